"""The no-allocation acceptance entry point against lz_spec_accept_temp
through the C ABI: same token, same accept flag, same generator state, on
two calls in a row with the second over a smaller vocabulary (the static
staging then still holds the first call's longer rows past the new end)."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as OL

pytestmark = pytest.mark.gpu


def dist(rng, n, zero_at=None):
    p = rng.random(n).astype(np.float32) ** 4
    if zero_at is not None:
        p[zero_at] = 0.0
    return (p / p.sum(dtype=np.float64)).astype(np.float32)


def both(lib, p, q, x, u, seed):
    ra, rb = C.c_uint64(seed), C.c_uint64(seed)
    aa, ab = C.c_int(-7), C.c_int(-7)
    ta = lib.lz_spec_accept_temp(OL.fp(p), OL.fp(q), x, len(p), u, C.byref(ra), C.byref(aa))
    tb = lib.l98_spec_accept_temp_noalloc(OL.fp(p), OL.fp(q), x, len(p), u, C.byref(rb), C.byref(ab))
    return (ta, aa.value, ra.value), (tb, ab.value, rb.value)


def test_noalloc_accept_matches_the_allocating_entry_point(pkg):
    lib = pkg.hip_lib()
    rng = np.random.default_rng(11)
    for V in (131072, 1000):                 # two calls in a row, the second smaller
        print(f"[case] no-alloc accept V={V}", flush=True)
        p, q = dist(rng, V), dist(rng, V, zero_at=5)
        for x, u in ((3, 0.999), (3, 0.0), (5, 0.5), (V - 1, 0.25)):
            ra, rb = both(lib, p, q, x, float(u), 1234 + x)
            assert ra == rb, (V, x, u, ra, rb)
            assert 0 <= ra[0] < V
    # a rejection that draws from the residual, and one whose ratio accepts
    p, q = dist(rng, 4096), dist(rng, 4096)
    x = int(np.argmax(q / np.maximum(p, 1e-30)))
    ra, rb = both(lib, p, q, x, 0.999999, 99)
    assert ra == rb and ra[1] == 0
    x = int(np.argmax(p / q))
    ra, rb = both(lib, p, q, x, 0.5, 99)
    assert ra == rb and ra[1] == 1


def test_noalloc_accept_refuses_oversize_and_bad_input(pkg):
    lib = pkg.hip_lib()
    big = pkg.L98_NOALLOC_MAX_VOCAB + 1
    p = np.full(big, 1.0 / big, np.float32)
    r, acc = C.c_uint64(1), C.c_int(5)
    assert lib.l98_spec_accept_temp_noalloc(OL.fp(p), OL.fp(p), 0, big, 0.5, C.byref(r), C.byref(acc)) == -2
    assert acc.value == 0 and r.value == 1
    assert lib.l98_spec_accept_temp_noalloc(OL.fp(p), OL.fp(p), 10, 8, 0.5, C.byref(r), C.byref(acc)) == -1
