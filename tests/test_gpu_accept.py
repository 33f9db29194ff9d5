"""Acceptance machinery on the GPU: the device argmax the rounds run (draft
steps: lz_argmax_p1's order; verify rows: lz_sample_argmax's), the library's
own lz_spec_accept / lz_argmax_p1, and draft width k = 7 (a verify of
M = 8 rows, past the reference's LZ_SPEC_K_MAX = 6) against the oracle's
same algorithm with an 8-slot ring and against the width invariant."""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as OL
from oracle_lib import Oracle, fp, ip

pytestmark = pytest.mark.gpu


def rows_with_specials(rng, rows, n):
    x = rng.standard_normal((rows, n)).astype(np.float32)
    x[0, 0] = np.nan                                   # NaN at 0: argmax_p1 answers 0
    x[1, n // 2] = np.nan                              # NaN elsewhere never wins
    x[1, 3] = 50.0
    x[2, :] = 0.0
    x[2, 5] = -0.0                                     # ties: first index
    x[3, 7] = np.inf
    x[3, 9] = np.inf
    x[4, :] = -np.inf
    x[5, n - 1] = 1e30                                 # the last element wins
    return x


@pytest.mark.parametrize("n", [64, 8191, 65536 + 7])
def test_device_argmax_matches_oracle(pkg, n):
    lib = pkg.hip_lib()
    L = OL.lib()
    rng = np.random.default_rng(n)
    x = rows_with_specials(rng, 8, n)
    for mode in (0, 1):
        out = np.zeros(8, np.int32)
        assert lib.l98_argmax_rows(fp(x), 8, n, mode, ip(out)) == 0
        for r in range(8):
            row = np.ascontiguousarray(x[r])
            if mode == 0:
                want = L.o_argmax(fp(row), n)
            else:
                p = C.c_float()
                want = L.o_argmax_p1(fp(row), n, C.byref(p))
            assert out[r] == want, (mode, r, out[r], want)


@pytest.mark.parametrize("M,gs", [(1, 0), (2, 0), (3, 0), (4, 0), (5, 0), (6, 0), (8, 0), (1, 64), (4, 64), (6, 64),
                                  (1, 128), (4, 128)])
def test_gemv_argmax_epilogue_matches_oracle(pkg, M, gs):
    # The rounds' argmax: per-tile candidates from the lm_head GEMV's
    # epilogue, reduced by l98k_argmax_part, with one scale per weight row
    # (gs = 0) or grouped scales (the instances a model.bin with Q8_0 groups
    # of 64 or 128 runs).  Row scales plant the special values in whole logit
    # columns: NaN at index 0 and elsewhere, +inf ties, a band of zeros (0
    # scale, and -0 scale), and a maximum in the last row.
    lib = pkg.hip_lib()
    L = OL.lib()
    N, K = 65536 + 40, 1024
    nws = K // gs if gs else 1
    rng = np.random.default_rng(M + gs)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    xq = rng.integers(-127, 128, (M, K), dtype=np.int8)
    xqs = (rng.random((M, K // 32)) * 0.01 + 1e-4).astype(np.float32)
    ws = (rng.random((N, nws)) * 0.01).astype(np.float32)
    ws[0] = np.nan
    ws[777] = np.nan
    ws[100:140] = 0.0
    ws[140:160] = -0.0
    ws[3000] = ws[5000] = np.inf
    ws[N - 1] = 1e30
    print(f"[case] gemv argmax M={M} gs={gs}", flush=True)
    for mode in (0, 1):
        for plant in (True, False):
            s = ws.copy()
            if not plant:                                # finite rows only: ties by value
                s[[0, 777, 3000, 5000, N - 1]] = 0.0
            logits = np.zeros((M, N), np.float32)
            out = np.zeros(M, np.int32)
            assert lib.l98_gemv_argmax(w.ctypes.data, fp(np.ascontiguousarray(s)), N, K, gs, xq.ctypes.data,
                                       fp(xqs), M, mode, fp(logits), ip(out)) == 0
            for r in range(M):
                row = np.ascontiguousarray(logits[r])
                if mode == 0:
                    want = L.o_argmax(fp(row), N)
                else:
                    p = C.c_float()
                    want = L.o_argmax_p1(fp(row), N, C.byref(p))
                assert out[r] == want, (mode, plant, r, out[r], want)


def test_library_spec_accept_exhaustive(pkg):
    """lz_spec_accept of the library (src/generate.c:232-243) against the
    oracle's and the definition, over every draft/target pair on 3 symbols
    up to length 4."""
    import itertools
    lib = pkg.hip_lib()
    L = OL.lib()
    for n in range(0, 5):
        for draft in itertools.product(range(3), repeat=n):
            for targ in itertools.product(range(3), repeat=n):
                d = np.array(draft + (0,), np.int32)
                t = np.array(targ + (0,), np.int32)
                a = np.full(n + 1, -9, np.int32)
                b = np.full(n + 1, -9, np.int32)
                ra = lib.lz_spec_accept(ip(d), ip(t), n, 7, ip(a))
                rb = L.o_spec_accept(ip(d), ip(t), n, 7, ip(b))
                assert ra == rb and np.array_equal(a[:ra + 1], b[:rb + 1]), (draft, targ)
                m = next((i for i in range(n) if draft[i] != targ[i]), n)
                assert ra == m


def test_library_argmax_p1_matches_oracle(pkg):
    lib = pkg.hip_lib()
    L = OL.lib()
    rng = np.random.default_rng(3)
    x = rows_with_specials(rng, 8, 4099)
    for r in range(8):
        row = np.ascontiguousarray(x[r])
        pa, pb = C.c_float(), C.c_float()
        ia = lib.lz_argmax_p1(fp(row), len(row), C.byref(pa))
        ib = L.o_argmax_p1(fp(row), len(row), C.byref(pb))
        assert ia == ib
        assert np.float32(pa.value).tobytes() == np.float32(pb.value).tobytes() or (
            np.isnan(pa.value) and np.isnan(pb.value))


@pytest.fixture(scope="module")
def echo(pkg, model_root):
    import os
    return pkg.ensure_model(os.path.join(model_root, "echo"), 11, seed=1234)


def test_k7_greedy_matches_oracle_and_spec1(pkg, echo):
    prompt = pkg.prompt_tokens(11, 24, 64)
    print("[case] echo greedy k=7", flush=True)
    ora = Oracle(echo, spec_k_max=7)
    try:
        ot, oke, ona, _ = ora.generate(prompt, 7, 180)
        o1 = ora.generate(prompt, 1, 180)[0]
    finally:
        ora.close()
    assert max(ona) == 7 and set(ona) >= {0, 7}
    assert np.array_equal(ot[:180], o1[:180]), "greedy k=7 must emit the k=1 sequence"
    eng = pkg.Engine(echo, spec_k_max=7)
    try:
        toks, ke, na = eng.generate(prompt, 7, 180)
        n = min(len(toks), len(ot))
        assert np.array_equal(toks[:n], ot[:n])
        assert list(ke) == list(oke) and list(na) == list(ona)
    finally:
        eng.close()


def test_k7_temperature_matches_oracle(pkg, echo):
    prompt = pkg.prompt_tokens(11, 24, 64)
    print("[case] echo temperature k=7", flush=True)
    ora = Oracle(echo, spec_k_max=7)
    try:
        ot, oke, ona, orng = ora.generate(prompt, 7, 120, 0.8, 0.95, 7)
    finally:
        ora.close()
    assert max(ona) >= 4
    eng = pkg.Engine(echo, spec_k_max=7)
    try:
        toks, ke, na = eng.generate(prompt, 7, 120, 0.8, 0.95, 7)
        n = min(len(toks), len(ot))
        assert np.array_equal(toks[:n], ot[:n])
        assert list(ke) == list(oke) and list(na) == list(ona)
        assert eng.last_rng == orng
    finally:
        eng.close()


def test_reference_entry_points_keep_the_reference_cap(pkg, echo):
    """lz_spec_round refuses k = 7 with LZ_ERR_SPEC_K_RANGE, as the
    reference does (src/generate.c:724-727), even on an 8-slot ring."""
    eng = pkg.Engine(echo, spec_k_max=7)
    try:
        prompt = pkg.prompt_tokens(11, 24, 64)
        eng.session_start(prompt)
        r = eng.spec_round(int(prompt[-1]), 23, 7)[0]
        assert r == -pkg.LZ_ERR["SPEC_K_RANGE"]
    finally:
        eng.close()


def test_verify_of_eight_rows_equals_single_steps(pkg, echo):
    """The M = 8 verify (k = 7) gives each row exactly the logits and hidden
    of forwarding that token alone."""
    prompt = pkg.prompt_tokens(3, 24, 64)
    toks = np.array([5, 17, 17, 40, 2, 63, 0, 31], np.int32)
    a = pkg.Engine(echo, spec_k_max=7)
    b = pkg.Engine(echo, spec_k_max=7)
    try:
        for e in (a, b):
            e.reset()
            assert e.batch_capture(prompt, 0) is not None
        lg, hd = a.verify(toks, len(prompt))
        for j, t in enumerate(toks):
            single = b.forward_capture(int(t), len(prompt) + j)
            assert np.array_equal(single.view(np.uint32), lg[j].view(np.uint32)), j
            assert np.array_equal(b.chain().view(np.uint32), hd[j].view(np.uint32)), j
    finally:
        a.close()
        b.close()
