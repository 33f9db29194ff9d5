"""The parallel index-order sum the RMSNorm kernels use for their sums of
squares (wave_sum_nonneg) against the serial float loop it replaces, on
inputs chosen to break it: exact ties against the running sum's grid,
binade crossings at every scale, leading zeros, denormals, powers of two
with few mantissa bits, huge values near the float range, single spikes,
and infinities / NaNs (which must take its serial path).  The model-level
parity tests only see ordinary activations; these rows cover the rest."""
import ctypes as C

import numpy as np
import pytest


def serial_sum(x):
    # s = 0; for v in x: s += v, in float32 (add.accumulate is sequential)
    return np.add.accumulate(x.astype(np.float32), dtype=np.float32)[-1] if len(x) else np.float32(0)


def rows_of(kind, n, count, rng):
    out = np.empty((count, n), np.float32)
    for r in range(count):
        if kind == "squares":
            v = rng.standard_normal(n).astype(np.float32) ** 2
        elif kind == "wide":
            v = (rng.standard_normal(n) * 2.0 ** rng.integers(-20, 20, n)).astype(np.float32) ** 2
        elif kind == "ties":
            v = (rng.integers(0, 16, n) * 0.5).astype(np.float32)
        elif kind == "short_mantissa":
            v = (rng.integers(0, 1024, n) / 1024.0).astype(np.float32)
        elif kind == "leading_zeros":
            v = rng.standard_normal(n).astype(np.float32) ** 2
            v[: n // 2] = 0
        elif kind == "denormal":
            v = np.ldexp(rng.random(n), -140).astype(np.float32)
        elif kind == "softmax_like":
            v = np.exp(rng.standard_normal(n) * 3).astype(np.float32)
        elif kind == "spikes":
            v = rng.random(n).astype(np.float32)
            hit = rng.random(n) < 0.02
            v[hit] = np.ldexp(1.0, rng.integers(0, 30, hit.sum())).astype(np.float32)
        elif kind == "tiny_first":
            v = rng.standard_normal(n).astype(np.float32) ** 2
            v[0] = 1e-30
        elif kind == "few_bits":
            v = np.ldexp(1.0 + rng.integers(0, 8, n) / 8.0, rng.integers(0, 6, n)).astype(np.float32)
        elif kind == "huge":
            v = np.ldexp(rng.random(n), 100).astype(np.float32)
            v[rng.random(n) < 0.15] = 0
        elif kind == "ones":
            v = np.ones(n, np.float32)
        elif kind == "inf":
            v = rng.random(n).astype(np.float32)
            v[rng.integers(0, n)] = np.inf
        elif kind == "nan":
            v = rng.random(n).astype(np.float32)
            v[rng.integers(0, n)] = np.nan
        else:
            raise ValueError(kind)
        out[r] = v
    return out


KINDS = ["squares", "wide", "ties", "short_mantissa", "leading_zeros", "denormal", "softmax_like", "spikes",
         "tiny_first", "few_bits", "huge", "ones", "inf", "nan"]


def test_serial_sum_is_the_float_loop():
    rng = np.random.default_rng(5)
    for n in (1, 7, 300):
        x = (rng.standard_normal(n) ** 2).astype(np.float32)
        s = np.float32(0)
        for v in x:
            s = np.float32(s + v)
        assert serial_sum(x).tobytes() == s.tobytes()


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 64, 77, 256, 512, 768, 1000, 1024, 1500, 2048])
def test_row_sums_match_serial_loop(pkg, n):
    lib = pkg.hip_lib()
    rng = np.random.default_rng(1000 + n)
    rows = np.concatenate([rows_of(k, n, 24, rng) for k in KINDS])
    out = np.zeros(len(rows), np.float32)
    fp = C.POINTER(C.c_float)
    assert lib.l98_row_sums(np.ascontiguousarray(rows).ctypes.data_as(fp), len(rows), n,
                            out.ctypes.data_as(fp)) == 0
    want = np.array([serial_sum(r) for r in rows], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(out), nan)
    bad = np.nonzero(out[~nan].view(np.uint32) != want[~nan].view(np.uint32))[0]
    kinds = np.repeat(KINDS, 24)[~nan]
    assert len(bad) == 0, f"n={n}: {len(bad)} rows differ, e.g. kind {kinds[bad[0]]}: " \
                          f"{out[~nan][bad[0]]!r} vs {want[~nan][bad[0]]!r}"


def serial_prefix(x):
    return np.add.accumulate(x.astype(np.float32), dtype=np.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 100, 1024, 5000, 32000, 65536, 131072])
def test_prefix_queries_match_serial_loop(pkg, n):
    """The sampler's engine (one block per row over global memory): totals,
    first prefix above a coin, first prefix reaching a limit."""
    lib = pkg.hip_lib()
    rng = np.random.default_rng(77 + n)
    kinds = [k for k in KINDS if k not in ("inf", "nan")]
    per = 2 if n >= 32000 else 4
    rows = np.concatenate([rows_of(k, n, per, rng) for k in kinds])
    pre = np.stack([serial_prefix(r) for r in rows])
    tot = pre[:, -1]
    fp, ip = C.POINTER(C.c_float), C.POINTER(C.c_int)
    xs = np.ascontiguousarray(rows)
    for mode in (0, 1, 2):
        # thresholds inside the range, at exact prefix values, and past the end
        c = np.empty(len(rows), np.float32)
        for r in range(len(rows)):
            pick = rng.integers(0, 3)
            if pick == 0:
                c[r] = np.float32(tot[r] * rng.random())
            elif pick == 1:
                c[r] = pre[r, rng.integers(0, n)]
            else:
                c[r] = np.float32(tot[r] * 2 + 1)
        out = np.zeros(len(rows), np.int32)
        outv = np.zeros(len(rows), np.float32)
        assert lib.l98_prefix_query(xs.ctypes.data_as(fp), len(rows), n, mode, c.ctypes.data_as(fp),
                                    out.ctypes.data_as(ip), outv.ctypes.data_as(fp)) == 0
        for r in range(len(rows)):
            if mode == 0:
                want_i, want_v = -1, tot[r]
            else:
                hit = np.nonzero(c[r] < pre[r] if mode == 1 else pre[r] >= c[r])[0]
                want_i = int(hit[0]) if len(hit) else -1
                want_v = pre[r, want_i] if len(hit) else tot[r]
            assert out[r] == want_i, f"n={n} mode={mode} row {r}: index {out[r]} vs {want_i}"
            assert outv[r].tobytes() == np.float32(want_v).tobytes(), \
                f"n={n} mode={mode} row {r}: {outv[r]!r} vs {want_v!r}"


@pytest.mark.gpu
@pytest.mark.parametrize("V", [16, 65536])
def test_spec_accept_temp_on_device_matches_oracle(pkg, V):
    """The library's lz_spec_accept_temp (host rows through the device
    acceptance kernel) against the oracle's restatement: u just below, at and
    above p[x]/q[x], a rejected draft's residual draw and the generator
    state it leaves, and q[x] = 0."""
    import oracle_lib as OL
    O = OL.lib()
    lib = pkg.hip_lib()
    lib.lz_spec_accept_temp.restype = C.c_int
    lib.lz_spec_accept_temp.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_float,
                                        C.POINTER(C.c_uint64), C.POINTER(C.c_int)]
    fp = C.POINTER(C.c_float)
    rng = np.random.default_rng(V)
    p = rng.dirichlet(np.ones(V)).astype(np.float32)
    q = rng.dirichlet(np.ones(V)).astype(np.float32)
    xs = range(V) if V <= 16 else rng.integers(0, V, 12)
    for x in xs:
        x = int(x)
        ratio = np.float32(p[x] / q[x])
        for u in (np.nextafter(ratio, np.float32(0)), ratio, np.nextafter(ratio, np.float32(2))):
            u = np.float32(min(u, np.float32(0.999999)))
            st, st2 = C.c_uint64(12345), C.c_uint64(12345)
            acc, acc2 = C.c_int(), C.c_int()
            tok = O.o_spec_accept_temp(p.ctypes.data_as(fp), q.ctypes.data_as(fp), x, V, float(u), C.byref(st),
                                       C.byref(acc))
            t2 = lib.lz_spec_accept_temp(p.ctypes.data, q.ctypes.data, x, V, C.c_float(u), C.byref(st2),
                                         C.byref(acc2))
            assert (t2, acc2.value, st2.value) == (tok, acc.value, st.value), (x, u)
    q0 = q.copy()
    q0[3] = 0.0
    st, st2 = C.c_uint64(1), C.c_uint64(1)
    acc, acc2 = C.c_int(), C.c_int()
    tok = O.o_spec_accept_temp(p.ctypes.data_as(fp), q0.ctypes.data_as(fp), 3, V, 0.0, C.byref(st), C.byref(acc))
    t2 = lib.lz_spec_accept_temp(p.ctypes.data, q0.ctypes.data, 3, V, C.c_float(0.0), C.byref(st2), C.byref(acc2))
    assert (t2, acc2.value, st2.value) == (tok, acc.value, st.value)
