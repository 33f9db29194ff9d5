"""Pins the oracle's block Walsh-Hadamard functions (the SubLN o_proj /
down_proj path, src/fwht.c and src/forward_kda.c:43-135) before the device
kernels are compared with them: the transforms against the reference's own
exported lz_fwht_i32 / lz_fwht and against a dense Sylvester matrix, the
quantization and the float rotation against closed forms."""
import ctypes as C

import numpy as np
import pytest
from scipy.linalg import hadamard

import oracle_lib as OL
from test_oracle import ref

IP = C.POINTER(C.c_int32)
FP = C.POINTER(C.c_float)


def o_fwht_i32(x):
    x = np.ascontiguousarray(x, np.int32)
    y = np.empty_like(x)
    OL.lib().o_fwht_i32(y.ctypes.data_as(IP), x.ctypes.data_as(IP), len(x))
    return y


def o_fwht_f32(x):
    v = np.array(x, np.float32)
    OL.lib().o_fwht_f32(v.ctypes.data_as(FP), len(v))
    return v


def o_subn_quant(x, blk, gw):
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(len(x), np.int8)
    s = np.empty(len(x) // 32, np.float32)
    OL.lib().o_subn_fwht_quant(x.ctypes.data_as(FP), len(x), blk, gw, q.ctypes.data, s.ctypes.data_as(FP))
    return q, s


def o_subn_rot(x, blk):
    v = np.array(x, np.float32)
    OL.lib().o_subn_rot_f32(v.ctypes.data_as(FP), len(v), blk)
    return v


def block_h(x, blk):
    """Block-diagonal Sylvester product in float64 / int64."""
    H = hadamard(blk)
    return (x.reshape(-1, blk) @ H.T).reshape(-1)


SIZES = [1, 2, 4, 8, 64, 256, 512]


@pytest.mark.parametrize("n", SIZES)
def test_fwht_i32_dense_product_and_involution(n):
    rng = np.random.default_rng(n)
    x = rng.integers(-(1 << 15), 1 << 15, n).astype(np.int32)
    y = o_fwht_i32(x)
    assert np.array_equal(y.astype(np.int64), block_h(x.astype(np.int64), n))
    # H H = n I
    assert np.array_equal(o_fwht_i32(y).astype(np.int64), n * x.astype(np.int64))
    # wrapping int32: the dense product mod 2^32
    big = rng.integers(-(1 << 31), 1 << 31, n, dtype=np.int64).astype(np.int32)
    want = (block_h(big.astype(np.int64), n) & 0xFFFFFFFF).astype(np.uint32).view(np.int32)
    assert np.array_equal(o_fwht_i32(big), want)


@pytest.mark.parametrize("n", SIZES)
def test_fwht_f32_dense_product(n):
    rng = np.random.default_rng(100 + n)
    # small integers: every partial sum is exact in float
    xi = rng.integers(-1000, 1000, n).astype(np.float32)
    assert np.array_equal(o_fwht_f32(xi), block_h(xi.astype(np.float64), n).astype(np.float32))
    xf = rng.standard_normal(n).astype(np.float32)
    assert np.allclose(o_fwht_f32(xf), block_h(xf.astype(np.float64), n), rtol=0, atol=1e-5 * n)


def test_fwht_bitwise_vs_reference():
    L = ref()
    L.lz_fwht_i32.argtypes = [IP, IP, C.c_int]
    L.lz_fwht.argtypes = [FP, C.c_int]
    rng = np.random.default_rng(7)
    for n in SIZES + [1024]:
        x = rng.integers(-(1 << 20), 1 << 20, n).astype(np.int32)
        yr = np.empty_like(x)
        L.lz_fwht_i32(yr.ctypes.data_as(IP), x.ctypes.data_as(IP), n)
        assert np.array_equal(o_fwht_i32(x), yr)
        v = (rng.standard_normal(n) * 2.0 ** rng.integers(-30, 30, n)).astype(np.float32)
        vr = v.copy()
        L.lz_fwht(vr.ctypes.data_as(FP), n)
        assert o_fwht_f32(v).tobytes() == vr.tobytes()


def subn_rows(n, rng):
    rows = [rng.standard_normal(n) * 3.0,
            rng.standard_normal(n) * 1e-6,
            rng.standard_normal(n) * 1e20,
            np.ldexp(rng.random(n), -130),                  # denormal-sized
            np.where(rng.random(n) < 0.05, 50.0, 0.01) * np.sign(rng.standard_normal(n)),
            np.r_[np.zeros(n - 1), 7.0],                    # one spike
            np.ones(n)]
    return [np.ascontiguousarray(r, np.float32) for r in rows]


@pytest.mark.parametrize("n,blk,gw", [(256, 64, 0), (512, 64, 32), (1024, 256, 0), (1024, 256, 128),
                                      (2048, 64, 2048), (768, 256, 96), (512, 512, 64)])
def test_subn_fwht_quant_closed_form(n, blk, gw):
    """Zero rows give q = 0, s = 1; S puts the row max in [2^14, 2^15);
    every group's largest code is 127; q * s reproduces H x / sqrt(blk) to
    half a code plus the fixed-point rounding of x * S."""
    rng = np.random.default_rng(n + blk + gw)
    q, s = o_subn_quant(np.zeros(n, np.float32), blk, gw)
    assert not q.any() and np.all(s == 1.0)
    g = gw if gw > 0 and gw % 32 == 0 and n % gw == 0 else n
    for x in subn_rows(n, rng):
        q, s = o_subn_quant(x, blk, gw)
        amax = np.abs(x).max()
        e = int((np.abs(x).view(np.uint32).max() >> 23) & 0xFF) - 127
        S = 2.0 ** min(14 - e, 127)
        if 14 - e <= 127:
            assert 2 ** 14 <= amax * S < 2 ** 15
        t = block_h(np.rint(x.astype(np.float64) * S), blk)           # the exact int32 transform
        want = block_h(x.astype(np.float64), blk) / np.sqrt(blk)
        sc = np.repeat(s, 32)
        for b in range(0, n, g):
            grp = slice(b, b + g)
            assert len(set(s[b // 32:(b + g) // 32].tolist())) == 1
            if np.abs(t[grp]).max() == 0:
                assert not q[grp].any() and s[b // 32] == 1.0
            else:
                assert np.abs(q[grp].astype(int)).max() == 127
        err = np.abs(q * sc.astype(np.float64) - want)
        bound = 0.5 * sc * 1.0001 + np.sqrt(blk) * 0.5 / S + 1e-6 * np.abs(want)
        live = sc != 1.0
        assert np.all(err[live] <= bound[live])


@pytest.mark.parametrize("n,blk", [(64, 64), (512, 64), (1024, 256), (2048, 512)])
def test_subn_rot_f32_dense_product(n, blk):
    rng = np.random.default_rng(n * blk)
    inv = OL.lib().o_rsqrt(float(blk))
    # unit vectors: the transform is exactly +-1, so the row is exactly +-inv
    for i in (0, blk - 1, n - 1):
        e = np.zeros(n, np.float32)
        e[i] = 1.0
        r = o_subn_rot(e, blk)
        b0 = (i // blk) * blk
        want = np.zeros(n, np.float32)
        want[b0:b0 + blk] = hadamard(blk)[:, i - b0] * np.float32(inv)
        assert r.tobytes() == want.tobytes()
    x = rng.standard_normal(n).astype(np.float32)
    assert np.allclose(o_subn_rot(x, blk), block_h(x.astype(np.float64), blk) / np.sqrt(blk), rtol=0, atol=1e-4)


@pytest.fixture(scope="module")
def ref_subn():
    """The reference's own static subn_fwht_quant / subn_rot_f32, exported by
    oracle/ref_subn.c (built by oracle/ref.mk), in the float-oracle mode."""
    import os
    path = os.path.join(OL.REF_DIR, "libl98ref_subn.so")
    if not os.path.exists(path):
        pytest.skip("reference build absent (oracle/_ref)")
    L = C.CDLL(path)
    L.lz_float_ref_select.restype = C.c_char_p
    L.lz_float_ref_select.argtypes = [C.c_char_p]
    L.lz_fastfp_select.restype = C.c_char_p
    L.lz_fastfp_select.argtypes = [C.c_char_p]
    L.lz_float_ref_select(b"off")
    L.lz_fastfp_select(b"off")
    L.l98ref_subn_fwht_quant.argtypes = [FP, C.c_int, C.c_int, C.c_int, C.c_void_p, FP]
    L.l98ref_subn_rot_f32.argtypes = [FP, C.c_int, C.c_int]
    return L


SUBN_SHAPES = [(256, 64, 0), (512, 64, 32), (1024, 256, 0), (1024, 256, 128), (2048, 64, 2048), (768, 256, 96),
               (512, 512, 64), (8192, 8192, 0), (4096, 128, 64)]


@pytest.mark.parametrize("n,blk,gw", SUBN_SHAPES)
def test_subn_fwht_quant_bitwise_vs_reference(ref_subn, n, blk, gw):
    """The oracle's subn_fwht_quant against the reference's own static
    function: codes and scales bit for bit, which pins the scale's multiply
    order (tam * inv_S) * rsqrt(blk) * (1/127)."""
    rng = np.random.default_rng(3 * n + blk + gw)
    rows = subn_rows(n, rng) + [np.zeros(n, np.float32),
                                (rng.standard_normal(n) * 2.0 ** rng.integers(-60, 60, n)).astype(np.float32)]
    for x in rows:
        x = np.ascontiguousarray(x, np.float32)
        q, s = o_subn_quant(x, blk, gw)
        qr = np.empty(n, np.int8)
        sr = np.empty(n // 32, np.float32)
        ref_subn.l98ref_subn_fwht_quant(x.ctypes.data_as(FP), n, blk, gw, qr.ctypes.data, sr.ctypes.data_as(FP))
        assert np.array_equal(q, qr)
        assert s.tobytes() == sr.tobytes()


@pytest.mark.parametrize("n,blk", [(64, 64), (512, 64), (1024, 256), (2048, 512), (8192, 8192)])
def test_subn_rot_f32_bitwise_vs_reference(ref_subn, n, blk):
    rng = np.random.default_rng(n + blk)
    for x in subn_rows(n, rng):
        vr = np.array(x, np.float32)
        ref_subn.l98ref_subn_rot_f32(vr.ctypes.data_as(FP), n, blk)
        assert o_subn_rot(x, blk).tobytes() == vr.tobytes()
