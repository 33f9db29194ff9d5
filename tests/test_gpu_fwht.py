"""The device's block Walsh-Hadamard kernels (the SubLN variant's o_proj /
down_proj input path: lz_fwht_i32, lz_fwht, subn_rot_f32, subn_fwht_quant)
against the oracle, bit for bit, through the C-ABI: integer transforms
including wrap-around, float transforms at every scale, the quantization on
ordinary, tiny, huge, denormal-sized, spiky, constant and all-zero rows,
with per-row and per-group scales (and group widths the reference ignores),
and the argument checks."""
import ctypes as C

import numpy as np
import pytest

from test_oracle_fwht import o_fwht_f32, o_fwht_i32, o_subn_quant, o_subn_rot, subn_rows

IP = C.POINTER(C.c_int32)
FP = C.POINTER(C.c_float)

SHAPES = [(1, 1), (64, 2), (64, 64), (256, 64), (1024, 256), (2048, 64), (2048, 512), (4096, 256),
          (8192, 8192)]


def by_blocks(fn, row, blk):
    return np.concatenate([fn(row[b:b + blk]) for b in range(0, len(row), blk)])


@pytest.mark.gpu
@pytest.mark.parametrize("n,blk", SHAPES)
def test_fwht_i32_matches_oracle(pkg, n, blk):
    lib = pkg.hip_lib()
    rng = np.random.default_rng(n + blk)
    rows = np.stack([rng.integers(-(1 << 15), 1 << 15, n),
                     rng.integers(-(1 << 31), 1 << 31, n, dtype=np.int64)]).astype(np.int32)
    y = np.zeros_like(rows)
    assert lib.l98_fwht_i32(rows.ctypes.data_as(IP), y.ctypes.data_as(IP), len(rows), n, blk) == 0
    for r in range(len(rows)):
        assert np.array_equal(y[r], by_blocks(o_fwht_i32, rows[r], blk)), f"n={n} blk={blk} row={r}"


@pytest.mark.gpu
@pytest.mark.parametrize("n,blk", SHAPES)
@pytest.mark.parametrize("rot", [0, 1])
def test_fwht_f32_matches_oracle(pkg, n, blk, rot):
    lib = pkg.hip_lib()
    rng = np.random.default_rng(7 * n + blk + rot)
    rows = np.stack([rng.standard_normal(n),
                     rng.standard_normal(n) * 2.0 ** rng.integers(-60, 60, n),
                     np.ldexp(rng.random(n), -140)]).astype(np.float32)
    v = rows.copy()
    assert lib.l98_fwht_f32(v.ctypes.data_as(FP), len(v), n, blk, rot) == 0
    for r in range(len(rows)):
        want = o_subn_rot(rows[r], blk) if rot else by_blocks(o_fwht_f32, rows[r], blk)
        assert v[r].tobytes() == want.tobytes(), f"n={n} blk={blk} rot={rot} row={r}"


@pytest.mark.gpu
@pytest.mark.parametrize("n,blk,gw", [(256, 64, 0), (512, 64, 32), (1024, 256, 0), (1024, 256, 128),
                                      (2048, 64, 2048), (768, 256, 96), (768, 256, 48), (4096, 256, 0),
                                      (8192, 256, 256), (8192, 8192, 0), (32, 32, 0), (64, 1, 0)])
def test_subn_fwht_quant_matches_oracle(pkg, n, blk, gw):
    lib = pkg.hip_lib()
    rng = np.random.default_rng(n + 3 * blk + gw)
    rows = np.stack(subn_rows(n, rng) + [np.zeros(n, np.float32),
                                         np.r_[np.zeros(n // 2), rng.standard_normal(n - n // 2)]]
                    ).astype(np.float32)
    q = np.zeros(rows.shape, np.int8)
    s = np.zeros((len(rows), n // 32), np.float32)
    assert lib.l98_subn_fwht_quant(rows.ctypes.data_as(FP), len(rows), n, blk, gw, q.ctypes.data,
                                   s.ctypes.data_as(FP)) == 0
    for r in range(len(rows)):
        qw, sw = o_subn_quant(rows[r], blk, gw)
        assert np.array_equal(q[r], qw), f"n={n} blk={blk} gw={gw} row={r}: codes differ"
        assert s[r].tobytes() == sw.tobytes(), f"n={n} blk={blk} gw={gw} row={r}: scales differ"


@pytest.mark.gpu
def test_fwht_argument_checks(pkg):
    lib = pkg.hip_lib()
    x = np.zeros(16384, np.float32)
    xi = np.zeros(16384, np.int32)
    q = np.zeros(16384, np.int8)
    s = np.zeros(512, np.float32)
    assert lib.l98_fwht_i32(xi.ctypes.data_as(IP), xi.ctypes.data_as(IP), 1, 16384, 64) == 1   # n > 8192
    assert lib.l98_fwht_i32(xi.ctypes.data_as(IP), xi.ctypes.data_as(IP), 1, 96, 48) == 1      # blk not 2^k
    assert lib.l98_fwht_f32(x.ctypes.data_as(FP), 1, 96, 64, 0) == 1                            # blk does not divide n
    assert lib.l98_fwht_f32(x.ctypes.data_as(FP), 0, 64, 64, 0) == 1                            # no rows
    assert lib.l98_subn_fwht_quant(x.ctypes.data_as(FP), 1, 48, 16, 0, q.ctypes.data, s.ctypes.data_as(FP)) == 1
    assert lib.l98_subn_fwht_quant(None, 1, 64, 64, 0, q.ctypes.data, s.ctypes.data_as(FP)) == 1
