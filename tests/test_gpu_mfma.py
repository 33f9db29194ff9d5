"""The wide int8 GEMM on the matrix cores (v_mfma_i32_16x16x32_i8, one
MFMA per 32-element quantization group) against the oracle's matmul
(o_matmul_q8: exact int32 group sums, the reference's epilogue order), bit
for bit, over shapes that leave partial row and token tiles."""
import numpy as np
import pytest

import oracle_lib as OL

pytestmark = pytest.mark.gpu


def case(rng, N, K, M):
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    w[0, :] = 127                                            # extreme codes
    ws = (rng.random(N).astype(np.float32) * 0.02 + 1e-4).astype(np.float32)
    x = rng.integers(-127, 128, (M, K), dtype=np.int8)
    x[-1, :] = -127
    xs = (rng.random((M, K // 32)).astype(np.float32) * 0.1).astype(np.float32)
    xs[0, 0] = 1.0                                           # a zero group's scale
    x[0, :32] = 0
    return w, ws, x, xs


@pytest.mark.parametrize("N,K,M", [(64, 32, 1), (100, 96, 70), (1024, 1024, 512), (2048, 1024, 33),
                                   (16, 64, 128), (8192, 256, 128), (768, 512, 65), (4096, 4096, 8),
                                   (256, 768, 100), (130, 2080, 64)])
def test_mfma_gemm_bit_exact(pkg, N, K, M):
    rng = np.random.default_rng(N * 7 + K + M)
    w, ws, x, xs = case(rng, N, K, M)
    out = np.zeros((M, N), np.float32)
    print(f"[case] mfma N={N} K={K} M={M}", flush=True)
    assert pkg.hip_lib().l98_gemm_q8(w.ctypes.data, OL.fp(ws), N, K, x.ctypes.data, OL.fp(xs), M, OL.fp(out)) == 0
    want = np.zeros((M, N), np.float32)
    OL.lib().o_matmul_q8(OL.fp(want), x.ctypes.data, OL.fp(xs), w.ctypes.data, OL.fp(ws), K, N, M, None)
    bad = np.nonzero(out.view(np.uint32) != want.view(np.uint32))
    assert len(bad[0]) == 0, (bad[0][:5], bad[1][:5], out[bad][:5], want[bad][:5])
