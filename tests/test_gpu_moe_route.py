"""The expert kernels' in-block MoE routing (route_block, through
l98_moe_route) against the oracle's lz_moe_route restatement, token by
token: random logits at every chunk size and top-k, and rows built to hit
the selection loop's edges (exact key ties, scores that underflow to zero so
the weights are not renormalized, NaN and infinite logits, keys at or below
the -1e30 sentinel that the loop never picks, top-k above the expert
count).  The model-level parity tests only route ordinary activations."""
import ctypes as C

import numpy as np
import pytest

CASES = [(1, 64, 6), (4, 64, 6), (8, 64, 8), (3, 40, 5), (8, 128, 8), (2, 100, 3), (5, 7, 7), (1, 1, 1),
         (6, 3, 5), (8, 65, 2), (7, 127, 4)]


def chunk_of(kind, nt, E, rng):
    lg = (rng.standard_normal((nt, E)) * 3).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    if kind == "ties":                   # few distinct keys: exact ties everywhere
        lg = (rng.integers(-2, 3, (nt, E)) * 0.5).astype(np.float32)
        bias = np.zeros(E, np.float32)
    elif kind == "underflow":            # scores 0: keys tie at the bias, weights sum to 0
        lg = np.full((nt, E), -200.0, np.float32)
        lg[:, ::5] = rng.standard_normal((nt, len(range(0, E, 5)))).astype(np.float32) * -300
        bias = (rng.integers(-1, 2, E) * 0.25).astype(np.float32)
    elif kind == "nan":                  # NaN first, in the middle, and everywhere
        lg[0, 0] = np.nan
        if nt > 1:
            lg[1, E // 2] = np.nan
        if nt > 2:
            lg[2, :] = np.nan
    elif kind == "inf":
        lg[:, rng.integers(0, E, max(1, E // 8))] = np.inf
        lg[:, rng.integers(0, E, max(1, E // 8))] = -np.inf
    elif kind == "sentinel":             # biases at and below -1e30 are never selected
        bias[rng.integers(0, E, max(1, E // 3))] = -1e30
        bias[rng.integers(0, E, max(1, E // 3))] = -3e30
        if nt > 1 and E > 1:
            bias[:] = -1e31                  # every key excluded: idx -1, w 0
    elif kind == "bias_inf":
        bias[rng.integers(0, E, max(1, E // 4))] = np.inf
    return np.ascontiguousarray(lg), np.ascontiguousarray(bias)


KINDS = ["random", "ties", "underflow", "nan", "inf", "sentinel", "bias_inf"]


@pytest.mark.gpu
@pytest.mark.parametrize("nt,E,topk", CASES)
def test_device_routing_matches_oracle(pkg, nt, E, topk):
    import oracle_lib as OL
    O = OL.lib()
    lib = pkg.hip_lib()
    fp, ip = C.POINTER(C.c_float), C.POINTER(C.c_int)
    rng = np.random.default_rng(nt * 1000 + E * 10 + topk)
    for kind in KINDS:
        for rep in range(6):
            lg, bias = chunk_of(kind, nt, E, rng)
            idx = np.full((nt, topk), -7, np.int32)
            w = np.full((nt, topk), 7.0, np.float32)
            print(f"route nt={nt} E={E} topk={topk} kind={kind} rep={rep}", flush=True)
            assert lib.l98_moe_route(lg.ctypes.data_as(fp), bias.ctypes.data_as(fp), nt, E, topk,
                                     idx.ctypes.data_as(ip), w.ctypes.data_as(fp)) == 0
            for t in range(nt):
                wi = np.zeros(topk, np.int32)
                ww = np.zeros(topk, np.float32)
                O.o_moe_route(np.ascontiguousarray(lg[t]).ctypes.data_as(fp), bias.ctypes.data_as(fp), E, topk,
                              wi.ctypes.data_as(ip), ww.ctypes.data_as(fp))
                where = f"{kind} rep {rep} token {t}"
                assert idx[t].tolist() == wi.tolist(), f"{where}: experts {idx[t]} vs {wi}"
                nan = np.isnan(ww)
                assert np.array_equal(np.isnan(w[t]), nan), f"{where}: weights {w[t]} vs {ww}"
                assert w[t][~nan].tobytes() == ww[~nan].tobytes(), f"{where}: weights {w[t]} vs {ww}"


@pytest.mark.gpu
def test_device_routing_null_bias_and_bad_arguments(pkg):
    import oracle_lib as OL
    O = OL.lib()
    lib = pkg.hip_lib()
    fp, ip = C.POINTER(C.c_float), C.POINTER(C.c_int)
    lg = np.random.default_rng(3).standard_normal((4, 64)).astype(np.float32)
    idx = np.zeros((4, 6), np.int32)
    w = np.zeros((4, 6), np.float32)
    assert lib.l98_moe_route(lg.ctypes.data_as(fp), None, 4, 64, 6, idx.ctypes.data_as(ip), w.ctypes.data_as(fp)) == 0
    for t in range(4):
        wi = np.zeros(6, np.int32)
        ww = np.zeros(6, np.float32)
        O.o_moe_route(np.ascontiguousarray(lg[t]).ctypes.data_as(fp), None, 64, 6, wi.ctypes.data_as(ip),
                      ww.ctypes.data_as(fp))
        assert idx[t].tolist() == wi.tolist() and w[t].tobytes() == ww.tobytes()
    for nt, E, topk in ((0, 64, 6), (9, 64, 6), (4, 129, 6), (4, 64, 9), (4, 0, 1)):
        assert lib.l98_moe_route(lg.ctypes.data_as(fp), None, nt, E, topk, idx.ctypes.data_as(ip),
                                 w.ctypes.data_as(fp)) == 1
