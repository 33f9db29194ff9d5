"""The temperature path's own pieces on the GPU:

  * the top-p candidates' order: the library's radix sort (three passes of
    10-bit digits, descending, equal keys in index order, as select_all's
    qsort orders the candidates, src/sampler.c:526-538) against numpy's
    stable sort, over ties, zeros, the largest key and tile boundaries;
  * the reference entry point lz_spec_round_temp driven round by round from
    the host against the reference's recorded temperature generations (the
    device-resident rounds of l98_generate are checked against the same
    fixtures in test_gpu_golden.py)."""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def want_order(keys):
    idx = np.arange(len(keys))
    return np.lexsort((idx, -keys.astype(np.int64)))


@pytest.mark.parametrize("n", [1, 5, 1023, 1024, 1025, 8192, 65536, 65537, 131072])
def test_radix_sort_is_stable_descending(pkg, n):
    lib = pkg.hip_lib()
    rng = np.random.default_rng(n)
    print(f"[case] radix sort n={n}", flush=True)
    cases = {
        # probabilities of a flat softmax, rounded so that many are equal
        "ties": np.round(rng.random(n) * 64).astype(np.float32) / np.float32(64 * n),
        # the candidates of a peaked row: a few large keys, most below the cutoff (0)
        "sparse": np.where(rng.random(n) < 0.05, rng.random(n), 0.0).astype(np.float32),
        "equal": np.full(n, 1.0 / n, np.float32),
        "extremes": np.where(rng.random(n) < 0.5, np.float32(1.0), np.float32(1e-30)).astype(np.float32),
    }
    for name, p in cases.items():
        keys = p.view(np.uint32).copy()
        if n > 3:
            keys[[0, n // 2, n - 1]] = [0, 0x3F800000, 1]
        out_k = np.zeros(n, np.uint32)
        out_i = np.zeros(n, np.int32)
        assert lib.l98_sort_desc(keys.ctypes.data, n, out_k.ctypes.data,
                                 out_i.ctypes.data_as(pkg.C.POINTER(pkg.C.c_int))) == 0
        order = want_order(keys)
        assert np.array_equal(out_i, order), name
        assert np.array_equal(out_k, keys[order]), name


TEMP_FIXTURES = sorted(f for f in os.listdir(GOLDEN)
                       if f.startswith("gen_") and f.endswith("_temp.json") and not f.startswith("gen_ds_"))


@pytest.mark.parametrize("fname", TEMP_FIXTURES)
def test_host_temperature_rounds_match_fixture(pkg, model_root, fname):
    g = json.load(open(os.path.join(GOLDEN, fname)))
    model = pkg.ensure_model(os.path.join(model_root, g["model"]), g["config_id"], seed=g["model_seed"])
    prompt = pkg.prompt_tokens(g["prompt_seed"], g["n_prompt"], g["vocab"])
    print(f"[case] host temperature rounds {fname}", flush=True)
    eng = pkg.Engine(model)
    try:
        toks, ke, na = eng.generate_host_temp(prompt, g["k"], g["n_new"], g["temp"], g["topp"], g["sampler_seed"])
        want = np.array(g["tokens"], np.int32)
        n = min(len(toks), len(want))
        assert n >= g["n_new"]
        bad = np.nonzero(toks[:n] != want[:n])[0]
        assert len(bad) == 0, f"first divergence at token {bad[0]}"
        assert list(ke) == g["k_eff"] and list(na) == g["n_accept"]
        assert eng.last_rng == g["rng"]
    finally:
        eng.close()
