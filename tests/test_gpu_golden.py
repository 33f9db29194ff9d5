"""GPU generations against the reference engine's recorded outputs
(tests/golden/, written by tests/golden/make_golden.py from the reference
build): micro, configs[0] (tiny) and configs[1] (base, the benchmark model),
greedy and fixed-seed temperature.  Needs no reference and no oracle at run
time."""
import hashlib
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(f for f in os.listdir(GOLDEN) if f.startswith("gen_") and f.endswith(".json"))


@pytest.mark.parametrize("fname", FIXTURES)
def test_generation_matches_reference_fixture(pkg, model_root, fname):
    g = json.load(open(os.path.join(GOLDEN, fname)))
    print(f"[case] golden {fname}", flush=True)
    model = pkg.ensure_model(os.path.join(model_root, g["model"]), g["config_id"], seed=g["model_seed"])
    h = hashlib.sha256()
    with open(os.path.join(model, "model.bin"), "rb") as f:
        for blk in iter(lambda: f.read(1 << 24), b""):
            h.update(blk)
    assert h.hexdigest() == g["model_sha256"], "synthetic model generator changed"
    prompt = pkg.prompt_tokens(g["prompt_seed"], g["n_prompt"], g["vocab"])
    eng = pkg.Engine(model)
    try:
        toks, ke, na = eng.generate(prompt, g["k"], g["n_new"], g["temp"], g["topp"], g["sampler_seed"])
        want = np.array(g["tokens"], np.int32)
        n = min(len(toks), len(want))
        assert n >= g["n_new"]
        bad = np.nonzero(toks[:n] != want[:n])[0]
        assert len(bad) == 0, f"first divergence at token {bad[0]}: {toks[bad[0]]} vs {want[bad[0]]}"
        assert list(ke) == g["k_eff"] and list(na) == g["n_accept"]
        if g["temp"] > 0:
            assert eng.last_rng == g["rng"]
    finally:
        eng.close()
