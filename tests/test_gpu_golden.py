"""GPU generations against the reference engine's recorded outputs
(tests/golden/, written by tests/golden/make_golden.py from the reference
build): micro, configs[0] (tiny), configs[1] (base, the benchmark model),
configs[3]'s and configs[4]'s models, and the echo model whose greedy drafts
are accepted at every depth.  Needs no reference and no oracle at run time.

Three drivers of the same rounds:
  * l98_generate: device-resident rounds, one HIP graph launch each;
  * l98_session_start + l98_greedy_rounds(use_graph=0): the same rounds
    enqueued kernel by kernel;
  * the reference's own loop over lz_forward_capture / lz_spec_round from the
    host (the only driver that takes p_min, n_min, debug_break_rollback and
    debug_skip_catchup, as the reference harness passes them)."""
import hashlib
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(f for f in os.listdir(GOLDEN) if f.startswith("gen_") and f.endswith(".json"))


def load(pkg, model_root, fname):
    g = json.load(open(os.path.join(GOLDEN, fname)))
    model = pkg.ensure_model(os.path.join(model_root, g["model"]), g["config_id"], seed=g["model_seed"])
    h = hashlib.sha256()
    with open(os.path.join(model, "model.bin"), "rb") as f:
        for blk in iter(lambda: f.read(1 << 24), b""):
            h.update(blk)
    assert h.hexdigest() == g["model_sha256"], "synthetic model generator changed"
    prompt = pkg.prompt_tokens(g["prompt_seed"], g["n_prompt"], g["vocab"])
    return g, model, prompt


def has_options(g):
    return g.get("p_min", 0) > 0 or g.get("n_min", 0) > 0 or g.get("brk", 0) or g.get("skipc", 0)


def check_tokens(toks, g):
    want = np.array(g["tokens"], np.int32)
    n = min(len(toks), len(want))
    assert n >= g["n_new"]
    bad = np.nonzero(np.asarray(toks[:n]) != want[:n])[0]
    assert len(bad) == 0, f"first divergence at token {bad[0]}: {toks[bad[0]]} vs {want[bad[0]]}"


@pytest.mark.parametrize("fname", FIXTURES)
def test_generation_matches_reference_fixture(pkg, model_root, fname):
    g, model, prompt = load(pkg, model_root, fname)
    print(f"[case] golden {fname}", flush=True)
    eng = pkg.Engine(model)
    try:
        if has_options(g):
            toks, ke, na = eng.generate_host(prompt, g["k"], g["n_new"], g["p_min"], g["n_min"], g["brk"],
                                             g["skipc"])
        else:
            toks, ke, na = eng.generate(prompt, g["k"], g["n_new"], g["temp"], g["topp"], g["sampler_seed"])
        check_tokens(toks, g)
        assert list(ke) == g["k_eff"] and list(na) == g["n_accept"]
        if g["temp"] > 0:
            assert eng.last_rng == g["rng"]
        assert eng.s.mtp_pos == g["mtp_pos"] and eng.s.ssm_slot == g["ssm_slot"]
    finally:
        eng.close()


GREEDY_PLAIN = [f for f in FIXTURES
                if f.startswith(("gen_echo", "gen_micro", "gen_tiny")) and f.endswith("_greedy.json")]


@pytest.mark.parametrize("fname", GREEDY_PLAIN)
def test_host_driven_rounds_match_fixture(pkg, model_root, fname):
    """Each round through lz_spec_round from the host (ctl in, ctl out)."""
    g, model, prompt = load(pkg, model_root, fname)
    print(f"[case] host rounds {fname}", flush=True)
    eng = pkg.Engine(model)
    try:
        toks, ke, na = eng.generate_host(prompt, g["k"], g["n_new"])
        check_tokens(toks, g)
        assert list(ke) == g["k_eff"] and list(na) == g["n_accept"]
        assert eng.s.mtp_pos == g["mtp_pos"] and eng.s.ssm_slot == g["ssm_slot"]
    finally:
        eng.close()


@pytest.mark.parametrize("fname", [f for f in GREEDY_PLAIN if f.startswith("gen_echo")])
def test_device_rounds_without_graph_match_fixture(pkg, model_root, fname):
    """l98_greedy_rounds with use_graph = 0: the round's kernels enqueued one
    by one, every scalar in the device control block."""
    g, model, prompt = load(pkg, model_root, fname)
    print(f"[case] device rounds, no graph {fname}", flush=True)
    eng = pkg.Engine(model)
    try:
        first = eng.session_start(prompt)
        rounds = len(g["n_accept"])
        try:
            toks, na, _ = eng.greedy_rounds(g["k"], rounds, use_graph=False)
        except RuntimeError:
            # the batch is refused up front (nothing ran) when rounds that all
            # accept every draft could pass the state's end; run them singly
            parts = [eng.greedy_rounds(g["k"], 1, use_graph=False) for _ in range(rounds)]
            toks = np.concatenate([p[0] for p in parts])
            na = np.concatenate([p[1] for p in parts])
        check_tokens(np.concatenate([[first], toks]).astype(np.int32), g)
        assert list(na) == g["n_accept"]
        assert eng.s.mtp_pos == g["mtp_pos"] and eng.s.ssm_slot == g["ssm_slot"]
    finally:
        eng.close()


def test_accept_paths_are_covered():
    """The fixtures above take every acceptance depth 0..k of a greedy round
    (k = 1, 3, 6), draft lengths cut by p_min, discards by n_min, and a
    temperature run that accepts drafts."""
    def g(name):
        return json.load(open(os.path.join(GOLDEN, name)))
    for k in (1, 3, 6):
        assert set(g(f"gen_echo_k{k}_greedy.json")["n_accept"]) == set(range(k + 1)), k
    assert set(g("gen_echo_k3_pmin.json")["k_eff"]) == {0, 1, 2, 3}
    assert -1 in g("gen_echo_k3_pmin_nmin.json")["n_accept"]
    assert max(g("gen_echo_k3_temp.json")["n_accept"]) == 3


ROUND_FIXTURES = [f for f in FIXTURES if "round_sha256" in json.load(open(os.path.join(GOLDEN, f)))]


@pytest.mark.parametrize("fname", ROUND_FIXTURES)
def test_round_values_match_reference_fixture(pkg, model_root, fname):
    """Bit for bit on the values, not only the tokens: the capture logits and,
    round after round, the verify logits, verify hidden rows and last draft
    logits that lz_spec_round leaves in the state hash to what the reference
    engine left in its own state (its harness's --dump-rounds files)."""
    import hashlib
    g, model, prompt = load(pkg, model_root, fname)
    print(f"[case] golden rounds {fname}", flush=True)
    want = g["round_sha256"]
    got = {}

    def keep(tag, a):
        if tag in want:
            got[tag] = hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()

    eng = pkg.Engine(model)
    try:
        eng.generate_host(prompt, g["k"], g["n_new"], on_round=keep)
    finally:
        eng.close()
    assert set(got) == set(want), sorted(set(want) - set(got))
    bad = [t for t in want if got[t] != want[t]]
    assert not bad, f"values differ from the reference at {bad}"
