"""The two attention paths of a session's chunk against the CPU
restatement: one launch per (q head, token) (path 1), and the scores by
64-position slice followed by the softmax and value chains per (q head,
token, 32-wide output group) (path 2: the exact wave sum over 2047-value
segments, the segment sums carried).  Contexts below, at and past one
segment (700, 2046-2049, 2200 positions on the 2304-position server model,
head_dim 128) and the micro / head_dim-128 shape models (head_dim 64 and
128): capture logits and MTP chain, verify logits and hidden rows, a draft
step and greedy generations, bit for bit."""
import numpy as np
import pytest

from oracle_lib import Oracle
from test_gpu_parity import diff_report, same_bits, start_both
from test_gpu_shapes import shape_model

pytestmark = pytest.mark.gpu


@pytest.fixture
def attn_path(pkg):
    yield lambda mode: pkg.set_attn_path(mode)
    pkg.set_attn_path(0)


@pytest.mark.parametrize("path", [1, 2])
@pytest.mark.parametrize("n_prompt", [700, 2047, 2049, 2200])
def test_long_capture_both_paths(pkg, server, attn_path, path, n_prompt):
    print(f"[case] attention path {path} capture server n_prompt={n_prompt}", flush=True)
    attn_path(path)
    prompt = pkg.prompt_tokens(5, n_prompt, 8192)
    eng, ora = start_both(pkg, server, prompt)
    n = len(prompt)
    lg = eng.forward_capture(prompt[-1], n - 1)
    lo = ora.forward_capture(prompt[-1], n - 1)
    assert same_bits(lg, lo), "capture logits: " + diff_report(lg, lo)
    assert same_bits(eng.chain(), ora.chain()), "mtp_chain: " + diff_report(eng.chain(), ora.chain())
    toks = np.array([int(np.argmax(lg)), 7, 300, 41], np.int32)
    v = eng.verify(toks, n)
    vo = ora.verify(toks, n)
    assert v is not None and vo is not None
    assert same_bits(v[0], vo[0]), "verify logits: " + diff_report(v[0], vo[0])
    assert same_bits(v[1], vo[1]), "verify hidden: " + diff_report(v[1], vo[1])
    eng.close()


@pytest.mark.parametrize("path", [1, 2])
@pytest.mark.parametrize("name", ["micro", "hd128"])
def test_short_models_both_paths(pkg, model_root, micro, attn_path, path, name):
    print(f"[case] attention path {path} model {name}", flush=True)
    attn_path(path)
    model = micro if name == "micro" else shape_model(pkg, model_root, name)
    prompt = pkg.prompt_tokens(3, 21, 512)
    eng, ora = start_both(pkg, model, prompt)
    n = len(prompt)
    lg = eng.forward_capture(prompt[-1], n - 1)
    lo = ora.forward_capture(prompt[-1], n - 1)
    assert same_bits(lg, lo), "capture logits: " + diff_report(lg, lo)
    toks = np.array([int(np.argmax(lg)), 7, 300, 41], np.int32)
    v = eng.verify(toks, n)
    vo = ora.verify(toks, n)
    assert same_bits(v[0], vo[0]), "verify logits: " + diff_report(v[0], vo[0])
    d = eng.draft_step(int(toks[0]), n)
    do = ora.draft_step(int(toks[0]), n)
    assert same_bits(d, do), "draft logits: " + diff_report(d, do)
    eng.close()
    e2, o2 = pkg.Engine(model), Oracle(model)
    t_gpu, _, _ = e2.generate(prompt, 3, 24)
    r = o2.generate(prompt, 3, 24)
    t_ora = r[0] if isinstance(r, tuple) else r["tokens"]
    m = min(len(t_gpu), len(t_ora))
    assert m >= 24 and np.array_equal(np.asarray(t_gpu[:m]), np.asarray(t_ora[:m])), (t_gpu[:m], t_ora[:m])
    e2.close()


def test_graph_rounds_both_paths(pkg, server, attn_path):
    """Device graph rounds on the server model from a 2040-token prompt, so
    the rounds cross the first segment's end: the same tokens on both
    paths."""
    print("[case] attention paths: graph rounds across 2047 positions", flush=True)
    prompt = pkg.prompt_tokens(11, 2040, 8192)
    out = {}
    for path in (1, 2):
        attn_path(path)
        eng = pkg.Engine(server)
        eng.session_start(prompt)
        toks, _ = eng.greedy_rounds(3, 12)[:2]
        out[path] = np.asarray(toks)
        eng.close()
    assert np.array_equal(out[1], out[2]), (out[1], out[2])
