"""GPU parity: the HIP path (through the C ABI) against the CPU restatement
of the reference, bit for bit, on seeded random-init models.

Each case prints its name before touching the GPU."""
import numpy as np
import pytest

from oracle_lib import Oracle

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def diff_report(a, b):
    a = np.asarray(a, np.float32).ravel()
    b = np.asarray(b, np.float32).ravel()
    bad = np.nonzero(a.view(np.uint32) != b.view(np.uint32))[0]
    if len(bad) == 0:
        return "equal"
    rel = np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)
    return f"{len(bad)}/{len(a)} differ, first at {bad[0]} ({a[bad[0]]} vs {b[bad[0]]}), max rel {rel:.3e}"


def start_both(pkg, model, prompt):
    eng = pkg.Engine(model)
    ora = Oracle(model)
    n = len(prompt)
    h_gpu = eng.batch_capture(prompt[:-1], 0)
    h_ora = ora.batch_capture(prompt[:-1], 0)
    assert h_gpu is not None and h_ora is not None
    assert same_bits(h_gpu, h_ora), "batch capture hidden: " + diff_report(h_gpu, h_ora)
    assert eng.mtp_prefill(h_gpu, prompt[1:], 0) == 0
    assert ora.mtp_prefill(h_ora, prompt[1:], 0) == 0
    eng.s.mtp_pos = n - 1          # the caller sets mtp_pos after the prefill (src/generate.c:2946)
    ora.set_mtp_pos(n - 1)
    return eng, ora


# server (seq_len 2304) contexts reach the softmax denominator's three
# exact-sum widths (up to 1024 and 2048 positions) and the serial loop past
# 2048
@pytest.mark.parametrize("name,n_prompt", [("micro", 20), ("tiny", 40), ("server", 700), ("server", 1500),
                                           ("server", 2200)])
def test_capture_and_prefill_bit_exact(pkg, request, name, n_prompt):
    print(f"[case] capture {name} n_prompt={n_prompt}", flush=True)
    model = request.getfixturevalue(name)
    V = 512 if name == "micro" else 8192
    prompt = pkg.prompt_tokens(0, n_prompt, V)
    eng, ora = start_both(pkg, model, prompt)
    lg = eng.forward_capture(prompt[-1], len(prompt) - 1)
    lo = ora.forward_capture(prompt[-1], len(prompt) - 1)
    assert same_bits(lg, lo), "capture logits: " + diff_report(lg, lo)
    assert same_bits(eng.chain(), ora.chain()), "mtp_chain: " + diff_report(eng.chain(), ora.chain())
    eng.close()


def test_verify_and_draft_bit_exact(pkg, tiny):
    print("[case] verify/draft tiny", flush=True)
    prompt = pkg.prompt_tokens(0, 40, 8192)
    eng, ora = start_both(pkg, tiny, prompt)
    n = len(prompt)
    lg = eng.forward_capture(prompt[-1], n - 1)
    ora.forward_capture(prompt[-1], n - 1)
    anchor = int(np.argmax(lg))
    # one draft step at mtp_pos = n-1
    dl = eng.draft_step(anchor, n - 1)
    do = ora.draft_step(anchor, n - 1)
    assert same_bits(dl, do), "draft logits: " + diff_report(dl, do)
    assert same_bits(eng.chain(), ora.chain()), "chain: " + diff_report(eng.chain(), ora.chain())
    toks = np.array([anchor, 5, 17, 4000], np.int32)
    v = eng.verify(toks, n)
    vo = ora.verify(toks, n)
    assert same_bits(v[0], vo[0]), "verify logits: " + diff_report(v[0], vo[0])
    assert same_bits(v[1], vo[1]), "verify hidden: " + diff_report(v[1], vo[1])
    assert eng.s.ssm_slot == ora.info()["ssm_slot"]
    eng.close()


# k = 4 and 5 run the 5- and 6-row instances of the verify's kernels
@pytest.mark.parametrize("k", [1, 3, 4, 5])
def test_spec_rounds_match(pkg, tiny, k):
    print(f"[case] spec rounds tiny k={k}", flush=True)
    prompt = pkg.prompt_tokens(0, 40, 8192)
    eng, ora = start_both(pkg, tiny, prompt)
    n = len(prompt)
    lg = eng.forward_capture(prompt[-1], n - 1)
    ora.forward_capture(prompt[-1], n - 1)
    anchor, apos = int(np.argmax(lg)), n - 1
    for r in range(12):
        g = eng.spec_round(anchor, apos, k)
        o = ora.spec_round(anchor, apos, k)
        assert g[0] == o[0] and g[2:] == o[2:], (r, g, o)
        assert list(g[1][:g[0]]) == list(o[1][:o[0]]), (r, g, o)
        assert eng.s.ssm_slot == ora.info()["ssm_slot"] and eng.s.mtp_pos == ora.info()["mtp_pos"]
        anchor, apos = int(g[1][g[2]]), g[3]
    assert same_bits(eng.chain(), ora.chain()), "chain: " + diff_report(eng.chain(), ora.chain())
    eng.close()


@pytest.mark.parametrize("name,k,n_new", [("micro", 3, 40), ("tiny", 1, 48), ("tiny", 3, 64)])
def test_generate_greedy_identical(pkg, request, name, k, n_new):
    print(f"[case] generate greedy {name} k={k}", flush=True)
    model = request.getfixturevalue(name)
    V = 512 if name == "micro" else 8192
    prompt = pkg.prompt_tokens(0, 32, V)
    eng = pkg.Engine(model)
    toks, ke, na = eng.generate(prompt, k, n_new)
    ora = Oracle(model)
    to, keo, nao, _ = ora.generate(prompt, k, n_new)
    m = min(len(toks), len(to))
    assert m >= n_new
    assert list(toks[:n_new]) == list(to[:n_new])
    assert list(na) == list(nao[:len(na)])
    eng.close()


def test_generate_temperature_identical(pkg, tiny):
    print("[case] generate temperature tiny", flush=True)
    prompt = pkg.prompt_tokens(0, 32, 8192)
    eng = pkg.Engine(tiny)
    toks, ke, na = eng.generate(prompt, 3, 40, temp=0.8, topp=0.95, seed=7)
    ora = Oracle(tiny)
    to, keo, nao, _ = ora.generate(prompt, 3, 40, temp=0.8, topp=0.95, seed=7)
    assert list(toks[:40]) == list(to[:40])
    eng.close()
