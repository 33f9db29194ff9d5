"""SubLN models on the GPU (use_subn = 1: no pre-layer norms, each projection
normalizes the raw residual with its own weight; the KDA o_proj and MTP
down_proj inputs take the block-Hadamard quantization; the MTP FFN gate / up
inputs one int8 scale per row), bit for bit against the CPU restatement of
the reference (src/forward.c:1426-1542, src/forward_kda.c:559-612, 954-996,
1102-1240, src/forward_attn.c:787-822, 1015-1024, src/forward_moe.c:349-525,
src/forward_mtp.c:74-105).  subln is the survey's C1s variant (configs[0]
shapes, hadamard_o = 64, hadamard_down = 256); micro_subln its d = 64 twin
whose 32-wide projections take the one-group epilogue."""
import numpy as np
import pytest

from oracle_lib import Oracle
from test_gpu_parity import diff_report, same_bits, start_both

pytestmark = pytest.mark.gpu

CASES = [("micro_subln", 512), ("subln", 8192)]


@pytest.mark.parametrize("name,V", CASES)
def test_subln_capture_verify_draft(pkg, request, name, V):
    print(f"[case] subln capture/verify/draft {name}", flush=True)
    model = request.getfixturevalue(name)
    prompt = pkg.prompt_tokens(4, 37, V)
    eng, ora = start_both(pkg, model, prompt)
    try:
        n = len(prompt)
        lg = eng.forward_capture(prompt[-1], n - 1)
        lo = ora.forward_capture(prompt[-1], n - 1)
        assert same_bits(lg, lo), "capture logits: " + diff_report(lg, lo)
        assert same_bits(eng.chain(), ora.chain()), "chain: " + diff_report(eng.chain(), ora.chain())
        anchor = int(np.argmax(lg))
        for j in range(3):
            dl = eng.draft_step(anchor, n - 1 + j)
            do = ora.draft_step(anchor, n - 1 + j)
            assert same_bits(dl, do), f"draft {j} logits: " + diff_report(dl, do)
            assert same_bits(eng.chain(), ora.chain()), f"draft {j} chain: " + diff_report(eng.chain(), ora.chain())
            anchor = int(np.argmax(dl))
        toks = np.array([anchor, 5, 17, V - 3], np.int32)
        v = eng.verify(toks, n)
        vo = ora.verify(toks, n)
        assert same_bits(v[0], vo[0]), "verify logits: " + diff_report(v[0], vo[0])
        assert same_bits(v[1], vo[1]), "verify hidden: " + diff_report(v[1], vo[1])
        assert eng.s.ssm_slot == ora.info()["ssm_slot"]
    finally:
        eng.close()
        ora.close()


@pytest.mark.parametrize("name,V,n_prompt", [("micro_subln", 512, 40), ("subln", 8192, 150)])
def test_subln_long_prefill_takes_the_chunked_path(pkg, request, name, V, n_prompt):
    """A prefill long enough for the many-row path on other models; a SubLN
    model takes 8-row chunks and must still equal the restatement."""
    print(f"[case] subln prefill {name} n={n_prompt}", flush=True)
    model = request.getfixturevalue(name)
    prompt = pkg.prompt_tokens(8, n_prompt, V)
    eng, ora = start_both(pkg, model, prompt)
    try:
        lg = eng.forward_capture(prompt[-1], n_prompt - 1)
        lo = ora.forward_capture(prompt[-1], n_prompt - 1)
        assert same_bits(lg, lo), "capture logits: " + diff_report(lg, lo)
    finally:
        eng.close()
        ora.close()


@pytest.mark.parametrize("name,V,k", [("micro_subln", 512, 3), ("subln", 8192, 1), ("subln", 8192, 3)])
def test_subln_rounds_and_generate(pkg, request, name, V, k):
    print(f"[case] subln rounds {name} k={k}", flush=True)
    model = request.getfixturevalue(name)
    prompt = pkg.prompt_tokens(6, 32, V)
    eng, ora = start_both(pkg, model, prompt)
    try:
        n = len(prompt)
        lg = eng.forward_capture(prompt[-1], n - 1)
        ora.forward_capture(prompt[-1], n - 1)
        anchor, apos = int(np.argmax(lg)), n - 1
        for r in range(8):
            g = eng.spec_round(anchor, apos, k)
            o = ora.spec_round(anchor, apos, k)
            assert g[0] == o[0] and g[2:] == o[2:], (r, g, o)
            assert list(g[1][:g[0]]) == list(o[1][:o[0]]), (r, g, o)
            assert eng.s.ssm_slot == ora.info()["ssm_slot"] and eng.s.mtp_pos == ora.info()["mtp_pos"]
            anchor, apos = int(g[1][g[2]]), g[3]
        assert same_bits(eng.chain(), ora.chain()), "chain: " + diff_report(eng.chain(), ora.chain())
        # the device-resident loop (HIP graph rounds) against the oracle's generation
        toks, ke, na = eng.generate(prompt, k, 40)
        to, keo, nao, _ = Oracle(model).generate(prompt, k, 40)
        assert list(toks[:40]) == list(to[:40]) and list(na) == list(nao[:len(na)])
    finally:
        eng.close()
        ora.close()


def test_subln_temperature_generate(pkg, subln):
    print("[case] subln temperature k=2", flush=True)
    prompt = pkg.prompt_tokens(3, 48, 8192)
    eng = pkg.Engine(subln)
    try:
        toks, ke, na = eng.generate(prompt, 2, 40, temp=0.8, topp=0.95, seed=9)
    finally:
        eng.close()
    ora = Oracle(subln)
    to, keo, nao, _ = ora.generate(prompt, 2, 40, temp=0.8, topp=0.95, seed=9)
    ora.close()
    assert list(toks[:40]) == list(to[:40]) and list(na) == list(nao[:len(na)])


def test_subln_verify_batch(pkg, subln):
    """The session batch on a SubLN model (its rows take the per-session
    chunked forward) against single sessions."""
    import ctypes as C
    print("[case] subln verify batch, 5 sessions", flush=True)
    eng = pkg.Engine(subln)
    lens = [21, 40, 33, 57, 26]
    batch, single = [], []
    try:
        for i, n in enumerate(lens):
            prompt = pkg.prompt_tokens(300 + i, n, 8192)
            for group in (batch, single):
                st = eng.add_session()
                eng.session_start_on(st, prompt)
                group.append(st)
        toks = np.array([[(11 * i + 5 * j + 2) % 8192 for j in range(4)] for i in range(len(lens))], np.int32)
        pos0 = np.array(lens, np.int32)
        _, out = eng.verify_batch(batch, toks, pos0)
        V, d = eng.V, eng.d
        for i, st in enumerate(single):
            t = np.ascontiguousarray(toks[i])
            assert eng.lib.lz_forward_verify(C.byref(eng.m), C.byref(st), t.ctypes.data_as(C.POINTER(C.c_int)), 4,
                                             int(pos0[i])) == 0
            lg = np.ctypeslib.as_array(st.mtp_logits, shape=(pkg.L98_SPEC_K_GPU + 1, V))[:4]
            assert same_bits(out[i][0], lg), f"session {i}: " + diff_report(out[i][0], lg)
    finally:
        for st in batch + single:
            eng.free_session(st)
        eng.close()
