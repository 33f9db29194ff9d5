"""model.bin versions 4-9 on the GPU (lz_open_bin's version ladder,
src/model.c:3925-4460, and its tensor reader, :3424-3812): grouped Q8_0
scales (groups of 32, 64, 128 instead of one per row: the epilogue takes the
reference's r == 1 and r > 1 forms, src/ops_epi.c:983-1022), binary16 and
row-base + u8 scale planes decoded at load, BF16 small tensors, and a
version-4 file without an MTP head.  Bit for bit against the CPU
restatement and the reference's recorded hashes (tests/golden/cap_*)."""
import hashlib
import json
import os

import numpy as np
import pytest

from oracle_lib import Oracle
from test_gpu_parity import diff_report, same_bits, start_both

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CAPTURES = sorted(f for f in os.listdir(GOLDEN) if f.startswith("cap_") and f.endswith(".json"))
MTP_CASES = [(13, 512), (14, 8192), (16, 512), (17, 512)]


def fmt_model(pkg, model_root, cid):
    return pkg.ensure_model(os.path.join(model_root, f"fmt{cid}"), cid, seed=1234)


@pytest.mark.parametrize("fname", CAPTURES)
def test_capture_matches_reference_hashes(pkg, model_root, fname):
    g = json.load(open(os.path.join(GOLDEN, fname)))
    print(f"[case] capture fixture {fname}", flush=True)
    model = pkg.ensure_model(os.path.join(model_root, g["model"]), g["config_id"], seed=g["model_seed"])
    prompt = pkg.prompt_tokens(g["prompt_seed"], g["n_prompt"], g["vocab"])
    eng = pkg.Engine(model)
    try:
        h = eng.batch_capture(prompt[:-1], 0)
        lg = eng.forward_capture(prompt[-1], len(prompt) - 1)
    finally:
        eng.close()
    assert hashlib.sha256(np.ascontiguousarray(h, np.float32).tobytes()).hexdigest() == g["sha256"]["hidden"]
    assert hashlib.sha256(np.ascontiguousarray(lg, np.float32).tobytes()).hexdigest() == g["sha256"]["capture"]


@pytest.mark.parametrize("cid,V", MTP_CASES)
def test_formats_verify_draft_rounds(pkg, model_root, cid, V):
    print(f"[case] format variant {cid}", flush=True)
    model = fmt_model(pkg, model_root, cid)
    prompt = pkg.prompt_tokens(2, 29, V)
    eng, ora = start_both(pkg, model, prompt)
    try:
        n = len(prompt)
        lg = eng.forward_capture(prompt[-1], n - 1)
        lo = ora.forward_capture(prompt[-1], n - 1)
        assert same_bits(lg, lo), "capture: " + diff_report(lg, lo)
        anchor = int(np.argmax(lg))
        dl = eng.draft_step(anchor, n - 1)
        do = ora.draft_step(anchor, n - 1)
        assert same_bits(dl, do), "draft: " + diff_report(dl, do)
        toks = np.array([anchor, 3, 7, V - 1], np.int32)
        v = eng.verify(toks, n)
        vo = ora.verify(toks, n)
        assert same_bits(v[0], vo[0]) and same_bits(v[1], vo[1]), "verify: " + diff_report(v[0], vo[0])
    finally:
        eng.close()
        ora.close()
    eng = pkg.Engine(model)
    try:
        toks, ke, na = eng.generate(prompt, 3, 32)
    finally:
        eng.close()
    to, keo, nao, _ = Oracle(model).generate(prompt, 3, 32)
    assert list(toks[:32]) == list(to[:32]) and list(na) == list(nao[:len(na)])


def test_version4_model_without_mtp_head(pkg, model_root):
    """A version-4 file carries no MTP head: the prefill and the capture run
    (against the oracle), and every entry point that needs the head refuses
    as the reference does (lz_forward_verify 1, lz_mtp_draft_step NULL,
    lz_spec_round -LZ_ERR_SPEC_NO_HEAD)."""
    import ctypes as C
    print("[case] version 4, no MTP head", flush=True)
    model = fmt_model(pkg, model_root, 15)
    prompt = pkg.prompt_tokens(4, 40, 8192)
    eng = pkg.Engine(model)
    ora = Oracle(model)
    try:
        h = eng.batch_capture(prompt[:-1], 0)
        ho = ora.batch_capture(prompt[:-1], 0)
        assert same_bits(h, ho), "prefill hidden: " + diff_report(h, ho)
        lg = eng.forward_capture(prompt[-1], len(prompt) - 1)
        lo = ora.forward_capture(prompt[-1], len(prompt) - 1)
        assert same_bits(lg, lo), "capture: " + diff_report(lg, lo)
        t = np.array([1, 2], np.int32)
        assert eng.lib.lz_forward_verify(C.byref(eng.m), C.byref(eng.s), t.ctypes.data_as(C.POINTER(C.c_int)), 2,
                                         len(prompt)) == 1
        assert not eng.lib.lz_mtp_draft_step(C.byref(eng.m), C.byref(eng.s), 1, len(prompt))
        r = eng.spec_round(int(np.argmax(lg)), len(prompt) - 1, 3)
        assert r[0] == -pkg.LZ_ERR["SPEC_NO_HEAD"]
    finally:
        eng.close()
        ora.close()
