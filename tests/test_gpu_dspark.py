"""DSpark heads (mtp_n_draft > 1) on the GPU: lz_mtp_draft_batch's k slots
as k rows of one pass (main_proj over [norm(h) | norm(emb or mask) | depth
row], the MTP block at position 0 with no history, the dense FFN, the exit
norm and the lm_head), and lz_spec_round_dspark's rounds, bit for bit
against the CPU restatement of the reference (src/forward_mtp.c:191-531,
src/generate.c:1000-1133).  ds_micro / ds_echo / ds_tiny / ds_subln are
synthetic configs 18-21 (micro, echo, tiny as a version-7 file with groups
of 64 and BF16 small tensors, micro-subln)."""
import ctypes as C

import numpy as np
import pytest

from oracle_lib import Oracle
from test_gpu_parity import diff_report, same_bits

pytestmark = pytest.mark.gpu

CASES = [("ds_micro", 512), ("ds_echo", 64), ("ds_tiny", 8192), ("ds_subln", 512)]


def start_both(pkg, model, prompt):
    """Body prefill on both (a DSpark session has no MTP prefill), then the
    capture forward of the last prompt token, which seeds the chain."""
    eng = pkg.Engine(model)
    ora = Oracle(model)
    n = len(prompt)
    h_gpu = eng.batch_capture(prompt[:-1], 0)
    h_ora = ora.batch_capture(prompt[:-1], 0)
    assert same_bits(h_gpu, h_ora), "batch capture hidden: " + diff_report(h_gpu, h_ora)
    lg = eng.forward_capture(prompt[-1], n - 1)
    lo = ora.forward_capture(prompt[-1], n - 1)
    assert same_bits(lg, lo), "capture logits: " + diff_report(lg, lo)
    return eng, ora, int(np.argmax(lo))


@pytest.mark.parametrize("name,V", CASES)
def test_draft_batch_bit_exact(pkg, request, name, V):
    print(f"[case] dspark draft batch {name}", flush=True)
    model = request.getfixturevalue(name)
    prompt = pkg.prompt_tokens(6, 33, V)
    eng, ora, anchor = start_both(pkg, model, prompt)
    try:
        nd = ora.n_draft
        assert eng.m.config.mtp_n_draft == nd and eng.m.config.mtp_markov_rank == 0
        chain = eng.chain()
        for k in sorted({1, 2, nd}):
            got = eng.draft_batch(anchor, k)
            want = ora.draft_batch(anchor, k)
            assert got is not None and want is not None
            assert same_bits(got, want), f"k={k} slot logits: " + diff_report(got, want)
            assert same_bits(eng.chain(), chain), "the draft batch changed the chain"
    finally:
        eng.close()
        ora.close()


@pytest.mark.parametrize("name,V,k", [("ds_micro", 512, 4), ("ds_echo", 64, 6), ("ds_echo", 64, 3),
                                      ("ds_tiny", 8192, 3), ("ds_subln", 512, 3)])
def test_dspark_rounds_bit_exact(pkg, request, name, V, k):
    """lz_spec_round_dspark round after round against the restatement: the
    emitted tokens, acceptance, ring slot, the verify logits and hidden rows
    and every slot's draft logits it leaves in the state, and mtp_pos kept."""
    print(f"[case] dspark rounds {name} k={k}", flush=True)
    model = request.getfixturevalue(name)
    prompt = pkg.prompt_tokens(12, 30, V)
    eng, ora, anchor = start_both(pkg, model, prompt)
    try:
        anchor_pos = len(prompt) - 1
        seen = set()
        for r in range(10):
            rg, og, nag, npg, keg = eng.spec_round(anchor, anchor_pos, k)
            ro, oo, nao, npo, keo = ora.spec_round_dspark(anchor, anchor_pos, k)
            assert (rg, nag, npg, keg) == (ro, nao, npo, keo), (r, rg, ro)
            assert np.array_equal(og[:nag + 1], oo[:nao + 1]), r
            lg = np.ctypeslib.as_array(eng.s.mtp_logits, shape=(keg + 1, V))
            lo = np.ctypeslib.as_array(pkg_ora_logits(ora), shape=(8, V))[:keo + 1]
            assert same_bits(lg, lo), f"round {r} verify logits: " + diff_report(lg, lo)
            hg = np.ctypeslib.as_array(eng.s.mtp_verify_hidden, shape=(keg + 1, eng.d))
            ho = np.ctypeslib.as_array(pkg_ora_hidden(ora), shape=(8, eng.d))[:keo + 1]
            assert same_bits(hg, ho), f"round {r} verify hidden: " + diff_report(hg, ho)
            dg = np.ctypeslib.as_array(eng.s.mtp_kdraft_logits, shape=(k, V))
            assert same_bits(dg, ora.kdraft_logits(k)), f"round {r} slot logits"
            assert same_bits(eng.chain(), ora.chain()), f"round {r} chain"
            assert eng.s.ssm_slot == ora.info()["ssm_slot"] and eng.s.mtp_pos == 0 == ora.info()["mtp_pos"]
            seen.add(nag)
            anchor, anchor_pos = int(og[nag]), npg
        if name == "ds_echo":
            assert len(seen) >= 2, seen
    finally:
        eng.close()
        ora.close()


def pkg_ora_logits(ora):
    import oracle_lib as OL
    return OL.lib().ora_mtp_logits(ora.s)


def pkg_ora_hidden(ora):
    import oracle_lib as OL
    return OL.lib().ora_mtp_hidden(ora.s)


def test_dspark_device_rounds_match_host_rounds(pkg, ds_echo):
    """l98_greedy_rounds (one HIP graph per round, every scalar on the device)
    equals the same rounds through lz_spec_round_dspark from the host."""
    print("[case] dspark device rounds vs host rounds", flush=True)
    prompt = pkg.prompt_tokens(11, 24, 64)
    a = pkg.Engine(ds_echo)
    try:
        first = a.session_start(prompt)
        toks, na, _ = a.greedy_rounds(4, 20, use_graph=True)
        slot, pos = a.s.ssm_slot, a.s.mtp_pos
    finally:
        a.close()
    b = pkg.Engine(ds_echo)
    try:
        want, ke, nb = b.generate_host(prompt, 4, 1 + len(toks))
    finally:
        b.close()
    got = np.concatenate([[first], toks]).astype(np.int32)
    n = min(len(got), len(want))
    assert np.array_equal(got[:n], want[:n]) and list(na) == list(nb[:len(na)])
    assert pos == 0 and max(na) >= 1


def test_dspark_refusals(pkg, ds_micro, micro):
    """The one-slot entry points refuse a DSpark head (it binds no fc), the
    DSpark rounds refuse a one-slot head, and k is bounded by mtp_n_draft."""
    print("[case] dspark refusals", flush=True)
    eng = pkg.Engine(ds_micro)
    try:
        prompt = pkg.prompt_tokens(3, 20, 512)
        eng.session_start(prompt)
        L = eng.lib
        err = C.create_string_buffer(256)
        out = np.zeros(8, np.int32)
        a, b, c_ = C.c_int(), C.c_int(), C.c_int()
        assert not L.lz_mtp_draft_step(C.byref(eng.m), C.byref(eng.s), 5, 20)
        r = L.lz_spec_round(C.byref(eng.m), C.byref(eng.s), 5, 19, 2, 0.0, 0, None, 0, 0,
                            out.ctypes.data_as(C.POINTER(C.c_int)), C.byref(a), C.byref(b), C.byref(c_), err, 256)
        assert r < 0 and b"DSpark" in err.value
        nd = eng.m.config.mtp_n_draft
        r = L.lz_spec_round_dspark(C.byref(eng.m), C.byref(eng.s), 5, 19, nd + 1, 0.0, 0, None, 0,
                                   out.ctypes.data_as(C.POINTER(C.c_int)), C.byref(a), C.byref(b), C.byref(c_),
                                   err, 256)
        assert r == -25                                   # LZ_ERR_SPEC_K_RANGE
        assert eng.draft_batch(5, nd + 1) is None
        # the Markov correction of a model.bin head adds zeros: values kept,
        # -0 becomes +0
        row = np.array([1.5, -0.0, 0.0, -3.25] * 128, np.float32)
        before = row.copy()
        L.lz_mtp_markov_correct(C.byref(eng.m), C.byref(eng.s), 7, row.ctypes.data_as(C.POINTER(C.c_float)))
        assert np.array_equal(row, before) and not np.signbit(row[1])
    finally:
        eng.close()
    one = pkg.Engine(micro)
    try:
        err = C.create_string_buffer(256)
        out = np.zeros(8, np.int32)
        a, b, c_ = C.c_int(), C.c_int(), C.c_int()
        r = one.lib.lz_spec_round_dspark(C.byref(one.m), C.byref(one.s), 5, 19, 2, 0.0, 0, None, 0,
                                         out.ctypes.data_as(C.POINTER(C.c_int)), C.byref(a), C.byref(b),
                                         C.byref(c_), err, 256)
        assert r < 0
        assert one.draft_batch(5, 2) is None
    finally:
        one.close()
