"""Session batches on the GPU (configs[4]'s server-style verify): several
independent sessions of one model advanced together, each on its own
stream.  Every session's results must equal what the same session gives
alone (the reference keeps one sequence per state, so n independent
reference runs are the specification), bit for bit against the CPU
restatement of the reference."""
import numpy as np
import pytest

from oracle_lib import Oracle
from test_gpu_parity import diff_report, same_bits

pytestmark = pytest.mark.gpu


def test_verify_batch_matches_single_sessions(pkg, server):
    print("[case] verify batch, server model, 6 sessions", flush=True)
    eng = pkg.Engine(server)
    lens = [17, 33, 48, 21, 60, 40]
    states, oras = [], []
    try:
        for i, n in enumerate(lens):
            st = eng.add_session()
            prompt = pkg.prompt_tokens(100 + i, n, 8192)
            eng.session_start_on(st, prompt)
            states.append(st)
            o = Oracle(server)
            o.session_start(prompt)             # prefill; l98_session_start also captures the last token
            o.forward_capture(prompt[-1], n - 1)
            oras.append(o)
        toks = np.array([[(7 * i + 3 * j + 1) % 8192 for j in range(4)] for i in range(len(lens))], np.int32)
        pos0 = np.array(lens, np.int32)
        _, out = eng.verify_batch(states, toks, pos0)
        for i, (lg, hd) in enumerate(out):
            ref = oras[i].verify(toks[i], lens[i])
            assert same_bits(lg, ref[0]), f"session {i} verify logits: " + diff_report(lg, ref[0])
            assert same_bits(hd, ref[1]), f"session {i} verify hidden: " + diff_report(hd, ref[1])
    finally:
        for st in states:
            eng.free_session(st)
        eng.close()


def test_greedy_rounds_batch_matches_single_sessions(pkg, server):
    print("[case] greedy rounds batch, server model, 5 sessions", flush=True)
    eng = pkg.Engine(server)
    lens = [24, 41, 30, 52, 19]
    k, n_rounds = 3, 12
    states, firsts = [], []
    try:
        for i, n in enumerate(lens):
            st = eng.add_session()
            prompt = pkg.prompt_tokens(200 + i, n, 8192)
            firsts.append(eng.session_start_on(st, prompt))
            states.append(st)
        _, toks = eng.greedy_rounds_batch(states, k, n_rounds)
        for i, n in enumerate(lens):
            prompt = pkg.prompt_tokens(200 + i, n, 8192)
            want = Oracle(server).generate(prompt, k, len(toks[i]) + 1)[0]
            got = np.concatenate([[firsts[i]], toks[i]])
            m = min(len(got), len(want))
            assert m >= n_rounds and np.array_equal(got[:m], want[:m]), (i, got[:m], want[:m])
    finally:
        for st in states:
            eng.free_session(st)
        eng.close()


def test_verify_batch_32_sessions_ragged_contexts(pkg, server):
    """configs[4]'s shape: 32 sessions with contexts uniform in [256, 2048],
    4 verify rows each, through the batch (one launch per kernel over all
    128 rows) against the same 32 sessions verified one by one, bit for
    bit; three of them also against the CPU restatement."""
    import ctypes as C
    print("[case] verify batch, 32 sessions, contexts 256-2048", flush=True)
    eng = pkg.Engine(server)
    rng = np.random.default_rng(0)
    ctx = rng.integers(256, 2049, size=32)
    batch, single = [], []
    try:
        for i, n in enumerate(ctx):
            prompt = pkg.prompt_tokens(1000 + i, int(n), 8192)
            for group in (batch, single):
                st = eng.add_session()
                eng.session_start_on(st, prompt)
                group.append(st)
        toks = np.array([[(13 * i + 7 * j + 5) % 8192 for j in range(4)] for i in range(32)], np.int32)
        pos0 = ctx.astype(np.int32)
        _, out = eng.verify_batch(batch, toks, pos0)
        V, d = eng.V, eng.d
        for i, st in enumerate(single):
            t = np.ascontiguousarray(toks[i])
            assert eng.lib.lz_forward_verify(C.byref(eng.m), C.byref(st), t.ctypes.data_as(C.POINTER(C.c_int)), 4,
                                             int(pos0[i])) == 0
            lg = np.ctypeslib.as_array(st.mtp_logits, shape=(pkg.L98_SPEC_K_GPU + 1, V))[:4]
            hd = np.ctypeslib.as_array(st.mtp_verify_hidden, shape=(pkg.L98_SPEC_K_GPU + 1, d))[:4]
            assert same_bits(out[i][0], lg), f"session {i} (ctx {ctx[i]}) logits: " + diff_report(out[i][0], lg)
            assert same_bits(out[i][1], hd), f"session {i} (ctx {ctx[i]}) hidden: " + diff_report(out[i][1], hd)
            assert batch[i].ssm_slot == st.ssm_slot
        for i in (0, int(np.argmax(ctx)), 17):
            o = Oracle(server)
            prompt = pkg.prompt_tokens(1000 + i, int(ctx[i]), 8192)
            o.session_start(prompt)
            o.forward_capture(prompt[-1], int(ctx[i]) - 1)
            ref = o.verify(toks[i], int(ctx[i]))
            assert same_bits(out[i][0], ref[0]) and same_bits(out[i][1], ref[1]), f"session {i} vs oracle"
            o.close()
    finally:
        for st in batch + single:
            eng.free_session(st)
        eng.close()


@pytest.fixture(scope="module")
def echo_model(pkg, model_root):
    import os
    return pkg.ensure_model(os.path.join(model_root, "echo"), 11, seed=1234)


@pytest.mark.parametrize("which", ["server", "echo"])
def test_batched_rounds_match_per_session_graphs(pkg, server, echo_model, which):
    """The batched rounds (each draft step one many-row pass over the
    sessions, one many-row verify, the acceptance and catch-up as one launch
    each) emit exactly what each session's own round graph emits; on the echo
    model, whose drafts are accepted, that covers the acceptance, the ring
    rollback and the catch-up.  The first session's tokens are also checked
    against the CPU restatement's generation."""
    model = server if which == "server" else echo_model
    print(f"[case] batched rounds vs per-session graphs, {which} model", flush=True)
    lens = [24, 41, 30, 52, 19, 33]
    k, n_rounds = 3, 10
    engs = [pkg.Engine(model), pkg.Engine(model)]
    V = engs[0].V
    assert engs[0].lib.l98_batched_rounds_ok(pkg.C.byref(engs[0].m), len(lens), k) == 1
    groups = [[], []]
    try:
        outs, firsts = [], []
        for g, eng in enumerate(engs):
            for i, n in enumerate(lens):
                st = eng.add_session()
                f = eng.session_start_on(st, pkg.prompt_tokens(300 + i, n, V))
                if g == 0:
                    firsts.append(f)
                groups[g].append(st)
            outs.append(eng.greedy_rounds_batch(groups[g], k, n_rounds, mode=g)[1])
        accepted = 0
        for i in range(len(lens)):
            assert np.array_equal(outs[0][i], outs[1][i]), (i, outs[0][i], outs[1][i])
            accepted += len(outs[0][i]) - n_rounds
        if which == "echo":
            assert accepted > 0
        prompt = pkg.prompt_tokens(300, lens[0], V)
        want = Oracle(model).generate(prompt, k, len(outs[0][0]) + 1)[0]
        got = np.concatenate([[firsts[0]], outs[0][0]])
        m = min(len(got), len(want))
        assert m > n_rounds and np.array_equal(got[:m], want[:m])
    finally:
        for g, eng in enumerate(engs):
            for st in groups[g]:
                eng.free_session(st)
            eng.close()
