"""The rest of the reference's export surface on the GPU library:
lz_read_weights, lz_forward, the exported counters the rounds update, and
the knobs (llama98.def:7-10, 102, 117-157)."""
import ctypes as C
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def echo(pkg, model_root):
    return pkg.ensure_model(os.path.join(model_root, "echo"), 11, seed=1234)


def test_read_weights_reports_open(pkg, echo):
    lib = pkg.hip_lib()
    err = C.create_string_buffer(128)
    closed = pkg.LZModel()
    assert lib.lz_read_weights(C.byref(closed), err, 128) == 1
    eng = pkg.Engine(echo)
    try:
        assert lib.lz_read_weights(C.byref(eng.m), err, 128) == 0
    finally:
        eng.close()


def test_forward_equals_capture_without_touching_the_chain(pkg, echo):
    prompt = pkg.prompt_tokens(4, 20, 64)
    a, b = pkg.Engine(echo), pkg.Engine(echo)
    try:
        for e in (a, b):
            e.reset()
            assert e.batch_capture(prompt[:-1], 0) is not None
        chain0 = a.chain()
        p = a.lib.lz_forward(C.byref(a.m), C.byref(a.s), int(prompt[-1]), len(prompt) - 1)
        assert p
        lg = np.ctypeslib.as_array(p, shape=(a.V,)).copy()
        want = b.forward_capture(int(prompt[-1]), len(prompt) - 1)
        assert np.array_equal(lg.view(np.uint32), want.view(np.uint32))
        assert np.array_equal(a.chain().view(np.uint32), chain0.view(np.uint32))
    finally:
        a.close()
        b.close()


def test_counters_follow_the_rounds(pkg, echo):
    """After a host-driven generation the reference's counters hold the
    rounds' rollbacks (n_accept < k_eff), catch-ups (n_accept > 1), captures
    and verify chunks; the timers moved."""
    g = json.load(open(os.path.join(GOLDEN, "gen_echo_k3_greedy.json")))
    prompt = pkg.prompt_tokens(g["prompt_seed"], g["n_prompt"], g["vocab"])
    names = ("lz_debug_n_ring_rollback", "lz_debug_n_catchup", "lz_debug_n_capture", "lz_debug_us_draft",
             "lz_debug_us_verify", "lz_debug_us_catchup")
    before = {n: pkg.hip_data(n).value for n in names}
    eng = pkg.Engine(echo)
    try:
        toks, ke, na = eng.generate_host(prompt, g["k"], g["n_new"])
    finally:
        eng.close()
    assert list(na) == g["n_accept"]
    d = {n: pkg.hip_data(n).value - before[n] for n in names}
    rounds = list(zip(g["k_eff"], g["n_accept"]))
    assert d["lz_debug_n_ring_rollback"] == sum(1 for k, n in rounds if 0 <= n < k)
    assert d["lz_debug_n_catchup"] == sum(1 for k, n in rounds if n > 1)
    # a capture opens the run and follows no round here (no discards)
    assert d["lz_debug_n_capture"] == 1
    assert d["lz_debug_us_draft"] > 0 and d["lz_debug_us_verify"] > 0 and d["lz_debug_us_catchup"] > 0


def test_knobs_outside_the_path_are_refused(pkg, echo):
    lib = pkg.hip_lib()
    assert pkg.hip_data("lz_kv_kfmt").value == 0 and pkg.hip_data("lz_attn_window").value == 0
    win = pkg.hip_data("lz_attn_window")
    win.value = 16
    try:
        m, s = pkg.LZModel(), pkg.LZRunState()
        err = C.create_string_buffer(256)
        assert lib.lz_open(C.byref(m), echo.encode(), err, 256) == 0
        try:
            assert lib.lz_state_alloc(C.byref(s), C.byref(m), 0, 3, err, 256) == 1
            assert b"window" in err.value
        finally:
            lib.lz_free(C.byref(m))
    finally:
        win.value = 0
    eng = pkg.Engine(echo)
    try:
        topk = pkg.hip_data("lz_moe_topk")
        topk.value = 1
        try:
            assert eng.forward_capture(3, 0) is None
        finally:
            topk.value = 0
        assert eng.forward_capture(3, 0) is not None
    finally:
        eng.close()
