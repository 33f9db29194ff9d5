"""Prefill through the wide path (512-row chunks: matrix-core projections,
grouped expert GEMMs, the KDA rows of a chunk in one launch) at long
contexts.

* A small model with configs[3]'s attention head size (128) and a 4608
  context: a 4200-token prompt's captured hidden rows, then a capture and
  a verify at position 4200, against the CPU restatement, bit for bit.
* configs[3] itself (d = 2048, 32 layers, 128 experts top-8): its
  4096-token prompt in 512-row chunks against the same prompt through the
  8-row chunked path (15-token calls), hidden rows and the next verify's
  logits bit for bit (the CPU restatement would take hours at this size;
  both paths are pinned against it on the shorter runs)."""
import ctypes as C
import os

import numpy as np
import pytest

from oracle_lib import Oracle
from test_gpu_parity import diff_report, same_bits
from test_gpu_shapes import SHAPES, shape_model

pytestmark = pytest.mark.gpu

SHAPES.setdefault("hd128_long", dict(n_heads=2, n_kv_heads=1, head_dim=128, seq_len=4608))


def test_long_prefill_matches_oracle(pkg, model_root):
    print("[case] prefill 4200 tokens, hd 128 model", flush=True)
    model = shape_model(pkg, model_root, "hd128_long")
    n = 4200
    prompt = pkg.prompt_tokens(5, n, 512)
    eng, ora = pkg.Engine(model), Oracle(model)
    try:
        eng.reset()
        h = eng.batch_capture(prompt[:-1], 0)
        ho = ora.batch_capture(prompt[:-1], 0)
        assert h is not None and ho is not None
        assert same_bits(h, ho), "prefill hidden rows: " + diff_report(h, ho)
        lg = eng.forward_capture(prompt[-1], n - 1)
        lo = ora.forward_capture(prompt[-1], n - 1)
        assert same_bits(lg, lo), "capture logits: " + diff_report(lg, lo)
        toks = np.array([int(np.argmax(lg)), 9, 77, 500], np.int32)
        v, vo = eng.verify(toks, n), ora.verify(toks, n)
        assert same_bits(v[0], vo[0]), "verify logits: " + diff_report(v[0], vo[0])
    finally:
        eng.close()
        ora.close()


def test_configs3_prompt_chunking_invariant(pkg, model_root):
    print("[case] configs[3] 4096-token prefill, wide chunks vs 8-row chunks", flush=True)
    model = pkg.ensure_model(os.path.join(model_root, "large"), 3, seed=1234)
    n = 4096
    prompt = pkg.prompt_tokens(0, n, 131072)
    eng = pkg.Engine(model)
    other = eng.add_session()
    try:
        eng.reset()
        h_wide = eng.batch_capture(prompt, 0)              # 8 chunks of 512 rows
        assert h_wide is not None
        lib, d = eng.lib, eng.d
        lib.lz_state_reset(C.byref(other), C.byref(eng.m))
        h_small = np.zeros((n, d), np.float32)
        for p0 in range(0, n, 15):                         # below the wide path's threshold
            t = np.ascontiguousarray(prompt[p0:p0 + 15], np.int32)
            out = h_small[p0:p0 + len(t)]
            buf = np.zeros((len(t), d), np.float32)
            assert lib.lz_forward_batch_capture(C.byref(eng.m), C.byref(other), t.ctypes.data_as(C.POINTER(C.c_int)),
                                                len(t), p0, buf.ctypes.data_as(C.POINTER(C.c_float)))
            out[:] = buf
        assert same_bits(h_wide, h_small), "hidden rows: " + diff_report(h_wide, h_small)
        toks = np.array([3, 1000, 77, 131071], np.int32)
        v_wide = eng.verify(toks, n)
        assert lib.lz_forward_verify(C.byref(eng.m), C.byref(other), toks.ctypes.data_as(C.POINTER(C.c_int)), 4, n) == 0
        lg = np.ctypeslib.as_array(other.mtp_logits, shape=(pkg.L98_SPEC_K_GPU + 1, eng.V))[:4]
        assert same_bits(v_wide[0], lg), "verify logits after the two prefills: " + diff_report(v_wide[0], lg)
    finally:
        eng.free_session(other)
        eng.close()


@pytest.mark.parametrize("n", [63, 64, 65, 97, 130, 600])
def test_split_prefill_matches_chunked(pkg, server, n):
    """A wide prefill chunk of 64 or more rows runs in three parts, each on
    its own stream (part p's layers wait for part p - 1's KDA recurrence and
    attention), when every part exceeds 8 rows; rows and the next verify's
    logits equal the 8-row chunked path bit for bit, at part sizes around the
    split's threshold and rounding, and over two wide chunks (600 rows)."""
    print(f"[case] split prefill n={n}", flush=True)
    prompt = pkg.prompt_tokens(9, n, 8192)
    eng = pkg.Engine(server)
    other = eng.add_session()
    try:
        eng.reset()
        h_wide = eng.batch_capture(prompt, 0)
        assert h_wide is not None
        lib, d = eng.lib, eng.d
        lib.lz_state_reset(C.byref(other), C.byref(eng.m))
        h_small = np.zeros((n, d), np.float32)
        for p0 in range(0, n, 15):                         # below the wide path's threshold
            t = np.ascontiguousarray(prompt[p0:p0 + 15], np.int32)
            buf = np.zeros((len(t), d), np.float32)
            assert lib.lz_forward_batch_capture(C.byref(eng.m), C.byref(other), t.ctypes.data_as(C.POINTER(C.c_int)),
                                                len(t), p0, buf.ctypes.data_as(C.POINTER(C.c_float)))
            h_small[p0:p0 + len(t)] = buf
        assert same_bits(h_wide, h_small), "hidden rows: " + diff_report(h_wide, h_small)
        toks = np.array([3, 1000, 77, 8191], np.int32)
        v_wide = eng.verify(toks, n)
        assert lib.lz_forward_verify(C.byref(eng.m), C.byref(other), toks.ctypes.data_as(C.POINTER(C.c_int)), 4, n) == 0
        lg = np.ctypeslib.as_array(other.mtp_logits, shape=(pkg.L98_SPEC_K_GPU + 1, eng.V))[:4]
        assert same_bits(v_wide[0], lg), "verify logits after the two prefills: " + diff_report(v_wide[0], lg)
    finally:
        eng.free_session(other)
        eng.close()
