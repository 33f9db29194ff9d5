"""Python bindings of the MI355X MTP speculative-decoding library.

The product is the C ABI of ``include/llama98_hip.h`` (``lib/libl98hip.so``,
hand-written gfx950 kernels behind the reference's ``lz_*`` entry points).
This module is a thin ctypes layer over it for tests and ``bench.py``, plus
the seeded synthetic-model writer (``lib/libl98synth.so``) and the prompt
generator the benchmark configs use.

The package directory is named ``llama98-zh_amd``; import it with
``load_package()`` from ``__graft_entry__`` or by path.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
HIP_LIB = os.path.join(LIB_DIR, "libl98hip.so")
SYNTH_LIB = os.path.join(LIB_DIR, "libl98synth.so")

LZ_SPEC_K_MAX = 6
L98_NOALLOC_MAX_VOCAB = 262144   # l98_spec_accept_temp_noalloc's static staging
L98_SPEC_K_GPU = 7      # the library's own loops take k up to 7 (verify M = 8)
LZ_BATCH_MAX = 8
LZ_ERR = {"NULL_ARG": 6, "STATE_ALLOC": 7, "FORWARD": 20, "SPEC_NO_HEAD": 24, "SPEC_K_RANGE": 25}


class LZModelConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "vocab_size", "hidden_size", "n_layers", "seq_len",
        "n_heads", "n_kv_heads", "head_dim", "rotary_dim",
        "lin_n_k_heads", "lin_n_v_heads", "lin_k_head_dim", "lin_v_head_dim", "conv_kernel",
        "n_linear_layers", "n_full_layers",
        "attn_q_dim", "attn_qgate_dim", "attn_kv_dim", "lin_key_dim", "lin_value_dim", "lin_conv_dim",
        "kda_gate_rank", "num_experts", "num_experts_per_token", "moe_latent_dim",
        "moe_intermediate_size", "moe_shared_width", "mtp_intermediate_size", "mtp_n_layers")] + [
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float), ("layer_types", C.c_int * 128),
        ("use_subn", C.c_int), ("hadamard_o", C.c_int), ("hadamard_down", C.c_int),
        ("mtp_n_draft", C.c_int), ("mtp_markov_rank", C.c_int),
        ("kda_has_gate_lower_bound", C.c_int), ("kda_gate_lower_bound", C.c_float)]


class LZModel(C.Structure):
    _fields_ = [("config", LZModelConfig), ("bytes_device", C.c_longlong), ("impl", C.c_void_p)]


class LZRunState(C.Structure):
    _fields_ = [("seq_len", C.c_int), ("ssm_slot", C.c_int), ("ssm_ring_depth", C.c_int),
                ("mtp_pos", C.c_int), ("nt_cap", C.c_int),
                ("logits", C.POINTER(C.c_float)), ("mtp_logits", C.POINTER(C.c_float)),
                ("mtp_verify_hidden", C.POINTER(C.c_float)), ("mtp_chain", C.POINTER(C.c_float)),
                ("mtp_draft_logits", C.POINTER(C.c_float)), ("mtp_kdraft_logits", C.POINTER(C.c_float)),
                ("bytes_device", C.c_longlong), ("impl", C.c_void_p)]


class LZSampleParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("temp_think", C.c_float), ("think_temp_enabled", C.c_int),
                ("topp", C.c_float), ("minp", C.c_float), ("topk", C.c_int),
                ("presence_penalty", C.c_float), ("frequency_penalty", C.c_float),
                ("repetition_penalty", C.c_float), ("repeat_last_n", C.c_int), ("minp_llamacpp", C.c_int)]


class LZSampler(C.Structure):
    _fields_ = [("vocab_size", C.c_int), ("p", LZSampleParams), ("rng_state", C.c_uint64)]


class L98SynthConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "vocab", "hidden", "n_layers", "seq_len", "attn_period", "n_heads", "n_kv_heads", "head_dim",
        "kda_heads", "kd", "vd", "conv_kernel", "gate_rank", "n_experts", "topk", "latent",
        "moe_inter", "shared_w", "mtp_inter")] + [
        ("w_std", C.c_float), ("router_std", C.c_float), ("bias_std", C.c_float), ("gate_lb", C.c_float),
        ("resid_std", C.c_float),
        ("mtp_echo", C.c_int), ("use_subn", C.c_int), ("hadamard_o", C.c_int), ("hadamard_down", C.c_int),
        ("bin_version", C.c_int), ("gs", C.c_int), ("scale_layout", C.c_int), ("bf16_small", C.c_int),
        ("mtp_n_draft", C.c_int)]


_P = C.c_void_p
_IP = C.POINTER(C.c_int)
_FP = C.POINTER(C.c_float)

# (name, restype, argtypes) of every entry point include/llama98_hip.h declares.
HIP_API = [
    ("lz_load_config", C.c_int, [C.POINTER(LZModelConfig), C.c_char_p, C.c_char_p, C.c_int]),
    ("lz_open", C.c_int, [C.POINTER(LZModel), C.c_char_p, C.c_char_p, C.c_int]),
    ("lz_read_weights", C.c_int, [C.POINTER(LZModel), C.c_char_p, C.c_int]),
    ("lz_forward", _FP, [C.POINTER(LZModel), C.POINTER(LZRunState), C.c_int, C.c_int]),
    ("lz_free", None, [C.POINTER(LZModel)]),
    ("lz_state_alloc", C.c_int, [C.POINTER(LZRunState), C.POINTER(LZModel), C.c_int, C.c_int, C.c_char_p, C.c_int]),
    ("lz_state_free", None, [C.POINTER(LZRunState)]),
    ("lz_state_reset", None, [C.POINTER(LZRunState), C.POINTER(LZModel)]),
    ("lz_forward_capture", _FP, [C.POINTER(LZModel), C.POINTER(LZRunState), C.c_int, C.c_int]),
    ("lz_forward_batch_capture", _FP, [C.POINTER(LZModel), C.POINTER(LZRunState), _IP, C.c_int, C.c_int, _FP]),
    ("lz_forward_verify", C.c_int, [C.POINTER(LZModel), C.POINTER(LZRunState), _IP, C.c_int, C.c_int]),
    ("lz_mtp_draft_step", _FP, [C.POINTER(LZModel), C.POINTER(LZRunState), C.c_int, C.c_int]),
    ("lz_mtp_prefill", C.c_int, [C.POINTER(LZModel), C.POINTER(LZRunState), _FP, _IP, C.c_int, C.c_int]),
    ("lz_mtp_draft_batch", _FP, [C.POINTER(LZModel), C.POINTER(LZRunState), C.c_int, C.c_int]),
    ("lz_mtp_markov_correct", None, [C.POINTER(LZModel), C.POINTER(LZRunState), C.c_int, _FP]),
    ("lz_mtp_catchup", C.c_int, [C.POINTER(LZModel), C.POINTER(LZRunState), _FP, _IP, C.c_int, C.c_int]),
    ("lz_spec_accept", C.c_int, [_IP, _IP, C.c_int, C.c_int, _IP]),
    ("lz_spec_accept_temp", C.c_int, [_FP, _FP, C.c_int, C.c_int, C.c_float, C.POINTER(C.c_uint64), _IP]),
    ("l98_spec_accept_temp_noalloc", C.c_int, [_FP, _FP, C.c_int, C.c_int, C.c_float, C.POINTER(C.c_uint64),
                                               _IP]),
    ("lz_spec_round", C.c_int, [C.POINTER(LZModel), C.POINTER(LZRunState), C.c_int, C.c_int, C.c_int, C.c_float,
                                C.c_int, C.POINTER(LZSampler), C.c_int, C.c_int, _IP, _IP, _IP, _IP,
                                C.c_char_p, C.c_int]),
    ("lz_spec_round_temp", C.c_int, [C.POINTER(LZModel), C.POINTER(LZRunState), C.c_int, C.c_int, C.c_int,
                                     C.c_float, C.c_int, C.POINTER(LZSampler), C.c_int, C.c_int, _IP, _IP, _IP,
                                     _IP, C.c_char_p, C.c_int]),
    ("lz_spec_round_dspark", C.c_int, [C.POINTER(LZModel), C.POINTER(LZRunState), C.c_int, C.c_int, C.c_int,
                                       C.c_float, C.c_int, C.POINTER(LZSampler), C.c_int, _IP, _IP, _IP, _IP,
                                       C.c_char_p, C.c_int]),
    ("lz_spec_round_dspark_temp", C.c_int, [C.POINTER(LZModel), C.POINTER(LZRunState), C.c_int, C.c_int,
                                            C.c_int, C.c_float, C.c_int, C.POINTER(LZSampler), C.c_int, _IP, _IP,
                                            _IP, _IP, C.c_char_p, C.c_int]),
    ("lz_sample_defaults", None, [C.POINTER(LZSampleParams)]),
    ("lz_sampler_init", C.c_int, [C.POINTER(LZSampler), C.c_int, C.POINTER(LZSampleParams), C.c_uint64]),
    ("lz_sampler_free", None, [C.POINTER(LZSampler)]),
    ("lz_random_f32", C.c_float, [C.POINTER(C.c_uint64)]),
    ("lz_sample_argmax", C.c_int, [_FP, C.c_int]),
    ("lz_argmax_p1", C.c_int, [_FP, C.c_int, _FP]),
    ("l98_generate", C.c_int, [C.POINTER(LZModel), C.POINTER(LZRunState), _IP, C.c_int, C.c_int, C.c_int,
                               C.POINTER(LZSampler), _IP, C.c_int, _IP, _IP, _IP]),
    ("l98_session_sampler", C.c_int, [C.POINTER(LZRunState), C.POINTER(LZSampler)]),
    ("l98_session_start", C.c_int, [C.POINTER(LZModel), C.POINTER(LZRunState), _IP, C.c_int,
                                    C.POINTER(LZSampler)]),
    ("l98_greedy_rounds", C.c_int, [C.POINTER(LZModel), C.POINTER(LZRunState), C.c_int, C.c_int, C.c_int, _IP,
                                    C.c_int, _IP, _FP]),
    ("l98_greedy_rounds_ex", C.c_int, [C.POINTER(LZModel), C.POINTER(LZRunState), C.c_int, C.c_int, C.c_int,
                                       _IP, C.c_int, _IP, _IP, _IP, _FP]),
    ("l98_time_kernel", C.c_int, [C.POINTER(LZModel), C.POINTER(LZRunState), C.c_int, C.c_int, C.c_int, _FP]),
    ("l98_time_stream", C.c_int, [C.POINTER(LZRunState), C.c_int, C.c_int, C.c_int, C.c_int, _FP]),
    ("l98_verify_batch", C.c_int, [C.POINTER(LZModel), C.POINTER(C.POINTER(LZRunState)), C.c_int, _IP, C.c_int,
                                   _IP, C.c_int, _FP]),
    ("l98_greedy_rounds_batch", C.c_int, [C.POINTER(LZModel), C.POINTER(C.POINTER(LZRunState)), C.c_int, C.c_int,
                                          C.c_int, _IP, C.c_int, _IP, _FP]),
    ("l98_greedy_rounds_batch_ex", C.c_int, [C.POINTER(LZModel), C.POINTER(C.POINTER(LZRunState)), C.c_int,
                                             C.c_int, C.c_int, _IP, C.c_int, _IP, _FP, C.c_int]),
    ("l98_batched_rounds_ok", C.c_int, [C.POINTER(LZModel), C.c_int, C.c_int]),
    ("l98_set_attn_path", None, [C.c_int]),
    ("l98_row_sums", C.c_int, [_FP, C.c_int, C.c_int, _FP]),
    ("l98_fwht_i32", C.c_int, [_IP, _IP, C.c_int, C.c_int, C.c_int]),
    ("l98_fwht_f32", C.c_int, [_FP, C.c_int, C.c_int, C.c_int, C.c_int]),
    ("l98_subn_fwht_quant", C.c_int, [_FP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, _FP]),
    ("l98_prefix_query", C.c_int, [_FP, C.c_int, C.c_int, C.c_int, _FP, _IP, _FP]),
    ("l98_moe_route", C.c_int, [_FP, _FP, C.c_int, C.c_int, C.c_int, _IP, _FP]),
    ("l98_argmax_rows", C.c_int, [_FP, C.c_int, C.c_int, C.c_int, _IP]),
    ("l98_sort_desc", C.c_int, [C.c_void_p, C.c_int, C.c_void_p, _IP]),
    ("l98_gemv_argmax", C.c_int, [C.c_void_p, _FP, C.c_int, C.c_int, C.c_int, C.c_void_p, _FP, C.c_int, C.c_int,
                                  _FP, _IP]),
    ("l98_gemm_q8", C.c_int, [C.c_void_p, _FP, C.c_int, C.c_int, C.c_void_p, _FP, C.c_int, _FP]),
    ("l98_device_name", C.c_char_p, []),
    ("l98_last_loop_seconds", C.c_double, []),
]

# Exported data (llama98.def:117-157): name -> ctypes type.
HIP_DATA = {n: C.c_longlong for n in (
    "lz_debug_us_draft", "lz_debug_us_verify", "lz_debug_us_capture", "lz_debug_us_catchup",
    "lz_debug_n_capture", "lz_debug_n_catchup", "lz_debug_n_ring_rollback", "lz_debug_n_chunks",
    "lz_debug_n_lmhead", "lz_debug_n_kv_rot", "lz_debug_attn_skip", "lz_debug_mtp_attn_rows")}
HIP_DATA.update({n: C.c_int for n in (
    "lz_debug_mtp_attn_window", "lz_kv_kfmt", "lz_kv_vfmt", "lz_kv_rot_enable", "lz_attn_sink", "lz_attn_window",
    "lz_moe_topk", "lz_prof_enable")})
HIP_DATA.update({"lz_debug_mtp_attn_scale": C.c_float, "lz_moe_tau": C.c_float, "lz_prof_us": C.c_float * 7})


def hip_data(name):
    """The library's exported variable `name` (a ctypes object: .value reads
    and writes it)."""
    return HIP_DATA[name].in_dll(hip_lib(), name)


_hip = None
_synth = None


def hip_lib(path=HIP_LIB):
    """Loads libl98hip.so (raises if it was not built: there is no fallback)."""
    global _hip
    if _hip is None:
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run __graft_entry__.build() first")
        lib = C.CDLL(path)
        for name, res, args in HIP_API:
            f = getattr(lib, name)
            f.restype = res
            f.argtypes = args
        _hip = lib
    return _hip


def set_attn_path(mode):
    """The attention path of a session's chunk for launches and graph
    captures from now on (l98_set_attn_path): 0 by the session's capacity,
    1 one launch per (q head, token), 2 scores by position slice, then the
    softmax and value chains per (q head, token, 32-wide group)."""
    hip_lib().l98_set_attn_path(int(mode))


def synth_lib():
    global _synth
    if _synth is None:
        if not os.path.exists(SYNTH_LIB):
            raise RuntimeError(f"{SYNTH_LIB} is missing: run __graft_entry__.build() first")
        lib = C.CDLL(SYNTH_LIB)
        lib.l98_synth_config.argtypes = [C.c_int, C.POINTER(L98SynthConfig)]
        lib.l98_synth_write.argtypes = [C.c_char_p, C.POINTER(L98SynthConfig), C.c_uint64, C.c_int,
                                        C.c_char_p, C.c_int]
        _synth = lib
    return _synth


def synth_config(config_id):
    cfg = L98SynthConfig()
    if synth_lib().l98_synth_config(config_id, C.byref(cfg)) != 0:
        raise ValueError(f"unknown synthetic config {config_id}")
    return cfg


def write_model(path, config_id, seed=1234, threads=8, cfg=None):
    """Writes path/model.bin for a named synthetic config (see csrc/synth.h)."""
    cfg = cfg or synth_config(config_id)
    os.makedirs(path, exist_ok=True)
    err = C.create_string_buffer(256)
    if synth_lib().l98_synth_write(path.encode(), C.byref(cfg), seed, threads, err, 256) != 0:
        raise RuntimeError(err.value.decode())
    return os.path.join(path, "model.bin")


def ensure_model(path, config_id, seed=1234):
    """Writes the model unless an identical one (same config id + seed) exists."""
    stamp = os.path.join(path, "synth.txt")
    want = f"config {config_id} seed {seed}\n"
    if os.path.exists(stamp) and os.path.exists(os.path.join(path, "model.bin")):
        if open(stamp).read() == want:
            return path
    write_model(path, config_id, seed)
    with open(stamp, "w") as f:
        f.write(want)
    return path


def prompt_tokens(seed, n, vocab):
    """Uniform random ids: splitmix64 stream from seed, id = z mod vocab."""
    out = np.empty(n, np.int64)
    st = seed & 0xFFFFFFFFFFFFFFFF
    M = 0xFFFFFFFFFFFFFFFF
    for i in range(n):
        st = (st + 0x9E3779B97F4A7C15) & M
        z = st
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        z = z ^ (z >> 31)
        out[i] = z % vocab
    return out.astype(np.int32)


def _ip(a):
    return a.ctypes.data_as(_IP)


def _fp(a):
    return a.ctypes.data_as(_FP)


class Engine:
    """One model + one run state on the current HIP device."""

    def __init__(self, model_dir, spec_k_max=LZ_SPEC_K_MAX, seq_len=0):
        lib = hip_lib()
        self.lib = lib
        self.m = LZModel()
        self.s = LZRunState()
        err = C.create_string_buffer(512)
        if lib.lz_open(C.byref(self.m), model_dir.encode(), err, 512) != 0:
            raise RuntimeError("lz_open: " + err.value.decode())
        if lib.lz_state_alloc(C.byref(self.s), C.byref(self.m), seq_len, spec_k_max, err, 512) != 0:
            lib.lz_free(C.byref(self.m))
            raise RuntimeError("lz_state_alloc: " + err.value.decode())
        self.cfg = self.m.config
        self.V = self.cfg.vocab_size
        self.d = self.cfg.hidden_size

    def close(self):
        if self.s.impl:
            self.lib.lz_state_free(C.byref(self.s))
        if self.m.impl:
            self.lib.lz_free(C.byref(self.m))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        self.lib.lz_state_reset(C.byref(self.s), C.byref(self.m))

    def forward_capture(self, token, pos):
        p = self.lib.lz_forward_capture(C.byref(self.m), C.byref(self.s), int(token), int(pos))
        if not p:
            return None
        return np.ctypeslib.as_array(p, shape=(self.V,)).copy()

    def batch_capture(self, tokens, pos0):
        tokens = np.ascontiguousarray(tokens, np.int32)
        h = np.zeros((len(tokens), self.d), np.float32)
        p = self.lib.lz_forward_batch_capture(C.byref(self.m), C.byref(self.s), _ip(tokens), len(tokens),
                                              int(pos0), _fp(h))
        return h if p else None

    def verify(self, tokens, pos0):
        tokens = np.ascontiguousarray(tokens, np.int32)
        n = len(tokens)
        rc = self.lib.lz_forward_verify(C.byref(self.m), C.byref(self.s), _ip(tokens), n, int(pos0))
        if rc != 0:
            return None
        lg = np.ctypeslib.as_array(self.s.mtp_logits, shape=(L98_SPEC_K_GPU + 1, self.V))[:n].copy()
        hd = np.ctypeslib.as_array(self.s.mtp_verify_hidden, shape=(L98_SPEC_K_GPU + 1, self.d))[:n].copy()
        return lg, hd

    def draft_step(self, token, pos):
        p = self.lib.lz_mtp_draft_step(C.byref(self.m), C.byref(self.s), int(token), int(pos))
        if not p:
            return None
        return np.ctypeslib.as_array(p, shape=(self.V,)).copy()

    def chain(self):
        return np.ctypeslib.as_array(self.s.mtp_chain, shape=(self.d,)).copy()

    def mtp_prefill(self, h, next_tokens, pos0):
        h = np.ascontiguousarray(h, np.float32)
        nt = np.ascontiguousarray(next_tokens, np.int32)
        return self.lib.lz_mtp_prefill(C.byref(self.m), C.byref(self.s), _fp(h), _ip(nt), len(nt), int(pos0))

    @property
    def dspark(self):
        return self.m.config.mtp_n_draft > 1

    def spec_round(self, anchor, anchor_pos, k, p_min=0.0, n_min=0, brk=0, skipc=0):
        """lz_spec_round, or lz_spec_round_dspark on a DSpark head (the
        driver's dispatch, src/generate.c:1929-1946)."""
        out = np.zeros(L98_SPEC_K_GPU + 1, np.int32)
        na, npos, ke = C.c_int(), C.c_int(), C.c_int()
        err = C.create_string_buffer(256)
        if self.dspark:
            r = self.lib.lz_spec_round_dspark(C.byref(self.m), C.byref(self.s), int(anchor), int(anchor_pos),
                                              int(k), float(p_min), int(n_min), None, brk, _ip(out), C.byref(na),
                                              C.byref(npos), C.byref(ke), err, 256)
        else:
            r = self.lib.lz_spec_round(C.byref(self.m), C.byref(self.s), int(anchor), int(anchor_pos), int(k),
                                       float(p_min), int(n_min), None, brk, skipc, _ip(out), C.byref(na),
                                       C.byref(npos), C.byref(ke), err, 256)
        return r, out, na.value, npos.value, ke.value

    def draft_batch(self, token, k):
        """lz_mtp_draft_batch: the k DSpark slots' logits, [k][V]."""
        p = self.lib.lz_mtp_draft_batch(C.byref(self.m), C.byref(self.s), int(token), int(k))
        return None if not p else np.ctypeslib.as_array(p, shape=(k, self.V)).copy()

    def session_start(self, prompt):
        prompt = np.ascontiguousarray(prompt, np.int32)
        r = self.lib.l98_session_start(C.byref(self.m), C.byref(self.s), _ip(prompt), len(prompt), None)
        if r < 0:
            raise RuntimeError(f"l98_session_start failed: {r}")
        return r

    def greedy_rounds(self, k, n_rounds, use_graph=True, detail=False):
        """Runs n greedy rounds on the device; returns (tokens, n_accept, device_ms)
        (plus per-round distinct experts and new_pos with detail=True)."""
        cap = n_rounds * (k + 1)
        toks = np.zeros(cap, np.int32)
        na = np.zeros(n_rounds, np.int32)
        ex = np.zeros(n_rounds, np.int32)
        npos = np.zeros(n_rounds, np.int32)
        ms = C.c_float()
        n = self.lib.l98_greedy_rounds_ex(C.byref(self.m), C.byref(self.s), k, n_rounds, 1 if use_graph else 0,
                                          _ip(toks), cap, _ip(na), _ip(ex), _ip(npos), C.byref(ms))
        if n < 0:
            raise RuntimeError(f"l98_greedy_rounds failed: {n}")
        if detail:
            return toks[:n], na, ms.value, ex, npos
        return toks[:n], na, ms.value

    def time_kernel(self, which, mrows, iters):
        ms = C.c_float()
        if self.lib.l98_time_kernel(C.byref(self.m), C.byref(self.s), which, mrows, iters, C.byref(ms)) != 0:
            raise RuntimeError("l98_time_kernel failed")
        return ms.value

    def time_stream(self, blocks, threads, kb_per_block, iters=4):
        us = C.c_float()
        if self.lib.l98_time_stream(C.byref(self.s), blocks, threads, kb_per_block, iters, C.byref(us)) != 0:
            raise RuntimeError("l98_time_stream failed")
        return us.value

    def add_session(self, seq_len=0, spec_k_max=LZ_SPEC_K_MAX):
        """Another run state on the same model (an independent session)."""
        st = LZRunState()
        err = C.create_string_buffer(512)
        if self.lib.lz_state_alloc(C.byref(st), C.byref(self.m), seq_len, spec_k_max, err, 512) != 0:
            raise RuntimeError("lz_state_alloc: " + err.value.decode())
        return st

    def free_session(self, st):
        if st.impl:
            self.lib.lz_state_free(C.byref(st))

    def session_start_on(self, st, prompt):
        prompt = np.ascontiguousarray(prompt, np.int32)
        r = self.lib.l98_session_start(C.byref(self.m), C.byref(st), _ip(prompt), len(prompt), None)
        if r < 0:
            raise RuntimeError(f"l98_session_start failed: {r}")
        return r

    def _state_ptrs(self, states):
        arr = (C.POINTER(LZRunState) * len(states))()
        for i, st in enumerate(states):
            arr[i] = C.pointer(st)
        return arr

    def verify_batch(self, states, tokens, pos0, copy_out=True):
        """l98_verify_batch; returns (wall_ms, [(logits, hidden) per session] or None)."""
        tokens = np.ascontiguousarray(tokens, np.int32)
        n_seq, n_tok = tokens.shape
        pos0 = np.ascontiguousarray(pos0, np.int32)
        ms = C.c_float()
        rc = self.lib.l98_verify_batch(C.byref(self.m), self._state_ptrs(states), n_seq, _ip(tokens), n_tok,
                                       _ip(pos0), 1 if copy_out else 0, C.byref(ms))
        if rc != 0:
            raise RuntimeError("l98_verify_batch failed")
        if not copy_out:
            return ms.value, None
        out = []
        for st in states:
            lg = np.ctypeslib.as_array(st.mtp_logits, shape=(L98_SPEC_K_GPU + 1, self.V))[:n_tok].copy()
            hd = np.ctypeslib.as_array(st.mtp_verify_hidden, shape=(L98_SPEC_K_GPU + 1, self.d))[:n_tok].copy()
            out.append((lg, hd))
        return ms.value, out

    def greedy_rounds_batch(self, states, k, n_rounds, mode=0):
        """l98_greedy_rounds_batch_ex (mode 0: batched when the model allows,
        1: each session's own round graph); returns (wall_ms, [tokens per
        session])."""
        cap = n_rounds * (k + 1)
        toks = np.zeros((len(states), cap), np.int32)
        n_out = np.zeros(len(states), np.int32)
        ms = C.c_float()
        n = self.lib.l98_greedy_rounds_batch_ex(C.byref(self.m), self._state_ptrs(states), len(states), k, n_rounds,
                                                _ip(toks), cap, _ip(n_out), C.byref(ms), mode)
        if n < 0:
            raise RuntimeError(f"l98_greedy_rounds_batch failed: {n}")
        return ms.value, [toks[i, :n_out[i]].copy() for i in range(len(states))]

    def generate_host(self, prompt, k, n_new, p_min=0.0, n_min=0, brk=0, skipc=0, on_round=None):
        """The reference's --spec generation loop driven from the host through
        the reference entry points (lz_forward_batch_capture, lz_mtp_prefill,
        lz_forward_capture, lz_sample_argmax, lz_spec_round), greedy, as
        src/generate.c:1822-2106 drives them; a discarded round records
        n_accept -1.  on_round(tag, array), when given, receives what the
        reference harness's --dump-rounds writes: "capture<r>" logits of each
        capture and, after each round r that emitted, "verify<r>" and
        "vhidden<r>" (the state's mtp_logits / mtp_verify_hidden rows) and
        "draft<r>" (mtp_draft_logits; a DSpark head's k slot rows,
        mtp_kdraft_logits).  A DSpark head's session is the body prefill
        alone (it has no fc for lz_mtp_prefill) and its rounds are
        lz_spec_round_dspark.  Returns (tokens, k_eff per round, n_accept
        per round)."""
        prompt = np.ascontiguousarray(prompt, np.int32)
        n_prompt = len(prompt)
        self.reset()
        h = self.batch_capture(prompt[:-1], 0)
        if h is None or (not self.dspark and self.mtp_prefill(h, prompt[1:], self.s.mtp_pos) != 0):
            raise RuntimeError("prefill failed")
        if not self.dspark:
            self.s.mtp_pos = n_prompt - 1
        toks, ke, na = [], [], []
        token, pos, have_seed = int(prompt[-1]), n_prompt - 1, False
        while len(toks) < n_new:
            if have_seed:
                anchor, anchor_pos = token, pos - 1
            else:
                lg = self.forward_capture(token, pos)
                if lg is None:
                    raise RuntimeError("lz_forward_capture failed")
                if on_round:
                    on_round(f"capture{len(ke)}", lg)
                anchor_pos = pos
                anchor = self.lib.lz_sample_argmax(_fp(lg), self.V)
                toks.append(anchor)
                if len(toks) >= n_new:
                    break
            r, out, n_acc, new_pos, k_eff = self.spec_round(anchor, anchor_pos, k, p_min, n_min, brk, skipc)
            if r < 0:
                raise RuntimeError(f"lz_spec_round failed: {r}")
            if on_round and r > 0:
                rnd = len(ke)
                on_round(f"verify{rnd}", np.ctypeslib.as_array(self.s.mtp_logits, shape=(k_eff + 1, self.V)).copy())
                on_round(f"vhidden{rnd}",
                         np.ctypeslib.as_array(self.s.mtp_verify_hidden, shape=(k_eff + 1, self.d)).copy())
                if self.dspark:
                    on_round(f"draft{rnd}", np.ctypeslib.as_array(self.s.mtp_kdraft_logits, shape=(k, self.V)).copy())
                else:
                    on_round(f"draft{rnd}", np.ctypeslib.as_array(self.s.mtp_draft_logits, shape=(self.V,)).copy())
            ke.append(k_eff)
            na.append(n_acc if r > 0 else -1)
            have_seed = r > 0
            if r > 0:
                toks.extend(int(t) for t in out[:n_acc + 1])
            pos = new_pos + 1
            token = int(out[n_acc])
        return np.array(toks, np.int32), np.array(ke, np.int32), np.array(na, np.int32)

    def generate_host_temp(self, prompt, k, n_new, temp, topp, seed):
        """Temperature generation driven from the host through the reference
        entry point lz_spec_round_temp, round by round (l98_session_start for
        the prefill and the first draw, then the session's sampler).  Returns
        (tokens, k_eff per round, n_accept per round); last_rng is the
        generator state after the run."""
        prompt = np.ascontiguousarray(prompt, np.int32)
        p = LZSampleParams()
        self.lib.lz_sample_defaults(C.byref(p))
        p.temperature, p.topp, p.topk, p.minp = temp, topp, 0, 0.0
        p.presence_penalty, p.frequency_penalty, p.repetition_penalty, p.repeat_last_n = 0.0, 0.0, 1.0, 0
        samp = LZSampler()
        self.lib.lz_sampler_init(C.byref(samp), self.V, C.byref(p), seed)
        anchor = self.lib.l98_session_start(C.byref(self.m), C.byref(self.s), _ip(prompt), len(prompt),
                                            C.byref(samp))
        if anchor < 0:
            raise RuntimeError(f"l98_session_start failed: {anchor}")
        assert self.lib.l98_session_sampler(C.byref(self.s), C.byref(samp)) == 0
        toks, ke, na = [anchor], [], []
        anchor_pos = len(prompt) - 1
        out = np.zeros(L98_SPEC_K_GPU + 1, np.int32)
        n_acc, npos, k_eff = C.c_int(), C.c_int(), C.c_int()
        err = C.create_string_buffer(256)
        while len(toks) < n_new:
            r = self.lib.lz_spec_round_temp(C.byref(self.m), C.byref(self.s), int(anchor), int(anchor_pos), int(k),
                                            0.0, 0, C.byref(samp), 0, 0, _ip(out),
                                            C.byref(n_acc), C.byref(npos), C.byref(k_eff), err, 256)
            if r < 0:
                raise RuntimeError(f"lz_spec_round_temp failed: {r} {err.value.decode()}")
            if r == 0:
                raise RuntimeError("a discarded round (p_min and n_min are 0 here)")
            ke.append(k_eff.value)
            na.append(n_acc.value)
            toks.extend(int(t) for t in out[:n_acc.value + 1])
            anchor, anchor_pos = int(out[n_acc.value]), npos.value
        self.last_rng = samp.rng_state
        return np.array(toks, np.int32), np.array(ke, np.int32), np.array(na, np.int32)

    def generate(self, prompt, k, n_new, temp=0.0, topp=1.0, seed=1):
        prompt = np.ascontiguousarray(prompt, np.int32)
        cap = n_new + L98_SPEC_K_GPU + 2
        toks = np.zeros(cap, np.int32)
        ke = np.zeros(n_new + 8, np.int32)
        na = np.zeros(n_new + 8, np.int32)
        nr = C.c_int()
        samp = None
        if temp > 0.0:
            p = LZSampleParams()
            self.lib.lz_sample_defaults(C.byref(p))
            p.temperature, p.topp, p.topk, p.minp = temp, topp, 0, 0.0
            p.presence_penalty, p.frequency_penalty, p.repetition_penalty, p.repeat_last_n = 0.0, 0.0, 1.0, 0
            samp = LZSampler()
            self.lib.lz_sampler_init(C.byref(samp), self.V, C.byref(p), seed)
        n = self.lib.l98_generate(C.byref(self.m), C.byref(self.s), _ip(prompt), len(prompt), k, n_new,
                                  C.byref(samp) if samp is not None else None, _ip(toks), cap, _ip(ke),
                                  _ip(na), C.byref(nr))
        if n < 0:
            raise RuntimeError(f"l98_generate failed: {n}")
        self.last_rng = samp.rng_state if samp is not None else None   # sampler state after the run
        return toks[:min(n, cap)], ke[:nr.value], na[:nr.value]
