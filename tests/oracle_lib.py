"""ctypes access to the checkers: the CPU restatement (oracle/_build/
libl98oracle.so) and the reference engine's own build (oracle/_ref/).

Test infrastructure only; the product never imports this module.
"""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "_build", "libl98oracle.so")
REF_DIR = os.path.join(ROOT, "oracle", "_ref")
REF_ORACLE_BIN = os.path.join(REF_DIR, "l98ref_oracle")
REF_SHIP_BIN = os.path.join(REF_DIR, "l98ref_ship")
REF_SO = os.path.join(REF_DIR, "libl98ref.so")

_P, _IP, _FP = C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_float)
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} missing: run __graft_entry__.build()")
        L = C.CDLL(ORACLE_SO)
        sig = {
            "ora_open": (_P, [C.c_char_p, C.c_char_p, C.c_int]),
            "ora_close": (None, [_P]),
            "ora_config": (C.c_int, [_P, _IP, C.c_int]),
            "ora_rope_table": (_FP, [_P]),
            "ora_state_new": (_P, [_P, C.c_int, C.c_int]),
            "ora_state_free": (None, [_P]),
            "ora_state_reset": (None, [_P]),
            "ora_session_start": (C.c_int, [_P, _IP, C.c_int]),
            "ora_forward_batch_capture": (C.c_int, [_P, _IP, C.c_int, C.c_int, _FP]),
            "ora_forward_capture": (_FP, [_P, C.c_int, C.c_int]),
            "ora_forward_verify": (C.c_int, [_P, _IP, C.c_int, C.c_int]),
            "ora_mtp_draft_step": (_FP, [_P, C.c_int, C.c_int]),
            "ora_mtp_prefill": (C.c_int, [_P, _FP, _IP, C.c_int, C.c_int]),
            "ora_spec_round": (C.c_int, [_P, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int, C.c_int, C.c_int,
                                         _IP, _IP, _IP, _IP]),
            "ora_generate": (C.c_int, [_P, _IP, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float, C.c_uint64,
                                       C.c_int, C.c_int, _IP, C.c_int, _IP, _IP, _IP, C.POINTER(C.c_uint64)]),
            "ora_generate_ex": (C.c_int, [_P, _IP, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float, C.c_uint64,
                                          C.c_int, C.c_int, C.c_float, C.c_int, _IP, C.c_int, _IP, _IP, _IP,
                                          C.POINTER(C.c_uint64)]),
            "ora_state_info": (C.c_int, [_P, _IP]),
            "ora_set_slot": (None, [_P, C.c_int]),
            "ora_set_mtp_pos": (None, [_P, C.c_int]),
            "ora_kda_state": (_FP, [_P, C.c_int]),
            "ora_conv_state": (_FP, [_P, C.c_int]),
            "ora_mtp_logits": (_FP, [_P]),
            "ora_mtp_hidden": (_FP, [_P]),
            "ora_draft_logits": (_FP, [_P]),
            "ora_mtp_chain": (_FP, [_P]),
            "ora_logits": (_FP, [_P]),
            "ora_kv_plane": (None, [_P, C.c_int, C.c_int, _P, _FP, _P, _FP]),
            "ora_set_tap": (None, [C.c_char_p]),
            "ora_mtp_draft_batch": (_FP, [_P, C.c_int, C.c_int]),
            "ora_mtp_markov_correct": (None, [_P, C.c_int, _FP]),
            "ora_kdraft_logits": (_FP, [_P]),
            "ora_spec_round_dspark": (C.c_int, [_P, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int, C.c_int,
                                                _IP, _IP, _IP, _IP]),
            "o_exp": (C.c_float, [C.c_float]),
            "o_rsqrt": (C.c_float, [C.c_float]),
            "o_sigmoid": (C.c_float, [C.c_float]),
            "o_silu": (C.c_float, [C.c_float]),
            "o_softplus": (C.c_float, [C.c_float]),
            "o_rmsnorm": (None, [_FP, _FP, _FP, C.c_int, C.c_float]),
            "o_l2norm": (None, [_FP, _FP, C.c_int, C.c_float]),
            "o_softmax": (None, [_FP, C.c_int]),
            "o_quantize_q8": (None, [_FP, C.c_int, _P, _FP]),
            "o_quantize_q8_tok": (None, [_FP, C.c_int, _P, _FP]),
            "o_fwht_i32": (None, [_IP, _IP, C.c_int]),
            "o_fwht_f32": (None, [_FP, C.c_int]),
            "o_subn_fwht_quant": (None, [_FP, C.c_int, C.c_int, C.c_int, _P, _FP]),
            "o_subn_rot_f32": (None, [_FP, C.c_int, C.c_int]),
            "o_matmul_q8": (None, [_FP, _P, _FP, _P, _FP, C.c_int, C.c_int, C.c_int, _IP]),
            "o_recur_step": (None, [_FP, _FP, _FP, _FP, _FP, _FP, _FP, C.c_float, C.c_int, C.c_int]),
            "o_moe_route": (None, [_FP, _FP, C.c_int, C.c_int, _IP, _FP]),
            "o_argmax": (C.c_int, [_FP, C.c_int]),
            "o_argmax_p1": (C.c_int, [_FP, C.c_int, _FP]),
            "o_spec_accept": (C.c_int, [_IP, _IP, C.c_int, C.c_int, _IP]),
            "o_spec_accept_temp": (C.c_int, [_FP, _FP, C.c_int, C.c_int, C.c_float, C.POINTER(C.c_uint64), _IP]),
            "o_random_f32": (C.c_float, [C.POINTER(C.c_uint64)]),
            "o_target_dist": (None, [_FP, C.c_int, C.c_float, C.c_float, _FP]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def fp(a):
    return a.ctypes.data_as(_FP)


def ip(a):
    return a.ctypes.data_as(_IP)


class Oracle:
    """CPU restatement of the reference engine on one model + state."""

    def __init__(self, model_dir, spec_k_max=6):
        L = lib()
        err = C.create_string_buffer(256)
        self.m = L.ora_open(model_dir.encode(), err, 256)
        if not self.m:
            raise RuntimeError("ora_open: " + err.value.decode())
        self.s = L.ora_state_new(self.m, 0, spec_k_max)
        cfg = (C.c_int * 30)()
        L.ora_config(self.m, cfg, 30)
        (self.V, self.d, self.n_layers, self.seq_len, self.nh, self.nkv, self.hd, self.nk, self.nv, self.kd,
         self.vd, self.K, self.n_lin, self.n_full, self.gate_rank, self.E, self.topk, self.latent,
         self.moe_inter, self.shared_w, self.mtp_inter, self.q_dim, self.kv_dim, self.conv_dim) = list(cfg)[:24]
        self.n_draft = cfg[29]

    def close(self):
        L = lib()
        if self.s:
            L.ora_state_free(self.s)
            self.s = None
        if self.m:
            L.ora_close(self.m)
            self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def session_start(self, prompt):
        p = np.ascontiguousarray(prompt, np.int32)
        return lib().ora_session_start(self.s, ip(p), len(p))

    def reset(self):
        lib().ora_state_reset(self.s)

    def batch_capture(self, tokens, pos0):
        t = np.ascontiguousarray(tokens, np.int32)
        h = np.zeros((len(t), self.d), np.float32)
        rc = lib().ora_forward_batch_capture(self.s, ip(t), len(t), int(pos0), fp(h))
        return h if rc == 0 else None

    def forward_capture(self, token, pos):
        p = lib().ora_forward_capture(self.s, int(token), int(pos))
        return None if not p else np.ctypeslib.as_array(p, shape=(self.V,)).copy()

    def verify(self, tokens, pos0):
        t = np.ascontiguousarray(tokens, np.int32)
        if lib().ora_forward_verify(self.s, ip(t), len(t), int(pos0)) != 0:
            return None
        lg = np.ctypeslib.as_array(lib().ora_mtp_logits(self.s), shape=(8, self.V))[:len(t)].copy()
        hd = np.ctypeslib.as_array(lib().ora_mtp_hidden(self.s), shape=(8, self.d))[:len(t)].copy()
        return lg, hd

    def draft_step(self, token, pos):
        p = lib().ora_mtp_draft_step(self.s, int(token), int(pos))
        return None if not p else np.ctypeslib.as_array(p, shape=(self.V,)).copy()

    def chain(self):
        return np.ctypeslib.as_array(lib().ora_mtp_chain(self.s), shape=(self.d,)).copy()

    def mtp_prefill(self, h, nxt, pos0):
        h = np.ascontiguousarray(h, np.float32)
        t = np.ascontiguousarray(nxt, np.int32)
        return lib().ora_mtp_prefill(self.s, fp(h), ip(t), len(t), int(pos0))

    def set_mtp_pos(self, pos):
        lib().ora_set_mtp_pos(self.s, int(pos))

    def info(self):
        out = (C.c_int * 5)()
        lib().ora_state_info(self.s, out)
        return dict(ssm_slot=out[0], mtp_pos=out[1], depth=out[2], planes=out[3], seq_len=out[4])

    def kda_state(self, slot):
        n = self.n_lin * self.nv * self.kd * self.vd
        return np.ctypeslib.as_array(lib().ora_kda_state(self.s, slot), shape=(n,)).copy()

    def spec_round(self, anchor, anchor_pos, k, p_min=0.0, n_min=0, brk=0, skipc=0):
        out = np.zeros(8, np.int32)
        na, npos, ke = C.c_int(), C.c_int(), C.c_int()
        r = lib().ora_spec_round(self.s, int(anchor), int(anchor_pos), int(k), float(p_min), int(n_min),
                                 brk, skipc, ip(out), C.byref(na), C.byref(npos), C.byref(ke))
        return r, out, na.value, npos.value, ke.value

    def draft_batch(self, token, k):
        """DSpark base logits of k slots from the current chain, [k][V]."""
        p = lib().ora_mtp_draft_batch(self.s, int(token), int(k))
        return None if not p else np.ctypeslib.as_array(p, shape=(k, self.V)).copy()

    def kdraft_logits(self, k):
        return np.ctypeslib.as_array(lib().ora_kdraft_logits(self.s), shape=(k, self.V)).copy()

    def spec_round_dspark(self, anchor, anchor_pos, k, p_min=0.0, n_min=0, brk=0):
        out = np.zeros(8, np.int32)
        na, npos, ke = C.c_int(), C.c_int(), C.c_int()
        r = lib().ora_spec_round_dspark(self.s, int(anchor), int(anchor_pos), int(k), float(p_min), int(n_min),
                                        brk, ip(out), C.byref(na), C.byref(npos), C.byref(ke))
        return r, out, na.value, npos.value, ke.value

    def generate(self, prompt, k, n_new, temp=0.0, topp=1.0, seed=1, brk=0, skipc=0, p_min=0.0, n_min=0):
        p = np.ascontiguousarray(prompt, np.int32)
        cap = n_new + 16
        toks = np.zeros(cap, np.int32)
        ke = np.zeros(2 * n_new + 8, np.int32)
        na = np.zeros(2 * n_new + 8, np.int32)
        nr = C.c_int()
        rng = C.c_uint64()
        n = lib().ora_generate_ex(self.s, ip(p), len(p), k, n_new, temp, topp, seed, brk, skipc, float(p_min),
                                  int(n_min), ip(toks), cap, ip(ke), ip(na), C.byref(nr), C.byref(rng))
        if n < 0:
            raise RuntimeError(f"ora_generate failed {n}")
        return toks[:min(n, cap)], ke[:nr.value], na[:nr.value], rng.value


def have_reference():
    return os.path.exists(REF_ORACLE_BIN)


def reference_generate(model_dir, prompt, k, n_new, temp=0.0, topp=1.0, seed=1, tmpdir=None, extra=(),
                       binary=REF_ORACLE_BIN):
    """Runs the reference engine's spec-decode loop (oracle/ref_harness.c)."""
    import tempfile
    tmpdir = tmpdir or tempfile.mkdtemp(prefix="l98ref_")
    pf = os.path.join(tmpdir, "prompt.bin")
    np.ascontiguousarray(prompt, np.int32).tofile(pf)
    out = os.path.join(tmpdir, "run")
    subprocess.run([binary, "gen", model_dir, pf, str(k), str(n_new), repr(float(temp)), repr(float(topp)),
                    str(seed), out, *extra], check=True)
    d = {}
    for line in open(out + ".txt"):
        f = line.split()
        d[f[0]] = f[1:]
    res = {
        "tokens": np.array(d["tokens"], np.int32),
        "k_eff": np.array(d["k_eff"], np.int32),
        "n_accept": np.array(d["n_accept"], np.int32),
        "rng": int(d["rng"][0]),
        "ssm_slot": int(d["ssm_slot"][0]),
        "mtp_pos": int(d["mtp_pos"][0]),
        "final_pos": int(d["final_pos"][0]),
        "prefix": out,
        "raw": d,
    }
    return res
