#!/usr/bin/env python3
"""Writes the golden generation fixtures (tests/golden/gen_*.json) from the
reference engine's own build (oracle/_ref/l98ref_oracle, compiled from the
reference sources by oracle/ref.mk) on the seeded synthetic models.

Run in a container that has the reference build:
    make -f oracle/ref.mk all && python3 tests/golden/make_golden.py
Each fixture holds the inputs (model generator id and seed, prompt seed and
length, k, sampling parameters) and the reference's outputs (emitted
tokens, per-round k_eff and n_accept, final RNG state and positions), plus
the sha256 of the generated model.bin so a change of the generator is
caught.  Greedy cases with the "dump" option also hold, for the first
rounds, the sha256 of the bytes of the capture logits, of each round's
verify logits and hidden rows and of its last draft step's logits (the
harness's --dump-rounds files), so a run can be checked bit for bit on the
values, not only on the emitted tokens.
"""
import hashlib
import json
import os
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

import oracle_lib as OL  # noqa: E402

# (fixture, model dir name, generator config id, vocab, n_prompt, k, n_new, temp, topp, sampler seed
#  [, options]); options: prompt_seed, p_min, n_min, brk (debug_break_rollback), skipc (debug_skip_catchup)
CASES = [
    ("gen_micro_k3_greedy", "micro", 10, 512, 24, 3, 40, 0.0, 1.0, 1),
    ("gen_micro_k2_temp", "micro", 10, 512, 24, 2, 32, 0.8, 0.95, 7),
    ("gen_tiny_k1_greedy", "tiny", 0, 8192, 64, 1, 128, 0.0, 1.0, 1),      # configs[0] as stated
    ("gen_tiny_k3_greedy", "tiny", 0, 8192, 64, 3, 128, 0.0, 1.0, 1),
    ("gen_tiny_k4_temp", "tiny", 0, 8192, 64, 4, 64, 0.8, 0.95, 7),
    ("gen_base_k3_greedy", "base", 1, 65536, 64, 3, 48, 0.0, 1.0, 1),
    ("gen_base_k2_temp", "base", 1, 65536, 64, 2, 32, 0.8, 0.95, 7),
    ("gen_large_k3_greedy", "large", 3, 131072, 40, 3, 24, 0.0, 1.0, 1),     # configs[3] shape, short run
    ("gen_server_k3_greedy", "server", 4, 8192, 48, 3, 48, 0.0, 1.0, 1),    # configs[4] model (skewed router)
    ("gen_tiny_k1_temp", "tiny", 0, 8192, 64, 1, 64, 0.8, 0.95, 7),          # configs[2] at k = 1
    # The echo model (config 11): greedy drafts are accepted at every depth,
    # so these runs take the accepted-draft branches of a round (bonus token,
    # partial rollback, catch-up rows, chain reseed from row n).
    ("gen_echo_k1_greedy", "echo", 11, 64, 24, 1, 160, 0.0, 1.0, 1, {"prompt_seed": 11}),
    ("gen_echo_k3_greedy", "echo", 11, 64, 24, 3, 160, 0.0, 1.0, 1, {"prompt_seed": 11}),
    ("gen_echo_k6_greedy", "echo", 11, 64, 24, 6, 200, 0.0, 1.0, 1, {"prompt_seed": 11}),
    ("gen_echo_k3_pmin", "echo", 11, 64, 24, 3, 100, 0.0, 1.0, 1, {"prompt_seed": 2, "p_min": 0.05775}),
    ("gen_echo_k3_pmin_nmin", "echo", 11, 64, 24, 3, 100, 0.0, 1.0, 1,
     {"prompt_seed": 2, "p_min": 0.05775, "n_min": 2}),
    ("gen_echo_k3_brk", "echo", 11, 64, 24, 3, 100, 0.0, 1.0, 1, {"prompt_seed": 11, "brk": 1}),
    ("gen_echo_k3_skipc", "echo", 11, 64, 24, 3, 100, 0.0, 1.0, 1, {"prompt_seed": 11, "skipc": 1}),
    ("gen_echo_k3_temp", "echo", 11, 64, 24, 3, 100, 0.8, 0.95, 7, {"prompt_seed": 11}),
    # Round values (--dump-rounds) of greedy runs, 32-wide projections (micro,
    # echo) included.
    ("gen_micro_k3_rounds", "micro", 10, 512, 24, 3, 40, 0.0, 1.0, 1, {"dump": 6}),
    ("gen_echo_k3_rounds", "echo", 11, 64, 24, 3, 60, 0.0, 1.0, 1, {"prompt_seed": 11, "dump": 6}),
    ("gen_tiny_k3_rounds", "tiny", 0, 8192, 64, 3, 32, 0.0, 1.0, 1, {"dump": 4}),
    # SubLN (use_subn = 1, the survey's C1s variant, and a micro twin).
    ("gen_subln_k3_greedy", "subln", 5, 8192, 64, 3, 96, 0.0, 1.0, 1, {"dump": 4}),
    ("gen_subln_k1_greedy", "subln", 5, 8192, 64, 1, 48, 0.0, 1.0, 1),
    ("gen_subln_k2_temp", "subln", 5, 8192, 64, 2, 48, 0.8, 0.95, 7),
    ("gen_micro_subln_k3_greedy", "micro_subln", 12, 512, 24, 3, 48, 0.0, 1.0, 1, {"dump": 6}),
    # model.bin versions 6-9 with grouped Q8_0 scales, binary16 and u8 scale
    # planes and BF16 small tensors.
    ("gen_fmt13_v9_k3_greedy", "fmt13", 13, 512, 24, 3, 40, 0.0, 1.0, 1, {"dump": 4}),
    ("gen_fmt14_v6_k3_greedy", "fmt14", 14, 8192, 48, 3, 40, 0.0, 1.0, 1, {"dump": 4}),
    ("gen_fmt14_v6_k2_temp", "fmt14", 14, 8192, 48, 2, 32, 0.8, 0.95, 7),
    ("gen_fmt16_v7_k2_greedy", "fmt16", 16, 512, 24, 2, 40, 0.0, 1.0, 1, {"dump": 4}),
    ("gen_fmt17_v8_k3_greedy", "fmt17", 17, 512, 24, 3, 40, 0.0, 1.0, 1, {"dump": 4}),
    # DSpark heads (mtp_n_draft > 1, lz_spec_round_dspark / _temp); the echo
    # one (config 19) accepts 0..k drafts.
    ("gen_ds_micro_k4_greedy", "ds_micro", 18, 512, 24, 4, 40, 0.0, 1.0, 1, {"dump": 4}),
    ("gen_ds_micro_k4_temp", "ds_micro", 18, 512, 24, 4, 40, 0.8, 0.95, 7),
    ("gen_ds_echo_k4_greedy", "ds_echo", 19, 64, 24, 4, 100, 0.0, 1.0, 1, {"prompt_seed": 11, "dump": 6}),
    ("gen_ds_echo_k6_greedy", "ds_echo", 19, 64, 24, 6, 100, 0.0, 1.0, 1, {"prompt_seed": 11}),
    ("gen_ds_echo_k3_temp", "ds_echo", 19, 64, 24, 3, 100, 0.8, 0.95, 7, {"prompt_seed": 11}),
    ("gen_ds_echo_k4_pmin_nmin", "ds_echo", 19, 64, 24, 4, 100, 0.0, 1.0, 1,
     {"prompt_seed": 11, "p_min": 0.025, "n_min": 2}),
    ("gen_ds_echo_k4_brk", "ds_echo", 19, 64, 24, 4, 100, 0.0, 1.0, 1, {"prompt_seed": 11, "brk": 1}),
    ("gen_ds_tiny_k3_greedy", "ds_tiny", 20, 8192, 48, 3, 40, 0.0, 1.0, 1, {"dump": 4}),
    ("gen_ds_subln_k3_greedy", "ds_subln", 21, 512, 24, 3, 40, 0.0, 1.0, 1, {"dump": 4}),
    ("gen_ds_subln_k2_temp", "ds_subln", 21, 512, 24, 2, 40, 0.8, 0.95, 7),
    ("gen_ds_base_k3_greedy", "base_dspark", 22, 65536, 64, 3, 32, 0.0, 1.0, 1, {"dump": 3}),
    # The KDA gate's lower-bound arm (kda_has_gate_lower_bound, lb = -5).
    ("gen_lb_k3_greedy", "lb", 24, 8192, 64, 3, 96, 0.0, 1.0, 1, {"dump": 4}),
    ("gen_lb_k2_temp", "lb", 24, 8192, 64, 2, 48, 0.8, 0.95, 7),
    ("gen_lb_micro_k3_greedy", "lb_micro", 25, 512, 24, 3, 48, 0.0, 1.0, 1, {"dump": 6}),
    # BASELINE.json's configs as stated (numbered from 0): configs[1] with its
    # 512-token prompt and 512 new tokens (the benchmarked workload);
    # configs[2] at temperature on configs[1]'s model and prompt, k = 1 and 4;
    # configs[3] with its 4096-token prompt and 512 new tokens; configs[4]'s
    # model (configs[3]'s shapes, unit-variance router logits, per-expert
    # bias N(0, 0.5)) at a short context.
    ("gen_base_p512_k3_greedy", "base", 1, 65536, 512, 3, 512, 0.0, 1.0, 1, {"dump": 4}),
    ("gen_base_p512_k1_temp", "base", 1, 65536, 512, 1, 128, 0.8, 0.95, 7),
    ("gen_base_p512_k4_temp", "base", 1, 65536, 512, 4, 128, 0.8, 0.95, 7),
    ("gen_large_p4096_k3_greedy", "large", 3, 131072, 4096, 3, 512, 0.0, 1.0, 1, {"dump": 2}),
    ("gen_xlserver_k3_greedy", "xlserver", 23, 131072, 48, 3, 32, 0.0, 1.0, 1, {"dump": 2}),
]
# Prefill + one capture (the harness's capture command; needs no MTP head):
# (fixture, model dir name, generator config id, vocab, n_prompt)
CAPTURES = [
    ("cap_fmt15_v4", "fmt15", 15, 8192, 40),       # version 4: no MTP head, groups of 64
    ("cap_fmt14_v6", "fmt14", 14, 8192, 40),
    ("cap_fmt13_v9", "fmt13", 13, 512, 40),
]
# Draft widths past the reference's cap (LZ_SPEC_K_MAX = 6): written by the
# CPU restatement (oracle/l98_oracle.c, pinned against the reference on every
# fixture above) extended to an 8-slot ring, as ora_*.json.
# (fixture, model dir name, generator config id, vocab, n_prompt, k, n_new, temp, topp, sampler seed)
ORACLE_CASES = [
    ("ora_base_p512_k7_temp", "base", 1, 65536, 512, 7, 128, 0.8, 0.95, 7),    # configs[2] at k = 7
]
MODEL_SEED = 1234
PROMPT_SEED = 0


def main():
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    if not OL.have_reference():
        sys.exit("reference build absent: make -f oracle/ref.mk all")
    root = os.environ.get("L98_MODEL_DIR") or os.path.join(tempfile.gettempdir(), "l98_models")
    only = set(sys.argv[1:])
    for case in CASES:
        name, mdir, cid, V, n_prompt, k, n_new, temp, topp, seed = case[:10]
        opt = case[10] if len(case) > 10 else {}
        if only and name not in only:
            continue
        pseed = opt.get("prompt_seed", PROMPT_SEED)
        p_min, n_min = float(opt.get("p_min", 0.0)), int(opt.get("n_min", 0))
        brk, skipc = int(opt.get("brk", 0)), int(opt.get("skipc", 0))
        extra = []
        if p_min > 0:
            extra += ["--pmin", repr(p_min)]
        if n_min > 0:
            extra += ["--nmin", str(n_min)]
        if brk:
            extra.append("--break-rollback")
        if skipc:
            extra.append("--skip-catchup")
        dump = int(opt.get("dump", 0))
        if dump:
            extra += ["--dump-rounds", str(dump)]
        model = pkg.ensure_model(os.path.join(root, mdir), cid, seed=MODEL_SEED)
        h = hashlib.sha256()
        with open(os.path.join(model, "model.bin"), "rb") as f:
            for blk in iter(lambda: f.read(1 << 24), b""):
                h.update(blk)
        digest = h.hexdigest()
        prompt = pkg.prompt_tokens(pseed, n_prompt, V)
        r = OL.reference_generate(model, prompt, k, n_new, temp, topp, seed=seed, extra=extra)
        out = {
            "model": mdir, "config_id": cid, "model_seed": MODEL_SEED, "model_sha256": digest, "vocab": V,
            "prompt_seed": pseed, "n_prompt": n_prompt, "k": k, "n_new": n_new, "temp": temp,
            "topp": topp, "sampler_seed": seed, "p_min": p_min, "n_min": n_min, "brk": brk, "skipc": skipc,
            "tokens": [int(t) for t in r["tokens"]],
            "k_eff": [int(t) for t in r["k_eff"]],
            "n_accept": [int(t) for t in r["n_accept"]],
            "rng": int(r["rng"]), "final_pos": r["final_pos"], "mtp_pos": r["mtp_pos"],
            "ssm_slot": r["ssm_slot"],
            "source": "oracle/_ref/l98ref_oracle gen (reference engine, float-oracle mode)",
        }
        if dump:
            sums = {}
            for tag in ["capture%d" % i for i in range(dump)] + \
                    ["%s%d" % (t, i) for i in range(dump) for t in ("verify", "vhidden", "draft")]:
                path = "%s.%s.bin" % (r["prefix"], tag)
                if os.path.exists(path):
                    sums[tag] = hashlib.sha256(open(path, "rb").read()).hexdigest()
            out["round_sha256"] = sums
        with open(os.path.join(HERE, name + ".json"), "w") as f:
            json.dump(out, f, indent=1)
        print(name, len(out["tokens"]), "tokens", flush=True)


def main_captures():
    import subprocess
    import __graft_entry__
    import numpy as np
    pkg = __graft_entry__.load_package()
    root = os.environ.get("L98_MODEL_DIR") or os.path.join(tempfile.gettempdir(), "l98_models")
    only = set(sys.argv[1:])
    for name, mdir, cid, V, n_prompt in CAPTURES:
        if only and name not in only:
            continue
        model = pkg.ensure_model(os.path.join(root, mdir), cid, seed=MODEL_SEED)
        digest = hashlib.sha256(open(os.path.join(model, "model.bin"), "rb").read()).hexdigest()
        prompt = pkg.prompt_tokens(PROMPT_SEED, n_prompt, V)
        tmp = tempfile.mkdtemp(prefix="l98cap_")
        pf = os.path.join(tmp, "prompt.bin")
        np.ascontiguousarray(prompt, np.int32).tofile(pf)
        subprocess.run([OL.REF_ORACLE_BIN, "capture", model, pf, os.path.join(tmp, "c")], check=True)
        sums = {t: hashlib.sha256(open(os.path.join(tmp, "c.%s.bin" % t), "rb").read()).hexdigest()
                for t in ("capture", "hidden")}
        out = {"model": mdir, "config_id": cid, "model_seed": MODEL_SEED, "model_sha256": digest, "vocab": V,
               "prompt_seed": PROMPT_SEED, "n_prompt": n_prompt, "sha256": sums,
               "source": "oracle/_ref/l98ref_oracle capture (reference engine, float-oracle mode)"}
        with open(os.path.join(HERE, name + ".json"), "w") as f:
            json.dump(out, f, indent=1)
        print(name, flush=True)


def main_oracle():
    import __graft_entry__
    from oracle_lib import Oracle
    pkg = __graft_entry__.load_package()
    root = os.environ.get("L98_MODEL_DIR") or os.path.join(tempfile.gettempdir(), "l98_models")
    only = set(sys.argv[1:])
    for name, mdir, cid, V, n_prompt, k, n_new, temp, topp, seed in ORACLE_CASES:
        if only and name not in only:
            continue
        model = pkg.ensure_model(os.path.join(root, mdir), cid, seed=MODEL_SEED)
        h = hashlib.sha256()
        with open(os.path.join(model, "model.bin"), "rb") as f:
            for blk in iter(lambda: f.read(1 << 24), b""):
                h.update(blk)
        prompt = pkg.prompt_tokens(PROMPT_SEED, n_prompt, V)
        o = Oracle(model, spec_k_max=k)
        try:
            toks, ke, na, rng = o.generate(prompt, k, n_new, temp, topp, seed)
        finally:
            o.close()
        out = {"model": mdir, "config_id": cid, "model_seed": MODEL_SEED, "model_sha256": h.hexdigest(),
               "vocab": V, "prompt_seed": PROMPT_SEED, "n_prompt": n_prompt, "k": k, "n_new": n_new, "temp": temp,
               "topp": topp, "sampler_seed": seed, "tokens": [int(t) for t in toks],
               "k_eff": [int(t) for t in ke], "n_accept": [int(t) for t in na], "rng": int(rng),
               "source": "oracle/l98_oracle.c ora_generate_ex (the CPU restatement; k past the reference's cap)"}
        with open(os.path.join(HERE, name + ".json"), "w") as f:
            json.dump(out, f, indent=1)
        print(name, len(out["tokens"]), "tokens", flush=True)


if __name__ == "__main__":
    main()
    main_captures()
    main_oracle()
