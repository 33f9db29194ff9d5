#!/usr/bin/env python3
"""Benchmark of the MTP speculative-decoding step on one MI355X.

Metric: accepted tokens/s at batch 1 with k = 3 drafts, and
the verify step's HBM bandwidth as a fraction of the MI355X peak.

Workload: the ~0.5B random-init KunMoe (d=1024, 24 layers in a
3:1 KDA:attention pattern, 16 heads x 64, 64 experts top-6, latent 256,
expert FFN 512, vocab 65536, int8 per-row weights), greedy, batch 1, a
512-token uniform-random prompt (seed 0), MTP drafting k = 3.

A step is one speculative round: k draft steps, the (k+1)-token verify
forward, acceptance, ring rollback and MTP catch-up, all on the device (one
HIP graph launch per round).  W warmup rounds, then K timed rounds between
device synchronizations; value = tokens emitted in the K rounds / wall time.

The JSON line also carries:
  roofline      the kernel with the largest share of the round's time: the
                RMSNorm-prologue GEMV k_gemv_q8<M, PJ, norm> (the verify's
                KDA, attention and MoE layer-input projections, one launch
                each per layer).  Each of its three launch shapes is timed
                with HIP events on the state's stream, every layer's launch
                in order, back to back; achieved = algorithmic bytes /
                duration summed over one round's launches; traffic from the
                committed rocprofv3 byte-counter summary;
  lm_head       the tied lm_head GEMV at M = k+1 (back to back, and cold);
  verify        the verify forward alone (M = k+1), algorithmic bytes / time,
                beside the reference's verify on the host;
  round         accepted tok/s against the round's HBM roofline
                E[n_accept+1] * 8e12 / bytes_per_round (bytes counted from
                the distinct experts and context each round actually used);
  prefill       the prompt's prefill (512-row matrix-core chunks);
  cpu_baseline  the reference engine's own shipping build (AVX2 tier,
                oracle/_ref/l98ref_ship) on one host core, same model and
                prompt, with its float-oracle build timed beside it.
"""
import argparse
import json
import os
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def model_bytes(cfg):
    """Per-component algorithmic bytes of the model (int8 weight + 4 B/row)."""
    d, V = cfg.hidden_size, cfg.vocab_size
    def mat(r, c):
        return r * c + 4 * r
    key, value = cfg.lin_key_dim, cfg.lin_value_dim
    nv, kd, vd = cfg.lin_n_v_heads, cfg.lin_k_head_dim, cfg.lin_v_head_dim
    kda = (2 * mat(key, d) + mat(value, d) + mat(cfg.kda_gate_rank, d) + mat(nv * kd, cfg.kda_gate_rank)
           + mat(nv, d) + mat(value, d) + mat(d, value) + 4 * cfg.lin_conv_dim * cfg.conv_kernel
           + 4 * (2 * nv * kd + vd) + 2 * 4 * nv * kd * vd            # params + fp32 state in and out
           + 2 * 4 * cfg.lin_conv_dim * (cfg.conv_kernel - 1))
    attn = (mat(cfg.attn_qgate_dim, d) + 2 * mat(cfg.attn_kv_dim, d) + mat(d, cfg.attn_q_dim)
            + 8 * cfg.head_dim)
    kv_row = 2 * cfg.attn_kv_dim + 2 * 4 * cfg.attn_kv_dim // 32       # Q8 K and V + scales, per position
    moe_fixed = (mat(cfg.num_experts, d) + 4 * cfg.num_experts + mat(cfg.moe_latent_dim, d)
                 + mat(d, cfg.moe_latent_dim) + 2 * mat(cfg.moe_shared_width, d) + mat(d, cfg.moe_shared_width))
    expert = 2 * mat(cfg.moe_intermediate_size, cfg.moe_latent_dim) + mat(cfg.moe_latent_dim,
                                                                            cfg.moe_intermediate_size)
    norms = 2 * 4 * d
    lm_head = mat(V, d)
    mtp = (mat(d, 2 * d) + attn + 2 * mat(cfg.mtp_intermediate_size, d) + mat(d, cfg.mtp_intermediate_size)
           + 5 * 4 * d)
    return dict(kda=kda, attn=attn, kv_row=kv_row, moe_fixed=moe_fixed, expert=expert, norms=norms,
                lm_head=lm_head, mtp=mtp)


def round_bytes(cfg, k, ctx_verify, experts):
    """Algorithmic HBM bytes of one round: k draft steps + an M = k+1 verify."""
    b = model_bytes(cfg)
    n_lin, n_full = cfg.n_linear_layers, cfg.n_full_layers
    M = k + 1
    draft = k * (b["mtp"] + b["lm_head"]) + b["kv_row"] * sum(ctx_verify + i for i in range(k))
    verify = (n_lin * b["kda"] + n_full * b["attn"] + (n_lin + n_full) * (b["moe_fixed"] + b["norms"])
              + experts * b["expert"] + b["lm_head"] + n_full * b["kv_row"] * (ctx_verify + M)
              + 4 * M * (cfg.vocab_size + cfg.hidden_size))
    return draft, verify


def norm_gemv_shapes(cfg, M):
    """The RMSNorm-prologue GEMV's launches in a verify of M rows: (name,
    l98_time_kernel mode, launches per round, algorithmic bytes per launch).
    Bytes: every weight row once (int8 + 4 B scale), the residual rows and
    addends read once (4 B each), the folded residual written once, the
    norm weight, and the outputs."""
    d = cfg.hidden_size
    def b(rows, addends):
        return rows * (d + 4) + 4 * M * d * (1 + addends) + 4 * M * d + 4 * d + 4 * M * rows
    kda_rows = 2 * cfg.lin_key_dim + 2 * cfg.lin_value_dim + cfg.kda_gate_rank + cfg.lin_n_v_heads
    attn_rows = cfg.attn_qgate_dim + 2 * cfg.attn_kv_dim
    moe_rows = cfg.num_experts + cfg.moe_latent_dim + 2 * cfg.moe_shared_width
    return [("kda input", 4, cfg.n_linear_layers, b(kda_rows, 2)),
            ("attention input", 5, cfg.n_full_layers, b(attn_rows, 2)),
            ("moe input", 6, cfg.n_layers, b(moe_rows, 1))]


def kda_step_bytes(cfg, M):
    """Algorithmic bytes of one KDA layer's token step over M verify rows
    (k_kda_step): the fp32 state read from its ring slot and written to the
    M slots after it, the conv history read and written per row, the taps,
    the f_b gate projection, A_log / dt_bias / output norm, the projected q,
    k, v, gate-input, f_a and b rows read, and the quantized output rows."""
    nv, kd, vd, K = cfg.lin_n_v_heads, cfg.lin_k_head_dim, cfg.lin_v_head_dim, cfg.conv_kernel
    key, value, conv, rank = cfg.lin_key_dim, cfg.lin_value_dim, cfg.lin_conv_dim, cfg.kda_gate_rank
    state = 4 * nv * kd * vd
    hist = 4 * conv * (K - 1)
    return (state * (1 + M) + hist * (1 + M) + 4 * conv * K + (nv * kd * rank + 4 * nv * kd)
            + 4 * nv + 4 * nv * kd + 4 * vd
            + 4 * M * (2 * key + 2 * value + rank + nv) + M * value + 4 * M * value // 32)


def moe_bytes(cfg, M, experts):
    """Algorithmic bytes of the routed experts of one MoE layer over M verify
    rows with `experts` distinct experts: k_moe_up (routing from the router
    logits, w1 and w3 of each distinct expert, the latent rows in, the
    (token, slot) pairs' h1 / h3 out) and k_expert_gemv (w2 of each distinct
    expert, h1 / h3 in, the pairs' latent rows out)."""
    lat, inter, E, topk = cfg.moe_latent_dim, cfg.moe_intermediate_size, cfg.num_experts, cfg.num_experts_per_token
    pairs = M * topk
    up = experts * 2 * inter * (lat + 4) + 4 * M * E + 4 * E + 4 * M * lat + 2 * 4 * pairs * inter
    down = experts * lat * (inter + 4) + 2 * 4 * pairs * inter + 4 * pairs * lat
    return up, down


def sources_sha(paths):
    """sha256 of the named source files' bytes, in order (ties a committed
    counter summary to the kernel code it measured)."""
    import hashlib
    h = hashlib.sha256()
    for p in paths:
        with open(os.path.join(ROOT, p), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


# the kernel sources the traffic summary's figures depend on
TRAFFIC_SOURCES = ["llama98-zh_amd/csrc/l98_gemv.h", "llama98-zh_amd/csrc/l98_k_gemv.hip",
                   "llama98-zh_amd/csrc/l98_devmath.h", "llama98-zh_amd/csrc/l98_k_kda.hip",
                   "llama98-zh_amd/csrc/l98_k_moe.hip"]
TRAFFIC_PROFILE = os.path.join("profiles", "traffic_configs1_m4.md")


def measured_traffic(config, k):
    """HBM bytes per round of the RMSNorm-prologue GEMV launches (and per
    lm_head launch) from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary (copy-calibrated), for the configs[1], k = 3 workload it was
    measured on; None otherwise."""
    path = os.path.join(ROOT, TRAFFIC_PROFILE)
    out = {}
    if config != 1 or k != 3 or not os.path.exists(path):
        return out
    vals = {}
    for line in open(path):
        if ":" in line and not line.startswith(("|", "#", " ")):
            key, val = line.split(":", 1)
            vals[key.strip()] = val.strip()
    if vals.get("kernel_sources_sha256") != sources_sha(TRAFFIC_SOURCES):
        out["traffic_source"] = f"{TRAFFIC_PROFILE} is stale (the kernel sources changed since it was measured)"
        return out
    out["traffic_source"] = f"{TRAFFIC_PROFILE} (kernel sources sha256 {vals['kernel_sources_sha256'][:16]})"
    for key in ("norm_gemv_traffic_bytes_per_round", "lm_head_traffic_bytes_per_launch"):
        if key in vals:
            out[key] = int(vals[key])
    for key in ("norm_gemv_rocprof_us_per_round", "norm_gemv_rocprof_frac"):
        if key in vals:
            out[key] = float(vals[key])
    return out


def cpu_baseline(model_dir, vocab, k, n_prompt):
    """The reference engine on one host core each, on a bounded sample of
    the benched workload (the same model and prompt; a few rounds): the
    shipping build (the baseline) and the float-oracle build, run side by
    side on two pinned cores.  Each times its prefill, its rounds and then
    its verify forward of M = k+1 rows alone."""
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    bins = {m: os.path.join(ROOT, "oracle", "_ref", f"l98ref_{m}") for m in ("ship", "oracle")}
    if not all(os.path.exists(b) for b in bins.values()):
        return None
    tmp = tempfile.mkdtemp(prefix="l98cpu_")
    pf = os.path.join(tmp, "prompt.bin")
    n_new = 12
    pkg.prompt_tokens(0, n_prompt, vocab).tofile(pf)
    cores = sorted(os.sched_getaffinity(0))
    procs = {}
    for i, (mode, binary) in enumerate(bins.items()):
        cmd = ["taskset", "-c", str(cores[-1 - i]), binary, "gen", model_dir, pf, str(k), str(n_new), "0", "1", "1",
               os.path.join(tmp, mode), "--timing", "--verify-iters", "3"]
        log("cpu baseline:", " ".join(cmd))
        procs[mode] = (subprocess.Popen(cmd), cores[-1 - i])
    res = {}
    for mode, (p, core) in procs.items():
        if p.wait(timeout=600) != 0:
            return None
        d = {}
        for line in open(os.path.join(tmp, mode + ".txt")):
            f = line.split()
            d[f[0]] = f[1:]
        res[mode] = d
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    def summary(d):
        n_tok, loop_s = int(d["n_tokens"][0]), float(d["loop_us"][0]) * 1e-6
        return {"tok_s": round(n_tok / loop_s, 3), "tokens": n_tok, "rounds": len(d["k_eff"]),
                "round_ms": round(loop_s * 1e3 / max(1, len(d["k_eff"])), 3),
                "prefill_s": round(float(d["prefill_us"][0]) * 1e-6, 2),
                "verify_ms": round(float(d["verify_us_median"][0]) * 1e-3, 3), "tier": d["kernel"][0]}
    ship, ora = summary(res["ship"]), summary(res["oracle"])
    ora["tokens"] = [int(t) for t in res["oracle"]["tokens"]]
    return {"value": ship["tok_s"], "unit": "tok/s", "cores": 1, "kind": "reference",
            "sample": f"reference shipping build (lz_spec_round, tier {ship['tier']}, gcc -O2 AVX2) on 1 core of "
                      f"{os.cpu_count()} ({cpu}): {n_prompt}-token prompt prefilled ({ship['prefill_s']} s), then "
                      f"{ship['tokens']} tokens in {ship['rounds']} rounds at k={k} on the same model; its verify "
                      f"forward of M={k + 1} rows alone: {ship['verify_ms']} ms",
            "round_ms": ship["round_ms"], "verify_ms": ship["verify_ms"], "prefill_s": ship["prefill_s"],
            "oracle_mode": ora, "ship_tokens": [int(t) for t in res["ship"]["tokens"]]}


def bench_server(args, pkg):
    """n_seq sessions of configs[3]'s model (128 experts top-8)
    with the skewed router (unit-variance logits plus a per-expert bias
    N(0, 0.5); synthetic config 23) and ragged contexts (uniform in
    [256, 2048], seed 0), k = 3.  Times the batched verify of k+1 tokens
    per session (all sessions in flight together, one stream each) and the
    batched greedy rounds; prints one JSON line."""
    import numpy as np
    mdir = os.path.join(args.model_dir, "xlserver")
    pkg.ensure_model(mdir, 23, seed=1234)
    eng = pkg.Engine(mdir)
    k, n_seq = args.k, args.sessions
    rng = np.random.default_rng(0)
    ctx = rng.integers(256, 2049, size=n_seq)
    states = []
    t0 = time.time()
    for i in range(n_seq):
        st = eng.add_session()
        eng.session_start_on(st, pkg.prompt_tokens(1000 + i, int(ctx[i]), eng.V))
        states.append(st)
    log(f"{n_seq} sessions prefilled ({int(ctx.sum())} prompt tokens) in {time.time() - t0:.1f}s")
    toks = np.array([[(13 * i + 7 * j + 5) % eng.V for j in range(k + 1)] for i in range(n_seq)], np.int32)
    pos0 = ctx.astype(np.int32)
    for _ in range(args.warmup):
        eng.verify_batch(states, toks, pos0, copy_out=False)
    ms = [eng.verify_batch(states, toks, pos0, copy_out=False)[0] for _ in range(args.steps)]
    step_ms = float(np.mean(ms))
    value = n_seq * (k + 1) / (step_ms * 1e-3)
    # batched greedy rounds (rounds continue from each session's prefill;
    # each session's round is a HIP graph launch, so --no-graph leaves them out)
    nr = min(args.steps, 32)
    rounds = None
    if not args.no_graph:
        r_ms, outs = eng.greedy_rounds_batch(states, k, nr)
        emitted = sum(len(o) for o in outs)
        rounds = {"rounds": nr, "wall_ms": round(r_ms, 3), "tokens": emitted, "tok_s": round(emitted / (r_ms * 1e-3), 1)}
    out = {
        "metric": f"batched verify tok/s ({n_seq} sessions x k+1={k + 1} tokens, ragged contexts 256-2048)",
        "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8xint8->int32, fp32 epilogue/state",
        "data": "synthetic (seeded random-init weights, router N(0,1) logits + N(0,0.5) expert bias; random prompts)",
        "config": {"workload": f"configs[4] server batch: {n_seq} sessions of the configs[3] model (d=2048, L=32, "
                               f"128 experts top-8, skewed router), k={k}, "
                               f"contexts {int(ctx.min())}-{int(ctx.max())}", "sessions": n_seq, "k": k},
        "rounds": rounds,
    }
    print(json.dumps(out))
    for st in states:
        eng.free_session(st)
    eng.close()


def bench_ksweep(args, pkg):
    """configs[1]'s model at temperature 0.8, top-p 0.95, a
    fixed sampler seed, draft widths k in {1, 2, 4, 7} (k = 7 through the
    library's own generation loop: the reference caps k at 6), after
    configs[1]'s 512-token prompt; per k the generation's tok/s and
    acceptance (prefill excluded), and the verify forward of M = k+1 rows
    timed alone.  Prints one JSON line."""
    import numpy as np
    mdir = os.path.join(args.model_dir, "base")
    pkg.ensure_model(mdir, 1, seed=1234)
    eng = pkg.Engine(mdir, spec_k_max=pkg.L98_SPEC_K_GPU)
    prompt = pkg.prompt_tokens(0, args.prompt, eng.V)
    rows = []
    n_new = 256
    for k in (1, 2, 4, 7):
        eng.generate(prompt, k, 16, 0.8, 0.95, 7)                 # warm: code load, the per-k graphs
        t0 = time.perf_counter()
        eng.session_start(prompt)
        prefill = time.perf_counter() - t0
        t0 = time.perf_counter()
        toks, ke, na = eng.generate(prompt, k, n_new, 0.8, 0.95, 7)
        wall = time.perf_counter() - t0
        ver_ms = eng.time_kernel(1, k + 1, 20)
        rows.append({"k": k, "M": k + 1, "tokens": int(len(toks)), "rounds": int(len(na)),
                     "alpha": round(float(np.clip(na, 0, None).sum()) / max(1, int(np.sum(ke))), 4),
                     "tok_s": round(len(toks) / (wall - prefill), 1), "wall_s_with_prefill": round(wall, 4),
                     "prefill_s": round(prefill, 4), "verify_ms": round(ver_ms, 4)})
    out = {"metric": "temperature spec decode tok/s and verify ms per draft width (configs[2])",
           "value": rows[-1]["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": n_new, "warmup": 16,
           "ms_per_step": rows[-1]["verify_ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "int8xint8->int32, fp32 epilogue/state",
           "data": f"synthetic (seeded random-init weights; {len(prompt)}-token random prompt; sampler seed 7)",
           "config": {"workload": f"configs[2]: configs[1] model, T=0.8 top-p 0.95, k in {{1,2,4,7}}, "
                                  f"generation of {n_new} tokens per k after a {len(prompt)}-token prompt "
                                  f"(tok/s with the prefill, timed alone, taken out), verify timed alone"},
           "sweep": rows}
    print(json.dumps(out))
    eng.close()


def bench_dspark(args, pkg):
    """A DSpark head (mtp_n_draft = 6) on configs[1]'s shapes (synthetic
    config 22): greedy rounds at k = 1..6, each one HIP graph launch whose
    k drafts are one k-row pass (lz_mtp_draft_batch) instead of k chained
    draft steps; the draft batch alone is timed too.  Prints one JSON line."""
    import numpy as np
    mdir = os.path.join(args.model_dir, "base_dspark")
    pkg.ensure_model(mdir, 22, seed=1234)
    eng = pkg.Engine(mdir, spec_k_max=pkg.L98_SPEC_K_GPU)
    prompt = pkg.prompt_tokens(0, args.prompt, eng.V)
    rows = []
    n_rounds = min(args.steps, 64)          # rounds that fit the 1280-row state at k = 6 after the prompt
    for k in range(1, 7):
        eng.session_start(prompt)
        eng.greedy_rounds(k, args.warmup)
        _, na, ms = eng.greedy_rounds(k, n_rounds, detail=False)
        emitted = int(np.sum(na)) + len(na)
        lg = eng.forward_capture(int(prompt[-1]), len(prompt) - 1)
        t0 = time.perf_counter()
        for _ in range(20):
            eng.draft_batch(int(np.argmax(lg)), k)
        batch_ms = (time.perf_counter() - t0) * 1e3 / 20
        rows.append({"k": k, "round_ms": round(ms / n_rounds, 4), "tok_s": round(emitted / (ms * 1e-3), 1),
                     "alpha": round(float(np.sum(na)) / (k * len(na)), 4),
                     "draft_batch_ms_host": round(batch_ms, 4)})
    out = {"metric": "DSpark greedy spec decode tok/s per draft width (configs[1] shapes, 6-slot head)",
           "value": rows[2]["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": n_rounds, "warmup": args.warmup,
           "ms_per_step": rows[2]["round_ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "int8xint8->int32, fp32 epilogue/state",
           "data": "synthetic (seeded random-init weights; random prompt)",
           "config": {"workload": f"configs[1] shapes + DSpark head (mtp_n_draft 6, model.bin v6), "
                                  f"{args.prompt}-token prompt, greedy rounds at k = 1..6; value at k = 3"},
           "sweep": rows}
    print(json.dumps(out))
    eng.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--k", type=int, default=None, help="draft width (default: the config's own, 1 for configs[0], else 3)")
    ap.add_argument("--config", type=int, default=1)
    ap.add_argument("--prompt", type=int, default=None,
                    help="prompt tokens (default: the config's own, 64 / 512 / 512 / 4096 for configs[0..3])")
    ap.add_argument("--model-dir", default=os.path.join(tempfile.gettempdir(), "l98_models"))
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--sessions", type=int, default=32, help="configs[4]: concurrent sessions")
    ap.add_argument("--dspark", action="store_true", help="a DSpark head on configs[1]'s shapes")
    ap.add_argument("--attn-path", type=int, default=0,
                    help="attention path of a session's chunk (l98_set_attn_path): 0 by capacity, 1 one launch, "
                         "2 slice scores + grouped value chains")
    args = ap.parse_args()
    if args.prompt is None:
        args.prompt = {0: 64, 3: 4096}.get(args.config, 512)
    if args.k is None:
        args.k = 1 if args.config == 0 else 3
    if args.gpus != 1:
        print(f"bench.py: this build runs the single-sequence path on one GPU; --gpus {args.gpus} "
              f"is not supported (see DESIGN.md for how the path would shard)", file=sys.stderr)
        sys.exit(2)

    import __graft_entry__
    pkg = __graft_entry__.load_package()
    pkg.set_attn_path(args.attn_path)
    if args.config == 4:
        bench_server(args, pkg)
        return
    if args.config == 2:
        bench_ksweep(args, pkg)
        return
    if args.dspark:
        bench_dspark(args, pkg)
        return
    name = {0: "tiny", 1: "base", 3: "large"}.get(args.config, f"c{args.config}")
    mdir = os.path.join(args.model_dir, name)
    t0 = time.time()
    pkg.ensure_model(mdir, args.config, seed=1234)
    log(f"model {mdir} ready in {time.time() - t0:.1f}s")
    eng = pkg.Engine(mdir, spec_k_max=pkg.L98_SPEC_K_GPU)    # ring depth 8: the sweep's M = 8 verify
    cfg = eng.cfg
    log(f"device {pkg.hip_lib().l98_device_name().decode()}; weights {eng.m.bytes_device / 1e9:.3f} GB, "
        f"state {eng.s.bytes_device / 1e6:.1f} MB")
    k = args.k
    prompt = pkg.prompt_tokens(0, args.prompt, cfg.vocab_size)
    eng.session_start(prompt)                   # first use: the wide scratch and code load
    t0 = time.perf_counter()
    eng.session_start(prompt)
    prefill_s = time.perf_counter() - t0
    log(f"prefill of {len(prompt)} tokens: {prefill_s:.3f}s")
    use_graph = not args.no_graph
    eng.greedy_rounds(k, args.warmup, use_graph)
    t0 = time.perf_counter()
    toks, na, dev_ms, experts, new_pos = eng.greedy_rounds(k, args.steps, use_graph, detail=True)
    t1 = time.perf_counter()
    wall = t1 - t0
    n_tok = len(toks)
    value = n_tok / wall
    log(f"{args.steps} rounds: {n_tok} tokens in {wall * 1e3:.1f} ms (device {dev_ms:.1f} ms), "
        f"alpha = {na.sum() / (k * args.steps):.4f}")

    # round roofline from the bytes the rounds actually moved
    rb_d = rb_v = 0.0
    for r in range(args.steps):
        ctx = int(new_pos[r]) - 1 - int(na[r])      # anchor position of the round
        dr, vr = round_bytes(cfg, k, ctx, int(experts[r]))
        rb_d += dr
        rb_v += vr
    mean_round = (rb_d + rb_v) / args.steps
    roof_toks = (n_tok / args.steps) * HBM_PEAK / mean_round
    # dominant kernel: the RMSNorm-prologue GEMV, its three launch shapes
    M = k + 1
    shapes = norm_gemv_shapes(cfg, M)
    ng_rows = []
    for name, mode, count, nbytes in shapes:
        t_ms = eng.time_kernel(mode, M, 10)
        ng_rows.append({"launch": name, "per_round": count, "bytes": nbytes, "us": round(t_ms * 1e3, 3),
                        "GB/s": round(nbytes / (t_ms * 1e-3) / 1e9, 1)})
    ng_bytes = sum(r["bytes"] * r["per_round"] for r in ng_rows)
    ng_s = sum(r["us"] * 1e-6 * r["per_round"] for r in ng_rows)
    ng_bw = ng_bytes / ng_s
    traffic = measured_traffic(args.config, k)
    # the tied lm_head GEMV at M = k+1 rows
    lm_ms = eng.time_kernel(0, M, 50)
    lm_cold_ms = eng.time_kernel(3, M, 10)      # each launch after a cache-evicting copy
    V, d = cfg.vocab_size, cfg.hidden_size
    lm_bytes = V * d + 4 * V + M * d + 4 * M * d // 32 + 4 * M * V
    lm_bw = lm_bytes / (lm_ms * 1e-3)
    # verify forward alone
    ver_ms = eng.time_kernel(1, M, 20)
    ctx_now = int(new_pos[-1])
    ver_bytes = round_bytes(cfg, k, ctx_now, int(experts.mean()))[1]
    ver_bw = ver_bytes / (ver_ms * 1e-3)
    # configs[2]'s verify widths on this model: M = k+1 rows timed alone
    sweep = []
    for ks in (1, 2, 4, 7):
        t_ms = eng.time_kernel(1, ks + 1, 10)
        vb = round_bytes(cfg, ks, ctx_now, int(experts.mean()))[1]
        sweep.append({"k": ks, "M": ks + 1, "ms": round(t_ms, 4), "GB/s": round(vb / (t_ms * 1e-3) / 1e9, 1)})
    # the launch floor: per launch of 64 dependent launches in one graph
    floor = {"graph_empty_1block_us": round(eng.time_kernel(7, M, 20) * 1e3, 3),
             "graph_empty_256blocks_us": round(eng.time_kernel(8, M, 20) * 1e3, 3),
             "graph_handoff_256blocks_us": round(eng.time_kernel(9, M, 20) * 1e3, 3),
             "stream_empty_256blocks_us": round(eng.time_kernel(10, M, 20) * 1e3, 3),
             "note": "chains of 64 dependent launches; handoff: every block reads the M x hidden floats the "
                     "previous launch wrote"}
    cpu = None if args.no_cpu else cpu_baseline(mdir, cfg.vocab_size, k, len(prompt))
    parity = bench_parity(eng, prompt, k, cpu)
    out = {
        "metric": "accepted tok/s @bs1 k=3; verify-step HBM GB/s as % of MI355X peak",
        "value": round(value, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xint8->int32, fp32 epilogue/state",
        "data": "synthetic (seeded random-init weights N(0,0.02), uniform random prompt)",
        "config": {"workload": f"configs[{args.config}] KunMoe d={d} L={cfg.n_layers} V={V} "
                               f"E={cfg.num_experts} top{cfg.num_experts_per_token}; k={k} greedy bs1, "
                               f"{len(prompt)}-token prompt", "k": k, "batch": 1,
                   "graph": use_graph},
        "roofline": {"bound": "hbm",
                     "kernel": f"k_gemv_q8<{M}, PJ, norm> (RMSNorm-prologue GEMV of the verify's layer inputs, "
                               f"{sum(r['per_round'] for r in ng_rows)} launches per round)",
                     "achieved": round(ng_bw / 1e9, 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(ng_bw / HBM_PEAK, 4),
                     "traffic": traffic.get("norm_gemv_traffic_bytes_per_round"),
                     "traffic_source": traffic.get("traffic_source"),
                     "frac_rocprof": traffic.get("norm_gemv_rocprof_frac"),
                     "bytes_per_round": int(ng_bytes), "us_per_round": round(ng_s * 1e6, 1),
                     "timing": "each launch shape's layers back to back, HIP events on the state's stream "
                               "(l98_time_kernel modes 4-6); frac_rocprof: the same launches' rocprofv3 mean "
                               "durations from the traffic summary",
                     "launches": ng_rows},
        "lm_head": {"kernel": f"k_gemv_q8<{M}, 0, pre-quantized> (tied lm_head, {V}x{d} int8)",
                    "bytes_per_launch": lm_bytes, "launch_ms": round(lm_ms, 5),
                    "frac": round(lm_bw / HBM_PEAK, 4), "cold_launch_ms": round(lm_cold_ms, 5),
                    "cold_frac": round(lm_bytes / (lm_cold_ms * 1e-3) / HBM_PEAK, 4),
                    "traffic": traffic.get("lm_head_traffic_bytes_per_launch")},
        "verify": {"M": M, "ms": round(ver_ms, 4), "bytes": int(ver_bytes),
                   "GB/s": round(ver_bw / 1e9, 1), "frac_of_peak": round(ver_bw / HBM_PEAK, 4),
                   "cpu_reference_ms": cpu["verify_ms"] if cpu else None, "sweep": sweep},
        "prefill": {"tokens": len(prompt) - 1, "s": round(prefill_s, 4),
                    "tok_s": round((len(prompt) - 1) / prefill_s, 1),
                    "note": "lz_forward_batch_capture in 512-row matrix-core chunks + MTP prefill + first capture",
                    "cpu_reference_s": cpu["prefill_s"] if cpu else None},
        "round": {"alpha": round(float(na.sum()) / (k * args.steps), 4),
                  "tokens_per_round": round(n_tok / args.steps, 4),
                  "bytes_per_round": int(mean_round),
                  "roofline_tok_s": round(roof_toks, 1),
                  "frac_of_roofline": round(value / roof_toks, 4),
                  "mean_distinct_experts": round(float(experts.mean()), 2)},
        "launch_floor": floor,
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(out))
    eng.close()


def bench_parity(eng, prompt, k, cpu):
    """The benched workload's own output against the reference: a fresh
    session on the same prompt, greedy rounds at the same k on the device
    (the timed path), and its first tokens compared with the tokens the
    reference engine's float-oracle build emitted in the CPU baseline's run
    (same model, prompt and k).  None when the CPU leg did not run."""
    import numpy as np
    if not cpu or "tokens" not in cpu.get("oracle_mode", {}):
        return None
    want = [int(t) for t in cpu["oracle_mode"]["tokens"]]
    first = eng.session_start(prompt)
    toks = [int(first)]
    while len(toks) < len(want):
        t, _, _ = eng.greedy_rounds(k, 1)
        toks.extend(int(x) for x in t)
    got = toks[:len(want)]
    bad = [i for i in range(len(want)) if got[i] != want[i]]
    return {"reference": "oracle/_ref/l98ref_oracle (the reference engine built from its sources, float-oracle "
                         "mode), same model, prompt and k",
            "tokens_compared": len(want), "identical": not bad, "first_divergence": bad[0] if bad else None,
            "gpu_tokens": got, "reference_tokens": want,
            "shipping_build_tokens": [int(t) for t in cpu.get("ship_tokens", [])]}


if __name__ == "__main__":
    main()
