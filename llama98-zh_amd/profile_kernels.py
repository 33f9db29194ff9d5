#!/usr/bin/env python3
"""Dispatches for the HBM byte counters of the round's kernels.

On the configs[1] model after a short prefill, runs `--iters` launches each
of (l98_time_kernel modes):
  0  the tied lm_head GEMV at M = k+1 = 4 token rows (back to back);
  4  the RMSNorm-prologue GEMV of every KDA layer's input projections;
  5  the same for the attention layers' inputs;
  6  the same for every layer's MoE input (4-6 back to back, in layer
     order);
  2  a device copy of the lm_head's vocab x hidden int8 bytes, the
     calibration kernel (its FETCH_SIZE and WRITE_SIZE per dispatch stand
     for a known byte count).
then 8 greedy rounds at k = 3 launched kernel by kernel (the verify's
KDA steps and routed experts) and prints one "SHAPES {json}" line: the
algorithmic bytes per launch of each kernel (bench.py's formulas), the
rounds' mean distinct experts per layer, the hipEvent timings above and the
sha256 of the kernel sources.  Meant to run under

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT -o pmc -- python3 llama98-zh_amd/profile_kernels.py
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d OUT -o pmc -- python3 llama98-zh_amd/profile_kernels.py

and, for the rocprof durations,

    rocprofv3 --kernel-trace --stats --output-format csv -d OUT -o tr -- python3 llama98-zh_amd/profile_kernels.py

all three summarized by llama98-zh_amd/trafficsum.py.

With --launch-floor it times the launch floor instead (l98_time_kernel
modes 7-10: chains of 64 dependent launches of an empty kernel of 1 and 256
blocks and of a 256-block kernel whose blocks read the M x hidden floats the
previous launch wrote, as a HIP graph and, for the empty 256-block kernel,
launched on the stream without a graph), printing microseconds per launch;
under `rocprofv3 --kernel-trace --stats` the probes' dispatches show as
k_nop and k_handoff.

With --prefill it runs two 512-token session starts instead (the prefill's
matrix-core GEMMs, k_mfma_q8, for the MFMA counters:
    rocprofv3 --pmc SQ_INSTS_VALU_MFMA_MOPS_I8 SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE \
        --output-format csv -d OUT -o pmc -- python3 llama98-zh_amd/profile_kernels.py --prefill
).
"""
import argparse
import os
import sys
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--model-dir", default=os.path.join(tempfile.gettempdir(), "l98_models"))
    ap.add_argument("--prefill", action="store_true", help="two 512-token session starts")
    ap.add_argument("--launch-floor", action="store_true", help="dependent-launch chains (modes 7-10)")
    args = ap.parse_args()
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    mdir = os.path.join(args.model_dir, "base")
    pkg.ensure_model(mdir, 1, seed=1234)
    eng = pkg.Engine(mdir)
    if args.prefill:
        for r in range(2):
            eng.reset()
            eng.session_start(pkg.prompt_tokens(0, 512, eng.V))
            print(f"prefill {r} done", flush=True)
        eng.close()
        return
    eng.session_start(pkg.prompt_tokens(0, 32, eng.V))
    if args.launch_floor:
        for which, name in ((7, "graph, empty kernel, 1 block"), (8, "graph, empty kernel, 256 blocks"),
                            (9, "graph, 256 blocks reading the previous launch's 4 x hidden floats"),
                            (10, "stream, empty kernel, 256 blocks"),
                            (11, "graph, mode 9 plus a last-block reduction per 8 blocks")):
            us = eng.time_kernel(which, 4, args.iters) * 1e3
            print(f"mode {which} ({name}): {us:.3f} us/launch", flush=True)
        # per-CU streaming: the same bytes per launch over few fat blocks or
        # many thin ones
        for blocks, threads, kb in ((16, 1024, 384), (24, 1024, 384), (32, 1024, 192), (64, 1024, 96),
                                    (64, 256, 96), (128, 256, 48), (256, 256, 24), (256, 256, 32),
                                    (256, 1024, 256), (2048, 256, 32)):
            us = eng.time_stream(blocks, threads, kb)
            print(f"stream {blocks} blocks x {threads} threads x {kb} KiB: {us:.3f} us/launch, "
                  f"{blocks * kb * 1024 / (us * 1e-6) / 1e9:.0f} GB/s, "
                  f"{kb * 1024 / (us * 1e-6) / 1e9:.1f} GB/s per block", flush=True)
        eng.close()
        return
    import json
    import numpy as np
    import bench
    cfg = eng.cfg
    M = 4
    timing = {}
    for which, name in ((0, "lm_head"), (4, "kda input"), (5, "attention input"), (6, "moe input"), (2, "copy")):
        ms = eng.time_kernel(which, M, args.iters)
        timing[name] = ms * 1e3
        print(f"mode {which} ({name}, M={M}): {ms * 1e3:.3f} us/launch (hipEvent, back to back)", flush=True)
    # greedy rounds at k = 3 launched kernel by kernel (the verify's KDA steps,
    # routed experts, attention, o_proj and tail GEMVs), with the distinct
    # experts each round's verify streamed
    eng.session_start(pkg.prompt_tokens(0, 64, eng.V))
    rounds = 8
    _, _, _, experts, _ = eng.greedy_rounds(3, rounds, use_graph=False, detail=True)
    mean_experts = float(np.mean(experts)) / cfg.n_layers
    up, down = bench.moe_bytes(cfg, M, mean_experts)
    V, d = cfg.vocab_size, cfg.hidden_size
    shapes = {
        "M": M, "rounds": rounds, "copy_bytes": V * d, "n_layers": cfg.n_layers,
        "n_kda_layers": cfg.n_linear_layers,
        "kda_instance": f"k_kda_step<{cfg.lin_k_head_dim}, {cfg.conv_kernel}, {M}>",
        "norm_gemv": [{"launch": n, "mode": mo, "per_round": pr, "bytes": b}
                      for n, mo, pr, b in bench.norm_gemv_shapes(cfg, M)],
        "lm_head_bytes": V * d + 4 * V + M * d + 4 * M * d // 32 + 4 * M * V,
        "kda_step_bytes": bench.kda_step_bytes(cfg, M),
        "moe_up_bytes": up, "expert_gemv_bytes": down, "mean_distinct_experts_per_layer": mean_experts,
        "hipevent_us": timing,
        "kernel_sources_sha256": bench.sources_sha(bench.TRAFFIC_SOURCES),
    }
    print("SHAPES " + json.dumps(shapes), flush=True)
    eng.close()


if __name__ == "__main__":
    main()
