#!/usr/bin/env python3
"""HBM traffic and rocprof durations of the round's kernels on configs[1]
(M = 4 verify rows), from three rocprofv3 runs of profile_kernels.py and
one without a profiler (its hipEvent timings, which the tracer inflates):

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT/fetch -o pmc -- python3 llama98-zh_amd/profile_kernels.py
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d OUT/write -o pmc -- python3 llama98-zh_amd/profile_kernels.py
    rocprofv3 --kernel-trace --stats --output-format csv -d OUT/trace -o tr -- \\
        python3 llama98-zh_amd/profile_kernels.py > OUT/profile_kernels.log
    python3 llama98-zh_amd/profile_kernels.py > OUT/plain.log
    python3 llama98-zh_amd/trafficsum.py --fetch OUT/fetch/pmc_counter_collection.csv \\
        --write OUT/write/pmc_counter_collection.csv --trace OUT/trace/tr_kernel_trace.csv \\
        --log OUT/profile_kernels.log --plain OUT/plain.log

FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are scaled by what they read
for the calibration copy of a known byte count; the algorithmic bytes per
launch come from profile_kernels.py's SHAPES line (bench.py's formulas).
Prints markdown, ending with the lines bench.py reads.
"""
import argparse
import collections
import csv
import json


def short(name):
    return name.split("(")[0].replace("void ", "").strip()


def load_counters(path):
    """Counter value per dispatch id: (kernel, grid size in threads, value)."""
    with open(path, newline="") as f:
        return {int(r["Dispatch_Id"]): (short(r["Kernel_Name"]), int(r["Grid_Size"]), float(r["Counter_Value"]))
                for r in csv.DictReader(f)}


def load_trace(path):
    """Per dispatch id: (kernel, grid x, grid y, grid size, duration us)."""
    out = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            x, y, z = int(r["Grid_Size_X"]), int(r["Grid_Size_Y"]), int(r["Grid_Size_Z"])
            out[int(r["Dispatch_Id"])] = (short(r["Kernel_Name"]), x, y, x * y * z,
                                          (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3)
    return out


def join(trace, fetch, write):
    """The three runs replay one deterministic dispatch sequence: the
    counter rows join the trace rows by dispatch id (kernel and grid size
    checked).  Returns {(kernel, grid x, grid y): [(fetch KiB, write KiB, us)]}."""
    if not (trace.keys() == fetch.keys() == write.keys()):
        raise SystemExit("the runs dispatched different sequences")
    groups = collections.defaultdict(list)
    for i, (name, x, y, g, us) in trace.items():
        if fetch[i][:2] != (name, g) or write[i][:2] != (name, g):
            raise SystemExit(f"dispatch {i}: {fetch[i][:2]} / {write[i][:2]} against {(name, g)} in the trace")
        groups[(name, x, y)].append((fetch[i][2], write[i][2], us))
    return groups


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--trace", required=True)
    ap.add_argument("--log", required=True, help="the traced run's output")
    ap.add_argument("--plain", required=True, help="the output of a run without a profiler")
    args = ap.parse_args()

    def shapes_of(path):
        for line in open(path):
            if line.startswith("SHAPES "):
                return json.loads(line[7:])
        raise SystemExit(f"no SHAPES line in {path}")
    shapes, plain = shapes_of(args.log), shapes_of(args.plain)
    if plain["kernel_sources_sha256"] != shapes["kernel_sources_sha256"]:
        raise SystemExit("the runs measured different kernel sources")
    groups = join(load_trace(args.trace), load_counters(args.fetch), load_counters(args.write))

    def mean(keys, j):
        v = [d[j] for k in keys for d in groups[k]]
        return sum(v) / len(v)
    copy_key = max((k for k in groups if k[0].startswith("__amd_rocclr_copyBuffer")), key=lambda k: k[1] * k[2])
    cb = shapes["copy_bytes"]
    kf = cb / (mean([copy_key], 0) * 1024.0)
    kw = cb / (mean([copy_key], 1) * 1024.0)
    print("### Calibration\n")
    print(f"The copy of {cb:,} bytes (`{copy_key[0]}`, grid {copy_key[1]}) reads FETCH_SIZE "
          f"{mean([copy_key], 0):.1f} KiB and WRITE_SIZE {mean([copy_key], 1):.1f} KiB per dispatch: one FETCH_SIZE "
          f"KiB stands for {kf:.3f} KiB read, one WRITE_SIZE KiB for {kw:.3f} KiB written.\n")
    M = shapes["M"]
    ng = {s["launch"]: s for s in shapes["norm_gemv"]}
    # the lm_head is the pre-quantized GEMV launch with the most tiles
    lm_x = max(k[1] for k in groups if k[0].startswith(f"k_gemv_q8<{M}, 0,"))
    # (label, kernel name prefix, predicate on (grid x, grid y), algorithmic bytes, launches per round)
    rows = [
        ("KDA layer input: RMSNorm GEMV q/k/v/f_a/b/g", f"k_gemv_q8<{M}, 4,", lambda gx, gy: gy == 6,
         ng["kda input"]["bytes"], ng["kda input"]["per_round"]),
        ("attention layer input: RMSNorm GEMV q/k/v", f"k_gemv_q8<{M}, 4,", lambda gx, gy: gy == 3,
         ng["attention input"]["bytes"], ng["attention input"]["per_round"]),
        ("MoE input: RMSNorm GEMV router/latent/shared", f"k_gemv_q8<{M}, 4,", lambda gx, gy: gy == 4,
         ng["moe input"]["bytes"], ng["moe input"]["per_round"]),
        ("tied lm_head GEMV (vocab rows)", f"k_gemv_q8<{M}, 0,", lambda gx, gy: gx == lm_x,
         shapes["lm_head_bytes"], 1),
        ("KDA token step", shapes["kda_instance"], lambda gx, gy: True, shapes["kda_step_bytes"], shapes["n_kda_layers"]),
        ("routed experts w1 / w3 with routing", f"k_moe_up<{M},", lambda gx, gy: True,
         shapes["moe_up_bytes"], shapes["n_layers"]),
        ("routed experts w2", f"k_expert_gemv<{M},", lambda gx, gy: True, shapes["expert_gemv_bytes"],
         shapes["n_layers"]),
    ]
    print("### Per launch\n")
    print("| launch | kernel | grid (x threads, y) | dispatches | read B | written B | traffic B | algorithmic B | "
          "traffic / alg | rocprof mean us | alg GB/s | of 8 TB/s |")
    print("|---|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|")
    out = {}
    for label, prefix, pred, alg, per_round in rows:
        keys = sorted(k for k in groups if k[0].startswith(prefix) and pred(k[1], k[2]))
        if not keys:
            print(f"| {label} | `{prefix}…` | | 0 | | | | {alg:,.0f} | | | | |")
            continue
        # every dispatch of those shapes (the experts' launches vary grid x with the groups)
        n = sum(len(groups[k]) for k in keys)
        rd, wr, tus = mean(keys, 0) * 1024 * kf, mean(keys, 1) * 1024 * kw, mean(keys, 2)
        names = sorted({k[0] for k in keys})
        gtxt = ", ".join(f"{k[1]} x {k[2]}" for k in keys[:2]) + (f" (+{len(keys) - 2} more)" if len(keys) > 2 else "")
        print(f"| {label} | {', '.join('`' + x + '`' for x in names)} | {gtxt} | {n} | {rd:,.0f} | {wr:,.0f} | "
              f"{rd + wr:,.0f} | {alg:,.0f} | {(rd + wr) / alg:.3f} | {tus:.2f} | {alg / (tus * 1e-6) / 1e9:.0f} | "
              f"{alg / (tus * 1e-6) / 8e12:.4f} |")
        out[label] = (rd + wr, alg, tus, per_round)
    norm = [v for k, v in out.items() if "RMSNorm GEMV" in k]
    print()
    if len(norm) == 3:
        traffic = sum(t * pr for t, a, u, pr in norm)
        alg = sum(a * pr for t, a, u, pr in norm)
        us = sum(u * pr for t, a, u, pr in norm)
        frac = alg / (us * 1e-6) / 8e12
        ev = plain["hipevent_us"]
        us_ev = sum(ev[n] * ng[n]["per_round"] for n in ("kda input", "attention input", "moe input"))
        print(f"RMSNorm-prologue GEMV over one round's {sum(pr for *_, pr in norm)} launches: "
              f"{alg:,.0f} algorithmic bytes, {traffic:,.0f} bytes of traffic ({traffic / alg:.3f}); "
              f"{us:.1f} us by the rocprof means ({alg / (us * 1e-6) / 1e9:.0f} GB/s, {frac:.4f} of 8 TB/s), "
              f"{us_ev:.1f} us by the hipEvent timing, without a profiler, of the same launch shapes back to back "
              f"({alg / (us_ev * 1e-6) / 8e12:.4f}).\n")
        print(f"hipEvent timings without a profiler (us per launch, l98_time_kernel modes 0, 4, 5, 6, 2): "
              + ", ".join(f"{k} {v:.3f}" for k, v in ev.items()) + "\n")
        print(f"Mean distinct experts per MoE layer over the profiled rounds: "
              f"{shapes['mean_distinct_experts_per_layer']:.2f}.\n")
        print(f"norm_gemv_traffic_bytes_per_round: {traffic:.0f}")
        print(f"norm_gemv_rocprof_us_per_round: {us:.1f}")
        print(f"norm_gemv_rocprof_frac: {frac:.4f}")
        print(f"norm_gemv_hipevent_us_per_round: {us_ev:.1f}")
        print(f"norm_gemv_hipevent_frac: {alg / (us_ev * 1e-6) / 8e12:.4f}")
    lm = out.get("tied lm_head GEMV (vocab rows)")
    if lm:
        print(f"lm_head_traffic_bytes_per_launch: {lm[0]:.0f}")
    print(f"kernel_sources_sha256: {shapes['kernel_sources_sha256']}")


if __name__ == "__main__":
    main()
