#!/usr/bin/env python3
"""Per-kernel mean of a rocprofv3 --pmc counter (FETCH_SIZE / WRITE_SIZE,
KiB per dispatch), per kernel name and grid, for the kernels and the
calibration copy that llama98-zh_amd/profile_kernels.py dispatches.

    python3 llama98-zh_amd/pmcsum.py OUT/pmc_counter_collection.csv [--vocab 65536 --hidden 1024]
"""
import argparse
import collections
import csv


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("csv")
    ap.add_argument("--vocab", type=int, default=65536)
    ap.add_argument("--hidden", type=int, default=1024)
    args = ap.parse_args()
    tot = collections.defaultdict(float)
    cnt = collections.defaultdict(int)
    with open(args.csv, newline="") as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"].split("(")[0].replace("void ", "")
            grid = int(r.get("Grid_Size", r.get("Grid_Size_X", 0)) or 0)
            key = (name, r["Counter_Name"], grid)
            tot[key] += float(r["Counter_Value"])
            cnt[key] += 1
    nbytes = args.vocab * args.hidden
    print(f"| kernel | grid | counter | dispatches | mean KiB | mean bytes | bytes / {nbytes} |")
    print("|---|---:|---|---:|---:|---:|---:|")
    for key in sorted(tot):
        name, ctr, grid = key
        mean = tot[key] / cnt[key]
        print(f"| `{name}` | {grid} | {ctr} | {cnt[key]} | {mean:.1f} | {mean * 1024:.0f} | "
              f"{mean * 1024 / nbytes:.3f} |")


if __name__ == "__main__":
    main()
