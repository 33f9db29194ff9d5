#!/usr/bin/env python3
"""Dispatches for the HBM byte counters of the tied lm_head GEMV.

Runs, on the configs[1] model after a short prefill, `--iters` launches of
the lm_head GEMV at M = k+1 = 4 token rows and `--iters` device copies of
the same vocab x hidden int8 bytes (the calibration kernel: its FETCH_SIZE
and WRITE_SIZE per dispatch are the known byte count).  Meant to run under

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT -o pmc -- python3 llama98-zh_amd/profile_lmhead.py
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d OUT -o pmc -- python3 llama98-zh_amd/profile_lmhead.py

and summarized by llama98-zh_amd/pmcsum.py.
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
    args = ap.parse_args()
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    mdir = os.path.join(args.model_dir, "base")
    pkg.ensure_model(mdir, 1, seed=1234)
    eng = pkg.Engine(mdir)
    eng.session_start(pkg.prompt_tokens(0, 32, eng.V))
    lm_ms = eng.time_kernel(0, 4, args.iters)
    cp_ms = eng.time_kernel(2, 4, args.iters)
    nbytes = eng.V * eng.d
    print(f"lm_head M=4: {lm_ms * 1e3:.2f} us/launch; copy of {nbytes} B: {cp_ms * 1e3:.2f} us/launch",
          flush=True)
    eng.close()


if __name__ == "__main__":
    main()
