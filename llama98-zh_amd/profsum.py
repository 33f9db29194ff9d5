"""Summarizes a rocprofv3 kernel trace of the speculative-decoding path.

    rocprofv3 --kernel-trace --stats --output-format csv -d OUT -o prof -- python3 bench.py --no-graph ...
    python3 llama98-zh_amd/profsum.py OUT/prof_kernel_trace.csv [--vocab V]
    python3 llama98-zh_amd/profsum.py OUT/prof_kernel_trace.csv --verify-batches N

With --verify-batches N (a trace of `bench.py --config 4 --no-graph`, whose
last N dispatch runs are the batched verifies), prints instead the whole
run and the mean of the last N batched verifies, each starting at its
many-row k_embed (the batch's token rows in one launch).

Prints, as markdown:
  * every kernel of the whole run (calls, total, mean, min, max);
  * one round of the timed loop: the dispatches after one k_accept up to and
    including the next (the last complete round), grouped by kernel;
  * the tied lm_head GEMV launches (k_gemv_q8 dispatches whose grid covers
    `vocab` rows), whose mean duration is the figure bench.py's roofline
    uses;
  * the prompt's many-row path: the dispatches from the last run of
    many-row k_embed dispatches (one per part of a split chunk) to the last
    many-row kernel (k_mfma_q8, k_kda_post, k_attn_prep) before the first
    k_accept, i.e. the session's prefill and MTP prefill.
"""
import argparse
import collections
import csv


def load(path):
    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            rows.append((r["Kernel_Name"], int(r["Start_Timestamp"]), int(r["End_Timestamp"]),
                         int(r["Grid_Size_X"]), int(r["Workgroup_Size_X"]), int(r.get("Grid_Size_Y") or 1)))
    rows.sort(key=lambda r: r[1])
    return rows


def short(name):
    return name.split("(")[0].replace("void ", "")


def table(groups, title, total_label):
    out = [f"### {title}", "", "| kernel | calls | total us | mean us | min us | max us | % |",
           "|---|---:|---:|---:|---:|---:|---:|"]
    tot = sum(sum(v) for v in groups.values())
    for k, v in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        out.append(f"| `{k}` | {len(v)} | {sum(v) / 1e3:.1f} | {sum(v) / len(v) / 1e3:.2f} | {min(v) / 1e3:.2f} | "
                   f"{max(v) / 1e3:.2f} | {100 * sum(v) / tot:.1f} |")
    out.append(f"| **{total_label}** | {sum(len(v) for v in groups.values())} | {tot / 1e3:.1f} | | | | |")
    return "\n".join(out)


def counters(paths):
    """Mean per dispatch of every counter in rocprofv3 --pmc CSVs, by kernel."""
    vals = collections.defaultdict(lambda: collections.defaultdict(list))
    for p in paths:
        with open(p, newline="") as f:
            for r in csv.DictReader(f):
                vals[short(r["Kernel_Name"]).strip()][r["Counter_Name"]].append(float(r["Counter_Value"]))
    for k, cs in vals.items():
        print(f"### `{k}`")
        print()
        print("| counter | dispatches | mean per dispatch |")
        print("|---|---:|---:|")
        for c in sorted(cs):
            v = cs[c]
            print(f"| {c} | {len(v)} | {sum(v) / len(v):.0f} |")
        print()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("trace", nargs="?")
    ap.add_argument("--counters", nargs="+", help="rocprofv3 --pmc counter CSVs: per-kernel means instead")
    ap.add_argument("--vocab", type=int, default=65536)
    ap.add_argument("--gemv-rows-per-block", type=int, default=32,
                    help="rows per GEMV tile at the lm_head's input width")
    ap.add_argument("--verify-batches", type=int, default=0, help="summarize the last N batched verifies")
    a = ap.parse_args()
    if a.counters:
        counters(a.counters)
        return
    rows = load(a.trace)
    whole = collections.defaultdict(list)
    for n, s, e, g, w, *_ in rows:
        whole[short(n)].append(e - s)
    print(table(whole, "Whole run", "all dispatches"))
    if a.verify_batches:
        emb = [i for i, r in enumerate(rows) if short(r[0]) == "k_embed" and r[5] >= 16]
        nb = min(a.verify_batches, len(emb))
        seg = rows[emb[-nb]:]
        grp = collections.defaultdict(list)
        for n, s, e, g, w, *_ in seg:
            grp[short(n)].append(e - s)
        span = (seg[-1][2] - seg[0][1]) / nb
        per = {k: [x / nb for x in v] for k, v in grp.items()}
        print()
        print(f"### Batched verify: the last {nb} (per verify: calls / {nb}, total / {nb}; span {span / 1e3:.1f} us "
              f"per verify, kernels launched one by one under the tracer)")
        print()
        print("| kernel | calls | total us | mean us | % |")
        print("|---|---:|---:|---:|---:|")
        tot = sum(sum(v) for v in grp.values())
        for k, v in sorted(grp.items(), key=lambda kv: -sum(kv[1])):
            print(f"| `{k}` | {len(v) / nb:g} | {sum(v) / nb / 1e3:.1f} | {sum(v) / len(v) / 1e3:.2f} | "
                  f"{100 * sum(v) / tot:.1f} |")
        print(f"| **verify** | {sum(len(v) for v in grp.values()) / nb:g} | {tot / nb / 1e3:.1f} | | |")
        return
    acc = [i for i, r in enumerate(rows) if short(r[0]) == "k_accept"]
    if len(acc) >= 2:
        seg = rows[acc[-2] + 1:acc[-1] + 1]
        grp = collections.defaultdict(list)
        for n, s, e, g, w, *_ in seg:
            grp[short(n)].append(e - s)
        span = seg[-1][2] - seg[0][1]
        print()
        print(table(grp, f"One round (last complete round; span {span / 1e3:.1f} us without graph replay)",
                    "round"))
    first_acc = acc[0] if acc else len(rows)
    # the many-row embeddings (a grid of at least 16 token rows in y) before
    # it; a prefill whose chunk runs in parts on several streams has one per
    # part, close together: take the first of the last such run (embeddings
    # less than 1 ms apart)
    emb = [i for i, r in enumerate(rows[:first_acc]) if short(r[0]) == "k_embed" and r[5] >= 16]
    while len(emb) >= 2 and rows[emb[-1]][1] - rows[emb[-2]][1] < 1_000_000:
        emb = emb[:-2] + emb[-2:-1]
    emb = emb[-1:]
    wide = [i for i, r in enumerate(rows[:first_acc])
            if short(r[0]).startswith(("k_mfma_q8", "k_kda_post", "k_attn_prep"))]
    if emb and wide and wide[-1] > emb[0]:
        seg = rows[emb[0]:wide[-1] + 1]
        grp = collections.defaultdict(list)
        for n, s, e, g, w, *_ in seg:
            grp[short(n)].append(e - s)
        span = seg[-1][2] - seg[0][1]
        print()
        print(table(grp, f"Prompt prefill and MTP prefill (span {span / 1e3:.1f} us)", "prefill"))
    tiles = (a.vocab + a.gemv_rows_per_block - 1) // a.gemv_rows_per_block
    lm = collections.defaultdict(list)
    for n, s, e, g, w, *_ in rows:
        if short(n).startswith("k_gemv_q8") and w > 0 and g // w == tiles:
            lm[short(n)].append(e - s)
    if lm:
        print()
        print(table(lm, f"Tied lm_head GEMV ({a.vocab} rows, {tiles} tiles)", "lm_head"))


if __name__ == "__main__":
    main()
