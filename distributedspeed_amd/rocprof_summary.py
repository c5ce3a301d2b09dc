"""Summarise rocprofv3 CSV output of the step's kernels.

    python -m distributedspeed_amd.rocprof_summary \
        --trace DIR (from --kernel-trace --stats) \
        --fetch DIR (from --pmc FETCH_SIZE) --write DIR (from --pmc WRITE_SIZE) \
        --numel N --out-md FILE --out-json FILE --command "..." [--title T --intro TEXT]

Byte counters are scaled by what they report for a plain copy kernel of
known size in the same run (the 1 GiB fp32 copy `bench.py --profile-kernels`
issues; it appears as __amd_rocclr_copyBuffer), so FETCH_SIZE/WRITE_SIZE
become HBM bytes per dispatch whatever unit or channel coverage the counter
has on this device.
"""
from __future__ import annotations

import argparse
import collections
import csv
import glob
import json
import os

KERNELS = {"k2_adamw_flat": 28, "k2_adamw_fold": 28, "k2_adamw_fold_dev": 28, "k1_unscale_norm": 2, "k0_finalize": 0,
           "k0_finalize_dev": 0, "k2_adamw_multi": 28, "k3_adamw_fold": 28, "k1_unscale_norm_multi": 2,
           "k2_traffic_probe": 28}

# The launches of one step, by form: K1, K0 (None where the finalize is
# folded into K2) and K2 (which may repeat: K2 over a partition above 2^26
# elements is several consecutive dispatches, and the folded form has one
# per parameter group). The folded K2 reading its group block from device
# memory (the graph form) is told apart by its template argument.
STEP_FORMS = {
    "flat, eager, two launches (K0 folded into K2)": ("k1_unscale_norm", None, "k2_adamw_fold"),
    "flat, HIP graph replay, two launches (K0 folded into K2)": ("k1_unscale_norm", None, "k2_adamw_fold_dev"),
    "flat, eager, three launches": ("k1_unscale_norm", "k0_finalize", "k2_adamw_flat"),
    "flat, HIP graph replay, three launches": ("k1_unscale_norm", "k0_finalize_dev", "k2_adamw_flat"),
    "ragged (chunk table)": ("k1_unscale_norm_multi", "k0_finalize", "k2_adamw_multi"),
    "ragged, two launches (K0 folded into K3)": ("k1_unscale_norm_multi", None, "k3_adamw_fold"),
}
# Above the fold's bound the folded K2 is a step's first part and K2's other
# parts follow it: they belong to the step, and to its K2 column.
STEP_TAIL = {"k2_adamw_fold": "k2_adamw_flat", "k2_adamw_fold_dev": "k2_adamw_flat"}
COPY_NAME = "__amd_rocclr_copyBuffer"
COPY_BYTES = 1 << 30


def _short(name: str) -> str | None:
    if "k2_adamw_fold<" in name and "DsxGroupsDev const*>" in name:
        return "k2_adamw_fold_dev"
    for k in sorted(KERNELS, key=len, reverse=True):
        if k in name:
            return k
    if COPY_NAME in name:
        return "copy"
    return None


def _csv(dirname: str, suffix: str) -> str:
    hits = glob.glob(os.path.join(dirname, "**", f"*{suffix}"), recursive=True)
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {dirname}")
    return hits[0]


def kernel_stats(trace_dir: str) -> dict:
    out = {}
    for r in csv.DictReader(open(_csv(trace_dir, "kernel_stats.csv"))):
        k = _short(r["Name"])
        if k and k != "copy":
            out[k] = {"calls": int(r["Calls"]), "avg_ns": float(r["AverageNs"]), "min_ns": float(r["MinNs"]),
                      "max_ns": float(r["MaxNs"]), "pct": float(r["Percentage"]), "name": r["Name"]}
    return out


def counter_per_dispatch(pmc_dir: str) -> dict:
    """{kernel: [KiB per dispatch, ...]} summed over the counter's instances."""
    per = collections.defaultdict(float)
    names = {}
    for r in csv.DictReader(open(_csv(pmc_dir, "counter_collection.csv"))):
        k = _short(r["Kernel_Name"])
        if k is None:
            continue
        if k == "copy" and int(r["Grid_Size"]) < 4096:
            continue  # small copies (parameter uploads), not the calibration copy
        per[(k, int(r["Dispatch_Id"]))] += float(r["Counter_Value"])
        names[k] = r["Counter_Name"]
    out = collections.defaultdict(list)
    for (k, _), v in sorted(per.items(), key=lambda x: x[0][1]):
        out[k].append(v)
    return dict(out)


# Kernels the library issues as consecutive dispatches over parts of the
# partition (dsx_set_tuning_k2_chunk): one call of the entry point is that
# many dispatches, and the figures below are per call.
PARTED = ("k2_adamw_flat", "k2_traffic_probe")


def parts_per_call(numel: int, part_elems: int) -> int:
    return -(-numel // part_elems) if part_elems > 0 and numel > part_elems else 1


def call_spans(trace_dir: str, kernel: str, parts: int) -> list[int]:
    """Per call of a parted kernel, in ns: from its first dispatch's start to
    its last dispatch's end in the kernel trace, gaps between the dispatches
    included (what events recorded around the call measure). The kernel's
    dispatches are taken in time order, `parts` to a call."""
    rows = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
                  for r in csv.DictReader(open(_csv(trace_dir, "kernel_trace.csv")))
                  if _short(r["Kernel_Name"]) == kernel)
    return [rows[i + parts - 1][1] - rows[i][0] for i in range(0, len(rows) - parts + 1, parts)]


def summarise(trace_dir, fetch_dir, write_dir, numel, part_elems: int = 1 << 26,
              kernel_numel: dict | None = None, timed_calls: int = 0) -> dict:
    """kernel_numel: elements one call of a kernel covers where that is not
    `numel` (a ragged list whose large tensors step through K2 and the rest
    through K3). timed_calls: for the parted kernels, the mean span is also
    taken over the last this many calls (a benchmark's timed calls, after
    its warm-up)."""
    kernel_numel = kernel_numel or {}
    stats = kernel_stats(trace_dir)
    fetch = counter_per_dispatch(fetch_dir)
    write = counter_per_dispatch(write_dir)
    # the calibration copies are the last three copy dispatches of the run
    # (earlier ones are the program's own copies, such as parameter clones)
    f_copy = sum(fetch["copy"][-3:]) / len(fetch["copy"][-3:])
    w_copy = sum(write["copy"][-3:]) / len(write["copy"][-3:])
    f_scale = COPY_BYTES / (f_copy * 1024)
    w_scale = COPY_BYTES / (w_copy * 1024)
    res = {"numel": int(numel), "fetch_scale": f_scale, "write_scale": w_scale,
           "copy_fetch_kib": f_copy, "copy_write_kib": w_copy, "part_elems": int(part_elems), "kernels": {}}
    for k, per_elt in KERNELS.items():
        if k not in fetch and k not in stats:
            continue
        kn = int(kernel_numel.get(k, numel))
        parts = parts_per_call(kn, part_elems) if k in PARTED else 1
        d = {"dispatches_per_call": parts, "numel": kn}
        if k in stats:
            # per call: the dispatches' own durations, without the gaps between them
            d.update(avg_ms=stats[k]["avg_ns"] * parts / 1e6, avg_dispatch_ms=stats[k]["avg_ns"] / 1e6,
                     calls=stats[k]["calls"] // parts, dispatches=stats[k]["calls"], pct=stats[k]["pct"])
        if k in fetch and k in write:
            fb = sum(fetch[k]) / len(fetch[k]) * 1024 * f_scale * parts
            wb = sum(write[k]) / len(write[k]) * 1024 * w_scale * parts
            d.update(fetch_bytes=fb, write_bytes=wb, hbm_bytes=fb + wb)
            if per_elt:
                d["algorithmic_bytes"] = per_elt * kn
                d["traffic_over_algorithmic"] = (fb + wb) / (per_elt * kn)
        if "avg_ms" in d and per_elt:
            d["achieved_gbs"] = per_elt * kn / (d["avg_ms"] * 1e-3) / 1e9
            d["frac_of_8tbs"] = d["achieved_gbs"] / 8000.0
        if k in PARTED and k in stats and per_elt:
            spans = call_spans(trace_dir, k, parts)
            if spans:
                tail = spans[-timed_calls:] if 0 < timed_calls <= len(spans) else spans
                d["span_calls"] = len(tail)
                d["span_ms"] = sum(tail) / len(tail) / 1e6
                d["span_achieved_gbs"] = per_elt * kn / (d["span_ms"] * 1e-3) / 1e9
                d["span_frac_of_8tbs"] = d["span_achieved_gbs"] / 8000.0
        res["kernels"][k] = d
    k2 = res["kernels"].get("k2_adamw_flat", {})
    res["k2_hbm_bytes_per_launch"] = k2.get("hbm_bytes")
    res["k1_hbm_bytes_per_launch"] = res["kernels"].get("k1_unscale_norm", {}).get("hbm_bytes")
    return res


def step_chains(trace_dir: str) -> dict:
    """Each step's launches found in the kernel trace (--kernel-trace CSV),
    by form: per step the kernels' own durations, their sum (the time the
    GPU spends in the step's kernels), the gaps between them, and the period
    from one step's first kernel to the next step's (all in microseconds,
    medians over the steps found)."""
    rows = []
    for r in csv.DictReader(open(_csv(trace_dir, "kernel_trace.csv"))):
        rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), _short(r["Kernel_Name"])))
    rows.sort()
    med = lambda xs: sorted(xs)[len(xs) // 2] / 1e3 if xs else None  # noqa: E731  (ns -> us)
    out = {}
    for form, full in STEP_FORMS.items():
        pat = [k for k in full if k is not None]
        steps, i = [], 0
        while i < len(rows):
            if all(i + q < len(rows) and rows[i + q][2] == k for q, k in enumerate(pat)):
                j = i + len(pat)
                while j < len(rows) and rows[j][2] in (pat[-1], STEP_TAIL.get(pat[-1])):
                    j += 1
                steps.append(rows[i:j])
                i = j
            else:
                i += 1
        if len(steps) < 3:  # a warm-up's launches, not a timed run of this form
            continue
        per = {}
        for k in full:
            ks = (k, STEP_TAIL.get(k))
            per[k or "k0 (folded)"] = (None if k is None else
                                       med([sum(e - s for s, e, n in st if n in ks) for st in steps]))
        busy = [sum(e - s for s, e, _ in st) for st in steps]
        span = [st[-1][1] - st[0][0] for st in steps]
        period = [steps[k + 1][0][0] - steps[k][0][0] for k in range(len(steps) - 1)]
        out[form] = {"steps": len(steps), "kernels_us": per, "kernel_busy_us": med(busy), "span_us": med(span),
                     "gaps_us": med([a - b for a, b in zip(span, busy)]), "period_us": med(period)}
    return out


def chains_markdown(res: dict, command: str, title: str, intro: str = "") -> str:
    lines = [f"# {title}", ""] + ([intro.strip(), ""] if intro.strip() else []) + [
             "Commands (run on one MI355X, from the repository root as $R):", "",
             "```", command.strip(), "```", "",
             "Per step, medians over the steps of each form in the trace, in microseconds: each kernel's "
             "duration (for K2 the sum of its dispatches), their sum (kernel-busy), the time from the first "
             "kernel's start to the last one's end (span), span minus kernel-busy (gaps), and the period from "
             "one step's first kernel to the next step's. The period under the tracer includes the tracer's "
             "own cost per dispatch.", "",
             "| form | steps | K1 | K0 | K2 | kernel-busy | span | gaps | period |", "|---|---|---|---|---|---|---|---|---|"]
    fmt = lambda x: "–" if x is None else f"{x:.2f}"  # noqa: E731
    for form, d in res.items():
        k = list(d["kernels_us"].values())
        lines.append(f"| {form} | {d['steps']} | {fmt(k[0])} | {fmt(k[1])} | {fmt(k[2])} | "
                     f"{d['kernel_busy_us']:.2f} | {d['span_us']:.2f} | {d['gaps_us']:.2f} | {fmt(d['period_us'])} |")
    return "\n".join(lines) + "\n"


def markdown(res: dict, command: str, title: str, intro: str = "") -> str:
    lines = [f"# {title}", ""] + ([intro.strip(), ""] if intro.strip() else []) + [
             "Commands (run on one MI355X, from the repository root as $R):", "",
             "```", command.strip(), "```", "",
             f"Byte-counter calibration: a {COPY_BYTES >> 20} MiB fp32 copy reads FETCH_SIZE "
             f"{res['copy_fetch_kib']:.1f} KiB and WRITE_SIZE {res['copy_write_kib']:.1f} KiB per dispatch, "
             f"so FETCH_SIZE is scaled by {res['fetch_scale']:.4f} and WRITE_SIZE by {res['write_scale']:.4f}.", "",
             f"n = {res['numel']:,} elements.", "",
             "Figures are per call of the entry point; K2 and its probe issue `dispatches / call` consecutive "
             "dispatches over parts of the partition, and `avg ms` is the sum of their durations (without the gaps "
             "between them).", "",
             "| kernel | elements / call | calls | dispatches / call | avg ms | algorithmic GB | achieved GB/s | % of 8 TB/s | HBM read GB | HBM write GB | traffic / algorithmic |",
             "|---|---|---|---|---|---|---|---|---|---|---|"]
    for k, d in res["kernels"].items():
        alg = d.get("algorithmic_bytes")
        lines.append("| {} | {:,} | {} | {} | {} | {} | {} | {} | {} | {} | {} |".format(
            k, d.get("numel", res["numel"]), d.get("calls", ""), d.get("dispatches_per_call", 1),
            f"{d['avg_ms']:.4f}" if "avg_ms" in d else "",
            f"{alg / 1e9:.3f}" if alg else "", f"{d['achieved_gbs']:.0f}" if "achieved_gbs" in d else "",
            f"{100 * d['frac_of_8tbs']:.1f}" if "frac_of_8tbs" in d else "",
            f"{d['fetch_bytes'] / 1e9:.3f}" if "fetch_bytes" in d else "",
            f"{d['write_bytes'] / 1e9:.3f}" if "write_bytes" in d else "",
            f"{d['traffic_over_algorithmic']:.4f}" if "traffic_over_algorithmic" in d else ""))
    spans = [(k, d) for k, d in res["kernels"].items() if "span_ms" in d]
    if spans:
        lines += ["", "The same calls timed as a benchmark's events time them: per call, from the first dispatch's "
                  "start to the last dispatch's end, gaps included (the mean over the last `calls` calls).", "",
                  "| kernel | calls | span ms | achieved GB/s | frac of 8 TB/s |", "|---|---|---|---|---|"]
        for k, d in spans:
            lines.append(f"| {k} | {d['span_calls']} | {d['span_ms']:.4f} | {d['span_achieved_gbs']:.0f} | "
                         f"{d['span_frac_of_8tbs']:.4f} |")
    b = res.get("bench_line")
    if b:
        rf = b.get("roofline", {})
        lines += ["", "The traced run's own bench line (events on the kernels' stream, same process):", "",
                  "| ms / step | % of 8 TB/s end to end | K1 ms | K0 ms | K2 ms | roofline.achieved GB/s | "
                  "roofline.frac |", "|---|---|---|---|---|---|---|",
                  "| {} | {} | {} | {} | {} | {} | {} |".format(
                      b.get("ms_per_step"), b.get("pct_of_8tbps_end_to_end"),
                      *(b.get("kernels_ms", {}).get(k) for k in ("k1_unscale_norm", "k0_finalize",
                                                                "k2_adamw_flat")),
                      rf.get("achieved"), rf.get("frac"))]
    return "\n".join(lines) + "\n"


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--trace", required=True)
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--numel", type=int)
    ap.add_argument("--chains", action="store_true",
                    help="summarise the trace's step launches (K1, K0, K2 per step) instead of the counters")
    ap.add_argument("--part-elems", type=int, default=1 << 26,
                    help="the library's K2 part size (dsx_set_tuning_k2_chunk; 0: one dispatch per call)")
    ap.add_argument("--out-md", required=True)
    ap.add_argument("--out-json", required=True)
    ap.add_argument("--command", default="")
    ap.add_argument("--title", default="rocprofv3 summary")
    ap.add_argument("--intro", default="", help="a paragraph placed under the title")
    ap.add_argument("--kernel-numel", action="append", default=[],
                    help="KERNEL=N: elements one call of KERNEL covers, where it is not --numel")
    ap.add_argument("--timed-calls", type=int, default=0,
                    help="take the parted kernels' mean span over the last this many calls")
    ap.add_argument("--bench-json", help="the traced run's bench.py output: its JSON line goes into the summary")
    a = ap.parse_args()
    if a.chains:
        res = step_chains(a.trace)
        with open(a.out_json, "w") as f:
            json.dump(res, f, indent=1)
        with open(a.out_md, "w") as f:
            f.write(chains_markdown(res, a.command, a.title, a.intro))
        print(json.dumps(res))
        return
    if not (a.fetch and a.write and a.numel):
        ap.error("--fetch, --write and --numel are required without --chains")
    kn = {k: int(v) for k, v in (x.split("=", 1) for x in a.kernel_numel)}
    res = summarise(a.trace, a.fetch, a.write, a.numel, a.part_elems, kn, a.timed_calls)
    if a.bench_json:
        lines = [x for x in open(a.bench_json).read().splitlines() if x.startswith("{")]
        if lines:
            b = json.loads(lines[-1])
            res["bench_line"] = {k: b.get(k) for k in ("ms_per_step", "pct_of_8tbps_end_to_end", "kernels_ms",
                                                       "roofline", "k2_traffic_probe")}
    with open(a.out_json, "w") as f:
        json.dump(res, f, indent=1)
    with open(a.out_md, "w") as f:
        f.write(markdown(res, a.command, a.title, a.intro))
    print(json.dumps({k: res[k] for k in ("k2_hbm_bytes_per_launch", "k1_hbm_bytes_per_launch", "fetch_scale")}))


if __name__ == "__main__":
    main()
