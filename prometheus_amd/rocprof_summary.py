"""Summaries of rocprofv3 CSV output for the committed profiles.

    python -m prometheus_amd.rocprof_summary stats DIR --cmd "..." [--bench-log LOG] -o OUT.md
    python -m prometheus_amd.rocprof_summary traffic FETCH_DIR WRITE_DIR --kernel NAME
        --cmd-fetch "..." --cmd-write "..." -o OUT.json
    python -m prometheus_amd.rocprof_summary mfma DIR --kernel NAME --cmd "..."
        [--algorithmic-flop F] -o OUT.json
    python -m prometheus_amd.rocprof_summary counters DIR --kernel NAME --cmd "..." -o OUT.md

``stats`` turns ``*_kernel_stats.csv`` (from ``--kernel-trace --stats``) into a
short markdown table.  ``traffic`` reads two ``--pmc`` runs (``FETCH_SIZE``,
then ``WRITE_SIZE``; both in KiB per dispatch) of a command that also ran
``bench.py --calib-copy`` (a plain elementwise fp32 copy of a known 1 GiB), and
scales the kernel's per-dispatch counters by ``known bytes / counted bytes``
of that copy, giving the HBM bytes one launch of the kernel moves.
``mfma`` reads one ``--pmc MfmaUtil MfmaFlopsBF16`` run (rocprofv3's derived
counters: MFMA busy cycles over GUI-active cycles times SIMDs, and
``SQ_INSTS_VALU_MFMA_MOPS_BF16 * 512``) and records their per-dispatch mean
for the kernel, beside its algorithmic flops.  ``counters`` reads any one
``--pmc`` run and tabulates the per-dispatch mean of every counter it holds
for the kernel (SQ counters are summed over the chip), with the LDS ratios.
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import statistics
import sys

CALIB_COPY_BYTES = 1 << 30
CALIB_KERNEL = "neg"  # torch.neg elementwise kernel launched by bench.py --calib-copy


def _one(pattern: str) -> str:
    hits = sorted(glob.glob(pattern, recursive=True))
    if not hits:
        raise FileNotFoundError(pattern)
    return hits[0]


def short_name(name: str) -> str:
    """Kernel name without return type and argument list (templates kept)."""
    name = re.sub(r"^void\s+", "", name).replace("(anonymous namespace)", "{anon}")
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            name = name[:i]
            break
    return name if len(name) <= 110 else name[:107] + "..."


def _bench_line(path: str) -> str:
    """One sentence with every leg's timing from a bench.py JSON line."""
    d = None
    for ln in open(path):
        if ln.startswith("{"):
            d = json.loads(ln)
    if d is None:
        return ""
    parts = [f"headline kernel_us (HIP events over the timed launches, per launch) = {d['kernel_us']:.1f}",
             f"value = {d['value']:.4g} {d['unit']}"]
    if d.get("bf16_out"):
        b = d["bf16_out"]
        parts.append(f"bf16-O kernel_us = {b['kernel_us']:.1f} (fp32-O {b['fp32_out_kernel_us_same_rounds']:.1f} "
                     f"in the same rounds)")
    for key in ("cfg3", "cfg2"):
        if d.get(key):
            c = d[key]
            extra = f", single-stage {c['single_stage']['kernel_us']:.1f}" if c.get("single_stage") else ""
            parts.append(f"{key} kernel_us = {c['kernel_us']:.1f} ({c['path']}{extra})")
    if d.get("decode"):
        parts.append(f"decode us_per_step = {d['decode']['us_per_step']:.1f}")
    for key, label in (("fp32_forward", "fp32 forward"), ("gated", "gated forward"), ("kda", "KDA forward")):
        if d.get(key):
            parts.append(f"{label} = {d[key]['ms_per_call']:.3f} ms")
    if d.get("kda") and d["kda"].get("per_token"):
        parts.append(f"KDA per-token = {d['kda']['per_token']['ms_per_call']:.3f} ms")
    if d.get("model_linear_attention"):
        m = d["model_linear_attention"]
        parts.append(f"model linear attention bf16 / fp32 = {m['bf16']['ms_per_call']:.3f} / "
                     f"{m['fp32']['ms_per_call']:.3f} ms")
    if d.get("backward"):
        b = d["backward"]
        parts.append(f"backward bf16 = {b['ms_per_call']:.3f} ms" +
                     (f", fp32 = {b['fp32']['ms_per_call']:.3f} ms" if b.get("fp32") else ""))
    return "bench.py line from the same run: " + "; ".join(parts) + "."


def stats(args) -> None:
    """Per-kernel durations.  With the kernel trace present, one row per (kernel, grid size),
    so that launches of one kernel at different shapes (cfg1 and a varlen batch, say)
    are told apart; otherwise rocprofv3's own per-kernel statistics."""
    out = ["# rocprofv3 kernel statistics", "", "Command:", "", "```", args.cmd, "```", ""]
    if args.bench_log:
        out += [_bench_line(args.bench_log), ""]
    hits = sorted(glob.glob(os.path.join(args.dir, "**", "*kernel_trace.csv"), recursive=True))
    if hits:
        groups: dict[tuple[str, int], list[float]] = {}
        with open(hits[0]) as f:
            for r in csv.DictReader(f):
                grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
                wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
                dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
                groups.setdefault((short_name(r["Kernel_Name"]), grid // max(wg, 1)), []).append(dur)
        total = sum(sum(v) for v in groups.values())
        rows = sorted(groups.items(), key=lambda kv: -sum(kv[1]))
        if args.prefix:
            rows = [kv for kv in rows if kv[0][0].startswith(args.prefix)]
            out += [f"Kernels named {args.prefix}* only (the rest are the bench's own torch set-up and "
                    f"reference work); total % is of every kernel's time.", ""]
        if args.skip:
            out += [f"`avg us` leaves out the first {args.skip} launches of a row that has more (the "
                    f"headline's warm-up, during which the shader clock ramps up); `avg all` is over every "
                    f"launch.", ""]
        out += ["| kernel | workgroups | calls | avg us | avg all | min us | max us | total % |",
                "|---|---:|---:|---:|---:|---:|---:|---:|"]
        for (name, n_wg), v in rows[: args.top]:
            w = v[args.skip:] if args.skip and len(v) > args.skip else v
            out.append(f"| `{name}` | {n_wg} | {len(v)} | {sum(w) / len(w):.1f} | {sum(v) / len(v):.1f} | "
                       f"{min(v):.1f} | {max(v):.1f} | {100 * sum(v) / total:.1f} |")
    else:
        path = _one(os.path.join(args.dir, "**", "*kernel_stats.csv"))
        with open(path) as f:
            rows = list(csv.DictReader(f))
        rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
        out += ["| kernel | calls | avg us | min us | max us | total % |",
                "|---|---:|---:|---:|---:|---:|"]
        for r in rows[: args.top]:
            out.append(f"| `{short_name(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                       f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | "
                       f"{float(r['Percentage']):.1f} |")
    text = "\n".join(out) + "\n"
    with open(args.out, "w") as f:
        f.write(text)
    print(text)


def _per_dispatch(dir_: str, counter: str) -> dict[str, list[float]]:
    """Kernel short name -> list of per-dispatch values of ``counter``."""
    path = _one(os.path.join(dir_, "**", "*counter_collection.csv"))
    acc: dict[tuple[str, str], float] = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            key = (r["Dispatch_Id"], r["Kernel_Name"])
            acc[key] = acc.get(key, 0.0) + float(r["Counter_Value"])
    out: dict[str, list[float]] = {}
    for (_, name), v in acc.items():
        out.setdefault(short_name(name), []).append(v)
    return out


def _pick(table: dict[str, list[float]], needle: str) -> tuple[str, list[float]]:
    hits = [(k, v) for k, v in table.items() if needle in k]
    if not hits:
        raise KeyError(f"no kernel matching {needle!r} in {sorted(table)}")
    hits.sort(key=lambda kv: -len(kv[1]))
    return hits[0]


def traffic(args) -> None:
    fetch = _per_dispatch(args.fetch_dir, "FETCH_SIZE")
    write = _per_dispatch(args.write_dir, "WRITE_SIZE")
    kname, kf = _pick(fetch, args.kernel)
    _, kw = _pick(write, args.kernel)
    cname, cf = _pick(fetch, CALIB_KERNEL)
    _, cw = _pick(write, CALIB_KERNEL)
    kib = CALIB_COPY_BYTES / 1024.0
    f_scale = kib / statistics.median(cf)
    w_scale = kib / statistics.median(cw)
    k_fetch = statistics.median(kf) * f_scale * 1024.0
    k_write = statistics.median(kw) * w_scale * 1024.0
    res = {
        "kernel": kname,
        "dispatches": {"fetch": len(kf), "write": len(kw)},
        "fetch_kib_per_dispatch": statistics.median(kf),
        "write_kib_per_dispatch": statistics.median(kw),
        "calib_kernel": cname,
        "calib_bytes_each_way": CALIB_COPY_BYTES,
        "calib_fetch_kib": statistics.median(cf),
        "calib_write_kib": statistics.median(cw),
        "fetch_scale": f_scale,
        "write_scale": w_scale,
        "fetch_bytes_per_launch": k_fetch,
        "write_bytes_per_launch": k_write,
        "bytes_per_launch": k_fetch + k_write,
        "algorithmic_bytes": args.algorithmic_bytes,
        "commands": {"fetch": args.cmd_fetch, "write": args.cmd_write},
    }
    if args.algorithmic_bytes:
        res["traffic_over_algorithmic"] = res["bytes_per_launch"] / args.algorithmic_bytes
    with open(args.out, "w") as f:
        json.dump(res, f, indent=1)
        f.write("\n")
    print(json.dumps(res, indent=1))


def mfma(args) -> None:
    kname, util = _pick(_per_dispatch(args.dir, "MfmaUtil"), args.kernel)
    _, flop = _pick(_per_dispatch(args.dir, "MfmaFlopsBF16"), args.kernel)
    res = {
        "kernel": kname,
        "dispatches": len(util),
        "mfma_util_pct": statistics.mean(util),
        "mfma_util_pct_per_dispatch": util,
        "executed_bf16_mfma_flop": statistics.mean(flop),
        "algorithmic_flop": args.algorithmic_flop,
        "counters": {
            "MfmaUtil": "reduce(SQ_VALU_MFMA_BUSY_CYCLES,sum)/(reduce(GRBM_GUI_ACTIVE,max)*SIMD_NUM)*100",
            "MfmaFlopsBF16": "SQ_INSTS_VALU_MFMA_MOPS_BF16*512"},
        "command": args.cmd,
    }
    if args.algorithmic_flop:
        res["executed_over_algorithmic"] = res["executed_bf16_mfma_flop"] / args.algorithmic_flop
    with open(args.out, "w") as f:
        json.dump(res, f, indent=1)
        f.write("\n")
    print(json.dumps(res, indent=1))


def counters(args) -> None:
    path = _one(os.path.join(args.dir, "**", "*counter_collection.csv"))
    names = []
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] not in names:
                names.append(r["Counter_Name"])
    vals = {}
    kname = None
    for n in names:
        kname, v = _pick(_per_dispatch(args.dir, n), args.kernel)
        vals[n] = statistics.mean(v)
    lines = ["# rocprofv3 counters: " + kname, "", "Command:", "", "```", args.cmd, "```", "",
             "Per-dispatch mean over the kernel's dispatches (SQ counters summed over the chip).",
             "", "| counter | per dispatch |", "|---|---:|"]
    lines += [f"| `{n}` | {vals[n]:.4g} |" for n in names]
    ratios = []
    if "SQ_WAIT_INST_LDS" in vals and "SQ_WAVE_CYCLES" in vals and vals["SQ_WAVE_CYCLES"]:
        ratios.append(("wave-cycles waiting to issue an LDS instruction / wave-cycles",
                       vals["SQ_WAIT_INST_LDS"] / vals["SQ_WAVE_CYCLES"]))
    if "SQ_WAIT_ANY" in vals and "SQ_WAVE_CYCLES" in vals and vals["SQ_WAVE_CYCLES"]:
        ratios.append(("wave-cycles waiting on anything / wave-cycles", vals["SQ_WAIT_ANY"] / vals["SQ_WAVE_CYCLES"]))
    if "SQ_LDS_BANK_CONFLICT" in vals and "SQ_LDS_IDX_ACTIVE" in vals and vals["SQ_LDS_IDX_ACTIVE"]:
        ratios.append(("LDS bank-conflict cycles / LDS active cycles",
                       vals["SQ_LDS_BANK_CONFLICT"] / vals["SQ_LDS_IDX_ACTIVE"]))
    if "SQ_ACTIVE_INST_LDS" in vals and "SQ_WAVE_CYCLES" in vals and vals["SQ_WAVE_CYCLES"]:
        ratios.append(("wave-cycles with an LDS instruction in flight / wave-cycles",
                       vals["SQ_ACTIVE_INST_LDS"] / vals["SQ_WAVE_CYCLES"]))
    if ratios:
        lines += ["", "| ratio | value |", "|---|---:|"] + [f"| {a} | {b:.3f} |" for a, b in ratios]
    with open(args.out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd_name", required=True)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--cmd", required=True)
    s.add_argument("--bench-log")
    s.add_argument("--top", type=int, default=40)
    s.add_argument("--prefix", default=None, help="list only kernels whose name starts with this")
    s.add_argument("--skip", type=int, default=0,
                   help="leave the first N launches of rows with more than N out of `avg us`")
    s.add_argument("-o", "--out", required=True)
    t = sub.add_parser("traffic")
    t.add_argument("fetch_dir")
    t.add_argument("write_dir")
    t.add_argument("--kernel", required=True)
    t.add_argument("--cmd-fetch", required=True)
    t.add_argument("--cmd-write", required=True)
    t.add_argument("--algorithmic-bytes", type=float, default=None)
    t.add_argument("-o", "--out", required=True)
    m = sub.add_parser("mfma")
    m.add_argument("dir")
    m.add_argument("--kernel", required=True)
    m.add_argument("--cmd", required=True)
    m.add_argument("--algorithmic-flop", type=float, default=None)
    m.add_argument("-o", "--out", required=True)
    c = sub.add_parser("counters")
    c.add_argument("dir")
    c.add_argument("--kernel", required=True)
    c.add_argument("--cmd", required=True)
    c.add_argument("-o", "--out", required=True)
    args = ap.parse_args(argv)
    {"stats": stats, "traffic": traffic, "mfma": mfma, "counters": counters}[args.cmd_name](args)


if __name__ == "__main__":
    main(sys.argv[1:])
