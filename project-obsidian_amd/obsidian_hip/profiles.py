"""Summaries of rocprofv3 runs for the repository's profiles/ folder.

    python -m obsidian_hip.profiles traffic --fetch F.csv --write W.csv \\
        --copy-fetch CF.csv --copy-write CW.csv [--out DIR]
    python -m obsidian_hip.profiles stats --stats S.csv [--line bench.json] [--out DIR]
    python -m obsidian_hip.profiles mfma --pmc P.csv [--kernel moe_ffn] [--out DIR]

`traffic` turns two `rocprofv3 --pmc` runs of bench.py (FETCH_SIZE, then
WRITE_SIZE, KiB per dispatch) into HBM bytes per launch, each counter scaled by
what it reads for a plain device copy of known size (bench.py --calibrate-copy),
and records for each kernel a digest of the sources it is built from, so a
reader (bench.py) can tell whether the figure still describes the code.
`stats` turns a `rocprofv3 --kernel-trace --stats` CSV into a Markdown table.
`mfma` turns a `rocprofv3 --pmc` run of the MFMA counters into the matrix
and vector pipes' busy fractions of one kernel.
"""
from __future__ import annotations

import argparse
import collections
import csv
import hashlib
import json
import os
import re
import sys
from typing import Dict, Optional, Tuple

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# kernel -> (pattern of its rocprofv3 name, the sources it is compiled from)
KERNELS = {
    "decode_fused": (r"decode_fused_kernel<2, false>",
                     ("csrc/obs_decode_fused.hip", "csrc/obs_moe_half.hpp", "csrc/obs_internal.hpp")),
    "decode_fused_norm": (r"decode_fused_kernel<2, true>",
                          ("csrc/obs_decode_fused.hip", "csrc/obs_moe_half.hpp", "csrc/obs_internal.hpp")),
    "layer_fused": (r"layer_fused_kernel<2>",
                    ("csrc/obs_layer_fused.hip", "csrc/obs_attn_half.hpp", "csrc/obs_moe_half.hpp",
                     "csrc/obs_internal.hpp")),
    "grouped_gemm_gateup": (r"grouped_gemm_kernel<1u, 3u>", ("csrc/obs_prefill.hip", "csrc/obs_internal.hpp")),
    "grouped_gemm_down": (r"grouped_gemm_kernel<2u, 5u>", ("csrc/obs_prefill.hip", "csrc/obs_internal.hpp")),
    "moe_ffn": (r"moe_ffn_kernel<2u>", ("csrc/obs_prefill.hip", "csrc/obs_internal.hpp")),
    "moe_group_count": (r"group_count_kernel", ("csrc/obs_prefill.hip",)),
    "moe_group_scan": (r"group_scan_kernel", ("csrc/obs_prefill.hip",)),
    "moe_group_rank": (r"group_rank_kernel", ("csrc/obs_prefill.hip",)),
    "moe_combine": (r"combine_kernel", ("csrc/obs_prefill.hip",)),
}
COPY = r"copyBuffer"

# algorithmic bytes per launch at the bench's shapes (H 2048, I 768, 128 experts, top-8, T 2048)
_PROJ = 768 * 2048 // 2 + 2 * 2 * (768 * 2048 // 64)
ALGORITHMIC = {
    "decode_fused": 8 * 3 * _PROJ + (128 * 2048 + 2 * 2 * (128 * 2048 // 64)) + 2 * 2 * 2048,
    # with the post-attention norm: its 2048 bf16 weights are read too
    "decode_fused_norm": 8 * 3 * _PROJ + (128 * 2048 + 2 * 2 * (128 * 2048 // 64)) + 2 * 2 * 2048 + 2 * 2048,
    "grouped_gemm_gateup": 128 * 2 * _PROJ + 2048 * 2048 * 2 + 2048 * 8 * 768 * 2,
    "grouped_gemm_down": 128 * _PROJ + 2048 * 8 * 768 * 2 + 2048 * 8 * 2048 * 2,
}
# both GEMMs in one launch: the same bytes (H is still written once and read once)
ALGORITHMIC["moe_ffn"] = ALGORITHMIC["grouped_gemm_gateup"] + ALGORITHMIC["grouped_gemm_down"]


def source_digest(kernel: str) -> Optional[str]:
    """sha256 (first 16 hex digits) over the sources `kernel` is built from."""
    if kernel not in KERNELS:
        return None
    h = hashlib.sha256()
    for rel in KERNELS[kernel][1]:
        with open(os.path.join(PKG, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def _short(name: str) -> Optional[str]:
    if re.search(COPY, name):
        return "__copy"
    for k, (pat, _) in KERNELS.items():
        if re.search(re.escape(pat) if "<" in pat else pat, name):
            return k
    return None


def pmc_per_dispatch(path: str, counter: str, first: int = 0) -> Dict[str, Tuple[float, int]]:
    """(mean counter value per dispatch, dispatches) per known kernel; with
    first > 0 only each kernel's first `first` dispatches count."""
    per = collections.defaultdict(dict)
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            k = _short(r["Kernel_Name"])
            if k is None:
                continue
            d = per[k]
            d[r["Dispatch_Id"]] = d.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
    out = {}
    for k, d in per.items():
        ids = sorted(d, key=int)
        vals = [d[i] for i in ids]
        if k == "__copy":  # the big copies only (a small readback copy runs too)
            vals = [v for v in vals if v >= 0.5 * max(vals)]
        elif first:
            vals = vals[:first]
        out[k] = (sum(vals) / len(vals), len(vals))
    return out


def traffic(fetch: str, write: str, copy_fetch: str, copy_write: str, copy_bytes: int, first: int = 0) -> Dict:
    cf = pmc_per_dispatch(copy_fetch, "FETCH_SIZE")["__copy"][0]
    cw = pmc_per_dispatch(copy_write, "WRITE_SIZE")["__copy"][0]
    fs, ws = copy_bytes / 1024 / cf, copy_bytes / 1024 / cw
    fe, wr = pmc_per_dispatch(fetch, "FETCH_SIZE", first), pmc_per_dispatch(write, "WRITE_SIZE", first)
    res = {"_calibration": {"copy_bytes": copy_bytes, "fetch_kib_per_copy": cf, "write_kib_per_copy": cw,
                            "fetch_scale": fs, "write_scale": ws}}
    for k in KERNELS:
        if k not in fe or k not in wr:
            continue
        f, n = fe[k]
        w, _ = wr[k]
        t = int(round(f * 1024 * fs + w * 1024 * ws))
        e = {"dispatches": n, "fetch_kib_per_dispatch": round(f, 1), "write_kib_per_dispatch": round(w, 1),
             "traffic_bytes_per_launch": t, "source_sha": source_digest(k)}
        if k in ALGORITHMIC:
            e["algorithmic_bytes_per_launch"] = ALGORITHMIC[k]
            e["traffic_over_algorithmic"] = round(t / ALGORITHMIC[k], 3)
        res[k] = e
    return res


def traffic_md(res: Dict, cmds) -> str:
    c = res["_calibration"]
    md = ["# HBM traffic per launch — rocprofv3 FETCH_SIZE / WRITE_SIZE", "",
          "Workloads: decode MoE layer T=1 (top-8 of 128 experts, H=2048, I=768, 48-layer table) and grouped "
          "prefill T=2048 (Zipf s=1.1 routing, seed 0), as run by `bench.py`.", "",
          "Commands (each counter in its own run, from the repository root):", "", "```", *cmds, "```", "",
          f"Calibration: a plain {c['copy_bytes'] >> 20} MiB device copy reads FETCH_SIZE = {c['fetch_kib_per_copy']:.0f} "
          f"KiB and WRITE_SIZE = {c['write_kib_per_copy']:.0f} KiB per dispatch for {c['copy_bytes'] >> 10:,} KiB moved "
          f"each way, so bytes = FETCH_SIZE x 1024 x {c['fetch_scale']:.4f} and WRITE_SIZE x 1024 x "
          f"{c['write_scale']:.4f}.", "",
          "| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | traffic bytes / launch | algorithmic bytes / "
          "launch | ratio | source digest |", "|---|---|---|---|---|---|---|---|"]
    for k, e in res.items():
        if k.startswith("_"):
            continue
        a = e.get("algorithmic_bytes_per_launch")
        md.append(f"| {k} | {e['dispatches']} | {e['fetch_kib_per_dispatch']:,.1f} | {e['write_kib_per_dispatch']:,.1f} "
                  f"| {e['traffic_bytes_per_launch']:,} | {'' if a is None else format(a, ',')} | "
                  f"{e.get('traffic_over_algorithmic', '')} | `{e['source_sha']}` |")
    md += ["", "Algorithmic bytes: decode = 8 experts x 2,654,208 + router 278,528 + 8,192 activations; gate/up GEMM = "
           "128 experts x 2 x 884,736 (weights, scales, biases) + X 8 MiB + H 24 MiB written; down GEMM = 128 x 884,736 "
           "+ H 24 MiB + Yp 64 MiB written. FETCH_SIZE counts L2-to-fabric reads, so Infinity Cache hits count too. "
           "The source digest is `obsidian_hip.profiles.source_digest` of the kernel's sources at measurement time; "
           "bench.py reports the traffic only while it matches."]
    return "\n".join(md) + "\n"


def stats_md(path: str, line: Optional[str], cmd: str) -> str:
    with open(path) as f:
        rows = list(csv.DictReader(f))
    md = ["# Kernel durations — rocprofv3 --kernel-trace --stats", "", "Command (from the repository root):", "",
          "```", cmd, "```", "", "| kernel | calls | average µs | min µs | max µs | % of traced time |",
          "|---|---|---|---|---|---|"]
    for r in rows:
        nm = re.sub(r"\(.*", "", r["Name"].replace("(anonymous namespace)::", "").replace("void ", ""))[:60]
        md.append(f"| `{nm}` | {r['Calls']} | {float(r['AverageNs']) / 1000:.2f} | {float(r['MinNs']) / 1000:.2f} | "
                  f"{float(r['MaxNs']) / 1000:.2f} | {float(r['Percentage']):.2f} |")
    if line:
        md += _roofline_check(rows, json.loads(line))
        md += ["", "bench.py's line from the same run:", "", "```json", line.strip(), "```"]
    return "\n".join(md) + "\n"


def _roofline_check(rows, line: Dict):
    """The line's decode roofline against this run's rocprof average of the
    kernel it names (the MoE sweep's launches alone: the decoder's MoE half is
    the `decode_fused_norm` instantiation, timed under its own name)."""
    rf = line.get("roofline") or {}
    k = rf.get("kernel")
    if k not in KERNELS or not line.get("config", {}).get("layers_per_step"):
        return []
    hit = [r for r in rows if _short(r["Name"]) == k]
    if not hit:
        return []
    avg_us = float(hit[0]["AverageNs"]) / 1000
    n = int(line["config"]["layers_per_step"])
    frac = rf["bytes_per_launch"] / (avg_us * 1e-6) / (rf["peak"] * 1e9)
    return ["", f"Roofline check for `{k}` ({hit[0]['Calls']} launches of the {n}-layer sweep):", "",
            f"- {n} x {avg_us:.3f} µs (rocprof average) = {n * avg_us / 1000:.4f} ms, against the line's "
            f"ms_per_step {line['ms_per_step']:.4f} (the rest is the gap between launches: "
            f"{(line['ms_per_step'] * 1000 / n - avg_us):.3f} µs per launch);",
            f"- {rf['bytes_per_launch']:,} B / {avg_us:.3f} µs / {rf['peak']:.0f} GB/s = frac {frac:.4f} against the "
            f"line's {rf['frac']:.4f}, which the timed region gives launch gaps included "
            f"({line['decode_us_per_layer']:.3f} µs per layer)."]


MFMA_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_MFMA", "SQ_INSTS_VALU", "SQ_ACTIVE_INST_VALU",
                 "SQ_VALU_MFMA_COEXEC_CYCLES", "SQ_WAVE_CYCLES", "SQ_WAIT_INST_ANY", "GRBM_GUI_ACTIVE")
# flop of one prefill FFN launch at T = 2048, top-8: gate/up 2 x T k x 2 I x H, down 2 x T k x H x I
PREFILL_FFN_FLOP = 2 * 2048 * 8 * (2 * 768) * 2048 + 2 * 2048 * 8 * 2048 * 768


def mfma_util(path: str, kernel: str, first: int = 10, simds: int = 1024, xcds: int = 8) -> Dict:
    """Per-dispatch means of the MFMA counters for `kernel`'s first `first`
    dispatches of a `rocprofv3 --pmc` CSV, and the figures derived from them.
    GRBM_GUI_ACTIVE is summed over the XCDs, so per XCD it is / xcds; a SIMD's
    busy fractions are counter / (cycles x simds); SQ_ACTIVE_INST_VALU counts
    in units of 4 cycles."""
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    span = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if _short(r["Kernel_Name"]) != kernel:
                continue
            d = int(r["Dispatch_Id"])
            per[d][r["Counter_Name"]] += float(r["Counter_Value"])
            if "Start_Timestamp" in r and r.get("End_Timestamp"):
                span[d] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
    ids = sorted(per)[:first]
    if not ids:
        raise ValueError(f"no dispatches of {kernel} in {path}")
    m = {c: sum(per[i].get(c, 0.0) for i in ids) / len(ids) for c in MFMA_COUNTERS}
    us = sum(span.get(i, 0.0) for i in ids) / len(ids)
    cyc = m["GRBM_GUI_ACTIVE"] / xcds
    mfma = m["SQ_VALU_MFMA_BUSY_CYCLES"] / (cyc * simds)
    valu = 4.0 * m["SQ_ACTIVE_INST_VALU"] / (cyc * simds)
    both = m["SQ_VALU_MFMA_COEXEC_CYCLES"] / (cyc * simds)
    return {"dispatches": len(ids), "us": us, "clock_ghz": cyc / us / 1e3 if us else None,
            "mfma_insts": m["SQ_INSTS_MFMA"], "mfma_util": mfma, "valu_per_mfma": m["SQ_INSTS_VALU"] / m["SQ_INSTS_MFMA"],
            "valu_busy": valu, "coexec": both, "neither": 1.0 - (mfma + valu - both),
            "tflops": PREFILL_FFN_FLOP / us / 1e6 if us else None,
            "padded_tflops": m["SQ_INSTS_MFMA"] * 32768 / us / 1e6 if us else None}


def mfma_md(res: Dict, kernel: str, cmd: str) -> str:
    md = ["# MFMA utilisation — the prefill's expert FFN (rocprofv3 --pmc)", "",
          "Workload: `bench.py` prefill, T=2048 tokens, top-8 of 128 experts with Zipf(s=1.1) routing (seed 0), "
          "gate/up [768, 2048] and down [2048, 768] 4-bit experts, both GEMMs in one launch.", "",
          "Command (from the repository root), then the summary:", "", "```", cmd,
          f"cd project-obsidian_amd && python -m obsidian_hip.profiles mfma --pmc ../gpurun_out/pmc_mfma/bench_counter_collection.csv --kernel {kernel} --out ../profiles",
          "```", "",
          "MfmaUtil = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD x 1024 SIMDs), rocprofv3's own MfmaUtil "
          "expression (one v_mfma_f32_32x32x16_bf16 keeps a SIMD's matrix unit busy 32 cycles). VALU busy = 4 x "
          "SQ_ACTIVE_INST_VALU over the same cycles; both = SQ_VALU_MFMA_COEXEC_CYCLES; neither = 1 - (MFMA + VALU - "
          "both). The clock is GRBM_GUI_ACTIVE per XCD / duration.", "",
          "| kernel | dispatches | duration µs | clock GHz | MFMA instructions | MfmaUtil | VALU instr / MFMA | VALU busy "
          "| both busy | neither busy | algorithmic TFLOP/s | padded-MFMA TFLOP/s |",
          "|---|---|---|---|---|---|---|---|---|---|---|---|",
          f"| {kernel} | {res['dispatches']} | {res['us']:.1f} | {res['clock_ghz']:.2f} | {res['mfma_insts']:,.0f} | "
          f"{100 * res['mfma_util']:.1f}% | {res['valu_per_mfma']:.1f} | {100 * res['valu_busy']:.1f}% | "
          f"{100 * res['coexec']:.1f}% | {100 * res['neither']:.1f}% | {res['tflops']:.0f} | {res['padded_tflops']:.0f} |", "",
          "Rows: the kernel's first dispatches, which are the Zipf prefill section of the bench. SQ_INSTS_VALU counts "
          "the MFMAs too. The padded-MFMA rate counts every issued MFMA (rows padded to 32 per expert tile); the "
          "algorithmic rate counts 2 x rows x N x K only. Durations are the dispatch timestamps of the counter run, "
          "whose clock runs below the 2.30 GHz the MFMA-only loop reaches (`achievable` in bench.py's line)."]
    return "\n".join(md) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m obsidian_hip.profiles")
    sub = ap.add_subparsers(dest="what", required=True)
    t = sub.add_parser("traffic")
    for a in ("fetch", "write", "copy-fetch", "copy-write"):
        t.add_argument("--" + a, required=True)
    t.add_argument("--copy-mib", type=int, default=1024)
    t.add_argument("--first", type=int, default=0, help="count only each kernel's first N dispatches")
    t.add_argument("--cmd", action="append", default=[], help="a command that made the CSVs (for the summary)")
    t.add_argument("--out", default="profiles")
    s = sub.add_parser("stats")
    s.add_argument("--stats", required=True)
    s.add_argument("--line", help="a file holding bench.py's JSON line from the same run")
    s.add_argument("--cmd", required=True)
    s.add_argument("--name", default="kernel_stats_bench.md")
    s.add_argument("--out", default="profiles")
    mm = sub.add_parser("mfma")
    mm.add_argument("--pmc", required=True)
    mm.add_argument("--kernel", default="moe_ffn")
    mm.add_argument("--first", type=int, default=10)
    mm.add_argument("--cmd", default="rocprofv3 --pmc " + " ".join(MFMA_COUNTERS) + " --kernel-include-regex moe_ffn "
                    "-d gpurun_out/pmc_mfma -o bench --output-format csv -- python3 bench.py --no-cpu --no-decoder "
                    "--steps 2 --warmup 1 --prof-reps 2")
    mm.add_argument("--out", default="profiles")
    args = ap.parse_args(argv)
    os.makedirs(args.out, exist_ok=True)
    if args.what == "traffic":
        res = traffic(args.fetch, args.write, args.copy_fetch, args.copy_write, args.copy_mib << 20, args.first)
        with open(os.path.join(args.out, "hbm_traffic.json"), "w") as f:
            json.dump(res, f, indent=1)
        with open(os.path.join(args.out, "hbm_traffic.md"), "w") as f:
            f.write(traffic_md(res, args.cmd))
        print(json.dumps({k: v.get("traffic_over_algorithmic") for k, v in res.items() if not k.startswith("_")}))
    elif args.what == "mfma":
        res = mfma_util(args.pmc, args.kernel, args.first)
        with open(os.path.join(args.out, "mfma_util_prefill.md"), "w") as f:
            f.write(mfma_md(res, args.kernel, args.cmd))
        print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in res.items()}))
    else:
        # the bench's JSON line: the last line that is one (rocprofv3 logs after it)
        objs = [ln for ln in open(args.line).read().splitlines() if ln.lstrip().startswith("{")] if args.line else []
        line = objs[-1] if objs else None
        with open(os.path.join(args.out, args.name), "w") as f:
            f.write(stats_md(args.stats, line, args.cmd))
    return 0


if __name__ == "__main__":
    sys.exit(main())
