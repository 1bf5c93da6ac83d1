"""Summaries of rocprofv3 CSV output, written to profiles/.

* ``stats``: a ``*_kernel_stats.csv`` (``--kernel-trace --stats``) as a
  markdown table of per-kernel calls and average durations.
* ``traffic``: two ``--pmc`` runs of ``bench.py --pmc-pass`` (one collecting
  FETCH_SIZE, one WRITE_SIZE; both in KiB per dispatch) turned into HBM bytes
  per launch for each kernel. Each counter is scaled by what it reads for the
  pass's calibration copy, a ``kv_copy_rows_kernel`` dispatch that reads and
  writes a known number of bytes (the largest-grid dispatch of that kernel).
  Each kernel's figure is its last dispatch in the pass (the hot-path launch;
  set-up work such as the prefix fill runs before it); for a kernel whose one
  call is several launches (the forward's and the dQ pass's 8-wave pair or
  4-wave launch and their two-group tail launch: ``MULTI_LAUNCH``) it is
  the sum over the last run of consecutive dispatches of that kernel.

* ``mfma``: ``--pmc`` runs of ``bench.py --pmc-pass`` collecting SQ and GRBM
  counters (any number of runs, each its own CSV) turned into per-kernel
  figures for the attention kernels: MFMA busy fraction (busy cycles of the
  MFMA units over all SIMDs' active cycles), the bf16 MFMA work the counters
  count against the credited work, and instructions per MFMA.
* ``clock``: one run with ``--pmc GRBM_GUI_ACTIVE --kernel-trace``: each
  dispatch's average clock, its GPU-active cycles per XCD
  (``GRBM_GUI_ACTIVE`` summed over the 8 XCDs, / 8) over its traced
  duration, median per attention kernel.

    python mtp-glora_amd/rocprof_summary.py stats TRACE_DIR/bench_kernel_stats.csv
    python mtp-glora_amd/rocprof_summary.py traffic --fetch F.csv --write W.csv \\
        --calib-read BYTES --calib-write BYTES --config 2 -o profiles/config2_traffic.json
    python mtp-glora_amd/rocprof_summary.py mfma --pass-json PASS.json A.csv B.csv \\
        -o profiles/config2_mfma.json
    python mtp-glora_amd/rocprof_summary.py clock COUNTERS.csv KERNEL_TRACE.csv
"""
from __future__ import annotations

import argparse
import csv
import json
import re
import sys

CALIB_KERNEL = "kv_copy_rows_kernel"


def kernel_base(name: str) -> str:
    """``attn_fwd_kernel`` from a mangled or demangled kernel name."""
    m = re.search(r"([a-z_]+_kernel)", name)
    return m.group(1).lstrip("_") if m else name[:48]


# kernels whose one call may be several consecutive launches
MULTI_LAUNCH = ("attn_fwd_kernel", "attn_bwd_dq_kernel")

# the forward's and the dQ pass's forms by their last template argument
FORMS = {"0": "4-wave", "1": "8-wave pair", "2": "two-group"}


def kernel_label(name: str) -> str:
    """kernel_base, telling the three forms of the forward and of the dQ pass
    apart (their last template argument) where the name carries it."""
    k = kernel_base(name)
    last = re.search(r"Li(\d)EEEv", name) or re.search(r",\s*(\d)>\(", name)
    if k in MULTI_LAUNCH and last and last.group(1) in FORMS:
        return f"{k} ({FORMS[last.group(1)]})"
    return k


def _last_call(seq):
    """seq: [(kernel, dispatch_id, payload)] in dispatch order -> {kernel:
    [payloads of its last call]}: the last dispatch, or for MULTI_LAUNCH
    kernels the last run of consecutive dispatches."""
    out = {}
    for i, (k, _, pay) in enumerate(seq):
        if k in MULTI_LAUNCH and i > 0 and seq[i - 1][0] == k:
            out[k].append(pay)
        else:
            out[k] = [pay]
    return out


def stats_markdown(path: str) -> str:
    rows = list(csv.DictReader(open(path)))
    out = ["| Kernel | Calls | Avg (us) | Share |", "|---|---|---|---|"]
    for r in rows:
        out.append(f"| {kernel_label(r['Name'])} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                   f"{float(r['Percentage']):.2f} % |")
    return "\n".join(out)


def _dispatches(path: str, counter: str):
    """[(kernel, grid_size, KiB)] in dispatch order for one counter."""
    out = []
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] != counter:
            continue
        out.append((kernel_base(r["Kernel_Name"]), int(r["Grid_Size"]), float(r["Counter_Value"]),
                    int(r["Dispatch_Id"])))
    out.sort(key=lambda t: t[3])
    return out


def traffic(fetch_csv: str, write_csv: str, calib_read: int, calib_write: int, config: int) -> dict:
    result = {"config": config, "counters": ["FETCH_SIZE", "WRITE_SIZE"], "unit": "bytes per launch"}
    scaled = {}
    for counter, path, known in (("FETCH_SIZE", fetch_csv, calib_read), ("WRITE_SIZE", write_csv, calib_write)):
        disp = _dispatches(path, counter)
        calib = max((d for d in disp if d[0] == CALIB_KERNEL), key=lambda d: d[1])
        factor = known / (calib[2] * 1024.0)
        result[f"{counter}_calibration"] = {"known_bytes": known, "counter_KiB": calib[2], "factor": factor}
        # the pass launches each hot-path kernel last (set-up copies come first)
        calls = _last_call([(d[0], d[3], d[2]) for d in disp if d is not calib])
        scaled[counter] = {k: sum(v) * 1024.0 * factor for k, v in calls.items()}
    kernels = {}
    for k in sorted(set(scaled["FETCH_SIZE"]) | set(scaled["WRITE_SIZE"])):
        f = scaled["FETCH_SIZE"].get(k, 0.0)
        w = scaled["WRITE_SIZE"].get(k, 0.0)
        kernels[k] = {"fetch_bytes": round(f), "write_bytes": round(w), "traffic_bytes": round(f + w)}
    result["kernels"] = kernels
    return result


SIMDS = 1024          # MI355X: 256 CUs x 4 SIMDs
XCDS = 8              # GRBM_GUI_ACTIVE is summed over the 8 XCDs in the CSV
MOP_FLOP = 512        # one SQ_INSTS_VALU_MFMA_MOPS_* unit (FLOP)
ATTN_KERNELS = ("attn_fwd_kernel", "attn_bwd_dq_kernel", "attn_bwd_dkdv_kernel")


def counters_by_kernel(paths) -> dict:
    """{kernel: {counter: value}} from the last dispatch of each kernel in
    every counter CSV (one rocprofv3 --pmc run each). Counters of a
    MULTI_LAUNCH kernel's launches are summed (cycles and instruction counts
    add over sequential launches); a derived percentage (MfmaUtil) is
    weighted by each launch's GRBM_GUI_ACTIVE when the run has it, else
    averaged."""
    out: dict = {}
    for path in paths:
        per: dict = {}
        for r in csv.DictReader(open(path)):
            d = int(r["Dispatch_Id"])
            e = per.setdefault(d, {"k": kernel_base(r["Kernel_Name"]), "c": {}})
            e["c"][r["Counter_Name"]] = float(r["Counter_Value"])
        calls = _last_call([(e["k"], d, e["c"]) for d, e in sorted(per.items())])
        for k, runs in calls.items():
            merged: dict = {}
            for name in runs[0]:
                vals = [c.get(name, 0.0) for c in runs]
                if name == "MfmaUtil":
                    w = [c.get("GRBM_GUI_ACTIVE", 1.0) for c in runs]
                    merged[name] = sum(v * x for v, x in zip(vals, w)) / sum(w)
                else:
                    merged[name] = sum(vals)
            out.setdefault(k, {}).update(merged)
    return out


def mfma_summary(paths, credited: dict) -> dict:
    c = counters_by_kernel(paths)
    res = {"simds": SIMDS, "xcds": XCDS, "mop_flop": MOP_FLOP, "kernels": {}}
    for k in ATTN_KERNELS:
        if k not in c:
            continue
        v = c[k]
        e = {"counters": v}
        gui = v.get("GRBM_GUI_ACTIVE")
        if gui and "SQ_VALU_MFMA_BUSY_CYCLES" in v:
            e["mfma_busy_frac"] = v["SQ_VALU_MFMA_BUSY_CYCLES"] / (gui / XCDS * SIMDS)
        if "SQ_VALU_MFMA_BUSY_CYCLES" in v and "SQ_BUSY_CU_CYCLES" in v and v["SQ_BUSY_CU_CYCLES"]:
            e["mfma_busy_per_busy_cu_simd"] = v["SQ_VALU_MFMA_BUSY_CYCLES"] / (4 * v["SQ_BUSY_CU_CYCLES"])
        if "SQ_INSTS_VALU_MFMA_MOPS_BF16" in v:
            fl = v["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * MOP_FLOP
            e["mfma_flop"] = fl
            if credited.get(k):
                e["credited_flop"] = credited[k]
                e["mfma_flop_over_credited"] = fl / credited[k]
        n_mfma = v.get("SQ_INSTS_MFMA") or v.get("SQ_INSTS_VALU_MFMA_BF16")
        if n_mfma:
            for name in ("SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_INSTS_VALU_TRANS_F32"):
                if name in v:
                    e[name[9:].lower() + "_per_mfma"] = v[name] / n_mfma
        if v.get("SQ_WAVE_CYCLES"):
            for name in ("SQ_WAIT_INST_ANY", "SQ_WAIT_INST_LDS", "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS",
                         "SQ_WAIT_ANY"):
                if name in v:
                    e[name[3:].lower() + "_frac_of_wave_cycles"] = v[name] / v["SQ_WAVE_CYCLES"]
        res["kernels"][k] = e
    return res


def kernel_clocks(counter_csv: str, trace_csv: str, xcds: int = 8) -> dict:
    """Median clock (GHz) and duration (us) per attention kernel: per
    dispatch, GRBM_GUI_ACTIVE (summed over the XCDs) / xcds cycles over the
    traced end - start nanoseconds."""
    cyc = {}
    for r in csv.DictReader(open(counter_csv)):
        if r["Counter_Name"] == "GRBM_GUI_ACTIVE":
            cyc[r["Dispatch_Id"]] = cyc.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
    per = {}
    for r in csv.DictReader(open(trace_csv)):
        d = r["Dispatch_Id"]
        if d not in cyc:
            continue
        k = kernel_base(r["Kernel_Name"])
        if k not in ATTN_KERNELS:
            continue
        ns = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        if ns > 0:
            per.setdefault(k, []).append((cyc[d] / xcds / ns, ns / 1e3))
    out = {}
    for k, v in per.items():
        ghz = sorted(x[0] for x in v)
        us = sorted(x[1] for x in v)
        out[k] = {"dispatches": len(v), "median_ghz": round(ghz[len(ghz) // 2], 3),
                  "min_ghz": round(ghz[0], 3), "max_ghz": round(ghz[-1], 3),
                  "median_us": round(us[len(us) // 2], 1)}
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--calib-read", type=int, required=True)
    t.add_argument("--calib-write", type=int, required=True)
    t.add_argument("--config", type=int, default=2)
    t.add_argument("-o", "--out")
    m = sub.add_parser("mfma")
    m.add_argument("csvs", nargs="+")
    m.add_argument("--pass-json", help="the JSON line bench.py --pmc-pass printed (credited FLOPs)")
    m.add_argument("-o", "--out")
    c = sub.add_parser("clock")
    c.add_argument("counters")
    c.add_argument("trace")
    c.add_argument("-o", "--out")
    args = ap.parse_args(argv)
    if args.cmd == "stats":
        print(stats_markdown(args.csv))
        return 0
    if args.cmd == "mfma":
        credited = {}
        if args.pass_json:
            for line in open(args.pass_json):
                line = line.strip()
                if line.startswith("{") and "pmc_pass" in line:
                    credited = json.loads(line).get("credited_flop", {})
        res = mfma_summary(args.csvs, credited)
    elif args.cmd == "clock":
        res = kernel_clocks(args.counters, args.trace)
    else:
        res = traffic(args.fetch, args.write, args.calib_read, args.calib_write, args.config)
    text = json.dumps(res, indent=1)
    if args.out:
        with open(args.out, "w") as f:
            f.write(text + "\n")
    print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
