"""Summaries of rocprofv3 results for profiles/ (reads the rocpd SQLite database rocprofv3 writes).

  python trellis.2-stableprojectorz_amd/profiling.py stats TRACE.db OUT.txt --command "..."
      per-kernel dispatch count, average / min / max duration and share of GPU time
  python trellis.2-stableprojectorz_amd/profiling.py counters PMC.db TRACE.db OUT.json OUT.txt \
          --command "..."
      per-kernel averages of every --pmc counter, with MFMA throughput / busy fraction / clock
      derived from them and the durations of a kernel-trace run of the same program
  python trellis.2-stableprojectorz_amd/profiling.py traffic FETCH.db WRITE.db OUT.json OUT.txt \
          --calib-bytes 268435456 --command "..."
      per-kernel average FETCH_SIZE and WRITE_SIZE (KiB per dispatch) scaled to bytes by the
      same counters on a device copy of --calib-bytes bytes (the largest copy dispatch in the run)

  python trellis.2-stableprojectorz_amd/profiling.py workload NAME TRACE.db MFMA.db FETCH.db \
          WRITE.db OUT.json --last 3 --calib-bytes 268435456 --command "..."
      one workload's record (a bench.py --profile-pass --workload NAME run under each of the four
      rocprofv3 passes): per kernel, the averages over its last --last dispatches (the warm
      launches) of duration, every counter, HBM bytes (FETCH_SIZE / WRITE_SIZE scaled by the
      calibration copy) and the derived MFMA figures
  python trellis.2-stableprojectorz_amd/profiling.py merge OUT.json OUT.txt IN.json...
      the per-workload records in one file, {workload: {kernel: record}}, and a text summary

Kernel names are shortened to the name the library's own profiler uses where possible
(e.g. conv_mfma_kernel<__bf16,256,256,64,4,2,4,0> -> conv_mfma_kernel<bf16,256x256,k64,s4>).
"""
from __future__ import annotations

import argparse
import json
import re
import sqlite3
from collections import defaultdict

_TYPES = {"DF16b": "bf16", "DF16_": "f16", "f": "f32"}


_DEMANGLED_TYPES = {"__bf16": "bf16", "_Float16": "f16", "float": "f32"}


def _conv_name(kind: str, t: str, nums: list) -> str:
    if kind == "conv_mfma_kernel":  # BM, BN, KB, STAGES, WM, WN, EPI
        bm, bn, kb, st, _, _, epi = nums
        tag = {"1": ",res", "2": ",ln"}.get(epi, "")
        return f"conv_mfma_kernel<{t},{bm}x{bn},k{kb},s{st}{tag}>"
    if kind == "conv_gather_kernel":  # EPI
        return f"conv_gather_kernel<{t}{',res' if nums[0] == '1' else ''}>"
    if kind == "conv_narrow_kernel":  # CO, EPI, threads
        co, epi, _ = nums
        return f"conv_narrow_kernel<{t},32x{co}{',res' if epi == '1' else ''}>"
    bm, bn, kb, _, _, epi = nums  # conv_regstage_kernel
    return f"conv_regstage_kernel<{t},{bm}x{bn},k{kb}{',res' if epi == '1' else ''}>"


def short_name(name: str) -> str:
    kinds = "conv_mfma_kernel|conv_regstage_kernel|conv_narrow_kernel|conv_gather_kernel"
    m = re.search(rf"({kinds})I(DF16b|DF16_|f)((?:Li\d+E)+)", name)  # mangled
    if m:
        return _conv_name(m.group(1), _TYPES[m.group(2)], re.findall(r"Li(\d+)E", m.group(3)))
    m = re.search(rf"({kinds})<(__bf16|_Float16|float), ([\d, ]+)>", name)  # demangled
    if m:
        return _conv_name(m.group(1), _DEMANGLED_TYPES[m.group(2)],
                          [x.strip() for x in m.group(3).split(",")])
    m = re.search(r"(?:tsc::\(anonymous namespace\)::|N_1\d+)(\w+_kernel)", name)
    if m:
        base = m.group(1)
        # key types: int32/int64 for the neighbor map's sort, uint32/uint64 for the gather plan's
        # Morton sort
        tm = re.search(r"<(unsigned int|unsigned long|int|long)", name)
        if "fill_columns_kernel" in name:
            base += "<radix>" if "ColumnLookup" in name else "<bitmap>"
        elif tm:
            base += "<" + {"int": "int32", "long": "int64", "unsigned int": "uint32",
                           "unsigned long": "uint64"}[tm.group(1)] + ">"
        return base
    m = re.search(r"(layernorm\w*_kernel|silu_kernel|add_kernel)", name)
    if m:
        return m.group(1)
    return name[:80]


def _rows(db_path: str, sql: str):
    con = sqlite3.connect(db_path)
    try:
        return con.execute(sql).fetchall()
    finally:
        con.close()


def stats(db: str, out: str, command: str) -> None:
    agg = defaultdict(list)
    for name, dur in _rows(db, "select name, duration from kernels"):
        agg[short_name(name)].append(dur / 1e3)
    total = sum(sum(v) for v in agg.values()) or 1.0
    lines = [f"# rocprofv3 kernel trace summary", f"# command: {command}", "",
             f"{'kernel':58s} {'calls':>6s} {'avg_us':>10s} {'min_us':>10s} {'max_us':>10s} {'share':>7s}"]
    for k, v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"{k:58s} {len(v):6d} {sum(v) / len(v):10.2f} {min(v):10.2f} {max(v):10.2f} "
                     f"{100 * sum(v) / total:6.2f}%")
    open(out, "w").write("\n".join(lines) + "\n")


def _counter(db: str, counter: str):
    per = defaultdict(list)
    for name, val, grid in _rows(db, "select kernel_name, value, grid_size from counters_collection "
                                     f"where counter_name = '{counter}'"):
        per[name].append((float(val), int(grid)))
    return per


def traffic(fetch_db: str, write_db: str, out_json: str, out_txt: str, calib_bytes: int,
            command: str) -> None:
    fetch, write = _counter(fetch_db, "FETCH_SIZE"), _counter(write_db, "WRITE_SIZE")

    def calib(per):
        copies = [(g, v) for n, vs in per.items() if "copyBuffer" in n for v, g in vs]
        g, kib = max(copies)  # the largest copy dispatch is the calibration copy
        return calib_bytes / (kib * 1024.0)

    ff, fw = calib(fetch), calib(write)
    res = {}
    for name in sorted(set(fetch) | set(write)):
        if "copyBuffer" in name or "at::native" in name:
            continue
        f = [v for v, _ in fetch.get(name, [])]
        w = [v for v, _ in write.get(name, [])]
        key = short_name(name)
        res[key] = {"fetch_bytes": round(sum(f) / len(f) * 1024 * ff) if f else None,
                    "write_bytes": round(sum(w) / len(w) * 1024 * fw) if w else None,
                    "dispatches": len(f)}
    doc = {"calibration": {"copy_bytes": calib_bytes, "fetch_scale": ff, "write_scale": fw},
           "kernels": res, "command": command}
    open(out_json, "w").write(json.dumps(doc, indent=1) + "\n")
    lines = ["# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per dispatch (HBM traffic)",
             f"# command: {command}",
             f"# scale: a {calib_bytes} B device copy reads FETCH_SIZE x {ff:.3f} and "
             f"WRITE_SIZE x {fw:.3f} bytes; both factors applied below", "",
             f"{'kernel':58s} {'fetch_MB':>10s} {'write_MB':>10s}"]
    for k, v in res.items():
        fb = "-" if v["fetch_bytes"] is None else f"{v['fetch_bytes'] / 1e6:10.2f}"
        wb = "-" if v["write_bytes"] is None else f"{v['write_bytes'] / 1e6:10.2f}"
        lines.append(f"{k:58s} {fb:>10s} {wb:>10s}")
    open(out_txt, "w").write("\n".join(lines) + "\n")


def _durations(db: str) -> dict:
    """{short kernel name: [duration us per dispatch]} from a kernel-trace database."""
    agg = defaultdict(list)
    for name, dur in _rows(db, "select name, duration from kernels"):
        agg[short_name(name)].append(dur / 1e3)
    return agg


# MI355X: 8 XCDs of 32 CUs x 4 SIMDs; one MOPS unit of SQ_INSTS_VALU_MFMA_MOPS_* is 512 flops.
# rocprofv3 reports GRBM_GUI_ACTIVE per dispatch summed over the 8 XCD instances.
SIMDS = 1024
XCDS = 8
MOPS_FLOPS = 512


def counters(pmc_db: str, trace_db: str, out_json: str, out_txt: str, command: str) -> None:
    """Per-kernel averages of every counter in a --pmc database, with the MFMA figures derived
    from them and the kernel durations of a --kernel-trace run of the same program:
      mfma_tflops_hw  (sum of SQ_INSTS_VALU_MFMA_MOPS_*) * 512 / average duration: the flops the
                      matrix cores executed, zero-padded work included
      mfma_busy       SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 * 1024 SIMDs): the fraction
                      of SIMD cycles with the MFMA unit busy while the GPU was active (rocprofv3's
                      MfmaUtil expression, which takes GRBM_GUI_ACTIVE of one XCD)
      clock_ghz       GRBM_GUI_ACTIVE / 8 / average duration: the engine clock the kernel ran at
                      (meaningful for kernels much longer than the counter set-up window)."""
    names = [r[0] for r in _rows(pmc_db, "select distinct counter_name from counters_collection")]
    per = {c: _counter(pmc_db, c) for c in names}
    durs = _durations(trace_db) if trace_db else {}
    res = {}
    kernels = sorted({k for c in per.values() for k in c})
    for name in kernels:
        if "copyBuffer" in name or "fillBuffer" in name or "at::native" in name:
            continue
        key = short_name(name)
        rec = {}
        for c in names:
            vals = [v for v, _ in per[c].get(name, [])]
            if vals:
                rec[c] = sum(vals) / len(vals)
        if not rec:
            continue
        d = durs.get(key)
        if d:
            rec["avg_us"] = sum(d) / len(d)
        mops = sum(rec.get(c, 0.0) for c in rec if c.startswith("SQ_INSTS_VALU_MFMA_MOPS_"))
        if mops and rec.get("avg_us"):
            rec["mfma_tflops_hw"] = mops * MOPS_FLOPS / (rec["avg_us"] * 1e-6) / 1e12
        if rec.get("SQ_VALU_MFMA_BUSY_CYCLES") is not None and rec.get("GRBM_GUI_ACTIVE"):
            xcd_cycles = rec["GRBM_GUI_ACTIVE"] / XCDS
            rec["mfma_busy"] = rec["SQ_VALU_MFMA_BUSY_CYCLES"] / (xcd_cycles * SIMDS)
            if rec.get("avg_us"):
                rec["clock_ghz"] = xcd_cycles / (rec["avg_us"] * 1e3)
        res[key] = rec
    doc = {"kernels": res, "command": command,
           "formulas": {"mfma_tflops_hw": "sum(SQ_INSTS_VALU_MFMA_MOPS_*) * 512 / avg duration",
                        "mfma_busy": "SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 * 1024 SIMDs)",
                        "clock_ghz": "GRBM_GUI_ACTIVE / 8 / avg duration"}}
    open(out_json, "w").write(json.dumps(doc, indent=1) + "\n")
    lines = ["# rocprofv3 --pmc counters, average per dispatch",
             f"# command: {command}",
             "# mfma_tflops_hw = sum(SQ_INSTS_VALU_MFMA_MOPS_*) * 512 / avg duration (kernel trace);",
             "# mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs * 1024 SIMDs);",
             "# clock_ghz = GRBM_GUI_ACTIVE / 8 / avg duration (GRBM_GUI_ACTIVE is summed over the",
             "# 8 XCDs; short kernels include the counter set-up window)", ""]
    for k, v in res.items():
        lines.append(k)
        for c, x in v.items():
            lines.append(f"    {c:36s} {x:16.4f}" if isinstance(x, float) else f"    {c:36s} {x}")
    open(out_txt, "w").write("\n".join(lines) + "\n")


def _last_per_kernel(rows, last: int, after: int = -1) -> dict:
    """{short name: [values of its last `last` dispatches]} from (dispatch order, name, value),
    counting only dispatches after dispatch `after`."""
    per = defaultdict(list)
    for d, name, val in sorted(rows, key=lambda r: r[0]):
        if d > after:
            per[name].append(val)
    return {short_name(k): v[-last:] for k, v in per.items()
            if "copyBuffer" not in k and "fillBuffer" not in k and "at::native" not in k}


def _trace_mark(trace_db: str) -> int:
    """Dispatch id of the calibration copy in a kernel trace: the device copy with the largest
    grid (host-to-device copies go through smaller staging blits)."""
    cols = [r[1] for r in _rows(trace_db, "pragma table_info(kernels)")]
    grid = [c for c in cols if c.startswith("grid") and c.endswith(("x", "size"))]
    if not grid:
        raise SystemExit(f"{trace_db}: no grid column in the kernels view ({cols})")
    rows = _rows(trace_db, f"select dispatch_id, {grid[0]} from kernels where name like '%copyBuffer%'")
    return max(rows, key=lambda r: r[1])[0] if rows else -1


def _calib_scale(db: str, counter: str, calib_bytes: int) -> tuple:
    """(bytes per counted byte, dispatch id) of the calibration copy: the largest device copy."""
    rows = _rows(db, "select dispatch_id, value, grid_size from counters_collection "
                     f"where counter_name = '{counter}' and kernel_name like '%copyBuffer%'")
    d, kib, _ = max(rows, key=lambda r: r[2])
    return calib_bytes / (float(kib) * 1024.0), d


def workload(name: str, trace_db: str, mfma_db: str, fetch_db: str, write_db: str, out_json: str,
             last: int, calib_bytes: int, command: str) -> None:
    """One workload's record from the four runs of `bench.py --profile-pass --workload NAME`,
    which makes its calibration copy between the warm-up launches and the measured ones: in each
    run only the dispatches after that copy count (so one-time work of the first launches, such
    as the GEMM library timing its candidate algorithms, stays out)."""
    trace = _rows(trace_db, "select dispatch_id, name, duration from kernels")
    durs = _last_per_kernel(trace, last, _trace_mark(trace_db))
    counters = [r[0] for r in _rows(mfma_db, "select distinct counter_name from counters_collection")]
    m_rows = _rows(mfma_db, "select dispatch_id, grid_size from counters_collection "
                            "where kernel_name like '%copyBuffer%'")
    m_mark = max(m_rows, key=lambda r: r[1])[0] if m_rows else -1
    per_counter = {c: _last_per_kernel(_rows(mfma_db, "select dispatch_id, kernel_name, value from "
                                                      f"counters_collection where counter_name = '{c}'"),
                                       last, m_mark) for c in counters}
    fs, f_mark = _calib_scale(fetch_db, "FETCH_SIZE", calib_bytes)
    ws, w_mark = _calib_scale(write_db, "WRITE_SIZE", calib_bytes)
    fetch = _last_per_kernel(_rows(fetch_db, "select dispatch_id, kernel_name, value from "
                                             "counters_collection where counter_name = 'FETCH_SIZE'"),
                             last, f_mark)
    write = _last_per_kernel(_rows(write_db, "select dispatch_id, kernel_name, value from "
                                             "counters_collection where counter_name = 'WRITE_SIZE'"),
                             last, w_mark)
    res = {}
    for k, d in durs.items():
        rec = {"dispatches": len(d), "avg_us": sum(d) / len(d) / 1e3}
        for c in counters:
            v = per_counter[c].get(k)
            if v:
                rec[c] = sum(v) / len(v)
        if k in fetch:
            rec["fetch_bytes"] = round(sum(fetch[k]) / len(fetch[k]) * 1024 * fs)
        if k in write:
            rec["write_bytes"] = round(sum(write[k]) / len(write[k]) * 1024 * ws)
        mops = sum(rec.get(c, 0.0) for c in rec if c.startswith("SQ_INSTS_VALU_MFMA_MOPS_"))
        if mops:
            rec["mfma_tflops_hw"] = mops * MOPS_FLOPS / (rec["avg_us"] * 1e-6) / 1e12
        if rec.get("SQ_VALU_MFMA_BUSY_CYCLES") is not None and rec.get("GRBM_GUI_ACTIVE"):
            xcd_cycles = rec["GRBM_GUI_ACTIVE"] / XCDS
            rec["mfma_busy"] = rec["SQ_VALU_MFMA_BUSY_CYCLES"] / (xcd_cycles * SIMDS)
            rec["clock_ghz"] = xcd_cycles / (rec["avg_us"] * 1e3)
        res[k] = rec
    doc = {"workload": name, "kernels": res, "command": command, "last_dispatches": last,
           "calibration": {"copy_bytes": calib_bytes, "fetch_scale": fs, "write_scale": ws}}
    open(out_json, "w").write(json.dumps(doc, indent=1) + "\n")


def merge(out_json: str, out_txt: str, inputs: list) -> None:
    docs = [json.loads(open(p).read()) for p in inputs]
    merged = {"workloads": {d["workload"]: d["kernels"] for d in docs},
              "commands": {d["workload"]: d["command"] for d in docs},
              "calibration": {d["workload"]: d["calibration"] for d in docs},
              "formulas": {"avg_us": "mean kernel-trace duration of the last dispatches",
                           "fetch_bytes / write_bytes": "FETCH_SIZE / WRITE_SIZE (KiB) x 1024 x the "
                                                        "scale a 256 MiB device copy gives",
                           "mfma_tflops_hw": "sum(SQ_INSTS_VALU_MFMA_MOPS_*) * 512 / avg_us",
                           "mfma_busy": "SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 * 1024 SIMDs)",
                           "clock_ghz": "GRBM_GUI_ACTIVE / 8 / avg_us"}}
    open(out_json, "w").write(json.dumps(merged, indent=1) + "\n")
    lines = ["# rocprofv3 per-workload kernel records: the last dispatches of each kernel in a "
             "bench.py --profile-pass --workload W run",
             "# durations from --kernel-trace; counters from one --pmc run per counter set; HBM "
             "bytes scaled by a 256 MiB device copy", ""]
    for d in docs:
        lines.append(f"## {d['workload']}")
        lines.append(f"# commands: {d['command']}")
        lines.append(f"{'kernel':52s} {'avg_us':>9s} {'fetch_MB':>9s} {'write_MB':>9s} "
                     f"{'mfma_busy':>9s} {'hw_TF/s':>8s} {'GHz':>5s}")
        for k, r in sorted(d["kernels"].items(), key=lambda kv: -kv[1]["avg_us"]):
            def f(key, scale=1.0, fmt="{:9.2f}"):
                v = r.get(key)
                return fmt.format(v * scale) if v is not None else f"{'-':>9s}"
            lines.append(f"{k:52s} {r['avg_us']:9.2f} {f('fetch_bytes', 1e-6)} "
                         f"{f('write_bytes', 1e-6)} {f('mfma_busy', 1.0, '{:9.3f}')} "
                         f"{f('mfma_tflops_hw', 1.0, '{:8.1f}')} {f('clock_ghz', 1.0, '{:5.2f}')}")
        lines.append("")
    open(out_txt, "w").write("\n".join(lines) + "\n")


def main() -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("db")
    s.add_argument("out")
    s.add_argument("--command", default="")
    c = sub.add_parser("counters")
    c.add_argument("pmc_db")
    c.add_argument("trace_db")
    c.add_argument("out_json")
    c.add_argument("out_txt")
    c.add_argument("--command", default="")
    t = sub.add_parser("traffic")
    t.add_argument("fetch_db")
    t.add_argument("write_db")
    t.add_argument("out_json")
    t.add_argument("out_txt")
    t.add_argument("--calib-bytes", type=int, default=256 << 20)
    t.add_argument("--command", default="")
    w = sub.add_parser("workload")
    for arg in ("name", "trace_db", "mfma_db", "fetch_db", "write_db", "out_json"):
        w.add_argument(arg)
    w.add_argument("--last", type=int, default=3)
    w.add_argument("--calib-bytes", type=int, default=256 << 20)
    w.add_argument("--command", default="")
    m = sub.add_parser("merge")
    m.add_argument("out_json")
    m.add_argument("out_txt")
    m.add_argument("inputs", nargs="+")
    a = ap.parse_args()
    if a.cmd == "workload":
        workload(a.name, a.trace_db, a.mfma_db, a.fetch_db, a.write_db, a.out_json, a.last,
                 a.calib_bytes, a.command)
        return
    if a.cmd == "merge":
        merge(a.out_json, a.out_txt, a.inputs)
        return
    if a.cmd == "stats":
        stats(a.db, a.out, a.command)
    elif a.cmd == "counters":
        counters(a.pmc_db, a.trace_db, a.out_json, a.out_txt, a.command)
    else:
        traffic(a.fetch_db, a.write_db, a.out_json, a.out_txt, a.calib_bytes, a.command)


if __name__ == "__main__":
    main()
