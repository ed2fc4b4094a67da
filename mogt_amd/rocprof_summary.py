"""Summaries of ``rocprofv3`` runs of this library's kernels, as committed text.

Reads the CSV output of up to three runs of the same command:

* ``--trace DIR``: ``rocprofv3 --kernel-trace --stats --output-format csv``
  (per-dispatch start / end timestamps, grid, registers);
* ``--fetch DIR`` and ``--write DIR``: ``rocprofv3 --pmc FETCH_SIZE`` and
  ``--pmc WRITE_SIZE`` (KiB per dispatch between L2 and the memory fabric).

The counters are calibrated on a plain device copy of known size in the same
runs (``bench.py --calib-copy`` copies 256 MiB five times): each counter is
scaled so the copy reads / writes exactly 256 MiB.  Kernels are grouped by
name (template arguments included) and launch shape.

The summary names the build it describes: the loaded library's build id and
the hashes of the sources behind the profiled kernel (``--sources``), taken
from the manifest compiled into the library (``mogt_build_manifest``).
``bench.py`` accepts a traffic figure only from a profile whose source hashes
match the library it runs.

Usage (after the three runs)::

    python -m mogt_amd.rocprof_summary --trace T --fetch F --write W \\
        --kernel 'diag_scan_kernel<0, float, float, float, 2, 32, 32, 8, false>' \\
        --algorithmic-bytes 301989888 --sources diag_kernel.h,diag_f32.hip,diag_scan.hip,common.h \\
        --title '...' --cmd '...' --cmd '...' [--bench-log LOG]
"""
from __future__ import annotations

import argparse
import csv
import shlex
import sys
import json
import re
import statistics
from collections import defaultdict
from pathlib import Path

COPY_KIB = 262144.0   # bench.py --calib-copy: 256 MiB each way


def _csv(dirpath: str | None, suffix: str) -> list[dict]:
    if not dirpath:
        return []
    files = sorted(Path(dirpath).rglob(f"*{suffix}"))
    rows: list[dict] = []
    for f in files:
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def short_name(name: str) -> str:
    """Kernel name without the parameter list (template arguments kept)."""
    # the parenthesis of an anonymous namespace is not a parameter list
    name = name.replace("(anonymous namespace)::", "")
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            name = name[:i]
            break
    for prefix in ("void ", "__global__ void "):
        if name.startswith(prefix):
            name = name[len(prefix):]
    return name.replace("mogt::", "").replace("(anonymous namespace)::", "").strip()


def display_name(name: str) -> str:
    """Table label: library GEMM kernels (Tensile names, hundreds of
    characters) by their macro tile, everything else as is."""
    if name.startswith(("Cijk_", "Custom_Cijk_")):
        m = re.search(r"_MT(\d+x\d+x\d+)_", name)
        return f"library GEMM MT{m.group(1)}" if m else "library GEMM"
    return name


def trace_table(rows: list[dict]) -> dict:
    """(name, work-groups, WG size) -> durations in microseconds + registers."""
    out: dict = defaultdict(lambda: {"us": [], "vgpr": 0, "agpr": 0, "lds": 0, "scratch": 0})
    for r in rows:
        wg = int(r["Workgroup_Size_X"]) * int(r.get("Workgroup_Size_Y", 1) or 1)
        grid = int(r["Grid_Size_X"]) * int(r.get("Grid_Size_Y", 1) or 1) * int(r.get("Grid_Size_Z", 1) or 1)
        key = (short_name(r["Kernel_Name"]), grid // max(wg, 1), wg)
        e = out[key]
        e["us"].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
        e["vgpr"] = int(r.get("VGPR_Count", 0) or 0)
        e["agpr"] = int(r.get("Accum_VGPR_Count", 0) or 0)
        e["lds"] = int(r.get("LDS_Block_Size", 0) or 0)
        e["scratch"] = int(r.get("Scratch_Size", 0) or 0)
    return out


def counter_table(rows: list[dict], counter: str) -> tuple[dict, float | None]:
    """(name, work-groups, WG size) -> mean KiB per dispatch; and the copy's mean."""
    per: dict = defaultdict(list)
    copies: list[tuple[int, float]] = []
    for r in rows:
        if r["Counter_Name"] != counter:
            continue
        v = float(r["Counter_Value"])
        wg = int(r["Workgroup_Size"])
        key = (short_name(r["Kernel_Name"]), int(r["Grid_Size"]) // max(wg, 1), wg)
        per[key].append(v)
        if "copyBuffer" in r["Kernel_Name"]:
            copies.append((int(r["Dispatch_Id"]), v))
    # the calibration copies are the process's first five copy dispatches
    # (bench.py --calib-copy runs them before anything else)
    first = [v for _, v in sorted(copies)[:5]]
    return ({k: sum(v) / len(v) for k, v in per.items()},
            (sum(first) / len(first)) if first else None)


def mfma_table(rows: list[dict]) -> dict:
    """(name, work-groups, WG size) -> mean per dispatch of each counter of an
    MFMA pass (SQ_INSTS_MFMA, SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE)."""
    per: dict = defaultdict(lambda: defaultdict(list))
    for r in rows:
        wg = int(r["Workgroup_Size"])
        key = (short_name(r["Kernel_Name"]), int(r["Grid_Size"]) // max(wg, 1), wg)
        per[key][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return {k: {c: sum(v) / len(v) for c, v in d.items()} for k, d in per.items()}


SIMDS = 1024          # MI355X: 256 CUs x 4 SIMDs
XCDS = 8              # GRBM_GUI_ACTIVE is summed over the XCDs


def mfma_busy(c: dict) -> float | None:
    """Fraction of SIMD cycles with the MFMA unit busy during the dispatch."""
    busy, active = c.get("SQ_VALU_MFMA_BUSY_CYCLES"), c.get("GRBM_GUI_ACTIVE")
    if not busy or not active:
        return None
    return busy / (SIMDS * active / XCDS)


def per_step_lines(rows: list[dict], steps: int, top: int) -> list[str]:
    """Kernel time per step of a run of `steps` steps (every dispatch of the
    run, warm-up and set-up included, divided by `steps`): by group (this
    library's kernels, library GEMMs, everything else), then by kernel."""
    groups: dict = defaultdict(float)
    per: dict = defaultdict(list)
    for r in rows:
        raw = r["Kernel_Name"]
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
        name = short_name(raw)
        if name.startswith(("Cijk_", "Custom_Cijk_")):
            grp = "hipBLASLt GEMMs"
        elif "mogt::" in raw:
            grp = "HIP kernels of this library"
        else:
            grp = "PyTorch kernels and copies"
        groups[grp] += us
        per[display_name(name)].append(us)
    total = sum(groups.values())
    out = [f"{total / steps:.0f} us of kernels per step", "", "| Group | us per step | share |", "|---|---|---|"]
    for g, us in sorted(groups.items(), key=lambda kv: -kv[1]):
        out.append(f"| {g} | {us / steps:.0f} | {us / total:.0%} |")
    out += ["", "| Kernel | Calls per step | Avg us | us per step |", "|---|---|---|---|"]
    ranked = sorted(per.items(), key=lambda kv: -sum(kv[1]))
    for name, d in ranked[:top or len(ranked)]:
        out.append(f"| `{name[:100]}` | {len(d) / steps:.1f} | {statistics.mean(d):.1f} | {sum(d) / steps:.0f} |")
    return out + [""]


def summarize(args) -> str:
    from . import _build, _lib

    trace = trace_table(_csv(args.trace, "kernel_trace.csv"))
    fetch, fcopy = counter_table(_csv(args.fetch, "counter_collection.csv"), "FETCH_SIZE")
    write, wcopy = counter_table(_csv(args.write, "counter_collection.csv"), "WRITE_SIZE")
    mfma = mfma_table(_csv(args.mfma, "counter_collection.csv"))
    fscale = COPY_KIB / fcopy if fcopy else None
    wscale = COPY_KIB / wcopy if wcopy else None
    manifest = _lib.build_manifest()
    tree = _build.source_manifest()

    lines = [f"# {args.title}", ""]
    lines += ["Commands (each run alone, from /tmp with `TMPDIR=/tmp`, repository at `$R`):", "", "```"]
    lines += list(args.cmd) + ["python3 -m mogt_amd.rocprof_summary " + shlex.join(args.argv), "```", ""]
    lines += [f"Build: library `{_lib.build_id()}`"
              + ("" if manifest == tree else " (NOT the checked-out sources: rebuild before profiling)"),
              "", "Sources behind the profiled kernel (name: SHA-256 prefix, from `mogt_build_manifest`):", ""]
    srcs = [s for s in args.sources.split(",") if s] + ["flags"]
    lines.append("kernel_sources=" + ",".join(f"{s}:{manifest.get(s, '?')}" for s in srcs))
    lines.append("")
    if fscale and wscale:
        lines.append(f"Counter calibration: the 256 MiB device copy reads FETCH_SIZE {fcopy:.1f} KiB and "
                     f"WRITE_SIZE {wcopy:.1f} KiB; bytes = FETCH_SIZE x {fscale:.4f} + WRITE_SIZE x "
                     f"{wscale:.4f} (KiB x 1024).")
        lines.append("")

    if args.per_step:
        lines += per_step_lines(_csv(args.trace, "kernel_trace.csv"), args.per_step, args.top)
        if args.note:
            lines += [args.note, ""]
        return "\n".join(lines)

    hdr = "| Kernel | WGs | WG size | VGPR | AGPR | LDS B | scratch B/lane | dispatches | avg us | median us | min us | max us |"
    sep = "|---|---|---|---|---|---|---|---|---|---|---|---|"
    if fscale and wscale:
        hdr += " read MB | write MB |"
        sep += "---|---|"
    if mfma:
        hdr += " MFMA insts | MFMA busy |"
        sep += "---|---|"
    lines += [hdr, sep]
    keys = sorted(trace, key=lambda k: -sum(trace[k]["us"]))
    mine = [k for k in keys if not args.match or any(m in k[0] for m in args.match)]
    rest = mine[args.top:] if args.top else []
    if args.top:
        mine = mine[:args.top]
    for k in mine:
        e = trace[k]
        d = e["us"]
        row = (f"| `{display_name(k[0])}` | {k[1]} | {k[2]} | {e['vgpr']} | {e['agpr']} | {e['lds']} | {e['scratch']} | "
               f"{len(d)} | {statistics.mean(d):.2f} | {statistics.median(d):.2f} | {min(d):.2f} | {max(d):.2f} |")
        if fscale and wscale:
            rd = fetch.get(k)
            wr = write.get(k)
            row += (f" {rd * fscale * 1024 / 1e6:.1f} |" if rd is not None else " - |")
            row += (f" {wr * wscale * 1024 / 1e6:.1f} |" if wr is not None else " - |")
        if mfma:
            c = mfma.get(k, {})
            fr = mfma_busy(c)
            row += f" {c['SQ_INSTS_MFMA']:.0f} |" if "SQ_INSTS_MFMA" in c else " - |"
            row += f" {fr:.1%} |" if fr is not None else " - |"
        lines.append(row)
    if rest:
        lines.append(f"| {len(rest)} more kernels / launch shapes | | | | | | | "
                     f"{sum(len(trace[k]['us']) for k in rest)} | | | | |"
                     + (" | |" if fscale and wscale else "") + (" | |" if mfma else ""))
        lines.append("")
        lines.append(f"(The table lists the {args.top} kernels / launch shapes with the most total time; the "
                     f"other {len(rest)} add {sum(sum(trace[k]['us']) for k in rest) / 1e3:.1f} ms of the "
                     f"{sum(sum(v['us']) for v in trace.values()) / 1e3:.1f} ms traced.)")
    lines.append("")

    if args.kernel:
        cand = [k for k in trace if k[0] == args.kernel]
        if not cand:
            # a unique-enough substring: the matching kernel with the most time
            sub = [k for k in trace if args.kernel in k[0]]
            cand = sorted(sub, key=lambda c: -sum(trace[c]["us"]))[:1]
        if not cand:
            raise SystemExit(f"kernel {args.kernel!r} not in the trace; have: {sorted({k[0] for k in trace})}")
        k = max(cand, key=lambda c: len(trace[c]["us"]))
        d = trace[k]["us"]
        kv = {"kernel": k[0], "work_groups": k[1], "dispatches": len(d),
              "avg_us": round(statistics.mean(d), 3), "median_us": round(statistics.median(d), 3)}
        if args.algorithmic_bytes:
            kv["algorithmic_bytes_per_launch"] = args.algorithmic_bytes
            kv["achieved_gbs_from_avg"] = round(args.algorithmic_bytes / (kv["avg_us"] * 1e-6) / 1e9, 1)
            kv["frac_of_8tbs_from_avg"] = round(kv["achieved_gbs_from_avg"] / 8000.0, 4)
        if fscale and wscale and k in fetch and k in write:
            rd = fetch[k] * fscale * 1024
            wr = write[k] * wscale * 1024
            kv.update(fetch_size_kib_raw=round(fetch[k], 1), write_size_kib_raw=round(write[k], 1),
                      fetch_scale=round(fscale, 4), write_scale=round(wscale, 4),
                      read_bytes_per_launch=int(rd), write_bytes_per_launch=int(wr),
                      hbm_bytes_per_launch=int(rd + wr))
            if args.algorithmic_bytes:
                kv["traffic_over_algorithmic"] = round((rd + wr) / args.algorithmic_bytes, 4)
        if args.bench_log:
            for ln in Path(args.bench_log).read_text().splitlines():
                if ln.startswith("{") and '"metric"' in ln:
                    b = json.loads(ln)
                    kv["bench_ms_per_step_same_run"] = b["ms_per_step"]
                    kv["bench_value_gbs_same_run"] = b["value"]
        lines.append("Profiled kernel (key=value, read by bench.py):")
        lines.append("")
        lines += [f"{a}={b}" for a, b in kv.items()]
        lines.append("")
    if args.note:
        lines += [args.note, ""]
    return "\n".join(lines)


def main(argv=None) -> None:
    p = argparse.ArgumentParser(description="Summarise rocprofv3 CSV runs of this library's kernels")
    p.add_argument("--trace", required=True)
    p.add_argument("--fetch")
    p.add_argument("--write")
    p.add_argument("--mfma", help="a run of --pmc SQ_INSTS_MFMA SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES "
                                   "GRBM_GUI_ACTIVE (MFMA busy = busy cycles / (1024 SIMDs x cycles per XCD))")
    p.add_argument("--title", required=True)
    p.add_argument("--cmd", action="append", default=[])
    p.add_argument("--match", action="append", default=[],
                   help="substrings of the kernel names listed in the table (default: every kernel)")
    p.add_argument("--kernel", help="full short name of the kernel the key=value block describes")
    p.add_argument("--top", type=int, default=0, help="list only this many kernels (most total time first)")
    p.add_argument("--per-step", type=int, default=0,
                   help="instead of the kernel table: kernel time per step of a run of this many steps")
    p.add_argument("--algorithmic-bytes", type=int, default=0)
    p.add_argument("--sources", default="")
    p.add_argument("--bench-log")
    p.add_argument("--note", default="")
    p.add_argument("--out")
    args = p.parse_args(argv)
    args.argv = [a for a in (sys.argv[1:] if argv is None else argv)]
    for flag in ("--out", "--title", "--cmd", "--note"):   # shown elsewhere in the summary
        while flag in args.argv:
            i = args.argv.index(flag)
            del args.argv[i:i + 2]
    if not args.match:
        args.match = [""]
    text = summarize(args)
    if args.out:
        Path(args.out).write_text(text)
    else:
        print(text)


if __name__ == "__main__":
    main()
