"""Summaries of rocprofv3 CSV output for the handoff kernels.

    python paged-batch-engine_amd/profiling.py stats <rocprof_dir> --out FILE --command "..."
    python paged-batch-engine_amd/profiling.py pmc <fetch_dir> <write_dir> --out FILE --command "..."
    python paged-batch-engine_amd/profiling.py legs <pmc_dir>... --launches K --out FILE --command "..."
    python paged-batch-engine_amd/profiling.py markers <trace_dir> --out FILE --command "..."
    python paged-batch-engine_amd/profiling.py req <pmc_dir> --grid G [--grid G2] --out FILE --command "..."

`stats` reads the kernel trace of a `rocprofv3 --kernel-trace --stats
--output-format csv` run and writes per-kernel call counts and durations.
`pmc` reads two counter runs (`--pmc FETCH_SIZE`, then `--pmc WRITE_SIZE`) of
`bench.py --calibrate`, which launches the config-2 handoff and a plain
contiguous copy of known size (CALIB_BYTES) with the same kernel; the plain
copy's counters give the bytes-per-unit factor used to turn the handoff's
counters into HBM bytes per launch.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics
from collections import defaultdict
from pathlib import Path

CALIB_BYTES = 256 << 20     # the --calibrate plain copy reads and writes this much
COPY_KERNEL = "copy_runs_kernel"


def _csv_rows(root: str, suffix: str):
    files = sorted(glob.glob(os.path.join(root, "**", f"*{suffix}"), recursive=True))
    if not files:
        raise FileNotFoundError(f"no *{suffix} under {root}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def _short(name: str) -> str:
    name = name.replace("(anonymous namespace)::", "").replace("void ", "")
    return name.split("(")[0]


def kernel_durations(root: str):
    """{(short kernel name, grid size): [durations ns]} from the kernel trace."""
    out = defaultdict(list)
    for r in _csv_rows(root, "kernel_trace.csv"):
        grid = int(r.get("Grid_Size_X", r.get("Grid_Size", 0)) or 0)
        dur = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        out[(_short(r["Kernel_Name"]), grid)].append(dur)
    return out


def stats(root: str, out: str, command: str, labels=None) -> None:
    """labels: {grid size: (workload label, algorithmic bytes per launch)}."""
    labels = labels or {}
    d = kernel_durations(root)
    lines = [f"# rocprofv3 kernel trace summary", f"command: {command}", "",
             f"{'kernel':<48} {'grid':>9} {'calls':>6} {'avg_us':>9} {'p50_us':>9} {'min_us':>9}"
             f"  {'workload':<28} {'GB/s':>8}"]
    for (name, grid), v in sorted(d.items(), key=lambda kv: -sum(kv[1])):
        label, alg = "", None
        for key, (lab, b) in labels.items():
            if key == (name, grid) or (isinstance(key, int) and key == grid and "pbe::" in name):
                label, alg = lab, b
        gbps = f"{alg / (statistics.mean(v) * 1e-9) / 1e9:8.1f}" if alg else ""
        lines.append(f"{name[:48]:<48} {grid:>9} {len(v):>6} {statistics.mean(v) / 1e3:>9.2f} "
                     f"{statistics.median(v) / 1e3:>9.2f} {min(v) / 1e3:>9.2f}  {label:<28} {gbps}")
    text = "\n".join(lines) + "\n"
    with open(out, "w") as fh:
        fh.write(text)
    print(text)


def _counter_per_dispatch(root: str, counter: str, kernel: str = COPY_KERNEL):
    """{grid size: [counter value per dispatch]} for kernels whose name holds `kernel`."""
    per = defaultdict(lambda: defaultdict(float))
    grids = {}
    for r in _csv_rows(root, "counter_collection.csv"):
        if kernel not in r["Kernel_Name"] or r["Counter_Name"] != counter:
            continue
        did = r["Dispatch_Id"]
        per[did][counter] += float(r["Counter_Value"])
        grids[did] = int(r.get("Grid_Size", 0) or 0)
    out = defaultdict(list)
    for did, v in per.items():
        out[grids[did]].append(v[counter])
    return out


def pmc(fetch_root: str, write_root: str, out: str, command: str, alg_bytes: int,
        handoff_grid: int, calib_grid: int, kernel: str = COPY_KERNEL,
        title: str = "HBM traffic of the config-2 handoff copy") -> None:
    f = _counter_per_dispatch(fetch_root, "FETCH_SIZE", kernel)
    w = _counter_per_dispatch(write_root, "WRITE_SIZE", kernel)
    fc = _counter_per_dispatch(fetch_root, "FETCH_SIZE")
    wc = _counter_per_dispatch(write_root, "WRITE_SIZE")
    f_h, f_c = statistics.median(f[handoff_grid]), statistics.median(fc[calib_grid])
    w_h, w_c = statistics.median(w[handoff_grid]), statistics.median(wc[calib_grid])
    f_scale = CALIB_BYTES / f_c  # bytes per counter unit (KiB nominal)
    w_scale = CALIB_BYTES / w_c
    traffic = f_h * f_scale + w_h * w_scale
    lines = [
        f"# rocprofv3 --pmc summary: {title}",
        f"command: {command}",
        f"kernel: {kernel} (grid {handoff_grid}); calibration: {COPY_KERNEL} (grid {calib_grid})",
        f"FETCH_SIZE per dispatch: handoff {f_h:.1f}, plain copy of {CALIB_BYTES} B {f_c:.1f}"
        f" -> {f_scale:.2f} bytes per unit",
        f"WRITE_SIZE per dispatch: handoff {w_h:.1f}, plain copy of {CALIB_BYTES} B {w_c:.1f}"
        f" -> {w_scale:.2f} bytes per unit",
        f"algorithmic_bytes_per_launch: {alg_bytes}",
        f"fetch_bytes_per_launch: {f_h * f_scale:.0f}",
        f"write_bytes_per_launch: {w_h * w_scale:.0f}",
        f"traffic_bytes_per_launch: {traffic:.0f}",
        f"traffic_over_algorithmic: {traffic / alg_bytes:.4f}",
    ]
    text = "\n".join(lines) + "\n"
    with open(out, "w") as fh:
        fh.write(text)
    print(text)


# bench.py --ceiling-legs K launches these legs K times each, in this order;
# the first three are the copy kernel, the last two the measurement streams.
LEGS = (("plan", COPY_KERNEL), ("sorted_destination", COPY_KERNEL), ("contiguous", COPY_KERNEL),
        ("read_only", "stream_read_kernel"), ("write_only", "stream_write_kernel"))


def _dispatch_counters(root: str):
    """[(dispatch id, kernel name, {counter: value summed over instances})] in
    dispatch order."""
    per, names = defaultdict(lambda: defaultdict(float)), {}
    for r in _csv_rows(root, "counter_collection.csv"):
        did = int(r["Dispatch_Id"])
        per[did][r["Counter_Name"]] += float(r["Counter_Value"])
        names[did] = r["Kernel_Name"]
    return [(d, names[d], dict(per[d])) for d in sorted(per)]


def _split_legs(items, launches: int, root: str):
    """{leg: [items]} from [(kernel name, item)] in dispatch order, by LEGS."""
    out = {}
    for leg_i, (leg, kern) in enumerate(LEGS):
        mine = [c for n, c in items if kern in n]
        if kern == COPY_KERNEL:  # the last 3k copy dispatches, in leg order
            mine = mine[-3 * launches:]
            k0 = leg_i * launches
            mine = mine[k0:k0 + launches]
        else:
            mine = mine[-launches:]
        if len(mine) != launches:
            raise RuntimeError(f"{root}: {leg}: {len(mine)} dispatches, expected {launches}")
        out[leg] = mine
    return out


def legs(roots, launches: int, out: str, command: str, trace: str | None = None,
         title: str = "config-2 handoff", alg_bytes: int = 0, copy_bytes: int = 0,
         kind: str = "DRAM-side counters") -> None:
    """Per-leg medians of every counter in the given --pmc runs of
    bench.py --ceiling-legs (one run per counter pass), and with `trace` (a
    --kernel-trace run of the same command) each leg's kernel durations."""
    table = defaultdict(dict)  # leg -> counter -> median
    for root in roots:
        rows = _dispatch_counters(root)
        for leg, mine in _split_legs([(n, c) for _, n, c in rows], launches, root).items():
            for counter in mine[0]:
                table[leg][counter] = statistics.median(m[counter] for m in mine)
    durations = {}
    if trace:
        rows = sorted(_csv_rows(trace, "kernel_trace.csv"), key=lambda r: int(r["Dispatch_Id"]))
        items = [(r["Kernel_Name"], int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) for r in rows]
        durations = {leg: statistics.mean(v) / 1e3 for leg, v in _split_legs(items, launches, trace).items()}
    counters = sorted({c for v in table.values() for c in v})
    w = max([len(c) for c in counters] + [26])
    lines = [f"# rocprofv3 --pmc summary: {kind} of the {title} and its "
             "ceiling legs", f"command: {command}",
             f"medians over {launches} launches per leg, each after a 1 GiB scrub; "
             "values summed over the counter's instances", "",
             f"{'counter':<{w}} " + " ".join(f"{leg:>19}" for leg, _ in LEGS)]
    if durations:
        lines.append(f"{'kernel avg_us (trace run)':<{w}} " +
                     " ".join(f"{durations[leg]:>19.2f}" for leg, _ in LEGS))
        if alg_bytes and copy_bytes:
            per = {"plan": alg_bytes, "sorted_destination": alg_bytes, "contiguous": alg_bytes,
                   "read_only": copy_bytes, "write_only": copy_bytes}
            lines.append(f"{'GB/s (algorithmic)':<{w}} " + " ".join(
                f"{per[leg] / (durations[leg] * 1e-6) / 1e9:>19.1f}" for leg, _ in LEGS))
    for c in counters:
        lines.append(f"{c:<{w}} " + " ".join(f"{table[leg].get(c, float('nan')):>19.0f}"
                                              for leg, _ in LEGS))
    # derived ratios where their inputs were collected
    def ratio(num, den, label):
        if all(num in table[l] and den in table[l] for l, _ in LEGS):
            lines.append(f"{label:<{w}} " + " ".join(
                f"{table[l][num] / max(table[l][den], 1):>19.3f}" for l, _ in LEGS))
    lines.append("")
    ratio("TCC_EA0_RDREQ_DRAM_CREDIT_STALL_sum", "TCC_EA0_RDREQ_sum", "rd credit stall / rd req")
    ratio("TCC_EA0_WRREQ_DRAM_CREDIT_STALL_sum", "TCC_EA0_WRREQ_sum", "wr credit stall / wr req")
    ratio("TCC_EA0_RDREQ_LEVEL_sum", "GRBM_GUI_ACTIVE", "rd req in flight (avg)")
    ratio("TCC_EA0_WRREQ_LEVEL_sum", "GRBM_GUI_ACTIVE", "wr req in flight (avg)")
    text = "\n".join(lines) + "\n"
    with open(out, "w") as fh:
        fh.write(text)
    print(text)


def markers(root: str, out: str, command: str) -> None:
    """roctx ranges of a rocprofv3 --marker-trace --kernel-trace run: per range
    name the count and durations, and per kernel how many of its dispatches
    ran entirely inside a range of each name (same host thread: the one that
    pushed the range and enqueued the kernel)."""
    ranges = defaultdict(list)  # name -> [(pid, start, end)]
    for r in _csv_rows(root, "marker_api_trace.csv"):
        name = r.get("Function") or r.get("Message") or ""
        ranges[name].append((r.get("Thread_Id", ""), int(r["Start_Timestamp"]),
                             int(r["End_Timestamp"])))
    kernels = defaultdict(list)
    for r in _csv_rows(root, "kernel_trace.csv"):
        kernels[_short(r["Kernel_Name"])].append((r.get("Thread_Id", ""), int(r["Start_Timestamp"]),
                                                  int(r["End_Timestamp"])))
    lines = ["# rocprofv3 --marker-trace --kernel-trace summary: roctx ranges around the handoff",
             f"command: {command}", "",
             f"{'range':<32} {'count':>6} {'median_us':>10} {'min_us':>9} {'max_us':>9}"]
    for name, v in sorted(ranges.items()):
        d = [(e - s) / 1e3 for _, s, e in v]
        lines.append(f"{name[:32]:<32} {len(v):>6} {statistics.median(d):>10.1f} {min(d):>9.1f} "
                     f"{max(d):>9.1f}")
    lines += ["", "kernel dispatches inside each range (start and end within it):",
              f"{'kernel':<40} {'dispatches':>10}  " + "  ".join(f"{n[:28]:>28}" for n in sorted(ranges))]
    for k, v in sorted(kernels.items(), key=lambda kv: -len(kv[1])):
        if "pbe::" not in k and "copy" not in k:
            continue
        inside = []
        for name in sorted(ranges):
            rs = ranges[name]
            inside.append(sum(any(p == rp and rs0 <= s and e <= re for rp, rs0, re in rs)
                              for p, s, e in v))
        lines.append(f"{k[:40]:<40} {len(v):>10}  " + "  ".join(f"{n:>28}" for n in inside))
    text = "\n".join(lines) + "\n"
    with open(out, "w") as fh:
        fh.write(text)
    print(text)


def req(root: str, grids, out: str, command: str, kernel: str = COPY_KERNEL) -> None:
    """Request counts at the memory interface per dispatch (a --pmc run of
    TCC_EA0_RDREQ / _32B and TCC_EA0_WRREQ / _64B): medians per grid, and the
    bytes per read request those give for the grid's known traffic."""
    rows = [(n, c) for _, n, c in _dispatch_counters(root) if kernel in n]
    lines = [f"# rocprofv3 --pmc summary: memory-interface request counts of {kernel}",
             f"command: {command}", ""]
    by_grid = defaultdict(list)
    for r in _csv_rows(root, "counter_collection.csv"):
        if kernel in r["Kernel_Name"]:
            by_grid[int(r.get("Grid_Size", 0) or 0)].append(int(r["Dispatch_Id"]))
    per = {d: c for d, _, c in _dispatch_counters(root)}
    for g in grids:
        ds = sorted(set(by_grid.get(g, [])))
        if not ds:
            raise RuntimeError(f"no {kernel} dispatch with grid {g}")
        med = {k: statistics.median(per[d][k] for d in ds) for k in per[ds[0]]}
        lines.append(f"grid {g} ({len(ds)} dispatches): " + ", ".join(
            f"{k} {v:.0f}" for k, v in sorted(med.items())))
    del rows
    text = "\n".join(lines) + "\n"
    with open(out, "w") as fh:
        fh.write(text)
    print(text)


def ceilings(bench_json: str, out: str, command: str) -> None:
    """The headline and its ceiling legs from one bench.py line (the last JSON
    line of its output), as a text summary."""
    line = [l for l in Path(bench_json).read_text().splitlines() if l.startswith("{")][-1]
    d = json.loads(line)
    c = d["ceilings"]
    rows = [("headline (the C2 plan)", d["latency_us"]["kernel_mean"], d["value"])]
    for k in ("sorted_destination", "contiguous_same_bytes", "slice_copy_no_run_list",
              "register_staged_copy"):
        leg = c.get(k) or d.get(k)
        if leg:
            rows.append((k, leg["us_mean"], leg["gbps"]))
    lines = ["# bench.py ceiling legs of the config-2 handoff (one run, mean kernel us)",
             f"command: {command}", "",
             f"{'leg':<32} {'us':>8} {'GB/s':>9}"]
    lines += [f"{n:<32} {u:>8.2f} {g:>9.1f}" for n, u, g in rows]
    v = c["vendor_memcpy"]
    lines.append(f"{'vendor_memcpy':<32} {v['us_mean']:>8.2f} {v['gbps']:>9.1f}   "
                 f"(after a read-only scrub: {v['us_mean_after_read_scrub']:.2f} us)")
    lines.append(f"{'read_only / write_only':<32} {c['read_only']['us_mean']:>8.2f} / "
                 f"{c['write_only']['us_mean']:.2f}   read then write: {c['read_then_write_us']:.2f}")
    ws = c["write_side"]
    lines.append(f"{'write_side (plan / contiguous)':<32} {ws['scattered_us']:>8.2f} / {ws['contiguous_us']:.2f}")
    lines.append(f"headline_over_best_of_sorted_and_vendor: {c['headline_over_best_of_sorted_and_vendor']}")
    lines.append(f"dispatch_only_us (empty kernel, the copy's grid): {c['dispatch_only_us']}")
    lines += ["", "wave timeline (times from the first wave's start, us; medians over launches):",
              f"{'':<28} {'plan':>10} {'contiguous':>11}"]
    t = c["wave_timeline"]
    for k in ("kernel_us", "first_slice_done_us", "p10_done_us", "p90_done_us",
              "last_slice_done_us", "steady_tbps_p10_p90", "load_wait_us_median",
              "store_wait_us_median"):
        lines.append(f"{k:<28} {t['plan'][k]:>10} {t['contiguous'][k]:>11}")
    text = "\n".join(lines) + "\n"
    Path(out).write_text(text)
    print(text)


def hostpaths(log: str, out: str, command: str) -> None:
    """The JSON line of bench.py --host-paths as a labelled table."""
    line = [l for l in Path(log).read_text().splitlines() if l.startswith("{")][-1]
    d = json.loads(line)
    g, r = d["generic_plan_form_us"], d["reference_call_order_us"]
    st = r["steps"]
    rows = [
        ("generic plan form (InProcKVBlockCopyConnector)", None),
        ("per-page BindComponents binding (BindManifestTransfers)", g["per_page_binding"]),
        ("template binding (BindManifestCopyOps)", g["copy_op_binding"]),
        ("pbe_copy_ops host call for the 17,640 component ops", g["copy_ops_call"]),
        ("connector submit -> drain", g["connector_submit_drain"]),
        *([("HIP TransferBackend, 315 page transfers (submit, drain)", g["hip_backend_315_transfers"]),
           ("the 17,640 ops, a hipMemcpyAsync each (reference pattern)", g["per_op_memcpy_17640"])]
          if "hip_backend_315_transfers" in g else []),
        ("", None),
        ("reference copy_shared_kv call order (serving::CopySharedKVToDecode)", None),
        ("append_slots, 28 layers (register_request + append_slots)", r["reserve_28_layers"]),
        ("end to end (reserve, manifest, copy, sync, commit_kv)", r["end_to_end"]),
        ("the copy and its wait alone (pbe_copy_shared_kv + sync)", r["copy_and_sync_alone"]),
        ("free_request afterwards", r["free_request"]),
        ("append_slots while 315 freed pages wait on fences", r["reserve_under_pending_fences"]),
        ("", None),
        ("the same steps through the same public calls, one timer between each (cold cache)", None),
        ("request copies (28 source lists)", st["request_copies"]),
        ("DecodeKVReservationManager::reserve (pages + manifest)", st["reserve_and_manifest"]),
        ("pbe_copy_shared_kv call (checks, runs, launch)", st["pbe_copy_shared_kv_call"]),
        ("stream wait (the kernel and its completion)", st["stream_wait"]),
        ("commit_kv", st["commit_kv"]),
    ]
    lines = [f"# Host costs of the handoff's C++ paths at config-2 size ({d['pages']} pages, "
             f"{d['layers']} layers), MI355X box", f"command: {command}",
             f"medians over {d['iterations']} iterations, microseconds", ""]
    for name, v in rows:
        lines.append(name if v is None else f"  {name:<58}{v:>8.1f}")
    lines += ["", "raw line:", line]
    text = "\n".join(lines) + "\n"
    Path(out).write_text(text)
    print(text)


def main() -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("root")
    s.add_argument("--out", required=True)
    s.add_argument("--command", required=True)
    s.add_argument("--label", action="append", default=[],
                   help="KERNEL_SUBSTRING:GRID=WORKLOAD:ALG_BYTES (repeatable)")
    p = sub.add_parser("pmc")
    p.add_argument("fetch_root")
    p.add_argument("write_root")
    p.add_argument("--out", required=True)
    p.add_argument("--command", required=True)
    p.add_argument("--alg-bytes", type=int, required=True)
    p.add_argument("--handoff-grid", type=int, required=True)
    p.add_argument("--calib-grid", type=int, required=True)
    p.add_argument("--kernel", default=COPY_KERNEL, help="substring of the measured kernel's name")
    p.add_argument("--title", default="HBM traffic of the config-2 handoff copy")
    q = sub.add_parser("legs")
    q.add_argument("roots", nargs="+")
    q.add_argument("--launches", type=int, required=True)
    q.add_argument("--out", required=True)
    q.add_argument("--command", required=True)
    q.add_argument("--trace", default=None, help="--kernel-trace run of the same command")
    q.add_argument("--title", default="config-2 handoff")
    q.add_argument("--kind", default="DRAM-side counters")
    q.add_argument("--alg-bytes", type=int, default=0)
    q.add_argument("--copy-bytes", type=int, default=0)
    rq = sub.add_parser("req")
    rq.add_argument("root")
    rq.add_argument("--grid", type=int, action="append", required=True)
    rq.add_argument("--out", required=True)
    rq.add_argument("--command", required=True)
    ce = sub.add_parser("ceilings")
    ce.add_argument("bench_json")
    ce.add_argument("--out", required=True)
    ce.add_argument("--command", required=True)
    hp = sub.add_parser("hostpaths")
    hp.add_argument("log")
    hp.add_argument("--out", required=True)
    hp.add_argument("--command", required=True)
    mk = sub.add_parser("markers")
    mk.add_argument("root")
    mk.add_argument("--out", required=True)
    mk.add_argument("--command", required=True)
    a = ap.parse_args()
    if a.cmd == "req":
        req(a.root, a.grid, a.out, a.command)
        return
    if a.cmd == "ceilings":
        ceilings(a.bench_json, a.out, a.command)
        return
    if a.cmd == "hostpaths":
        hostpaths(a.log, a.out, a.command)
        return
    if a.cmd == "markers":
        markers(a.root, a.out, a.command)
        return
    if a.cmd == "legs":
        legs(a.roots, a.launches, a.out, a.command, a.trace, a.title, a.alg_bytes, a.copy_bytes,
             a.kind)
        return
    if a.cmd == "stats":
        labels = {}
        if a.label:
            names = {k[0] for k in kernel_durations(a.root)}
            for spec in a.label:
                key, val = spec.split("=", 1)
                sub_name, grid = key.rsplit(":", 1)
                lab, alg = val.rsplit(":", 1)
                for n in names:
                    if sub_name in n:
                        labels[(n, int(grid))] = (lab, int(alg))
        stats(a.root, a.out, a.command, labels)
    else:
        pmc(a.fetch_root, a.write_root, a.out, a.command, a.alg_bytes, a.handoff_grid,
            a.calib_grid, a.kernel, a.title)


if __name__ == "__main__":
    main()
