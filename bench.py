"""Benchmark: prefill->decode KV handoff on one MI355X.

Workload: Qwen2.5-1.5B-shaped BF16 pool (28 layers, 2 KV
heads x 128, 16-token pages of 448 KiB) in a 2112 MiB arena; a 5040-token
prefix = 315 pages whose destination runs are uniform in 1..5 pages.

A step is one handoff launch over the device-resident run list (all layers'
K and V of all 315 pages). Before every step a 1 GiB scrub write evicts the
source and destination from L2 / MALL (Infinity Cache), so every step reads
from and writes to HBM; the scrub is outside the per-launch HIP-event timing.

Prints ONE JSON line. value = algorithmic bytes (read + write of every copied
page) / mean kernel duration, in GB/s. ms_per_step = that mean handoff kernel
latency. The CPU baseline is the oracle's restatement of the reference's
per-run memcpy loop (split_pd_engine.cpp:96-108), one thread, on a host copy of
the same pool and plan.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "paged-batch-engine_amd"))
sys.path.insert(0, str(ROOT))

PEAK_GBPS = 8000.0
METRIC = "KV handoff HBM GB/s (% of peak) + latency for 5040-tok Qwen2.5-1.5B prefix"
PMC_SUMMARY = ROOT / "profiles" / "handoff_copy_c2_pmc.txt"


def _traffic_from_profile():
    """HBM bytes per launch from the committed rocprofv3 --pmc summary (FETCH_SIZE
    + WRITE_SIZE of copy_runs_kernel, scaled by the plain-copy calibration)."""
    if not PMC_SUMMARY.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", PMC_SUMMARY.read_text(), re.M)
    return float(m.group(1)) if m else None


def _cpu_model() -> str:
    """The host CPU's model name from /proc/cpuinfo."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(w, host_arena, seconds: float):
    """Reference-faithful host copy: coalesce + one memcpy per run, 1 thread."""
    from oracle import oracle as O
    import numpy as np
    g = w.geometry
    reps, t0 = 0, time.perf_counter()
    O.copy_handoff(host_arena, w.src_ids, w.dst_ids, g.half(), g.layers)  # first touch
    t0 = time.perf_counter()
    while True:
        O.copy_handoff(host_arena, w.src_ids, w.dst_ids, g.half(), g.layers)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per = el / reps
    # the same port on every host core: the page list cut into one contiguous
    # share per thread (pages are independent), ctypes releasing the GIL
    from concurrent.futures import ThreadPoolExecutor
    threads = max(1, min(16, os.cpu_count() or 1))
    cut = np.linspace(0, len(w.src_ids), threads + 1).astype(int)
    shares = [(w.src_ids[cut[i]:cut[i + 1]], w.dst_ids[cut[i]:cut[i + 1]]) for i in range(threads)]
    with ThreadPoolExecutor(threads) as pool:
        def one_handoff():
            list(pool.map(lambda sd: O.copy_handoff(host_arena, sd[0], sd[1], g.half(), g.layers), shares))
        one_handoff()
        treps, t0 = 0, time.perf_counter()
        while True:
            one_handoff()
            treps += 1
            tel = time.perf_counter() - t0
            if tel >= seconds / 2:
                break
    tper = tel / treps
    # generic plan form: 2*layers component memcpys of `half` bytes per page
    # (ExecuteCpuTransfer over the bound manifest, transfer_plan.cpp:392-403)
    creps, t0 = 0, time.perf_counter()
    while True:
        O.copy_components(host_arena, w.src_ids, w.dst_ids, g.half(), g.layers)
        creps += 1
        cel = time.perf_counter() - t0
        if cel >= seconds / 2:
            break
    cper = cel / creps
    # the same generic path as the reference's own code runs it: oracle/_ref
    # (its TransferPlanner / BoundTransfer / ExecuteCpuTransfer compiled from
    # its sources), binding included, on the same host arena and plan
    ref = {"skipped": "oracle/_ref not built"}
    if O.REF_LIB_PATH.exists():
        after_port = host_arena.copy()
        geo = (g.layers, g.kv_heads, g.head_dim)
        t0 = time.perf_counter()
        ok = O.ref_cpu_handoff(O.REF_LIB_PATH, host_arena, w.src_ids, w.dst_ids, *geo) == w.copied_bytes()
        one = time.perf_counter() - t0
        rreps = max(1, int(seconds / 2 / max(one, 1e-6)))
        t0 = time.perf_counter()
        ok = ok and O.ref_cpu_handoff(O.REF_LIB_PATH, host_arena, w.src_ids, w.dst_ids, *geo,
                                      repeats=rreps) == w.copied_bytes()
        rel = time.perf_counter() - t0
        rper = rel / rreps
        ref = {"value": round(w.algorithmic_bytes() / rper / 1e9, 3), "unit": "GB/s", "cores": 1,
               "kind": "reference-with-glog-stub", "ms_per_handoff": round(rper * 1e3, 3),
               "what": "the reference's TransferPlanner + per-page BoundTransfer::BindComponents + "
                       "ExecuteCpuTransfer (pd_handoff.cpp:192-213), compiled from its sources "
                       "against the glog stand-in of its own CPU tests (test/cache_core/stubs): "
                       "a timing of the reference's code, not a parity pin",
               "same_bytes_as_port": bool(ok and np.array_equal(host_arena, after_port)),
               "sample": f"{rreps} handoffs in {rel:.1f} s"}
        # the same driver over this repository's drop-in TransferPlanner / BoundTransfer
        api = Path(__file__).resolve().parent / "paged-batch-engine_amd" / "lib" / "libpbe_api_driver.so"
        if api.exists():
            t0 = time.perf_counter()
            aok = O.ref_cpu_handoff(api, host_arena, w.src_ids, w.dst_ids, *geo,
                                    repeats=rreps) == w.copied_bytes()
            ael = time.perf_counter() - t0
            ref["drop_in_build"] = {"ms_per_handoff": round(ael / rreps * 1e3, 3),
                                    "value": round(w.algorithmic_bytes() / (ael / rreps) / 1e9, 3),
                                    "same_bytes_as_port": bool(aok and np.array_equal(host_arena, after_port))}
    return {"value": round(w.algorithmic_bytes() / per / 1e9, 3), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"{reps} handoffs of the config-2 plan (315 pages, {w.copied_bytes()} B "
                      f"copied each, one memcpy per coalesced run) in {el:.1f} s; "
                      f"{per * 1e3:.2f} ms per handoff",
            "ms_per_handoff": round(per * 1e3, 3),
            "all_host_cores": {"value": round(w.algorithmic_bytes() / tper / 1e9, 3), "unit": "GB/s",
                               "cores": threads, "kind": "port",
                               "ms_per_handoff": round(tper * 1e3, 3),
                               "sample": f"{treps} handoffs, the page list in {threads} shares"},
            "generic_plan_form": {"value": round(w.algorithmic_bytes() / cper / 1e9, 3),
                                  "unit": "GB/s", "ms_per_handoff": round(cper * 1e3, 3),
                                  "memcpys_per_handoff": w.pages * 2 * g.layers,
                                  "sample": f"{creps} handoffs in {cel:.1f} s"},
            "reference_generic_plan_form": ref}


class TimingEvents:
    """HIP timing events created with hipEventDisableSystemFence. A default
    event runs a system-scope release (L2 writeback and invalidate) when it
    completes; that fence lands inside the measured interval and adds ~2 us to
    a ~50 us kernel. The flag exists for events used only to measure time."""
    FLAGS = 0x20000000  # hipEventDisableSystemFence (timing stays enabled)

    def __init__(self, n: int):
        import ctypes as C
        self.C = C
        self.hip = C.CDLL("libamdhip64.so.7")
        self.hip.hipEventCreateWithFlags.argtypes = [C.POINTER(C.c_void_p), C.c_uint]
        self.hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.hip.hipEventDestroy.argtypes = [C.c_void_p]
        self.ev = []
        for _ in range(n):
            e = C.c_void_p()
            rc = self.hip.hipEventCreateWithFlags(C.byref(e), self.FLAGS)
            if rc != 0:
                raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
            self.ev.append(e)

    def handle(self, i: int) -> int:
        return self.ev[i].value

    def record(self, i: int, stream: int) -> None:
        if self.hip.hipEventRecord(self.ev[i], self.C.c_void_p(stream)) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed_ms(self, i: int, j: int) -> float:
        ms = self.C.c_float()
        if self.hip.hipEventElapsedTime(self.C.byref(ms), self.ev[i], self.ev[j]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return float(ms.value)

    def close(self) -> None:
        for e in self.ev:
            self.hip.hipEventDestroy(e)
        self.ev = []


def _timed(torch, stream, scrub, fn, n, scrub_fn=None):
    """Mean/min event time (ms) of fn() over n cold launches (scrub before
    each: a 1 GiB fill unless scrub_fn is given), between fence-free timing
    events recorded on the stream."""
    import numpy as np
    ev = TimingEvents(2 * (n + 2))
    sp = stream.cuda_stream
    ts = []
    for i in range(n + 2):
        if scrub_fn is None:
            scrub.fill_(i & 0xff)
        else:
            scrub_fn(i)
        ev.record(2 * i, sp)
        fn()
        ev.record(2 * i + 1, sp)
        torch.cuda.synchronize()
        if i >= 2:
            ts.append(ev.elapsed_ms(2 * i, 2 * i + 1))
    ev.close()
    return float(np.mean(ts)), float(np.min(ts))


def _kernel_timed(torch, scrub, launch, n):
    """Mean/min kernel duration (ms) of n cold launches (1 GiB scrub before
    each), between fence-free events the runtime stamps at the kernel's own
    start and end: launch(start_event, stop_event) must launch through
    hipExtLaunchKernel (RunList.copy_timed, the ceiling kernels). The same
    method as the headline, so the legs compare like for like."""
    import numpy as np
    ev = TimingEvents(2)
    ts = []
    for i in range(n + 2):
        scrub.fill_(i & 0xff)
        launch(ev.handle(0), ev.handle(1))
        torch.cuda.synchronize()
        if i >= 2:
            ts.append(ev.elapsed_ms(0, 1))
    ev.close()
    return float(np.mean(ts)), float(np.min(ts))


def gpu_reference_pattern(torch, stream, scrub, base, runs, g, alg, n, scrub_each):
    """Times the reference's copy loop as the reference issues it, on this GPU:
    one hipMemcpyAsync (device to device) per coalesced run, on one stream,
    between two events, plus the end-to-end time including the host loop and
    the final stream synchronize. Uses the HIP runtime already loaded by torch."""
    import ctypes as C
    import numpy as np
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    hip.hipMemcpyAsync.restype = C.c_int
    half, page = g.half(), g.page_bytes()
    calls = [(base + d * half, base + s * half, k * page) for s, d, k in runs]
    sp = C.c_void_p(stream.cuda_stream)

    def issue():
        for dst, src, nbytes in calls:
            rc = hip.hipMemcpyAsync(dst, src, nbytes, 3, sp)  # hipMemcpyDeviceToDevice
            if rc != 0:
                raise RuntimeError(f"hipMemcpyAsync failed with {rc}")

    issue()
    torch.cuda.synchronize()
    tev = TimingEvents(2 * n)
    ev, wall = [], []
    for i in range(n):
        if scrub_each:
            scrub.fill_(i & 0xff)
        torch.cuda.synchronize()
        t = time.perf_counter()
        tev.record(2 * i, stream.cuda_stream)
        issue()
        tev.record(2 * i + 1, stream.cuda_stream)
        stream.synchronize()
        wall.append(time.perf_counter() - t)
        ev.append(tev.elapsed_ms(2 * i, 2 * i + 1))
    tev.close()
    us = float(np.mean(ev)) * 1e3
    return {"what": "one hipMemcpyAsync per coalesced run on this GPU (the reference's loop)",
            "calls": len(calls), "us_mean": round(us, 2),
            "gbps": round(alg / (us * 1e-6) / 1e9, 1),
            "e2e_us_p50": round(float(np.median(wall)) * 1e6, 1)}


def host_paths_timing():
    """JSON line of lib/pbe_host_paths (tests/cpp/bench_host_paths.cpp) run as
    a child process, or None when it is not built."""
    import subprocess
    exe = Path(__file__).resolve().parent / "paged-batch-engine_amd" / "lib" / "pbe_host_paths"
    if not exe.exists():
        print(f"bench.py: {exe} is missing; the reference call order is not timed", file=sys.stderr)
        return None
    out = subprocess.run([str(exe)], stdout=subprocess.PIPE, timeout=300, check=True, text=True)
    return json.loads(out.stdout.strip().splitlines()[-1])


def measure_ceilings(torch, P, w, runs, kv, arena, scrub, alg: int, n: int) -> dict:
    """Ceilings the config-2 kernel time is held against, measured in this run
    on the same byte count with the same 1 GiB write scrub before each launch:
      sorted_destination  the same kernel and the plan's own source runs, the
                          destinations packed into one ascending contiguous
                          region (what the decode allocator's page placement
                          costs);
      vendor_memcpy       one hipMemcpyAsync device-to-device of the same bytes,
                          contiguous on both sides (also after a read-only scrub,
                          which the vendor copy is sensitive to);
      read_only/write_only the copy kernel's two halves alone
                          (lib/libpbe_ceiling.so): a copy's steady state cannot
                          beat HBM's rate for either stream at this size;
      register_staged_copy a contiguous copy whose waves each read 32 KiB before
                          writing it, the test of whether separating the two
                          streams in time pays;
      write_side          a cache-resident source written to the plan's scattered
                          destinations and to a contiguous region: the write path
                          alone (C2's runs are at most 5 pages, the source's size)."""
    import ctypes as C
    import numpy as np
    g = w.geometry
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    nbytes = w.pages * g.page_bytes()
    out = {}
    # (b) plan sources, contiguous ascending destination in a separate buffer
    dbuf = torch.empty(nbytes, dtype=torch.uint8, device=arena.device)
    dview = P.view_of(dbuf.data_ptr(), nbytes)
    sview = P.view_of(arena.data_ptr(), arena.numel())
    stride = 2 * g.layers
    packed, at = [], 0
    for s_id, _d, k in runs:
        packed.append((s_id, at * stride, k))
        at += k
    with P.RunList.bf16(sview, dview, packed, kv) as srl:
        ms = _kernel_timed(torch, scrub, lambda a, b: srl.copy_timed(sp, a, b), n)
    out["sorted_destination"] = {
        "what": "same kernel, the plan's source runs, destinations packed into one ascending "
                "contiguous region", "runs": len(packed),
        "us_mean": round(ms[0] * 1e3, 2), "gbps": round(alg / (ms[0] * 1e-3) / 1e9, 1)}
    # the write side alone: a 5-page source that stays cache-resident after
    # its first read, copied into the plan's destinations and into one
    # contiguous region (reads nearly free, so the difference is what the
    # scattered destinations cost the writes)
    hot = torch.empty(5 * g.page_bytes(), dtype=torch.uint8, device=arena.device)
    hview = P.view_of(hot.data_ptr(), hot.numel())
    hot_runs = [(0, d, k) for _s, d, k in runs]
    with P.RunList.bf16(hview, sview, hot_runs, kv) as hrl:
        ms_scat = _kernel_timed(torch, scrub, lambda a, b: hrl.copy_timed(sp, a, b), n)
    with P.RunList.bf16(hview, dview, [(0, pk[1], pk[2]) for pk in packed], kv) as hrl:
        ms_cont = _kernel_timed(torch, scrub, lambda a, b: hrl.copy_timed(sp, a, b), n)
    del hot
    out["write_side"] = {
        "what": "a cache-resident 5-page source copied to the plan's destinations / to one "
                "contiguous region (the plan's run lengths): the write path alone",
        "scattered_us": round(ms_scat[0] * 1e3, 2), "contiguous_us": round(ms_cont[0] * 1e3, 2)}
    # (a) vendor copy of the same bytes
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    hip.hipMemcpyAsync.restype = C.c_int

    def vendor():
        if hip.hipMemcpyAsync(dbuf.data_ptr(), arena.data_ptr(), nbytes, 3, C.c_void_p(sp)) != 0:
            raise RuntimeError("hipMemcpyAsync failed")
    ms = _timed(torch, stream, scrub, vendor, n)
    sums = scrub.view(torch.int64)
    ms_r = _timed(torch, stream, scrub, vendor, n, scrub_fn=lambda i: sums.sum())
    out["vendor_memcpy"] = {
        "what": "one hipMemcpyAsync device-to-device of the same bytes, contiguous; timed "
                "between events recorded on the stream around the call (the vendor copy "
                "cannot be bracketed at its kernel, so this includes a launch gap of ~1 us)",
        "us_mean": round(ms[0] * 1e3, 2), "gbps": round(alg / (ms[0] * 1e-3) / 1e9, 1),
        "us_mean_after_read_scrub": round(ms_r[0] * 1e3, 2),
        "gbps_after_read_scrub": round(alg / (ms_r[0] * 1e-3) / 1e9, 1)}
    # (c) the two halves of a copy alone
    so = Path(__file__).resolve().parent / "paged-batch-engine_amd" / "lib" / "libpbe_ceiling.so"
    if so.exists():
        cl = C.CDLL(str(so))
        cl.pbe_ceiling_read.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p,
                                        C.c_void_p, C.c_void_p]
        cl.pbe_ceiling_write.argtypes = [C.c_void_p, C.c_uint64, C.c_uint32, C.c_void_p,
                                         C.c_void_p, C.c_void_p]
        sink = torch.empty(1024, dtype=torch.uint8, device=arena.device)
        def leg(fn):
            return _kernel_timed(torch, scrub, fn, n)[0]
        r_ms = leg(lambda a, b: cl.pbe_ceiling_read(arena.data_ptr(), nbytes, sink.data_ptr(), sp, a, b))
        w_ms = leg(lambda a, b: cl.pbe_ceiling_write(dbuf.data_ptr(), nbytes, 7, sp, a, b))
        cl.pbe_ceiling_phase_copy.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p,
                                              C.c_void_p, C.c_void_p]
        p_ms = leg(lambda a, b: cl.pbe_ceiling_phase_copy(arena.data_ptr(), dbuf.data_ptr(), nbytes,
                                                          sp, a, b))
        cl.pbe_ceiling_slice_copy.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p,
                                              C.c_void_p, C.c_void_p]
        t_ms = leg(lambda a, b: cl.pbe_ceiling_slice_copy(arena.data_ptr(), dbuf.data_ptr(), nbytes,
                                                          sp, a, b))
        out["read_only"] = {"what": "the copy kernel's loads alone over the same bytes",
                            "bytes": nbytes, "us_mean": round(r_ms * 1e3, 2),
                            "gbps": round(nbytes / (r_ms * 1e-3) / 1e9, 1)}
        out["write_only"] = {"what": "the copy kernel's stores alone over the same bytes",
                             "bytes": nbytes, "us_mean": round(w_ms * 1e3, 2),
                             "gbps": round(nbytes / (w_ms * 1e-3) / 1e9, 1)}
        out["read_then_write_us"] = round((r_ms + w_ms) * 1e3, 2)
        out["slice_copy_no_run_list"] = {
            "what": "the copy kernel's slices and cache policies over one contiguous span, "
                    "no run list to search", "us_mean": round(t_ms * 1e3, 2),
            "gbps": round(alg / (t_ms * 1e-3) / 1e9, 1)}
        out["register_staged_copy"] = {
            "what": "contiguous copy of the same bytes, each wave loading 32 KiB into registers "
                    "before storing it (long read-only then write-only bursts)",
            "us_mean": round(p_ms * 1e3, 2), "gbps": round(alg / (p_ms * 1e-3) / 1e9, 1)}
        out.update(wave_timeline(torch, cl, w, runs, arena, dbuf, scrub, sp, n))
    del dbuf
    return out


def wave_timeline(torch, cl, w, runs, arena, dbuf, scrub, sp, n: int) -> dict:
    """The copy at the product's one-region geometry (1 KiB slices, 512-thread
    workgroups) from the plan's contiguous sources into the plan's destinations
    and into one contiguous region, every wave stamping the 100 MHz real-time
    counter at its start, when its load returned and when its store completed
    (lib/libpbe_ceiling.so, timeline_copy_kernel); and an empty kernel with the
    same grid (the dispatch alone). Medians over n launches, each after the
    1 GiB scrub."""
    import ctypes as C
    import numpy as np
    g = w.geometry
    half, slice_bytes = g.half(), 1024
    per_page = g.page_bytes() // slice_bytes
    stride = 2 * g.layers
    cl.pbe_ceiling_timeline_copy.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p,
                                             C.c_void_p, C.c_void_p, C.c_void_p]
    cl.pbe_ceiling_empty.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
    src_ids = [r[0] for r in runs]
    assert all(src_ids[i + 1] == src_ids[i] + runs[i][2] * stride for i in range(len(runs) - 1)), \
        "the timeline legs need the plan's sources in one region"
    src = arena.data_ptr() + runs[0][0] * half
    n_slices = w.pages * per_page
    within = np.arange(per_page * max(r[2] for r in runs), dtype=np.uint64) * slice_bytes
    plan = np.concatenate([np.uint64(arena.data_ptr() + d * half) + within[:k * per_page]
                           for _s, d, k in runs])
    region = np.uint64(dbuf.data_ptr()) + np.arange(n_slices, dtype=np.uint64) * slice_bytes
    stamps = torch.empty(3 * n_slices, dtype=torch.int64, device=arena.device)
    ev = TimingEvents(2)
    res = {}
    for name, table in (("plan", plan), ("contiguous", region)):
        dst_of = torch.from_numpy(table.view(np.int64)).to(arena.device)
        rows = []
        for i in range(n + 2):
            scrub.fill_(i & 0xff)
            rc = cl.pbe_ceiling_timeline_copy(src, dst_of.data_ptr(), n_slices, stamps.data_ptr(),
                                              sp, ev.handle(0), ev.handle(1))
            if rc:
                raise RuntimeError(f"timeline copy failed ({rc})")
            torch.cuda.synchronize()
            if i < 2:
                continue
            t = stamps.cpu().numpy().reshape(-1, 3).astype(np.int64)
            t0 = t[:, 0].min()
            done = np.sort(t[:, 2] - t0) * 0.01  # us
            lo, hi = done[int(0.1 * n_slices)], done[int(0.9 * n_slices)]
            rows.append([ev.elapsed_ms(0, 1) * 1e3, done[0], lo, hi, done[-1],
                         0.8 * n_slices * 2 * slice_bytes / ((hi - lo) * 1e-6) / 1e12,
                         np.median(t[:, 1] - t[:, 0]) * 0.01, np.median(t[:, 2] - t[:, 1]) * 0.01])
        m = np.median(np.array(rows), axis=0)
        res[name] = {"kernel_us": round(m[0], 2), "first_slice_done_us": round(m[1], 2),
                     "p10_done_us": round(m[2], 2), "p90_done_us": round(m[3], 2),
                     "last_slice_done_us": round(m[4], 2), "steady_tbps_p10_p90": round(m[5], 3),
                     "load_wait_us_median": round(m[6], 2), "store_wait_us_median": round(m[7], 2)}
        del dst_of
    sink = torch.empty(4096, dtype=torch.uint8, device=arena.device)
    ts = []
    for i in range(n + 2):
        rc = cl.pbe_ceiling_empty(n_slices, sink.data_ptr(), sp, ev.handle(0), ev.handle(1))
        if rc:
            raise RuntimeError(f"empty kernel failed ({rc})")
        torch.cuda.synchronize()
        if i >= 2:
            ts.append(ev.elapsed_ms(0, 1) * 1e3)
    ev.close()
    return {"wave_timeline": {
                "what": "one-region copy geometry into the plan's destinations / one contiguous "
                        "region, every wave stamping the 100 MHz real-time counter at start, "
                        "load return and store completion; times from the first wave's start",
                **res},
            "dispatch_only_us": round(float(np.median(ts)), 2)}


LEG_ORDER = ("plan", "sorted_destination", "contiguous", "read_only", "write_only")


def ceiling_legs(torch, P, w, runs, kv, arena, scrub, rl, k: int) -> dict:
    """Launches each leg k times, in LEG_ORDER, each launch after the 1 GiB
    scrub: the workload's plan (config 2 or 3), the same sources into one contiguous ascending
    destination, the same bytes as one contiguous run, and the copy's
    read-only and write-only halves. Under rocprofv3 --pmc the copy kernel's
    dispatches are told apart by this order (profiling.py legs)."""
    import ctypes as C
    g = w.geometry
    sp = torch.cuda.current_stream().cuda_stream
    nbytes = w.pages * g.page_bytes()
    stride = 2 * g.layers
    dbuf = torch.empty(nbytes, dtype=torch.uint8, device=arena.device)
    dview = P.view_of(dbuf.data_ptr(), nbytes)
    sview = P.view_of(arena.data_ptr(), arena.numel())
    rl_own = rl is None
    if rl_own:
        rl = P.RunList.bf16(sview, sview, runs, kv)
    packed, at = [], 0
    for s_id, _d, n_pages in runs:
        packed.append((s_id, at * stride, n_pages))
        at += n_pages
    n_arena = w.arena_bytes // g.page_bytes()
    srl = P.RunList.bf16(sview, dview, packed, kv)
    crl = P.RunList.bf16(sview, sview, [(0, stride * (n_arena - w.pages), w.pages)], kv)
    so = Path(__file__).resolve().parent / "paged-batch-engine_amd" / "lib" / "libpbe_ceiling.so"
    cl = C.CDLL(str(so))
    cl.pbe_ceiling_read.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_void_p]
    cl.pbe_ceiling_write.argtypes = [C.c_void_p, C.c_uint64, C.c_uint32, C.c_void_p,
                                     C.c_void_p, C.c_void_p]
    sink = torch.empty(1024, dtype=torch.uint8, device=arena.device)
    legs = {
        "plan": lambda: rl.copy(sp),
        "sorted_destination": lambda: srl.copy(sp),
        "contiguous": lambda: crl.copy(sp),
        "read_only": lambda: cl.pbe_ceiling_read(arena.data_ptr(), nbytes, sink.data_ptr(), sp,
                                                 None, None),
        "write_only": lambda: cl.pbe_ceiling_write(dbuf.data_ptr(), nbytes, 7, sp, None, None),
    }
    for name in LEG_ORDER:
        for i in range(k):
            scrub.fill_(i & 0xff)
            rc = legs[name]()
            if rc:
                raise RuntimeError(f"{name}: launch failed ({rc})")
        torch.cuda.synchronize()
        print(f"leg {name}: {k} launches", file=sys.stderr, flush=True)
    srl.close()
    crl.close()
    if rl_own:
        rl.close()
    return {"workload": w.name, "legs": list(LEG_ORDER), "launches_each": k, "bytes": nbytes,
            "algorithmic_bytes": w.algorithmic_bytes(), "runs": len(runs)}


def measure_extra_configs(torch, P, W, scrub, n: int):
    """Kernel timings of the other handoff configurations (parity-test cases,
    reported beside the headline line)."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    out = []

    def rec(name, alg, ms, extra=None):
        r = {"workload": name, "algorithmic_bytes": alg, "kernel_us_mean": round(ms[0] * 1e3, 2),
             "kernel_us_min": round(ms[1] * 1e3, 2),
             "gbps": round(alg / (ms[0] * 1e-3) / 1e9, 1),
             "pct_of_peak": round(100 * alg / (ms[0] * 1e-3) / 1e9 / PEAK_GBPS, 1)}
        r.update(extra or {})
        out.append(r)
        print(json.dumps(r), file=sys.stderr, flush=True)

    for cfg in (1, 3, 5):
        w = W.CONFIGS[cfg](0)
        g = w.geometry
        kv = P.shape(g.layers, g.kv_heads, g.head_dim, g.page_tokens)
        seg = w.segment_bytes or w.arena_bytes
        bufs = [torch.empty(min(seg, w.arena_bytes - o), dtype=torch.uint8, device=dev)
                for o in range(0, w.arena_bytes, seg)]
        view = P.view_of([b.data_ptr() for b in bufs], w.arena_bytes, seg)
        runs = P.build_runs(w.src_ids, w.dst_ids, kv, 2, w.segment_bytes)
        rl = P.RunList.bf16(view, view, runs, kv)
        rec(w.name, w.algorithmic_bytes(), _timed(torch, stream, scrub, lambda: rl.copy(sp), n),
            {"pages": w.pages, "runs": len(runs), "launches": 1})
        rl.close()
        if cfg == 3:
            # generic plan form: 2*layers component copies of `half` bytes per
            # page in one op-list launch (op list staged per call, included)
            half = g.half()
            ops = P.op_array([(view.base[0] + (s + plane) * half,
                               view.base[0] + (d + plane) * half, half)
                              for s, d in zip(w.src_ids.tolist(), w.dst_ids.tolist())
                              for plane in range(2 * g.layers)])
            rec(w.name + "_component_ops", w.algorithmic_bytes(),
                _timed(torch, stream, scrub, lambda: P.copy_ops(ops, 0, sp), n),
                {"pages": w.pages, "ops": ops[1], "launches": 1,
                 "note": "includes host validation and op-list staging per call"})
        if cfg == 3:  # one launch per request
            lists = []
            for r in w.requests:
                rr = P.build_runs(r.src_ids, r.dst_ids, kv)
                lists.append(P.RunList.bf16(view, view, rr, kv))
            rec(w.name + "_per_request", w.algorithmic_bytes(),
                _timed(torch, stream, scrub, lambda: [x.copy(sp) for x in lists], n),
                {"pages": w.pages, "launches": len(lists)})
            for x in lists:
                x.close()
        del bufs

    out.extend(measure_fp8(torch, P, W, scrub, n))
    out.extend(measure_decode(torch, P, scrub, n))
    out.extend(measure_scatter(torch, P, scrub, n))
    return out


def measure_decode_loop(torch, P, scrub, n: int, batch: int = 64, seq: int = 5040):
    """The KV side of one whole decode step of a 28-layer Qwen2.5-1.5B over
    FP8 pages: per layer, the new token of every sequence written to its slot
    (pbe_scatter_kv) and the decode reader (split-K pass + combine), i.e. 84
    kernels per step. Timed eagerly and as one captured HIP graph replayed per
    step, and eagerly in the fused form (pbe_paged_decode_append: the reader
    writes the new token itself, 56 kernels per step)."""
    import numpy as np
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    L, H, D, kvm, B = 28, 2, 128, 6, 16
    blocks = (seq + 1 + B - 1) // B
    n_pages = batch * blocks
    half = B * H * D
    plane = B * H
    g = torch.Generator(device=dev)
    g.manual_seed(23)
    arena = torch.randint(0, 0x70, (n_pages * 2 * L * half,), generator=g, device=dev,
                          dtype=torch.uint8)
    scales = torch.rand(n_pages * 2 * L * plane, generator=g, device=dev) * 0.1 + 0.01
    perm = torch.randperm(n_pages, generator=g, device=dev).to(torch.int32)
    tables = (perm * (2 * L)).view(batch, blocks).contiguous()
    lens = torch.full((batch,), seq + 1, dtype=torch.int32, device=dev)
    slots = (tables[:, seq // B] * B + seq % B).contiguous()
    new_kv = torch.randn((2, batch, H * D), generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn((batch, H * kvm, D), generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    view = P.view_of(arena.data_ptr(), arena.numel())
    kv = P.shape(L, H, D)
    splits = P.decode_splits(batch, H, blocks, P.PBE_KV_FP8_E4M3)
    ws_bytes = P.decode_workspace_bytes(batch, H * kvm, D, splits)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    total, total_sc = arena.numel(), scales.numel() * 4

    def step(sp):
        for layer in range(L):
            ko, vo = 2 * layer * half, (2 * layer + 1) * half
            so, svo = 4 * 2 * layer * plane, 4 * (2 * layer + 1) * plane
            P.scatter_kv(new_kv[0].data_ptr(), new_kv[1].data_ptr(), P.PBE_IN_BF16, batch,
                         slots.data_ptr(), B, H, D, P.PBE_KV_FP8_E4M3, arena.data_ptr() + ko,
                         total - ko, arena.data_ptr() + vo, total - vo, scales.data_ptr() + so,
                         total_sc - so, scales.data_ptr() + svo, total_sc - svo, stream=sp)
            P.paged_decode(view, P.PBE_KV_FP8_E4M3, scales.data_ptr(), total_sc, kv, layer,
                           q.data_ptr(), out.data_ptr(), batch, H * kvm, tables.data_ptr(),
                           lens.data_ptr(), blocks, splits, ws.data_ptr(), ws_bytes, sp)

    def fused_step(sp):
        for layer in range(L):
            ko, vo = 2 * layer * half, (2 * layer + 1) * half
            so, svo = 4 * 2 * layer * plane, 4 * (2 * layer + 1) * plane
            P.paged_decode_append(arena.data_ptr() + ko, arena.data_ptr() + vo, total - vo,
                                  scales.data_ptr() + so, scales.data_ptr() + svo, total_sc - svo,
                                  P.PBE_KV_FP8_E4M3, H, D, new_kv[0].data_ptr(),
                                  new_kv[1].data_ptr(), q.data_ptr(), out.data_ptr(), batch,
                                  H * kvm, tables.data_ptr(), lens.data_ptr(), blocks, splits,
                                  ws.data_ptr(), ws_bytes, sp)

    eager_ms = _timed(torch, stream, scrub, lambda: step(stream.cuda_stream), n)
    fused_ms = _timed(torch, stream, scrub, lambda: fused_step(stream.cuda_stream), n)
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            step(side.cuda_stream)
    torch.cuda.synchronize()
    graph_ms = _timed(torch, stream, scrub, graph.replay, n)
    alg = L * (batch * (seq + 1) * H * (2 * D + 8) + 2 * q.numel() * 2 + batch * H * D * 2 * 2)
    r = {"workload": f"decode_step_28_layers_fp8_b{batch}_s{seq}", "algorithmic_bytes": alg,
         "splits": splits, "kernels_per_step": 3 * L,
         "eager_us_per_step": round(eager_ms[0] * 1e3, 1),
         "graph_us_per_step": round(graph_ms[0] * 1e3, 1),
         "fused_eager_us_per_step": round(fused_ms[0] * 1e3, 1), "fused_kernels_per_step": 2 * L,
         "graph_gbps": round(alg / (graph_ms[0] * 1e-3) / 1e9, 1)}
    print(json.dumps(r), file=sys.stderr, flush=True)
    del graph
    return [r]


def measure_scatter(torch, P, scrub, n: int):
    """The page writer (pbe_scatter_kv) on Qwen2.5-1.5B geometry (H=2, D=128,
    28 layers): the C2 prompt's 5040 tokens of one layer written to random
    page-major slots (BF16 pages, FP8 pages + scales), and one decode token for
    each of 64 sequences. Algorithmic bytes: K and V read, rows written (+ FP8
    scales), slot ids read."""
    import numpy as np
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    out = []
    L, H, D, B, layer, pages = 28, 2, 128, 16, 27, 400
    rng = np.random.default_rng(17)
    for tokens, fp8, name in ((5040, False, "scatter_c2_prompt_bf16_pages"),
                              (5040, True, "scatter_c2_prompt_fp8_pages"),
                              (64, True, "scatter_decode_b64_fp8_pages")):
        e_out = 1 if fp8 else 2
        half = B * H * D * e_out
        arena = torch.empty(pages * 2 * L * half, dtype=torch.uint8, device=dev)
        plane = B * H
        sc = torch.empty(pages * 2 * L * plane, dtype=torch.float32, device=dev)
        if tokens >= B:  # one sequence: consecutive slots of shuffled pages
            ids = rng.permutation(pages)[: (tokens + B - 1) // B] * 2 * L
            slots = np.array([ids[t // B] * B + t % B for t in range(tokens)], np.int32)
        else:  # one token of each sequence, each on its own page
            ids = rng.permutation(pages)[:tokens] * 2 * L
            slots = (ids * B + rng.integers(0, B, tokens)).astype(np.int32)
        kv = torch.randn((2, tokens, H * D), device=dev).to(torch.bfloat16)
        d_slots = torch.from_numpy(slots).to(dev)
        k_off, v_off = 2 * layer * half, (2 * layer + 1) * half
        s_args = ([sc.data_ptr() + 4 * 2 * layer * plane, 4 * (sc.numel() - 2 * layer * plane),
                   sc.data_ptr() + 4 * (2 * layer + 1) * plane,
                   4 * (sc.numel() - (2 * layer + 1) * plane)] if fp8 else [0, 0, 0, 0])
        alg = 2 * tokens * H * D * 2 + 2 * tokens * H * D * e_out + tokens * 4
        if fp8:
            alg += 2 * tokens * H * 4
        fn = lambda: P.scatter_kv(kv[0].data_ptr(), kv[1].data_ptr(), P.PBE_IN_BF16, tokens,
                                  d_slots.data_ptr(), B, H, D,
                                  P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16,
                                  arena.data_ptr() + k_off, arena.numel() - k_off,
                                  arena.data_ptr() + v_off, arena.numel() - v_off, *s_args,
                                  stream=sp)
        ms = _timed(torch, stream, scrub, fn, n)
        r = {"workload": name, "algorithmic_bytes": alg, "kernel_us_mean": round(ms[0] * 1e3, 2),
             "kernel_us_min": round(ms[1] * 1e3, 2),
             "gbps": round(alg / (ms[0] * 1e-3) / 1e9, 1),
             "pct_of_peak": round(100 * alg / (ms[0] * 1e-3) / 1e9 / PEAK_GBPS, 1),
             "tokens": tokens, "launches": 1}
        out.append(r)
        print(json.dumps(r), file=sys.stderr, flush=True)
        del arena, sc, kv
    return out


def measure_fp8(torch, P, W, scrub, n: int):
    """Config 4: the fused BF16 -> FP8 E4M3 handoff in both scale modes."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    out = []

    def rec(name, alg, ms, extra=None):
        r = {"workload": name, "algorithmic_bytes": alg, "kernel_us_mean": round(ms[0] * 1e3, 2),
             "kernel_us_min": round(ms[1] * 1e3, 2),
             "gbps": round(alg / (ms[0] * 1e-3) / 1e9, 1),
             "pct_of_peak": round(100 * alg / (ms[0] * 1e-3) / 1e9 / PEAK_GBPS, 1)}
        r.update(extra or {})
        out.append(r)
        print(json.dumps(r), file=sys.stderr, flush=True)

    w = W.config4(0)
    g = w.geometry
    kv = P.shape(g.layers, g.kv_heads, g.head_dim, g.page_tokens)
    n_pages = w.meta["n_pages"]
    src = torch.empty(n_pages * g.page_bytes(2), dtype=torch.uint8, device=dev)
    src.view(torch.bfloat16).normal_()
    dst = torch.empty(n_pages * g.page_bytes(1), dtype=torch.uint8, device=dev)
    scale_page = 2 * g.layers * g.page_tokens * g.kv_heads * 4
    scales = torch.empty(n_pages * scale_page, dtype=torch.uint8, device=dev)
    table = torch.tensor(w.amax_table.ravel(), device=dev)
    runs = P.build_runs(w.src_ids, w.dst_ids, kv)
    rl = P.RunList.fp8(P.view_of(src.data_ptr(), src.numel()), P.view_of(dst.data_ptr(), dst.numel()),
                       scales.data_ptr(), scales.numel(), runs, kv)
    alg = w.algorithmic_bytes()
    rec(w.name + "_per_token_head", alg + w.pages * scale_page,
        _timed(torch, stream, scrub, lambda: rl.copy_fp8(P.PBE_FP8_SCALE_PER_TOKEN_HEAD, 0, sp), n),
        {"pages": w.pages, "scale_bytes": w.pages * scale_page})
    rec(w.name + "_table", alg + table.numel() * 4,
        _timed(torch, stream, scrub,
               lambda: rl.copy_fp8(P.PBE_FP8_SCALE_TABLE, table.data_ptr(), sp), n),
        {"pages": w.pages})
    rl.close()
    return out


def measure_decode(torch, P, scrub, n: int, batch: int = 64, seq: int = 5040, placement: str = "chunks"):
    """Decode-side reader after the handoff: one decode step (one layer) of
    `batch` sequences holding the 5040-token Qwen2.5-1.5B prefix, reading FP8
    pages + per-token-head scales, and BF16 pages. Algorithmic bytes = the K
    and V rows (and scales) of every valid token + queries + outputs."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    L, H, D, kvm = 28, 2, 128, 6
    kv = P.shape(L, H, D)
    blocks = (seq + 15) // 16
    n_pages = batch * blocks
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    if placement == "one_page":  # diagnostic: every block reads page 0 (cache-resident)
        perm = torch.zeros(n_pages, dtype=torch.int32, device=dev)
    elif placement == "random":    # every block on a random page of the arena
        perm = torch.randperm(n_pages, generator=g, device=dev).to(torch.int32)
    else:                          # 5-page Chunks (the shared arena's 2 MiB Chunks), shuffled
        chunks = torch.randperm(n_pages // 5, generator=g, device=dev).to(torch.int32)
        perm = (chunks[:, None] * 5 + torch.arange(5, device=dev, dtype=torch.int32)).view(-1)
    tables = (perm * (2 * L)).view(batch, blocks).contiguous()
    seq_lens = torch.full((batch,), seq, dtype=torch.int32, device=dev)
    q = (torch.randn(batch, H * kvm, D, generator=g, device=dev)).to(torch.bfloat16)
    o = torch.empty_like(q)
    res = []
    for fp8 in (True, False):
        E = 1 if fp8 else 2
        splits = P.decode_splits(batch, H, blocks, P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16)
        ws_bytes = P.decode_workspace_bytes(batch, H * kvm, D, splits)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        arena = torch.empty(n_pages * 2 * L * 16 * H * D * E, dtype=torch.uint8, device=dev)
        if fp8:
            arena.copy_(torch.randint(0, 0x70, arena.shape, generator=g, device=dev, dtype=torch.uint8)
                        | (torch.randint(0, 2, arena.shape, generator=g, device=dev,
                                         dtype=torch.uint8) << 7))
            scales = torch.rand(n_pages * 2 * L * 16 * H, generator=g, device=dev) * 0.1 + 0.01
        else:
            arena.view(torch.bfloat16).normal_(generator=g)
            scales = None
        view = P.view_of(arena.data_ptr(), arena.numel())

        def step():
            P.paged_decode(view, P.PBE_KV_FP8_E4M3 if fp8 else P.PBE_KV_BF16,
                           scales.data_ptr() if fp8 else 0, scales.numel() * 4 if fp8 else 0, kv,
                           L - 1, q.data_ptr(), o.data_ptr(), batch, H * kvm, tables.data_ptr(),
                           seq_lens.data_ptr(), blocks, splits, ws.data_ptr(), ws_bytes, sp)

        ms = _timed(torch, stream, scrub, step, n)
        alg = batch * seq * H * (2 * D * E + (8 if fp8 else 0)) + 2 * q.numel() * 2
        r = {"workload": f"decode_reader_{'fp8' if fp8 else 'bf16'}_qwen15b_b{batch}_s{seq}",
             "placement": placement,
             "algorithmic_bytes": alg, "kernel_us_mean": round(ms[0] * 1e3, 2),
             "kernel_us_min": round(ms[1] * 1e3, 2),
             "gbps": round(alg / (ms[0] * 1e-3) / 1e9, 1),
             "pct_of_peak": round(100 * alg / (ms[0] * 1e-3) / 1e9 / PEAK_GBPS, 1),
             "splits": splits, "launches": 2,
             "note": "both launches (split-K attention + combine) between the events"}
        print(json.dumps(r), file=sys.stderr, flush=True)
        res.append(r)
        del arena
    return res


def read_ceiling(torch, scrub, n: int, nbytes: int = 170_704_896) -> dict:
    """Streaming-read ceilings for the decode reader: about `nbytes` (the FP8
    reader's bytes per step at 64 x 5,040 tokens) read at shuffled positions
    by short-lived waves (1 step each) and by long-lived ones (8 and 20 steps
    each; the reader's waves hold ~20 blocks at 16 splits), each wave keeping
    4 steps in flight (lib/libpbe_ceiling.so, stream_read_steps_kernel), in two
    access shapes: contiguous 4 KiB steps, and the FP8 reader's own (8 KiB
    blocks, each read as two KV heads' 128-byte halves of 256-byte token rows
    by a pair of waves)."""
    import ctypes as C
    import numpy as np
    so = Path(__file__).resolve().parent / "paged-batch-engine_amd" / "lib" / "libpbe_ceiling.so"
    cl = C.CDLL(str(so))
    cl.pbe_ceiling_read_steps.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_int,
                                          C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
    dev = torch.device("cuda:0")
    sp = torch.cuda.current_stream().cuda_stream
    buf = torch.empty(nbytes // 8192 * 8192, dtype=torch.uint8, device=dev)
    buf.view(torch.int32).random_()
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    sink = torch.empty(1024, dtype=torch.uint8, device=dev)
    ev = TimingEvents(2)
    out = {"what": "reads at shuffled positions, non-temporal loads, 4 steps in flight per wave"}
    for shape, step in (("contiguous_4k_steps", 4096), ("reader_shape_8k_blocks", 8192)):
        n_steps = buf.numel() // step
        order = torch.randperm(n_steps, generator=g, device=dev).to(torch.int32)
        legs = {"bytes": n_steps * step}
        for spw in (1, 8, 20):
            ts = []
            for i in range(n + 2):
                scrub.fill_(i & 0xff)
                rc = cl.pbe_ceiling_read_steps(buf.data_ptr(), order.data_ptr(), n_steps, spw,
                                               1 if step == 8192 else 0, sink.data_ptr(), sp,
                                               ev.handle(0), ev.handle(1))
                if rc:
                    raise RuntimeError(f"read-steps launch failed ({rc})")
                torch.cuda.synchronize()
                if i >= 2:
                    ts.append(ev.elapsed_ms(0, 1))
            ms = float(np.mean(ts))
            waves = (n_steps + spw - 1) // spw * (2 if step == 8192 else 1)
            legs[f"steps_per_wave_{spw}"] = {
                "waves": waves, "us_mean": round(ms * 1e3, 2),
                "gbps": round(n_steps * step / (ms * 1e-3) / 1e9, 1),
                "grid_threads": (waves + 3) // 4 * 256}
            print(json.dumps({"read_steps": shape, "spw": spw, **legs[f"steps_per_wave_{spw}"]}),
                  file=sys.stderr, flush=True)
        out[shape] = legs
    ev.close()
    return out


def calibration_copy(torch, P, scrub, steps: int, sp: int) -> dict:
    """One plain 256 MiB run (1024 pages of 256 KiB, offset 0 to offset 256 MiB)
    with the copy kernel: the known byte count that rocprofv3 --pmc counters
    are scaled by."""
    import numpy as np
    ckv = P.shape(1, 1, 4096, 16)
    cbuf = torch.empty(2 * (256 << 20), dtype=torch.uint8, device="cuda")
    cview = P.view_of(cbuf.data_ptr(), cbuf.numel())
    crl = P.RunList.bf16(cview, cview, [(0, (256 << 20) // ckv.half_bytes(), 1024)], ckv)
    ct = []
    cev = TimingEvents(2)
    for i in range(steps):
        scrub.fill_(i & 0xff)
        cev.record(0, sp)
        crl.copy(sp)
        cev.record(1, sp)
        torch.cuda.synchronize()
        ct.append(cev.elapsed_ms(0, 1))
    cev.close()
    calib = {"bytes": 256 << 20, "grid_threads": int(crl.info().slices) * 64,
             "gbps": round(2 * (256 << 20) / (float(np.mean(ct)) * 1e-3) / 1e9, 1)}
    crl.close()
    return calib


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-scrub", action="store_true", help="hot-cache timing (diagnostic)")
    ap.add_argument("--extra-configs", default="",
                    help="also time configs 1, 3, 4 and 5 and write them as JSON to this file")
    ap.add_argument("--decode-only", action="store_true",
                    help="time only the decode reader (FP8 and BF16 pages) and print it as JSON")
    ap.add_argument("--decode-batch", type=int, default=64,
                    help="with --decode-only: sequences per decode step")
    ap.add_argument("--decode-seq", type=int, default=5040,
                    help="with --decode-only: tokens per sequence")
    ap.add_argument("--fp8-only", action="store_true",
                    help="time only the fused FP8 handoff (config 4, both scale modes)")
    ap.add_argument("--host-paths", action="store_true",
                    help="run lib/pbe_host_paths: host costs of the C++ connector and of the "
                         "reference's copy_shared_kv call order at config-2 size (one JSON line)")
    ap.add_argument("--decode-loop-only", action="store_true",
                    help="time only a 28-layer decode step (page write + reader), eager and graph")
    ap.add_argument("--scatter-only", action="store_true",
                    help="time only the page writer (prompt and decode-token scatters)")
    ap.add_argument("--ceiling-legs", type=int, default=0, metavar="K",
                    help="only launch the config-2 plan and its ceiling legs K times each, in a "
                         "fixed order (for rocprofv3 --pmc; summarised by profiling.py legs)")
    ap.add_argument("--legs-config", type=int, default=2, choices=(2, 3),
                    help="with --ceiling-legs: the workload whose plan the legs follow")
    ap.add_argument("--read-ceiling", action="store_true",
                    help="time the decode reader (FP8 and BF16) beside plain streaming reads of "
                         "the FP8 reader's bytes by short- and long-lived waves")
    ap.add_argument("--headline-only", action="store_true",
                    help="time only the config-2 headline kernel (no ceiling legs, no contiguous "
                         "leg, no reference-pattern or host-path legs): for rocprofv3 runs whose "
                         "per-kernel averages must be the headline kernel's alone")
    ap.add_argument("--calibrate", action="store_true",
                    help="also launch a plain contiguous copy of 256 MiB with the same kernel "
                         "(rocprofv3 --pmc byte-count calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the handoff is a same-GPU page migration.", file=sys.stderr)
        return 2
    if args.host_paths:  # a child process: this one never touches the GPU
        import subprocess
        exe = Path(__file__).resolve().parent / "paged-batch-engine_amd" / "lib" / "pbe_host_paths"
        if not exe.exists():
            print(f"bench.py: {exe} is missing: run __graft_entry__.build()", file=sys.stderr)
            return 2
        return subprocess.run([str(exe)], timeout=300).returncode

    import numpy as np
    import torch
    import pbe_handoff as P
    import workload as W

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    if args.read_ceiling:
        scrub = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        out = {"decode": measure_decode(torch, P, scrub, max(3, args.steps), 64, 5040, "chunks"),
               "read_ceiling": read_ceiling(torch, scrub, max(3, args.steps))}
        print(json.dumps(out))
        return 0
    if args.decode_only or args.fp8_only or args.scatter_only or args.decode_loop_only:
        scrub = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        sp = torch.cuda.current_stream().cuda_stream
        if args.decode_only:
            placement = "chunks" if (args.decode_batch * ((args.decode_seq + 15) // 16)) % 5 == 0 \
                else "random"
            out = {"decode": measure_decode(torch, P, scrub, max(3, args.steps), args.decode_batch,
                                            args.decode_seq, placement)}
        elif args.decode_loop_only:
            out = {"decode_loop": measure_decode_loop(torch, P, scrub, max(3, args.steps // 4),
                                                      args.decode_batch, args.decode_seq)}
        elif args.fp8_only:
            out = {"fp8": measure_fp8(torch, P, W, scrub, max(3, args.steps))}
        else:
            out = {"scatter": measure_scatter(torch, P, scrub, max(3, args.steps))}
        if args.calibrate:
            out["calibration"] = calibration_copy(torch, P, scrub, args.steps, sp)
        print(json.dumps(out))
        return 0
    if args.ceiling_legs:
        w = W.CONFIGS[args.legs_config](0)
        g = w.geometry
        kv = P.shape(g.layers, g.kv_heads, g.head_dim, g.page_tokens)
        arena = torch.empty(w.arena_bytes, dtype=torch.uint8, device=dev)
        arena.view(torch.int32).random_()
        scrub = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        runs = P.build_runs(w.src_ids, w.dst_ids, kv)
        print(json.dumps(ceiling_legs(torch, P, w, runs, kv, arena, scrub, None, args.ceiling_legs)))
        return 0
    w = W.config2(0)
    g = w.geometry
    kv = P.shape(g.layers, g.kv_heads, g.head_dim, g.page_tokens)

    arena = torch.empty(w.arena_bytes, dtype=torch.uint8, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(2)
    vals = arena.view(torch.bfloat16)
    chunk = 1 << 26
    for i in range(0, vals.numel(), chunk):
        v = vals[i:i + chunk]
        v.copy_((torch.randn(v.numel(), generator=gen, device=dev) * w.sigma).to(torch.bfloat16))
    scrub = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    view = P.view_of(arena.data_ptr(), w.arena_bytes)
    runs = P.build_runs(w.src_ids, w.dst_ids, kv)
    rl = P.RunList.bf16(view, view, runs, kv)
    info = rl.info()
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream


    # correctness of this exact run: device result vs oracle on the same pool
    from oracle import oracle as O
    torch.cuda.synchronize()
    host_before = arena.cpu().numpy()
    expected = host_before.copy()
    O.copy_handoff(expected, w.src_ids, w.dst_ids, g.half(), g.layers)
    rl.copy(sp)
    torch.cuda.synchronize()
    parity = bool(np.array_equal(arena.cpu().numpy(), expected))
    del expected

    for i in range(args.warmup):
        if not args.no_scrub:
            scrub.fill_(i & 0xff)
        rl.copy(sp)
    torch.cuda.synchronize()

    # Timed region: each step's kernel is bracketed by two HIP events that
    # the runtime stamps at the kernel's own start and end (hipExtLaunchKernel
    # through pbe_handoff_copy_timed), on the stream the kernel runs on.
    ev = TimingEvents(2 * args.steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        if not args.no_scrub:
            scrub.fill_((i + 1) & 0xff)
        rl.copy_timed(sp, ev.handle(2 * i), ev.handle(2 * i + 1))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    times_ms = np.array([ev.elapsed_ms(2 * i, 2 * i + 1) for i in range(args.steps)])
    ev.close()
    mean_ms = float(times_ms.mean())
    # the same launches between events recorded on the stream around them
    # (adds the dispatch gap on both sides)
    outer_ms = _timed(torch, stream, scrub, lambda: rl.copy(sp), max(10, args.steps // 4))
    alg = w.algorithmic_bytes()
    achieved = alg / (mean_ms * 1e-3) / 1e9

    # end-to-end handoff latency of the one-call form (validate, coalesce,
    # stage, launch, wait), as copy_shared_kv does before commit_kv
    lat, lat_stream = [], []
    src_np = np.ascontiguousarray(w.src_ids, dtype=np.int32)  # the id lists as the
    dst_np = np.ascontiguousarray(w.dst_ids, dtype=np.int32)  # engine holds them
    for i in range(20):
        if not args.no_scrub:
            scrub.fill_(i & 0xff)
        torch.cuda.synchronize()
        t = time.perf_counter()
        P.copy_shared_kv(view, src_np, dst_np, kv, 0, sp)
        torch.cuda.synchronize()
        lat.append(time.perf_counter() - t)
    # the same call waited on with its own stream's synchronize, as copy_shared_kv
    # waits on the model stream (split_pd_engine.cpp:110)
    for i in range(20):
        if not args.no_scrub:
            scrub.fill_(i & 0xff)
        torch.cuda.synchronize()
        t = time.perf_counter()
        P.copy_shared_kv(view, src_np, dst_np, kv, 0, sp)
        P.stream_synchronize(sp)
        lat_stream.append(time.perf_counter() - t)
    e2e_us = float(np.median(lat) * 1e6)
    e2e_stream_us = float(np.median(lat_stream) * 1e6)

    # the reference's own GPU pattern on this GPU: one hipMemcpyAsync per
    # coalesced run (split_pd_engine.cpp:102-108), then a stream sync (:110)
    refpat = gpu_reference_pattern(torch, stream, scrub, arena.data_ptr(), runs, g, alg,
                                   max(10, args.steps // 4), not args.no_scrub)
    refpat["kernel_speedup"] = round(refpat["us_mean"] / (mean_ms * 1e3), 2)

    # the same bytes as one contiguous run, same kernel: the difference to
    # the headline is the cost of the plan's page placement in HBM
    contiguous = ceilings = None
    if not args.headline_only:
        stride = 2 * g.layers
        n_arena = w.arena_bytes // g.page_bytes()
        with P.RunList.bf16(view, view, [(0, stride * (n_arena - w.pages), w.pages)], kv) as crl:
            c_ms = _kernel_timed(torch, scrub, lambda a, b: crl.copy_timed(sp, a, b),
                                 max(10, args.steps // 4))
        contiguous = {"what": "same kernel, same bytes, one contiguous run (pages 0.. -> end of "
                              "arena)", "us_mean": round(c_ms[0] * 1e3, 2),
                      "gbps": round(alg / (c_ms[0] * 1e-3) / 1e9, 1)}
        ceilings = measure_ceilings(torch, P, w, runs, kv, arena, scrub, alg,
                                    max(10, args.steps // 4))
        ceilings["contiguous_same_bytes"] = contiguous
        best = min(ceilings["sorted_destination"]["us_mean"], ceilings["vendor_memcpy"]["us_mean"])
        ceilings["headline_over_best_of_sorted_and_vendor"] = round(mean_ms * 1e3 / best, 4)

    calib = calibration_copy(torch, P, scrub, args.steps, sp) if args.calibrate else None

    if args.extra_configs:
        extra = measure_extra_configs(torch, P, W, scrub, max(10, args.steps // 4))
        Path(args.extra_configs).write_text(json.dumps(extra, indent=1) + "\n")

    # the reference's copy_shared_kv call order through the C++ drop-in API
    # (serving::CopySharedKVToDecode: reserve over 28 layers, manifest, the
    # one-launch copy, stream sync, commit_kv) at config-2 size, timed by the
    # C++ host-path runner in a child process on this GPU
    ref_order = None if args.headline_only else host_paths_timing()

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(w, host_before, args.cpu_seconds)
        cpu["cores_on_host"] = os.cpu_count()
        cpu["cpu_model"] = _cpu_model()

    traffic = _traffic_from_profile()
    line = {
        "metric": METRIC,
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mean_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1.5) BF16 pool, seeded page plan)",
        "config": {"workload": w.name, "layers": g.layers, "kv_heads": g.kv_heads,
                   "head_dim": g.head_dim, "page_tokens": g.page_tokens,
                   "page_bytes": g.page_bytes(), "prefix_tokens": 5040, "pages": w.pages,
                   "runs": int(info.runs), "arena_mib": w.arena_bytes >> 20,
                   "cache": "cold (1 GiB scrub before each step)" if not args.no_scrub else "hot"},
        "latency_us": {"kernel_mean": round(mean_ms * 1e3, 2),
                       "kernel_p50": round(float(np.median(times_ms)) * 1e3, 2),
                       "kernel_min": round(float(times_ms.min()) * 1e3, 2),
                       "launch_between_stream_events_mean": round(outer_ms[0] * 1e3, 2),
                       "handoff_e2e_p50": round(e2e_us, 1),
                       "handoff_e2e_stream_sync_p50": round(e2e_stream_us, 1),
                       "reference_call_order_p50":
                           ref_order["reference_call_order_us"]["end_to_end"] if ref_order else None},
        "pct_of_peak": round(100 * achieved / PEAK_GBPS, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_GBPS, 4),
                     "traffic": traffic, "algorithmic_bytes": alg,
                     "traffic_source": "profiles/handoff_copy_c2_pmc.txt (rocprofv3 --pmc FETCH_SIZE, "
                                       "WRITE_SIZE of the same kernel and plan, scaled by a plain copy)"},
        "cpu_baseline": cpu,
        "parity_vs_oracle": parity,
        "wall_ms_per_step_incl_scrub": round(wall / args.steps * 1e3, 4),
        "grid_threads": int(info.slices) * 64,
    }
    line["gpu_reference_pattern"] = refpat
    if contiguous:
        line["contiguous_same_bytes"] = contiguous
        line["ceilings"] = ceilings
    if ref_order:
        line["reference_call_order_us"] = dict(
            ref_order["reference_call_order_us"],
            what="serving::CopySharedKVToDecode at config-2 size (315 pages, 28 layers), medians of "
                 f"{ref_order['iterations']} calls: reserve = register_request + append_slots; "
                 "end_to_end = checks, reserve, manifest, one-launch copy, stream sync, commit_kv; "
                 "copy_and_sync_alone = pbe_copy_shared_kv + stream sync on the same pages")
    if calib:
        line["calibration_copy"] = calib
    print(json.dumps(line))
    rl.close()
    return 0 if parity else 3


if __name__ == "__main__":
    sys.exit(main())
