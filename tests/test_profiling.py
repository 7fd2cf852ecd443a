"""The rocprofv3 summarisers behind profiles/ (paged-batch-engine_amd/profiling.py),
on synthetic CSV and JSON input whose figures are known by hand."""
import csv
import json

import pytest

import profiling as PR

COPY = "void pbe::(anonymous namespace)::copy_runs_kernel<512>(pbe::DevRun const*)"


def _write_csv(path, rows):
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def _trace_rows(kernel, grid, durations_ns, t0=1000):
    rows = []
    for d in durations_ns:
        rows.append({"Kernel_Name": kernel, "Grid_Size_X": grid, "Start_Timestamp": t0,
                     "End_Timestamp": t0 + d, "Dispatch_Id": len(rows) + 1})
        t0 += d + 500
    return rows


def test_stats_mean_median_min_and_bandwidth(tmp_path):
    _write_csv(tmp_path / "run" / "h" / "x_kernel_trace.csv",
               _trace_rows(COPY, 9031680, [45000, 46000, 50000]))
    out = tmp_path / "s.txt"
    PR.stats(str(tmp_path / "run"), str(out), "cmd", {9031680: ("c2", 289013760)})
    line = [l for l in out.read_text().splitlines() if "copy_runs_kernel" in l][0]
    f = line.split()
    # name grid calls avg p50 min workload GB/s
    assert f[0] == "pbe::copy_runs_kernel<512>" and f[1] == "9031680" and f[2] == "3"
    assert f[3:6] == ["47.00", "46.00", "45.00"]
    assert f[6] == "c2"
    assert float(f[7]) == pytest.approx(289013760 / 47e-6 / 1e9, abs=0.05)


def test_pmc_scales_counters_by_the_plain_copy(tmp_path):
    # plain copy of CALIB_BYTES: 131072 FETCH units and 262144 WRITE units,
    # so 2048 and 1024 bytes per unit; the handoff: 1000 and 2000 units
    def rows(counter, handoff, calib):
        return [{"Dispatch_Id": 1, "Kernel_Name": COPY, "Grid_Size": 100, "Counter_Name": counter,
                 "Counter_Value": handoff / 2},
                {"Dispatch_Id": 1, "Kernel_Name": COPY, "Grid_Size": 100, "Counter_Name": counter,
                 "Counter_Value": handoff / 2},
                {"Dispatch_Id": 2, "Kernel_Name": COPY, "Grid_Size": 200, "Counter_Name": counter,
                 "Counter_Value": calib}]
    _write_csv(tmp_path / "f" / "a_counter_collection.csv", rows("FETCH_SIZE", 1000, 131072))
    _write_csv(tmp_path / "w" / "a_counter_collection.csv", rows("WRITE_SIZE", 2000, 262144))
    out = tmp_path / "p.txt"
    alg = 1000 * 2048 + 2000 * 1024
    PR.pmc(str(tmp_path / "f"), str(tmp_path / "w"), str(out), "cmd", alg, 100, 200)
    got = dict(l.split(": ", 1) for l in out.read_text().splitlines() if ": " in l)
    assert got["fetch_bytes_per_launch"] == str(1000 * 2048)
    assert got["write_bytes_per_launch"] == str(2000 * 1024)
    assert got["traffic_over_algorithmic"] == "1.0000"


def test_split_legs_takes_the_last_copy_dispatches_in_leg_order():
    k = 2
    items = [("copy_runs_kernel<256>", "warmup")]  # an earlier copy dispatch is ignored
    for leg in ("plan", "sorted_destination", "contiguous"):
        items += [("pbe::copy_runs_kernel<512>", f"{leg}{i}") for i in range(k)]
    items += [("stream_read_kernel", f"r{i}") for i in range(k)]
    items += [("stream_write_kernel", f"w{i}") for i in range(k)]
    legs = PR._split_legs(items, k, "root")
    assert legs["plan"] == ["plan0", "plan1"]
    assert legs["sorted_destination"] == ["sorted_destination0", "sorted_destination1"]
    assert legs["contiguous"] == ["contiguous0", "contiguous1"]
    assert legs["read_only"] == ["r0", "r1"] and legs["write_only"] == ["w0", "w1"]
    with pytest.raises(RuntimeError):
        PR._split_legs(items[:-1], k, "root")


def test_hostpaths_table_from_the_bench_line(tmp_path):
    d = {"workload": "c2_host_paths", "pages": 315, "layers": 28, "iterations": 25,
         "generic_plan_form_us": {"per_page_binding": 1917.8, "copy_op_binding": 153.0,
                                  "copy_ops_call": 72.7, "connector_submit_drain": 215.3},
         "reference_call_order_us": {"reserve_28_layers": 22.6, "end_to_end": 89.2,
                                     "copy_and_sync_alone": 55.3, "free_request": 39.6,
                                     "reserve_under_pending_fences": 25.4,
                                     "steps": {"request_copies": 0.9, "reserve_and_manifest": 26.2,
                                               "pbe_copy_shared_kv_call": 3.6, "stream_wait": 52.3,
                                               "commit_kv": 0.0}}}
    log = tmp_path / "h.log"
    log.write_text("some progress line\n" + json.dumps(d) + "\n")
    out = tmp_path / "h.txt"
    PR.hostpaths(str(log), str(out), "cmd")
    text = out.read_text()
    assert "(315 pages, 28 layers)" in text
    rows = {l.rsplit(None, 1)[0].strip(): float(l.rsplit(None, 1)[1])
            for l in text.splitlines() if l.startswith("  ")}
    assert rows["connector submit -> drain"] == 215.3
    assert rows["end to end (reserve, manifest, copy, sync, commit_kv)"] == 89.2
    assert rows["stream wait (the kernel and its completion)"] == 52.3
    assert text.rstrip().endswith(json.dumps(d))
