"""Build recipe for the MI355X KV-handoff library (gfx950).

Compiles, in-tree:
  lib/libpbe_handoff.so   HIP kernels + C ABI (include/pbe_handoff.h) + the C++
                          drop-in API (include/{base,cache,serving}/*.h)
  lib/pbe_cpp_tests       C++ unit tests of the drop-in API (host-only parts)
  lib/pbe_cpp_gpu_tests   C++ tests that need a GPU (HIP backend, connector)
  lib/libpbe_ceiling.so   measurement-only read/write stream kernels (bench.py)

Usage: python paged-batch-engine_amd/build.py [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIB = PKG / "lib"
OBJ = PKG / "lib" / "obj"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # Packed FP32 (v_pk_*_f32) stays off: hand-verified scalar FP32 only.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the decode reader rescales them with VALU
    # ops, and AGPR accumulators cost a copy each way per block.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-command-line-argument",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter"]
INCLUDES = [f"-I{ROOT / 'include'}", f"-I{PKG / 'include'}", f"-I{PKG / 'csrc'}"]

# Host-only C++ of the drop-in API (no HIP headers): also built with g++ into
# the CPU unit-test binary.
HOST_SOURCES = [
    "csrc/base/base.cpp",
    "csrc/base/global_chunk_allocator.cpp",
    "csrc/cache/page_schema.cpp",
    "csrc/cache/layout_codec.cpp",
    "csrc/cache/transfer_plan.cpp",
    "csrc/cache/page_migration.cpp",
    "csrc/serving/pd_handoff_common.cpp",
    "csrc/base/trace_range.cpp",
]
# Host C++ that reaches the GPU only through the C ABI (in the library, not in
# the CPU-only unit-test binary).
ABI_HOST_SOURCES = [
    "csrc/base/shared_kv_arena.cpp",
    "csrc/base/block_allocator.cpp",
    "csrc/base/kv_cache_manager.cpp",
    "csrc/cache/hip_transfer_backend.cpp",
    "csrc/serving/shared_kv_handoff.cpp",
    "csrc/serving/decode_kv_reservation.cpp",
    "csrc/serving/split_pd_handoff.cpp",
    "csrc/serving/plan_kv_connector.cpp",
    "csrc/serving/kv_page_wire.cpp",
    "csrc/model/paged_kv_runtime.cpp",
]
# Sources that call HIP (compiled by hipcc).
HIP_SOURCES = [
    "csrc/kernels/handoff_kernels.hip",
    "csrc/kernels/decode_kernels.hip",
    "csrc/kernels/scatter_kernels.hip",
    "csrc/capi/capi_core.hip",
    "csrc/capi/capi_arena.hip",
    "csrc/capi/capi_plan.hip",
    "csrc/capi/capi_copy.hip",
    "csrc/capi/capi_decode.hip",
    "csrc/capi/capi_scatter.hip",
]
CPU_TESTS = ["tests/cpp/test_drop_in_api.cpp"]
GPU_TESTS = ["tests/cpp/test_gpu_backend.cpp"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops" not in l and "hip-link" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def _obj(src: str, tag: str) -> Path:
    return OBJ / (src.replace("/", "_").rsplit(".", 1)[0] + f".{tag}.o")


def build(jobs: int = 8) -> Path:
    if not shutil.which(HIPCC) and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    OBJ.mkdir(parents=True, exist_ok=True)
    steps = []
    for src in HIP_SOURCES:
        steps.append([HIPCC, *HIP_FLAGS, *INCLUDES, "-c", str(PKG / src), "-o", str(_obj(src, "hip"))])
    for src in HOST_SOURCES + ABI_HOST_SOURCES:
        steps.append([HIPCC, "-x", "c++", *CXX_FLAGS, *INCLUDES, "-c", str(PKG / src),
                      "-o", str(_obj(src, "host"))])
    for src in HOST_SOURCES:
        steps.append(["g++", *CXX_FLAGS, *INCLUDES, "-c", str(PKG / src), "-o", str(_obj(src, "gcc"))])
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        for fut in [pool.submit(_run, s) for s in steps]:
            fut.result()
    so = LIB / "libpbe_handoff.so"
    tmp = LIB / "libpbe_handoff.so.tmp"
    objs = [str(_obj(s, "hip")) for s in HIP_SOURCES] + \
        [str(_obj(s, "host")) for s in HOST_SOURCES + ABI_HOST_SOURCES]
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs])
    os.replace(tmp, so)
    # C++ CPU tests link the library (its HIP runtime dependency loads without
    # a GPU; the tests only use host paths and metadata-only page groups).
    cpu_objs = [str(_obj(s, "gcc")) for s in HOST_SOURCES]
    for t in CPU_TESTS:
        _run(["g++", *CXX_FLAGS, *INCLUDES, f"-I{ROOT / 'tests' / 'cpp'}", str(ROOT / t),
              f"-L{LIB}", "-lpbe_handoff", "-Wl,-rpath,$ORIGIN", "-o", str(LIB / "pbe_cpp_tests")])
    # The scenario driver of oracle/ref_driver.cpp built against this API, so
    # tests can replay identical scenarios on it and on the reference build.
    _run(["g++", *CXX_FLAGS, "-shared", *INCLUDES, str(ROOT / "oracle" / "ref_driver.cpp"), *cpu_objs,
          "-o", str(LIB / "libpbe_api_driver.so")])
    for t in GPU_TESTS:
        _run([HIPCC, *HIP_FLAGS, *INCLUDES, f"-I{ROOT / 'tests' / 'cpp'}", str(ROOT / t),
              f"-L{LIB}", "-lpbe_handoff", "-Wl,-rpath,$ORIGIN",
              "-o", str(LIB / "pbe_cpp_gpu_tests")])
    # bench.py --host-paths: the C++ paths' host costs at config-2 size
    _run([HIPCC, *HIP_FLAGS, *INCLUDES, str(ROOT / "tests" / "cpp" / "bench_host_paths.cpp"),
          f"-L{LIB}", "-lpbe_handoff", "-Wl,-rpath,$ORIGIN", "-o", str(LIB / "pbe_host_paths")])
    # bench.py only: read-only and write-only streams at the copy's geometry
    # (csrc/diag/hbm_ceiling.hip), the HBM ceilings the handoff is held against
    _run([HIPCC, *HIP_FLAGS, "-shared", str(PKG / "csrc" / "diag" / "hbm_ceiling.hip"),
          "-o", str(LIB / "libpbe_ceiling.so")])
    return so


SAN = ["-fsanitize=address,undefined", "-fno-omit-frame-pointer"]


def build_sanitized(jobs: int = 8) -> Path:
    """Host code under AddressSanitizer + UBSan (device code unchanged): lib/asan/
    holds libpbe_handoff.so and pbe_cpp_tests. The C++ suite runs as is; the
    Python CPU suite runs against the library with the runtime preloaded:
      LD_PRELOAD=<clang>/libclang_rt.asan-x86_64.so ASAN_OPTIONS=detect_leaks=0
    and pbe_handoff.LIB_PATH pointed at lib/asan/libpbe_handoff.so."""
    out = LIB / "asan"
    out.mkdir(parents=True, exist_ok=True)
    host_flags = [f for f in CXX_FLAGS if f != "-O2"] + ["-O1", "-g", *SAN]
    steps, objs = [], []
    for src in HOST_SOURCES + ABI_HOST_SOURCES:
        o = out / (src.replace("/", "_") + ".o")
        steps.append([HIPCC, "-x", "c++", *host_flags, *INCLUDES, "-c", str(PKG / src), "-o", str(o)])
        objs.append(str(o))
    for src in HIP_SOURCES:
        o = out / (src.replace("/", "_") + ".o")
        host_san = [x for f in SAN for x in ("-Xarch_host", f)]
        steps.append([HIPCC, *HIP_FLAGS, *host_san, *INCLUDES, "-c", str(PKG / src), "-o", str(o)])
        objs.append(str(o))
    t_obj = out / "test_drop_in_api.o"
    steps.append([HIPCC, "-x", "c++", *host_flags, *INCLUDES, f"-I{ROOT / 'tests' / 'cpp'}",
                  "-c", str(ROOT / CPU_TESTS[0]), "-o", str(t_obj)])
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        for fut in [pool.submit(_run, s) for s in steps]:
            fut.result()
    link = [HIPCC, f"--offload-arch={ARCH}", *SAN, "-fno-gpu-sanitize"]
    _run([*link, "-shared", "-fPIC", "-shared-libsan", "-o", str(out / "libpbe_handoff.so"), *objs])
    _run([*link, "-o", str(out / "pbe_cpp_tests"), str(t_obj), *objs])
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--sanitize", action="store_true",
                    help="also build lib/asan/ (host code under ASan + UBSan)")
    args = ap.parse_args()
    print(build(args.jobs))
    if args.sanitize:
        print(build_sanitized(args.jobs))
