// Internal interface between the C ABI layer and the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pbe {

constexpr int kThreadsPerBlock = 256;
// Workgroup of the one-region path (1 KiB slices): 8 waves, half as many
// workgroups to dispatch. MI355X, config 2: 46.0 us against 46.4 us with 256
// threads and 46.9 us with 128; config 3 (general path) keeps 256 threads
// (119.2 us against 121.6 us with 512).
constexpr int kLinearThreadsPerBlock = 512;
// Slice (the bytes one wave moves) of the identity copy, by path. Plans whose
// sources form one region take 1 KiB slices (one 16-byte vector per lane):
// the kernel issues a slice's loads before it looks its run up. Other plans
// look the run up first and take 2 KiB slices, which spend that lookup on
// twice the bytes. Measured on MI355X (kernel-bracketing events, 1 GiB scrub
// before each launch), slices of 4 / 2 / 1 KiB: config 2 (one source
// region) 48.5-48.9 / 48.1-48.5 / 46.9-47.1 us; config 3 (scattered
// sources) 124.1-126.0 / 119.5-121.3 / 135.3-136.4 us; config 5 646.6-646.9 /
// 635.4-636.0 / 729.0-730.2 us. 512-byte slices are bound by workgroup
// dispatch (64.8 us on config 2), as are 1024-thread workgroups (50.0 us).
constexpr int kLinearUnroll = 1;
constexpr uint32_t kLinearSliceBytes = 64u * 16u * kLinearUnroll;  // 1 KiB per wave
constexpr int kCopyUnroll = 2;  // 16-byte vectors per lane per slice of the identity copy
constexpr uint32_t kCopySliceBytes = 64u * 16u * kCopyUnroll;      // 2 KiB per wave
// The one-region path searches at most this many runs (one vector probe per
// lane, then a scalar scan of at most 8 entries); longer lists take the
// general path.
constexpr uint32_t kLinearMaxRuns = 512;
// Workgroups per XCD group (xcd_grouped in xcd_order.h), by path: 24 on the
// one-region path (192 KiB per group), 48 on the general path (384 KiB).
// MI355X, kernel-bracketing events, three alternating runs of 60 launches,
// mean us, (one-region, general) groups: (24, 48) config 2 45.64, one
// contiguous run 44.11, config 3 115.31, config 5 598.8; (16, 64) 45.96 /
// 44.70 / 115.96 / 601.0; (20, 40) 45.78 / 44.23 / 116.06 / 605.6; (32, 48)
// 46.43 / 44.72 / 115.33 / 599.1. Dispatch order: config 2 45.7-46.3,
// config 3 119.3-121.0, config 5 635-638. Further from these: one-region 4 /
// 8 / 12 / 256 (config 2 47.2 / 46.4 / 46.1 / 46.1); general 16 / 96 / 256
// (config 3 116.5 / 115.2 / 116.0) and 4 KiB general slices at 32 (123.9).
constexpr uint32_t kLinearXcdGroup = 24;
constexpr uint32_t kCopyXcdGroup = 48;
constexpr int kFp8Unroll = 4;   // 16-byte BF16 vectors per lane per slice of the FP8 copy
constexpr uint32_t kFp8SliceBytes = 64u * 16u * kFp8Unroll;    // 4 KiB of BF16 source per wave
// The FP8 copy's slice on the one-region path (loads before the run lookup):
// 2 KiB of BF16 source. MI355X, config 4 (bench events), slices of 4 / 2 /
// 1 KiB on that path: per-token-head scales 40.4 / 39.1 / 50.6 us, table
// mode 39.4 / 39.1 / 48.7 us. The general path keeps 4 KiB (2 KiB there, with
// the lookup first: 42.9 against 40.9 us).
constexpr int kFp8LinearUnroll = 2;
constexpr uint32_t kFp8LinearSliceBytes = 64u * 16u * kFp8LinearUnroll;

// Device form of one run: resolved addresses in this process's mapping.
// slice_begin is the exclusive prefix of slices over the preceding runs.
struct DevRun {
  uint64_t src;          // first source byte
  uint64_t dst;          // first destination payload byte
  uint64_t aux;          // first destination scale byte (FP8 per-token-head), else 0
  uint32_t slice_begin;  // first global slice of this run
  uint32_t pages;        // whole pages in the run
};
static_assert(sizeof(DevRun) == 32, "device run entry is 32 bytes");

// Ops larger than this are split into pieces before upload.
constexpr uint64_t kOpPieceBytes = 16384;

struct DevOp {
  uint64_t src;
  uint64_t dst;
  uint64_t bytes;
};

// Optional events that bracket the kernel itself (hipExtLaunchKernel), for
// timing without the launch gap.
struct LaunchEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};

// Run lists this short travel in the kernel arguments (3.6 KB of the 4 KB
// kernarg space) instead of a staged device copy.
constexpr uint32_t kKernargRuns = 112;
struct KernargRunList {
  uint32_t n_runs;
  uint32_t total_slices;
  uint64_t page_bytes;
  uint64_t linear_src;  // see launch_copy_runs
  DevRun runs[kKernargRuns];
};
static_assert(sizeof(KernargRunList) <= 4096 - 256, "kernel arguments are limited to 4 KiB");

// One slice per wave (kLinearSliceBytes when linear_src is set, else
// kCopySliceBytes), 256-thread workgroups.
hipError_t launch_copy_runs_kernarg(const KernargRunList& list, hipStream_t stream);

// Kernel-argument form of a one-region plan (linear_src set): only what that
// path reads, so up to 256 runs fit: each run's first slice and its first
// destination byte. Slices are kLinearSliceBytes. Slots past n_runs hold
// starts 0xffffffff (the kernel's search reads all 256).
constexpr uint32_t kKernargLinearRuns = 256;
struct KernargLinearList {
  uint32_t n_runs;
  uint32_t total_slices;
  uint64_t linear_src;
  uint32_t starts[kKernargLinearRuns];
  uint64_t dst[kKernargLinearRuns];
};
static_assert(sizeof(KernargLinearList) <= 4096 - 256, "kernel arguments are limited to 4 KiB");
hipError_t launch_copy_runs_kernarg_linear(const KernargLinearList& list, hipStream_t stream);

// linear_src: 0, or the first run's source address when every run's source
// directly follows the previous run's, every run holds whole slices of
// kLinearSliceBytes and there are at most kLinearMaxRuns runs (then slice s,
// counted in kLinearSliceBytes, reads linear_src + s * kLinearSliceBytes,
// known without the run list). Otherwise slices are kCopySliceBytes.
// starts: null, or (with linear_src) the runs' slice_begin values as a
// compact device array, which the one-region search probes.
hipError_t launch_copy_runs(const DevRun* runs, const uint32_t* starts, uint32_t n_runs,
                            uint32_t total_slices, uint64_t page_bytes, uint64_t linear_src,
                            const LaunchEvents& events, hipStream_t stream);

// linear_src: as for launch_copy_runs, with slices of kFp8LinearSliceBytes
// source bytes (kFp8SliceBytes without it).
hipError_t launch_copy_runs_fp8(const DevRun* runs, const uint32_t* starts, uint32_t n_runs,
                                uint32_t total_slices,
                                uint64_t page_bytes, uint32_t lanes_per_row,
                                uint32_t rows_per_plane, uint32_t kv_heads,
                                uint32_t rows_per_page, bool table, const float* amax_table,
                                uint64_t linear_src, const LaunchEvents& events, hipStream_t stream);

hipError_t launch_copy_ops(const DevOp* ops, uint32_t n_ops, hipStream_t stream);

}  // namespace pbe
