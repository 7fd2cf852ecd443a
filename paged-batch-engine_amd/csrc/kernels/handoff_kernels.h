// Internal interface between the C ABI layer and the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pbe {

constexpr int kThreadsPerBlock = 256;
constexpr int kCopyUnroll = 4;  // 16-byte vectors per lane per slice of the identity copy
constexpr uint32_t kCopySliceBytes = 64u * 16u * kCopyUnroll;  // 4 KiB per wave
constexpr int kFp8Unroll = 4;   // 16-byte BF16 vectors per lane per slice of the FP8 copy
constexpr uint32_t kFp8SliceBytes = 64u * 16u * kFp8Unroll;    // 4 KiB of BF16 source per wave

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

// One slice of kCopySliceBytes per wave, 256-thread workgroups.
hipError_t launch_copy_runs_kernarg(const KernargRunList& list, hipStream_t stream);

// linear_src: 0, or the first run's source address when every run's source
// directly follows the previous run's and every run holds whole slices
// (then slice s reads linear_src + s * kCopySliceBytes, known without the
// run list).
hipError_t launch_copy_runs(const DevRun* runs, uint32_t n_runs, uint32_t total_slices,
                            uint64_t page_bytes, uint64_t linear_src, const LaunchEvents& events,
                            hipStream_t stream);

hipError_t launch_copy_runs_fp8(const DevRun* runs, uint32_t n_runs, uint32_t total_slices,
                                uint64_t page_bytes, uint32_t lanes_per_row,
                                uint32_t rows_per_plane, uint32_t kv_heads,
                                uint32_t rows_per_page, bool table, const float* amax_table,
                                const LaunchEvents& events, hipStream_t stream);

hipError_t launch_copy_ops(const DevOp* ops, uint32_t n_ops, hipStream_t stream);

}  // namespace pbe
