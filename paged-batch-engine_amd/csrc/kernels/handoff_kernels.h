// Internal interface between the C ABI layer and the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pbe {

constexpr int kThreadsPerBlock = 256;
constexpr int kCopyUnroll = 4;  // 4 KiB per wave slice for the identity copy
// Cache policy of the identity copy: buffer loads with the non-temporal bit,
// buffer stores with sc1 + nt (measured 1-2% faster on MI355X than global
// nt stores; stores without nt are 50% slower).
constexpr int kCopyPolicy = 10;
constexpr int kFp8Unroll = 4;   // 4 KiB of BF16 source per wave slice

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

enum class KernelKind { kCopy, kFp8 };

// Identity-copy variant: 16-byte vectors per lane per slice (unroll), cache
// policy of loads/stores (index into the kernel's policy table), workgroup
// size, and dynamic LDS per workgroup (caps workgroups per CU).
struct CopyConfig {
  int unroll = kCopyUnroll;
  int policy = kCopyPolicy;
  int block = 256;
  uint32_t lds_bytes = 0;
};

struct LaunchShape {
  uint32_t slices_per_wave = 1;
  CopyConfig copy;
  // Optional events that bracket the kernel itself (hipExtLaunchKernel).
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};

uint32_t slice_bytes(KernelKind kind, const CopyConfig& cfg);

// Run lists this short travel in the kernel arguments (3.6 KB of the 4 KB
// kernarg space) instead of a staged device copy.
constexpr uint32_t kKernargRuns = 112;
struct KernargRunList {
  uint32_t n_runs;
  uint32_t total_slices;
  uint64_t page_bytes;
  DevRun runs[kKernargRuns];
};
static_assert(sizeof(KernargRunList) <= 4096 - 256, "kernel arguments are limited to 4 KiB");

// Default copy variant (unroll 4, global nt, 256 threads, one slice per wave).
hipError_t launch_copy_runs_kernarg(const KernargRunList& list, hipStream_t stream);

hipError_t launch_copy_runs(const DevRun* runs, uint32_t n_runs, uint32_t total_slices,
                            uint64_t page_bytes, const LaunchShape& shape, hipStream_t stream);

hipError_t launch_copy_runs_fp8(const DevRun* runs, uint32_t n_runs, uint32_t total_slices,
                                uint64_t page_bytes, uint32_t lanes_per_row,
                                uint32_t rows_per_plane, uint32_t kv_heads,
                                uint32_t rows_per_page, bool table, const float* amax_table,
                                const LaunchShape& shape, hipStream_t stream);

hipError_t launch_copy_ops(const DevOp* ops, uint32_t n_ops, hipStream_t stream);

}  // namespace pbe
