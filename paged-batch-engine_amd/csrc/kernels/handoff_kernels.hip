// gfx950 kernels of the prefill->decode KV handoff.
//
// The handoff is a pure HBM stream: every copied page is read once and written
// once, so the kernels are bound by HBM bandwidth and use no MFMA.
//
// Work unit: one wavefront (64 lanes) moves one "slice" of a run, 64 lanes x
// 16-byte vectors x kUnroll. A run is contiguous on both sides across all of
// its pages (page = every layer's K and V planes, shared_kv_arena.h:35-36), so
// a slice never needs page or layer arithmetic: it is a contiguous byte span.
// Each wave copies one slice and finds its run with a wave-parallel search
// over the device run list. Loads and stores are non-temporal: the source
// pages are dead after the handoff and the destination is not read until the
// next decode step, so neither should evict the decode working set from L2 /
// MALL.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <hip/hip_ext.h>

#include "fp8_device.h"
#include "handoff_kernels.h"
#include "xcd_order.h"

namespace pbe {
namespace {

constexpr int kWavesPerBlock = kThreadsPerBlock / kWave;

__device__ __forceinline__ u32x4 ld16(gsrc_t p, uint32_t off) {
  return __builtin_nontemporal_load(reinterpret_cast<PBE_GLOBAL const u32x4*>(p + off));
}
__device__ __forceinline__ void st8(gdst_t p, uint32_t off, u32x2 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<PBE_GLOBAL u32x2*>(p + off));
}
// Largest index r in [lo, n) with runs[r].slice_begin <= s, given
// runs[lo].slice_begin <= s. Each level lets the 64 lanes probe 64 evenly
// spaced candidates at once, so n runs take ceil(log64(n)) dependent loads.
__device__ __forceinline__ uint32_t find_run(const DevRun* __restrict__ runs, uint32_t lo,
                                             uint32_t n, uint32_t s, uint32_t lane) {
  uint32_t count = n - lo;
  for (;;) {
    const uint32_t stride = (count + kWave - 1) / kWave;
    const uint32_t probe = lane * stride;
    const bool hit = probe < count && runs[lo + probe].slice_begin <= s;
    const uint64_t mask = __ballot(hit);
    const uint32_t k = (uint32_t)__popcll(mask) - 1u;
    lo += k * stride;
    if (stride == 1) return lo;
    count = min(stride, count - k * stride);
  }
}

// Cache policy bits of gfx950 buffer instructions (bit0 sc0, bit1 nt,
// bit4 sc1). Loads stream (nt): the source pages are dead after the handoff.
// Stores are sc1 + nt: written through without allocating, so the copy does
// not evict the decode working set; measured on MI355X 1-2% faster than
// global nt stores and 50% faster than stores without nt.
constexpr int kLoadPolicy = 0x02;
constexpr int kStorePolicy = 0x12;

// One slice: every lane moves kCopyUnroll 16-byte vectors, all loads issued
// before the first store. Buffer resources clamp to the slice, so a short
// last slice of a run (or an op) needs no per-lane bound test: out-of-range
// lanes read 0 and the hardware drops their stores.
__device__ __forceinline__ void copy_slice(uint64_t src, uint64_t dst, uint64_t nbytes, uint32_t lane) {
  const uint32_t n = nbytes >= kCopySliceBytes ? kCopySliceBytes : (uint32_t)nbytes;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(src), (short)0, n, 0x00020000);
  const __amdgpu_buffer_rsrc_t rd =
      __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(dst), (short)0, n, 0x00020000);
  u32x4 v[kCopyUnroll];
#pragma unroll
  for (int u = 0; u < kCopyUnroll; ++u)
    v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, (u * kWave + lane) * 16u, 0, kLoadPolicy);
#pragma unroll
  for (int u = 0; u < kCopyUnroll; ++u)
    __builtin_amdgcn_raw_buffer_store_b128(v[u], rd, (u * kWave + lane) * 16u, 0, kStorePolicy);
}

// Slice s when the sources form one region (linear_src: the first run's
// source; every run's source follows the previous one and holds whole
// slices of kLinearSliceBytes): the source of slice s is linear_src + s *
// slice whatever the run, so its loads go out before the run is known, and
// the lookup of the destination runs while they are in flight. Vector loads
// return in issue order, so only the first search level (one probe per lane,
// sent before the copy loads) is a vector load; the rest of the search and
// the run record are scalar loads, which are counted apart and do not wait
// for the copy's data. n_runs <= kLinearMaxRuns = 64 * kLinearScan (the host
// sets linear_src only then): the second level reads at most kLinearScan
// entries. The probe reads `starts`, the runs' first slices as a compact
// array, when the list has one (its 64 probes then touch a few cache lines
// instead of one 32-byte record each: config 2 46.9 -> 46.3 us on MI355X),
// else the records' slice_begin (run lists in the kernel arguments). The
// scalar scan reads the records (from the compact array: 46.5 us).
constexpr uint32_t kLinearScan = 8;
static_assert(kLinearMaxRuns == kWave * kLinearScan, "one probe per lane, then kLinearScan entries");
__device__ __forceinline__ uint32_t probe_start(const DevRun* __restrict__ runs,
                                                const uint32_t* __restrict__ starts, uint32_t i) {
  return starts ? starts[i] : runs[i].slice_begin;
}

__device__ __forceinline__ void copy_slice_linear_src(const DevRun* __restrict__ runs,
                                                      const uint32_t* __restrict__ starts,
                                                      uint32_t n_runs, uint32_t s,
                                                      uint64_t linear_src, uint32_t lane) {
  const uint32_t stride = (n_runs + kWave - 1) / kWave;  // <= kLinearScan
  const uint32_t probe = lane * stride;
  const uint32_t first = probe < n_runs ? probe_start(runs, starts, probe) : 0xffffffffu;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<void*>(linear_src + (uint64_t)s * kLinearSliceBytes), (short)0,
      kLinearSliceBytes, 0x00020000);
  u32x4 v[kLinearUnroll];
#pragma unroll
  for (int u = 0; u < kLinearUnroll; ++u)
    v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, (u * kWave + lane) * 16u, 0, kLoadPolicy);
  // level 1: the last probe at or below s (probe 0 is run 0, slice 0)
  const uint64_t mask = __ballot(first <= s);
  uint32_t r = ((uint32_t)__popcll(mask) - 1u) * stride;
  // level 2: up to stride - 1 following entries, scalar
  const uint32_t end = min(r + stride, n_runs);
  uint32_t next[kLinearScan];
#pragma unroll
  for (uint32_t i = 1; i < kLinearScan; ++i)
    next[i] = r + i < end ? runs[r + i].slice_begin : 0xffffffffu;
#pragma unroll
  for (uint32_t i = 1; i < kLinearScan; ++i) r += next[i] <= s ? 1u : 0u;
  const uint64_t dst = runs[r].dst + (uint64_t)(s - runs[r].slice_begin) * kLinearSliceBytes;
  const __amdgpu_buffer_rsrc_t rd =
      __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(dst), (short)0, kLinearSliceBytes,
                                        0x00020000);
#pragma unroll
  for (int u = 0; u < kLinearUnroll; ++u)
    __builtin_amdgcn_raw_buffer_store_b128(v[u], rd, (u * kWave + lane) * 16u, 0, kStorePolicy);
}

// Identity copy of every run: the device form of the reference's per-run
// cudaMemcpyAsync loop (split_pd_engine.cpp:96-108). Wave w copies global
// slice w; it finds its run with the wave-parallel search over the run list.
template <int kThreads>
__device__ __forceinline__ void copy_runs_body(const DevRun* __restrict__ runs,
                                               const uint32_t* __restrict__ starts, uint32_t n_runs,
                                               uint32_t total_slices, uint64_t page_bytes,
                                               uint64_t linear_src) {
  const uint32_t lane = threadIdx.x % kWave;
  // The slice index is wave-uniform; saying so keeps the run, the addresses
  // and the buffer resources in SGPRs (a resource the compiler cannot prove
  // uniform is rebuilt per lane in a readfirstlane loop around every load
  // and store).
  const uint32_t s = __builtin_amdgcn_readfirstlane(
      xcd_grouped(blockIdx.x, gridDim.x, kThreads == kLinearThreadsPerBlock ? kLinearXcdGroup : kCopyXcdGroup) *
          (kThreads / kWave) +
      threadIdx.x / kWave);
  if (s >= total_slices) return;
  if (linear_src) {
    copy_slice_linear_src(runs, starts, n_runs, s, linear_src, lane);
    return;
  }
  const uint32_t r = find_run(runs, 0, n_runs, s, lane);
  const DevRun& run = runs[r];
  const uint64_t rel = (uint64_t)(s - run.slice_begin) * kCopySliceBytes;
  copy_slice(run.src + rel, run.dst + rel, (uint64_t)run.pages * page_bytes - rel, lane);
}

// kThreads: kLinearThreadsPerBlock for one-region plans, else kThreadsPerBlock.
template <int kThreads>
__global__ __launch_bounds__(kThreads) void copy_runs_kernel(
    const DevRun* __restrict__ runs, const uint32_t* __restrict__ starts, uint32_t n_runs,
    uint32_t total_slices, uint64_t page_bytes, uint64_t linear_src) {
  copy_runs_body<kThreads>(runs, starts, n_runs, total_slices, page_bytes, linear_src);
}

// The same copy with the run list in the kernel arguments (no staging copy).
// An aggregate kernel argument stays in the kernarg segment and is read there.
__global__ __launch_bounds__(kThreadsPerBlock) void copy_runs_kernarg_kernel(const KernargRunList list) {
  copy_runs_body<kThreadsPerBlock>(list.runs, nullptr, list.n_runs, list.total_slices,
                                   list.page_bytes, list.linear_src);
}

// The one-region path with its runs in the kernel arguments: the slice's
// loads go out first, then a binary search over the runs' first slices with
// scalar loads from the argument segment (counted apart from the copy's
// loads, so the search runs while the data is in flight), then the stores.
__global__ __launch_bounds__(kLinearThreadsPerBlock) void copy_runs_kernarg_linear_kernel(
    const KernargLinearList list) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t s = __builtin_amdgcn_readfirstlane(xcd_grouped(blockIdx.x, gridDim.x, kLinearXcdGroup) * (kLinearThreadsPerBlock / kWave) +
                                                    threadIdx.x / kWave);
  if (s >= list.total_slices) return;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<void*>(list.linear_src + (uint64_t)s * kLinearSliceBytes), (short)0,
      kLinearSliceBytes, 0x00020000);
  u32x4 v[kLinearUnroll];
#pragma unroll
  for (int u = 0; u < kLinearUnroll; ++u)
    v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, (u * kWave + lane) * 16u, 0, kLoadPolicy);
  // largest r with starts[r] <= s (starts[0] = 0; slots past n_runs hold
  // 0xffffffff): eight halving steps over the 256 slots, straight-line so
  // the loads above stay first
  uint32_t lo = 0;
#pragma unroll
  for (uint32_t step = kKernargLinearRuns / 2; step >= 1; step /= 2) {
    const uint32_t mid = lo + step;  // <= 255
    lo = list.starts[mid] <= s ? mid : lo;
  }
  const uint64_t dst = list.dst[lo] + (uint64_t)(s - list.starts[lo]) * kLinearSliceBytes;
  const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<void*>(dst), (short)0, kLinearSliceBytes, 0x00020000);
#pragma unroll
  for (int u = 0; u < kLinearUnroll; ++u)
    __builtin_amdgcn_raw_buffer_store_b128(v[u], rd, (u * kWave + lane) * 16u, 0, kStorePolicy);
}

// Fused BF16 -> FP8 handoff. A row is one (token, kv head) of one K or V
// plane: head_dim BF16 values = kLanesPerRow lanes x 8 values. Rows are laid
// out [layer][K|V][token][head] within a page on both sides, so a row's index
// inside the run (source offset / row bytes) is also its scale index.
//   per-token-head: amax over the row, scale = amax/448 | 1, inv = 448/amax | 0
//                   (scatter_kv_kernel.cu:166-190), scale written per row;
//   table:          amax = table[(2*layer+kv)*heads + head], nothing written.
template <int kLanesPerRow, bool kTable>
__device__ __forceinline__ void fp8_step(const u32x4& v, uint32_t row, uint32_t lane,
                                         gdst_t dst, uint32_t dst_off, uint64_t scales,
                                         uint32_t rows_per_plane, uint32_t kv_heads,
                                         uint32_t rows_per_page,
                                         const float* __restrict__ amax_table) {
  float inv;
  if constexpr (kTable) {
    const uint32_t in_page = row % rows_per_page;
    const float amax = amax_table[(in_page / rows_per_plane) * kv_heads + in_page % kv_heads];
    inv = amax > 0.f ? 448.f / amax : 0.f;
  } else {
    const float m = group_max<kLanesPerRow>(amax8(v));
    inv = m > 0.f ? 448.f / m : 0.f;
    if (lane % kLanesPerRow == 0)
      __builtin_nontemporal_store(m > 0.f ? m / 448.f : 1.f,
                                  reinterpret_cast<PBE_GLOBAL float*>(scales) + row);
  }
  st8(dst, dst_off, quantise8(v, inv));
}

// A whole slice of the FP8 copy, loaded into v: quantises it into dst and
// writes its rows' scales (per-token-head) at scales + row. row0 is the row
// (within its run) of this lane's first 16-byte vector.
template <int kLanesPerRow, bool kTable, int kUnroll>
__device__ __forceinline__ void fp8_full_slice(const u32x4 (&v)[kUnroll], uint32_t lane,
                                               gdst_t dst, uint32_t row0, uint64_t scales,
                                               uint32_t rows_per_plane, uint32_t kv_heads,
                                               uint32_t rows_per_page,
                                               const float* __restrict__ amax_table) {
  constexpr uint32_t kRowsPerStep = kWave / kLanesPerRow;
  constexpr uint32_t kRowsPerSlice = kUnroll * kRowsPerStep;
  if constexpr (kRowsPerSlice <= kWave) {
    // Batched per slice: lane j owns row j of the slice. It obtains the
    // row's amax (per-token-head: the row maximum gathered from the row's
    // lanes; table: the (layer, K|V, head) entry of the row), computes
    // 448/amax (and the scale) once, and every lane then fetches its row's
    // multiplier. Divisions and index arithmetic run once per slice instead
    // of once per 1 KiB step.
    const uint32_t slice_row0 = row0 - lane / kLanesPerRow;  // first row of the slice
    float row_amax;
    if constexpr (kTable) {
      const uint32_t in_page = (slice_row0 + lane) % rows_per_page;
      row_amax = amax_table[(in_page / rows_per_plane) * kv_heads + in_page % kv_heads];
    } else {
      float m[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) m[u] = group_max<kLanesPerRow>(amax8(v[u]));
      const uint32_t j_step = lane / kRowsPerStep, j_row = lane % kRowsPerStep;
      row_amax = 0.f;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const float t = __shfl(m[u], (int)(j_row * kLanesPerRow), kWave);
        if (j_step == (uint32_t)u) row_amax = t;
      }
      if (lane < kRowsPerSlice)
        __builtin_nontemporal_store(row_amax > 0.f ? row_amax / 448.f : 1.f,
                                    reinterpret_cast<PBE_GLOBAL float*>(scales) + slice_row0 + lane);
    }
    const float row_inv = row_amax > 0.f ? 448.f / row_amax : 0.f;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const float inv = __shfl(row_inv, (int)(u * kRowsPerStep + lane / kLanesPerRow), kWave);
      st8(dst, (u * kWave + lane) * 8u, quantise8(v[u], inv));
    }
  } else {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      fp8_step<kLanesPerRow, kTable>(v[u], row0 + u * kRowsPerStep, lane, dst, (u * kWave + lane) * 8u,
                                     scales, rows_per_plane, kv_heads, rows_per_page, amax_table);
  }
}

// Fused BF16 -> FP8 copy of every run, one slice per wave: kFp8SliceBytes of
// source, kFp8LinearSliceBytes with kLinear. kLinear: the sources form one
// region and every run holds whole slices (linear_src, as for the identity
// copy), so the slice's loads
// go out before its run is looked up: one vector probe per lane first, the
// loads, then the ballot, a scalar scan of at most kLinearScan entries and
// the scalar run record (n_runs <= kLinearMaxRuns).
// Workgroup of the FP8 copy: kLinearThreadsPerBlock on the one-region path
// (table mode 39.0-39.1 against 39.5-39.6 us with 256 threads on config 4,
// per-token-head unchanged), else kThreadsPerBlock.
template <bool kLinear>
constexpr int fp8_threads() { return kLinear ? kLinearThreadsPerBlock : kThreadsPerBlock; }

template <int kLanesPerRow, bool kTable, bool kLinear>
__global__ __launch_bounds__(fp8_threads<kLinear>()) void copy_runs_fp8_kernel(
    const DevRun* __restrict__ runs, const uint32_t* __restrict__ starts, uint32_t n_runs,
    uint32_t total_slices, uint64_t page_bytes, uint32_t rows_per_plane, uint32_t kv_heads,
    uint32_t rows_per_page, const float* __restrict__ amax_table, uint64_t linear_src) {
  constexpr int kUnroll = kLinear ? kFp8LinearUnroll : kFp8Unroll;
  constexpr uint32_t kSlice = 64u * 16u * kUnroll;       // source bytes per slice
  constexpr uint32_t kRowBytes = kLanesPerRow * 16u;     // source bytes per row
  constexpr uint32_t kRowsPerStep = kWave / kLanesPerRow;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t s = __builtin_amdgcn_readfirstlane(blockIdx.x * (fp8_threads<kLinear>() / kWave) +
                                                    threadIdx.x / kWave);
  if (s >= total_slices) return;
  if constexpr (kLinear) {
    const uint32_t stride = (n_runs + kWave - 1) / kWave;  // <= kLinearScan
    const uint32_t probe = lane * stride;
    const uint32_t first = probe < n_runs ? probe_start(runs, starts, probe) : 0xffffffffu;
    gsrc_t src = reinterpret_cast<gsrc_t>(linear_src + (uint64_t)s * kSlice);
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = ld16(src, (u * kWave + lane) * 16u);
    const uint64_t mask = __ballot(first <= s);
    uint32_t r = ((uint32_t)__popcll(mask) - 1u) * stride;
    const uint32_t end = min(r + stride, n_runs);
    uint32_t next[kLinearScan];
#pragma unroll
    for (uint32_t i = 1; i < kLinearScan; ++i)
      next[i] = r + i < end ? runs[r + i].slice_begin : 0xffffffffu;
#pragma unroll
    for (uint32_t i = 1; i < kLinearScan; ++i) r += next[i] <= s ? 1u : 0u;
    const uint64_t rel = (uint64_t)(s - runs[r].slice_begin) * kSlice;
    fp8_full_slice<kLanesPerRow, kTable, kUnroll>(v, lane, reinterpret_cast<gdst_t>(runs[r].dst + rel / 2),
                                         (uint32_t)(rel / kRowBytes) + lane / kLanesPerRow,
                                         runs[r].aux, rows_per_plane, kv_heads, rows_per_page,
                                         amax_table);
    return;
  }
  const uint32_t r = __builtin_amdgcn_readfirstlane(find_run(runs, 0, n_runs, s, lane));
  const DevRun& run = runs[r];
  const uint64_t rel = (uint64_t)(s - run.slice_begin) * kSlice;
  const uint64_t nbytes = (uint64_t)run.pages * page_bytes - rel;
  gsrc_t src = reinterpret_cast<gsrc_t>(run.src + rel);
  gdst_t dst = reinterpret_cast<gdst_t>(run.dst + rel / 2);
  const uint64_t scales = run.aux;
  const uint32_t row0 = (uint32_t)(rel / kRowBytes) + lane / kLanesPerRow;  // row in the run
  if (nbytes >= kSlice) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = ld16(src, (u * kWave + lane) * 16u);
    fp8_full_slice<kLanesPerRow, kTable, kUnroll>(v, lane, dst, row0, scales, rows_per_plane, kv_heads,
                                         rows_per_page, amax_table);
  } else {
    // Last, partial slice of a run: whole rows only (slices are multiples
    // of the row size), one 1 KiB step at a time.
    for (uint32_t u = 0; u * kWave * 16u < nbytes; ++u) {
      const uint32_t off = (u * kWave + lane) * 16u;
      const u32x4 v = off < nbytes ? ld16(src, off) : u32x4{0u, 0u, 0u, 0u};
      if (off < nbytes)
        fp8_step<kLanesPerRow, kTable>(v, row0 + u * kRowsPerStep, lane, dst, off / 2, scales,
                                       rows_per_plane, kv_heads, rows_per_page, amax_table);
    }
  }
}

// Generic op-list copy (ops are pre-split on the host into pieces of at most
// kOpPieceBytes). One wave per piece, grid-stride over pieces. Pieces whose
// addresses and size are 16-byte multiples move as 16-byte vectors, four in
// flight per lane; others byte by byte.
__global__ __launch_bounds__(kThreadsPerBlock) void copy_ops_kernel(
    const DevOp* __restrict__ ops, uint32_t n_ops) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t waves = gridDim.x * kWavesPerBlock;
  for (uint32_t i = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave; i < n_ops; i += waves) {
    const DevOp op = ops[__builtin_amdgcn_readfirstlane(i)];
    if (((op.src | op.dst | op.bytes) & 15u) == 0) {
      // Up to 8 KiB per round (a whole K or V plane of a 1.5B page in one
      // round trip): all loads first, then all stores, against buffer
      // resources clamped to the op (out-of-range lanes load 0, stores drop).
      // A piece is at most kOpPieceBytes, so the 32-bit range holds it. Loads
      // are non-temporal, stores sc1+nt, as in the run-list kernel.
      const uint32_t bytes = (uint32_t)op.bytes;
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)op.src, (short)0, bytes, 0x00020000);
      const __amdgpu_buffer_rsrc_t rd =
          __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)op.dst, (short)0, bytes, 0x00020000);
      for (uint32_t base = 0; base < bytes; base += 8u * kWave * 16u) {
        u32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, base + (u * kWave + lane) * 16u, 0, 0x02);
#pragma unroll
        for (int u = 0; u < 8; ++u)
          __builtin_amdgcn_raw_buffer_store_b128(v[u], rd, base + (u * kWave + lane) * 16u, 0, 0x12);
      }
    } else {
      const uint8_t* src = reinterpret_cast<const uint8_t*>(op.src);
      uint8_t* dst = reinterpret_cast<uint8_t*>(op.dst);
      for (uint64_t off = lane; off < op.bytes; off += kWave) dst[off] = src[off];
    }
  }
}

}  // namespace

hipError_t launch_copy_runs_kernarg(const KernargRunList& list, hipStream_t stream) {
  if (list.n_runs == 0 || list.n_runs > kKernargRuns) return hipErrorInvalidValue;
  const uint32_t waves = list.total_slices ? list.total_slices : 1u;
  hipLaunchKernelGGL(copy_runs_kernarg_kernel, dim3((waves + kWavesPerBlock - 1) / kWavesPerBlock),
                     dim3(kThreadsPerBlock), 0, stream, list);
  return hipGetLastError();
}

hipError_t launch_copy_runs_kernarg_linear(const KernargLinearList& list, hipStream_t stream) {
  if (list.n_runs == 0 || list.n_runs > kKernargLinearRuns || !list.linear_src)
    return hipErrorInvalidValue;
  const uint32_t waves = list.total_slices ? list.total_slices : 1u;
  constexpr uint32_t kWavesLinear = kLinearThreadsPerBlock / kWave;
  hipLaunchKernelGGL(copy_runs_kernarg_linear_kernel,
                     dim3((waves + kWavesLinear - 1) / kWavesLinear), dim3(kLinearThreadsPerBlock), 0,
                     stream, list);
  return hipGetLastError();
}

hipError_t launch_copy_runs(const DevRun* runs, const uint32_t* starts, uint32_t n_runs,
                            uint32_t total_slices, uint64_t page_bytes, uint64_t linear_src,
                            const LaunchEvents& ev, hipStream_t stream) {
  const uint32_t waves = total_slices ? total_slices : 1u;
  if (linear_src) {
    constexpr uint32_t kWavesLinear = kLinearThreadsPerBlock / kWave;
    hipExtLaunchKernelGGL(copy_runs_kernel<kLinearThreadsPerBlock>,
                          dim3((waves + kWavesLinear - 1) / kWavesLinear),
                          dim3(kLinearThreadsPerBlock), 0, stream, ev.start, ev.stop, 0, runs,
                          starts, n_runs, total_slices, page_bytes, linear_src);
  } else {
    hipExtLaunchKernelGGL(copy_runs_kernel<kThreadsPerBlock>,
                          dim3((waves + kWavesPerBlock - 1) / kWavesPerBlock),
                          dim3(kThreadsPerBlock), 0, stream, ev.start, ev.stop, 0, runs, starts,
                          n_runs, total_slices, page_bytes, linear_src);
  }
  return hipGetLastError();
}

namespace {
template <int L, bool kLinear>
void launch_fp8_path(bool table, uint32_t waves, hipStream_t stream, const LaunchEvents& ev,
                     const DevRun* runs, const uint32_t* starts, uint32_t n_runs,
                     uint32_t total_slices, uint64_t page_bytes, uint32_t rows_per_plane,
                     uint32_t kv_heads, uint32_t rows_per_page, const float* amax_table,
                     uint64_t linear_src) {
  constexpr uint32_t per_block = fp8_threads<kLinear>() / kWave;
  const dim3 blocks((waves + per_block - 1) / per_block), threads(fp8_threads<kLinear>());
  if (table)
    hipExtLaunchKernelGGL((copy_runs_fp8_kernel<L, true, kLinear>), blocks, threads,
                          0, stream, ev.start, ev.stop, 0, runs, starts, n_runs, total_slices,
                          page_bytes, rows_per_plane, kv_heads, rows_per_page, amax_table, linear_src);
  else
    hipExtLaunchKernelGGL((copy_runs_fp8_kernel<L, false, kLinear>), blocks, threads,
                          0, stream, ev.start, ev.stop, 0, runs, starts, n_runs, total_slices,
                          page_bytes, rows_per_plane, kv_heads, rows_per_page, amax_table, linear_src);
}

template <int L>
void launch_fp8(bool table, uint32_t waves, hipStream_t stream, const LaunchEvents& ev,
                const DevRun* runs, const uint32_t* starts, uint32_t n_runs, uint32_t total_slices,
                uint64_t page_bytes, uint32_t rows_per_plane, uint32_t kv_heads,
                uint32_t rows_per_page, const float* amax_table, uint64_t linear_src) {
  if (linear_src)
    launch_fp8_path<L, true>(table, waves, stream, ev, runs, starts, n_runs, total_slices,
                             page_bytes, rows_per_plane, kv_heads, rows_per_page, amax_table,
                             linear_src);
  else
    launch_fp8_path<L, false>(table, waves, stream, ev, runs, nullptr, n_runs, total_slices,
                              page_bytes, rows_per_plane, kv_heads, rows_per_page, amax_table, 0);
}
}  // namespace

hipError_t launch_copy_runs_fp8(const DevRun* runs, const uint32_t* starts, uint32_t n_runs,
                                uint32_t total_slices,
                                uint64_t page_bytes, uint32_t lanes_per_row,
                                uint32_t rows_per_plane, uint32_t kv_heads,
                                uint32_t rows_per_page, bool table, const float* amax_table,
                                uint64_t linear_src, const LaunchEvents& ev, hipStream_t stream) {
  const uint32_t waves = total_slices ? total_slices : 1u;
  // One instantiation per row width (head_dim / 8 lanes), a shape, not a tuning choice.
#define PBE_FP8_CASE(L)                                                                      \
  case L:                                                                                    \
    launch_fp8<L>(table, waves, stream, ev, runs, starts, n_runs, total_slices, page_bytes,  \
                  rows_per_plane, kv_heads, rows_per_page, amax_table, linear_src);          \
    return hipGetLastError();
  switch (lanes_per_row) {
    PBE_FP8_CASE(1)
    PBE_FP8_CASE(2)
    PBE_FP8_CASE(4)
    PBE_FP8_CASE(8)
    PBE_FP8_CASE(16)
    PBE_FP8_CASE(32)
    PBE_FP8_CASE(64)
    default:
      return hipErrorInvalidValue;
  }
#undef PBE_FP8_CASE
}

hipError_t launch_copy_ops(const DevOp* ops, uint32_t n_ops, hipStream_t stream) {
  uint32_t blocks = (n_ops + kWavesPerBlock - 1) / kWavesPerBlock;
  if (blocks > 16384u) blocks = 16384u;
  hipLaunchKernelGGL(copy_ops_kernel, dim3(blocks), dim3(kThreadsPerBlock), 0, stream, ops,
                     n_ops);
  return hipGetLastError();
}

}  // namespace pbe
