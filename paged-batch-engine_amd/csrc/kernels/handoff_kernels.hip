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

#include "handoff_kernels.h"

namespace pbe {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Global-address-space pointers: lets the compiler emit global_* instructions
// with a wave-uniform scalar base instead of flat_* with per-lane 64-bit bases.
#define PBE_GLOBAL __attribute__((address_space(1)))
typedef PBE_GLOBAL const uint8_t* gsrc_t;
typedef PBE_GLOBAL uint8_t* gdst_t;

constexpr int kWave = 64;
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
// last slice of a run needs no per-lane bound test: out-of-range lanes read 0
// and the hardware drops their stores.
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

// Identity copy of every run: the device form of the reference's per-run
// cudaMemcpyAsync loop (split_pd_engine.cpp:96-108). Wave w copies global
// slice w; it finds its run with the wave-parallel search over the run list.
__device__ __forceinline__ void copy_runs_body(const DevRun* __restrict__ runs, uint32_t n_runs,
                                               uint32_t total_slices, uint64_t page_bytes) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t s = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (s >= total_slices) return;
  const uint32_t r = find_run(runs, 0, n_runs, s, lane);
  const DevRun& run = runs[r];
  const uint64_t rel = (uint64_t)(s - run.slice_begin) * kCopySliceBytes;
  copy_slice(run.src + rel, run.dst + rel, (uint64_t)run.pages * page_bytes - rel, lane);
}

__global__ __launch_bounds__(kThreadsPerBlock) void copy_runs_kernel(
    const DevRun* __restrict__ runs, uint32_t n_runs, uint32_t total_slices, uint64_t page_bytes) {
  copy_runs_body(runs, n_runs, total_slices, page_bytes);
}

// The same copy with the run list in the kernel arguments (no staging copy).
// An aggregate kernel argument stays in the kernarg segment and is read there.
__global__ __launch_bounds__(kThreadsPerBlock) void copy_runs_kernarg_kernel(const KernargRunList list) {
  copy_runs_body(list.runs, list.n_runs, list.total_slices, list.page_bytes);
}

// ---- FP8 E4M3 (OCP v1.0, "fn": no infinities, 0x7F NaN, max 448) ----
// Round to nearest even with saturation to +-448, the conversion the reference
// asks of __nv_cvt_float_to_fp8(v, __NV_SATFINITE, __NV_E4M3)
// (scatter_kv_kernel.cu:207-210). gfx950's v_cvt_pk_fp8_f32 rounds to nearest
// even in the OCP format; clamping to +-448 first makes it saturate. A NaN
// product would be absorbed by the clamp, so lanes that can produce one (a NaN
// input, or an infinite multiplier meeting a zero) take a path that writes the
// NaN code explicitly.
template <bool kHi>
__device__ __forceinline__ uint32_t cvt_pair_e4m3(float a, float b, uint32_t old) {
  const float ca = fminf(fmaxf(a, -448.f), 448.f);
  const float cb = fminf(fmaxf(b, -448.f), 448.f);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, (int)old, kHi);
}

template <bool kHi>
__device__ __forceinline__ uint32_t cvt_pair_e4m3_nan(float a, float b, uint32_t old) {
  uint32_t packed = cvt_pair_e4m3<kHi>(a, b, old);
  const uint32_t sh = kHi ? 16u : 0u;
  if (a != a) packed = (packed & ~(0xffu << sh)) | (0x7fu << sh);
  if (b != b) packed = (packed & ~(0xff00u << sh)) | (0x7f00u << sh);
  return packed;
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Non-zero iff one of the 8 BF16 values is a NaN ((h & 0x7fff) > 0x7f80 per
// half-word, evaluated on both halves of each word at once).
__device__ __forceinline__ uint32_t bf16x8_nan(u32x4 x) {
  const uint32_t m = 0x7fff7fffu, k = 0x007f007fu;
  return (((x.x & m) + k) | ((x.y & m) + k) | ((x.z & m) + k) | ((x.w & m) + k)) & 0x80008000u;
}

// Quantise 8 BF16 values (one 16-byte vector) with multiplier inv into 8 FP8
// bytes; inv == 0 yields +0 codes as in scatter_kv_kernel.cu:205-206.
__device__ __forceinline__ u32x2 quantise8(u32x4 x, float inv) {
  u32x2 out{0u, 0u};
  if (!(inv > 0.f)) return out;
  if (__builtin_expect(bf16x8_nan(x) != 0u || !(inv <= 3.402823466e38f), 0)) {
    uint32_t w0 = cvt_pair_e4m3_nan<false>(bf16_lo(x.x) * inv, bf16_hi(x.x) * inv, 0u);
    w0 = cvt_pair_e4m3_nan<true>(bf16_lo(x.y) * inv, bf16_hi(x.y) * inv, w0);
    uint32_t w1 = cvt_pair_e4m3_nan<false>(bf16_lo(x.z) * inv, bf16_hi(x.z) * inv, 0u);
    w1 = cvt_pair_e4m3_nan<true>(bf16_lo(x.w) * inv, bf16_hi(x.w) * inv, w1);
    out.x = w0;
    out.y = w1;
    return out;
  }
  uint32_t w0 = cvt_pair_e4m3<false>(bf16_lo(x.x) * inv, bf16_hi(x.x) * inv, 0u);
  w0 = cvt_pair_e4m3<true>(bf16_lo(x.y) * inv, bf16_hi(x.y) * inv, w0);
  uint32_t w1 = cvt_pair_e4m3<false>(bf16_lo(x.z) * inv, bf16_hi(x.z) * inv, 0u);
  w1 = cvt_pair_e4m3<true>(bf16_lo(x.w) * inv, bf16_hi(x.w) * inv, w1);
  out.x = w0;
  out.y = w1;
  return out;
}

__device__ __forceinline__ float amax8(u32x4 x) {
  float m = fabsf(bf16_lo(x.x));
  m = fmaxf(m, fabsf(bf16_hi(x.x)));
  m = fmaxf(m, fabsf(bf16_lo(x.y)));
  m = fmaxf(m, fabsf(bf16_hi(x.y)));
  m = fmaxf(m, fabsf(bf16_lo(x.z)));
  m = fmaxf(m, fabsf(bf16_hi(x.z)));
  m = fmaxf(m, fabsf(bf16_lo(x.w)));
  m = fmaxf(m, fabsf(bf16_hi(x.w)));
  return m;
}

template <int kCtrl>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xf, 0xf, false));
}

// Max over aligned groups of kLanes lanes, result in every lane of the group.
// Groups up to a 16-lane DPP row use DPP lane swaps (quad_perm [1,0,3,2],
// quad_perm [2,3,0,1], row_half_mirror, row_mirror); wider groups add
// cross-row shuffles. fmaxf keeps the non-NaN operand, as the reference's
// warp reduction does.
template <int kLanes>
__device__ __forceinline__ float group_max(float m) {
  if constexpr (kLanes >= 2) m = fmaxf(m, dpp_f<0xb1>(m));
  if constexpr (kLanes >= 4) m = fmaxf(m, dpp_f<0x4e>(m));
  if constexpr (kLanes >= 8) m = fmaxf(m, dpp_f<0x141>(m));
  if constexpr (kLanes >= 16) m = fmaxf(m, dpp_f<0x140>(m));
  if constexpr (kLanes >= 32) m = fmaxf(m, __shfl_xor(m, 16, kWave));
  if constexpr (kLanes >= 64) m = fmaxf(m, __shfl_xor(m, 32, kWave));
  return m;
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

template <int kLanesPerRow, bool kTable>
__global__ __launch_bounds__(kThreadsPerBlock) void copy_runs_fp8_kernel(
    const DevRun* __restrict__ runs, uint32_t n_runs, uint32_t total_slices, uint64_t page_bytes,
    uint32_t rows_per_plane, uint32_t kv_heads, uint32_t rows_per_page,
    const float* __restrict__ amax_table) {
  constexpr int kUnroll = kFp8Unroll;
  constexpr uint32_t kSlice = kFp8SliceBytes;           // source bytes per slice
  constexpr uint32_t kRowBytes = kLanesPerRow * 16u;     // source bytes per row
  constexpr uint32_t kRowsPerStep = kWave / kLanesPerRow;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t s = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (s >= total_slices) return;
  {
    const uint32_t r = __builtin_amdgcn_readfirstlane(find_run(runs, 0, n_runs, s, lane));
    const DevRun& run = runs[r];
    const uint64_t rel = (uint64_t)(s - run.slice_begin) * kSlice;
    const uint64_t nbytes = (uint64_t)run.pages * page_bytes - rel;
    gsrc_t src = reinterpret_cast<gsrc_t>(run.src + rel);
    gdst_t dst = reinterpret_cast<gdst_t>(run.dst + rel / 2);
    const uint64_t scales = run.aux;
    const uint32_t row0 = (uint32_t)(rel / kRowBytes) + lane / kLanesPerRow;  // row in the run
    constexpr uint32_t kRowsPerSlice = kUnroll * kRowsPerStep;
    if (nbytes >= kSlice) {
      u32x4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = ld16(src, (u * kWave + lane) * 16u);
      if constexpr (kRowsPerSlice <= kWave) {
        // Batched per slice: lane j owns row j of the slice. It obtains the
        // row's amax (per-token-head: the row maximum gathered from the
        // row's lanes; table: the (layer, K|V, head) entry of the row),
        // computes 448/amax (and the scale) once, and every lane then
        // fetches its row's multiplier. Divisions and index arithmetic run
        // once per slice instead of once per 1 KiB step.
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
                                        reinterpret_cast<PBE_GLOBAL float*>(scales) + slice_row0 +
                                            lane);
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
          fp8_step<kLanesPerRow, kTable>(v[u], row0 + u * kRowsPerStep, lane, dst,
                                                  (u * kWave + lane) * 8u, scales, rows_per_plane,
                                                  kv_heads, rows_per_page, amax_table);
      }
    } else {
      // Last, partial slice of a run: whole rows only (slices are multiples
      // of the row size), one 1 KiB step at a time.
      for (uint32_t u = 0; u * kWave * 16u < nbytes; ++u) {
        const uint32_t off = (u * kWave + lane) * 16u;
        const u32x4 v = off < nbytes ? ld16(src, off) : u32x4{0u, 0u, 0u, 0u};
        if (off < nbytes)
          fp8_step<kLanesPerRow, kTable>(v, row0 + u * kRowsPerStep, lane, dst, off / 2,
                                                  scales, rows_per_plane, kv_heads,
                                                  rows_per_page, amax_table);
      }
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

hipError_t launch_copy_runs(const DevRun* runs, uint32_t n_runs, uint32_t total_slices,
                            uint64_t page_bytes, const LaunchEvents& ev, hipStream_t stream) {
  const uint32_t waves = total_slices ? total_slices : 1u;
  hipExtLaunchKernelGGL(copy_runs_kernel, dim3((waves + kWavesPerBlock - 1) / kWavesPerBlock),
                        dim3(kThreadsPerBlock), 0, stream, ev.start, ev.stop, 0, runs, n_runs,
                        total_slices, page_bytes);
  return hipGetLastError();
}

namespace {
template <int L>
void launch_fp8(bool table, uint32_t blocks, hipStream_t stream, const LaunchEvents& ev,
                const DevRun* runs, uint32_t n_runs, uint32_t total_slices, uint64_t page_bytes,
                uint32_t rows_per_plane, uint32_t kv_heads, uint32_t rows_per_page,
                const float* amax_table) {
  if (table)
    hipExtLaunchKernelGGL((copy_runs_fp8_kernel<L, true>), dim3(blocks), dim3(kThreadsPerBlock), 0,
                          stream, ev.start, ev.stop, 0, runs, n_runs, total_slices, page_bytes,
                          rows_per_plane, kv_heads, rows_per_page, amax_table);
  else
    hipExtLaunchKernelGGL((copy_runs_fp8_kernel<L, false>), dim3(blocks), dim3(kThreadsPerBlock), 0,
                          stream, ev.start, ev.stop, 0, runs, n_runs, total_slices, page_bytes,
                          rows_per_plane, kv_heads, rows_per_page, amax_table);
}
}  // namespace

hipError_t launch_copy_runs_fp8(const DevRun* runs, uint32_t n_runs, uint32_t total_slices,
                                uint64_t page_bytes, uint32_t lanes_per_row,
                                uint32_t rows_per_plane, uint32_t kv_heads,
                                uint32_t rows_per_page, bool table, const float* amax_table,
                                const LaunchEvents& ev, hipStream_t stream) {
  const uint32_t waves = total_slices ? total_slices : 1u;
  const uint32_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  // One instantiation per row width (head_dim / 8 lanes), a shape, not a tuning choice.
#define PBE_FP8_CASE(L)                                                                      \
  case L:                                                                                    \
    launch_fp8<L>(table, blocks, stream, ev, runs, n_runs, total_slices, page_bytes,         \
                  rows_per_plane, kv_heads, rows_per_page, amax_table);                      \
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
