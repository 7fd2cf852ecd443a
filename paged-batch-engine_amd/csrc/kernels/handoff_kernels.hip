// gfx950 kernels of the prefill->decode KV handoff.
//
// The handoff is a pure HBM stream: every copied page is read once and written
// once, so the kernels are bound by HBM bandwidth and use no MFMA.
//
// Work unit: one wavefront (64 lanes) moves one "slice" of a run, 64 lanes x
// 16-byte vectors x kUnroll. A run is contiguous on both sides across all of
// its pages (page = every layer's K and V planes, shared_kv_arena.h:35-36), so
// a slice never needs page or layer arithmetic: it is a contiguous byte span.
// Each wave owns a contiguous range of slices, finds its first run with a
// wave-parallel search over the device run list and then walks runs forward.
// Loads and stores are non-temporal: the source pages are dead after the
// handoff and the destination is not read until the next decode step, so
// neither should evict the decode working set from L2 / MALL.
#include <hip/hip_runtime.h>
#include <stdint.h>

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

__device__ __forceinline__ u32x4 ld16(gsrc_t p, uint32_t off) {
  return __builtin_nontemporal_load(reinterpret_cast<PBE_GLOBAL const u32x4*>(p + off));
}
__device__ __forceinline__ void st16(gdst_t p, uint32_t off, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<PBE_GLOBAL u32x4*>(p + off));
}
__device__ __forceinline__ void st8(gdst_t p, uint32_t off, u32x2 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<PBE_GLOBAL u32x2*>(p + off));
}

constexpr int kWave = 64;
constexpr int kWavesPerBlock = kThreadsPerBlock / kWave;

// Largest index r in [0, n) with runs[r].slice_begin <= s (runs[0] starts at 0).
// Each level lets the 64 lanes probe 64 evenly spaced candidates at once, so
// n runs take ceil(log64(n)) dependent loads instead of log2(n).
__device__ __forceinline__ uint32_t find_run(const DevRun* __restrict__ runs, uint32_t n,
                                             uint32_t s, uint32_t lane) {
  uint32_t lo = 0, count = n;
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

template <int kUnroll>
__device__ __forceinline__ void copy_slice(gsrc_t src, gdst_t dst, uint64_t nbytes,
                                           uint32_t lane) {
  constexpr uint32_t kSlice = kWave * 16u * kUnroll;
  u32x4 v[kUnroll];
  if (nbytes >= kSlice) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = ld16(src, (u * kWave + lane) * 16u);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) st16(dst, (u * kWave + lane) * 16u, v[u]);
  } else {
    // Last, partial slice of a run: rare, so keep it small rather than wide.
    for (uint32_t off = lane * 16u; off < nbytes; off += kWave * 16u) st16(dst, off, ld16(src, off));
  }
}

// Identity copy of every run: the device form of the reference's per-run
// cudaMemcpyAsync loop (split_pd_engine.cpp:96-108).
template <int kUnroll>
__global__ __launch_bounds__(kThreadsPerBlock) void copy_runs_kernel(
    const DevRun* __restrict__ runs, uint32_t n_runs, uint32_t total_slices,
    uint32_t slices_per_wave, uint64_t page_bytes) {
  constexpr uint32_t kSlice = kWave * 16u * kUnroll;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  const uint32_t s_begin = wave * slices_per_wave;
  if (s_begin >= total_slices) return;
  const uint32_t s_end = min(s_begin + slices_per_wave, total_slices);
  uint32_t r = find_run(runs, n_runs, s_begin, lane);
  uint32_t next = r + 1 < n_runs ? runs[r + 1].slice_begin : 0xffffffffu;
  for (uint32_t s = s_begin; s < s_end; ++s) {
    while (s >= next) {
      ++r;
      next = r + 1 < n_runs ? runs[r + 1].slice_begin : 0xffffffffu;
    }
    const DevRun& run = runs[r];
    const uint64_t rel = (uint64_t)(s - run.slice_begin) * kSlice;
    const uint64_t run_bytes = (uint64_t)run.pages * page_bytes;
    copy_slice<kUnroll>(reinterpret_cast<gsrc_t>(run.src + rel),
                        reinterpret_cast<gdst_t>(run.dst + rel), run_bytes - rel, lane);
  }
}

// ---- FP8 E4M3 (OCP v1.0, "fn": no infinities, 0x7F NaN, max 448) ----
// Round to nearest even with saturation to +-448, the conversion the reference
// asks of __nv_cvt_float_to_fp8(v, __NV_SATFINITE, __NV_E4M3)
// (scatter_kv_kernel.cu:207-210). gfx950's v_cvt_pk_fp8_f32 rounds to nearest
// even in the OCP format; clamping to +-448 first makes it saturate, and NaN
// is mapped explicitly because the clamp would otherwise absorb it.
template <bool kHi>
__device__ __forceinline__ uint32_t cvt_pair_e4m3(float a, float b, uint32_t old) {
  const float ca = fminf(fmaxf(a, -448.f), 448.f);
  const float cb = fminf(fmaxf(b, -448.f), 448.f);
  uint32_t packed = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, (int)old, kHi);
  const uint32_t sh = kHi ? 16u : 0u;
  if (a != a) packed = (packed & ~(0xffu << sh)) | (0x7fu << sh);
  if (b != b) packed = (packed & ~(0xff00u << sh)) | (0x7f00u << sh);
  return packed;
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Quantise 8 BF16 values (one 16-byte vector) with multiplier inv into 8 FP8
// bytes; inv == 0 yields +0 codes as in scatter_kv_kernel.cu:205-206.
__device__ __forceinline__ u32x2 quantise8(u32x4 x, float inv) {
  u32x2 out;
  if (inv > 0.f) {
    uint32_t w0 = cvt_pair_e4m3<false>(bf16_lo(x.x) * inv, bf16_hi(x.x) * inv, 0u);
    w0 = cvt_pair_e4m3<true>(bf16_lo(x.y) * inv, bf16_hi(x.y) * inv, w0);
    uint32_t w1 = cvt_pair_e4m3<false>(bf16_lo(x.z) * inv, bf16_hi(x.z) * inv, 0u);
    w1 = cvt_pair_e4m3<true>(bf16_lo(x.w) * inv, bf16_hi(x.w) * inv, w1);
    out.x = w0;
    out.y = w1;
  } else {
    out.x = 0u;
    out.y = 0u;
  }
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

// Fused BF16 -> FP8 handoff. A row is one (token, kv head) of one K or V
// plane: head_dim BF16 values = kLanesPerRow lanes x 8 values. Rows are laid
// out [layer][K|V][token][head] within a page on both sides, so a row's index
// inside the run (source offset / row bytes) is also its scale index.
//   per-token-head: amax over the row, scale = amax/448 | 1, inv = 448/amax | 0
//                   (scatter_kv_kernel.cu:166-190), scale written per row;
//   table:          amax = table[(2*layer+kv)*heads + head], nothing written.
template <int kUnroll, int kLanesPerRow, bool kTable>
__global__ __launch_bounds__(kThreadsPerBlock) void copy_runs_fp8_kernel(
    const DevRun* __restrict__ runs, uint32_t n_runs, uint32_t total_slices,
    uint32_t slices_per_wave, uint64_t page_bytes, uint32_t rows_per_plane,
    uint32_t kv_heads, uint32_t rows_per_page, const float* __restrict__ amax_table) {
  constexpr uint32_t kSlice = kWave * 16u * kUnroll;    // source bytes per slice
  constexpr uint32_t kRowBytes = kLanesPerRow * 16u;     // source bytes per row
  constexpr uint32_t kRowsPerStep = kWave / kLanesPerRow;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t wave = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  const uint32_t s_begin = wave * slices_per_wave;
  if (s_begin >= total_slices) return;
  const uint32_t s_end = min(s_begin + slices_per_wave, total_slices);
  uint32_t r = find_run(runs, n_runs, s_begin, lane);
  uint32_t next = r + 1 < n_runs ? runs[r + 1].slice_begin : 0xffffffffu;
  for (uint32_t s = s_begin; s < s_end; ++s) {
    while (s >= next) {
      ++r;
      next = r + 1 < n_runs ? runs[r + 1].slice_begin : 0xffffffffu;
    }
    const DevRun& run = runs[r];
    const uint64_t rel = (uint64_t)(s - run.slice_begin) * kSlice;
    const uint64_t run_bytes = (uint64_t)run.pages * page_bytes;
    const uint64_t nbytes = run_bytes - rel;
    gsrc_t src = reinterpret_cast<gsrc_t>(run.src + rel);
    gdst_t dst = reinterpret_cast<gdst_t>(run.dst + rel / 2);
    const uint32_t row0 = (uint32_t)(rel / kRowBytes);  // row index inside the run
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t off = (u * kWave + lane) * 16u;
      if (off < nbytes) v[u] = ld16(src, off);
      else v[u] = u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t off = (u * kWave + lane) * 16u;
      const uint32_t row = row0 + u * kRowsPerStep + lane / kLanesPerRow;
      float inv;
      if constexpr (kTable) {
        const uint32_t in_page = row % rows_per_page;
        const uint32_t plane = in_page / rows_per_plane;
        const float amax = amax_table[plane * kv_heads + in_page % kv_heads];
        inv = amax > 0.f ? 448.f / amax : 0.f;
      } else {
        float m = amax8(v[u]);
#pragma unroll
        for (int w = kLanesPerRow / 2; w >= 1; w /= 2) m = fmaxf(m, __shfl_xor(m, w, kWave));
        inv = m > 0.f ? 448.f / m : 0.f;
        if (lane % kLanesPerRow == 0 && off < nbytes) {
          const float scale = m > 0.f ? m / 448.f : 1.f;
          __builtin_nontemporal_store(scale, reinterpret_cast<PBE_GLOBAL float*>(run.aux) + row);
        }
      }
      if (off < nbytes) st8(dst, off / 2, quantise8(v[u], inv));
    }
  }
}

// Generic op-list copy: one wave per op slice. Ops whose addresses and size
// are 16-byte multiples take the vector path; others fall back to bytes.
__global__ __launch_bounds__(kThreadsPerBlock) void copy_ops_kernel(
    const DevOp* __restrict__ ops, uint32_t n_ops) {
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t waves = gridDim.x * kWavesPerBlock;
  for (uint32_t i = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave; i < n_ops; i += waves) {
    const DevOp op = ops[i];
    const uint8_t* src = reinterpret_cast<const uint8_t*>(op.src);
    uint8_t* dst = reinterpret_cast<uint8_t*>(op.dst);
    if (((op.src | op.dst | op.bytes) & 15u) == 0) {
      for (uint64_t off = (uint64_t)lane * 16u; off < op.bytes; off += kWave * 16u) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + off));
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst + off));
      }
    } else {
      for (uint64_t off = lane; off < op.bytes; off += kWave) dst[off] = src[off];
    }
  }
}

}  // namespace

uint32_t slice_bytes(KernelKind kind) {
  return kind == KernelKind::kCopy ? kWave * 16u * kCopyUnroll : kWave * 16u * kFp8Unroll;
}

hipError_t launch_copy_runs(const DevRun* runs, uint32_t n_runs, uint32_t total_slices,
                            uint64_t page_bytes, const LaunchShape& shape, hipStream_t stream) {
  const uint32_t waves = (total_slices + shape.slices_per_wave - 1) / shape.slices_per_wave;
  const uint32_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  hipLaunchKernelGGL(copy_runs_kernel<kCopyUnroll>, dim3(blocks), dim3(kThreadsPerBlock), 0,
                     stream, runs, n_runs, total_slices, shape.slices_per_wave, page_bytes);
  return hipGetLastError();
}

hipError_t launch_copy_runs_fp8(const DevRun* runs, uint32_t n_runs, uint32_t total_slices,
                                uint64_t page_bytes, uint32_t lanes_per_row,
                                uint32_t rows_per_plane, uint32_t kv_heads,
                                uint32_t rows_per_page, bool table, const float* amax_table,
                                const LaunchShape& shape, hipStream_t stream) {
  const uint32_t waves = (total_slices + shape.slices_per_wave - 1) / shape.slices_per_wave;
  const uint32_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
#define PBE_FP8_CASE(L)                                                                     \
  case L:                                                                                   \
    if (table)                                                                              \
      hipLaunchKernelGGL((copy_runs_fp8_kernel<kFp8Unroll, L, true>), dim3(blocks),         \
                         dim3(kThreadsPerBlock), 0, stream, runs, n_runs, total_slices,     \
                         shape.slices_per_wave, page_bytes, rows_per_plane, kv_heads,       \
                         rows_per_page, amax_table);                                        \
    else                                                                                    \
      hipLaunchKernelGGL((copy_runs_fp8_kernel<kFp8Unroll, L, false>), dim3(blocks),        \
                         dim3(kThreadsPerBlock), 0, stream, runs, n_runs, total_slices,     \
                         shape.slices_per_wave, page_bytes, rows_per_plane, kv_heads,       \
                         rows_per_page, amax_table);                                        \
    break;
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
  return hipGetLastError();
}

hipError_t launch_copy_ops(const DevOp* ops, uint32_t n_ops, hipStream_t stream) {
  const uint32_t waves = n_ops;
  uint32_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  if (blocks > 65535u) blocks = 65535u;
  hipLaunchKernelGGL(copy_ops_kernel, dim3(blocks), dim3(kThreadsPerBlock), 0, stream, ops,
                     n_ops);
  return hipGetLastError();
}

}  // namespace pbe
