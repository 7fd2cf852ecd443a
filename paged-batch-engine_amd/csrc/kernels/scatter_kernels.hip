// gfx950 writer of new tokens' K/V into their page slots: the device side of
// scatter_kv_batch_to_pages_cu / scatter_kv_batch_to_pages_fp8_e4m3_cu
// (scatter_kv_kernel.cu:99-216).
//
// Work unit: one lane moves one 16-byte vector of an input row. Units run
// token-major ([token][K|V][vector]), so a wave reads a contiguous stretch of
// the token-major K and V inputs and writes whole rows of the pages. A row
// (token, K|V) shares one slot, so every lane of a row takes the same
// skip-or-write decision; for FP8 a (token, K|V, head) group of lanes shares
// one amax through DPP, and the group's first lane writes the scale.
//
// Memory: each input vector is read once (non-temporal load); the pages are
// read by this layer's attention next, so stores keep the default policy.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fp8_device.h"
#include "scatter_kernels.h"

namespace pbe {
namespace {

__device__ __forceinline__ uint32_t div_by(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.mul) + n) >> f.shift;
}

template <bool kF32, bool kFp8, int kLanesPerHead>
__global__ __launch_bounds__(kThreadsPerBlock) void scatter_kv_kernel(const ScatterParams p) {
  const uint32_t u = blockIdx.x * kThreadsPerBlock + threadIdx.x;
  if (u >= p.units) return;
  const uint32_t token = div_by(u, p.by_row_pair);           // 2 rows (K, V) per token
  const uint32_t in_pair = u - token * 2u * p.vecs_per_row;
  const uint32_t kv = in_pair >= p.vecs_per_row ? 1u : 0u;
  const uint32_t vec = in_pair - kv * p.vecs_per_row;
  // The input vector does not depend on the slot: both loads go out together,
  // so a wave waits for one memory round trip before its store, not two.
  const uint8_t* in = (kv ? p.values : p.keys) + (uint64_t)token * p.row_in_bytes;
  const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(in + (uint64_t)vec * 16u));
  const int32_t slot = p.slots ? p.slots[token] : p.fixed_slot;
  if (slot < 0) return;  // scatter_kv_kernel.cu:147-149
  const uint32_t block = div_by((uint32_t)slot, p.by_block_size);
  const uint32_t offset = (uint32_t)slot - block * p.block_size;
  const uint64_t out_row = (uint64_t)block * p.block_out_bytes + (uint64_t)offset * p.row_out_bytes;
  if (out_row + p.row_out_bytes > (kv ? p.value_pool_bytes : p.key_pool_bytes)) return;
  uint8_t* out = (kv ? p.value_pool : p.key_pool) + out_row;
  if constexpr (!kFp8) {
    *reinterpret_cast<u32x4*>(out + (uint64_t)vec * 16u) = x;  // plain: the pool holds the input type
  } else {
    const uint32_t head = vec / kLanesPerHead;
    const uint64_t scale_idx = ((uint64_t)block * p.block_size + offset) * p.kv_heads + head;
    if (scale_idx >= (kv ? p.value_scale_count : p.key_scale_count)) return;
    const float m = group_max<kLanesPerHead>(kF32 ? amax4(x) : amax8(x));
    const float inv = m > 0.f ? 448.f / m : 0.f;
    if (vec % kLanesPerHead == 0) (kv ? p.value_scales : p.key_scales)[scale_idx] = m > 0.f ? m / 448.f : 1.f;
    if constexpr (kF32)
      *reinterpret_cast<uint32_t*>(out + (uint64_t)vec * 4u) = quantise4(x, inv);
    else
      *reinterpret_cast<u32x2*>(out + (uint64_t)vec * 8u) = quantise8(x, inv);
  }
}

template <bool kF32, bool kFp8>
hipError_t launch_lanes(const ScatterParams& p, uint32_t lanes_per_head, hipStream_t stream) {
  const dim3 grid((p.units + kThreadsPerBlock - 1) / kThreadsPerBlock), block(kThreadsPerBlock);
  if constexpr (!kFp8) {  // plain rows need no per-head grouping
    hipLaunchKernelGGL((scatter_kv_kernel<kF32, false, 1>), grid, block, 0, stream, p);
    return hipGetLastError();
  }
  switch (lanes_per_head) {
    case 1: hipLaunchKernelGGL((scatter_kv_kernel<kF32, kFp8, 1>), grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL((scatter_kv_kernel<kF32, kFp8, 2>), grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL((scatter_kv_kernel<kF32, kFp8, 4>), grid, block, 0, stream, p); break;
    case 8: hipLaunchKernelGGL((scatter_kv_kernel<kF32, kFp8, 8>), grid, block, 0, stream, p); break;
    case 16: hipLaunchKernelGGL((scatter_kv_kernel<kF32, kFp8, 16>), grid, block, 0, stream, p); break;
    case 32: hipLaunchKernelGGL((scatter_kv_kernel<kF32, kFp8, 32>), grid, block, 0, stream, p); break;
    case 64: hipLaunchKernelGGL((scatter_kv_kernel<kF32, kFp8, 64>), grid, block, 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_scatter_kv(const ScatterParams& p, bool f32_input, bool fp8, uint32_t lanes_per_head,
                             hipStream_t stream) {
  if (p.units == 0) return hipSuccess;
  if (!fp8) return f32_input ? launch_lanes<true, false>(p, 1, stream) : launch_lanes<false, false>(p, 1, stream);
  return f32_input ? launch_lanes<true, true>(p, lanes_per_head, stream)
                   : launch_lanes<false, true>(p, lanes_per_head, stream);
}

}  // namespace pbe
