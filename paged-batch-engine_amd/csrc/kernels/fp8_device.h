// Device helpers shared by the gfx950 kernels that move BF16 KV into pages:
// 16-byte vector types, global-address-space pointers, and the FP8 E4M3
// conversion of the reference's KV writer (scatter_kv_kernel.cu:166-211).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pbe {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Global-address-space pointers: lets the compiler emit global_* instructions
// with a wave-uniform scalar base instead of flat_* with per-lane 64-bit bases.
#define PBE_GLOBAL __attribute__((address_space(1)))
typedef PBE_GLOBAL const uint8_t* gsrc_t;
typedef PBE_GLOBAL uint8_t* gdst_t;

constexpr int kWave = 64;

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

// FP32 input (scatter_kv_kernel.cu accepts FP32 K/V as well as BF16): four
// values per 16-byte vector. Products are checked for NaN directly.
__device__ __forceinline__ float amax4(u32x4 x) {
  float m = fabsf(__uint_as_float(x.x));
  m = fmaxf(m, fabsf(__uint_as_float(x.y)));
  m = fmaxf(m, fabsf(__uint_as_float(x.z)));
  return fmaxf(m, fabsf(__uint_as_float(x.w)));
}

__device__ __forceinline__ uint32_t quantise4(u32x4 x, float inv) {
  if (!(inv > 0.f)) return 0u;
  const uint32_t w = cvt_pair_e4m3_nan<false>(__uint_as_float(x.x) * inv, __uint_as_float(x.y) * inv, 0u);
  return cvt_pair_e4m3_nan<true>(__uint_as_float(x.z) * inv, __uint_as_float(x.w) * inv, w);
}

}  // namespace pbe
