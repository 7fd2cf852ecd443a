// Decode-side reader of handed-off KV pages: split-K paged attention for one
// query token per sequence, over the page-major arena (FP8 E4M3 planes with
// per-(token, head) scales, or BF16 planes). Same arithmetic as the
// reference's splitkv_paged_mha_fp8_stage1_kernel / _fast_stage1_kernel and
// splitkv_paged_mha_fast_stage2_kernel (paged_mha_fast_kernel.cu:391-800):
// score = (q . k) * (log2(e)/sqrt(D) * k_scale), online softmax in base 2,
// acc += v * (p * v_scale), output = acc / sum as BF16 (round to nearest even).
//
// gfx950 mapping. One wave owns one (sequence, KV head, split) and walks its
// blocks of 16 tokens:
//  - scores: one v_mfma_f32_16x16x32_bf16 per 32 head dims. A = the query
//    heads sharing the KV head (rows, padded to 16), B = the block's 16 keys
//    (columns). FP8 keys become BF16 exactly (an E4M3 value has at most 3
//    mantissa bits). The contraction order over head dims is permuted the
//    same way in A and B so each lane reads one contiguous run of its key.
//  - softmax: row max / row sum over the 16 token lanes with DPP row ops.
//  - values: lane (g, j) accumulates tokens 4g..4g+3 of the block for head
//    dims j*D/16.., all query heads of the group, in fp32 registers; the
//    four token groups are summed once at the end.
// A second kernel combines the splits.
#include "decode_kernels.h"

namespace pbe {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWavesPerBlock = 4;
constexpr int kBlockTokens = 16;

template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xf, 0xf, false));
}

// Reductions over the 16 lanes of a DPP row: quad_perm [1,0,3,2],
// quad_perm [2,3,0,1], row_half_mirror, row_mirror.
__device__ __forceinline__ float row_max16(float x) {
  x = fmaxf(x, dpp<0xb1>(x));
  x = fmaxf(x, dpp<0x4e>(x));
  x = fmaxf(x, dpp<0x141>(x));
  return fmaxf(x, dpp<0x140>(x));
}

__device__ __forceinline__ float row_sum16(float x) {
  x += dpp<0xb1>(x);
  x += dpp<0x4e>(x);
  x += dpp<0x141>(x);
  return x + dpp<0x140>(x);
}

__device__ __forceinline__ float wave_max(float x) {
  x = row_max16(x);
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}

__device__ __forceinline__ float wave_sum(float x) {
  x = row_sum16(x);
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

// Orders this wave's LDS writes before its other lanes' reads.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Four E4M3 bytes -> four BF16 (exact), packed in two words.
__device__ __forceinline__ u32x2 e4m3x4_to_bf16x4(uint32_t w) {
  const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  return u32x2{(__float_as_uint(lo[0]) >> 16) | (__float_as_uint(lo[1]) & 0xffff0000u),
               (__float_as_uint(hi[0]) >> 16) | (__float_as_uint(hi[1]) & 0xffff0000u)};
}

__device__ __forceinline__ void e4m3x4_to_f32(uint32_t w, float* out) {
  const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  out[0] = lo[0];
  out[1] = lo[1];
  out[2] = hi[0];
  out[3] = hi[1];
}

// fp32 -> bf16, round to nearest even; NaN stays NaN (quiet).
__device__ __forceinline__ uint16_t to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ const char* arena_at(const DecodeView& v, uint64_t off) {
  const uint64_t seg = off / v.segment_bytes;
  return v.base[seg] + (off - seg * v.segment_bytes);
}

template <int D, bool kFp8>
__global__ __launch_bounds__(kWavesPerBlock * 64) void paged_decode_kernel(const DecodeParams p) {
  constexpr int E = kFp8 ? 1 : 2;  // bytes per stored element
  constexpr int NK = D / 32;       // score MFMAs per block
  constexpr int DG = D / 4;        // head dims per lane group in the score tile
  constexpr int DV = D / 16;       // head dims per lane in the value sum
  constexpr int KVM = kDecodeMaxKvMul;
  __shared__ float lds_p[kWavesPerBlock][kBlockTokens][17];
  __shared__ float lds_alpha[kWavesPerBlock][16];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t unit = (int64_t)blockIdx.x * kWavesPerBlock + w;
  if (unit >= (int64_t)p.batch * p.kv_heads * p.splits) return;
  const int split = (int)(unit % p.splits);
  const int kvh = (int)((unit / p.splits) % p.kv_heads);
  const int b = (int)(unit / p.splits / p.kv_heads);
  const int kvm = p.q_heads / p.kv_heads;
  const int g = lane >> 4, j = lane & 15;
  const int seq = p.seq_lens[b];
  const int nblk = seq > 0 ? (seq + kBlockTokens - 1) / kBlockTokens : 0;
  bool bad = seq < 0 || nblk > p.max_blocks;
  // Each sequence's blocks are cut into `splits` equal ranges
  // (paged_mha_fast_kernel.cu:596-601).
  const int per_split = (nblk + p.splits - 1) / p.splits;
  const int blk0 = split * per_split;
  const int blk1 = bad ? blk0 : min(blk0 + per_split, nblk);

  // Query rows (A operand): lane (g, j) holds head j's dims g*DG + 8kk + 0..7.
  bf16x8 qa[NK];
  {
    const bool has = j < kvm;
    const uint16_t* qrow =
        p.q + ((int64_t)b * p.q_heads + (int64_t)kvh * kvm + (has ? j : 0)) * D + g * DG;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      const u32x4 v = has ? *reinterpret_cast<const u32x4*>(qrow + kk * 8) : u32x4{0u, 0u, 0u, 0u};
      qa[kk] = __builtin_bit_cast(bf16x8, v);
    }
  }
  float m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
  }
  float acc[KVM][DV];
#pragma unroll
  for (int h = 0; h < KVM; ++h)
#pragma unroll
    for (int e = 0; e < DV; ++e) acc[h][e] = 0.f;

  const uint64_t H = (uint64_t)p.kv_heads;
  const uint64_t token_stride = H * D * E;
  const uint64_t stride = 2ull * p.layers;
  for (int blk = blk0; blk < blk1; ++blk) {
    const int32_t id = p.tables[(int64_t)b * p.max_blocks + blk];
    if (id < 0 || (uint64_t)id % stride != 0 || ((uint64_t)id + stride) * p.half > p.kv.bytes ||
        (kFp8 && ((uint64_t)id + stride) * kBlockTokens * H * 4ull > p.scale_bytes)) {
      bad = true;
      break;
    }
    const int valid = blk == nblk - 1 ? seq - kBlockTokens * (nblk - 1) : kBlockTokens;
    const char* page = arena_at(p.kv, (uint64_t)id * p.half);
    const char* kplane = page + 2ull * p.layer * p.half + (uint64_t)kvh * D * E;
    const char* vplane = kplane + p.half;

    // ---- scores of the block's 16 tokens (B operand: lane (g, j) = token j)
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    const char* krow = kplane + (uint64_t)j * token_stride + (uint64_t)g * DG * E;
    if constexpr (kFp8) {
      uint32_t words[DG / 4];
#pragma unroll
      for (int v = 0; v < DG / 16; ++v) {
        const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(krow) + v);
        words[4 * v] = x[0];
        words[4 * v + 1] = x[1];
        words[4 * v + 2] = x[2];
        words[4 * v + 3] = x[3];
      }
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
        const u32x2 lo = e4m3x4_to_bf16x4(words[2 * kk]);
        const u32x2 hi = e4m3x4_to_bf16x4(words[2 * kk + 1]);
        const bf16x8 kb = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[kk], kb, s, 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
        const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(krow) + kk);
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[kk], __builtin_bit_cast(bf16x8, x), s, 0, 0, 0);
      }
    }
    const bool tok_ok = j < valid;
    float ks = 1.f, vs = 1.f;
    if constexpr (kFp8) {
      if (tok_ok) {
        const uint64_t kidx = ((uint64_t)id + 2ull * p.layer) * kBlockTokens + j;
        ks = p.scales[kidx * H + kvh];
        vs = p.scales[(kidx + kBlockTokens) * H + kvh];
      }
    }
    const float c = p.scale * ks;
    // ---- online softmax; lane (g, j) holds heads 4g..4g+3 of token j
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sv = tok_ok ? s[i] * c : -INFINITY;
      const float mn = fmaxf(m[i], row_max16(sv));
      const float alpha = mn == -INFINITY ? 1.f : exp2f(m[i] - mn);
      const float pr = tok_ok ? exp2f(sv - mn) : 0.f;
      l[i] = l[i] * alpha + row_sum16(pr);
      m[i] = mn;
      lds_p[w][j][4 * g + i] = pr * vs;
      if (j == 0) lds_alpha[w][4 * g + i] = alpha;
    }
    wave_sync();
    // ---- values: lane (g, j) takes tokens 4g..4g+3, dims j*DV..j*DV+DV-1
#pragma unroll
    for (int h = 0; h < KVM; ++h) {
      if (h < kvm) {
        const float a = lds_alpha[w][h];
#pragma unroll
        for (int e = 0; e < DV; ++e) acc[h][e] *= a;
      }
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int t = 4 * g + tt;
      const bool ok = t < valid;  // tail slots may hold anything, even NaN
      const char* vrow = vplane + (uint64_t)t * token_stride + (uint64_t)j * DV * E;
      float vf[DV];
      if constexpr (kFp8) {
        if constexpr (DV == 8) {
          const u32x2 x = ok ? *reinterpret_cast<const u32x2*>(vrow) : u32x2{0u, 0u};
          e4m3x4_to_f32(x[0], vf);
          e4m3x4_to_f32(x[1], vf + 4);
        } else {
          const uint32_t x = ok ? *reinterpret_cast<const uint32_t*>(vrow) : 0u;
          e4m3x4_to_f32(x, vf);
        }
      } else {
        uint32_t x[DV / 2];
        if constexpr (DV == 8) {
          const u32x4 y = ok ? *reinterpret_cast<const u32x4*>(vrow) : u32x4{0u, 0u, 0u, 0u};
          x[0] = y[0];
          x[1] = y[1];
          x[2] = y[2];
          x[3] = y[3];
        } else {
          const u32x2 y = ok ? *reinterpret_cast<const u32x2*>(vrow) : u32x2{0u, 0u};
          x[0] = y[0];
          x[1] = y[1];
        }
#pragma unroll
        for (int e = 0; e < DV / 2; ++e) {
          vf[2 * e] = __uint_as_float(x[e] << 16);
          vf[2 * e + 1] = __uint_as_float(x[e] & 0xffff0000u);
        }
      }
#pragma unroll
      for (int h = 0; h < KVM; ++h) {
        if (h < kvm) {
          const float ph = lds_p[w][t][h];
#pragma unroll
          for (int e = 0; e < DV; ++e) acc[h][e] = fmaf(ph, vf[e], acc[h][e]);
        }
      }
    }
    wave_sync();
  }

  // ---- sum the four token groups and write this split's partials
#pragma unroll
  for (int h = 0; h < KVM; ++h) {
    if (h < kvm) {
#pragma unroll
      for (int e = 0; e < DV; ++e) {
        acc[h][e] += __shfl_xor(acc[h][e], 16);
        acc[h][e] += __shfl_xor(acc[h][e], 32);
      }
    }
  }
  const int64_t row0 = (int64_t)b * p.q_heads + (int64_t)kvh * kvm;
  const float nan = __builtin_nanf("");
  if (g == 0) {
#pragma unroll
    for (int h = 0; h < KVM; ++h) {
      if (h < kvm) {
        float* dst = p.part_acc + ((row0 + h) * p.splits + split) * D + j * DV;
#pragma unroll
        for (int e = 0; e < DV; ++e) dst[e] = bad ? nan : acc[h][e];
      }
    }
  }
  if (j == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * g + i;
      if (h < kvm) {
        p.part_m[(row0 + h) * p.splits + split] = bad ? nan : m[i];
        p.part_l[(row0 + h) * p.splits + split] = bad ? nan : l[i];
      }
    }
  }
}

// One wave per (sequence, query head): combines the splits as
// splitkv_paged_mha_fast_stage2_kernel does (paged_mha_fast_kernel.cu:730-799).
template <int D>
__global__ __launch_bounds__(kWavesPerBlock * 64) void decode_combine_kernel(const DecodeParams p) {
  constexpr int PER = D / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + w;
  if (row >= (int64_t)p.batch * p.q_heads) return;
  const int S = p.splits;
  float ms = -INFINITY, ls = 0.f;
  if (lane < S) {
    ms = p.part_m[row * S + lane];
    ls = p.part_l[row * S + lane];
  }
  const bool any_nan = __ballot(ls != ls) != 0;
  const float m = wave_max(ms);
  const float denom = wave_sum((lane < S && ls > 0.f) ? ls * exp2f(ms - m) : 0.f);
  float o[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) o[e] = 0.f;
  for (int s = 0; s < S; ++s) {
    const float sl = __shfl(ls, s), sm = __shfl(ms, s);
    if (!(sl > 0.f)) continue;
    const float a = exp2f(sm - m);
    const float* src = p.part_acc + (row * S + s) * D + lane * PER;
#pragma unroll
    for (int e = 0; e < PER; ++e) o[e] += src[e] * a;
  }
  uint16_t* dst = p.out + row * D + lane * PER;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const float v = any_nan ? __builtin_nanf("") : (denom > 0.f ? o[e] / denom : 0.f);
    dst[e] = to_bf16(v);
  }
}

template <int D, bool kFp8>
void launch(const DecodeParams& p, hipStream_t stream) {
  const int64_t units = (int64_t)p.batch * p.kv_heads * p.splits;
  const int64_t rows = (int64_t)p.batch * p.q_heads;
  hipLaunchKernelGGL((paged_decode_kernel<D, kFp8>),
                     dim3((unsigned)((units + kWavesPerBlock - 1) / kWavesPerBlock)),
                     dim3(kWavesPerBlock * 64), 0, stream, p);
  hipLaunchKernelGGL((decode_combine_kernel<D>),
                     dim3((unsigned)((rows + kWavesPerBlock - 1) / kWavesPerBlock)),
                     dim3(kWavesPerBlock * 64), 0, stream, p);
}

}  // namespace

uint64_t decode_workspace_bytes(int32_t batch, int32_t q_heads, int32_t head_dim, int32_t splits) {
  const uint64_t rows = (uint64_t)batch * q_heads * splits;
  return rows * head_dim * 4ull + 2ull * rows * 4ull;
}

hipError_t launch_paged_decode(const DecodeParams& p, bool fp8, hipStream_t stream) {
  if (p.head_dim == 128) {
    if (fp8) launch<128, true>(p, stream);
    else launch<128, false>(p, stream);
  } else if (p.head_dim == 64) {
    if (fp8) launch<64, true>(p, stream);
    else launch<64, false>(p, stream);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace pbe
