// Decode-side reader of handed-off KV pages: split-K paged attention for one
// query token per sequence, over the page-major arena (FP8 E4M3 planes with
// per-(token, head) scales, or BF16 planes). Same arithmetic as the
// reference's splitkv_paged_mha_fp8_stage1_kernel / _fast_stage1_kernel and
// splitkv_paged_mha_fast_stage2_kernel (paged_mha_fast_kernel.cu:391-800):
// score = (q . k) * (log2(e)/sqrt(D) * k_scale), online softmax in base 2,
// acc += v * (p * v_scale), output = acc / sum as BF16 (round to nearest even).
//
// gfx950 mapping. One wave owns one (sequence, KV head, split) and walks its
// blocks of 16 tokens; the KV heads of one (sequence, split) are neighbouring
// waves of a workgroup, so a block's rows are read together:
//  - loads: a key load instruction covers 64 contiguous bytes of each of the
//    16 rows (the MFMA wants one row per lane). A value load instruction
//    covers whole rows, i.e. full 128-byte lines, since the value tile is
//    rearranged in LDS anyway; requesting half lines instead costs 10% of
//    the BF16 step. 2 to 8 register sets rotate so that the next blocks are
//    in flight while one is computed.
//  - scores, transposed: one v_mfma_f32_16x16x32_bf16 per 32 head dims,
//    A = the block's 16 keys (rows), B = the query heads sharing the KV head
//    (columns, padded to 16). FP8 keys become BF16 exactly (an E4M3 value has
//    at most 3 mantissa bits). The contraction order over head dims follows
//    the load order, in A and B alike. Lane (g, j) ends with tokens 4g..4g+3
//    of query head j.
//  - softmax: per head in-lane, across the four lane groups with the gfx950
//    row swaps (v_permlane32_swap / v_permlane16_swap).
//  - values: the value tile goes through LDS once and comes back transposed
//    with ds_read_b64_tr_b8 / _b16, four tokens of one head dim per lane, as
//    the A operand of O^T += V^T P^T (P^T as held, split into a BF16 high and
//    low part, K = 32).
// A second kernel combines the splits.
//
// Append variant (kAppend): the step's new token of every sequence, at its
// last position, is written into its page slot by the one wave that reads
// that block (per KV head only one wave reads a given row), with the page
// writer's arithmetic (scatter_kv_kernel.cu:128-216). The wave takes the row
// from its registers rather than from memory, so no ordering between the
// store and any load is needed, and the result equals writing the row first
// and reading the pages afterwards, byte for byte.
#include "decode_kernels.h"
#include "fp8_device.h"

namespace pbe {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

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

// Max / sum over the four lanes j, j+16, j+32, j+48 with the gfx950 row
// swaps (VALU only, no LDS round trip). Every lane ends with the same value,
// combined in the same order.
__device__ __forceinline__ float group_max4(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float group_sum4(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Orders this wave's LDS writes before its other lanes' reads.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// fp32 -> bf16, round to nearest even; NaN stays NaN (quiet).
__device__ __forceinline__ uint16_t to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ uint32_t fast_div(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.mul) + n) >> f.shift;
}

// Four E4M3 bytes -> four BF16 with the gfx950 scaled converter (scale 1: exact).
__device__ __forceinline__ u32x2 e4m3x4_to_bf16x4_cvt(uint32_t w) {
  return u32x2{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, true))};
}

// Per-lane registers of one block of 16 tokens of one KV head: the lane's
// part of key row j, its whole-row-mapped part of the value tile and one scale.
template <int D, bool kFp8>
struct Geo {
  static constexpr int E = kFp8 ? 1 : 2;
  static constexpr int WORDS = D * E / 16;   // key words = value words per lane
  static constexpr int PITCH = D * E + 16;   // LDS row pitch of the value tile
};

template <int W, bool kFp8>
struct BlockRegs {
  uint32_t k[W];
  uint32_t v[W];
  // FP8: lane (g, n): log2(e)/sqrt(D) * key scale (n%8 < 4) or value scale
  // (otherwise) of token 4g + n%4
  float scale;
};

constexpr int kDecodeWaves = 4;

// kSets register sets per wave: kSets-1 blocks in flight while one is
// computed (chosen at launch, see sets_for).
template <int D, bool kFp8, int KVM, bool kAppend, int kSets>
__global__ __launch_bounds__(kDecodeWaves * 64) void paged_decode_kernel(
    const DecodeParams p, const int32_t* __restrict__ tables) {
  using G = Geo<D, kFp8>;
  constexpr int E = G::E;
  constexpr int NK = D / 32;  // score MFMAs per block
  constexpr int NT = D / 16;  // value MFMAs (16 head dims each) per block
  constexpr int W = G::WORDS, SETS = kSets, PITCH = G::PITCH;
  __shared__ __attribute__((aligned(16))) unsigned char lds_v[kDecodeWaves][kBlockTokens * PITCH];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t unit = (int64_t)blockIdx.x * kDecodeWaves + w;
  if (unit >= (int64_t)p.batch * p.kv_heads * p.splits) return;
  const int kvh = (int)(unit % p.kv_heads);
  const int split = (int)((unit / p.kv_heads) % p.splits);
  const int b = (int)(unit / p.kv_heads / p.splits);
  const int g = lane >> 4, j = lane & 15;
  const int seq = p.seq_lens[b];
  const int nblk = seq > 0 ? (seq + kBlockTokens - 1) / kBlockTokens : 0;
  bool bad = seq < 0 || nblk > p.max_blocks;
  // Each sequence's blocks are cut into `splits` equal ranges
  // (paged_mha_fast_kernel.cu:596-601).
  const int per_split = (nblk + p.splits - 1) / p.splits;
  const int blk0 = split * per_split;
  int blk1 = bad ? blk0 : min(blk0 + per_split, nblk);

  // Query rows as the B operand of the scores: lane (g, j) holds head j's
  // dims matching the key bytes MFMA kk consumes (rows past the group's
  // heads are zero).
  bf16x8 qa[NK];
  {
    const bool has = j < KVM;
    const uint16_t* qrow =
        p.q + ((int64_t)b * p.q_heads + (int64_t)kvh * KVM + (has ? j : 0)) * D;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      // the head dims of the key bytes this MFMA consumes (see key_off)
      const int cb = kk * 8 * E;
      const int dim0 = (64 / E) * (cb / 16) + (16 / E) * g + (cb % 16) / E;
      const u32x4 v = has ? *reinterpret_cast<const u32x4*>(qrow + dim0) : u32x4{0u, 0u, 0u, 0u};
      qa[kk] = __builtin_bit_cast(bf16x8, v);
    }
  }

  const uint64_t H = (uint64_t)p.kv_heads;
  const uint32_t token_stride = (uint32_t)(H * D * E);
  const uint64_t stride = p.by_stride.d;
  // Block ids are uniform: read through the read-only table with scalar loads.
  const int32_t* table = tables + (int64_t)b * p.max_blocks;
  const uint64_t head_off = 2ull * p.layer * p.half + (uint64_t)kvh * D * E;
  // Key load v of lane (g, j) reads bytes 64v + 16g.. of key row j: 64
  // contiguous bytes of every row per instruction. The key's head dims are
  // consumed in that order; the queries are read in the same order.
  const uint32_t key_off = (uint32_t)j * token_stride + (uint32_t)(16 * g);
  // Value load v of lane l reads the 16 bytes at column vcol of row
  // v * RPI + vrow0: each instruction covers RPI whole rows.
  constexpr int LPR = D * E / 16, RPI = 64 / LPR;  // lanes per row, rows per load
  constexpr int RL = D / 8;  // append: 16-byte BF16 input vectors per head row
  const int vrow0 = lane / LPR, vcol = 16 * (lane % LPR);
  const uint32_t val_off = (uint32_t)vrow0 * token_stride + (uint32_t)vcol;
  // lane (g, j): scale of token 4g + j%4 from the key (j%8 < 4) or value plane
  const int64_t scale_off =
      (int64_t)((2u * p.layer * kBlockTokens + 4u * g + (j & 3)) * H + kvh) + ((j >> 2) & 1 ? p.vscale_delta : 0);
  // Loads block `blk` into `r`. Every call issues the same loads (an
  // unconditional count keeps the compiler's in-flight accounting exact): a
  // block past the split's end, or whose id is not a page id inside the arena
  // and scale pool, reads page 0 instead and reports false when it was wanted.
  auto load = [&](int blk, BlockRegs<W, kFp8>& r) -> bool {
    const bool want = blk < blk1;
    int32_t id = want ? table[blk] : 0;
    uint32_t page = fast_div((uint32_t)max(id, 0), p.by_stride);
    const bool ok = id >= 0 && id <= p.id_max && page * p.by_stride.d == (uint32_t)id;
    if (!ok) id = 0, page = 0;
    const uint32_t seg = fast_div(page, p.by_seg_pages);
    const char* kplane =
        p.kv.base[seg] + (uint64_t)(page - seg * p.by_seg_pages.d) * stride * p.half + head_off;
#pragma unroll
    for (int v = 0; v < W / 4; ++v) {
      const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kplane + key_off + 64 * v));
      const u32x4 y = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(kplane + p.v_delta + val_off + (uint64_t)v * RPI * token_stride));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        r.k[4 * v + e] = x[e];
        r.v[4 * v + e] = y[e];
      }
    }
    if constexpr (kFp8) {  // key scales carry the score scale: p.scale * k_scale
      // Non-temporal like the page rows: plain loads cost 8% of the FP8 step.
      const float sc = __builtin_nontemporal_load(p.scales + (uint64_t)id * kBlockTokens * H + scale_off);
      r.scale = (j & 4) ? sc : p.scale * sc;
    }
    return ok || !want;
  };

  float m = -INFINITY, l = 0.f;  // of head j
  f32x4 acc[NT];                 // O^T: lane (g, j) = head j, dims 16nt + 4g + 0..3
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Append: the new token's row of this KV head as lane (g, j) holds key row
  // j (nk), as the value writer lanes computed it (nv), its scales, and the
  // block it lands in (-1: nothing to write here).
  uint32_t nk[kAppend ? W : 1], nv[kAppend ? 4 : 1];
  float nks = 0.f, nvs = 0.f;
  int patch_blk = -1, slot_row = 0;

  unsigned char* vt_w = &lds_v[w][0];
  auto compute = [&](int blk, const BlockRegs<W, kFp8>& r) {
    const int valid = blk == nblk - 1 ? seq - kBlockTokens * (nblk - 1) : kBlockTokens;
    const bool patch = kAppend && blk == patch_blk;
    // Value tile -> LDS rows (tail rows zeroed: tail slots may hold anything, even NaN).
    {
      unsigned char* dst = vt_w + vrow0 * PITCH + vcol;
#pragma unroll
      for (int v = 0; v < W / 4; ++v) {
        const u32x4 x = v * RPI + vrow0 < valid
                            ? u32x4{r.v[4 * v], r.v[4 * v + 1], r.v[4 * v + 2], r.v[4 * v + 3]}
                            : u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(dst + v * RPI * PITCH) = x;
      }
      // The new row replaces what was read (LDS writes of one wave land in
      // issue order).
      if constexpr (kAppend) {
        if (patch && lane >= 32 && (lane & 31) < RL) {
          unsigned char* row = vt_w + slot_row * PITCH + (kFp8 ? 8 : 16) * (lane & 31);
          if constexpr (kFp8) *reinterpret_cast<u32x2*>(row) = u32x2{nv[0], nv[1]};
          else *reinterpret_cast<u32x4*>(row) = u32x4{nv[0], nv[1], nv[2], nv[3]};
        }
      }
    }
    // Scores, transposed: lane (g, j) gets tokens 4g..4g+3 of head j.
    uint32_t kw[W];
#pragma unroll
    for (int i = 0; i < W; ++i) kw[i] = r.k[i];
    float rscale = kFp8 ? r.scale : 0.f;
    if constexpr (kAppend) {
      if (patch) {
        const bool mine = j == slot_row;
#pragma unroll
        for (int i = 0; i < W; ++i) kw[i] = mine ? nk[i] : kw[i];
        if (4 * g + (j & 3) == slot_row) rscale = (j & 4) ? nvs : p.scale * nks;
      }
    }
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      bf16x8 kb;
      if constexpr (kFp8) {
        const u32x2 lo = e4m3x4_to_bf16x4_cvt(kw[2 * kk]);
        const u32x2 hi = e4m3x4_to_bf16x4_cvt(kw[2 * kk + 1]);
        kb = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
      } else {
        kb = __builtin_bit_cast(bf16x8, u32x4{kw[4 * kk], kw[4 * kk + 1], kw[4 * kk + 2], kw[4 * kk + 3]});
      }
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kb, qa[kk], s, 0, 0, 0);
    }
    wave_sync();
    float ks[4] = {p.scale, p.scale, p.scale, p.scale}, vs[4] = {1.f, 1.f, 1.f, 1.f};
    if constexpr (kFp8) {  // broadcast within each 16-lane row
      ks[0] = dpp<0x150>(rscale);
      ks[1] = dpp<0x151>(rscale);
      ks[2] = dpp<0x152>(rscale);
      ks[3] = dpp<0x153>(rscale);
      vs[0] = dpp<0x154>(rscale);
      vs[1] = dpp<0x155>(rscale);
      vs[2] = dpp<0x156>(rscale);
      vs[3] = dpp<0x157>(rscale);
    }
    // Online softmax of head j over the block's 16 tokens.
    float sv[4], tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sv[i] = 4 * g + i < valid ? s[i] * ks[i] : -INFINITY;
      tmax = fmaxf(tmax, sv[i]);
    }
    tmax = group_max4(tmax);
    const float mn = fmaxf(m, tmax);
    const float alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - mn);
    float psum = 0.f;
    uint32_t phi[2], plo[2];
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
      const bool ok0 = 4 * g + i < valid, ok1 = 4 * g + i + 1 < valid;
      const float p0 = ok0 ? __builtin_amdgcn_exp2f(sv[i] - mn) : 0.f;
      const float p1 = ok1 ? __builtin_amdgcn_exp2f(sv[i + 1] - mn) : 0.f;
      psum += p0 + p1;
      // p * v_scale as a bf16 hi + bf16 lo pair by truncation: hi keeps the
      // top 8 significant bits, lo the next 8 of the exact remainder, so the
      // pair is within 2^-15 of the fp32 product.
      const float a0 = ok0 ? p0 * vs[i] : 0.f, a1 = ok1 ? p1 * vs[i + 1] : 0.f;
      const uint32_t h0 = __float_as_uint(a0) & 0xffff0000u, h1 = __float_as_uint(a1) & 0xffff0000u;
      const uint32_t l0 = __float_as_uint(a0 - __uint_as_float(h0)) & 0xffff0000u;
      const uint32_t l1 = __float_as_uint(a1 - __uint_as_float(h1)) & 0xffff0000u;
      phi[i / 2] = (h0 >> 16) | h1;
      plo[i / 2] = (l0 >> 16) | l1;
    }
    psum = group_sum4(psum);
    l = l * alpha + psum;
    m = mn;
    const bf16x8 pb = __builtin_bit_cast(bf16x8, u32x4{phi[0], phi[1], plo[0], plo[1]});
    // Rescale: the accumulators hold O^T, lane (g, j) = head j, so alpha is
    // in-lane; skipped when no head's maximum moved (the common case).
    if (__ballot(alpha != 1.f) != 0) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[nt][i] *= alpha;
    }
    // O^T += V^T P^T: A = value rows 4g..4g+3 at head dim 16nt + j, B = P^T as held.
    // Transposing LDS reads: lane (g, j) gets tokens 4g..4g+3 of head dim
    // 16nt + j. ds_read_b64_tr_b8 hands lane i of a 16-lane group byte e of
    // the row addressed by lane 2e + i/8 (at byte i%8); tr_b16 hands it
    // element e of the row addressed by lane 4e + i/4 (at element i%4).
    const unsigned char* vt;
    if constexpr (kFp8) vt = vt_w + (4 * g + ((j >> 1) & 3)) * PITCH + 8 * (j & 1);
    else vt = vt_w + (4 * g + (j >> 2)) * PITCH + 8 * (j & 3);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      u32x2 vw;
      if constexpr (kFp8) {
        typedef int i32x2 __attribute__((ext_vector_type(2)));
        const i32x2 t = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) i32x2*)(vt + 16 * nt));
        vw = e4m3x4_to_bf16x4_cvt((uint32_t)t[0]);
      } else {
        const s16x4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(vt + 32 * nt));
        vw = __builtin_bit_cast(u32x2, t);
      }
      // K = 32: the four tokens twice, against p_hi then p_lo.
      acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, u32x4{vw[0], vw[1], vw[0], vw[1]}),
                                                         pb, acc[nt], 0, 0, 0);
    }
    wave_sync();  // the next block rewrites the tile
  };

  // SETS register sets in rotation: while one block is computed, the next
  // SETS-1 are in flight.
  static_assert(SETS >= 2 && SETS <= 8, "2 to 8 register sets");
  BlockRegs<W, kFp8> r[SETS];
  auto prime = [&](int blk, BlockRegs<W, kFp8>& rr) {
    if (!load(blk, rr)) bad = true, blk1 = min(blk1, blk);
  };
  auto step = [&](int blk, BlockRegs<W, kFp8>& rr) {
    if (blk < blk1) compute(blk, rr);
    if (!load(blk + SETS, rr)) bad = true, blk1 = min(blk1, blk + SETS);
  };
#pragma unroll
  for (int i = 0; i < SETS; ++i) prime(blk0 + i, r[i]);
  if constexpr (kAppend) {
    // The wave whose split holds the sequence's last block writes the new
    // token there (while its first blocks are in flight). Lanes 0..RL-1 take
    // the key row, lanes 32..32+RL-1 the value row, 16 input bytes each, as
    // the page writer does with D/8 lanes per head.
    const int last = nblk - 1;
    if (seq > 0 && nblk <= p.max_blocks && last >= blk0 && last < blk0 + per_split) {
      const int32_t id = table[last];
      const uint32_t page = fast_div((uint32_t)max(id, 0), p.by_stride);
      if (id >= 0 && id <= p.id_max && page * p.by_stride.d == (uint32_t)id) {
        const int row = seq - 1 - kBlockTokens * last;
        const uint32_t seg = fast_div(page, p.by_seg_pages);
        char* krow = p.wbase[seg] + (uint64_t)(page - seg * p.by_seg_pages.d) * stride * p.half +
                     head_off + (uint64_t)row * token_stride;
        const bool is_v = lane >= 32;
        const int li = lane & 31;
        const bool act = li < RL;
        const uint16_t* src = (is_v ? p.new_v : p.new_k) + ((int64_t)b * p.kv_heads + kvh) * D + 8 * (act ? li : 0);
        const u32x4 x = act ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src)) : u32x4{0u, 0u, 0u, 0u};
        char* dst = krow + (is_v ? p.v_delta : 0);
        if constexpr (kFp8) {
          const float mx = group_max<RL>(amax8(x));
          const float inv = mx > 0.f ? 448.f / mx : 0.f;
          const float sc = mx > 0.f ? mx / 448.f : 1.f;
          const u32x2 c = quantise8(x, inv);
          if (act) *reinterpret_cast<u32x2*>(dst + 8 * li) = c;
          if (act && li == 0)
            p.wscales[(uint64_t)id * kBlockTokens * H +
                                         (2u * p.layer * kBlockTokens + row) * H + kvh + (is_v ? p.vscale_delta : 0)] = sc;
          nks = __shfl(sc, 0);
          nvs = __shfl(sc, 32);
#pragma unroll
          for (int i = 0; i < W; ++i) nk[i] = __shfl(c[i & 1], (64 * (i / 4) + 16 * g + 4 * (i % 4)) / 8);
          nv[0] = c[0];
          nv[1] = c[1];
        } else {
          if (act) *reinterpret_cast<u32x4*>(dst + 16 * li) = x;
#pragma unroll
          for (int i = 0; i < W; ++i) nk[i] = __shfl(x[i % 4], 4 * (i / 4) + g);
#pragma unroll
          for (int e = 0; e < 4; ++e) nv[e] = x[e];
        }
        patch_blk = last;
        slot_row = row;
      }
    }
  }
  for (int base = blk0; base < blk1; base += SETS) {
#pragma unroll
    for (int i = 0; i < SETS; ++i) step(base + i, r[i]);
  }

  // ---- this split's partials (lane (g, j): head j, dims 16nt + 4g + i)
  const int64_t row0 = (int64_t)b * p.q_heads + (int64_t)kvh * KVM;
  const float nan = __builtin_nanf("");
  if (j < KVM) {
    float* dst = p.part_acc + ((row0 + j) * p.splits + split) * D + 4 * g;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      *reinterpret_cast<f32x4*>(dst + 16 * nt) = bad ? f32x4{nan, nan, nan, nan} : acc[nt];
    if (g == 0) {
      p.part_m[(row0 + j) * p.splits + split] = bad ? nan : m;
      p.part_l[(row0 + j) * p.splits + split] = bad ? nan : l;
    }
  }
}

// Combines the splits as splitkv_paged_mha_fast_stage2_kernel does
// (paged_mha_fast_kernel.cu:730-799): M = max over splits of m_s,
// w_s = 2^(m_s - M) for splits with l_s > 0, out = sum_s w_s acc_s / sum_s w_s
// l_s, and NaN when any split met a bad block id. A row's D/4 float4 columns
// are shared by `groups` workgroups (gridDim.y), so a step with few rows and
// hundreds of splits (small batches, long sequences) still spreads over the
// GPU. In a workgroup, thread t is (split lane t / CPW, column t % CPW): it
// sums the splits s = lane, lane + LANES, ... of its column, and the lanes'
// sums meet in an LDS tree.
constexpr int kCombineThreads = 256;

template <int D>
__global__ __launch_bounds__(kCombineThreads) void decode_combine_kernel(const DecodeParams p) {
  constexpr int WAVES = kCombineThreads / 64;
  __shared__ float w_lds[kDecodeMaxSplits];
  __shared__ float red_m[WAVES], red_s[WAVES];
  __shared__ int red_nan[WAVES];
  __shared__ f32x4 part[kCombineThreads];
  const int t = threadIdx.x, wv = t >> 6, ln = t & 63;
  const int64_t row = blockIdx.x;
  const int cpw = (D / 4) / (int)gridDim.y;  // float4 columns of this workgroup
  const int lanes = kCombineThreads / cpw;
  const int S = p.splits;
  const float* m_row = p.part_m + row * S;
  const float* l_row = p.part_l + row * S;
  float mx = -INFINITY;
  int nan = 0;
  for (int s = t; s < S; s += kCombineThreads) {
    const float l = l_row[s];
    nan |= l != l;
    mx = fmaxf(mx, m_row[s]);
  }
  mx = wave_max(mx);
  const bool wave_nan = __ballot(nan) != 0;
  if (ln == 0) {
    red_m[wv] = mx;
    red_nan[wv] = wave_nan;
  }
  __syncthreads();
  float M = red_m[0];
  int any_nan = red_nan[0];
#pragma unroll
  for (int i = 1; i < WAVES; ++i) {
    M = fmaxf(M, red_m[i]);
    any_nan |= red_nan[i];
  }
  float den = 0.f;
  for (int s = t; s < S; s += kCombineThreads) {
    const float l = l_row[s];
    const float w = l > 0.f ? exp2f(m_row[s] - M) : 0.f;
    w_lds[s] = w;
    den += w > 0.f ? l * w : 0.f;
  }
  den = wave_sum(den);
  if (ln == 0) red_s[wv] = den;
  __syncthreads();
  den = red_s[0];
#pragma unroll
  for (int i = 1; i < WAVES; ++i) den += red_s[i];
  // Weighted sum: every split of the row wrote its partial (zeros for an
  // empty split, whose weight is 0), so the loads need no guard.
  const int col = (int)blockIdx.y * cpw + t % cpw, lane = t / cpw;
  const float* acc = p.part_acc + row * S * D + 4 * col;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int s = lane; s < S; s += lanes) {
    const float w = w_lds[s];
    const f32x4 x = *reinterpret_cast<const f32x4*>(acc + (int64_t)s * D);
    if (w > 0.f) o += x * w;
  }
  part[t] = o;
  __syncthreads();
  for (int stride = kCombineThreads / 2; stride >= cpw; stride >>= 1) {
    if (t < stride) part[t] += part[t + stride];
    __syncthreads();
  }
  if (t < cpw) {
    const f32x4 sum = part[t];
    uint16_t* dst = p.out + row * D + 4 * col;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v = any_nan ? __builtin_nanf("") : (den > 0.f ? sum[e] / den : 0.f);
      dst[e] = to_bf16(v);
    }
  }
}

// Workgroups per row for the combine: enough to give the GPU ~512
// workgroups when rows are few (a batch of 64 keeps one per row: splitting
// its 768 rows measured 4.5 against 4.2 us), at most one per float4 column.
int combine_groups(int64_t rows, int D) {
  int g = 1;
  while (g < D / 4 && rows * g < 512) g *= 2;
  return g;
}

// Register sets of one wave. BF16: two. FP8: two (one block in flight)
// while a split holds at most 48 blocks, four beyond. Both launches on
// MI355X, FP8, 2 KV heads x 6 query heads, 1 GiB scrub before each step,
// two sets against four: 64 x 5,040 tokens (16 splits, 20 blocks each)
// 39.2-39.5 against 41.2-41.3 us; 64 x 10,080 (40 blocks) 68.9 against
// 72.0; 128 x 5,040 (8 splits, 40 blocks) 68.8-69.2 against 68.0-71.5;
// 8 x 5,040 (5 blocks) 17.0 against 18.1; 1 x 32,768 (4 blocks) 18.4
// against 18.9; 64 x 20,160 (79 blocks) 123.2 against 120.7.
constexpr int kSetsLongSplit = 48;

template <int D, bool kFp8, int KVM, int kSets>
void launch_sets(const DecodeParams& p, hipStream_t stream, dim3 grid, dim3 block) {
  if (p.new_k)
    hipLaunchKernelGGL((paged_decode_kernel<D, kFp8, KVM, true, kSets>), grid, block, 0, stream, p, p.tables);
  else
    hipLaunchKernelGGL((paged_decode_kernel<D, kFp8, KVM, false, kSets>), grid, block, 0, stream, p, p.tables);
}

template <int D, bool kFp8, int KVM>
void launch(const DecodeParams& p, hipStream_t stream) {
  const int64_t units = (int64_t)p.batch * p.kv_heads * p.splits;
  const int64_t rows = (int64_t)p.batch * p.q_heads;
  const dim3 grid((unsigned)((units + kDecodeWaves - 1) / kDecodeWaves)), block(kDecodeWaves * 64);
  const int per_split = (p.max_blocks + p.splits - 1) / p.splits;
  if (kFp8 && per_split > kSetsLongSplit) launch_sets<D, kFp8, KVM, 4>(p, stream, grid, block);
  else launch_sets<D, kFp8, KVM, 2>(p, stream, grid, block);
  hipLaunchKernelGGL((decode_combine_kernel<D>), dim3((unsigned)rows, (unsigned)combine_groups(rows, D)),
                     dim3(kCombineThreads), 0, stream, p);
}

template <int D, bool kFp8>
bool launch_kvm(const DecodeParams& p, hipStream_t stream) {
  switch (p.q_heads / p.kv_heads) {
    case 1: launch<D, kFp8, 1>(p, stream); return true;
    case 2: launch<D, kFp8, 2>(p, stream); return true;
    case 3: launch<D, kFp8, 3>(p, stream); return true;
    case 4: launch<D, kFp8, 4>(p, stream); return true;
    case 5: launch<D, kFp8, 5>(p, stream); return true;
    case 6: launch<D, kFp8, 6>(p, stream); return true;
    case 7: launch<D, kFp8, 7>(p, stream); return true;
    case 8: launch<D, kFp8, 8>(p, stream); return true;
    default: return false;
  }
}

}  // namespace

FastDiv make_fast_div(uint32_t d) {
  FastDiv f;
  f.d = d ? d : 1;
  uint32_t s = 0;
  while ((1ull << s) < f.d) ++s;
  f.shift = s;
  f.mul = (uint32_t)(((1ull << 32) * ((1ull << s) - f.d)) / f.d + 1);
  return f;
}

uint64_t decode_workspace_bytes(int32_t batch, int32_t q_heads, int32_t head_dim, int32_t splits) {
  const uint64_t rows = (uint64_t)batch * q_heads * splits;
  return rows * head_dim * 4ull + 2ull * rows * 4ull;
}

hipError_t launch_paged_decode(const DecodeParams& p, bool fp8, hipStream_t stream) {
  bool ok = false;
  if (p.head_dim == 128) ok = fp8 ? launch_kvm<128, true>(p, stream) : launch_kvm<128, false>(p, stream);
  else if (p.head_dim == 64) ok = fp8 ? launch_kvm<64, true>(p, stream) : launch_kvm<64, false>(p, stream);
  if (!ok) return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace pbe
