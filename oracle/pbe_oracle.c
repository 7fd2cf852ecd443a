/*
 * TEST INFRASTRUCTURE ONLY: CPU restatement of PagedBatchEngine's
 * prefill->decode KV handoff. It is the checker for the HIP path and the CPU
 * baseline in bench.py. Nothing in the product library links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root).
 *
 * Pinning (how each function is checked independently of this file):
 *   orc_coalesce            brute-force maximality/concatenation property and the
 *                           hand-derived run lists in tests/golden/handoff_runs.json
 *   orc_copy_runs/_handoff  closed form (identity on every copied page, canary
 *                           bytes untouched) and the page-major probe pattern of
 *                           demo/shared_kv_reuse_probe.cpp:76-83
 *   orc_copy_components     must agree byte-for-byte with orc_copy_runs (two
 *                           different decompositions of the same copy)
 *   orc_bf16_from_f32       torch's float32->bfloat16 cast (round-to-nearest-even)
 *   orc_e4m3_from_f32       OCP FP8 v1.0 E4M3 value table (nearest value, ties to
 *                           even code, saturate-to-finite) checked against
 *                           torch.float8_e4m3fn for |x| <= 448, and the
 *                           hand-worked vectors in tests/golden/e4m3_cases.json
 *   orc_fp8_*               per-row reduction checked against a numpy restatement
 *                           on small pools; FP8 rounding parity against CUDA's
 *                           __nv_cvt_float_to_fp8 is pinned by the OCP spec only.
 *   orc_scatter_kv          plain form: pages it writes, read back by the pinned
 *                           paged-decode oracle, give the attention torch computes
 *                           on the unpaged K/V; FP8 form: byte-identical to the
 *                           pinned FP8 handoff of the plain pages it would write
 *                           (same rows, same per-(token, head) rule); FP32 input
 *                           checked element-wise against numpy x*inv + E4M3.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ---- run coalescing: infMain/source/serving/split_pd_engine.cpp:96-101 ----
 * Extend a run while both the source and destination block id advance by one
 * page (2*layers half-planes). Returns the number of runs written. */
int64_t orc_coalesce(const int32_t* src, const int32_t* dst, int64_t n,
                     int32_t page_stride, int32_t* run_src, int32_t* run_dst,
                     int32_t* run_pages) {
  int64_t runs = 0;
  for (int64_t i = 0; i < n;) {
    int64_t end = i + 1;
    while (end < n && src[end] == src[end - 1] + page_stride &&
           dst[end] == dst[end - 1] + page_stride)
      ++end;
    run_src[runs] = src[i];
    run_dst[runs] = dst[i];
    run_pages[runs] = (int32_t)(end - i);
    ++runs;
    i = end;
  }
  return runs;
}

/* ---- copy one coalesced run per memcpy: split_pd_engine.cpp:102-108 ----
 * dst.key/src.key are the layer-0 K plane addresses arena + id*half
 * (block_allocator.cpp:382-389 with key_base(0) = arena, shared_kv_arena.cpp:224);
 * bytes = run_pages * page_bytes with page_bytes = 2*layers*half. */
uint64_t orc_copy_runs(uint8_t* arena, const int32_t* run_src,
                       const int32_t* run_dst, const int32_t* run_pages,
                       int64_t n_runs, uint64_t half, int32_t layers) {
  const uint64_t page_bytes = 2ull * (uint64_t)layers * half;
  uint64_t copied = 0;
  for (int64_t r = 0; r < n_runs; ++r) {
    const uint64_t bytes = (uint64_t)run_pages[r] * page_bytes;
    memcpy(arena + (uint64_t)run_dst[r] * half, arena + (uint64_t)run_src[r] * half,
           bytes);
    copied += bytes;
  }
  return copied;
}

/* Whole data effect of copy_shared_kv (split_pd_engine.cpp:94-109): coalesce,
 * then one memcpy per run. Scratch arrays hold n entries each. */
uint64_t orc_copy_handoff(uint8_t* arena, const int32_t* src, const int32_t* dst,
                          int64_t n, uint64_t half, int32_t layers,
                          int32_t* scratch_src, int32_t* scratch_dst,
                          int32_t* scratch_pages) {
  const int64_t runs = orc_coalesce(src, dst, n, 2 * layers, scratch_src,
                                    scratch_dst, scratch_pages);
  return orc_copy_runs(arena, scratch_src, scratch_dst, scratch_pages, runs, half,
                       layers);
}

/* ---- generic plan form: pd_handoff.cpp:192-213 over transfer_plan.cpp:392-403 ----
 * One memcpy of `half` bytes per (page, layer, K|V) component. The K plane of
 * layer l of block id b sits at arena + (2l)*half + b*half and the V plane at
 * arena + (2l+1)*half + b*half (shared_kv_arena.cpp:224-229). */
uint64_t orc_copy_components(uint8_t* arena, const int32_t* src, const int32_t* dst,
                             int64_t n, uint64_t half, int32_t layers) {
  uint64_t copied = 0;
  for (int64_t p = 0; p < n; ++p)
    for (int32_t l = 0; l < layers; ++l)
      for (int32_t plane = 0; plane < 2; ++plane) {
        const uint64_t base = (2ull * (uint64_t)l + (uint64_t)plane) * half;
        memcpy(arena + base + (uint64_t)dst[p] * half,
               arena + base + (uint64_t)src[p] * half, half);
        copied += half;
      }
  return copied;
}

/* ---- source id validation: split_pd_engine.cpp:70-77 ----
 * Returns the index of the first id the reference rejects, or -1. */
int64_t orc_validate_ids(const int32_t* ids, int64_t n, int32_t layers, uint64_t half,
                         uint64_t arena_bytes) {
  for (int64_t i = 0; i < n; ++i) {
    const int32_t id = ids[i];
    if (id < 0 || ((uint64_t)id + 2ull * (uint64_t)layers) * half > arena_bytes ||
        id % (2 * layers) != 0)
      return i;
  }
  return -1;
}

/* ---- BF16: infMain/include/base/bf16.h:14-28 ---- */
uint16_t orc_bf16_from_f32(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof(bits));
  const uint32_t lsb = (bits >> 16) & 1u;
  bits += 0x7fffu + lsb;
  return (uint16_t)(bits >> 16);
}

float orc_f32_from_bf16(uint16_t value) {
  const uint32_t bits = (uint32_t)value << 16;
  float out;
  memcpy(&out, &bits, sizeof(out));
  return out;
}

void orc_bf16_from_f32_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_from_f32(in[i]);
}

/* ---- FP8 E4M3 per the OCP 8-bit Floating Point Specification v1.0 ----
 * Codes 0x00-0x7E are the finite non-negative values: exponent field e = c>>3
 * (bias 7), mantissa m = c&7; e == 0 is subnormal m*2^-9, otherwise
 * (1+m/8)*2^(e-7). 0x7F is NaN; there is no infinity. This is the conversion
 * the reference requests with __nv_cvt_float_to_fp8(v, __NV_SATFINITE,
 * __NV_E4M3) (scatter_kv_kernel.cu:207-210): round to nearest, ties to even,
 * magnitudes beyond 448 saturate to 448. */
static double e4m3_value(int code) {
  const int e = (code >> 3) & 15, m = code & 7;
  if (e == 0) return ldexp((double)m, -9);
  return ldexp(1.0 + m / 8.0, e - 7);
}

float orc_e4m3_to_f32(uint8_t code) {
  if ((code & 0x7f) == 0x7f) return NAN;
  const double v = e4m3_value(code & 0x7f);
  return (float)((code & 0x80) ? -v : v);
}

uint8_t orc_e4m3_from_f32(float x) {
  static double table[127];
  static int ready = 0;
  if (!ready) {
    for (int c = 0; c < 127; ++c) table[c] = e4m3_value(c);
    ready = 1;
  }
  if (isnan(x)) return 0x7f;
  const uint8_t sign = signbit(x) ? 0x80 : 0x00;
  const double a = fabs((double)x);
  if (a >= 448.0) return sign | 0x7e; /* SATFINITE */
  /* largest code with table[c] <= a (table is strictly increasing) */
  int lo = 0, hi = 126;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (table[mid] <= a) lo = mid; else hi = mid - 1;
  }
  int code = lo;
  if (code < 126) {
    const double below = a - table[code], above = table[code + 1] - a;
    if (above < below || (above == below && (code & 1))) code += 1;
  }
  return sign | (uint8_t)code;
}

void orc_e4m3_from_f32_array(const float* in, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_e4m3_from_f32(in[i]);
}

/* ---- fused BF16 -> FP8 handoff, per-(token, kv head) scales ----
 * Per row of head_dim elements: scatter_kv_kernel.cu:166-211.
 *   amax = max |x|;  scale = amax>0 ? amax/448 : 1;  inv = amax>0 ? 448/amax : 0
 *   q = e4m3(inv>0 ? x*inv : 0)   (fp32 multiply, no contraction)
 * Scale layout follows the reference pool [block][token*heads + head]
 * (scatter_kv_kernel.cu:188-190), one plane per (layer, K|V) of the page, so a
 * scale page is [layer][K|V][token][head] fp32.
 * Source: BF16 page-major arena, half16 = T*H*D*2 bytes, ids = offset/half16.
 * Destination: FP8 page-major arena, half8 = T*H*D bytes, ids = offset/half8;
 * scale page of dst id d is at scales + (d / (2L)) * (2L*T*H*4). */
/* One row of d_count values: amax, scale = amax/448 (1 for amax 0),
 * inv = 448/amax (0 for amax 0), q = E4M3(x * inv) (scatter_kv_kernel.cu:166-211).
 * fmaxf drops NaN inputs from the amax, as the reference's reduction does. */
static void fp8_row_f32(const float* x, uint8_t* q, int32_t d_count, float inv_given,
                        int use_given, float* scale_out) {
  float amax = 0.f;
  float inv;
  if (use_given) {
    inv = inv_given;
  } else {
    for (int32_t d = 0; d < d_count; ++d) amax = fmaxf(amax, fabsf(x[d]));
    *scale_out = amax > 0.f ? amax / 448.f : 1.f;
    inv = amax > 0.f ? 448.f / amax : 0.f;
  }
  for (int32_t d = 0; d < d_count; ++d) {
    volatile float v = inv > 0.f ? x[d] * inv : 0.f;
    q[d] = orc_e4m3_from_f32(v);
  }
}

static void fp8_row(const uint16_t* x, uint8_t* q, int32_t d_count, float inv_given,
                    int use_given, float* scale_out) {
  float row[1024];
  for (int32_t d = 0; d < d_count; ++d) row[d] = orc_f32_from_bf16(x[d]);
  fp8_row_f32(row, q, d_count, inv_given, use_given, scale_out);
}

void orc_fp8_handoff_token_head(const uint8_t* src_arena, uint8_t* dst_arena,
                                uint8_t* dst_scales, const int32_t* src_ids,
                                const int32_t* dst_ids, int64_t n, int32_t layers,
                                int32_t tokens, int32_t heads, int32_t head_dim) {
  const uint64_t rows = (uint64_t)tokens * (uint64_t)heads;
  const uint64_t half16 = rows * (uint64_t)head_dim * 2u;
  const uint64_t half8 = rows * (uint64_t)head_dim;
  const uint64_t scale_page = 2ull * (uint64_t)layers * rows * 4u;
  for (int64_t p = 0; p < n; ++p) {
    const uint8_t* s = src_arena + (uint64_t)src_ids[p] * half16;
    uint8_t* d = dst_arena + (uint64_t)dst_ids[p] * half8;
    float* sc = (float*)(dst_scales + (uint64_t)(dst_ids[p] / (2 * layers)) * scale_page);
    for (uint64_t plane = 0; plane < 2ull * (uint64_t)layers; ++plane)
      for (uint64_t r = 0; r < rows; ++r) {
        const uint64_t row = plane * rows + r;
        float scale;
        fp8_row((const uint16_t*)(s + row * head_dim * 2u), d + row * head_dim, head_dim,
                0.f, 0, &scale);
        sc[row] = scale;
      }
  }
}

/* ---- fused BF16 -> FP8 handoff, static per-(layer, K|V, kv head) scales ----
 * amax_table[(2l+kv)*H + h] holds the seeded amax; scale = amax/448 and
 * inv = 448/amax with the same guards as the per-row form. No scales are
 * written: the table itself is the scale state. */
void orc_fp8_handoff_table(const uint8_t* src_arena, uint8_t* dst_arena,
                           const float* amax_table, const int32_t* src_ids,
                           const int32_t* dst_ids, int64_t n, int32_t layers,
                           int32_t tokens, int32_t heads, int32_t head_dim) {
  const uint64_t rows = (uint64_t)tokens * (uint64_t)heads;
  const uint64_t half16 = rows * (uint64_t)head_dim * 2u;
  const uint64_t half8 = rows * (uint64_t)head_dim;
  for (int64_t p = 0; p < n; ++p) {
    const uint8_t* s = src_arena + (uint64_t)src_ids[p] * half16;
    uint8_t* d = dst_arena + (uint64_t)dst_ids[p] * half8;
    for (uint64_t plane = 0; plane < 2ull * (uint64_t)layers; ++plane)
      for (uint64_t t = 0; t < (uint64_t)tokens; ++t)
        for (uint64_t h = 0; h < (uint64_t)heads; ++h) {
          const float amax = amax_table[plane * (uint64_t)heads + h];
          const float inv = amax > 0.f ? 448.f / amax : 0.f;
          const uint64_t row = plane * rows + t * (uint64_t)heads + h;
          fp8_row((const uint16_t*)(s + row * head_dim * 2u), d + row * head_dim, head_dim,
                  inv, 1, 0);
        }
  }
}

/* scale = amax/448 (or 1) for each table entry, as the decode side reads it. */
void orc_fp8_table_scales(const float* amax_table, float* scales, int64_t n) {
  for (int64_t i = 0; i < n; ++i) scales[i] = amax_table[i] > 0.f ? amax_table[i] / 448.f : 1.f;
}

/* ---- page writer: scatter_kv_kernel.cu:99-127 (plain), :128-216 (FP8) ----
 * keys/values: n rows of kv_dim = heads*head_dim elements, BF16 (in_f32 = 0)
 * or FP32 (in_f32 = 1). Row t goes to slot s = slots[t], block s/B and offset
 * s%B. Plain pools hold the input type, head h of the row at
 *   pool + ((s/B)*B*kv_dim + (s%B)*kv_dim + h*head_dim) * E;
 * FP8 pools hold E4M3 bytes (E = 1) and the (token, head) scale at
 * scales[((s/B)*B + s%B)*heads + h]. A negative slot, a row that would end
 * beyond its pool, or (FP8) a head whose scale would fall beyond its scale
 * pool, is skipped; the reference skips negative slots in its FP8 form
 * (:147-149) and does not check bounds. */
void orc_scatter_kv(const uint8_t* keys, const uint8_t* values, int32_t in_f32, int64_t n,
                    const int32_t* slots, int32_t block_size, int32_t heads, int32_t head_dim,
                    int32_t fp8, uint8_t* key_pool, uint64_t key_pool_bytes, uint8_t* value_pool,
                    uint64_t value_pool_bytes, float* key_scales, uint64_t key_scale_count,
                    float* value_scales, uint64_t value_scale_count) {
  const uint64_t kv_dim = (uint64_t)heads * (uint64_t)head_dim;
  const uint64_t e_in = in_f32 ? 4u : 2u, e_out = fp8 ? 1u : e_in;
  float row[1024];
  for (int64_t t = 0; t < n; ++t) {
    const int32_t s = slots[t];
    if (s < 0) continue;
    const uint64_t block = (uint64_t)s / (uint64_t)block_size, off = (uint64_t)s % (uint64_t)block_size;
    const uint64_t out_row = (block * (uint64_t)block_size + off) * kv_dim * e_out;
    for (int kv = 0; kv < 2; ++kv) {
      const uint8_t* in = (kv ? values : keys) + (uint64_t)t * kv_dim * e_in;
      uint8_t* pool = kv ? value_pool : key_pool;
      if (out_row + kv_dim * e_out > (kv ? value_pool_bytes : key_pool_bytes)) continue;
      if (!fp8) {
        memcpy(pool + out_row, in, kv_dim * e_in);
        continue;
      }
      float* scales = kv ? value_scales : key_scales;
      for (int32_t h = 0; h < heads; ++h) {
        const uint64_t idx = (block * (uint64_t)block_size + off) * (uint64_t)heads + (uint64_t)h;
        if (idx >= (kv ? value_scale_count : key_scale_count)) continue;
        for (int32_t d = 0; d < head_dim; ++d) {
          const uint64_t i = (uint64_t)h * (uint64_t)head_dim + (uint64_t)d;
          if (in_f32) memcpy(&row[d], in + i * 4u, 4);
          else {
            uint16_t b;
            memcpy(&b, in + i * 2u, 2);
            row[d] = orc_f32_from_bf16(b);
          }
        }
        fp8_row_f32(row, pool + out_row + (uint64_t)h * (uint64_t)head_dim, head_dim, 0.f, 0,
                    &scales[idx]);
      }
    }
  }
}
