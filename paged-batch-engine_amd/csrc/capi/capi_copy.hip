// C ABI: device run lists and their launches, the one-call handoff
// (pbe_copy_shared_kv) and generic op lists (pbe_copy_ops).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "base/trace_range.h"
#include "capi_internal.h"

using namespace pbe_capi;

// ---------------------------------------------------------------- run lists
namespace {

struct Resolved {
  std::vector<pbe::DevRun> runs;
  pbe_runlist_info info{};
  // The first run's source when linear slices were asked for, the sources
  // form one region in run order, every run holds whole linear slices and
  // the list fits the kernel's one-region search (the copy kernel then reads
  // slice s at linear_src + s * linear_slice without looking the run up
  // first; slices are counted in linear_slice); else 0.
  uint64_t linear_src = 0;
  // With linear_src: the runs' first slices as a compact array, which the
  // kernel's one-region search probes (4 bytes per run instead of one
  // 32-byte record per probe). Device images place it after the records.
  std::vector<uint32_t> starts;

  size_t image_bytes() const { return runs.size() * sizeof(pbe::DevRun) + starts.size() * 4; }
  void image(void* dst) const {
    std::memcpy(dst, runs.data(), runs.size() * sizeof(pbe::DevRun));
    if (!starts.empty())
      std::memcpy(static_cast<char*>(dst) + runs.size() * sizeof(pbe::DevRun), starts.data(),
                  starts.size() * 4);
  }
  const uint32_t* starts_in(const void* dev_image) const {
    return starts.empty() ? nullptr
                          : reinterpret_cast<const uint32_t*>(static_cast<const char*>(dev_image) +
                                                              runs.size() * sizeof(pbe::DevRun));
  }
};

// Builds device run entries for either kernel. src pages are src_page_bytes
// long in the src view, dst pages dst_page_bytes long in the dst view;
// scale pages (FP8) scale_page_bytes long at scales. Slices are `slice`
// source bytes, or `linear_slice` when the one-region path applies (0: the
// kernel has no such path).
int resolve_runs(const pbe_arena_view& src, const pbe_arena_view& dst, uint64_t src_half,
                 uint64_t dst_half, int32_t stride, const pbe_run* runs, int64_t n_runs,
                 uint64_t scales, uint64_t scales_bytes, uint64_t scale_page_bytes,
                 uint32_t slice, uint32_t linear_slice, Resolved* out) {
  if (n_runs <= 0 || n_runs > 0x7fffffff) return fail(PBE_ERR_INVALID, "run count out of range");
  const uint64_t src_page = (uint64_t)stride * src_half;
  const uint64_t dst_page = (uint64_t)stride * dst_half;
  std::vector<std::pair<uint64_t, uint64_t>> dst_spans, src_spans;
  out->runs.resize((size_t)n_runs);
  uint64_t slices = 0;
  for (int64_t i = 0; i < n_runs; ++i) {
    const pbe_run& r = runs[i];
    if (r.src_block < 0 || r.dst_block < 0 || r.pages <= 0 || r.src_block % stride ||
        r.dst_block % stride)
      return fail(PBE_ERR_INVALID, "run %lld: ids must be non-negative page ids, pages > 0",
                  (long long)i);
    pbe::DevRun d{};
    const uint64_t sb = (uint64_t)r.pages * src_page, db = (uint64_t)r.pages * dst_page;
    if (!resolve(src, (uint64_t)r.src_block * src_half, sb, &d.src))
      return fail(PBE_ERR_INVALID, "run %lld: source span outside one arena segment", (long long)i);
    if (!resolve(dst, (uint64_t)r.dst_block * dst_half, db, &d.dst))
      return fail(PBE_ERR_INVALID, "run %lld: destination span outside one arena segment",
                  (long long)i);
    if (scale_page_bytes) {
      const uint64_t off = (uint64_t)(r.dst_block / stride) * scale_page_bytes;
      const uint64_t len = (uint64_t)r.pages * scale_page_bytes;
      if (off > scales_bytes || len > scales_bytes - off)
        return fail(PBE_ERR_INVALID, "run %lld: scale span outside the scale pool", (long long)i);
      d.aux = scales + off;
      dst_spans.emplace_back(d.aux, d.aux + len);
    }
    d.pages = (uint32_t)r.pages;
    d.slice_begin = (uint32_t)slices;
    slices += (sb + slice - 1) / slice;
    if (slices > 0xfffffff0ull) return fail(PBE_ERR_INVALID, "run list too large for one launch");
    src_spans.emplace_back(d.src, d.src + sb);
    dst_spans.emplace_back(d.dst, d.dst + db);
    out->info.src_bytes += sb;
    out->info.dst_bytes += db;
    out->info.pages += r.pages;
    if (scale_page_bytes) out->info.scale_bytes += (uint64_t)r.pages * scale_page_bytes;
    out->runs[(size_t)i] = d;
  }
  if (!spans_disjoint(dst_spans, src_spans))
    return fail(PBE_ERR_INVALID, "run list writes a byte twice or overwrites its own source");
  out->info.runs = n_runs;
  bool linear = linear_slice && src_page % linear_slice == 0 && (uint64_t)n_runs <= pbe::kLinearMaxRuns;
  for (size_t i = 1; linear && i < src_spans.size(); ++i)
    linear = src_spans[i].first == src_spans[i - 1].second;
  if (linear) {  // recount in linear slices (whole ones: src_page is a multiple)
    slices = 0;
    for (pbe::DevRun& d : out->runs) {
      d.slice_begin = (uint32_t)slices;
      slices += (uint64_t)d.pages * (src_page / linear_slice);
      if (slices > 0xfffffff0ull) return fail(PBE_ERR_INVALID, "run list too large for one launch");
    }
  }
  if (!linear) {
    // The general path takes its runs in destination address order, the
    // slices renumbered in that order. MI355X, config 3 (kernel-bracketing
    // events, means of three alternating runs, two boxes): 113.9-114.0
    // against 114.9-115.2 us in the caller's order (114.6 in source order);
    // config 5 596.7-597.9 against 597.4-598.3 us. The one-region path keeps
    // source order, which its slice-to-source mapping needs.
    std::sort(out->runs.begin(), out->runs.end(),
              [](const pbe::DevRun& a, const pbe::DevRun& b) { return a.dst < b.dst; });
    slices = 0;
    for (pbe::DevRun& d : out->runs) {
      d.slice_begin = (uint32_t)slices;
      slices += ((uint64_t)d.pages * src_page + slice - 1) / slice;
    }
  }
  out->info.slices = slices;
  out->linear_src = linear ? out->runs.front().src : 0;
  out->starts.clear();
  if (linear)
    for (const pbe::DevRun& d : out->runs) out->starts.push_back(d.slice_begin);
  return PBE_OK;
}

int upload_runlist(Resolved& res, int device, bool fp8, bool has_scales, uint64_t page_bytes,
                   const pbe_kv_shape& kv, pbe_runlist** out) {
  PBE_DEVICE_SCOPE(device);
  pbe_runlist* list = new (std::nothrow) pbe_runlist;
  if (!list) return fail(PBE_ERR_NOMEM, "run list object");
  const size_t bytes = res.image_bytes();
  std::vector<char> image(bytes);
  res.image(image.data());
  hipError_t e = hipMalloc(&list->runs, bytes);
  if (e == hipSuccess) e = hipMemcpy(list->runs, image.data(), bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    if (list->runs) (void)hipFree(list->runs);
    delete list;
    return hip_fail(e, "upload run list");
  }
  list->device = device;
  list->fp8 = fp8;
  list->has_scales = has_scales;
  list->n_runs = (uint32_t)res.runs.size();
  list->total_slices = (uint32_t)res.info.slices;
  list->page_bytes = page_bytes;
  list->linear_src = res.linear_src;
  list->starts = res.starts_in(list->runs);
  list->info = res.info;
  list->kv = kv;
  *out = list;
  return PBE_OK;
}

}  // namespace

extern "C" {

int pbe_runlist_create(const pbe_arena_view* src, const pbe_arena_view* dst, const pbe_run* runs,
                       int64_t n_runs, const pbe_kv_shape* shape, uint32_t elem_bytes, int device,
                       pbe_runlist** out) {
  if (!out) return fail(PBE_ERR_INVALID, "null output");
  *out = nullptr;
  if (!view_ok(src) || !view_ok(dst) || !runs || !shape_ok(shape) || !elem_bytes)
    return fail(PBE_ERR_INVALID, "invalid arena view, run list or shape");
  const uint64_t half = half_bytes(*shape, elem_bytes);
  if (half % 16) return fail(PBE_ERR_INVALID, "half-plane bytes must be a multiple of 16");
  {
    PBE_DEVICE_SCOPE(device);
    std::vector<Range> known;
    if (!view_accessible(*src, device, &known) || !view_accessible(*dst, device, &known))
      return fail(PBE_ERR_INVALID, "arena view is not device memory of device %d", device);
  }
  Resolved res;
  int rc = resolve_runs(*src, *dst, half, half, 2 * shape->layers, runs, n_runs, 0, 0, 0,
                        pbe::kCopySliceBytes, pbe::kLinearSliceBytes, &res);
  if (rc != PBE_OK) return rc;
  return upload_runlist(res, device, false, false, 2ull * shape->layers * half, *shape, out);
}

int pbe_runlist_create_fp8(const pbe_arena_view* src, const pbe_arena_view* dst, void* dst_scales,
                           uint64_t dst_scales_bytes, const pbe_run* runs, int64_t n_runs,
                           const pbe_kv_shape* shape, int device, pbe_runlist** out) {
  if (!out) return fail(PBE_ERR_INVALID, "null output");
  *out = nullptr;
  if (!view_ok(src) || !view_ok(dst) || !runs || !shape_ok(shape))
    return fail(PBE_ERR_INVALID, "invalid arena view, run list or shape");
  const uint32_t lanes = (uint32_t)shape->head_dim / 8u;
  if (shape->head_dim % 8 || lanes == 0 || lanes > 64 || (lanes & (lanes - 1)))
    return fail(PBE_ERR_UNSUPPORTED, "FP8 handoff needs head_dim = 8 * 2^k <= 512");
  const uint64_t half16 = half_bytes(*shape, 2), half8 = half_bytes(*shape, 1);
  const uint64_t rows = (uint64_t)shape->page_tokens * shape->kv_heads;
  const uint64_t scale_page = dst_scales ? 2ull * shape->layers * rows * 4u : 0;
  if (dst_scales && (reinterpret_cast<uint64_t>(dst_scales) % 4))
    return fail(PBE_ERR_INVALID, "scale pool must be 4-byte aligned");
  if (half16 % 16) return fail(PBE_ERR_INVALID, "half-plane bytes must be a multiple of 16");
  {
    PBE_DEVICE_SCOPE(device);
    std::vector<Range> known;
    if (!view_accessible(*src, device, &known) || !view_accessible(*dst, device, &known) ||
        (dst_scales && !accessible(dst_scales, dst_scales_bytes, device, &known)))
      return fail(PBE_ERR_INVALID, "arena view or scale pool is not memory of device %d", device);
  }
  Resolved res;
  int rc = resolve_runs(*src, *dst, half16, half8, 2 * shape->layers, runs, n_runs,
                        reinterpret_cast<uint64_t>(dst_scales), dst_scales_bytes, scale_page,
                        pbe::kFp8SliceBytes, pbe::kFp8LinearSliceBytes, &res);
  if (rc != PBE_OK) return rc;
  return upload_runlist(res, device, true, dst_scales != nullptr, 2ull * shape->layers * half16,
                        *shape, out);
}

int pbe_runlist_get_info(const pbe_runlist* list, pbe_runlist_info* out) {
  if (!list || !out) return fail(PBE_ERR_INVALID, "null argument");
  *out = list->info;
  return PBE_OK;
}

int pbe_runlist_destroy(pbe_runlist* list) {
  if (!list) return PBE_OK;
  PBE_DEVICE_SCOPE(list->device);
  const hipError_t e = hipFree(list->runs);
  delete list;
  if (e != hipSuccess) return hip_fail(e, "hipFree(run list)");
  return PBE_OK;
}

int pbe_handoff_copy_timed(const pbe_runlist* list, void* stream, void* start_event,
                           void* stop_event) {
  if (!list) return fail(PBE_ERR_INVALID, "null run list");
  if (list->fp8) return fail(PBE_ERR_INVALID, "FP8 run list passed to the BF16 copy");
  PBE_DEVICE_SCOPE(list->device);
  const pbe::LaunchEvents ev{static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event)};
  PBE_HIP(pbe::launch_copy_runs(list->runs, list->starts, list->n_runs, list->total_slices,
                                list->page_bytes, list->linear_src, ev,
                                static_cast<hipStream_t>(stream)));
  return PBE_OK;
}

int pbe_handoff_copy(const pbe_runlist* list, void* stream) {
  return pbe_handoff_copy_timed(list, stream, nullptr, nullptr);
}

int pbe_handoff_copy_fp8(const pbe_runlist* list, int scale_mode, const float* amax_table,
                         void* stream) {
  return pbe_handoff_copy_fp8_timed(list, scale_mode, amax_table, stream, nullptr, nullptr);
}

int pbe_handoff_copy_fp8_timed(const pbe_runlist* list, int scale_mode, const float* amax_table,
                               void* stream, void* start_event, void* stop_event) {
  if (!list) return fail(PBE_ERR_INVALID, "null run list");
  if (!list->fp8) return fail(PBE_ERR_INVALID, "BF16 run list passed to the FP8 copy");
  if (scale_mode == PBE_FP8_SCALE_PER_TOKEN_HEAD && !list->has_scales)
    return fail(PBE_ERR_INVALID, "per-token-head scales need a scale pool");
  if (scale_mode == PBE_FP8_SCALE_TABLE && !amax_table)
    return fail(PBE_ERR_INVALID, "table mode needs an amax table");
  if (scale_mode != PBE_FP8_SCALE_PER_TOKEN_HEAD && scale_mode != PBE_FP8_SCALE_TABLE)
    return fail(PBE_ERR_INVALID, "unknown scale mode %d", scale_mode);
  PBE_DEVICE_SCOPE(list->device);
  const pbe_kv_shape& kv = list->kv;
  const uint32_t rows_per_plane = (uint32_t)(kv.page_tokens * kv.kv_heads);
  const pbe::LaunchEvents ev{static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event)};
  PBE_HIP(pbe::launch_copy_runs_fp8(
      list->runs, list->starts, list->n_runs, list->total_slices, list->page_bytes,
      (uint32_t)kv.head_dim / 8u,
      rows_per_plane, (uint32_t)kv.kv_heads, rows_per_plane * 2u * (uint32_t)kv.layers,
      scale_mode == PBE_FP8_SCALE_TABLE, amax_table, list->linear_src, ev,
      static_cast<hipStream_t>(stream)));
  return PBE_OK;
}

}  // extern "C"

// ---------------------------------------------------------------- one-call forms
namespace {

// Per-device ring of pinned staging + device buffers for the one-call entry
// points. A slot is reused only after the launch that read it has completed,
// so back-to-back calls block the host only when the whole ring is in flight.
constexpr int kStagingSlots = 4;

struct StagingSlot {
  void* host = nullptr;
  void* dev = nullptr;
  size_t cap = 0;
  hipEvent_t done = nullptr;
  bool pending = false;
};

struct Staging {
  std::mutex mu;
  StagingSlot slots[kStagingSlots];
  int next = 0;
};

Staging& staging_for(int device) {
  static Staging per_device[64];
  return per_device[device & 63];
}

// Copies `bytes` of `data` into the next ring slot's device buffer, ordered on
// `stream`, and returns the slot. Caller holds st.mu and calls stage_done()
// after the launch that reads the buffer.
int stage(Staging& st, const void* data, size_t bytes, hipStream_t stream, StagingSlot** slot_out,
          void** dev_out) {
  StagingSlot& sl = st.slots[st.next];
  st.next = (st.next + 1) % kStagingSlots;
  if (sl.pending) {
    PBE_HIP(hipEventSynchronize(sl.done));
    sl.pending = false;
  }
  if (bytes > sl.cap) {
    if (sl.host) (void)hipHostFree(sl.host);
    if (sl.dev) (void)hipFree(sl.dev);
    sl.host = sl.dev = nullptr;
    sl.cap = 0;
    size_t cap = 4096;
    while (cap < bytes) cap *= 2;
    PBE_HIP(hipHostMalloc(&sl.host, cap, hipHostMallocDefault));
    PBE_HIP(hipMalloc(&sl.dev, cap));
    sl.cap = cap;
  }
  if (!sl.done) PBE_HIP(hipEventCreateWithFlags(&sl.done, hipEventDisableTiming));
  std::memcpy(sl.host, data, bytes);
  PBE_HIP(hipMemcpyAsync(sl.dev, sl.host, bytes, hipMemcpyHostToDevice, stream));
  *slot_out = &sl;
  *dev_out = sl.dev;
  return PBE_OK;
}

// The staging ring reuses its buffers after four calls: a graph captured with
// a staged list would replay stale or freed memory, so staged calls refuse a
// stream that is being captured (prebuilt run lists are the capturable form).
int refuse_capture(hipStream_t stream, const char* what) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  PBE_HIP(hipStreamIsCapturing(stream, &status));
  if (status != hipStreamCaptureStatusNone)
    return fail(PBE_ERR_UNSUPPORTED,
                "%s stages its list per call and cannot be captured into a graph; capture "
                "pbe_handoff_copy with a prebuilt run list instead", what);
  return PBE_OK;
}

int stage_done(StagingSlot& sl, hipStream_t stream) {
  PBE_HIP(hipEventRecord(sl.done, stream));
  sl.pending = true;
  return PBE_OK;
}

}  // namespace

extern "C" {

int pbe_copy_shared_kv(const pbe_arena_view* arena, const int32_t* src_ids, const int32_t* dst_ids,
                       int64_t n, const pbe_kv_shape* shape, int device, void* stream,
                       uint64_t* copied) {
  const base::TraceRange trace("pbe_copy_shared_kv");
  if (copied) *copied = 0;
  if (!view_ok(arena) || !shape_ok(shape) || n <= 0 || !src_ids || !dst_ids || device < 0)
    return fail(PBE_ERR_INVALID, "invalid handoff arguments");
  int64_t bad = -1;
  int rc = pbe_validate_ids(src_ids, n, shape, 2, arena->bytes, &bad);
  if (rc != PBE_OK) return rc;
  rc = pbe_validate_ids(dst_ids, n, shape, 2, arena->bytes, &bad);
  if (rc != PBE_OK) return rc;
  std::vector<pbe_run> runs((size_t)n);
  int64_t n_runs = 0;
  rc = pbe_build_runs(src_ids, dst_ids, n, shape, 2, arena->nseg > 1 ? arena->segment_bytes : 0,
                      runs.data(), &n_runs);
  if (rc != PBE_OK) return rc;
  const uint64_t half = half_bytes(*shape, 2);
  if (half % 16) return fail(PBE_ERR_INVALID, "half-plane bytes must be a multiple of 16");
  {
    PBE_DEVICE_SCOPE(device);
    std::vector<Range> known;
    if (!view_accessible(*arena, device, &known))
      return fail(PBE_ERR_INVALID, "arena view is not device memory of device %d", device);
  }
  Resolved res;
  rc = resolve_runs(*arena, *arena, half, half, 2 * shape->layers, runs.data(), n_runs, 0, 0, 0,
                    pbe::kCopySliceBytes, pbe::kLinearSliceBytes, &res);
  if (rc != PBE_OK) return rc;
  PBE_DEVICE_SCOPE(device);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (res.linear_src && (uint64_t)n_runs <= pbe::kKernargLinearRuns) {
    // A one-region plan rides in the kernel arguments as run starts and
    // destinations (up to 256 runs): no staging copy, no fence.
    pbe::KernargLinearList list{};
    list.n_runs = (uint32_t)n_runs;
    list.total_slices = (uint32_t)res.info.slices;
    list.linear_src = res.linear_src;
    std::fill(std::begin(list.starts), std::end(list.starts), 0xffffffffu);
    for (size_t i = 0; i < res.runs.size(); ++i) {
      list.starts[i] = res.runs[i].slice_begin;
      list.dst[i] = res.runs[i].dst;
    }
    PBE_HIP(pbe::launch_copy_runs_kernarg_linear(list, s));
    if (copied) *copied = res.info.src_bytes;
    return PBE_OK;
  }
  if ((uint64_t)n_runs <= pbe::kKernargRuns) {
    // Short lists ride in the kernel arguments: no staging copy, no fence.
    pbe::KernargRunList list{};
    list.n_runs = (uint32_t)n_runs;
    list.total_slices = (uint32_t)res.info.slices;
    list.page_bytes = 2ull * shape->layers * half;
    list.linear_src = res.linear_src;
    std::memcpy(list.runs, res.runs.data(), res.runs.size() * sizeof(pbe::DevRun));
    PBE_HIP(pbe::launch_copy_runs_kernarg(list, s));
    if (copied) *copied = res.info.src_bytes;
    return PBE_OK;
  }
  rc = refuse_capture(s, "pbe_copy_shared_kv with a run list longer than the kernel arguments hold");
  if (rc != PBE_OK) return rc;
  Staging& st = staging_for(device);
  std::lock_guard<std::mutex> lock(st.mu);
  void* dev = nullptr;
  StagingSlot* slot = nullptr;
  std::vector<char> image(res.image_bytes());
  res.image(image.data());
  rc = stage(st, image.data(), image.size(), s, &slot, &dev);
  if (rc != PBE_OK) return rc;
  PBE_HIP(pbe::launch_copy_runs(static_cast<const pbe::DevRun*>(dev), res.starts_in(dev),
                                (uint32_t)n_runs, (uint32_t)res.info.slices,
                                2ull * shape->layers * half, res.linear_src, pbe::LaunchEvents{}, s));
  rc = stage_done(*slot, s);
  if (rc != PBE_OK) return rc;
  if (copied) *copied = res.info.src_bytes;
  return PBE_OK;
}

int pbe_copy_ops(const pbe_copy_op* ops, int64_t n_ops, int device, void* stream) {
  if (n_ops < 0 || (n_ops && !ops) || n_ops > 0x7fffffff)
    return fail(PBE_ERR_INVALID, "invalid op list");
  if (!n_ops) return PBE_OK;
  PBE_DEVICE_SCOPE(device);
  // Every op's endpoints are checked as given; then ops that continue the
  // previous one on both sides (the 2L component copies of one page, and
  // consecutive pages of a run, in a bound manifest) are merged, so the
  // overlap check, the staging and the kernel see runs instead of planes.
  std::vector<pbe_copy_op> merged;
  merged.reserve(64);
  {
    std::vector<Range> known;
    // The allocations last found to hold a source and a destination: most ops
    // of a bound manifest fall inside them, and the full check (which asks
    // the runtime once per allocation) runs only for the others.
    Range last_src{1, 0}, last_dst{1, 0};
    auto inside = [](const Range& r, uint64_t p, uint64_t n) { return p >= r.begin && p + n <= r.end; };
    auto check = [&](uint64_t p, uint64_t n, Range* last) {
      if (inside(*last, p, n)) return true;
      if (!accessible(reinterpret_cast<const void*>(p), n, device, &known)) return false;
      for (const Range& r : known)
        if (inside(r, p, n)) *last = r;
      return true;
    };
    for (int64_t i = 0; i < n_ops; ++i) {
      const pbe_copy_op& o = ops[i];
      if (!o.src || !o.dst || !o.bytes)
        return fail(PBE_ERR_INVALID, "op %lld: null pointer or zero bytes", (long long)i);
      if (o.bytes > ~0ull - o.src || o.bytes > ~0ull - o.dst)
        return fail(PBE_ERR_INVALID, "op %lld: span wraps the address space", (long long)i);
      if (!check(o.src, o.bytes, &last_src) || !check(o.dst, o.bytes, &last_dst))
        return fail(PBE_ERR_INVALID, "op %lld: endpoint is not device or pinned memory", (long long)i);
      if (!merged.empty()) {
        pbe_copy_op& last = merged.back();
        if (last.src + last.bytes == o.src && last.dst + last.bytes == o.dst) {
          last.bytes += o.bytes;
          continue;
        }
      }
      merged.push_back(o);
    }
  }
  {
    std::vector<std::pair<uint64_t, uint64_t>> dst, src;
    dst.reserve(merged.size());
    src.reserve(merged.size());
    for (const pbe_copy_op& o : merged) {
      dst.emplace_back(o.dst, o.dst + o.bytes);
      src.emplace_back(o.src, o.src + o.bytes);
    }
    if (!spans_disjoint(dst, src))
      return fail(PBE_ERR_INVALID, "op list writes a byte twice or overwrites its own source");
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // Spans whose addresses and sizes are all 16-byte multiples are runs of
  // 16-byte pages for the run kernel: 2 KiB per wave, one launch, and up to
  // kKernargRuns spans in the kernel arguments (no staging, so capturable).
  const bool aligned = std::all_of(merged.begin(), merged.end(), [](const pbe_copy_op& o) {
    return ((o.src | o.dst | o.bytes) & 15u) == 0 && o.bytes / 16 <= 0xffffffffull;
  });
  if (aligned) {
    std::vector<pbe::DevRun> runs(merged.size());
    uint64_t slices = 0;
    for (size_t i = 0; i < merged.size(); ++i) {
      const pbe_copy_op& o = merged[i];
      runs[i] = pbe::DevRun{o.src, o.dst, 0, (uint32_t)slices, (uint32_t)(o.bytes / 16)};
      slices += (o.bytes + pbe::kCopySliceBytes - 1) / pbe::kCopySliceBytes;
      if (slices > 0xfffffff0ull) return fail(PBE_ERR_INVALID, "op list too large for one launch");
    }
    if (runs.size() <= pbe::kKernargRuns) {
      pbe::KernargRunList list{};
      list.n_runs = (uint32_t)runs.size();
      list.total_slices = (uint32_t)slices;
      list.page_bytes = 16;
      std::memcpy(list.runs, runs.data(), runs.size() * sizeof(pbe::DevRun));
      PBE_HIP(pbe::launch_copy_runs_kernarg(list, s));
      return PBE_OK;
    }
    int rc = refuse_capture(s, "pbe_copy_ops with more than 112 spans");
    if (rc != PBE_OK) return rc;
    Staging& st = staging_for(device);
    std::lock_guard<std::mutex> lock(st.mu);
    void* dev = nullptr;
    StagingSlot* slot = nullptr;
    rc = stage(st, runs.data(), runs.size() * sizeof(pbe::DevRun), s, &slot, &dev);
    if (rc != PBE_OK) return rc;
    PBE_HIP(pbe::launch_copy_runs(static_cast<const pbe::DevRun*>(dev), nullptr,
                                  (uint32_t)runs.size(), (uint32_t)slices, 16, 0,
                                  pbe::LaunchEvents{}, s));
    return stage_done(*slot, s);
  }
  // Otherwise: split ops so that every wave moves at most kOpPieceBytes.
  std::vector<pbe::DevOp> pieces;
  for (const pbe_copy_op& o : merged)
    for (uint64_t off = 0; off < o.bytes; off += pbe::kOpPieceBytes)
      pieces.push_back({o.src + off, o.dst + off, std::min<uint64_t>(pbe::kOpPieceBytes, o.bytes - off)});
  if (pieces.size() > 0xffffffffull) return fail(PBE_ERR_INVALID, "op list too large");
  int rc = refuse_capture(s, "pbe_copy_ops with unaligned spans");
  if (rc != PBE_OK) return rc;
  Staging& st = staging_for(device);
  std::lock_guard<std::mutex> lock(st.mu);
  void* dev = nullptr;
  StagingSlot* slot = nullptr;
  rc = stage(st, pieces.data(), pieces.size() * sizeof(pbe::DevOp), s, &slot, &dev);
  if (rc != PBE_OK) return rc;
  PBE_HIP(pbe::launch_copy_ops(static_cast<const pbe::DevOp*>(dev), (uint32_t)pieces.size(), s));
  return stage_done(*slot, s);
}

}  // extern "C"
