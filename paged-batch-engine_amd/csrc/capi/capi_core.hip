// C ABI, shared pieces: the calling thread's last error, host-side checks of
// shapes, views and pointers (so a bad pointer is rejected instead of
// faulting the GPU), version and device queries, streams.
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

#include "capi_internal.h"

namespace pbe_capi {
namespace {
thread_local std::string g_error;
}  // namespace

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(PBE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

const char* last_error() { return g_error.c_str(); }

bool shape_ok(const pbe_kv_shape* s) {
  return s && s->layers > 0 && s->kv_heads > 0 && s->head_dim > 0 && s->page_tokens > 0;
}

// half = one layer's K or V plane of one page (block_allocator.cpp:369-372).
uint64_t half_bytes(const pbe_kv_shape& s, uint32_t elem_bytes) {
  return (uint64_t)s.page_tokens * (uint64_t)s.kv_heads * (uint64_t)s.head_dim * elem_bytes;
}

bool view_ok(const pbe_arena_view* v) {
  if (!v || v->nseg == 0 || v->nseg > PBE_MAX_SEGMENTS || v->bytes == 0 || v->segment_bytes == 0)
    return false;
  if ((v->bytes + v->segment_bytes - 1) / v->segment_bytes != v->nseg) return false;
  for (uint32_t i = 0; i < v->nseg; ++i)
    if (!v->base[i]) return false;
  return true;
}

// Resolves [offset, offset+len) of a view to a device address; the span must
// lie inside one segment and inside the view.
bool resolve(const pbe_arena_view& v, uint64_t offset, uint64_t len, uint64_t* addr) {
  if (offset > v.bytes || len > v.bytes - offset) return false;
  const uint64_t seg = offset / v.segment_bytes;
  const uint64_t in_seg = offset % v.segment_bytes;
  if (seg >= v.nseg || len > v.segment_bytes - in_seg) return false;
  *addr = reinterpret_cast<uint64_t>(v.base[seg]) + in_seg;
  return true;
}

// Rejects any destination span overlapping another destination span or any
// source span (a copy must never race with itself).
bool spans_disjoint(std::vector<std::pair<uint64_t, uint64_t>> dst,
                    std::vector<std::pair<uint64_t, uint64_t>> src) {
  std::sort(dst.begin(), dst.end());
  for (size_t i = 1; i < dst.size(); ++i)
    if (dst[i].first < dst[i - 1].second) return false;
  std::sort(src.begin(), src.end());
  size_t j = 0;
  for (const auto& s : src) {
    while (j < dst.size() && dst[j].second <= s.first) ++j;
    if (j < dst.size() && dst[j].first < s.second) return false;
  }
  return true;
}

ArenaRegistry& arena_registry() {
  static ArenaRegistry r;
  return r;
}

bool accessible(const void* ptr, uint64_t bytes, int device, std::vector<Range>* known) {
  const uint64_t p = reinterpret_cast<uint64_t>(ptr);
  if (!p || bytes > ~0ull - p) return false;
  for (const Range& r : *known)
    if (p >= r.begin && p + bytes <= r.end) return true;
  {
    Range seg{};
    if (arena_registry().segment_of(p, bytes, device, &seg.begin, &seg.end)) {
      known->push_back(seg);  // later checks of this segment stay in `known`
      return true;
    }
  }
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, const_cast<void*>(ptr)) != hipSuccess || !base) {
    (void)hipGetLastError();
    return false;
  }
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, ptr) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  const bool ok_type = (attr.type == hipMemoryTypeDevice && attr.device == device) ||
                       attr.type == hipMemoryTypeHost;
  const Range r{reinterpret_cast<uint64_t>(base), reinterpret_cast<uint64_t>(base) + size};
  if (!ok_type || p < r.begin || p + bytes > r.end) return false;
  known->push_back(r);
  return true;
}

bool view_accessible(const pbe_arena_view& v, int device, std::vector<Range>* known) {
  for (uint32_t i = 0; i < v.nseg; ++i) {
    const uint64_t len = std::min(v.segment_bytes, v.bytes - (uint64_t)i * v.segment_bytes);
    if (!accessible(v.base[i], len, device, known)) return false;
  }
  return true;
}

}  // namespace pbe_capi

using namespace pbe_capi;

extern "C" {

const char* pbe_last_error(void) { return last_error(); }

const char* pbe_version(void) { return "pbe-handoff 1.0 gfx950"; }

int pbe_device_uuid(int device, uint8_t out[16]) {
  if (!out) return fail(PBE_ERR_INVALID, "null output");
  hipUUID uuid;
  PBE_HIP(hipDeviceGetUuid(&uuid, device));
  std::memcpy(out, uuid.bytes, 16);
  return PBE_OK;
}

}  // extern "C"

extern "C" {

// ---------------------------------------------------------------- streams
int pbe_stream_create(int device, void** out) {
  if (!out) return fail(PBE_ERR_INVALID, "null output");
  *out = nullptr;
  PBE_DEVICE_SCOPE(device);
  hipStream_t s = nullptr;
  PBE_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *out = s;
  return PBE_OK;
}

int pbe_stream_destroy(int device, void* stream) {
  if (!stream) return PBE_OK;
  PBE_DEVICE_SCOPE(device);
  PBE_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)));
  return PBE_OK;
}

int pbe_stream_synchronize(int device, void* stream) {
  PBE_DEVICE_SCOPE(device);
  const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(PBE_ERR_UNKNOWN, "hipStreamSynchronize: %s", hipGetErrorString(e));
  return PBE_OK;
}

int pbe_stream_wait_raw_event(int device, void* stream, void* hip_event) {
  if (!hip_event) return fail(PBE_ERR_INVALID, "null event");
  PBE_DEVICE_SCOPE(device);
  PBE_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(hip_event), 0));
  return PBE_OK;
}

int pbe_pointer_kind(const void* ptr, uint64_t bytes, int* kind, int* device_out) {
  if (!kind) return fail(PBE_ERR_INVALID, "null output");
  *kind = PBE_PTR_UNKNOWN;
  if (device_out) *device_out = -1;
  if (!ptr) return PBE_OK;
  const int arena_device = arena_registry().device_of(reinterpret_cast<uint64_t>(ptr), bytes);
  if (arena_device >= 0) {
    *kind = PBE_PTR_DEVICE;
    if (device_out) *device_out = arena_device;
    return PBE_OK;
  }
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, const_cast<void*>(ptr)) != hipSuccess || !base) {
    (void)hipGetLastError();
    return PBE_OK;
  }
  const uint64_t p = reinterpret_cast<uint64_t>(ptr), b = reinterpret_cast<uint64_t>(base);
  if (bytes > ~0ull - p || p + bytes > b + size) return PBE_OK;
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, ptr) != hipSuccess) {
    (void)hipGetLastError();
    return PBE_OK;
  }
  if (attr.type == hipMemoryTypeDevice) {
    *kind = PBE_PTR_DEVICE;
    if (device_out) *device_out = attr.device;
  } else if (attr.type == hipMemoryTypeHost) {
    *kind = PBE_PTR_PINNED_HOST;
  }
  return PBE_OK;
}

}  // extern "C"
