// Internal interface shared by the translation units of the C ABI: the
// calling thread's error message, device scoping, host-side pointer and view
// checks, and the definitions of the ABI's opaque handle types.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <utility>
#include <vector>

#include "../kernels/handoff_kernels.h"
#include "pbe_handoff.h"

namespace pbe_capi {

// Records a message for pbe_last_error() and returns `code`.
int fail(int code, const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);
const char* last_error();

// Makes `device` current for the scope and restores the caller's device.
class DeviceScope {
 public:
  explicit DeviceScope(int device) {
    if (hipGetDevice(&old_) != hipSuccess) {
      err_ = hipErrorNoDevice;
      return;
    }
    if (old_ == device) return;  // already current: nothing to switch or restore
    err_ = hipSetDevice(device);
    switched_ = err_ == hipSuccess;
  }
  ~DeviceScope() {
    if (switched_) (void)hipSetDevice(old_);
  }
  hipError_t error() const { return err_; }

 private:
  int old_ = 0;
  bool switched_ = false;
  hipError_t err_ = hipSuccess;
};

bool shape_ok(const pbe_kv_shape* s);
// half = one layer's K or V plane of one page (block_allocator.cpp:369-372).
uint64_t half_bytes(const pbe_kv_shape& s, uint32_t elem_bytes);
bool view_ok(const pbe_arena_view* v);
// Resolves [offset, offset+len) of a view to a device address; the span must
// lie inside one segment and inside the view.
bool resolve(const pbe_arena_view& v, uint64_t offset, uint64_t len, uint64_t* addr);
// Rejects any destination span overlapping another destination span or any
// source span (a copy must never race with itself).
bool spans_disjoint(std::vector<std::pair<uint64_t, uint64_t>> dst,
                    std::vector<std::pair<uint64_t, uint64_t>> src);

// Checks on the host that [ptr, ptr+bytes) lies inside one allocation a kernel
// on `device` may touch (device memory of that GPU, or pinned host memory), so
// a bad pointer is rejected instead of faulting the GPU. Verified allocation
// ranges are remembered in `known` for the rest of the call.
struct Range {
  uint64_t begin, end;
};

// Segments of arenas this library created or imported over IPC, per device.
// IPC mappings are device memory but need not be visible to the runtime's
// allocation-range queries, so they are recognised here first.
struct ArenaRegistry {
  std::mutex mu;
  struct Entry {
    uint64_t begin, end;
    int device;
  };
  std::vector<Entry> entries;
  void add(const void* p, uint64_t bytes, int device) {
    std::lock_guard<std::mutex> lock(mu);
    entries.push_back({reinterpret_cast<uint64_t>(p), reinterpret_cast<uint64_t>(p) + bytes, device});
  }
  void remove(const void* p) {
    std::lock_guard<std::mutex> lock(mu);
    const uint64_t b = reinterpret_cast<uint64_t>(p);
    entries.erase(std::remove_if(entries.begin(), entries.end(),
                                 [b](const Entry& e) { return e.begin == b; }),
                  entries.end());
  }
  bool contains(uint64_t p, uint64_t bytes, int device) { return device_of(p, bytes) == device; }
  // The registered segment of `device` holding [p, p+bytes), if any.
  bool segment_of(uint64_t p, uint64_t bytes, int device, uint64_t* begin, uint64_t* end) {
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& e : entries)
      if (p >= e.begin && bytes <= e.end - p && p < e.end && e.device == device) {
        *begin = e.begin;
        *end = e.end;
        return true;
      }
    return false;
  }
  // Device of the registered segment holding [p, p+bytes), or -1.
  int device_of(uint64_t p, uint64_t bytes) {
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& e : entries)
      if (p >= e.begin && bytes <= e.end - p && p < e.end) return e.device;
    return -1;
  }
};
ArenaRegistry& arena_registry();

bool accessible(const void* ptr, uint64_t bytes, int device, std::vector<Range>* known);
bool view_accessible(const pbe_arena_view& v, int device, std::vector<Range>* known);

}  // namespace pbe_capi

#define PBE_HIP(call)                                        \
  do {                                                       \
    const hipError_t pbe_e_ = (call);                        \
    if (pbe_e_ != hipSuccess) return pbe_capi::hip_fail(pbe_e_, #call); \
  } while (0)

#define PBE_DEVICE_SCOPE(dev)                                          \
  pbe_capi::DeviceScope pbe_scope_(dev);                                         \
  if (pbe_scope_.error() != hipSuccess) return pbe_capi::hip_fail(pbe_scope_.error(), "select device")

struct pbe_arena {
  int device = 0;
  bool owner = false;
  uint64_t bytes = 0, segment_bytes = 0, epoch = 0;
  uint32_t nseg = 0;
  void* base[PBE_MAX_SEGMENTS] = {};
  uint8_t uuid[16] = {};
};

struct pbe_event {
  int device = 0;
  bool imported = false;
  bool interprocess = false;
  hipEvent_t event = nullptr;
};

struct pbe_signal {
  int device = 0;
  bool imported = false;
  void* word = nullptr;  // 8-byte sequence value at the start of a 4 KiB allocation
};

struct pbe_runlist {
  int device = 0;
  bool fp8 = false;
  bool has_scales = false;
  pbe::DevRun* runs = nullptr;  // device memory
  uint32_t n_runs = 0;
  uint32_t total_slices = 0;
  uint64_t page_bytes = 0;      // source bytes per page
  uint64_t linear_src = 0;      // see pbe::launch_copy_runs
  const uint32_t* starts = nullptr;  // with linear_src: the runs' first slices, inside `runs`
  pbe_runlist_info info{};
  pbe_kv_shape kv{};
};
