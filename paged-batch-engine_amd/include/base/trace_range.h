// Named host-time ranges for rocprofv3 --marker-trace (roctx), the MI355X
// counterpart of the NVTX range the reference puts around its handoff
// (split_pd_engine.cpp:51). The roctx library is looked up at run time
// (dlopen of librocprofiler-sdk-roctx.so.1, then libroctx64.so.4): a build or
// a host without it gets ranges that do nothing, and the library never links
// against it. PBE_NO_ROCTX=1 in the environment turns the ranges off.
#pragma once

namespace base {

class TraceRange {
 public:
  explicit TraceRange(const char* name);
  ~TraceRange();
  TraceRange(const TraceRange&) = delete;
  TraceRange& operator=(const TraceRange&) = delete;

  // True when a roctx library was found and ranges are recorded.
  static bool enabled();

 private:
  bool pushed_ = false;
};

}  // namespace base
