// roctx ranges through a run-time lookup (see base/trace_range.h).
#include "base/trace_range.h"

#include <dlfcn.h>

#include <cstdlib>
#include <cstring>
#include <initializer_list>

namespace base {
namespace {

struct Roctx {
  int (*push)(const char*) = nullptr;
  int (*pop)() = nullptr;
  Roctx() {
    const char* off = std::getenv("PBE_NO_ROCTX");
    if (off && std::strcmp(off, "0") != 0) return;
    for (const char* name : {"librocprofiler-sdk-roctx.so.1", "libroctx64.so.4"}) {
      void* h = dlopen(name, RTLD_NOW | RTLD_LOCAL);
      if (!h) continue;
      auto push_fn = reinterpret_cast<int (*)(const char*)>(dlsym(h, "roctxRangePushA"));
      auto pop_fn = reinterpret_cast<int (*)()>(dlsym(h, "roctxRangePop"));
      if (push_fn && pop_fn) {
        push = push_fn;
        pop = pop_fn;
        return;  // the handle stays open for the life of the process
      }
      dlclose(h);
    }
  }
};

const Roctx& roctx() {
  static const Roctx r;  // looked up once, thread-safe
  return r;
}

}  // namespace

TraceRange::TraceRange(const char* name) {
  const Roctx& r = roctx();
  if (r.push) pushed_ = r.push(name) >= 0;
}

TraceRange::~TraceRange() {
  if (pushed_) roctx().pop();
}

bool TraceRange::enabled() { return roctx().push != nullptr; }

}  // namespace base
