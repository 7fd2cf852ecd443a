// TEST INFRASTRUCTURE ONLY. A C-callable scenario driver over the
// GlobalChunkAllocator API (global_chunk_allocator.h:27-44). It is compiled
// twice: against the reference sources (oracle/_ref/libpbe_ref.so) and against
// this repository's drop-in implementation (tests), so both run the exact same
// operation sequence and their outcome logs can be compared entry by entry.
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "base/global_chunk_allocator.h"

namespace {
enum : int64_t {
  kOk = 0,
  kStaleOrDuplicate = 10,
  kIdentityMismatch = 11,
  kInvalidArgument = 12,
  kRuntimeError = 13,
};

int64_t classify_invalid(const std::invalid_argument& e) {
  const std::string what = e.what();
  if (what == "stale_or_duplicate_chunk_release") return kStaleOrDuplicate;
  if (what == "chunk_identity_mismatch") return kIdentityMismatch;
  return kInvalidArgument;
}
}  // namespace

extern "C" {

// Runs n_ops operations on a fresh allocator and writes 4 int64 per op to out:
//   [code, offset, generation, free_bytes]
// op kind 0: acquire(model[op_model], "layout" + op_layout, op_bytes, op_align)
// op kind 1: release(live[op_index]) and drop it from the live list
// op kind 2: release a copy of live[op_index] with field op_align mutated
//            (0 epoch,1 generation,2 offset,3 bytes,4 model,5 layout,6 id)
// op kind 3: release(live[op_index]) without dropping it (duplicate release)
// Then leased_bytes(model m) for every model is appended (n_models int64).
// Returns 0, or -1 if the scenario itself is malformed.
int ref_alloc_run(uint64_t arena_bytes, uint64_t epoch, int32_t n_models, const uint64_t* limits,
                  int32_t n_ops, const int32_t* op_kind, const int32_t* op_model,
                  const int32_t* op_layout, const uint64_t* op_bytes, const uint64_t* op_align,
                  const int32_t* op_index, int64_t* out, int64_t* model_bytes_out) {
  try {
    base::GlobalChunkAllocator pool(arena_bytes, epoch);
    for (int32_t m = 0; m < n_models; ++m) pool.register_model("M" + std::to_string(m), limits[m]);
    std::vector<base::ChunkLease> live;
    for (int32_t i = 0; i < n_ops; ++i) {
      int64_t* o = out + 4 * i;
      o[0] = kOk;
      o[1] = o[2] = -1;
      try {
        if (op_kind[i] == 0) {
          auto lease = pool.acquire("M" + std::to_string(op_model[i]),
                                    "layout" + std::to_string(op_layout[i]), op_bytes[i], op_align[i]);
          o[1] = (int64_t)lease.offset;
          o[2] = (int64_t)lease.generation;
          live.push_back(lease);
        } else {
          if (live.empty()) return -1;
          const size_t idx = (size_t)op_index[i] % live.size();
          base::ChunkLease lease = live[idx];
          if (op_kind[i] == 2) {
            switch (op_align[i]) {
              case 0: ++lease.epoch; break;
              case 1: ++lease.generation; break;
              case 2: ++lease.offset; break;
              case 3: ++lease.bytes; break;
              case 4: lease.model = "other"; break;
              case 5: lease.layout = "wrong"; break;
              default: ++lease.id; break;
            }
          }
          o[1] = (int64_t)lease.offset;
          pool.release(lease);
          if (op_kind[i] == 1) live.erase(live.begin() + (long)idx);
        }
      } catch (const base::ChunkAllocationError& e) {
        o[0] = static_cast<int64_t>(e.code());
      } catch (const std::invalid_argument& e) {
        o[0] = classify_invalid(e);
      } catch (const std::runtime_error&) {
        o[0] = kRuntimeError;
      }
      o[3] = (int64_t)pool.free_bytes();
    }
    for (int32_t m = 0; m < n_models; ++m)
      model_bytes_out[m] = (int64_t)pool.leased_bytes("M" + std::to_string(m));
    return 0;
  } catch (...) {
    return -1;
  }
}

}  // extern "C"
