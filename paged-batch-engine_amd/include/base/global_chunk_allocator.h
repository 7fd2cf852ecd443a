// Owner-side metadata of the shared KV arena: leases byte ranges ("Chunks")
// to models with per-model hard limits. Drop-in for the reference's
// base::GlobalChunkAllocator (infMain/include/base/global_chunk_allocator.h:9-44):
// same types, error codes/messages and placement (best fit by least leftover,
// lowest offset on ties; released ranges coalesce with their neighbours).
// CPU metadata only; the owner serializes every call.
#ifndef PBE_INCLUDE_BASE_GLOBAL_CHUNK_ALLOCATOR_H_
#define PBE_INCLUDE_BASE_GLOBAL_CHUNK_ALLOCATOR_H_

#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace base {

enum class ChunkAllocationFailure { kQuota = 1, kFragmented = 2, kExhausted = 3 };

class ChunkAllocationError : public std::runtime_error {
 public:
  explicit ChunkAllocationError(ChunkAllocationFailure code);
  ChunkAllocationFailure code() const { return code_; }

 private:
  ChunkAllocationFailure code_;
};

struct ChunkLease {
  uint64_t epoch = 0, id = 0, generation = 0;
  uint64_t offset = 0, bytes = 0;
  std::string model, layout;
};

class GlobalChunkAllocator {
 public:
  // Throws std::invalid_argument for a zero size or epoch.
  GlobalChunkAllocator(uint64_t bytes, uint64_t epoch);
  // Throws std::invalid_argument for an empty/duplicate model or a limit of 0
  // or above the arena size.
  void register_model(const std::string& model, uint64_t hard_limit);
  // Throws std::invalid_argument for an unknown model, empty layout, zero
  // size/alignment or bytes % alignment != 0; ChunkAllocationError kQuota
  // when the model's limit would be exceeded, kFragmented when enough bytes
  // are free but no aligned range fits, kExhausted otherwise. A failed call
  // changes nothing.
  ChunkLease acquire(const std::string& model, const std::string& layout, uint64_t bytes,
                     uint64_t alignment);
  // Throws std::invalid_argument("stale_or_duplicate_chunk_release") for a
  // foreign epoch or unknown id and ("chunk_identity_mismatch") when any other
  // field differs from the live lease.
  void release(const ChunkLease& lease);
  // Zero-copy page takeover (no counterpart in the reference, whose decode
  // side always copies, docs/single-gpu-2p1d-2026-10-12.md:34): re-attributes
  // the live Chunks `leases` (as their holder sees them) to `to_model`, all or
  // nothing. Same identity checks as release(); std::invalid_argument for an
  // unknown target model, a Chunk listed twice or one already held by
  // `to_model`; ChunkAllocationError kQuota when the target's limit cannot take
  // their bytes. Returns the new leases (same id, offset, bytes and layout, a
  // fresh generation, model = to_model): the old identities become stale.
  std::vector<ChunkLease> transfer(const std::vector<ChunkLease>& leases, const std::string& to_model);
  uint64_t free_bytes() const;
  uint64_t leased_bytes(const std::string& model) const;
  uint64_t epoch() const { return epoch_; }
  uint64_t bytes() const { return bytes_; }
  size_t lease_count() const { return leases_.size(); }

 private:
  struct Quota {
    uint64_t limit = 0;
    uint64_t used = 0;
  };
  const ChunkLease& live_lease(const ChunkLease& lease) const;  // identity checks of release()
  uint64_t bytes_, epoch_, next_generation_ = 1;
  std::map<uint64_t, uint64_t> free_;  // offset -> length, disjoint, never adjacent
  std::unordered_map<uint64_t, ChunkLease> leases_;
  std::unordered_map<std::string, Quota> quotas_;
};

}  // namespace base

#endif  // PBE_INCLUDE_BASE_GLOBAL_CHUNK_ALLOCATOR_H_
