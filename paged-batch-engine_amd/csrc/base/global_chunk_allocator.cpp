// Placement and release rules follow infMain/source/base/global_chunk_allocator.cpp:25-81.
#include "base/global_chunk_allocator.h"

#include <iterator>
#include <limits>

namespace base {
namespace {
const char* failure_name(ChunkAllocationFailure code) {
  switch (code) {
    case ChunkAllocationFailure::kQuota: return "model_kv_quota_exhausted";
    case ChunkAllocationFailure::kFragmented: return "arena_fragmented";
    default: return "arena_exhausted";
  }
}
}  // namespace

ChunkAllocationError::ChunkAllocationError(ChunkAllocationFailure code)
    : std::runtime_error(failure_name(code)), code_(code) {}

GlobalChunkAllocator::GlobalChunkAllocator(uint64_t bytes, uint64_t epoch)
    : bytes_(bytes), epoch_(epoch) {
  if (bytes == 0 || epoch == 0) throw std::invalid_argument("invalid arena size/epoch");
  free_.emplace(0, bytes);
}

void GlobalChunkAllocator::register_model(const std::string& model, uint64_t hard_limit) {
  if (model.empty() || hard_limit == 0 || hard_limit > bytes_ || quotas_.count(model))
    throw std::invalid_argument("invalid/duplicate model or KV hard limit");
  quotas_[model] = Quota{hard_limit, 0};
}

uint64_t GlobalChunkAllocator::leased_bytes(const std::string& model) const {
  return quotas_.at(model).used;
}

uint64_t GlobalChunkAllocator::free_bytes() const {
  uint64_t total = 0;
  for (const auto& range : free_) total += range.second;
  return total;
}

ChunkLease GlobalChunkAllocator::acquire(const std::string& model, const std::string& layout,
                                         uint64_t bytes, uint64_t alignment) {
  auto quota = quotas_.find(model);
  if (quota == quotas_.end() || layout.empty() || bytes == 0 || alignment == 0 ||
      bytes % alignment != 0)
    throw std::invalid_argument("invalid chunk request");
  if (bytes > quota->second.limit - quota->second.used)
    throw ChunkAllocationError(ChunkAllocationFailure::kQuota);

  // Best fit: the free range whose leftover after an aligned placement is
  // smallest; on equal leftover the lower offset (scanned first) wins.
  auto chosen = free_.end();
  uint64_t place_at = 0;
  uint64_t least_leftover = std::numeric_limits<uint64_t>::max();
  for (auto it = free_.begin(); it != free_.end(); ++it) {
    const uint64_t start = it->first, length = it->second;
    const uint64_t skip = (alignment - start % alignment) % alignment;
    if (skip > length || length - skip < bytes) continue;
    const uint64_t leftover = length - bytes;
    if (leftover < least_leftover) {
      least_leftover = leftover;
      chosen = it;
      place_at = start + skip;
    }
  }
  if (chosen == free_.end())
    throw ChunkAllocationError(free_bytes() >= bytes ? ChunkAllocationFailure::kFragmented
                                                     : ChunkAllocationFailure::kExhausted);

  const uint64_t range_start = chosen->first, range_end = chosen->first + chosen->second;
  free_.erase(chosen);
  if (place_at > range_start) free_.emplace(range_start, place_at - range_start);
  if (place_at + bytes < range_end) free_.emplace(place_at + bytes, range_end - place_at - bytes);

  ChunkLease lease;
  lease.epoch = epoch_;
  lease.id = next_generation_;
  lease.generation = next_generation_;
  lease.offset = place_at;
  lease.bytes = bytes;
  lease.model = model;
  lease.layout = layout;
  ++next_generation_;
  leases_.emplace(lease.id, lease);
  quota->second.used += bytes;
  return lease;
}

const ChunkLease& GlobalChunkAllocator::live_lease(const ChunkLease& lease) const {
  auto live = leases_.find(lease.id);
  if (lease.epoch != epoch_ || live == leases_.end())
    throw std::invalid_argument("stale_or_duplicate_chunk_release");
  const ChunkLease& held = live->second;
  if (held.generation != lease.generation || held.model != lease.model ||
      held.layout != lease.layout || held.offset != lease.offset || held.bytes != lease.bytes)
    throw std::invalid_argument("chunk_identity_mismatch");
  return held;
}

std::vector<ChunkLease> GlobalChunkAllocator::transfer(const std::vector<ChunkLease>& leases,
                                                       const std::string& to_model) {
  auto target = quotas_.find(to_model);
  if (target == quotas_.end()) throw std::invalid_argument("invalid chunk transfer target");
  uint64_t bytes = 0;
  std::unordered_map<uint64_t, int> seen;
  for (const ChunkLease& lease : leases) {
    const ChunkLease& held = live_lease(lease);
    if (held.model == to_model || seen[held.id]++) throw std::invalid_argument("invalid chunk transfer");
    bytes += held.bytes;
  }
  if (bytes > target->second.limit - target->second.used)
    throw ChunkAllocationError(ChunkAllocationFailure::kQuota);
  std::vector<ChunkLease> moved;
  moved.reserve(leases.size());
  for (const ChunkLease& lease : leases) {
    ChunkLease& held = leases_.at(lease.id);
    quotas_.at(held.model).used -= held.bytes;
    target->second.used += held.bytes;
    held.model = to_model;
    held.generation = next_generation_++;
    moved.push_back(held);
  }
  return moved;
}

void GlobalChunkAllocator::release(const ChunkLease& lease) {
  const ChunkLease& held = live_lease(lease);
  auto live = leases_.find(held.id);

  uint64_t start = held.offset, length = held.bytes;
  quotas_.at(held.model).used -= length;
  leases_.erase(live);

  // Merge with the free range ending at `start` and the one beginning at the end.
  auto after = free_.lower_bound(start);
  if (after != free_.begin()) {
    auto before = std::prev(after);
    if (before->first + before->second == start) {
      start = before->first;
      length += before->second;
      free_.erase(before);
    }
  }
  after = free_.lower_bound(start);
  if (after != free_.end() && after->first == start + length) {
    length += after->second;
    free_.erase(after);
  }
  free_.emplace(start, length);
}

}  // namespace base
