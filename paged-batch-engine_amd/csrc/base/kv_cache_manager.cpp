// Request page tables over per-layer block allocators. Semantics follow
// infMain/source/base/kv_cache_manager.cpp:167-244,639-760 and the growth rule
// of sequence_kv_manager.cpp:204-290 (new blocks per layer =
// ceil((n+k)/B) - ceil(n/B), allocated layer by layer, rolled back as a whole).
#include "base/kv_cache_manager.h"

#include <algorithm>
#include <climits>
#include <stdexcept>
#include <string>

namespace base {
namespace {
constexpr uint32_t kSlotBits = 20;
constexpr uint64_t kSlotMask = (uint64_t{1} << kSlotBits) - 1;
constexpr uint64_t kMaxReuse = (uint64_t{1} << (63 - kSlotBits)) - 1;

int32_t blocks_for(int32_t tokens, int32_t block_size) {
  return tokens <= 0 ? 0 : static_cast<int32_t>((static_cast<int64_t>(tokens) + block_size - 1) / block_size);
}
}  // namespace

KVCacheManager::KVCacheManager(int32_t block_size, int32_t num_layers,
                               std::vector<std::unique_ptr<BlockAllocator>> layer_allocators)
    : block_size_(block_size), num_layers_(num_layers), layers_(std::move(layer_allocators)) {
  if (block_size_ <= 0 || num_layers_ <= 0)
    throw std::invalid_argument("KV cache manager needs positive block size and layer count");
  if (static_cast<int32_t>(layers_.size()) != num_layers_)
    throw std::invalid_argument("KV cache manager needs one allocator per layer");
  for (const auto& a : layers_)
    if (!a || a->block_size() != block_size_)
      throw std::invalid_argument("KV cache manager allocator block size mismatch");
}

RequestId KVCacheManager::register_request() {
  uint32_t slot;
  if (!idle_slots_.empty()) {
    slot = idle_slots_.back();
    idle_slots_.pop_back();
    ++requests_[slot].reuse;
  } else {
    if (requests_.size() > kSlotMask) throw std::runtime_error("request slot capacity exhausted");
    slot = static_cast<uint32_t>(requests_.size());
    requests_.emplace_back();
  }
  Request& r = requests_[slot];
  r.live = true;
  r.tokens = 0;
  r.committed = 0;
  r.blocks.assign(num_layers_, {});
  ++active_;
  return static_cast<RequestId>((r.reuse << kSlotBits) | slot);
}

bool KVCacheManager::is_valid_request(RequestId id) const {
  if (id < 0) return false;
  const uint64_t slot = static_cast<uint64_t>(id) & kSlotMask;
  if (slot >= requests_.size()) return false;
  const Request& r = requests_[slot];
  return r.live && r.reuse == (static_cast<uint64_t>(id) >> kSlotBits);
}

KVCacheManager::Request& KVCacheManager::live_request(RequestId id) {
  if (!is_valid_request(id)) throw std::invalid_argument("unknown or released request id " + std::to_string(id));
  return requests_[static_cast<uint64_t>(id) & kSlotMask];
}

const KVCacheManager::Request& KVCacheManager::live_request(RequestId id) const {
  if (!is_valid_request(id)) throw std::invalid_argument("unknown or released request id " + std::to_string(id));
  return requests_[static_cast<uint64_t>(id) & kSlotMask];
}

void KVCacheManager::check_layer(int32_t layer_idx) const {
  if (layer_idx < 0 || layer_idx >= num_layers_) throw std::out_of_range("layer index out of range");
}

void KVCacheManager::free_request(RequestId id) {
  Request& r = live_request(id);
  // Later layers first: for a shared page group, layer 0's release is the one
  // that fences the page once every other layer has let go of it.
  for (int32_t l = num_layers_; l-- > 0;) layers_[l]->free_many(r.blocks[l]);
  r.blocks.assign(num_layers_, {});
  r.tokens = r.committed = 0;
  r.live = false;
  const uint32_t slot = static_cast<uint32_t>(static_cast<uint64_t>(id) & kSlotMask);
  if (r.reuse < kMaxReuse) idle_slots_.push_back(slot);  // an exhausted slot is never reused
  --active_;
}

bool KVCacheManager::append_slots(RequestId id, int32_t num_tokens) {
  Request& r = live_request(id);
  if (num_tokens <= 0 || num_tokens > INT32_MAX - r.tokens - (block_size_ - 1)) return false;
  const int32_t need = blocks_for(r.tokens + num_tokens, block_size_) - blocks_for(r.tokens, block_size_);
  if (need > 0) {
    for (int32_t l = 0; l < num_layers_; ++l)
      if (layers_[l]->num_free_blocks() < need) return false;
    // Appended in place; on failure (a false return or an exception) every
    // layer's new blocks are freed and the tables cut back to where they were
    // (all or nothing).
    const size_t had = r.blocks[0].size();
    int32_t l = 0;
    // best_effort: on the exception path a block the failed call left
    // half-registered may refuse its free; the cut-back goes on and the
    // original exception is the one reported.
    auto cut_back = [&](bool best_effort) {
      for (int32_t m = std::min(l, num_layers_ - 1); m >= 0; --m) {
        for (size_t k = had; k < r.blocks[m].size(); ++k) {
          if (!best_effort) {
            layers_[m]->free(r.blocks[m][k]);
            continue;
          }
          try {
            layers_[m]->free(r.blocks[m][k]);
          } catch (...) {
          }
        }
        r.blocks[m].resize(had);
      }
    };
    try {
      for (; l < num_layers_; ++l) {
        r.blocks[l].reserve(had + need);
        if (!layers_[l]->allocate_many(need, &r.blocks[l])) {
          cut_back(false);
          return false;
        }
      }
    } catch (...) {
      cut_back(true);
      throw;
    }
  }
  r.tokens += num_tokens;
  return true;
}

bool KVCacheManager::commit_kv(RequestId id, int32_t tokens) {
  if (!is_valid_request(id)) return false;
  Request& r = live_request(id);
  if (tokens < r.committed || tokens > r.tokens) return false;
  r.committed = tokens;
  return true;
}

int32_t KVCacheManager::kv_committed_tokens(RequestId id) const { return live_request(id).committed; }

const std::vector<int32_t>& KVCacheManager::get_block_ids(RequestId id, int32_t layer_idx) const {
  check_layer(layer_idx);
  return live_request(id).blocks[layer_idx];
}

int32_t KVCacheManager::get_context_len(RequestId id) const { return live_request(id).tokens; }

int32_t KVCacheManager::num_tokens_in_last_block(RequestId id) const {
  const int32_t n = live_request(id).tokens;
  if (n == 0) return 0;
  return n % block_size_ == 0 ? block_size_ : n % block_size_;
}

std::pair<int32_t, int32_t> KVCacheManager::get_slot(RequestId id, int32_t layer_idx,
                                                     int32_t token_pos) const {
  check_layer(layer_idx);
  const Request& r = live_request(id);
  if (token_pos < 0 || token_pos >= r.tokens) throw std::out_of_range("token position out of range");
  return {r.blocks[layer_idx][token_pos / block_size_], token_pos % block_size_};
}

std::pair<int32_t, int32_t> KVCacheManager::current_slot(RequestId id, int32_t layer_idx) const {
  check_layer(layer_idx);
  const Request& r = live_request(id);
  if (r.tokens == 0) return {-1, -1};
  return get_slot(id, layer_idx, r.tokens - 1);
}

std::vector<int32_t> KVCacheManager::build_slot_mapping(const std::vector<RequestId>& ids,
                                                        int32_t layer_idx) const {
  std::vector<int32_t> out;
  out.reserve(ids.size());
  for (RequestId id : ids) {
    const auto s = current_slot(id, layer_idx);
    out.push_back(s.first * block_size_ + s.second);
  }
  return out;
}

std::pair<std::vector<int32_t>, int32_t> KVCacheManager::build_block_tables(
    const std::vector<RequestId>& ids, int32_t layer_idx) const {
  int32_t width = 0;
  for (RequestId id : ids) width = std::max(width, static_cast<int32_t>(get_block_ids(id, layer_idx).size()));
  std::vector<int32_t> table(ids.size() * static_cast<size_t>(width), -1);
  for (size_t b = 0; b < ids.size(); ++b) {
    const auto& blocks = get_block_ids(ids[b], layer_idx);
    std::copy(blocks.begin(), blocks.end(), table.begin() + b * width);
  }
  return {std::move(table), width};
}

std::vector<int32_t> KVCacheManager::build_seq_lens(const std::vector<RequestId>& ids) const {
  std::vector<int32_t> out;
  out.reserve(ids.size());
  for (RequestId id : ids) out.push_back(get_context_len(id));
  return out;
}

const BlockAllocator& KVCacheManager::allocator(int32_t layer_idx) const {
  check_layer(layer_idx);
  return *layers_[layer_idx];
}

BlockAllocator& KVCacheManager::allocator_mut(int32_t layer_idx) {
  check_layer(layer_idx);
  return *layers_[layer_idx];
}

void KVCacheManager::set_radix_cache_enabled(bool enabled) {
  if (enabled) throw std::invalid_argument("this KV cache manager has no radix prefix cache");
}

int32_t KVCacheManager::num_free_blocks(int32_t layer_idx) const { return allocator(layer_idx).num_free_blocks(); }
int32_t KVCacheManager::num_total_blocks(int32_t layer_idx) const { return allocator(layer_idx).num_total_blocks(); }

}  // namespace base
