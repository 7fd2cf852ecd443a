// Shared-arena mode of the block allocator; rules follow
// infMain/source/base/block_allocator.cpp:139-401 (reference counts and
// generations per block id, the page group deciding allocation and retire).
#include "base/block_allocator.h"

#include <atomic>
#include <limits>
#include <stdexcept>
#include <string>

namespace base {

BlockAllocator::BlockAllocator(int32_t block_size, int32_t num_kv_heads, int32_t head_size,
                               std::shared_ptr<SharedKVPageGroup> group, int32_t layer)
    : group_(std::move(group)), block_size_(block_size), num_kv_heads_(num_kv_heads),
      head_size_(head_size), layer_(layer),
      storage_spec_(MakeKVCacheStorageSpec(DataType::kDataTypeBf16, BlockStorageMode::kPlain)) {
  if (!group_ || block_size <= 0 || num_kv_heads <= 0 || head_size <= 0 || layer < 0 ||
      layer >= group_->layers())
    throw std::invalid_argument("invalid shared-arena block allocator");
  if (key_value_bytes_per_block() != group_->half_bytes())
    throw std::invalid_argument("block geometry does not match the shared page group");
  num_blocks_ = group_->addressable_blocks();
  if (num_blocks_ <= 0 || static_cast<int64_t>(num_blocks_) * block_size_ > INT32_MAX)
    throw std::invalid_argument("Shared arena exceeds int32 slot mapping range");
  static std::atomic<uint64_t> next_pool_id{uint64_t{1} << 62};
  pool_id_ = next_pool_id.fetch_add(1);
  ref_counts_.assign(num_blocks_, 0);
  generations_.assign(num_blocks_, 0);
}

void BlockAllocator::check_id(int32_t block_id) const {
  if (block_id < 0 || block_id >= num_blocks_) throw std::out_of_range("block_id out of range");
}

int32_t BlockAllocator::allocate() {
  const int32_t id = group_->allocate(layer_);
  if (id < 0) return -1;
  check_id(id);
  if (ref_counts_[id] != 0) throw std::logic_error("allocated block still has outstanding references");
  if (generations_[id] == std::numeric_limits<uint64_t>::max())
    throw std::logic_error("block generation exhausted");
  ++generations_[id];
  ref_counts_[id] = 1;
  return id;
}

void BlockAllocator::incref(int32_t block_id) {
  check_id(block_id);
  if (ref_counts_[block_id] <= 0) throw std::logic_error("Cannot incref a free block");
  ++ref_counts_[block_id];
}

void BlockAllocator::free(int32_t block_id) {
  check_id(block_id);
  if (ref_counts_[block_id] <= 0) throw std::logic_error("Double free of block");
  if (--ref_counts_[block_id] == 0) group_->retire(layer_, block_id);
}

int32_t BlockAllocator::ref_count(int32_t block_id) const {
  check_id(block_id);
  return ref_counts_[block_id];
}

BlockHandle BlockAllocator::handle(int32_t block_id) const {
  check_id(block_id);
  if (ref_counts_[block_id] <= 0) throw std::logic_error("handle of a free block");
  return {block_id, generations_[block_id], pool_id_};
}

bool BlockAllocator::is_current(BlockHandle h) const {
  return h.pool_id == pool_id_ && h.block_id >= 0 && h.block_id < num_blocks_ &&
         ref_counts_[h.block_id] > 0 && generations_[h.block_id] == h.generation;
}

size_t BlockAllocator::key_value_bytes_per_block() const {
  return static_cast<size_t>(block_size_) * num_kv_heads_ * head_size_ *
         DataTypeSize(storage_spec_.storage_dtype);
}

std::pair<void*, void*> BlockAllocator::get_block_ptrs(int32_t block_id) const {
  const KVBlockPayloadPtrs p = get_block_payload_ptrs(block_id);
  return {p.key, p.value};
}

KVBlockPayloadPtrs BlockAllocator::get_block_payload_ptrs(int32_t block_id) const {
  check_id(block_id);
  KVBlockPayloadPtrs ptrs;
  ptrs.key = group_->plane_address(static_cast<int64_t>(block_id) + 2 * layer_);
  ptrs.value = group_->plane_address(static_cast<int64_t>(block_id) + 2 * layer_ + 1);
  ptrs.key_value_bytes = key_value_bytes_per_block();
  return ptrs;
}

int32_t BlockAllocator::num_free_blocks() const {
  group_->collect();
  return group_->free_blocks(layer_);
}

int32_t BlockAllocator::num_total_blocks() const { return group_->capacity(); }
size_t BlockAllocator::shared_leased_bytes() const { return group_->leased_bytes(); }
size_t BlockAllocator::shared_arena_bytes() const { return group_->arena_bytes(); }
uint64_t BlockAllocator::shared_arena_epoch() const { return group_->arena_epoch(); }

KVPoolView BlockAllocator::pool_view() const {
  return KVPoolView(group_->key_base(layer_), group_->value_base(layer_), nullptr, nullptr,
                    key_value_bytes_per_block(), storage_spec_, DeviceType::kDeviceHIP);
}

}  // namespace base
