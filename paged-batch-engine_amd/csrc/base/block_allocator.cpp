// Block allocator in shared-arena and local-pool mode; rules follow
// infMain/source/base/block_allocator.cpp:17-428 (reference counts and
// generations per block id; the page group or a FIFO free queue deciding
// allocation and reuse).
#include "base/block_allocator.h"

#include <atomic>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <string>

namespace base {
namespace {
uint64_t next_pool_id() {
  static std::atomic<uint64_t> next{1};
  return next.fetch_add(1);
}
}  // namespace

BlockAllocator::BlockAllocator(int32_t num_blocks, int32_t block_size, int32_t num_kv_heads,
                               int32_t head_size, const KVCacheStorageSpec& storage_spec,
                               DeviceType device)
    : block_size_(block_size), num_kv_heads_(num_kv_heads), head_size_(head_size),
      num_blocks_(num_blocks), device_(device), storage_spec_(storage_spec) {
  if (num_blocks <= 0 || block_size <= 0 || num_kv_heads <= 0 || head_size <= 0)
    throw std::invalid_argument("block pool dimensions must be positive");
  if (device != DeviceType::kDeviceHIP && device != DeviceType::kDeviceCPU)
    throw std::invalid_argument("block pool device must be HIP or CPU");
  const Status ok = ValidateKVCacheStorageSpec(storage_spec_, device_, storage_spec_.logical_dtype);
  if (!ok) throw std::invalid_argument(ok.get_err_msg());
  const uint64_t kv = static_cast<uint64_t>(num_blocks) * key_value_bytes_per_block();
  const uint64_t sc = static_cast<uint64_t>(num_blocks) * scale_bytes_per_block();
  // Every pool starts on a 256-byte boundary.
  const uint64_t kv_pad = (kv + 255) / 256 * 256, sc_pad = (sc + 255) / 256 * 256;
  const uint64_t total = 2 * kv_pad + 2 * sc_pad;
  uint8_t* base = nullptr;
  if (device_ == DeviceType::kDeviceHIP) {
    if (pbe_current_device(&device_index_) != PBE_OK ||
        pbe_arena_create(device_index_, total, 0, 1, &device_pools_) != PBE_OK)
      throw std::runtime_error(std::string("block pool allocation: ") + pbe_last_error());
    pbe_arena_view v;
    pbe_arena_get_view(device_pools_, &v);
    base = static_cast<uint8_t*>(v.base[0]);
  } else {
    host_pools_.assign(total, 0);
    base = host_pools_.data();
  }
  key_pool_ = base;
  value_pool_ = base + kv_pad;
  if (sc) {
    key_scale_pool_ = base + 2 * kv_pad;
    value_scale_pool_ = base + 2 * kv_pad + sc_pad;
  }
  pool_id_ = next_pool_id();
  ref_counts_.assign(num_blocks_, 0);
  generations_.assign(num_blocks_, 0);
  for (int32_t i = 0; i < num_blocks_; ++i) free_queue_.push_back(i);
}

BlockAllocator::BlockAllocator(int32_t num_blocks, int32_t block_size, int32_t num_kv_heads,
                               int32_t head_size, DataType dtype, DeviceType device,
                               BlockStorageMode storage_mode)
    : BlockAllocator(num_blocks, block_size, num_kv_heads, head_size,
                     MakeKVCacheStorageSpec(dtype, storage_mode), device) {}

BlockAllocator::~BlockAllocator() {
  if (device_pools_) pbe_arena_destroy(device_pools_);
}

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
  device_ = DeviceType::kDeviceHIP;
  device_index_ = group_->device();
  num_blocks_ = group_->addressable_blocks();
  if (num_blocks_ <= 0 || static_cast<int64_t>(num_blocks_) * block_size_ > INT32_MAX)
    throw std::invalid_argument("Shared arena exceeds int32 slot mapping range");
  pool_id_ = next_pool_id();
  // Only page ids (multiples of 2L) are ever handed out here, so the counts
  // are kept per page: dense for the pages of one request, where an array
  // per addressable id put every page's entry on its own cache line.
  id_stride_ = 2 * group_->layers();
  page_index_ = PageIndex(id_stride_);
  const int32_t pages = (num_blocks_ + id_stride_ - 1) / id_stride_;
  ref_counts_.assign(pages, 0);
  generations_.assign(pages, 0);
}

void BlockAllocator::check_id(int32_t block_id) const {
  if (block_id < 0 || block_id >= num_blocks_) throw std::out_of_range("block_id out of range");
}

int32_t BlockAllocator::slot(int32_t block_id) const {
  check_id(block_id);
  return id_stride_ == 1 ? block_id : page_index_.of(block_id);
}

int32_t BlockAllocator::allocate() {
  int32_t id;
  if (group_) {
    id = group_->allocate(layer_);
    if (id < 0) return -1;
  } else {
    if (free_queue_.empty()) return -1;
    id = free_queue_.front();
    free_queue_.pop_front();
  }
  const int32_t k = slot(id);
  if (k < 0) throw std::logic_error("page group handed out a non-page id");
  if (ref_counts_[k] != 0) throw std::logic_error("allocated block still has outstanding references");
  if (generations_[k] == std::numeric_limits<uint64_t>::max())
    throw std::logic_error("block generation exhausted");
  ++generations_[k];
  ref_counts_[k] = 1;
  return id;
}

bool BlockAllocator::allocate_many(int32_t n, std::vector<int32_t>* out) {
  if (!group_) {
    for (int32_t k = 0; k < n; ++k) {
      const int32_t id = allocate();
      if (id < 0) return false;
      out->push_back(id);
    }
    return true;
  }
  const size_t first = out->size();
  const bool all = group_->allocate_many(layer_, n, out);
  for (size_t i = first; i < out->size(); ++i) {
    const int32_t k = slot((*out)[i]);
    if (k < 0) throw std::logic_error("page group handed out a non-page id");
    if (ref_counts_[k] != 0) throw std::logic_error("allocated block still has outstanding references");
    if (generations_[k] == std::numeric_limits<uint64_t>::max())
      throw std::logic_error("block generation exhausted");
    ++generations_[k];
    ref_counts_[k] = 1;
  }
  return all;
}

void BlockAllocator::incref(int32_t block_id) {
  const int32_t k = slot(block_id);
  if (k < 0 || ref_counts_[k] <= 0) throw std::logic_error("Cannot incref a free block");
  ++ref_counts_[k];
}

void BlockAllocator::free(int32_t block_id) {
  const int32_t k = slot(block_id);
  if (k < 0 || ref_counts_[k] <= 0) throw std::logic_error("Double free of block");
  if (--ref_counts_[k] == 0) {
    if (group_) group_->retire(layer_, block_id);
    else free_queue_.push_back(block_id);
  }
}

void BlockAllocator::free_many(const std::vector<int32_t>& block_ids) {
  if (!group_) {
    for (int32_t id : block_ids) free(id);
    return;
  }
  std::vector<int32_t> released;
  released.reserve(block_ids.size());
  try {
    for (int32_t id : block_ids) {
      const int32_t k = slot(id);
      if (k < 0 || ref_counts_[k] <= 0) throw std::logic_error("Double free of block");
      if (--ref_counts_[k] == 0) released.push_back(id);
    }
  } catch (...) {
    group_->retire_many(layer_, released);
    throw;
  }
  group_->retire_many(layer_, released);
}

int32_t BlockAllocator::ref_count(int32_t block_id) const {
  const int32_t k = slot(block_id);
  return k < 0 ? 0 : ref_counts_[k];
}

BlockHandle BlockAllocator::handle(int32_t block_id) const {
  const int32_t k = slot(block_id);
  if (k < 0 || ref_counts_[k] <= 0) throw std::logic_error("handle of a free block");
  return {block_id, generations_[k], pool_id_};
}

bool BlockAllocator::is_current(BlockHandle h) const {
  if (h.pool_id != pool_id_ || h.block_id < 0 || h.block_id >= num_blocks_) return false;
  const int32_t k = slot(h.block_id);
  return k >= 0 && ref_counts_[k] > 0 && generations_[k] == h.generation;
}

size_t BlockAllocator::key_value_bytes_per_block() const {
  return static_cast<size_t>(block_size_) * num_kv_heads_ * head_size_ *
         DataTypeSize(storage_spec_.storage_dtype);
}

std::pair<void*, void*> BlockAllocator::get_block_ptrs(int32_t block_id) const {
  const KVBlockPayloadPtrs p = get_block_payload_ptrs(block_id);
  return {p.key, p.value};
}

size_t BlockAllocator::scale_bytes_per_block() const {
  if (!storage_spec_.has_scales()) return 0;
  return static_cast<size_t>(block_size_) * num_kv_heads_ * DataTypeSize(storage_spec_.scale_dtype);
}

KVBlockPayloadPtrs BlockAllocator::get_block_payload_ptrs(int32_t block_id) const {
  check_id(block_id);
  KVBlockPayloadPtrs ptrs;
  ptrs.key_value_bytes = key_value_bytes_per_block();
  if (group_) {
    ptrs.key = group_->plane_address(static_cast<int64_t>(block_id) + 2 * layer_);
    ptrs.value = group_->plane_address(static_cast<int64_t>(block_id) + 2 * layer_ + 1);
    return ptrs;
  }
  const size_t kv = static_cast<size_t>(block_id) * ptrs.key_value_bytes;
  ptrs.key = key_pool_ + kv;
  ptrs.value = value_pool_ + kv;
  ptrs.scale_bytes = scale_bytes_per_block();
  if (ptrs.scale_bytes) {
    const size_t s = static_cast<size_t>(block_id) * ptrs.scale_bytes;
    ptrs.key_scale = key_scale_pool_ + s;
    ptrs.value_scale = value_scale_pool_ + s;
  }
  return ptrs;
}

void BlockAllocator::copy_block_payload(int32_t source_block_id, int32_t destination_block_id) const {
  if (source_block_id == destination_block_id)
    throw std::logic_error("block payload copy onto itself");
  if (ref_count(source_block_id) <= 0 || ref_count(destination_block_id) <= 0)
    throw std::logic_error("block payload copy between free blocks");
  const KVBlockPayloadPtrs src = get_block_payload_ptrs(source_block_id);
  const KVBlockPayloadPtrs dst = get_block_payload_ptrs(destination_block_id);
  pbe_copy_op ops[4];
  int n = 0;
  auto add = [&](const void* s, void* d, size_t bytes) {
    if (bytes) ops[n++] = {reinterpret_cast<uint64_t>(s), reinterpret_cast<uint64_t>(d), bytes};
  };
  add(src.key, dst.key, src.key_value_bytes);
  add(src.value, dst.value, src.key_value_bytes);
  add(src.key_scale, dst.key_scale, src.scale_bytes);
  add(src.value_scale, dst.value_scale, src.scale_bytes);
  if (device_ == DeviceType::kDeviceCPU) {
    for (int i = 0; i < n; ++i)
      std::memcpy(reinterpret_cast<void*>(ops[i].dst), reinterpret_cast<const void*>(ops[i].src), ops[i].bytes);
  } else {
    void* stream = group_ ? group_->stream() : nullptr;
    if (pbe_copy_ops(ops, n, device_index_, stream) != PBE_OK ||
        pbe_stream_synchronize(device_index_, stream) != PBE_OK)
      throw std::runtime_error(std::string("block payload copy failed: ") + pbe_last_error());
  }
  payload_copy_bytes_ += 2 * src.key_value_bytes + 2 * src.scale_bytes;
}

int32_t BlockAllocator::num_free_blocks() const {
  if (!group_) return static_cast<int32_t>(free_queue_.size());
  group_->collect();
  return group_->free_blocks(layer_);
}

int32_t BlockAllocator::num_total_blocks() const { return group_ ? group_->capacity() : num_blocks_; }
size_t BlockAllocator::shared_leased_bytes() const { return group_ ? group_->leased_bytes() : 0; }
size_t BlockAllocator::shared_arena_bytes() const { return group_ ? group_->arena_bytes() : 0; }
uint64_t BlockAllocator::shared_arena_epoch() const { return group_ ? group_->arena_epoch() : 0; }

KVPoolView BlockAllocator::pool_view() const {
  const size_t half = key_value_bytes_per_block();
  if (!group_) {
    const size_t n = static_cast<size_t>(num_blocks_);
    return KVPoolView(key_pool_, value_pool_, key_scale_pool_, value_scale_pool_, half, storage_spec_,
                      device_, n * half, n * half, n * scale_bytes_per_block());
  }
  // Shared arena: this layer's K plane of block b at key_base + b * half, up to
  // the end of the arena (flat single-segment arenas only; otherwise no base).
  void* key = group_->key_base(layer_);
  void* value = group_->value_base(layer_);
  const size_t arena = group_->arena_bytes();
  const size_t k_off = 2 * static_cast<size_t>(layer_) * half;
  return KVPoolView(key, value, nullptr, nullptr, half, storage_spec_, DeviceType::kDeviceHIP,
                    key && arena > k_off ? arena - k_off : 0,
                    value && arena > k_off + half ? arena - k_off - half : 0, 0);
}

}  // namespace base
