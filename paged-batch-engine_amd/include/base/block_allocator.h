// The reference's block allocator (infMain/include/base/block_allocator.h:113-240,
// block_allocator.cpp:17-428) in two of its modes:
//  - shared-arena mode: the per-layer view of a SharedKVPageGroup that
//    copy_shared_kv and the decode runtime use. Block ids are page-major (byte
//    offset / half), so layer l's K plane of block b is half-plane b + 2l of
//    the arena and its V plane b + 2l + 1;
//  - local-pool mode: one layer's own [num_blocks][block] K and V pools (and,
//    for FP8 storage, [num_blocks][block_size * heads] fp32 K and V scale
//    pools) with a FIFO free queue, on the GPU or in host memory.
// Device pointers are plain pointers (no tensor type). The external-pool
// binding of the reference belongs to its data service, outside this build.
#ifndef PBE_INCLUDE_BASE_BLOCK_ALLOCATOR_H_
#define PBE_INCLUDE_BASE_BLOCK_ALLOCATOR_H_

#include <cstddef>
#include <cstdint>
#include <deque>
#include <memory>
#include <utility>
#include <vector>

#include "base/base.h"
#include "base/kv_cache_format.h"
#include "base/page_index.h"
#include "base/shared_kv_arena.h"

namespace base {

struct BlockHandle {
  int32_t block_id = -1;
  uint64_t generation = 0;
  uint64_t pool_id = 0;
};

struct KVBlockPayloadPtrs {
  void* key = nullptr;
  void* value = nullptr;
  void* key_scale = nullptr;
  void* value_scale = nullptr;
  size_t key_value_bytes = 0;
  size_t scale_bytes = 0;
};

// Non-owning binding used by compute kernels (block_allocator.h:86-112). In
// the shared arena, block b of this layer starts at key + b * block_stride
// (single-segment arenas; segmented arenas resolve per block through
// BlockAllocator::get_block_payload_ptrs).
class KVPoolView {
 public:
  KVPoolView() = default;
  KVPoolView(void* key, void* value, void* key_scale, void* value_scale, size_t block_stride,
             KVCacheStorageSpec storage_spec, DeviceType device)
      : key_(key), value_(value), key_scale_(key_scale), value_scale_(value_scale),
        block_stride_(block_stride), storage_spec_(storage_spec), device_(device) {}
  // With the bytes addressable from each pool pointer (the reference's pool
  // tensors carry their sizes; kernels bound their writes by them).
  KVPoolView(void* key, void* value, void* key_scale, void* value_scale, size_t block_stride,
             KVCacheStorageSpec storage_spec, DeviceType device, size_t key_bytes,
             size_t value_bytes, size_t scale_bytes)
      : KVPoolView(key, value, key_scale, value_scale, block_stride, storage_spec, device) {
    key_bytes_ = key_bytes;
    value_bytes_ = value_bytes;
    scale_bytes_ = scale_bytes;
  }
  bool valid() const { return key_ != nullptr && value_ != nullptr; }
  bool uses_fp8_storage() const { return storage_spec_.uses_fp8_storage(); }
  DeviceType device_type() const { return device_; }
  const KVCacheStorageSpec& storage_spec() const { return storage_spec_; }
  void* key_pool() const { return key_; }
  void* value_pool() const { return value_; }
  void* key_scale_pool() const { return key_scale_; }
  void* value_scale_pool() const { return value_scale_; }
  size_t block_stride() const { return block_stride_; }
  // 0 when unknown.
  size_t key_pool_bytes() const { return key_bytes_; }
  size_t value_pool_bytes() const { return value_bytes_; }
  size_t scale_pool_bytes() const { return scale_bytes_; }  // each of the K and V scale pools

 private:
  void* key_ = nullptr;
  void* value_ = nullptr;
  void* key_scale_ = nullptr;
  void* value_scale_ = nullptr;
  size_t block_stride_ = 0;
  KVCacheStorageSpec storage_spec_;
  DeviceType device_ = DeviceType::kDeviceUnknown;
  size_t key_bytes_ = 0;
  size_t value_bytes_ = 0;
  size_t scale_bytes_ = 0;
};

class BlockAllocator {
 public:
  // Local-pool mode (block_allocator.cpp:17-84): kDeviceHIP pools live on the
  // calling thread's current GPU, kDeviceCPU pools in host memory. Throws
  // std::invalid_argument for a bad geometry or an invalid storage spec and
  // std::runtime_error when the pools cannot be allocated.
  BlockAllocator(int32_t num_blocks, int32_t block_size, int32_t num_kv_heads, int32_t head_size,
                 const KVCacheStorageSpec& storage_spec, DeviceType device);
  BlockAllocator(int32_t num_blocks, int32_t block_size, int32_t num_kv_heads, int32_t head_size,
                 DataType dtype, DeviceType device,
                 BlockStorageMode storage_mode = BlockStorageMode::kPlain);
  ~BlockAllocator();
  // Shared-arena mode (block_allocator.cpp:139-163): BF16 plain storage, one
  // allocator per layer over a page group whose half-plane equals
  // block_size * num_kv_heads * head_size * 2 bytes. Throws
  // std::invalid_argument on a mismatch.
  BlockAllocator(int32_t block_size, int32_t num_kv_heads, int32_t head_size,
                 std::shared_ptr<SharedKVPageGroup> group, int32_t layer);
  BlockAllocator(const BlockAllocator&) = delete;
  BlockAllocator& operator=(const BlockAllocator&) = delete;

  // Block id of a fresh page for this layer, or -1 when the group is out of
  // quota (block_allocator.cpp:206-216). Layers allocate in order.
  int32_t allocate();
  // allocate() up to n times, appending the ids to *out; false at the first
  // -1 (ids already appended stay allocated). One page-group lock per call in
  // shared-arena mode. No counterpart in the reference.
  bool allocate_many(int32_t n, std::vector<int32_t>* out);
  void incref(int32_t block_id);
  // Drops one reference; the last one retires the page in the group.
  void free(int32_t block_id);
  // free() of each id in order; in shared-arena mode the blocks that reach no
  // references retire together (SharedKVPageGroup::retire_many). An invalid
  // id throws as free() would, after the ids before it are freed. No
  // counterpart in the reference.
  void free_many(const std::vector<int32_t>& block_ids);
  int32_t ref_count(int32_t block_id) const;
  BlockHandle handle(int32_t block_id) const;
  bool is_current(BlockHandle handle) const;

  std::pair<void*, void*> get_block_ptrs(int32_t block_id) const;
  KVBlockPayloadPtrs get_block_payload_ptrs(int32_t block_id) const;
  // Bitwise copy of one block's K and V payload (and scales) onto another
  // block of this layer, both allocated (block_allocator.cpp:403-428). On the
  // GPU it is one copy-kernel launch, ordered on the page group's stream in
  // shared-arena mode, and returns once the copy has completed. Throws
  // std::logic_error for equal or free blocks, std::runtime_error when the
  // device copy fails.
  void copy_block_payload(int32_t source_block_id, int32_t destination_block_id) const;
  uint64_t payload_copy_bytes() const { return payload_copy_bytes_; }

  int32_t num_free_blocks() const;
  int32_t num_total_blocks() const;
  bool uses_shared_arena() const { return group_ != nullptr; }
  size_t shared_leased_bytes() const;
  size_t shared_arena_bytes() const;
  uint64_t shared_arena_epoch() const;
  // Shared-arena mode: this process's mapping of the arena and its GPU
  // (nullptr / -1 in local-pool mode).
  const pbe_arena_view* shared_arena_view() const { return group_ ? &group_->arena_view() : nullptr; }
  int device_index() const { return device_index_; }

  int32_t block_size() const { return block_size_; }
  int32_t num_kv_heads() const { return num_kv_heads_; }
  int32_t head_size() const { return head_size_; }
  int32_t layer() const { return layer_; }
  const KVCacheStorageSpec& storage_spec() const { return storage_spec_; }
  BlockStorageMode storage_mode() const { return storage_spec_.storage_mode; }
  bool uses_fp8_storage() const { return storage_spec_.uses_fp8_storage(); }
  DeviceType device_type() const { return device_; }
  size_t key_value_bytes_per_block() const;
  size_t scale_bytes_per_block() const;
  KVPoolView pool_view() const;

 private:
  void check_id(int32_t block_id) const;
  // Index of block_id in ref_counts_ / generations_: the id itself in
  // local-pool mode; id / 2L in shared-arena mode, -1 for an id that is not a
  // page id (never allocated there). Throws out_of_range like check_id.
  int32_t slot(int32_t block_id) const;
  std::shared_ptr<SharedKVPageGroup> group_;  // shared-arena mode only
  int32_t block_size_, num_kv_heads_, head_size_, layer_ = 0;
  int32_t num_blocks_ = 0;
  uint64_t pool_id_ = 0;
  DeviceType device_ = DeviceType::kDeviceHIP;
  int device_index_ = -1;
  KVCacheStorageSpec storage_spec_;
  int32_t id_stride_ = 1;  // shared-arena mode: 2L (page ids only)
  PageIndex page_index_;   // id / id_stride_ without a division (slot())
  std::vector<int32_t> ref_counts_;
  std::vector<uint64_t> generations_;
  // Local-pool mode: [K pool][V pool][K scales][V scales] in one allocation.
  pbe_arena* device_pools_ = nullptr;
  std::vector<uint8_t> host_pools_;
  uint8_t* key_pool_ = nullptr;
  uint8_t* value_pool_ = nullptr;
  uint8_t* key_scale_pool_ = nullptr;
  uint8_t* value_scale_pool_ = nullptr;
  std::deque<int32_t> free_queue_;
  mutable uint64_t payload_copy_bytes_ = 0;
};

}  // namespace base

#endif  // PBE_INCLUDE_BASE_BLOCK_ALLOCATOR_H_
