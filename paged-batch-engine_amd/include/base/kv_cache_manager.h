// Request-level KV bookkeeping over per-layer block allocators: the subset of
// the reference's base::KVCacheManager (infMain/include/base/kv_cache_manager.h:121-214)
// that the prefill->decode handoff and the decode reader call:
//   register_request / free_request / is_valid_request
//   append_slot(s), get_block_ids, get_slot, current_slot, get_context_len
//   commit_kv / kv_committed_tokens
//   build_block_tables / build_seq_lens / build_slot_mapping
//   allocator(layer), num_layers(), block_size(), num_free_blocks()
// (callers: decode_kv_reservation.cpp:73-91,125-127 and split_pd_engine.cpp:51-112).
// The radix prefix cache, host demotion, snapshots and forks of the
// reference's manager belong to the model runtime, which this build does not
// contain; a request here owns a plain page table per layer.
//
// Request ids are opaque 63-bit values: the low 20 bits name a slot, the bits
// above count how often the slot has been reused, so a stale id never
// aliases a later request (kv_cache_manager.h:262-271 uses the same split).
#ifndef PBE_INCLUDE_BASE_KV_CACHE_MANAGER_H_
#define PBE_INCLUDE_BASE_KV_CACHE_MANAGER_H_

#include <cstdint>
#include <memory>
#include <utility>
#include <vector>

#include "base/block_allocator.h"

namespace base {

using RequestId = int64_t;

class KVCacheManager {
 public:
  // One allocator per layer, all with block_size tokens per block. Throws
  // std::invalid_argument when the counts or block sizes disagree.
  KVCacheManager(int32_t block_size, int32_t num_layers,
                 std::vector<std::unique_ptr<BlockAllocator>> layer_allocators);
  KVCacheManager(const KVCacheManager&) = delete;
  KVCacheManager& operator=(const KVCacheManager&) = delete;

  RequestId register_request();
  // Drops the request's reference on every block of every layer. Throws
  // std::invalid_argument for an id that is not live.
  void free_request(RequestId id);
  bool is_valid_request(RequestId id) const;

  // Grows the request by num_tokens slots, allocating
  // ceil((n+k)/B) - ceil(n/B) new blocks in every layer. All or nothing:
  // returns false (and holds nothing new) when any layer runs out.
  bool append_slots(RequestId id, int32_t num_tokens);
  bool append_slot(RequestId id) { return append_slots(id, 1); }

  // Marks the first `tokens` slots as holding valid KV. Only moves forward
  // and never past the slots appended (kv_cache_manager.cpp:238-244). The
  // caller must have observed the producer's completion first.
  bool commit_kv(RequestId id, int32_t tokens);
  int32_t kv_committed_tokens(RequestId id) const;

  const std::vector<int32_t>& get_block_ids(RequestId id, int32_t layer_idx) const;
  int32_t get_context_len(RequestId id) const;
  int32_t num_tokens_in_last_block(RequestId id) const;
  // (block id, offset in block) of token `token_pos`, and of the last token
  // ({-1, -1} for an empty request).
  std::pair<int32_t, int32_t> get_slot(RequestId id, int32_t layer_idx, int32_t token_pos) const;
  std::pair<int32_t, int32_t> current_slot(RequestId id, int32_t layer_idx) const;

  // Decode-batch inputs: slot = block_id * block_size + offset of each
  // request's last token; [batch, max_blocks] tables padded with -1; lengths.
  std::vector<int32_t> build_slot_mapping(const std::vector<RequestId>& ids, int32_t layer_idx) const;
  std::pair<std::vector<int32_t>, int32_t> build_block_tables(const std::vector<RequestId>& ids,
                                                              int32_t layer_idx) const;
  std::vector<int32_t> build_seq_lens(const std::vector<RequestId>& ids) const;

  const BlockAllocator& allocator(int32_t layer_idx) const;
  BlockAllocator& allocator_mut(int32_t layer_idx);
  int32_t block_size() const { return block_size_; }
  int32_t num_layers() const { return num_layers_; }
  int32_t num_free_blocks(int32_t layer_idx) const;
  int32_t num_total_blocks(int32_t layer_idx) const;
  int32_t num_active_requests() const { return active_; }
  // This build has no radix prefix cache: the shared-arena setup's
  // set_radix_cache_enabled(false) (qwen2.cpp:1137) is accepted, true throws
  // std::invalid_argument.
  void set_radix_cache_enabled(bool enabled);
  bool radix_cache_enabled() const { return false; }

 private:
  struct Request {
    uint64_t reuse = 0;  // generation of the slot
    bool live = false;
    int32_t tokens = 0;
    int32_t committed = 0;
    std::vector<std::vector<int32_t>> blocks;  // per layer
  };
  Request& live_request(RequestId id);
  const Request& live_request(RequestId id) const;
  void check_layer(int32_t layer_idx) const;

  int32_t block_size_;
  int32_t num_layers_;
  std::vector<std::unique_ptr<BlockAllocator>> layers_;
  std::vector<Request> requests_;
  std::vector<uint32_t> idle_slots_;
  int32_t active_ = 0;
};

}  // namespace base

#endif  // PBE_INCLUDE_BASE_KV_CACHE_MANAGER_H_
