// Decode-side reservation of destination pages for a handoff and the
// manifest that maps them (infMain/include/serving/decode_kv_reservation.h:13-55).
// Destination pages come from KVCacheManager::append_slots, which for a
// shared arena lands in SharedKVPageGroup::allocate for every layer
// (kv_cache_manager.cpp:644-659 -> block_allocator.cpp:205 ->
// shared_kv_arena.cpp:115); the reservation is a registered decode request
// whose first ceil(computed/block_size) pages the manifest maps.
#ifndef PBE_INCLUDE_SERVING_DECODE_KV_RESERVATION_H_
#define PBE_INCLUDE_SERVING_DECODE_KV_RESERVATION_H_

#include <cstdint>
#include <vector>

#include "base/base.h"
#include "base/kv_cache_manager.h"
#include "serving/pd_handoff.h"

namespace serving {

struct DecodeKVReservationRequest {
  GlobalRequestId client_request_id;
  HandoffId handoff_id;
  int32_t prompt_tokens = 0;
  int32_t computed_tokens = 0;
  int32_t first_token = -1;
  KVPoolDescriptor src_pool;
  std::vector<std::vector<int32_t>> src_block_ids_per_layer;
};

struct DecodeKVReservation {
  base::RequestId decode_request_id = -1;
  int32_t reserved_tokens = 0;
  int32_t first_token = -1;
  std::vector<std::vector<int32_t>> dst_block_ids_per_layer;

  bool valid() const { return decode_request_id >= 0; }
};

class DecodeKVReservationManager {
 public:
  // dst_pool describes the decode pool; its layer count and block size must
  // match the manager's. Throws std::invalid_argument for a null manager.
  DecodeKVReservationManager(base::KVCacheManager* kv_manager, KVPoolDescriptor dst_pool);

  // Validates the request (decode_kv_reservation.cpp:14-47), registers a
  // decode request holding computed_tokens slots (ceil(computed_tokens /
  // block_size) pages in every layer) and fills the manifest (src ids
  // truncated to that count). On failure nothing stays reserved and both
  // outputs are reset. The caller commits the tokens with
  // KVCacheManager::commit_kv once the copy has completed.
  base::Status reserve(const DecodeKVReservationRequest& request, DecodeKVReservation* reservation,
                       KVBlockManifest* manifest);
  // Frees the decode request (its pages return to the free list once the
  // page group's stream passes their completion fence).
  void release(DecodeKVReservation* reservation);

  const KVPoolDescriptor& dst_pool() const { return dst_pool_; }

 private:
  base::Status validate_request(const DecodeKVReservationRequest& request) const;
  int32_t required_blocks(int32_t tokens) const;

  base::KVCacheManager* kv_manager_ = nullptr;
  KVPoolDescriptor dst_pool_;
};

}  // namespace serving

#endif  // PBE_INCLUDE_SERVING_DECODE_KV_RESERVATION_H_
