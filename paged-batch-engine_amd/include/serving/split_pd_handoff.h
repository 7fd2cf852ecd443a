// The decode side of a same-GPU split prefill/decode handoff as one library
// call with the reference's semantics: copy_shared_kv
// (infMain/source/serving/split_pd_engine.cpp:49-115), whose inputs are the
// prefill result received over the control plane and the decode process's
// KVCacheManager.
#ifndef PBE_INCLUDE_SERVING_SPLIT_PD_HANDOFF_H_
#define PBE_INCLUDE_SERVING_SPLIT_PD_HANDOFF_H_

#include <cstdint>
#include <vector>

#include "base/kv_cache_manager.h"
#include "serving/decode_kv_reservation.h"
#include "serving/kv_page_wire.h"
#include "serving/pd_handoff.h"

namespace serving {

// The fields of the reference's RemotePrefillResult (serving_zmq_rpc.h:86-99)
// that the shared-arena handoff reads.
struct SharedKVPrefillResult {
  uint64_t shared_arena_epoch = 0;
  GlobalRequestId client_request_id;
  HandoffId handoff_id;
  std::vector<int32_t> prompt_tokens;
  int32_t computed_tokens = 0;
  int32_t first_token = -1;
  KVPoolDescriptor src_pool;
  std::vector<RemoteKVLayerPayload> layers;
};

// In order, as split_pd_engine.cpp:51-112 does:
//  1. the source epoch must equal the decode mapping's (allocator 0's);
//  2. one payload per layer, layer_idx == position, every allocator in
//     shared-arena mode, ids page-major and inside the arena, all layers'
//     lists identical;
//  3. DecodeKVReservationManager(manager, decode_pool).reserve(...) -> the
//     manifest; its destination lists must be page-major too;
//  4. runs coalesced and copied by one gfx950 kernel on `stream` (the
//     reference's per-run cudaMemcpyAsync loop);
//  5. the stream is synchronized and manager->commit_kv(reservation,
//     computed_tokens) marks the copied KV valid.
// Returns the bytes copied. Throws std::runtime_error with the reference's
// messages on a rejected input (nothing written, nothing reserved) and when
// the copy's completion cannot be established (the reservation is then kept:
// the copy may still write it).
uint64_t CopySharedKVToDecode(base::KVCacheManager* manager, const KVPoolDescriptor& decode_pool,
                              const SharedKVPrefillResult& source, void* stream,
                              DecodeKVReservation* reservation);

}  // namespace serving

#endif  // PBE_INCLUDE_SERVING_SPLIT_PD_HANDOFF_H_
