// Compact wire form of a prefill result's KV page list.
//
// The reference ships the page list of a prefill result as one JSON integer
// array per layer (RemoteKVLayerPayload::src_block_ids,
// infMain/include/serving/serving_zmq_rpc.h:80-98; serialized by
// remote_prefill_result_to_json, serving_zmq_rpc.cpp:222-253), and
// copy_shared_kv insists that every layer's array is the same page-major list
// (split_pd_engine.cpp:63-80). These helpers encode that list once, as spans
// of consecutive page ids, in the binary layout of pbe_page_list_encode
// (include/pbe_handoff.h), and decode it back into the per-layer payloads the
// decode side's reservation code consumes.
#ifndef PBE_INCLUDE_SERVING_KV_PAGE_WIRE_H_
#define PBE_INCLUDE_SERVING_KV_PAGE_WIRE_H_

#include <cstdint>
#include <string>
#include <vector>

#include "base/base.h"

namespace serving {

// The id part of the reference's RemoteKVLayerPayload (serving_zmq_rpc.h:80-84);
// inline block payloads (`blocks`) belong to the non-shared-arena transport.
struct RemoteKVLayerPayload {
  int32_t layer_idx = -1;
  std::vector<int32_t> src_block_ids;
};

// Checks the layers as copy_shared_kv does (layer_idx == position, identical
// page-major lists, ids >= 0 and multiples of 2*layers) and encodes them.
// Arena bounds are the decode side's check (it knows its mapping).
base::Status EncodeKVPageList(uint64_t shared_arena_epoch,
                              const std::vector<RemoteKVLayerPayload>& layers, std::string* wire);

constexpr int64_t kMaxWirePages = int64_t{1} << 22;

// Decodes and checks a page list; fills one payload per layer, all with the
// same ids, ready for DecodeKVReservationRequest::src_block_ids_per_layer.
// A few bytes of spans can claim millions of pages: `max_pages` (the arena's
// page capacity, say) bounds what is allocated for input from another
// process; longer lists are rejected before any allocation. The default,
// 2^22 pages, exceeds any one-GPU arena (1.8 TB of 448 KiB pages).
base::Status DecodeKVPageList(const std::string& wire, uint64_t* shared_arena_epoch,
                              std::vector<RemoteKVLayerPayload>* layers,
                              int64_t max_pages = kMaxWirePages);

// Decodes the page-major id list once (no per-layer copies).
base::Status DecodeKVPageIds(const std::string& wire, uint64_t* shared_arena_epoch,
                             int32_t* layers, std::vector<int32_t>* ids,
                             int64_t max_pages = kMaxWirePages);

}  // namespace serving

#endif  // PBE_INCLUDE_SERVING_KV_PAGE_WIRE_H_
