// copy_shared_kv (infMain/source/serving/split_pd_engine.cpp:49-115) over the
// KVCacheManager subset and the one-launch run copy of the C ABI.
#include "serving/split_pd_handoff.h"

#include <stdexcept>
#include <string>

#include "base/trace_range.h"

namespace serving {

uint64_t CopySharedKVToDecode(base::KVCacheManager* manager, const KVPoolDescriptor& decode_pool,
                              const SharedKVPrefillResult& source, void* stream,
                              DecodeKVReservation* reservation) {
  const base::TraceRange trace("split_pd_shared_kv_copy");  // split_pd_engine.cpp:51
  if (manager == nullptr || reservation == nullptr)
    throw std::invalid_argument("shared KV handoff needs a manager and a reservation output");
  const base::BlockAllocator& first = manager->allocator(0);
  if (!source.shared_arena_epoch || source.shared_arena_epoch != first.shared_arena_epoch())
    throw std::runtime_error("PD arena epoch mismatch");
  const int32_t layers = manager->num_layers();
  if (source.layers.size() != static_cast<size_t>(layers))
    throw std::runtime_error("PD layer count mismatch");
  const int64_t stride = 2ll * layers;
  DecodeKVReservationRequest request;
  request.client_request_id = source.client_request_id;
  request.handoff_id = source.handoff_id;
  request.prompt_tokens = static_cast<int32_t>(source.prompt_tokens.size());
  request.computed_tokens = source.computed_tokens;
  request.first_token = source.first_token;
  request.src_pool = source.src_pool;
  request.src_block_ids_per_layer.resize(layers);
  // Every layer must carry layer 0's page-major ids (split_pd_engine.cpp:78-79,
  // 91-93), and every layer's allocator views the same arena with the same
  // plane size, so the bounds and alignment checks run once, on layer 0's
  // list; the other layers are compared with it as a whole.
  const std::vector<int32_t>& ids0 = source.layers.front().src_block_ids;
  const base::BlockAllocator& a0 = manager->allocator(0);
  const uint64_t half = a0.key_value_bytes_per_block();
  const uint64_t arena_bytes = a0.shared_arena_bytes();
  const uint32_t page_stride = static_cast<uint32_t>(stride);
  for (int32_t l = 0; l < layers; ++l) {
    const RemoteKVLayerPayload& layer = source.layers[l];
    const base::BlockAllocator& a = manager->allocator(l);
    if (layer.layer_idx != l || !a.uses_shared_arena() || a.key_value_bytes_per_block() != half ||
        a.shared_arena_bytes() != arena_bytes)
      throw std::runtime_error("PD shared layout mismatch");
    // a layer that differs from layer 0 is checked in full first, so its
    // error is the one the per-layer order reports
    if (l == 0 || layer.src_block_ids != ids0) {
      for (int32_t id : layer.src_block_ids)
        if (id < 0 || (static_cast<uint64_t>(id) + stride) * half > arena_bytes ||
            static_cast<uint32_t>(id) % page_stride != 0)
          throw std::runtime_error("PD source block outside shared page layout");
      if (l > 0) throw std::runtime_error("PD page-major layer IDs disagree");
    }
    request.src_block_ids_per_layer[l] = layer.src_block_ids;
  }
  DecodeKVReservationManager reservations(manager, decode_pool);
  KVBlockManifest manifest;
  const base::Status status = reservations.reserve(request, reservation, &manifest);
  if (!status) throw std::runtime_error(status.get_err_msg());
  const KVBlockMapping& mapping = manifest.layer_mappings.front();
  for (const KVBlockMapping& m : manifest.layer_mappings)
    if (m.dst_block_ids != mapping.dst_block_ids) {
      reservations.release(reservation);
      throw std::runtime_error("PD destination is not page-major");
    }
  const pbe_kv_shape shape{layers, decode_pool.kv_head_num, decode_pool.head_size, decode_pool.block_size};
  const int device = first.device_index();
  uint64_t copied = 0;
  const int64_t n = static_cast<int64_t>(mapping.src_block_ids.size());
  const int rc = pbe_copy_shared_kv(first.shared_arena_view(), mapping.src_block_ids.data(),
                                    mapping.dst_block_ids.data(), n, &shape, device, stream, &copied);
  if (rc != PBE_OK) {
    const std::string why = pbe_last_error();
    // A rejected call queued nothing, so the reservation can go; after any
    // other failure the copy's effect is unknown and the pages stay held.
    if (rc == PBE_ERR_INVALID) reservations.release(reservation);
    throw std::runtime_error("PD copy failed; discard the complete IPC domain: " + why);
  }
  if (pbe_stream_synchronize(device, stream) != PBE_OK)
    throw std::runtime_error("PD copy completion unknown; retain source until domain shutdown");
  if (!manager->commit_kv(reservation->decode_request_id, source.computed_tokens))
    throw std::runtime_error("PD destination KV commit failed");
  return copied;
}

}  // namespace serving
