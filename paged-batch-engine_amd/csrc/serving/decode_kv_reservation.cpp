// Rules follow infMain/source/serving/decode_kv_reservation.cpp:14-130.
#include "serving/decode_kv_reservation.h"

#include <stdexcept>

namespace serving {
namespace {
using base::error::InvalidArgument;
}

DecodeKVReservationManager::DecodeKVReservationManager(base::SharedKVPageGroup* pages,
                                                       KVPoolDescriptor dst_pool)
    : pages_(pages), dst_pool_(std::move(dst_pool)) {
  if (pages_ == nullptr) throw std::invalid_argument("decode kv reservation needs a page group");
}

base::Status DecodeKVReservationManager::validate_request(const DecodeKVReservationRequest& r) const {
  if (r.client_request_id.empty()) return InvalidArgument("decode kv reservation missing client_request_id");
  if (!r.handoff_id.valid()) return InvalidArgument("decode kv reservation missing handoff_id");
  if (r.prompt_tokens <= 0) return InvalidArgument("decode kv reservation prompt_tokens must be positive");
  if (r.computed_tokens <= 0 || r.computed_tokens > r.prompt_tokens)
    return InvalidArgument("decode kv reservation computed_tokens is invalid");
  if (!r.src_pool.compatible_with(dst_pool_))
    return InvalidArgument("decode kv reservation source/destination pools are incompatible");
  if (dst_pool_.layer_num != pages_->layers())
    return InvalidArgument("decode kv reservation dst layer_num mismatch");
  if (dst_pool_.block_size <= 0 ||
      static_cast<uint64_t>(dst_pool_.bytes_per_block_per_layer()) != 2 * pages_->half_bytes())
    return InvalidArgument("decode kv reservation dst block_size mismatch");
  if (static_cast<int32_t>(r.src_block_ids_per_layer.size()) != dst_pool_.layer_num)
    return InvalidArgument("decode kv reservation source layer count mismatch");
  const int32_t blocks = required_blocks(r.computed_tokens);
  for (const auto& ids : r.src_block_ids_per_layer)
    if (static_cast<int32_t>(ids.size()) < blocks)
      return InvalidArgument("decode kv reservation source block count is insufficient");
  return base::error::Success();
}

int32_t DecodeKVReservationManager::required_blocks(int32_t tokens) const {
  if (tokens <= 0) return 0;
  return (tokens + dst_pool_.block_size - 1) / dst_pool_.block_size;
}

base::Status DecodeKVReservationManager::reserve(const DecodeKVReservationRequest& request,
                                                 DecodeKVReservation* reservation,
                                                 KVBlockManifest* manifest) {
  if (reservation == nullptr) return InvalidArgument("decode kv reservation output is null");
  if (manifest == nullptr) return InvalidArgument("decode kv reservation manifest output is null");
  *reservation = {};
  *manifest = {};
  base::Status status = validate_request(request);
  if (!status) return status;

  const int32_t blocks = required_blocks(request.computed_tokens);
  const int32_t layers = dst_pool_.layer_num;
  DecodeKVReservation held;
  held.decode_request_id = next_request_id_++;
  held.reserved_tokens = request.computed_tokens;
  held.first_token = request.first_token;
  held.dst_block_ids_per_layer.assign(layers, {});
  // Page by page: layer 0 picks the page, layers 1..L-1 take its reservation.
  for (int32_t b = 0; b < blocks; ++b) {
    const int id = pages_->allocate(0);
    if (id < 0) {
      release(&held);
      return base::error::InternalError("decode kv reservation failed to allocate dst KV blocks");
    }
    held.dst_block_ids_per_layer[0].push_back(id);
    for (int32_t l = 1; l < layers; ++l) held.dst_block_ids_per_layer[l].push_back(pages_->allocate(l));
  }

  manifest->client_request_id = request.client_request_id;
  manifest->handoff_id = request.handoff_id;
  manifest->prompt_tokens = request.prompt_tokens;
  manifest->computed_tokens = request.computed_tokens;
  manifest->first_token = request.first_token;
  manifest->src_pool = request.src_pool;
  manifest->dst_pool = dst_pool_;
  manifest->layer_mappings.reserve(layers);
  for (int32_t l = 0; l < layers; ++l) {
    KVBlockMapping m;
    m.layer_idx = l;
    m.src_block_ids.assign(request.src_block_ids_per_layer[l].begin(),
                           request.src_block_ids_per_layer[l].begin() + blocks);
    m.dst_block_ids = held.dst_block_ids_per_layer[l];
    manifest->layer_mappings.push_back(std::move(m));
  }
  status = manifest->validate();
  if (!status) {
    release(&held);
    *manifest = {};
    return status;
  }
  *reservation = std::move(held);
  return base::error::Success();
}

void DecodeKVReservationManager::release(DecodeKVReservation* reservation) {
  if (reservation == nullptr || !reservation->valid()) return;
  auto& ids = reservation->dst_block_ids_per_layer;
  // Retire the later layers first so layer 0's retire finds nothing to roll
  // back, then layer 0 (which fences the page once all layers are retired).
  for (size_t l = ids.size(); l-- > 1;)
    for (int id : ids[l]) pages_->retire(static_cast<int>(l), id);
  if (!ids.empty())
    for (int id : ids[0]) pages_->retire(0, id);
  *reservation = {};
}

}  // namespace serving
