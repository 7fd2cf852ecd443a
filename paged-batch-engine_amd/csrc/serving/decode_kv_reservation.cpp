// Rules follow infMain/source/serving/decode_kv_reservation.cpp:14-130.
#include "serving/decode_kv_reservation.h"

#include <stdexcept>

namespace serving {
namespace {
using base::error::InvalidArgument;
}

DecodeKVReservationManager::DecodeKVReservationManager(base::KVCacheManager* kv_manager,
                                                       KVPoolDescriptor dst_pool)
    : kv_manager_(kv_manager), dst_pool_(std::move(dst_pool)) {
  if (kv_manager_ == nullptr) throw std::invalid_argument("decode kv reservation needs a KV cache manager");
}

base::Status DecodeKVReservationManager::validate_request(const DecodeKVReservationRequest& r) const {
  if (r.client_request_id.empty()) return InvalidArgument("decode kv reservation missing client_request_id");
  if (!r.handoff_id.valid()) return InvalidArgument("decode kv reservation missing handoff_id");
  if (r.prompt_tokens <= 0) return InvalidArgument("decode kv reservation prompt_tokens must be positive");
  if (r.computed_tokens <= 0 || r.computed_tokens > r.prompt_tokens)
    return InvalidArgument("decode kv reservation computed_tokens is invalid");
  if (!r.src_pool.compatible_with(dst_pool_))
    return InvalidArgument("decode kv reservation source/destination pools are incompatible");
  if (dst_pool_.layer_num != kv_manager_->num_layers())
    return InvalidArgument("decode kv reservation dst layer_num mismatch");
  // The reference compares block sizes only; the per-layer payload bytes are
  // checked as well so a pool whose head geometry differs from the manager's
  // allocators cannot be mapped.
  if (dst_pool_.block_size != kv_manager_->block_size() ||
      static_cast<uint64_t>(dst_pool_.bytes_per_block_per_layer()) !=
          2 * kv_manager_->allocator(0).key_value_bytes_per_block())
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
  const base::RequestId id = kv_manager_->register_request();
  if (!kv_manager_->append_slots(id, request.computed_tokens)) {
    kv_manager_->free_request(id);
    return base::error::InternalError("decode kv reservation failed to allocate dst KV blocks");
  }
  DecodeKVReservation held;
  held.decode_request_id = id;
  held.reserved_tokens = request.computed_tokens;
  held.first_token = request.first_token;
  held.dst_block_ids_per_layer.resize(layers);
  for (int32_t l = 0; l < layers; ++l) {
    const std::vector<int32_t>& got = kv_manager_->get_block_ids(id, l);
    if (static_cast<int32_t>(got.size()) < blocks) {
      release(&held);
      return base::error::InternalError("decode kv reservation dst block count is insufficient");
    }
    held.dst_block_ids_per_layer[l].assign(got.begin(), got.begin() + blocks);
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
  if (kv_manager_->is_valid_request(reservation->decode_request_id))
    kv_manager_->free_request(reservation->decode_request_id);
  *reservation = {};
}

}  // namespace serving
