// Descriptor, manifest and status helpers: infMain/source/serving/pd_handoff_common.cpp:302-381.
#include "serving/pd_handoff.h"

namespace serving {

int64_t KVPoolDescriptor::bytes_per_block_per_layer() const {
  const auto storage = base::MakeKVCacheStorageSpec(dtype, storage_mode);
  const int64_t elem = static_cast<int64_t>(base::DataTypeSize(storage.storage_dtype));
  if (elem <= 0 || block_size <= 0 || kv_head_num <= 0 || head_size <= 0) return 0;
  const int64_t rows = static_cast<int64_t>(2) * block_size * kv_head_num;
  int64_t bytes = rows * head_size * elem;
  if (storage.has_scales()) bytes += rows * static_cast<int64_t>(base::DataTypeSize(storage.scale_dtype));
  return bytes;
}

bool KVPoolDescriptor::compatible_with(const KVPoolDescriptor& o) const {
  return layer_num == o.layer_num && block_size == o.block_size && kv_head_num == o.kv_head_num &&
         head_size == o.head_size && dtype == o.dtype && storage_mode == o.storage_mode;
}

base::Status KVBlockManifest::validate() const {
  using base::error::InvalidArgument;
  if (client_request_id.empty()) return InvalidArgument("pd handoff manifest missing client_request_id");
  if (!handoff_id.valid()) return InvalidArgument("pd handoff manifest missing handoff_id");
  if (prompt_tokens <= 0) return InvalidArgument("pd handoff manifest prompt_tokens must be positive");
  if (computed_tokens <= 0 || computed_tokens > prompt_tokens)
    return InvalidArgument("pd handoff manifest computed_tokens is invalid");
  if (!src_pool.compatible_with(dst_pool))
    return InvalidArgument("pd handoff source/destination KV pools are incompatible");
  if (src_pool.layer_num <= 0) return InvalidArgument("pd handoff KV pool layer_num must be positive");
  if (static_cast<int32_t>(layer_mappings.size()) != src_pool.layer_num)
    return InvalidArgument("pd handoff layer mapping count does not match layer_num");
  for (const auto& m : layer_mappings) {
    if (m.layer_idx < 0 || m.layer_idx >= src_pool.layer_num)
      return InvalidArgument("pd handoff layer_idx out of range");
    if (m.src_block_ids.size() != m.dst_block_ids.size())
      return InvalidArgument("pd handoff src/dst block mapping size mismatch");
    if (m.src_block_ids.empty()) return InvalidArgument("pd handoff block mapping cannot be empty");
  }
  return base::error::Success();
}

KVTransferStatus KVTransferStatus::Pending() { return {KVTransferState::kPending, ""}; }
KVTransferStatus KVTransferStatus::Completed() { return {KVTransferState::kCompleted, ""}; }
KVTransferStatus KVTransferStatus::Failed(std::string m) { return {KVTransferState::kFailed, std::move(m)}; }
KVTransferStatus KVTransferStatus::Cancelled(std::string m) {
  return {KVTransferState::kCancelled, std::move(m)};
}
bool KVTransferStatus::done() const { return state != KVTransferState::kPending; }
bool KVTransferStatus::ok() const { return state == KVTransferState::kCompleted; }

}  // namespace serving
