// Compact KV page-list wire form over the C ABI codec (pbe_page_list_*).
#include "serving/kv_page_wire.h"

#include "pbe_handoff.h"

namespace serving {
namespace {
using base::error::InvalidArgument;
}  // namespace

base::Status EncodeKVPageList(uint64_t shared_arena_epoch,
                              const std::vector<RemoteKVLayerPayload>& layers, std::string* wire) {
  if (wire == nullptr) return InvalidArgument("page list output is null");
  wire->clear();
  if (layers.empty()) return InvalidArgument("PD layer count mismatch");
  const auto& first = layers.front().src_block_ids;
  for (size_t i = 0; i < layers.size(); ++i) {
    if (layers[i].layer_idx != static_cast<int32_t>(i)) return InvalidArgument("PD shared layout mismatch");
    if (i > 0 && layers[i].src_block_ids != first) return InvalidArgument("PD page-major layer IDs disagree");
  }
  const int32_t n_layers = static_cast<int32_t>(layers.size());
  const uint64_t bytes = pbe_page_list_bytes(first.data(), static_cast<int64_t>(first.size()), n_layers);
  if (bytes == 0) return InvalidArgument("PD source block outside shared page layout");
  wire->resize(bytes);
  uint64_t written = 0;
  if (pbe_page_list_encode(first.data(), static_cast<int64_t>(first.size()), n_layers, shared_arena_epoch,
                           &(*wire)[0], bytes, &written) != PBE_OK) {
    wire->clear();
    return InvalidArgument(pbe_last_error());
  }
  return base::error::Success();
}

base::Status DecodeKVPageIds(const std::string& wire, uint64_t* shared_arena_epoch, int32_t* layers,
                             std::vector<int32_t>* ids, int64_t max_pages) {
  if (!shared_arena_epoch || !layers || !ids) return InvalidArgument("page list output is null");
  int64_t n = 0;
  if (pbe_page_list_decode(wire.data(), wire.size(), nullptr, 0, &n, layers, shared_arena_epoch) != PBE_OK)
    return InvalidArgument(pbe_last_error());
  if (n > max_pages)
    return InvalidArgument("page list claims " + std::to_string(n) + " pages, more than the " +
                           std::to_string(max_pages) + " allowed");
  ids->assign(static_cast<size_t>(n), 0);
  if (pbe_page_list_decode(wire.data(), wire.size(), ids->data(), n, &n, layers, shared_arena_epoch) !=
      PBE_OK) {
    ids->clear();
    return InvalidArgument(pbe_last_error());
  }
  return base::error::Success();
}

base::Status DecodeKVPageList(const std::string& wire, uint64_t* shared_arena_epoch,
                              std::vector<RemoteKVLayerPayload>* layers, int64_t max_pages) {
  if (layers == nullptr) return InvalidArgument("page list output is null");
  layers->clear();
  int32_t n_layers = 0;
  std::vector<int32_t> ids;
  base::Status status = DecodeKVPageIds(wire, shared_arena_epoch, &n_layers, &ids, max_pages);
  if (!status) return status;
  layers->resize(static_cast<size_t>(n_layers));
  for (int32_t l = 0; l < n_layers; ++l) {
    (*layers)[l].layer_idx = l;
    (*layers)[l].src_block_ids = ids;
  }
  return base::error::Success();
}

}  // namespace serving
