// Logical description of one KV page as a set of components
// (layer, K|V|K-scale|V-scale, token count, head range, dtype). Drop-in for
// the reference's cache/page_schema.h (infMain/include/cache/page_schema.h:14-61).
#ifndef PBE_INCLUDE_CACHE_PAGE_SCHEMA_H_
#define PBE_INCLUDE_CACHE_PAGE_SCHEMA_H_

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "base/base.h"
#include "base/kv_cache_format.h"

namespace cache {

enum class ComponentKind : uint8_t {
  kKey = 0,
  kValue = 1,
  kKeyScale = 2,
  kValueScale = 3,
};

const char* ComponentKindName(ComponentKind kind);

struct ComponentDescriptor {
  int32_t layer = -1;
  ComponentKind kind = ComponentKind::kKey;
  int32_t token_count = 0;
  int32_t head_begin = 0;
  int32_t head_count = 0;
  int32_t elements_per_head = 0;
  base::DataType dtype = base::DataType::kDataTypeUnknown;

  // tokens * heads * elements_per_head, 0 on non-positive dims or overflow.
  size_t element_count() const;
  // element_count * dtype size, 0 on unknown dtype or overflow.
  size_t byte_size() const;
  // "layer:kind:tokens:head_begin:head_count:width:dtype", the identity used
  // for matching and ordering components.
  std::string semantic_key() const;
  bool operator==(const ComponentDescriptor& other) const;
};

// Hash over the same fields as semantic_key() and operator==, for maps keyed
// by component without building key strings.
struct ComponentDescriptorHash {
  size_t operator()(const ComponentDescriptor& c) const noexcept;
};

struct PageSchema {
  uint32_t version = 1;
  int32_t layer_count = 0;
  int32_t page_size = 0;
  int32_t kv_head_count = 0;
  int32_t head_size = 0;
  base::KVCacheStorageSpec storage;
  std::vector<ComponentDescriptor> components;

  // Every layer's K and V (and scales iff the storage has them) must be
  // covered by components whose head ranges tile [0, kv_head_count) exactly.
  base::Status validate() const;
  // Model-compute identity: version, dims and logical dtype only.
  std::string logical_fingerprint() const;
  // Physical identity: storage spec plus the sorted component keys.
  std::string fingerprint() const;
};

// One full-head-range component per (layer, K, V[, K-scale, V-scale]).
base::Status MakeKVPageSchema(uint32_t version, int32_t layer_count, int32_t page_size,
                              int32_t kv_head_count, int32_t head_size,
                              const base::KVCacheStorageSpec& storage, PageSchema* schema);

}  // namespace cache

#endif  // PBE_INCLUDE_CACHE_PAGE_SCHEMA_H_
