// Validation rules follow infMain/source/cache/page_schema.cpp:84-170; the
// fingerprint text formats follow :172-199 so identities match across builds.
#include "cache/page_schema.h"

#include <cstdio>

#include <algorithm>
#include <array>
#include <limits>
#include <sstream>
#include <unordered_set>
#include <utility>

namespace cache {
namespace {

bool is_scale(ComponentKind kind) {
  return kind == ComponentKind::kKeyScale || kind == ComponentKind::kValueScale;
}

bool known_kind(ComponentKind kind) { return static_cast<uint8_t>(kind) <= 3; }

// Multiplies with overflow detection; returns 0 on overflow.
size_t checked_mul(size_t a, size_t b) {
  if (a != 0 && b > std::numeric_limits<size_t>::max() / a) return 0;
  return a * b;
}

}  // namespace

const char* ComponentKindName(ComponentKind kind) {
  switch (kind) {
    case ComponentKind::kKey: return "key";
    case ComponentKind::kValue: return "value";
    case ComponentKind::kKeyScale: return "key_scale";
    case ComponentKind::kValueScale: return "value_scale";
  }
  return "unknown";
}

size_t ComponentDescriptor::element_count() const {
  if (token_count <= 0 || head_count <= 0 || elements_per_head <= 0) return 0;
  return checked_mul(checked_mul(static_cast<size_t>(token_count), static_cast<size_t>(head_count)),
                     static_cast<size_t>(elements_per_head));
}

size_t ComponentDescriptor::byte_size() const {
  const size_t width = base::DataTypeSize(dtype);
  if (width == 0) return 0;
  return checked_mul(element_count(), width);
}

std::string ComponentDescriptor::semantic_key() const {
  char buf[96];
  const int n = std::snprintf(buf, sizeof(buf), "%d:%d:%d:%d:%d:%d:%d", (int)layer, (int)kind,
                              (int)token_count, (int)head_begin, (int)head_count,
                              (int)elements_per_head, (int)dtype);
  return std::string(buf, (size_t)n);
}

size_t ComponentDescriptorHash::operator()(const ComponentDescriptor& c) const noexcept {
  uint64_t h = 1469598103934665603ull;  // FNV-1a over the seven fields
  const int64_t f[7] = {c.layer, (int64_t)c.kind, c.token_count, c.head_begin, c.head_count,
                        c.elements_per_head, (int64_t)c.dtype};
  for (int64_t v : f) {
    h ^= (uint64_t)v;
    h *= 1099511628211ull;
  }
  return (size_t)h;
}

bool ComponentDescriptor::operator==(const ComponentDescriptor& o) const {
  return layer == o.layer && kind == o.kind && token_count == o.token_count &&
         head_begin == o.head_begin && head_count == o.head_count &&
         elements_per_head == o.elements_per_head && dtype == o.dtype;
}

base::Status PageSchema::validate() const {
  using base::error::InvalidArgument;
  if (version == 0 || layer_count <= 0 || page_size <= 0 || kv_head_count <= 0 || head_size <= 0)
    return InvalidArgument("Page schema dimensions and version must be positive.");
  if (storage.logical_dtype == base::DataType::kDataTypeUnknown ||
      storage.storage_dtype == base::DataType::kDataTypeUnknown)
    return InvalidArgument("Page schema storage spec is incomplete.");
  switch (storage.storage_mode) {
    case base::BlockStorageMode::kPlain:
      if (storage.storage_dtype != storage.logical_dtype || storage.has_scales())
        return InvalidArgument("Plain page storage must use logical dtype without scales.");
      break;
    case base::BlockStorageMode::kFp8E4M3PerTokenHead:
      if (storage.logical_dtype != base::DataType::kDataTypeBf16 ||
          storage.storage_dtype != base::DataType::kDataTypeInt8 ||
          storage.scale_dtype != base::DataType::kDataTypeFp32)
        return InvalidArgument("FP8 page storage requires BF16 logical, int8 payload, and fp32 scales.");
      break;
    default:
      return InvalidArgument("Page schema storage mode is unsupported.");
  }

  // Head ranges seen per (layer, kind).
  std::vector<std::array<std::vector<std::pair<int32_t, int32_t>>, 4>> heads(
      static_cast<size_t>(layer_count));
  std::unordered_set<ComponentDescriptor, ComponentDescriptorHash> keys;
  for (const ComponentDescriptor& c : components) {
    if (c.layer < 0 || c.token_count <= 0 || c.head_begin < 0 || c.head_count <= 0 ||
        c.elements_per_head <= 0 || c.dtype == base::DataType::kDataTypeUnknown ||
        !known_kind(c.kind))
      return InvalidArgument("Component descriptor has an invalid shape or dtype.");
    if (c.byte_size() == 0) return InvalidArgument("Component byte size is zero or overflows size_t.");
    if (c.layer >= layer_count || c.token_count != page_size || c.head_begin > kv_head_count ||
        c.head_count > kv_head_count - c.head_begin)
      return InvalidArgument("Page component lies outside the schema head coverage.");
    const bool scale = is_scale(c.kind);
    const base::DataType want_dtype = scale ? storage.scale_dtype : storage.storage_dtype;
    if (want_dtype == base::DataType::kDataTypeUnknown || c.dtype != want_dtype ||
        c.elements_per_head != (scale ? 1 : head_size))
      return InvalidArgument("Page component shape or dtype disagrees with storage.");
    if (scale && !storage.has_scales())
      return InvalidArgument("Plain storage must not contain scale components.");
    if (!keys.insert(c).second)
      return InvalidArgument("Page schema contains a duplicate component.");
    heads[static_cast<size_t>(c.layer)][static_cast<size_t>(c.kind)].emplace_back(
        c.head_begin, c.head_begin + c.head_count);
  }

  const size_t kinds_needed = storage.has_scales() ? 4 : 2;
  for (auto& per_layer : heads) {
    for (size_t kind = 0; kind < 4; ++kind) {
      auto& ranges = per_layer[kind];
      if (kind >= kinds_needed) {
        if (!ranges.empty())
          return InvalidArgument("Page schema contains scales for a representation without scales.");
        continue;
      }
      std::sort(ranges.begin(), ranges.end());
      int32_t next = 0;
      for (const auto& r : ranges) {
        if (r.first != next) return InvalidArgument("Page schema head coverage is missing or overlapping.");
        next = r.second;
      }
      if (next != kv_head_count)
        return InvalidArgument("Page schema is missing required K/V/scale head coverage.");
    }
  }
  return base::error::Success();
}

std::string PageSchema::logical_fingerprint() const {
  std::ostringstream out;
  out << version << '|' << layer_count << '|' << page_size << '|' << kv_head_count << '|'
      << head_size << '|' << static_cast<int>(storage.logical_dtype);
  return out.str();
}

std::string PageSchema::fingerprint() const {
  std::vector<std::string> keys;
  keys.reserve(components.size());
  size_t total = 64;
  for (const auto& c : components) {
    keys.push_back(c.semantic_key());
    total += keys.back().size() + 1;
  }
  std::sort(keys.begin(), keys.end());
  char head[128];
  const int n = std::snprintf(head, sizeof(head), "%u|%d|%d|%d|%d|%d|%d|%d|%d", (unsigned)version,
                              (int)layer_count, (int)page_size, (int)kv_head_count, (int)head_size,
                              static_cast<int>(storage.storage_mode),
                              static_cast<int>(storage.logical_dtype),
                              static_cast<int>(storage.storage_dtype),
                              static_cast<int>(storage.scale_dtype));
  std::string out;
  out.reserve(total);
  out.append(head, (size_t)n);
  for (const auto& k : keys) {
    out.push_back('|');
    out += k;
  }
  return out;
}

base::Status MakeKVPageSchema(uint32_t version, int32_t layer_count, int32_t page_size,
                              int32_t kv_head_count, int32_t head_size,
                              const base::KVCacheStorageSpec& storage, PageSchema* schema) {
  if (schema == nullptr) return base::error::InvalidArgument("Page schema output is null.");
  PageSchema built;
  built.version = version;
  built.layer_count = layer_count;
  built.page_size = page_size;
  built.kv_head_count = kv_head_count;
  built.head_size = head_size;
  built.storage = storage;
  const ComponentKind kinds[4] = {ComponentKind::kKey, ComponentKind::kValue,
                                  ComponentKind::kKeyScale, ComponentKind::kValueScale};
  const int n_kinds = storage.has_scales() ? 4 : 2;
  for (int32_t layer = 0; layer < layer_count; ++layer)
    for (int k = 0; k < n_kinds; ++k) {
      const bool scale = k >= 2;
      built.components.push_back({layer, kinds[k], page_size, 0, kv_head_count,
                                  scale ? 1 : head_size,
                                  scale ? storage.scale_dtype : storage.storage_dtype});
    }
  base::Status status = built.validate();
  if (!status) return status;
  *schema = std::move(built);
  return base::error::Success();
}

}  // namespace cache
