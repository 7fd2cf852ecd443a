// KV page storage description (plain BF16 or FP8 E4M3 with per-(token, head)
// fp32 scales). Same enum values and field meaning as the reference
// (infMain/include/base/kv_cache_format.h:10-52); FP8 pools are accepted on
// HIP devices here instead of CUDA.
#ifndef PBE_INCLUDE_BASE_KV_CACHE_FORMAT_H_
#define PBE_INCLUDE_BASE_KV_CACHE_FORMAT_H_

#include <cstddef>
#include <cstdint>

#include "base/base.h"

namespace base {

enum class BlockStorageMode : uint8_t {
  kPlain = 0,
  kFp8E4M3PerTokenHead = 1,
};

const char* BlockStorageModeName(BlockStorageMode storage_mode);

struct KVCacheStorageSpec {
  BlockStorageMode storage_mode = BlockStorageMode::kPlain;
  DataType logical_dtype = DataType::kDataTypeUnknown;
  DataType storage_dtype = DataType::kDataTypeUnknown;
  DataType scale_dtype = DataType::kDataTypeUnknown;

  bool has_scales() const { return scale_dtype != DataType::kDataTypeUnknown; }
  bool uses_fp8_storage() const { return storage_mode == BlockStorageMode::kFp8E4M3PerTokenHead; }
};

// Plain: storage = logical, no scales. FP8: int8 payload + fp32 scales.
KVCacheStorageSpec MakeKVCacheStorageSpec(DataType logical_dtype, BlockStorageMode storage_mode);

// Rejects incomplete specs, plain specs with scales or converted payloads, and
// FP8 specs that are not BF16 -> int8 + fp32 on a GPU device.
Status ValidateKVCacheStorageSpec(const KVCacheStorageSpec& spec, DeviceType device_type,
                                  DataType runtime_data_type);

// Bytes of KV state one token occupies across all layers (payload + scales).
size_t KVCacheBytesPerToken(const KVCacheStorageSpec& spec, int32_t layer_num, int32_t kv_head_num,
                            int32_t head_size);

}  // namespace base

#endif  // PBE_INCLUDE_BASE_KV_CACHE_FORMAT_H_
