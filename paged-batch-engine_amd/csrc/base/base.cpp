#include "base/base.h"

#include <utility>

namespace base {

size_t DataTypeSize(DataType data_type) {
  switch (data_type) {
    case DataType::kDataTypeFp32: return 4;
    case DataType::kDataTypeInt8: return 1;
    case DataType::kDataTypeInt32: return 4;
    case DataType::kDataTypeBf16: return 2;
    default: return 0;
  }
}

Status::Status(int code, std::string err_message) : code_(code), message_(std::move(err_message)) {}

Status& Status::operator=(int code) {
  code_ = code;
  return *this;
}

namespace error {
Status Success(const std::string& m) { return Status(kSuccess, m); }
Status FunctionNotImplement(const std::string& m) { return Status(kFunctionUnImplement, m); }
Status PathNotValid(const std::string& m) { return Status(kPathNotValid, m); }
Status ModelParseError(const std::string& m) { return Status(kModelParseError, m); }
Status InternalError(const std::string& m) { return Status(kInternalError, m); }
Status KeyHasExits(const std::string& m) { return Status(kKeyValueHasExist, m); }
Status InvalidArgument(const std::string& m) { return Status(kInvalidArgument, m); }
}  // namespace error

std::ostream& operator<<(std::ostream& os, const Status& x) { return os << x.get_err_msg(); }

std::ostream& operator<<(std::ostream& os, DeviceType x) {
  switch (x) {
    case DeviceType::kDeviceCPU: return os << "cpu";
    case DeviceType::kDeviceCUDA: return os << "cuda";
    case DeviceType::kDeviceHIP: return os << "hip";
    case DeviceType::kDeviceTPU: return os << "tpu";
    default: return os << "unknown";
  }
}

std::ostream& operator<<(std::ostream& os, DataType x) {
  switch (x) {
    case DataType::kDataTypeFp32: return os << "fp32";
    case DataType::kDataTypeInt8: return os << "int8";
    case DataType::kDataTypeInt32: return os << "int32";
    case DataType::kDataTypeBf16: return os << "bf16";
    default: return os << "unknown";
  }
}

}  // namespace base

#include "base/kv_cache_format.h"

namespace base {

const char* BlockStorageModeName(BlockStorageMode storage_mode) {
  switch (storage_mode) {
    case BlockStorageMode::kPlain: return "plain";
    case BlockStorageMode::kFp8E4M3PerTokenHead: return "fp8_e4m3_per_token_head";
  }
  return "unknown";
}

KVCacheStorageSpec MakeKVCacheStorageSpec(DataType logical_dtype, BlockStorageMode storage_mode) {
  KVCacheStorageSpec spec;
  spec.storage_mode = storage_mode;
  spec.logical_dtype = logical_dtype;
  const bool fp8 = storage_mode == BlockStorageMode::kFp8E4M3PerTokenHead;
  spec.storage_dtype = fp8 ? DataType::kDataTypeInt8 : logical_dtype;
  spec.scale_dtype = fp8 ? DataType::kDataTypeFp32 : DataType::kDataTypeUnknown;
  return spec;
}

Status ValidateKVCacheStorageSpec(const KVCacheStorageSpec& spec, DeviceType device_type,
                                  DataType runtime_data_type) {
  if (spec.logical_dtype == DataType::kDataTypeUnknown ||
      spec.storage_dtype == DataType::kDataTypeUnknown)
    return error::InternalError("KV cache storage spec is incomplete.");
  switch (spec.storage_mode) {
    case BlockStorageMode::kPlain:
      if (spec.storage_dtype != spec.logical_dtype || spec.has_scales())
        return error::InternalError("Plain KV cache spec must use runtime dtype without scales.");
      return error::Success();
    case BlockStorageMode::kFp8E4M3PerTokenHead:
      if (device_type != DeviceType::kDeviceHIP && device_type != DeviceType::kDeviceCUDA)
        return error::InternalError("FP8 KV cache is only supported on GPU devices.");
      if (runtime_data_type != DataType::kDataTypeBf16 ||
          spec.logical_dtype != DataType::kDataTypeBf16)
        return error::InternalError("FP8 KV cache requires BF16 runtime.");
      if (spec.storage_dtype != DataType::kDataTypeInt8 ||
          spec.scale_dtype != DataType::kDataTypeFp32)
        return error::InternalError("FP8 KV cache spec must use int8 storage and fp32 scales.");
      return error::Success();
  }
  return error::InternalError("Unsupported KV cache storage mode.");
}

size_t KVCacheBytesPerToken(const KVCacheStorageSpec& spec, int32_t layer_num, int32_t kv_head_num,
                            int32_t head_size) {
  const size_t planes = 2u * static_cast<size_t>(layer_num) * static_cast<size_t>(kv_head_num);
  size_t bytes = planes * static_cast<size_t>(head_size) * DataTypeSize(spec.storage_dtype);
  if (spec.has_scales()) bytes += planes * DataTypeSize(spec.scale_dtype);
  return bytes;
}

}  // namespace base
