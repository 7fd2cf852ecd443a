// Core value types of the drop-in API: device/data type enums and the Status
// result used by every fallible call. Names, values and conversions match the
// reference's base/base.h (infMain/include/base/base.h:52-186) so callers of
// the reference compile unchanged; logging macros are not part of this layer.
#ifndef PBE_INCLUDE_BASE_BASE_H_
#define PBE_INCLUDE_BASE_BASE_H_

#include <cstddef>
#include <cstdint>
#include <ostream>
#include <string>

namespace base {

enum class DeviceType : uint8_t {
  kDeviceUnknown = 0,
  kDeviceCPU = 1,
  kDeviceCUDA = 2,
  kDeviceHIP = 3,
  kDeviceTPU = 4,
};

enum class DataType : uint8_t {
  kDataTypeUnknown = 0,
  kDataTypeFp32 = 1,
  kDataTypeInt8 = 2,
  kDataTypeInt32 = 3,
  kDataTypeBf16 = 4,
};

// Element size in bytes; 0 for kDataTypeUnknown.
size_t DataTypeSize(DataType data_type);

enum StatusCode : uint8_t {
  kSuccess = 0,
  kFunctionUnImplement = 1,
  kPathNotValid = 2,
  kModelParseError = 3,
  kInternalError = 5,
  kKeyValueHasExist = 6,
  kInvalidArgument = 7,
};

// Result of a fallible call. Converts to true exactly when the code is
// kSuccess, and to the integer code.
class Status {
 public:
  Status(int code = StatusCode::kSuccess, std::string err_message = "");
  Status(const Status& other) = default;
  Status& operator=(const Status& other) = default;
  Status& operator=(int code);
  bool operator==(int code) const { return code_ == code; }
  bool operator!=(int code) const { return code_ != code; }
  operator int() const { return code_; }
  operator bool() const { return code_ == kSuccess; }
  int32_t get_err_code() const { return code_; }
  const std::string& get_err_msg() const { return message_; }
  void set_err_msg(const std::string& err_msg) { message_ = err_msg; }

 private:
  int code_ = StatusCode::kSuccess;
  std::string message_;
};

namespace error {
Status Success(const std::string& err_msg = "");
Status FunctionNotImplement(const std::string& err_msg = "");
Status PathNotValid(const std::string& err_msg = "");
Status ModelParseError(const std::string& err_msg = "");
Status InternalError(const std::string& err_msg = "");
Status KeyHasExits(const std::string& err_msg = "");
Status InvalidArgument(const std::string& err_msg = "");
}  // namespace error

std::ostream& operator<<(std::ostream& os, const Status& x);
std::ostream& operator<<(std::ostream& os, DeviceType x);
std::ostream& operator<<(std::ostream& os, DataType x);

}  // namespace base

#endif  // PBE_INCLUDE_BASE_BASE_H_
