// Page index of a page-major block id: id / stride for an id that is a
// multiple of stride (2 * layers), else -1, without a hardware division: the
// quotient is (id * mul) >> shift with shift = 32 + ceil(log2 stride) and
// mul = floor(2^shift / stride) + 1, the round-up method for unsigned division
// by a constant, exact for every 32-bit id (checked exhaustively for every
// even stride up to 64). The reservation and retire paths index pages once per
// layer and id (8,820 times for a 315-page, 28-layer request).
#pragma once
#include <cstdint>

namespace base {

class PageIndex {
 public:
  PageIndex() = default;
  explicit PageIndex(int32_t stride) : stride_(stride) {
    int lg = 0;
    while ((int64_t{1} << lg) < stride) ++lg;
    shift_ = 32 + lg;
    mul_ = (uint64_t{1} << shift_) / static_cast<uint64_t>(stride) + 1;
  }
  int32_t stride() const { return stride_; }
  // id / stride for a non-negative multiple of stride, else -1.
  int32_t of(int32_t id) const {
    if (id < 0) return -1;
    const int32_t k = static_cast<int32_t>((static_cast<uint64_t>(id) * mul_) >> shift_);
    return k * stride_ == id ? k : -1;
  }

 private:
  int32_t stride_ = 1;
  uint64_t mul_ = uint64_t{1} << 32;  // stride 1: the id itself
  int shift_ = 32;
};

}  // namespace base
