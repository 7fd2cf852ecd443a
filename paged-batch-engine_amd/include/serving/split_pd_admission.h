// Per-lane admission of split prefill/decode requests on the decode owner
// thread: the interface of the reference's serving::SplitPDAdmission
// (infMain/include/serving/split_pd_admission.h:8-41), which decides whether a
// handoff may reserve decode pages at all (split_pd_engine.cpp:275-291). Lane 0
// serves short outputs, lane 1 long ones; each has its own slot count and KV
// token budget, so one lane cannot starve the other.
#ifndef PBE_INCLUDE_SERVING_SPLIT_PD_ADMISSION_H_
#define PBE_INCLUDE_SERVING_SPLIT_PD_ADMISSION_H_

#include <array>
#include <cstdint>
#include <stdexcept>

namespace serving {

class SplitPDAdmission {
 public:
  // slots[lane]: requests a lane may hold at once; tokens[lane]: its KV budget.
  SplitPDAdmission(std::array<int, 2> slots, std::array<int64_t, 2> tokens) {
    for (int lane = 0; lane < 2; ++lane) {
      lanes_[lane].slots = slots[lane];
      lanes_[lane].budget = tokens[lane];
    }
  }

  // KV tokens a request will occupy once its output is complete: prompt plus
  // output, rounded up to whole pages of block_size tokens.
  static int64_t charge(int64_t prompt, int64_t output, int block_size) {
    const int64_t pages = (prompt + output + block_size - 1) / block_size;
    return pages * block_size;
  }

  // Whether a request of `tokens` could ever be admitted to `lane`.
  bool fits_request(int lane, int64_t tokens) const {
    const Lane& l = at(lane);
    return tokens > 0 && tokens <= l.budget;
  }
  // Whether it can be admitted now: a free slot and room in the budget.
  bool can_acquire(int lane, int64_t tokens) const {
    if (!fits_request(lane, tokens)) return false;
    const Lane& l = at(lane);
    return l.active < l.slots && tokens <= l.budget - l.used;
  }
  // Throws std::logic_error when can_acquire is false.
  void acquire(int lane, int64_t tokens) {
    if (!can_acquire(lane, tokens)) throw std::logic_error("split PD admission exceeded");
    Lane& l = at(lane);
    l.active += 1;
    l.used += tokens;
  }
  // Throws std::logic_error when the lane holds no request or fewer tokens.
  void release(int lane, int64_t tokens) {
    Lane& l = at(lane);
    if (l.active == 0 || tokens > l.used) throw std::logic_error("split PD admission double release");
    l.active -= 1;
    l.used -= tokens;
  }
  int active(int lane) const { return at(lane).active; }
  int64_t used(int lane) const { return at(lane).used; }

 private:
  struct Lane {
    int slots = 0, active = 0;
    int64_t budget = 0, used = 0;
  };
  // Lanes are 0 and 1; any other index throws std::out_of_range.
  Lane& at(int lane) {
    if (lane < 0 || lane > 1) throw std::out_of_range("split PD admission lane");
    return lanes_[lane];
  }
  const Lane& at(int lane) const {
    if (lane < 0 || lane > 1) throw std::out_of_range("split PD admission lane");
    return lanes_[lane];
  }
  Lane lanes_[2];
};

}  // namespace serving

#endif  // PBE_INCLUDE_SERVING_SPLIT_PD_ADMISSION_H_
