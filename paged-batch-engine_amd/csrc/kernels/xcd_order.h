// Workgroup renumbering for MI355X's eight XCDs. Header-only and constexpr,
// so the kernels call it on the device and the host tests check it.
#pragma once
#include <stdint.h>

namespace pbe {

// MI355X dispatches workgroup b of a launch to XCD b % 8. Each XCD has its
// own L2 and each CU its own address-translation cache.
constexpr uint32_t kXcds = 8;

// The slice-order position of workgroup `b` of `nb` when each XCD takes `g`
// consecutive workgroups' slices in turn: rounds of kXcds * g workgroups, XCD
// x taking positions [x*g, x*g + g) of each round. The trailing partial round
// keeps its own numbering. A bijection on [0, nb) for every nb and g >= 1.
//
// In dispatch order, consecutive slices land on different XCDs, so every XCD
// reads and writes in every run in flight; in groups, each XCD streams
// through its own stretch of the plan. Measured, not derived: on MI355X the
// scattered plans (configs 3 and 5) run 3-6% faster, while rocprofv3 shows
// the same UTCL1 translation misses (config 2: 2,090-2,189 per launch
// against 2,256 in dispatch order) and 2-4% more DRAM requests in flight.
constexpr uint32_t xcd_grouped(uint32_t b, uint32_t nb, uint32_t g) {
  const uint32_t round = kXcds * g;
  const uint32_t tail = nb / round * round;
  if (b >= tail) return b;
  const uint32_t x = b % kXcds, k = b / kXcds;
  return k / g * round + x * g + k % g;
}

}  // namespace pbe
