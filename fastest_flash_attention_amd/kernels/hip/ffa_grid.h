// Workgroup -> work-item maps of the prefill and backward grids, and the host-side
// choice of map for a launch. Plain integer C++: the functions are constexpr, so the
// kernels call them on the device (clang compiles constexpr functions for host and
// device) and tests/hip/grid_check.cpp, built by g++, checks on the CPU that every map
// the launchers select is a bijection from workgroup ids onto (unit, tile) pairs.
//
// The hardware deals linear workgroup ids round-robin to the 8 XCDs of MI355X
// (id % 8 = XCD); each XCD has its own L2, so the maps keep a unit's tiles (one
// (batch, head): the K/V, or Q/dO, they share) on one XCD.
#pragma once

#include <stdint.h>

namespace ffa {

// Prefill: grid = n_units * n_qt workgroups, unit = batch x q-head, jq = query tile
// (jq = 0 is the heaviest causal tile). With xcd_group = G > 0 (needs n_units % 8 ==
// 0), XCD x owns units [x HX, (x + 1) HX) (HX = n_units / 8) and runs them one after
// another, heaviest tile first, except its last min(HX, G) units, whose tiles run
// interleaved (tile j of each in turn), so the launch ends on light tiles instead of
// the last unit's heaviest tiles starting near the end. Without a group, xcd_remap
// (needs grid % 8 == 0) places consecutive ids on one XCD; otherwise ids map in order.
constexpr void prefill_work_item(int bid, int grid, int n_qt, int xcd_group, int xcd_remap,
                                 int& unit, int& jq) {
  if (xcd_group > 0) {
    const int hx = (grid / n_qt) >> 3;
    const int x = bid & 7;
    const int k = bid >> 3;
    const int gl = hx < xcd_group ? hx : xcd_group;
    const int k0 = (hx - gl) * n_qt;  // tiles of the units run one after another
    if (k < k0) {
      const int u = k / n_qt;
      unit = x * hx + u;
      jq = k - u * n_qt;
    } else {
      const int r = k - k0;
      jq = r / gl;
      unit = x * hx + (hx - gl) + (r - jq * gl);
    }
    return;
  }
  if (xcd_remap) {
    const int per_xcd = grid >> 3;
    bid = (bid & 7) * per_xcd + (bid >> 3);
  }
  unit = bid / n_qt;
  jq = bid - unit * n_qt;
}

// The prefill launcher's choice: causal grids (whose tiles differ in weight) with
// n_units % 8 == 0 interleave the last units of each XCD: all of them when an XCD has at
// most 8 (cfg3 and cfg5: 64 units), else the last four for units of at most 32 tiles
// (cfg2) and the last two for longer ones (the north star). On MI355X, over unit after
// unit: +2-3 % at S = 8192 and +4-8 % at S = 4096 for the last two; then all 8 +2 % at
// cfg3 and +3.5 % at cfg5, the last four +1.5 % at cfg2 (-0.5 % at the north star,
// all 16 there -2.6 %). Other grids that split evenly over the XCDs keep consecutive
// ids on one XCD.
constexpr void prefill_grid_order(bool causal, int64_t n_units, int64_t grid, int& xcd_group,
                                  int& xcd_remap) {
  xcd_remap = (grid % 8 == 0) ? 1 : 0;
  const int64_t n_qt = n_units > 0 ? grid / n_units : 0;
  xcd_group = (causal && n_units % 8 == 0) ? (n_units / 8 <= 8 ? 8 : (n_qt <= 32 ? 4 : 2)) : 0;
}

// The backward's dK/dV and dQ grids (unit = batch x head, tile j = 0 the heaviest causal
// tile) use the same map and the same launcher choice as the prefill.

}  // namespace ffa
