// CPU check of the kernels' workgroup -> work-item maps (ffa_grid.h, the code the
// prefill and backward kernels run): for every grid shape of a sweep that includes
// each BASELINE configuration, the map the launcher selects must send the workgroup
// ids [0, grid) one-to-one onto the (unit, tile) pairs, so no output tile is left
// unwritten and none is written twice. Built with g++ by tests/test_grid_maps.py.
//
// Usage: grid_check  -> prints "grid_check ok: <n> grids" or the first failure, and
// exits 0 / 1.

#include <cstdio>
#include <vector>

#include "ffa_grid.h"

namespace {

long g_checked = 0;

template <typename Map>
bool check(const char* what, int n_units, int n_t, int group, int remap, Map map) {
  const long grid = static_cast<long>(n_units) * n_t;
  std::vector<unsigned char> seen(static_cast<size_t>(grid), 0);
  for (long bid = 0; bid < grid; ++bid) {
    int u = -1;
    int j = -1;
    map(static_cast<int>(bid), static_cast<int>(grid), u, j);
    if (u < 0 || u >= n_units || j < 0 || j >= n_t) {
      std::printf("%s: units %d tiles %d group %d remap %d: id %ld -> (%d, %d) out of range\n",
                  what, n_units, n_t, group, remap, bid, u, j);
      return false;
    }
    unsigned char& s = seen[static_cast<size_t>(u) * n_t + j];
    if (s) {
      std::printf("%s: units %d tiles %d group %d remap %d: (%d, %d) hit twice (id %ld)\n",
                  what, n_units, n_t, group, remap, u, j, bid);
      return false;
    }
    s = 1;
  }
  ++g_checked;
  return true;  // grid ids and pairs are equally many: injective means bijective
}

bool check_prefill(int n_units, int n_qt, bool causal) {
  int group = 0;
  int remap = 0;
  ffa::prefill_grid_order(causal, n_units, static_cast<int64_t>(n_units) * n_qt, group, remap);
  return check("prefill", n_units, n_qt, group, remap, [&](int bid, int grid, int& u, int& j) {
    ffa::prefill_work_item(bid, grid, n_qt, group, remap, u, j);
  });
}

// the backward grids: the prefill map, chosen per launch as the prefill's is, over the
// dK/dV grid's (batch x kv-head, key tile) and the dQ grid's (batch x q-head, row tile)
bool check_bwd(int n_units, int n_t, bool causal) {
  int group = 0;
  int remap = 0;
  ffa::prefill_grid_order(causal, n_units, static_cast<int64_t>(n_units) * n_t, group, remap);
  return check("backward", n_units, n_t, group, remap, [&](int bid, int grid, int& u, int& j) {
    ffa::prefill_work_item(bid, grid, n_t, group, remap, u, j);
  });
}

}  // namespace

int main() {
  // (units, tiles) of the BASELINE configurations at 128 rows / keys per workgroup:
  // cfg1 B2 H8 S1024, cfg2 B4 H32 S4096, north star B4 H32 S8192, cfg3 B2 Hq32 (Hkv 8
  // for the dK/dV grid) S8192, cfg5 B2 H32 S4096.
  const int baseline[][2] = {{16, 8}, {128, 32}, {128, 64}, {64, 64}, {16, 64}, {64, 32}};
  for (const auto& c : baseline) {
    for (bool causal : {false, true}) {
      if (!check_prefill(c[0], c[1], causal) || !check_bwd(c[0], c[1], causal)) return 1;
    }
  }
  // every unit count up to 96 (each residue mod 8 and mod 16, groups of one unit per
  // XCD and of odd sizes) against every tile count up to 70, plus large grids
  for (int units = 1; units <= 96; ++units) {
    for (int tiles = 1; tiles <= 70; ++tiles) {
      for (bool causal : {false, true}) {
        if (!check_prefill(units, tiles, causal) || !check_bwd(units, tiles, causal)) return 1;
      }
    }
  }
  const int big[][2] = {{256, 64}, {512, 128}, {1024, 33}, {4096, 2}, {8, 1024}, {24, 129},
                        {160, 130}, {1000, 7}};
  for (const auto& c : big) {
    for (bool causal : {false, true}) {
      if (!check_prefill(c[0], c[1], causal) || !check_bwd(c[0], c[1], causal)) return 1;
    }
  }
  std::printf("grid_check ok: %ld grids\n", g_checked);
  return 0;
}
