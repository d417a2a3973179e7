// Pieces of the gfx950 prefill kernels (ffa_prefill.hip): the launch parameter block, the LDS row swizzles of K/V tiles and the reference's
// per-tile 1e-30 floor of the softmax sum (the LSE of rows that see no key, and its
// share in rows that do).
#pragma once

#include "ffa_common.h"

namespace ffa {
namespace pf {

constexpr float kRescaleThresh = 8.0f;  // log2 units: the running max moves only past this
// 16-bit kernels: the running max moves when a 16-key chunk's 8 exponentials per lane sum
// past this (some p > 2^5), so every accumulated p stays <= 2^8.
constexpr float kChunkLimit = 256.0f;

struct PrefillParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int64_t l_sb, l_sh, l_ss;
  int B, Hq, Hkv, Sq, Skv, D;
  int Dv;  // V's head dim (<= D): O's dims past it are written as 0
  int q_offset, causal, window;
  int ratio;
  int n_qt;
  float score_mul;  // scale*log2e, or scale/softcap with softcap
  float cap_mul;    // softcap*log2e (softcap only)
  uint32_t q_neg;   // 1: Q's sign bits are flipped as it is loaded (negative scale)
  int ref_bq, ref_bkv;
  int masked_lse_mode;
  int xcd_remap;
  int xcd_group;  // > 0: how many last heads of each XCD run interleaved (work_item)
  const uint64_t* kmask;  // block mask expanded to keys, [n_br][kmask_words], or null
  int kmask_words;
  const int32_t* visited;  // reference tiles visited per row block (with kmask)
};

// Row swizzles (XOR on the 16-byte chunk index) of the K and V tiles in LDS. They make
// the 16 rows read together by a K operand load, and the 4 rows x 64 bytes read
// together by a transposed V load, land in distinct bank groups.
template <int DP>
__device__ inline int kswz(int r) {
  if constexpr (DP == 32) return (r >> 2) & 3;
  if constexpr (DP == 64 || DP == 192) return (r >> 1) & 7;
  return r & 15;
}
template <int DP>
__device__ inline int vswz(int r) {
  if constexpr (DP == 32) return 0;
  if constexpr (DP == 64 || DP == 192) return 4 * ((r >> 1) & 1);
  return 4 * (r & 3);
}

// The reference tiles (ref_bq x ref_bkv) that the reference loop visits for `row`'s row
// block (cpu_reference.py:215-231): the block mask's count per row block, or the
// causal / window range.
__device__ inline int ref_visited_tiles(const PrefillParams& p, int row) {
  if (p.kmask != nullptr) return p.visited[row / p.ref_bq];
  const int bq = p.ref_bq;
  const int bkv = p.ref_bkv;
  const int iq = row / bq;
  const int qs_abs = p.q_offset + iq * bq;
  const int qe_abs = p.q_offset + min((iq + 1) * bq, p.Sq);
  const int n_bc = (p.Skv + bkv - 1) / bkv;
  int j_hi = n_bc - 1;
  if (p.causal) {
    const int last = qe_abs - 1;
    j_hi = last < 0 ? -1 : min(j_hi, last / bkv);
  }
  int j_lo = 0;
  if (p.window > 0) {
    const int thr = qs_abs - p.window + 1;
    int j = (thr + 1 <= 0) ? 0 : (thr + bkv) / bkv - 1;
    if (j >= n_bc - 1) j = (p.Skv - 1 >= thr) ? n_bc - 1 : n_bc;
    j_lo = j;
  }
  return max(j_hi - j_lo + 1, 0);
}

// LSE of a row with no visible key, as the reference loop produces it: each visited
// tile floors its row sum at 1e-30 and adds it by logaddexp (cpu_reference.py:288-297),
// so n visited tiles give log(n) + log(1e-30); no visited tile leaves -inf.
__device__ inline float masked_row_lse(const PrefillParams& p, int row) {
  if (p.masked_lse_mode != 0) return kNegInf;
  const int n = ref_visited_tiles(p, row);
  return n > 0 ? logf(static_cast<float>(n)) + logf(1e-30f) : kNegInf;
}

// The same floor for a row that does see keys: every visited reference tile in which
// the row sees none adds 1e-30 to its softmax sum. The kernels add it at the end:
// lse becomes logaddexp(lse, log(k 1e-30)) and O is scaled by exp(lse_old - lse_new).
// It only shows where the row's own sum is below about k 1e-30 (every visible logit
// under about -69 + log k); elsewhere the correction is below fp32 resolution and is
// skipped without counting the tiles. Not with the two-pass LSE (masked_lse_mode),
// which the reference takes exactly.
__device__ inline void ref_tile_floor(const PrefillParams& p, int row, float& lse, float& inv) {
  // n < 2^31 tiles: log(n 1e-30) - lse <= -40 whenever lse > -8
  if (p.masked_lse_mode != 0 || lse > -8.0f) return;
  const int n = ref_visited_tiles(p, row);
  if (n <= 0 || logf(static_cast<float>(n)) + logf(1e-30f) - lse <= -40.0f) return;
  // visited tiles that hold a key this row sees: they all lie in [lo, hi] / ref_bkv
  const int qa = p.q_offset + row;
  const int lo = p.window > 0 ? max(0, qa - p.window + 1) : 0;
  const int hi = p.causal ? min(qa, p.Skv - 1) : p.Skv - 1;
  if (lo > hi) return;  // no visible key: the masked-row path
  const int bkv = p.ref_bkv;
  int seen = 0;
  if (p.kmask != nullptr) {
    // the key mask holds the block mask's bit at every key of a tile
    const uint64_t* mrow = p.kmask + static_cast<int64_t>(row / p.ref_bq) * p.kmask_words;
    for (int j = lo / bkv; j <= hi / bkv; ++j) {
      const int key = j * bkv;
      seen += static_cast<int>((mrow[key >> 6] >> (key & 63)) & 1u);
    }
  } else {
    seen = hi / bkv - lo / bkv + 1;
  }
  const int k = n - seen;
  if (k <= 0) return;
  const float e = expf(logf(static_cast<float>(k)) + logf(1e-30f) - lse);
  inv *= 1.0f / (1.0f + e);
  lse += log1pf(e);
}

}  // namespace pf
}  // namespace ffa
