// Attention backward (recompute from q, k, v, O, LSE) for gfx950.
//
// Semantics follow flash_attn_cpu_backward (reference kernels/cpu_reference.py:319-427):
//   P    = exp(S - lse)               S = softcap(q.k * scale) with the forward's masks
//   D_i  = rowsum(dO * O)             (O as stored by the forward, fp32 sum)
//   dV   = P^T dO
//   dS   = P * (dO V^T - D_i)         times (1 - tanh^2(q.k * scale / cap)) with softcap
//   dQ   = scale * dS K,   dK = scale * dS^T Q
// GQA (q head h reads kv head h / ratio) is reduced inside the kernel: dK / dV of a KV
// head sum over the q heads of its group. A row whose LSE is -inf (no visible key in
// the two-pass forward) contributes nothing (P = 0).
//
// Three launches on the caller's stream, no atomics (results are run-to-run
// deterministic):
//   1. bwd_pre_kernel   lse2 = lse * log2e (+inf for -inf rows and the padding rows up
//                       to the next 128-row boundary) and D_i, both fp32, into the
//                       workspace [B * Hq][Sq_pad].
//   2. bwd_dkdv_kernel  keys stationary: one workgroup (4 waves) per 128 keys of one
//                       (batch, kv head); each wave holds 32 keys' K and V rows as MFMA
//                       B operands and their dK^T / dV^T accumulators in registers, and
//                       sweeps 32-row tiles of Q, dO, lse2, D_i of every q head of its
//                       group (direct global -> LDS loads, double-buffered):
//                         S  = Q K^T, dP = dO V^T      lane l holds key l % 32
//                         dV^T += dO^T P, dK^T += Q^T dS   A = ds_read_b64_tr_b16 of the
//                         Q / dO tile, B = P / dS packed from the accumulators
//   3. bwd_dq_kernel    queries stationary: one workgroup per 128 query rows of one
//                       (batch, q head), the forward kernel's decomposition; per 64-key
//                       tile S^T = K Q^T, dP^T = V dO^T (lane = query, lse2 / D_i in
//                       one register each), dQ^T += K^T dS^T with K^T transposed-read
//                       from the same LDS tile.
// The Q / dO (kernel 2) and K (kernel 3) tiles are read both row-wise (MFMA A rows)
// and transposed; one XOR swizzle of the 16-byte chunk index keeps both access forms
// free of LDS bank conflicts.
// P and dS are rounded to the input's 16-bit type for the MFMAs; everything else is
// fp32. Inputs are 16-byte aligned with head_dim % 8 == 0 (the host pads otherwise);
// head_dim up to 256 (kernel widths 64, 128, 192, 256). fp32 inputs run the fp32
// kernels at the end of this file (fp32 MFMA up to head_dim 128, FMA above), with no
// rounding.

#include <type_traits>

#include "ffa_common.h"
#include "ffa_grid.h"
#include "ffa_internal.h"

namespace ffa {
namespace {

constexpr int kThreads = 256;
constexpr int kQTile = 128;   // q rows per dQ workgroup, and the Sq padding unit
constexpr int kKeyTile = 64;  // keys per dQ k-tile
constexpr int kDkvKeys = 128; // keys per dK/dV workgroup
constexpr int kDkvRows = 32;  // q rows per dK/dV tile

struct BwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  const float* lse;
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  float* lse2;  // workspace [B * Hq][sq_pad]
  float* di;    // workspace [B * Hq][sq_pad]
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int64_t do_sb, do_sh, do_ss;
  int64_t dq_sb, dq_sh, dq_ss;
  int64_t dk_sb, dk_sh, dk_ss;
  int64_t dv_sb, dv_sh, dv_ss;
  int64_t l_sb, l_sh, l_ss;
  int B, Hq, Hkv, Sq, Skv, D;
  int q_offset, causal, window;
  int ratio;
  int sq_pad;
  int n_qt;        // dQ workgroups per (batch, q head)
  int n_kt;        // dK/dV workgroups per (batch, kv head)
  float score_mul; // scale*log2e, or scale/softcap with softcap
  float cap_mul;   // softcap*log2e
  float tanh_mul;  // 2*log2e*scale/softcap: tanh(x) = 1 - 2 / (1 + exp2(q.k * tanh_mul))
  float scale;
  int xcd_remap_dq, xcd_remap_dkv;
  int xcd_group_dq, xcd_group_dkv;  // > 0: units per interleaved group on one XCD
  int Dv;  // V's (and dV's) head dim, <= D: V is taken as zero-padded to D
};

// Workgroup -> (unit u = batch x head, tile j; j = 0 the heaviest causal tile): the
// XCD-aware order of ffa_grid.h, the same as the forward kernel's grid, with the
// group the launcher chose (prefill_grid_order).
__device__ inline void bwd_item(int bid, int n_t, int g, int remap, int& u, int& j) {
  prefill_work_item(bid, static_cast<int>(gridDim.x), n_t, g, remap, u, j);
  u = __builtin_amdgcn_readfirstlane(u);
  j = __builtin_amdgcn_readfirstlane(j);
}

// XOR swizzle of the 16-byte chunk index of tile row r. Row-wise MFMA operand reads
// (16 lanes, 16 rows, one chunk each) need r -> swz(r) injective over 16 rows (within
// one row parity for 128-byte rows); ds_read_b64_tr_b16 (rows r0..r0+3, r0 % 4 == 0,
// 4 consecutive chunks) needs swz(r) >> 2 distinct over those 4 rows (128-byte rows:
// rows of one parity distinct). swz(r + 16) == swz(r) for both widths.
// Rows of 256 or 512 bytes (DP = 128, 256) start in the same bank group: a 4-bit
// swizzle over the low chunk bits; rows of 128 or 384 bytes (DP = 64, 192) alternate
// between two half bank rows: a 3-bit swizzle injective over rows of one parity.
template <int DP>
constexpr int kSwBits = (DP == 64 || DP == 192) ? 3 : 4;

template <int DP>
__device__ inline int bswz(int r) {
  if constexpr (kSwBits<DP> == 4) {
    return ((r & 3) << 2) | ((r >> 2) & 3);
  } else {
    const int s = (r >> 1) & 7;
    return ((s & 1) << 2) | (s >> 1);
  }
}

template <int DP>
struct BShape {
  static constexpr int CPR = DP / 8;  // 16-byte chunks per row
  static constexpr int KS = DP / 16;  // MFMA k-steps over the head dim
  static constexpr int DB = DP / 32;  // 32-dim output blocks
};

// Row `row` of a [*, DP] tile as the MFMA register operand of k-step ks: dims
// 16 ks + 8 g .. +7, zero at and beyond D.
template <int DP>
__device__ inline void load_row_operand(const uint16_t* row, int D, int g,
                                        u32x4 (&reg)[BShape<DP>::KS]) {
#pragma unroll
  for (int ks = 0; ks < BShape<DP>::KS; ++ks) {
    const int d0 = min(16 * ks + 8 * g, D - 8);
    const u32x4 v = *reinterpret_cast<const u32x4*>(row + d0);
    reg[ks] = (16 * ks + 8 * g < D) ? v : u32x4{0u, 0u, 0u, 0u};
  }
}

// Store one 32-row block of MFMA accumulators (lane l32 = row, dims 32 db + 8 i + 4 g + j)
// times `mul` as 16-bit elements. A v_permlane32_swap per dword gives lane g = 0 both
// 4-dim halves of the 8-dim chunks i = 0, 2 and lane g = 1 those of i = 1, 3, so each
// store is 16 contiguous bytes (half as many stores as 8-byte pieces). Lanes l and l + 32
// hold the same row, so they are active together wherever this is called. On MI355X the
// backward gained 1-5 % (north star +0.9 %, head_dim 64 +5 %), bit-identical.
template <typename Tag, int DP>
__device__ inline void store_rows(uint16_t* row, const f32x16 (&acc)[BShape<DP>::DB], float mul,
                                  int D, int g) {
  using E = Elem<Tag>;
#pragma unroll
  for (int db = 0; db < BShape<DP>::DB; ++db) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int i0 = 2 * k;
      const int i1 = 2 * k + 1;
      const uint32_t a0 = E::pack2(acc[db][4 * i0 + 0] * mul, acc[db][4 * i0 + 1] * mul);
      const uint32_t b0 = E::pack2(acc[db][4 * i1 + 0] * mul, acc[db][4 * i1 + 1] * mul);
      const uint32_t a1 = E::pack2(acc[db][4 * i0 + 2] * mul, acc[db][4 * i0 + 3] * mul);
      const uint32_t b1 = E::pack2(acc[db][4 * i1 + 2] * mul, acc[db][4 * i1 + 3] * mul);
      const auto x0 = __builtin_amdgcn_permlane32_swap(a0, b0, false, false);
      const auto x1 = __builtin_amdgcn_permlane32_swap(a1, b1, false, false);
      const int d0 = 32 * db + 16 * k + 8 * g;  // D is a multiple of 8
      if (d0 < D) *reinterpret_cast<u32x4*>(row + d0) = u32x4{x0[0], x1[0], x0[1], x1[1]};
    }
  }
}

// Element offsets inside a swizzled [rows, DP] tile are row * DP + chunk' * 8 + elem,
// chunk' = chunk ^ bswz(row), which only touches the low SW = kSwBits chunk bits; row * DP
// is a multiple of 8 * 2^SW for every DP. So moving from one chunk to another is an XOR
// inside the low SW + 3 offset bits plus an addition above them: one base offset per
// lane serves every k-step and dim block (the per-step offsets are not held in
// registers).
//
// Row-wise A operand of k-step ks: tile row l32, chunk 2 ks + g.
template <int DP>
__device__ inline int row_rd0(int lane) {
  const int l32 = lane & 31;
  return l32 * DP + ((((lane >> 5)) ^ bswz<DP>(l32)) << 3);
}
template <int DP>
__device__ inline int row_rd(int base, int ks) {
  constexpr int SW = kSwBits<DP>;
  return (base ^ ((ks & ((1 << (SW - 1)) - 1)) << 4)) + ((ks >> (SW - 1)) << (SW + 3));
}

// The two ds_read_b64_tr_b16 reads (rows 4g + 0..3 and 8 + 4g + 0..3 of a 16-row chunk;
// dims colw .. colw + 3 of a 32-dim block) that form the A operand [32 dims x 16 rows]
// of dims 32 db .. +31 are at base ^ (db << 5). The row order they produce is the row
// order an accumulator's lane half holds in elements 8c .. 8c + 7.
template <int DP>
__device__ inline void tr_offsets(int lane, int& lo, int& hi) {
  const int g = lane >> 5;
  const int rowoff = 4 * g + ((lane & 15) >> 2);
  const int colw = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const int cg = colw >> 3;
  lo = rowoff * DP + ((cg ^ bswz<DP>(rowoff)) << 3) + (colw & 7);
  hi = (rowoff + 8) * DP + ((cg ^ bswz<DP>(rowoff + 8)) << 3) + (colw & 7);
}

// Hide a value's origin from the optimizer: the offsets derived from it inside a
// loop are recomputed there (one XOR each) instead of being hoisted into registers.
__device__ inline int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

template <int DP>
__device__ inline int tr_at(int base, int db) {
  constexpr int SW = kSwBits<DP>;
  return (base ^ ((db & ((1 << (SW - 2)) - 1)) << 5)) + ((db >> (SW - 2)) << (SW + 3));
}

template <int DP>
__device__ inline u32x4 tr_operand(const uint16_t* tile, int lo, int hi, int db) {
  const u32x2 a = lds_read_tr16(tile + tr_at<DP>(lo, db));
  const u32x2 b = lds_read_tr16(tile + tr_at<DP>(hi, db));
  return u32x4{a[0], a[1], b[0], b[1]};
}

// ---------------------------------------------------------------------------------
// 1. lse2 and D_i. 32 rows per workgroup, 8 lanes per row.
// ---------------------------------------------------------------------------------
// 8 elements of O or dO starting at `row + 8 c` as fp32 (16-bit tags, or F32Tag).
struct F32Tag {};
template <typename Tag>
__device__ inline void load8_f32(const uint16_t* row, int c, float (&x)[8]) {
  if constexpr (std::is_same_v<Tag, F32Tag>) {
    const float* r = reinterpret_cast<const float*>(row) + 8 * c;
    const f32x4 a = *reinterpret_cast<const f32x4*>(r);
    const f32x4 b = *reinterpret_cast<const f32x4*>(r + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = a[e];
      x[4 + e] = b[e];
    }
  } else {
    const u32x4 v = *reinterpret_cast<const u32x4*>(row + 8 * c);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      x[2 * w] = Elem<Tag>::to_f32(static_cast<uint16_t>(v[w] & 0xffffu));
      x[2 * w + 1] = Elem<Tag>::to_f32(static_cast<uint16_t>(v[w] >> 16));
    }
  }
}

template <typename Tag>
__global__ __launch_bounds__(kThreads) void bwd_pre_kernel(const BwdParams p) {
  constexpr int EB = std::is_same_v<Tag, F32Tag> ? 2 : 1;  // element size in 16-bit units
  const int tid = threadIdx.x;
  const int part = tid & 7;
  const int64_t rg = static_cast<int64_t>(blockIdx.x) * 32 + (tid >> 3);  // < B*Hq*sq_pad
  const int bh = static_cast<int>(rg / p.sq_pad);
  const int s = static_cast<int>(rg - static_cast<int64_t>(bh) * p.sq_pad);
  const int b = bh / p.Hq;
  const int h = bh - b * p.Hq;
  float acc = 0.0f;
  if (s < p.Sq) {
    const uint16_t* orow =
        p.o + EB * (b * p.o_sb + h * p.o_sh + static_cast<int64_t>(s) * p.o_ss);
    const uint16_t* drow =
        p.dout + EB * (b * p.do_sb + h * p.do_sh + static_cast<int64_t>(s) * p.do_ss);
    for (int c = part; c < (p.D >> 3); c += 8) {
      float ov[8], dv[8];
      load8_f32<Tag>(orow, c, ov);
      load8_f32<Tag>(drow, c, dv);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = fmaf(ov[e], dv[e], acc);
    }
  }
  acc += __shfl_xor(acc, 1);
  acc += __shfl_xor(acc, 2);
  acc += __shfl_xor(acc, 4);
  if (part == 0) {
    float l2 = __builtin_inff();
    float di = 0.0f;
    if (s < p.Sq) {
      const float l = p.lse[b * p.l_sb + h * p.l_sh + static_cast<int64_t>(s) * p.l_ss];
      l2 = (l == kNegInf) ? __builtin_inff() : l * kLog2e;
      di = acc;
    }
    p.lse2[rg] = l2;
    p.di[rg] = di;
  }
}

// ---------------------------------------------------------------------------------
// 2. dK, dV: keys stationary.
// ---------------------------------------------------------------------------------
// Two workgroups per CU up to head_dim 128; wider rows keep their dK / dV (or dQ)
// accumulators in AGPRs at one workgroup per CU.
template <int DP>
constexpr int kBwdMinBlocks = DP <= 128 ? 2 : 1;

// DV: the width of V, dO's used dims and dV (<= DP). It is DP except for head_dim 192
// over a V of at most 128 dims (the MLA module's V, which the reference zero-pads):
// with V's padding zero, dP = dO V^T needs dO's first DV dims only, and dV's padding
// dims are not outputs, so dP and dV run over DV dims.
template <typename Tag, int DP, int DV, bool SOFTCAP>
__global__ __launch_bounds__(kThreads, kBwdMinBlocks<DP>) void bwd_dkdv_kernel(const BwdParams p) {
  using S = BShape<DP>;   // Q, K, dK
  using SV = BShape<DV>;  // dO, V, dV
  using E = Elem<Tag>;
  constexpr int TILE = kDkvRows * DP;
  constexpr int TILE_V = kDkvRows * DV;
  constexpr int LPT = kDkvRows * S::CPR / kThreads;    // Q tile loads per thread
  constexpr int LPTV = kDkvRows * SV::CPR / kThreads;  // dO tile loads per thread
  static_assert(kDkvRows * S::CPR % kThreads == 0 && kDkvRows * SV::CPR % kThreads == 0,
                "tile must split evenly");
  __shared__ __attribute__((aligned(1024))) uint16_t q_lds[2][TILE];
  __shared__ __attribute__((aligned(1024))) uint16_t do_lds[2][TILE_V];
  __shared__ __attribute__((aligned(1024))) float st_lds[2][256];  // [0,32) lse2, [32,64) D_i
  __shared__ __attribute__((aligned(1024))) uint16_t v_lds[4][32 * DV];  // each wave's V rows

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;

  int bh, kt;  // causal: low key tiles are seen by the most rows (heaviest first)
  bwd_item(blockIdx.x, p.n_kt, p.xcd_group_dkv, p.xcd_remap_dkv, bh, kt);
  const int b = bh / p.Hkv;
  const int hk = bh - b * p.Hkv;
  const int D = p.D;
  const int Sq = p.Sq;

  const int k0 = kt * kDkvKeys;
  const int kw0 = k0 + wave * 32;
  const int key = kw0 + l32;
  const bool wave_live = kw0 < p.Skv;
  const int k_last = min(k0 + kDkvKeys, p.Skv) - 1;

  // q rows whose visible keys meet [k0, k_last]: causal q_abs >= key, window
  // q_abs <= key + window - 1.
  const int q_lo = p.causal ? max(0, k0 - p.q_offset) : 0;
  const int q_hi = p.window > 0
                       ? static_cast<int>(min<int64_t>(Sq, static_cast<int64_t>(k_last) + p.window -
                                                               p.q_offset))
                       : Sq;
  const int qt_begin = q_lo / kDkvRows;
  const int ntq = q_hi > q_lo ? (q_hi + kDkvRows - 1) / kDkvRows - qt_begin : 0;
  const int nit = ntq * p.ratio;

  const float c = SOFTCAP ? p.cap_mul : p.score_mul;

  // K row of this lane's key as the B operand of S (clamped row; keys >= Skv are never
  // stored). The wave's 32 V rows go to its own LDS slice (swizzled like the tiles) and
  // are read back as the B operand of dP: registers for both would not fit. Dims at and
  // beyond D are zero in the slice (the dO tile's padding dims are not).
  const int dchunks = D >> 3;
  constexpr bool NARROW = DV < DP;
  const int Dv = NARROW ? p.Dv : D;
  const int dvchunks = Dv >> 3;
  u32x4 kreg[S::KS];
  load_row_operand<DP>(p.k + b * p.k_sb + hk * p.k_sh +
                           static_cast<int64_t>(min(key, p.Skv - 1)) * p.k_ss, D, g, kreg);
  if (wave_live) {
    const uint16_t* vb = p.v + b * p.v_sb + hk * p.v_sh + static_cast<int64_t>(kw0) * p.v_ss;
#pragma unroll
    for (int j = 0; j < 32 * SV::CPR / 64; ++j) {
      const int pos = j * 64 + lane;
      const int row = pos / SV::CPR;
      const int cq = (pos - row * SV::CPR) ^ bswz<DV>(row);
      const int rr = min(row, p.Skv - 1 - kw0);
      u32x4 val = {0u, 0u, 0u, 0u};
      if (cq < dvchunks) val = *reinterpret_cast<const u32x4*>(vb + static_cast<int64_t>(rr) * p.v_ss + 8 * cq);
      *reinterpret_cast<u32x4*>(&v_lds[wave][8 * pos]) = val;
    }
  }
  const uint16_t* vw = v_lds[wave];

  // Tile loads: load j of this thread fills chunk position P = (4j + wave) * 64 + lane;
  // LDS (row, c) holds global chunk c ^ bswz(row), clamped below head_dim (dO: below
  // V's width).
  uint32_t q_off[LPT], do_off[LPTV];
  if constexpr (!NARROW) {
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int pos = (4 * j + wave) * 64 + lane;
      const int row = pos / S::CPR;
      const int cq = min((pos - row * S::CPR) ^ bswz<DP>(row), dchunks - 1);
      q_off[j] = static_cast<uint32_t>(row * p.q_ss * 2 + cq * 16);
      do_off[j] = static_cast<uint32_t>(row * p.do_ss * 2 + cq * 16);
    }
  } else {
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int pos = (4 * j + wave) * 64 + lane;
      const int row = pos / S::CPR;
      const int cq = min((pos - row * S::CPR) ^ bswz<DP>(row), dchunks - 1);
      q_off[j] = static_cast<uint32_t>(row * p.q_ss * 2 + cq * 16);
    }
#pragma unroll
    for (int j = 0; j < LPTV; ++j) {
      const int pos = (4 * j + wave) * 64 + lane;
      const int row = pos / SV::CPR;
      const int cq = min((pos - row * SV::CPR) ^ bswz<DV>(row), dvchunks - 1);
      do_off[j] = static_cast<uint32_t>(row * p.do_ss * 2 + cq * 16);
    }
  }
  // Tiles are visited q head by q head of the group, q tiles ascending within each.
  // The next tile to issue is tracked incrementally (head r of the group, tile index
  // qi, running byte pointers) instead of dividing the iteration index.
  int is_r = 0;
  int is_qi = 0;
  const char* is_qb = nullptr;
  const char* is_db = nullptr;
  int64_t is_ws = 0;
  const int64_t q_tile_bytes = static_cast<int64_t>(kDkvRows) * p.q_ss * 2;
  const int64_t do_tile_bytes = static_cast<int64_t>(kDkvRows) * p.do_ss * 2;
  auto is_head = [&]() {
    const int hq = hk * p.ratio + is_r;
    const int q0 = qt_begin * kDkvRows;
    is_qb = reinterpret_cast<const char*>(p.q + b * p.q_sb + hq * p.q_sh +
                                          static_cast<int64_t>(q0) * p.q_ss);
    is_db = reinterpret_cast<const char*>(p.dout + b * p.do_sb + hq * p.do_sh +
                                          static_cast<int64_t>(q0) * p.do_ss);
    is_ws = (static_cast<int64_t>(b) * p.Hq + hq) * p.sq_pad + q0;
  };
  is_head();
  auto issue = [&](int buf) {
    const int q0 = (qt_begin + is_qi) * kDkvRows;
    if (q0 + kDkvRows <= Sq) {
#pragma unroll
      for (int j = 0; j < LPT; ++j) {
        load_lds16_async(is_qb, q_off[j], lds_addr(&q_lds[buf][(4 * j + wave) * 512]));
        if (j < LPTV) load_lds16_async(is_db, do_off[j], lds_addr(&do_lds[buf][(4 * j + wave) * 512]));
      }
    } else {
      // rows past Sq re-read row Sq - 1: their lse2 is +inf, so P = dS = 0
#pragma unroll
      for (int j = 0; j < LPT; ++j) {
        const int row = ((4 * j + wave) * 64 + lane) / S::CPR;
        const int over = max(0, q0 + row - (Sq - 1));
        const uint32_t qback = static_cast<uint32_t>(over * p.q_ss * 2);
        load_lds16_async(is_qb, q_off[j] - qback, lds_addr(&q_lds[buf][(4 * j + wave) * 512]));
        if constexpr (!NARROW) {
          const uint32_t dback = static_cast<uint32_t>(over * p.do_ss * 2);
          load_lds16_async(is_db, do_off[j] - dback, lds_addr(&do_lds[buf][(4 * j + wave) * 512]));
        }
      }
      if constexpr (NARROW) {
#pragma unroll
        for (int j = 0; j < LPTV; ++j) {
          const int row = ((4 * j + wave) * 64 + lane) / SV::CPR;
          const int over = max(0, q0 + row - (Sq - 1));
          const uint32_t dback = static_cast<uint32_t>(over * p.do_ss * 2);
          load_lds16_async(is_db, do_off[j] - dback, lds_addr(&do_lds[buf][(4 * j + wave) * 512]));
        }
      }
    }
    if (wave == 0) {
      // lanes 0-7: lse2 rows q0 .. q0+31, lanes 8-15: D_i; the other lanes repeat them
      // into the unused rest of the 1 KiB stats buffer
      const float* src = ((lane & 8) ? p.di : p.lse2) + is_ws + 4 * (lane & 7);
      load_lds16_async(src, lds_addr(&st_lds[buf][0]));
    }
    if (++is_qi == ntq) {
      is_qi = 0;
      ++is_r;
      if (is_r < p.ratio) is_head();
    } else {
      is_qb += q_tile_bytes;
      is_db += do_tile_bytes;
      is_ws += kDkvRows;
    }
  };

  const int a_rd0 = row_rd0<DP>(lane);
  int t_lo0, t_hi0;
  tr_offsets<DP>(lane, t_lo0, t_hi0);
  // the dO / V tiles' offsets (the same as Q's unless V is narrower)
  const int a_rd0v = row_rd0<DV>(lane);
  int tv_lo0, tv_hi0;
  tr_offsets<DV>(lane, tv_lo0, tv_hi0);

  f32x16 dkacc[S::DB], dvacc[SV::DB];
#pragma unroll
  for (int db = 0; db < S::DB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dkacc[db][r] = 0.0f;
      if (db < SV::DB) dvacc[db][r] = 0.0f;
    }
    if constexpr (kBwdMinBlocks<DP> == 1) {
      pin_agpr(dkacc[db]);
      if (db < SV::DB) pin_agpr(dvacc[db]);
    }
  }

  if (nit > 0) issue(0);
  int cur_qi = 0;  // q tile index (within [0, ntq)) of iteration it
  for (int it = 0; it < nit; ++it) {
    const int buf = it & 1;
    wait_vmcnt0();
    __syncthreads();
    if (it + 1 < nit) issue(buf ^ 1);
    const int q0 = (qt_begin + cur_qi) * kDkvRows;
    if (++cur_qi == ntq) cur_qi = 0;
    const int q0_abs = p.q_offset + q0;
    if (!wave_live) continue;
    if (p.causal && kw0 > q0_abs + kDkvRows - 1) continue;
    if (p.window > 0 && kw0 + 31 < q0_abs - p.window + 1) continue;
    const uint16_t* ql = q_lds[buf];
    const uint16_t* dl = do_lds[buf];
    const float* st = st_lds[buf];
    const int a_rd = opaque(a_rd0);
    const int t_lo = opaque(t_lo0);
    const int t_hi = opaque(t_hi0);
    const int a_rdv = NARROW ? opaque(a_rd0v) : a_rd;
    const int tv_lo = NARROW ? opaque(tv_lo0) : t_lo;
    const int tv_hi = NARROW ? opaque(tv_hi0) : t_hi;

    f32x16 sacc, dpacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sacc[r] = 0.0f;
      dpacc[r] = 0.0f;
    }
    // operands one k-step ahead of the MFMAs that consume them (dP runs over V's
    // SV::KS k-steps, S over head_dim's S::KS)
    u32x4 aq = *reinterpret_cast<const u32x4*>(ql + row_rd<DP>(a_rd, 0));
    u32x4 ad = *reinterpret_cast<const u32x4*>(dl + row_rd<DV>(a_rdv, 0));
    u32x4 bv = *reinterpret_cast<const u32x4*>(vw + row_rd<DV>(a_rdv, 0));
#pragma unroll
    for (int ks = 0; ks < S::KS; ++ks) {
      u32x4 aq_n, ad_n, bv_n;
      if (ks + 1 < S::KS) aq_n = *reinterpret_cast<const u32x4*>(ql + row_rd<DP>(a_rd, ks + 1));
      if (ks + 1 < SV::KS) {
        ad_n = *reinterpret_cast<const u32x4*>(dl + row_rd<DV>(a_rdv, ks + 1));
        bv_n = *reinterpret_cast<const u32x4*>(vw + row_rd<DV>(a_rdv, ks + 1));
      }
      __builtin_amdgcn_sched_barrier(0);
      sacc = E::mfma32(aq, kreg[ks], sacc);
      if (ks < SV::KS) dpacc = E::mfma32(ad, bv, dpacc);
      if (ks + 1 < S::KS) aq = aq_n;
      if (ks + 1 < SV::KS) {
        ad = ad_n;
        bv = bv_n;
      }
    }

    // element (row 8i + 4g + j, key l32) sits in accumulator 4i + j
    const bool need_mask = (p.causal && kw0 + 31 > q0_abs) ||
                           (p.window > 0 && kw0 < q0_abs + kDkvRows - 1 - p.window + 1);
    float pv[16], dsv[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 l2 = *reinterpret_cast<const f32x4*>(st + 8 * i + 4 * g);
      const f32x4 di = *reinterpret_cast<const f32x4*>(st + 32 + 8 * i + 4 * g);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * i + j;
        if constexpr (SOFTCAP) {
          const float t = tanh_fast(sacc[r] * p.tanh_mul);
          pv[r] = fast_exp2(fmaf(t, c, -l2[j]));
          dsv[r] = pv[r] * (dpacc[r] - di[j]) * fmaf(-t, t, 1.0f);
        } else {
          pv[r] = fast_exp2(fmaf(sacc[r], c, -l2[j]));
          dsv[r] = pv[r] * (dpacc[r] - di[j]);
        }
      }
    }
    if (need_mask) {
      // row qa0 + off (off = 8 (r >> 2) + (r & 3), a compile-time offset) sees this
      // lane's key iff lo <= off <= hi: causal key <= row, window key >= row - w + 1
      const int qa0 = q0_abs + 4 * g;
      const int lo = p.causal ? key - qa0 : -0x7fffffff;
      const int hi = p.window > 0 ? key + p.window - 1 - qa0 : 0x7fffffff;  // window clamped on the host
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int off = 8 * (r >> 2) + (r & 3);
        const bool ok = (off >= lo) & (off <= hi);
        pv[r] = ok ? pv[r] : 0.0f;
        dsv[r] = ok ? dsv[r] : 0.0f;
      }
    }
    // dV^T[d, key] += dO^T[d, row] P[row, key]; dK^T[d, key] += Q^T[d, row] dS[row, key]
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      const int e0 = 8 * cc;
      const u32x4 bp = {E::pack2(pv[e0 + 0], pv[e0 + 1]), E::pack2(pv[e0 + 2], pv[e0 + 3]),
                        E::pack2(pv[e0 + 4], pv[e0 + 5]), E::pack2(pv[e0 + 6], pv[e0 + 7])};
      const u32x4 bs = {E::pack2(dsv[e0 + 0], dsv[e0 + 1]), E::pack2(dsv[e0 + 2], dsv[e0 + 3]),
                        E::pack2(dsv[e0 + 4], dsv[e0 + 5]), E::pack2(dsv[e0 + 6], dsv[e0 + 7])};
#pragma unroll
      for (int db = 0; db < S::DB; ++db) {
        u32x4 ado;
        if (db < SV::DB) ado = tr_operand<DV>(dl + 16 * cc * DV, tv_lo, tv_hi, db);
        const u32x4 aq = tr_operand<DP>(ql + 16 * cc * DP, t_lo, t_hi, db);
        if (db < SV::DB) dvacc[db] = E::mfma32(ado, bp, dvacc[db]);
        dkacc[db] = E::mfma32(aq, bs, dkacc[db]);
      }
    }
    if constexpr (kBwdMinBlocks<DP> == 1) {
#pragma unroll
      for (int db = 0; db < S::DB; ++db) {
        pin_agpr(dkacc[db]);
        if (db < SV::DB) pin_agpr(dvacc[db]);
      }
    }
  }

  if (wave_live && key < p.Skv) {
    store_rows<Tag, DP>(p.dk + b * p.dk_sb + hk * p.dk_sh + static_cast<int64_t>(key) * p.dk_ss,
                        dkacc, p.scale, D, g);
    store_rows<Tag, DV>(p.dv + b * p.dv_sb + hk * p.dv_sh + static_cast<int64_t>(key) * p.dv_ss,
                        dvacc, 1.0f, Dv, g);
  }
}

// ---------------------------------------------------------------------------------
// 3. dQ: queries stationary.
// ---------------------------------------------------------------------------------
template <typename Tag, int DP, int DV, bool SOFTCAP>
__global__ __launch_bounds__(kThreads, kBwdMinBlocks<DP>) void bwd_dq_kernel(const BwdParams p) {
  using S = BShape<DP>;   // Q, K, dQ
  using SV = BShape<DV>;  // dO, V (dP^T = V dO^T over V's dims)
  using E = Elem<Tag>;
  constexpr int BN = kKeyTile;
  constexpr int TILE = BN * DP;
  constexpr int TILE_V = BN * DV;
  constexpr int LPT = BN * S::CPR / kThreads;
  constexpr int LPTV = BN * SV::CPR / kThreads;
  static_assert(BN * S::CPR % kThreads == 0 && BN * SV::CPR % kThreads == 0, "tile must split evenly");
  __shared__ __attribute__((aligned(1024))) uint16_t k_lds[2][TILE];
  __shared__ __attribute__((aligned(1024))) uint16_t v_lds[2][TILE_V];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;

  int bh, jq;
  bwd_item(blockIdx.x, p.n_qt, p.xcd_group_dq, p.xcd_remap_dq, bh, jq);
  const int qt = p.causal ? (p.n_qt - 1 - jq) : jq;
  const int b = bh / p.Hq;
  const int h = bh - b * p.Hq;
  const int hk = h / p.ratio;
  const int D = p.D;
  const int Skv = p.Skv;

  const int q0 = qt * kQTile;
  const int q_last = min(q0 + kQTile, p.Sq) - 1;
  const int q0_abs = p.q_offset + q0;
  const int ql_abs = p.q_offset + q_last;
  const int kv_lo = p.window > 0 ? max(0, q0_abs - p.window + 1) : 0;
  const int kv_hi = p.causal ? min(Skv, ql_abs + 1) : Skv;
  const int t_begin = kv_lo / BN;
  const int nt = kv_hi > kv_lo ? (kv_hi + BN - 1) / BN - t_begin : 0;

  const int qw0 = q0 + wave * 32;
  const int qrow = qw0 + l32;
  const bool wave_live = qw0 < p.Sq;
  const int qw0_abs = p.q_offset + qw0;
  const int qwl_abs = p.q_offset + min(qw0 + 31, p.Sq - 1);
  const int qa = p.q_offset + qrow;

  const float c = SOFTCAP ? p.cap_mul : p.score_mul;
  // this lane's row statistics (padding rows: lse2 = +inf, D_i = 0)
  const int64_t ws = static_cast<int64_t>(bh) * p.sq_pad + qrow;
  const float lse2 = p.lse2[ws];
  const float di = p.di[ws];

  constexpr bool NARROW = DV < DP;
  const int Dv = NARROW ? p.Dv : D;
  u32x4 qreg[S::KS], doreg[SV::KS];
  {
    const int qr = min(qrow, p.Sq - 1);
    load_row_operand<DP>(p.q + b * p.q_sb + h * p.q_sh + static_cast<int64_t>(qr) * p.q_ss, D, g, qreg);
    load_row_operand<DV>(p.dout + b * p.do_sb + h * p.do_sh + static_cast<int64_t>(qr) * p.do_ss, Dv, g,
                         doreg);
  }

  const char* kbytes = reinterpret_cast<const char*>(p.k + b * p.k_sb + hk * p.k_sh);
  const char* vbytes = reinterpret_cast<const char*>(p.v + b * p.v_sb + hk * p.v_sh);
  const int dchunks = D >> 3;
  const int dvchunks = Dv >> 3;
  uint32_t k_off[LPT], v_off[LPTV];
  if constexpr (!NARROW) {
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int pos = (4 * j + wave) * 64 + lane;
      const int row = pos / S::CPR;
      const int cq = min((pos - row * S::CPR) ^ bswz<DP>(row), dchunks - 1);
      k_off[j] = static_cast<uint32_t>(row * p.k_ss * 2 + cq * 16);
      v_off[j] = static_cast<uint32_t>(row * p.v_ss * 2 + cq * 16);
    }
  } else {
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int pos = (4 * j + wave) * 64 + lane;
      const int row = pos / S::CPR;
      const int cq = min((pos - row * S::CPR) ^ bswz<DP>(row), dchunks - 1);
      k_off[j] = static_cast<uint32_t>(row * p.k_ss * 2 + cq * 16);
    }
#pragma unroll
    for (int j = 0; j < LPTV; ++j) {
      const int pos = (4 * j + wave) * 64 + lane;
      const int row = pos / SV::CPR;
      const int cq = min((pos - row * SV::CPR) ^ bswz<DV>(row), dvchunks - 1);
      v_off[j] = static_cast<uint32_t>(row * p.v_ss * 2 + cq * 16);
    }
  }
  auto issue = [&](int t, int buf) {
    const int kt0 = t * BN;
    const char* kb = kbytes + static_cast<int64_t>(kt0) * p.k_ss * 2;
    const char* vb = vbytes + static_cast<int64_t>(kt0) * p.v_ss * 2;
    if (kt0 + BN <= Skv) {
#pragma unroll
      for (int j = 0; j < LPT; ++j) {
        load_lds16_async(kb, k_off[j], lds_addr(&k_lds[buf][(4 * j + wave) * 512]));
        if (j < LPTV) load_lds16_async(vb, v_off[j], lds_addr(&v_lds[buf][(4 * j + wave) * 512]));
      }
    } else {
      // rows past Skv re-read row Skv - 1 (masked below)
#pragma unroll
      for (int j = 0; j < LPT; ++j) {
        const int row = ((4 * j + wave) * 64 + lane) / S::CPR;
        const int over = max(0, kt0 + row - (Skv - 1));
        load_lds16_async(kb, k_off[j] - static_cast<uint32_t>(over * p.k_ss * 2),
                         lds_addr(&k_lds[buf][(4 * j + wave) * 512]));
        if constexpr (!NARROW) {
          load_lds16_async(vb, v_off[j] - static_cast<uint32_t>(over * p.v_ss * 2),
                           lds_addr(&v_lds[buf][(4 * j + wave) * 512]));
        }
      }
      if constexpr (NARROW) {
#pragma unroll
        for (int j = 0; j < LPTV; ++j) {
          const int row = ((4 * j + wave) * 64 + lane) / SV::CPR;
          const int over = max(0, kt0 + row - (Skv - 1));
          load_lds16_async(vb, v_off[j] - static_cast<uint32_t>(over * p.v_ss * 2),
                           lds_addr(&v_lds[buf][(4 * j + wave) * 512]));
        }
      }
    }
  };

  const int a_rd0 = row_rd0<DP>(lane);
  const int a_rd0v = row_rd0<DV>(lane);
  int t_lo0, t_hi0;
  tr_offsets<DP>(lane, t_lo0, t_hi0);

  f32x16 dqacc[S::DB];
#pragma unroll
  for (int db = 0; db < S::DB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) dqacc[db][r] = 0.0f;
    if constexpr (kBwdMinBlocks<DP> == 1) pin_agpr(dqacc[db]);
  }

  if (nt > 0) issue(t_begin, 0);
  for (int i = 0; i < nt; ++i) {
    const int buf = i & 1;
    const int t = t_begin + i;
    const int kt0 = t * BN;
    wait_vmcnt0();
    __syncthreads();
    if (i + 1 < nt) issue(t + 1, buf ^ 1);
    if (!wave_live) continue;
    if (p.causal && kt0 > qwl_abs) continue;
    const uint16_t* kl = k_lds[buf];
    const uint16_t* vl = v_lds[buf];
    const int a_rd = opaque(a_rd0);
    const int a_rdv = NARROW ? opaque(a_rd0v) : a_rd;
    const int t_lo = opaque(t_lo0);
    const int t_hi = opaque(t_hi0);

    f32x16 sacc[2], dpacc[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sacc[nb][r] = 0.0f;
        dpacc[nb][r] = 0.0f;
      }
    }
#pragma unroll
    for (int ks = 0; ks < S::KS; ++ks) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const u32x4 ak = *reinterpret_cast<const u32x4*>(kl + row_rd<DP>(a_rd, ks) + nb * 32 * DP);
        sacc[nb] = E::mfma32(ak, qreg[ks], sacc[nb]);
        if (ks < SV::KS) {
          const u32x4 av = *reinterpret_cast<const u32x4*>(vl + row_rd<DV>(a_rdv, ks) + nb * 32 * DV);
          dpacc[nb] = E::mfma32(av, doreg[ks < SV::KS ? ks : 0], dpacc[nb]);
        }
      }
    }

    // element (key 32 nb + 8 i + 4 g + j, query l32) sits in sacc[nb][4i + j]
    const bool need_mask = (kt0 + BN > Skv) || (p.causal && kt0 + BN - 1 > qw0_abs) ||
                           (p.window > 0 && kt0 < qwl_abs - p.window + 1);
    float dsv[2][16];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if constexpr (SOFTCAP) {
          const float tt = tanh_fast(sacc[nb][r] * p.tanh_mul);
          dsv[nb][r] = fast_exp2(fmaf(tt, c, -lse2)) * (dpacc[nb][r] - di) * fmaf(-tt, tt, 1.0f);
        } else {
          dsv[nb][r] = fast_exp2(fmaf(sacc[nb][r], c, -lse2)) * (dpacc[nb][r] - di);
        }
      }
    }
    if (need_mask) {
      // key key0 + off (off a compile-time offset) is visible to this lane's row iff
      // off <= hi (below Skv and, causal, at or before the row) and off >= lo (window)
      const int key0 = kt0 + 4 * g;
      const int hi = min(Skv - 1, p.causal ? qa : 0x7fffffff) - key0;
      const int lo = p.window > 0 ? qa - p.window + 1 - key0 : -0x7fffffff;  // window clamped on the host
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int off = 32 * nb + 8 * (r >> 2) + (r & 3);
          const bool ok = (off >= lo) & (off <= hi);
          dsv[nb][r] = ok ? dsv[nb][r] : 0.0f;
        }
      }
    }
    // dQ^T[d, q] += K^T[d, key] dS^T[key, q]
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int nb = cc >> 1;
      const int e0 = (cc & 1) * 8;
      const u32x4 bs = {E::pack2(dsv[nb][e0 + 0], dsv[nb][e0 + 1]),
                        E::pack2(dsv[nb][e0 + 2], dsv[nb][e0 + 3]),
                        E::pack2(dsv[nb][e0 + 4], dsv[nb][e0 + 5]),
                        E::pack2(dsv[nb][e0 + 6], dsv[nb][e0 + 7])};
#pragma unroll
      for (int db = 0; db < S::DB; ++db) {
        const u32x4 ak = tr_operand<DP>(kl + 16 * cc * DP, t_lo, t_hi, db);
        dqacc[db] = E::mfma32(ak, bs, dqacc[db]);
      }
    }
    if constexpr (kBwdMinBlocks<DP> == 1) {
#pragma unroll
      for (int db = 0; db < S::DB; ++db) pin_agpr(dqacc[db]);
    }
  }

  if (wave_live && qrow < p.Sq) {
    store_rows<Tag, DP>(p.dq + b * p.dq_sb + h * p.dq_sh + static_cast<int64_t>(qrow) * p.dq_ss,
                        dqacc, p.scale, D, g);
  }
}

// ---------------------------------------------------------------------------------
// fp32 inputs with head_dim > 128: the reference computes them in fp32
// (cpu_reference.py:319-427), so they run on fp32 FMAs (head_dim <= 128 runs the MFMA
// kernels below). A workgroup (256 threads) owns 32 keys (dK / dV) or 32 query rows
// (dQ) and sweeps 32-row tiles of the other side through LDS, rows padded by one float
// so the 32 rows read together at one dim fall in 32 distinct banks. Per tile, thread t
// computes the scores of key (or row) t % 32 against rows t / 32 + 8 i (i < 4), and
// P / dS go through LDS to the accumulation, where thread t owns dims t / 32 + 8 j of
// key (or row) t % 32.
// ---------------------------------------------------------------------------------
constexpr int kF32T = 32;  // keys or rows per workgroup, rows per tile

// P and dS of the pairs (row rb + 8 i of the row tile, key kk of the key tile) from the
// two fp32 tiles in LDS; `row_ok(i)` / `key_of` give the mask inputs.
template <bool SOFTCAP, int PITCH>
__device__ inline void f32_pairs(const BwdParams& p, const float* rowt_q, const float* rowt_do,
                                 const float* keyt_k, const float* keyt_v, const float* stats,
                                 int kk, int rb, int q0_abs, int q_valid, int key, bool key_ok,
                                 float (&pv)[4], float (&dsv)[4]) {
  float sc[4] = {0.f, 0.f, 0.f, 0.f};
  float dp[4] = {0.f, 0.f, 0.f, 0.f};
  const float* kr = keyt_k + kk * PITCH;
  const float* vr = keyt_v + kk * PITCH;
  for (int d = 0; d < p.D; ++d) {
    const float kv = kr[d];
    const float vv = vr[d];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = fmaf(rowt_q[(rb + 8 * i) * PITCH + d], kv, sc[i]);
      dp[i] = fmaf(rowt_do[(rb + 8 * i) * PITCH + d], vv, dp[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = rb + 8 * i;
    const int qa = q0_abs + r;
    const bool ok = key_ok && r < q_valid && (!p.causal || key <= qa) &&
                    (p.window <= 0 || key >= qa - p.window + 1);
    const float l2 = stats[r];
    const float di = stats[kF32T + r];
    float pr, ds;
    if constexpr (SOFTCAP) {
      const float t = tanh_fast(sc[i] * p.tanh_mul);
      pr = fast_exp2(fmaf(t, p.cap_mul, -l2));
      ds = pr * (dp[i] - di) * fmaf(-t, t, 1.0f);
    } else {
      pr = fast_exp2(fmaf(sc[i], p.score_mul, -l2));
      ds = pr * (dp[i] - di);
    }
    pv[i] = ok ? pr : 0.0f;
    dsv[i] = ok ? ds : 0.0f;
  }
}

// rows [r0, r0 + 32) of a [*, D] fp32 tensor (row stride ss elements, rows past `last`
// clamped to it) into a padded LDS tile; dims >= D are not read
template <int PITCH>
__device__ inline void f32_tile(float* t, const float* base, int64_t ss, int r0, int last, int D) {
  for (int idx = threadIdx.x; idx < kF32T * D; idx += kThreads) {
    const int r = idx / D;
    const int d = idx - r * D;
    t[r * PITCH + d] = base[static_cast<int64_t>(min(r0 + r, last)) * ss + d];
  }
}

template <int DP, bool SOFTCAP>
__global__ __launch_bounds__(kThreads) void bwd_f32_dkdv_kernel(const BwdParams p) {
  constexpr int PITCH = DP + 1;
  constexpr int NJ = DP / 8;
  __shared__ float kt[kF32T * PITCH], vt[kF32T * PITCH], qt[kF32T * PITCH], dt[kF32T * PITCH];
  __shared__ float pt[kF32T][kF32T + 1], st[kF32T][kF32T + 1];
  __shared__ float stats[2 * kF32T];
  const int tid = threadIdx.x;
  const int kk = tid & 31;
  const int rb = tid >> 5;
  const int n_kt = (p.Skv + kF32T - 1) / kF32T;
  const int bh = blockIdx.x / n_kt;
  const int k0 = (blockIdx.x - bh * n_kt) * kF32T;
  const int b = bh / p.Hkv;
  const int hk = bh - b * p.Hkv;
  const int D = p.D;
  const float* q = reinterpret_cast<const float*>(p.q);
  const float* k = reinterpret_cast<const float*>(p.k);
  const float* v = reinterpret_cast<const float*>(p.v);
  const float* dout = reinterpret_cast<const float*>(p.dout);
  f32_tile<PITCH>(kt, k + b * p.k_sb + hk * p.k_sh, p.k_ss, k0, p.Skv - 1, D);
  f32_tile<PITCH>(vt, v + b * p.v_sb + hk * p.v_sh, p.v_ss, k0, p.Skv - 1, D);
  const int key = k0 + kk;
  const int k_last = min(k0 + kF32T, p.Skv) - 1;
  // q rows that can see a key of [k0, k_last]
  const int q_lo = p.causal ? max(0, k0 - p.q_offset) : 0;
  const int q_hi = p.window > 0 ? static_cast<int>(min<int64_t>(
                                      p.Sq, static_cast<int64_t>(k_last) + p.window - p.q_offset))
                                : p.Sq;
  float dk[NJ], dv[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    dk[j] = 0.0f;
    dv[j] = 0.0f;
  }
  for (int r = 0; r < p.ratio; ++r) {
    const int hq = hk * p.ratio + r;
    const float* qb = q + b * p.q_sb + hq * p.q_sh;
    const float* db = dout + b * p.do_sb + hq * p.do_sh;
    const int64_t ws = (static_cast<int64_t>(b) * p.Hq + hq) * p.sq_pad;
    for (int q0 = q_lo / kF32T * kF32T; q0 < q_hi; q0 += kF32T) {
      __syncthreads();  // the previous tile's reads are done
      f32_tile<PITCH>(qt, qb, p.q_ss, q0, p.Sq - 1, D);
      f32_tile<PITCH>(dt, db, p.do_ss, q0, p.Sq - 1, D);
      if (tid < 2 * kF32T) {
        stats[tid] = (tid < kF32T ? p.lse2 : p.di)[ws + q0 + (tid & (kF32T - 1))];
      }
      __syncthreads();
      float pv[4], dsv[4];
      f32_pairs<SOFTCAP, PITCH>(p, qt, dt, kt, vt, stats, kk, rb, p.q_offset + q0, p.Sq - q0, key,
                                key < p.Skv, pv, dsv);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pt[rb + 8 * i][kk] = pv[i];
        st[rb + 8 * i][kk] = dsv[i];
      }
      __syncthreads();
      // dV[key, d] += P[row, key] dO[row, d];  dK[key, d] += dS[row, key] Q[row, d]
      for (int row = 0; row < kF32T; ++row) {
        const float pr = pt[row][kk];
        const float ds = st[row][kk];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int d = rb + 8 * j;
          if (d < D) {
            dv[j] = fmaf(pr, dt[row * PITCH + d], dv[j]);
            dk[j] = fmaf(ds, qt[row * PITCH + d], dk[j]);
          }
        }
      }
    }
  }
  if (key < p.Skv) {
    float* dkr = reinterpret_cast<float*>(p.dk) + b * p.dk_sb + hk * p.dk_sh +
                 static_cast<int64_t>(key) * p.dk_ss;
    float* dvr = reinterpret_cast<float*>(p.dv) + b * p.dv_sb + hk * p.dv_sh +
                 static_cast<int64_t>(key) * p.dv_ss;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int d = rb + 8 * j;
      if (d < D) {
        dkr[d] = dk[j] * p.scale;
        dvr[d] = dv[j];
      }
    }
  }
}

template <int DP, bool SOFTCAP>
__global__ __launch_bounds__(kThreads) void bwd_f32_dq_kernel(const BwdParams p) {
  constexpr int PITCH = DP + 1;
  constexpr int NJ = DP / 8;
  __shared__ float qt[kF32T * PITCH], dt[kF32T * PITCH], kt[kF32T * PITCH], vt[kF32T * PITCH];
  __shared__ float st[kF32T][kF32T + 1];
  __shared__ float stats[2 * kF32T];
  const int tid = threadIdx.x;
  const int kk = tid & 31;  // key of the pair phase, row of the accumulation phase
  const int rb = tid >> 5;
  const int n_qt = (p.Sq + kF32T - 1) / kF32T;
  const int bh = blockIdx.x / n_qt;
  const int q0 = (blockIdx.x - bh * n_qt) * kF32T;
  const int b = bh / p.Hq;
  const int h = bh - b * p.Hq;
  const int hk = h / p.ratio;
  const int D = p.D;
  f32_tile<PITCH>(qt, reinterpret_cast<const float*>(p.q) + b * p.q_sb + h * p.q_sh, p.q_ss, q0,
                  p.Sq - 1, D);
  f32_tile<PITCH>(dt, reinterpret_cast<const float*>(p.dout) + b * p.do_sb + h * p.do_sh,
                  p.do_ss, q0, p.Sq - 1, D);
  const int64_t ws = static_cast<int64_t>(bh) * p.sq_pad;
  if (tid < 2 * kF32T) stats[tid] = (tid < kF32T ? p.lse2 : p.di)[ws + q0 + (tid & (kF32T - 1))];
  const float* kb = reinterpret_cast<const float*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const float* vb = reinterpret_cast<const float*>(p.v) + b * p.v_sb + hk * p.v_sh;
  const int q0_abs = p.q_offset + q0;
  const int ql_abs = p.q_offset + min(q0 + kF32T, p.Sq) - 1;
  const int kv_lo = p.window > 0 ? max(0, q0_abs - p.window + 1) : 0;
  const int kv_hi = p.causal ? min(p.Skv, ql_abs + 1) : p.Skv;
  float dq[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) dq[j] = 0.0f;
  for (int k0 = kv_lo / kF32T * kF32T; k0 < kv_hi; k0 += kF32T) {
    __syncthreads();  // the previous tile's reads are done
    f32_tile<PITCH>(kt, kb, p.k_ss, k0, p.Skv - 1, D);
    f32_tile<PITCH>(vt, vb, p.v_ss, k0, p.Skv - 1, D);
    __syncthreads();
    float pv[4], dsv[4];
    const int key = k0 + kk;
    f32_pairs<SOFTCAP, PITCH>(p, qt, dt, kt, vt, stats, kk, rb, q0_abs, p.Sq - q0, key,
                              key < p.Skv, pv, dsv);
#pragma unroll
    for (int i = 0; i < 4; ++i) st[rb + 8 * i][kk] = dsv[i];
    __syncthreads();
    // dQ[row, d] += dS[row, key] K[key, d]  (row = kk here)
    for (int kx = 0; kx < kF32T; ++kx) {
      const float ds = st[kk][kx];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int d = rb + 8 * j;
        if (d < D) dq[j] = fmaf(ds, kt[kx * PITCH + d], dq[j]);
      }
    }
  }
  if (q0 + kk < p.Sq) {
    float* dqr = reinterpret_cast<float*>(p.dq) + b * p.dq_sb + h * p.dq_sh +
                 static_cast<int64_t>(q0 + kk) * p.dq_ss;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int d = rb + 8 * j;
      if (d < D) dqr[d] = dq[j] * p.scale;
    }
  }
}

template <int DP, bool SOFTCAP>
void launch_f32_dp(const BwdParams& p, hipStream_t s) {
  const int grid_dkv = p.B * p.Hkv * ((p.Skv + kF32T - 1) / kF32T);
  const int grid_dq = p.B * p.Hq * ((p.Sq + kF32T - 1) / kF32T);
  if (grid_dkv > 0) {
    hipLaunchKernelGGL((bwd_f32_dkdv_kernel<DP, SOFTCAP>), dim3(grid_dkv), dim3(kThreads), 0, s, p);
  }
  hipLaunchKernelGGL((bwd_f32_dq_kernel<DP, SOFTCAP>), dim3(grid_dq), dim3(kThreads), 0, s, p);
}

// ---------------------------------------------------------------------------------
// fp32 inputs up to head_dim 128 on v_mfma_f32_32x32x2_f32 (fp32 operands, no
// rounding). A workgroup of 4 waves owns 32 keys (dK / dV) or 32 query rows (dQ); its
// waves split the other side's 32-row tiles between them (wave w takes tiles w, w + 4,
// ...), each staging its own tiles in a wave-private LDS region with the next tile
// prefetched into registers, and their partial sums meet in LDS at the end in a fixed
// order (deterministic). Small problems (cfg1: 16 heads of 1024 rows) still fill the
// chip: one workgroup per 32 keys or rows, four waves each.
//   dK / dV: lane (g, l) holds key l's K and V dims [g D/2, (g + 1) D/2) as B operands.
//     S = Q K^T and dP = dO V^T (reduction dim ks for lanes 0-31, D/2 + ks for 32-63);
//     accumulator element r of lane (g, l) is row 8 (r / 4) + 4 g + r % 4, key l, so
//     P and dS are directly the B operands of dV^T += dO^T P and dK^T += Q^T dS.
//   dQ: the same with rows and keys exchanged (S^T = K Q^T, dP^T = V dO^T, lane =
//     query row with its lse2 / D_i in one register), dQ^T += K^T dS^T.
// Rows are padded by 4 floats (the forward fp32 kernel's conflict-free pitch).
// ---------------------------------------------------------------------------------
constexpr int kM32 = 32;  // keys or rows per workgroup, rows per tile
static_assert(F32WaveTile<64>::ROWS == kM32, "a wave tile is one 32-row tile");

// dims [g DP/2, (g + 1) DP/2) of one fp32 row (zero past D): the stationary operand
template <int DP>
__device__ inline void load_half_row_f32(const float* row, int D, int g, float (&x)[DP / 2]) {
#pragma unroll
  for (int c4 = 0; c4 < DP / 2; c4 += 4) {
    const int d0 = g * (DP / 2) + c4;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (d0 < D) v = *reinterpret_cast<const f32x4*>(row + d0);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[c4 + e] = v[e];
  }
}

// P and dS of one (row, key) pair from its raw score s = q.k and dP
template <bool SOFTCAP>
__device__ inline void f32_pds(const BwdParams& p, float s, float dp, float l2, float di, bool ok,
                               float& pr, float& ds) {
  if constexpr (SOFTCAP) {
    const float t = tanh_fast(s * p.tanh_mul);
    pr = fast_exp2(fmaf(t, p.cap_mul, -l2));
    ds = pr * (dp - di) * fmaf(-t, t, 1.0f);
  } else {
    pr = fast_exp2(fmaf(s, p.score_mul, -l2));
    ds = pr * (dp - di);
  }
  pr = ok ? pr : 0.0f;
  ds = ok ? ds : 0.0f;
}

// Sum the partial accumulators of the four waves in LDS (wave order 0, 1, 2, 3) into
// wave 0's registers. `red` holds 3 x 64 x NA floats and no tile is in use any more.
template <int NA>
__device__ inline void wave_reduce4(float* red, f32x16 (&acc)[NA], int wave, int lane) {
  __syncthreads();  // every wave is done with its tiles
  if (wave > 0) {
#pragma unroll
    for (int a = 0; a < NA; ++a) {
#pragma unroll
      for (int r = 0; r < 16; ++r) red[(((wave - 1) * NA + a) * 16 + r) * 64 + lane] = acc[a][r];
    }
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 0; w < 3; ++w) {
#pragma unroll
      for (int a = 0; a < NA; ++a) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][r] += red[((w * NA + a) * 16 + r) * 64 + lane];
      }
    }
  }
}

// accumulator element (db, r) of lane (g, l32): row dim 32 db + 8 (r / 4) + 4 g + r % 4
template <int DB>
__device__ inline void store_acc_row_f32(float* row, const f32x16* acc, float mul, int D, int g) {
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int d0 = 32 * db + 8 * ii + 4 * g;
      const f32x4 w = {acc[db][4 * ii] * mul, acc[db][4 * ii + 1] * mul, acc[db][4 * ii + 2] * mul,
                       acc[db][4 * ii + 3] * mul};
      if (d0 < D) *reinterpret_cast<f32x4*>(row + d0) = w;
    }
  }
}

// dK / dV: one workgroup per CU (its 4 waves hold K, V, dK and dV of 32 keys plus a
// prefetched tile at head_dim 64; at 128 the tile is loaded when it is needed). dQ: two
// per CU at head_dim 64.
template <int DP>
constexpr int kF32mDqBlocks = DP <= 64 ? 2 : 1;
template <int DP>
constexpr bool kF32mDkvPrefetch = DP <= 64;

template <int DP, bool SOFTCAP>
__global__ __launch_bounds__(kThreads, 1) void bwd_f32m_dkdv_kernel(const BwdParams p) {
  using T = F32WaveTile<DP>;
  constexpr int PITCH = T::PITCH;
  constexpr int HALF = DP / 2;
  constexpr int DB = DP / 32;
  static_assert(3 * 64 * 32 * DB <= 4 * 2 * kM32 * PITCH, "reduction fits in the tiles");
  __shared__ __attribute__((aligned(16))) float lds[4 * 2 * kM32 * PITCH];
  __shared__ __attribute__((aligned(16))) float stl[4][2 * kM32];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;
  float* qt = lds + wave * 2 * kM32 * PITCH;
  float* dt = qt + kM32 * PITCH;
  float* st = stl[wave];

  // heaviest key blocks (causal: block 0 sees every row) first, all heads at once
  const int units = p.B * p.Hkv;
  const int kb = static_cast<int>(blockIdx.x) / units;
  const int bh = static_cast<int>(blockIdx.x) - kb * units;
  const int b = bh / p.Hkv;
  const int hk = bh - b * p.Hkv;
  const int D = p.D;
  const int k0 = kb * kM32;
  const int key = k0 + l32;
  const int k_last = min(k0 + kM32, p.Skv) - 1;
  const int q_lo = p.causal ? max(0, k0 - p.q_offset) : 0;
  const int q_hi = p.window > 0 ? static_cast<int>(min<int64_t>(
                                      p.Sq, static_cast<int64_t>(k_last) + p.window - p.q_offset))
                                : p.Sq;
  const int j_lo = q_lo / kM32;
  const int nj = q_hi > q_lo ? (q_hi + kM32 - 1) / kM32 - j_lo : 0;
  const int n_items = p.ratio * nj;

  const float* qf = reinterpret_cast<const float*>(p.q);
  const float* dof = reinterpret_cast<const float*>(p.dout);
  float kreg[HALF], vreg[HALF];
  {
    const int kr = min(key, p.Skv - 1);
    load_half_row_f32<DP>(reinterpret_cast<const float*>(p.k) + b * p.k_sb + hk * p.k_sh +
                              static_cast<int64_t>(kr) * p.k_ss, D, g, kreg);
    load_half_row_f32<DP>(reinterpret_cast<const float*>(p.v) + b * p.v_sb + hk * p.v_sh +
                              static_cast<int64_t>(kr) * p.v_ss, D, g, vreg);
  }
  f32x16 acc[2 * DB];  // dK^T blocks, then dV^T blocks
#pragma unroll
  for (int a = 0; a < 2 * DB; ++a) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[a][r] = 0.0f;
    pin_agpr(acc[a]);
  }

  T qn, dn;
  float statn = 0.0f;
  // item i: q head hk * ratio + i / nj, row tile j_lo + i % nj
  auto fetch = [&](int i) {
    const int hq = hk * p.ratio + i / nj;
    const int q0 = (j_lo + i % nj) * kM32;
    qn.load(qf + b * p.q_sb + hq * p.q_sh, p.q_ss, q0, p.Sq - 1, D, lane);
    dn.load(dof + b * p.do_sb + hq * p.do_sh, p.do_ss, q0, p.Sq - 1, D, lane);
    // lanes 0-31: lse2 of row q0 + l32, lanes 32-63: D_i (rows < sq_pad)
    const int64_t ws = (static_cast<int64_t>(b) * p.Hq + hq) * p.sq_pad + q0 + l32;
    statn = (g == 0 ? p.lse2 : p.di)[ws];
  };
  constexpr bool PREFETCH = kF32mDkvPrefetch<DP>;
  if (PREFETCH && wave < n_items) fetch(wave);
  for (int i = wave; i < n_items; i += 4) {
    const int q0 = (j_lo + i % nj) * kM32;
    if (!PREFETCH) fetch(i);
    qn.store(qt, lane);
    dn.store(dt, lane);
    st[lane] = statn;
    wave_lds_order();
    if (PREFETCH && i + 4 < n_items) fetch(i + 4);

    f32x16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = 0.0f;
      dp[r] = 0.0f;
    }
    const float* qrow = qt + l32 * PITCH + g * HALF;
    const float* drow = dt + l32 * PITCH + g * HALF;
#pragma unroll
    for (int ks = 0; ks < HALF; ++ks) {
      s = mfma_f32(qrow[ks], kreg[ks], s);
      dp = mfma_f32(drow[ks], vreg[ks], dp);
    }
    const int qa0 = p.q_offset + q0;
    const bool need_mask = q0 + kM32 > p.Sq || k0 + kM32 > p.Skv || (p.causal && qa0 < k0 + kM32 - 1) ||
                           (p.window > 0 && k0 < qa0 + kM32 - p.window);
    float pv[16], dsv[16];
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const f32x4 l2 = *reinterpret_cast<const f32x4*>(st + 8 * ii + 4 * g);
      const f32x4 di = *reinterpret_cast<const f32x4*>(st + kM32 + 8 * ii + 4 * g);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int r = 4 * ii + jj;
        const int row = 8 * ii + 4 * g + jj;
        bool ok = true;
        if (need_mask) {
          const int qa = qa0 + row;
          ok = q0 + row < p.Sq && key < p.Skv && (!p.causal || key <= qa) &&
               (p.window <= 0 || key >= qa - p.window + 1);
        }
        f32_pds<SOFTCAP>(p, s[r], dp[r], l2[jj], di[jj], ok, pv[r], dsv[r]);
      }
    }
    // dV^T[d, key] += dO[row, d] P[row, key];  dK^T[d, key] += Q[row, d] dS[row, key]
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 8 * (r >> 2) + 4 * g + (r & 3);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        acc[DB + db] = mfma_f32(dt[row * PITCH + 32 * db + l32], pv[r], acc[DB + db]);
        acc[db] = mfma_f32(qt[row * PITCH + 32 * db + l32], dsv[r], acc[db]);
      }
    }
#pragma unroll
    for (int a = 0; a < 2 * DB; ++a) pin_agpr(acc[a]);
    wave_lds_order();
  }

  wave_reduce4<2 * DB>(lds, acc, wave, lane);
  if (wave == 0 && key < p.Skv) {
    float* dkr = reinterpret_cast<float*>(p.dk) + b * p.dk_sb + hk * p.dk_sh + static_cast<int64_t>(key) * p.dk_ss;
    float* dvr = reinterpret_cast<float*>(p.dv) + b * p.dv_sb + hk * p.dv_sh + static_cast<int64_t>(key) * p.dv_ss;
    store_acc_row_f32<DB>(dkr, acc, p.scale, D, g);
    store_acc_row_f32<DB>(dvr, acc + DB, 1.0f, D, g);
  }
}

template <int DP, bool SOFTCAP>
__global__ __launch_bounds__(kThreads, kF32mDqBlocks<DP>) void bwd_f32m_dq_kernel(const BwdParams p) {
  using T = F32WaveTile<DP>;
  constexpr int PITCH = T::PITCH;
  constexpr int HALF = DP / 2;
  constexpr int DB = DP / 32;
  static_assert(3 * 64 * 16 * DB <= 4 * 2 * kM32 * PITCH, "reduction fits in the tiles");
  __shared__ __attribute__((aligned(16))) float lds[4 * 2 * kM32 * PITCH];
  __shared__ __attribute__((aligned(16))) float dos[kM32 * PITCH];  // the 32 rows' dO, shared
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;
  float* kt = lds + wave * 2 * kM32 * PITCH;
  float* vt = kt + kM32 * PITCH;

  // heaviest row blocks (causal: the last) first, all heads at once
  const int units = p.B * p.Hq;
  const int n_rb = (p.Sq + kM32 - 1) / kM32;
  const int jb = static_cast<int>(blockIdx.x) / units;
  const int bh = static_cast<int>(blockIdx.x) - jb * units;
  const int rb = p.causal ? n_rb - 1 - jb : jb;
  const int b = bh / p.Hq;
  const int h = bh - b * p.Hq;
  const int hk = h / p.ratio;
  const int D = p.D;
  const int q0 = rb * kM32;
  const int qrow = q0 + l32;
  const int qa = p.q_offset + qrow;
  const int qa0 = p.q_offset + q0;
  const int kv_lo = p.window > 0 ? max(0, qa0 - p.window + 1) : 0;
  const int kv_hi = p.causal ? min(p.Skv, p.q_offset + min(q0 + kM32, p.Sq)) : p.Skv;
  const int t_lo = kv_lo / kM32;
  const int nt = kv_hi > kv_lo ? (kv_hi + kM32 - 1) / kM32 - t_lo : 0;

  // Q^T operand in registers; dO^T (the same for all four waves) from LDS
  float qreg[HALF];
  load_half_row_f32<DP>(reinterpret_cast<const float*>(p.q) + b * p.q_sb + h * p.q_sh +
                            static_cast<int64_t>(min(qrow, p.Sq - 1)) * p.q_ss, D, g, qreg);
  {
    const float* dob = reinterpret_cast<const float*>(p.dout) + b * p.do_sb + h * p.do_sh;
    for (int idx = tid; idx < kM32 * T::CPR; idx += kThreads) {
      const int r = idx / T::CPR;
      const int c4 = idx - r * T::CPR;
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      if (4 * c4 < D) {
        x = *reinterpret_cast<const f32x4*>(dob + static_cast<int64_t>(min(q0 + r, p.Sq - 1)) * p.do_ss + 4 * c4);
      }
      *reinterpret_cast<f32x4*>(dos + r * PITCH + 4 * c4) = x;
    }
  }
  const int64_t ws = static_cast<int64_t>(bh) * p.sq_pad + qrow;  // qrow < sq_pad
  const float l2 = p.lse2[ws];
  const float di = p.di[ws];
  const float* kb = reinterpret_cast<const float*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const float* vb = reinterpret_cast<const float*>(p.v) + b * p.v_sb + hk * p.v_sh;

  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.0f;
    if constexpr (kF32mDqBlocks<DP> == 1) pin_agpr(acc[db]);
  }
  T kn, vn;
  if (wave < nt) {
    kn.load(kb, p.k_ss, (t_lo + wave) * kM32, p.Skv - 1, D, lane);
    vn.load(vb, p.v_ss, (t_lo + wave) * kM32, p.Skv - 1, D, lane);
  }
  __syncthreads();  // dO tile written
  for (int t = wave; t < nt; t += 4) {
    const int k0 = (t_lo + t) * kM32;
    kn.store(kt, lane);
    vn.store(vt, lane);
    wave_lds_order();
    if (t + 4 < nt) {
      kn.load(kb, p.k_ss, k0 + 4 * kM32, p.Skv - 1, D, lane);
      vn.load(vb, p.v_ss, k0 + 4 * kM32, p.Skv - 1, D, lane);
    }

    f32x16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = 0.0f;
      dp[r] = 0.0f;
    }
    const float* krow = kt + l32 * PITCH + g * HALF;
    const float* vrow = vt + l32 * PITCH + g * HALF;
    const float* dorow = dos + l32 * PITCH + g * HALF;
#pragma unroll
    for (int ks = 0; ks < HALF; ++ks) {
      s = mfma_f32(krow[ks], qreg[ks], s);
      dp = mfma_f32(vrow[ks], dorow[ks], dp);
    }
    const bool need_mask = k0 + kM32 > p.Skv || q0 + kM32 > p.Sq || (p.causal && k0 + kM32 - 1 > qa0) ||
                           (p.window > 0 && k0 < qa0 + kM32 - p.window);
    float dsv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      bool ok = true;
      if (need_mask) {
        const int kk = k0 + 8 * (r >> 2) + 4 * g + (r & 3);
        ok = kk < p.Skv && qrow < p.Sq && (!p.causal || kk <= qa) && (p.window <= 0 || kk >= qa - p.window + 1);
      }
      float pr;
      f32_pds<SOFTCAP>(p, s[r], dp[r], l2, di, ok, pr, dsv[r]);
    }
    // dQ^T[d, row] += K[key, d] dS[row, key]
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kk = 8 * (r >> 2) + 4 * g + (r & 3);
#pragma unroll
      for (int db = 0; db < DB; ++db) acc[db] = mfma_f32(kt[kk * PITCH + 32 * db + l32], dsv[r], acc[db]);
    }
    if constexpr (kF32mDqBlocks<DP> == 1) {
#pragma unroll
      for (int db = 0; db < DB; ++db) pin_agpr(acc[db]);
    }
    wave_lds_order();
  }

  wave_reduce4<DB>(lds, acc, wave, lane);
  if (wave == 0 && qrow < p.Sq) {
    float* dqr = reinterpret_cast<float*>(p.dq) + b * p.dq_sb + h * p.dq_sh + static_cast<int64_t>(qrow) * p.dq_ss;
    store_acc_row_f32<DB>(dqr, acc, p.scale, D, g);
  }
}

template <int DP, bool SOFTCAP>
void launch_f32m_dp(const BwdParams& p, hipStream_t s) {
  const int grid_dkv = p.B * p.Hkv * ((p.Skv + kM32 - 1) / kM32);
  const int grid_dq = p.B * p.Hq * ((p.Sq + kM32 - 1) / kM32);
  if (grid_dkv > 0) {
    hipLaunchKernelGGL((bwd_f32m_dkdv_kernel<DP, SOFTCAP>), dim3(grid_dkv), dim3(kThreads), 0, s, p);
  }
  hipLaunchKernelGGL((bwd_f32m_dq_kernel<DP, SOFTCAP>), dim3(grid_dq), dim3(kThreads), 0, s, p);
}

void launch_f32(const BwdParams& p, bool softcap, int grid_pre, hipStream_t s) {
  hipLaunchKernelGGL((bwd_pre_kernel<F32Tag>), dim3(grid_pre), dim3(kThreads), 0, s, p);
  if (p.D <= 64) {
    softcap ? launch_f32m_dp<64, true>(p, s) : launch_f32m_dp<64, false>(p, s);
  } else if (p.D <= 128) {
    softcap ? launch_f32m_dp<128, true>(p, s) : launch_f32m_dp<128, false>(p, s);
  } else {
    softcap ? launch_f32_dp<256, true>(p, s) : launch_f32_dp<256, false>(p, s);
  }
}

template <typename Tag, int DP, bool SOFTCAP, int DV = DP>
void launch_main(const BwdParams& p, int grid_dkv, int grid_dq, hipStream_t s) {
  if (grid_dkv > 0) {
    hipLaunchKernelGGL((bwd_dkdv_kernel<Tag, DP, DV, SOFTCAP>), dim3(grid_dkv), dim3(kThreads), 0, s, p);
  }
  hipLaunchKernelGGL((bwd_dq_kernel<Tag, DP, DV, SOFTCAP>), dim3(grid_dq), dim3(kThreads), 0, s, p);
}

template <typename Tag>
void launch_tag(const BwdParams& p, bool softcap, int grid_pre, int grid_dkv, int grid_dq,
                hipStream_t s) {
  hipLaunchKernelGGL((bwd_pre_kernel<Tag>), dim3(grid_pre), dim3(kThreads), 0, s, p);
  if (p.D <= 64) {
    softcap ? launch_main<Tag, 64, true>(p, grid_dkv, grid_dq, s)
            : launch_main<Tag, 64, false>(p, grid_dkv, grid_dq, s);
  } else if (p.D <= 128) {
    softcap ? launch_main<Tag, 128, true>(p, grid_dkv, grid_dq, s)
            : launch_main<Tag, 128, false>(p, grid_dkv, grid_dq, s);
  } else if (p.D <= 192) {
    if (p.Dv <= 128) {  // V narrower than q / k (the MLA module's)
      softcap ? launch_main<Tag, 192, true, 128>(p, grid_dkv, grid_dq, s)
              : launch_main<Tag, 192, false, 128>(p, grid_dkv, grid_dq, s);
    } else {
      softcap ? launch_main<Tag, 192, true>(p, grid_dkv, grid_dq, s)
              : launch_main<Tag, 192, false>(p, grid_dkv, grid_dq, s);
    }
  } else {
    softcap ? launch_main<Tag, 256, true>(p, grid_dkv, grid_dq, s)
            : launch_main<Tag, 256, false>(p, grid_dkv, grid_dq, s);
  }
}

int64_t sq_padded(int32_t seqlen_q) {
  return (static_cast<int64_t>(seqlen_q) + kQTile - 1) / kQTile * kQTile;
}

}  // namespace

size_t attn_bwd_workspace_bytes(int32_t batch, int32_t heads_q, int32_t seqlen_q) {
  return static_cast<size_t>(2) * batch * heads_q * sq_padded(seqlen_q) * sizeof(float);
}

int launch_attn_bwd(const ffa_attn_bwd_args& a, hipStream_t stream) {
  BwdParams p{};
  p.q = static_cast<const uint16_t*>(a.q);
  p.k = static_cast<const uint16_t*>(a.k);
  p.v = static_cast<const uint16_t*>(a.v);
  p.o = static_cast<const uint16_t*>(a.o);
  p.dout = static_cast<const uint16_t*>(a.dout);
  p.lse = a.lse;
  p.dq = static_cast<uint16_t*>(a.dq);
  p.dk = static_cast<uint16_t*>(a.dk);
  p.dv = static_cast<uint16_t*>(a.dv);
  p.q_sb = a.q_stride[0];
  p.q_sh = a.q_stride[1];
  p.q_ss = a.q_stride[2];
  p.k_sb = a.k_stride[0];
  p.k_sh = a.k_stride[1];
  p.k_ss = a.k_stride[2];
  p.v_sb = a.v_stride[0];
  p.v_sh = a.v_stride[1];
  p.v_ss = a.v_stride[2];
  p.o_sb = a.o_stride[0];
  p.o_sh = a.o_stride[1];
  p.o_ss = a.o_stride[2];
  p.do_sb = a.do_stride[0];
  p.do_sh = a.do_stride[1];
  p.do_ss = a.do_stride[2];
  p.dq_sb = a.dq_stride[0];
  p.dq_sh = a.dq_stride[1];
  p.dq_ss = a.dq_stride[2];
  p.dk_sb = a.dk_stride[0];
  p.dk_sh = a.dk_stride[1];
  p.dk_ss = a.dk_stride[2];
  p.dv_sb = a.dv_stride[0];
  p.dv_sh = a.dv_stride[1];
  p.dv_ss = a.dv_stride[2];
  p.l_sb = a.lse_stride[0];
  p.l_sh = a.lse_stride[1];
  p.l_ss = a.lse_stride[2];
  p.B = a.batch;
  p.Hq = a.heads_q;
  p.Hkv = a.heads_kv;
  p.Sq = a.seqlen_q;
  p.Skv = a.seqlen_kv;
  p.D = a.head_dim;
  p.Dv = a.v_head_dim > 0 ? a.v_head_dim : a.head_dim;
  p.q_offset = a.q_offset;
  p.causal = a.causal ? 1 : 0;
  p.window = clamp_window(a.window, a.q_offset, a.seqlen_q);
  p.ratio = a.heads_q / a.heads_kv;
  p.sq_pad = static_cast<int>(sq_padded(a.seqlen_q));
  p.n_qt = p.sq_pad / kQTile;
  p.n_kt = (a.seqlen_kv + kDkvKeys - 1) / kDkvKeys;
  const bool softcap = a.softcap > 0.0f;
  if (softcap) {
    p.score_mul = a.scale / a.softcap;
    p.cap_mul = a.softcap * kLog2e;
    p.tanh_mul = 2.0f * kLog2e * a.scale / a.softcap;
  } else {
    p.score_mul = a.scale * kLog2e;
    p.cap_mul = 0.0f;
    p.tanh_mul = 0.0f;
  }
  p.scale = a.scale;
  float* ws = static_cast<float*>(a.workspace);
  const int64_t rows = static_cast<int64_t>(a.batch) * a.heads_q * p.sq_pad;
  p.lse2 = ws;
  p.di = ws + rows;

  const int64_t grid_pre = rows / 32;
  const int64_t grid_dq = static_cast<int64_t>(p.n_qt) * a.batch * a.heads_q;
  const int64_t grid_dkv = static_cast<int64_t>(p.n_kt) * a.batch * a.heads_kv;
  if (grid_pre > 0x7fffffff || grid_dq > 0x7fffffff || grid_dkv > 0x7fffffff) {
    return FFA_ERR_TOO_LARGE;
  }
  if (grid_pre == 0 || grid_dq == 0) return FFA_OK;
  // the forward's grid order: each XCD runs its units one after another (their K / V,
  // or Q / dO, stay in its L2) and interleaves only its last ones. At the north-star
  // shape the step reads 0.53 GB less than with every pair interleaved (4.24 against
  // 4.78 GB per backward); time within +-0.5 %, +5 % at head_dim 64.
  prefill_grid_order(p.causal, static_cast<int64_t>(a.batch) * a.heads_q, grid_dq, p.xcd_group_dq,
                     p.xcd_remap_dq);
  prefill_grid_order(p.causal, static_cast<int64_t>(a.batch) * a.heads_kv, grid_dkv,
                     p.xcd_group_dkv, p.xcd_remap_dkv);
  if (a.dtype == FFA_DTYPE_FP32) {
    // 32-row / 32-key workgroups
    const int64_t g32 = static_cast<int64_t>(a.batch) * a.heads_q * ((a.seqlen_q + 31) / 32) +
                        static_cast<int64_t>(a.batch) * a.heads_kv * ((a.seqlen_kv + 31) / 32);
    if (g32 > 0x7fffffff) return FFA_ERR_TOO_LARGE;
    launch_f32(p, softcap, static_cast<int>(grid_pre), stream);
  } else if (a.dtype == FFA_DTYPE_BF16) {
    launch_tag<Bf16Tag>(p, softcap, static_cast<int>(grid_pre), static_cast<int>(grid_dkv),
                        static_cast<int>(grid_dq), stream);
  } else {
    launch_tag<F16Tag>(p, softcap, static_cast<int>(grid_pre), static_cast<int>(grid_dkv),
                       static_cast<int>(grid_dq), stream);
  }
  return hipGetLastError() == hipSuccess ? FFA_OK : FFA_ERR_LAUNCH;
}

}  // namespace ffa
