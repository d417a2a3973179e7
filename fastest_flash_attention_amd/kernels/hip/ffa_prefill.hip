// Fused forward attention (prefill) for gfx950.
//
// Semantics follow flash_attn_cpu_forward (reference kernels/cpu_reference.py:132-312):
// scores in fp32, softcap before masking, causal / one-sided sliding window relative to
// q_offset, GQA head map h -> h / (Hq / Hkv), natural-log LSE.
//
// Work decomposition: one workgroup (4 waves, 256 threads) per (batch, q-head, 128-row
// query tile); each wave owns 32 query rows for the whole KV sweep. The narrow-V
// kernels on sequences of 4096 rows or more use 8 waves and 256-row tiles instead.
// Inputs must be 16-byte aligned with head_dim % 8 == 0 (the host pads / copies
// otherwise).
//
// Per KV tile of BN keys (BN = 64 for head_dim <= 128, 32 above):
//   S^T[key, q] = K Q^T   v_mfma_f32_32x32x16 with K (LDS) as A and Q (registers) as B,
//                         so lane l holds BN/2 scores of ONE query (l % 32): the row max
//                         needs one lane swap (l ^ 32), the row sum none until the end.
//   P = exp2(S*c - m*c)   fp32 (c = scale*log2e, one FMA per score); m moves only when
//                         the max grows by more than 2^8, so O and l are rarely rescaled.
//                         The reference's per-tile 1e-30 floor of the row sum is added
//                         at the end (ref_tile_floor, masked_row_lse).
//   O^T[d, q] += V^T P^T  B = P packed to 16 bit straight from the S^T accumulators;
//                         A = V^T from LDS by two ds_read_b64_tr_b16 (4 keys x 1 dim per
//                         lane each) on the row-major V tile: the key order they produce
//                         is the key order the S^T accumulator layout hands to P.
// Data movement: K and V tiles go global -> LDS with global_load_lds_dwordx4 (no VGPR
// staging), double-buffered, issued one tile ahead; the global side picks the 16-byte
// chunk each lane fetches so the LDS image is XOR-swizzled per row, which makes the
// K operand reads and the transposed V reads bank-conflict free. S^T of tile t+1 is
// computed during the softmax and P V of tile t (its k-steps spread over the 16-key
// chunks of P V for head_dim <= 128, ahead of them above) so MFMA and VALU work overlap
// within a wave; one barrier per tile.
// Causal / window tiles outside a workgroup's band are never loaded; tiles past a
// wave's causal band skip the wave's work; element masks run only on band-edge tiles.
// Grid order: heaviest causal query tiles first, and (when the grid is a multiple of
// 8) consecutive tiles of one head are placed on one XCD so its K/V stay in that L2.

#include <type_traits>

#include "ffa_common.h"
#include "ffa_grid.h"
#include "ffa_internal.h"
#include "ffa_prefill_common.h"

namespace ffa {
namespace {

using namespace pf;

constexpr int kThreads = 256;
constexpr int kBlockM = 128;
// With a block mask, a workgroup first lists the KV tiles that hold any visible key for
// its rows and visits only those; sweeps longer than this many tiles visit every tile.
constexpr int kMaxLiveTiles = 2048;
// Key tile of the narrow-V kernels (head_dim 192, V <= 128 dims): K 2 x 24 KiB + V 2 x
// 16 KiB of LDS still fit two workgroups per CU (the block mask's tile list is dynamic
// LDS). On MI355X at the MLA prefill shape (B 2, H 32, S 4096, causal): 0.332 ms against
// 0.351 ms with 32-key tiles and 0.397 ms for the zero-padded V on the 192-dim kernel.
constexpr int kNarrowBN = 64;
constexpr int kTileFull = 0x8000;  // list entry flag: the block mask keeps the whole tile
constexpr size_t kLiveLdsBytes = 8 * sizeof(int) + kMaxLiveTiles * sizeof(uint16_t);
// Workgroup -> (batch x head, query tile j; j = 0 is the heaviest causal tile): the
// XCD-aware order of ffa_grid.h, with the group / remap the launcher chose.
__device__ inline void work_item(const PrefillParams& p, int bid, int& bh, int& jq) {
  prefill_work_item(bid, static_cast<int>(gridDim.x), p.n_qt, p.xcd_group, p.xcd_remap, bh, jq);
}

template <int DP, int BN, int NW = 4>
struct Shape {
  static constexpr int CPR = DP / 8;            // 16-byte chunks per row
  static constexpr int TILE = BN * DP;          // elements per K (or V) tile
  static constexpr int LPT = BN * CPR / (64 * NW);  // direct loads per thread per tile
  static constexpr int NB = BN / 32;
  static constexpr int NC = BN / 16;
  static constexpr int KS = DP / 16;
  static constexpr int DB = DP / 32;
  static_assert(BN * CPR % (64 * NW) == 0, "tile must split evenly over the workgroup");
};

// Two workgroups per CU (2 waves per SIMD, <= 256 VGPRs) up to head_dim 192; the
// 256-dim variant keeps 128 fp32 accumulators per lane and runs one wave per SIMD.
// head_dim 64 without softcap fits 168 VGPRs without spills: three workgroups per CU
// (+4 % at S = 8192 on MI355X; with softcap that bound spills). head_dim 32 needs
// fewer than 168 VGPRs anyway.
template <int DP, bool SOFTCAP>
constexpr int kMinBlocks = (DP == 64 && !SOFTCAP) ? 3 : (DP <= 192 ? 2 : 1);

// DV: the V tile / O accumulator width (<= DP). It is DP except for head_dim 192 over
// a V of at most 128 dims (the MLA prefill's V, which its caller would otherwise
// zero-pad to 192): P V then runs over the 128 real dims only.
// NW: waves per workgroup, each owning 32 query rows (a workgroup covers 32 NW rows).
// Four, two workgroups per CU, except the narrow-V kernels on long sequences: eight
// waves, one workgroup per CU, so each K/V tile is loaded once for 256 rows (half the
// tile loads per FLOP of two 4-wave workgroups). On MI355X at the MLA prefill shape
// (B 2, H 32, S 4096): +4-6 % causal, +5 % non-causal, +-0-2 % with softcap, outputs
// bit-identical, and the kernel stops spilling; the head_dim-128 kernels lose 3-8 %
// with eight waves, and shorter causal sequences lose too (-10 % at S = 2048).
template <typename Tag, int DP, int DV, int BN, bool SOFTCAP, int NW>
__global__ __launch_bounds__((64 * NW), (kMinBlocks<DP, SOFTCAP> * 4 / NW)) void prefill_kernel(const PrefillParams p) {
  constexpr int BM = 32 * NW;  // query rows per workgroup
  using S = Shape<DP, BN, NW>;   // Q, K tiles, S^T
  using SV = Shape<DV, BN, NW>;  // V tiles, O^T
  using E = Elem<Tag>;
  __shared__ __attribute__((aligned(1024))) uint16_t k_lds[2][S::TILE];
  __shared__ __attribute__((aligned(1024))) uint16_t v_lds[2][SV::TILE];
  // Block mask: the tiles to visit, in dynamic LDS that only launches with a block mask
  // request (kLiveLdsBytes), so that the K/V buffers alone set the occupancy otherwise.
  extern __shared__ __attribute__((aligned(16))) int live_dyn[];
  int* const live_cnt = live_dyn;                                       // [NW <= 8]
  uint16_t* const live_lds = reinterpret_cast<uint16_t*>(live_dyn + 8);  // [kMaxLiveTiles]

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;

  int bh, jq;
  work_item(p, blockIdx.x, bh, jq);
  bh = __builtin_amdgcn_readfirstlane(bh);  // uniform: keeps the tile bases in SGPRs
  jq = __builtin_amdgcn_readfirstlane(jq);
  const int qt = p.causal ? (p.n_qt - 1 - jq) : jq;
  const int b = bh / p.Hq;
  const int h = bh - b * p.Hq;
  const int hk = h / p.ratio;

  const uint16_t* __restrict__ qbase = p.q + b * p.q_sb + h * p.q_sh;
  const char* kbytes = reinterpret_cast<const char*>(p.k + b * p.k_sb + hk * p.k_sh);
  const char* vbytes = reinterpret_cast<const char*>(p.v + b * p.v_sb + hk * p.v_sh);
  const int D = p.D;
  const int Skv = p.Skv;

  const int q0 = qt * BM;
  const int q_last = min(q0 + BM, p.Sq) - 1;
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
  // block mask: this lane's row block in the expanded key mask
  const uint64_t* kmask_row =
      p.kmask != nullptr ? p.kmask + static_cast<int64_t>(min(qrow, p.Sq - 1) / p.ref_bq) * p.kmask_words
                         : nullptr;

  // Block mask: list the tiles of [t_begin, t_begin + nt) whose keys have any set bit
  // in the key mask of the workgroup's rows (rows q0 .. q_last, i.e. reference row
  // blocks rb0 .. rb1). A tile without one contributes nothing (every score is masked),
  // so skipping it changes no result; the fully-masked-row LSE comes from the
  // reference's visited-tile counts, not from the tiles this kernel visits.
  const bool use_list = p.kmask != nullptr && nt <= kMaxLiveTiles;
  int n_it = nt;  // iterations of the sweep: nt, or the live tiles with a block mask
  if (use_list) {
    const int rb0 = q0 / p.ref_bq;
    const int rb1 = q_last / p.ref_bq;
    int n_live = 0;
    for (int base = 0; base < nt; base += 64 * NW) {
      const int i = base + tid;
      bool live = false;
      bool full = true;  // every key of the tile set for every row: no element mask
      if (i < nt) {
        const int kt0 = (t_begin + i) * BN;
        const uint64_t all = BN < 64 ? (uint64_t{1} << (BN & 63)) - 1 : ~uint64_t{0};
        for (int rb = rb0; rb <= rb1; ++rb) {
          uint64_t w = p.kmask[static_cast<int64_t>(rb) * p.kmask_words + (kt0 >> 6)];
          if constexpr (BN < 64) w = (w >> (kt0 & 63)) & all;
          live = live || w != 0;
          full = full && w == all;
        }
      }
      const uint64_t bal = __ballot(live);
      if (lane == 0) live_cnt[wave] = __popcll(bal);
      __syncthreads();
      int off = n_live;
      for (int w = 0; w < wave; ++w) off += live_cnt[w];
      if (live) {
        live_lds[off + __popcll(bal & ((uint64_t{1} << lane) - 1))] =
            static_cast<uint16_t>(i | (full ? kTileFull : 0));
      }
#pragma unroll
      for (int w = 0; w < NW; ++w) n_live += live_cnt[w];
      __syncthreads();
    }
    n_it = n_live;
  }
  auto tile_at = [&](int i) {
    return t_begin + (use_list ? static_cast<int>(live_lds[i] & (kTileFull - 1)) : i);
  };
  // whether the block mask needs element tests on sweep position i
  auto kmask_partial = [&](int i) {
    return p.kmask != nullptr && !(use_list && (live_lds[i] & kTileFull));
  };

  // Scores stay in raw units until the exponent: p = exp2(s*c - m*c), with s = q.k and
  // c = scale*log2e, or with softcap s = tanh(q.k * scale / cap) and c = cap*log2e.
  const float c = SOFTCAP ? p.cap_mul : p.score_mul;
  const float tanh_mul = 2.0f * kLog2e * p.score_mul;  // softcap: e^{2y} = exp2(s * tanh_mul)

  // ---- direct global -> LDS tile loads -------------------------------------------
  // Load j of this thread fills chunk position P = (4j + wave) * 64 + lane of the tile
  // (each wave instruction writes 1 KiB of LDS); row = P / CPR, and the global chunk
  // fetched is (P % CPR) ^ swz(row), clamped below head_dim (padding dims multiply a
  // zero Q dim or feed O dims that are never stored).
  const int dchunks = D >> 3;
  constexpr bool NARROW = DV < DP;  // V (and O's computed dims) narrower than Q / K
  const int dvchunks = NARROW ? p.Dv >> 3 : dchunks;
  uint32_t k_off[S::LPT], v_off[SV::LPT];
#pragma unroll
  for (int j = 0; j < S::LPT; ++j) {
    const int pos = (NW * j + wave) * 64 + lane;
    const int row = pos / S::CPR;
    const int q = pos - row * S::CPR;
    const int kc = min(q ^ kswz<DP>(row), dchunks - 1);
    k_off[j] = static_cast<uint32_t>(row * p.k_ss * 2 + kc * 16);
  }
#pragma unroll
  for (int j = 0; j < SV::LPT; ++j) {
    const int pos = (NW * j + wave) * 64 + lane;
    const int row = pos / SV::CPR;
    const int q = pos - row * SV::CPR;
    const int vc = min(q ^ vswz<DV>(row), dvchunks - 1);
    v_off[j] = static_cast<uint32_t>(row * p.v_ss * 2 + vc * 16);
  }
  // The loads are issued from inline asm (wave-uniform tile base + 32-bit lane offset):
  // the compiler neither holds a 64-bit address per load nor guards later LDS reads
  // with vmcnt waits; completion is the explicit wait_vmcnt0 before each tile barrier.
  // K and V tiles are issued in order, so each tensor keeps a running tile base that
  // advances by one tile per issue (one 64-bit scalar add per tile).
  const int64_t k_tile_bytes = static_cast<int64_t>(BN) * p.k_ss * 2;
  const int64_t v_tile_bytes = static_cast<int64_t>(BN) * p.v_ss * 2;
  const int t_full = Skv / BN;  // tiles below this index hold BN keys
  auto issue_tile = [&](auto shp, const char*& tb, int64_t tile_bytes, int64_t stride,
                        const auto& off, uint16_t* dst, int t) __attribute__((always_inline)) {
    using SH = decltype(shp);
    if (t < t_full) {
#pragma unroll
      for (int j = 0; j < SH::LPT; ++j) {
        load_lds16_async(tb, off[j], lds_addr(dst + (NW * j + wave) * 512));
      }
    } else {
      // last tile: rows past Skv re-read row Skv-1 (their scores are masked to -inf)
      const int kt0 = t * BN;
#pragma unroll
      for (int j = 0; j < SH::LPT; ++j) {
        const int row = ((NW * j + wave) * 64 + lane) / SH::CPR;
        const int over = max(0, kt0 + row - (Skv - 1));
        const uint32_t back = static_cast<uint32_t>(over * stride * 2);
        load_lds16_async(tb, off[j] - back, lds_addr(dst + (NW * j + wave) * 512));
      }
    }
    tb += tile_bytes;
  };
  // LDS byte address of this wave's first load slot in buffer 0 of K and of V (uniform,
  // SGPRs): load j of buffer b writes at base + b * TILE * 2 + j * NW KiB.
  const uint32_t k_wlds = __builtin_amdgcn_readfirstlane(lds_addr(&k_lds[0][0]) + wave * 1024);
  const uint32_t v_wlds = __builtin_amdgcn_readfirstlane(lds_addr(&v_lds[0][0]) + wave * 1024);
  // A tile known to hold BN keys (no tail handling, no test) into buffer B.
  auto issue_full = [&](auto shp, const char*& tb, int64_t tile_bytes, const auto& off,
                        uint32_t wlds, auto buf) __attribute__((always_inline)) {
    using SH = decltype(shp);
    constexpr uint32_t B = decltype(buf)::value;
#pragma unroll
    for (int j = 0; j < SH::LPT; ++j) {
      load_lds16_async(tb, off[j], wlds + B * SH::TILE * 2 + j * 1024 * NW);
    }
    tb += tile_bytes;
  };
  const char* k_next = kbytes + static_cast<int64_t>(t_begin) * k_tile_bytes;
  const char* v_next = vbytes + static_cast<int64_t>(t_begin) * v_tile_bytes;
  // Issue K (V) tile t: in tile order the running pointer is already there; a live-tile
  // list can jump, so there the pointer is set from t first.
  auto issue_k = [&](int t, uint16_t* dst) __attribute__((always_inline)) {
    if (use_list) k_next = kbytes + static_cast<int64_t>(t) * k_tile_bytes;
    issue_tile(S{}, k_next, k_tile_bytes, p.k_ss, k_off, dst, t);
  };
  auto issue_v = [&](int t, uint16_t* dst) __attribute__((always_inline)) {
    if (use_list) v_next = vbytes + static_cast<int64_t>(t) * v_tile_bytes;
    issue_tile(SV{}, v_next, v_tile_bytes, p.v_ss, v_off, dst, t);
  };

  // ---- per-lane LDS operand addresses (element offsets inside one tile buffer) ----
  // K operand of k-step ks for 32-key block nb: row 32nb + l32, chunk 2ks + g. The row
  // swizzle XORs only the low log2(KSW) bits of the chunk index, so the address is a
  // per-lane part for ks % KP plus the compile-time KSW * 8 * (ks / KP) (one register
  // per KP k-steps instead of one per k-step: 4 rather than 12 at head_dim 192).
  constexpr int KSW = (DP == 32) ? 4 : (DP == 64 || DP == 192) ? 8 : 16;
  constexpr int KP = KSW / 2 < S::KS ? KSW / 2 : S::KS;
  int k_rd4[KP];
#pragma unroll
  for (int kp = 0; kp < KP; ++kp) k_rd4[kp] = l32 * DP + (((2 * kp + g) ^ kswz<DP>(l32)) << 3);
  auto k_rd = [&](int ks) __attribute__((always_inline)) { return k_rd4[ks % KP] + KSW * 8 * (ks / KP); };
  // V^T operand of dim block db: this lane supplies row (key) rowoff of a 4-key group
  // and dims colw .. colw+3 of the block (ds_read_b64_tr_b16 law: lanes 4k..4k+3 of a
  // 16-lane group supply row k, lane i receives dim i of rows 0..3).
  const int rowoff = 4 * g + ((lane & 15) >> 2);
  const int colw = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  int v_rd[SV::DB];
#pragma unroll
  for (int db = 0; db < SV::DB; ++db) {
    const int cg = 4 * db + (colw >> 3);
    v_rd[db] = rowoff * DV + ((cg ^ vswz<DV>(rowoff)) << 3) + (colw & 7);
  }

  // Q^T as the B operand: lane holds row qrow (clamped: rows past Sq are never
  // stored), dims 16*ks + 8g .. +7. The loads are issued from inline asm ahead of the
  // first tiles' global -> LDS loads, so that one memory round trip serves both: the
  // compiler, which would wait for compiler-issued Q loads before issuing anything
  // else, does not see them, and the prologue's wait for K(0) also covers Q (loads
  // retire in issue order). On MI355X: -1 round trip of start-up per workgroup.
  u32x4 qreg[S::KS];
  {
    const uint16_t* qr = qbase + static_cast<int64_t>(min(qrow, p.Sq - 1)) * p.q_ss;
#pragma unroll
    for (int ks = 0; ks < S::KS; ++ks) {
      const int d0 = min(16 * ks + 8 * g, D - 8);
      asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(qreg[ks]) : "v"(qr + d0) : "memory");
    }
  }
  // Once the loads are complete (wait_q below): a negative scale is applied as
  // q.k * scale = (-q).k * |scale|, the sign bits of Q flipped (exact), so the kernel's
  // multiplier stays positive; dims past head_dim are zero.
  auto finish_q = [&]() __attribute__((always_inline)) {
    const uint32_t qx = p.q_neg ? 0x80008000u : 0u;
#pragma unroll
    for (int ks = 0; ks < S::KS; ++ks) {
      qreg[ks] = (16 * ks + 8 * g < D) ? (qreg[ks] ^ qx) : u32x4{0u, 0u, 0u, 0u};
    }
  };

  f32x16 oacc[SV::DB];
#pragma unroll
  for (int db = 0; db < SV::DB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.0f;
  }
  float m_run = kNegInf;
  float l_run = 0.0f;
  float negmc = 0.0f;   // -m_run * c (0 while m_run = -inf)
  float lim = -1.0f;    // chunk exp-sum limit; < 0: no max yet, the first chunk sets it

  // S^T of one tile. FENCE keeps each k-step's MFMAs behind a scheduling barrier (the
  // K operand reads stay one k-step ahead). Without it (the fast step at head_dim >= 192,
  // where S^T(t+1) is a block of 24-32 MFMAs ahead of softmax(t)) the compiler spreads
  // the tile's max and softcap VALU work of tile t between those MFMAs: +2 % at the MLA
  // prefill shape, +5-6 % at head_dim 192 with softcap and at 256 on MI355X,
  // bit-identical (two head_dim-192 kernels then use 12 B per lane of scratch, reloaded in
  // the general-step loops, not in the fast loop; still faster).
  auto qk = [&](const uint16_t* kl, f32x16 (&sacc)[S::NB], auto fence) __attribute__((always_inline)) {
    constexpr bool FENCE = decltype(fence)::value;
#pragma unroll
    for (int nb = 0; nb < S::NB; ++nb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[nb][r] = 0.0f;
    }
    // K operands one k-step ahead of the MFMAs that consume them
    u32x4 a_cur[S::NB], a_nxt[S::NB];
#pragma unroll
    for (int nb = 0; nb < S::NB; ++nb) {
      a_cur[nb] = *reinterpret_cast<const u32x4*>(kl + k_rd(0) + nb * 32 * DP);
    }
    // head_dim 192 (32-key tiles, one 32-key block): the 12 k-steps would form one chain
    // of dependent MFMAs, so even and odd k-steps go to two accumulators summed at the
    // end (+2.3 % at cfg5 on MI355X; with softcap it spills, and at 256 it is slower)
    if constexpr (DP == 192 && BN == 32 && !SOFTCAP) {
      f32x16 s_odd;
#pragma unroll
      for (int r = 0; r < 16; ++r) s_odd[r] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < S::KS; ++ks) {
        if (ks + 1 < S::KS) a_nxt[0] = *reinterpret_cast<const u32x4*>(kl + k_rd(ks + 1));
        __builtin_amdgcn_sched_barrier(0);
        if (ks & 1) {
          s_odd = E::mfma32(a_cur[0], qreg[ks], s_odd);
        } else {
          sacc[0] = E::mfma32(a_cur[0], qreg[ks], sacc[0]);
        }
        a_cur[0] = a_nxt[0];
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[0][r] += s_odd[r];
      return;
    }
#pragma unroll
    for (int ks = 0; ks < S::KS; ++ks) {
      if (ks + 1 < S::KS) {
#pragma unroll
        for (int nb = 0; nb < S::NB; ++nb) {
          a_nxt[nb] = *reinterpret_cast<const u32x4*>(kl + k_rd(ks + 1) + nb * 32 * DP);
        }
      }
      if constexpr (FENCE) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int nb = 0; nb < S::NB; ++nb) sacc[nb] = E::mfma32(a_cur[nb], qreg[ks], sacc[nb]);
#pragma unroll
      for (int nb = 0; nb < S::NB; ++nb) a_cur[nb] = a_nxt[nb];
    }
  };

  // Online softmax of tile t (scores in sacc) then O^T += V^T P^T from V tile vl.
  // MAYMASK (std::true_type / std::false_type): whether this tile can need an element
  // mask at all; the fast steps below only handle tiles that cannot.
  // With IL it also computes S^T of the next tile into nxt (from the K tile kl, when
  // do_qk): 16-key chunk cc runs k-steps KS cc / NC .. KS (cc + 1) / NC - 1 of it right
  // after the chunk's V reads, their K operands read at the end of the chunk before.
  // S^T alone is two accumulator chains of dependent MFMAs; interleaved with the four
  // P V chains (and with the chunk's exp work) the matrix core rarely waits on a
  // result. On MI355X: +3.7 % at the north-star shape, +10 % with window and softcap.
  // Not for head_dim > 128 (BN = 32 and 128 accumulators: it would spill) nor for the
  // three-workgroup head_dim 64 variant (168 VGPRs).
  constexpr bool IL = DP <= 128 && kMinBlocks<DP, SOFTCAP> <= 2;
  auto softmax_pv = [&](f32x16 (&sacc)[S::NB], int t, const uint16_t* vl, auto maymask,
                        bool kpartial, f32x16 (&nxt)[S::NB], const uint16_t* kl, bool do_qk,
                        auto chunk_hook) __attribute__((always_inline)) {
    constexpr bool MAYMASK = decltype(maymask)::value;
    const int kt0 = t * BN;
    constexpr int KPC = (S::KS + S::NC - 1) / S::NC;
    u32x4 ak[KPC][S::NB];
    auto rd_k = [&](int cc) __attribute__((always_inline)) {
#pragma unroll
      for (int ks = S::KS * cc / S::NC; ks < S::KS * (cc + 1) / S::NC; ++ks) {
#pragma unroll
        for (int nb = 0; nb < S::NB; ++nb) {
          ak[ks - S::KS * cc / S::NC][nb] = *reinterpret_cast<const u32x4*>(kl + k_rd(ks) + nb * 32 * DP);
        }
      }
    };
    if (IL && do_qk) {
#pragma unroll
      for (int nb = 0; nb < S::NB; ++nb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) nxt[nb][r] = 0.0f;
      }
      rd_k(0);
    }
    // Softcap: the scores are kept as r = 1 / (1 + e^{2y}), tanh(y) = 1 - 2r, so the
    // exponent c tanh(y) - m c = c (1 - 2r) - m c is one FMA of r (the FMA that would
    // form tanh from r is folded into it). A masked element is r = +inf (tanh = -inf).
    // LATE_CAP (softcap in the interleaved kernels' fast step): the transform of each
    // chunk's scores runs inside that chunk, beside its S^T(t+1) MFMAs (one MFMA to
    // twelve VALU instructions), instead of as a pass over the whole tile before the
    // chunks; the rare path takes the tile max on raw scores. On MI355X +1 % at cfg3,
    // +1.3 % non-causal GQA with softcap, +3.7 % at head_dim 64 with softcap,
    // bit-identical. The general step (masks) transforms first: a masked score must
    // become r = +inf, which no raw score maps to.
    constexpr bool LATE_CAP = SOFTCAP && IL && !MAYMASK;
    if constexpr (SOFTCAP && !LATE_CAP) {
#pragma unroll
      for (int nb = 0; nb < S::NB; ++nb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          sacc[nb][r] = __builtin_amdgcn_rcpf(1.0f + fast_exp2(sacc[nb][r] * tanh_mul));
        }
      }
    }
    constexpr float kMasked = SOFTCAP ? __builtin_inff() : kNegInf;
    // the tile's row max in score units (softcap: 1 - 2 min r)
    auto tile_max = [&]() __attribute__((always_inline)) {
      if constexpr (LATE_CAP) {
        // raw scores: r = 1 / (1 + 2^x) decreases in x = s * tanh_mul, so the tile's
        // smallest r (largest tanh) is the transform of the largest x: of the largest s,
        // or of the smallest for a negative multiplier (a negative scale). Both are taken
        // on s itself (max of s or of -s), so no product s * tanh_mul is formed here for
        // the compiler to keep live for the chunks' own transform.
        const bool up = tanh_mul >= 0.0f;  // uniform
        float mx = kNegInf;
        if (up) {
#pragma unroll
          for (int nb2 = 0; nb2 < S::NB; ++nb2) {
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[nb2][r]);
          }
        } else {
#pragma unroll
          for (int nb2 = 0; nb2 < S::NB; ++nb2) {
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, -sacc[nb2][r]);
          }
        }
        mx = wave_pair_max(mx);
        const float x = (up ? mx : -mx) * tanh_mul;
        return fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + fast_exp2(x)), 1.0f);
      }
      float mt = SOFTCAP ? __builtin_inff() : kNegInf;
#pragma unroll
      for (int nb2 = 0; nb2 < S::NB; ++nb2) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = SOFTCAP ? fminf(mt, sacc[nb2][r]) : fmaxf(mt, sacc[nb2][r]);
      }
      if constexpr (SOFTCAP) {
        mt = -wave_pair_max(-mt);
        return fmaf(-2.0f, mt, 1.0f);
      } else {
        return wave_pair_max(mt);
      }
    };
    const bool need_mask = MAYMASK && ((kt0 + BN > Skv) || (p.causal && kt0 + BN - 1 > qw0_abs) ||
                                       (p.window > 0 && kt0 < qwl_abs - p.window + 1) ||
                                       kpartial);
    if (need_mask) {
      const int key0 = kt0 + 4 * g;
      // (not in the three-workgroup head_dim 64 kernel: its 168-VGPR budget spills with
      // both paths)
      if (kMinBlocks<DP, SOFTCAP> <= 2 && p.kmask == nullptr && kt0 + BN <= Skv) {
        // Causal / window edges of a full tile without a block mask (the diagonal of a
        // causal sweep, the left edge of a window): element (key0 + off) is visible iff
        // lo <= off <= hi, compares against a compile-time offset per score instead of
        // the general test below.
        const int hi = p.causal ? qa - key0 : 0x7fffffff;
        if (p.window <= 0) {
#pragma unroll
          for (int nb = 0; nb < S::NB; ++nb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int off = 32 * nb + 8 * (r >> 2) + (r & 3);
              sacc[nb][r] = off <= hi ? sacc[nb][r] : kMasked;
            }
          }
        } else {
          const int lo = qa - p.window + 1 - key0;  // no overflow: the host clamps the window
#pragma unroll
          for (int nb = 0; nb < S::NB; ++nb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int off = 32 * nb + 8 * (r >> 2) + (r & 3);
              sacc[nb][r] = (off >= lo && off <= hi) ? sacc[nb][r] : kMasked;
            }
          }
        }
      } else {
        // keys kt0 .. kt0 + BN - 1 of the block mask (BN divides 64, kt0 % BN == 0)
        // pre-shifted by this lane half's key offset 4g, so each element tests a bit at
        // a compile-time position (no per-element 64-bit shift constants to hold)
        const uint64_t kbits =
            p.kmask != nullptr ? kmask_row[kt0 >> 6] >> ((kt0 & 63) + 4 * g) : ~uint64_t{0};
#pragma unroll
        for (int nb = 0; nb < S::NB; ++nb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int off = 32 * nb + 8 * (r >> 2) + (r & 3);
            const int key = key0 + off;
            const bool ok = key < Skv && (!p.causal || key <= qa) &&
                            (p.window <= 0 || key >= qa - p.window + 1) && ((kbits >> off) & 1u);
            sacc[nb][r] = ok ? sacc[nb][r] : kMasked;
          }
        }
      }
    }
    // Running max. CHUNK_CHECK (the interleaved kernels, head_dim <= 128): the max moves
    // only when a chunk shows it must. The exponents are taken against the current
    // m_run, and a chunk whose exp sum exceeds kChunkLimit (some p > 2^5, i.e. a score
    // well above m_run), or any row without a max yet (lim < 0), takes the rare path
    // below, which sets m_run to the tile's max and rescales O and l, then redoes the
    // chunk. Every accumulated p is thus <= kChunkLimit, and the common tile spends no
    // VALU work on its max (-13 % VALU instructions per tile). The other kernels (no
    // registers to spare for the rare path inside the chunk loop) take the tile's max
    // first and move m_run when it grows by more than kRescaleThresh.
    constexpr bool CHUNK_CHECK = IL;
    if constexpr (!CHUNK_CHECK) {
      const float mt = tile_max();
      const float m_new = fmaxf(m_run, mt);
      const bool need = m_new > m_run + kRescaleThresh / c;
      if (__any(need)) {
        const float alpha = need ? fast_exp2((m_run - m_new) * c) : 1.0f;
        m_run = need ? m_new : m_run;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < SV::DB; ++db) {
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
        }
      }
      negmc = (m_run == kNegInf) ? 0.0f : -m_run * c;
    }
    bool checked = !CHUNK_CHECK;  // uniform: this tile's max is known, later chunks are safe
    auto chunk_exp = [&](int nb, int base, float (&pv)[8]) __attribute__((always_inline)) {
      if constexpr (LATE_CAP) {
        const float cn = c + negmc;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float rr = __builtin_amdgcn_rcpf(1.0f + fast_exp2(sacc[nb][base + e] * tanh_mul));
          pv[e] = fast_exp2(fmaf(rr, -2.0f * c, cn));
        }
      } else if constexpr (SOFTCAP) {
        const float cn = c + negmc;
#pragma unroll
        for (int e = 0; e < 8; ++e) pv[e] = fast_exp2(fmaf(sacc[nb][base + e], -2.0f * c, cn));
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) pv[e] = fast_exp2(fmaf(sacc[nb][base + e], c, negmc));
      }
      return ((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7]));
    };
#pragma unroll
    for (int cc = 0; cc < S::NC; ++cc) {
      const int nb = cc >> 1;
      const int base = (cc & 1) * 8;
      chunk_hook(cc);
      // V^T operands of the chunk first: their LDS latency overlaps the exp work
      u32x4 av[SV::DB];
#pragma unroll
      for (int db = 0; db < SV::DB; ++db) {
        const uint16_t* r0 = vl + v_rd[db] + 16 * cc * DV;
        const u32x2 lo2 = lds_read_tr16(r0);             // keys 16cc + 4g + 0..3
        const u32x2 hi2 = lds_read_tr16(r0 + 8 * DV);    // keys 16cc + 8 + 4g + 0..3
        av[db] = u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
      }
      __builtin_amdgcn_sched_barrier(0);
      if (IL && do_qk) {
#pragma unroll
        for (int ks = S::KS * cc / S::NC; ks < S::KS * (cc + 1) / S::NC; ++ks) {
#pragma unroll
          for (int nb2 = 0; nb2 < S::NB; ++nb2) {
            nxt[nb2] = E::mfma32(ak[ks - S::KS * cc / S::NC][nb2], qreg[ks], nxt[nb2]);
          }
        }
      }
      float pv[8];
      float csum = chunk_exp(nb, base, pv);
      if constexpr (IL) {
        // one S^T(t+1) MFMA, then four VALU instructions of the chunk's exponentials,
        // and so on: on MI355X +1.6 % at the north-star shape, +3 % at S = 4096
        // against the compiler's own order, bit-identical
        if (do_qk) {
#pragma unroll
          for (int m = 0; m < S::KS * S::NB / S::NC; ++m) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, LATE_CAP ? 12 : 4, 0);
          }
        }
      }
      if (!checked && __any(!(csum <= lim))) {
        checked = true;
        const float mt = tile_max();
        const float m_new = fmaxf(m_run, mt);
        const float alpha = m_new > m_run ? fast_exp2((m_run - m_new) * c) : 1.0f;
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < SV::DB; ++db) {
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
        }
        const bool no_max = m_run == kNegInf;  // every key so far masked
        negmc = no_max ? 0.0f : -m_run * c;
        lim = no_max ? -1.0f : kChunkLimit;
        csum = chunk_exp(nb, base, pv);
      }
      l_run += csum;
      const u32x4 pk = {E::pack2(pv[0], pv[1]), E::pack2(pv[2], pv[3]),
                        E::pack2(pv[4], pv[5]), E::pack2(pv[6], pv[7])};
#pragma unroll
      for (int db = 0; db < SV::DB; ++db) oacc[db] = E::mfma32(av[db], pk, oacc[db]);
      if (IL && do_qk && cc + 1 < S::NC) rd_k(cc + 1);
    }
  };

  f32x16 s_cur[S::NB];
  f32x16 s_nxt[S::NB];
  if (n_it > 0) {
    issue_k(tile_at(0), k_lds[0]);
    issue_v(tile_at(0), v_lds[0]);
    // S^T(0) needs Q and K(0) only: the loads retire in issue order, so waiting until
    // V(0) and K(1) alone may be outstanding (SV::LPT + S::LPT loads per thread; V
    // tiles are narrower than K tiles in the narrow-V kernels) leaves Q and K(0)
    // complete, and their latency overlaps S^T(0) (the first step's wait and barrier
    // cover them)
    if (n_it > 1) {
      issue_k(tile_at(1), k_lds[1]);
      wait_vmcnt<SV::LPT + S::LPT>();
    } else {
      wait_vmcnt<SV::LPT>();
    }
  } else {
    wait_vmcnt0();
  }
  // The Q registers hold the loaded values from here on (the asm below orders every
  // use after the wait, and keeps the registers allocated to Q until then).
#pragma unroll
  for (int ks = 0; ks < S::KS; ++ks) asm volatile("" : "+v"(qreg[ks]) :: "memory");
  finish_q();
  if (n_it > 0) {
    __syncthreads();
    if (wave_live) qk(k_lds[0], s_cur, std::true_type{});
  }
  // Iteration i computes tile t = t_begin + i. Entering it, K(t+1) and V(t) are in
  // LDS; it issues K(t+2) and V(t+1) into the buffers iteration i-1 finished reading,
  // computes S^T(t+1) (MFMA) ahead of softmax(t) (VALU), then P V(t). The loop body is
  // written twice so the two score buffers swap roles without copies.
  auto step = [&](int i, f32x16 (&cur)[S::NB], f32x16 (&nxt)[S::NB]) __attribute__((always_inline)) {
    const int t = tile_at(i);
    wait_vmcnt0();
    __syncthreads();
    if (i + 2 < n_it) issue_k(tile_at(i + 2), k_lds[i & 1]);
    if (i + 1 < n_it) issue_v(tile_at(i + 1), v_lds[(i + 1) & 1]);
    if (!wave_live) return;
    if (p.causal && t * BN > qwl_abs) return;  // past this wave's causal band
    if (!IL && i + 1 < n_it) qk(k_lds[(i + 1) & 1], nxt, std::true_type{});
    softmax_pv(cur, t, v_lds[i & 1], std::true_type{}, kmask_partial(i), nxt, k_lds[(i + 1) & 1],
               i + 1 < n_it, [](int) {});
  };
  // The same iteration for a tile where every test above is known to pass: K(t+2) and
  // V(t+1) exist and hold BN keys, the wave is live and the tile needs no element mask.
  // The same barrier count and the same loads as `step`, without the tests.
  // PAR = i & 1, known at compile time in the fast loop (it starts at an even i).
  auto fast_step = [&](int i, f32x16 (&cur)[S::NB], f32x16 (&nxt)[S::NB], auto par) __attribute__((always_inline)) {
    constexpr int PAR = decltype(par)::value;
    const int t = t_begin + i;
    wait_vmcnt0();
    __syncthreads();
    if (!IL) {
      issue_full(S{}, k_next, k_tile_bytes, k_off, k_wlds, std::integral_constant<uint32_t, PAR>{});
      issue_full(SV{}, v_next, v_tile_bytes, v_off, v_wlds, std::integral_constant<uint32_t, 1 - PAR>{});
      qk(k_lds[1 - PAR], nxt, std::integral_constant<bool, (DP < 192)>{});
      softmax_pv(cur, t, v_lds[PAR], std::false_type{}, false, nxt, k_lds[1 - PAR], true, [](int) {});
    } else {
      // The tile loads spread over the P V chunks (chunk cc issues loads
      // LPT cc / NC .. LPT (cc + 1) / NC - 1 of K(t+2) and of V(t+1)) rather than all
      // right after the barrier, where the four waves' 32 KiB of requests at once stall
      // their issue: +2-4 % on MI355X.
      softmax_pv(cur, t, v_lds[PAR], std::false_type{}, false, nxt, k_lds[1 - PAR], true,
                 [&](int cc) __attribute__((always_inline)) {
#pragma unroll
                   for (int j = S::LPT * cc / S::NC; j < S::LPT * (cc + 1) / S::NC; ++j) {
                     load_lds16_async(k_next, k_off[j], k_wlds + PAR * S::TILE * 2 + j * 1024 * NW);
                   }
#pragma unroll
                   for (int j = SV::LPT * cc / S::NC; j < SV::LPT * (cc + 1) / S::NC; ++j) {
                     load_lds16_async(v_next, v_off[j], v_wlds + (1 - PAR) * SV::TILE * 2 + j * 1024 * NW);
                   }
                 });
      k_next += k_tile_bytes;
      v_next += v_tile_bytes;
    }
  };
  // This wave's fast range [i_lo, i_hi) (wave-uniform): tiles t + 2 < nt and holding BN
  // keys, right of the window's left edge for the wave's last row, and (causal) wholly
  // at or left of the wave's first row. No block mask.
  int i_lo = 0;
  int i_hi = 0;
  if (wave_live && p.kmask == nullptr) {
    i_hi = min(nt - 2, t_full - t_begin - 2);
    if (p.causal) i_hi = min(i_hi, (qw0_abs + 1) / BN - t_begin);
    if (p.window > 0) {
      const int edge = qwl_abs - p.window + 1;  // first key every row of the wave sees
      i_lo = edge > 0 ? (edge + BN - 1) / BN - t_begin : 0;
      i_lo = max(i_lo, 0);
    }
  }
  // Three loops over tile pairs (the loop body is written twice so the two score
  // buffers swap roles without copies): general pairs up to the fast range, fast pairs,
  // general pairs to the end.
  int i = 0;
  for (; i < n_it && !(i >= i_lo && i + 1 < i_hi); i += 2) {
    step(i, s_cur, s_nxt);
    if (i + 1 < n_it) step(i + 1, s_nxt, s_cur);
  }
  for (; i + 1 < i_hi; i += 2) {
    fast_step(i, s_cur, s_nxt, std::integral_constant<int, 0>{});
    fast_step(i + 1, s_nxt, s_cur, std::integral_constant<int, 1>{});
  }
  for (; i < n_it; i += 2) {
    step(i, s_cur, s_nxt);
    if (i + 1 < n_it) step(i + 1, s_nxt, s_cur);
  }

  const float l_tot = wave_pair_sum(l_run);
  if (wave_live && qrow < p.Sq) {
    float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    float lse = l_tot > 0.0f ? (m_run * c + fast_log2(l_tot)) * kLn2 : masked_row_lse(p, qrow);
    if (l_tot > 0.0f) ref_tile_floor(p, qrow, lse, inv);
    uint16_t* orow = p.o + b * p.o_sb + h * p.o_sh + static_cast<int64_t>(qrow) * p.o_ss;
    const int Dv = NARROW ? p.Dv : D;
    if constexpr (NARROW) {
      // Lane (row, g) holds dims 32 db + 8 i + 4 g .. +3. A v_permlane32_swap per dword
      // gives lane g = 0 both halves of the 8-dim chunks i = 0, 2 and lane g = 1 those of
      // i = 1, 3, so every store is 16 contiguous bytes (half as many stores, each row's
      // 32 bytes per instruction in one piece). On MI355X +5-8 % at the MLA prefill
      // shapes with the zero padding below stored the same way; in the equal-width
      // kernels it measured within noise and is not used there.
#pragma unroll
      for (int db = 0; db < SV::DB; ++db) {
        uint32_t w[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          w[i][0] = E::pack2(oacc[db][4 * i + 0] * inv, oacc[db][4 * i + 1] * inv);
          w[i][1] = E::pack2(oacc[db][4 * i + 2] * inv, oacc[db][4 * i + 3] * inv);
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const auto x0 = __builtin_amdgcn_permlane32_swap(w[2 * k][0], w[2 * k + 1][0], false, false);
          const auto x1 = __builtin_amdgcn_permlane32_swap(w[2 * k][1], w[2 * k + 1][1], false, false);
          const int d0 = 32 * db + 16 * k + 8 * g;
          if (d0 < Dv) *reinterpret_cast<u32x4*>(orow + d0) = u32x4{x0[0], x1[0], x0[1], x1[1]};
        }
      }
      // a V narrower than head_dim is zero-padded: O's dims past it are 0 (D and Dv are
      // multiples of 8, so each 16-byte store ends at or before D)
      for (int d0 = Dv + 8 * g; d0 < D; d0 += 16) {
        *reinterpret_cast<u32x4*>(orow + d0) = u32x4{0u, 0u, 0u, 0u};
      }
    } else {
#pragma unroll
      for (int db = 0; db < SV::DB; ++db) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d0 = 32 * db + 8 * i + 4 * g;
          const uint32_t w0 = E::pack2(oacc[db][4 * i + 0] * inv, oacc[db][4 * i + 1] * inv);
          const uint32_t w1 = E::pack2(oacc[db][4 * i + 2] * inv, oacc[db][4 * i + 3] * inv);
          if (d0 < Dv) *reinterpret_cast<u32x2*>(orow + d0) = u32x2{w0, w1};
        }
      }
    }
    if (p.lse != nullptr && g == 0) {
      p.lse[b * p.l_sb + h * p.l_sh + static_cast<int64_t>(qrow) * p.l_ss] = lse;
    }
  }
}

template <typename Tag, int DP, int DV, int BN, int NW>
void launch_nw(const PrefillParams& p, bool softcap, int grid, hipStream_t s) {
  const size_t dyn = p.kmask != nullptr ? kLiveLdsBytes : 0;
  if (softcap) {
    hipLaunchKernelGGL((prefill_kernel<Tag, DP, DV, BN, true, NW>), dim3(grid), dim3(64 * NW), dyn, s, p);
  } else {
    hipLaunchKernelGGL((prefill_kernel<Tag, DP, DV, BN, false, NW>), dim3(grid), dim3(64 * NW), dyn, s, p);
  }
}

template <typename Tag, int DP, int DV, int BN>
void launch_dp(const PrefillParams& p, bool softcap, int grid, hipStream_t s) {
  launch_nw<Tag, DP, DV, BN, 4>(p, softcap, grid, s);
}

// The narrow-V kernels run eight waves (256-row workgroups) from kWideRowsFrom query
// rows on: the query tiles, the grid and its XCD order are re-derived for 256 rows.
constexpr int kWideRowsFrom = 4096;

template <typename Tag>
void launch_narrow(const PrefillParams& p0, bool softcap, int grid, hipStream_t s) {
  if (p0.Sq < kWideRowsFrom) {
    launch_nw<Tag, 192, 128, kNarrowBN, 4>(p0, softcap, grid, s);
    return;
  }
  PrefillParams p = p0;
  p.n_qt = (p.Sq + 255) / 256;
  const int grid8 = p.n_qt * p.B * p.Hq;
  prefill_grid_order(p.causal != 0, static_cast<int64_t>(p.B) * p.Hq, grid8, p.xcd_group, p.xcd_remap);
  launch_nw<Tag, 192, 128, kNarrowBN, 8>(p, softcap, grid8, s);
}

template <typename Tag>
void launch_tag(const PrefillParams& p, bool softcap, int grid, hipStream_t s) {
  if (p.D <= 32) {
    launch_dp<Tag, 32, 32, 64>(p, softcap, grid, s);
  } else if (p.D <= 64) {
    launch_dp<Tag, 64, 64, 64>(p, softcap, grid, s);
  } else if (p.D <= 128) {
    launch_dp<Tag, 128, 128, 64>(p, softcap, grid, s);
  } else if (p.D <= 192) {
    if (p.Dv <= 128) {
      launch_narrow<Tag>(p, softcap, grid, s);
    } else {
      launch_dp<Tag, 192, 192, 32>(p, softcap, grid, s);
    }
  } else {
    launch_dp<Tag, 256, 256, 32>(p, softcap, grid, s);
  }
}

// ---------------------------------------------------------------------------------
// fp32 inputs: the reference computes them in fp32 (cpu_reference.py:262), so they run
// on v_mfma_f32_32x32x2_f32 instead of being rounded to 16 bits. One workgroup of 4
// waves per 128 query rows, 32-key tiles of K and V staged in LDS (rows padded by 4
// floats: the K operand reads of 32 rows and the V reads of 32 dims are conflict
// free). S^T = K Q^T with the reduction dims permuted per lane half (k-step ks: dim ks
// for lanes 0-31, DP/2 + ks for lanes 32-63) so every lane's Q and K operands are
// contiguous. For O^T += V^T P^T the keys are permuted so that k-step (i, j) covers
// keys 8i + j and 8i + 4 + j: each lane's B operand is then its own S^T accumulator
// 4i + j (fp32 P, no shuffle).
// ---------------------------------------------------------------------------------
constexpr int kF32BN = 32;

template <int DP, bool SOFTCAP>
__global__ __launch_bounds__(kThreads, 1) void prefill_f32_kernel(const PrefillParams p) {
  constexpr int PITCH = DP + 4;
  constexpr int HALF = DP / 2;
  constexpr int DB = DP / 32;
  __shared__ __attribute__((aligned(16))) float kt[kF32BN * PITCH];
  __shared__ __attribute__((aligned(16))) float vt[kF32BN * PITCH];
  const float* qf = reinterpret_cast<const float*>(p.q);
  const float* kf = reinterpret_cast<const float*>(p.k);
  const float* vf = reinterpret_cast<const float*>(p.v);
  float* of = reinterpret_cast<float*>(p.o);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;

  int bh, jq;
  work_item(p, blockIdx.x, bh, jq);
  bh = __builtin_amdgcn_readfirstlane(bh);  // uniform: keeps the tile bases in SGPRs
  jq = __builtin_amdgcn_readfirstlane(jq);
  const int qt = p.causal ? (p.n_qt - 1 - jq) : jq;
  const int b = bh / p.Hq;
  const int h = bh - b * p.Hq;
  const int hk = h / p.ratio;
  const int D = p.D;
  const int Skv = p.Skv;

  const int q0 = qt * kBlockM;
  const int q_last = min(q0 + kBlockM, p.Sq) - 1;
  const int q0_abs = p.q_offset + q0;
  const int ql_abs = p.q_offset + q_last;
  const int kv_lo = p.window > 0 ? max(0, q0_abs - p.window + 1) : 0;
  const int kv_hi = p.causal ? min(Skv, ql_abs + 1) : Skv;
  const int t_begin = kv_lo / kF32BN;
  const int nt = kv_hi > kv_lo ? (kv_hi + kF32BN - 1) / kF32BN - t_begin : 0;

  const int qw0 = q0 + wave * 32;
  const int qrow = qw0 + l32;
  const bool wave_live = qw0 < p.Sq;
  const int qw0_abs = p.q_offset + qw0;
  const int qwl_abs = p.q_offset + min(qw0 + 31, p.Sq - 1);
  const int qa = p.q_offset + qrow;
  const uint64_t* kmask_row =
      p.kmask != nullptr ? p.kmask + static_cast<int64_t>(min(qrow, p.Sq - 1) / p.ref_bq) * p.kmask_words
                         : nullptr;
  const float c = SOFTCAP ? 1.0f : p.score_mul;
  const float thresh = SOFTCAP ? kRescaleThresh : kRescaleThresh / p.score_mul;

  // Q^T operand: lane holds row qrow, dims g*HALF .. g*HALF + HALF - 1 (zero past D)
  float qreg[HALF];
  {
    const float* qr = qf + b * p.q_sb + h * p.q_sh + static_cast<int64_t>(min(qrow, p.Sq - 1)) * p.q_ss;
#pragma unroll
    for (int c4 = 0; c4 < HALF; c4 += 4) {
      const int d0 = g * HALF + c4;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (d0 < D) v = *reinterpret_cast<const f32x4*>(qr + d0);  // D % 8 == 0
#pragma unroll
      for (int e = 0; e < 4; ++e) qreg[c4 + e] = p.q_neg ? -v[e] : v[e];  // negative scale
    }
  }
  f32x16 oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.0f;
  }
  float m_run = kNegInf;
  float l_run = 0.0f;
  const float* kbase = kf + b * p.k_sb + hk * p.k_sh;
  const float* vbase = vf + b * p.v_sb + hk * p.v_sh;
  const int dq = D >> 2;  // float4 chunks per row

  for (int i = 0; i < nt; ++i) {
    const int kt0 = (t_begin + i) * kF32BN;
    __syncthreads();  // previous tile's reads are done
    for (int idx = tid; idx < kF32BN * (DP / 4); idx += kThreads) {
      const int r = idx / (DP / 4);
      const int c4 = idx - r * (DP / 4);
      const int key = min(kt0 + r, Skv - 1);  // rows past Skv are masked below
      f32x4 kv = {0.f, 0.f, 0.f, 0.f}, vv = {0.f, 0.f, 0.f, 0.f};
      if (c4 < dq) {
        kv = *reinterpret_cast<const f32x4*>(kbase + static_cast<int64_t>(key) * p.k_ss + 4 * c4);
        vv = *reinterpret_cast<const f32x4*>(vbase + static_cast<int64_t>(key) * p.v_ss + 4 * c4);
      }
      *reinterpret_cast<f32x4*>(kt + r * PITCH + 4 * c4) = kv;
      *reinterpret_cast<f32x4*>(vt + r * PITCH + 4 * c4) = vv;
    }
    __syncthreads();
    if (!wave_live) continue;
    if (p.causal && kt0 > qwl_abs) continue;  // past this wave's causal band

    f32x16 sacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[r] = 0.0f;
    const float* krow = kt + l32 * PITCH + g * HALF;
#pragma unroll
    for (int ks = 0; ks < HALF; ++ks) sacc = mfma_f32(krow[ks], qreg[ks], sacc);

    if constexpr (SOFTCAP) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] = p.cap_mul * tanh_approx(sacc[r] * p.score_mul);
    }
    const bool need_mask = (kt0 + kF32BN > Skv) || (p.causal && kt0 + kF32BN - 1 > qw0_abs) ||
                           (p.window > 0 && kt0 < qwl_abs - p.window + 1) || p.kmask != nullptr;
    if (need_mask) {
      const uint64_t kbits =
          p.kmask != nullptr ? kmask_row[kt0 >> 6] >> (kt0 & 63) : ~uint64_t{0};
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int off = 8 * (r >> 2) + 4 * g + (r & 3);
        const int key = kt0 + off;
        const bool ok = key < Skv && (!p.causal || key <= qa) &&
                        (p.window <= 0 || key >= qa - p.window + 1) && ((kbits >> off) & 1u);
        sacc[r] = ok ? sacc[r] : kNegInf;
      }
    }
    float mt = kNegInf;
#pragma unroll
    for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sacc[r]);
    mt = wave_pair_max(mt);
    const float m_new = fmaxf(m_run, mt);
    const bool need = m_new > m_run + thresh;
    if (__any(need)) {
      const float alpha = need ? fast_exp2((m_run - m_new) * c) : 1.0f;
      m_run = need ? m_new : m_run;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
      }
    }
    const float mc = (m_run == kNegInf) ? 0.0f : m_run * c;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sacc[r] = fast_exp2(fmaf(sacc[r], c, -mc));
      l_run += sacc[r];
    }
    // O^T[d, q] += sum over keys 8ii + 4g + jj of V[key][d] P[q][key]
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 8 * (r >> 2) + 4 * g + (r & 3);
        oacc[db] = mfma_f32(vt[key * PITCH + 32 * db + l32], sacc[r], oacc[db]);
      }
    }
  }

  const float l_tot = wave_pair_sum(l_run);
  if (wave_live && qrow < p.Sq) {
    float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    float lse = l_tot > 0.0f ? (m_run * c + fast_log2(l_tot)) * kLn2 : masked_row_lse(p, qrow);
    if (l_tot > 0.0f) ref_tile_floor(p, qrow, lse, inv);
    float* orow = of + b * p.o_sb + h * p.o_sh + static_cast<int64_t>(qrow) * p.o_ss;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int d0 = 32 * db + 8 * ii + 4 * g;
        const f32x4 w = {oacc[db][4 * ii + 0] * inv, oacc[db][4 * ii + 1] * inv,
                         oacc[db][4 * ii + 2] * inv, oacc[db][4 * ii + 3] * inv};
        if (d0 < D) *reinterpret_cast<f32x4*>(orow + d0) = w;
      }
    }
    if (p.lse != nullptr && g == 0) {
      p.lse[b * p.l_sb + h * p.l_sh + static_cast<int64_t>(qrow) * p.l_ss] = lse;
    }
  }
}

// ---------------------------------------------------------------------------------
// fp32 inputs on grids too small for the kernel above (fewer than 2048 128-row
// workgroups; cfg1 has 128): one workgroup per 32 query rows, and its 4 waves
// split the key range (wave w takes 32-key tiles w, w + 4, ...), each staging its own
// tiles in a wave-private LDS region with the next one prefetched into registers, and
// each keeping its own running max, sum and O^T for the 32 rows (the per-tile math is
// the kernel above's). The four partial states meet in LDS at the end and wave 0
// merges them in a fixed order: O = sum_w 2^((m_w - m) c) O_w / sum_w 2^((m_w - m) c) l_w.
// ---------------------------------------------------------------------------------
template <int DP>
constexpr int kF32SplitBlocks = DP <= 64 ? 2 : 1;

template <int DP, bool SOFTCAP>
__global__ __launch_bounds__(kThreads, kF32SplitBlocks<DP>) void prefill_f32_split_kernel(const PrefillParams p) {
  using T = F32WaveTile<DP>;
  constexpr int PITCH = T::PITCH;
  constexpr int HALF = DP / 2;
  constexpr int DB = DP / 32;
  constexpr int NE = 16 * DB + 2;  // floats per lane in the merge: O^T, m, l
  static_assert(T::ROWS == kF32BN, "a wave tile is one key tile");
  static_assert(3 * NE * 64 <= 4 * 2 * kF32BN * PITCH, "merge fits in the tiles");
  __shared__ __attribute__((aligned(16))) float lds[4 * 2 * kF32BN * PITCH];
  const float* qf = reinterpret_cast<const float*>(p.q);
  const float* kf = reinterpret_cast<const float*>(p.k);
  const float* vf = reinterpret_cast<const float*>(p.v);
  float* of = reinterpret_cast<float*>(p.o);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;
  float* kt = lds + wave * 2 * kF32BN * PITCH;
  float* vt = kt + kF32BN * PITCH;

  // heaviest row blocks (causal: the last) first, all heads at once
  const int units = p.B * p.Hq;
  const int n_rb = (p.Sq + kF32BN - 1) / kF32BN;
  const int jb = static_cast<int>(blockIdx.x) / units;
  const int bh = static_cast<int>(blockIdx.x) - jb * units;
  const int rb = p.causal ? n_rb - 1 - jb : jb;
  const int b = bh / p.Hq;
  const int h = bh - b * p.Hq;
  const int hk = h / p.ratio;
  const int D = p.D;
  const int Skv = p.Skv;

  const int q0 = rb * kF32BN;
  const int qrow = q0 + l32;
  const int qa = p.q_offset + qrow;
  const int qa0 = p.q_offset + q0;
  const int ql_abs = p.q_offset + min(q0 + kF32BN, p.Sq) - 1;
  const int kv_lo = p.window > 0 ? max(0, qa0 - p.window + 1) : 0;
  const int kv_hi = p.causal ? min(Skv, ql_abs + 1) : Skv;
  const int t_lo = kv_lo / kF32BN;
  const int nt = kv_hi > kv_lo ? (kv_hi + kF32BN - 1) / kF32BN - t_lo : 0;
  const uint64_t* kmask_row =
      p.kmask != nullptr ? p.kmask + static_cast<int64_t>(min(qrow, p.Sq - 1) / p.ref_bq) * p.kmask_words
                         : nullptr;
  const float c = SOFTCAP ? 1.0f : p.score_mul;
  const float thresh = SOFTCAP ? kRescaleThresh : kRescaleThresh / p.score_mul;

  // Q^T operand: lane holds row qrow, dims g*HALF .. g*HALF + HALF - 1 (zero past D)
  float qreg[HALF];
  {
    const float* qr = qf + b * p.q_sb + h * p.q_sh + static_cast<int64_t>(min(qrow, p.Sq - 1)) * p.q_ss;
#pragma unroll
    for (int c4 = 0; c4 < HALF; c4 += 4) {
      const int d0 = g * HALF + c4;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (d0 < D) v = *reinterpret_cast<const f32x4*>(qr + d0);  // D % 8 == 0
#pragma unroll
      for (int e = 0; e < 4; ++e) qreg[c4 + e] = p.q_neg ? -v[e] : v[e];  // negative scale
    }
  }
  f32x16 oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.0f;
  }
  float m_run = kNegInf;
  float l_run = 0.0f;
  const float* kbase = kf + b * p.k_sb + hk * p.k_sh;
  const float* vbase = vf + b * p.v_sb + hk * p.v_sh;

  T kn, vn;
  if (wave < nt) {
    kn.load(kbase, p.k_ss, (t_lo + wave) * kF32BN, Skv - 1, D, lane);
    vn.load(vbase, p.v_ss, (t_lo + wave) * kF32BN, Skv - 1, D, lane);
  }
  for (int t = wave; t < nt; t += 4) {
    const int kt0 = (t_lo + t) * kF32BN;
    kn.store(kt, lane);
    vn.store(vt, lane);
    wave_lds_order();
    if (t + 4 < nt) {
      kn.load(kbase, p.k_ss, kt0 + 4 * kF32BN, Skv - 1, D, lane);
      vn.load(vbase, p.v_ss, kt0 + 4 * kF32BN, Skv - 1, D, lane);
    }

    f32x16 sacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[r] = 0.0f;
    const float* krow = kt + l32 * PITCH + g * HALF;
#pragma unroll
    for (int ks = 0; ks < HALF; ++ks) sacc = mfma_f32(krow[ks], qreg[ks], sacc);

    if constexpr (SOFTCAP) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] = p.cap_mul * tanh_approx(sacc[r] * p.score_mul);
    }
    const bool need_mask = (kt0 + kF32BN > Skv) || (p.causal && kt0 + kF32BN - 1 > qa0) ||
                           (p.window > 0 && kt0 < ql_abs - p.window + 1) || p.kmask != nullptr;
    if (need_mask) {
      const uint64_t kbits =
          p.kmask != nullptr ? kmask_row[kt0 >> 6] >> (kt0 & 63) : ~uint64_t{0};
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int off = 8 * (r >> 2) + 4 * g + (r & 3);
        const int key = kt0 + off;
        const bool ok = key < Skv && (!p.causal || key <= qa) &&
                        (p.window <= 0 || key >= qa - p.window + 1) && ((kbits >> off) & 1u);
        sacc[r] = ok ? sacc[r] : kNegInf;
      }
    }
    float mt = kNegInf;
#pragma unroll
    for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sacc[r]);
    mt = wave_pair_max(mt);
    const float m_new = fmaxf(m_run, mt);
    const bool need = m_new > m_run + thresh;
    if (__any(need)) {
      const float alpha = need ? fast_exp2((m_run - m_new) * c) : 1.0f;
      m_run = need ? m_new : m_run;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
      }
    }
    const float mc = (m_run == kNegInf) ? 0.0f : m_run * c;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sacc[r] = fast_exp2(fmaf(sacc[r], c, -mc));
      l_run += sacc[r];
    }
    // O^T[d, q] += sum over keys 8ii + 4g + jj of V[key][d] P[q][key]
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 8 * (r >> 2) + 4 * g + (r & 3);
        oacc[db] = mfma_f32(vt[key * PITCH + 32 * db + l32], sacc[r], oacc[db]);
      }
    }
    wave_lds_order();
  }

  // merge: waves 1-3 leave (O^T, m, l) in LDS, wave 0 combines them with its own
  const float l_w = wave_pair_sum(l_run);
  __syncthreads();  // every wave is done with its tiles
  if (wave > 0) {
    float* dst = lds + (wave - 1) * NE * 64 + lane;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[(16 * db + r) * 64] = oacc[db][r];
    }
    dst[(16 * DB) * 64] = m_run;
    dst[(16 * DB + 1) * 64] = l_w;
  }
  __syncthreads();
  if (wave != 0 || qrow >= p.Sq) return;
  float mw[4], lw[4];
  mw[0] = m_run;
  lw[0] = l_w;
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    mw[w] = lds[((w - 1) * NE + 16 * DB) * 64 + lane];
    lw[w] = lds[((w - 1) * NE + 16 * DB + 1) * 64 + lane];
  }
  const float m = fmaxf(fmaxf(mw[0], mw[1]), fmaxf(mw[2], mw[3]));
  float sc[4];
  float l_tot = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    sc[w] = mw[w] == kNegInf ? 0.0f : fast_exp2((mw[w] - m) * c);  // a wave with no key: 0
    l_tot = fmaf(sc[w], lw[w], l_tot);
  }
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float o = sc[0] * oacc[db][r];
#pragma unroll
      for (int w = 1; w < 4; ++w) o = fmaf(sc[w], lds[((w - 1) * NE + 16 * db + r) * 64 + lane], o);
      oacc[db][r] = o;
    }
  }
  float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  float lse = l_tot > 0.0f ? (m * c + fast_log2(l_tot)) * kLn2 : masked_row_lse(p, qrow);
  if (l_tot > 0.0f) ref_tile_floor(p, qrow, lse, inv);
  float* orow = of + b * p.o_sb + h * p.o_sh + static_cast<int64_t>(qrow) * p.o_ss;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int d0 = 32 * db + 8 * ii + 4 * g;
      const f32x4 w = {oacc[db][4 * ii + 0] * inv, oacc[db][4 * ii + 1] * inv,
                       oacc[db][4 * ii + 2] * inv, oacc[db][4 * ii + 3] * inv};
      if (d0 < D) *reinterpret_cast<f32x4*>(orow + d0) = w;
    }
  }
  if (p.lse != nullptr && g == 0) {
    p.lse[b * p.l_sb + h * p.l_sh + static_cast<int64_t>(qrow) * p.l_ss] = lse;
  }
}

// Workgroups of the 128-row fp32 kernel below which the split kernel runs instead
// (fewer than eight per CU). Measured on MI355X: 2.4x at cfg1 (128 workgroups), 1.7x
// at 512, 1.4x at 1024; at 4096 and more the two are within -9 % .. +4 % of each other.
constexpr int64_t kF32SplitBelow = 2048;

template <int DP>
void launch_f32_dp(const PrefillParams& p, bool softcap, int grid, hipStream_t s) {
  if constexpr (DP <= 128) {
    if (grid < kF32SplitBelow) {
      const int grid_s = p.B * p.Hq * ((p.Sq + kF32BN - 1) / kF32BN);  // <= 4 * grid
      if (softcap) {
        hipLaunchKernelGGL((prefill_f32_split_kernel<DP, true>), dim3(grid_s), dim3(kThreads), 0, s, p);
      } else {
        hipLaunchKernelGGL((prefill_f32_split_kernel<DP, false>), dim3(grid_s), dim3(kThreads), 0, s, p);
      }
      return;
    }
  }
  if (softcap) {
    hipLaunchKernelGGL((prefill_f32_kernel<DP, true>), dim3(grid), dim3(kThreads), 0, s, p);
  } else {
    hipLaunchKernelGGL((prefill_f32_kernel<DP, false>), dim3(grid), dim3(kThreads), 0, s, p);
  }
}

void launch_f32(const PrefillParams& p, bool softcap, int grid, hipStream_t s) {
  if (p.D <= 32) {
    launch_f32_dp<32>(p, softcap, grid, s);
  } else if (p.D <= 64) {
    launch_f32_dp<64>(p, softcap, grid, s);
  } else if (p.D <= 128) {
    launch_f32_dp<128>(p, softcap, grid, s);
  } else if (p.D <= 192) {
    launch_f32_dp<192>(p, softcap, grid, s);
  } else {
    launch_f32_dp<256>(p, softcap, grid, s);
  }
}


}  // namespace

int launch_prefill(const ffa_prefill_args& a, hipStream_t stream) {
  PrefillParams p{};
  p.q = static_cast<const uint16_t*>(a.q);
  p.k = static_cast<const uint16_t*>(a.k);
  p.v = static_cast<const uint16_t*>(a.v);
  p.o = static_cast<uint16_t*>(a.o);
  p.lse = a.lse;
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
  p.n_qt = (a.seqlen_q + kBlockM - 1) / kBlockM;
  const bool softcap = a.softcap > 0.0f;
  // Without softcap the kernels keep the running max of raw q.k, so their multiplier
  // must be positive: a negative scale flips Q's sign instead (q.k * scale =
  // (-q).k * |scale|), and a zero or tiny scale becomes 1e-30, which rounds every
  // exponent q.k * 1e-30 * log2 e (|q.k| < 1e20) to 0: the uniform softmax with
  // LSE = log(n) that scale 0 gives. With softcap the scores are tanh-transformed
  // before the max (tanh is odd), so any finite scale is used as it is.
  float scale = a.scale;
  p.q_neg = 0;
  if (!softcap) {
    if (scale < 0.0f) {
      scale = -scale;
      p.q_neg = 1;
    }
    scale = fmaxf(scale, 1e-30f);
  }
  if (softcap) {
    p.score_mul = scale / a.softcap;
    p.cap_mul = a.softcap * kLog2e;
  } else {
    p.score_mul = scale * kLog2e;
    p.cap_mul = 0.0f;
  }
  p.ref_bq = a.ref_block_q > 0 ? a.ref_block_q : 64;
  p.ref_bkv = a.ref_block_kv > 0 ? a.ref_block_kv : 64;
  p.masked_lse_mode = a.masked_lse_mode;
  p.kmask = a.block_key_mask;
  p.kmask_words = a.block_key_mask_words;
  p.visited = a.block_visited;

  // The kernels move 16-byte chunks: callers guarantee 16-byte aligned bases, strides
  // that are multiples of 8 elements and head_dim % 8 == 0 (checked by ffa_prefill_fwd),
  // and per-tile byte offsets that fit 32 bits.
  const int64_t grid64 = static_cast<int64_t>(p.n_qt) * a.batch * a.heads_q;
  if (grid64 <= 0) return FFA_OK;
  if (grid64 > 0x7fffffff) return FFA_ERR_TOO_LARGE;
  const int grid = static_cast<int>(grid64);
  prefill_grid_order(p.causal != 0, static_cast<int64_t>(a.batch) * a.heads_q, grid,
                     p.xcd_group, p.xcd_remap);

  if (a.dtype == FFA_DTYPE_BF16) {
    launch_tag<Bf16Tag>(p, softcap, grid, stream);
  } else if (a.dtype == FFA_DTYPE_FP16) {
    launch_tag<F16Tag>(p, softcap, grid, stream);
  } else {
    launch_f32(p, softcap, grid, stream);
  }
  return hipGetLastError() == hipSuccess ? FFA_OK : FFA_ERR_LAUNCH;
}

}  // namespace ffa
