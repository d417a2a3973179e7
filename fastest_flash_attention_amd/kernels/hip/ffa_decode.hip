// Paged KV decode and paged gather for gfx950.
//
// Pool layout and index law of PagedKVCache (reference ops/kv_cache.py:142-149,194-203):
// pages [num_pages, heads_kv, page_size, head_dim]; token t of a sequence lives in
// physical page block_table[t / page_size], slot t % page_size.
//
// Decode (one query token per sequence, GQA group of G = Hq / Hkv query heads per KV
// head) is split-K:
//   split kernel  grid (batch * Hkv * column_groups, splits), 4 waves per workgroup.
//                 A workgroup streams tokens_per_split tokens of one (sequence, KV head)
//                 straight from the pages; every K/V byte is read once and serves all
//                 G query heads of the group (no repeat_kv). The block-table entries of
//                 the split are staged in LDS first, so no tile waits on a dependent
//                 block-table load. Each wave owns every 4th 16-token tile and keeps a
//                 2-stage ring in LDS: K and V rows go HBM -> LDS by asm-issued
//                 global_load_lds_dwordx4 (no VGPR staging, completion tracked by
//                 explicit vmcnt waits only), XOR-swizzled per row so the K operand
//                 reads and the transposed V reads are bank-conflict free.
//                 Per tile: S^T[key, head] = K Q^T (v_mfma_f32_16x16x32), fp32 softmax
//                 with exp2 and lane swaps, rescale deferred until the max grows by 2^8,
//                 O^T += V^T P^T (v_mfma_f32_16x16x16) whose B operand is exactly the
//                 lane's four P values. The waves' partials are merged through LDS and
//                 one normalised (O, lse) partial per query head goes to the workspace.
//   combine kernel one wave per (sequence, query head): O = sum_s exp(lse_s - lse) O_s,
//                 lse = logsumexp_s lse_s.
// Page ids outside [0, num_pages) never address memory: the tokens such a page would
// hold are excluded from the attention like tokens past context_len (a split whose
// staged ids are all valid pays nothing for this check).

#include <atomic>
#include <mutex>

#include "ffa_common.h"
#include "ffa_internal.h"

// Split-K partials of ffa_paged_decode_fwd_noalloc: one array per GPU the library runs
// on (a device global), held until the process ends. Host code never uses the name
// itself as memory (on the host it is only a handle): noalloc_scratch() resolves the
// array's device address per device with hipGetSymbolAddress, and that address is
// what the kernels are given.
static __device__ __attribute__((aligned(256))) unsigned char scratch[FFA_NOALLOC_SCRATCH_BYTES];

namespace ffa {
namespace {

constexpr int kDecWaves = 4;
constexpr int kDecThreads = 64 * kDecWaves;
constexpr int kTile = 16;            // tokens per wave tile
constexpr int kCols = 16;            // query heads per workgroup (MFMA N)
constexpr int kDefaultSplit = 1024;  // tokens per split
constexpr int kMaxSplit = 2048;      // bounds the LDS block-table stage
constexpr int kMinSplit = 32;
constexpr float kRescaleThresh = 8.0f;

struct DecodeParams {
  const uint16_t* q;
  const uint16_t* kp;
  const uint16_t* vp;
  uint16_t* o;
  float* lse;
  const int32_t* bt;
  const int32_t* lens;
  float* ws_o;    // [B][Hq][n_splits][DP] fp32 partials (paged decode)
  const uint16_t* ws_o16;  // [B][Hq][n_splits][DP] 16-bit partials (MLA decode)
  float* ws_lse;  // [B][Hq][n_splits]
  int64_t q_sb, q_sh, o_sb, o_sh, l_sb, l_sh;
  int64_t page_stride;  // Hkv * P * D elements
  int64_t head_stride;  // P * D elements
  int bt_stride;
  int B, Hq, Hkv, G, D, P, log2P, num_pages;
  int n_splits, tps, window;
  int max_len;  // context lengths are clamped to this (it sizes the grid)
  int n_cg;
  int dp;
  float score_mul, cap_mul;
};

template <int DP>
struct DShape {
  static constexpr int KS = DP / 32;          // k-steps of the 16x16x32 QK product
  static constexpr int DB = DP / 16;          // 16-dim blocks of O^T
};

__device__ inline int page_of(const DecodeParams& p, int tok, int& slot) {
  if (p.log2P >= 0) {
    slot = tok & (p.P - 1);
    return tok >> p.log2P;
  }
  const int pi = tok / p.P;
  slot = tok - pi * p.P;
  return pi;
}

template <int DP>
constexpr int kDecMinBlocks = DP <= 128 ? 2 : 1;

// XOR swizzle (16-byte chunk index) of the V rows in LDS: the 8 rows x 32 bytes a
// transposed read fetches per half-wave land in distinct bank groups.
template <int DP>
__device__ inline int dec_vswz(int r) {
  if constexpr (DP == 32) return 2 * ((r >> 2) & 1);
  if constexpr (DP == 64 || DP == 192) return 2 * ((r >> 1) & 3);
  return 2 * (r & 7);
}

// XOR swizzle (16-byte chunk index) of the K rows in LDS: the 16 rows x 16 bytes one
// K operand read fetches per 16 lanes land in distinct bank groups.
template <int DP>
__device__ inline int dec_kswz(int r) {
  if constexpr (DP == 32) return (r >> 2) & 3;
  if constexpr (DP == 64 || DP == 192) return (r >> 1) & 7;
  return r & 15;
}

template <typename Tag, int DP, bool SOFTCAP>
__global__ __launch_bounds__(kDecThreads, kDecMinBlocks<DP>) void decode_split_kernel(
    const DecodeParams p) {
  using S = DShape<DP>;
  using E = Elem<Tag>;
  constexpr int CPR = DP / 8;                    // 16-byte chunks per row
  constexpr int TILE = kTile * DP;               // elements of one K (or V) tile
  constexpr int NLD = kTile * CPR / 64;          // direct loads per lane per tile, per tensor
  constexpr int NL = 2 * NLD;                    // vector memory ops per lane per tile
  static_assert(kTile * CPR % 64 == 0, "tile rows must fill whole wave loads");
  // Per wave: 2 stages x (K tile, V tile); reused for the wave merge afterwards.
  constexpr int kStageBytes = kDecWaves * 2 * 2 * TILE * 2;
  constexpr int kRedBytes = kDecWaves * kCols * (DP + 4) * 4;
  __shared__ __attribute__((aligned(1024))) char smem[kStageBytes > kRedBytes ? kStageBytes : kRedBytes];
  __shared__ int bt_lds[kMaxSplit + 2];
  __shared__ int bad_lds[kDecWaves];
  __shared__ float red_m[kDecWaves][kCols];
  __shared__ float red_l[kDecWaves][kCols];
  auto red_o = reinterpret_cast<float(*)[kCols][DP + 4]>(smem);

  // blockIdx.x = (sequence, KV head, column group), blockIdx.y = split: workgroups are
  // dealt to the 8 XCDs round-robin by linear id, so every XCD gets whole KV heads of
  // every sequence (with the split as the fast index, an XCD would get one split
  // position of every sequence, and uneven lengths would load the XCDs unevenly).
  const int split = blockIdx.y;
  const int per_b = p.Hkv * p.n_cg;
  const int b = blockIdx.x / per_b;
  const int hkcg = blockIdx.x - b * per_b;
  const int hk = hkcg / p.n_cg;
  const int cg = hkcg - hk * p.n_cg;
  const int L = min(max(p.lens[b], 0), p.max_len);
  const int lo = p.window > 0 ? max(0, L - p.window) : 0;
  const int s_begin = max(split * p.tps, lo);
  const int s_end = min(split * p.tps + p.tps, L);
  if (s_begin >= s_end) return;  // uniform across the workgroup: no barrier reached

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int c16 = lane & 15;  // MFMA column = query head within the group
  const int g4 = lane >> 4;   // 0..3
  const int gcols = min(kCols, p.G - cg * kCols);
  const int head0 = hk * p.G + cg * kCols;
  const int D = p.D;
  const int dchunks = D >> 3;

  // Stage the split's physical page ids (entries [pg0, pg1]) in LDS.
  int slot0;
  const int pg0 = page_of(p, s_begin, slot0);
  int slot1;
  const int pg1 = page_of(p, s_end - 1, slot1);
  // Invalid ids are staged as -1: loads read page 0 instead (in bounds) and the
  // compute masks the tokens, which only splits holding such an id test (any_bad).
  bool bad = false;
  {
    const int32_t* btrow = p.bt + static_cast<int64_t>(b) * p.bt_stride;
    for (int i = tid; i <= pg1 - pg0; i += kDecThreads) {
      const int phys = btrow[pg0 + i];
      const bool ok = phys >= 0 && phys < p.num_pages;
      bt_lds[i] = ok ? phys : -1;
      bad = bad || !ok;
    }
  }
  const bool wave_bad = __any(bad);  // every lane votes
  if (lane == 0) bad_lds[wave] = wave_bad ? 1 : 0;
  const char* kpool = reinterpret_cast<const char*>(p.kp);
  const char* vpool = reinterpret_cast<const char*>(p.vp);
  // byte offset of token `tok` (clamped into the split) of this KV head in a pool
  auto row_off = [&](int tok) -> int64_t {
    tok = min(tok, s_end - 1);
    int slot;
    const int pg = page_of(p, tok, slot);
    const int phys = max(bt_lds[pg - pg0], 0);
    return (static_cast<int64_t>(phys) * p.page_stride + hk * p.head_stride +
            static_cast<int64_t>(slot) * D) * 2;
  };

  // Q^T as the B operand: lane holds head (head0 + c16), dims 32*ks + 8*g4 .. +7.
  u32x4 qreg[S::KS];
  {
    const bool col_live = c16 < gcols;
    const uint16_t* qr = p.q + b * p.q_sb + (col_live ? head0 + c16 : head0) * p.q_sh;
#pragma unroll
    for (int ks = 0; ks < S::KS; ++ks) {
      const int d0 = min(32 * ks + 8 * g4, D - 8);
      const u32x4 v = *reinterpret_cast<const u32x4*>(qr + d0);
      qreg[ks] = (col_live && 32 * ks + 8 * g4 < D) ? v : u32x4{0u, 0u, 0u, 0u};
    }
  }
  // Every compiler-issued load (block table, Q) is complete before the tile loop: the
  // tile loads below are asm direct-to-LDS loads whose completion the loop tracks with
  // explicit vmcnt waits, and no compiler wait inside the loop may count them.
  wait_vmcnt0();
  __syncthreads();  // bt_lds ready
  const bool any_bad = (bad_lds[0] | bad_lds[1] | bad_lds[2] | bad_lds[3]) != 0;

  f32x4 oacc[S::DB];
#pragma unroll
  for (int db = 0; db < S::DB; ++db) oacc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf;
  float l_run = 0.0f;

  const int n_tiles = (s_end - s_begin + kTile - 1) / kTile;
  // stage st of this wave: K tile at kst(st), V tile right after it
  uint16_t* const wbase = reinterpret_cast<uint16_t*>(smem) + wave * 2 * 2 * TILE;
  auto kst = [&](int st) { return wbase + st * 2 * TILE; };
  auto vst = [&](int st) { return wbase + st * 2 * TILE + TILE; };

  // Per-lane constants of the direct loads: load j fills chunk position j * 64 + lane
  // of a tile -> row, swizzled source chunk (K and V swizzles differ).
  int lrow[NLD];
  int kchk[NLD];
  int vchk[NLD];
#pragma unroll
  for (int j = 0; j < NLD; ++j) {
    const int pos = j * 64 + lane;
    lrow[j] = pos / CPR;
    const int q = pos - lrow[j] * CPR;
    kchk[j] = min(q ^ dec_kswz<DP>(lrow[j]), dchunks - 1) * 16;
    vchk[j] = min(q ^ dec_vswz<DP>(lrow[j]), dchunks - 1) * 16;
  }
  // Per-lane K operand addresses: key c16, chunk 4*ks + g4 (dims 32ks + 8g4).
  int krd[S::KS];
#pragma unroll
  for (int ks = 0; ks < S::KS; ++ks) {
    krd[ks] = c16 * DP + (((4 * ks + g4) ^ dec_kswz<DP>(c16)) << 3);
  }
  // Per-lane V^T operand addresses (elements) of dim block db inside a V tile: this
  // lane supplies row 4*g4 + (c16 >> 2) of a 4-key group and dims 4*(c16 & 3) .. +3
  // of the 16-dim block (ds_read_b64_tr_b16 law).
  const int vr = 4 * g4 + (c16 >> 2);
  int vrd[S::DB];
#pragma unroll
  for (int db = 0; db < S::DB; ++db) {
    const int col = 16 * db + 4 * (c16 & 3);
    vrd[db] = vr * DP + (((col >> 3) ^ dec_vswz<DP>(vr)) << 3) + (col & 7);
  }

  auto issue = [&](int it, int st) {
    const int t0 = s_begin + it * kTile;
    uint16_t* kd = kst(st);
    uint16_t* vd = vst(st);
#pragma unroll
    for (int j = 0; j < NLD; ++j) {
      const int64_t ro = row_off(t0 + lrow[j]);
      load_lds16_async(kpool + ro + kchk[j], lds_addr(kd + j * 512));
      load_lds16_async(vpool + ro + vchk[j], lds_addr(vd + j * 512));
    }
  };

  // One 16-token tile: S^T[key, head] = K Q^T (v_mfma_f32_16x16x32: lane holds keys
  // 4*g4 + j of head c16), fp32 softmax, then O^T += V^T P^T with v_mfma_f32_16x16x16:
  // its B operand (keys 4*g4 .. +3 of head c16) is exactly this lane's four P values.
  auto compute = [&](int it, int st) {
    const int t0 = s_begin + it * kTile;
    const uint16_t* kl = kst(st);
    f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < S::KS; ++ks) {
      // dims >= head_dim of K were clamped re-reads: the zero Q dims cancel them
      const u32x4 a = *reinterpret_cast<const u32x4*>(kl + krd[ks]);
      sacc = E::mfma16(a, qreg[ks], sacc);
    }
    float mt = kNegInf;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float x = sacc[j];
      if constexpr (SOFTCAP) {
        x = p.cap_mul * tanh_approx(x * p.score_mul);
      } else {
        x = x * p.score_mul;
      }
      const int tok = t0 + 4 * g4 + j;
      bool live = tok < s_end;  // tokens below `lo` never enter a split range
      if (any_bad && live) {
        int slot;
        live = bt_lds[page_of(p, tok, slot) - pg0] >= 0;
      }
      x = live ? x : kNegInf;
      sacc[j] = x;
      mt = fmaxf(mt, x);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = wave_pair_max(mt);
    const float m_new = fmaxf(m_run, mt);
    const bool need = m_new > m_run + kRescaleThresh;
    if (__any(need)) {
      const float alpha = need ? fast_exp2(m_run - m_new) : 1.0f;
      m_run = need ? m_new : m_run;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < S::DB; ++db) {
#pragma unroll
        for (int j = 0; j < 4; ++j) oacc[db][j] *= alpha;
      }
    }
    const float mu = (m_run == kNegInf) ? 0.0f : m_run;
    float pv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pv[j] = fast_exp2(sacc[j] - mu);
      l_run += pv[j];
    }
    const u32x2 pk = {E::pack2(pv[0], pv[1]), E::pack2(pv[2], pv[3])};
    const uint16_t* vl = vst(st);
#pragma unroll
    for (int db = 0; db < S::DB; ++db) {
      const u32x2 a = lds_read_tr16(vl + vrd[db]);  // dim 16db + c16, keys 4*g4 + 0..3
      oacc[db] = E::mfma16k16(a, pk, oacc[db]);
    }
  };

  // Wave w owns tiles w, w + W, ... (W waves); its i-th tile uses stage i & 1. Entering
  // the compute of tile i, tiles i and i+1 are in flight: waiting until at most one
  // tile's NL loads remain leaves tile i complete (the counter retires in order).
  const int my_tiles = n_tiles > wave ? (n_tiles - wave + kDecWaves - 1) / kDecWaves : 0;
  if (my_tiles > 0) issue(wave, 0);
  if (my_tiles > 1) issue(wave + kDecWaves, 1);
  auto step = [&](int i, int st) {
    if (i + 1 < my_tiles) {
      wait_vmcnt<NL>();
    } else {
      wait_vmcnt0();
    }
    compute(wave + i * kDecWaves, st);
    if (i + 2 < my_tiles) {
      wait_lgkmcnt0();  // this stage's LDS reads are done before it is refilled
      issue(wave + (i + 2) * kDecWaves, st);
    }
  };
  for (int i = 0; i < my_tiles; i += 2) {
    step(i, 0);
    if (i + 1 < my_tiles) step(i + 1, 1);
  }

  // Per-wave totals, then merge the waves through LDS.
  float l_w = l_run + __shfl_xor(l_run, 16);
  l_w += __shfl_xor(l_w, 32);
  __syncthreads();  // every wave is done with its V stages
  if (g4 == 0) {
    red_m[wave][c16] = m_run;
    red_l[wave][c16] = l_w;
  }
  if (c16 < gcols) {
#pragma unroll
    for (int db = 0; db < S::DB; ++db) {
      *reinterpret_cast<f32x4*>(&red_o[wave][c16][16 * db + 4 * g4]) = oacc[db];
    }
  }
  __syncthreads();

  // Merge of the four waves' partials: 16 threads per column n (query head), 8
  // consecutive dims each, the waves' weights computed once per thread; 16-byte LDS
  // reads and workspace stores (rows are padded by 4 floats, keeping them 16-byte
  // aligned).
  const int n = tid >> 4;
  if (n < gcols) {
    float mm = kNegInf;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) mm = fmaxf(mm, red_m[w][n]);
    float wt[kDecWaves];
    float lsum = 0.0f;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
      wt[w] = mm != kNegInf ? fast_exp2(red_m[w][n] - mm) : 0.0f;
      lsum += wt[w] * red_l[w][n];
    }
    const int hq = head0 + n;
    const int64_t slot = (static_cast<int64_t>(b) * p.Hq + hq) * p.n_splits + split;
    for (int d0 = (tid & 15) * 8; d0 < D; d0 += 128) {
      float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) {
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(&red_o[w][n][d0]);
        const f32x4 x1 = *reinterpret_cast<const f32x4*>(&red_o[w][n][d0 + 4]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[e] += wt[w] * x0[e];
          o[4 + e] += wt[w] * x1[e];
        }
      }
      f32x4 r0, r1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        r0[e] = lsum > 0.0f ? o[e] / lsum : 0.0f;
        r1[e] = lsum > 0.0f ? o[4 + e] / lsum : 0.0f;
      }
      *reinterpret_cast<f32x4*>(p.ws_o + slot * p.dp + d0) = r0;
      *reinterpret_cast<f32x4*>(p.ws_o + slot * p.dp + d0 + 4) = r1;
    }
    if ((tid & 15) == 0) p.ws_lse[slot] = lsum > 0.0f ? (mm + fast_log2(lsum)) * kLn2 : kNegInf;
  }
}

// Partial s of dims d0, d0 + 1 in fp32 (P16: stored in the input's 16-bit type).
template <typename Tag, bool P16>
__device__ inline f32x2 load_partial(const DecodeParams& p, int64_t row, int d0) {
  if constexpr (P16) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p.ws_o16 + row * p.dp + d0);
    return f32x2{Elem<Tag>::to_f32(static_cast<uint16_t>(w & 0xffffu)),
                 Elem<Tag>::to_f32(static_cast<uint16_t>(w >> 16))};
  } else {
    return *reinterpret_cast<const f32x2*>(p.ws_o + row * p.dp + d0);
  }
}

// One workgroup per (sequence, query head): O = sum_s w_s O_s / sum_s w_s with
// w_s = exp(lse_s - max lse). Lane l owns dims 2l, 2l + 1 of a 128-dim slice, so a
// split's partial row is one coalesced 512-byte read; splits are walked 8 at a time
// to keep eight reads in flight per lane. Wave w of the workgroup (blockDim.x / 64
// waves) takes slices w, w + waves, ...: wide rows (the 512 MLA latent dims) are
// launched with one wave per slice, so all slices' reads are in flight at once.
template <typename Tag, bool P16>
__global__ __launch_bounds__(256) void decode_combine_kernel(const DecodeParams p) {
  using E = Elem<Tag>;
  const int bh = blockIdx.x;
  const int b = bh / p.Hq;
  const int hq = bh - b * p.Hq;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n_waves = blockDim.x >> 6;
  const int L = min(max(p.lens[b], 0), p.max_len);
  const int lo = p.window > 0 ? max(0, L - p.window) : 0;
  const int s0 = lo / p.tps;
  const int s1 = L > 0 ? (L + p.tps - 1) / p.tps : 0;
  const int64_t base = (static_cast<int64_t>(b) * p.Hq + hq) * p.n_splits;
  const float* lse_row = p.ws_lse + base;

  float mm = kNegInf;
  for (int s = s0 + lane; s < s1; s += 64) mm = fmaxf(mm, lse_row[s]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mm = fmaxf(mm, __shfl_xor(mm, off));

  float wsum = 0.0f;
  if (mm != kNegInf) {
    for (int s = s0 + lane; s < s1; s += 64) wsum += __expf(lse_row[s] - mm);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) wsum += __shfl_xor(wsum, off);
  const float inv = (mm != kNegInf && wsum > 0.0f) ? 1.0f / wsum : 0.0f;

  uint16_t* orow = p.o + b * p.o_sb + hq * p.o_sh;
  const bool o_pair_aligned = (reinterpret_cast<uintptr_t>(orow) & 3u) == 0;
  for (int d0 = 2 * lane + 128 * wave; d0 < p.D; d0 += 128 * n_waves) {
    f32x2 acc = {0.0f, 0.0f};
    if (mm != kNegInf) {
      int s = s0;
      for (; s + 8 <= s1; s += 8) {
        f32x2 v[8];
        float w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          v[u] = load_partial<Tag, P16>(p, base + s + u, d0);
          w[u] = __expf(lse_row[s + u] - mm);  // exp(-inf) = 0 for empty partials
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          acc[0] += w[u] * v[u][0];
          acc[1] += w[u] * v[u][1];
        }
      }
      for (; s < s1; ++s) {
        const f32x2 v = load_partial<Tag, P16>(p, base + s, d0);
        const float w = __expf(lse_row[s] - mm);
        acc[0] += w * v[0];
        acc[1] += w * v[1];
      }
    }
    const uint32_t pr = E::pack2(acc[0] * inv, acc[1] * inv);
    if (d0 + 1 < p.D && o_pair_aligned) {
      *reinterpret_cast<uint32_t*>(orow + d0) = pr;
    } else {
      orow[d0] = static_cast<uint16_t>(pr & 0xffffu);
      if (d0 + 1 < p.D) orow[d0 + 1] = static_cast<uint16_t>(pr >> 16);
    }
  }
  if (threadIdx.x == 0 && p.lse != nullptr) {
    p.lse[b * p.l_sb + hq * p.l_sh] = (mm != kNegInf && wsum > 0.0f) ? mm + logf(wsum) : kNegInf;
  }
}

// Split-K merge of the MLA decode for up to NS splits: one wave per (sequence, query
// head), lane l owns latent dims 8l .. 8l + 7 (one 16-byte read per split). Every read
// it needs (the context length, each split's lse and 16-bit partial row) is issued at
// once, so the merge costs one memory round trip rather than three dependent ones
// (length, then lse, then partials); splits past the sequence's length are read (the
// workspace holds n_splits rows per head) and given weight 0.
template <typename Tag, int NS>
__global__ __launch_bounds__(256) void mla_combine_kernel(const DecodeParams p) {
  using E = Elem<Tag>;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int lane = threadIdx.x & 63;
  const int bh = blockIdx.x * 4 + wave;
  if (bh >= p.B * p.Hq) return;  // wave-uniform; the kernel has no barrier
  const int b = bh / p.Hq;
  const int hq = bh - b * p.Hq;
  const int64_t base = static_cast<int64_t>(bh) * p.n_splits;
  const float* lse_row = p.ws_lse + base;
  const int d0 = 8 * lane;
  const bool dlive = d0 < p.D;  // D is a multiple of 8
  const int len = p.lens[b];
  float ls[NS];
  u32x4 v[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const bool in = s < p.n_splits;
    ls[s] = in ? lse_row[s] : kNegInf;
    v[s] = (in && dlive) ? *reinterpret_cast<const u32x4*>(p.ws_o16 + (base + s) * p.dp + d0)
                         : u32x4{0u, 0u, 0u, 0u};
  }
  const int L = min(max(len, 0), p.max_len);
  const int s1 = L > 0 ? (L + p.tps - 1) / p.tps : 0;  // splits that ran (no window)
  float mm = kNegInf;
#pragma unroll
  for (int s = 0; s < NS; ++s) mm = s < s1 ? fmaxf(mm, ls[s]) : mm;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float wsum = 0.0f;
  if (mm != kNegInf) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const bool use = s < s1;
      const float w = use ? __expf(ls[s] - mm) : 0.0f;  // exp(-inf) = 0 for empty partials
      wsum += w;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t word = v[s][e >> 1];
        const float x = E::to_f32(static_cast<uint16_t>((e & 1) ? (word >> 16) : (word & 0xffffu)));
        acc[e] = fmaf(w, use ? x : 0.0f, acc[e]);
      }
    }
  }
  const bool ok = mm != kNegInf && wsum > 0.0f;
  const float inv = ok ? 1.0f / wsum : 0.0f;
  uint16_t* orow = p.o + b * p.o_sb + hq * p.o_sh;
  if (dlive) {
    const u32x4 out = {E::pack2(acc[0] * inv, acc[1] * inv), E::pack2(acc[2] * inv, acc[3] * inv),
                       E::pack2(acc[4] * inv, acc[5] * inv), E::pack2(acc[6] * inv, acc[7] * inv)};
    if ((reinterpret_cast<uintptr_t>(orow) & 15u) == 0) {
      *reinterpret_cast<u32x4*>(orow + d0) = out;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        orow[d0 + e] = static_cast<uint16_t>((e & 1) ? (out[e >> 1] >> 16) : (out[e >> 1] & 0xffffu));
      }
    }
  }
  if (lane == 0 && p.lse != nullptr) {
    p.lse[b * p.l_sb + hq * p.l_sh] = ok ? mm + logf(wsum) : kNegInf;
  }
}

// ---------------------------------------------------------------------------------
// MLA decode over the compressed latent cache (absorbed form of the reference
// FastestFlashMLA attention, modules/flash_mla.py:116-172). With W_uk / W_uv the
// per-head slices of kv_up_proj, head h scores token t as
//   q_nope.(W_uk c_t) + q_rope.r_t = [W_uk^T q_nope, q_rope] . [c_t, r_t]
// and outputs sum_t p_t W_uv c_t = W_uv (sum_t p_t c_t). So every head attends over
// ONE shared KV row per token, [c_t (DV dims) | r_t (64 rope dims)], with V = its first
// DV dims: an MQA decode with D_qk = DV + 64, D_v = DV, whose latent-space output the
// host up-projects with W_uv. Each token costs (DV + 64) * 2 bytes for all heads.
//
// Pool layout: [num_pages, page_size, DV + 64], token t of sequence b at page
// block_tables[b][t / page_size], slot t % page_size (the PagedKVCache index law).
// Workgroup = 8 waves for (sequence, 32-head group) x split (mla_decode_split8_kernel
// below). 32-key tiles of the shared rows go HBM -> LDS (asm global_load_lds_dwordx4)
// into a 2-stage ring; S^T = K Q^T on v_mfma_f32_16x16x32, fp32 softmax with exp2 and
// deferred rescale, O^T += V^T P^T on v_mfma_f32_16x16x32 (V^T by ds_read_b64_tr_b16).
// Normalised (O, lse) partials per split are merged by mla_combine_kernel (up to 16
// splits) or decode_combine_kernel.
// ---------------------------------------------------------------------------------
constexpr int kMlaTile = 32;
constexpr int kMlaRope = 64;
constexpr int kMlaMaxSplit = 1024;
constexpr int kMlaDefaultSplit = 512;

struct MlaParams {
  const uint16_t* q;
  const uint16_t* kv;
  const int32_t* bt;
  const int32_t* lens;
  uint16_t* ws_o;  // [B][Hq][n_splits][DV] partials in the input's 16-bit type
  float* ws_lse;
  int64_t q_sb, q_sh;
  int bt_stride;
  int B, Hq, P, log2P, num_pages;
  int n_splits, tps, max_len;
  int n_hg;  // 32-head groups
  float score_mul;  // scale * log2e
};

__device__ inline int mla_page_of(const MlaParams& p, int tok, int& slot) {
  if (p.log2P >= 0) {
    slot = tok & (p.P - 1);
    return tok >> p.log2P;
  }
  const int pi = tok / p.P;
  slot = tok - pi * p.P;
  return pi;
}

// XOR swizzle of 16-byte chunks inside each aligned group of 8: a row is (DV+64)*2 bytes
// = 8 (mod 16) chunks, so rows r and r+2 would share banks; (r >> 1) & 7 spreads the 16
// rows of a K operand read, and the 4 rows of a transposed V read, over distinct banks.
__device__ inline int mla_swz(int r) { return (r >> 1) & 7; }

// ---------------------------------------------------------------------------------
// Eight-wave MLA split kernel (latent DV = 512 or 256): two waves per SIMD. Wave w
// takes head subgroup hs = w >> 2 (16 heads as MFMA columns) and output quarter
// dq = w & 3 (DV / 4 latent dims). S^T of a 32-token tile is cut into four pieces per
// head subgroup: key block kb = dq & 1 over k-step half kh = dq >> 1 (half of the
// (DV + 64) / 32 k-steps); each wave computes its piece and the four are summed from LDS
// as (kh 0 + kh 1) in every wave of the subgroup, so the subgroup's waves hold identical
// scores and softmax state. Against a four-wave layout (two waves per head subgroup,
// each computing a key block over all k-steps) this issues half the MFMAs per wave with
// the same LDS operand bytes per workgroup and measured 8-12 % faster except at
// whole-tile pages (latent 512, unchanged). At latent 512: 84 KiB of LDS (ring, staged
// block table, 8 KiB of pieces), one workgroup, eight waves, per CU.
// TILE_PAGE: page_size is a multiple of the 32-token tile, so a tile (they start at
// multiples of 32) never straddles a page: one wave-uniform page lookup per tile, and
// each load is the tile's base (SGPRs) plus a per-lane 32-bit offset fixed for the whole
// sweep. Otherwise every row of a tile finds its own page.
// ---------------------------------------------------------------------------------
constexpr int kMla8Waves = 8;
constexpr int kMla8Threads = 64 * kMla8Waves;

template <typename Tag, int DV, bool TILE_PAGE>
__global__ __launch_bounds__(kMla8Threads, 1) void mla_decode_split8_kernel(const MlaParams p) {
  using E = Elem<Tag>;
  constexpr int DQK = DV + kMlaRope;             // 576
  constexpr int CH = DQK / 8;                    // 72 chunks per row
  constexpr int TILE = kMlaTile * DQK;           // elements per tile
  constexpr int NPOS = kMlaTile * CH;            // 2304 chunk positions per tile
  constexpr int LPT = NPOS / kMla8Threads;       // 4 loads per lane per tile ...
  constexpr int XW = (NPOS - LPT * kMla8Threads) / 64;  // ... and one more in waves 0..XW-1
  static_assert((NPOS - LPT * kMla8Threads) % 64 == 0 && XW < kMla8Waves, "tile split");
  constexpr int KS = DQK / 32;                   // 18 k-steps
  constexpr int KH = KS / 2;                     // per k-step half
  static_assert(KS % 2 == 0, "k-step halves");
  constexpr int DW = DV / 4;                     // 128 output dims per wave
  constexpr int DBW = DW / 16;                   // 8 dim blocks per wave
  __shared__ __attribute__((aligned(1024))) uint16_t ring[2][TILE];
  __shared__ int bt_lds[kMlaMaxSplit];
  __shared__ __attribute__((aligned(16))) f32x4 xbuf[kMla8Waves][64];
  int* const bad_lds = reinterpret_cast<int*>(&xbuf[0][0]);

  const int split = blockIdx.y;
  const int b = blockIdx.x / p.n_hg;
  const int hg = blockIdx.x - b * p.n_hg;
  const int L = min(max(p.lens[b], 0), p.max_len);
  const int s_begin = split * p.tps;
  const int s_end = min(s_begin + p.tps, L);
  if (s_begin >= s_end) return;  // uniform across the workgroup: no barrier reached

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  const int hs = wave >> 2;  // head subgroup: MFMA columns = heads 16 hs + c16
  const int dq = wave & 3;   // output dim quarter
  const int kb = dq & 1;     // S^T key block of this wave's piece
  const int kh = dq >> 1;    // S^T k-step half of this wave's piece
  const int head = hg * 32 + hs * 16 + c16;
  const bool head_live = head < p.Hq;

  int slot0;
  const int pg0 = mla_page_of(p, s_begin, slot0);
  int slot1;
  const int pg1 = mla_page_of(p, s_end - 1, slot1);
  bool bad = false;
  {
    const int32_t* btrow = p.bt + static_cast<int64_t>(b) * p.bt_stride;
    for (int i = tid; i <= pg1 - pg0; i += kMla8Threads) {
      const int phys = btrow[pg0 + i];
      const bool ok = phys >= 0 && phys < p.num_pages;
      bt_lds[i] = ok ? phys : -1;
      bad = bad || !ok;
    }
  }
  const bool wave_bad = __any(bad);
  if (lane == 0) bad_lds[wave] = wave_bad ? 1 : 0;
  // Q^T as the B operand for this wave's k-steps: lane holds head `head`, dims
  // 32 (KH kh + i) + 8 g4 .. +7.
  u32x4 qreg[KH];
  {
    const uint16_t* qr = p.q + b * p.q_sb + static_cast<int64_t>(head_live ? head : 0) * p.q_sh;
#pragma unroll
    for (int i = 0; i < KH; ++i) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(qr + 32 * (KH * kh + i) + 8 * g4);
      qreg[i] = head_live ? v : u32x4{0u, 0u, 0u, 0u};
    }
  }
  wait_vmcnt0();
  __syncthreads();
  bool any_bad = false;
#pragma unroll
  for (int w = 0; w < kMla8Waves; ++w) any_bad = any_bad || bad_lds[w] != 0;

  const char* pool = reinterpret_cast<const char*>(p.kv);
  const int n_tiles = (s_end - s_begin + kMlaTile - 1) / kMlaTile;
  // Load j of this lane fills chunk position (8 j + wave) * 64 + lane of a tile (load
  // LPT only in waves 0 .. XW - 1).
  auto ld_pos = [&](int j) { return (kMla8Waves * j + wave) * 64 + lane; };
  uint32_t ld_off[LPT + 1];
#pragma unroll
  for (int j = 0; j <= LPT; ++j) {
    const int pos = min(ld_pos(j), NPOS - 1);
    const int row = pos / CH;
    const int pc = pos - row * CH;
    ld_off[j] = static_cast<uint32_t>(row * DQK * 2 + (pc ^ mla_swz(row)) * 16);
  }
  const bool extra = wave < XW;  // wave-uniform
  const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_addr(&ring[0][0]) + wave * 1024);
  auto tile_page = [&](int t0) {
    int slot;
    const int pg = mla_page_of(p, t0, slot);
    return __builtin_amdgcn_readfirstlane(bt_lds[pg - pg0]);
  };
  auto issue = [&](int t, int st) {
    const int t0 = s_begin + t * kMlaTile;
    if constexpr (TILE_PAGE) {
      int slot;
      mla_page_of(p, t0, slot);
      const int phys = max(tile_page(t0), 0);
      const char* tb = pool + (static_cast<int64_t>(phys) * p.P + slot) * DQK * 2;
      const uint32_t dst = ring_lds + st * TILE * 2;
      if (t0 + kMlaTile <= s_end) {
#pragma unroll
        for (int j = 0; j < LPT; ++j) load_lds16_async(tb, ld_off[j], dst + j * 1024 * kMla8Waves);
        if (extra) load_lds16_async(tb, ld_off[LPT], dst + LPT * 1024 * kMla8Waves);
      } else {
        // last tile of the split: rows past s_end - 1 re-read that row (masked)
        const int last = s_end - 1 - t0;
#pragma unroll
        for (int j = 0; j <= LPT; ++j) {
          if (j == LPT && !extra) break;
          const uint32_t back = static_cast<uint32_t>(max(0, ld_pos(j) / CH - last) * DQK * 2);
          load_lds16_async(tb, ld_off[j] - back, dst + j * 1024 * kMla8Waves);
        }
      }
    } else {
      uint16_t* dst = ring[st];
#pragma unroll
      for (int j = 0; j <= LPT; ++j) {
        if (j == LPT && !extra) break;
        const int pos = ld_pos(j);
        const int row = pos / CH;
        const int pc = pos - row * CH;
        const int tok = min(t0 + row, s_end - 1);  // rows past the split are masked
        int slot;
        const int pg = mla_page_of(p, tok, slot);
        const int64_t ro = (static_cast<int64_t>(max(bt_lds[pg - pg0], 0)) * p.P + slot) * DQK * 2;
        load_lds16_async(pool + ro + (pc ^ mla_swz(row)) * 16, lds_addr(dst + (kMla8Waves * j + wave) * 512));
      }
    }
  };

  const int ksw = mla_swz(c16);
  const int k_rd0 = c16 * DQK + (((0 + g4) ^ ksw) << 3);
  const int k_rd1 = c16 * DQK + (((4 + g4) ^ ksw) << 3);
  const int vrow = 4 * g4 + (c16 >> 2);
  const int vsw = mla_swz(vrow);
  int v_rd[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int col = dq * DW + 16 * u + 4 * (c16 & 3);
    v_rd[u] = vrow * DQK + (((col >> 3) ^ vsw) << 3) + (col & 7);
  }

  f32x4 oacc[DBW];
#pragma unroll
  for (int db = 0; db < DBW; ++db) oacc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf;
  float l_run = 0.0f;

  auto compute = [&](int t, const uint16_t* tl) {
    const int t0 = s_begin + t * kMlaTile;
    auto k_at = [&](int ks, int kbb) {
      return *reinterpret_cast<const u32x4*>(tl + ((ks & 1) ? k_rd1 : k_rd0) + (ks >> 1) * 64 +
                                             kbb * 16 * DQK);
    };
    f32x4 sp[2];
    sp[0] = f32x4{0.f, 0.f, 0.f, 0.f};
    sp[1] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 a_cur = k_at(KH * kh, kb);
#pragma unroll
    for (int i = 0; i < KH; ++i) {
      u32x4 a_nxt;
      if (i + 1 < KH) a_nxt = k_at(KH * kh + i + 1, kb);
      __builtin_amdgcn_sched_barrier(0);
      sp[i & 1] = E::mfma16(a_cur, qreg[i], sp[i & 1]);
      if (i + 1 < KH) a_cur = a_nxt;
    }
    xbuf[wave][lane] = sp[0] + sp[1];
    __syncthreads();  // every piece of every head subgroup is in xbuf
    f32x4 sacc[2];
#pragma unroll
    for (int kbb = 0; kbb < 2; ++kbb) {
      sacc[kbb] = xbuf[4 * hs + kbb][lane] + xbuf[4 * hs + 2 + kbb][lane];
    }
    const bool tile_ok = !TILE_PAGE || !any_bad || tile_page(t0) >= 0;  // uniform
    float mt = kNegInf;
#pragma unroll
    for (int kbb = 0; kbb < 2; ++kbb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tok = t0 + 16 * kbb + 4 * g4 + j;
        bool live = tok < s_end && tile_ok;
        if (!TILE_PAGE && any_bad && live) {
          int slot;
          live = bt_lds[mla_page_of(p, tok, slot) - pg0] >= 0;
        }
        const float x = live ? sacc[kbb][j] * p.score_mul : kNegInf;
        sacc[kbb][j] = x;
        mt = fmaxf(mt, x);
      }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = wave_pair_max(mt);
    const float m_new = fmaxf(m_run, mt);
    const bool need = m_new > m_run + kRescaleThresh;
    if (__any(need)) {
      const float alpha = need ? fast_exp2(m_run - m_new) : 1.0f;
      m_run = need ? m_new : m_run;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DBW; ++db) {
#pragma unroll
        for (int j = 0; j < 4; ++j) oacc[db][j] *= alpha;
      }
    }
    const float mu = (m_run == kNegInf) ? 0.0f : m_run;
    u32x2 pk[2];
#pragma unroll
    for (int kbb = 0; kbb < 2; ++kbb) {
      float e[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        e[j] = fast_exp2(sacc[kbb][j] - mu);
        l_run += e[j];
      }
      pk[kbb] = u32x2{E::pack2(e[0], e[1]), E::pack2(e[2], e[3])};
    }
    const u32x4 pb = {pk[0][0], pk[0][1], pk[1][0], pk[1][1]};
#pragma unroll
    for (int db = 0; db < DBW; ++db) {
      const int off = v_rd[db & 3] + (db >> 2) * 64;
      const u32x2 a0 = lds_read_tr16(tl + off);
      const u32x2 a1 = lds_read_tr16(tl + off + 16 * DQK);
      oacc[db] = E::mfma16(u32x4{a0[0], a0[1], a1[0], a1[1]}, pb, oacc[db]);
    }
  };

  if (n_tiles > 0) issue(0, 0);
  for (int t = 0; t < n_tiles; ++t) {
    wait_vmcnt0();
    __syncthreads();  // tile t is in LDS; every wave is done with stage (t + 1) & 1
    if (t + 1 < n_tiles) issue(t + 1, (t + 1) & 1);
    compute(t, ring[t & 1]);
  }

  float l_tot = l_run + __shfl_xor(l_run, 16);
  l_tot = wave_pair_sum(l_tot);
  if (!head_live) return;
  const int64_t row = (static_cast<int64_t>(b) * p.Hq + head) * p.n_splits + split;
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  uint16_t* wo = p.ws_o + row * DV + dq * DW + 4 * g4;
#pragma unroll
  for (int db = 0; db < DBW; ++db) {
    const u32x2 v = {E::pack2(oacc[db][0] * inv, oacc[db][1] * inv),
                     E::pack2(oacc[db][2] * inv, oacc[db][3] * inv)};
    *reinterpret_cast<u32x2*>(wo + 16 * db) = v;
  }
  if (dq == 0 && g4 == 0) {
    p.ws_lse[row] = l_tot > 0.0f ? (m_run + fast_log2(l_tot)) * kLn2 : kNegInf;
  }
}

// get_kv: copy the first context_len tokens of one sequence into [H, L, D].
template <typename U>
__global__ __launch_bounds__(256) void paged_gather_kernel(const U* __restrict__ kp,
                                                           const U* __restrict__ vp,
                                                           U* __restrict__ ko, U* __restrict__ vo,
                                                           const int32_t* __restrict__ pt,
                                                           int num_pages, int H, int P,
                                                           int row_units, int L) {
  const int64_t total = static_cast<int64_t>(H) * L * row_units;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int u = static_cast<int>(i % row_units);
    const int64_t ht = i / row_units;
    const int t = static_cast<int>(ht % L);
    const int h = static_cast<int>(ht / L);
    const int phys = pt[t / P];
    const int slot = t - (t / P) * P;
    U kv = U{};
    U vv = U{};
    if (phys >= 0 && phys < num_pages) {
      const int64_t src = ((static_cast<int64_t>(phys) * H + h) * P + slot) * row_units + u;
      kv = kp[src];
      vv = vp[src];
    }
    ko[i] = kv;
    vo[i] = vv;
  }
}

// append_tokens: token t (0 <= t < n) of [H, n, D] new K/V goes to page
// pt[(start + t) / P], slot (start + t) % P of every head. One thread per unit U of
// a row; consecutive threads cover consecutive units of one (head, token) row, so the
// reads of a row and its write into the page are both contiguous.
template <typename U>
__global__ __launch_bounds__(256) void paged_append_kernel(
    U* __restrict__ kp, U* __restrict__ vp, const U* __restrict__ kn, const U* __restrict__ vn,
    const int32_t* __restrict__ pt, int64_t k_sh, int64_t k_st, int64_t v_sh, int64_t v_st,
    int num_pages, int H, int P, int row_units, int start, int n) {
  const int64_t total = static_cast<int64_t>(H) * n * row_units;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int u = static_cast<int>(i % row_units);
    const int64_t ht = i / row_units;
    const int t = static_cast<int>(ht % n);
    const int h = static_cast<int>(ht / n);
    const int pos = start + t;
    const int phys = pt[pos / P];
    if (phys < 0 || phys >= num_pages) continue;
    const int slot = pos - (pos / P) * P;
    const int64_t dst = ((static_cast<int64_t>(phys) * H + h) * P + slot) * row_units + u;
    kp[dst] = kn[h * k_sh + t * k_st + u];
    if (vp != nullptr) vp[dst] = vn[h * v_sh + t * v_st + u];
  }
}

template <typename Tag, int DP>
void launch_decode_dp(const DecodeParams& p, bool softcap, dim3 grid, hipStream_t s) {
  if (softcap) {
    hipLaunchKernelGGL((decode_split_kernel<Tag, DP, true>), grid, dim3(kDecThreads), 0, s, p);
  } else {
    hipLaunchKernelGGL((decode_split_kernel<Tag, DP, false>), grid, dim3(kDecThreads), 0, s, p);
  }
}

template <typename Tag>
void launch_decode_tag(DecodeParams& p, bool softcap, dim3 grid, hipStream_t s) {
  if (p.D <= 32) {
    p.dp = 32;
    launch_decode_dp<Tag, 32>(p, softcap, grid, s);
  } else if (p.D <= 64) {
    p.dp = 64;
    launch_decode_dp<Tag, 64>(p, softcap, grid, s);
  } else if (p.D <= 128) {
    p.dp = 128;
    launch_decode_dp<Tag, 128>(p, softcap, grid, s);
  } else if (p.D <= 192) {
    p.dp = 192;
    launch_decode_dp<Tag, 192>(p, softcap, grid, s);
  } else {
    p.dp = 256;
    launch_decode_dp<Tag, 256>(p, softcap, grid, s);
  }
  hipLaunchKernelGGL((decode_combine_kernel<Tag, false>), dim3(p.B * p.Hq), dim3(64), 0, s, p);
}

int dp_of(int d) { return d <= 32 ? 32 : d <= 64 ? 64 : d <= 128 ? 128 : d <= 192 ? 192 : 256; }

}  // namespace

int32_t decode_tokens_per_split(int32_t tokens_per_split) {
  if (tokens_per_split <= 0) return kDefaultSplit;
  const int32_t t = ((tokens_per_split + kTile - 1) / kTile) * kTile;
  return t < kMinSplit ? kMinSplit : (t > kMaxSplit ? kMaxSplit : t);
}

int32_t decode_num_splits(int32_t max_context_len, int32_t tokens_per_split) {
  const int32_t tps = decode_tokens_per_split(tokens_per_split);
  return max_context_len <= 0 ? 1 : (max_context_len + tps - 1) / tps;
}

size_t decode_workspace_bytes(int32_t batch, int32_t heads_q, int32_t head_dim,
                              int32_t max_context_len, int32_t tokens_per_split) {
  const size_t ns = static_cast<size_t>(decode_num_splits(max_context_len, tokens_per_split));
  const size_t rows = static_cast<size_t>(batch) * heads_q * ns;
  return rows * (static_cast<size_t>(dp_of(head_dim)) + 1) * sizeof(float);
}

int launch_paged_decode(const ffa_paged_decode_args& a, hipStream_t stream) {
  DecodeParams p{};
  p.q = static_cast<const uint16_t*>(a.q);
  p.kp = static_cast<const uint16_t*>(a.k_pages);
  p.vp = static_cast<const uint16_t*>(a.v_pages);
  p.o = static_cast<uint16_t*>(a.o);
  p.lse = a.lse;
  p.bt = a.block_tables;
  p.lens = a.context_lens;
  p.B = a.batch;
  p.Hq = a.heads_q;
  p.Hkv = a.heads_kv;
  p.G = a.heads_q / a.heads_kv;
  p.D = a.head_dim;
  p.P = a.page_size;
  p.log2P = ((a.page_size & (a.page_size - 1)) == 0) ? __builtin_ctz(a.page_size) : -1;
  p.num_pages = a.num_pages;
  p.tps = decode_tokens_per_split(a.tokens_per_split);
  p.n_splits = decode_num_splits(a.max_context_len, a.tokens_per_split);
  p.window = a.window > 0 ? a.window : 0;
  p.max_len = a.max_context_len;
  p.n_cg = (p.G + kCols - 1) / kCols;
  p.dp = dp_of(a.head_dim);
  p.q_sb = a.q_stride[0];
  p.q_sh = a.q_stride[1];
  p.o_sb = a.o_stride[0];
  p.o_sh = a.o_stride[1];
  p.l_sb = a.lse_stride[0];
  p.l_sh = a.lse_stride[1];
  p.page_stride = static_cast<int64_t>(a.heads_kv) * a.page_size * a.head_dim;
  p.head_stride = static_cast<int64_t>(a.page_size) * a.head_dim;
  p.bt_stride = a.block_table_stride;
  const bool softcap = a.softcap > 0.0f;
  if (softcap) {
    p.score_mul = a.scale / a.softcap;
    p.cap_mul = a.softcap * kLog2e;
  } else {
    p.score_mul = a.scale * kLog2e;
    p.cap_mul = 0.0f;
  }
  const size_t rows = static_cast<size_t>(a.batch) * a.heads_q * p.n_splits;
  p.ws_o = static_cast<float*>(a.workspace);
  p.ws_lse = p.ws_o + rows * p.dp;

  const int64_t gx = static_cast<int64_t>(a.batch) * a.heads_kv * p.n_cg;
  if (gx > 0x7fffffff || p.n_splits > 65535 ||
      static_cast<int64_t>(a.batch) * a.heads_q > 0x7fffffff) {
    return FFA_ERR_TOO_LARGE;
  }
  const dim3 grid(static_cast<unsigned>(gx), p.n_splits);
  if (a.dtype == FFA_DTYPE_BF16) {
    launch_decode_tag<Bf16Tag>(p, softcap, grid, stream);
  } else {
    launch_decode_tag<F16Tag>(p, softcap, grid, stream);
  }
  return hipGetLastError() == hipSuccess ? FFA_OK : FFA_ERR_LAUNCH;
}

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the current device's scratch array, resolved once per device
// (with that device current) and kept.
int noalloc_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    return FFA_ERR_NO_DEVICE;
  }
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
        (void)hipGetLastError();  // leave no error behind for the next call's launch check
        return FFA_ERR_NO_DEVICE;
      }
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return FFA_OK;
}

}  // namespace

int launch_paged_decode_noalloc(const ffa_paged_decode_args& a, hipStream_t stream) {
  const size_t need = decode_workspace_bytes(a.batch, a.heads_q, a.head_dim, a.max_context_len,
                                             a.tokens_per_split);
  if (need > FFA_NOALLOC_SCRATCH_BYTES) return FFA_ERR_SCRATCH_LIMIT;
  void* ptr = nullptr;
  const int rc = noalloc_scratch(&ptr);
  if (rc != FFA_OK) return rc;
  ffa_paged_decode_args b = a;
  b.workspace = ptr;
  b.workspace_bytes = FFA_NOALLOC_SCRATCH_BYTES;
  return launch_paged_decode(b, stream);
}

int launch_paged_gather(const ffa_paged_gather_args& a, hipStream_t stream) {
  const int64_t row_bytes = static_cast<int64_t>(a.head_dim) * a.elem_bytes;
  const uintptr_t align = reinterpret_cast<uintptr_t>(a.k_pages) |
                          reinterpret_cast<uintptr_t>(a.v_pages) |
                          reinterpret_cast<uintptr_t>(a.k_out) |
                          reinterpret_cast<uintptr_t>(a.v_out);
  const int64_t units_total = static_cast<int64_t>(a.heads_kv) * a.context_len;
  auto grid_for = [&](int64_t units) {
    const int64_t blocks = (units + 255) / 256;
    return static_cast<unsigned>(blocks < 65536 ? (blocks < 1 ? 1 : blocks) : 65536);
  };
  if (row_bytes % 16 == 0 && (align & 15u) == 0) {
    const int ru = static_cast<int>(row_bytes / 16);
    hipLaunchKernelGGL(paged_gather_kernel<u32x4>, dim3(grid_for(units_total * ru)), dim3(256), 0,
                       stream, static_cast<const u32x4*>(a.k_pages),
                       static_cast<const u32x4*>(a.v_pages), static_cast<u32x4*>(a.k_out),
                       static_cast<u32x4*>(a.v_out), a.page_table, a.num_pages, a.heads_kv,
                       a.page_size, ru, a.context_len);
  } else if (row_bytes % 4 == 0 && (align & 3u) == 0) {
    const int ru = static_cast<int>(row_bytes / 4);
    hipLaunchKernelGGL(paged_gather_kernel<uint32_t>, dim3(grid_for(units_total * ru)), dim3(256),
                       0, stream, static_cast<const uint32_t*>(a.k_pages),
                       static_cast<const uint32_t*>(a.v_pages), static_cast<uint32_t*>(a.k_out),
                       static_cast<uint32_t*>(a.v_out), a.page_table, a.num_pages, a.heads_kv,
                       a.page_size, ru, a.context_len);
  } else {
    const int ru = static_cast<int>(row_bytes / 2);
    hipLaunchKernelGGL(paged_gather_kernel<uint16_t>, dim3(grid_for(units_total * ru)), dim3(256),
                       0, stream, static_cast<const uint16_t*>(a.k_pages),
                       static_cast<const uint16_t*>(a.v_pages), static_cast<uint16_t*>(a.k_out),
                       static_cast<uint16_t*>(a.v_out), a.page_table, a.num_pages, a.heads_kv,
                       a.page_size, ru, a.context_len);
  }
  return hipGetLastError() == hipSuccess ? FFA_OK : FFA_ERR_LAUNCH;
}

int launch_paged_append(const ffa_paged_append_args& a, hipStream_t stream) {
  const int64_t row_bytes = static_cast<int64_t>(a.head_dim) * a.elem_bytes;
  const uintptr_t align = reinterpret_cast<uintptr_t>(a.k_pages) |
                          reinterpret_cast<uintptr_t>(a.v_pages) |
                          reinterpret_cast<uintptr_t>(a.k_new) |
                          reinterpret_cast<uintptr_t>(a.v_new);
  // strides in bytes must keep every row on the unit's alignment
  const int64_t sb[4] = {a.k_new_stride[0] * a.elem_bytes, a.k_new_stride[1] * a.elem_bytes,
                         a.v_new_stride[0] * a.elem_bytes, a.v_new_stride[1] * a.elem_bytes};
  auto fits = [&](int64_t unit) {
    if (row_bytes % unit != 0 || (align % unit) != 0) return false;
    for (int64_t x : sb) {
      if (x % unit != 0) return false;
    }
    return true;
  };
  const int64_t rows = static_cast<int64_t>(a.heads_kv) * a.n_tokens;
  auto grid_for = [&](int64_t units) {
    const int64_t blocks = (units + 255) / 256;
    return static_cast<unsigned>(blocks < 65536 ? (blocks < 1 ? 1 : blocks) : 65536);
  };
  auto run = [&](auto unit_tag, int64_t unit) {
    using U = decltype(unit_tag);
    const int ru = static_cast<int>(row_bytes / unit);
    const int64_t eu = unit / a.elem_bytes;  // elements per unit
    hipLaunchKernelGGL(paged_append_kernel<U>, dim3(grid_for(rows * ru)), dim3(256), 0, stream,
                       static_cast<U*>(a.k_pages), static_cast<U*>(a.v_pages),
                       static_cast<const U*>(a.k_new), static_cast<const U*>(a.v_new),
                       a.page_table, a.k_new_stride[0] / eu, a.k_new_stride[1] / eu,
                       a.v_new_stride[0] / eu, a.v_new_stride[1] / eu, a.num_pages, a.heads_kv,
                       a.page_size, ru, a.start, a.n_tokens);
  };
  if (fits(16)) {
    run(u32x4{}, 16);
  } else if (fits(4)) {
    run(uint32_t{}, 4);
  } else if (a.elem_bytes == 2) {
    run(uint16_t{}, 2);
  } else {
    return FFA_ERR_MISALIGNED;  // 4-byte elements off 4-byte alignment
  }
  return hipGetLastError() == hipSuccess ? FFA_OK : FFA_ERR_LAUNCH;
}


int32_t mla_decode_tokens_per_split(int32_t tokens_per_split) {
  if (tokens_per_split <= 0) return kMlaDefaultSplit;
  const int32_t t = ((tokens_per_split + kMlaTile - 1) / kMlaTile) * kMlaTile;
  return t > kMlaMaxSplit ? kMlaMaxSplit : t;
}

int32_t mla_decode_num_splits(int32_t max_context_len, int32_t tokens_per_split) {
  const int32_t tps = mla_decode_tokens_per_split(tokens_per_split);
  return max_context_len <= 0 ? 1 : (max_context_len + tps - 1) / tps;
}

size_t mla_decode_workspace_bytes(int32_t batch, int32_t heads_q, int32_t dim_v,
                                  int32_t max_context_len, int32_t tokens_per_split) {
  const size_t ns = static_cast<size_t>(mla_decode_num_splits(max_context_len, tokens_per_split));
  const size_t rows = static_cast<size_t>(batch) * heads_q * ns;
  // 16-bit O partials, then fp32 lse partials (rows * dim_v * 2 keeps them 16-byte aligned)
  return rows * (static_cast<size_t>(dim_v) * 2 + sizeof(float));
}

namespace {

template <typename Tag>
void launch_mla_tag(const MlaParams& mp, const DecodeParams& cp, int dim_v, dim3 grid,
                    hipStream_t s) {
  // The whole-tile page path serves latent 512 only: a latent-256 instantiation of it
  // (in an earlier four-wave kernel) gave wrong scores on MI355X (deterministically, for
  // some lanes of one key block: a K operand read returned the 16 bytes of a later
  // k-step's read) although its LDS tile and Q registers were verified correct; latent
  // 256 uses per-row page lookups at every page size.
  const bool tile_page = mp.P % kMlaTile == 0 && dim_v == 512;
  if (dim_v == 512) {
    if (tile_page) {
      hipLaunchKernelGGL((mla_decode_split8_kernel<Tag, 512, true>), grid, dim3(kMla8Threads), 0, s, mp);
    } else {
      hipLaunchKernelGGL((mla_decode_split8_kernel<Tag, 512, false>), grid, dim3(kMla8Threads), 0, s, mp);
    }
  } else {
    hipLaunchKernelGGL((mla_decode_split8_kernel<Tag, 256, false>), grid, dim3(kMla8Threads), 0, s, mp);
  }
  const unsigned heads4 = static_cast<unsigned>((static_cast<int64_t>(cp.B) * cp.Hq + 3) / 4);
  if (cp.n_splits <= 8) {
    hipLaunchKernelGGL((mla_combine_kernel<Tag, 8>), dim3(heads4), dim3(256), 0, s, cp);
  } else if (cp.n_splits <= 16) {
    hipLaunchKernelGGL((mla_combine_kernel<Tag, 16>), dim3(heads4), dim3(256), 0, s, cp);
  } else {
    // many splits: one wave per 128-dim slice of the latent output dims, splits walked in
    // groups of eight
    hipLaunchKernelGGL((decode_combine_kernel<Tag, true>), dim3(cp.B * cp.Hq), dim3(dim_v / 2), 0, s, cp);
  }
}

}  // namespace

int launch_mla_decode(const ffa_mla_decode_args& a, hipStream_t stream) {
  MlaParams mp{};
  mp.q = static_cast<const uint16_t*>(a.q);
  mp.kv = static_cast<const uint16_t*>(a.kv_pages);
  mp.bt = a.block_tables;
  mp.lens = a.context_lens;
  mp.q_sb = a.q_stride[0];
  mp.q_sh = a.q_stride[1];
  mp.bt_stride = a.block_table_stride;
  mp.B = a.batch;
  mp.Hq = a.heads_q;
  mp.P = a.page_size;
  mp.log2P = ((a.page_size & (a.page_size - 1)) == 0) ? __builtin_ctz(a.page_size) : -1;
  mp.num_pages = a.num_pages;
  mp.tps = mla_decode_tokens_per_split(a.tokens_per_split);
  mp.n_splits = mla_decode_num_splits(a.max_context_len, a.tokens_per_split);
  mp.max_len = a.max_context_len;
  mp.score_mul = a.scale * kLog2e;
  const size_t rows = static_cast<size_t>(a.batch) * a.heads_q * mp.n_splits;
  mp.ws_o = static_cast<uint16_t*>(a.workspace);
  mp.ws_lse = reinterpret_cast<float*>(mp.ws_o + rows * a.dim_v);

  // the split-K merge is the paged-decode combine kernel over dim_v output dims
  DecodeParams cp{};
  cp.o = static_cast<uint16_t*>(a.o);
  cp.lse = a.lse;
  cp.lens = a.context_lens;
  cp.ws_o16 = mp.ws_o;
  cp.ws_lse = mp.ws_lse;
  cp.o_sb = a.o_stride[0];
  cp.o_sh = a.o_stride[1];
  cp.l_sb = a.lse_stride[0];
  cp.l_sh = a.lse_stride[1];
  cp.B = a.batch;
  cp.Hq = a.heads_q;
  cp.D = a.dim_v;
  cp.dp = a.dim_v;
  cp.n_splits = mp.n_splits;
  cp.tps = mp.tps;
  cp.window = 0;
  cp.max_len = a.max_context_len;

  mp.n_hg = (a.heads_q + 31) / 32;
  const int64_t gx = static_cast<int64_t>(a.batch) * mp.n_hg;
  if (gx > 0x7fffffff || mp.n_splits > 65535 ||
      static_cast<int64_t>(a.batch) * a.heads_q > 0x7fffffff) {
    return FFA_ERR_TOO_LARGE;
  }
  const dim3 grid(static_cast<unsigned>(gx), mp.n_splits);
  if (a.dtype == FFA_DTYPE_BF16) {
    launch_mla_tag<Bf16Tag>(mp, cp, a.dim_v, grid, stream);
  } else {
    launch_mla_tag<F16Tag>(mp, cp, a.dim_v, grid, stream);
  }
  return hipGetLastError() == hipSuccess ? FFA_OK : FFA_ERR_LAUNCH;
}

}  // namespace ffa
