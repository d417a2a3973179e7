// Fused forward attention (prefill) for gfx950.
//
// Semantics follow flash_attn_cpu_forward (reference kernels/cpu_reference.py:132-312):
// scores in fp32, softcap before masking, causal / one-sided sliding window relative to
// q_offset, GQA head map h -> h / (Hq / Hkv), natural-log LSE.
//
// Work decomposition: one workgroup (4 waves, 256 threads) per (batch, q-head, 128-row
// query tile); each wave owns 32 query rows for the whole KV sweep.
//
// Per KV tile of BN keys (BN = 64 for head_dim <= 128, 32 above):
//   S^T[key, q] = K Q^T   v_mfma_f32_32x32x16 with K (LDS) as A and Q (registers) as B,
//                         so lane l holds 32*BN/64 scores of ONE query (l % 32): the
//                         row max needs one lane swap (l ^ 32), the row sum none until
//                         the epilogue.
//   P = exp2(S*scale*log2e - m)   fp32, m updated only when it grows by more than
//                         2^8 (deferred rescale: O and l are rescaled only then).
//   O^T[d, q] += V^T P^T  A = V^T from LDS, B = P packed to 16 bit straight from the
//                         S^T accumulator registers: the MFMA C layout of S^T holds,
//                         per lane, exactly the keys the B operand of the next MFMA
//                         needs once the PV contraction uses the matching key order.
// V is stored in LDS as key quads ([key/4][dim][4 keys]) so each A operand of the PV
// product is two 8-byte LDS reads, with no transpose instruction.
// K/V tiles are double-buffered in LDS; the global loads of tile t+2 are in flight
// while tile t is computed, so each iteration has a single barrier.
// Causal / window tiles outside a workgroup's band are never loaded; tiles outside a
// wave's band are loaded but skip the wave's MFMA work; element masks are evaluated
// only on band-edge tiles.
// Grid order: heaviest causal query tiles first, and (when the grid is a multiple of
// 8) consecutive tiles of one head are placed on one XCD so its K/V stay in that L2.

#include "ffa_common.h"
#include "ffa_internal.h"

namespace ffa {
namespace {

constexpr int kThreads = 256;
constexpr int kBlockM = 128;
constexpr float kRescaleThresh = 8.0f;  // log2 units

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
  int q_offset, causal, window;
  int ratio;
  int n_qt;
  float score_mul;  // scale*log2e, or scale/softcap with softcap
  float cap_mul;    // softcap*log2e (softcap only)
  int ref_bq, ref_bkv;
  int masked_lse_mode;
  int vec;
  int xcd_remap;
};

template <int DP, int BN>
struct Shape {
  static constexpr int KSTR = DP + 8;  // K row stride in 16-bit elements (16 B pad)
  static constexpr int VSTR = DP * 4;  // V key-quad row stride in 16-bit elements
  static constexpr int K_ELEMS = BN * KSTR;
  static constexpr int V_ELEMS = (BN / 4) * VSTR;
  static constexpr int KCHUNKS = BN * DP / 8;
  static constexpr int KPT = (KCHUNKS + kThreads - 1) / kThreads;
  static constexpr int VITEMS = (BN / 4) * (DP / 8);
  static constexpr int VPT = (VITEMS + kThreads - 1) / kThreads;
  static constexpr int NB = BN / 32;
  static constexpr int NC = BN / 16;
  static constexpr int KS = DP / 16;
  static constexpr int DB = DP / 32;
};

// LSE of a row with no visible key, as the reference loop produces it: each visited
// tile adds log(1e-30) by logaddexp (cpu_reference.py:288-297), so n visited tiles
// give log(n) + log(1e-30); no visited tile leaves -inf. Tiles are the reference's
// (ref_bq x ref_bkv) tiles, visited per cpu_reference.py:215-231.
__device__ float masked_row_lse(const PrefillParams& p, int row) {
  if (p.masked_lse_mode != 0) return kNegInf;
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
  const int n = j_hi - j_lo + 1;
  if (n <= 0) return kNegInf;
  return logf(static_cast<float>(n)) + logf(1e-30f);
}

// Two workgroups per CU (2 waves per SIMD, <= 256 VGPRs) up to head_dim 192; the
// 256-dim variant keeps 128 fp32 accumulators per lane and runs one wave per SIMD.
template <int DP>
constexpr int kMinBlocks = DP <= 192 ? 2 : 1;

template <typename Tag, int DP, int BN, bool SOFTCAP>
__global__ __launch_bounds__(kThreads, kMinBlocks<DP>) void prefill_kernel(const PrefillParams p) {
  using S = Shape<DP, BN>;
  using E = Elem<Tag>;
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][S::K_ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][S::V_ELEMS];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;

  int bid = blockIdx.x;
  if (p.xcd_remap) {
    const int per_xcd = gridDim.x >> 3;
    bid = (bid & 7) * per_xcd + (bid >> 3);
  }
  const int bh = bid / p.n_qt;
  const int jq = bid - bh * p.n_qt;
  const int qt = p.causal ? (p.n_qt - 1 - jq) : jq;
  const int b = bh / p.Hq;
  const int h = bh - b * p.Hq;
  const int hk = h / p.ratio;

  const uint16_t* __restrict__ qbase = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* __restrict__ kbase = p.k + b * p.k_sb + hk * p.k_sh;
  const uint16_t* __restrict__ vbase = p.v + b * p.v_sb + hk * p.v_sh;
  const bool vec = p.vec != 0;
  const int D = p.D;
  const int Skv = p.Skv;

  const int q0 = qt * kBlockM;
  const int q_last = min(q0 + kBlockM, p.Sq) - 1;
  const int q0_abs = p.q_offset + q0;
  const int ql_abs = p.q_offset + q_last;
  const int kv_lo = p.window > 0 ? max(0, q0_abs - p.window + 1) : 0;
  const int kv_hi = p.causal ? min(Skv, ql_abs + 1) : Skv;
  const int t_begin = kv_lo / BN;
  const int t_end = kv_hi > kv_lo ? (kv_hi + BN - 1) / BN : t_begin;

  const int qw0 = q0 + wave * 32;
  const int qrow = qw0 + l32;
  const bool wave_live = qw0 < p.Sq;
  const int qw0_abs = p.q_offset + qw0;
  const int qwl_abs = p.q_offset + min(qw0 + 31, p.Sq - 1);
  const int qa = p.q_offset + qrow;

  // Q^T as the B operand: lane holds row qrow, dims 16*ks + 8g .. +7.
  u32x4 qreg[S::KS];
  {
    const bool rv = qrow < p.Sq;
    const uint16_t* qr = qbase + static_cast<int64_t>(qrow) * p.q_ss;
#pragma unroll
    for (int ks = 0; ks < S::KS; ++ks) {
      qreg[ks] = rv ? load_row8(qr, 16 * ks + 8 * g, D, vec) : u32x4{0u, 0u, 0u, 0u};
    }
  }

  f32x16 oacc[S::DB];
#pragma unroll
  for (int db = 0; db < S::DB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.0f;
  }
  float m_run = kNegInf;
  float l_run = 0.0f;

  u32x4 kst[S::KPT];
  u32x4 vst[S::VPT][4];

  auto gload = [&](int t) {
    const int kt0 = t * BN;
#pragma unroll
    for (int i = 0; i < S::KPT; ++i) {
      const int idx = tid + i * kThreads;
      if (idx < S::KCHUNKS) {
        const int row = idx / (DP / 8);
        const int c8 = idx - row * (DP / 8);
        const int key = kt0 + row;
        kst[i] = key < Skv ? load_row8(kbase + static_cast<int64_t>(key) * p.k_ss, c8 * 8, D, vec)
                           : u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int i = 0; i < S::VPT; ++i) {
      const int idx = tid + i * kThreads;
      if (idx < S::VITEMS) {
        const int kq = idx / (DP / 8);
        const int c8 = idx - kq * (DP / 8);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = kt0 + 4 * kq + r;
          vst[i][r] = key < Skv
                          ? load_row8(vbase + static_cast<int64_t>(key) * p.v_ss, c8 * 8, D, vec)
                          : u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
  };

  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < S::KPT; ++i) {
      const int idx = tid + i * kThreads;
      if (idx < S::KCHUNKS) {
        const int row = idx / (DP / 8);
        const int c8 = idx - row * (DP / 8);
        *reinterpret_cast<u32x4*>(&k_lds[buf][row * S::KSTR + c8 * 8]) = kst[i];
      }
    }
#pragma unroll
    for (int i = 0; i < S::VPT; ++i) {
      const int idx = tid + i * kThreads;
      if (idx < S::VITEMS) {
        const int kq = idx / (DP / 8);
        const int c8 = idx - kq * (DP / 8);
        u32x4 out[4];
        quad_interleave(vst[i][0], vst[i][1], vst[i][2], vst[i][3], out);
        u32x4* dst = reinterpret_cast<u32x4*>(&v_lds[buf][kq * S::VSTR + c8 * 32]);
#pragma unroll
        for (int w = 0; w < 4; ++w) dst[w] = out[w];
      }
    }
  };

  auto compute = [&](int buf, int t) {
    const int kt0 = t * BN;
    if (!wave_live) return;
    if (p.causal && kt0 > qwl_abs) return;
    if (p.window > 0 && kt0 + BN - 1 < qw0_abs - p.window + 1) return;
    const bool need_mask = (kt0 + BN > Skv) || (p.causal && kt0 + BN - 1 > qw0_abs) ||
                           (p.window > 0 && kt0 < qwl_abs - p.window + 1);

    f32x16 sacc[S::NB];
#pragma unroll
    for (int nb = 0; nb < S::NB; ++nb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[nb][r] = 0.0f;
    }
    const uint16_t* kl = &k_lds[buf][0];
#pragma unroll
    for (int ks = 0; ks < S::KS; ++ks) {
#pragma unroll
      for (int nb = 0; nb < S::NB; ++nb) {
        const u32x4 a =
            *reinterpret_cast<const u32x4*>(kl + (32 * nb + l32) * S::KSTR + 16 * ks + 8 * g);
        sacc[nb] = E::mfma32(a, qreg[ks], sacc[nb]);
      }
    }

    float mt = kNegInf;
#pragma unroll
    for (int nb = 0; nb < S::NB; ++nb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = sacc[nb][r];
        if constexpr (SOFTCAP) {
          x = p.cap_mul * tanh_approx(x * p.score_mul);
        } else {
          x = x * p.score_mul;
        }
        if (need_mask) {
          const int key = kt0 + 32 * nb + 8 * (r >> 2) + 4 * g + (r & 3);
          const bool ok = key < Skv && (!p.causal || key <= qa) &&
                          (p.window <= 0 || key >= qa - p.window + 1);
          x = ok ? x : kNegInf;
        }
        sacc[nb][r] = x;
        mt = fmaxf(mt, x);
      }
    }
    mt = fmaxf(mt, wave_xor32(mt));
    const float m_new = fmaxf(m_run, mt);
    const bool need = m_new > m_run + kRescaleThresh;
    if (__any(need)) {
      const float alpha = need ? fast_exp2(m_run - m_new) : 1.0f;
      m_run = need ? m_new : m_run;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < S::DB; ++db) {
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
      }
    }
    const float mu = (m_run == kNegInf) ? 0.0f : m_run;

    u32x4 pk[S::NC];
#pragma unroll
    for (int c = 0; c < S::NC; ++c) {
      const int nb = c >> 1;
      const int base = (c & 1) * 8;
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pv[e] = fast_exp2(sacc[nb][base + e] - mu);
        l_run += pv[e];
      }
      pk[c] = u32x4{E::pack2(pv[0], pv[1]), E::pack2(pv[2], pv[3]), E::pack2(pv[4], pv[5]),
                    E::pack2(pv[6], pv[7])};
    }

    const uint16_t* vl = &v_lds[buf][0];
#pragma unroll
    for (int c = 0; c < S::NC; ++c) {
      const int kq0 = 4 * c + g;
      const int kq1 = 4 * c + 2 + g;
#pragma unroll
      for (int db = 0; db < S::DB; ++db) {
        const int d = 32 * db + l32;
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vl + kq0 * S::VSTR + d * 4);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vl + kq1 * S::VSTR + d * 4);
        const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
        oacc[db] = E::mfma32(a, pk[c], oacc[db]);
      }
    }
  };

  if (t_begin < t_end) {
    gload(t_begin);
    lstore(0);
  }
  if (t_begin + 1 < t_end) gload(t_begin + 1);
  for (int t = t_begin; t < t_end; ++t) {
    const int buf = (t - t_begin) & 1;
    __syncthreads();
    if (t + 1 < t_end) lstore(buf ^ 1);
    if (t + 2 < t_end) gload(t + 2);
    compute(buf, t);
  }

  const float l_tot = l_run + wave_xor32(l_run);
  if (wave_live && qrow < p.Sq) {
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    uint16_t* orow = p.o + b * p.o_sb + h * p.o_sh + static_cast<int64_t>(qrow) * p.o_ss;
#pragma unroll
    for (int db = 0; db < S::DB; ++db) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d0 = 32 * db + 8 * i + 4 * g;
        const uint32_t w0 = E::pack2(oacc[db][4 * i + 0] * inv, oacc[db][4 * i + 1] * inv);
        const uint32_t w1 = E::pack2(oacc[db][4 * i + 2] * inv, oacc[db][4 * i + 3] * inv);
        if (vec && d0 + 4 <= D) {
          *reinterpret_cast<u32x2*>(orow + d0) = u32x2{w0, w1};
        } else {
          const uint16_t hv[4] = {static_cast<uint16_t>(w0 & 0xffffu),
                                  static_cast<uint16_t>(w0 >> 16),
                                  static_cast<uint16_t>(w1 & 0xffffu),
                                  static_cast<uint16_t>(w1 >> 16)};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (d0 + j < D) orow[d0 + j] = hv[j];
          }
        }
      }
    }
    if (p.lse != nullptr && g == 0) {
      const float lse = l_tot > 0.0f ? (m_run + fast_log2(l_tot)) * kLn2 : masked_row_lse(p, qrow);
      p.lse[b * p.l_sb + h * p.l_sh + static_cast<int64_t>(qrow) * p.l_ss] = lse;
    }
  }
}

template <typename Tag, int DP, int BN>
void launch_dp(const PrefillParams& p, bool softcap, int grid, hipStream_t s) {
  if (softcap) {
    hipLaunchKernelGGL((prefill_kernel<Tag, DP, BN, true>), dim3(grid), dim3(kThreads), 0, s, p);
  } else {
    hipLaunchKernelGGL((prefill_kernel<Tag, DP, BN, false>), dim3(grid), dim3(kThreads), 0, s, p);
  }
}

template <typename Tag>
void launch_tag(const PrefillParams& p, bool softcap, int grid, hipStream_t s) {
  if (p.D <= 32) {
    launch_dp<Tag, 32, 64>(p, softcap, grid, s);
  } else if (p.D <= 64) {
    launch_dp<Tag, 64, 64>(p, softcap, grid, s);
  } else if (p.D <= 128) {
    launch_dp<Tag, 128, 64>(p, softcap, grid, s);
  } else if (p.D <= 192) {
    launch_dp<Tag, 192, 32>(p, softcap, grid, s);
  } else {
    launch_dp<Tag, 256, 32>(p, softcap, grid, s);
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

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
  p.q_offset = a.q_offset;
  p.causal = a.causal ? 1 : 0;
  p.window = a.window > 0 ? a.window : 0;
  p.ratio = a.heads_q / a.heads_kv;
  p.n_qt = (a.seqlen_q + kBlockM - 1) / kBlockM;
  const bool softcap = a.softcap > 0.0f;
  if (softcap) {
    p.score_mul = a.scale / a.softcap;
    p.cap_mul = a.softcap * kLog2e;
  } else {
    p.score_mul = a.scale * kLog2e;
    p.cap_mul = 0.0f;
  }
  p.ref_bq = a.ref_block_q > 0 ? a.ref_block_q : 64;
  p.ref_bkv = a.ref_block_kv > 0 ? a.ref_block_kv : 64;
  p.masked_lse_mode = a.masked_lse_mode;

  bool vec = (a.head_dim % 8) == 0 && aligned16(a.q) && aligned16(a.k) && aligned16(a.v) &&
             aligned16(a.o);
  const int64_t* strides[4] = {a.q_stride, a.k_stride, a.v_stride, a.o_stride};
  for (int t = 0; t < 4 && vec; ++t) {
    for (int i = 0; i < 3; ++i) {
      if (strides[t][i] % 8 != 0) vec = false;
    }
  }
  p.vec = vec ? 1 : 0;

  const int64_t grid64 = static_cast<int64_t>(p.n_qt) * a.batch * a.heads_q;
  if (grid64 <= 0) return FFA_OK;
  if (grid64 > 0x7fffffff) return FFA_ERR_TOO_LARGE;
  const int grid = static_cast<int>(grid64);
  p.xcd_remap = (grid % 8 == 0) ? 1 : 0;

  if (a.dtype == FFA_DTYPE_BF16) {
    launch_tag<Bf16Tag>(p, softcap, grid, stream);
  } else {
    launch_tag<F16Tag>(p, softcap, grid, stream);
  }
  return hipGetLastError() == hipSuccess ? FFA_OK : FFA_ERR_LAUNCH;
}

}  // namespace ffa
