// Shared device helpers of the gfx950 attention kernels: operand vector types,
// MFMA wrappers, 16-bit element conversion and guarded row loads.
//
// MFMA v_mfma_f32_32x32x16_{bf16,f16} operand layout (wave64, lane l, g = l / 32):
//   A [32 x 16] : lane l holds A[l % 32][8g .. 8g+7]
//   B [16 x 32] : lane l holds B[8g .. 8g+7][l % 32]
//   C [32 x 32] : lane l holds C[8i + 4g + j][l % 32] in acc[4i + j], i, j in 0..3
// (checked on the device by tests/test_gpu_mfma_layout.py).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ffa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

// Element tags: 16-bit storage types the kernels accept.
struct Bf16Tag {};
struct F16Tag {};

template <typename Tag>
struct Elem;

template <>
struct Elem<Bf16Tag> {
  // 32x32x16 MFMA on raw 16-bit patterns.
  __device__ static inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // 16x16x16 MFMA: A lane l = A[l % 16][4(l/16) .. +3], B lane l = B[4(l/16) .. +3][l % 16].
  __device__ static inline f32x4 mfma16k16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a),
                                                     __builtin_bit_cast(s16x4_t, b), c, 0, 0, 0);
  }
  // Two fp32 -> packed pair (x in the low half), round to nearest even.
  __device__ static inline uint32_t pack2(float x, float y) {
    f32x2 v = {x, y};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  }
  __device__ static inline float to_f32(uint16_t h) {
    return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
  }
};

template <>
struct Elem<F16Tag> {
  __device__ static inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static inline f32x4 mfma16k16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                 __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float x, float y) {
    f32x2 v = {x, y};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
  }
  __device__ static inline float to_f32(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
  }
};

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ inline float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// tanh(y) = sign(y) * (1 - e) / (1 + e), e = exp(-2|y|); |error| ~ 1e-7 absolute.
__device__ inline float tanh_approx(float y) {
  const float e = fast_exp2(fabsf(y) * (-2.0f * kLog2e));
  const float t = (1.0f - e) * __builtin_amdgcn_rcpf(1.0f + e);
  return __builtin_copysignf(t, y);
}

// tanh(y) = 1 - 2 / (1 + e^{2y}), given x = 2y * log2(e): exp2, add, rcp, fma. It
// saturates to -1 / +1 for large |y| (e^{2y} = 0 / inf); |error| ~ 1e-7 absolute.
__device__ inline float tanh_fast(float x) {
  return fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + fast_exp2(x)), 1.0f);
}

// Ties an MFMA accumulator to the accumulation registers (AGPRs) at this point; emits
// no instruction. Kernels that run one workgroup per CU (512 registers per lane) call it
// on their loop-carried accumulators: left alone, the register allocator keeps them in
// VGPRs and copies them into AGPRs and back around the MFMAs (hundreds of
// v_accvgpr_write / read per tile), or spills.
__device__ inline void pin_agpr(f32x16& acc) { asm volatile("" : "+a"(acc)); }

// fp32 x fp32 -> fp32 MFMA, 32x32 output, k = 2: lane (g, l) supplies A[l][g] and
// B[g][l]; accumulator element r of lane (g, l) is C[8 (r / 4) + 4 g + r % 4][l].
__device__ inline f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Keeps the compiler from moving LDS accesses across this point. One wave's LDS
// operations complete in issue order, so a wave-private tile needs no wait or barrier
// between its writes and the other lanes' reads.
__device__ inline void wave_lds_order() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

// 32 rows of a [*, D] fp32 tensor held by one wave as f32x4 chunks (chunk j of lane l:
// row (64 j + l) / (DP / 4), dims 4 x the remainder; rows past `last` re-read it, dims
// past D are zero), then stored to a wave-private LDS tile of pitch DP + 4 (rows
// 16-byte aligned; 32 rows read at one dim offset hit distinct banks).
template <int DP>
struct F32WaveTile {
  static constexpr int ROWS = 32;
  static constexpr int PITCH = DP + 4;
  static constexpr int CPR = DP / 4;
  static constexpr int NL = ROWS * CPR / 64;
  f32x4 x[NL];
  __device__ inline void load(const float* base, int64_t ss, int r0, int last, int D, int lane) {
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int idx = j * 64 + lane;
      const int r = idx / CPR;
      const int c4 = idx - r * CPR;
      x[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (4 * c4 < D) {  // D % 8 == 0: a chunk is wholly inside or outside
        x[j] = *reinterpret_cast<const f32x4*>(base + static_cast<int64_t>(min(r0 + r, last)) * ss + 4 * c4);
      }
    }
  }
  __device__ inline void store(float* t, int lane) const {
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int idx = j * 64 + lane;
      const int r = idx / CPR;
      *reinterpret_cast<f32x4*>(t + r * PITCH + 4 * (idx - r * CPR)) = x[j];
    }
  }
};

// Positions (q_offset + row, key index) are int32 inside the kernels; the C ABI keeps
// |q_offset|, q_offset + S_q and S_kv at most kMaxPos.
constexpr int kMaxPos = 0x1fffffff;

// One-sided window as the kernels use it: 0 for none, else at most q_offset + S_q + 1
// (at least 1). A longer window masks no key that a query can see (row r sees keys
// >= r - window + 1 <= 0), so the clamp changes no result, and with positions bounded
// by kMaxPos every position - window + 1 - key stays inside int32.
__host__ __device__ inline int clamp_window(int window, int q_offset, int seqlen_q) {
  if (window <= 0) return 0;
  const int64_t lim = static_cast<int64_t>(q_offset) + seqlen_q + 1;
  return static_cast<int>(window < lim ? window : (lim < 1 ? 1 : lim));
}

// Eight consecutive 16-bit elements row[d0 .. d0+7] as one 128-bit value, zero
// beyond `dlim`. `vec` promises 16-byte alignment of row + d0 whenever d0 + 8 <= dlim.
__device__ inline u32x4 load_row8(const uint16_t* __restrict__ row, int d0, int dlim, bool vec) {
  if (vec && d0 + 8 <= dlim) {
    return *reinterpret_cast<const u32x4*>(row + d0);
  }
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if (d0 + e < dlim) {
      w[e >> 1] |= static_cast<uint32_t>(row[d0 + e]) << ((e & 1) * 16);
    }
  }
  u32x4 r = {w[0], w[1], w[2], w[3]};
  return r;
}

// Interleave four key rows (8 dims each) into key-quad order: for every dim d the
// output holds keys 0..3 contiguously (8 bytes). out[2*dd + 0] = (key0, key1) of
// dim dd, out[2*dd + 1] = (key2, key3) of dim dd.
__device__ inline void quad_interleave(const u32x4& r0, const u32x4& r1, const u32x4& r2,
                                       const u32x4& r3, u32x4 out[4]) {
  uint32_t o[16];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    o[4 * w + 0] = (r0[w] & 0xffffu) | (r1[w] << 16);
    o[4 * w + 1] = (r2[w] & 0xffffu) | (r3[w] << 16);
    o[4 * w + 2] = (r0[w] >> 16) | (r1[w] & 0xffff0000u);
    o[4 * w + 3] = (r2[w] >> 16) | (r3[w] & 0xffff0000u);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[i] = u32x4{o[4 * i + 0], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
  }
}

__device__ inline float wave_xor32(float x) { return __shfl_xor(x, 32); }

// max / sum of x over the lane pair (l, l ^ 32), on the VALU: v_permlane32_swap
// exchanges the upper half of its first operand with the lower half of its second, so
// swapping x with itself yields {x[l & 31], x[(l & 31) + 32]} in every lane.
__device__ inline float wave_pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float wave_pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// gfx950 data-movement builtins, wrapped in __device__ functions (called from lambdas
// inside kernels they must not appear in host-side code).
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

// global_load_lds_dwordx4: this lane's 16 bytes at `src` land at lds_base + 16 * lane.
__device__ inline void load_lds16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)lds_base, 16, 0, 0);
}

// The same load issued from inline asm, for pipelined tile loads. The compiler does
// not see an asm load, so it neither counts it nor guards later LDS reads with
// s_waitcnt vmcnt(0): loads of a future tile stay in flight while the current tile's
// LDS is read. The caller owns completion (explicit wait_vmcnt before the barrier that
// publishes the tile) and must not overwrite LDS another wave may still be reading.
// Address = wave-uniform `base` (SGPR pair) + per-lane 32-bit byte offset `voff`;
// `lds_base` is the LDS byte address (wave-uniform), carried in M0.
__device__ inline void load_lds16_async(const void* base, uint32_t voff, uint32_t lds_base) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds_base))
               : "memory");
}

// Same, with a per-lane 64-bit address (sources that need not share a 4 GiB window).
__device__ inline void load_lds16_async(const void* src, uint32_t lds_base) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds_base))
               : "memory");
}

// LDS byte address of a pointer into a __shared__ array (low 32 bits of its flat
// address are the LDS offset).
__device__ inline uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// ds_read_b64_tr_b16: within each 16-lane group, lanes 4k..4k+3 point at 16 contiguous
// 16-bit elements of row k (4 each); lane i receives element i of rows 0..3.
__device__ inline u32x2 lds_read_tr16(const uint16_t* lds_ptr) {
  const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)lds_ptr);
  return __builtin_bit_cast(u32x2, v);
}

__device__ inline void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// s_waitcnt vmcnt(N) (gfx9 encoding: N[3:0] in bits 3:0, N[5:4] in bits 15:14).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}
__device__ inline void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

}  // namespace ffa
