// Device-side check of the MFMA operand/accumulator layouts the kernels rely on.
// One wave runs one MFMA on operands loaded with the assumed lane layout and writes
// every lane's accumulator registers out; the test compares them against A @ B.
//   32x32x16: A lane l = A[l%32][8(l/32)..+7], B lane l = B[8(l/32)..+7][l%32],
//             acc[4i+j] = C[8i+4(l/32)+j][l%32]
//   16x16x32: A lane l = A[l%16][8(l/16)..+7], B lane l = B[8(l/16)..+7][l%16],
//             acc[j]    = C[4(l/16)+j][l%16]
// All indexes stay inside the 32x16 / 16x32 / 64x16 buffers the launchers document.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ffa_common.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

__global__ void probe32(const uint16_t* A, const uint16_t* B, float* out) {
  const int l = threadIdx.x;
  u16x8 a, b;
  for (int e = 0; e < 8; ++e) {
    a[e] = A[(l % 32) * 16 + 8 * (l / 32) + e];   // A: [32][16]
    b[e] = B[(8 * (l / 32) + e) * 32 + (l % 32)]; // B: [16][32]
  }
  f32x16 acc = {};
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
  for (int r = 0; r < 16; ++r) out[l * 16 + r] = acc[r];  // out: [64][16]
}

__global__ void probe16(const uint16_t* A, const uint16_t* B, float* out) {
  const int l = threadIdx.x;
  u16x8 a, b;
  for (int e = 0; e < 8; ++e) {
    a[e] = A[(l % 16) * 32 + 8 * (l / 16) + e];   // A: [16][32]
    b[e] = B[(8 * (l / 16) + e) * 16 + (l % 16)]; // B: [32][16]
  }
  f32x4 acc = {};
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
  for (int r = 0; r < 4; ++r) out[l * 4 + r] = acc[r];    // out: [64][4]
}

extern "C" int ffa_probe_mfma32(const void* A, const void* B, void* out) {
  hipLaunchKernelGGL(probe32, dim3(1), dim3(64), 0, 0, static_cast<const uint16_t*>(A),
                     static_cast<const uint16_t*>(B), static_cast<float*>(out));
  return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}

extern "C" int ffa_probe_mfma16(const void* A, const void* B, void* out) {
  hipLaunchKernelGGL(probe16, dim3(1), dim3(64), 0, 0, static_cast<const uint16_t*>(A),
                     static_cast<const uint16_t*>(B), static_cast<float*>(out));
  return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}

// ds_read_b64_tr_b16: LDS holds elements 0..1023 (value = index). Lane l reads
// 64 bits at element address addr(l); out[l][0..3] are the element indices returned.
//   mode 0: addr(l) = 4 l                      (64 rows x 4 elements, row-major)
//   mode 1: addr(l) = 64 (l % 16) + 4 (l / 16) (16 rows of 64 elements per group)
// Every address stays inside the 1024-element LDS array.
typedef short s16x4 __attribute__((ext_vector_type(4)));
__global__ void probe_tr16(int mode, short* out) {
  __shared__ __attribute__((aligned(16))) short lds[1024];
  const int l = threadIdx.x;
  for (int i = l; i < 1024; i += 64) lds[i] = static_cast<short>(i);
  __syncthreads();
  const int addr = mode == 0 ? 4 * l : 64 * (l % 16) + 4 * (l / 16);
  typedef __attribute__((address_space(3))) short lds_short;
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((lds_short*)lds + addr));
  for (int e = 0; e < 4; ++e) out[l * 4 + e] = v[e];
}

// global_load_lds_dwordx4: lane l loads the 16-byte chunk (63 - l) of a 1 KiB global
// buffer; the LDS image (1 KiB) is copied out.
__global__ void probe_load_lds(const unsigned* g, unsigned* out) {
  __shared__ __attribute__((aligned(16))) unsigned lds[256];
  const int l = threadIdx.x;
  for (int i = l; i < 256; i += 64) lds[i] = 0xdeadbeefu;
  __syncthreads();
  __builtin_amdgcn_global_load_lds(g + (63 - l) * 4,
                                   (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int i = l; i < 256; i += 64) out[i] = lds[i];
}

extern "C" int ffa_probe_tr16(int mode, void* out) {
  hipLaunchKernelGGL(probe_tr16, dim3(1), dim3(64), 0, 0, mode, static_cast<short*>(out));
  return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}

extern "C" int ffa_probe_load_lds(const void* g, void* out) {
  hipLaunchKernelGGL(probe_load_lds, dim3(1), dim3(64), 0, 0, static_cast<const unsigned*>(g),
                     static_cast<unsigned*>(out));
  return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}

// Lane-pair reductions of the kernels (ffa::wave_pair_max / wave_pair_sum over lanes
// l and l ^ 32): one wave, 64 inputs, 64 + 64 outputs.
__global__ void probe_pair(const float* x, float* out) {
  const int l = threadIdx.x;
  out[l] = ffa::wave_pair_max(x[l]);
  out[64 + l] = ffa::wave_pair_sum(x[l]);
}

extern "C" int ffa_probe_pair(const void* x, void* out) {
  hipLaunchKernelGGL(probe_pair, dim3(1), dim3(64), 0, 0, static_cast<const float*>(x),
                     static_cast<float*>(out));
  return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}

// v_mfma_f32_16x16x16bf16_1k: A lane l = A[l%16][4(l/16)..+3], B lane l =
// B[4(l/16)..+3][l%16], acc[j] = C[4(l/16)+j][l%16] (A, B 16x16, out 64x4).
__global__ void probe16k16(const uint16_t* A, const uint16_t* B, float* out) {
  const int l = threadIdx.x;
  ffa::u32x2 a, b;
  uint16_t av[4], bv[4];
  for (int e = 0; e < 4; ++e) {
    av[e] = A[(l % 16) * 16 + 4 * (l / 16) + e];
    bv[e] = B[(4 * (l / 16) + e) * 16 + l % 16];
  }
  a[0] = av[0] | (uint32_t(av[1]) << 16);
  a[1] = av[2] | (uint32_t(av[3]) << 16);
  b[0] = bv[0] | (uint32_t(bv[1]) << 16);
  b[1] = bv[2] | (uint32_t(bv[3]) << 16);
  ffa::f32x4 c = {0.f, 0.f, 0.f, 0.f};
  c = ffa::Elem<ffa::Bf16Tag>::mfma16k16(a, b, c);
  for (int j = 0; j < 4; ++j) out[l * 4 + j] = c[j];
}

extern "C" int ffa_probe_mfma16k16(const void* A, const void* B, void* out) {
  hipLaunchKernelGGL(probe16k16, dim3(1), dim3(64), 0, 0, static_cast<const uint16_t*>(A),
                     static_cast<const uint16_t*>(B), static_cast<float*>(out));
  return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}

// v_mfma_f32_32x32x2_f32: A lane l = A[l%32][l/32], B lane l = B[l/32][l%32],
// acc[4i+j] = C[8i+4(l/32)+j][l%32] (A 32x2, B 2x32 fp32, out 64x16).
__global__ void probe32f32(const float* A, const float* B, float* out) {
  const int l = threadIdx.x;
  ffa::f32x16 c;
  for (int r = 0; r < 16; ++r) c[r] = 0.0f;
  c = __builtin_amdgcn_mfma_f32_32x32x2f32(A[(l % 32) * 2 + l / 32], B[(l / 32) * 32 + l % 32], c,
                                           0, 0, 0);
  for (int r = 0; r < 16; ++r) out[l * 16 + r] = c[r];
}

extern "C" int ffa_probe_mfma32f32(const void* A, const void* B, void* out) {
  hipLaunchKernelGGL(probe32f32, dim3(1), dim3(64), 0, 0, static_cast<const float*>(A),
                     static_cast<const float*>(B), static_cast<float*>(out));
  return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}
