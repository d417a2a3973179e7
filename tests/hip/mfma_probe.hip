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
