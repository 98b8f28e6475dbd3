// Test helper: one wave runs a chain of v_mfma_f32_32x32x16_{bf16,f16} on given
// operands so a test can compare the fp32 accumulation with exact sums.
// Operand layout: a[s][m][k] (32x16), b[s][k][n] (16x32), 16-bit patterns.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <bool F16>
__global__ void mfma_chain(const uint16_t* a, const uint16_t* b, const float* acc0, float* c,
                           int steps) {
  const int l = threadIdx.x, l32 = l & 31, h = l >> 5;
  f32x16 acc;
  for (int e = 0; e < 16; ++e) acc[e] = acc0[(8 * (e / 4) + 4 * h + (e % 4)) * 32 + l32];
  for (int s = 0; s < steps; ++s) {
    uint16_t av[8], bv[8];
    for (int t = 0; t < 8; ++t) {
      av[t] = a[(s * 32 + l32) * 16 + 8 * h + t];
      bv[t] = b[(s * 16 + 8 * h + t) * 32 + l32];
    }
    const uint4 ra = *reinterpret_cast<uint4*>(av), rb = *reinterpret_cast<uint4*>(bv);
    if constexpr (F16)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, ra),
                                                  __builtin_bit_cast(f16x8, rb), acc, 0, 0, 0);
    else
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ra),
                                                   __builtin_bit_cast(bf16x8, rb), acc, 0, 0, 0);
  }
  for (int e = 0; e < 16; ++e) c[(8 * (e / 4) + 4 * h + (e % 4)) * 32 + l32] = acc[e];
}

extern "C" int mfma_chain_run(int f16, const void* a, const void* b, const void* acc0, void* c,
                              int steps) {
  if (steps < 1 || steps > 64) return -1;
  if (f16)
    hipLaunchKernelGGL(mfma_chain<true>, dim3(1), dim3(64), 0, 0, (const uint16_t*)a,
                       (const uint16_t*)b, (const float*)acc0, (float*)c, steps);
  else
    hipLaunchKernelGGL(mfma_chain<false>, dim3(1), dim3(64), 0, 0, (const uint16_t*)a,
                       (const uint16_t*)b, (const float*)acc0, (float*)c, steps);
  if (hipGetLastError() != hipSuccess) return -2;
  return hipDeviceSynchronize() == hipSuccess ? 0 : -3;
}
