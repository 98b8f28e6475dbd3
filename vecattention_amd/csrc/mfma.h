// bf16 / fp16 32x32x16 MFMA helpers shared by the selection and attention kernels.
#pragma once
#include "common.h"

namespace va {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <typename T> struct Mfma;
template <> struct Mfma<bf16_t> {
  typedef bf16x8_t vec;
  __device__ static f32x16_t run(vec a, vec b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static vec pack(const float* x) {
    vec r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = __bf16(x[e]);
    return r;
  }
  // acc + x[2i] + x[2i+1] (v_dot2c_f32_bf16 against (1, 1)).
  __device__ static float add_pair(vec x, int i, float acc) {
    typedef __bf16 pair __attribute__((ext_vector_type(2)));
    const pair one = {__bf16(1.f), __bf16(1.f)};
    return __builtin_amdgcn_fdot2_f32_bf16(pair{x[2 * i], x[2 * i + 1]}, one, acc, false);
  }
};
template <> struct Mfma<f16_t> {
  typedef f16x8_t vec;
  __device__ static f32x16_t run(vec a, vec b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static vec pack(const float* x) {
    vec r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = _Float16(x[e]);
    return r;
  }
  // acc + x[2i] + x[2i+1] (v_dot2c_f32_f16 against (1, 1)).
  __device__ static float add_pair(vec x, int i, float acc) {
    typedef _Float16 pair __attribute__((ext_vector_type(2)));
    const pair one = {_Float16(1.f), _Float16(1.f)};
    return __builtin_amdgcn_fdot2(pair{x[2 * i], x[2 * i + 1]}, one, acc, false);
  }
};

}  // namespace va
