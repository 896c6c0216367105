// MFMA building blocks for gfx950 (CDNA4), 64-wide wavefronts.
//
// Each op multiplies an (M x KK) A fragment by a (KK x N) B fragment into an
// M x N accumulator held across the wave. Lane l supplies one A value
// A[l % M][l / M] and one B value B[l / M][l % N] per instruction, and holds
// ACC accumulator values; acc_row(l, r) / acc_col(l) give the output element
// of accumulator register r.
#pragma once

#include "pt_common.h"

namespace pt {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef double doublex4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma;

// v_mfma_f32_32x32x2_f32: 32x32 output, 2-deep contraction, 16 VGPRs of accumulator.
template <>
struct Mfma<float> {
  static constexpr int M = 32, N = 32, KK = 2, ACC = 16;
  using acc_t = floatx16;
  __device__ __forceinline__ static acc_t zero() {
    acc_t z;
#pragma unroll
    for (int i = 0; i < ACC; ++i) z[i] = 0.0f;
    return z;
  }
  __device__ __forceinline__ static acc_t mma(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static int acc_row(int lane, int r) {
    return 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
  }
  __device__ __forceinline__ static int acc_col(int lane) { return lane % 32; }
};

// v_mfma_f64_16x16x4_f64: 16x16 output, 4-deep contraction, 4 doubles of accumulator.
template <>
struct Mfma<double> {
  static constexpr int M = 16, N = 16, KK = 4, ACC = 4;
  using acc_t = doublex4;
  __device__ __forceinline__ static acc_t zero() {
    acc_t z;
#pragma unroll
    for (int i = 0; i < ACC; ++i) z[i] = 0.0;
    return z;
  }
  __device__ __forceinline__ static acc_t mma(double a, double b, acc_t c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
  // Unlike the fp32 16x16 layouts, register r of lane l holds row 4 r + l / 16.
  __device__ __forceinline__ static int acc_row(int lane, int r) { return 4 * r + lane / 16; }
  __device__ __forceinline__ static int acc_col(int lane) { return lane % 16; }
};

}  // namespace pt
