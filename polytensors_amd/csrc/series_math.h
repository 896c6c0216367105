// Series helpers shared by the activation and cross-entropy kernels.
#pragma once

#include "pt_common.h"

namespace pt {

__device__ __forceinline__ float tanh_acc(float x) { return tanhf(x); }
__device__ __forceinline__ double tanh_acc(double x) { return tanh(x); }

// Standard normal cdf Phi(x) = 0.5 erfc(-x / sqrt 2) and density phi(x).
// float: erfc by the Chebyshev fit "erfcc" of Press, Teukolsky, Vetterling and
// Flannery, Numerical Recipes in C (2nd ed.), sec. 6.2 -- fractional error
// below 1.2e-7 for every argument -- with the hardware reciprocal and exp (a
// third of the cost of the library erfcf); double: the library erfc and exp.
__device__ __forceinline__ float normal_cdf(float x) {
  const float z = fabsf(x) * 0.70710678118654752f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
  float poly = fmaf(t, 0.17087277f, -0.82215223f);
  poly = fmaf(t, poly, 1.48851587f);
  poly = fmaf(t, poly, -1.13520398f);
  poly = fmaf(t, poly, 0.27886807f);
  poly = fmaf(t, poly, -0.18628806f);
  poly = fmaf(t, poly, 0.09678418f);
  poly = fmaf(t, poly, 0.37409196f);
  poly = fmaf(t, poly, 1.00002368f);
  poly = fmaf(t, poly, -1.26551223f);
  const float half_tail = 0.5f * t * __expf(fmaf(-z, z, poly));   // 0.5 erfc(z)
  return x >= 0.0f ? 1.0f - half_tail : half_tail;
}
__device__ __forceinline__ double normal_cdf(double x) { return 0.5 * erfc(-x * 0.70710678118654752440); }
__device__ __forceinline__ float normal_density(float x) {
  return 0.39894228040143267794f * __expf(-0.5f * x * x);
}
__device__ __forceinline__ double normal_density(double x) {
  return 0.39894228040143267794 * exp(-0.5 * x * x);
}

// c = a (*) b, truncated at K.
template <typename A, int K>
__device__ __forceinline__ void cauchy_mul(const A (&a)[K + 1], const A (&b)[K + 1], A (&c)[K + 1]) {
#pragma unroll
  for (int k = K; k >= 0; --k) {
    A s = a[0] * b[k];
#pragma unroll
    for (int i = 1; i <= k; ++i) s = fma(a[i], b[k - i], s);
    c[k] = s;
  }
}

// y and d of y' = d u' where d_k = sign * sum_{a+b=k} y_a y_b (+ y_k when
// LINEAR): tanh (d = 1 - y^2) and sigmoid (d = y - y^2). y[0], d[0] given.
template <typename A, int K, bool LINEAR>
__device__ __forceinline__ void output_ode(const A (&ju)[K + 1], A (&y)[K + 1], A (&d)[K + 1]) {
#pragma unroll
  for (int k = 1; k <= K; ++k) {
    A s = A(0);
#pragma unroll
    for (int j = 1; j <= k; ++j) s = fma(ju[j], d[k - j], s);
    y[k] = s * (A(1) / A(k));
    // d_k = (LINEAR ? y_k : 0) - 2 y_0 y_k - sum_{a=1..k-1} y_a y_{k-a}
    A q = y[k] * ((LINEAR ? A(1) : A(0)) - A(2) * y[0]);
#pragma unroll
    for (int a = 1; a < k; ++a) q = fma(-y[a], y[k - a], q);
    d[k] = q;
  }
}

template <typename A, int K>
__device__ __forceinline__ void tanh_series(const A (&u)[K + 1], const A (&ju)[K + 1], A (&y)[K + 1],
                                            A (&d)[K + 1]) {
  y[0] = tanh_acc(u[0]);
  d[0] = (A(1) - y[0]) * (A(1) + y[0]);
  output_ode<A, K, false>(ju, y, d);
}

// tanh(v) and 1 - tanh(v)^2 from e = exp(-2|v|): sign(v) (1 - e) / (1 + e) and
// 4 e / (1 + e)^2 -- absolutely accurate everywhere and relatively accurate in
// both tails; float uses the hardware exp and reciprocal.
__device__ __forceinline__ void tanh_pair(float v, float& t, float& dt) {
  const float e = __expf(-2.0f * fabsf(v));
  const float inv = __builtin_amdgcn_rcpf(1.0f + e);
  t = copysignf((1.0f - e) * inv, v);
  dt = 4.0f * e * inv * inv;
}
__device__ __forceinline__ void tanh_pair(double v, double& t, double& dt) {
  t = tanh(v);
  dt = (1.0 - t) * (1.0 + t);
}

// Softcap of a series in place: z(t) <- cap tanh(z(t) / cap), by the tanh series
// of w = z / cap (the capped logits of the reference's fused cross entropy,
// /root/reference/src/polytensors/_cross_entropy_kernels.py:7-17, at degree K).
// dt receives the series of the cap's derivative 1 - tanh(z / cap)^2.
template <typename A, int K>
__device__ __forceinline__ void softcap_series(A (&z)[K + 1], A cap, A inv_cap, A (&dt)[K + 1]) {
  A jw[K + 1], t[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) jw[k] = A(k) * (z[k] * inv_cap);
  tanh_pair(z[0] * inv_cap, t[0], dt[0]);
  output_ode<A, K, false>(jw, t, dt);
#pragma unroll
  for (int k = 0; k <= K; ++k) z[k] = cap * t[k];
}
template <typename A, int K>
__device__ __forceinline__ void softcap_series(A (&z)[K + 1], A cap, A inv_cap) {
  A dt[K + 1];
  softcap_series<A, K>(z, cap, inv_cap, dt);
}

}  // namespace pt
