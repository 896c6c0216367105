// Elementwise product and quotient of two degree-K series, one streaming pass.
//
//   mul: y_k = sum_{i+j=k} a_i b_j           (the Cauchy rule of
//        /root/reference/src/polytensors/_range_ops.py:143-144 with _plain.py:118-128)
//   div: y_k = (a_k - sum_{i=1..k} b_i y_{k-i}) / b_0
//        (quotient, /root/reference/src/polytensors/_range_ops.py:86-93)
// Each thread streams one 16-byte vector of every order of both operands per
// step with non-temporal accesses; arithmetic float32 (float64 for float64).
#pragma once

#include <algorithm>

#include "series_binary.h"

namespace pt {

constexpr int kBinaryThreads = 256;

template <typename A, int K>
__device__ __forceinline__ void binary_element(int op, const A (&a)[K + 1], const A (&b)[K + 1],
                                               A (&y)[K + 1]) {
  if (op == PT_BINARY_MUL) {
#pragma unroll
    for (int k = K; k >= 0; --k) {
      A s = a[0] * b[k];
#pragma unroll
      for (int i = 1; i <= k; ++i) s = fma(a[i], b[k - i], s);
      y[k] = s;
    }
  } else {
    const A inv0 = A(1) / b[0];
#pragma unroll
    for (int k = 0; k <= K; ++k) {
      A r = a[k];
#pragma unroll
      for (int i = 1; i <= k; ++i) r = fma(-b[i], y[k - i], r);
      y[k] = r * inv0;
    }
  }
}

template <typename T, int K>
__global__ __launch_bounds__(kBinaryThreads) void series_binary_kernel(int op, CPtrs<T, kMaxElementwiseOrders> a,
                                                                       CPtrs<T, kMaxElementwiseOrders> b,
                                                                       MPtrs<T, kMaxElementwiseOrders> y,
                                                                       int64_t numel, bool vec) {
  using A = typename AccOf<T>::type;
  constexpr int V = VecWidth<T>::value;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBinaryThreads;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kBinaryThreads + threadIdx.x;
  int64_t scalar_from = 0;
  if (vec) {
    const int64_t nvec = numel / V;
    for (int64_t i = first; i < nvec; i += stride) {
      Vec<T, V> ra[K + 1], rb[K + 1];
#pragma unroll
      for (int k = 0; k <= K; ++k) {
        ra[k] = load_vec_nt<T, V>(a.p[k] + i * V);
        rb[k] = load_vec_nt<T, V>(b.p[k] + i * V);
      }
      A fa[K + 1][V], fb[K + 1][V];
#pragma unroll
      for (int k = 0; k <= K; ++k) {
        unpack_vec(ra[k], fa[k]);
        unpack_vec(rb[k], fb[k]);
      }
#pragma unroll
      for (int e = 0; e < V; ++e) {
        A u[K + 1], w[K + 1], out[K + 1];
#pragma unroll
        for (int k = 0; k <= K; ++k) {
          u[k] = fa[k][e];
          w[k] = fb[k][e];
        }
        binary_element<A, K>(op, u, w, out);
#pragma unroll
        for (int k = 0; k <= K; ++k) fa[k][e] = out[k];
      }
#pragma unroll
      for (int k = 0; k <= K; ++k) {
        pack_vec(fa[k], ra[k]);
        store_vec_nt<T, V>(y.p[k] + i * V, ra[k]);
      }
    }
    scalar_from = nvec * V;
  }
  for (int64_t i = scalar_from + first; i < numel; i += stride) {
    A u[K + 1], w[K + 1], out[K + 1];
#pragma unroll
    for (int k = 0; k <= K; ++k) {
      u[k] = to_acc(a.p[k][i]);
      w[k] = to_acc(b.p[k][i]);
    }
    binary_element<A, K>(op, u, w, out);
#pragma unroll
    for (int k = 0; k <= K; ++k) y.p[k][i] = from_acc<T>(out[k]);
  }
}

template <typename T, int K>
static int launch_binary_k(const BinaryArgs& a) {
  constexpr int V = VecWidth<T>::value;
  CPtrs<T, kMaxElementwiseOrders> pa{}, pb{};
  MPtrs<T, kMaxElementwiseOrders> py{};
  // 16-byte vectors of every order of both operands in registers up to 72 values each; above
  // that (16-bit types past degree 8) the element-by-element path
  bool vec = (K + 1) * V <= 72;
  for (int k = 0; k <= K; ++k) {
    pa.p[k] = static_cast<const T*>(a.a[k]);
    pb.p[k] = static_cast<const T*>(a.b[k]);
    py.p[k] = static_cast<T*>(a.y[k]);
    vec = vec && pt_host::aligned16(a.a[k]) && pt_host::aligned16(a.b[k]) && pt_host::aligned16(a.y[k]);
  }
  const int64_t work = vec ? (a.numel / V + a.numel % V) : a.numel;
  const int64_t blocks =
      std::max<int64_t>(1, std::min<int64_t>((work + kBinaryThreads - 1) / kBinaryThreads, 256 * 32));
  series_binary_kernel<T, K><<<dim3(blocks), dim3(kBinaryThreads), 0, a.stream>>>(a.op, pa, pb, py, a.numel, vec);
  PT_LAUNCH_CHECK();
  return PT_OK;
}

template <typename T>
int launch_binary(const BinaryArgs& a) {
  switch (a.degree) {
    case 0: return launch_binary_k<T, 0>(a);
    case 1: return launch_binary_k<T, 1>(a);
    case 2: return launch_binary_k<T, 2>(a);
    case 3: return launch_binary_k<T, 3>(a);
    case 4: return launch_binary_k<T, 4>(a);
    case 5: return launch_binary_k<T, 5>(a);
    case 6: return launch_binary_k<T, 6>(a);
    case 7: return launch_binary_k<T, 7>(a);
    case 8: return launch_binary_k<T, 8>(a);
    case 9: return launch_binary_k<T, 9>(a);
    case 10: return launch_binary_k<T, 10>(a);
    case 11: return launch_binary_k<T, 11>(a);
    case 12: return launch_binary_k<T, 12>(a);
    case 13: return launch_binary_k<T, 13>(a);
    case 14: return launch_binary_k<T, 14>(a);
    case 15: return launch_binary_k<T, 15>(a);
    case 16: return launch_binary_k<T, 16>(a);
    default: break;
  }
  pt_host::set_error("series product: degree outside 0..PT_MAX_ELEMENTWISE_DEGREE");
  return PT_UNSUPPORTED;
}

}  // namespace pt
