// Complex directions over a real base, carried through the real kernels.
//
// A series with complex higher coefficients is evaluated as real-direction
// variants: variant v of order o is alpha_v Re(c_o) + beta_v Im(c_o) (the real
// nodes lam_v of a Lagrange evaluation at i use (1, lam_v); a real/imaginary
// split of a bilinear operation uses (1, 0) and (0, 1)). The results are
// recombined as c_o = sum_v (wre_v + i wim_v) y_{v,o}. Both passes are
// streaming, one read and one write per value (HBM-bound), replacing strided
// elementwise passes over complex views. The reference defines complex
// directions as the multilinear extension of the real derivatives
// (/root/reference/docs/notes.md:59-76) and splits linear operations on complex
// coefficients into real and imaginary parts
// (/root/reference/src/polytensors/_dispatch.py:12-26).
#include "pt_common.h"

namespace pt {

// K+1 real nodes and orders 1..K at most, up to the elementwise kernels' degree (the kernel
// arguments then hold 17 x 16 destination pointers, 2.2 KB)
constexpr int kMaxPlaneVariants = kMaxElementwiseOrders;
constexpr int kMaxComplexOrders = PT_MAX_ELEMENTWISE_DEGREE;

template <typename T>
struct ToRealArgs {
  const T* src[kMaxComplexOrders];   // interleaved (re, im) planes
  T* dst[kMaxPlaneVariants * kMaxComplexOrders];
  T alpha[kMaxPlaneVariants], beta[kMaxPlaneVariants];
};

template <typename T>
struct ToComplexArgs {
  const T* src[kMaxPlaneVariants * kMaxComplexOrders];
  T* dst[kMaxComplexOrders];   // interleaved (re, im) planes
  T wre[kMaxPlaneVariants], wim[kMaxPlaneVariants];
};

// Values per thread and step: one 16-byte store per real plane.
template <typename T>
struct PlaneVec {
  static constexpr int value = 16 / sizeof(T);
};

// VEC: every plane 16-byte aligned (16-byte accesses); otherwise one value per step.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void complex_to_real_kernel(ToRealArgs<T> a, int orders, int variants,
                                                              int64_t numel) {
  constexpr int E = VEC ? PlaneVec<T>::value : 1;
  const int64_t groups = numel / E;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; g < groups; g += stride) {
    for (int o = 0; o < orders; ++o) {
      T re[E], im[E];
      if constexpr (VEC) {
        // E complex values: two 16-byte loads of interleaved (re, im)
        const Vec<T, E> c0 = load_vec_nt<T, E>(a.src[o] + 2 * E * g);
        const Vec<T, E> c1 = load_vec_nt<T, E>(a.src[o] + 2 * E * g + E);
#pragma unroll
        for (int e = 0; e < E / 2; ++e) {
          re[e] = c0.v[2 * e];
          im[e] = c0.v[2 * e + 1];
          re[E / 2 + e] = c1.v[2 * e];
          im[E / 2 + e] = c1.v[2 * e + 1];
        }
      } else {
        re[0] = a.src[o][2 * g];
        im[0] = a.src[o][2 * g + 1];
      }
      for (int v = 0; v < variants; ++v) {
        if constexpr (VEC) {
          Vec<T, E> r;
#pragma unroll
          for (int e = 0; e < E; ++e) r.v[e] = a.alpha[v] * re[e] + a.beta[v] * im[e];
          store_vec_nt<T, E>(a.dst[v * orders + o] + E * g, r);
        } else {
          a.dst[v * orders + o][g] = a.alpha[v] * re[0] + a.beta[v] * im[0];
        }
      }
    }
  }
  // tail (fewer than E values), by the first threads
  const int64_t t = groups * E + static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t < numel && t < groups * E + E) {
    for (int o = 0; o < orders; ++o)
      for (int v = 0; v < variants; ++v)
        a.dst[v * orders + o][t] = a.alpha[v] * a.src[o][2 * t] + a.beta[v] * a.src[o][2 * t + 1];
  }
}

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void real_to_complex_kernel(ToComplexArgs<T> a, int orders, int variants,
                                                              int64_t numel) {
  constexpr int E = VEC ? PlaneVec<T>::value : 1;
  const int64_t groups = numel / E;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; g < groups; g += stride) {
    for (int o = 0; o < orders; ++o) {
      T re[E], im[E];
#pragma unroll
      for (int e = 0; e < E; ++e) re[e] = im[e] = T(0);
      for (int v = 0; v < variants; ++v) {
        if constexpr (VEC) {
          const Vec<T, E> y = load_vec_nt<T, E>(a.src[v * orders + o] + E * g);
#pragma unroll
          for (int e = 0; e < E; ++e) {
            re[e] += a.wre[v] * y.v[e];
            im[e] += a.wim[v] * y.v[e];
          }
        } else {
          const T y = a.src[v * orders + o][g];
          re[0] += a.wre[v] * y;
          im[0] += a.wim[v] * y;
        }
      }
      if constexpr (VEC) {
        Vec<T, E> c0, c1;
#pragma unroll
        for (int e = 0; e < E / 2; ++e) {
          c0.v[2 * e] = re[e];
          c0.v[2 * e + 1] = im[e];
          c1.v[2 * e] = re[E / 2 + e];
          c1.v[2 * e + 1] = im[E / 2 + e];
        }
        store_vec_nt<T, E>(a.dst[o] + 2 * E * g, c0);
        store_vec_nt<T, E>(a.dst[o] + 2 * E * g + E, c1);
      } else {
        a.dst[o][2 * g] = re[0];
        a.dst[o][2 * g + 1] = im[0];
      }
    }
  }
  const int64_t t = groups * E + static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t < numel && t < groups * E + E) {
    for (int o = 0; o < orders; ++o) {
      T re = T(0), im = T(0);
      for (int v = 0; v < variants; ++v) {
        const T y = a.src[v * orders + o][t];
        re += a.wre[v] * y;
        im += a.wim[v] * y;
      }
      a.dst[o][2 * t] = re;
      a.dst[o][2 * t + 1] = im;
    }
  }
}

static unsigned plane_blocks(int64_t numel, int E) {
  const int64_t groups = (numel + E - 1) / E;
  const int64_t blocks = (groups + 255) / 256;
  return static_cast<unsigned>(blocks < 256 * 16 ? (blocks > 0 ? blocks : 1) : 256 * 16);
}

template <typename T>
static int launch_to_real(int orders, const void* const* src, int variants, const double* alpha, const double* beta,
                          void* const* dst, int64_t numel, hipStream_t stream) {
  ToRealArgs<T> a{};
  for (int o = 0; o < orders; ++o) a.src[o] = static_cast<const T*>(src[o]);
  for (int i = 0; i < orders * variants; ++i) a.dst[i] = static_cast<T*>(dst[i]);
  for (int v = 0; v < variants; ++v) {
    a.alpha[v] = static_cast<T>(alpha[v]);
    a.beta[v] = static_cast<T>(beta[v]);
  }
  bool vec = true;
  for (int o = 0; o < orders; ++o) vec = vec && pt_host::aligned16(src[o]);
  for (int i = 0; i < orders * variants; ++i) vec = vec && pt_host::aligned16(dst[i]);
  if (vec)
    complex_to_real_kernel<T, true><<<plane_blocks(numel, PlaneVec<T>::value), 256, 0, stream>>>(
        a, orders, variants, numel);
  else
    complex_to_real_kernel<T, false><<<plane_blocks(numel, 1), 256, 0, stream>>>(a, orders, variants, numel);
  PT_LAUNCH_CHECK();
  return PT_OK;
}

template <typename T>
static int launch_to_complex(int orders, int variants, const void* const* src, const double* wre, const double* wim,
                             void* const* dst, int64_t numel, hipStream_t stream) {
  ToComplexArgs<T> a{};
  for (int i = 0; i < orders * variants; ++i) a.src[i] = static_cast<const T*>(src[i]);
  for (int o = 0; o < orders; ++o) a.dst[o] = static_cast<T*>(dst[o]);
  for (int v = 0; v < variants; ++v) {
    a.wre[v] = static_cast<T>(wre[v]);
    a.wim[v] = static_cast<T>(wim[v]);
  }
  bool vec = true;
  for (int i = 0; i < orders * variants; ++i) vec = vec && pt_host::aligned16(src[i]);
  for (int o = 0; o < orders; ++o) vec = vec && pt_host::aligned16(dst[o]);
  if (vec)
    real_to_complex_kernel<T, true><<<plane_blocks(numel, PlaneVec<T>::value), 256, 0, stream>>>(
        a, orders, variants, numel);
  else
    real_to_complex_kernel<T, false><<<plane_blocks(numel, 1), 256, 0, stream>>>(a, orders, variants, numel);
  PT_LAUNCH_CHECK();
  return PT_OK;
}

}  // namespace pt

namespace {

int check_planes(int dtype, int orders, int variants, const void* const* a, const void* const* b,
                 const double* p, const double* q, int64_t numel) {
  PT_REQUIRE(dtype == PT_FLOAT32 || dtype == PT_FLOAT64, PT_UNSUPPORTED,
             "complex planes: float32 (complex64) or float64 (complex128) only");
  PT_REQUIRE(orders >= 0 && orders <= pt::kMaxComplexOrders && variants >= 1 && variants <= pt::kMaxPlaneVariants,
             PT_INVALID_ARGUMENT, "complex planes: 0..16 complex orders and 1..17 variants");
  PT_REQUIRE(numel >= 0, PT_INVALID_ARGUMENT, "complex planes: numel must be >= 0");
  PT_REQUIRE(p != nullptr && q != nullptr, PT_INVALID_ARGUMENT, "complex planes: coefficient arrays are required");
  if (numel == 0 || orders == 0) return PT_OK;
  PT_REQUIRE(a != nullptr && b != nullptr, PT_INVALID_ARGUMENT, "complex planes: pointer arrays are required");
  return -1;
}

}  // namespace

extern "C" {

int pt_complex_to_real(int dtype, int orders, const void* const* src, int variants, const double* alpha,
                       const double* beta, void* const* dst, int64_t numel, void* stream) {
  pt_host::clear_error();
  const int early = check_planes(dtype, orders, variants, src, dst, alpha, beta, numel);
  if (early >= 0) return early;
  for (int o = 0; o < orders; ++o)
    PT_REQUIRE(src[o] != nullptr, PT_INVALID_ARGUMENT, "complex planes: null source plane");
  for (int i = 0; i < orders * variants; ++i)
    PT_REQUIRE(dst[i] != nullptr, PT_INVALID_ARGUMENT, "complex planes: null destination plane");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == PT_FLOAT32 ? pt::launch_to_real<float>(orders, src, variants, alpha, beta, dst, numel, s)
                             : pt::launch_to_real<double>(orders, src, variants, alpha, beta, dst, numel, s);
}

int pt_real_to_complex(int dtype, int orders, int variants, const void* const* src, const double* wre,
                       const double* wim, void* const* dst, int64_t numel, void* stream) {
  pt_host::clear_error();
  const int early = check_planes(dtype, orders, variants, src, dst, wre, wim, numel);
  if (early >= 0) return early;
  for (int i = 0; i < orders * variants; ++i)
    PT_REQUIRE(src[i] != nullptr, PT_INVALID_ARGUMENT, "complex planes: null source plane");
  for (int o = 0; o < orders; ++o)
    PT_REQUIRE(dst[o] != nullptr, PT_INVALID_ARGUMENT, "complex planes: null destination plane");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == PT_FLOAT32 ? pt::launch_to_complex<float>(orders, variants, src, wre, wim, dst, numel, s)
                             : pt::launch_to_complex<double>(orders, variants, src, wre, wim, dst, numel, s);
}

}  // extern "C"
