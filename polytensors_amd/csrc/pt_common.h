// Shared device and host helpers of the gfx950 truncated-Taylor kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/polytaylor.h"

namespace pt {

constexpr int kMaxDegree = PT_MAX_DEGREE;
constexpr int kMaxOrders = kMaxDegree + 1;
constexpr int kWave = 64;

// bfloat16 storage is raw 16-bit words.
struct bf16 {
  uint16_t bits;
};

// K+1 coefficient pointers passed to a kernel by value.
template <typename T>
struct CPtrs {
  const T* p[kMaxOrders];
};
template <typename T>
struct MPtrs {
  T* p[kMaxOrders];
};

template <typename T>
struct AccOf {
  using type = float;
};
template <>
struct AccOf<double> {
  using type = double;
};

// ---- scalar conversions to/from the arithmetic type ----------------------
__device__ __forceinline__ float to_acc(float x) { return x; }
__device__ __forceinline__ double to_acc(double x) { return x; }
__device__ __forceinline__ float to_acc(_Float16 x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_acc(bf16 x) {
  return __uint_as_float(static_cast<uint32_t>(x.bits) << 16);
}

template <typename T>
__device__ __forceinline__ T from_acc(typename AccOf<T>::type x);
template <>
__device__ __forceinline__ float from_acc<float>(float x) { return x; }
template <>
__device__ __forceinline__ double from_acc<double>(double x) { return x; }
template <>
__device__ __forceinline__ _Float16 from_acc<_Float16>(float x) {
  return static_cast<_Float16>(x);
}
template <>
__device__ __forceinline__ bf16 from_acc<bf16>(float x) {
  // Round to nearest, ties to even; NaN stays a quiet NaN.
  uint32_t u = __float_as_uint(x);
  bf16 r;
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    r.bits = static_cast<uint16_t>((u >> 16) | 0x0040u);
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
    r.bits = static_cast<uint16_t>(u >> 16);
  }
  return r;
}

// ---- 16-byte vectors of storage elements ---------------------------------
template <typename T>
struct VecWidth {
  static constexpr int value = 16 / sizeof(T);
};

template <typename T, int V>
struct alignas(sizeof(T) * V) Vec {
  T v[V];
};

template <typename T, int V>
__device__ __forceinline__ Vec<T, V> load_vec(const T* p) {
  return *reinterpret_cast<const Vec<T, V>*>(p);
}
template <typename T, int V>
__device__ __forceinline__ void store_vec(T* p, const Vec<T, V>& v) {
  *reinterpret_cast<Vec<T, V>*>(p) = v;
}

// ---- wave and block reductions (fixed order: deterministic) ---------------
template <typename A>
__device__ __forceinline__ A wave_sum(A x) {
#pragma unroll
  for (int off = kWave / 2; off >= 1; off >>= 1) x += __shfl_xor(x, off, kWave);
  return x;
}

template <typename A>
__device__ __forceinline__ A wave_max(A x) {
#pragma unroll
  for (int off = kWave / 2; off >= 1; off >>= 1) x = fmax(x, __shfl_xor(x, off, kWave));
  return x;
}

// Accurate exp/log in the arithmetic type.
__device__ __forceinline__ float exp_acc(float x) { return expf(x); }
__device__ __forceinline__ double exp_acc(double x) { return exp(x); }
__device__ __forceinline__ float log_acc(float x) { return logf(x); }
__device__ __forceinline__ double log_acc(double x) { return log(x); }
__device__ __forceinline__ float rsqrt_acc(float x) { return 1.0f / sqrtf(x); }
__device__ __forceinline__ double rsqrt_acc(double x) { return 1.0 / sqrt(x); }

}  // namespace pt

// ---- host-side error reporting --------------------------------------------
namespace pt_host {

void set_error(const std::string& message);
void clear_error();

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

}  // namespace pt_host

#define PT_REQUIRE(cond, code, msg)        \
  do {                                     \
    if (!(cond)) {                         \
      pt_host::set_error(msg);             \
      return (code);                       \
    }                                      \
  } while (0)

#define PT_LAUNCH_CHECK()                                                   \
  do {                                                                      \
    hipError_t e__ = hipGetLastError();                                     \
    if (e__ != hipSuccess) {                                                \
      pt_host::set_error(std::string("HIP launch failed: ") +               \
                         hipGetErrorString(e__));                           \
      return PT_DEVICE_ERROR;                                               \
    }                                                                       \
  } while (0)

namespace pt {
// exp on the hardware exp2 unit for float (relative error of a few ulp plus
// |x| * 2^-24 from rounding x * log2(e)); the accurate routine for double.
__device__ __forceinline__ float exp_fast(float x) { return __expf(x); }
__device__ __forceinline__ double exp_fast(double x) { return exp(x); }
}  // namespace pt
