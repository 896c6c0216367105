// Shared device and host helpers of the gfx950 truncated-Taylor kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/polytaylor.h"

namespace pt {

constexpr int kMaxDegree = PT_MAX_DEGREE;
constexpr int kMaxOrders = kMaxDegree + 1;
constexpr int kMaxElementwiseOrders = PT_MAX_ELEMENTWISE_DEGREE + 1;
constexpr int kWave = 64;

// bfloat16 storage is raw 16-bit words.
struct bf16 {
  uint16_t bits;
};

// K+1 coefficient pointers passed to a kernel by value (N slots: kMaxOrders for the MFMA and
// row kernels, kMaxElementwiseOrders for the elementwise ones).
template <typename T, int N = kMaxOrders>
struct CPtrs {
  const T* p[N];
};
template <typename T, int N = kMaxOrders>
struct MPtrs {
  T* p[N];
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
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float floatx2_t __attribute__((ext_vector_type(2)));

// Two floats to two bfloat16 in one 32-bit word (a in the low half) with
// gfx950's v_cvt_pk_bf16_f32: round to nearest even, NaN stays NaN.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const floatx2_t f = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

template <>
__device__ __forceinline__ bf16 from_acc<bf16>(float x) {
  bf16 r;
  r.bits = static_cast<uint16_t>(pack_bf16x2(x, 0.0f));
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

// Streaming (non-temporal) 16-byte accesses, for data touched exactly once.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
template <typename T, int V>
__device__ __forceinline__ Vec<T, V> load_vec_nt(const T* p) {
  static_assert(sizeof(Vec<T, V>) == 16, "16-byte vectors only");
  return __builtin_bit_cast(Vec<T, V>, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)));
}
template <typename T, int V>
__device__ __forceinline__ void store_vec_nt(T* p, const Vec<T, V>& v) {
  static_assert(sizeof(Vec<T, V>) == 16, "16-byte vectors only");
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v), reinterpret_cast<u32x4_t*>(p));
}

// Storage vector <-> arithmetic values. bfloat16 pairs are unpacked from
// 32-bit words with one shift or mask each and packed with one conversion
// instruction per pair.
template <typename T, int V>
__device__ __forceinline__ void unpack_vec(const Vec<T, V>& v, typename AccOf<T>::type (&f)[V]) {
#pragma unroll
  for (int e = 0; e < V; ++e) f[e] = to_acc(v.v[e]);
}
template <int V>
__device__ __forceinline__ void unpack_vec(const Vec<bf16, V>& v, float (&f)[V]) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(&v);
#pragma unroll
  for (int i = 0; i < V / 2; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

// Element e of a storage vector in the arithmetic type, and a pair (e, e+1)
// written back (one conversion instruction per bfloat16 pair).
template <typename T, int V>
__device__ __forceinline__ typename AccOf<T>::type vec_get(const Vec<T, V>& v, int e) {
  return to_acc(v.v[e]);
}
template <int V>
__device__ __forceinline__ float vec_get(const Vec<bf16, V>& v, int e) {
  const uint32_t w = reinterpret_cast<const uint32_t*>(&v)[e / 2];
  return __uint_as_float((e % 2 == 0) ? (w << 16) : (w & 0xffff0000u));
}
template <typename T, int V>
__device__ __forceinline__ void vec_put2(Vec<T, V>& v, int e, typename AccOf<T>::type a,
                                         typename AccOf<T>::type b) {
  v.v[e] = from_acc<T>(a);
  v.v[e + 1] = from_acc<T>(b);
}
template <int V>
__device__ __forceinline__ void vec_put2(Vec<bf16, V>& v, int e, float a, float b) {
  reinterpret_cast<uint32_t*>(&v)[e / 2] = pack_bf16x2(a, b);
}

template <typename T, int V>
__device__ __forceinline__ void pack_vec(const typename AccOf<T>::type (&f)[V], Vec<T, V>& v) {
#pragma unroll
  for (int e = 0; e < V; ++e) v.v[e] = from_acc<T>(f[e]);
}
template <int V>
__device__ __forceinline__ void pack_vec(const float (&f)[V], Vec<bf16, V>& v) {
  uint32_t* w = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
  for (int i = 0; i < V / 2; ++i) w[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
}

// ---- wave and block reductions (fixed order: deterministic) ---------------
template <typename A>
__device__ __forceinline__ A wave_sum(A x) {
#pragma unroll
  for (int off = kWave / 2; off >= 1; off >>= 1) x += __shfl_xor(x, off, kWave);
  return x;
}

// float: DPP moves within each row of 16 lanes (quad swaps, half-row and row
// mirrors), then two lane exchanges across rows. Each step adds a lane's
// value to its partner's, so every lane ends with the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum(float x) {
  x += dpp_mov<0xB1>(x);    // quad_perm [1,0,3,2]
  x += dpp_mov<0x4E>(x);    // quad_perm [2,3,0,1]
  x += dpp_mov<0x141>(x);   // row_half_mirror
  x += dpp_mov<0x140>(x);   // row_mirror
  x += __shfl_xor(x, 16, kWave);
  x += __shfl_xor(x, 32, kWave);
  return x;
}

// Max and sum over the four 16-lane rows of a wave, for each lane position within a row: the
// exchanges of __shfl_xor by 16 and by 32 without their LDS round trips. v_permlane16_swap(x, x)
// yields rows (x0, x0, x2, x2) and (x1, x1, x3, x3), v_permlane32_swap(y, y) halves (lo, lo) and
// (hi, hi) (both checked on gfx950 with a lane-layout probe). Every lane ends with the same bits,
// those of the __shfl_xor form. Other types take that form.
template <typename A>
__device__ __forceinline__ A rows_max(A x) {
  if constexpr (sizeof(A) == 4) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
  } else {
    x = fmax(x, __shfl_xor(x, 16, kWave));
    return fmax(x, __shfl_xor(x, 32, kWave));
  }
}
template <typename A>
__device__ __forceinline__ A rows_sum(A x) {
  if constexpr (sizeof(A) == 4) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
  } else {
    x += __shfl_xor(x, 16, kWave);
    return x + __shfl_xor(x, 32, kWave);
  }
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
