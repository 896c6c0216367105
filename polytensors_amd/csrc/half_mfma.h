// 16-bit MFMA operands and LDS DMA on gfx950 (CDNA4), shared by the bfloat16 /
// float16 kernels.
#pragma once

#include "pt_common.h"
#include "mfma.h"

namespace pt {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct HalfMfma;

template <>
struct HalfMfma<bf16> {
  typedef __bf16 op_t __attribute__((ext_vector_type(8)));
  __device__ __forceinline__ static floatx4 mma(u32x4 a, u32x4 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(op_t, a), __builtin_bit_cast(op_t, b), c,
                                                   0, 0, 0);
  }
  // two values, round to nearest even, first in the low half
  __device__ __forceinline__ static uint32_t pack2(float a, float b) { return pack_bf16x2(a, b); }
  // the two values of a packed word
  __device__ __forceinline__ static float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ __forceinline__ static float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  // acc + lo(w) + hi(w) in one instruction (v_dot2c_f32_bf16 against (1, 1)): the products are
  // exact, the sum is in float32
  __device__ __forceinline__ static float sum2(uint32_t w, float acc) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, w), __builtin_bit_cast(bf2, 0x3F803F80u), acc, false);
  }
  // lazy-rescale slack (natural-log units): p <= e^8 (bf16 has the fp32 exponent range)
  static constexpr float kSlack = 8.0f;
};

template <>
struct HalfMfma<_Float16> {
  typedef _Float16 op_t __attribute__((ext_vector_type(8)));
  __device__ __forceinline__ static floatx4 mma(u32x4 a, u32x4 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(op_t, a), __builtin_bit_cast(op_t, b), c,
                                                  0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack2(float a, float b) {
    const _Float16 x = static_cast<_Float16>(a), y = static_cast<_Float16>(b);   // round to nearest even
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, x)) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, y)) << 16);
  }
  __device__ __forceinline__ static float lo(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
  }
  __device__ __forceinline__ static float hi(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
  }
  // acc + lo(w) + hi(w) in one instruction (v_dot2c_f32_f16 against (1, 1))
  __device__ __forceinline__ static float sum2(uint32_t w, float acc) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, w), __builtin_bit_cast(h2, 0x3C003C00u), acc, false);
  }
  // float16 overflows at 65504: the running maximum is exact (p <= 1)
  static constexpr float kSlack = 0.0f;
};

// ---------------------------------------------------------------------------
// LDS DMA: buffer_load_dwordx4 ... lds moves 16 bytes per lane from global memory
// into LDS, lane l's bytes landing at M0 + 16 l (so one wave instruction fills 1 KB
// of LDS, contiguous). The source is a raw buffer resource (base, stride 0,
// num_records bytes) and a 32-bit lane offset: a lane whose offset is at or past
// num_records is out of range and loads zeros, which is how the kernels pad
// ragged tiles.
//
// It is issued from inline assembly. The compiler's wait insertion treats an LDS
// DMA it knows of as a store to all of LDS and waits for it (vmcnt(0)) before
// every later LDS read, even of another buffer; hidden from it, the DMA is waited
// for where the kernel says so: s_waitcnt vmcnt(0) before the barrier that hands
// the buffer to its readers. Vector memory loads complete in issue order, so the
// compiler's own counted waits for its ordinary loads stay sufficient with these
// loads in flight (they can only wait longer).
typedef int BufferRsrc __attribute__((ext_vector_type(4)));

// Raw buffer resource over [base, base + bytes): 48-bit base, stride 0, dword 3 = 0x00020000.
__device__ __forceinline__ BufferRsrc buffer_rsrc(const void* base, int bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  return BufferRsrc{static_cast<int>(b), static_cast<int>((b >> 32) & 0xffff), bytes, 0x00020000};
}

// An offset that is out of range for every resource (loads zeros).
constexpr int kBufferOutOfRange = 0x7ffffff0;

// This wave's 64 x 16 bytes at lane offsets voff into LDS at lds (wave-uniform, 16-byte aligned).
__device__ __forceinline__ void lds_dma16(void* lds, const BufferRsrc& rsrc, int voff) {
  const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void*)lds));
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(m0), "v"(voff), "s"(rsrc)
      : "memory", "m0");
}

// Two 8-byte LDS transpose reads (ds_read_b64_tr_b16) as one 16-byte operand. Within each
// 16-lane group, lane 4a + b receives element b of the 8-byte pieces addressed by lanes a,
// a+4, a+8, a+12 (checked on gfx950 with a lane-layout probe).
typedef short Shortx4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 lds_read_tr16x2(const void* first, const void* second) {
  typedef __attribute__((address_space(3))) Shortx4 lds_x4;
  const Shortx4 f = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_x4*)(first));
  const Shortx4 s = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_x4*)(second));
  const uint2 a = __builtin_bit_cast(uint2, f), b = __builtin_bit_cast(uint2, s);
  return u32x4{a.x, a.y, b.x, b.y};
}

}  // namespace pt
