// Streaming probes: the HBM rates of a plain copy and a plain read with the
// access pattern of the memory-bound series kernels (16-byte non-temporal loads
// and stores, kProbeUnroll vectors in flight per thread; a contiguous chunk per
// block or a grid-stride walk).
// They measure the practical ceiling those kernels are compared with beside the
// published 8 TB/s; they compute nothing of the series and have no counterpart
// in the reference.
#include <algorithm>

#include "pt_common.h"

namespace pt {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 4;
constexpr int kProbeDefaultBlocks = 2048;   // 8 resident waves per SIMD on 256 CUs
constexpr int kProbeMaxBlocks = 65536;

// The vectors a thread visits: CHUNKED, block b owns the contiguous chunk
// [b * chunk, (b + 1) * chunk) (as a series kernel's block owns its rows) and
// its threads step by the block width; otherwise the whole grid steps through
// the buffer together (grid-stride). Which is faster depends on the size.
template <bool CHUNKED>
struct ProbeRange {
  int64_t i, end, step;
  __device__ __forceinline__ explicit ProbeRange(int64_t n) {
    if constexpr (CHUNKED) {
      const int64_t chunk = (n + gridDim.x - 1) / gridDim.x;
      const int64_t begin = min(static_cast<int64_t>(blockIdx.x) * chunk, n);
      end = min(begin + chunk, n);
      i = begin + threadIdx.x;
      step = kProbeThreads;
    } else {
      end = n;
      i = static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
      step = static_cast<int64_t>(gridDim.x) * kProbeThreads;
    }
  }
};

template <bool CHUNKED>
__global__ __launch_bounds__(kProbeThreads) void stream_copy_kernel(const u32x4_t* __restrict__ src,
                                                                    u32x4_t* __restrict__ dst, int64_t n) {
  ProbeRange<CHUNKED> r(n);
  int64_t i = r.i;
  for (; i + (kProbeUnroll - 1) * r.step < r.end; i += kProbeUnroll * r.step) {
    u32x4_t v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * r.step);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) __builtin_nontemporal_store(v[u], dst + i + u * r.step);
  }
  for (; i < r.end; i += r.step) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// Reads every 32-bit word once; out[block] = XOR of the block's words, so the
// loads cannot be dropped and the result is checkable on the host.
template <bool CHUNKED>
__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(const u32x4_t* __restrict__ src, int64_t n,
                                                                    uint32_t* __restrict__ out) {
  __shared__ uint32_t part[kProbeThreads / kWave];
  ProbeRange<CHUNKED> r(n);
  int64_t i = r.i;
  u32x4_t acc = {0u, 0u, 0u, 0u};
  for (; i + (kProbeUnroll - 1) * r.step < r.end; i += kProbeUnroll * r.step) {
    u32x4_t v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * r.step);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u];
  }
  for (; i < r.end; i += r.step) acc ^= __builtin_nontemporal_load(src + i);
  uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
#pragma unroll
  for (int off = kWave / 2; off > 0; off /= 2) x ^= __shfl_xor(x, off);
  if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < kProbeThreads / kWave; ++w) t ^= part[w];
    out[blockIdx.x] = t;
  }
}

// Series-kernel pattern: ns source and nd destination buffers of n vectors each
// (the K+1 orders of a series and their outputs). Each thread takes one 16-byte
// vector of every source at its index, reads them all, then writes their XOR to
// every destination (or, with none, accumulates it into out[block]), as the
// elementwise series kernels take one vector of every order per thread; a block
// per 256 indices, striding past kProbeMaxSeriesBlocks blocks.
constexpr int kProbeMaxStreams = 2 * kMaxOrders;
constexpr int64_t kProbeMaxSeriesBlocks = int64_t(1) << 20;
struct ProbeStreams {
  const u32x4_t* src[kProbeMaxStreams];
  u32x4_t* dst[kMaxOrders];
};

__global__ __launch_bounds__(kProbeThreads) void stream_series_kernel(ProbeStreams p, int ns, int nd, int64_t n,
                                                                      uint32_t* __restrict__ out) {
  __shared__ uint32_t part[kProbeThreads / kWave];
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kProbeThreads;
  u32x4_t total = {0u, 0u, 0u, 0u};
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x; i < n; i += stride) {
    u32x4_t v[kProbeMaxStreams];
#pragma unroll
    for (int s = 0; s < kProbeMaxStreams; ++s)
      if (s < ns) v[s] = __builtin_nontemporal_load(p.src[s] + i);
    u32x4_t x = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int s = 0; s < kProbeMaxStreams; ++s)
      if (s < ns) x ^= v[s];
#pragma unroll
    for (int d = 0; d < kMaxOrders; ++d)
      if (d < nd) __builtin_nontemporal_store(x, p.dst[d] + i);
    total ^= x;
  }
  if (nd > 0) return;
  uint32_t x = total.x ^ total.y ^ total.z ^ total.w;
#pragma unroll
  for (int off = kWave / 2; off > 0; off /= 2) x ^= __shfl_xor(x, off);
  if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < kProbeThreads / kWave; ++w) t ^= part[w];
    out[blockIdx.x] = t;
  }
}

}  // namespace pt

namespace {

int check_probe(const void* src, int64_t bytes, int blocks, const char* what) {
  PT_REQUIRE(bytes >= 0 && bytes % 16 == 0, PT_INVALID_ARGUMENT,
             std::string(what) + ": bytes must be a non-negative multiple of 16");
  PT_REQUIRE(blocks >= 0 && blocks <= pt::kProbeMaxBlocks, PT_INVALID_ARGUMENT,
             std::string(what) + ": blocks must be 0 (default) .. 65536");
  PT_REQUIRE(bytes == 0 || (src != nullptr && pt_host::aligned16(src)), PT_INVALID_ARGUMENT,
             std::string(what) + ": source must be a 16-byte aligned device pointer");
  return -1;
}

}  // namespace

extern "C" {

int pt_stream_copy(const void* src, void* dst, int64_t bytes, int blocks, int chunked, void* stream) {
  pt_host::clear_error();
  const int early = check_probe(src, bytes, blocks, "stream copy");
  if (early >= 0) return early;
  if (bytes == 0) return PT_OK;
  PT_REQUIRE(dst != nullptr && pt_host::aligned16(dst), PT_INVALID_ARGUMENT,
             "stream copy: destination must be a 16-byte aligned device pointer");
  const unsigned grid = static_cast<unsigned>(blocks > 0 ? blocks : pt::kProbeDefaultBlocks);
  const auto* s = static_cast<const pt::u32x4_t*>(src);
  auto* d = static_cast<pt::u32x4_t*>(dst);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (chunked)
    pt::stream_copy_kernel<true><<<grid, pt::kProbeThreads, 0, st>>>(s, d, bytes / 16);
  else
    pt::stream_copy_kernel<false><<<grid, pt::kProbeThreads, 0, st>>>(s, d, bytes / 16);
  PT_LAUNCH_CHECK();
  return PT_OK;
}

int pt_stream_read(const void* src, int64_t bytes, int blocks, int chunked, void* out, void* stream) {
  pt_host::clear_error();
  const int early = check_probe(src, bytes, blocks, "stream read");
  if (early >= 0) return early;
  PT_REQUIRE(out != nullptr, PT_INVALID_ARGUMENT, "stream read: out (one uint32 per block) is required");
  const unsigned grid = static_cast<unsigned>(blocks > 0 ? blocks : pt::kProbeDefaultBlocks);
  const auto* s = static_cast<const pt::u32x4_t*>(src);
  auto* o = static_cast<uint32_t*>(out);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (chunked)
    pt::stream_read_kernel<true><<<grid, pt::kProbeThreads, 0, st>>>(s, bytes / 16, o);
  else
    pt::stream_read_kernel<false><<<grid, pt::kProbeThreads, 0, st>>>(s, bytes / 16, o);
  PT_LAUNCH_CHECK();
  return PT_OK;
}

int pt_stream_probe_blocks(void) { return pt::kProbeDefaultBlocks; }

int pt_stream_series(const void* const* src, int ns, void* const* dst, int nd, int64_t bytes_each, void* out,
                     void* stream) {
  pt_host::clear_error();
  PT_REQUIRE(ns >= 1 && ns <= pt::kProbeMaxStreams && nd >= 0 && nd <= pt::kMaxOrders, PT_INVALID_ARGUMENT,
             "stream series: 1..18 sources and 0..9 destinations");
  PT_REQUIRE(bytes_each >= 0 && bytes_each % 16 == 0, PT_INVALID_ARGUMENT,
             "stream series: bytes_each must be a non-negative multiple of 16");
  PT_REQUIRE(src != nullptr && (nd == 0 || dst != nullptr), PT_INVALID_ARGUMENT,
             "stream series: pointer arrays are required");
  PT_REQUIRE(nd > 0 || out != nullptr, PT_INVALID_ARGUMENT,
             "stream series: out (one uint32 per block) is required without destinations");
  pt::ProbeStreams p{};
  for (int s = 0; s < ns; ++s) {
    PT_REQUIRE(bytes_each == 0 || (src[s] != nullptr && pt_host::aligned16(src[s])), PT_INVALID_ARGUMENT,
               "stream series: sources must be 16-byte aligned device pointers");
    p.src[s] = static_cast<const pt::u32x4_t*>(src[s]);
  }
  for (int d = 0; d < nd; ++d) {
    PT_REQUIRE(bytes_each == 0 || (dst[d] != nullptr && pt_host::aligned16(dst[d])), PT_INVALID_ARGUMENT,
               "stream series: destinations must be 16-byte aligned device pointers");
    p.dst[d] = static_cast<pt::u32x4_t*>(dst[d]);
  }
  const int64_t n = bytes_each / 16;
  if (n == 0) return PT_OK;
  const int64_t blocks = std::min<int64_t>((n + pt::kProbeThreads - 1) / pt::kProbeThreads, pt::kProbeMaxSeriesBlocks);
  pt::stream_series_kernel<<<static_cast<unsigned>(blocks), pt::kProbeThreads, 0, static_cast<hipStream_t>(stream)>>>(
      p, ns, nd, n, static_cast<uint32_t*>(out));
  PT_LAUNCH_CHECK();
  return PT_OK;
}

int64_t pt_stream_series_blocks(int64_t bytes_each) {
  if (bytes_each <= 0) return 0;
  return std::min<int64_t>((bytes_each / 16 + pt::kProbeThreads - 1) / pt::kProbeThreads, pt::kProbeMaxSeriesBlocks);
}

}  // extern "C"
