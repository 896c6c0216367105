// C ABI of the Taylor attention kernels.
#include "taylor_attention.h"

namespace {

// The mask map of the C ABI (NULL: one mask shared by every head), checked.
bool read_mask_map(const int64_t* map, pt::AttnMaskMap& m) {
  if (map == nullptr) return true;
  m.div = map[0];
  m.outer = map[1];
  m.inner = map[2];
  return m.div >= 1 && m.outer >= 0 && m.inner >= 0;
}

}  // namespace

extern "C" {

int pt_taylor_attention_fwd(int dtype, int degree, const void* const* q, int q_orders,
                            const void* const* k, int k_orders, const void* const* v, int v_orders,
                            void* const* out, void* const* lse, int64_t bh, int64_t lq, int64_t lk,
                            int64_t d, int causal, const uint8_t* mask, const int32_t* mask_ranges, double scale,
                            void* stream) {
  return pt_taylor_attention_fwd_ws(dtype, degree, q, q_orders, k, k_orders, v, v_orders, out, lse, bh, lq, lk, d,
                                    causal, mask, mask_ranges, nullptr, nullptr, scale, nullptr, 0, stream);
}

size_t pt_taylor_attention_fwd_workspace_size(int dtype, int degree, int q_orders, int k_orders, int v_orders,
                                              int64_t bh, int64_t lq, int64_t lk, int64_t d) {
  if (degree < 0 || degree > PT_MAX_DEGREE || bh < 0 || lq < 0 || lk < 0 || d <= 0) return 0;
  const pt::AttnSplit sp = pt::attention_split(dtype, degree, q_orders, k_orders, v_orders, bh, lq, lk, d);
  return sp.chunks > 1 ? sp.bytes : 0;
}

int pt_taylor_attention_fwd_ws(int dtype, int degree, const void* const* q, int q_orders,
                               const void* const* k, int k_orders, const void* const* v, int v_orders,
                               void* const* out, void* const* lse, int64_t bh, int64_t lq, int64_t lk,
                               int64_t d, int causal, const uint8_t* mask, const int32_t* mask_ranges,
                               const void* mask_add, const int64_t* mask_map, double scale, void* workspace,
                               size_t workspace_bytes, void* stream) {
  pt_host::clear_error();
  pt::AttnMaskMap map;
  PT_REQUIRE(read_mask_map(mask_map, map), PT_INVALID_ARGUMENT,
             "Taylor attention: mask_map must hold div >= 1, outer >= 0, inner >= 0");
  PT_REQUIRE(workspace_bytes == 0 || pt_host::aligned16(workspace), PT_INVALID_ARGUMENT,
             "Taylor attention: workspace must be 16-byte aligned");
  PT_REQUIRE(degree >= 0 && degree <= PT_MAX_DEGREE, PT_UNSUPPORTED,
             "Taylor attention: degree must be in 0..8");
  PT_REQUIRE(mask_ranges == nullptr || mask != nullptr, PT_INVALID_ARGUMENT,
             "Taylor attention: mask_ranges without a mask");
  PT_REQUIRE(mask_add == nullptr || mask != nullptr, PT_INVALID_ARGUMENT,
             "Taylor attention: an additive mask needs the boolean mask of its finite entries");
  PT_REQUIRE(dtype == PT_FLOAT32 || dtype == PT_FLOAT64 || dtype == PT_BFLOAT16 || dtype == PT_FLOAT16,
             PT_UNSUPPORTED, "Taylor attention: float32, float64, bfloat16 or float16");
  PT_REQUIRE(q != nullptr && k != nullptr && v != nullptr && out != nullptr, PT_INVALID_ARGUMENT,
             "Taylor attention: q, k, v and out pointer arrays are required");
  for (int o : {q_orders, k_orders, v_orders})
    PT_REQUIRE(o == 1 || o == degree + 1, PT_INVALID_ARGUMENT,
               "Taylor attention: operand orders must be 1 or degree+1");
  PT_REQUIRE(bh >= 0 && lq >= 0 && lk >= 0, PT_INVALID_ARGUMENT, "Taylor attention: negative size");
  PT_REQUIRE(d == 16 || d == 32 || d == 64 || d == 128, PT_UNSUPPORTED,
             "Taylor attention: head dim must be 16, 32, 64 or 128");
  PT_REQUIRE(!(causal && mask != nullptr), PT_INVALID_ARGUMENT,
             "Taylor attention: causal and mask are exclusive");
  PT_REQUIRE(lq <= INT32_MAX && lk <= INT32_MAX && (lq + 63) / 64 * bh <= (int64_t{1} << 24), PT_UNSUPPORTED,
             "Taylor attention: sizes beyond the launch grid (query blocks x heads > 2^24)");
  // empty sequences may come with null buffers (nothing is read or written)
  const bool no_rows = bh == 0 || lq == 0;
  for (int o = 0; o < q_orders; ++o) PT_REQUIRE(q[o] != nullptr || no_rows, PT_INVALID_ARGUMENT, "null q");
  for (int o = 0; o < k_orders; ++o) PT_REQUIRE(k[o] != nullptr || lk == 0, PT_INVALID_ARGUMENT, "null k");
  for (int o = 0; o < v_orders; ++o) PT_REQUIRE(v[o] != nullptr || lk == 0, PT_INVALID_ARGUMENT, "null v");
  for (int o = 0; o <= degree; ++o) {
    PT_REQUIRE(out[o] != nullptr || no_rows, PT_INVALID_ARGUMENT, "null out");
    PT_REQUIRE(lse == nullptr || lse[o] != nullptr || no_rows, PT_INVALID_ARGUMENT, "null lse entry");
  }
  if (bh == 0 || lq == 0) return PT_OK;
  pt::AttnArgs a{degree, q, q_orders, k, k_orders, v, v_orders, out, lse, bh, lq, lk, d,
                 causal != 0, mask, mask_ranges, scale, static_cast<hipStream_t>(stream),
                 workspace_bytes > 0 ? workspace : nullptr, workspace_bytes, mask_add, map};
  switch (dtype) {
    case PT_FLOAT32: return pt::launch_attention<float>(a);
    case PT_FLOAT64: return pt::launch_attention<double>(a);
    case PT_BFLOAT16: return pt::launch_attention_half<pt::bf16>(a);
    default: return pt::launch_attention_half<_Float16>(a);
  }
}

int64_t pt_attention_mask_ranges_count(int64_t lq, int64_t lk) {
  if (lq < 0 || lk < 0) return 0;
  return pt::attention_mask_ranges_count(lq, lk);
}

int pt_attention_mask_ranges(const uint8_t* mask, int64_t n_masks, int64_t lq, int64_t lk, int32_t* ranges,
                             void* stream) {
  pt_host::clear_error();
  PT_REQUIRE(lq >= 0 && lk >= 0 && lq <= INT32_MAX && lk <= INT32_MAX, PT_INVALID_ARGUMENT,
             "attention mask ranges: sizes out of range");
  PT_REQUIRE(n_masks >= 0 && n_masks <= 65535, PT_INVALID_ARGUMENT,
             "attention mask ranges: n_masks must be in 0..65535");
  PT_REQUIRE((mask != nullptr || lq * lk == 0) && (ranges != nullptr || lq + lk == 0), PT_INVALID_ARGUMENT,
             "attention mask ranges: mask and ranges are required");
  return pt::launch_attention_mask_ranges(mask, n_masks, lq, lk, ranges, static_cast<hipStream_t>(stream));
}

size_t pt_taylor_attention_bwd_workspace_size(int dtype, int degree, int64_t bh, int64_t lq, int64_t lk,
                                              int materialize) {
  if (degree < 0 || degree > PT_MAX_DEGREE || bh < 0 || lq < 0 || lk < 0) return 0;
  if (dtype == PT_BFLOAT16 || dtype == PT_FLOAT16)   // stored tiles at degrees 1..4
    return pt::attention_bwd_half_layout(degree, bh, lq, lk, materialize != 0 && degree >= 1 && degree <= 4).total;
  // the rowsum(G O) series in the accumulator type (float64, else float32); the stored tiles (float32
  // only) in the element type
  const size_t size = dtype == PT_FLOAT64 ? sizeof(double) : sizeof(float);
  return pt::attention_bwd_layout(size, size, degree, bh, lq, lk, materialize != 0).total;
}

int pt_taylor_attention_bwd(int dtype, int degree, const void* const* q, const void* const* k,
                            const void* const* v, const void* const* out, const void* const* lse,
                            const void* const* grad, void* const* dq, void* const* dk, void* const* dv,
                            void* workspace, int materialize, int64_t bh, int64_t lq, int64_t lk, int64_t d,
                            int causal, const uint8_t* mask, const int32_t* mask_ranges, const void* mask_add,
                            const int64_t* mask_map, double scale, void* stream) {
  pt_host::clear_error();
  pt::AttnMaskMap map;
  PT_REQUIRE(read_mask_map(mask_map, map), PT_INVALID_ARGUMENT,
             "Taylor attention backward: mask_map must hold div >= 1, outer >= 0, inner >= 0");
  PT_REQUIRE(mask_ranges == nullptr || mask != nullptr, PT_INVALID_ARGUMENT,
             "Taylor attention backward: mask_ranges without a mask");
  PT_REQUIRE(mask_add == nullptr || mask != nullptr, PT_INVALID_ARGUMENT,
             "Taylor attention backward: an additive mask needs the boolean mask of its finite entries");
  // The stored-tile path is float32 and 16-bit only: a float64 run of it (degree 8, head dim 64)
  // took a GPU memory fault whose cause is not established, so float64 always recomputes.
  PT_REQUIRE(!materialize || dtype != PT_FLOAT64, PT_UNSUPPORTED,
             "Taylor attention backward: materialize is not available for float64 (float32 and 16-bit only)");
  PT_REQUIRE(degree >= 0 && degree <= PT_MAX_DEGREE, PT_UNSUPPORTED,
             "Taylor attention backward: degree must be in 0..8");
  PT_REQUIRE(dtype == PT_FLOAT32 || dtype == PT_FLOAT64 || dtype == PT_BFLOAT16 || dtype == PT_FLOAT16,
             PT_UNSUPPORTED, "Taylor attention backward: dtype must be float32, float64, bfloat16 or float16");
  PT_REQUIRE(q != nullptr && k != nullptr && v != nullptr && out != nullptr && lse != nullptr &&
                 grad != nullptr,
             PT_INVALID_ARGUMENT, "Taylor attention backward: q, k, v, out, lse and grad are required");
  PT_REQUIRE(bh >= 0 && lq >= 0 && lk >= 0, PT_INVALID_ARGUMENT, "Taylor attention backward: negative size");
  PT_REQUIRE(d == 16 || d == 32 || d == 64 || d == 128, PT_UNSUPPORTED,
             "Taylor attention backward: head dim must be 16, 32, 64 or 128");
  PT_REQUIRE(!(causal && mask != nullptr), PT_INVALID_ARGUMENT,
             "Taylor attention backward: causal and mask are exclusive");
  // grids: (query blocks x heads x slices) and (key blocks x heads x slices), at most 8 slices
  PT_REQUIRE(lq <= INT32_MAX && lk <= INT32_MAX && (lq + 63) / 64 * bh <= (int64_t{1} << 24) &&
                 (lk + 63) / 64 * bh <= (int64_t{1} << 24),
             PT_UNSUPPORTED, "Taylor attention backward: sizes beyond the launch grid (blocks x heads > 2^24)");
  PT_REQUIRE((bh * lq == 0 && !materialize) || workspace != nullptr, PT_INVALID_ARGUMENT,
             "Taylor attention backward: the workspace is required");
  PT_REQUIRE(pt_host::aligned16(workspace), PT_INVALID_ARGUMENT,
             "Taylor attention backward: workspace must be 16-byte aligned");
  const bool need_q = bh * lq > 0, need_k = bh * lk > 0;
  for (int o = 0; o <= degree; ++o) {
    PT_REQUIRE((q[o] != nullptr || !need_q) && (out[o] != nullptr || !need_q) &&
                   (grad[o] != nullptr || !need_q) && (lse[o] != nullptr || !need_q),
               PT_INVALID_ARGUMENT, "Taylor attention backward: null q/out/grad/lse entry");
    PT_REQUIRE((k[o] != nullptr && v[o] != nullptr) || !need_k, PT_INVALID_ARGUMENT,
               "Taylor attention backward: null k/v entry");
    PT_REQUIRE(pt_host::aligned16(q[o]) && pt_host::aligned16(k[o]) && pt_host::aligned16(v[o]) &&
                   pt_host::aligned16(out[o]) && pt_host::aligned16(grad[o]),
               PT_INVALID_ARGUMENT, "Taylor attention backward: operands must be 16-byte aligned");
    PT_REQUIRE(dq == nullptr || dq[o] != nullptr || !need_q, PT_INVALID_ARGUMENT, "null dq entry");
    PT_REQUIRE(dk == nullptr || dk[o] != nullptr || !need_k, PT_INVALID_ARGUMENT, "null dk entry");
    PT_REQUIRE(dv == nullptr || dv[o] != nullptr || !need_k, PT_INVALID_ARGUMENT, "null dv entry");
    PT_REQUIRE((dq == nullptr || pt_host::aligned16(dq[o])) && (dk == nullptr || pt_host::aligned16(dk[o])) &&
                   (dv == nullptr || pt_host::aligned16(dv[o])),
               PT_INVALID_ARGUMENT, "Taylor attention backward: outputs must be 16-byte aligned");
  }
  if (bh == 0) return PT_OK;
  pt::AttnBwdArgs a{degree, q, k, v, out, lse, grad, dq, dk, dv, workspace, bh, lq, lk, d,
                    causal != 0, mask, mask_ranges, scale, materialize != 0, static_cast<hipStream_t>(stream),
                    mask_add, map};
  switch (dtype) {
    case PT_FLOAT32: return pt::launch_attention_bwd<float>(a);
    case PT_FLOAT64: return pt::launch_attention_bwd<double>(a);
    case PT_BFLOAT16: return pt::launch_attention_bwd_half<pt::bf16>(a);
    default: return pt::launch_attention_bwd_half<_Float16>(a);
  }
}

}  // extern "C"
