// C ABI of the Taylor attention kernels.
#include "taylor_attention.h"

extern "C" {

int pt_taylor_attention_fwd(int dtype, int degree, const void* const* q, int q_orders,
                            const void* const* k, int k_orders, const void* const* v, int v_orders,
                            void* const* out, void* const* lse, int64_t bh, int64_t lq, int64_t lk,
                            int64_t d, int causal, const uint8_t* mask, double scale, void* stream) {
  pt_host::clear_error();
  PT_REQUIRE(degree >= 0 && degree <= PT_MAX_DEGREE, PT_UNSUPPORTED,
             "Taylor attention: degree must be in 0..8");
  PT_REQUIRE(dtype == PT_FLOAT32 || dtype == PT_FLOAT64, PT_UNSUPPORTED,
             "Taylor attention: float32 and float64 only");
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
  for (int o = 0; o < q_orders; ++o) PT_REQUIRE(q[o] != nullptr, PT_INVALID_ARGUMENT, "null q");
  // an empty key sequence may come with null key/value buffers (nothing is read)
  for (int o = 0; o < k_orders; ++o) PT_REQUIRE(k[o] != nullptr || lk == 0, PT_INVALID_ARGUMENT, "null k");
  for (int o = 0; o < v_orders; ++o) PT_REQUIRE(v[o] != nullptr || lk == 0, PT_INVALID_ARGUMENT, "null v");
  for (int o = 0; o <= degree; ++o) {
    PT_REQUIRE(out[o] != nullptr, PT_INVALID_ARGUMENT, "null out");
    PT_REQUIRE(lse == nullptr || lse[o] != nullptr, PT_INVALID_ARGUMENT, "null lse entry");
  }
  if (bh == 0 || lq == 0) return PT_OK;
  pt::AttnArgs a{degree, q, q_orders, k, k_orders, v, v_orders, out, lse, bh, lq, lk, d,
                 causal != 0, mask, scale, static_cast<hipStream_t>(stream)};
  return dtype == PT_FLOAT32 ? pt::launch_attention<float>(a) : pt::launch_attention<double>(a);
}

}  // extern "C"
