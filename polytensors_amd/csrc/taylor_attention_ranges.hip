// Block ranges of boolean attention masks (launcher of attn_mask_ranges_kernel).
#include "taylor_attention.inl"

namespace pt {

static_assert(kAttnRangeBlock == 64, "attn_ranges_count assumes 64-row blocks");

int64_t attention_mask_ranges_count(int64_t lq, int64_t lk) { return attn_ranges_count(lq, lk); }

int launch_attention_mask_ranges(const uint8_t* mask, int64_t n_masks, int64_t lq, int64_t lk, int32_t* ranges,
                                 hipStream_t stream) {
  const int64_t blocks = attention_mask_ranges_count(lq, lk) / 2;
  if (blocks == 0 || n_masks == 0) return PT_OK;
  attn_mask_ranges_kernel<><<<dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(n_masks)), dim3(256), 0,
                              stream>>>(mask, static_cast<int>(lq), static_cast<int>(lk), ranges);
  PT_LAUNCH_CHECK();
  return PT_OK;
}

}  // namespace pt
