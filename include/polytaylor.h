/*
 * polytaylor.h — C ABI of the MI355X (gfx950) truncated-Taylor kernels.
 *
 * A degree-K series tensor is passed the way the reference stores it: as K+1
 * coefficient buffers, one device pointer per order (the reference keeps a
 * tuple of K+1 tensors, /root/reference/src/polytensors/_tensor.py:147).
 * Every pointer array is a HOST array of device pointers; each coefficient
 * buffer is dense row-major with the shape stated per entry point. An
 * operand given with fewer orders (`*_orders` < K+1) has zero higher orders:
 * a plain tensor is passed with one order, as the reference's lift pads it
 * with zeros (/root/reference/src/polytensors/_range_ops.py:37-45).
 *
 * dtype codes: PT_FLOAT32, PT_FLOAT64, PT_BFLOAT16, PT_FLOAT16. Arithmetic is
 * float32 for the 32/16-bit types and float64 for PT_FLOAT64.
 *
 * All entry points are asynchronous on `stream` (a hipStream_t; NULL is the
 * null stream), allocate nothing, never synchronise the host, and return a
 * pt_status. On failure pt_last_error() gives a message (thread-local).
 * Outputs never alias inputs.
 */
#ifndef POLYTAYLOR_H
#define POLYTAYLOR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PT_ABI_VERSION 13
#define PT_MAX_DEGREE 8
/* Largest degree of the elementwise kernels (pt_activation_series_*, pt_series_binary): their
 * register plans are per element, so they run above PT_MAX_DEGREE. */
#define PT_MAX_ELEMENTWISE_DEGREE 16

typedef enum pt_dtype {
  PT_FLOAT32 = 0,
  PT_FLOAT64 = 1,
  PT_BFLOAT16 = 2,
  PT_FLOAT16 = 3
} pt_dtype;

typedef enum pt_status {
  PT_OK = 0,
  PT_INVALID_ARGUMENT = 1, /* shapes, pointers or sizes inconsistent */
  PT_UNSUPPORTED = 2,      /* valid call outside what the kernels implement */
  PT_DEVICE_ERROR = 3      /* the HIP runtime reported an error */
} pt_status;

typedef enum pt_reduction {
  PT_REDUCTION_NONE = 0,
  PT_REDUCTION_MEAN = 1,
  PT_REDUCTION_SUM = 2
} pt_reduction;

/* Message of the last failing call on this thread ("" if none). */
const char* pt_last_error(void);

/* PT_ABI_VERSION of the built library. */
int pt_abi_version(void);

/* Largest supported degree K (PT_MAX_DEGREE). */
int pt_max_degree(void);

/* Largest degree of the elementwise kernels (PT_MAX_ELEMENTWISE_DEGREE). */
int pt_max_elementwise_degree(void);

/*
 * RMSNorm of a degree-K series over the last `n` elements of each of `rows`
 * rows:  y(t) = x(t) * rsqrt(mean(x(t)^2) + eps) [* w(t)].
 * x, y: K+1 pointers, each [rows, n] of `dtype`.
 * weight: NULL, or `weight_orders` pointers (1 = plain weight, K+1 = series),
 *         each [n] of `dtype`.
 * Replaces the fused degree-1 RMSNorm of the reference
 *   /root/reference/src/polytensors/_fused_norm.py:24-40 (_run) and
 *   /root/reference/src/polytensors/_norm_kernels.py:7-19 (_forward),
 * generalised to degree K with the series of the reference's general rule
 *   /root/reference/src/polytensors/_decompositions.py:14-22 (_rms_norm) and
 *   /root/reference/src/polytensors/_series.py:83-96 (poly_rsqrt);
 * the weight multiply is the reference's separate `result * weight`
 *   (/root/reference/src/polytensors/_fused_norm.py:69), fused here.
 */
int pt_rms_norm_series_fwd(int dtype, int degree, const void* const* x,
                           const void* const* weight, int weight_orders,
                           void* const* y, int64_t rows, int64_t n, double eps,
                           void* stream);

/*
 * LayerNorm of a degree-K series over the last `n` elements of each row:
 *   c(t) = x(t) - mean(x(t)),
 *   y(t) = c(t) * rsqrt(mean(c(t)^2) + eps) [* w(t)] [+ b(t)].
 * Shapes as pt_rms_norm_series_fwd; bias like weight.
 * The reference has no layer-norm rule (native layer norm is listed as
 * missing, /root/reference/docs/notes.md:33-35); this is the series of the
 * composite built from its mean/mul/rsqrt rules
 *   (/root/reference/src/polytensors/_range_ops.py:133-149,178-193,
 *    /root/reference/src/polytensors/_series.py:83-96).
 */
int pt_layer_norm_series_fwd(int dtype, int degree, const void* const* x,
                             const void* const* weight, int weight_orders,
                             const void* const* bias, int bias_orders,
                             void* const* y, int64_t rows, int64_t n,
                             double eps, void* stream);

/*
 * Gradient series of the RMSNorm / LayerNorm normalization (no affine terms):
 *   dx(t) = J(x(t))^T g(t), the reverse-mode series of the output cotangent g.
 * RMSNorm:   dx = r (*) g - (1/n) r^3 (*) c (*) x,   c = sum_row g (*) x;
 * LayerNorm: with d = x - mean(x), the same for d and g - mean(g).
 * x, g, dx: K+1 pointers, each [rows, n] of `dtype`; eps as the forward.
 * Replaces the degree-1 backward of the reference
 *   /root/reference/src/polytensors/_norm_kernels.py:22-38 (_backward) and
 *   /root/reference/src/polytensors/_fused_norm.py:43-60 (_SeriesNorm, whose
 *   general formula :52-56 this evaluates in series arithmetic), at degree K.
 */
int pt_rms_norm_series_bwd(int dtype, int degree, const void* const* x,
                           const void* const* g, void* const* dx, int64_t rows,
                           int64_t n, double eps, void* stream);
int pt_layer_norm_series_bwd(int dtype, int degree, const void* const* x,
                             const void* const* g, void* const* dx,
                             int64_t rows, int64_t n, double eps, void* stream);

/*
 * Cross entropy of a degree-K series of logits z(t) with integer targets.
 * logits: K+1 pointers, each `rows` rows of `classes` values, row i at
 *         element offset i * row_stride (row_stride >= classes).
 * target: [rows] int64 device array; rows whose target == ignore_index get
 *         zero loss and are excluded from the mean's count.
 * reduction PT_REDUCTION_NONE: loss = K+1 pointers, each [rows] of the
 *           arithmetic type (float32, or float64 for PT_FLOAT64).
 *           PT_REDUCTION_MEAN / _SUM: loss = K+1 pointers, each one scalar of
 *           the arithmetic type; `workspace` must hold
 *           pt_cross_entropy_series_workspace_size(...) bytes (else unused).
 * lse: NULL, or K+1 pointers, each [rows] of the arithmetic type (float32, or
 *      float64 for PT_FLOAT64): the log-sum-exp series of each row.
 * softcap: 0 for none; else every logit series is first capped as
 *          softcap * tanh(z(t) / softcap) (the series of the cap), on the fly,
 *          as the reference's fused kernel caps its degree-1 logits
 *          (/root/reference/src/polytensors/_cross_entropy_kernels.py:7-17,
 *          _fused_cross_entropy.py:173-187); lse and loss refer to the capped logits.
 * loss_0 = lse_0 - z_0[y]; loss_k = lse_k - z_k[y] for k >= 1.
 * Replaces the fused degree-1 forward of the reference
 *   /root/reference/src/polytensors/_fused_cross_entropy.py:54-63 (forward),
 *   /root/reference/src/polytensors/_cross_entropy_kernels.py:20-55 (_forward)
 * and its reductions (/root/reference/src/polytensors/_fused_cross_entropy.py:163-170),
 * generalised to degree K with the log-softmax series of the general rule
 *   /root/reference/src/polytensors/_plain.py:262-273 (plain_softmax_family)
 *   and per-order NLL /root/reference/src/polytensors/_dispatch.py:537-543.
 */
int pt_cross_entropy_series_fwd(int dtype, int degree, const void* const* logits,
                                int64_t rows, int64_t classes, int64_t row_stride,
                                const int64_t* target, int64_t ignore_index,
                                double softcap, int reduction, void* const* loss,
                                void* const* lse, void* workspace, void* stream);

/*
 * Gradient series of the per-row cross-entropy losses:
 *   dz(t) = c(t) (*) (softmax(z(t)) - e_y)  per row (times the series of
 *   1 - tanh(z / softcap)^2 with a softcap), c the row's cotangent series.
 * logits, rows, classes, row_stride, target, ignore_index, softcap: as the
 *   forward; lse: the forward's lse output (K+1 pointers [rows], arithmetic
 *   type); cot: K+1 pointers [rows] of the arithmetic type; dz: K+1 pointers,
 *   each [rows, classes] contiguous of `dtype`. Ignored rows get zero.
 * Replaces the degree-1 backward of the reference
 *   /root/reference/src/polytensors/_cross_entropy_kernels.py:58-85 (_backward),
 *   /root/reference/src/polytensors/_fused_cross_entropy.py:101-128 (_SeriesCrossEntropy),
 * at degree K.
 */
int pt_cross_entropy_series_bwd(int dtype, int degree, const void* const* logits,
                                int64_t rows, int64_t classes, int64_t row_stride,
                                const int64_t* target, int64_t ignore_index,
                                double softcap, const void* const* lse,
                                const void* const* cot, void* const* dz, void* stream);

/* Bytes of device workspace pt_cross_entropy_series_fwd needs for a
 * reduction (0 for PT_REDUCTION_NONE). */
size_t pt_cross_entropy_series_workspace_size(int dtype, int degree,
                                              int64_t rows, int reduction);

/*
 * pt_cross_entropy_series_fwd without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. It calls
 * no hipMalloc, hipFree or allocating routine: a mean/sum reduction keeps its
 * per-row losses in a file-scope device array of PT_CE_NOALLOC_SCRATCH_BYTES
 * (4 MiB) that each GPU the library runs on holds until the process ends; its
 * address is looked up once per device on the first call there.
 * Arguments and results as pt_cross_entropy_series_fwd. A reduction whose
 * per-row losses, pt_cross_entropy_series_workspace_size(...) bytes, exceed
 * the array returns PT_UNSUPPORTED (before any device work).
 * All calls on one GPU share its array: calls that overlap on one GPU (other
 * streams or host threads) race and must be serialised by the caller.
 */
#define PT_CE_NOALLOC_SCRATCH_BYTES ((size_t)4 << 20)
int pt_cross_entropy_series_fwd_noalloc(int dtype, int degree, const void* const* logits,
                                        int64_t rows, int64_t classes, int64_t row_stride,
                                        const int64_t* target, int64_t ignore_index,
                                        double softcap, int reduction, void* const* loss,
                                        void* const* lse, void* stream);

/* PT_CE_NOALLOC_SCRATCH_BYTES of the built library. */
size_t pt_cross_entropy_series_noalloc_max_bytes(void);

/*
 * Cauchy-product (truncated series) matrix product
 *   C_k = sum_{i+j=k} A_i @ B_j,   k = 0..K,
 * the i-sum in increasing i as the reference's plain_polynomial_product
 *   (/root/reference/src/polytensors/_plain.py:118-128), reached from the
 *   mm/bmm/matmul/linear rules (/root/reference/src/polytensors/_range_ops.py:78-84,160-176).
 * a: a_orders pointers (1 or K+1), each [batch, m, k] (batch stride
 *    a_batch_stride elements; 0 broadcasts one matrix over the batch).
 * b: b_orders pointers (1 or K+1), each [batch, k, n], or [batch, n, k] if
 *    trans_b (then B_j is used transposed), batch stride b_batch_stride.
 * c: K+1 pointers, each [batch, m, n] contiguous.
 * dtype: PT_FLOAT32 (fp32 MFMA), PT_FLOAT64 (fp64 MFMA), or PT_BFLOAT16 / PT_FLOAT16 (16-bit MFMA
 * operands, fp32 accumulation, each output element rounded once; needs k and, unless trans_b, n
 * to be multiples of 8, 16-byte aligned operands, batch strides that are multiples of 8 and each
 * matrix below 1 GiB, else PT_UNSUPPORTED). Any alignment of c is accepted: 16-bit outputs are
 * written 8 bytes at a time where n is a multiple of 4 and every c[o] is 8-byte aligned, else one
 * element at a time).
 */
int pt_cauchy_matmul(int dtype, int degree, const void* const* a, int a_orders,
                     const void* const* b, int b_orders, void* const* c,
                     int64_t batch, int64_t m, int64_t n, int64_t k,
                     int64_t a_batch_stride, int64_t b_batch_stride,
                     int trans_b, void* stream);

/*
 * Flash-style attention forward of degree-K series:
 *   S(t) = scale * Q(t) K(t)^T (masked), P(t) = softmax(S(t)), O(t) = P(t) V(t).
 * q: q_orders pointers (1 or K+1), each [bh, lq, d];
 * k, v: k_orders / v_orders pointers, each [bh, lk, d];
 * out: K+1 pointers, each [bh, lq, d] of `dtype`.
 * lse: NULL, or K+1 pointers, each [bh, lq] of the arithmetic type: the
 *      log-sum-exp series of each score row (+inf, 0, ... for a row with no
 *      admissible key, whose output is zero, as the reference's fused kernel
 *      /root/reference/src/polytensors/_attention_kernels.py:70-76).
 * causal: key j admissible for query i iff j <= i.
 * mask: NULL, or [lq, lk] uint8 (nonzero = admissible); not with causal.
 * mask_ranges: NULL, or pt_attention_mask_ranges(mask, ...) of this mask: key
 *   blocks outside each query block's admissible range are then skipped.
 * Replaces the degree-1 fused forward
 *   /root/reference/src/polytensors/_fused_attention.py:126-141 (forward),
 *   /root/reference/src/polytensors/_attention_kernels.py:27-82 (_forward),
 * generalised to degree K; the series follow the general decomposition
 *   /root/reference/src/polytensors/_decompositions.py:28-43 (_attention).
 * dtype: PT_FLOAT32 or PT_FLOAT64 (fp32 / fp64 MFMA), or PT_BFLOAT16 or
 * PT_FLOAT16 (16-bit MFMA operands, fp32 accumulation and lse, as the
 * reference's half-type kernel, _fused_attention.py:72-78; the probability
 * series is rounded to the storage type as the value product's operand;
 * pointers 16-byte aligned, out 8-byte aligned).
 */
int pt_taylor_attention_fwd(int dtype, int degree, const void* const* q,
                            int q_orders, const void* const* k, int k_orders,
                            const void* const* v, int v_orders,
                            void* const* out, void* const* lse, int64_t bh,
                            int64_t lq, int64_t lk, int64_t d, int causal,
                            const uint8_t* mask, const int32_t* mask_ranges,
                            double scale, void* stream);

/*
 * pt_taylor_attention_fwd with a workspace for launches of few workgroups (no counterpart in
 * the reference; its kernels have no such split): the float32/float64 generic kernel then
 * divides each query block's key range over several workgroups, which write partial sums
 * into the workspace, and a second kernel merges them (same results up to the order of the
 * floating-point sums). pt_taylor_attention_fwd_workspace_size gives the bytes this needs
 * (0: the launch does not split, and the workspace may be NULL); a smaller workspace
 * runs the launch unsplit. The workspace must be 16-byte aligned.
 * mask_add: NULL, or an additive float mask, the reference's float attn_mask
 *   (/root/reference/src/polytensors/_decompositions.py:38-40: added to the scores, so to
 *   their constant order, after scaling): [lq, lk] values of the accumulator type (double for
 *   PT_FLOAT64, float for PT_FLOAT32, PT_BFLOAT16 and PT_FLOAT16). mask must then
 *   be given and mark exactly its finite entries (an entry of -inf excludes its key; a row
 *   with none admissible gets the empty-row output above).
 * mask_map: NULL (mask, mask_ranges and mask_add hold one mask, shared by every head), or
 *   three int64 {div, outer, inner} in host memory: they then hold a set of masks, [n, lq, lk]
 *   each (mask_ranges: n sets of pt_attention_mask_ranges_count(lq, lk) entries), and head b
 *   (0 .. bh-1) uses mask (b / div) * outer + (b % div) * inner. This is the broadcast of the
 *   reference's attn_mask over batch and heads (a [B, 1, lq, lk] mask over H heads per batch
 *   is {H, 1, 0}; [1, H, lq, lk] is {H, 0, 1}; one per head is {1, 1, 0}).
 */
size_t pt_taylor_attention_fwd_workspace_size(int dtype, int degree, int q_orders, int k_orders, int v_orders,
                                              int64_t bh, int64_t lq, int64_t lk, int64_t d);
int pt_taylor_attention_fwd_ws(int dtype, int degree, const void* const* q, int q_orders,
                               const void* const* k, int k_orders, const void* const* v, int v_orders,
                               void* const* out, void* const* lse, int64_t bh, int64_t lq, int64_t lk,
                               int64_t d, int causal, const uint8_t* mask, const int32_t* mask_ranges,
                               const void* mask_add, const int64_t* mask_map, double scale, void* workspace,
                               size_t workspace_bytes, void* stream);

/*
 * Block ranges of a boolean [lq, lk] attention mask (nonzero = admissible),
 * the reference's _mask_ranges
 *   /root/reference/src/polytensors/_fused_attention.py:81-99:
 * for each 64-row query block the first and one-past-last admissible key,
 * then for each 64-key block the first and one-past-last query admitting one of
 * its keys ((0, 0) when none). mask: n_masks masks [n_masks, lq, lk] (n_masks
 * at most 65535); ranges: n_masks * pt_attention_mask_ranges_count(lq, lk)
 * int32 of device memory, the masks' ranges one after the other. Computed once
 * per mask, reused by any number of forward and backward calls with that mask.
 */
int64_t pt_attention_mask_ranges_count(int64_t lq, int64_t lk);
int pt_attention_mask_ranges(const uint8_t* mask, int64_t n_masks, int64_t lq, int64_t lk,
                             int32_t* ranges, void* stream);

/*
 * Gradient series of pt_taylor_attention_fwd for an output cotangent series G:
 * coefficient j of dQ, dK, dV is sum_{k<=j} J_{j-k}^T G_k, i.e. the VJP
 *   P = exp(scale Q K^T - lse), dV = P^T G, dP = G V^T,
 *   dS = P (dP - rowsum(G O)), dQ = scale dS K, dK = scale dS^T Q
 * in truncated series arithmetic (products are Cauchy products of orders).
 * dtype: PT_FLOAT32, PT_FLOAT64, or PT_BFLOAT16 / PT_FLOAT16 (16-bit MFMA
 *   operands, fp32 accumulation; lse float32, as the forward writes it).
 * q, k, v, out, grad: K+1 pointers each (a plain operand or cotangent passes
 *   zeros for orders 1..K); shapes as in pt_taylor_attention_fwd; out and lse
 *   are that call's outputs for the same q, k, v, mask and scale.
 * dq ([bh, lq, d]), dk, dv ([bh, lk, d]): K+1 pointers each, or NULL when that
 *   gradient is not wanted.
 * workspace: pt_taylor_attention_bwd_workspace_size(...) bytes of device memory.
 * materialize: nonzero stores the P and dS series of every visited 16 x 16
 *   tile in the workspace (2 (K+1) bh lq lk values): five series products per
 *   admissible pair instead of eight (S and dP are then not recomputed for dK
 *   and dV), at the cost of that workspace. PT_FLOAT32, and PT_BFLOAT16 /
 *   PT_FLOAT16 at degrees 1..4 and head dims 32..128 (other 16-bit calls
 *   recompute and ignore it); PT_UNSUPPORTED for PT_FLOAT64.
 * mask, mask_ranges: as in pt_taylor_attention_fwd; mask_add, mask_map: as in
 *   pt_taylor_attention_fwd_ws (the forward's additive mask, [lq, lk] values of the
 *   accumulator type: double for PT_FLOAT64, float for the other types). With it the
 *   PT_FLOAT32 / PT_FLOAT64 kernels recompute the scores and materialize does not apply;
 *   the 16-bit stored-tile kernels take it as they are.
 * Pointers must be 16-byte aligned. Deterministic (no atomics).
 * Replaces the degree-1 fused backward
 *   /root/reference/src/polytensors/_fused_attention.py:144-163 (backward),
 *   /root/reference/src/polytensors/_fused_attention.py:267-295 (_SeriesAttention.backward),
 *   /root/reference/src/polytensors/_attention_kernels.py:85-201 (_block_terms,
 *   _backward_kv, _backward_q), generalised to degree K.
 */
int pt_taylor_attention_bwd(int dtype, int degree, const void* const* q,
                            const void* const* k, const void* const* v,
                            const void* const* out, const void* const* lse,
                            const void* const* grad, void* const* dq,
                            void* const* dk, void* const* dv, void* workspace,
                            int materialize, int64_t bh, int64_t lq, int64_t lk, int64_t d,
                            int causal, const uint8_t* mask,
                            const int32_t* mask_ranges, const void* mask_add, const int64_t* mask_map,
                            double scale,
                            void* stream);

/* Bytes of device workspace pt_taylor_attention_bwd needs (the per-row
 * rowsum(G O) series in the arithmetic type, and with materialize the P and
 * dS tiles). */
size_t pt_taylor_attention_bwd_workspace_size(int dtype, int degree, int64_t bh, int64_t lq,
                                              int64_t lk, int materialize);

/*
 * Complex directions through the real kernels. A series with a real constant
 * term and complex higher coefficients is run as real-direction variants and
 * recombined (the result is the multilinear extension of the real derivatives,
 *   /root/reference/docs/notes.md:59-76, and linear operations on complex
 * coefficients split into real and imaginary parts as the reference's
 *   /root/reference/src/polytensors/_dispatch.py:12-26 (_linear_complex_split)).
 * pt_complex_to_real: src holds `orders` complex planes of `numel` values
 *   (interleaved re, im); writes dst[v * orders + o] = alpha[v] Re(src[o]) +
 *   beta[v] Im(src[o]) for v < variants (real nodes: (1, lam_v); a real /
 *   imaginary split: (1, 0), (0, 1)).
 * pt_real_to_complex: writes dst[o] = sum_v (wre[v] + i wim[v]) src[v * orders + o].
 * orders <= 16, variants <= 17; PT_FLOAT32 (complex64) or PT_FLOAT64
 * (complex128); alpha/beta/wre/wim are host arrays. 16-byte aligned planes take
 * 16-byte accesses, others a scalar path.
 */
int pt_complex_to_real(int dtype, int orders, const void* const* src, int variants,
                       const double* alpha, const double* beta, void* const* dst,
                       int64_t numel, void* stream);
int pt_real_to_complex(int dtype, int orders, int variants, const void* const* src,
                       const double* wre, const double* wim, void* const* dst,
                       int64_t numel, void* stream);

/* Activation kinds of pt_activation_series_fwd / _bwd. */
typedef enum pt_activation {
  PT_ACT_GELU = 0,      /* x * Phi(x) (erf form, torch approximate='none') */
  PT_ACT_GELU_TANH = 1, /* 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) */
  PT_ACT_TANH = 2,
  PT_ACT_SIGMOID = 3,
  PT_ACT_SILU = 4,      /* x * sigmoid(x) */
  PT_ACT_EXP = 5,       /* forward only */
  PT_ACT_LOG = 6,       /* forward only */
  PT_ACT_SIN = 7,       /* forward only */
  PT_ACT_COS = 8,       /* forward only */
  PT_ACT_SQRT = 9,      /* forward only */
  PT_ACT_RSQRT = 10     /* forward only */
} pt_activation;

/*
 * Elementwise activation of a degree-K series: y(t) = f(x(t)), K up to
 * PT_MAX_ELEMENTWISE_DEGREE.
 * x, y: K+1 pointers, each `numel` elements of `dtype` (any shape, dense).
 * Arithmetic float32 (float64 for PT_FLOAT64); order 0 is f(x_0).
 * PT_ACT_SIN / PT_ACT_COS follow s' = c u', c' = -s u'; PT_ACT_SQRT / PT_ACT_RSQRT the power
 * recurrence k x_0 y_k = sum_{j=1..k} ((p+1) j - k) x_j y_{k-j} with p = 1/2, -1/2 (for
 * PT_ACT_RSQRT the reference's poly_rsqrt, /root/reference/src/polytensors/_series.py:83-96).
 * Replaces the fused degree-1 activation of the reference
 *   /root/reference/src/polytensors/_fused_activation.py:5-24 (maybe_activation),
 *   /root/reference/src/polytensors/_activation_kernels.py:8-38 (_activation),
 * generalised to degree K with the series of its plain-range rules
 *   /root/reference/src/polytensors/_plain.py:153-171 (plain_exp, plain_log),
 *   /root/reference/src/polytensors/_plain.py:174-259 (plain_activation: gelu,
 *   tanh, sigmoid by Faa di Bruno composition), dispatched from
 *   /root/reference/src/polytensors/_plain.py:276-355 (plain_rule),
 * and for silu / gelu_tanh the jets of
 *   /root/reference/src/polytensors/_activations.py:89-115 (_scalar_taylor),
 *   dispatched from /root/reference/src/polytensors/_dispatch.py:460-473.
 */
int pt_activation_series_fwd(int dtype, int degree, int kind,
                             const void* const* x, void* const* y,
                             int64_t numel, void* stream);

/*
 * Gradient series of the native activation backward operations:
 *   dx(t) = g(t) * f'(x(t)), Cauchy product truncated at K.
 * saved: for PT_ACT_GELU, PT_ACT_GELU_TANH and PT_ACT_SILU the forward INPUT
 *        series x; for PT_ACT_TANH and PT_ACT_SIGMOID the forward OUTPUT
 *        series y (as aten.tanh_backward / aten.sigmoid_backward take it).
 * g, saved, dx: K+1 pointers, each `numel` elements of `dtype`.
 * The forward-only kinds (PT_ACT_EXP, PT_ACT_LOG, PT_ACT_SIN, PT_ACT_COS, PT_ACT_SQRT,
 * PT_ACT_RSQRT: their gradients are products of forward series) return PT_UNSUPPORTED.
 * Replaces the BACKWARD mode of
 *   /root/reference/src/polytensors/_activation_kernels.py:8-38 (degree 1),
 * generalised with the reference's gradient-series rules
 *   /root/reference/src/polytensors/_plain.py:310-325 (gelu_backward,
 *   tanh_backward, sigmoid_backward) and
 *   /root/reference/src/polytensors/_dispatch.py:629-630 (silu_backward).
 */
int pt_activation_series_bwd(int dtype, int degree, int kind,
                             const void* const* g, const void* const* saved,
                             void* const* dx, int64_t numel, void* stream);

/* Operations of pt_series_binary. */
typedef enum pt_binary {
  PT_BINARY_MUL = 0,
  PT_BINARY_DIV = 1
} pt_binary;

/*
 * Elementwise product or quotient of two degree-K series of one shape (K up to
 * PT_MAX_ELEMENTWISE_DEGREE):
 *   PT_BINARY_MUL  y_k = sum_{i+j=k} a_i b_j,
 *   PT_BINARY_DIV  y_k = (a_k - sum_{i=1..k} b_i y_{k-i}) / b_0.
 * a, b, y: K+1 pointers, each `numel` elements of `dtype`.
 * Replaces the reference's general rules for a series times / over a series
 *   /root/reference/src/polytensors/_range_ops.py:133-149 (mul -> convolution,
 *   _plain.py:118-128; div -> quotient, _range_ops.py:86-93); an ordinary
 *   operand takes the constant-operand path there (:109-132) and needs no kernel.
 */
int pt_series_binary(int dtype, int degree, int op, const void* const* a,
                     const void* const* b, void* const* y, int64_t numel,
                     void* stream);

/*
 * Streaming probes (measurement only; no counterpart in the reference): the
 * practical HBM ceiling beside the published peak, with the access pattern of
 * the memory-bound series kernels (16-byte non-temporal loads and stores).
 * pt_stream_copy copies `bytes` (a multiple of 16, 16-byte aligned pointers);
 * pt_stream_read reads them and writes out[b] = XOR of the 32-bit words read by
 * block b, for b < the block count (`out` holds one uint32 per block).
 * blocks = 0 takes pt_stream_probe_blocks(); at most 65536. chunked != 0: block
 * b walks its own contiguous chunk; 0: the grid walks the buffer together.
 */
int pt_stream_copy(const void* src, void* dst, int64_t bytes, int blocks, int chunked, void* stream);
int pt_stream_read(const void* src, int64_t bytes, int blocks, int chunked, void* out, void* stream);
int pt_stream_probe_blocks(void);
/*
 * The series kernels' own pattern over separate buffers (the K+1 orders of a series): ns
 * sources (1..18) and nd destinations (0..9) of bytes_each bytes each; every thread reads one
 * 16-byte vector of every source at its index and writes their XOR to every destination, a
 * block per 256 indices. With nd = 0 it writes out[b] = XOR of block b's words (out holds
 * pt_stream_series_blocks(bytes_each) uint32 values).
 */
int pt_stream_series(const void* const* src, int ns, void* const* dst, int nd, int64_t bytes_each, void* out,
                     void* stream);
int64_t pt_stream_series_blocks(int64_t bytes_each);

#ifdef __cplusplus
}
#endif

#endif /* POLYTAYLOR_H */
