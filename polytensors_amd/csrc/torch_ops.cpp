// PyTorch registration of the gfx950 Taylor kernels: the polytensors_amd::*
// operators (TORCH_LIBRARY schemas, CUDA/HIP implementations) over the C ABI
// of libpolytaylor.so (include/polytaylor.h). Each implementation checks its
// arguments (ValueError), allocates the coefficient-stacked [K+1, ...] result,
// passes the K+1 coefficient pointers of every series as they are stored (no
// stacking copies) and launches on the current HIP stream of the operands'
// device; a non-zero status becomes RuntimeError with pt_last_error(). The
// fake (shape) and autograd registrations of these operators are made from
// Python (polytensors_amd/_ops.py).
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <array>
#include <limits>
#include <string>
#include <vector>

#include "../../include/polytaylor.h"

namespace {

using at::Tensor;
using TensorList = std::vector<Tensor>;

hipStream_t stream_of(const Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

void check_abi() {
  static const bool ok = pt_abi_version() == PT_ABI_VERSION;
  TORCH_CHECK(ok, "polytensors_amd: libpolytaylor.so has ABI ", pt_abi_version(), ", this extension was built for ",
              PT_ABI_VERSION, ": rebuild both with `python -m polytensors_amd.build`");
}

void check_status(int status, const std::string& what) {
  if (status == PT_OK) return;
  const char* kind = status == PT_INVALID_ARGUMENT ? "invalid argument"
                     : status == PT_UNSUPPORTED    ? "unsupported"
                     : status == PT_DEVICE_ERROR   ? "device error"
                                                   : "error";
  TORCH_CHECK(false, what, ": ", kind, ": ", pt_last_error());
}

bool has_code(at::ScalarType t) {
  return t == at::kFloat || t == at::kDouble || t == at::kBFloat16 || t == at::kHalf;
}

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return PT_FLOAT32;
    case at::kDouble: return PT_FLOAT64;
    case at::kBFloat16: return PT_BFLOAT16;
    case at::kHalf: return PT_FLOAT16;
    default: break;
  }
  TORCH_CHECK_VALUE(false, "polytensors_amd: unsupported dtype ", t);
}

at::ScalarType acc_type(at::ScalarType t) { return t == at::kDouble ? at::kDouble : at::kFloat; }

std::vector<const void*> cptrs(const TensorList& ts) {
  std::vector<const void*> p(std::max<size_t>(1, ts.size()), nullptr);
  for (size_t i = 0; i < ts.size(); ++i) p[i] = ts[i].data_ptr();
  return p;
}

// The leading slices of a coefficient-stacked (contiguous) result.
std::vector<void*> slices(const Tensor& stacked) {
  std::vector<void*> p(std::max<int64_t>(1, stacked.size(0)), nullptr);
  char* base = static_cast<char*>(stacked.data_ptr());
  const int64_t step = stacked.stride(0) * static_cast<int64_t>(stacked.element_size());
  for (int64_t i = 0; i < stacked.size(0); ++i) p[i] = base + i * step;
  return p;
}

std::vector<int64_t> stacked_shape(int64_t orders, at::IntArrayRef shape) {
  std::vector<int64_t> s{orders};
  s.insert(s.end(), shape.begin(), shape.end());
  return s;
}

void check_series(const std::string& name, const TensorList& c, c10::optional<at::ScalarType> want = c10::nullopt) {
  TORCH_CHECK_VALUE(!c.empty(), name, ": at least one coefficient is required");
  const Tensor& first = c[0];
  const at::ScalarType dtype = want ? *want : first.scalar_type();
  for (const Tensor& t : c) {
    TORCH_CHECK_VALUE(t.scalar_type() == dtype, name, ": coefficient dtypes differ (", t.scalar_type(), " vs ",
                      dtype, ")");
    TORCH_CHECK_VALUE(t.device() == first.device(), name, ": coefficients on different devices");
    TORCH_CHECK_VALUE(t.sizes() == first.sizes(), name, ": coefficient shapes differ");
    TORCH_CHECK_VALUE(t.is_contiguous(), name, ": coefficients must be contiguous");
  }
  TORCH_CHECK_VALUE(has_code(dtype), name, ": unsupported dtype ", dtype);
}

// ---- RMSNorm / LayerNorm series ----------------------------------------------

Tensor norm_series(const TensorList& x, const TensorList& weight, const TensorList& bias, int64_t n, double eps,
                   bool layer) {
  check_abi();
  check_series("norm_series", x);
  const int64_t degree = static_cast<int64_t>(x.size()) - 1;
  const int64_t numel = x[0].numel();
  TORCH_CHECK_VALUE(n >= 1 && numel % n == 0, "norm_series: n must divide the element count");
  for (const auto& [name, aff] : {std::pair<const char*, const TensorList*>{"weight", &weight}, {"bias", &bias}}) {
    const int64_t len = static_cast<int64_t>(aff->size());
    TORCH_CHECK_VALUE(len == 0 || len == 1 || len == degree + 1, "norm_series: ", name,
                      " needs 0, 1 or degree+1 coefficients");
    for (const Tensor& c : *aff)
      TORCH_CHECK_VALUE(c.scalar_type() == x[0].scalar_type() && c.device() == x[0].device() && c.numel() == n &&
                            c.is_contiguous(),
                        "norm_series: ", name, " coefficients must be contiguous [n] of the input dtype");
  }
  TORCH_CHECK_VALUE(layer || bias.empty(), "norm_series: bias is a LayerNorm argument");
  c10::DeviceGuard guard(x[0].device());
  Tensor out = at::empty(stacked_shape(degree + 1, x[0].sizes()), x[0].options());
  auto xs = cptrs(x), ws = cptrs(weight), bs = cptrs(bias);
  auto ys = slices(out);
  const int code = dtype_code(x[0].scalar_type());
  int status;
  if (layer) {
    status = pt_layer_norm_series_fwd(code, static_cast<int>(degree), xs.data(), weight.empty() ? nullptr : ws.data(),
                                      static_cast<int>(weight.size()), bias.empty() ? nullptr : bs.data(),
                                      static_cast<int>(bias.size()), ys.data(), numel / n, n, eps, stream_of(x[0]));
  } else {
    status = pt_rms_norm_series_fwd(code, static_cast<int>(degree), xs.data(), weight.empty() ? nullptr : ws.data(),
                                    static_cast<int>(weight.size()), ys.data(), numel / n, n, eps, stream_of(x[0]));
  }
  check_status(status, layer ? "layer_norm_series" : "rms_norm_series");
  return out;
}

Tensor norm_series_backward(const TensorList& x, const TensorList& grad, int64_t n, double eps, bool layer) {
  check_abi();
  check_series("norm_series_backward x", x);
  check_series("norm_series_backward grad", grad);
  TORCH_CHECK_VALUE(x.size() == grad.size() && x[0].sizes() == grad[0].sizes() &&
                        x[0].scalar_type() == grad[0].scalar_type() && x[0].device() == grad[0].device(),
                    "norm_series_backward: x and grad series must match");
  const int64_t degree = static_cast<int64_t>(x.size()) - 1;
  const int64_t numel = x[0].numel();
  TORCH_CHECK_VALUE(n >= 1 && numel % n == 0, "norm_series_backward: n must divide the element count");
  c10::DeviceGuard guard(x[0].device());
  Tensor out = at::empty(stacked_shape(degree + 1, x[0].sizes()), x[0].options());
  auto xs = cptrs(x), gs = cptrs(grad);
  auto ys = slices(out);
  const int code = dtype_code(x[0].scalar_type());
  const int status = (layer ? pt_layer_norm_series_bwd : pt_rms_norm_series_bwd)(
      code, static_cast<int>(degree), xs.data(), gs.data(), ys.data(), numel / n, n, eps, stream_of(x[0]));
  check_status(status, layer ? "layer_norm_series_bwd" : "rms_norm_series_bwd");
  return out;
}

// ---- Cross-entropy series ----------------------------------------------------

void check_logit_rows(const std::string& name, const TensorList& z) {
  TORCH_CHECK_VALUE(!z.empty(), name, ": at least one coefficient is required");
  const Tensor& first = z[0];
  TORCH_CHECK_VALUE(first.dim() == 2, name, ": logits must be (N, C)");
  TORCH_CHECK_VALUE(has_code(first.scalar_type()), name, ": unsupported dtype ", first.scalar_type());
  for (const Tensor& c : z) {
    TORCH_CHECK_VALUE(c.scalar_type() == first.scalar_type() && c.device() == first.device() &&
                          c.sizes() == first.sizes(),
                      name, ": coefficients must share dtype, device and shape");
    TORCH_CHECK_VALUE(c.strides() == first.strides() && c.stride(1) == 1, name,
                      ": coefficient rows must be contiguous with one common row stride");
  }
}

std::tuple<Tensor, Tensor> cross_entropy_series(const TensorList& z, const Tensor& target, int64_t ignore_index,
                                                int64_t reduction, double softcap) {
  check_abi();
  check_logit_rows("cross_entropy_series", z);
  const Tensor& first = z[0];
  TORCH_CHECK_VALUE(target.scalar_type() == at::kLong && target.dim() == 1 && target.size(0) == first.size(0) &&
                        target.is_contiguous() && target.device() == first.device(),
                    "cross_entropy_series: target must be contiguous int64 [N]");
  TORCH_CHECK_VALUE(reduction >= 0 && reduction <= 2, "cross_entropy_series: reduction must be 0, 1 or 2");
  TORCH_CHECK_VALUE(softcap >= 0.0 && softcap != std::numeric_limits<double>::infinity(),
                    "cross_entropy_series: softcap must be 0 or a positive cap");
  const int64_t degree = static_cast<int64_t>(z.size()) - 1;
  const int64_t rows = first.size(0), classes = first.size(1);
  c10::DeviceGuard guard(first.device());
  const auto acc = first.options().dtype(acc_type(first.scalar_type()));
  Tensor lse = at::empty({degree + 1, rows}, acc);
  Tensor loss = reduction == 0 ? at::empty({degree + 1, rows}, acc) : at::empty({degree + 1}, acc);
  const int code = dtype_code(first.scalar_type());
  const size_t wbytes =
      pt_cross_entropy_series_workspace_size(code, static_cast<int>(degree), rows, static_cast<int>(reduction));
  Tensor workspace = at::empty({static_cast<int64_t>(std::max<size_t>(1, wbytes))}, first.options().dtype(at::kByte));
  auto zs = cptrs(z);
  auto ls = slices(loss), es = slices(lse);
  const int status = pt_cross_entropy_series_fwd(
      code, static_cast<int>(degree), zs.data(), rows, classes, rows ? first.stride(0) : classes,
      target.data_ptr<int64_t>(), ignore_index, softcap, static_cast<int>(reduction), ls.data(), es.data(),
      workspace.data_ptr(), stream_of(first));
  check_status(status, "cross_entropy_series");
  return {loss, lse};
}

Tensor cross_entropy_series_backward(const TensorList& z, const Tensor& target, int64_t ignore_index, double softcap,
                                     const Tensor& lse, const TensorList& cot) {
  check_abi();
  TORCH_CHECK_VALUE(!z.empty() && cot.size() == z.size() && lse.dim() >= 1 &&
                        lse.size(0) == static_cast<int64_t>(z.size()),
                    "cross_entropy_series_backward: z, lse and cot need the same number of orders");
  check_logit_rows("cross_entropy_series_backward", z);
  const Tensor& first = z[0];
  const int64_t rows = first.size(0), classes = first.size(1);
  const at::ScalarType acc = acc_type(first.scalar_type());
  TORCH_CHECK_VALUE(lse.scalar_type() == acc && lse.is_contiguous() && lse.dim() == 2 && lse.size(1) == rows,
                    "cross_entropy_series_backward: lse must be contiguous [K+1, N] of the arithmetic type");
  for (const Tensor& c : cot)
    TORCH_CHECK_VALUE(c.scalar_type() == acc && c.is_contiguous() && c.dim() == 1 && c.size(0) == rows,
                      "cross_entropy_series_backward: cotangents must be contiguous [N] of the arithmetic type");
  TORCH_CHECK_VALUE(target.scalar_type() == at::kLong && target.is_contiguous() && target.dim() == 1 &&
                        target.size(0) == rows,
                    "cross_entropy_series_backward: target must be contiguous int64 [N]");
  const int64_t degree = static_cast<int64_t>(z.size()) - 1;
  c10::DeviceGuard guard(first.device());
  Tensor out = at::empty({degree + 1, rows, classes}, first.options());
  auto zs = cptrs(z), cs = cptrs(cot);
  auto es = slices(lse);
  std::vector<const void*> ec(es.begin(), es.end());
  auto os = slices(out);
  const int status = pt_cross_entropy_series_bwd(dtype_code(first.scalar_type()), static_cast<int>(degree), zs.data(),
                                                 rows, classes, rows ? first.stride(0) : classes,
                                                 target.data_ptr<int64_t>(), ignore_index, softcap, ec.data(),
                                                 cs.data(), os.data(), stream_of(first));
  check_status(status, "cross_entropy_series_bwd");
  return out;
}

// ---- Cauchy-product matmul ---------------------------------------------------

// x zero-padded at the end of dim to a multiple of `multiple` (x itself if it is one).
Tensor pad_dim(const Tensor& x, int64_t dim, int64_t multiple) {
  const int64_t size = x.size(dim);
  const int64_t extra = (multiple - size % multiple) % multiple;
  if (extra == 0) return x;
  std::vector<int64_t> pad(2 * (x.dim() - 1 - ((dim % x.dim() + x.dim()) % x.dim())), 0);
  pad.push_back(0);
  pad.push_back(extra);
  return at::constant_pad_nd(x, pad, 0);
}

Tensor aligned16(const Tensor& x) {
  return reinterpret_cast<uintptr_t>(x.data_ptr()) % 16 == 0 ? x : x.clone();
}

Tensor cauchy_matmul(const TensorList& a_in, const TensorList& b_in, int64_t degree, bool trans_b) {
  check_abi();
  for (const auto& [name, s] : {std::pair<const char*, const TensorList*>{"a", &a_in}, {"b", &b_in}}) {
    const int64_t len = static_cast<int64_t>(s->size());
    TORCH_CHECK_VALUE(len == 1 || len == degree + 1, "cauchy_matmul: ", name, " needs 1 or degree+1 coefficients");
    check_series(std::string("cauchy_matmul ") + name, *s);
    TORCH_CHECK_VALUE((*s)[0].dim() == 3, "cauchy_matmul: ", name, " must be 3-D [batch, rows, cols]");
  }
  const at::ScalarType dtype = a_in[0].scalar_type();
  TORCH_CHECK_VALUE(b_in[0].scalar_type() == dtype && b_in[0].device() == a_in[0].device(),
                    "cauchy_matmul: operand dtype/device differ");
  const int64_t ba = a_in[0].size(0), m = a_in[0].size(1);
  int64_t kd = a_in[0].size(2);
  const int64_t bb = b_in[0].size(0);
  int64_t n = trans_b ? b_in[0].size(1) : b_in[0].size(2);
  const int64_t kb = trans_b ? b_in[0].size(2) : b_in[0].size(1);
  TORCH_CHECK_VALUE(kb == kd, "cauchy_matmul: inner dimensions differ");
  TORCH_CHECK_VALUE(ba == bb || ba == 1 || bb == 1, "cauchy_matmul: batch dimensions do not broadcast");
  const int64_t batch = std::max(ba, bb);
  const int64_t n_out = n;
  c10::DeviceGuard guard(a_in[0].device());
  TensorList a = a_in, b = b_in;
  if (dtype == at::kBFloat16 || dtype == at::kHalf) {
    // the 16-bit kernel moves 16-byte chunks: zero-pad the contraction (which leaves every product
    // unchanged) and, for B stored [k, n], the columns to multiples of 8, and give it 16-byte
    // aligned operands
    for (Tensor& t : a) t = aligned16(pad_dim(t, -1, 8));
    for (Tensor& t : b) t = aligned16(pad_dim(t, trans_b ? -1 : -2, 8));
    if (!trans_b) {
      for (Tensor& t : b) t = pad_dim(t, -1, 8);
      n = b[0].size(2);
    }
    kd = a[0].size(2);
  }
  Tensor out = at::empty({degree + 1, batch, m, n}, a[0].options());
  auto as = cptrs(a), bs = cptrs(b);
  auto cs = slices(out);
  const int status = pt_cauchy_matmul(dtype_code(dtype), static_cast<int>(degree), as.data(),
                                      static_cast<int>(a.size()), bs.data(), static_cast<int>(b.size()), cs.data(),
                                      batch, m, n, kd, ba == 1 ? 0 : m * kd, bb == 1 ? 0 : n * kd, trans_b ? 1 : 0,
                                      stream_of(a[0]));
  check_status(status, "cauchy_matmul");
  if (n == n_out) return out;
  return out.narrow(-1, 0, n_out).contiguous();
}

// ---- Taylor attention --------------------------------------------------------

// An attention mask as the kernels take it: the boolean mask of the admissible entries (a
// floating mask's entries above -inf), a floating mask's values in the accumulator type (added
// to the constant-order scores), and for a set of masks [n, L, S] the map of heads to masks.
struct AttnMask {
  c10::optional<Tensor> keep, add;
  int64_t count = 1;
  std::array<int64_t, 3> map{1, 0, 0};
  bool mapped = false;
  const uint8_t* keep_ptr() const { return keep ? static_cast<const uint8_t*>(keep->data_ptr()) : nullptr; }
  const void* add_ptr() const { return add ? add->data_ptr() : nullptr; }
  const int64_t* map_ptr() const { return mapped ? map.data() : nullptr; }
};

// mask: (L, S), shared by every head, or (n, L, S) with mask_map (div, outer, inner): head b
// uses mask (b / div) * outer + (b % div) * inner (without a map, n == bh and head b uses mask b).
AttnMask attention_mask(const c10::optional<Tensor>& mask, at::OptionalIntArrayRef mask_map, const Tensor& q0,
                        int64_t bh, int64_t lq, int64_t lk, bool causal, const char* name) {
  AttnMask m;
  const bool has_map = mask_map.has_value() && !mask_map->empty();
  if (!mask) {
    TORCH_CHECK_VALUE(!has_map, name, ": mask_map without a mask");
    return m;
  }
  const at::ScalarType type = mask->scalar_type();
  const int64_t dim = mask->dim();
  TORCH_CHECK_VALUE((type == at::kBool || at::isFloatingType(type)) && (dim == 2 || dim == 3) &&
                        mask->size(dim - 2) == lq && mask->size(dim - 1) == lk && mask->device() == q0.device(),
                    name, ": mask must be a bool or floating (L, S) or (n, L, S) tensor on the query's device");
  TORCH_CHECK_VALUE(!causal, name, ": mask and causal are exclusive");
  if (dim == 3) {
    m.count = mask->size(0);
    TORCH_CHECK_VALUE(m.count >= 1 && m.count <= 65535, name, ": a mask set holds 1 to 65535 masks");
    if (has_map) {
      TORCH_CHECK_VALUE(mask_map->size() == 3 && (*mask_map)[0] >= 1 && (*mask_map)[1] >= 0 && (*mask_map)[2] >= 0,
                        name, ": mask_map must be (div >= 1, outer >= 0, inner >= 0)");
      m.map = {(*mask_map)[0], (*mask_map)[1], (*mask_map)[2]};
    } else {
      TORCH_CHECK_VALUE(m.count == bh, name, ": an (n, L, S) mask without mask_map needs one mask per head");
      m.map = {1, 1, 0};
    }
    if (bh > 0) {   // the largest mask index any head takes
      const int64_t top = ((bh - 1) / m.map[0]) * m.map[1] + (std::min(m.map[0], bh) - 1) * m.map[2];
      TORCH_CHECK_VALUE(top < m.count, name, ": mask_map sends a head past the ", m.count, " masks given");
    }
    m.mapped = true;
  } else {
    TORCH_CHECK_VALUE(!has_map, name, ": mask_map needs an (n, L, S) mask");
  }
  if (type == at::kBool) {
    m.keep = mask->contiguous();
    return m;
  }
  m.add = mask->to(acc_type(q0.scalar_type())).contiguous();
  m.keep = at::ne(*m.add, -std::numeric_limits<double>::infinity());
  return m;
}

// Block ranges of every mask of m on its device (the key / query blocks the kernels visit).
c10::optional<Tensor> mask_ranges(const AttnMask& m, int64_t lq, int64_t lk) {
  if (!m.keep) return c10::nullopt;
  const int64_t per = pt_attention_mask_ranges_count(lq, lk);
  Tensor ranges = at::empty({std::max<int64_t>(1, m.count * per)}, m.keep->options().dtype(at::kInt));
  check_status(pt_attention_mask_ranges(m.keep_ptr(), m.count, lq, lk, ranges.data_ptr<int32_t>(), stream_of(*m.keep)),
               "attention_mask_ranges");
  return ranges;
}

std::tuple<Tensor, Tensor> taylor_attention_fwd(const TensorList& q, const TensorList& k, const TensorList& v,
                                                const c10::optional<Tensor>& mask_in, bool causal, double scale,
                                                int64_t degree, at::OptionalIntArrayRef mask_map) {
  check_abi();
  for (const auto& [name, s] :
       {std::pair<const char*, const TensorList*>{"q", &q}, {"k", &k}, {"v", &v}}) {
    const int64_t len = static_cast<int64_t>(s->size());
    TORCH_CHECK_VALUE(len == 1 || len == degree + 1, "taylor_attention: ", name,
                      " needs 1 or degree+1 coefficients");
    check_series(std::string("taylor_attention ") + name, *s);
    TORCH_CHECK_VALUE((*s)[0].dim() >= 3, "taylor_attention: ", name, " must be [..., length, d]");
  }
  // batch dimensions [...] (flattened to bh heads in order), then length and head dim
  const at::ScalarType dtype = q[0].scalar_type();
  const int64_t nd = q[0].dim();
  const auto batch = q[0].sizes().slice(0, nd - 2);
  const int64_t lq = q[0].size(nd - 2), d = q[0].size(nd - 1);
  int64_t bh = 1;
  for (const int64_t b : batch) bh *= b;
  TORCH_CHECK_VALUE(k[0].sizes() == v[0].sizes() && k[0].dim() == nd && k[0].sizes().slice(0, nd - 2) == batch &&
                        k[0].size(nd - 1) == d,
                    "taylor_attention: key/value shapes must be [..., S, d] matching the query");
  TORCH_CHECK_VALUE(k[0].scalar_type() == dtype && v[0].scalar_type() == dtype, "taylor_attention: dtypes differ");
  const int64_t lk = k[0].size(nd - 2);
  c10::DeviceGuard guard(q[0].device());
  const auto mask = attention_mask(mask_in, mask_map, q[0], bh, lq, lk, causal, "taylor_attention");
  std::vector<int64_t> out_shape{degree + 1};
  out_shape.insert(out_shape.end(), batch.begin(), batch.end());
  out_shape.push_back(lq);
  out_shape.push_back(d);
  Tensor out = at::empty(out_shape, q[0].options());
  Tensor lse = at::empty({degree + 1, bh, lq}, q[0].options().dtype(acc_type(dtype)));
  const auto ranges = mask_ranges(mask, lq, lk);
  auto qs = cptrs(q), ks = cptrs(k), vs = cptrs(v);
  auto os = slices(out), ls = slices(lse);
  const int code = dtype_code(dtype);
  // launches of few workgroups split each key range over several (partial sums in a workspace)
  const size_t wbytes = pt_taylor_attention_fwd_workspace_size(
      code, static_cast<int>(degree), static_cast<int>(q.size()), static_cast<int>(k.size()),
      static_cast<int>(v.size()), bh, lq, lk, d);
  Tensor workspace;
  if (wbytes > 0) workspace = at::empty({static_cast<int64_t>(wbytes)}, q[0].options().dtype(at::kByte));
  const int status = pt_taylor_attention_fwd_ws(
      code, static_cast<int>(degree), qs.data(), static_cast<int>(q.size()), ks.data(),
      static_cast<int>(k.size()), vs.data(), static_cast<int>(v.size()), os.data(), ls.data(), bh, lq, lk, d,
      causal ? 1 : 0, mask.keep_ptr(), ranges ? ranges->data_ptr<int32_t>() : nullptr, mask.add_ptr(),
      mask.map_ptr(), scale, wbytes > 0 ? workspace.data_ptr() : nullptr, wbytes, stream_of(q[0]));
  check_status(status, "taylor_attention_fwd");
  return {out, lse};
}

std::tuple<Tensor, Tensor, Tensor> taylor_attention_bwd(const TensorList& q, const TensorList& k,
                                                        const TensorList& v, const Tensor& out, const Tensor& lse,
                                                        const TensorList& grad, const c10::optional<Tensor>& mask_in,
                                                        bool causal, double scale, int64_t materialize,
                                                        at::OptionalIntArrayRef mask_map) {
  check_abi();
  const int64_t degree = static_cast<int64_t>(q.size()) - 1;
  for (const auto& [name, s] : {std::pair<const char*, const TensorList*>{"q", &q}, {"k", &k}, {"v", &v},
                                {"grad", &grad}}) {
    TORCH_CHECK_VALUE(static_cast<int64_t>(s->size()) == degree + 1, "taylor_attention_bwd: ", name,
                      " needs degree+1 coefficients");
    check_series(std::string("taylor_attention_bwd ") + name, *s);
    TORCH_CHECK_VALUE((*s)[0].dim() == 3, "taylor_attention_bwd: ", name, " must be [bh, length, d]");
  }
  const at::ScalarType dtype = q[0].scalar_type();
  TORCH_CHECK_VALUE(has_code(dtype), "taylor_attention_bwd: float32, float64, bfloat16 or float16 only");
  const int64_t bh = q[0].size(0), lq = q[0].size(1), d = q[0].size(2);
  TORCH_CHECK_VALUE(k[0].sizes() == v[0].sizes() && k[0].size(0) == bh && k[0].size(2) == d,
                    "taylor_attention_bwd: key/value shapes must be [bh, S, d] matching the query");
  TORCH_CHECK_VALUE(grad[0].sizes() == q[0].sizes(), "taylor_attention_bwd: grad must have the query's shape");
  TORCH_CHECK_VALUE(k[0].scalar_type() == dtype && v[0].scalar_type() == dtype && grad[0].scalar_type() == dtype,
                    "taylor_attention_bwd: dtypes differ");
  TORCH_CHECK_VALUE(out.scalar_type() == dtype && out.is_contiguous() &&
                        out.sizes() == at::IntArrayRef({degree + 1, bh, lq, d}),
                    "taylor_attention_bwd: out must be the forward's contiguous [K+1, bh, L, d] output");
  TORCH_CHECK_VALUE(lse.scalar_type() == acc_type(dtype) && lse.is_contiguous() &&
                        lse.sizes() == at::IntArrayRef({degree + 1, bh, lq}),
                    "taylor_attention_bwd: lse must be the forward's contiguous [K+1, bh, L] output");
  const int64_t lk = k[0].size(1);
  c10::DeviceGuard guard(q[0].device());
  const auto mask = attention_mask(mask_in, mask_map, q[0], bh, lq, lk, causal, "taylor_attention_bwd");
  // float32 and float64 recompute with an additive mask (materialize is ignored); the 16-bit
  // stored tiles carry it
  if (mask.add && (dtype == at::kFloat || dtype == at::kDouble)) materialize = 0;
  Tensor dq = at::empty({degree + 1, bh, lq, d}, q[0].options());
  Tensor dk = at::empty({degree + 1, bh, lk, d}, q[0].options());
  Tensor dv = at::empty_like(dk);
  const auto ranges = mask_ranges(mask, lq, lk);
  const int code = dtype_code(dtype);
  auto workspace_for = [&](int64_t mat) {
    const size_t wbytes =
        pt_taylor_attention_bwd_workspace_size(code, static_cast<int>(degree), bh, lq, lk, static_cast<int>(mat));
    return at::empty({static_cast<int64_t>(std::max<size_t>(1, wbytes))}, q[0].options().dtype(at::kByte));
  };
  Tensor workspace;
  if (materialize < 0) {   // stored tiles where the workspace takes at most a quarter of the device
                           // and can be allocated now (else recompute); the library refuses them for
                           // float64
    const size_t size = pt_taylor_attention_bwd_workspace_size(code, static_cast<int>(degree), bh, lq, lk, 1);
    size_t free_bytes = 0, total_bytes = 0;
    if (hipMemGetInfo(&free_bytes, &total_bytes) != hipSuccess) total_bytes = 0;
    materialize = dtype != at::kDouble && total_bytes > 0 && size <= total_bytes / 4 ? 1 : 0;
    if (materialize) {
      try {
        workspace = workspace_for(1);
      } catch (const c10::OutOfMemoryError&) {   // a busy device: the recomputing kernels need none
        materialize = 0;
      }
    }
  }
  if (!workspace.defined()) workspace = workspace_for(materialize);
  auto qs = cptrs(q), ks = cptrs(k), vs = cptrs(v), gs = cptrs(grad);
  auto os = slices(out), ls = slices(lse);
  std::vector<const void*> oc(os.begin(), os.end()), lc(ls.begin(), ls.end());
  auto dqs = slices(dq), dks = slices(dk), dvs = slices(dv);
  const int status = pt_taylor_attention_bwd(
      code, static_cast<int>(degree), qs.data(), ks.data(), vs.data(), oc.data(), lc.data(), gs.data(), dqs.data(),
      dks.data(), dvs.data(), workspace.data_ptr(), static_cast<int>(materialize), bh, lq, lk, d, causal ? 1 : 0,
      mask.keep_ptr(), ranges ? ranges->data_ptr<int32_t>() : nullptr, mask.add_ptr(), mask.map_ptr(), scale,
      stream_of(q[0]));
  check_status(status, "taylor_attention_bwd");
  return {dq, dk, dv};
}

// ---- Complex directions ------------------------------------------------------

Tensor complex_to_real(const TensorList& src, at::ArrayRef<double> alpha, at::ArrayRef<double> beta) {
  check_abi();
  TORCH_CHECK_VALUE(!src.empty() && !alpha.empty() && alpha.size() == beta.size(),
                    "complex_to_real: planes and variants required");
  const Tensor& first = src[0];
  TORCH_CHECK_VALUE(first.scalar_type() == at::kComplexFloat || first.scalar_type() == at::kComplexDouble,
                    "complex_to_real: complex64 or complex128 planes");
  for (const Tensor& c : src)
    TORCH_CHECK_VALUE(c.scalar_type() == first.scalar_type() && c.sizes() == first.sizes() &&
                          c.device() == first.device() && c.is_contiguous(),
                      "complex_to_real: planes must share dtype, shape and device and be contiguous");
  const at::ScalarType real = first.scalar_type() == at::kComplexFloat ? at::kFloat : at::kDouble;
  c10::DeviceGuard guard(first.device());
  std::vector<int64_t> shape{static_cast<int64_t>(alpha.size()), static_cast<int64_t>(src.size())};
  shape.insert(shape.end(), first.sizes().begin(), first.sizes().end());
  Tensor out = at::empty(shape, first.options().dtype(real));
  std::vector<void*> dst;   // plane (variant a, order o) at a * orders + o
  char* base = static_cast<char*>(out.data_ptr());
  const int64_t plane = out.stride(1) * static_cast<int64_t>(out.element_size());
  for (int64_t i = 0; i < out.size(0) * out.size(1); ++i) dst.push_back(base + i * plane);
  auto ss = cptrs(src);
  const int status = pt_complex_to_real(dtype_code(real), static_cast<int>(src.size()), ss.data(),
                                        static_cast<int>(alpha.size()), alpha.data(), beta.data(), dst.data(),
                                        first.numel(), stream_of(first));
  check_status(status, "complex_to_real");
  return out;
}

Tensor real_to_complex(const TensorList& src, int64_t orders, at::ArrayRef<double> wre, at::ArrayRef<double> wim) {
  check_abi();
  const int64_t variants = static_cast<int64_t>(wre.size());
  TORCH_CHECK_VALUE(variants >= 1 && static_cast<int64_t>(wim.size()) == variants &&
                        static_cast<int64_t>(src.size()) == variants * orders && orders >= 1,
                    "real_to_complex: src must hold variants x orders planes");
  const Tensor& first = src[0];
  TORCH_CHECK_VALUE(first.scalar_type() == at::kFloat || first.scalar_type() == at::kDouble,
                    "real_to_complex: float32 or float64 planes");
  for (const Tensor& c : src)
    TORCH_CHECK_VALUE(c.scalar_type() == first.scalar_type() && c.sizes() == first.sizes() &&
                          c.device() == first.device() && c.is_contiguous(),
                      "real_to_complex: planes must share dtype, shape and device and be contiguous");
  const at::ScalarType cplx = first.scalar_type() == at::kFloat ? at::kComplexFloat : at::kComplexDouble;
  c10::DeviceGuard guard(first.device());
  Tensor out = at::empty(stacked_shape(orders, first.sizes()), first.options().dtype(cplx));
  auto ss = cptrs(src);
  auto os = slices(out);
  const int status = pt_real_to_complex(dtype_code(first.scalar_type()), static_cast<int>(orders),
                                        static_cast<int>(variants), ss.data(), wre.data(), wim.data(), os.data(),
                                        first.numel(), stream_of(first));
  check_status(status, "real_to_complex");
  return out;
}

// ---- Elementwise series ------------------------------------------------------

int activation_code(const std::string& kind, bool backward, const char* name) {
  static const std::pair<const char*, int> kinds[] = {
      {"gelu", PT_ACT_GELU}, {"gelu_tanh", PT_ACT_GELU_TANH}, {"tanh", PT_ACT_TANH}, {"sigmoid", PT_ACT_SIGMOID},
      {"silu", PT_ACT_SILU}, {"exp", PT_ACT_EXP},             {"log", PT_ACT_LOG},   {"sin", PT_ACT_SIN},
      {"cos", PT_ACT_COS},   {"sqrt", PT_ACT_SQRT},           {"rsqrt", PT_ACT_RSQRT}};
  for (const auto& [k, code] : kinds)
    if (kind == k && !(backward && code > PT_ACT_SILU)) return code;   // the forward-only kinds
  TORCH_CHECK_VALUE(false, name, backward ? ": no backward for kind '" : ": unknown kind '", kind, "'");
}

Tensor activation_series(const TensorList& x, c10::string_view kind) {
  check_abi();
  check_series("activation_series", x);
  const std::string k(kind);
  const int code = activation_code(k, false, "activation_series");
  const int64_t degree = static_cast<int64_t>(x.size()) - 1;
  c10::DeviceGuard guard(x[0].device());
  Tensor out = at::empty(stacked_shape(degree + 1, x[0].sizes()), x[0].options());
  auto xs = cptrs(x);
  auto ys = slices(out);
  check_status(pt_activation_series_fwd(dtype_code(x[0].scalar_type()), static_cast<int>(degree), code, xs.data(),
                                        ys.data(), x[0].numel(), stream_of(x[0])),
               "activation_series(" + k + ")");
  return out;
}

Tensor activation_series_backward(const TensorList& grad, const TensorList& saved, c10::string_view kind) {
  check_abi();
  check_series("activation_series_backward grad", grad);
  check_series("activation_series_backward saved", saved);
  TORCH_CHECK_VALUE(grad.size() == saved.size() && grad[0].sizes() == saved[0].sizes() &&
                        grad[0].scalar_type() == saved[0].scalar_type() && grad[0].device() == saved[0].device(),
                    "activation_series_backward: grad and saved series must match in degree, shape, dtype and "
                    "device");
  const std::string k(kind);
  const int code = activation_code(k, true, "activation_series_backward");
  const int64_t degree = static_cast<int64_t>(grad.size()) - 1;
  c10::DeviceGuard guard(grad[0].device());
  Tensor out = at::empty(stacked_shape(degree + 1, grad[0].sizes()), grad[0].options());
  auto gs = cptrs(grad), ss = cptrs(saved);
  auto ys = slices(out);
  check_status(pt_activation_series_bwd(dtype_code(grad[0].scalar_type()), static_cast<int>(degree), code, gs.data(),
                                        ss.data(), ys.data(), grad[0].numel(), stream_of(grad[0])),
               "activation_series_backward(" + k + ")");
  return out;
}

Tensor series_binary(const TensorList& a, const TensorList& b, c10::string_view op) {
  check_abi();
  check_series("series_binary a", a);
  check_series("series_binary b", b);
  TORCH_CHECK_VALUE(a.size() == b.size() && a[0].sizes() == b[0].sizes() &&
                        a[0].scalar_type() == b[0].scalar_type() && a[0].device() == b[0].device(),
                    "series_binary: operands must match in degree, shape, dtype and device");
  const std::string o(op);
  TORCH_CHECK_VALUE(o == "mul" || o == "div", "series_binary: unknown operation '", o, "'");
  const int64_t degree = static_cast<int64_t>(a.size()) - 1;
  c10::DeviceGuard guard(a[0].device());
  Tensor out = at::empty(stacked_shape(degree + 1, a[0].sizes()), a[0].options());
  auto as = cptrs(a), bs = cptrs(b);
  auto ys = slices(out);
  check_status(pt_series_binary(dtype_code(a[0].scalar_type()), static_cast<int>(degree),
                                o == "mul" ? PT_BINARY_MUL : PT_BINARY_DIV, as.data(), bs.data(), ys.data(),
                                a[0].numel(), stream_of(a[0])),
               "series_binary(" + o + ")");
  return out;
}

}  // namespace

TORCH_LIBRARY(polytensors_amd, m) {
  m.def("norm_series(Tensor[] x, Tensor[] weight, Tensor[] bias, int n, float eps, bool layer) -> Tensor");
  m.def("norm_series_backward(Tensor[] x, Tensor[] grad, int n, float eps, bool layer) -> Tensor");
  m.def("cross_entropy_series(Tensor[] z, Tensor target, int ignore_index, int reduction, float softcap) "
        "-> (Tensor, Tensor)");
  m.def("cross_entropy_series_backward(Tensor[] z, Tensor target, int ignore_index, float softcap, Tensor lse, "
        "Tensor[] cot) -> Tensor");
  m.def("cauchy_matmul(Tensor[] a, Tensor[] b, int degree, bool trans_b) -> Tensor");
  m.def("taylor_attention_fwd(Tensor[] q, Tensor[] k, Tensor[] v, Tensor? mask, bool causal, float scale, "
        "int degree, int[]? mask_map=None) -> (Tensor, Tensor)");
  m.def("taylor_attention_bwd(Tensor[] q, Tensor[] k, Tensor[] v, Tensor out, Tensor lse, Tensor[] grad, "
        "Tensor? mask, bool causal, float scale, int materialize=-1, int[]? mask_map=None) -> (Tensor, Tensor, Tensor)");
  m.def("complex_to_real(Tensor[] src, float[] alpha, float[] beta) -> Tensor");
  m.def("real_to_complex(Tensor[] src, int orders, float[] wre, float[] wim) -> Tensor");
  m.def("activation_series(Tensor[] x, str kind) -> Tensor");
  m.def("activation_series_backward(Tensor[] grad, Tensor[] saved, str kind) -> Tensor");
  m.def("series_binary(Tensor[] a, Tensor[] b, str op) -> Tensor");
}

TORCH_LIBRARY_IMPL(polytensors_amd, CUDA, m) {
  m.impl("norm_series", &norm_series);
  m.impl("norm_series_backward", &norm_series_backward);
  m.impl("cross_entropy_series", &cross_entropy_series);
  m.impl("cross_entropy_series_backward", &cross_entropy_series_backward);
  m.impl("cauchy_matmul", &cauchy_matmul);
  m.impl("taylor_attention_fwd", &taylor_attention_fwd);
  m.impl("taylor_attention_bwd", &taylor_attention_bwd);
  m.impl("complex_to_real", &complex_to_real);
  m.impl("real_to_complex", &real_to_complex);
  m.impl("activation_series", &activation_series);
  m.impl("activation_series_backward", &activation_series_backward);
  m.impl("series_binary", &series_binary);
}
