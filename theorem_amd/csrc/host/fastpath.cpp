// Host fast path of the four custom_kernel wrappers (theorem_amd.kernels.*):
// the argument checks, the output allocation and the C-ABI launch of one call
// in C++ (pybind11 over torch tensors), instead of Python attribute queries,
// torch.empty calls from Python and a ctypes call with 17 arguments.
//
// It is an accelerator only.  Each function handles the common case (every
// tensor on one GPU, dense row-major, 16-byte aligned, the dtypes and shapes
// the kernels take) and returns None for anything else; the Python wrapper
// then runs its own path, which raises the reference's errors.  When the C
// ABI returns a nonzero status, the function returns that status (an int)
// and the wrapper raises it at once (ValueError for an argument the C side
// rejected, RuntimeError for a launch error), with no second attempt.  The
// kernels, their arguments and the outputs' allocation (torch's caching
// allocator, the current stream) are the same on both paths.
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include "theorem_mi355x.h"

namespace py = pybind11;

namespace {

constexpr int64_t kBT = 64;

int32_t dtype_code(const at::Tensor& t) {
  if (t.scalar_type() == at::kFloat) return THM_DTYPE_F32;
  if (t.scalar_type() == at::kBFloat16) return THM_DTYPE_BF16;
  return -1;
}

// On GPU `dev`, dense row-major and 16-byte aligned.
bool ok(const at::Tensor& t, int dev) {
  return t.is_cuda() && t.get_device() == dev && t.is_contiguous() &&
         (reinterpret_cast<uintptr_t>(t.data_ptr()) & 15) == 0;
}
bool ok_opt(const c10::optional<at::Tensor>& t, int dev) { return !t.has_value() || ok(*t, dev); }
const void* ptr(const c10::optional<at::Tensor>& t) { return t.has_value() ? t->data_ptr() : nullptr; }
bool is_f32(const c10::optional<at::Tensor>& t) { return !t.has_value() || t->scalar_type() == at::kFloat; }

void* stream_of(int dev) { return c10::hip::getCurrentHIPStream(dev).stream(); }

// causal_conv1d.custom_kernel((x, weight, bias), activation) for x [B, D, S] contiguous.
py::object conv1d(const at::Tensor& x, const at::Tensor& weight, const c10::optional<at::Tensor>& bias,
                  int32_t activation) {
  if (!x.is_cuda() || x.dim() != 3 || weight.dim() != 2) return py::none();
  const int dev = x.get_device();
  if (!ok(x, dev) || !ok(weight, dev) || !ok_opt(bias, dev)) return py::none();
  const int64_t B = x.size(0), D = x.size(1), S = x.size(2), W = weight.size(1);
  if (weight.size(0) != D || (bias.has_value() && (bias->dim() != 1 || bias->size(0) != D ||
                                                   bias->scalar_type() != weight.scalar_type())))
    return py::none();
  const int32_t xd = dtype_code(x), wd = dtype_code(weight);
  if (xd < 0 || wd < 0 || W > INT32_MAX) return py::none();
  at::Tensor out = at::empty_like(x);
  const int st = thm_causal_conv1d_fwd(x.data_ptr(), weight.data_ptr(), ptr(bias), out.data_ptr(), B, D, S,
                                       (int32_t)W, xd, wd, activation, stream_of(dev));
  if (st != THM_OK) return py::int_(st);
  return py::cast(out);
}

// recompute_w_u: (w, u) from k, v [B, T, H, K / V], beta [B, T, H], A [B, T, H, 64], g.
py::object wu(const at::Tensor& k, const at::Tensor& v, const at::Tensor& beta, const at::Tensor& A,
              const c10::optional<at::Tensor>& g) {
  if (!k.is_cuda() || k.dim() != 4 || v.dim() != 4) return py::none();
  const int dev = k.get_device();
  if (!ok(k, dev) || !ok(v, dev) || !ok(beta, dev) || !ok(A, dev) || !ok_opt(g, dev)) return py::none();
  const int64_t B = k.size(0), T = k.size(1), H = k.size(2), K = k.size(3), V = v.size(3);
  const std::vector<int64_t> bth{B, T, H};
  if (T % kBT || v.sizes().slice(0, 3) != at::IntArrayRef(bth) || beta.sizes() != at::IntArrayRef(bth) ||
      A.sizes() != at::IntArrayRef({B, T, H, kBT}) || (g.has_value() && g->sizes() != at::IntArrayRef(bth)))
    return py::none();
  if (beta.scalar_type() != at::kFloat || A.scalar_type() != at::kFloat || !is_f32(g) ||
      k.scalar_type() != v.scalar_type())
    return py::none();
  const int32_t code = dtype_code(k);
  if (code < 0) return py::none();
  at::Tensor w = at::empty_like(k), u = at::empty_like(v);
  const int st = thm_recompute_w_u_fwd(k.data_ptr(), v.data_ptr(), beta.data_ptr(), A.data_ptr(), ptr(g),
                                       w.data_ptr(), u.data_ptr(), B, T, H, K, V, (int32_t)kBT, code,
                                       stream_of(dev));
  if (st != THM_OK) return py::int_(st);
  return py::make_tuple(w, u);
}

// chunk_fwd_h: (h, v_new or None, final state or None); w given selects the delta form.
py::object h(const at::Tensor& k, const c10::optional<at::Tensor>& w, const at::Tensor& vu,
             const c10::optional<at::Tensor>& g, const c10::optional<at::Tensor>& h0, bool delta, bool want_vn,
             bool want_ht) {
  if (!k.is_cuda() || k.dim() != 4 || vu.dim() != 4 || delta != w.has_value()) return py::none();
  const int dev = k.get_device();
  if (!ok(k, dev) || !ok_opt(w, dev) || !ok(vu, dev) || !ok_opt(g, dev) || !ok_opt(h0, dev)) return py::none();
  const int64_t B = k.size(0), T = k.size(1), H = k.size(2), K = k.size(3), V = vu.size(3);
  if (T % kBT || vu.sizes().slice(0, 3) != at::IntArrayRef({B, T, H}) || (w.has_value() && w->sizes() != k.sizes()) ||
      (g.has_value() && g->sizes() != at::IntArrayRef({B, T, H})) ||
      (h0.has_value() && h0->sizes() != at::IntArrayRef({B, H, K, V})))
    return py::none();
  if (k.scalar_type() != vu.scalar_type() || (w.has_value() && w->scalar_type() != k.scalar_type()) ||
      !is_f32(g) || !is_f32(h0))
    return py::none();
  const int32_t code = dtype_code(k);
  if (code < 0) return py::none();
  const auto f32 = k.options().dtype(at::kFloat);
  at::Tensor hs = at::empty({B, T / kBT, H, K, V}, f32);
  c10::optional<at::Tensor> vn, ht;
  if (delta && want_vn) vn = at::empty_like(vu);
  if (want_ht) ht = at::empty({B, H, K, V}, f32);
  const int st = thm_chunk_fwd_h(k.data_ptr(), ptr(w), vu.data_ptr(), ptr(g), ptr(h0), hs.data_ptr(),
                                 vn.has_value() ? vn->data_ptr() : nullptr, ht.has_value() ? ht->data_ptr() : nullptr,
                                 B, T, H, K, V, (int32_t)kBT, code, delta ? THM_H_DELTA : 0, stream_of(dev));
  if (st != THM_OK) return py::int_(st);
  return py::make_tuple(hs, vn.has_value() ? py::cast(*vn) : py::none(), ht.has_value() ? py::cast(*ht) : py::none());
}

// chunk_fwd_o: o from q, k, v [B, T, H, K / V], g, h [B, T/64, H, K, V], scale.
py::object o(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const c10::optional<at::Tensor>& g,
             const at::Tensor& hs, double scale) {
  if (!q.is_cuda() || q.dim() != 4 || v.dim() != 4 || hs.dim() != 5) return py::none();
  const int dev = q.get_device();
  if (!ok(q, dev) || !ok(k, dev) || !ok(v, dev) || !ok_opt(g, dev) || !ok(hs, dev)) return py::none();
  const int64_t B = q.size(0), T = q.size(1), H = q.size(2), K = q.size(3), V = v.size(3);
  if (T % kBT || k.sizes() != q.sizes() || v.sizes().slice(0, 3) != at::IntArrayRef({B, T, H}) ||
      hs.sizes() != at::IntArrayRef({B, T / kBT, H, K, V}) ||
      (g.has_value() && g->sizes() != at::IntArrayRef({B, T, H})))
    return py::none();
  if (k.scalar_type() != q.scalar_type() || v.scalar_type() != q.scalar_type() || hs.scalar_type() != at::kFloat ||
      !is_f32(g))
    return py::none();
  const int32_t code = dtype_code(q);
  if (code < 0) return py::none();
  at::Tensor out = at::empty_like(v);
  const int st = thm_chunk_fwd_o(q.data_ptr(), k.data_ptr(), v.data_ptr(), ptr(g), hs.data_ptr(), out.data_ptr(),
                                 (float)scale, B, T, H, K, V, (int32_t)kBT, code, stream_of(dev));
  if (st != THM_OK) return py::int_(st);
  return py::cast(out);
}

}  // namespace

PYBIND11_MODULE(_fastpath, m) {
  m.doc() = "Host fast path of the custom_kernel wrappers (None: use the Python path; int: C status to raise)";
  m.def("conv1d", &conv1d, py::arg("x"), py::arg("weight"), py::arg("bias"), py::arg("activation"));
  m.def("wu", &wu, py::arg("k"), py::arg("v"), py::arg("beta"), py::arg("A"), py::arg("g"));
  m.def("h", &h, py::arg("k"), py::arg("w"), py::arg("vu"), py::arg("g"), py::arg("h0"), py::arg("delta"),
        py::arg("want_vn"), py::arg("want_ht"));
  m.def("o", &o, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("g"), py::arg("h"), py::arg("scale"));
}
