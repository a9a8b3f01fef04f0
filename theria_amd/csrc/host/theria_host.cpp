// Python binding of the hot C ABI entry points (theria_sdpa_fwd, _bwd, _jvp, _bwd_bwd) for torch tensors.
//
// The autograd operator calls these once per forward, backward, JVP and double backward. Building the
// theria_tensor_t views, the output tensors and the stream handle here costs about a microsecond per call,
// against ~3 us per tensor view through ctypes from Python (a double backward passes fifteen). The semantics are
// those of theria_amd/_ops.py (same argument meaning, same output dtypes, same error types): shape and device
// mismatches raise AssertionError, as the reference's guards do (theria/attention/triton_sdpa_backward.py:23-103),
// and the C ABI's own contract errors keep their status (THERIA_ERR_CONTRACT -> AssertionError,
// THERIA_ERR_HIP -> RuntimeError). Dtype and 4-D checks of the primary inputs stay in Python
// (_ops.check_inputs), which runs once per autograd operator.
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include <optional>
#include <string>

#include "theria_sdpa.h"

namespace py = pybind11;

namespace {

using OptT = std::optional<at::Tensor>;

[[noreturn]] void raise_assertion(const std::string& msg) {
  PyErr_SetString(PyExc_AssertionError, msg.c_str());
  throw py::error_already_set();
}

void need(bool ok, const char* msg) {
  if (!ok) raise_assertion(msg);
}

void check_rc(int rc, const char* what) {
  if (rc == THERIA_OK) return;
  std::string msg = std::string(what) + ": " + theria_last_error();
  if (rc == THERIA_ERR_CONTRACT) raise_assertion(msg);
  PyErr_SetString(PyExc_RuntimeError, msg.c_str());
  throw py::error_already_set();
}

// The tensor a torch.func wrapper holds (SDPAOp.jvp receives its saved tensors wrapped under torch.func.jvp).
// A wrapper has no storage of its own; such calls are rare, so torch's own Python helpers unwrap it. The helpers
// are looked up once and deliberately never released: a static py::object would be destroyed after the
// interpreter has shut down, and its reference-count decrement would then crash the process at exit.
at::Tensor plain(const at::Tensor& t) {
  if (t.has_storage()) return t;
  static py::object* is_wrapped = nullptr;
  static py::object* unwrap = nullptr;
  if (!unwrap) {
    const py::object ft = py::module_::import("torch._C._functorch");
    is_wrapped = new py::object(ft.attr("is_functorch_wrapped_tensor"));
    unwrap = new py::object(ft.attr("get_unwrapped"));
  }
  at::Tensor cur = t;
  while (!cur.has_storage() && (*is_wrapped)(cur).cast<bool>()) cur = (*unwrap)(cur).cast<at::Tensor>();
  return cur;
}

// The kernels need a contiguous last dimension; any other strides (broadcast rows included) are fine.
at::Tensor rowmajor(at::Tensor t) {
  t = plain(t);
  if (t.size(-1) > 1 && t.stride(-1) != 1) t = t.contiguous();
  return t;
}

// A (B, H, rows, D) operand in the compute dtype on q's device.
at::Tensor like_rows(const at::Tensor& t_in, const at::Tensor& q, int64_t rows, const char* msg) {
  const at::Tensor t = plain(t_in);
  need(t.dim() == 4 && t.size(0) == q.size(0) && t.size(1) == q.size(1) && t.size(2) == rows &&
           t.size(3) == q.size(3) && t.device() == q.device(),
       msg);
  return rowmajor(t.scalar_type() == q.scalar_type() ? t : t.to(q.scalar_type()));
}

OptT like_rows(const OptT& t, const at::Tensor& q, int64_t rows, const char* msg) {
  if (!t) return std::nullopt;
  return like_rows(*t, q, rows, msg);
}

at::Tensor rowstat(const at::Tensor& t, const at::Tensor& q, const char* msg) {
  need(t.scalar_type() == at::kFloat && t.numel() == q.size(0) * q.size(1) * q.size(2) && t.device() == q.device(),
       msg);
  return plain(t).contiguous();
}

// Views and pointers are taken from the plain tensor: under a torch.func transform the outputs allocated here are
// wrappers too (at::empty returns one), and they are returned as such while the kernels write the storage.
theria_tensor_t view(const at::Tensor& t_in) {
  const at::Tensor t = plain(t_in);
  return {t.data_ptr(), t.stride(0), t.stride(1), t.stride(2)};
}
theria_tensor_t view(const OptT& t) { return t ? view(*t) : theria_tensor_t{nullptr, 0, 0, 0}; }
float* fptr(const at::Tensor& t) { return plain(t).data_ptr<float>(); }
float* fptr(const OptT& t) { return t ? fptr(*t) : nullptr; }

int32_t dtype_code(at::ScalarType st) {
  switch (st) {
    case at::kFloat: return THERIA_DTYPE_F32;
    case at::kHalf: return THERIA_DTYPE_F16;
    case at::kBFloat16: return THERIA_DTYPE_BF16;
    default: raise_assertion(std::string("Unsupported dtype: ") + c10::toString(st));
  }
}

theria_sdpa_problem_t problem(const at::Tensor& q, const at::Tensor& k, double scale, bool causal) {
  return {dtype_code(q.scalar_type()), (int32_t)q.size(0), (int32_t)q.size(1), (int32_t)q.size(2),
          (int32_t)k.size(2),           (int32_t)q.size(3), (float)scale,       causal ? 1 : 0};
}

void* stream_of(const at::Tensor& q) { return c10::hip::getCurrentHIPStream(q.get_device()).stream(); }

// (q, k, v) in row-major layout with matching shapes (dtype and rank were checked in Python).
void kv_shapes(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v) {
  need(k.size(0) == q.size(0) && k.size(1) == q.size(1) && k.size(3) == q.size(3),
       "k must have shape (B,H,M,D) with D matching q");
  need(v.size(0) == q.size(0) && v.size(1) == q.size(1) && v.size(2) == k.size(2) && v.size(3) == q.size(3),
       "v must have shape (B,H,M,D) matching k");
  need(k.device() == q.device() && v.device() == q.device(), "q, k and v must be on one device");
}

py::tuple fwd(at::Tensor q, at::Tensor k, at::Tensor v, double scale, bool causal, bool out_fp32, bool stats) {
  q = rowmajor(q), k = rowmajor(k), v = rowmajor(v);
  kv_shapes(q, k, v);
  const c10::hip::HIPGuard guard(q.get_device());
  const auto o = at::empty(q.sizes(), q.options().dtype(out_fp32 ? at::kFloat : q.scalar_type()));
  const auto f = q.options().dtype(at::kFloat);
  const auto lse = at::empty({q.size(0), q.size(1), q.size(2)}, f);
  OptT m, l;
  if (stats) m = at::empty_like(lse), l = at::empty_like(lse);
  const auto p = problem(q, k, scale, causal);
  const auto tq = view(q), tk = view(k), tv = view(v), to = view(o);
  check_rc(theria_sdpa_fwd(&p, &tq, &tk, &tv, &to, out_fp32 ? 1 : 0, fptr(lse), fptr(m), fptr(l),
                           stream_of(q)),
           "theria_sdpa_fwd");
  return py::make_tuple(o, lse, m ? py::cast(*m) : py::none(), l ? py::cast(*l) : py::none());
}

// dQ, dK, dV and the row term, as _ops.bwd. out: (dq, dk, dv) to write instead of new tensors.
py::tuple bwd(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor o, const at::Tensor& lse_in,
              const at::Tensor& dout_in, double scale, bool causal, bool need_dq, bool need_dk,
              const std::optional<std::vector<at::Tensor>>& out) {
  q = rowmajor(q), k = rowmajor(k), v = rowmajor(v);
  kv_shapes(q, k, v);
  const int64_t T = q.size(2), M = k.size(2);
  const auto dout = like_rows(dout_in, q, T, "dout must have shape (B,H,T,D)");
  o = rowmajor(o);
  need(o.dim() == 4 && o.sizes() == q.sizes(), "o must have shape (B,H,T,D)");
  const bool o_f32 = o.scalar_type() == at::kFloat && q.scalar_type() != at::kFloat;
  if (!o_f32 && o.scalar_type() != q.scalar_type()) o = o.to(q.scalar_type());
  const auto lse = rowstat(lse_in, q, "lse must be a float32 (B,H,T) tensor on q's device");
  const c10::hip::HIPGuard guard(q.get_device());
  const auto delta = at::empty({q.size(0), q.size(1), T}, q.options().dtype(at::kFloat));
  OptT dq, dk;
  at::Tensor dv;
  if (out) {
    need(out->size() == 3, "out must hold (dq, dk, dv)");
    const int64_t rows[3] = {T, M, M};
    for (int i = 0; i < 3; ++i) {
      const auto& t = (*out)[i];
      need(t.dim() == 4 && t.size(0) == q.size(0) && t.size(1) == q.size(1) && t.size(2) == rows[i] &&
               t.size(3) == q.size(3) && t.scalar_type() == q.scalar_type() && t.device() == q.device() &&
               t.stride(3) == 1,
           "out tensors must match q's dtype and device, shaped like (dq, dk, dv), last dimension contiguous");
    }
    dq = (*out)[0], dk = (*out)[1], dv = (*out)[2];
  } else {
    if (need_dq) dq = at::empty(q.sizes(), q.options());
    if (need_dk) dk = at::empty({q.size(0), q.size(1), M, q.size(3)}, q.options());
    dv = at::empty({q.size(0), q.size(1), M, q.size(3)}, q.options());
  }
  const auto p = problem(q, k, scale, causal);
  const auto tq = view(q), tk = view(k), tv = view(v), to = view(o), tdo = view(dout), tdq = view(dq), tdk = view(dk),
             tdv = view(dv);
  check_rc(theria_sdpa_bwd(&p, &tq, &tk, &tv, &to, o_f32 ? 1 : 0, &tdo, fptr(lse),
                           fptr(delta), &tdq, &tdk, &tdv, stream_of(q)),
           "theria_sdpa_bwd");
  return py::make_tuple(dq ? py::cast(*dq) : py::none(), dk ? py::cast(*dk) : py::none(), dv, delta);
}

at::Tensor jvp(at::Tensor q, at::Tensor k, at::Tensor v, OptT o, const at::Tensor& lse_in, const OptT& tq_in,
               const OptT& tk_in, const OptT& tv_in, double scale, bool causal, bool normalize) {
  q = rowmajor(q), k = rowmajor(k), v = rowmajor(v);
  kv_shapes(q, k, v);
  const int64_t T = q.size(2), M = k.size(2);
  const auto tq = like_rows(tq_in, q, T, "tq must have shape (B,H,T,D)");
  const auto tk = like_rows(tk_in, q, M, "tk must have shape (B,H,M,D)");
  const auto tv = like_rows(tv_in, q, M, "tv must have shape (B,H,M,D)");
  if (o) {  // a float32 O of a low-precision op is rebuilt at full precision inside the kernel instead
    if (o->scalar_type() != q.scalar_type())
      o = std::nullopt;
    else
      o = like_rows(*o, q, T, "o must have shape (B,H,T,D)");
  }
  const auto lse = rowstat(lse_in, q, "lse must be a float32 (B,H,T) tensor on q's device");
  const c10::hip::HIPGuard guard(q.get_device());
  const auto out = at::empty(q.sizes(), q.options());
  const auto p = problem(q, k, scale, causal);
  const auto vq = view(q), vk = view(k), vv = view(v), vo = view(o), vtq = view(tq), vtk = view(tk), vtv = view(tv),
             vout = view(out);
  check_rc(theria_sdpa_jvp(&p, &vq, &vk, &vv, &vo, fptr(lse), &vtq, &vtk, &vtv, &vout,
                           normalize ? 1 : 0, stream_of(q)),
           "theria_sdpa_jvp");
  return out;
}

// (G_Q, G_K, G_V, G_dO) as _ops.bwd_bwd; delta is not read by the library and may be None.
py::tuple bwd_bwd(at::Tensor q, at::Tensor k, at::Tensor v, OptT o, const at::Tensor& dout_in,
                  const at::Tensor& lse_in, const OptT& gq_in, const OptT& gk_in, const OptT& gv_in, double scale,
                  bool causal, bool noalloc, const std::optional<std::vector<at::Tensor>>& out) {
  q = rowmajor(q), k = rowmajor(k), v = rowmajor(v);
  kv_shapes(q, k, v);
  const int64_t B = q.size(0), H = q.size(1), T = q.size(2), M = k.size(2), D = q.size(3);
  const auto dout = like_rows(dout_in, q, T, "dout must have shape (B,H,T,D)");
  const auto gq = like_rows(gq_in, q, T, "gq must have shape (B,H,T,D)");
  const auto gk = like_rows(gk_in, q, M, "gk must have shape (B,H,M,D)");
  const auto gv = like_rows(gv_in, q, M, "gv must have shape (B,H,M,D)");
  if (o) {
    if (o->scalar_type() != q.scalar_type())
      o = std::nullopt;
    else
      o = like_rows(*o, q, T, "o must have shape (B,H,T,D)");
  }
  const auto lse = rowstat(lse_in, q, "lse must be a float32 (B,H,T) tensor on q's device");
  const c10::hip::HIPGuard guard(q.get_device());
  at::Tensor oq, ok, ov;
  if (out) {
    need(out->size() == 3, "out must hold (out_gq, out_gk, out_gv)");
    const int64_t rows[3] = {T, M, M};
    for (int i = 0; i < 3; ++i) {
      const auto& t = (*out)[i];
      need(t.dim() == 4 && t.size(0) == B && t.size(1) == H && t.size(2) == rows[i] && t.size(3) == D &&
               t.scalar_type() == q.scalar_type() && t.device() == q.device() && t.stride(3) == 1,
           "out tensors must match q's dtype and device, shaped like (gq, gk, gv), last dimension contiguous");
    }
    oq = (*out)[0], ok = (*out)[1], ov = (*out)[2];
  } else {
    oq = at::empty(q.sizes(), q.options());
    ok = at::empty({B, H, M, D}, q.options());
    ov = at::empty({B, H, M, D}, q.options());
  }
  const auto odo = at::empty(q.sizes(), q.options());
  const auto p = problem(q, k, scale, causal);
  const auto vq = view(q), vk = view(k), vv = view(v), vo = view(o), vdo = view(dout), vgq = view(gq), vgk = view(gk),
             vgv = view(gv), voq = view(oq), vok = view(ok), vov = view(ov), vodo = view(odo);
  int rc;
  if (noalloc) {
    rc = theria_sdpa_bwd_bwd_noalloc(&p, &vq, &vk, &vv, &vo, &vdo, fptr(lse), nullptr, &vgq, &vgk, &vgv,
                                     &voq, &vok, &vov, &vodo, stream_of(q));
    check_rc(rc, "theria_sdpa_bwd_bwd_noalloc");
  } else {
    const auto ws = at::empty({5 * B * H * T}, q.options().dtype(at::kFloat));
    rc = theria_sdpa_bwd_bwd(&p, &vq, &vk, &vv, &vo, &vdo, fptr(lse), nullptr, &vgq, &vgk, &vgv, &voq,
                             &vok, &vov, &vodo, fptr(ws), stream_of(q));
    check_rc(rc, "theria_sdpa_bwd_bwd");
  }
  return py::make_tuple(oq, ok, ov, odo);
}

}  // namespace

PYBIND11_MODULE(_theria_host, m) {
  m.doc() = "torch-tensor binding of the hot C ABI entry points of libtheria_sdpa.so";
  m.def("abi_version", &theria_abi_version);
  m.def("fwd", &fwd, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("scale"), py::arg("causal"),
        py::arg("out_fp32"), py::arg("stats"));
  m.def("bwd", &bwd, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("o"), py::arg("lse"), py::arg("dout"),
        py::arg("scale"), py::arg("causal"), py::arg("need_dq"), py::arg("need_dk"), py::arg("out"));
  m.def("jvp", &jvp, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("o"), py::arg("lse"), py::arg("tq"),
        py::arg("tk"), py::arg("tv"), py::arg("scale"), py::arg("causal"), py::arg("normalize"));
  m.def("bwd_bwd", &bwd_bwd, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("o"), py::arg("dout"),
        py::arg("lse"), py::arg("gq"), py::arg("gk"), py::arg("gv"), py::arg("scale"), py::arg("causal"),
        py::arg("noalloc"), py::arg("out"));
}
