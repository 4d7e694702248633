// Tensor-level front door to the C ABI for eager callers, as a torch C++
// extension (flash_hog/_lib/_fhog_torch*.so, built by flash-hog_amd/build.py).
//
// It does in C++ what flash_hog/_hip.py's attention_fwd / attention_bwd /
// attention_bwdbwd do in Python (the same checks with the same messages, the
// same allocations, the caller's device made current around the call, the
// current stream of that device) and then calls the C-ABI entry point, so a
// call costs a few microseconds of host time instead of the Python wrapper's
// 9-20 us. That host time is what bounds an eager Hessian-vector product at
// short sequences, whose GPU work is shorter than the host's.
//
// The entry points are not linked: bind() receives their addresses from the
// library _hip.py loaded (which honours its FLASH_HOG_HIP_LIB override), and
// the Python exception class to raise for a non-zero status. _hip.py uses this
// module when it is built and falls back to its own wrappers when it is not;
// both reach the same kernels.
//
// attention() is dot_product_attention's eager autograd path in C++: two
// torch::autograd::Function nodes with the rules of
// flash_hog/torch/attention.py (the forward saving (q, k, v, L, O); its
// backward, itself differentiable once, saving (q, k, v, O, L, dO); the double
// backward with no cotangent for L and O), so that a Hessian-vector product
// runs no Python between the autograd engine and the kernels.
//
// The calls themselves (the *_core functions) touch no Python object: the
// autograd engine runs backward nodes on its own threads, without the GIL.
// They throw ArgError and StatusError; the Python-facing functions release the
// GIL around them and turn those into ValueError and the bound FlashHogError.
#include <ATen/core/Tensor.h>
#include <ATen/ops/empty.h>
#include <ATen/ops/empty_like.h>
#include <c10/core/DeviceGuard.h>
#include <c10/core/GradMode.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/autograd/custom_function.h>
#include <torch/csrc/utils/pybind.h>

#include <cstdint>
#include <sstream>
#include <stdexcept>
#include <string>
#include <tuple>

#include "flash_hog.h"

namespace py = pybind11;

namespace {

struct Api {
  decltype(&fhog_attention_fwd) fwd = nullptr;
  decltype(&fhog_attention_bwd) bwd = nullptr;
  decltype(&fhog_attention_bwdbwd) bwdbwd = nullptr;
  decltype(&fhog_last_error) last_error = nullptr;
  decltype(&fhog_status_string) status_string = nullptr;
  py::object error_cls;
};

Api& api() {
  static Api a;
  return a;
}

void bind(std::uintptr_t fwd, std::uintptr_t bwd, std::uintptr_t bwdbwd, std::uintptr_t last_error,
          std::uintptr_t status_string, py::object error_cls) {
  Api& a = api();
  a.fwd = reinterpret_cast<decltype(a.fwd)>(fwd);
  a.bwd = reinterpret_cast<decltype(a.bwd)>(bwd);
  a.bwdbwd = reinterpret_cast<decltype(a.bwdbwd)>(bwdbwd);
  a.last_error = reinterpret_cast<decltype(a.last_error)>(last_error);
  a.status_string = reinterpret_cast<decltype(a.status_string)>(status_string);
  a.error_cls = std::move(error_cls);
}

std::string shape_str(const at::Tensor& t) {
  std::ostringstream os;
  os << "(";
  for (int64_t i = 0; i < t.dim(); ++i) os << (i ? ", " : "") << t.size(i);
  os << (t.dim() == 1 ? ",)" : ")");
  return os.str();
}

std::string dtype_str(at::ScalarType s) {
  switch (s) {
    case at::kFloat: return "torch.float32";
    case at::kHalf: return "torch.float16";
    case at::kBFloat16: return "torch.bfloat16";
    default: return std::string("torch.") + c10::toString(s);
  }
}

std::string device_str(const at::Tensor& t) {
  std::ostringstream os;
  os << t.device();
  return os.str();
}

// A bad argument (ValueError in Python) and a non-zero C-ABI status
// (FlashHogError(status, message) in Python).
struct ArgError : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct StatusError : std::runtime_error {
  int status;
  StatusError(int s, const std::string& msg) : std::runtime_error(msg), status(s) {}
};

[[noreturn]] void value_error(const std::string& msg) { throw ArgError(msg); }

int dtype_code(at::ScalarType s) {
  switch (s) {
    case at::kFloat: return FHOG_DTYPE_F32;
    case at::kHalf: return FHOG_DTYPE_F16;
    case at::kBFloat16: return FHOG_DTYPE_BF16;
    default: value_error("unsupported dtype " + dtype_str(s));
  }
}

// Every tensor on the first one's GPU device, with dtype `dtype` unless it is
// None (_hip.py _check_inputs).
void check_inputs(std::initializer_list<std::pair<const char*, const at::Tensor*>> named,
                  c10::optional<at::ScalarType> dtype) {
  const at::Tensor* first = nullptr;
  for (const auto& [name, t] : named) {
    if (!t->is_cuda()) value_error(std::string(name) + " must be on a GPU device, got " + device_str(*t));
    if (!first) {
      first = t;
    } else if (t->get_device() != first->get_device()) {
      value_error(std::string(name) + " is on " + device_str(*t) + ", expected " + device_str(*first));
    }
    if (dtype && t->scalar_type() != *dtype)
      value_error(std::string(name) + " has dtype " + dtype_str(t->scalar_type()) + ", expected " +
                  dtype_str(*dtype));
  }
}

struct Dims {
  int B, Tq, Tk, N, Nk, H;
};

// (B, Tq, Tk, N, Nk, H) of q (B, Tq, N, H) and k (B, Tk, Nk, H) (_hip.py _dims).
Dims dims(const at::Tensor& q, const at::Tensor& k) {
  if (q.dim() != 4 || k.dim() != 4)
    value_error("expected (B, T, N, H) tensors, got q" + shape_str(q) + " k" + shape_str(k));
  if (k.size(0) != q.size(0) || k.size(3) != q.size(3))
    value_error("q" + shape_str(q) + " and k" + shape_str(k) + " disagree on batch or head_dim");
  if (k.size(2) == 0 || q.size(2) % k.size(2) != 0) {
    std::ostringstream os;
    os << "query heads (" << q.size(2) << ") must be a multiple of key/value heads (" << k.size(2) << ")";
    value_error(os.str());
  }
  dtype_code(q.scalar_type());
  for (int64_t s : q.sizes())
    if (s > INT32_MAX) value_error("q" + shape_str(q) + " has a dimension beyond the C ABI's int range");
  if (k.size(1) > INT32_MAX) value_error("k" + shape_str(k) + " has a dimension beyond the C ABI's int range");
  return {(int)q.size(0), (int)q.size(1), (int)k.size(1), (int)q.size(2), (int)k.size(2), (int)q.size(3)};
}

void expect(const char* name, const at::Tensor& t, at::IntArrayRef shape,
            c10::optional<at::ScalarType> dtype = c10::nullopt) {
  if (t.sizes() != shape) {
    std::ostringstream os;
    os << "(";
    for (size_t i = 0; i < shape.size(); ++i) os << (i ? ", " : "") << shape[i];
    os << (shape.size() == 1 ? ",)" : ")");
    value_error(std::string(name) + " has shape " + shape_str(t) + ", expected " + os.str());
  }
  if (dtype && t.scalar_type() != *dtype)
    value_error(std::string(name) + " has dtype " + dtype_str(t.scalar_type()) + ", expected " + dtype_str(*dtype));
}

at::Tensor contig(const at::Tensor& t) { return t.is_contiguous() ? t : t.contiguous(); }

// The current stream of t's device (torch's, as _hip.py takes it).
fhog_stream_t current_stream(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// The message comes from the calling thread's fhog_last_error.
void check_status(int status) {
  if (status == FHOG_OK) return;
  const Api& a = api();
  std::string msg = a.last_error();
  if (msg.empty()) msg = a.status_string(status);
  throw StatusError(status, msg);
}

void require_bound(const void* fn) {
  if (!fn) throw std::runtime_error("_fhog_torch.bind() has not been called");
}

std::tuple<at::Tensor, at::Tensor> fwd_core(const at::Tensor& q_, const at::Tensor& k_, const at::Tensor& v_,
                                            int causal, double scale) {
  require_bound((const void*)api().fwd);
  check_inputs({{"q", &q_}, {"k", &k_}, {"v", &v_}}, q_.scalar_type());
  const Dims d = dims(q_, k_);
  expect("v", v_, k_.sizes());
  const at::Tensor q = contig(q_), k = contig(k_), v = contig(v_);
  at::Tensor o = at::empty_like(q);
  at::Tensor lse = at::empty({(int64_t)d.B, (int64_t)d.N, (int64_t)d.Tq}, q.options().dtype(at::kFloat));
  c10::DeviceGuard guard(q.device());
  const int status = api().fwd(current_stream(q), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                               lse.data_ptr<float>(), d.B, d.Tq, d.Tk, d.N, d.Nk, d.H, dtype_code(q.scalar_type()),
                               causal, (float)scale);
  check_status(status);
  return {o, lse};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> bwd_core(
    const at::Tensor& q_, const at::Tensor& k_, const at::Tensor& v_, const at::Tensor& o_, const at::Tensor& dout_,
    const at::Tensor& lse_, int causal, double scale) {
  require_bound((const void*)api().bwd);
  check_inputs({{"q", &q_}, {"k", &k_}, {"v", &v_}, {"o", &o_}, {"dout", &dout_}}, q_.scalar_type());
  check_inputs({{"q", &q_}, {"lse", &lse_}}, c10::nullopt);
  const Dims d = dims(q_, k_);
  expect("v", v_, k_.sizes());
  expect("o", o_, q_.sizes());
  expect("dout", dout_, q_.sizes());
  expect("lse", lse_, {(int64_t)d.B, (int64_t)d.N, (int64_t)d.Tq}, at::kFloat);
  const at::Tensor q = contig(q_), k = contig(k_), v = contig(v_), o = contig(o_), dout = contig(dout_),
                   lse = contig(lse_);
  at::Tensor dq = at::empty_like(q), dk = at::empty_like(k), dv = at::empty_like(v);
  at::Tensor delta = at::empty({(int64_t)d.B, (int64_t)d.N, (int64_t)d.Tq}, q.options().dtype(at::kFloat));
  c10::DeviceGuard guard(q.device());
  const int status =
      api().bwd(current_stream(q), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), dout.data_ptr(),
                lse.data_ptr<float>(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), delta.data_ptr<float>(), d.B,
                d.Tq, d.Tk, d.N, d.Nk, d.H, dtype_code(q.scalar_type()), causal, (float)scale);
  check_status(status);
  return {dq, dk, dv, delta};
}

// dq2, dk2, dv2, ddo and the (3, B, N, Tq) fp32 row statistics D, dD, B.
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor> bwdbwd_core(
    const at::Tensor& q_, const at::Tensor& k_, const at::Tensor& v_, const at::Tensor& o_, const at::Tensor& dout_,
    const at::Tensor& ddq_, const at::Tensor& ddk_, const at::Tensor& ddv_, const at::Tensor& lse_, int causal,
    double scale) {
  require_bound((const void*)api().bwdbwd);
  check_inputs({{"q", &q_}, {"k", &k_}, {"v", &v_}, {"o", &o_}, {"dout", &dout_}, {"ddq", &ddq_}, {"ddk", &ddk_},
                {"ddv", &ddv_}},
               q_.scalar_type());
  check_inputs({{"q", &q_}, {"lse", &lse_}}, c10::nullopt);
  const Dims d = dims(q_, k_);
  expect("v", v_, k_.sizes());
  expect("o", o_, q_.sizes());
  expect("dout", dout_, q_.sizes());
  expect("ddq", ddq_, q_.sizes());
  expect("ddk", ddk_, k_.sizes());
  expect("ddv", ddv_, k_.sizes());
  expect("lse", lse_, {(int64_t)d.B, (int64_t)d.N, (int64_t)d.Tq}, at::kFloat);
  const at::Tensor q = contig(q_), k = contig(k_), v = contig(v_), o = contig(o_), dout = contig(dout_),
                   ddq = contig(ddq_), ddk = contig(ddk_), ddv = contig(ddv_), lse = contig(lse_);
  at::Tensor dq2 = at::empty_like(q), dk2 = at::empty_like(k), dv2 = at::empty_like(v), ddo = at::empty_like(dout);
  at::Tensor stats = at::empty({3, (int64_t)d.B, (int64_t)d.N, (int64_t)d.Tq}, q.options().dtype(at::kFloat));
  float* st = stats.data_ptr<float>();
  const int64_t n_stat = (int64_t)d.B * d.N * d.Tq;
  c10::DeviceGuard guard(q.device());
  const int status = api().bwdbwd(current_stream(q), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                  dout.data_ptr(), ddq.data_ptr(), ddk.data_ptr(), ddv.data_ptr(),
                                  lse.data_ptr<float>(), dq2.data_ptr(), dk2.data_ptr(), dv2.data_ptr(),
                                  ddo.data_ptr(), st, st + n_stat, st + 2 * n_stat, d.B, d.Tq, d.Tk, d.N, d.Nk, d.H,
                                  dtype_code(q.scalar_type()), causal, (float)scale);
  check_status(status);
  return {dq2, dk2, dv2, ddo, stats};
}

// ------------------------------------------------------------------ autograd

using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

// Refuses a third derivative as the once_differentiable double backward of
// flash_hog/torch/attention.py does. Under create_graph, with cotangents that
// require grad, the double backward's results are detached, marked as
// requiring grad and passed through this node (as copies), whose backward
// raises: a backward() through them raises, while a grad() with respect to
// the inputs finds no path through them.
struct NoThirdOrder : public torch::autograd::Function<NoThirdOrder> {
  static variable_list forward(AutogradContext*, const at::Tensor& dq2, const at::Tensor& dk2,
                               const at::Tensor& dv2, const at::Tensor& ddo) {
    return {dq2.clone(), dk2.clone(), dv2.clone(), ddo.clone()};
  }
  static variable_list backward(AutogradContext*, variable_list) {
    throw std::runtime_error("trying to differentiate twice a function that was marked with @once_differentiable");
  }
};

// Primal (q, k, v, O, L, dO) -> (dQ, dK, dV), differentiable once in q, k, v
// and dO: _DotProductAttentionBwd (the rule
// dot_product_attention_bwd_rule_fwd_rule and its rule
// dot_product_attention_bwd_rule_bwd_rule).
struct AttentionBwdFn : public torch::autograd::Function<AttentionBwdFn> {
  static variable_list forward(AutogradContext* ctx, int64_t causal, double scale, const at::Tensor& q,
                               const at::Tensor& k, const at::Tensor& v, const at::Tensor& lse, const at::Tensor& o,
                               const at::Tensor& g) {
    auto [dq, dk, dv, delta] = bwd_core(q, k, v, o, g, lse, (int)causal, scale);
    ctx->save_for_backward({q, k, v, o, lse, g});
    ctx->saved_data["causal"] = causal;
    ctx->saved_data["scale"] = scale;
    return {dq, dk, dv};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const variable_list r = ctx->get_saved_variables();  // q, k, v, O, L, dO
    auto [dq2, dk2, dv2, ddo, stats] =
        bwdbwd_core(r[0], r[1], r[2], r[3], r[5], grads[0], grads[1], grads[2], r[4],
                    (int)ctx->saved_data["causal"].toInt(), ctx->saved_data["scale"].toDouble());
    if (c10::GradMode::is_enabled() &&
        (grads[0].requires_grad() || grads[1].requires_grad() || grads[2].requires_grad())) {
      auto mark = [](const at::Tensor& t) { return t.detach().requires_grad_(true); };
      const variable_list w = NoThirdOrder::apply(mark(dq2), mark(dk2), mark(dv2), mark(ddo));
      dq2 = w[0], dk2 = w[1], dv2 = w[2], ddo = w[3];
    }
    // no cotangent for L and O (flash_hog/jax/_attention_impl.py:278-303)
    return {at::Tensor(), at::Tensor(), dq2, dk2, dv2, at::Tensor(), at::Tensor(), ddo};
  }
};

// Primal (q, k, v) -> (O, L), L not differentiable: _DotProductAttention (the
// rule dot_product_attention_fwd_rule and its rule
// dot_product_attention_bwd_rule, through AttentionBwdFn).
struct AttentionFn : public torch::autograd::Function<AttentionFn> {
  static variable_list forward(AutogradContext* ctx, const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                               int64_t causal, double scale) {
    auto [o, lse] = fwd_core(q, k, v, (int)causal, scale);
    ctx->save_for_backward({q, k, v, lse, o});
    ctx->saved_data["causal"] = causal;
    ctx->saved_data["scale"] = scale;
    ctx->mark_non_differentiable({lse});
    return {o, lse};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const variable_list r = ctx->get_saved_variables();  // q, k, v, L, O
    // O enters the first backward as a constant: the double backward returns
    // no cotangent for it, and detaching it keeps this node out of a second
    // derivative's graph.
    const variable_list d = AttentionBwdFn::apply(ctx->saved_data["causal"].toInt(),
                                                  ctx->saved_data["scale"].toDouble(), r[0], r[1], r[2], r[3],
                                                  r[4].detach(), grads[0]);
    return {d[0], d[1], d[2], at::Tensor(), at::Tensor()};
  }
};

// ----------------------------------------------------------- Python-facing

// Runs f without the GIL and raises its errors as Python exceptions.
template <class F>
auto py_call(F&& f) {
  try {
    py::gil_scoped_release nogil;
    return f();
  } catch (const ArgError& e) {
    throw py::value_error(e.what());
  } catch (const StatusError& e) {
    PyErr_SetObject(api().error_cls.ptr(), py::make_tuple(e.status, std::string(e.what())).ptr());
    throw py::error_already_set();
  }
}

std::tuple<at::Tensor, at::Tensor> attention_fwd(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                                 int causal, double scale) {
  require_bound((const void*)api().fwd);
  return py_call([&] { return fwd_core(q, k, v, causal, scale); });
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> attention_bwd(
    const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& o, const at::Tensor& dout,
    const at::Tensor& lse, int causal, double scale) {
  require_bound((const void*)api().bwd);
  return py_call([&] { return bwd_core(q, k, v, o, dout, lse, causal, scale); });
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor> attention_bwdbwd(
    const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& o, const at::Tensor& dout,
    const at::Tensor& ddq, const at::Tensor& ddk, const at::Tensor& ddv, const at::Tensor& lse, int causal,
    double scale) {
  require_bound((const void*)api().bwdbwd);
  return py_call([&] { return bwdbwd_core(q, k, v, o, dout, ddq, ddk, ddv, lse, causal, scale); });
}

// O of attention(q, k, v) with the autograd nodes above (when q, k or v
// require grad and grad mode is on).
at::Tensor attention(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, int64_t causal, double scale) {
  require_bound((const void*)api().bwdbwd);
  return py_call([&] { return AttentionFn::apply(q, k, v, causal, scale)[0]; });
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "Tensor-level calls of the Flash-HOG C ABI (see flash_hog/_hip.py)";
  m.def("bind", &bind, "bind(fwd, bwd, bwdbwd, last_error, status_string, error_cls): entry-point addresses");
  m.def("attention_fwd", &attention_fwd);
  m.def("attention_bwd", &attention_bwd);
  m.def("attention_bwdbwd", &attention_bwdbwd);
  m.def("attention", &attention, "attention(q, k, v, causal, scale) -> O, differentiable twice");
}
