// Autograd nodes of the fused DWT chains in C++ (a torch extension): the same transforms as
// dwt.py's _AnalysisChain / _SynthesisChain (each the other's backward, reference
// src/fdwt/dwt.py:36-82), for chains that run as one launch.  Python-level Function objects
// cost tens of microseconds per call and per backward node (the engine's device thread takes
// the GIL for each); here a node costs a few.  The kernels are the C ABI of libfdwt_hip.so,
// whose entry points the Python loader hands over as addresses (set_entry_points), so this
// module does not link against it.  Launches go to torch's current HIP stream.

#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <vector>

namespace {

typedef int (*AnalysisFnPtr)(const void*, void* const*, void*, const void*, const void*, int64_t,
                             const int64_t*, const int64_t*, int32_t, int32_t, int32_t, int32_t,
                             int32_t, void*);
typedef int (*SynthesisFnPtr)(const void*, const void* const*, void*, const void*, const void*,
                              int64_t, const int64_t*, const int64_t*, int32_t, int32_t, int32_t,
                              int32_t, int32_t, void*);
typedef const char* (*ErrorFnPtr)(int);

AnalysisFnPtr g_analysis = nullptr;
SynthesisFnPtr g_synthesis = nullptr;
ErrorFnPtr g_error = nullptr;

void set_entry_points(int64_t analysis, int64_t synthesis, int64_t error) {
  g_analysis = reinterpret_cast<AnalysisFnPtr>(analysis);
  g_synthesis = reinterpret_cast<SynthesisFnPtr>(synthesis);
  g_error = reinterpret_cast<ErrorFnPtr>(error);
}

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return 0;
    case at::kDouble: return 1;
    case at::kHalf: return 2;
    case at::kBFloat16: return 3;
    default: TORCH_CHECK(false, "unsupported dtype ", t);
  }
}

void check(int rc, const char* what) {
  TORCH_CHECK(rc == 0, what, ": ", g_error ? g_error(rc) : "error", " (code ", rc, ")");
}

void* stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

std::vector<int64_t> reversed(const std::vector<int64_t>& v) {
  return std::vector<int64_t>(v.rbegin(), v.rend());
}

// Levels 0 .. J-1 of an analysis chain on x (..., n_in[0]): details d_0 .. d_{J-1}, then a_J,
// each shaped (..., n).  x's dtype is the storage dtype, h0 / h1 the compute-dtype taps.
std::vector<at::Tensor> analysis_run(const at::Tensor& x_, const at::Tensor& h0,
                                     const at::Tensor& h1, int64_t mode, int64_t off,
                                     const std::vector<int64_t>& n_in,
                                     const std::vector<int64_t>& n_out) {
  TORCH_CHECK(g_analysis, "fdwt: entry points not set");
  TORCH_CHECK(x_.is_cuda(), "pytorch_morlet_fdwt_amd runs on ROCm GPU tensors only");
  const at::Tensor x = x_.contiguous();
  const int J = (int)n_in.size();
  std::vector<int64_t> shape(x.sizes().begin(), x.sizes().end());
  const int64_t R = shape.back() ? x.numel() / shape.back() : 0;
  std::vector<at::Tensor> outs;
  outs.reserve(J + 1);
  std::vector<void*> ptrs(J);
  for (int l = 0; l < J; ++l) {
    shape.back() = n_out[l];
    outs.push_back(at::empty(shape, x.options()));
    ptrs[l] = outs.back().data_ptr();
  }
  shape.back() = n_out[J - 1];
  outs.push_back(at::empty(shape, x.options()));
  if (R)
    check(g_analysis(x.data_ptr(), ptrs.data(), outs.back().data_ptr(), h0.data_ptr(),
                     h1.data_ptr(), R, n_in.data(), n_out.data(), J, (int32_t)h0.numel(),
                     (int32_t)mode, (int32_t)off, dtype_code(x.scalar_type()), stream_of(x)),
          "fdwt_analysis_chain");
  return outs;
}

// Levels (coarsest first) of a synthesis chain from the low band a and the high bands ds (an
// undefined tensor is a band of zeros); the output is shaped (..., n_out[-1]).
at::Tensor synthesis_run(const at::Tensor& h0, const at::Tensor& h1, int64_t mode, int64_t off,
                         const std::vector<int64_t>& nc, const std::vector<int64_t>& n_out,
                         const at::Tensor& a, const std::vector<at::Tensor>& ds) {
  TORCH_CHECK(g_synthesis, "fdwt: entry points not set");
  const int K = (int)nc.size();
  const at::Tensor* ref = a.defined() ? &a : nullptr;
  for (int k = 0; !ref && k < K; ++k)
    if (ds[k].defined()) ref = &ds[k];
  TORCH_CHECK(ref, "fdwt: synthesis of no bands");
  TORCH_CHECK(ref->is_cuda(), "pytorch_morlet_fdwt_amd runs on ROCm GPU tensors only");
  std::vector<at::Tensor> keep;  // contiguous copies that must outlive the launch
  keep.reserve(K + 1);
  auto contig = [&](const at::Tensor& t) -> const void* {
    if (!t.defined()) return nullptr;
    TORCH_CHECK(t.is_cuda(), "pytorch_morlet_fdwt_amd runs on ROCm GPU tensors only");
    keep.push_back(t.contiguous());
    return keep.back().data_ptr();
  };
  const void* ap = contig(a);
  std::vector<const void*> dp(K);
  for (int k = 0; k < K; ++k) dp[k] = contig(ds[k]);
  std::vector<int64_t> shape(ref->sizes().begin(), ref->sizes().end());
  const int64_t R = shape.back() ? ref->numel() / shape.back() : 0;
  shape.back() = n_out[K - 1];
  at::Tensor out = at::empty(shape, ref->options());
  if (R)
    check(g_synthesis(ap, dp.data(), out.data_ptr(), h0.data_ptr(), h1.data_ptr(), R, nc.data(),
                      n_out.data(), K, (int32_t)h0.numel(), (int32_t)mode, (int32_t)off,
                      dtype_code(ref->scalar_type()), stream_of(*ref)),
          "fdwt_synthesis_chain");
  return out;
}

using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

struct SynthesisChain;

// (d_0, ..., d_{J-1}, a_J) = A x; backward: the synthesis chain with the transposed levels
struct AnalysisChain : public torch::autograd::Function<AnalysisChain> {
  static variable_list forward(AutogradContext* ctx, const at::Tensor& x, const at::Tensor& h0,
                               const at::Tensor& h1, int64_t mode, int64_t off,
                               std::vector<int64_t> n_in, std::vector<int64_t> n_out) {
    ctx->set_materialize_grads(false);  // unused outputs: no gradient tensors of zeros
    ctx->save_for_backward({h0, h1});
    ctx->saved_data["mode"] = mode;
    ctx->saved_data["off"] = off;
    ctx->saved_data["n_in"] = n_in;
    ctx->saved_data["n_out"] = n_out;
    return analysis_run(x, h0, h1, mode, off, n_in, n_out);
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads);
};

// y = A^T (a, ds); backward: the analysis chain with the transposed levels
struct SynthesisChain : public torch::autograd::Function<SynthesisChain> {
  static variable_list forward(AutogradContext* ctx, const at::Tensor& h0, const at::Tensor& h1,
                               int64_t mode, int64_t off, std::vector<int64_t> nc,
                               std::vector<int64_t> n_out, const at::Tensor& a,
                               at::TensorList ds) {
    ctx->set_materialize_grads(false);
    ctx->save_for_backward({h0, h1});
    ctx->saved_data["mode"] = mode;
    ctx->saved_data["off"] = off;
    ctx->saved_data["nc"] = nc;
    ctx->saved_data["n_out"] = n_out;
    ctx->saved_data["n_ds"] = (int64_t)ds.size();
    return {synthesis_run(h0, h1, mode, off, nc, n_out, a, ds.vec())};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const auto saved = ctx->get_saved_variables();
    const int64_t mode = ctx->saved_data["mode"].toInt(), off = ctx->saved_data["off"].toInt();
    const auto nc = ctx->saved_data["nc"].toIntVector();
    const auto n_out = ctx->saved_data["n_out"].toIntVector();
    const int64_t n_ds = ctx->saved_data["n_ds"].toInt();
    const at::Tensor& gy = grads[0];
    variable_list res(6);  // h0, h1, mode, off, nc, n_out
    if (!gy.defined()) {
      res.resize(7 + n_ds);
      return res;
    }
    variable_list outs;
    if (torch::GradMode::is_enabled())  // the backward is differentiated: a graph node
      outs = AnalysisChain::apply(gy, saved[0], saved[1], mode, off, reversed(n_out),
                                  reversed(nc));
    else
      outs = analysis_run(gy, saved[0], saved[1], mode, off, reversed(n_out), reversed(nc));
    // outs: (g of the finest band .. g of the coarsest band, g of a)
    res.push_back(outs.back());                                      // a
    for (int64_t k = 0; k < n_ds; ++k) res.push_back(outs[n_ds - 1 - k]);  // ds, coarsest first
    return res;
  }
};

variable_list AnalysisChain::backward(AutogradContext* ctx, variable_list grads) {
  const auto saved = ctx->get_saved_variables();
  const int64_t mode = ctx->saved_data["mode"].toInt(), off = ctx->saved_data["off"].toInt();
  const auto n_in = ctx->saved_data["n_in"].toIntVector();
  const auto n_out = ctx->saved_data["n_out"].toIntVector();
  const size_t J = n_in.size();
  // transpose: coarsest level first; the coarsest low band's gradient is grads[J]
  variable_list ds(J);
  bool any = grads[J].defined();
  for (size_t k = 0; k < J; ++k) {
    ds[k] = grads[J - 1 - k];
    any = any || ds[k].defined();
  }
  if (!any) return variable_list(7);
  at::Tensor gx;
  if (torch::GradMode::is_enabled())
    gx = SynthesisChain::apply(saved[0], saved[1], mode, off, reversed(n_out), reversed(n_in),
                               grads[J], at::TensorList(ds))[0];
  else
    gx = synthesis_run(saved[0], saved[1], mode, off, reversed(n_out), reversed(n_in), grads[J],
                       ds);
  return {gx, at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(),
          at::Tensor()};
}

variable_list analysis_chain(const at::Tensor& x, const at::Tensor& h0, const at::Tensor& h1,
                             int64_t mode, int64_t off, std::vector<int64_t> n_in,
                             std::vector<int64_t> n_out) {
  return AnalysisChain::apply(x, h0, h1, mode, off, std::move(n_in), std::move(n_out));
}

at::Tensor synthesis_chain(const at::Tensor& h0, const at::Tensor& h1, int64_t mode, int64_t off,
                           std::vector<int64_t> nc, std::vector<int64_t> n_out,
                           const c10::optional<at::Tensor>& a,
                           const std::vector<c10::optional<at::Tensor>>& ds) {
  variable_list d;
  d.reserve(ds.size());
  for (const auto& t : ds) d.push_back(t.has_value() ? *t : at::Tensor());
  return SynthesisChain::apply(h0, h1, mode, off, std::move(nc), std::move(n_out),
                               a.has_value() ? *a : at::Tensor(), at::TensorList(d))[0];
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("set_entry_points", &set_entry_points);
  m.def("analysis_chain", &analysis_chain);
  m.def("synthesis_chain", &synthesis_chain);
}
