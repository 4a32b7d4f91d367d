// fa_torch.cpp - native host path of the dense forward / backward for
// PyTorch callers.
//
// The C ABI (include/fa_mi355x.h) takes plain pointers; this library is the
// PyTorch-side caller of it for dense (B, H, S, D) attention.  It fills
// fa_fwd_params / fa_bwd_params from tensors, allocates outputs and the
// optional dS scratch through torch's caching allocator, launches on torch's
// current HIP stream, and defines the autograd function of
// flash_attention (reference fa_rdna3/interface.py:316-333, `_flash_fwd`'s
// registered autograd) in C++.  A training step's backward then runs on
// the autograd engine's device thread without taking the Python interpreter
// lock, and neither pass pays for Python parameter packing: the host cost of
// a config-2 step was close to its GPU time with the Python path.
//
// Registered operators (namespace fa_mi355x):
//   attention(q, k, v, causal, scale, window_left, window_right, softcap,
//             bias?, alibi?, dropout_p, dropout_seed) -> out   (differentiable)
//   forward(...same...) -> (out, lse)
//   backward(dout, q, k, v, out, lse, ...same options...) -> (dq, dk, dv)
//   set_ds_scratch_limit(bytes) / ds_scratch_limit() -> bytes
// Argument contracts are checked by the Python layer with the reference's
// messages before any of these is called; the C ABI re-checks what could
// make a kernel access memory out of bounds.
#include <ATen/ATen.h>
#include <ATen/core/dispatch/Dispatcher.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/autograd.h>
#include <torch/library.h>

#include <atomic>
#include <cstring>
#include <initializer_list>
#include <optional>
#include <tuple>

#include "../../include/fa_mi355x.h"

namespace {

using at::Tensor;
using OptTensor = std::optional<Tensor>;

// Smallest head dim the kernels take; smaller ones are zero-padded to it
// (zeros add nothing to q.k^T or p.v; the scale is the caller's).
constexpr int64_t kMinKernelHeadDim = 32;

// Largest dS scratch a backward allocates.  A problem whose dS exceeds it
// runs in two chunks of KV heads when one chunk fits and the library chunks
// it (fa_bwd_workspace_min_bytes); otherwise dQ recomputes the scores.  0
// disables the dS path.
std::atomic<int64_t> g_ds_limit{int64_t(12) << 30};

// Scratch bytes for the backward of p under `limit`: the whole dS, else one
// chunk's, else 0.
int64_t ds_scratch_bytes(const fa_bwd_params& p, int64_t limit) {
  const int64_t full = (int64_t)fa_bwd_workspace_bytes(&p);
  if (full <= 0) return 0;
  if (full <= limit) return full;
  const int64_t half = (int64_t)fa_bwd_workspace_min_bytes(&p);
  return (half > 0 && half < full && half <= limit) ? half : 0;
}

struct Options {
  bool causal;
  double scale;
  int64_t window_left, window_right;
  double softcap;
  OptTensor bias, alibi;
  double dropout_p;
  int64_t dropout_seed;
};

int32_t dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kHalf: return FA_DTYPE_F16;
    case at::kBFloat16: return FA_DTYPE_BF16;
    case at::kFloat: return FA_DTYPE_F32;
    default: TORCH_CHECK(false, "fa_mi355x: unsupported dtype ", t);
  }
  return -1;
}

void check_status(int rc, const char* what) {
  TORCH_CHECK(rc == 0, what, " failed (status ", rc, "): ", fa_last_error_string());
}

// Rows must start 16-byte aligned with a unit last stride (the kernels'
// vector-load contract); anything else is copied to a contiguous tensor.
Tensor kernel_ready(const Tensor& t) {
  const int64_t esize = t.element_size();
  bool ok = t.stride(-1) == 1 || t.size(-1) == 1;
  ok = ok && reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0;
  for (int64_t i = 0; ok && i + 1 < t.dim(); ++i)
    if (t.size(i) > 1 && (t.stride(i) * esize) % 16 != 0) ok = false;
  if (ok && t.stride(-1) == 1) return t;
  return t.contiguous();
}

Tensor pad_head_dim(const Tensor& t, int64_t dim) {
  const int64_t pad = dim - t.size(-1);
  return pad > 0 ? at::constant_pad_nd(t, {0, pad}) : t;
}

// Element strides for the ABI: size-1 dims (never stepped over) get stride
// 0 and the last dim is contiguous (see kernel_ready).
void abi_strides4(int64_t* dst, const Tensor& t) {
  for (int i = 0; i < 4; ++i) dst[i] = t.size(i) > 1 ? t.stride(i) : 0;
  dst[3] = 1;
}

void abi_strides3(int64_t* dst, const Tensor& t) {
  for (int i = 0; i < 3; ++i) dst[i] = t.size(i) > 1 ? t.stride(i) : 0;
}

void* stream_of(const Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

// Tensors a launch reads besides q / k / v: the broadcast bias view and the
// fp32 ALiBi slopes.  They must outlive the launch call.
struct Extras {
  Tensor bias, alibi;
};

// reference interface.py:115-133 (_bias_args, _alibi_args)
Extras fill_fwd(fa_fwd_params& p, const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& out,
                const Tensor& lse, const Options& o) {
  std::memset(&p, 0, sizeof(p));
  p.abi_version = FA_ABI_VERSION;
  p.dtype = dtype_code(q.scalar_type());
  p.q = q.data_ptr();
  p.k = k.data_ptr();
  p.v = v.data_ptr();
  p.out = out.data_ptr();
  p.lse = lse.data_ptr<float>();
  abi_strides4(p.q_stride, q);
  abi_strides4(p.k_stride, k);
  abi_strides4(p.v_stride, v);
  abi_strides4(p.out_stride, out);
  abi_strides3(p.lse_stride, lse);
  p.batch = (int32_t)q.size(0);
  p.heads_q = (int32_t)q.size(1);
  p.seqlen_q = (int32_t)q.size(2);
  p.head_dim = (int32_t)q.size(3);
  p.heads_kv = (int32_t)k.size(1);
  p.seqlen_k = (int32_t)k.size(2);
  p.softmax_scale = (float)o.scale;
  p.causal = o.causal ? 1 : 0;
  p.window_left = (int32_t)o.window_left;
  p.window_right = (int32_t)o.window_right;
  p.softcap = (float)o.softcap;
  p.dropout_p = (float)o.dropout_p;
  p.dropout_seed = (uint64_t)o.dropout_seed;
  Extras ex;
  if (o.bias.has_value() && o.bias->defined()) {
    ex.bias = o.bias->expand({q.size(0), q.size(1), q.size(2), k.size(2)});
    p.bias = ex.bias.data_ptr();
    p.bias_dtype = dtype_code(ex.bias.scalar_type());
    for (int i = 0; i < 4; ++i) p.bias_stride[i] = ex.bias.stride(i);
  }
  if (o.alibi.has_value() && o.alibi->defined()) {
    ex.alibi = o.alibi->to(at::kFloat).contiguous();
    p.alibi_slopes = ex.alibi.data_ptr<float>();
  }
  return ex;
}

// Every tensor a launch touches must live on the query's GPU: the C ABI
// receives bare pointers and cannot tell host memory from device memory.
void check_on_gpu(const Tensor& query, std::initializer_list<const Tensor*> others, const Options& o) {
  TORCH_CHECK(query.is_cuda(), "fa_mi355x: tensors must be on a GPU");
  for (const Tensor* t : others)
    TORCH_CHECK(t->device() == query.device(), "fa_mi355x: all tensors must be on the query's device");
  if (o.bias.has_value() && o.bias->defined())
    TORCH_CHECK(o.bias->device() == query.device(), "fa_mi355x: bias must be on the query's device");
  if (o.alibi.has_value() && o.alibi->defined())
    TORCH_CHECK(o.alibi->device() == query.device(), "fa_mi355x: alibi slopes must be on the query's device");
}

// reference interface.py:154-199 (_forward)
std::tuple<Tensor, Tensor> forward_impl(const Tensor& query, const Tensor& key, const Tensor& value,
                                        const Options& o) {
  check_on_gpu(query, {&key, &value}, o);
  c10::DeviceGuard guard(query.device());
  const int64_t head_dim = query.size(3);
  const int64_t kdim = std::max(kMinKernelHeadDim, head_dim);
  const Tensor q = kernel_ready(pad_head_dim(query, kdim));
  const Tensor k = kernel_ready(pad_head_dim(key, kdim));
  const Tensor v = kernel_ready(pad_head_dim(value, kdim));
  Tensor out = at::empty({q.size(0), q.size(1), q.size(2), kdim}, query.options());
  Tensor lse = at::empty({q.size(0), q.size(1), q.size(2)}, query.options().dtype(at::kFloat));
  fa_fwd_params p;
  const Extras ex = fill_fwd(p, q, k, v, out, lse, o);
  check_status(fa_fwd(&p, stream_of(query)), "fa_fwd");
  if (kdim != head_dim) out = out.narrow(-1, 0, head_dim).contiguous();
  return {out, lse};
}

// reference interface.py:202-277 (_backward): delta, dK/dV and dQ in one
// fa_bwd call, with the dS scratch when it fits under the limit.
std::tuple<Tensor, Tensor, Tensor> backward_impl(const Tensor& dout, const Tensor& query, const Tensor& key,
                                                 const Tensor& value, const Tensor& out, const Tensor& lse_in,
                                                 const Options& o) {
  check_on_gpu(query, {&dout, &key, &value, &out, &lse_in}, o);
  c10::DeviceGuard guard(query.device());
  const int64_t head_dim = query.size(3);
  const int64_t kdim = std::max(kMinKernelHeadDim, head_dim);
  const Tensor q = kernel_ready(pad_head_dim(query, kdim));
  const Tensor k = kernel_ready(pad_head_dim(key, kdim));
  const Tensor v = kernel_ready(pad_head_dim(value, kdim));
  const Tensor ot = kernel_ready(pad_head_dim(out, kdim));
  const Tensor dot = kernel_ready(pad_head_dim(dout.contiguous(), kdim));
  const Tensor lse = lse_in.contiguous();
  Tensor delta = at::empty_like(lse);
  Tensor dq = at::empty(q.sizes(), query.options());
  Tensor dk = at::empty(k.sizes(), key.options());
  Tensor dv = at::empty(v.sizes(), value.options());
  fa_bwd_params p;
  std::memset(&p, 0, sizeof(p));
  const Extras ex = fill_fwd(p.fwd, q, k, v, ot, lse, o);
  p.dout = dot.data_ptr();
  p.dq = dq.data_ptr();
  p.dk = dk.data_ptr();
  p.dv = dv.data_ptr();
  p.delta = delta.data_ptr<float>();
  abi_strides4(p.dout_stride, dot);
  abi_strides4(p.dq_stride, dq);
  abi_strides4(p.dk_stride, dk);
  abi_strides4(p.dv_stride, dv);
  abi_strides3(p.delta_stride, delta);
  Tensor ds;
  const int64_t bytes = ds_scratch_bytes(p, g_ds_limit.load(std::memory_order_relaxed));
  if (bytes > 0) {
    ds = at::empty({bytes}, query.options().dtype(at::kByte));
    p.ds_workspace = ds.data_ptr();
    p.ds_workspace_bytes = bytes;
  }
  check_status(fa_bwd(&p, stream_of(query)), "fa_bwd");
  if (kdim != head_dim) {
    dq = dq.narrow(-1, 0, head_dim).contiguous();
    dk = dk.narrow(-1, 0, head_dim).contiguous();
    dv = dv.narrow(-1, 0, head_dim).contiguous();
  }
  return {dq, dk, dv};
}

Options make_options(bool causal, double scale, int64_t wl, int64_t wr, double softcap, const OptTensor& bias,
                     const OptTensor& alibi, double dropout_p, int64_t seed) {
  return Options{causal, scale, wl, wr, softcap, bias, alibi, dropout_p, seed};
}

std::tuple<Tensor, Tensor> forward_op(const Tensor& q, const Tensor& k, const Tensor& v, bool causal, double scale,
                                      int64_t wl, int64_t wr, double softcap, const OptTensor& bias,
                                      const OptTensor& alibi, double dropout_p, int64_t seed) {
  return forward_impl(q, k, v, make_options(causal, scale, wl, wr, softcap, bias, alibi, dropout_p, seed));
}

std::tuple<Tensor, Tensor, Tensor> backward_op(const Tensor& dout, const Tensor& q, const Tensor& k,
                                               const Tensor& v, const Tensor& out, const Tensor& lse, bool causal,
                                               double scale, int64_t wl, int64_t wr, double softcap,
                                               const OptTensor& bias, const OptTensor& alibi, double dropout_p,
                                               int64_t seed) {
  return backward_impl(dout, q, k, v, out, lse,
                       make_options(causal, scale, wl, wr, softcap, bias, alibi, dropout_p, seed));
}

// Autograd of the dense attention: q, k, v differentiable; bias and ALiBi
// slopes are not (reference interface.py:316-333).
// Shape functions of forward / backward (Meta kernels): FakeTensorMode,
// make_fx and other tracers run these instead of the launches.
std::tuple<Tensor, Tensor> forward_meta(const Tensor& q, const Tensor& k, const Tensor& v, bool causal, double scale,
                                        int64_t wl, int64_t wr, double softcap, const OptTensor& bias,
                                        const OptTensor& alibi, double dropout_p, int64_t seed) {
  return {at::empty(q.sizes(), q.options()), at::empty({q.size(0), q.size(1), q.size(2)}, q.options().dtype(at::kFloat))};
}

std::tuple<Tensor, Tensor, Tensor> backward_meta(const Tensor& dout, const Tensor& q, const Tensor& k,
                                                 const Tensor& v, const Tensor& out, const Tensor& lse, bool causal,
                                                 double scale, int64_t wl, int64_t wr, double softcap,
                                                 const OptTensor& bias, const OptTensor& alibi, double dropout_p,
                                                 int64_t seed) {
  return {at::empty(q.sizes(), q.options()), at::empty(k.sizes(), k.options()), at::empty(v.sizes(), v.options())};
}

// The autograd function calls forward / backward through the dispatcher, so
// a tracer (FakeTensorMode, make_fx) sees those operators and their Meta
// kernels rather than raw launches on its tensors.
std::tuple<Tensor, Tensor> call_forward(const Tensor& q, const Tensor& k, const Tensor& v, const Options& o) {
  static const auto op = c10::Dispatcher::singleton()
                             .findSchemaOrThrow("fa_mi355x::forward", "")
                             .typed<decltype(forward_op)>();
  return op.call(q, k, v, o.causal, o.scale, o.window_left, o.window_right, o.softcap, o.bias, o.alibi, o.dropout_p,
                 o.dropout_seed);
}

std::tuple<Tensor, Tensor, Tensor> call_backward(const Tensor& dout, const Tensor& q, const Tensor& k,
                                                 const Tensor& v, const Tensor& out, const Tensor& lse,
                                                 const Options& o) {
  static const auto op = c10::Dispatcher::singleton()
                             .findSchemaOrThrow("fa_mi355x::backward", "")
                             .typed<decltype(backward_op)>();
  return op.call(dout, q, k, v, out, lse, o.causal, o.scale, o.window_left, o.window_right, o.softcap, o.bias,
                 o.alibi, o.dropout_p, o.dropout_seed);
}

class AttentionFn : public torch::autograd::Function<AttentionFn> {
 public:
  static Tensor forward(torch::autograd::AutogradContext* ctx, const Tensor& q, const Tensor& k, const Tensor& v,
                        bool causal, double scale, int64_t wl, int64_t wr, double softcap, const OptTensor& bias,
                        const OptTensor& alibi, double dropout_p, int64_t seed) {
    auto [out, lse] = call_forward(q, k, v, make_options(causal, scale, wl, wr, softcap, bias, alibi, dropout_p, seed));
    ctx->save_for_backward({q, k, v, out, lse, bias.value_or(Tensor()), alibi.value_or(Tensor())});
    ctx->saved_data["causal"] = causal;
    ctx->saved_data["scale"] = scale;
    ctx->saved_data["wl"] = wl;
    ctx->saved_data["wr"] = wr;
    ctx->saved_data["softcap"] = softcap;
    ctx->saved_data["dropout_p"] = dropout_p;
    ctx->saved_data["seed"] = seed;
    ctx->mark_non_differentiable({lse});
    return out;
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const auto saved = ctx->get_saved_variables();
    const Tensor& bias = saved[5];
    const Tensor& alibi = saved[6];
    Options o{ctx->saved_data["causal"].toBool(),
              ctx->saved_data["scale"].toDouble(),
              ctx->saved_data["wl"].toInt(),
              ctx->saved_data["wr"].toInt(),
              ctx->saved_data["softcap"].toDouble(),
              bias.defined() ? OptTensor(bias) : std::nullopt,
              alibi.defined() ? OptTensor(alibi) : std::nullopt,
              ctx->saved_data["dropout_p"].toDouble(),
              ctx->saved_data["seed"].toInt()};
    auto [dq, dk, dv] = call_backward(grads[0], saved[0], saved[1], saved[2], saved[3], saved[4], o);
    return {dq, dk, dv, Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
  }
};

Tensor attention_op(const Tensor& q, const Tensor& k, const Tensor& v, bool causal, double scale, int64_t wl,
                    int64_t wr, double softcap, const OptTensor& bias, const OptTensor& alibi, double dropout_p,
                    int64_t seed) {
  return AttentionFn::apply(q, k, v, causal, scale, wl, wr, softcap, bias, alibi, dropout_p, seed);
}

int64_t set_ds_scratch_limit(int64_t bytes) {
  return g_ds_limit.exchange(bytes < 0 ? 0 : bytes);
}

int64_t ds_scratch_limit() { return g_ds_limit.load(); }

}  // namespace

TORCH_LIBRARY(fa_mi355x, m) {
  m.def("attention(Tensor q, Tensor k, Tensor v, bool causal, float scale, int window_left, int window_right, "
        "float softcap, Tensor? bias, Tensor? alibi, float dropout_p, int dropout_seed) -> Tensor");
  m.def("forward(Tensor q, Tensor k, Tensor v, bool causal, float scale, int window_left, int window_right, "
        "float softcap, Tensor? bias, Tensor? alibi, float dropout_p, int dropout_seed) -> (Tensor, Tensor)");
  m.def("backward(Tensor dout, Tensor q, Tensor k, Tensor v, Tensor out, Tensor lse, bool causal, float scale, "
        "int window_left, int window_right, float softcap, Tensor? bias, Tensor? alibi, float dropout_p, "
        "int dropout_seed) -> (Tensor, Tensor, Tensor)");
  m.def("set_ds_scratch_limit(int bytes) -> int", &set_ds_scratch_limit);
  m.def("ds_scratch_limit() -> int", &ds_scratch_limit);
}

TORCH_LIBRARY_IMPL(fa_mi355x, CompositeImplicitAutograd, m) { m.impl("attention", &attention_op); }

TORCH_LIBRARY_IMPL(fa_mi355x, CUDA, m) {
  m.impl("forward", &forward_op);
  m.impl("backward", &backward_op);
}

TORCH_LIBRARY_IMPL(fa_mi355x, Meta, m) {
  m.impl("forward", &forward_meta);
  m.impl("backward", &backward_meta);
}
