// PyTorch operators over the C ABI of libsffft.so, registered from C++.
//
// The reference names a library with a PyTorch binding as its next step (README.md:177),
// for the long-convolution layers of Hyena/H3/S4-style models (README.md:11):
//
//   sffft::spectrum(Tensor k, int[] plan, bool conj=False) -> Tensor
//                                    k [H, L] fp32 -> [H, 2L] complex64 (conj: its conjugate)
//   sffft::conv(Tensor u, Tensor kf, int[] plan) -> Tensor  u [B, H, L] fp32 or bf16
//
// `plan` is the nine sffft_plan fields (r0, r1, r2, waves, acc, cached, seqs, mode, channels).
// Each operator launches on the current stream of its input's device, so it is ordered with
// the caller's work and captures into graphs. The GPU kernels are the library's; this file is
// host code only (no kernel of its own), built with the host compiler against torch's headers.
//
// Registering here rather than through torch.library.custom_op keeps the per-call host cost
// at the dispatcher's: the Python wrappers of custom_op (autograd, aliasing checks) took about
// 9 us per call, longer than the kernel itself at L <= 2048. The fake (meta) implementations,
// used only while tracing, stay in Python (sffft_amd/torch_ops.py).
//
// Gradients: sffft::conv is differentiable in u. The adjoint of causal convolution is the
// anti-causal correlation du[m] = sum_{n >= m} dy[n] k[n - m]. With the N = 2L zero padding
// that is IDFT(DFT(dy) * conj(K))[m] for m < L: the same kernel on the conjugated spectrum
// (elementwise conjugation of the kernel-order buffer is the kernel-order buffer of conj(K),
// Hermitian halves included), with no time reversal of dy or du. sffft::spectrum has no
// gradient; backpropagating through it raises.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/autograd.h>
#include <torch/library.h>

#include "sffft.h"

namespace {

sffft_plan to_plan(c10::IntArrayRef f) {
  TORCH_CHECK(f.size() == 9, "a plan has 9 fields (r0, r1, r2, waves, acc, cached, seqs, mode, channels), got ",
              f.size());
  return sffft_plan{(int)f[0], (int)f[1], (int)f[2], (int)f[3], (int)f[4],
                    (int)f[5], (int)f[6], (int)f[7], (int)f[8]};
}

void* current_stream() { return c10::hip::getCurrentHIPStream().stream(); }

void check(int rc, const char* what) {
  TORCH_CHECK(rc == SFFFT_OK, what, " failed: ", sffft_strerror(rc), " (", rc, ") ", sffft_last_error());
}

at::Tensor spectrum_gpu(const at::Tensor& k_in, c10::IntArrayRef plan_fields, bool conj) {
  TORCH_CHECK(k_in.is_cuda() && k_in.scalar_type() == at::kFloat && k_in.dim() == 2,
              "sffft::spectrum: k must be a [H, L] float32 GPU tensor");
  // torch labels GPU tensors CUDA on this backend too; the generic guard picks the
  // backend's own device guard for that label
  const c10::DeviceGuard guard(k_in.device());
  const at::Tensor k = k_in.contiguous();
  const int64_t H = k.size(0), L = k.size(1);
  TORCH_CHECK(H <= INT32_MAX && L <= INT32_MAX, "sffft::spectrum: shape too large");
  const sffft_plan p = to_plan(plan_fields);
  at::Tensor kf = at::empty({H, 2 * L}, k.options().dtype(at::kComplexFloat));
  at::Tensor work = at::empty_like(kf);  // sffft_spectrum_bytes(H, L): scratch, clobbered
  check((conj ? sffft_spectrum_conj : sffft_spectrum)(k.data_ptr<float>(), (int)H, (int)L, &p, kf.data_ptr(),
                                                       work.data_ptr(), current_stream()),
        "sffft_spectrum");
  return kf;
}

at::Tensor conv_gpu(const at::Tensor& u_in, const at::Tensor& kf, c10::IntArrayRef plan_fields) {
  TORCH_CHECK(u_in.is_cuda() && u_in.dim() == 3, "sffft::conv: u must be a [B, H, L] GPU tensor");
  TORCH_CHECK(u_in.scalar_type() == at::kFloat || u_in.scalar_type() == at::kBFloat16,
              "sffft::conv: u must be float32 or bfloat16");
  TORCH_CHECK(kf.is_cuda() && kf.scalar_type() == at::kComplexFloat && kf.is_contiguous(),
              "sffft::conv: kf must be a contiguous complex64 GPU tensor from sffft::spectrum");
  TORCH_CHECK(kf.device() == u_in.device(), "sffft::conv: u and kf must be on the same device");
  const c10::DeviceGuard guard(u_in.device());
  const at::Tensor u = u_in.contiguous();
  const int64_t B = u.size(0), H = u.size(1), L = u.size(2);
  TORCH_CHECK(B <= INT32_MAX && H <= INT32_MAX && L <= INT32_MAX, "sffft::conv: shape too large");
  // the kernels read H rows of 2L values from the start of kf (row h is channel h's
  // spectrum): a spectrum of fewer channels or of another length would be read past its end
  TORCH_CHECK(kf.dim() == 2 && kf.size(0) == H && kf.size(1) == 2 * L, "sffft::conv: kf must be [H, 2L] = [", H,
              ", ", 2 * L, "] for u of shape ", u.sizes(), ", got ", kf.sizes());
  const sffft_plan p = to_plan(plan_fields);
  at::Tensor y = at::empty_like(u);
  const bool bf16 = u.scalar_type() == at::kBFloat16;
  void* s = current_stream();
  if (p.mode == 2) {  // multi-pass: the workspace comes from torch's allocator
    const size_t wb = sffft_work_bytes((int)B, (int)H, (int)L, &p);
    at::Tensor work = at::empty({(int64_t)std::max<size_t>(wb, 16)}, u.options().dtype(at::kByte));
    const size_t have = (size_t)work.numel();
    check(bf16 ? sffft_conv_long_bf16(reinterpret_cast<const uint16_t*>(u.data_ptr()), kf.data_ptr(),
                                      reinterpret_cast<uint16_t*>(y.data_ptr()), work.data_ptr(), have, (int)B,
                                      (int)H, (int)L, &p, s)
               : sffft_conv_long_f32(u.data_ptr<float>(), kf.data_ptr(), y.data_ptr<float>(), work.data_ptr(), have,
                                     (int)B, (int)H, (int)L, &p, s),
          "sffft_conv_long");
  } else {
    check(bf16 ? sffft_conv_bf16(reinterpret_cast<const uint16_t*>(u.data_ptr()), kf.data_ptr(),
                                 reinterpret_cast<uint16_t*>(y.data_ptr()), (int)B, (int)H, (int)L, &p, s)
               : sffft_conv_f32(u.data_ptr<float>(), kf.data_ptr(), y.data_ptr<float>(), (int)B, (int)H, (int)L, &p,
                                s),
          "sffft_conv");
  }
  return y;
}

at::Tensor call_conv(const at::Tensor& u, const at::Tensor& kf, c10::IntArrayRef plan) {
  static const auto op = c10::Dispatcher::singleton()
                             .findSchemaOrThrow("sffft::conv", "")
                             .typed<at::Tensor(const at::Tensor&, const at::Tensor&, c10::IntArrayRef)>();
  return op.call(u, kf, plan);
}

at::Tensor call_spectrum(const at::Tensor& k, c10::IntArrayRef plan, bool conj) {
  static const auto op = c10::Dispatcher::singleton()
                             .findSchemaOrThrow("sffft::spectrum", "")
                             .typed<at::Tensor(const at::Tensor&, c10::IntArrayRef, bool)>();
  return op.call(k, plan, conj);
}

using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

class ConvFn : public torch::autograd::Function<ConvFn> {
 public:
  static at::Tensor forward(AutogradContext* ctx, const at::Tensor& u, const at::Tensor& kf,
                            c10::IntArrayRef plan) {
    ctx->save_for_backward({kf});
    ctx->saved_data["plan"] = plan.vec();
    at::AutoDispatchBelowADInplaceOrView guard;
    return call_conv(u, kf, plan);
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const at::Tensor kf = ctx->get_saved_variables()[0];
    const std::vector<int64_t> plan = ctx->saved_data["plan"].toIntVector();
    at::Tensor du;
    if (ctx->needs_input_grad(0)) du = call_conv(grads[0].contiguous(), at::conj_physical(kf), plan);
    return {du, at::Tensor(), at::Tensor()};
  }
};

class SpectrumFn : public torch::autograd::Function<SpectrumFn> {
 public:
  static at::Tensor forward(AutogradContext*, const at::Tensor& k, c10::IntArrayRef plan, bool conj) {
    at::AutoDispatchBelowADInplaceOrView guard;
    return call_spectrum(k, plan, conj);
  }
  static variable_list backward(AutogradContext*, variable_list) {
    TORCH_CHECK(false, "sffft::spectrum has no gradient with respect to the filter");
    return {};
  }
};

at::Tensor conv_autograd(const at::Tensor& u, const at::Tensor& kf, c10::IntArrayRef plan) {
  return ConvFn::apply(u, kf, plan);
}

at::Tensor spectrum_autograd(const at::Tensor& k, c10::IntArrayRef plan, bool conj) {
  return SpectrumFn::apply(k, plan, conj);
}

}  // namespace

TORCH_LIBRARY(sffft, m) {
  m.def("spectrum(Tensor k, int[] plan, bool conj=False) -> Tensor");
  m.def("conv(Tensor u, Tensor kf, int[] plan) -> Tensor");
}

// torch names its GPU dispatch key CUDA on every backend, this one included.
TORCH_LIBRARY_IMPL(sffft, CUDA, m) {
  m.impl("spectrum", &spectrum_gpu);
  m.impl("conv", &conv_gpu);
}

TORCH_LIBRARY_IMPL(sffft, Autograd, m) {
  m.impl("spectrum", &spectrum_autograd);
  m.impl("conv", &conv_autograd);
}
