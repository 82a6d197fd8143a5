// muon_polar_step_binding.cpp — registers muon_ascend950::polar_step for ROCm
// devices and forwards to the C ABI (include/muon_polar.h).
//
// Reference counterpart: csrc/muon_polar_step_binding.cpp:613-685.  Same schema,
// same preconditions and error texts; differences by design:
//   * dispatch key CUDA (how PyTorch-ROCm names HIP devices) instead of PrivateUse1;
//   * no zero-padded input copy and no output crop (binding.cpp:630-640, 667-672):
//     the kernels mask edge tiles, so the output is allocated at the input shape;
//   * A and P come from one caching-allocator workspace tensor (binding.cpp:646,657);
//   * the launch-configuration cache lives in the C ABI library.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "muon_polar.h"

namespace {

// Contiguous copy of x whose data is 16-byte aligned (a fresh allocation always
// is).  The DMA-fed kernels read X in 16-byte chunks; a contiguous view at an odd
// offset (e.g. buf[1:].view(...)) would otherwise take the register-staged kernels
// (m <= n, about 3.5x slower) or be rejected (m > n).
at::Tensor aligned_contiguous(const at::Tensor &x) {
    at::Tensor t = x.contiguous();
    if (reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 != 0) t = t.clone();
    return t;
}

at::Tensor MuonPolarStepHip(const at::Tensor &x, double a, double b, double c) {
    TORCH_CHECK(x.defined(), "muon_polar_step: x must be defined");
    TORCH_CHECK(x.device().is_cuda(), "muon_polar_step: x must be a ROCm (HIP) device tensor");
    TORCH_CHECK(x.scalar_type() == at::kBFloat16, "muon_polar_step: only bfloat16 is supported");
    TORCH_CHECK(x.dim() == 3, "muon_polar_step: x must have shape [batch, M, N]");
    TORCH_CHECK(x.size(0) > 0 && x.size(1) > 0 && x.size(2) > 0,
                "muon_polar_step: all dimensions must be positive");
    TORCH_CHECK(x.size(1) <= x.size(2),
                "muon_polar_step: current prototype expects M <= N; transpose policy stays "
                "outside this op");
    const c10::OptionalDeviceGuard device_guard(x.device());
    const at::Tensor input = aligned_contiguous(x);
    const int64_t batch = input.size(0), m = input.size(1), n = input.size(2);

    muon_polar_shape_info info{};
    int st = muon_polar_query(batch, m, n, &info);
    TORCH_CHECK(st == MUON_POLAR_OK, "muon_polar_step: ", muon_polar_last_error());

    at::Tensor workspace =
        at::empty({static_cast<int64_t>(info.workspace_bytes)}, input.options().dtype(at::kByte));
    at::Tensor out =
        at::empty_like(input, input.options().memory_format(c10::MemoryFormat::Contiguous));
    hipStream_t stream = c10::hip::getCurrentHIPStream(x.device().index()).stream();
    st = muon_polar_step(input.data_ptr(), out.data_ptr(), workspace.data_ptr(),
                         info.workspace_bytes, batch, m, n, a, b, c, stream);
    TORCH_CHECK(st == MUON_POLAR_OK, "muon_polar_step: ", muon_polar_last_error());
    return out;
}

// One step on X [batch, M, N] with M > N in the right-Gram form
// Y = a·X + X·(b·G + c·G²), G = Xᵀ·X: no transposed copies of X and Y (the
// reference's wrapper transposes around the op, ops.py:26-32).  Needs N % 8 == 0.
at::Tensor MuonPolarStepTallHip(const at::Tensor &x, double a, double b, double c) {
    TORCH_CHECK(x.defined(), "muon_polar_step_tall: x must be defined");
    TORCH_CHECK(x.device().is_cuda(), "muon_polar_step_tall: x must be a ROCm (HIP) device tensor");
    TORCH_CHECK(x.scalar_type() == at::kBFloat16, "muon_polar_step_tall: only bfloat16 is supported");
    TORCH_CHECK(x.dim() == 3, "muon_polar_step_tall: x must have shape [batch, M, N]");
    TORCH_CHECK(x.size(0) > 0 && x.size(1) > 0 && x.size(2) > 0,
                "muon_polar_step_tall: all dimensions must be positive");
    TORCH_CHECK(x.size(1) > x.size(2) && x.size(2) % 8 == 0,
                "muon_polar_step_tall: expects M > N with N % 8 == 0");
    const c10::OptionalDeviceGuard device_guard(x.device());
    const at::Tensor input = aligned_contiguous(x);
    const int64_t batch = input.size(0), m = input.size(1), n = input.size(2);
    muon_polar_shape_info info{};
    int st = muon_polar_query(batch, m, n, &info);
    TORCH_CHECK(st == MUON_POLAR_OK, "muon_polar_step_tall: ", muon_polar_last_error());
    at::Tensor workspace =
        at::empty({static_cast<int64_t>(info.workspace_bytes)}, input.options().dtype(at::kByte));
    at::Tensor out =
        at::empty_like(input, input.options().memory_format(c10::MemoryFormat::Contiguous));
    hipStream_t stream = c10::hip::getCurrentHIPStream(x.device().index()).stream();
    st = muon_polar_step(input.data_ptr(), out.data_ptr(), workspace.data_ptr(),
                         info.workspace_bytes, batch, m, n, a, b, c, stream);
    TORCH_CHECK(st == MUON_POLAR_OK, "muon_polar_step_tall: ", muon_polar_last_error());
    return out;
}

// Several steps (and the optional per-matrix normalisation) in one call; no
// reference counterpart (the reference's examples/five_steps.py:17-20 loops in
// Python).  Preconditions of polar_step, except that M > N is accepted when
// N % 8 == 0 (right-Gram form); coefficients are flattened triples.
at::Tensor MuonPolarExpressHip(const at::Tensor &x, at::ArrayRef<double> coefficients,
                               bool normalize) {
    TORCH_CHECK(x.defined(), "muon_polar_express: x must be defined");
    TORCH_CHECK(x.device().is_cuda(), "muon_polar_express: x must be a ROCm (HIP) device tensor");
    TORCH_CHECK(x.scalar_type() == at::kBFloat16, "muon_polar_express: only bfloat16 is supported");
    TORCH_CHECK(x.dim() == 3, "muon_polar_express: x must have shape [batch, M, N]");
    TORCH_CHECK(x.size(0) > 0 && x.size(1) > 0 && x.size(2) > 0,
                "muon_polar_express: all dimensions must be positive");
    TORCH_CHECK(x.size(1) <= x.size(2) || x.size(2) % 8 == 0,
                "muon_polar_express: M > N needs N % 8 == 0; otherwise transpose outside this op");
    TORCH_CHECK(coefficients.size() % 3 == 0,
                "muon_polar_express: coefficients must be (a, b, c) triples");
    TORCH_CHECK(!coefficients.empty() || normalize,
                "muon_polar_express: no coefficients and no normalisation");
    const c10::OptionalDeviceGuard device_guard(x.device());
    const at::Tensor input = aligned_contiguous(x);
    const int64_t batch = input.size(0), m = input.size(1), n = input.size(2);

    muon_polar_shape_info info{};
    int st = muon_polar_query(batch, m, n, &info);
    TORCH_CHECK(st == MUON_POLAR_OK, "muon_polar_express: ", muon_polar_last_error());
    at::Tensor workspace = at::empty({static_cast<int64_t>(info.express_workspace_bytes)},
                                     input.options().dtype(at::kByte));
    at::Tensor out =
        at::empty_like(input, input.options().memory_format(c10::MemoryFormat::Contiguous));
    hipStream_t stream = c10::hip::getCurrentHIPStream(x.device().index()).stream();
    st = muon_polar_express(input.data_ptr(), out.data_ptr(), workspace.data_ptr(),
                            info.express_workspace_bytes, batch, m, n, coefficients.data(),
                            static_cast<int64_t>(coefficients.size() / 3), normalize ? 1 : 0,
                            stream);
    TORCH_CHECK(st == MUON_POLAR_OK, "muon_polar_express: ", muon_polar_last_error());
    return out;
}

// Muon update of param (in place) and momentum_buffer (in place) from grad; no
// reference counterpart (the reference leaves the update to its caller,
// README.md:130).  All three fp32 [batch, M, N], contiguous, on one device.
void MuonUpdateHip(const at::Tensor &param, const at::Tensor &grad,
                   const at::Tensor &momentum_buffer, double momentum, bool nesterov,
                   at::ArrayRef<double> coefficients, double lr, double weight_decay,
                   double lr_scale) {
    for (const at::Tensor *t : {&param, &grad, &momentum_buffer}) {
        TORCH_CHECK(t->defined(), "muon_update: tensors must be defined");
        TORCH_CHECK(t->device().is_cuda(), "muon_update: tensors must be ROCm (HIP) device tensors");
        TORCH_CHECK(t->device() == param.device(), "muon_update: tensors must share one device");
        TORCH_CHECK(t->scalar_type() == at::kFloat, "muon_update: param, grad and momentum_buffer must be float32");
        TORCH_CHECK(t->sizes() == param.sizes(), "muon_update: param, grad and momentum_buffer must have one shape");
    }
    TORCH_CHECK(param.dim() == 3, "muon_update: tensors must have shape [batch, M, N]");
    TORCH_CHECK(param.size(0) > 0 && param.size(1) > 0 && param.size(2) > 0,
                "muon_update: all dimensions must be positive");
    TORCH_CHECK(param.is_contiguous() && momentum_buffer.is_contiguous(),
                "muon_update: param and momentum_buffer must be contiguous (they are updated in place)");
    TORCH_CHECK(coefficients.size() % 3 == 0, "muon_update: coefficients must be (a, b, c) triples");
    const c10::OptionalDeviceGuard device_guard(param.device());
    const at::Tensor g = grad.contiguous();
    const int64_t batch = param.size(0), m = param.size(1), n = param.size(2);
    muon_polar_shape_info info{};
    int st = muon_polar_query(batch, m, n, &info);
    TORCH_CHECK(st == MUON_POLAR_OK, "muon_update: ", muon_polar_last_error());
    at::Tensor workspace = at::empty({static_cast<int64_t>(info.muon_workspace_bytes)},
                                     param.options().dtype(at::kByte));
    hipStream_t stream = c10::hip::getCurrentHIPStream(param.device().index()).stream();
    st = muon_polar_muon_update(param.data_ptr(), g.data_ptr(), momentum_buffer.data_ptr(),
                                workspace.data_ptr(), info.muon_workspace_bytes, batch, m, n,
                                momentum, nesterov ? 1 : 0, coefficients.data(),
                                static_cast<int64_t>(coefficients.size() / 3), lr, weight_decay,
                                lr_scale, stream);
    TORCH_CHECK(st == MUON_POLAR_OK, "muon_update: ", muon_polar_last_error());
}

}  // namespace

TORCH_LIBRARY(muon_ascend950, m) {
    m.def("polar_step(Tensor x, float a, float b, float c) -> Tensor");
    m.def("polar_step_tall(Tensor x, float a, float b, float c) -> Tensor");
    m.def("polar_express(Tensor x, float[] coefficients, bool normalize) -> Tensor");
    m.def("muon_update(Tensor(a!) param, Tensor grad, Tensor(b!) momentum_buffer, float momentum, "
          "bool nesterov, float[] coefficients, float lr, float weight_decay, float lr_scale) -> ()");
}

TORCH_LIBRARY_IMPL(muon_ascend950, CUDA, m) {
    m.impl("polar_step", &MuonPolarStepHip);
    m.impl("polar_step_tall", &MuonPolarStepTallHip);
    m.impl("polar_express", &MuonPolarExpressHip);
    m.impl("muon_update", &MuonUpdateHip);
}
