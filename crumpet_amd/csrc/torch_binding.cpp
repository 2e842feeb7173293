// Dispatcher registration of the crumpet_ops operators on ROCm PyTorch.
//
// Same five op schemas and tags as the reference
// (torch-ext/torch_binding.cpp:10-31), plus `fused_swin_attention`, which
// the reference launched from Python through Triton, and
// `fused_swin_attention_shifted` (attention with the shifted-window mask
// derived from the volume geometry instead of a mask tensor),
// `attn_mask_tiles` / `fused_swin_attention_tiled` (a 16-bit mask's tiled
// copy and attention reading it), the fused block projections
// `window_qkv_3d` / `window_proj_3d`, and `window_msa_3d`, which runs those
// three kernels for a whole block half in one dispatcher call.  Every impl checks
// shapes, dtypes and devices (so no launch can index outside its tensors),
// takes the current HIP stream of the tensor's device (ROCm torch tags HIP
// devices as "cuda", hence the masquerading guard/stream helpers) and forwards to the
// C ABI of libcrumpet_hip.so (include/crumpet_hip.h).  A non-OK status
// becomes a RuntimeError carrying crumpet_last_error().
#include <ATen/core/Tensor.h>
#include <ATen/ops/empty.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include "crumpet_hip.h"

namespace {

const std::vector<at::Tag> kCrumpetOpTags = {
    at::Tag::pt2_compliant_tag,
    at::Tag::needs_fixed_stride_order,
};

void* stream_of(const at::Tensor& t) {
    return static_cast<void*>(
        c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream());
}

void check_status(int status) {
    TORCH_CHECK(status == CRUMPET_OK, "crumpet_ops: ", crumpet_last_error(), " (",
                crumpet_status_string(status), ")");
}

void check_device_pair(const at::Tensor& out, const at::Tensor& in, const char* what) {
    TORCH_CHECK(out.is_cuda() && in.is_cuda(), what, ": tensors must be on a HIP device");
    TORCH_CHECK(out.device() == in.device(), what, ": tensors must be on the same device");
    TORCH_CHECK(out.scalar_type() == in.scalar_type(), what, ": dtype mismatch");
    TORCH_CHECK(out.is_contiguous() && in.is_contiguous(), what, ": tensors must be contiguous");
    TORCH_CHECK(out.numel() == in.numel(), what, ": output and input sizes differ");
}

int32_t dtype_code(at::ScalarType t) {
    switch (t) {
        case at::kFloat: return CRUMPET_DTYPE_F32;
        case at::kHalf: return CRUMPET_DTYPE_F16;
        case at::kBFloat16: return CRUMPET_DTYPE_BF16;
        default: return -1;
    }
}

void compute_attn_mask_3d(at::Tensor& output, int64_t D, int64_t H, int64_t W, int64_t ws_d,
                          int64_t ws_h, int64_t ws_w, int64_t ss_d, int64_t ss_h, int64_t ss_w) {
    TORCH_CHECK(output.is_cuda(), "compute_attn_mask_3d: output must be on a HIP device");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(output.device());
    if (output.numel() == 0) return;
    const int32_t dt = dtype_code(output.scalar_type());
    TORCH_CHECK(dt >= 0, "compute_attn_mask_3d: output dtype must be float32, float16 or bfloat16");
    TORCH_CHECK(output.is_contiguous(), "compute_attn_mask_3d: output must be contiguous");
    TORCH_CHECK(ws_d > 0 && ws_h > 0 && ws_w > 0 && D % ws_d == 0 && H % ws_h == 0 && W % ws_w == 0,
                "compute_attn_mask_3d: D, H and W must be divisible by window_size");
    const int64_t vol = ws_d * ws_h * ws_w;
    const int64_t nW = (D / ws_d) * (H / ws_h) * (W / ws_w);
    TORCH_CHECK(output.numel() == nW * vol * vol, "compute_attn_mask_3d: output must hold ", nW,
                " x ", vol, " x ", vol, " elements");
    check_status(crumpet_compute_attn_mask_3d(output.data_ptr(), dt, D, H, W, ws_d, ws_h, ws_w,
                                              ss_d, ss_h, ss_w, stream_of(output)));
}

void fused_shift_partition_3d(at::Tensor& output, const at::Tensor& x, int64_t ws_d, int64_t ws_h,
                              int64_t ws_w, int64_t ss_d, int64_t ss_h, int64_t ss_w) {
    TORCH_CHECK(x.dim() == 5, "fused_shift_partition_3d: x must have shape [B, D, H, W, C]");
    check_device_pair(output, x, "fused_shift_partition_3d");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    if (output.numel() == 0) return;
    check_status(crumpet_shift_partition_3d(output.data_ptr(), x.data_ptr(), x.size(0), x.size(1),
                                            x.size(2), x.size(3), x.size(4), x.element_size(),
                                            ws_d, ws_h, ws_w, ss_d, ss_h, ss_w, stream_of(x)));
}

void fused_unshift_unpartition_3d(at::Tensor& output, const at::Tensor& windows, int64_t B,
                                  int64_t D, int64_t H, int64_t W, int64_t C, int64_t ws_d,
                                  int64_t ws_h, int64_t ws_w, int64_t ss_d, int64_t ss_h,
                                  int64_t ss_w) {
    check_device_pair(output, windows, "fused_unshift_unpartition_3d");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(windows.device());
    if (output.numel() == 0) return;
    TORCH_CHECK(output.numel() == B * D * H * W * C,
                "fused_unshift_unpartition_3d: output must hold B*D*H*W*C elements");
    check_status(crumpet_unshift_unpartition_3d(output.data_ptr(), windows.data_ptr(), B, D, H, W,
                                                C, windows.element_size(), ws_d, ws_h, ws_w, ss_d,
                                                ss_h, ss_w, stream_of(windows)));
}

void fused_shift_partition_3d_backward(at::Tensor& grad_x, const at::Tensor& grad_windows,
                                       int64_t B, int64_t D, int64_t H, int64_t W, int64_t C,
                                       int64_t ws_d, int64_t ws_h, int64_t ws_w, int64_t ss_d,
                                       int64_t ss_h, int64_t ss_w) {
    check_device_pair(grad_x, grad_windows, "fused_shift_partition_3d_backward");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(grad_windows.device());
    if (grad_x.numel() == 0) return;
    TORCH_CHECK(grad_x.numel() == B * D * H * W * C,
                "fused_shift_partition_3d_backward: grad_x must hold B*D*H*W*C elements");
    check_status(crumpet_shift_partition_3d_backward(
        grad_x.data_ptr(), grad_windows.data_ptr(), B, D, H, W, C, grad_windows.element_size(),
        ws_d, ws_h, ws_w, ss_d, ss_h, ss_w, stream_of(grad_windows)));
}

void fused_unshift_unpartition_3d_backward(at::Tensor& grad_windows, const at::Tensor& grad_x,
                                           int64_t ws_d, int64_t ws_h, int64_t ws_w,
                                           int64_t ss_d, int64_t ss_h, int64_t ss_w) {
    TORCH_CHECK(grad_x.dim() == 5,
                "fused_unshift_unpartition_3d_backward: grad_x must have shape [B, D, H, W, C]");
    check_device_pair(grad_windows, grad_x, "fused_unshift_unpartition_3d_backward");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(grad_x.device());
    if (grad_windows.numel() == 0) return;
    check_status(crumpet_unshift_unpartition_3d_backward(
        grad_windows.data_ptr(), grad_x.data_ptr(), grad_x.size(0), grad_x.size(1),
        grad_x.size(2), grad_x.size(3), grad_x.size(4), grad_x.element_size(), ws_d, ws_h, ws_w,
        ss_d, ss_h, ss_w, stream_of(grad_x)));
}

// fused_swin_attention, and with `tiles` (the tiled copy of the mask, from
// attn_mask_tiles) fused_swin_attention_tiled
void run_fused_swin_attention(const char* what, at::Tensor& out, const at::Tensor& q, const at::Tensor& k,
                              const at::Tensor& v, const at::Tensor& bias,
                              const std::optional<at::Tensor>& mask, const at::Tensor* tiles,
                              const std::optional<at::Tensor>& boundary, double scale) {
    TORCH_CHECK(q.dim() == 4, what, ": q must have shape [B, H, N, D]");
    TORCH_CHECK(k.sizes() == q.sizes() && v.sizes() == q.sizes() && out.sizes() == q.sizes(), what,
                ": q, k, v and out must have the same shape");
    TORCH_CHECK(k.scalar_type() == q.scalar_type() && v.scalar_type() == q.scalar_type() &&
                    out.scalar_type() == q.scalar_type(),
                what, ": q, k, v and out must have the same dtype");
    const int32_t dt = dtype_code(q.scalar_type());
    TORCH_CHECK(dt >= 0, what, ": dtype must be float32, float16 or bfloat16");
    const at::Device dev = q.device();
    TORCH_CHECK(q.is_cuda() && k.device() == dev && v.device() == dev && out.device() == dev &&
                    bias.device() == dev,
                what, ": all tensors must be on the same HIP device");
    const int64_t B = q.size(0), Hh = q.size(1), N = q.size(2), Dh = q.size(3);
    TORCH_CHECK(bias.dim() == 3 && bias.size(0) == Hh && bias.size(1) == N && bias.size(2) == N,
                what, ": relative_position_bias must have shape [H, N, N]");
    const int32_t bdt = dtype_code(bias.scalar_type());
    TORCH_CHECK(bdt >= 0, what, ": bias dtype must be float32, float16 or bfloat16");
    const void* mptr = nullptr;
    int32_t mdt = 0;
    int64_t mbatch = 1;
    int64_t ms[3] = {0, 0, 0};
    at::Tensor mask_t;
    if (mask.has_value()) {
        // the kernels read mask rows with unit key stride, rows not overlapping
        mask_t = (mask->stride(2) == 1 && (N < 2 || mask->stride(1) >= N)) ? *mask : mask->contiguous();
        const at::Tensor& m = mask_t;
        TORCH_CHECK(m.device() == dev, what, ": mask must be on the same device");
        TORCH_CHECK(m.dim() == 3 && m.size(1) == N && m.size(2) == N, what,
                    ": mask must have shape [M, N, N]");
        mdt = dtype_code(m.scalar_type());
        TORCH_CHECK(mdt >= 0, what, ": mask dtype must be float32, float16 or bfloat16");
        mbatch = m.size(0);
        TORCH_CHECK(mbatch > 0 && B % mbatch == 0, what, ": mask batch ", mbatch,
                    " must divide the window batch ", B);
        for (int i = 0; i < 3; ++i) ms[i] = m.stride(i);
        if (mbatch == 1) ms[0] = 0;
        mptr = m.data_ptr();
    }
    const uint8_t* bptr = nullptr;
    if (boundary.has_value()) {
        const at::Tensor& bd = *boundary;
        TORCH_CHECK(bd.device() == dev, what, ": boundary must be on the same device");
        TORCH_CHECK(bd.scalar_type() == at::kByte || bd.scalar_type() == at::kBool, what,
                    ": boundary must be uint8 or bool");
        TORCH_CHECK(bd.dim() == 1 && bd.size(0) == B && bd.is_contiguous(), what,
                    ": boundary must be a contiguous [B] tensor");
        bptr = static_cast<const uint8_t*>(bd.data_ptr());
    }
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(dev);
    if (out.numel() == 0) return;
    int64_t qs[4], ks[4], vs[4], os[4], bs[3];
    for (int i = 0; i < 4; ++i) {
        qs[i] = q.stride(i);
        ks[i] = k.stride(i);
        vs[i] = v.stride(i);
        os[i] = out.stride(i);
    }
    // the kernels read bias rows with unit key stride, rows not overlapping
    const at::Tensor bk = (bias.stride(2) == 1 && (N < 2 || bias.stride(1) >= N)) ? bias : bias.contiguous();
    for (int i = 0; i < 3; ++i) bs[i] = bk.stride(i);
    if (tiles != nullptr) {
        TORCH_CHECK(mask.has_value(), what, ": mask is required");
        TORCH_CHECK(tiles->device() == dev && tiles->scalar_type() == mask->scalar_type() &&
                        tiles->is_contiguous() &&
                        tiles->numel() == crumpet_attn_mask_tiles_elements(mbatch, N),
                    what, ": mask_tiles must be attn_mask_tiles(mask)");
        check_status(crumpet_fused_swin_attention_tiled(
            out.data_ptr(), os, q.data_ptr(), qs, k.data_ptr(), ks, v.data_ptr(), vs, dt, B, Hh, N, Dh,
            bk.data_ptr(), bdt, bs, mptr, mdt, mbatch, ms, tiles->data_ptr(), bptr,
            static_cast<float>(scale), stream_of(q)));
        return;
    }
    check_status(crumpet_fused_swin_attention(
        out.data_ptr(), os, q.data_ptr(), qs, k.data_ptr(), ks, v.data_ptr(), vs, dt, B, Hh, N, Dh,
        bk.data_ptr(), bdt, bs, mptr, mdt, mbatch, ms, bptr, static_cast<float>(scale),
        stream_of(q)));
}

void fused_swin_attention(at::Tensor& out, const at::Tensor& q, const at::Tensor& k,
                          const at::Tensor& v, const at::Tensor& bias,
                          const std::optional<at::Tensor>& mask,
                          const std::optional<at::Tensor>& boundary, double scale) {
    run_fused_swin_attention("fused_swin_attention", out, q, k, v, bias, mask, nullptr, boundary, scale);
}

void fused_swin_attention_tiled(at::Tensor& out, const at::Tensor& q, const at::Tensor& k,
                                const at::Tensor& v, const at::Tensor& bias, const at::Tensor& mask,
                                const at::Tensor& mask_tiles, const std::optional<at::Tensor>& boundary,
                                double scale) {
    run_fused_swin_attention("fused_swin_attention_tiled", out, q, k, v, bias, mask, &mask_tiles, boundary,
                             scale);
}

void attn_mask_tiles(at::Tensor& out, const at::Tensor& mask) {
    const char* what = "attn_mask_tiles";
    TORCH_CHECK(mask.dim() == 3 && mask.size(1) == mask.size(2), what, ": mask must have shape [M, N, N]");
    const int32_t mdt = dtype_code(mask.scalar_type());
    TORCH_CHECK(mdt == CRUMPET_DTYPE_F16 || mdt == CRUMPET_DTYPE_BF16, what,
                ": mask dtype must be float16 or bfloat16");
    TORCH_CHECK(out.is_cuda() && mask.is_cuda() && out.device() == mask.device(), what,
                ": out and mask must be on the same HIP device");
    const int64_t M = mask.size(0), N = mask.size(1);
    const int64_t n = crumpet_attn_mask_tiles_elements(M, N);
    TORCH_CHECK(n >= 0, what, ": N = ", N, " is outside 1 .. 512");
    TORCH_CHECK(out.scalar_type() == mask.scalar_type() && out.is_contiguous() && out.numel() == n, what,
                ": out must be a contiguous tensor of the mask's dtype with attn_mask_tiles_elements(M, N) elements");
    if (n == 0) return;
    const at::Tensor m = mask.stride(2) == 1 ? mask : mask.contiguous();
    const int64_t ms[3] = {m.stride(0), m.stride(1), m.stride(2)};
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(mask.device());
    check_status(crumpet_attn_mask_tiles(out.data_ptr(), m.data_ptr(), mdt, M, N, ms, stream_of(mask)));
}

void fused_swin_attention_shifted(at::Tensor& out, const at::Tensor& q, const at::Tensor& k,
                                  const at::Tensor& v, const at::Tensor& bias, int64_t D,
                                  int64_t H, int64_t W, int64_t ws_d, int64_t ws_h, int64_t ws_w,
                                  int64_t ss_d, int64_t ss_h, int64_t ss_w, double scale) {
    const char* what = "fused_swin_attention_shifted";
    TORCH_CHECK(q.dim() == 4, what, ": q must have shape [B, H, N, D]");
    TORCH_CHECK(k.sizes() == q.sizes() && v.sizes() == q.sizes() && out.sizes() == q.sizes(), what,
                ": q, k, v and out must have the same shape");
    TORCH_CHECK(k.scalar_type() == q.scalar_type() && v.scalar_type() == q.scalar_type() &&
                    out.scalar_type() == q.scalar_type(),
                what, ": q, k, v and out must have the same dtype");
    const int32_t dt = dtype_code(q.scalar_type());
    TORCH_CHECK(dt >= 0, what, ": dtype must be float32, float16 or bfloat16");
    const at::Device dev = q.device();
    TORCH_CHECK(q.is_cuda() && k.device() == dev && v.device() == dev && out.device() == dev &&
                    bias.device() == dev,
                what, ": all tensors must be on the same HIP device");
    const int64_t B = q.size(0), Hh = q.size(1), N = q.size(2), Dh = q.size(3);
    TORCH_CHECK(bias.dim() == 3 && bias.size(0) == Hh && bias.size(1) == N && bias.size(2) == N,
                what, ": relative_position_bias must have shape [H, N, N]");
    const int32_t bdt = dtype_code(bias.scalar_type());
    TORCH_CHECK(bdt >= 0, what, ": bias dtype must be float32, float16 or bfloat16");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(dev);
    if (out.numel() == 0) return;
    int64_t qs[4], ks[4], vs[4], os[4], bs[3];
    for (int i = 0; i < 4; ++i) {
        qs[i] = q.stride(i);
        ks[i] = k.stride(i);
        vs[i] = v.stride(i);
        os[i] = out.stride(i);
    }
    // the kernels read bias rows with unit key stride, rows not overlapping
    const at::Tensor bk = (bias.stride(2) == 1 && (N < 2 || bias.stride(1) >= N)) ? bias : bias.contiguous();
    for (int i = 0; i < 3; ++i) bs[i] = bk.stride(i);
    check_status(crumpet_fused_swin_attention_shifted(
        out.data_ptr(), os, q.data_ptr(), qs, k.data_ptr(), ks, v.data_ptr(), vs, dt, B, Hh, N, Dh,
        bk.data_ptr(), bdt, bs, D, H, W, ws_d, ws_h, ws_w, ss_d, ss_h, ss_w,
        static_cast<float>(scale), stream_of(q)));
}

// Linear weight [n_out, C] and optional bias [n_out], contiguous, in `dt`.
void check_linear_params(const at::Tensor& weight, const std::optional<at::Tensor>& bias,
                         int64_t C, at::ScalarType dt, const at::Device& dev, const char* what) {
    TORCH_CHECK(weight.dim() == 2 && weight.size(1) == C, what, ": weight must have shape [n_out, ", C,
                "]");
    TORCH_CHECK(weight.scalar_type() == dt && weight.device() == dev && weight.is_contiguous(), what,
                ": weight must be a contiguous tensor of the output dtype on the output's device");
    if (bias.has_value()) {
        TORCH_CHECK(bias->dim() == 1 && bias->size(0) == weight.size(0), what,
                    ": bias must have shape [n_out]");
        TORCH_CHECK(bias->scalar_type() == dt && bias->device() == dev && bias->is_contiguous(), what,
                    ": bias must be a contiguous tensor of the output dtype on the output's device");
    }
}

void window_qkv_3d(at::Tensor& out, const at::Tensor& x, const std::optional<at::Tensor>& norm_weight,
                   const std::optional<at::Tensor>& norm_bias, double eps, bool normalize,
                   const at::Tensor& weight, const std::optional<at::Tensor>& bias, int64_t ws_d,
                   int64_t ws_h, int64_t ws_w, int64_t ss_d, int64_t ss_h, int64_t ss_w) {
    const char* what = "window_qkv_3d";
    TORCH_CHECK(x.dim() == 5, what, ": x must have shape [B, D, H, W, C]");
    TORCH_CHECK(x.is_cuda() && out.device() == x.device(), what,
                ": x and out must be on the same HIP device");
    TORCH_CHECK(x.is_contiguous() && out.is_contiguous(), what, ": x and out must be contiguous");
    const int32_t xdt = dtype_code(x.scalar_type());
    const int32_t dt = dtype_code(out.scalar_type());
    TORCH_CHECK(xdt >= 0 && dt >= 0, what, ": dtypes must be float32, float16 or bfloat16");
    const int64_t B = x.size(0), D = x.size(1), H = x.size(2), W = x.size(3), C = x.size(4);
    check_linear_params(weight, bias, C, out.scalar_type(), x.device(), what);
    const int64_t n_out = weight.size(0);
    TORCH_CHECK(ws_d > 0 && ws_h > 0 && ws_w > 0, what, ": window_size values must be positive");
    const int64_t Dp = (D + ws_d - 1) / ws_d * ws_d, Hp = (H + ws_h - 1) / ws_h * ws_h,
                  Wp = (W + ws_w - 1) / ws_w * ws_w;
    const int64_t N = ws_d * ws_h * ws_w;
    TORCH_CHECK(out.dim() == 3 && out.size(0) == B * (Dp / ws_d) * (Hp / ws_h) * (Wp / ws_w) &&
                    out.size(1) == N && out.size(2) == n_out,
                what, ": out must have shape [B*nW, N, n_out] over the volume padded to the window grid");
    const void* lw = nullptr;
    const void* lb = nullptr;
    int32_t ldt = CRUMPET_DTYPE_F32;
    for (const auto* p : {&norm_weight, &norm_bias}) {
        if (!p->has_value()) continue;
        const at::Tensor& t = p->value();
        TORCH_CHECK(t.dim() == 1 && t.size(0) == C && t.is_contiguous() && t.device() == x.device(), what,
                    ": LayerNorm parameters must be contiguous [C] tensors on x's device");
        ldt = dtype_code(t.scalar_type());
        TORCH_CHECK(ldt >= 0, what, ": LayerNorm parameter dtype must be float32, float16 or bfloat16");
    }
    if (norm_weight.has_value() && norm_bias.has_value())
        TORCH_CHECK(norm_weight->scalar_type() == norm_bias->scalar_type(), what,
                    ": LayerNorm weight and bias must share a dtype");
    if (norm_weight.has_value()) lw = norm_weight->data_ptr();
    if (norm_bias.has_value()) lb = norm_bias->data_ptr();
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    check_status(crumpet_window_qkv_3d(out.data_ptr(), dt, x.data_ptr(), xdt, B, D, H, W, C,
                                       normalize ? 1 : 0, lw, lb, ldt, static_cast<float>(eps),
                                       weight.data_ptr(), bias.has_value() ? bias->data_ptr() : nullptr,
                                       n_out, ws_d, ws_h, ws_w, ss_d, ss_h, ss_w, stream_of(x)));
}

void window_proj_3d(at::Tensor& out, const at::Tensor& windows, const at::Tensor& weight,
                    const std::optional<at::Tensor>& bias, int64_t ws_d, int64_t ws_h, int64_t ws_w,
                    int64_t ss_d, int64_t ss_h, int64_t ss_w) {
    const char* what = "window_proj_3d";
    TORCH_CHECK(out.dim() == 5, what, ": out must have shape [B, D, H, W, n_out]");
    TORCH_CHECK(windows.is_cuda() && out.device() == windows.device(), what,
                ": windows and out must be on the same HIP device");
    TORCH_CHECK(windows.is_contiguous() && out.is_contiguous(), what,
                ": windows and out must be contiguous");
    TORCH_CHECK(windows.scalar_type() == out.scalar_type(), what, ": windows and out dtypes differ");
    const int32_t dt = dtype_code(out.scalar_type());
    TORCH_CHECK(dt >= 0, what, ": dtype must be float32, float16 or bfloat16");
    TORCH_CHECK(windows.dim() == 3, what, ": windows must have shape [B*nW, N, C]");
    const int64_t C = windows.size(2);
    check_linear_params(weight, bias, C, out.scalar_type(), out.device(), what);
    const int64_t B = out.size(0), D = out.size(1), H = out.size(2), W = out.size(3);
    TORCH_CHECK(out.size(4) == weight.size(0), what, ": out's last dim must equal n_out");
    TORCH_CHECK(ws_d > 0 && ws_h > 0 && ws_w > 0, what, ": window_size values must be positive");
    const int64_t Dp = (D + ws_d - 1) / ws_d * ws_d, Hp = (H + ws_h - 1) / ws_h * ws_h,
                  Wp = (W + ws_w - 1) / ws_w * ws_w;
    TORCH_CHECK(windows.size(0) == B * (Dp / ws_d) * (Hp / ws_h) * (Wp / ws_w) &&
                    windows.size(1) == ws_d * ws_h * ws_w,
                what, ": windows must have shape [B*nW, N, C] over the volume padded to the window grid");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(out.device());
    check_status(crumpet_window_proj_3d(out.data_ptr(), windows.data_ptr(), dt, B, D, H, W, C,
                                        weight.data_ptr(), bias.has_value() ? bias->data_ptr() : nullptr,
                                        weight.size(0), ws_d, ws_h, ws_w, ss_d, ss_h, ss_w,
                                        stream_of(out)));
}

// The attention half of a Swin block (norm1, pad to the window grid, roll,
// partition, qkv -> window attention -> proj, reverse, roll back, crop) as
// one call: window_qkv_3d, the fused attention and window_proj_3d launched
// back to back, with the qkv and attention intermediates allocated here.
// A call from Python then costs one dispatch instead of three plus the
// allocations and views between them, which is most of a block's time at
// the deep stages.  A nonzero shift takes the shifted-window mask from the
// padded volume's geometry (fused_swin_attention_shifted); without a shift
// there is no mask.  Weights are in the compute dtype, which the outputs
// take.
at::Tensor window_msa_3d(const at::Tensor& x, const std::optional<at::Tensor>& norm_weight,
                         const std::optional<at::Tensor>& norm_bias, double eps, const at::Tensor& w_qkv,
                         const std::optional<at::Tensor>& b_qkv, const at::Tensor& w_proj,
                         const std::optional<at::Tensor>& b_proj, const at::Tensor& bias, int64_t heads,
                         double scale, int64_t ws_d, int64_t ws_h, int64_t ws_w, int64_t ss_d, int64_t ss_h,
                         int64_t ss_w) {
    const char* what = "window_msa_3d";
    TORCH_CHECK(x.dim() == 5, what, ": x must have shape [B, D, H, W, C]");
    TORCH_CHECK(w_qkv.dim() == 2 && w_qkv.size(0) % 3 == 0, what, ": w_qkv must have shape [3 C, C_in]");
    const int64_t Ca = w_qkv.size(0) / 3;  // attention width
    TORCH_CHECK(heads > 0 && Ca % heads == 0, what, ": heads must divide the attention width");
    TORCH_CHECK(w_proj.dim() == 2, what, ": w_proj must have shape [C_out, C]");
    TORCH_CHECK(ws_d > 0 && ws_h > 0 && ws_w > 0, what, ": window_size values must be positive");
    const int64_t B = x.size(0), D = x.size(1), H = x.size(2), W = x.size(3);
    const int64_t Dp = (D + ws_d - 1) / ws_d * ws_d, Hp = (H + ws_h - 1) / ws_h * ws_h,
                  Wp = (W + ws_w - 1) / ws_w * ws_w;
    const int64_t nwin = B * (Dp / ws_d) * (Hp / ws_h) * (Wp / ws_w), n = ws_d * ws_h * ws_w;
    const auto opts = x.options().dtype(w_qkv.scalar_type());
    at::Tensor qkv = at::empty({nwin, n, 3 * Ca}, opts);
    window_qkv_3d(qkv, x.contiguous(), norm_weight, norm_bias, eps, true, w_qkv, b_qkv, ws_d, ws_h, ws_w, ss_d,
                  ss_h, ss_w);
    // q, k, v: [nwin, heads, n, hd] views of the [token][3][heads][hd] rows
    const at::Tensor t = qkv.view({nwin, n, 3, heads, Ca / heads}).permute({2, 0, 3, 1, 4});
    at::Tensor attn = at::empty({nwin, n, heads, Ca / heads}, opts);
    at::Tensor ov = attn.permute({0, 2, 1, 3});
    if (ss_d > 0 || ss_h > 0 || ss_w > 0)
        fused_swin_attention_shifted(ov, t.select(0, 0), t.select(0, 1), t.select(0, 2), bias, Dp, Hp, Wp, ws_d,
                                     ws_h, ws_w, ss_d, ss_h, ss_w, scale);
    else
        fused_swin_attention(ov, t.select(0, 0), t.select(0, 1), t.select(0, 2), bias, std::nullopt,
                             std::nullopt, scale);
    at::Tensor y = at::empty({B, D, H, W, w_proj.size(0)}, opts);
    window_proj_3d(y, attn.view({nwin, n, Ca}), w_proj, b_proj, ws_d, ws_h, ws_w, ss_d, ss_h, ss_w);
    return y;
}

}  // namespace

TORCH_LIBRARY(crumpet_ops, ops) {
    ops.def(
        "compute_attn_mask_3d(Tensor! output, int D, int H, int W, int ws_d, int ws_h, int ws_w, "
        "int ss_d, int ss_h, int ss_w) -> ()",
        kCrumpetOpTags);
    ops.def(
        "fused_shift_partition_3d(Tensor! output, Tensor x, int ws_d, int ws_h, int ws_w, "
        "int ss_d, int ss_h, int ss_w) -> ()",
        kCrumpetOpTags);
    ops.def(
        "fused_shift_partition_3d_backward(Tensor! grad_x, Tensor grad_windows, int B, int D, "
        "int H, int W, int C, int ws_d, int ws_h, int ws_w, int ss_d, int ss_h, int ss_w) -> ()",
        kCrumpetOpTags);
    ops.def(
        "fused_unshift_unpartition_3d(Tensor! output, Tensor windows, int B, int D, int H, int W, "
        "int C, int ws_d, int ws_h, int ws_w, int ss_d, int ss_h, int ss_w) -> ()",
        kCrumpetOpTags);
    ops.def(
        "fused_unshift_unpartition_3d_backward(Tensor! grad_windows, Tensor grad_x, int ws_d, "
        "int ws_h, int ws_w, int ss_d, int ss_h, int ss_w) -> ()",
        kCrumpetOpTags);
    ops.def(
        "fused_swin_attention(Tensor! out, Tensor q, Tensor k, Tensor v, Tensor bias, "
        "Tensor? mask, Tensor? boundary, float scale) -> ()",
        kCrumpetOpTags);
    ops.def(
        "fused_swin_attention_tiled(Tensor! out, Tensor q, Tensor k, Tensor v, Tensor bias, "
        "Tensor mask, Tensor mask_tiles, Tensor? boundary, float scale) -> ()",
        kCrumpetOpTags);
    ops.def("attn_mask_tiles(Tensor! out, Tensor mask) -> ()", kCrumpetOpTags);
    ops.def(
        "fused_swin_attention_shifted(Tensor! out, Tensor q, Tensor k, Tensor v, Tensor bias, "
        "int D, int H, int W, int ws_d, int ws_h, int ws_w, int ss_d, int ss_h, int ss_w, "
        "float scale) -> ()",
        kCrumpetOpTags);
    ops.def(
        "window_qkv_3d(Tensor! out, Tensor x, Tensor? norm_weight, Tensor? norm_bias, float eps, "
        "bool normalize, Tensor weight, Tensor? bias, int ws_d, int ws_h, int ws_w, int ss_d, "
        "int ss_h, int ss_w) -> ()",
        kCrumpetOpTags);
    ops.def(
        "window_proj_3d(Tensor! out, Tensor windows, Tensor weight, Tensor? bias, int ws_d, int ws_h, "
        "int ws_w, int ss_d, int ss_h, int ss_w) -> ()",
        kCrumpetOpTags);
    ops.def(
        "window_msa_3d(Tensor x, Tensor? norm_weight, Tensor? norm_bias, float eps, Tensor w_qkv, "
        "Tensor? b_qkv, Tensor w_proj, Tensor? b_proj, Tensor bias, int heads, float scale, int ws_d, "
        "int ws_h, int ws_w, int ss_d, int ss_h, int ss_w) -> Tensor",
        kCrumpetOpTags);
}

TORCH_LIBRARY_IMPL(crumpet_ops, CUDA, ops) {
    ops.impl("compute_attn_mask_3d", &compute_attn_mask_3d);
    ops.impl("fused_shift_partition_3d", &fused_shift_partition_3d);
    ops.impl("fused_shift_partition_3d_backward", &fused_shift_partition_3d_backward);
    ops.impl("fused_unshift_unpartition_3d", &fused_unshift_unpartition_3d);
    ops.impl("fused_unshift_unpartition_3d_backward", &fused_unshift_unpartition_3d_backward);
    ops.impl("fused_swin_attention", &fused_swin_attention);
    ops.impl("fused_swin_attention_shifted", &fused_swin_attention_shifted);
    ops.impl("fused_swin_attention_tiled", &fused_swin_attention_tiled);
    ops.impl("attn_mask_tiles", &attn_mask_tiles);
    ops.impl("window_qkv_3d", &window_qkv_3d);
    ops.impl("window_proj_3d", &window_proj_3d);
    ops.impl("window_msa_3d", &window_msa_3d);
}
