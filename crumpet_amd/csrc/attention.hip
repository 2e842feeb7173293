// Host side of the fused window attention: argument checks, the padded
// fp32 bias workspace, and dispatch to the per-dtype kernel instantiations
// (attention_f16.hip, attention_bf16.hip, attention_f32.hip; the kernel
// itself is in attention_kernel.h).
//
// Replaces the Triton launch of torch-ext/crumpet/fused_attention.py:149-226.
#include <hip/hip_runtime.h>

#include <math.h>

#include "attention_kernel.h"
#include "crumpet_common.h"
#include "crumpet_hip.h"

namespace crumpet {
namespace {

constexpr int kPrepThreads = 256;

// Padded fp32 copy of the bias: ws[h][i][j] = bias[h][i][j] for i, j < N,
// -inf in padded key columns, 0 in padded query rows of real keys.
template <typename TB>
__global__ void __launch_bounds__(kPrepThreads)
bias_prep_kernel(float* __restrict__ ws, const TB* __restrict__ bias, int64_t sh, int64_t si,
                 int64_t sj, int32_t H, int32_t N, int32_t NP) {
    const int64_t total = int64_t(H) * NP * NP;
    for (int64_t idx = int64_t(blockIdx.x) * kPrepThreads + threadIdx.x; idx < total;
         idx += int64_t(gridDim.x) * kPrepThreads) {
        const int32_t j = static_cast<int32_t>(idx % NP);
        const int64_t r = idx / NP;
        const int32_t i = static_cast<int32_t>(r % NP);
        const int32_t h = static_cast<int32_t>(r / NP);
        float val;
        if (j >= N)
            val = -INFINITY;
        else if (i >= N)
            val = 0.0f;
        else
            val = static_cast<float>(bias[h * sh + i * si + j * sj]);
        ws[idx] = val;
    }
}

int dtype_size(int32_t dt) {
    switch (dt) {
        case CRUMPET_DTYPE_F32: return 4;
        case CRUMPET_DTYPE_F16: return 2;
        case CRUMPET_DTYPE_BF16: return 2;
        default: return 0;
    }
}

}  // namespace
}  // namespace crumpet

extern "C" size_t crumpet_fused_swin_attention_workspace_size(int64_t Hh, int64_t N) {
    if (Hh <= 0 || N <= 0) return 0;
    const int nt = crumpet::attn::select_tiles(N);
    if (nt < 0) return 0;
    const int64_t np = 16 * nt;
    return static_cast<size_t>(Hh * np * np * int64_t(sizeof(float)));
}

extern "C" int crumpet_fused_swin_attention(
    void* out, const int64_t out_strides[4], const void* q, const int64_t q_strides[4],
    const void* k, const int64_t k_strides[4], const void* v, const int64_t v_strides[4],
    int32_t dtype, int64_t B, int64_t Hh, int64_t N, int64_t Dh, const void* bias,
    int32_t bias_dtype, const int64_t bias_strides[3], const void* mask, int32_t mask_dtype,
    int64_t mask_batch, const int64_t mask_strides[3], const uint8_t* boundary, float scale,
    void* workspace, size_t workspace_bytes, void* stream) {
    using namespace crumpet;
    const char* what = "crumpet_fused_swin_attention";
    const int esize = dtype_size(dtype);
    if (esize == 0) return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: unsupported dtype %d", what, dtype);
    if (B < 0 || Hh < 0 || N < 0 || Dh <= 0)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: negative size", what);
    if (B == 0 || Hh == 0 || N == 0) return CRUMPET_OK;
    if (Dh != 16)
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: head_dim %lld is not supported (16)", what,
                    (long long)Dh);
    if (N > 512)
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: N = %lld exceeds 512 tokens per window", what,
                    (long long)N);
    if (B * Hh > 0x7fffffffLL)
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: too many (window, head) pairs", what);
    if (!out || !q || !k || !v || !bias || !out_strides || !q_strides || !k_strides ||
        !v_strides || !bias_strides)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: null pointer argument", what);
    if (dtype_size(bias_dtype) == 0)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: unsupported bias dtype %d", what, bias_dtype);
    if (mask != nullptr) {
        if (dtype_size(mask_dtype) == 0)
            return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: unsupported mask dtype %d", what,
                        mask_dtype);
        if (!mask_strides)
            return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: null mask strides", what);
        if (mask_strides[2] != 1)
            return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: mask must have unit stride along keys",
                        what);
        if (mask_strides[0] < 0 || mask_strides[1] < 0 ||
            ((N - 1) * mask_strides[1] + N) * 4 >= (int64_t(1) << 31))
            return fail(CRUMPET_ERR_UNSUPPORTED, "%s: mask row stride out of range", what);
        if (mask_batch <= 0 || B % mask_batch != 0)
            return fail(CRUMPET_ERR_INVALID_ARGUMENT,
                        "%s: mask batch %lld must divide the window batch %lld", what,
                        (long long)mask_batch, (long long)B);
    }
    const size_t need = crumpet_fused_swin_attention_workspace_size(Hh, N);
    if (workspace == nullptr || workspace_bytes < need ||
        reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT,
                    "%s: workspace must be 16-byte aligned and hold %zu bytes", what, need);

    const int NT = attn::select_tiles(N);
    const int NP = 16 * NT;
    attn::Params p;
    p.q = q; p.k = k; p.v = v; p.out = out;
    for (int i = 0; i < 4; ++i) {
        p.qs[i] = q_strides[i];
        p.ks[i] = k_strides[i];
        p.vs[i] = v_strides[i];
        p.os[i] = out_strides[i];
    }
    p.bias_ws = static_cast<const float*>(workspace);
    p.mask = mask;
    for (int i = 0; i < 3; ++i) p.ms[i] = mask ? mask_strides[i] : 0;
    p.mask_batch = mask ? static_cast<int32_t>(mask_batch) : 1;
    p.boundary = boundary;
    p.scale = scale;
    p.B = static_cast<int32_t>(B);
    p.H = static_cast<int32_t>(Hh);
    p.N = static_cast<int32_t>(N);
    p.strips = static_cast<int32_t>((N + 15) / 16);

    // 4-element vector IO needs unit d stride, 4-element aligned row strides and bases.
    bool vec = true;
    const int64_t* st[4] = {q_strides, k_strides, v_strides, out_strides};
    const void* ptr[4] = {q, k, v, out};
    for (int i = 0; i < 4; ++i) {
        if (st[i][3] != 1 || st[i][0] % 4 || st[i][1] % 4 || st[i][2] % 4 ||
            reinterpret_cast<uintptr_t>(ptr[i]) % (4 * esize))
            vec = false;
    }
    p.vec_io = vec ? 1 : 0;
    p.chunks = static_cast<uint32_t>(B * Hh);
    p.launched = xcd_launch_count(p.chunks);

    hipStream_t s = static_cast<hipStream_t>(stream);
    {
        const int64_t total = Hh * NP * NP;
        int64_t blocks = (total + kPrepThreads - 1) / kPrepThreads;
        if (blocks > 4096) blocks = 4096;
        float* ws = static_cast<float*>(workspace);
        if (bias_dtype == CRUMPET_DTYPE_F16)
            hipLaunchKernelGGL(bias_prep_kernel<_Float16>, dim3(blocks), dim3(kPrepThreads), 0, s, ws,
                               static_cast<const _Float16*>(bias), bias_strides[0],
                               bias_strides[1], bias_strides[2], p.H, p.N, NP);
        else if (bias_dtype == CRUMPET_DTYPE_BF16)
            hipLaunchKernelGGL(bias_prep_kernel<__bf16>, dim3(blocks), dim3(kPrepThreads), 0, s, ws,
                               static_cast<const __bf16*>(bias), bias_strides[0],
                               bias_strides[1], bias_strides[2], p.H, p.N, NP);
        else
            hipLaunchKernelGGL(bias_prep_kernel<float>, dim3(blocks), dim3(kPrepThreads), 0, s, ws,
                               static_cast<const float*>(bias), bias_strides[0], bias_strides[1],
                               bias_strides[2], p.H, p.N, NP);
        const int st2 = check_launch(what);
        if (st2 != CRUMPET_OK) return st2;
    }
    const int kmask = mask == nullptr                     ? attn::kNoMask
                      : mask_dtype == CRUMPET_DTYPE_F32  ? attn::kMaskF32
                      : mask_dtype == CRUMPET_DTYPE_BF16 ? attn::kMaskBF16
                                                         : attn::kMaskF16;
    if (dtype == CRUMPET_DTYPE_F16)
        attn::launch_f16(p, NT, kmask, s);
    else if (dtype == CRUMPET_DTYPE_BF16)
        attn::launch_bf16(p, NT, kmask, s);
    else
        attn::launch_f32(p, NT, kmask, s);
    return check_launch(what);
}
