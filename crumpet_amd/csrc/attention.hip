// Host side of the fused window attention: argument checks, the window-type
// table of the region mode, the work decomposition, and dispatch to the
// per-dtype kernel instantiations (attention_f16.hip, attention_bf16.hip,
// attention_f32.hip; the kernel itself is in attention_kernel.h).  Nothing
// here allocates: the kernel builds its bias tiles from the bias tensor.
//
// Replaces the Triton launch of torch-ext/crumpet/fused_attention.py:149-226.
#include <hip/hip_runtime.h>

#include <math.h>

#include <algorithm>

#include "attention_kernel.h"
#include "crumpet_common.h"
#include "crumpet_hip.h"

namespace crumpet {
namespace {

// Workgroups a call aims for: each walks win_per_wg windows.  1536 = two
// full rounds of 3 resident workgroups on each of the 256 CUs (the 2-byte
// vector-IO kernels run 3 waves per SIMD); a partial last round costs more
// than the extra prologues of smaller ranges.
constexpr int64_t kTargetWorkgroups = 1536;
// Workgroups of kHeadsPerWg slots (heads, or head-dim-32 strip groups)
// take most of a CU's LDS: one per CU, 256 CUs
constexpr int64_t kTargetWorkgroupsMultiHead = 256;

int dtype_size(int32_t dt) {
    switch (dt) {
        case CRUMPET_DTYPE_F32: return 4;
        case CRUMPET_DTYPE_F16: return 2;
        case CRUMPET_DTYPE_BF16: return 2;
        default: return 0;
    }
}

struct Region {
    int64_t D, H, W, ws[3], ss[3];
};

// Shared path of both entry points.  mask/boundary describe tensor mode;
// region (nullable) selects region mode.
int run_attention(const char* what, void* out, const int64_t out_strides[4], const void* q,
                  const int64_t q_strides[4], const void* k, const int64_t k_strides[4],
                  const void* v, const int64_t v_strides[4], int32_t dtype, int64_t B, int64_t Hh,
                  int64_t N, int64_t Dh, const void* bias, int32_t bias_dtype,
                  const int64_t bias_strides[3], const void* mask, int32_t mask_dtype,
                  int64_t mask_batch, const int64_t mask_strides[3], const void* mask_tiles,
                  const uint8_t* boundary, const Region* region, float scale, void* stream) {
    const int esize = dtype_size(dtype);
    if (esize == 0) return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: unsupported dtype %d", what, dtype);
    if (B < 0 || Hh < 0 || N < 0 || Dh <= 0)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: negative size", what);
    if (B == 0 || Hh == 0 || N == 0) return CRUMPET_OK;
    // head dim 16 with N <= 512 (every Swin UNETR stage) runs the tuned
    // kernel; other head dims and larger windows the general one
    if (Dh != 16 && Dh != 32 && Dh != 64 && Dh != 128 && Dh != 256)
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: head_dim %lld is not supported (16, 32, 64, 128 or 256)",
                    what, (long long)Dh);
    // The tuned kernel feeds q * scale * log2(e) to the score product (its
    // scores come out in log2 units).  An fp16 q is at most 65504, so that
    // product can overflow fp16 only for |scale| > ln 2; such calls run the
    // general kernel, which rounds q * scale as the reference does.
    const bool fold_log2e = !(dtype == CRUMPET_DTYPE_F16 && fabsf(scale) > 0.6931472f);
    const bool wide = Dh != 16 || N > 512 || !fold_log2e;
    if (wide && N > 0x3fffffffLL)
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: N = %lld is too large", what, (long long)N);
    if (wide && region != nullptr && N > attn::kWideMaxRegionN)
        return fail(CRUMPET_ERR_UNSUPPORTED,
                    "%s: shifted windows of %lld tokens exceed %d", what, (long long)N,
                    attn::kWideMaxRegionN);
    if (wide && B * Hh * ((N + attn::kWideQueries - 1) / attn::kWideQueries) >= 0x7fffff00LL)
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: too many (window, head, query block) triples", what);
    if (B * Hh > 0x7fffffffLL || B > 0x3fffffffLL)
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: too many (window, head) pairs", what);
    if (!out || !q || !k || !v || !bias || !out_strides || !q_strides || !k_strides ||
        !v_strides || !bias_strides)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: null pointer argument", what);
    if (dtype_size(bias_dtype) == 0)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: unsupported bias dtype %d", what, bias_dtype);
    if (bias_strides[2] != 1 || bias_strides[0] < 0 || bias_strides[1] < 0)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT,
                    "%s: bias must have unit stride along keys", what);
    // rows are read with multi-element loads: they must not overlap
    if (N > 1 && bias_strides[1] < N)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: bias rows must not overlap (row stride < N)", what);
    if (((N - 1) * bias_strides[1] + N) * dtype_size(bias_dtype) >= (int64_t(1) << 31))
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: bias row stride out of range", what);
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
        if (N > 1 && mask_strides[1] < N)
            return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: mask rows must not overlap (row stride < N)",
                        what);
        if (mask_batch <= 0 || B % mask_batch != 0)
            return fail(CRUMPET_ERR_INVALID_ARGUMENT,
                        "%s: mask batch %lld must divide the window batch %lld", what,
                        (long long)mask_batch, (long long)B);
    }

    attn::Params p = {};
    for (int a = 0; a < 3; ++a) {
        p.ws[a] = 1;
        p.ss[a] = 0;
    }
    if (region != nullptr) {
        const Region& rg = *region;
        for (int a = 0; a < 3; ++a) {
            if (rg.ws[a] <= 0 || rg.ss[a] < 0 || rg.ss[a] >= rg.ws[a])
                return fail(CRUMPET_ERR_INVALID_ARGUMENT,
                            "%s: shift_size must satisfy 0 <= shift < window_size", what);
        }
        if (rg.D <= 0 || rg.H <= 0 || rg.W <= 0 || rg.D % rg.ws[0] || rg.H % rg.ws[1] ||
            rg.W % rg.ws[2])
            return fail(CRUMPET_ERR_INVALID_ARGUMENT,
                        "%s: D, H and W must be divisible by window_size", what);
        if (rg.ws[0] * rg.ws[1] * rg.ws[2] != N)
            return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: window volume must equal N", what);
        const int64_t nWd = rg.D / rg.ws[0], nWh = rg.H / rg.ws[1], nWw = rg.W / rg.ws[2];
        const int64_t nW = nWd * nWh * nWw;
        if (B % nW != 0)
            return fail(CRUMPET_ERR_INVALID_ARGUMENT,
                        "%s: window batch %lld must be a multiple of the %lld windows per volume",
                        what, (long long)B, (long long)nW);
        p.nWd = nWd;
        p.nWh = nWh;
        p.nWw = nWw;
        p.nW = nW;
        const int64_t batches = B / nW;
        const int64_t nwin[3] = {nWd, nWh, nWw};
        int nt = 0;
        int64_t off = 0;
        for (int code = 0; code < 8; ++code) {
            int64_t ch[3];
            bool ok = true;
            for (int a = 0; a < 3; ++a) {
                const bool last = (code >> (2 - a)) & 1;
                const bool shifted = rg.ss[a] > 0;
                if (last && !shifted) ok = false;
                ch[a] = last ? 1 : (shifted ? nwin[a] - 1 : nwin[a]);
            }
            if (!ok) continue;
            const int64_t count = ch[0] * ch[1] * ch[2] * batches;
            if (count == 0) continue;
            p.types.code[nt] = code;
            for (int a = 0; a < 3; ++a) p.types.choices[nt][a] = static_cast<int32_t>(ch[a]);
            p.types.offset[nt] = static_cast<int32_t>(off);
            off += count;
            ++nt;
        }
        p.types.ntypes = nt;
        p.types.offset[nt] = static_cast<int32_t>(off);
        for (int a = 0; a < 3; ++a) {
            p.ws[a] = static_cast<int32_t>(rg.ws[a]);
            p.ss[a] = static_cast<int32_t>(rg.ss[a]);
        }
    }

    p.q = q;
    p.k = k;
    p.v = v;
    p.out = out;
    for (int i = 0; i < 4; ++i) {
        p.qs[i] = q_strides[i];
        p.ks[i] = k_strides[i];
        p.vs[i] = v_strides[i];
        p.os[i] = out_strides[i];
    }
    p.bias = bias;
    for (int i = 0; i < 3; ++i) p.bsd[i] = bias_strides[i];
    p.bias_dtype = bias_dtype;
    p.mask = mask;
    for (int i = 0; i < 3; ++i) p.ms[i] = mask ? mask_strides[i] : 0;
    p.mask_batch = mask ? static_cast<int32_t>(mask_batch) : 1;
    p.boundary = boundary;
    p.scale = scale;
    p.B = static_cast<int32_t>(B);
    p.H = static_cast<int32_t>(Hh);
    p.N = static_cast<int32_t>(N);
    // 4-element vector IO needs unit d stride, 4-element aligned row strides and bases.
    bool vec = true;
    const int64_t* st[4] = {q_strides, k_strides, v_strides, out_strides};
    const void* ptr[4] = {q, k, v, out};
    for (int i = 0; i < 4; ++i) {
        if (st[i][3] != 1 || st[i][0] % 4 || st[i][1] % 4 || st[i][2] % 4 ||
            reinterpret_cast<uintptr_t>(ptr[i]) % (4 * esize))
            vec = false;
    }
    // the vector paths address q/k/v and out rows of one (window, head) with
    // 32-bit byte offsets
    for (int i = 0; i < 4; ++i) {
        if (st[i][2] < 0 || ((N - 1) * st[i][2] + 16) * esize >= (int64_t(1) << 31)) vec = false;
    }
    p.vec_io = vec ? 1 : 0;

    hipStream_t s = static_cast<hipStream_t>(stream);
    const int kmask = region != nullptr                  ? attn::kMaskRegion
                      : mask == nullptr                  ? attn::kNoMask
                      : mask_dtype == CRUMPET_DTYPE_F32  ? attn::kMaskF32
                      : mask_dtype == CRUMPET_DTYPE_BF16 ? attn::kMaskBF16
                                                         : attn::kMaskF16;
    // head dim 32 runs the tuned kernel for 2-byte types with vector IO at
    // 14 or 22 tiles (129 <= N <= 352), addressed with 32-bit byte offsets
    bool tuned32 = Dh == 32 && dtype != CRUMPET_DTYPE_F32 && vec && N <= 512 && fold_log2e &&
                   attn::d32_tiles(attn::select_tiles(N));
    for (int i = 0; i < 3; ++i) {
        if (((N - 1) * st[i][2] + 32) * esize >= (int64_t(1) << 31)) tuned32 = false;
    }
    if (wide && !tuned32) {
        attn::launch_wide(p, static_cast<int>(Dh), kmask, dtype, mask_dtype, s);
        return check_launch(what);
    }

    const int NT = attn::select_tiles(N);
    p.strips = static_cast<int32_t>((N + 15) / 16);
    p.groups = (p.strips + attn::kWaves - 1) / attn::kWaves;
    // several heads per workgroup: 2-byte LDS-DMA path, large windows, no
    // mask tensor or a 16-bit one without boundary flags, H a multiple, heads
    // adjacent in the K and V rows and V at a fixed distance after K (same
    // strides), addressed from K's base with 32-bit byte offsets
    const int64_t kv_bytes = static_cast<const char*>(v) - static_cast<const char*>(k);
    const bool records = k_strides[1] == 16 && v_strides[1] == 16 && k_strides[0] == v_strides[0] &&
                         k_strides[2] == v_strides[2] && kv_bytes >= 0 && kv_bytes % esize == 0 &&
                         k_strides[2] >= 0 &&
                         ((N - 1) * k_strides[2] + kv_bytes / esize + 16 * attn::kHeadsPerWg) * esize <
                             (int64_t(1) << 31);
    p.hpw = (!tuned32 && dtype != CRUMPET_DTYPE_F32 && p.vec_io && attn::multi_head_tiles(NT) &&
             (!attn::mask_tensor(kmask) || (boundary == nullptr && kmask != attn::kMaskF32)) &&
             Hh % attn::kHeadsPerWg == 0 && records)
                ? attn::kHeadsPerWg
                : 1;
    p.kv_delta = p.hpw > 1 ? static_cast<int32_t>(kv_bytes / esize) : 0;
    // head dim 32 at 21 or 22 strips (321 <= N <= 352: the 7^3 windows):
    // kHeadsPerWg strip groups of one head per workgroup, sharing
    // double-buffered K and V (3 of 24 waves idle at most, as in the 4-wave
    // form; fewer strips would idle more of them).  fp32 masks need 2 waves
    // per SIMD, too few for the 12-wave workgroup.  With boundary flags the
    // 4-wave form stays: its three workgroups per CU mix flagged and clear
    // windows, where the strip groups would all wait on a flagged window's
    // mask together.
    const bool group_slots = tuned32 && attn::d32_group_slots(NT, p.strips) && kmask != attn::kMaskF32 &&
                             (!attn::mask_tensor(kmask) || boundary == nullptr);
    if (group_slots) {
        p.hpw = attn::kHeadsPerWg;
        p.kv_delta = 0;
        p.groups = (p.groups + attn::kHeadsPerWg - 1) / attn::kHeadsPerWg;  // blocks of strip groups
    }
    const int64_t units = (group_slots ? Hh : Hh / p.hpw) * p.groups;
    // At most `target` chunks (whole rounds of resident workgroups), so that
    // none waits for an extra round behind full ranges: ranges of
    // ceil(B * units / target) windows gave 264 chunks for 256 CUs at stages
    // 1 and 2.
    const int64_t target = p.hpw > 1 ? kTargetWorkgroupsMultiHead : kTargetWorkgroups;
    const int64_t max_ranges = std::max<int64_t>(1, target / units);
    int64_t wpw = (B + max_ranges - 1) / max_ranges;
    if (wpw < 1) wpw = 1;
    p.win_per_wg = static_cast<int32_t>(wpw);
    p.ranges = static_cast<int32_t>((B + wpw - 1) / wpw);
    const int64_t chunks = int64_t(p.ranges) * units;
    if (chunks > 0x7fffffffLL)
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: too many workgroups", what);
    p.chunks = static_cast<uint32_t>(chunks);
    p.launched = xcd_launch_count(p.chunks);

    // A 16-bit mask also given in the tiled layout (crumpet_attn_mask_tiles)
    // is read from there by the 2-byte kernels at 14 or 22 tiles with vector
    // IO: a wave's 4 keys per lane of a key tile are then 512 contiguous
    // bytes instead of 16 row pieces.  p.ms[0] becomes the elements of one
    // window's block.
    int kmask_run = kmask;
    if (mask_tiles != nullptr && (kmask == attn::kMaskF16 || kmask == attn::kMaskBF16) &&
        dtype != CRUMPET_DTYPE_F32 && p.vec_io && attn::multi_head_tiles(NT)) {
        p.mask = mask_tiles;
        p.ms[0] = int64_t(p.strips) * NT * 256;
        p.ms[1] = 0;
        p.ms[2] = 0;
        kmask_run = kmask == attn::kMaskF16 ? attn::kMaskF16T : attn::kMaskBF16T;
    }

    if (tuned32)
        attn::launch_d32(p, NT, kmask_run, dtype, s);
    else if (dtype == CRUMPET_DTYPE_F16)
        attn::launch_f16(p, NT, kmask_run, s);
    else if (dtype == CRUMPET_DTYPE_BF16)
        attn::launch_bf16(p, NT, kmask_run, s);
    else
        attn::launch_f32(p, NT, kmask_run, s);
    return check_launch(what);
}

}  // namespace
}  // namespace crumpet

extern "C" int crumpet_fused_swin_attention(
    void* out, const int64_t out_strides[4], const void* q, const int64_t q_strides[4],
    const void* k, const int64_t k_strides[4], const void* v, const int64_t v_strides[4],
    int32_t dtype, int64_t B, int64_t Hh, int64_t N, int64_t Dh, const void* bias,
    int32_t bias_dtype, const int64_t bias_strides[3], const void* mask, int32_t mask_dtype,
    int64_t mask_batch, const int64_t mask_strides[3], const uint8_t* boundary, float scale,
    void* stream) {
    return crumpet::run_attention("crumpet_fused_swin_attention", out, out_strides, q, q_strides,
                                  k, k_strides, v, v_strides, dtype, B, Hh, N, Dh, bias,
                                  bias_dtype, bias_strides, mask, mask_dtype, mask_batch,
                                  mask_strides, nullptr, boundary, nullptr, scale, stream);
}

extern "C" int crumpet_fused_swin_attention_tiled(
    void* out, const int64_t out_strides[4], const void* q, const int64_t q_strides[4],
    const void* k, const int64_t k_strides[4], const void* v, const int64_t v_strides[4],
    int32_t dtype, int64_t B, int64_t Hh, int64_t N, int64_t Dh, const void* bias,
    int32_t bias_dtype, const int64_t bias_strides[3], const void* mask, int32_t mask_dtype,
    int64_t mask_batch, const int64_t mask_strides[3], const void* mask_tiles,
    const uint8_t* boundary, float scale, void* stream) {
    if (mask == nullptr || mask_tiles == nullptr)
        return crumpet::fail(CRUMPET_ERR_INVALID_ARGUMENT,
                             "crumpet_fused_swin_attention_tiled: mask and mask_tiles are required");
    return crumpet::run_attention("crumpet_fused_swin_attention_tiled", out, out_strides, q, q_strides,
                                  k, k_strides, v, v_strides, dtype, B, Hh, N, Dh, bias,
                                  bias_dtype, bias_strides, mask, mask_dtype, mask_batch,
                                  mask_strides, mask_tiles, boundary, nullptr, scale, stream);
}

extern "C" int crumpet_fused_swin_attention_shifted(
    void* out, const int64_t out_strides[4], const void* q, const int64_t q_strides[4],
    const void* k, const int64_t k_strides[4], const void* v, const int64_t v_strides[4],
    int32_t dtype, int64_t B, int64_t Hh, int64_t N, int64_t Dh, const void* bias,
    int32_t bias_dtype, const int64_t bias_strides[3], int64_t D, int64_t H, int64_t W,
    int64_t ws_d, int64_t ws_h, int64_t ws_w, int64_t ss_d, int64_t ss_h, int64_t ss_w,
    float scale, void* stream) {
    const crumpet::Region rg = {D, H, W, {ws_d, ws_h, ws_w}, {ss_d, ss_h, ss_w}};
    return crumpet::run_attention("crumpet_fused_swin_attention_shifted", out, out_strides, q,
                                  q_strides, k, k_strides, v, v_strides, dtype, B, Hh, N, Dh, bias,
                                  bias_dtype, bias_strides, nullptr, 0, 1, nullptr, nullptr, nullptr,
                                  &rg, scale, stream);
}
