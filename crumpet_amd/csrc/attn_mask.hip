// Shifted-window additive attention mask for gfx950: a write-bound kernel.
//
// The mask [nW, vol, vol] is written as one flat array of 16-byte vectors
// (8 fp16/bf16 or 4 fp32 elements), so every store is a full, aligned,
// coalesced 16-byte non-temporal store, whatever the odd window volume
// (vol^2 = 117649 at ws=7 leaves the per-window blocks only 2-byte aligned).
//
// Which value an element holds follows from two 3-bit codes:
//   cls[loc]  : for each axis, whether the local coordinate lies at or past
//               ws - ss (the "upper" part of a window that the cyclic shift
//               split).  Depends only on ws and ss; kept in LDS.
//   split(win): for each axis, whether this window is the last one along
//               the axis with a non-zero shift (only those windows straddle
//               two shift regions).
// out[win, i, j] = ((cls[i] ^ cls[j]) & split(win)) ? -100 : 0.
//
// This equals the reference's region-label compare: for a window that is
// not the last along an axis every coordinate lies in region 0; in the last
// window the coordinate x = dim - ws + loc is in region 1 when loc < ws - ss
// and in region 2 otherwise (region(x) definition: cuda/attn_mask_3d.cu:42-50,
// torch-ext/crumpet/reference.py:80-98).  Interior windows (split == 0) take
// a zero-store fast path with no table reads.
#include <hip/hip_runtime.h>

#include "crumpet_common.h"
#include "crumpet_hip.h"

namespace crumpet {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxVolume = 1024;  // same limit as cuda/attn_mask_3d.cu:143
constexpr int kVecPerThread = 4;

struct MaskGeom {
    uint32_t total_elems;  // elements written by this launch (< 2^31)
    uint32_t win0;         // first window of this launch
    uint32_t vol;
    uint32_t ws_d, ws_h, ws_w;
    uint32_t ss_d, ss_h, ss_w;
    uint32_t nWd, nWh, nWw;
    FastDiv f_vol, f_nWw, f_nWh, f_wsw, f_wsh;
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t split_of(uint32_t win, const MaskGeom& g) {
    uint32_t t, ww, wd, wh;
    g.f_nWw.divmod(win, t, ww);
    g.f_nWh.divmod(t, wd, wh);
    return ((wd == g.nWd - 1 && g.ss_d) ? 4u : 0u) | ((wh == g.nWh - 1 && g.ss_h) ? 2u : 0u) |
           ((ww == g.nWw - 1 && g.ss_w) ? 1u : 0u);
}

// kEsize: 2 (fp16/bf16) or 4 (fp32); kNeg: bit pattern of -100 in that type.
template <int kEsize, uint32_t kNeg>
__global__ void __launch_bounds__(kThreads)
attn_mask_kernel(u32x4* __restrict__ out, const MaskGeom g, const uint32_t chunks,
                 const uint32_t launched) {
    constexpr uint32_t kEpv = 16 / kEsize;  // elements per vector
    __shared__ uint8_t cls[kMaxVolume];

    uint32_t chunk;
    const bool active = xcd_chunk(blockIdx.x, launched, chunks, chunk);
    if (!active) return;  // whole workgroup exits together

    for (uint32_t loc = threadIdx.x; loc < g.vol; loc += kThreads) {
        uint32_t lt, lw, ld, lh;
        g.f_wsw.divmod(loc, lt, lw);
        g.f_wsh.divmod(lt, ld, lh);
        cls[loc] = static_cast<uint8_t>(((ld >= g.ws_d - g.ss_d) ? 4 : 0) |
                                        ((lh >= g.ws_h - g.ss_h) ? 2 : 0) |
                                        ((lw >= g.ws_w - g.ss_w) ? 1 : 0));
    }
    __syncthreads();

    const uint32_t nvec = (g.total_elems + kEpv - 1) / kEpv;
    const uint32_t base = chunk * (kThreads * kVecPerThread) + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) {
        const uint32_t vi = base + u * kThreads;
        if (vi >= nvec) break;
        const uint32_t e0 = vi * kEpv;
        uint32_t row, j0, wl, i;
        g.f_vol.divmod(e0, row, j0);
        g.f_vol.divmod(row, wl, i);
        const uint32_t sm = split_of(g.win0 + wl, g);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (j0 + kEpv <= g.vol && e0 + kEpv <= g.total_elems) {
            // the whole vector lies in one mask row
            if (sm != 0) {
                const uint32_t ci = cls[i];
                uint32_t bits[kEpv];
#pragma unroll
                for (uint32_t k = 0; k < kEpv; ++k)
                    bits[k] = ((cls[j0 + k] ^ ci) & sm) ? kNeg : 0u;
#pragma unroll
                for (uint32_t m = 0; m < 4; ++m) {
                    if (kEsize == 2)
                        v[m] = bits[2 * m] | (bits[2 * m + 1] << 16);
                    else
                        v[m] = bits[m];
                }
            }
            __builtin_nontemporal_store(v, out + vi);
        } else {
            // vector crosses a row (or window) boundary, or is the tail
            uint32_t bits[kEpv];
#pragma unroll
            for (uint32_t k = 0; k < kEpv; ++k) {
                const uint32_t e = e0 + k;
                uint32_t r, j, w, ii;
                g.f_vol.divmod(e, r, j);
                g.f_vol.divmod(r, w, ii);
                const uint32_t s = split_of(g.win0 + w, g);
                bits[k] = (e < g.total_elems && ((cls[j] ^ cls[ii]) & s)) ? kNeg : 0u;
            }
            if (e0 + kEpv <= g.total_elems) {
#pragma unroll
                for (uint32_t m = 0; m < 4; ++m) {
                    if (kEsize == 2)
                        v[m] = bits[2 * m] | (bits[2 * m + 1] << 16);
                    else
                        v[m] = bits[m];
                }
                __builtin_nontemporal_store(v, out + vi);
            } else {
                // partial tail vector: scalar stores of the elements in range
                for (uint32_t k = 0; k < kEpv && e0 + k < g.total_elems; ++k) {
                    if (kEsize == 2)
                        reinterpret_cast<uint16_t*>(out)[e0 + k] = static_cast<uint16_t>(bits[k]);
                    else
                        reinterpret_cast<uint32_t*>(out)[e0 + k] = bits[k];
                }
            }
        }
    }
}

}  // namespace
}  // namespace crumpet

extern "C" int crumpet_compute_attn_mask_3d(void* out, int32_t dtype, int64_t D, int64_t H,
                                            int64_t W, int64_t ws_d, int64_t ws_h, int64_t ws_w,
                                            int64_t ss_d, int64_t ss_h, int64_t ss_w,
                                            void* stream) {
    using namespace crumpet;
    const char* what = "crumpet_compute_attn_mask_3d";
    if (D <= 0 || H <= 0 || W <= 0)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: D, H and W must be positive", what);
    if (ws_d <= 0 || ws_h <= 0 || ws_w <= 0)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: window_size values must be positive", what);
    if (D % ws_d || H % ws_h || W % ws_w)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT,
                    "%s: D, H and W must be divisible by window_size", what);
    if (ss_d < 0 || ss_d >= ws_d || ss_h < 0 || ss_h >= ws_h || ss_w < 0 || ss_w >= ws_w)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT,
                    "%s: shift_size must satisfy 0 <= shift < window_size", what);
    int esize;
    uint32_t neg;
    switch (dtype) {
        case CRUMPET_DTYPE_F32: esize = 4; neg = 0xC2C80000u; break;
        case CRUMPET_DTYPE_F16: esize = 2; neg = 0xD640u; break;
        case CRUMPET_DTYPE_BF16: esize = 2; neg = 0xC2C8u; break;
        default: return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: unsupported dtype %d", what, dtype);
    }
    const int64_t vol = ws_d * ws_h * ws_w;
    if (vol > kMaxVolume)
        return fail(CRUMPET_ERR_UNSUPPORTED,
                    "CRUMPET mask kernel supports window volumes up to 1024");
    const int64_t nWd = D / ws_d, nWh = H / ws_h, nWw = W / ws_w;
    const int64_t nW = nWd * nWh * nWw;
    if (out == nullptr) return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: null output", what);
    if (reinterpret_cast<uintptr_t>(out) % 16 != 0)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: output must be 16-byte aligned", what);
    if (nWd > 0x7fffffff || nWh > 0x7fffffff || nWw > 0x7fffffff || nW > 0x7fffffff)
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: too many windows", what);

    MaskGeom g;
    g.vol = vol;
    g.ws_d = ws_d; g.ws_h = ws_h; g.ws_w = ws_w;
    g.ss_d = ss_d; g.ss_h = ss_h; g.ss_w = ss_w;
    g.nWd = nWd; g.nWh = nWh; g.nWw = nWw;
    g.f_vol.init(vol);
    g.f_nWw.init(nWw);
    g.f_nWh.init(nWh);
    g.f_wsw.init(ws_w);
    g.f_wsh.init(ws_h);

    // Launch over groups of windows whose byte size keeps every launch base
    // 16-byte aligned and its element count within 31 bits.
    const int64_t pair = vol * vol;
    const int64_t align_group = (esize == 2) ? 8 : 4;  // windows per 16-byte multiple
    int64_t per_launch = ((int64_t(1) << 31) - 4096) / pair;
    per_launch = per_launch / align_group * align_group;
    if (per_launch <= 0) per_launch = align_group;
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* base = static_cast<char*>(out);
    for (int64_t w0 = 0; w0 < nW; w0 += per_launch) {
        const int64_t nwin = (nW - w0 < per_launch) ? nW - w0 : per_launch;
        g.win0 = static_cast<uint32_t>(w0);
        g.total_elems = static_cast<uint32_t>(nwin * pair);
        const int64_t epv = 16 / esize;
        const int64_t nvec = (nwin * pair + epv - 1) / epv;
        const uint32_t chunks =
            static_cast<uint32_t>((nvec + kThreads * kVecPerThread - 1) / (kThreads * kVecPerThread));
        const uint32_t launched = xcd_launch_count(chunks);
        u32x4* dst = reinterpret_cast<u32x4*>(base + w0 * pair * esize);
        if (esize == 4)
            hipLaunchKernelGGL((attn_mask_kernel<4, 0xC2C80000u>), dim3(launched), dim3(kThreads),
                               0, s, dst, g, chunks, launched);
        else if (neg == 0xD640u)
            hipLaunchKernelGGL((attn_mask_kernel<2, 0xD640u>), dim3(launched), dim3(kThreads), 0,
                               s, dst, g, chunks, launched);
        else
            hipLaunchKernelGGL((attn_mask_kernel<2, 0xC2C8u>), dim3(launched), dim3(kThreads), 0,
                               s, dst, g, chunks, launched);
        const int st = check_launch(what);
        if (st != CRUMPET_OK) return st;
    }
    return CRUMPET_OK;
}
