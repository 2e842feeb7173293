// Fused cyclic shift + 3D window partition, and its inverse, for gfx950.
//
// Both directions are written as one output-ordered gather: every lane owns
// one VB-byte vector of the OUTPUT, decodes where that vector lives in the
// input and copies it.  Writes are therefore perfectly coalesced and
// contiguous; reads are contiguous runs of ws_w tokens (7 * C * elem bytes,
// 672 B at C=48 fp16), split in two only where the cyclic shift wraps.
//
// Index math uses FastDiv (one mulhi + add + shift per division), so the
// VALU cost is ~50 instructions per 16-byte vector, a third of the VALU
// budget at HBM speed.  One vector per thread with non-temporal stores and
// the hardware's own workgroup order measured fastest on MI355X for the
// window-ordered direction (5.8 TB/s for the 98^3 C=48 fp16 partition, 98%
// of a plain streaming copy); more vectors per thread were slower.  The
// volume-ordered direction groups workgroups in runs per XCD (3-4% faster)
// and runs 512-thread workgroups (1-2% faster than 256 there).
//
// Reference semantics: torch-ext/crumpet/reference.py:141-184 (roll then
// view/permute, and the inverse); kernels replaced:
// cuda/shift_partition_3d.cu:60-181 and cuda/unshift_unpartition_3d.cu:34-142.
#include <hip/hip_runtime.h>

#include "crumpet_common.h"
#include "crumpet_hip.h"

namespace crumpet {
namespace {

// Threads per workgroup: 256 for the window-ordered gather, 512 for the
// volume-ordered one (measured fastest for each at config 1).
template <bool kToWindows>
constexpr int threads_for() {
    return kToWindows ? 256 : 512;
}
constexpr uint32_t kXcdRun = 16;  // workgroups per XCD run in the volume-ordered gather

struct GatherGeom {
    uint32_t total;  // output vectors
    uint32_t D, H, W;
    uint32_t ws_d, ws_h, ws_w;
    uint32_t ss_d, ss_h, ss_w;
    uint32_t nWh, nWw, nW, vol;
    uint32_t cvec;  // vectors per token
    FastDiv f_cvec;
    // windows -> (b, win, loc) decode
    FastDiv f_vol, f_nW, f_nWw, f_nWh, f_wsw, f_wsh;
    // volume -> (b, d, h, w) decode
    FastDiv f_W, f_H, f_D, f_wsd;
};

template <int VB>
struct VecOf;
template <>
struct VecOf<16> {
    typedef uint32_t type __attribute__((ext_vector_type(4)));
};
template <>
struct VecOf<8> {
    typedef uint32_t type __attribute__((ext_vector_type(2)));
};
template <>
struct VecOf<4> {
    typedef uint32_t type;
};
template <>
struct VecOf<2> {
    typedef uint16_t type;
};
template <>
struct VecOf<1> {
    typedef uint8_t type;
};

// Output is [B*nW, vol, C]: find the source vector in [B, D, H, W, C].
__device__ __forceinline__ uint32_t src_for_windows(uint32_t o, const GatherGeom& g) {
    uint32_t tok, cv, bw, loc, b, win, t, ww, wd, wh, lt, lw, ld, lh;
    g.f_cvec.divmod(o, tok, cv);
    g.f_vol.divmod(tok, bw, loc);
    g.f_nW.divmod(bw, b, win);
    g.f_nWw.divmod(win, t, ww);
    g.f_nWh.divmod(t, wd, wh);
    g.f_wsw.divmod(loc, lt, lw);
    g.f_wsh.divmod(lt, ld, lh);
    uint32_t d = wd * g.ws_d + ld + g.ss_d;
    uint32_t h = wh * g.ws_h + lh + g.ss_h;
    uint32_t w = ww * g.ws_w + lw + g.ss_w;
    d -= (d >= g.D) ? g.D : 0u;
    h -= (h >= g.H) ? g.H : 0u;
    w -= (w >= g.W) ? g.W : 0u;
    return (((b * g.D + d) * g.H + h) * g.W + w) * g.cvec + cv;
}

// Output is [B, D, H, W, C]: find the source vector in [B*nW, vol, C].
__device__ __forceinline__ uint32_t src_for_volume(uint32_t o, const GatherGeom& g) {
    uint32_t tok, cv, t1, w, t2, h, b, d, wd, ld, wh, lh, ww, lw;
    g.f_cvec.divmod(o, tok, cv);
    g.f_W.divmod(tok, t1, w);
    g.f_H.divmod(t1, t2, h);
    g.f_D.divmod(t2, b, d);
    // position in the rolled frame: (x - ss) mod dim
    d = (d >= g.ss_d) ? d - g.ss_d : d + g.D - g.ss_d;
    h = (h >= g.ss_h) ? h - g.ss_h : h + g.H - g.ss_h;
    w = (w >= g.ss_w) ? w - g.ss_w : w + g.W - g.ss_w;
    g.f_wsd.divmod(d, wd, ld);
    g.f_wsh.divmod(h, wh, lh);
    g.f_wsw.divmod(w, ww, lw);
    const uint32_t win = (wd * g.nWh + wh) * g.nWw + ww;
    const uint32_t loc = (ld * g.ws_h + lh) * g.ws_w + lw;
    return ((b * g.nW + win) * g.vol + loc) * g.cvec + cv;
}

template <int VB, bool kToWindows, int U>
__global__ void __launch_bounds__(threads_for<kToWindows>())
window_gather_kernel(typename VecOf<VB>::type* __restrict__ out,
                     const typename VecOf<VB>::type* __restrict__ in, const GatherGeom g) {
    typedef typename VecOf<VB>::type V;
    constexpr int kThreads = threads_for<kToWindows>();
    uint32_t blk = blockIdx.x;
    if constexpr (!kToWindows) {
        // Volume-ordered output: consecutive rows read the two halves of the
        // partial cache lines at the ends of each window row.  Give each XCD
        // runs of kXcdRun consecutive workgroups (hardware ids go round-robin
        // over the XCDs) so those rows share one L2; the tail keeps the
        // identity mapping.
        constexpr uint32_t kSpan = kNumXcd * kXcdRun;
        const uint32_t sup = blk / kSpan;
        if ((sup + 1) * kSpan <= gridDim.x) {
            const uint32_t within = blk - sup * kSpan;
            blk = sup * kSpan + (within % kNumXcd) * kXcdRun + within / kNumXcd;
        }
    }
    const uint32_t base = blk * (kThreads * U) + threadIdx.x;
    V vals[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t o = base + u * kThreads;
        if (o < g.total) {
            const uint32_t s = kToWindows ? src_for_windows(o, g) : src_for_volume(o, g);
            vals[u] = in[s];
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t o = base + u * kThreads;
        if (o < g.total) __builtin_nontemporal_store(vals[u], out + o);
    }
}

int validate_windows(const char* what, int64_t B, int64_t D, int64_t H, int64_t W, int64_t C,
                     int64_t elem_size, int64_t ws_d, int64_t ws_h, int64_t ws_w,
                     int64_t ss_d, int64_t ss_h, int64_t ss_w) {
    if (B < 0 || D <= 0 || H <= 0 || W <= 0 || C < 0)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT,
                    "%s: B, C must be non-negative and D, H, W positive", what);
    if (ws_d <= 0 || ws_h <= 0 || ws_w <= 0)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: window_size values must be positive", what);
    if (D % ws_d || H % ws_h || W % ws_w)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT,
                    "%s: D, H and W must be divisible by window_size", what);
    if (ss_d < 0 || ss_d >= ws_d || ss_h < 0 || ss_h >= ws_h || ss_w < 0 || ss_w >= ws_w)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT,
                    "%s: shift_size must satisfy 0 <= shift < window_size", what);
    if (elem_size != 1 && elem_size != 2 && elem_size != 4 && elem_size != 8)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: elem_size must be 1, 2, 4 or 8", what);
    return CRUMPET_OK;
}

int launch_gather(bool to_windows, void* out, const void* in, int64_t B, int64_t D, int64_t H,
                  int64_t W, int64_t C, int64_t elem_size, int64_t ws_d, int64_t ws_h,
                  int64_t ws_w, int64_t ss_d, int64_t ss_h, int64_t ss_w, void* stream,
                  const char* what) {
    int st = validate_windows(what, B, D, H, W, C, elem_size, ws_d, ws_h, ws_w, ss_d, ss_h, ss_w);
    if (st != CRUMPET_OK) return st;
    const int64_t tokens = B * D * H * W;
    const int64_t token_bytes = C * elem_size;
    if (tokens == 0 || token_bytes == 0) return CRUMPET_OK;
    if (out == nullptr || in == nullptr)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: null data pointer", what);

    int vb = 16;
    const uintptr_t a = reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(in);
    while (vb > 1 && ((token_bytes % vb) != 0 || (a % vb) != 0)) vb >>= 1;
    const int64_t cvec = token_bytes / vb;
    const int64_t total = tokens * cvec;
    const int64_t kLimit = (int64_t(1) << 31) - (int64_t(1) << 16);
    if (total >= kLimit)
        return fail(CRUMPET_ERR_UNSUPPORTED,
                    "%s: %lld vectors of %d bytes exceed the 31-bit index range", what,
                    (long long)total, vb);

    GatherGeom g;
    g.total = static_cast<uint32_t>(total);
    g.D = D; g.H = H; g.W = W;
    g.ws_d = ws_d; g.ws_h = ws_h; g.ws_w = ws_w;
    g.ss_d = ss_d; g.ss_h = ss_h; g.ss_w = ss_w;
    g.nWh = H / ws_h; g.nWw = W / ws_w;
    g.nW = (D / ws_d) * g.nWh * g.nWw;
    g.vol = ws_d * ws_h * ws_w;
    g.cvec = cvec;
    g.f_cvec.init(cvec);
    g.f_vol.init(g.vol);
    g.f_nW.init(g.nW);
    g.f_nWw.init(g.nWw);
    g.f_nWh.init(g.nWh);
    g.f_wsw.init(ws_w);
    g.f_wsh.init(ws_h);
    g.f_W.init(W);
    g.f_H.init(H);
    g.f_D.init(D);
    g.f_wsd.init(ws_d);

    constexpr int U = 1;
    const int threads = to_windows ? threads_for<true>() : threads_for<false>();
    const uint32_t blocks = static_cast<uint32_t>((total + threads * U - 1) / (threads * U));
    hipStream_t s = static_cast<hipStream_t>(stream);

#define CRUMPET_LAUNCH_GATHER(VBV)                                                           \
    do {                                                                                     \
        typedef typename VecOf<VBV>::type V;                                                 \
        if (to_windows)                                                                      \
            hipLaunchKernelGGL((window_gather_kernel<VBV, true, U>), dim3(blocks),           \
                               dim3(threads), 0, s, static_cast<V*>(out),                   \
                               static_cast<const V*>(in), g);                                \
        else                                                                                 \
            hipLaunchKernelGGL((window_gather_kernel<VBV, false, U>), dim3(blocks),          \
                               dim3(threads), 0, s, static_cast<V*>(out),                   \
                               static_cast<const V*>(in), g);                                \
    } while (0)

    switch (vb) {
        case 16: CRUMPET_LAUNCH_GATHER(16); break;
        case 8: CRUMPET_LAUNCH_GATHER(8); break;
        case 4: CRUMPET_LAUNCH_GATHER(4); break;
        case 2: CRUMPET_LAUNCH_GATHER(2); break;
        default: CRUMPET_LAUNCH_GATHER(1); break;
    }
#undef CRUMPET_LAUNCH_GATHER
    return check_launch(what);
}

}  // namespace
}  // namespace crumpet

extern "C" int crumpet_shift_partition_3d(void* out, const void* x, int64_t B, int64_t D,
                                          int64_t H, int64_t W, int64_t C, int64_t elem_size,
                                          int64_t ws_d, int64_t ws_h, int64_t ws_w,
                                          int64_t ss_d, int64_t ss_h, int64_t ss_w,
                                          void* stream) {
    return crumpet::launch_gather(true, out, x, B, D, H, W, C, elem_size, ws_d, ws_h, ws_w,
                                  ss_d, ss_h, ss_w, stream, "crumpet_shift_partition_3d");
}

extern "C" int crumpet_unshift_unpartition_3d(void* out, const void* windows, int64_t B,
                                              int64_t D, int64_t H, int64_t W, int64_t C,
                                              int64_t elem_size, int64_t ws_d, int64_t ws_h,
                                              int64_t ws_w, int64_t ss_d, int64_t ss_h,
                                              int64_t ss_w, void* stream) {
    return crumpet::launch_gather(false, out, windows, B, D, H, W, C, elem_size, ws_d, ws_h,
                                  ws_w, ss_d, ss_h, ss_w, stream,
                                  "crumpet_unshift_unpartition_3d");
}

extern "C" int crumpet_shift_partition_3d_backward(void* grad_x, const void* grad_windows,
                                                   int64_t B, int64_t D, int64_t H, int64_t W,
                                                   int64_t C, int64_t elem_size, int64_t ws_d,
                                                   int64_t ws_h, int64_t ws_w, int64_t ss_d,
                                                   int64_t ss_h, int64_t ss_w, void* stream) {
    return crumpet::launch_gather(false, grad_x, grad_windows, B, D, H, W, C, elem_size, ws_d,
                                  ws_h, ws_w, ss_d, ss_h, ss_w, stream,
                                  "crumpet_shift_partition_3d_backward");
}

extern "C" int crumpet_unshift_unpartition_3d_backward(void* grad_windows, const void* grad_x,
                                                       int64_t B, int64_t D, int64_t H,
                                                       int64_t W, int64_t C, int64_t elem_size,
                                                       int64_t ws_d, int64_t ws_h, int64_t ws_w,
                                                       int64_t ss_d, int64_t ss_h, int64_t ss_w,
                                                       void* stream) {
    return crumpet::launch_gather(true, grad_windows, grad_x, B, D, H, W, C, elem_size, ws_d,
                                  ws_h, ws_w, ss_d, ss_h, ss_w, stream,
                                  "crumpet_unshift_unpartition_3d_backward");
}
