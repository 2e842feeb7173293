// The two token-wise projections of a Swin window-attention block, with the
// layout changes around them folded into their memory access (gfx950):
//
//   window_qkv   : qkv[t] = LN(xpad[src(t)]) @ Wqkv^T + bqkv
//   window_proj  : y[src(t)] = win[t] @ Wproj^T + bproj   (src(t) inside y)
//
// t runs over window-ordered tokens (b, window, position in window) and
// src(t) is the volume position that the cyclic shift + window partition
// puts at t: d = (wd*ws_d + ld + ss_d) mod D, likewise for h and w, on the
// volume zero-padded to the window grid (D, H, W multiples of ws).  Tokens
// whose src lies in the padding read zeros (the padding is applied after
// the LayerNorm); window_proj produces only the tokens inside the caller's
// volume (the crop).
//
// This is the eager chain of MONAI's SwinTransformerBlock.forward_part1 and
// WindowAttention (norm1, F.pad, torch.roll, window_partition, qkv Linear;
// proj Linear, window_reverse, torch.roll back, crop), as driven by
// torch-ext/crumpet/monai_patch.py:72-114 and :153-198 in the reference.
// Fusing it removes the LayerNorm output, the padded copy, the window
// partition and its inverse as separate HBM round trips: window_qkv reads the
// block input once and writes qkv once; window_proj reads the attention
// output once and writes the block output once.
//
// Both kernels are one GEMM with M = output features, N = tokens, K = C on
// the matrix cores, in output order: a workgroup of 4 waves owns 64
// consecutive output tokens (window-ordered for window_qkv, volume-ordered
// for window_proj, so padding is never loaded or computed there), gathers
// their input rows and stages them in LDS as the B
// operand; each wave walks a quarter of the 16-feature output tiles,
// reading its weight fragments (the A operand) straight from the
// L2-resident weight matrix.  The MFMA result layout gives each lane 4
// consecutive output features of one token; they go to an LDS output chunk
// that the workgroup writes back as consecutive 16-byte vectors.
// With a 2-byte compute type and small C (stage 0), window_proj (C and
// n_out at most 64, or 96 -> 96) and window_qkv (n_out = 3 C, C at most 48)
// take window_proj_stream_kernel / window_qkv_stream_kernel instead:
// independent persistent waves with the weights in registers (stage 0: 74%
// and 77% of HBM against 60% and 69% for the tiled kernels, whose
// workgroups drain the memory queue at every barrier).  window_qkv at C = 96
// and 192 (stages 1 and 2) takes window_qkv_stream_lds_kernel: the same
// persistent waves, with the weights in LDS.
//
// Numerics: LayerNorm in fp32 (two passes: mean, then the mean of squared
// deviations; biased variance, as torch), the normalised value rounded once
// to the compute type (what autocast does at the Linear's input), products
// accumulated in fp32, the bias added in fp32, one rounding at the store.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "crumpet_common.h"
#include "crumpet_hip.h"

namespace crumpet {
namespace {

constexpr int kThreads = 256;
constexpr int kTileTokens = 64;  // tokens per workgroup: 4 MFMA column tiles
constexpr uint32_t kPadRow = 0xffffffffu;
constexpr int64_t kMaxLdsBytes = 64 * 1024;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

// One 16x16x16 multiply-accumulate step D += A B for the compute type.
template <typename T>
struct Mma;

template <>
struct Mma<_Float16> {
    typedef f16x4 x4;
    static __device__ __forceinline__ f32x4 step(x4 a, x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mma<__bf16> {
    typedef bf16x4 x4;
    static __device__ __forceinline__ f32x4 step(x4 a, x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                         __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
    }
};

template <>
struct Mma<float> {
    typedef f32x4 x4;
    // four K=4 steps; lane group g contracts k = 4g + j in step j, for A and
    // B alike, so the 16 products of a row are each taken once
    static __device__ __forceinline__ f32x4 step(x4 a, x4 b, f32x4 c) {
#pragma unroll
        for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], c, 0, 0, 0);
        return c;
    }
};

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
    return static_cast<float>(v);
}

// Element offset of a row padding that keeps 16 consecutive LDS rows on
// distinct banks for the 8/16-byte fragment reads.
template <typename T>
constexpr int row_pad() {
    return 16 / static_cast<int>(sizeof(T));
}

struct WinGeom {
    uint32_t tokens;      // B * nW * vol, window order
    uint32_t D0, H0, W0;  // the caller's volume
    uint32_t D, H, W;     // padded to the window grid
    uint32_t ws_d, ws_h, ws_w;
    uint32_t ss_d, ss_h, ss_w;
    FastDiv f_vol, f_nW, f_nWw, f_nWh, f_wsw, f_wsh;
    // volume order -> window order (window_proj)
    uint32_t vtokens;           // B * D0 * H0 * W0
    uint32_t nWh, nWw, nW, vol;
    FastDiv f_W0, f_H0, f_D0, f_wsd;
};

// Row of window-ordered token t in the caller's [B, D0, H0, W0] volume, or
// kPadRow when the token falls in the padding.
__device__ __forceinline__ uint32_t token_row(uint32_t t, const WinGeom& g) {
    uint32_t bw, loc, b, win, tq, ww, wd, wh, lt, lw, ld, lh;
    g.f_vol.divmod(t, bw, loc);
    g.f_nW.divmod(bw, b, win);
    g.f_nWw.divmod(win, tq, ww);
    g.f_nWh.divmod(tq, wd, wh);
    g.f_wsw.divmod(loc, lt, lw);
    g.f_wsh.divmod(lt, ld, lh);
    uint32_t d = wd * g.ws_d + ld + g.ss_d;
    uint32_t h = wh * g.ws_h + lh + g.ss_h;
    uint32_t w = ww * g.ws_w + lw + g.ss_w;
    d -= (d >= g.D) ? g.D : 0u;
    h -= (h >= g.H) ? g.H : 0u;
    w -= (w >= g.W) ? g.W : 0u;
    if (d >= g.D0 || h >= g.H0 || w >= g.W0) return kPadRow;
    return ((b * g.D0 + d) * g.H0 + h) * g.W0 + w;
}

// Window-ordered token of volume token v (< vtokens): the inverse of
// token_row over the caller's volume.
__device__ __forceinline__ uint32_t window_token(uint32_t v, const WinGeom& g) {
    uint32_t t1, w, t2, h, b, d, wd, ld, wh, lh, ww, lw;
    g.f_W0.divmod(v, t1, w);
    g.f_H0.divmod(t1, t2, h);
    g.f_D0.divmod(t2, b, d);
    // position in the rolled, padded frame: (x - ss) mod padded dim
    d = (d >= g.ss_d) ? d - g.ss_d : d + g.D - g.ss_d;
    h = (h >= g.ss_h) ? h - g.ss_h : h + g.H - g.ss_h;
    w = (w >= g.ss_w) ? w - g.ss_w : w + g.W - g.ss_w;
    g.f_wsd.divmod(d, wd, ld);
    g.f_wsh.divmod(h, wh, lh);
    g.f_wsw.divmod(w, ww, lw);
    const uint32_t win = (wd * g.nWh + wh) * g.nWw + ww;
    const uint32_t loc = (ld * g.ws_h + lh) * g.ws_w + lw;
    return (b * g.nW + win) * g.vol + loc;
}

// Four consecutive elements of type T as floats (8- or 16-byte load).
template <typename T>
__device__ __forceinline__ f32x4 load4(const T* p) {
    f32x4 r;
    if constexpr (sizeof(T) == 4) {
        r = *reinterpret_cast<const f32x4*>(p);
    } else {
        typedef T T4 __attribute__((ext_vector_type(4)));
        const T4 v = *reinterpret_cast<const T4*>(p);
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = to_f32(v[e]);
    }
    return r;
}

template <typename T>
__device__ __forceinline__ void store4(T* p, f32x4 v) {
    typedef T T4 __attribute__((ext_vector_type(4)));
    T4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = static_cast<T>(v[e]);
    *reinterpret_cast<T4*>(p) = o;
}

// Per-channel LayerNorm parameter (fp32 or the input's type), 4 at a time.
__device__ __forceinline__ f32x4 load_param4(const void* p, int32_t dtype, int c, float dflt) {
    if (p == nullptr) return f32x4{dflt, dflt, dflt, dflt};
    if (dtype == CRUMPET_DTYPE_F32) return load4(static_cast<const float*>(p) + c);
    if (dtype == CRUMPET_DTYPE_F16) return load4(static_cast<const _Float16*>(p) + c);
    return load4(static_cast<const __bf16*>(p) + c);
}

// Launch shape shared by both kernels (host-computed).
struct TileShape {
    int32_t C, n_out;
    int32_t fchunk;   // features per LDS output chunk (multiple of 16)
    int32_t fgroup;   // features per workgroup along grid y (multiple of fchunk)
    int32_t astride;  // LDS row stride of the input tile (elements)
    int32_t ostride;  // LDS row stride of the output chunk (elements)
};

// Weight fragments and bias of a wave's first kPre 16-feature tiles,
// requested once the tile's rows are staged, before the barrier that
// publishes them, so that their round trip overlaps the wait at that
// barrier instead of following it.  Wave w's tiles in the first output chunk
// are w, w + 4, ...
template <typename Tc, int kKSteps, int kPre>
struct WeightPrefetch {
    typename Mma<Tc>::x4 wf[kPre > 0 ? kPre : 1][kKSteps];
    f32x4 b4[kPre > 0 ? kPre : 1];

    __device__ __forceinline__ void load(const Tc* __restrict__ w, const Tc* __restrict__ bias,
                                         const TileShape& ts, int f_begin, int f_end) {
        typedef typename Mma<Tc>::x4 X4;
        const int lane = threadIdx.x & 63;
        const int wave = threadIdx.x >> 6;
        const int col = lane & 15;
        const int g = lane >> 4;
        const int ksteps = ts.C >> 4;
        const int ft_end = min(f_end, f_begin + ts.fchunk) >> 4;
#pragma unroll
        for (int i = 0; i < kPre; ++i) {
            const int ft = (f_begin >> 4) + wave + 4 * i;
            if (ft < ft_end) {
                const Tc* wrow = w + int64_t(16 * ft + col) * ts.C + 4 * g;
#pragma unroll
                for (int kk = 0; kk < kKSteps; ++kk)
                    if (kk < ksteps) wf[i][kk] = *reinterpret_cast<const X4*>(wrow + 16 * kk);
                b4[i] = bias ? load4(bias + 16 * ft + 4 * g) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
    }
};

// Tiles per wave whose weights are requested before the barrier: the first
// one from C = 96 up (stages 1-3 of Swin UNETR: 9-17% faster); none at
// C <= 48, where the registers held across the barrier cost more than the
// overlap gains (stage 0: 7% slower).
template <int kKSteps>
constexpr int prefetch_tiles() {
    return kKSteps > 3 ? 1 : 0;
}

// GEMM over the staged tile and a coalesced store of the result:
//   out^T[f][t] = sum_k W[f][k] a[t][k] + bias[f]
// for this workgroup's features [f_begin, f_end), in chunks of fchunk.
// Per chunk, wave w takes the 16-feature tiles w, w+4, ...; the first kPre
// tiles of the first chunk use the fragments in `pre`, later tiles request
// theirs (from L2) right before their MFMAs.  Lane (col, g) ends with
// features 4g..4g+3 of token 16 s + col, which go to the LDS output chunk.
// (Requesting the next tile's fragments during the current one measured
// slower: the extra registers cost occupancy.)  After a barrier the 256
// threads write the chunk as 16-byte vectors, row by row: row r of the tile
// goes to element offset rows_lds[r] * n_out (rows_lds[r] < 0: not stored).
template <typename Tc, int kKSteps, int kPre>
__device__ __forceinline__ void gemm_store(const Tc* __restrict__ a_lds, Tc* __restrict__ o_lds,
                                           const int32_t* __restrict__ rows_lds, const Tc* __restrict__ w,
                                           const Tc* __restrict__ bias, Tc* __restrict__ out,
                                           const TileShape& ts, int f_begin, int f_end,
                                           const WeightPrefetch<Tc, kKSteps, kPre>& pre) {
    typedef typename Mma<Tc>::x4 X4;
    typedef Tc T8 __attribute__((ext_vector_type(16 / sizeof(Tc))));
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int C = ts.C;
    const int ksteps = C >> 4;
    constexpr int kEpv = 16 / sizeof(Tc);  // elements per 16-byte vector

    // one 16-feature tile: MFMAs over the staged rows, result to the LDS chunk
    auto tile = [&](int ft, int c0, const X4 (&wf)[kKSteps], const f32x4& b4) {
        f32x4 acc[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) acc[s] = b4;
#pragma unroll
        for (int kk = 0; kk < kKSteps; ++kk) {
            if (kk < ksteps) {
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const X4 bf = *reinterpret_cast<const X4*>(&a_lds[(16 * s + col) * ts.astride + 16 * kk + 4 * g]);
                    acc[s] = Mma<Tc>::step(wf[kk], bf, acc[s]);
                }
            }
        }
        const int f0 = 16 * ft + 4 * g;
#pragma unroll
        for (int s = 0; s < 4; ++s) store4(&o_lds[(16 * s + col) * ts.ostride + (f0 - c0)], acc[s]);
    };

    for (int c0 = f_begin; c0 < f_end; c0 += ts.fchunk) {
        const int c1 = min(f_end, c0 + ts.fchunk);
        int ft = (c0 >> 4) + wave;
        if (c0 == f_begin) {
#pragma unroll
            for (int i = 0; i < kPre; ++i, ft += 4)
                if (ft < (c1 >> 4)) tile(ft, c0, pre.wf[i], pre.b4[i]);
        }
        for (; ft < (c1 >> 4); ft += 4) {
            const Tc* wrow = w + int64_t(16 * ft + col) * C + 4 * g;
            X4 wf[kKSteps];
#pragma unroll
            for (int kk = 0; kk < kKSteps; ++kk)
                if (kk < ksteps) wf[kk] = *reinterpret_cast<const X4*>(wrow + 16 * kk);
            const f32x4 b4 = bias ? load4(bias + 16 * ft + 4 * g) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            tile(ft, c0, wf, b4);
        }
        __syncthreads();
        const int vpr = (c1 - c0) / kEpv;  // vectors per row of this chunk
        for (int i = threadIdx.x; i < kTileTokens * vpr; i += kThreads) {
            const int r = i / vpr;
            const int j = i - r * vpr;
            const int32_t row = rows_lds[r];
            if (row >= 0)
                __builtin_nontemporal_store(*reinterpret_cast<const T8*>(&o_lds[r * ts.ostride + j * kEpv]),
                                            reinterpret_cast<T8*>(out + int64_t(row) * ts.n_out + c0 + j * kEpv));
        }
        if (c1 < f_end) __syncthreads();  // the next chunk reuses o_lds
    }
}

// Dynamic LDS of a tile: input rows, output chunk, 64 output row indices.
template <typename Tc>
struct TileLds {
    Tc* a;
    Tc* o;
    int32_t* rows;
    __device__ __forceinline__ TileLds(unsigned char* smem, const TileShape& ts) {
        a = reinterpret_cast<Tc*>(smem);
        o = a + kTileTokens * ts.astride;
        rows = reinterpret_cast<int32_t*>(o + kTileTokens * ts.ostride);
    }
};

// LN + pad + shift + partition + qkv projection.  kCpl: 4-element chunks of
// a token row held per lane (4 lanes per token), C <= 16 * kCpl.
template <typename Tx, typename Tc, int kCpl>
__global__ void __launch_bounds__(kThreads)
window_qkv_kernel(Tc* __restrict__ out, const Tx* __restrict__ x, const void* ln_w, const void* ln_b,
                  int32_t ln_dtype, int32_t normalize, float eps, const Tc* __restrict__ w,
                  const Tc* __restrict__ bias, const TileShape ts, const WinGeom g) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const TileLds<Tc> L(smem, ts);
    const int C = ts.C;
    const uint32_t t0 = blockIdx.x * kTileTokens;
    const int f_begin = blockIdx.y * ts.fgroup;
    const int f_end = min(ts.n_out, f_begin + ts.fgroup);
    if (threadIdx.x < kTileTokens) {
        // the tile's qkv rows are consecutive
        const uint32_t t = t0 + threadIdx.x;
        L.rows[threadIdx.x] = t < g.tokens ? static_cast<int32_t>(t) : -1;
    }
    {
        // 16 tokens per wave, 4 lanes per token; lane part p holds the
        // chunks p, p + 4, ... (channels 4c .. 4c + 3 of chunk c)
        const int lane = threadIdx.x & 63;
        const int tl = (threadIdx.x >> 6) * 16 + (lane >> 2);
        const int part = lane & 3;
        const int nch = C >> 2;
        const uint32_t t = t0 + tl;
        const uint32_t row = t < g.tokens ? token_row(t, g) : kPadRow;
        // LayerNorm parameters requested with the rows (C <= 48), so that
        // the normalisation does not wait for a second round trip after
        // them (6% at stage 0; larger C would cost occupancy).
        constexpr bool kPreLn = kCpl <= 3;
        f32x4 gmv[kPreLn ? kCpl : 1], btv[kPreLn ? kCpl : 1];
        if constexpr (kPreLn) {
#pragma unroll
            for (int j = 0; j < kCpl; ++j) {
                const int c = part + 4 * j;
                gmv[j] = load_param4(ln_w, ln_dtype, 4 * (c < nch ? c : 0), 1.0f);
                btv[j] = load_param4(ln_b, ln_dtype, 4 * (c < nch ? c : 0), 0.0f);
            }
        }
        f32x4 v[kCpl];
        const Tx* xr = x + int64_t(row == kPadRow ? 0 : row) * C;
#pragma unroll
        for (int j = 0; j < kCpl; ++j) {
            const int c = part + 4 * j;
            v[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if (c < nch && row != kPadRow) v[j] = load4(xr + 4 * c);
        }
        if (normalize && row != kPadRow) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < kCpl; ++j) s += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
            s += __shfl_xor(s, 1, 4);
            s += __shfl_xor(s, 2, 4);
            const float mean = s / static_cast<float>(C);
            float q = 0.0f;
#pragma unroll
            for (int j = 0; j < kCpl; ++j) {
                if (part + 4 * j < nch) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float dv = v[j][e] - mean;
                        q = __builtin_fmaf(dv, dv, q);
                    }
                }
            }
            q += __shfl_xor(q, 1, 4);
            q += __shfl_xor(q, 2, 4);
            const float rstd = rsqrtf(q / static_cast<float>(C) + eps);
#pragma unroll
            for (int j = 0; j < kCpl; ++j) {
                const int c = part + 4 * j;
                if (c < nch) {
                    f32x4 gm, bt;
                    if constexpr (kPreLn) {
                        gm = gmv[j];
                        bt = btv[j];
                    } else {
                        gm = load_param4(ln_w, ln_dtype, 4 * c, 1.0f);
                        bt = load_param4(ln_b, ln_dtype, 4 * c, 0.0f);
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[j][e] = __builtin_fmaf((v[j][e] - mean) * rstd, gm[e], bt[e]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < kCpl; ++j) {
            const int c = part + 4 * j;
            if (c < nch) store4(&L.a[tl * ts.astride + 4 * c], v[j]);
        }
    }
    WeightPrefetch<Tc, kCpl, prefetch_tiles<kCpl>()> pre;
    pre.load(w, bias, ts, f_begin, f_end);
    __syncthreads();
    gemm_store<Tc, kCpl>(L.a, L.o, L.rows, w, bias, out, ts, f_begin, f_end, pre);
}

// proj projection + inverse partition + reverse shift + crop, in output
// (volume) order: a workgroup owns 64 consecutive tokens of the caller's
// volume, gathers their window rows as 16-byte vectors (adjacent lanes on
// adjacent parts of a row) and writes 64 consecutive output rows.
template <typename Tc, int kKSteps>
__global__ void __launch_bounds__(kThreads)
window_proj_kernel(Tc* __restrict__ y, const Tc* __restrict__ win, const Tc* __restrict__ w,
                   const Tc* __restrict__ bias, const TileShape ts, const WinGeom g) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const TileLds<Tc> L(smem, ts);
    const int C = ts.C;
    const uint32_t t0 = blockIdx.x * kTileTokens;
    const int f_begin = blockIdx.y * ts.fgroup;
    const int f_end = min(ts.n_out, f_begin + ts.fgroup);
    if (threadIdx.x < kTileTokens) {
        const uint32_t v = t0 + threadIdx.x;
        L.rows[threadIdx.x] = v < g.vtokens ? static_cast<int32_t>(v) : -1;
    }
    {
        // Rows are copied as 16-byte vectors, vector i of the tile being
        // (token i / vpt, part i mod vpt): adjacent lanes read adjacent parts
        // of a row, and the rows of tokens adjacent along W within a window
        // are adjacent in the window buffer, so a wave reads whole runs.  All
        // of a lane's loads are issued before its LDS stores.
        typedef uint32_t V16 __attribute__((ext_vector_type(4)));
        constexpr int kEpv16 = 16 / sizeof(Tc);
        constexpr int kIters = (kTileTokens * (16 * kKSteps / kEpv16) + kThreads - 1) / kThreads;
        constexpr int kBatch = kIters < 3 ? kIters : 3;  // loads in flight per lane
        const int vpt = C / kEpv16;
        const int total = kTileTokens * vpt;
        for (int i0 = threadIdx.x; i0 < total; i0 += kBatch * kThreads) {
            V16 xv[kBatch];
            int dst[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int i = i0 + u * kThreads;
                const int tl = i / vpt;
                const int part = i - tl * vpt;
                const uint32_t v = t0 + tl;
                xv[u] = V16{0u, 0u, 0u, 0u};
                dst[u] = i < total ? tl * ts.astride + part * kEpv16 : -1;
                if (i < total && v < g.vtokens)
                    xv[u] = *reinterpret_cast<const V16*>(win + int64_t(window_token(v, g)) * C + part * kEpv16);
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (dst[u] >= 0) *reinterpret_cast<V16*>(&L.a[dst[u]]) = xv[u];
        }
    }
    WeightPrefetch<Tc, kKSteps, prefetch_tiles<kKSteps>()> pre;
    pre.load(w, bias, ts, f_begin, f_end);
    __syncthreads();
    gemm_store<Tc, kKSteps>(L.a, L.o, L.rows, w, bias, y, ts, f_begin, f_end, pre);
}

// Orders a wave's LDS accesses to its own LDS slice across its lanes (the
// streaming kernels below run their waves independently: no workgroup
// barrier).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// window_proj for 2-byte types with C and n_out at most 64 (stage 0 of Swin
// UNETR: 48 and 48): the whole weight matrix fits in a wave's registers,
// so waves run independently, without workgroup barriers.  A wave takes
// 16-token tiles of the output volume, one per step, and requests the next
// kDepth - 1 tiles' rows before computing the current one.
//
// Fragment layout (v_mfma_f32_16x16x16, token = B column = lane & 15, lane
// group q = lane >> 4): the contraction order is free as long as A and B
// agree, so step kk, element j of lane group q contracts channel
// 4*KS*q + 4*kk + j: lane group q loads the contiguous channels
// [4*KS*q, 4*KS*(q+1)) of its token's window row as KS 8-byte pieces.
// Likewise output row 4*q + i of feature tile ft is feature
// 4*FT*q + 4*ft + i, so the lane's FT result quads are the contiguous
// features [4*FT*q, 4*FT*(q+1)) of its token; they go to the wave's LDS
// slice, and the tile's 16 consecutive output rows leave as 16-byte
// non-temporal vectors (per-lane 8-byte non-temporal stores were 2.4x
// slower: partial-line non-temporal writes; staging the input rows through
// LDS as well measured no faster).
//
// Tile assignment: at step s, logical wave L takes tile s * waves + L, with
// L numbered so that the waves of one XCD (workgroups x, x + 8, ... under
// round-robin dispatch) hold a contiguous run of tiles; the window-buffer
// lines that straddle two neighbouring tiles are then fetched into one L2.
// The grid (stream_grid, kStreamWorkgroups) keeps 3 workgroups per CU
// resident, so the kernel asks for 3 waves per SIMD: 96 -> 96 fits that in
// 165 VGPRs, where the compiler's own choice (171 with AGPRs) gave 2.
template <typename Tc, int KS, int FT, int kDepth>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3)))
window_proj_stream_kernel(Tc* __restrict__ y, const Tc* __restrict__ win, const Tc* __restrict__ w,
                          const Tc* __restrict__ bias, const WinGeom g, uint32_t tiles) {
    typedef typename Mma<Tc>::x4 X4;
    typedef Tc T4 __attribute__((ext_vector_type(4)));
    typedef uint32_t V16 __attribute__((ext_vector_type(4)));
    constexpr int C = 16 * KS, NO = 16 * FT;
    constexpr int kWavesPerWg = kThreads / 64;
    constexpr int kPad = 8;  // elements: rows 16 bytes apart in bank order
    constexpr int kOutVecs = 16 * NO / 8;
    __shared__ __attribute__((aligned(16))) Tc out_lds[kWavesPerWg][16 * (NO + kPad)];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15;
    const int q = lane >> 4;
    const uint32_t wgs = gridDim.x;  // a multiple of 8
    const uint32_t wg = (blockIdx.x & 7u) * (wgs >> 3) + (blockIdx.x >> 3);
    const uint32_t waves = wgs * kWavesPerWg;
    const uint32_t L = wg * kWavesPerWg + wave;

    X4 wf[FT][KS];
    f32x4 b4[FT];
#pragma unroll
    for (int ft = 0; ft < FT; ++ft) {
        const Tc* wr = w + (4 * FT * (col >> 2) + 4 * ft + (col & 3)) * C + 4 * KS * q;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) wf[ft][kk] = *reinterpret_cast<const X4*>(wr + 4 * kk);
        b4[ft] = bias ? load4(bias + 4 * FT * q + 4 * ft) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    // the lane's fragments of tile t (tiles clamped to the last, so that the
    // loads are unconditional; tokens past the volume read row 0 and are not
    // stored)
    auto load_tile = [&](uint32_t t, X4(&xf)[KS]) {
        const uint32_t v = min(t, tiles - 1) * 16 + col;
        const uint32_t row = v < g.vtokens ? window_token(v, g) : 0u;
        const Tc* src = win + int64_t(row) * C + 4 * KS * q;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) xf[kk] = *reinterpret_cast<const X4*>(src + 4 * kk);
    };
    auto run_tile = [&](uint32_t t, const X4(&xf)[KS]) {
        const uint32_t t16 = t * 16;
        Tc* ol = out_lds[wave];
        wave_lds_sync();  // the previous tile's vectors have been read
#pragma unroll
        for (int ft = 0; ft < FT; ++ft) {
            f32x4 acc = b4[ft];
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) acc = Mma<Tc>::step(wf[ft][kk], xf[kk], acc);
            T4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = static_cast<Tc>(acc[e]);
            *reinterpret_cast<T4*>(&ol[col * (NO + kPad) + 4 * FT * q + 4 * ft]) = o;
        }
        wave_lds_sync();
#pragma unroll
        for (int it = 0; it < (kOutVecs + 63) / 64; ++it) {
            const int i = lane + 64 * it;
            const int tok = i / (NO / 8);
            const int part = i - tok * (NO / 8);
            if (i < kOutVecs && t16 + tok < g.vtokens)
                __builtin_nontemporal_store(*reinterpret_cast<const V16*>(&ol[tok * (NO + kPad) + 8 * part]),
                                            reinterpret_cast<V16*>(y + int64_t(t16 + tok) * NO + 8 * part));
        }
    };

    X4 xb[kDepth][KS];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) load_tile(L + d * waves, xb[d]);
    for (uint32_t t0 = L; t0 < tiles; t0 += kDepth * waves) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            const uint32_t t = t0 + d * waves;
            if (t < tiles) {  // wave-uniform
                run_tile(t, xb[d]);
                load_tile(t + kDepth * waves, xb[d]);
            }
        }
    }
}

// window_qkv for 2-byte compute types with n_out = 3 C and C at most 48
// (stage 0 of Swin UNETR: 48 -> 144): the weight matrix, its bias and the
// LayerNorm parameters stay in registers; waves run independently over
// 16-token tiles of the window-ordered output, as in
// window_proj_stream_kernel and with its fragment layout: lane group q holds
// channels [4*KS*q, 4*KS*(q+1)) of its token, so the LayerNorm statistics
// are sums over the token's 4 lanes (lanes col + 16 q), and features
// [4*FT*q, 4*FT*(q+1)) of the result.  The tile's 16 output rows are
// consecutive; they leave through the wave's LDS slice as 16-byte vectors.
template <typename Tx, typename Tc, int KS, int kDepth>
__global__ void __launch_bounds__(kThreads)
window_qkv_stream_kernel(Tc* __restrict__ out, const Tx* __restrict__ x, const void* ln_w, const void* ln_b,
                         int32_t ln_dtype, int32_t normalize, float eps, const Tc* __restrict__ w,
                         const Tc* __restrict__ bias, const WinGeom g, uint32_t tiles) {
    typedef typename Mma<Tc>::x4 X4;
    typedef Tc T4 __attribute__((ext_vector_type(4)));
    typedef Tx Tx4 __attribute__((ext_vector_type(4)));
    typedef uint32_t V16 __attribute__((ext_vector_type(4)));
    constexpr int C = 16 * KS, FT = 3 * KS, NO = 16 * FT;
    constexpr int kWavesPerWg = kThreads / 64;
    constexpr int kPad = 8;
    constexpr int kOutVecs = 16 * NO / 8;
    __shared__ __attribute__((aligned(16))) Tc out_lds[kWavesPerWg][16 * (NO + kPad)];
    // fp32 bias and LayerNorm parameters, shared by the workgroup's waves
    // (read per tile: in registers they would cost a wave per SIMD)
    __shared__ __attribute__((aligned(16))) float par_lds[NO + 2 * C];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15;
    const int q = lane >> 4;
    const uint32_t wgs = gridDim.x;  // a multiple of 8
    const uint32_t wg = (blockIdx.x & 7u) * (wgs >> 3) + (blockIdx.x >> 3);
    const uint32_t waves = wgs * kWavesPerWg;
    const uint32_t L = wg * kWavesPerWg + wave;

    for (int i = threadIdx.x; i < (NO + 2 * C) / 4; i += kThreads) {
        f32x4 v;
        if (4 * i < NO)
            v = bias ? load4(bias + 4 * i) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        else if (4 * i < NO + C)
            v = load_param4(ln_w, ln_dtype, 4 * i - NO, 1.0f);
        else
            v = load_param4(ln_b, ln_dtype, 4 * i - NO - C, 0.0f);
        *reinterpret_cast<f32x4*>(&par_lds[4 * i]) = v;
    }
    X4 wf[FT][KS];
#pragma unroll
    for (int ft = 0; ft < FT; ++ft) {
        const Tc* wr = w + (4 * FT * (col >> 2) + 4 * ft + (col & 3)) * C + 4 * KS * q;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) wf[ft][kk] = *reinterpret_cast<const X4*>(wr + 4 * kk);
    }
    __syncthreads();  // par_lds is written (every wave passes here once)
    const float* b_lds = par_lds + 4 * FT * q;
    const float* gm_lds = par_lds + NO + 4 * KS * q;
    const float* bt_lds = par_lds + NO + C + 4 * KS * q;

    struct Raw {
        Tx4 v[KS];
        bool pad;
    };
    // the lane's channels of window-ordered token t (tiles clamped to the
    // last, so that the loads are unconditional; padding reads row 0)
    auto load_tile = [&](uint32_t t, Raw& r) {
        const uint32_t tok = min(t, tiles - 1) * 16 + col;
        const uint32_t row = tok < g.tokens ? token_row(tok, g) : kPadRow;
        r.pad = row == kPadRow;
        const Tx* src = x + int64_t(r.pad ? 0u : row) * C + 4 * KS * q;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) r.v[kk] = *reinterpret_cast<const Tx4*>(src + 4 * kk);
    };
    auto run_tile = [&](uint32_t t, const Raw& r) {
        f32x4 v[KS];
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[kk][e] = r.pad ? 0.0f : to_f32(r.v[kk][e]);
        if (normalize) {
            float sm = 0.0f;
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) sm += (v[kk][0] + v[kk][1]) + (v[kk][2] + v[kk][3]);
            sm += __shfl_xor(sm, 16);
            sm += __shfl_xor(sm, 32);
            const float mean = sm / static_cast<float>(C);
            float qs = 0.0f;
#pragma unroll
            for (int kk = 0; kk < KS; ++kk)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float dv = v[kk][e] - mean;
                    qs = __builtin_fmaf(dv, dv, qs);
                }
            qs += __shfl_xor(qs, 16);
            qs += __shfl_xor(qs, 32);
            const float rstd = rsqrtf(qs / static_cast<float>(C) + eps);
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) {
                const f32x4 gm = *reinterpret_cast<const f32x4*>(gm_lds + 4 * kk);
                const f32x4 bt = *reinterpret_cast<const f32x4*>(bt_lds + 4 * kk);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v[kk][e] = r.pad ? 0.0f : __builtin_fmaf((v[kk][e] - mean) * rstd, gm[e], bt[e]);
            }
        }
        X4 xf[KS];
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
#pragma unroll
            for (int e = 0; e < 4; ++e) xf[kk][e] = static_cast<Tc>(v[kk][e]);
        Tc* ol = out_lds[wave];
        wave_lds_sync();  // the previous tile's vectors have been read
#pragma unroll
        for (int ft = 0; ft < FT; ++ft) {
            f32x4 acc = *reinterpret_cast<const f32x4*>(b_lds + 4 * ft);
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) acc = Mma<Tc>::step(wf[ft][kk], xf[kk], acc);
            T4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = static_cast<Tc>(acc[e]);
            *reinterpret_cast<T4*>(&ol[col * (NO + kPad) + 4 * FT * q + 4 * ft]) = o;
        }
        wave_lds_sync();
        const uint32_t t16 = t * 16;
#pragma unroll
        for (int it = 0; it < (kOutVecs + 63) / 64; ++it) {
            const int i = lane + 64 * it;
            const int tok = i / (NO / 8);
            const int part = i - tok * (NO / 8);
            if (i < kOutVecs && t16 + tok < g.tokens)
                __builtin_nontemporal_store(*reinterpret_cast<const V16*>(&ol[tok * (NO + kPad) + 8 * part]),
                                            reinterpret_cast<V16*>(out + int64_t(t16 + tok) * NO + 8 * part));
        }
    };

    Raw raw[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) load_tile(L + d * waves, raw[d]);
    for (uint32_t t0 = L; t0 < tiles; t0 += kDepth * waves) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            const uint32_t t = t0 + d * waves;
            if (t < tiles) {  // wave-uniform
                run_tile(t, raw[d]);
                load_tile(t + kDepth * waves, raw[d]);
            }
        }
    }
}

// window_qkv for 2-byte compute types at C = 96 and 192 (stages 1 and 2 of
// Swin UNETR at feature size 48: 96 -> 288, 192 -> 576), whose weights do
// not fit a wave's registers.  A workgroup holds NCH chunks of 96 output
// features in LDS for the whole launch (stage 1 all three, 55 KB; stage 2
// one of six, 37 KB), in fragment order: fragment (c, ft, kk) is 64 lanes x
// 4 elements, contiguous, so each A-operand read is one conflict-free
// 8-byte LDS load per lane.  Twelve persistent waves per workgroup (one
// workgroup per CU, 3 waves per SIMD) stream 16-token tiles as in
// window_qkv_stream_kernel: lane group q holds channels [4 KS q, 4 KS (q +
// 1)) of its token (LayerNorm sums over the token's 4 lanes).  Chunk groups
// alternate between neighbouring workgroups, which share an XCD and so read
// the same tiles through one L2.  Within chunk c, lane group q computes
// features c * 96 + 24 q + [4 ft, 4 ft + 4), staged through the wave's LDS
// slice and stored as 16-byte vectors.
constexpr int kLdsQkvWaves = 12;
constexpr int kLdsQkvDepth = 2;  // tiles in flight per wave (C = 96; 1 at C = 192)
constexpr int kLdsQkvChunk = 96;  // output features per chunk

template <typename Tx, typename Tc, int KS, int NCH, int kDepth>
__global__ void __launch_bounds__(64 * kLdsQkvWaves)
window_qkv_stream_lds_kernel(Tc* __restrict__ out, const Tx* __restrict__ x, const void* ln_w, const void* ln_b,
                             int32_t ln_dtype, int32_t normalize, float eps, const Tc* __restrict__ w,
                             const Tc* __restrict__ bias, const WinGeom g, uint32_t tiles) {
    typedef typename Mma<Tc>::x4 X4;
    typedef Tc T4 __attribute__((ext_vector_type(4)));
    typedef Tx Tx4 __attribute__((ext_vector_type(4)));
    typedef uint32_t V16 __attribute__((ext_vector_type(4)));
    constexpr int C = 16 * KS, NOC = kLdsQkvChunk, NOW = NCH * NOC, NO = 3 * C;
    constexpr int CG = NO / NOW;             // chunk groups
    constexpr int kFtc = NOC / 16;           // feature tiles per chunk (6)
    constexpr int kFrags = NCH * kFtc * KS;  // A-operand fragments held
    constexpr int kThreadsL = 64 * kLdsQkvWaves;
    constexpr int kPad = 8;
    constexpr int kOutVecs = 16 * NOC / 8;  // 16-byte vectors per chunk of a tile
    static_assert(NO % NOW == 0 && NOC == 4 * 24, "chunk geometry");
    __shared__ __attribute__((aligned(16))) Tc w_lds[kFrags * 64 * 4];
    __shared__ __attribute__((aligned(16))) Tc out_lds[kLdsQkvWaves][16 * (NOC + kPad)];
    __shared__ __attribute__((aligned(16))) float par_lds[NOW + 2 * C];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15;
    const int q = lane >> 4;
    const uint32_t wgs = gridDim.x;  // a multiple of 8 and of CG
    const uint32_t wg = (blockIdx.x & 7u) * (wgs >> 3) + (blockIdx.x >> 3);
    const int cg = static_cast<int>(wg % CG);
    const uint32_t waves = wgs / CG * kLdsQkvWaves;  // per chunk group
    const uint32_t L = wg / CG * kLdsQkvWaves + wave;
    const int f0 = cg * NOW;  // the workgroup's first output feature

    // fragment j = (c * kFtc + ft) * KS + kk, lane (lc, lq): weight row
    // f0 + c * 96 + 24 (lc >> 2) + 4 ft + (lc & 3), channels 4 KS lq + 4 kk .. + 3
    // (every load of the fill is issued before the first store waits)
    constexpr int kFill = (kFrags * 64 + kThreadsL - 1) / kThreadsL;
    X4 wtmp[kFill];
#pragma unroll
    for (int it = 0; it < kFill; ++it) {
        const int i = static_cast<int>(threadIdx.x) + it * kThreadsL;
        if (i < kFrags * 64) {
            const int j = i >> 6, l = i & 63;
            const int kk = j % KS, cf = j / KS;
            const int c = cf / kFtc, ft = cf - c * kFtc;
            const int lc = l & 15, lq = l >> 4;
            const int row = f0 + c * NOC + 24 * (lc >> 2) + 4 * ft + (lc & 3);
            wtmp[it] = *reinterpret_cast<const X4*>(w + row * C + 4 * KS * lq + 4 * kk);
        }
    }
#pragma unroll
    for (int it = 0; it < kFill; ++it) {
        const int i = static_cast<int>(threadIdx.x) + it * kThreadsL;
        if (i < kFrags * 64) *reinterpret_cast<X4*>(&w_lds[4 * i]) = wtmp[it];
    }
    for (int i = threadIdx.x; i < (NOW + 2 * C) / 4; i += kThreadsL) {
        f32x4 v;
        if (4 * i < NOW)
            v = bias ? load4(bias + f0 + 4 * i) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        else if (4 * i < NOW + C)
            v = load_param4(ln_w, ln_dtype, 4 * i - NOW, 1.0f);
        else
            v = load_param4(ln_b, ln_dtype, 4 * i - NOW - C, 0.0f);
        *reinterpret_cast<f32x4*>(&par_lds[4 * i]) = v;
    }
    __syncthreads();  // weights and parameters are in LDS (every wave passes here once)
    const float* gm_lds = par_lds + NOW + 4 * KS * q;
    const float* bt_lds = par_lds + NOW + C + 4 * KS * q;

    struct Raw {
        Tx4 v[KS];
        bool pad;
    };
    // the lane's channels of window-ordered token t (tiles clamped to the
    // last, so that the loads are unconditional; padding reads row 0)
    auto load_tile = [&](uint32_t t, Raw& r) {
        const uint32_t tok = min(t, tiles - 1) * 16 + col;
        const uint32_t row = tok < g.tokens ? token_row(tok, g) : kPadRow;
        r.pad = row == kPadRow;
        const Tx* src = x + int64_t(r.pad ? 0u : row) * C + 4 * KS * q;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) r.v[kk] = *reinterpret_cast<const Tx4*>(src + 4 * kk);
    };
    auto run_tile = [&](uint32_t t, const Raw& r) {
        f32x4 v[KS];
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[kk][e] = r.pad ? 0.0f : to_f32(r.v[kk][e]);
        if (normalize) {
            float sm = 0.0f;
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) sm += (v[kk][0] + v[kk][1]) + (v[kk][2] + v[kk][3]);
            sm += __shfl_xor(sm, 16);
            sm += __shfl_xor(sm, 32);
            const float mean = sm / static_cast<float>(C);
            float qs = 0.0f;
#pragma unroll
            for (int kk = 0; kk < KS; ++kk)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float dv = v[kk][e] - mean;
                    qs = __builtin_fmaf(dv, dv, qs);
                }
            qs += __shfl_xor(qs, 16);
            qs += __shfl_xor(qs, 32);
            const float rstd = rsqrtf(qs / static_cast<float>(C) + eps);
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) {
                const f32x4 gm = *reinterpret_cast<const f32x4*>(gm_lds + 4 * kk);
                const f32x4 bt = *reinterpret_cast<const f32x4*>(bt_lds + 4 * kk);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v[kk][e] = r.pad ? 0.0f : __builtin_fmaf((v[kk][e] - mean) * rstd, gm[e], bt[e]);
            }
        }
        X4 xf[KS];
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
#pragma unroll
            for (int e = 0; e < 4; ++e) xf[kk][e] = static_cast<Tc>(v[kk][e]);
        Tc* ol = out_lds[wave];
        const uint32_t t16 = t * 16;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            wave_lds_sync();  // the previous chunk's vectors have been read
#pragma unroll
            for (int ft = 0; ft < kFtc; ++ft) {
                f32x4 acc = *reinterpret_cast<const f32x4*>(par_lds + c * NOC + 24 * q + 4 * ft);
#pragma unroll
                for (int kk = 0; kk < KS; ++kk) {
                    const X4 wf = *reinterpret_cast<const X4*>(&w_lds[(((c * kFtc + ft) * KS + kk) * 64 + lane) * 4]);
                    acc = Mma<Tc>::step(wf, xf[kk], acc);
                }
                T4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = static_cast<Tc>(acc[e]);
                *reinterpret_cast<T4*>(&ol[col * (NOC + kPad) + 24 * q + 4 * ft]) = o;
            }
            wave_lds_sync();
#pragma unroll
            for (int it = 0; it < (kOutVecs + 63) / 64; ++it) {
                const int i = lane + 64 * it;
                const int tok = i / (NOC / 8);
                const int part = i - tok * (NOC / 8);
                if (i < kOutVecs && t16 + tok < g.tokens)
                    __builtin_nontemporal_store(
                        *reinterpret_cast<const V16*>(&ol[tok * (NOC + kPad) + 8 * part]),
                        reinterpret_cast<V16*>(out + int64_t(t16 + tok) * NO + f0 + c * NOC + 8 * part));
            }
        }
    };

    Raw raw[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) load_tile(L + d * waves, raw[d]);
    for (uint32_t t0 = L; t0 < tiles; t0 += kDepth * waves) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            const uint32_t t = t0 + d * waves;
            if (t < tiles) {  // wave-uniform
                run_tile(t, raw[d]);
                load_tile(t + kDepth * waves, raw[d]);
            }
        }
    }
}

int elem_size(int32_t dtype) {
    switch (dtype) {
        case CRUMPET_DTYPE_F32: return 4;
        case CRUMPET_DTYPE_F16: return 2;
        case CRUMPET_DTYPE_BF16: return 2;
        default: return 0;
    }
}

// Shared validation; fills g.  The caller's volume is [B, D, H, W] with
// channels C_in; tokens run over the volume padded to the window grid.
int make_geometry(const char* what, int64_t B, int64_t D, int64_t H, int64_t W, int64_t ws_d,
                  int64_t ws_h, int64_t ws_w, int64_t ss_d, int64_t ss_h, int64_t ss_w, WinGeom& g) {
    if (B < 0 || D <= 0 || H <= 0 || W <= 0)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: B must be non-negative and D, H, W positive", what);
    if (ws_d <= 0 || ws_h <= 0 || ws_w <= 0)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: window_size values must be positive", what);
    if (ss_d < 0 || ss_d >= ws_d || ss_h < 0 || ss_h >= ws_h || ss_w < 0 || ss_w >= ws_w)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT,
                    "%s: shift_size must satisfy 0 <= shift < window_size", what);
    const int64_t Dp = (D + ws_d - 1) / ws_d * ws_d;
    const int64_t Hp = (H + ws_h - 1) / ws_h * ws_h;
    const int64_t Wp = (W + ws_w - 1) / ws_w * ws_w;
    const int64_t tokens = B * Dp * Hp * Wp;
    if (tokens >= (int64_t(1) << 31) - kTileTokens || B * D * H * W >= (int64_t(1) << 31))
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: more than 2^31 tokens", what);
    g.tokens = static_cast<uint32_t>(tokens);
    g.D0 = D; g.H0 = H; g.W0 = W;
    g.D = Dp; g.H = Hp; g.W = Wp;
    g.ws_d = ws_d; g.ws_h = ws_h; g.ws_w = ws_w;
    g.ss_d = ss_d; g.ss_h = ss_h; g.ss_w = ss_w;
    const uint32_t nWh = Hp / ws_h, nWw = Wp / ws_w;
    g.f_vol.init(ws_d * ws_h * ws_w);
    g.f_nW.init((Dp / ws_d) * nWh * nWw);
    g.f_nWw.init(nWw);
    g.f_nWh.init(nWh);
    g.f_wsw.init(ws_w);
    g.f_wsh.init(ws_h);
    g.vtokens = static_cast<uint32_t>(B * D * H * W);
    g.nWh = nWh;
    g.nWw = nWw;
    g.nW = (Dp / ws_d) * nWh * nWw;
    g.vol = ws_d * ws_h * ws_w;
    g.f_W0.init(W);
    g.f_H0.init(H);
    g.f_D0.init(D);
    g.f_wsd.init(ws_d);
    return CRUMPET_OK;
}

// Validates the projection and plans its tile: the LDS output chunk is as
// wide as fits next to the staged input rows (at most 192 16-bit or 96 fp32
// features), and small token counts split the features over grid y so that
// the launch still covers the chip.
int plan_tile(const char* what, int64_t C, int64_t n_out, int32_t dtype, const void* weight, uint32_t tokens,
              TileShape& ts, size_t& lds, dim3& grid) {
    if (C <= 0 || C % 16 != 0)
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: channels (%lld) must be a positive multiple of 16",
                    what, (long long)C);
    if (C > 16 * 24) return fail(CRUMPET_ERR_UNSUPPORTED, "%s: at most 384 channels", what);
    if (n_out <= 0 || n_out % 16 != 0 || n_out > (int64_t(1) << 20))
        return fail(CRUMPET_ERR_UNSUPPORTED,
                    "%s: output features (%lld) must be a positive multiple of 16 (at most 2^20)", what,
                    (long long)n_out);
    const int es = elem_size(dtype);
    if (es == 0) return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: unsupported compute dtype %d", what, dtype);
    if (weight == nullptr) return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: null weight", what);
    const int pad = 16 / es;
    const int64_t a_bytes = int64_t(kTileTokens) * (C + pad) * es;
    const int64_t rows_bytes = int64_t(kTileTokens) * 4;
    int fchunk = static_cast<int>(std::min<int64_t>(n_out, es == 2 ? 192 : 96));
    while (fchunk >= 16 && a_bytes + int64_t(kTileTokens) * (fchunk + pad) * es + rows_bytes > kMaxLdsBytes)
        fchunk -= 16;
    if (fchunk < 16)
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: %lld channels of %d bytes exceed the staging tile",
                    what, (long long)C, es);
    const uint32_t tiles = (tokens + kTileTokens - 1) / kTileTokens;
    const int nft = static_cast<int>(n_out / 16);
    int groups = static_cast<int>(std::min<int64_t>(std::max<int64_t>(1, (1024 + tiles - 1) / std::max(tiles, 1u)),
                                                    std::max(1, nft / 4)));
    const int fgroup = (nft + groups - 1) / groups * 16;
    groups = static_cast<int>((n_out + fgroup - 1) / fgroup);
    ts.C = static_cast<int32_t>(C);
    ts.n_out = static_cast<int32_t>(n_out);
    ts.fgroup = fgroup;
    ts.fchunk = std::min(fchunk, fgroup);
    ts.astride = static_cast<int32_t>(C) + pad;
    ts.ostride = ts.fchunk + pad;
    lds = static_cast<size_t>(a_bytes + int64_t(kTileTokens) * ts.ostride * es + rows_bytes);
    grid = dim3(tiles, groups);
    return CRUMPET_OK;
}

template <typename Tx, typename Tc>
void launch_qkv(dim3 grid, size_t lds, hipStream_t s, void* out, const void* x, const void* ln_w,
                const void* ln_b, int32_t ln_dtype, int32_t normalize, float eps, const void* w,
                const void* bias, const TileShape& ts, const WinGeom& g) {
#define CRUMPET_QKV(K)                                                                            \
    hipLaunchKernelGGL((window_qkv_kernel<Tx, Tc, K>), grid, dim3(kThreads), lds, s,             \
                       static_cast<Tc*>(out), static_cast<const Tx*>(x), ln_w, ln_b, ln_dtype,  \
                       normalize, eps, static_cast<const Tc*>(w), static_cast<const Tc*>(bias), \
                       ts, g)
    const int cpl = ts.C / 16;
    if (cpl <= 3)
        CRUMPET_QKV(3);
    else if (cpl <= 6)
        CRUMPET_QKV(6);
    else if (cpl <= 12)
        CRUMPET_QKV(12);
    else
        CRUMPET_QKV(24);
#undef CRUMPET_QKV
}

template <typename Tx>
void launch_qkv_x(int32_t dtype, dim3 grid, size_t lds, hipStream_t s, void* out, const void* x,
                  const void* ln_w, const void* ln_b, int32_t ln_dtype, int32_t normalize, float eps,
                  const void* w, const void* bias, const TileShape& ts, const WinGeom& g) {
    if (dtype == CRUMPET_DTYPE_F16)
        launch_qkv<Tx, _Float16>(grid, lds, s, out, x, ln_w, ln_b, ln_dtype, normalize, eps, w, bias, ts, g);
    else if (dtype == CRUMPET_DTYPE_BF16)
        launch_qkv<Tx, __bf16>(grid, lds, s, out, x, ln_w, ln_b, ln_dtype, normalize, eps, w, bias, ts, g);
    else
        launch_qkv<Tx, float>(grid, lds, s, out, x, ln_w, ln_b, ln_dtype, normalize, eps, w, bias, ts, g);
}

template <typename Tc>
void launch_proj(dim3 grid, size_t lds, hipStream_t s, void* y, const void* win, const void* w,
                 const void* bias, const TileShape& ts, const WinGeom& g) {
#define CRUMPET_PROJ(K)                                                                           \
    hipLaunchKernelGGL((window_proj_kernel<Tc, K>), grid, dim3(kThreads), lds, s, static_cast<Tc*>(y), \
                       static_cast<const Tc*>(win), static_cast<const Tc*>(w),                   \
                       static_cast<const Tc*>(bias), ts, g)
    const int ks = ts.C / 16;
    if (ks <= 3)
        CRUMPET_PROJ(3);
    else if (ks <= 6)
        CRUMPET_PROJ(6);
    else if (ks <= 12)
        CRUMPET_PROJ(12);
    else
        CRUMPET_PROJ(24);
#undef CRUMPET_PROJ
}

// The register-resident projection: 2-byte types, C and n_out at most 64.
constexpr int kStreamDepth = 2;               // tiles in flight per wave
constexpr uint32_t kStreamWorkgroups = 768;  // 3 per CU, 12 waves per CU

// C and n_out up to 64, and 96 -> 96 (stage 1 of Swin UNETR at feature size
// 48: 72 weight VGPRs per lane, still 3 waves per SIMD)
bool proj_streams(int32_t dtype, int64_t C, int64_t n_out) {
    return elem_size(dtype) == 2 && ((C <= 64 && n_out <= 64) || (C == 96 && n_out == 96));
}

constexpr int kQkvStreamDepth = 1;
constexpr uint32_t kQkvStreamWorkgroups = 512;

bool qkv_streams(int32_t dtype, int64_t C, int64_t n_out) {
    return elem_size(dtype) == 2 && C <= 48 && n_out == 3 * C;
}

// 96 -> 288 and 192 -> 576 (stages 1 and 2): the weights in LDS, one
// 12-wave workgroup per CU
constexpr uint32_t kLdsQkvWorkgroups = 256;

bool qkv_streams_lds(int32_t dtype, int64_t C, int64_t n_out) {
    return elem_size(dtype) == 2 && (C == 96 || C == 192) && n_out == 3 * C;
}

// Grid of a streaming kernel: the fewest steps that `cap` workgroups allow,
// then the fewest workgroups (a multiple of 8, one per XCD) that take every
// tile in that many steps, so that the last step is nearly full for every
// wave.
dim3 stream_grid(uint32_t tiles, uint32_t cap) {
    constexpr uint32_t kWaves = kThreads / 64;
    const uint32_t steps = std::max(1u, (tiles + cap * kWaves - 1) / (cap * kWaves));
    const uint32_t wgs = (tiles + steps * kWaves - 1) / (steps * kWaves);
    return dim3(std::max(8u, (wgs + 7) / 8 * 8));
}

template <typename Tx, typename Tc>
void launch_qkv_stream(int KS, hipStream_t s, void* out, const void* x, const void* ln_w, const void* ln_b,
                       int32_t ln_dtype, int32_t normalize, float eps, const void* w, const void* bias,
                       const WinGeom& g) {
    const uint32_t tiles = (g.tokens + 15) / 16;
    const dim3 grid = stream_grid(tiles, kQkvStreamWorkgroups);
#define CRUMPET_QKV_STREAM(K)                                                                          \
    hipLaunchKernelGGL((window_qkv_stream_kernel<Tx, Tc, K, kQkvStreamDepth>), grid, dim3(kThreads), 0, s, \
                       static_cast<Tc*>(out), static_cast<const Tx*>(x), ln_w, ln_b, ln_dtype, normalize, eps,  \
                       static_cast<const Tc*>(w), static_cast<const Tc*>(bias), g, tiles)
    switch (KS) {
        case 1: CRUMPET_QKV_STREAM(1); break;
        case 2: CRUMPET_QKV_STREAM(2); break;
        default: CRUMPET_QKV_STREAM(3); break;
    }
#undef CRUMPET_QKV_STREAM
}

template <typename Tx>
void launch_qkv_stream_x(int32_t dtype, int KS, hipStream_t s, void* out, const void* x, const void* ln_w,
                         const void* ln_b, int32_t ln_dtype, int32_t normalize, float eps, const void* w,
                         const void* bias, const WinGeom& g) {
    if (dtype == CRUMPET_DTYPE_F16)
        launch_qkv_stream<Tx, _Float16>(KS, s, out, x, ln_w, ln_b, ln_dtype, normalize, eps, w, bias, g);
    else
        launch_qkv_stream<Tx, __bf16>(KS, s, out, x, ln_w, ln_b, ln_dtype, normalize, eps, w, bias, g);
}

// Per chunk group the fewest steps that its share of kLdsQkvWorkgroups
// allows, then the fewest workgroups that take every tile in that many
// steps; the total is a multiple of 8 (one per XCD) and of the chunk groups.
template <typename Tx, typename Tc, int KS, int NCH, int kDepth>
void launch_qkv_stream_lds_k(hipStream_t s, void* out, const void* x, const void* ln_w, const void* ln_b,
                             int32_t ln_dtype, int32_t normalize, float eps, const void* w, const void* bias,
                             const WinGeom& g) {
    constexpr uint32_t CG = 3 * 16 * KS / (NCH * kLdsQkvChunk);
    constexpr uint32_t kStep = CG % 8 == 0 ? 1 : (CG % 4 == 0 ? 2 : (CG % 2 == 0 ? 4 : 8));
    const uint32_t tiles = (g.tokens + 15) / 16;
    const uint32_t cap = std::max(1u, kLdsQkvWorkgroups / CG) * kLdsQkvWaves;  // waves per chunk group
    const uint32_t steps = std::max(1u, (tiles + cap - 1) / cap);
    uint32_t wpc = (tiles + steps * kLdsQkvWaves - 1) / (steps * kLdsQkvWaves);
    wpc = (wpc + kStep - 1) / kStep * kStep;
    hipLaunchKernelGGL((window_qkv_stream_lds_kernel<Tx, Tc, KS, NCH, kDepth>), dim3(CG * wpc),
                       dim3(64 * kLdsQkvWaves), 0, s, static_cast<Tc*>(out), static_cast<const Tx*>(x), ln_w, ln_b,
                       ln_dtype, normalize, eps, static_cast<const Tc*>(w), static_cast<const Tc*>(bias), g, tiles);
}

template <typename Tx, typename Tc>
void launch_qkv_stream_lds(int64_t C, hipStream_t s, void* out, const void* x, const void* ln_w, const void* ln_b,
                           int32_t ln_dtype, int32_t normalize, float eps, const void* w, const void* bias,
                           const WinGeom& g) {
    if (C == 96)  // all three chunks per workgroup (55 KB)
        launch_qkv_stream_lds_k<Tx, Tc, 6, 3, kLdsQkvDepth>(s, out, x, ln_w, ln_b, ln_dtype, normalize, eps, w,
                                                           bias, g);
    else  // C = 192: one chunk of six per workgroup (37 KB)
        launch_qkv_stream_lds_k<Tx, Tc, 12, 1, 1>(s, out, x, ln_w, ln_b, ln_dtype, normalize, eps, w, bias, g);
}

template <typename Tx>
void launch_qkv_stream_lds_x(int32_t dtype, int64_t C, hipStream_t s, void* out, const void* x, const void* ln_w,
                             const void* ln_b, int32_t ln_dtype, int32_t normalize, float eps, const void* w,
                             const void* bias, const WinGeom& g) {
    if (dtype == CRUMPET_DTYPE_F16)
        launch_qkv_stream_lds<Tx, _Float16>(C, s, out, x, ln_w, ln_b, ln_dtype, normalize, eps, w, bias, g);
    else
        launch_qkv_stream_lds<Tx, __bf16>(C, s, out, x, ln_w, ln_b, ln_dtype, normalize, eps, w, bias, g);
}

template <typename Tc, int KS>
void launch_proj_stream_ks(int FT, dim3 grid, hipStream_t s, void* y, const void* win, const void* w,
                           const void* bias, const WinGeom& g, uint32_t tiles) {
#define CRUMPET_PROJ_STREAM(F)                                                                        \
    hipLaunchKernelGGL((window_proj_stream_kernel<Tc, KS, F, kStreamDepth>), grid, dim3(kThreads), 0, s, \
                       static_cast<Tc*>(y), static_cast<const Tc*>(win), static_cast<const Tc*>(w),   \
                       static_cast<const Tc*>(bias), g, tiles)
    if constexpr (KS == 6) {
        (void)FT;  // 96 -> 96 only (proj_streams)
        CRUMPET_PROJ_STREAM(6);
    } else {
        switch (FT) {
            case 1: CRUMPET_PROJ_STREAM(1); break;
            case 2: CRUMPET_PROJ_STREAM(2); break;
            case 3: CRUMPET_PROJ_STREAM(3); break;
            default: CRUMPET_PROJ_STREAM(4); break;
        }
    }
#undef CRUMPET_PROJ_STREAM
}

template <typename Tc>
void launch_proj_stream(int KS, int FT, hipStream_t s, void* y, const void* win, const void* w,
                        const void* bias, const WinGeom& g) {
    const uint32_t tiles = (g.vtokens + 15) / 16;
    const dim3 grid = stream_grid(tiles, kStreamWorkgroups);
    switch (KS) {
        case 1: launch_proj_stream_ks<Tc, 1>(FT, grid, s, y, win, w, bias, g, tiles); break;
        case 2: launch_proj_stream_ks<Tc, 2>(FT, grid, s, y, win, w, bias, g, tiles); break;
        case 3: launch_proj_stream_ks<Tc, 3>(FT, grid, s, y, win, w, bias, g, tiles); break;
        case 4: launch_proj_stream_ks<Tc, 4>(FT, grid, s, y, win, w, bias, g, tiles); break;
        default: launch_proj_stream_ks<Tc, 6>(FT, grid, s, y, win, w, bias, g, tiles); break;
    }
}

}  // namespace
}  // namespace crumpet

using namespace crumpet;

extern "C" int crumpet_window_qkv_3d(void* out, int32_t dtype, const void* x, int32_t x_dtype,
                                     int64_t B, int64_t D, int64_t H, int64_t W, int64_t C,
                                     int32_t normalize, const void* ln_weight, const void* ln_bias,
                                     int32_t ln_dtype, float eps, const void* weight, const void* bias,
                                     int64_t n_out, int64_t ws_d, int64_t ws_h, int64_t ws_w,
                                     int64_t ss_d, int64_t ss_h, int64_t ss_w, void* stream) {
    const char* what = "crumpet_window_qkv_3d";
    WinGeom g;
    int st = make_geometry(what, B, D, H, W, ws_d, ws_h, ws_w, ss_d, ss_h, ss_w, g);
    if (st != CRUMPET_OK) return st;
    TileShape ts;
    size_t lds;
    dim3 grid;
    st = plan_tile(what, C, n_out, dtype, weight, g.tokens, ts, lds, grid);
    if (st != CRUMPET_OK) return st;
    if (elem_size(x_dtype) == 0)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: unsupported input dtype %d", what, x_dtype);
    if (normalize && (ln_weight || ln_bias) && ln_dtype != CRUMPET_DTYPE_F32 && ln_dtype != x_dtype)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT,
                    "%s: LayerNorm parameters must be float32 or the input dtype", what);
    if (!(eps >= 0.0f))
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: eps must be non-negative", what);
    if (g.tokens == 0) return CRUMPET_OK;
    if (out == nullptr || x == nullptr)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: null data pointer", what);
    if ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(x) |
         reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(bias) |
         reinterpret_cast<uintptr_t>(ln_weight) | reinterpret_cast<uintptr_t>(ln_bias)) % 16 != 0)
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: pointers must be 16-byte aligned", what);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (qkv_streams(dtype, C, n_out)) {
        const int KS = static_cast<int>(C / 16);
        if (x_dtype == CRUMPET_DTYPE_F32)
            launch_qkv_stream_x<float>(dtype, KS, s, out, x, ln_weight, ln_bias, ln_dtype, normalize, eps, weight,
                                       bias, g);
        else if (x_dtype == CRUMPET_DTYPE_F16)
            launch_qkv_stream_x<_Float16>(dtype, KS, s, out, x, ln_weight, ln_bias, ln_dtype, normalize, eps,
                                          weight, bias, g);
        else
            launch_qkv_stream_x<__bf16>(dtype, KS, s, out, x, ln_weight, ln_bias, ln_dtype, normalize, eps,
                                        weight, bias, g);
        return check_launch(what);
    }
    if (qkv_streams_lds(dtype, C, n_out)) {
        if (x_dtype == CRUMPET_DTYPE_F32)
            launch_qkv_stream_lds_x<float>(dtype, C, s, out, x, ln_weight, ln_bias, ln_dtype, normalize, eps,
                                           weight, bias, g);
        else if (x_dtype == CRUMPET_DTYPE_F16)
            launch_qkv_stream_lds_x<_Float16>(dtype, C, s, out, x, ln_weight, ln_bias, ln_dtype, normalize, eps,
                                              weight, bias, g);
        else
            launch_qkv_stream_lds_x<__bf16>(dtype, C, s, out, x, ln_weight, ln_bias, ln_dtype, normalize, eps,
                                            weight, bias, g);
        return check_launch(what);
    }
    if (x_dtype == CRUMPET_DTYPE_F32)
        launch_qkv_x<float>(dtype, grid, lds, s, out, x, ln_weight, ln_bias, ln_dtype, normalize, eps, weight,
                            bias, ts, g);
    else if (x_dtype == CRUMPET_DTYPE_F16)
        launch_qkv_x<_Float16>(dtype, grid, lds, s, out, x, ln_weight, ln_bias, ln_dtype, normalize, eps,
                               weight, bias, ts, g);
    else
        launch_qkv_x<__bf16>(dtype, grid, lds, s, out, x, ln_weight, ln_bias, ln_dtype, normalize, eps, weight,
                             bias, ts, g);
    return check_launch(what);
}

extern "C" int crumpet_window_proj_3d(void* y, const void* windows, int32_t dtype, int64_t B, int64_t D,
                                      int64_t H, int64_t W, int64_t C, const void* weight,
                                      const void* bias, int64_t n_out, int64_t ws_d, int64_t ws_h,
                                      int64_t ws_w, int64_t ss_d, int64_t ss_h, int64_t ss_w,
                                      void* stream) {
    const char* what = "crumpet_window_proj_3d";
    WinGeom g;
    int st = make_geometry(what, B, D, H, W, ws_d, ws_h, ws_w, ss_d, ss_h, ss_w, g);
    if (st != CRUMPET_OK) return st;
    TileShape ts;
    size_t lds;
    dim3 grid;
    st = plan_tile(what, C, n_out, dtype, weight, g.vtokens, ts, lds, grid);
    if (st != CRUMPET_OK) return st;
    if (g.vtokens == 0) return CRUMPET_OK;
    if (y == nullptr || windows == nullptr)
        return fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: null data pointer", what);
    if ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(windows) |
         reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(bias)) % 16 != 0)
        return fail(CRUMPET_ERR_UNSUPPORTED, "%s: pointers must be 16-byte aligned", what);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (proj_streams(dtype, C, n_out)) {
        const int KS = static_cast<int>(C / 16), FT = static_cast<int>(n_out / 16);
        if (dtype == CRUMPET_DTYPE_F16)
            launch_proj_stream<_Float16>(KS, FT, s, y, windows, weight, bias, g);
        else
            launch_proj_stream<__bf16>(KS, FT, s, y, windows, weight, bias, g);
        return check_launch(what);
    }
    if (dtype == CRUMPET_DTYPE_F16)
        launch_proj<_Float16>(grid, lds, s, y, windows, weight, bias, ts, g);
    else if (dtype == CRUMPET_DTYPE_BF16)
        launch_proj<__bf16>(grid, lds, s, y, windows, weight, bias, ts, g);
    else
        launch_proj<float>(grid, lds, s, y, windows, weight, bias, ts, g);
    return check_launch(what);
}
