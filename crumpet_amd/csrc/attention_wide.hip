// General fused window attention for the shapes the head-dim-16 kernel does
// not cover: head dims 32, 64, 128 and 256, and windows of more than 512
// tokens (any head dim of 16..256 that is a power of two, any N).  At head
// dim 256 a wave holds about 330 registers (one wave per SIMD).  Same contract
// and the same three mask modes as swin_attention_tuned_kernel
// (attention_kernel.h); the numerics are the reference's:
//
//   S = (q * scale) k^T + bias[h] + mask,  out = softmax_rows(S) v
//
// with q scaled in fp32 and rounded back to the input type, S and the
// softmax in fp32, P rounded to the input type for the P v product, the row
// sums accumulated from the unrounded fp32 P, and one division at the end:
// the steps of torch-ext/crumpet/fused_attention.py:82-146 in the reference.
//
// Decomposition: a workgroup of 4 waves owns one (window, head) and 64
// queries (a 16-query strip per wave); it walks the keys in chunks of 64
// (32 from head dim 32 up: the smaller register prefetch raises occupancy,
// 12% faster than 64-key chunks at head dim 32),
// with K (row-major) and V^T double-buffered in LDS, and keeps the strip's Q
// fragments, the online-softmax state and the O^T accumulators in
// registers.  The next chunk's K/V rows and bias (+ mask) values are
// requested into registers before the current chunk is computed, so their
// latency overlaps the compute; one barrier per chunk.  Per 16-key tile:
// S^T = K Q^T on the matrix cores over D/16 16-dim steps, starting from the
// bias (+ mask) tile; per chunk one online-softmax update; then
// O^T += V^T P^T with P straight from the score registers (the score tile's
// layout is the B-operand layout).  Bias and mask are read as floats of
// their own dtype with their own strides.  Nothing is allocated.
#include <hip/hip_runtime.h>

#include <math.h>

#include "attention_kernel.h"
#include "crumpet_common.h"
#include "crumpet_hip.h"

namespace crumpet {
namespace attn {
namespace {

constexpr int kWideThreads = 256;
constexpr int kWideWaves = 4;
constexpr float kWideLog2e = 1.4426950408889634f;

typedef float f32x4w __attribute__((ext_vector_type(4)));
typedef short i16x4w __attribute__((ext_vector_type(4)));

// One 16x16x16 step D += A B; fp32 contracts k = 4g + j in step j for A and
// B alike, so each product is taken once.
template <typename T>
struct WideMma;

template <>
struct WideMma<_Float16> {
    typedef _Float16 x4 __attribute__((ext_vector_type(4)));
    static __device__ __forceinline__ f32x4w step(x4 a, x4 b, f32x4w c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
    }
};

template <>
struct WideMma<__bf16> {
    typedef __bf16 x4 __attribute__((ext_vector_type(4)));
    static __device__ __forceinline__ f32x4w step(x4 a, x4 b, f32x4w c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4w, a),
                                                         __builtin_bit_cast(i16x4w, b), c, 0, 0, 0);
    }
};

template <>
struct WideMma<float> {
    typedef f32x4w x4;
    static __device__ __forceinline__ f32x4w step(x4 a, x4 b, f32x4w c) {
#pragma unroll
        for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], c, 0, 0, 0);
        return c;
    }
};

// Element i of a float tensor of dtype dt (uniform branch).
__device__ __forceinline__ float load_as_float(const void* base, int64_t i, int32_t dt) {
    if (dt == CRUMPET_DTYPE_F32) return static_cast<const float*>(base)[i];
    if (dt == CRUMPET_DTYPE_F16) return static_cast<float>(static_cast<const _Float16*>(base)[i]);
    return static_cast<float>(static_cast<const __bf16*>(base)[i]);
}

// Elements d0..d0+3 of a row with element stride sd: one vector access
// when the row has unit stride and 4-element alignment (vec), else four.
template <typename T>
__device__ __forceinline__ auto load4v(const T* row, int d0, int64_t sd, bool vec) {
    typedef T V4 __attribute__((ext_vector_type(4)));
    if (vec) return *reinterpret_cast<const V4*>(row + d0);
    V4 v;
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = row[int64_t(d0 + r) * sd];
    return v;
}

template <typename T, typename V4>
__device__ __forceinline__ void store4v(T* row, int d0, int64_t sd, bool vec, V4 v) {
    if (vec) {
        *reinterpret_cast<V4*>(row + d0) = v;
        return;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) row[int64_t(d0 + r) * sd] = v[r];
}

// One element of type T at byte offset off of a buffer resource, as a
// float (offsets past the resource's extent read 0).
template <typename T>
__device__ __forceinline__ float buffer_elem(__amdgpu_buffer_rsrc_t rs, int off) {
    if constexpr (sizeof(T) == 4) {
        return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
    } else {
        const uint16_t h = __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
        return static_cast<float>(__builtin_bit_cast(T, h));
    }
}

// The lane's bias (+ mask) values of keys kc0 + 16 t + 4 g + r of a chunk
// (t < kKC / 16, r < 4) as floats, through buffer resources spanning the
// head's bias and the window's mask; boff / moff are the lane's row
// offsets in bytes.  Keys past N become -inf (their loads read the next row
// or 0).  TB / TM are the bias / mask element types; the key offsets are
// instruction immediates.
template <typename TB, typename TM, int kKC>
__device__ __forceinline__ void fetch_bias_rows(float (&bq)[kKC / 4], __amdgpu_buffer_rsrc_t brs, int boff,
                                                __amdgpu_buffer_rsrc_t mrs, int moff, bool use_mask, int kc0,
                                                int g, int N) {
    const int k4 = kc0 + 4 * g;
#pragma unroll
    for (int t = 0; t < kKC / 16; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int k0 = k4 + 16 * t + r;
            float bv = buffer_elem<TB>(brs, boff + k4 * int(sizeof(TB)) + (16 * t + r) * int(sizeof(TB)));
            if (use_mask) bv += buffer_elem<TM>(mrs, moff + k4 * int(sizeof(TM)) + (16 * t + r) * int(sizeof(TM)));
            bq[4 * t + r] = k0 < N ? bv : -INFINITY;
        }
}

template <typename TB, int kKC>
__device__ __forceinline__ void fetch_bias_m(float (&bq)[kKC / 4], __amdgpu_buffer_rsrc_t brs, int boff,
                                             __amdgpu_buffer_rsrc_t mrs, int moff, bool use_mask, int32_t mdt,
                                             int kc0, int g, int N) {
    if (!use_mask || mdt == CRUMPET_DTYPE_F32)
        fetch_bias_rows<TB, float, kKC>(bq, brs, boff, mrs, moff, use_mask, kc0, g, N);
    else if (mdt == CRUMPET_DTYPE_F16)
        fetch_bias_rows<TB, _Float16, kKC>(bq, brs, boff, mrs, moff, use_mask, kc0, g, N);
    else
        fetch_bias_rows<TB, __bf16, kKC>(bq, brs, boff, mrs, moff, use_mask, kc0, g, N);
}

// Dispatch on the (uniform) bias dtype.
template <int kKC>
__device__ __forceinline__ void fetch_bias_any(float (&bq)[kKC / 4], __amdgpu_buffer_rsrc_t brs, int32_t bdt,
                                               int boff, __amdgpu_buffer_rsrc_t mrs, int moff, bool use_mask,
                                               int32_t mdt, int kc0, int g, int N) {
    if (bdt == CRUMPET_DTYPE_F32)
        fetch_bias_m<float, kKC>(bq, brs, boff, mrs, moff, use_mask, mdt, kc0, g, N);
    else if (bdt == CRUMPET_DTYPE_F16)
        fetch_bias_m<_Float16, kKC>(bq, brs, boff, mrs, moff, use_mask, mdt, kc0, g, N);
    else
        fetch_bias_m<__bf16, kKC>(bq, brs, boff, mrs, moff, use_mask, mdt, kc0, g, N);
}

// kMode: 0 no mask, 1 mask tensor (mask[b mod mask_batch], skipped where a
// boundary flag is 0), 2 shifted-window regions of the [D, H, W] volume.
template <typename T, int D, int kMode>
__global__ void __launch_bounds__(kWideThreads)
swin_attention_wide_kernel(const Params p, int32_t mask_dtype, uint32_t qblocks, uint32_t chunks,
                           uint32_t launched) {
    typedef WideMma<T> M;
    typedef typename M::x4 X4;
    constexpr int kDC = D / 16;                                 // 16-dim steps
    constexpr int kKC = D <= 16 ? 64 : 32;                      // keys per chunk (registers of the prefetch)
    constexpr int kPad = 16 / static_cast<int>(sizeof(T));      // 16 bytes per LDS row
    constexpr int kKStride = D + kPad;                          // K row stride (elements)
    constexpr int kVStride = kKC + kPad;                  // V^T row stride (elements)
    constexpr int kUnits = kKC * (D / 4) / kWideThreads;  // 4-element K/V units per thread and chunk
    static_assert(kUnits >= 1 && kKC * (D / 4) % kWideThreads == 0, "chunk units per thread");
    typedef T V4 __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(16))) T k_lds[2][kKC * kKStride];
    __shared__ __attribute__((aligned(16))) T vt_lds[2][D * kVStride];
    __shared__ uint8_t cls_lds[kMode == 2 ? kWideMaxRegionN : 4];
    // (fp32 at head dim 128 takes about 70 KB: more than the 64 KB of earlier CDNA parts)
    static_assert(sizeof(k_lds) + sizeof(vt_lds) + sizeof(cls_lds) <= 160 * 1024,
                  "LDS footprint exceeds the 160 KB of a gfx950 CU");

    uint32_t chunk;
    if (!xcd_chunk(blockIdx.x, launched, chunks, chunk)) return;
    // chunk = (b * H + h) * qblocks + qb: the query blocks of one
    // (window, head) are consecutive, hence on one XCD, and share its L2.
    const int qb = static_cast<int>(chunk % qblocks);
    const uint32_t bh = chunk / qblocks;
    const int h = static_cast<int>(bh % static_cast<uint32_t>(p.H));
    const int b = static_cast<int>(bh / static_cast<uint32_t>(p.H));
    const int N = p.N;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int qi = qb * kWideQueries + wave * 16 + col;
    const int qr = qi < N ? qi : N - 1;  // padded query rows are computed, never stored

    // region mode: shift-region class of every token (one bit per axis, set
    // at or past ws - ss) and the split bits of this window (axes along which
    // it is the last window of a shifted axis); tokens of different regions
    // along a split axis see -100
    int split = 0;
    if constexpr (kMode == 2) {
        for (int j = threadIdx.x; j < N; j += kWideThreads) {
            const int lw = j % p.ws[2];
            const int t = j / p.ws[2];
            const int lh = t % p.ws[1];
            const int ld = t / p.ws[1];
            cls_lds[j] = static_cast<uint8_t>(((ld >= p.ws[0] - p.ss[0]) ? 4 : 0) |
                                              ((lh >= p.ws[1] - p.ss[1]) ? 2 : 0) |
                                              ((lw >= p.ws[2] - p.ss[2]) ? 1 : 0));
        }
        const int wi = b % p.nW;
        const int ww = wi % p.nWw;
        const int wt = wi / p.nWw;
        const int wh = wt % p.nWh;
        const int wd = wt / p.nWh;
        split = ((wd == p.nWd - 1 && p.ss[0] > 0) ? 4 : 0) | ((wh == p.nWh - 1 && p.ss[1] > 0) ? 2 : 0) |
                ((ww == p.nWw - 1 && p.ss[2] > 0) ? 1 : 0);
    }
    // bias and mask rows through buffer resources: the head's bias [N, N]
    // and the window's mask [N, N] extents (the host checked that they fit
    // 31 bits); the lane's row offset is a per-lane byte offset
    const int bsz = p.bias_dtype == CRUMPET_DTYPE_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(static_cast<const char*>(p.bias) + int64_t(h) * p.bsd[0] * bsz), 0,
        __builtin_amdgcn_readfirstlane(static_cast<int>((int64_t(N - 1) * p.bsd[1] + N) * bsz)), 0x00020000);
    const int boff = static_cast<int>(int64_t(qr) * p.bsd[1] * bsz);
    bool use_mask = false;
    __amdgpu_buffer_rsrc_t mrs = brs;
    int moff = 0;
    if constexpr (kMode == 1) {
        use_mask = p.boundary == nullptr || p.boundary[b] != 0;
        const int msz = mask_dtype == CRUMPET_DTYPE_F32 ? 4 : 2;
        mrs = __builtin_amdgcn_make_buffer_rsrc(
            uniform_ptr(static_cast<const char*>(p.mask) + int64_t(b % p.mask_batch) * p.ms[0] * msz), 0,
            __builtin_amdgcn_readfirstlane(static_cast<int>((int64_t(N - 1) * p.ms[1] + N) * msz)), 0x00020000);
        moff = static_cast<int>(int64_t(qr) * p.ms[1] * msz);
    }

    // B operand of S^T = K Q^T: Q[qr][16 dc + 4 g + r], scaled in fp32 and
    // rounded back to T
    const bool vec = p.vec_io != 0;  // unit d stride, 4-element aligned rows and bases
    const T* qrow = static_cast<const T*>(p.q) + int64_t(b) * p.qs[0] + int64_t(h) * p.qs[1] +
                    int64_t(qr) * p.qs[2];
    X4 qf[kDC];
#pragma unroll
    for (int dc = 0; dc < kDC; ++dc) {
        const V4 qv = load4v(qrow, 16 * dc + 4 * g, p.qs[3], vec);
#pragma unroll
        for (int r = 0; r < 4; ++r) qf[dc][r] = static_cast<T>(static_cast<float>(qv[r]) * p.scale);
    }

    const T* kbase = static_cast<const T*>(p.k) + int64_t(b) * p.ks[0] + int64_t(h) * p.ks[1];
    const T* vbase = static_cast<const T*>(p.v) + int64_t(b) * p.vs[0] + int64_t(h) * p.vs[1];

    // K and V rows of the next key chunk travel through registers: they are
    // requested before the current chunk is computed and written to the
    // other LDS buffer after it, so the loads overlap the compute.  Thread
    // unit e covers key e / (D / 4), dims 4 (e mod (D / 4)) .. + 3.
    V4 kr[kUnits], vr[kUnits];
    // Keys past N re-read row N - 1: their scores are -inf (bias) and their
    // P is 0, so any finite K/V row serves, and no branch is needed.
    auto fetch_kv = [&](int kc0) {
#pragma unroll
        for (int u = 0; u < kUnits; ++u) {
            const int e = threadIdx.x + u * kWideThreads;
            const int kk = min(kc0 + e / (D / 4), N - 1);
            const int d0 = (e % (D / 4)) * 4;
            kr[u] = load4v(kbase + int64_t(kk) * p.ks[2], d0, p.ks[3], vec);
            vr[u] = load4v(vbase + int64_t(kk) * p.vs[2], d0, p.vs[3], vec);
        }
    };
    auto stash_kv = [&](int buf) {
#pragma unroll
        for (int u = 0; u < kUnits; ++u) {
            const int e = threadIdx.x + u * kWideThreads;
            const int key = e / (D / 4);
            const int d0 = (e % (D / 4)) * 4;
            *reinterpret_cast<V4*>(&k_lds[buf][key * kKStride + d0]) = kr[u];
#pragma unroll
            for (int r = 0; r < 4; ++r) vt_lds[buf][(d0 + r) * kVStride + key] = vr[u][r];
        }
    };
    // bias (+ mask tensor) of the lane's scores of a chunk, also one chunk
    // ahead (the dtype choice is uniform and outside the loops)
    float bq[kKC / 4];
    auto fetch_bias = [&](int kc0) __attribute__((always_inline)) {
        fetch_bias_any<kKC>(bq, brs, p.bias_dtype, boff, mrs, moff, use_mask, mask_dtype, kc0, g, N);
    };

    f32x4w o[kDC];  // O^T: o[dd][r] = O[query col][16 dd + 4 g + r]
#pragma unroll
    for (int dd = 0; dd < kDC; ++dd) o[dd] = f32x4w{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY;
    float l_part = 0.0f;  // this lane's share of the row sum (its keys 4g..4g+3 of each tile)

    fetch_kv(0);
    fetch_bias(0);
    stash_kv(0);
    __syncthreads();  // chunk 0 and (region mode) the class table are in LDS
    int my_cls = 0;   // region class of this lane's query
    if constexpr (kMode == 2) my_cls = cls_lds[qr];

    const int nchunks = (N + kKC - 1) / kKC;
    for (int c = 0; c < nchunks; ++c) {
        const int kc0 = c * kKC;
        const int buf = c & 1;
        const bool more = c + 1 < nchunks;
        float bc[kKC / 4];
#pragma unroll
        for (int i = 0; i < kKC / 4; ++i) bc[i] = bq[i];
        if (more) {
            fetch_kv(kc0 + kKC);
            fetch_bias(kc0 + kKC);
        }

        // scores of the chunk's 4 key tiles: lane (col, g) holds
        // S[query col][key kc0 + 16 t + 4 g + r]
        f32x4w S[kKC / 16];
#pragma unroll
        for (int t = 0; t < kKC / 16; ++t) {
            f32x4w acc;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                acc[r] = bc[4 * t + r];
            }
            if constexpr (kMode == 2) {
                if (split != 0) {  // windows not last along a shifted axis see no mask
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int kk = min(kc0 + 16 * t + 4 * g + r, N - 1);
                        acc[r] += ((my_cls ^ cls_lds[kk]) & split) ? -100.0f : 0.0f;
                    }
                }
            }
#pragma unroll
            for (int dc = 0; dc < kDC; ++dc) {
                const X4 kf = *reinterpret_cast<const X4*>(&k_lds[buf][(16 * t + col) * kKStride + 16 * dc + 4 * g]);
                acc = M::step(kf, qf[dc], acc);
            }
            S[t] = acc;
        }

        // online softmax over the chunk: row max across the 4 lane groups
        float cm = -INFINITY;
#pragma unroll
        for (int t = 0; t < kKC / 16; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) cm = fmaxf(cm, S[t][r]);
        cm = fmaxf(cm, __shfl_xor(cm, 16));
        cm = fmaxf(cm, __shfl_xor(cm, 32));
        const float m_new = fmaxf(m_run, cm);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;  // rows with no finite score yet
        const float alpha = __builtin_amdgcn_exp2f((m_run - m_use) * kWideLog2e);
        l_part *= alpha;
#pragma unroll
        for (int dd = 0; dd < kDC; ++dd) o[dd] *= alpha;
        m_run = m_new;
        const float mb = m_use * kWideLog2e;

#pragma unroll
        for (int t = 0; t < kKC / 16; ++t) {
            X4 pb;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(S[t][r], kWideLog2e, -mb));
                l_part += pv;
                pb[r] = static_cast<T>(pv);
            }
            // O^T += V^T P^T: A = V^T[16 dd + col][keys 16 t + 4 g ..], B = P^T
#pragma unroll
            for (int dd = 0; dd < kDC; ++dd) {
                const X4 vf =
                    *reinterpret_cast<const X4*>(&vt_lds[buf][(16 * dd + col) * kVStride + 16 * t + 4 * g]);
                o[dd] = M::step(vf, pb, o[dd]);
            }
        }
        // the other buffer was last read before the previous barrier
        if (more) stash_kv(buf ^ 1);
        __syncthreads();
    }

    float l = l_part;
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (qi < N) {
        T* orow = static_cast<T*>(p.out) + int64_t(b) * p.os[0] + int64_t(h) * p.os[1] + int64_t(qi) * p.os[2];
#pragma unroll
        for (int dd = 0; dd < kDC; ++dd) {
            V4 ov;
#pragma unroll
            for (int r = 0; r < 4; ++r) ov[r] = static_cast<T>(o[dd][r] / l);
            store4v(orow, 16 * dd + 4 * g, p.os[3], vec, ov);
        }
    }
}

template <typename T, int D>
void launch_d(const Params& p, int mode, int32_t mask_dtype, uint32_t qblocks, uint32_t chunks,
              uint32_t launched, hipStream_t s) {
    const dim3 grid(launched), block(kWideThreads);
    if (mode == 0)
        hipLaunchKernelGGL((swin_attention_wide_kernel<T, D, 0>), grid, block, 0, s, p, mask_dtype, qblocks,
                           chunks, launched);
    else if (mode == 1)
        hipLaunchKernelGGL((swin_attention_wide_kernel<T, D, 1>), grid, block, 0, s, p, mask_dtype, qblocks,
                           chunks, launched);
    else
        hipLaunchKernelGGL((swin_attention_wide_kernel<T, D, 2>), grid, block, 0, s, p, mask_dtype, qblocks,
                           chunks, launched);
}

template <typename T>
void launch_t(const Params& p, int Dh, int mode, int32_t mask_dtype, uint32_t qblocks, uint32_t chunks,
              uint32_t launched, hipStream_t s) {
    switch (Dh) {
        case 16: launch_d<T, 16>(p, mode, mask_dtype, qblocks, chunks, launched, s); break;
        case 32: launch_d<T, 32>(p, mode, mask_dtype, qblocks, chunks, launched, s); break;
        case 64: launch_d<T, 64>(p, mode, mask_dtype, qblocks, chunks, launched, s); break;
        case 128: launch_d<T, 128>(p, mode, mask_dtype, qblocks, chunks, launched, s); break;
        default: launch_d<T, 256>(p, mode, mask_dtype, qblocks, chunks, launched, s); break;
    }
}

}  // namespace

void launch_wide(const Params& p, int Dh, int kmask, int32_t dtype, int32_t mask_dtype, hipStream_t s) {
    const uint32_t qblocks = static_cast<uint32_t>((p.N + kWideQueries - 1) / kWideQueries);
    const uint32_t chunks = static_cast<uint32_t>(uint64_t(p.B) * uint64_t(p.H) * qblocks);
    const uint32_t launched = xcd_launch_count(chunks);
    const int mode = kmask == kMaskRegion ? 2 : kmask == kNoMask ? 0 : 1;
    if (dtype == CRUMPET_DTYPE_F16)
        launch_t<_Float16>(p, Dh, mode, mask_dtype, qblocks, chunks, launched, s);
    else if (dtype == CRUMPET_DTYPE_BF16)
        launch_t<__bf16>(p, Dh, mode, mask_dtype, qblocks, chunks, launched, s);
    else
        launch_t<float>(p, Dh, mode, mask_dtype, qblocks, chunks, launched, s);
}

}  // namespace attn
}  // namespace crumpet
