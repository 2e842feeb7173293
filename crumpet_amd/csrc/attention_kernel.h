// Fused 3D Swin window attention kernel for gfx950 (MFMA 16x16 tiles, wave64).
//
// Per window b and head h:
//   S   = (q * scale) k^T + bias[h] + (boundary[b] ? mask[b mod M] : 0)
//   out = softmax_rows(S) v
//
// Work decomposition
//   One workgroup (4 waves) per (window, head).  K and V of that pair are
//   staged once in LDS (K row-major, V transposed), zero-padded to 16*NT
//   keys.  Each wave then owns 16-query strips.  For a strip it computes the
//   transposed score block S^T = K Q^T tile by tile, one MFMA per 16 keys x
//   16 queries; the accumulator input is the bias tile (plus the mask tile on
//   boundary windows), so those adds cost no VALU work.  The whole strip row
//   (NT * 16 keys) stays in registers, so the softmax is an exact two-pass
//   one (max, then exp2 and sum) with no online rescaling.
//
// Layout trick
//   In the 16x16 MFMA output a lane holds 4 consecutive rows of one column.
//   With S^T (keys as rows, queries as columns) lane l holds 4 keys of query
//   l%16, which is exactly the B-operand layout of the second product
//   O^T = V^T P^T.  P therefore never leaves registers: it is rounded to the
//   input type in place and fed straight into v_mfma_f32_16x16x32_{f16,bf16}
//   (two key tiles per instruction).  O^T lands as 4 consecutive head-dim
//   values of one query per lane, which is one 8-byte store.
//
// Control flow
//   The tile count NT is a template parameter (one of kTileCounts) and the
//   masked / unmasked strip bodies are separate instantiations chosen once
//   per workgroup, so the unrolled tile loop has no per-tile branches.
//   Padded query rows load the last real row (their output is never
//   stored); mask loads go through a buffer descriptor bounded by the
//   window, so padded keys need no test either (their bias is -inf).
//
// Padding
//   The bias is first copied into a padded fp32 workspace [H][NP][NP]
//   (NP = 16*NT) whose padded key columns hold -inf (probability exactly 0)
//   and whose padded query rows hold 0.
//
// Numerics follow torch-ext/crumpet/fused_attention.py:82-146: q is scaled
// in fp32 and rounded back to the input type, products accumulate in fp32,
// bias then mask are added in fp32, the row sum is taken over fp32
// probabilities, P is rounded (RNE) to the input type before the second
// product, and the output is acc / rowsum rounded to the output type.
#pragma once

#include <hip/hip_runtime.h>

#include <math.h>

#include "crumpet_common.h"
#include "crumpet_hip.h"

namespace crumpet {
namespace attn {

// Per-dtype entry points (one translation unit each, compiled in parallel).
struct Params;
void launch_f16(const Params& p, int NT, int kmask, hipStream_t s);
void launch_bf16(const Params& p, int NT, int kmask, hipStream_t s);
void launch_f32(const Params& p, int NT, int kmask, hipStream_t s);

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr float kLog2e = 1.4426950408889634f;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

struct Params {
    const void* q;
    const void* k;
    const void* v;
    void* out;
    int64_t qs[4], ks[4], vs[4], os[4];  // element strides (b, h, n, d)
    const float* bias_ws;                // [H][NP][NP] fp32, NP = 16 * NT
    const void* mask;                    // [M][N][N] or null, unit key stride
    int64_t ms[3];
    int32_t mask_batch;
    const uint8_t* boundary;
    float scale;
    int32_t B, H, N;
    int32_t strips;  // ceil(N / 16)
    int32_t vec_io;  // q/k/v/out rows are 4-element aligned with unit d stride
    uint32_t chunks, launched;
};

// Tile counts the kernel is compiled for; a call runs with the smallest one
// that covers ceil(N / 16).
constexpr int kTileCounts[] = {1, 2, 4, 8, 14, 22, 32};

inline int select_tiles(int64_t N) {
    const int64_t need = (N + 15) / 16;
    for (int c : kTileCounts)
        if (c >= need) return c;
    return -1;
}

// Kernels and device helpers have internal linkage: every translation unit
// that instantiates them gets its own copy, and none is exported.
namespace {

template <typename T>
struct Frag;

template <>
struct Frag<_Float16> {
    typedef f16x4 x4;
    typedef f16x8 x8;
    static __device__ __forceinline__ f32x4 mma16(x4 a, x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 mma32(x8 a, x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Frag<__bf16> {
    typedef bf16x4 x4;
    typedef bf16x8 x8;
    static __device__ __forceinline__ f32x4 mma16(x4 a, x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                         __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 mma32(x8 a, x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Frag<float> {
    typedef f32x4 x4;
};

// 4 consecutive head-dim elements (d0..d0+3) of one row.
template <typename T>
__device__ __forceinline__ typename Frag<T>::x4 load_row4(const T* row, int64_t sd, int d0, bool vec) {
    typedef typename Frag<T>::x4 X4;
    if (vec) return *reinterpret_cast<const X4*>(row + d0);
    X4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = row[(d0 + e) * sd];
    return r;
}

// Waves per SIMD the register allocation targets; the strip's score row
// (NT * 4 fp32 per lane) dominates the budget.
template <typename T, int NT, int kMask>
constexpr int waves_per_eu() {
    return NT <= 8 ? 4 : (NT <= 22 ? 3 : 2);
}

// Mask storage types (template parameter kMask).
enum MaskKind { kNoMask = 0, kMaskF16 = 1, kMaskF32 = 2, kMaskBF16 = 3 };

// One 16-query strip s of window b, head h.  q_lds holds Q already scaled
// and rounded, K row-major, V transposed; padded rows/keys are zero.
template <typename T, int NT, int kMask, bool kUseMask>
__device__ __forceinline__ void attend_strip(const Params& p, const T* __restrict__ q_lds,
                                             const T* __restrict__ k_lds,
                                             const T* __restrict__ vt_lds, int vt_stride, T* ob,
                                             int b, int h, int s, int col, int g, bool vec) {
    typedef typename Frag<T>::x4 X4;
    constexpr int NP = NT * 16;
    constexpr int kPrefetch = NT < 6 ? NT : 6;
    const int N = p.N;
    const int qi = s * 16 + col;

    // B operand of S^T = K Q^T: Q[qi][4g..4g+3]
    const X4 qf = *reinterpret_cast<const X4*>(&q_lds[qi * 16 + 4 * g]);

    const float* brow = p.bias_ws + (int64_t(h) * NP + qi) * NP + 4 * g;

    // Mask of this window read through a buffer descriptor spanning exactly
    // the window's [N, N] extent: offsets past it return 0 in hardware, so the
    // loads need no per-key test.  Padded keys of a row read a finite
    // neighbour value, harmless under their -inf bias; padded query rows read
    // row N-1 and are never stored.  Per-tile offsets are instruction
    // immediates.
    constexpr int kMaskBytes = (kMask == kMaskF32) ? 4 : 2;
    __amdgpu_buffer_rsrc_t mrsrc;
    int mvoff = 0;
    if constexpr (kUseMask) {
        const int qr = qi < N ? qi : N - 1;
        const char* mbase = static_cast<const char*>(p.mask) +
                            int64_t(b % p.mask_batch) * p.ms[0] * kMaskBytes;
        const int extent = static_cast<int>(((N - 1) * p.ms[1] + N) * kMaskBytes);
        mrsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(mbase), 0, extent, 0x00020000);
        mvoff = static_cast<int>((qr * p.ms[1] + 4 * g) * kMaskBytes);
    }

    // accumulator input of tile t, fetched kPrefetch tiles ahead
    f32x4 bq[kPrefetch];
    uint32_t mq[kUseMask ? 4 * kPrefetch : 1];
    auto fetch = [&](int t, int slot) {
        bq[slot] = *reinterpret_cast<const f32x4*>(brow + 16 * t);
        if constexpr (kUseMask) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int off = mvoff + (16 * t + r) * kMaskBytes;
                if constexpr (kMaskBytes == 2)
                    mq[4 * slot + r] = __builtin_amdgcn_raw_buffer_load_b16(mrsrc, off, 0, 0);
                else
                    mq[4 * slot + r] = __builtin_amdgcn_raw_buffer_load_b32(mrsrc, off, 0, 0);
            }
        }
    };
#pragma unroll
    for (int t = 0; t < kPrefetch; ++t) fetch(t, t);

    f32x4 S[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int slot = t % kPrefetch;
        f32x4 c = bq[slot];
        if constexpr (kUseMask) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t bits = mq[4 * slot + r];
                if constexpr (kMask == kMaskF16)
                    c[r] += static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
                else if constexpr (kMask == kMaskBF16)
                    c[r] += __uint_as_float(bits << 16);
                else
                    c[r] += __uint_as_float(bits);
            }
        }
        if (t + kPrefetch < NT) fetch(t + kPrefetch, slot);
        if constexpr (sizeof(T) == 2) {
            const X4 kf = *reinterpret_cast<const X4*>(&k_lds[(16 * t + col) * 16 + 4 * g]);
            S[t] = Frag<T>::mma16(kf, qf, c);
        } else {
            const f32x4 kf = *reinterpret_cast<const f32x4*>(&k_lds[(16 * t + col) * 16 + 4 * g]);
            f32x4 acc = c;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[kk], qf[kk], acc, 0, 0, 0);
            S[t] = acc;
        }
        // keep the ring: no load of a later tile may be hoisted above this point
        __builtin_amdgcn_sched_barrier(0);
    }

    // exact row max over all keys: two 3-input maxes per tile on two
    // independent chains, then across the 4 lane groups
    float m0 = -INFINITY, m1 = -INFINITY;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        if (t & 1) {
            m1 = fmaxf(fmaxf(m1, S[t][0]), S[t][1]);
            m1 = fmaxf(fmaxf(m1, S[t][2]), S[t][3]);
        } else {
            m0 = fmaxf(fmaxf(m0, S[t][0]), S[t][1]);
            m0 = fmaxf(fmaxf(m0, S[t][2]), S[t][3]);
        }
    }
    float m = fmaxf(m0, m1);
    m = fmaxf(m, __shfl_xor(m, 16));
    m = fmaxf(m, __shfl_xor(m, 32));
    const float mb = m * kLog2e;

#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) S[t][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(S[t][r], kLog2e, -mb));

    // O^T = V^T P^T; the row sums ride on the matrix pipe as ones^T P^T
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
    float l;
    const T* vrow = &vt_lds[col * vt_stride + 4 * g];
    if constexpr (sizeof(T) == 2) {
        typedef typename Frag<T>::x8 X8;
        f32x4 lacc = {0.0f, 0.0f, 0.0f, 0.0f};
        X8 ones8;
        X4 ones4;
#pragma unroll
        for (int r = 0; r < 8; ++r) ones8[r] = T(1.0f);
#pragma unroll
        for (int r = 0; r < 4; ++r) ones4[r] = T(1.0f);
#pragma unroll
        for (int t = 0; t + 1 < NT; t += 2) {
            X8 pb, va;
            const X4 v0 = *reinterpret_cast<const X4*>(vrow + 16 * t);
            const X4 v1 = *reinterpret_cast<const X4*>(vrow + 16 * t + 16);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pb[r] = T(S[t][r]);
                pb[r + 4] = T(S[t + 1][r]);
                va[r] = v0[r];
                va[r + 4] = v1[r];
            }
            o = Frag<T>::mma32(va, pb, o);
            lacc = Frag<T>::mma32(ones8, pb, lacc);
        }
        if constexpr (NT % 2 == 1) {
            X4 pb;
#pragma unroll
            for (int r = 0; r < 4; ++r) pb[r] = T(S[NT - 1][r]);
            const X4 v0 = *reinterpret_cast<const X4*>(vrow + 16 * (NT - 1));
            o = Frag<T>::mma16(v0, pb, o);
            lacc = Frag<T>::mma16(ones4, pb, lacc);
        }
        l = lacc[0];  // every row of ones^T P^T holds the sum for query col
    } else {
        float ls = 0.0f;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const f32x4 v0 = *reinterpret_cast<const f32x4*>(vrow + 16 * t);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                o = __builtin_amdgcn_mfma_f32_16x16x4f32(v0[r], S[t][r], o, 0, 0, 0);
                ls += S[t][r];
            }
        }
        ls += __shfl_xor(ls, 16);
        l = ls + __shfl_xor(ls, 32);
    }

    // lane holds O[qi][4g + r], r = 0..3
    if (qi < N) {
        T* orow = ob + qi * p.os[2];
        const float inv = 1.0f / l;
        X4 res;
#pragma unroll
        for (int r = 0; r < 4; ++r) res[r] = T(o[r] * inv);
        if (vec) {
            *reinterpret_cast<X4*>(orow + 4 * g) = res;
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) orow[(4 * g + r) * p.os[3]] = res[r];
        }
    }
}

template <typename T, int NT, int kMask>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(waves_per_eu<T, NT, kMask>(), waves_per_eu<T, NT, kMask>())))
swin_attention_d16_kernel(const Params p) {
    typedef typename Frag<T>::x4 X4;
    constexpr int NP = NT * 16;
    constexpr int kVtStride = NP + 4;  // keeps 8/16-byte row alignment, breaks bank aliasing
    __shared__ __attribute__((aligned(16))) T q_lds[NP * 16];
    __shared__ __attribute__((aligned(16))) T k_lds[NP * 16];
    __shared__ __attribute__((aligned(16))) T vt_lds[16 * kVtStride];

    uint32_t chunk;
    if (!xcd_chunk(blockIdx.x, p.launched, p.chunks, chunk)) return;
    const int b = static_cast<int>(chunk / p.H);
    const int h = static_cast<int>(chunk % p.H);
    const int N = p.N;
    const bool vec = p.vec_io != 0;

    // ---- stage Q (scaled in fp32, rounded back), K (row-major) and V
    //      (transposed) of this (b, h) in LDS; rows past N are zero ----
    const T* qb = static_cast<const T*>(p.q) + b * p.qs[0] + h * p.qs[1];
    const T* kb = static_cast<const T*>(p.k) + b * p.ks[0] + h * p.ks[1];
    const T* vb = static_cast<const T*>(p.v) + b * p.vs[0] + h * p.vs[1];
    for (int c = threadIdx.x; c < NP * 4; c += kThreads) {
        const int n = c >> 2;
        const int d0 = (c & 3) * 4;
        X4 qv, kv, vv;
        if (n < N) {
            qv = load_row4<T>(qb + n * p.qs[2], p.qs[3], d0, vec);
            kv = load_row4<T>(kb + n * p.ks[2], p.ks[3], d0, vec);
            vv = load_row4<T>(vb + n * p.vs[2], p.vs[3], d0, vec);
#pragma unroll
            for (int e = 0; e < 4; ++e) qv[e] = T(static_cast<float>(qv[e]) * p.scale);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) qv[e] = kv[e] = vv[e] = T(0.0f);
        }
        *reinterpret_cast<X4*>(&q_lds[n * 16 + d0]) = qv;
        *reinterpret_cast<X4*>(&k_lds[n * 16 + d0]) = kv;
#pragma unroll
        for (int e = 0; e < 4; ++e) vt_lds[(d0 + e) * kVtStride + n] = vv[e];
    }
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15;
    const int g = lane >> 4;
    T* ob = static_cast<T*>(p.out) + b * p.os[0] + h * p.os[1];
    const bool use_mask = kMask != kNoMask && (p.boundary == nullptr || p.boundary[b] != 0);

    if constexpr (kMask != kNoMask) {
        if (use_mask) {
            for (int s = wave; s < p.strips; s += kWaves)
                attend_strip<T, NT, kMask, true>(p, q_lds, k_lds, vt_lds, kVtStride, ob, b, h, s, col, g, vec);
            return;
        }
    }
    for (int s = wave; s < p.strips; s += kWaves)
        attend_strip<T, NT, kMask, false>(p, q_lds, k_lds, vt_lds, kVtStride, ob, b, h, s, col, g, vec);
}

// Launch for element type T; NT from kTileCounts, kmask a MaskKind.
template <typename T>
void launch(const Params& p, int NT, int kmask, hipStream_t s) {
    const dim3 grid(p.launched), block(kThreads);
#define CRUMPET_ATTN_MASK(NTV, MK) \
    hipLaunchKernelGGL((swin_attention_d16_kernel<T, NTV, MK>), grid, block, 0, s, p)
#define CRUMPET_ATTN_NT(NTV)                                        \
    case NTV:                                                       \
        switch (kmask) {                                            \
            case kNoMask: CRUMPET_ATTN_MASK(NTV, kNoMask); break;   \
            case kMaskF16: CRUMPET_ATTN_MASK(NTV, kMaskF16); break; \
            case kMaskF32: CRUMPET_ATTN_MASK(NTV, kMaskF32); break; \
            default: CRUMPET_ATTN_MASK(NTV, kMaskBF16); break;      \
        }                                                           \
        break;
    switch (NT) {
        CRUMPET_ATTN_NT(1)
        CRUMPET_ATTN_NT(2)
        CRUMPET_ATTN_NT(4)
        CRUMPET_ATTN_NT(8)
        CRUMPET_ATTN_NT(14)
        CRUMPET_ATTN_NT(22)
        CRUMPET_ATTN_NT(32)
        default: break;
    }
#undef CRUMPET_ATTN_NT
#undef CRUMPET_ATTN_MASK
}

}  // namespace

}  // namespace attn
}  // namespace crumpet
