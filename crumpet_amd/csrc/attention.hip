// Fused 3D Swin window attention for gfx950 (MFMA 16x16 tiles, wave64).
//
// Per window b and head h:
//   S   = (q * scale) k^T + bias[h] + (boundary[b] ? mask[b mod M] : 0)
//   out = softmax_rows(S) v
//
// Work decomposition
//   One workgroup (4 waves) per (window, head).  K and V of that pair are
//   staged once in LDS (K row-major, V transposed), zero-padded to NP = 16*nt
//   keys.  Each wave then owns 16-query strips.  For a strip it computes the
//   transposed score block S^T = K Q^T tile by tile with one MFMA per
//   16 keys x 16 queries tile; the accumulator is initialised with the bias
//   tile, so the bias add is free.  A whole strip row (up to NT_MAX * 16
//   keys) stays in registers, so the softmax is exact two-pass (max, then
//   exp2 and sum) with no online rescaling.
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
// Padding
//   The bias is first copied into a padded fp32 workspace [H][NP][NP] whose
//   padded key columns hold -inf (so padded keys get probability exactly 0
//   without any per-element test) and whose padded query rows hold 0.
//
// Numerics follow torch-ext/crumpet/fused_attention.py:82-146: q is scaled
// in fp32 and rounded back to the input type, products accumulate in fp32,
// bias then mask are added in fp32, the row sum is taken over fp32
// probabilities, P is rounded (RNE) to the input type before the second
// product, and the output is acc / rowsum rounded to the output type.
#include <hip/hip_runtime.h>

#include <math.h>

#include "crumpet_common.h"
#include "crumpet_hip.h"

namespace crumpet {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr float kLog2e = 1.4426950408889634f;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

struct AttnParams {
    const void* q;
    const void* k;
    const void* v;
    void* out;
    int64_t qs[4], ks[4], vs[4], os[4];  // element strides (b, h, n, d)
    const float* bias_ws;                // [H][NP][NP] fp32
    const void* mask;                    // [M][N][N] or null
    int64_t ms[3];
    int32_t mask_batch;
    int32_t mask_dtype;
    const uint8_t* boundary;
    float scale;
    int32_t B, H, N, nt, NP;
    int32_t vec_io;  // q/k/v/out rows are 4-element aligned with unit d stride
    uint32_t chunks, launched;
};

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

// Load 4 consecutive head-dim elements (d0..d0+3) of one row, or zeros.
template <typename T>
__device__ __forceinline__ typename Frag<T>::x4 load_row4(const T* row, int64_t sd, int d0,
                                                          bool valid, bool vec) {
    typedef typename Frag<T>::x4 X4;
    X4 r;
    if (!valid) {
        for (int e = 0; e < 4; ++e) r[e] = T(0.0f);
        return r;
    }
    if (vec) return *reinterpret_cast<const X4*>(row + d0);
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = row[(d0 + e) * sd];
    return r;
}

// Mask element as fp32.  kMask = 1: 16-bit storage (fp16, or bf16 when
// mask_bf16), kMask = 2: fp32 storage.
template <int kMask>
__device__ __forceinline__ float load_mask(const void* base, int64_t off, bool mask_bf16) {
    if constexpr (kMask == 2) {
        return static_cast<const float*>(base)[off];
    } else {
        const uint16_t u = static_cast<const uint16_t*>(base)[off];
        const float as_bf16 = __uint_as_float(static_cast<uint32_t>(u) << 16);
        const float as_f16 = static_cast<float>(__builtin_bit_cast(_Float16, u));
        return mask_bf16 ? as_bf16 : as_f16;
    }
}

// Padded fp32 copy of the bias: ws[h][i][j] = bias[h][i][j] for i, j < N,
// -inf in padded key columns, 0 in padded query rows of real keys.
template <typename TB>
__global__ void __launch_bounds__(kThreads)
bias_prep_kernel(float* __restrict__ ws, const TB* __restrict__ bias, int64_t sh, int64_t si,
                 int64_t sj, int32_t H, int32_t N, int32_t NP) {
    const int64_t total = int64_t(H) * NP * NP;
    for (int64_t idx = int64_t(blockIdx.x) * kThreads + threadIdx.x; idx < total;
         idx += int64_t(gridDim.x) * kThreads) {
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

template <typename T, int NT_MAX, int kMask>
__global__ void __launch_bounds__(kThreads)
swin_attention_d16_kernel(const AttnParams p) {
    typedef typename Frag<T>::x4 X4;
    constexpr int kNP = NT_MAX * 16;
    constexpr int kVtStride = kNP + 4;  // keeps 8/16-byte row alignment, breaks bank aliasing
    __shared__ __attribute__((aligned(16))) T k_lds[kNP * 16];
    __shared__ __attribute__((aligned(16))) T vt_lds[16 * kVtStride];

    uint32_t chunk;
    if (!xcd_chunk(blockIdx.x, p.launched, p.chunks, chunk)) return;
    const int b = static_cast<int>(chunk / p.H);
    const int h = static_cast<int>(chunk % p.H);
    const int N = p.N;
    const int nt = p.nt;
    const int NP = p.NP;
    const bool vec = p.vec_io != 0;

    // ---- stage K (row-major) and V (transposed) of this (b, h) in LDS ----
    const T* kb = static_cast<const T*>(p.k) + b * p.ks[0] + h * p.ks[1];
    const T* vb = static_cast<const T*>(p.v) + b * p.vs[0] + h * p.vs[1];
    for (int c = threadIdx.x; c < NP * 4; c += kThreads) {
        const int n = c >> 2;
        const int d0 = (c & 3) * 4;
        const bool valid = n < N;
        const X4 kv = load_row4<T>(kb + n * p.ks[2], p.ks[3], d0, valid, vec);
        *reinterpret_cast<X4*>(&k_lds[n * 16 + d0]) = kv;
        const X4 vv = load_row4<T>(vb + n * p.vs[2], p.vs[3], d0, valid, vec);
#pragma unroll
        for (int e = 0; e < 4; ++e) vt_lds[(d0 + e) * kVtStride + n] = vv[e];
    }
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15;
    const int g = lane >> 4;
    const bool use_mask = kMask != 0 && (p.boundary == nullptr || p.boundary[b] != 0);
    const bool mask_bf16 = p.mask_dtype == CRUMPET_DTYPE_BF16;
    const T* qb = static_cast<const T*>(p.q) + b * p.qs[0] + h * p.qs[1];
    T* ob = static_cast<T*>(p.out) + b * p.os[0] + h * p.os[1];

    for (int s = wave; s < nt; s += kWaves) {
        const int qi = s * 16 + col;
        const bool qvalid = qi < N;

        // B operand of S^T = K Q^T: Q[qi][4g..4g+3], scaled in fp32 and rounded back.
        X4 qf = load_row4<T>(qb + qi * p.qs[2], p.qs[3], 4 * g, qvalid, vec);
#pragma unroll
        for (int e = 0; e < 4; ++e) qf[e] = T(static_cast<float>(qf[e]) * p.scale);

        f32x4 S[NT_MAX];
        const float* brow = p.bias_ws + (int64_t(h) * NP + qi) * NP + 4 * g;
        const int64_t mrow = int64_t(b % p.mask_batch) * p.ms[0] + int64_t(qi) * p.ms[1];
#pragma unroll
        for (int t = 0; t < NT_MAX; ++t) {
            if (t < nt) {
                f32x4 c = *reinterpret_cast<const f32x4*>(brow + 16 * t);
                if (kMask != 0 && use_mask && qvalid) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int key = 16 * t + 4 * g + r;
                        if (key < N) c[r] += load_mask<kMask>(p.mask, mrow + key * p.ms[2], mask_bf16);
                    }
                }
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
            }
        }

        // exact row max over all keys: in-lane, then across the 4 lane groups
        float m = -INFINITY;
#pragma unroll
        for (int t = 0; t < NT_MAX; ++t)
            if (t < nt) m = fmaxf(m, fmaxf(fmaxf(S[t][0], S[t][1]), fmaxf(S[t][2], S[t][3])));
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        const float mb = m * kLog2e;

        float l = 0.0f;
#pragma unroll
        for (int t = 0; t < NT_MAX; ++t) {
            if (t < nt) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    S[t][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(S[t][r], kLog2e, -mb));
                    l += S[t][r];
                }
            }
        }
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);

        // O^T = V^T P^T
        f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
        const T* vrow = &vt_lds[col * kVtStride + 4 * g];
        if constexpr (sizeof(T) == 2) {
            typedef typename Frag<T>::x8 X8;
#pragma unroll
            for (int t = 0; t < NT_MAX; t += 2) {
                if (t + 1 < nt) {
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
                } else if (t < nt) {
                    X4 pb;
#pragma unroll
                    for (int r = 0; r < 4; ++r) pb[r] = T(S[t][r]);
                    const X4 v0 = *reinterpret_cast<const X4*>(vrow + 16 * t);
                    o = Frag<T>::mma16(v0, pb, o);
                }
            }
        } else {
#pragma unroll
            for (int t = 0; t < NT_MAX; ++t) {
                if (t < nt) {
                    const f32x4 v0 = *reinterpret_cast<const f32x4*>(vrow + 16 * t);
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        o = __builtin_amdgcn_mfma_f32_16x16x4f32(v0[r], S[t][r], o, 0, 0, 0);
                }
            }
        }

        // lane holds O[qi][4g + r], r = 0..3
        if (qvalid) {
            T* orow = ob + qi * p.os[2];
            X4 res;
#pragma unroll
            for (int r = 0; r < 4; ++r) res[r] = T(o[r] / l);
            if (vec) {
                *reinterpret_cast<X4*>(orow + 4 * g) = res;
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) orow[(4 * g + r) * p.os[3]] = res[r];
            }
        }
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

template <typename T, int kMask>
void launch_attention_nt(const AttnParams& p, hipStream_t s) {
    const dim3 grid(p.launched), block(kThreads);
    if (p.nt <= 8)
        hipLaunchKernelGGL((swin_attention_d16_kernel<T, 8, kMask>), grid, block, 0, s, p);
    else if (p.nt <= 22)
        hipLaunchKernelGGL((swin_attention_d16_kernel<T, 22, kMask>), grid, block, 0, s, p);
    else
        hipLaunchKernelGGL((swin_attention_d16_kernel<T, 32, kMask>), grid, block, 0, s, p);
}

template <typename T>
int launch_attention_t(const AttnParams& p, hipStream_t s) {
    if (p.mask == nullptr)
        launch_attention_nt<T, 0>(p, s);
    else if (p.mask_dtype == CRUMPET_DTYPE_F32)
        launch_attention_nt<T, 2>(p, s);
    else
        launch_attention_nt<T, 1>(p, s);
    return check_launch("crumpet_fused_swin_attention");
}

}  // namespace
}  // namespace crumpet

extern "C" size_t crumpet_fused_swin_attention_workspace_size(int64_t Hh, int64_t N) {
    if (Hh <= 0 || N <= 0) return 0;
    const int64_t np = (N + 15) / 16 * 16;
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

    AttnParams p;
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
    p.mask_dtype = mask_dtype;
    p.boundary = boundary;
    p.scale = scale;
    p.B = static_cast<int32_t>(B);
    p.H = static_cast<int32_t>(Hh);
    p.N = static_cast<int32_t>(N);
    p.nt = static_cast<int32_t>((N + 15) / 16);
    p.NP = p.nt * 16;

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
        const int64_t total = Hh * p.NP * p.NP;
        int64_t blocks = (total + kThreads - 1) / kThreads;
        if (blocks > 4096) blocks = 4096;
        float* ws = static_cast<float*>(workspace);
        if (bias_dtype == CRUMPET_DTYPE_F16)
            hipLaunchKernelGGL(bias_prep_kernel<_Float16>, dim3(blocks), dim3(kThreads), 0, s, ws,
                               static_cast<const _Float16*>(bias), bias_strides[0],
                               bias_strides[1], bias_strides[2], p.H, p.N, p.NP);
        else if (bias_dtype == CRUMPET_DTYPE_BF16)
            hipLaunchKernelGGL(bias_prep_kernel<__bf16>, dim3(blocks), dim3(kThreads), 0, s, ws,
                               static_cast<const __bf16*>(bias), bias_strides[0],
                               bias_strides[1], bias_strides[2], p.H, p.N, p.NP);
        else
            hipLaunchKernelGGL(bias_prep_kernel<float>, dim3(blocks), dim3(kThreads), 0, s, ws,
                               static_cast<const float*>(bias), bias_strides[0], bias_strides[1],
                               bias_strides[2], p.H, p.N, p.NP);
        const int st2 = check_launch(what);
        if (st2 != CRUMPET_OK) return st2;
    }
    if (dtype == CRUMPET_DTYPE_F16) return launch_attention_t<_Float16>(p, s);
    if (dtype == CRUMPET_DTYPE_BF16) return launch_attention_t<__bf16>(p, s);
    return launch_attention_t<float>(p, s);
}
