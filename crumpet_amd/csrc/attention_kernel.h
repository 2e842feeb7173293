// Fused 3D Swin window attention kernel for gfx950 (MFMA 16x16 tiles, wave64).
//
// Per window b and head h:
//   S   = (q * scale) k^T + bias[h] + mask_b
//   out = softmax_rows(S) v
// where mask_b is, depending on the mode,
//   tensor : boundary[b] ? mask[b mod M] : 0          (a mask tensor)
//   region : the shifted-window mask of window b      (from the geometry)
//   none   : 0
//
// Work decomposition (bias-stationary, persistent)
//   The relative-position bias is the same for every window, so it is kept in
//   registers instead of being re-read per window: a workgroup of 4 waves
//   owns one head h and a group of 4 consecutive 16-query strips, and walks a
//   range of windows (contiguous; every ranges-th window with a mask tensor,
//   whose boundary windows cost more and come in runs).  Each wave builds the fp32 bias tiles of its
//   strip (NT tiles of 16 keys x 16 queries, 4 values per lane each) once,
//   straight from the caller's bias tensor (any float dtype and strides),
//   and uses them as the accumulator input of every window's S^T = K Q^T
//   MFMAs, so the bias add costs neither memory traffic nor VALU work.
//
//   Q (the group's 64 rows, pre-scaled and rounded), K and V of a window
//   live in LDS, double-buffered, one barrier per window.  While the waves
//   compute window i, window i+1 is fetched into the other buffer: for 2-byte
//   types with unit d stride, K and V rows go straight from memory to LDS
//   (buffer loads with the lds flag) and only Q passes through registers;
//   otherwise each thread holds its share in registers and stores it after
//   the compute (fp32 keeps V transposed; 2-byte types keep V row-major and
//   read V^T with the LDS transpose read).
//
//   In region mode the windows are visited grouped by type (which axes the
//   window is last on; at most 8 types).  The shifted-window mask of a window
//   depends only on its type, so it is folded into the bias tiles when the
//   type changes (at most 8 times per workgroup) and costs nothing per
//   window.  Logical index -> window uses per-type offsets and mixed-radix
//   decoding (Params::types).
//
// Layout trick
//   In the 16x16 MFMA output a lane holds 4 consecutive rows of one column.
//   With S^T (keys as rows, queries as columns) lane l holds 4 keys of query
//   l%16, which is exactly the B-operand layout of the second product
//   O^T = V^T P^T.  P therefore never leaves registers: it is rounded to the
//   input type in place and fed straight into v_mfma_f32_16x16x32_{f16,bf16}
//   (two key tiles per instruction); the row sums ride on the same pipe as
//   ones^T P^T.  O^T lands as 4 consecutive head-dim values of one query per
//   lane, which is one 8-byte store.
//
// Softmax
//   Online over key chunks of at most 6 tiles, with a lazy rescale: the
//   first chunk fixes the row max, later chunks exponentiate against the
//   running max and refresh it (with a cross-lane reduction and a rescale of
//   O and the row sums) only when a score exceeds it by more than
//   kLazyMargin.  The small chunks keep 2-byte vector-IO kernels within 168
//   VGPRs, i.e. 3 waves per SIMD, which this latency-bound loop needs more
//   than it needs a larger register budget.
//
// Padding
//   Keys are padded to NP = 16*NT: padded key columns get a -inf bias
//   (probability exactly 0), padded query rows a 0 bias (never stored).  K, V
//   and Q rows past N are copies of row N-1 in LDS (zero on the register
//   path), harmless under those biases.  The kernel needs no workspace.
//
// Numerics follow torch-ext/crumpet/fused_attention.py:82-146: q is scaled
// in fp32 and rounded back to the input type, products accumulate in fp32,
// bias and mask are added in fp32, P is rounded (RNE) to the input type
// before the second product, and the output is acc / rowsum rounded to the
// output type.  The row sum is taken over the rounded P (the same values the
// numerator uses).
#pragma once

#include <hip/hip_runtime.h>

#include <math.h>

#include "crumpet_common.h"
#include "crumpet_hip.h"

namespace crumpet {
namespace attn {

constexpr int kWaves = 4;  // waves (strips) per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr float kLog2e = 1.4426950408889634f;
// After the first key chunk of a strip, scores may exceed the running row
// max by this much (natural-log units) before the max is refreshed: the
// chunk's exps start right away with the running max, and P = exp(s - m)
// stays below e^8, well inside fp16 / bf16 range.
constexpr float kLazyMargin = 8.0f;

// Mask modes (template parameter kMask).
enum MaskKind { kNoMask = 0, kMaskF16 = 1, kMaskF32 = 2, kMaskBF16 = 3, kMaskRegion = 4 };

// Window-type table of region mode: logical window index -> window.
struct TypeTable {
    int32_t ntypes;
    int32_t offset[9];     // first logical index of each type (offset[ntypes] = B)
    int32_t code[8];       // 3-bit type code: bit2 = last along D, bit1 = H, bit0 = W
    int32_t choices[8][3]; // window choices per axis for the type
};

struct Params {
    const void* q;
    const void* k;
    const void* v;
    void* out;
    int64_t qs[4], ks[4], vs[4], os[4];  // element strides (b, h, n, d)
    const void* bias;                    // [H][N][N], element strides bsd (bsd[2] == 1)
    int64_t bsd[3];
    int32_t bias_dtype;                  // crumpet_dtype code
    const void* mask;                    // tensor mode: [M][N][N], unit key stride
    int64_t ms[3];
    int32_t mask_batch;
    const uint8_t* boundary;  // tensor mode: [B] flags or null
    float scale;
    int32_t B, H, N;
    int32_t strips;          // ceil(N / 16)
    int32_t groups;          // ceil(strips / kWaves)
    int32_t win_per_wg;      // windows walked by one workgroup
    int32_t ranges;          // ceil(B / win_per_wg)
    int32_t vec_io;          // q/k/v/out rows are 4-element aligned with unit d stride
    uint32_t chunks, launched;
    // region mode geometry
    int32_t nWd, nWh, nWw, nW;  // windows per volume along D, H, W and in total
    int32_t ws[3], ss[3];       // window and shift sizes
    TypeTable types;
};

// Per-dtype entry points (one translation unit each, compiled in parallel).
void launch_f16(const Params& p, int NT, int kmask, hipStream_t s);
void launch_bf16(const Params& p, int NT, int kmask, hipStream_t s);
void launch_f32(const Params& p, int NT, int kmask, hipStream_t s);

// General kernel (attention_wide.hip): head dims 16, 32, 64 and 128, any N
// (shifted-window regions up to kWideMaxRegionN tokens).  The caller has
// checked the head dim, the region size and that B * H * ceil(N / 64) fits
// in 31 bits.
constexpr int kWideMaxRegionN = 2048;
constexpr int kWideQueries = 64;  // queries per workgroup of the general kernel
void launch_wide(const Params& p, int Dh, int kmask, int32_t dtype, int32_t mask_dtype, hipStream_t s);

// Tile counts the kernel is compiled for; a call runs with the smallest one
// that covers ceil(N / 16).
constexpr int kTileCounts[] = {1, 2, 4, 8, 14, 22, 32};

inline int select_tiles(int64_t N) {
    const int64_t need = (N + 15) / 16;
    for (int c : kTileCounts)
        if (c >= need) return c;
    return -1;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

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

// 4 consecutive head-dim elements (d0..d0+3) of one row: one vector load
// when rows have unit d stride and 4-element alignment (kVec), else 4 loads.
template <typename T, bool kVec>
__device__ __forceinline__ typename Frag<T>::x4 load_row4(const T* row, int64_t sd, int d0) {
    typedef typename Frag<T>::x4 X4;
    if constexpr (kVec) {
        return *reinterpret_cast<const X4*>(row + d0);
    } else {
        X4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = row[(d0 + e) * sd];
        return r;
    }
}

// q * scale in fp32, rounded back to the input type (the reference scales q
// before the dot product: torch-ext/crumpet/fused_attention.py:88).  Applied
// when Q is written to LDS, not when its load is issued, so no wait for the
// load lands between the issue of a window's rows and the compute that
// should hide them.
template <typename T>
__device__ __forceinline__ typename Frag<T>::x4 scaled(typename Frag<T>::x4 v, float scale) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = T(static_cast<float>(v[e]) * scale);
    return v;
}

// K layout in LDS.  2-byte types: each 16-row key tile stores the first 8
// dims of its 16 rows (16 B each), then the last 8, so the 32 lanes of a
// half-wave that read one key fragment (rows 0-15, dims 4g..4g+3, g = 0, 1)
// cover 256 contiguous bytes; with plain 32-byte rows they would cover only
// half of each row and collide on the banks.  fp32: plain rows.
template <typename T>
__device__ __forceinline__ constexpr int kidx(int row, int d) {
    if constexpr (sizeof(T) == 2)
        return (row >> 4) * 256 + (d >> 3) * 128 + (row & 15) * 8 + (d & 7);
    else
        return row * 16 + d;
}

template <typename T>
__device__ __forceinline__ typename Frag<T>::x4 zero4() {
    typename Frag<T>::x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = T(0.0f);
    return r;
}

// Waves per SIMD the register allocation targets: the strip's fp32 bias
// tiles (4 * NT per lane) and one chunk of scores dominate the budget.  With
// 2-byte types and vector IO (K and V arrive by LDS DMA, no staging
// registers) up to 22 tiles fit 168 VGPRs, i.e. 3 waves; the latency-bound
// loop gains more from the third wave than it loses to the smaller budget.
template <typename T, int NT, int kMask, bool kVec>
constexpr int waves_per_eu() {
    // (an fp32 mask's prefetch ring needs a few more registers than 168 at
    // 22 tiles)
    if constexpr (sizeof(T) == 2 && kVec && !(kMask == kMaskF32 && NT > 14))
        return NT <= 4 ? 4 : (NT <= 22 ? 3 : 2);
    return NT <= 4 ? 4 : (NT <= 8 ? 3 : 2);
}

// Walks the logical window indices [i0, i1) of a workgroup.  In region mode
// windows are visited grouped by type: logical index -> (type t, outer batch,
// window choice per axis) in mixed radix.  The start is decoded once; each
// step is a carry chain of scalar compares (no divisions per window).  In
// the other modes logical index i is window base + i * stride.
template <int kMask>
struct WindowIter {
    int i;
    int t, batch, jd, jh, jw;  // region mode position
    int cd, ch, cw, code;      // choices of the current type, its code
    int batches;               // outer batches (B / nW)
    int base = 0, stride = 1;  // other modes: window = base + i * stride

    __device__ __forceinline__ void load_type(const Params& p) {
        code = p.types.code[t];
        cd = p.types.choices[t][0];
        ch = p.types.choices[t][1];
        cw = p.types.choices[t][2];
    }

    __device__ __forceinline__ void init(const Params& p, int i0) {
        i = i0;
        if constexpr (kMask == kMaskRegion) {
            batches = p.B / p.nW;
            t = 0;
            while (t + 1 < p.types.ntypes && i0 >= p.types.offset[t + 1]) ++t;
            load_type(p);
            int j = i0 - p.types.offset[t];
            const int per = cd * ch * cw;
            batch = j / per;
            j -= batch * per;
            jw = j % cw;
            j /= cw;
            jh = j % ch;
            jd = j / ch;
        }
    }

    // window index b of the current position; type_code of its mask
    __device__ __forceinline__ int window(const Params& p, int& type_code) const {
        if constexpr (kMask != kMaskRegion) {
            type_code = 0;
            return base + i * stride;
        } else {
            const int wd = (code & 4) ? p.nWd - 1 : jd;
            const int wh = (code & 2) ? p.nWh - 1 : jh;
            const int ww = (code & 1) ? p.nWw - 1 : jw;
            type_code = code;
            return batch * p.nW + (wd * p.nWh + wh) * p.nWw + ww;
        }
    }

    __device__ __forceinline__ void next(const Params& p) {
        ++i;
        if constexpr (kMask == kMaskRegion) {
            if (++jw < cw) return;
            jw = 0;
            if (++jh < ch) return;
            jh = 0;
            if (++jd < cd) return;
            jd = 0;
            if (++batch < batches) return;
            batch = 0;
            if (t + 1 < p.types.ntypes) {
                ++t;
                load_type(p);
            }
        }
    }
};

// A workgroup-uniform 64-bit address made provably uniform (scalar
// registers).  readfirstlane returns a signed int: both halves are taken as
// uint32_t so that the low word is zero-extended, not sign-extended.
__device__ __forceinline__ char* uniform_ptr(const void* ptr) {
    const uint64_t a = reinterpret_cast<uint64_t>(ptr);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a)));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32)));
    return reinterpret_cast<char*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// 2-byte element types keep V row-major in LDS (like K) and read the
// V^T MFMA fragments with the gfx950 LDS transpose read: within each group
// of 16 lanes, lane j receives element j%4 of the 8-byte vectors addressed by
// lanes 4e + j/4 (e = 0..3).  Lane (col, g) addressing V row 16t + 4g + col/4
// at dims 4*(col%4) therefore receives V[16t + 4g + e][col], e = 0..3.  fp32
// keeps a transposed V (no 32-bit transpose read is used).
template <typename T>
constexpr bool v_row_major() {
    return sizeof(T) == 2;
}

template <typename T>
__device__ __forceinline__ typename Frag<T>::x4 lds_read_tr(const T* ptr) {
    typedef __attribute__((address_space(3))) i16x4 LdsI16x4;
    const i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LdsI16x4*)(const_cast<T*>(ptr)));
    return __builtin_bit_cast(typename Frag<T>::x4, r);
}

// Staging of one window's Q (this group's rows), K and V into LDS.  Each
// thread owns chunks c = tid + k * kThreads of 4 elements; kQChunks Q chunks
// come first, then NP*4 K chunks, then NP*4 V chunks.
template <typename T, int NT, bool kVec>
struct Stage {
    static constexpr int NP = NT * 16;
    static constexpr int kQRows = 16 * kWaves;
    static constexpr int kQChunks = kQRows * 4;
    static constexpr int kChunks = kQChunks + 2 * NP * 4;
    static constexpr int kPerThread = (kChunks + kThreads - 1) / kThreads;
    static constexpr int kRows = NP;           // K / V rows held in LDS
    static constexpr int kVtStride = NP + 4;  // keeps 8/16-byte rows, breaks bank aliasing
    static constexpr int kVLds = v_row_major<T>() ? kRows * 16 : 16 * kVtStride;
    typedef typename Frag<T>::x4 X4;

    X4 r[kPerThread];

    __device__ __forceinline__ void load(const Params& p, int b, int h, int q0, T*, T*) {
        const T* qb = static_cast<const T*>(p.q) + b * p.qs[0] + h * p.qs[1];
        const T* kb = static_cast<const T*>(p.k) + b * p.ks[0] + h * p.ks[1];
        const T* vb = static_cast<const T*>(p.v) + b * p.vs[0] + h * p.vs[1];
#pragma unroll
        for (int k = 0; k < kPerThread; ++k) {
            const int c = threadIdx.x + k * kThreads;
            r[k] = zero4<T>();
            if (c < kQChunks) {
                const int n = q0 + (c >> 2);
                if (n < p.N) r[k] = load_row4<T, kVec>(qb + n * p.qs[2], p.qs[3], (c & 3) * 4);
            } else if (c < kChunks) {
                const int cc = c - kQChunks;
                const bool isv = cc >= NP * 4;
                const int c2 = isv ? cc - NP * 4 : cc;
                const int n = c2 >> 2;
                if (n < p.N)
                    r[k] = isv ? load_row4<T, kVec>(vb + n * p.vs[2], p.vs[3], (c2 & 3) * 4)
                               : load_row4<T, kVec>(kb + n * p.ks[2], p.ks[3], (c2 & 3) * 4);
            }
        }
    }

    __device__ __forceinline__ void store(float scale, T* q_lds, T* k_lds, T* vt_lds) const {
#pragma unroll
        for (int k = 0; k < kPerThread; ++k) {
            const int c = threadIdx.x + k * kThreads;
            if (c < kQChunks) {
                *reinterpret_cast<X4*>(&q_lds[c * 4]) = scaled<T>(r[k], scale);
            } else if (c < kChunks) {
                const int cc = c - kQChunks;
                if (cc < NP * 4) {
                    *reinterpret_cast<X4*>(&k_lds[kidx<T>(cc >> 2, (cc & 3) * 4)]) = r[k];
                } else {
                    const int c2 = cc - NP * 4;
                    if constexpr (v_row_major<T>()) {
                        *reinterpret_cast<X4*>(&vt_lds[c2 * 4]) = r[k];
                    } else {
                        const int n = c2 >> 2, d0 = (c2 & 3) * 4;
#pragma unroll
                        for (int e = 0; e < 4; ++e) vt_lds[(d0 + e) * kVtStride + n] = r[k][e];
                    }
                }
            }
        }
    }
};

// Staging for rows with unit d stride and 4-element alignment (the MONAI
// qkv layout).  Thread tid owns 4 dims (4*(tid&3)..) of rows tid/4 + 64k:
// one Q row of this group and kKC rows each of K and V.  Loads go through
// per-window buffer descriptors with 32-bit offsets; row indices past N are
// clamped to N-1, which is harmless: padded keys have a -inf bias, padded V
// rows meet P = 0 and padded query rows are never stored.  No branches and
// no 64-bit address arithmetic per row.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Buffer descriptor words (base, stride 0, num_records, dword-3 flags) for a
// window's rows, workgroup-uniform.
template <typename T>
__device__ __forceinline__ u32x4 desc_words(const void* base, int64_t off, int64_t s2, int N) {
    const char* ub = uniform_ptr(static_cast<const char*>(base) + off * int64_t(sizeof(T)));
    const uint64_t a = reinterpret_cast<uint64_t>(ub);
    u32x4 d;
    d[0] = static_cast<uint32_t>(a);
    d[1] = static_cast<uint32_t>(a >> 32) & 0xffffu;
    d[2] = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
        static_cast<int>((int64_t(N - 1) * s2 + 16) * int64_t(sizeof(T)))));
    d[3] = 0x00020000u;
    return d;
}

// 16 bytes per lane from buffer offset voff straight into LDS at
// lds_addr + 16 * lane (lds_addr wave-uniform).  Written as inline asm so
// that the compiler does not treat it as an LDS store it must wait for
// before unrelated LDS reads; the caller waits (vmcnt(0)) before the barrier
// that publishes the rows.  gfx950 needs one wait state between an SALU
// write of M0 and an LDS-DMA load that reads it; the compiler's hazard
// recognizer does not look inside inline asm, hence the explicit s_nop.
__device__ __forceinline__ void dma16(u32x4 desc, uint32_t lds_addr, int voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_addr), "v"(voff), "s"(desc)
                 : "memory", "m0");
}

template <typename T, int NT>
struct Stage<T, NT, true> {
    static constexpr int NP = NT * 16;
    static constexpr int kQRows = 16 * kWaves;
    static constexpr bool kDma = v_row_major<T>();
    static constexpr int kKC = (NP + 63) / 64;          // register path: rows per thread
    static constexpr int kRows = kDma ? (NP + 31) / 32 * 32 : kKC * 64;
    static constexpr int kRounds = (kRows + 127) / 128;  // DMA path: 32-row loads per wave
    static constexpr int kVtStride = kRows + 4;
    static constexpr int kVLds = v_row_major<T>() ? kRows * 16 : 16 * kVtStride;
    typedef typename Frag<T>::x4 X4;

    X4 rq, rk[kDma ? 1 : kKC], rv[kDma ? 1 : kKC];

    static __device__ __forceinline__ X4 ld(__amdgpu_buffer_rsrc_t rs, int off) {
        if constexpr (sizeof(X4) == 8)
            return __builtin_bit_cast(X4, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0));
        else
            return __builtin_bit_cast(X4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }

    static __device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t off,
                                                                 int64_t s2, int N) {
        char* ub = uniform_ptr(static_cast<const char*>(base) + off * int64_t(sizeof(T)));
        const int extent = __builtin_amdgcn_readfirstlane(
            static_cast<int>((int64_t(N - 1) * s2 + 16) * int64_t(sizeof(T))));
        return __builtin_amdgcn_make_buffer_rsrc(ub, 0, extent, 0x00020000);
    }

    __device__ __forceinline__ void load(const Params& p, int b, int h, int q0, T* k_dst, T* v_dst) {
        const int N = p.N;
        const int n0 = threadIdx.x >> 2;
        const int d0 = (threadIdx.x & 3) * 4;
        const auto qr = rsrc(p.q, int64_t(b) * p.qs[0] + int64_t(h) * p.qs[1], p.qs[2], N);
        const auto kr = rsrc(p.k, int64_t(b) * p.ks[0] + int64_t(h) * p.ks[1], p.ks[2], N);
        const auto vr = rsrc(p.v, int64_t(b) * p.vs[0] + int64_t(h) * p.vs[1], p.vs[2], N);
        const int qs2 = static_cast<int>(p.qs[2]), ks2 = static_cast<int>(p.ks[2]),
                  vs2 = static_cast<int>(p.vs[2]);
        constexpr int es = sizeof(T);
        const int nq = min(q0 + n0, N - 1);
        rq = ld(qr, (nq * qs2 + d0) * es);
        if constexpr (kDma) {
            // 16 bytes per lane straight into LDS: the 64 lanes of wave w in
            // round r fill the 1 KB of rows 32*(4r + w) .. +31 at a
            // wave-uniform LDS address, lane l writing its 16-byte chunk l;
            // which row half each lane fetches sets the layout (kidx for K,
            // plain rows for V)
            const int lane = threadIdx.x & 63;
            const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
            const u32x4 kd = desc_words<T>(p.k, int64_t(b) * p.ks[0] + int64_t(h) * p.ks[1], p.ks[2], N);
            const u32x4 vd = desc_words<T>(p.v, int64_t(b) * p.vs[0] + int64_t(h) * p.vs[1], p.vs[2], N);
            typedef __attribute__((address_space(3))) T LdsT;
            const uint32_t kl = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((LdsT*)k_dst));
            const uint32_t vl = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((LdsT*)v_dst));
#pragma unroll
            for (int r = 0; r < kRounds; ++r) {
                const int row0 = 32 * (4 * r + wave);
                if (row0 < kRows) {  // wave-uniform
                    // K: chunk l of these two tiles is (tile l/32, dims 8*((l/16)&1), row l&15)
                    const int nk = min(row0 + ((lane >> 5) << 4) + (lane & 15), N - 1);
                    const int hk = ((lane >> 4) & 1) * 8;
                    dma16(kd, kl + row0 * 32, (nk * ks2 + hk) * es);
                    // V: plain 32-byte rows (its transpose reads are conflict-free)
                    const int nv = min(row0 + (lane >> 1), N - 1);
                    dma16(vd, vl + row0 * 32, (nv * vs2 + (lane & 1) * 8) * es);
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < kKC; ++k) {
                const int n = min(n0 + 64 * k, N - 1);
                rk[k] = ld(kr, (n * ks2 + d0) * es);
                rv[k] = ld(vr, (n * vs2 + d0) * es);
            }
        }
    }

    __device__ __forceinline__ void store(float scale, T* q_lds, T* k_lds, T* vt_lds) const {
        const int tid = threadIdx.x;
        const int n0 = tid >> 2, d0 = (tid & 3) * 4;
        *reinterpret_cast<X4*>(&q_lds[tid * 4]) = scaled<T>(rq, scale);
        if constexpr (!kDma) {
#pragma unroll
            for (int k = 0; k < kKC; ++k) {
                *reinterpret_cast<X4*>(&k_lds[(tid + k * kThreads) * 4]) = rk[k];
                if constexpr (v_row_major<T>()) {
                    *reinterpret_cast<X4*>(&vt_lds[(tid + k * kThreads) * 4]) = rv[k];
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) vt_lds[(d0 + e) * kVtStride + n0 + 64 * k] = rv[k][e];
                }
            }
        }
    }
};

// Bias (+ region mask) tiles of one strip, built in registers from the
// caller's bias tensor: lane (col, g) holds keys 16t + 4g + r of query qi.
// The head's [N, N] bias is read through a buffer descriptor, so every load
// is one instruction with an immediate offset; keys past N read 0 or the
// next row and are replaced by -inf (probability exactly 0).  Padded query
// rows get 0 (never stored).  In region mode a key whose shift-region class
// differs from the query's on an axis that the window type `code` splits
// gets -100.  Runs when the window type changes (at most 8 times per
// workgroup), never per window.
template <int NT, int kMask>
__device__ __forceinline__ void build_tiles(f32x4 (&bs)[NT], const Params& prm, int h, int qi, int g,
                                            int code, const uint8_t* cls) {
    // Re-read the kernel arguments (Params is the kernel's only argument, at
    // offset 0 of the kernarg segment) through an opaque copy of the segment
    // pointer, so that the compiler loads them here instead of keeping them
    // live in scalar registers across the whole window loop.
    (void)prm;
    typedef const __attribute__((address_space(4))) Params KParams;
    KParams* pp = (KParams*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(pp));
    const int N = pp->N;
    const int bias_dtype = pp->bias_dtype;
    const int64_t bsd0 = pp->bsd[0], bsd1 = pp->bsd[1];
    const void* bias_ptr = pp->bias;
    const bool row = qi < N;
    const int qr = row ? qi : N - 1;
    const int es = bias_dtype == CRUMPET_DTYPE_F32 ? 4 : 2;
    const bool bf16 = bias_dtype == CRUMPET_DTYPE_BF16;
    // base and extent are workgroup-uniform; readfirstlane keeps the
    // descriptor in SGPRs (a VGPR descriptor costs a waterfall loop per load)
    char* hb = uniform_ptr(static_cast<const char*>(bias_ptr) + int64_t(h) * bsd0 * es);
    const int extent =
        __builtin_amdgcn_readfirstlane(static_cast<int>((int64_t(N - 1) * bsd1 + N) * es));
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(hb, 0, extent, 0x00020000);
    const int voff = static_cast<int>((int64_t(qr) * bsd1 + 4 * g) * es);
    uint32_t cq = 0, cmask = 0;
    if constexpr (kMask == kMaskRegion) {
        cq = uint32_t(cls[qr]) * 0x01010101u;  // query class in every byte
        cmask = uint32_t(code) * 0x01010101u;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        uint32_t split = 0;  // byte r nonzero: key 16t+4g+r is masked by the region rule
        if constexpr (kMask == kMaskRegion)
            split = (*reinterpret_cast<const uint32_t*>(&cls[16 * t + 4 * g]) ^ cq) & cmask;
        float v4[4];
        if (es == 4) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                v4[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, voff + (16 * t + r) * 4, 0, 0));
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t bits = __builtin_amdgcn_raw_buffer_load_b16(rs, voff + (16 * t + r) * 2, 0, 0);
                const float fh = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
                v4[r] = bf16 ? __uint_as_float(bits << 16) : fh;
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float val = v4[r];
            if constexpr (kMask == kMaskRegion) {
                if ((split >> (8 * r)) & 0xffu) val += -100.0f;
            }
            val = row ? val : 0.0f;
            bs[t][r] = (16 * t + 4 * g + r) < N ? val : -INFINITY;
        }
    }
}


// max(m[l], m[l ^ 16]) and max(m[l], m[l ^ 32]) with the gfx950 VALU row
// swaps: with both operands m, v_permlane16_swap returns m[l] and m[l ^ 16]
// (in some order), v_permlane32_swap m[l] and m[l ^ 32]; no LDS round trip.
__device__ __forceinline__ float xmax16(float m) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xmax32(float m) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// One strip (16 queries, NT*16 keys) of one window.
template <typename T, int NT, int kMask, bool kUseMask, bool kVec>
__device__ __forceinline__ void attend(const Params& p, const f32x4 (&bs)[NT], const T* __restrict__ q_lds,
                                       const T* __restrict__ k_lds, const T* __restrict__ vt_lds,
                                       int b, int h, int wave, int qi, int col, int g) {
    typedef typename Frag<T>::x4 X4;
    constexpr int kVtStride = Stage<T, NT, kVec>::kVtStride;
    constexpr int kMaskBytes = (kMask == kMaskF32) ? 4 : 2;
    constexpr int kPrefetch = NT < 6 ? NT : 6;
    const int N = p.N;

    // B operand of S^T = K Q^T: Q[qi][4g..4g+3] (pre-scaled in LDS)
    const X4 qf = *reinterpret_cast<const X4*>(&q_lds[(wave * 16 + col) * 16 + 4 * g]);

    // Tensor mask through a buffer descriptor spanning exactly the window's
    // [N, N] extent: offsets past it return 0, so no per-key test is needed;
    // padded keys read a finite neighbour (their bias is -inf) and padded
    // query rows read row N-1 (never stored).  A lane's 4 keys of a tile are
    // contiguous in the mask row, so each tile is one 8-byte (16-bit masks)
    // or 16-byte (fp32 masks) load; the target accesses memory unaligned, so
    // an odd row stride is fine.  Only the last tile of row N-1 can reach
    // past the extent, and a range check at dword or access granularity
    // would then zero in-range keys sharing the load, so those lanes read
    // that tile again element by element.  Offsets are immediates.
    typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
    constexpr int kMaskWords = kMaskBytes;  // 32-bit words per lane and tile
    __amdgpu_buffer_rsrc_t mrsrc;
    int mvoff = 0;
    uint32_t mq[kUseMask ? kMaskWords * kPrefetch : 1];
    if constexpr (kUseMask) {
        const int qr = qi < N ? qi : N - 1;
        // uniform base and extent, kept in scalar registers (see build_tiles)
        char* mb = uniform_ptr(static_cast<const char*>(p.mask) +
                               int64_t(b % p.mask_batch) * p.ms[0] * kMaskBytes);
        const int extent =
            __builtin_amdgcn_readfirstlane(static_cast<int>(((N - 1) * p.ms[1] + N) * kMaskBytes));
        mrsrc = __builtin_amdgcn_make_buffer_rsrc(mb, 0, extent, 0x00020000);
        mvoff = static_cast<int>((qr * p.ms[1] + 4 * g) * kMaskBytes);
    }
    auto fetch = [&](int t, int slot) {
        if constexpr (kUseMask) {
            const int off = mvoff + 16 * t * kMaskBytes;
            if constexpr (kMaskBytes == 2) {
                const u32x2v w = __builtin_amdgcn_raw_buffer_load_b64(mrsrc, off, 0, 0);
                mq[2 * slot] = w[0];
                mq[2 * slot + 1] = w[1];
            } else {
                const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(mrsrc, off, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) mq[4 * slot + r] = w[r];
            }
            // the load that reaches past the extent end (row N-1, last tile)
            // is read again element by element (compile-time tile test)
            if (t == NT - 1 && qi == N - 1 && 16 * t + 4 * g + 3 >= N) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (kMaskBytes == 2) {
                        const uint32_t h = __builtin_amdgcn_raw_buffer_load_b16(mrsrc, off + 2 * r, 0, 0);
                        if (r & 1)
                            mq[2 * slot + (r >> 1)] |= h << 16;
                        else
                            mq[2 * slot + (r >> 1)] = h;
                    } else {
                        mq[4 * slot + r] = __builtin_amdgcn_raw_buffer_load_b32(mrsrc, off + 4 * r, 0, 0);
                    }
                }
            }
        }
    };
    if constexpr (kUseMask) {
#pragma unroll
        for (int t = 0; t < kPrefetch; ++t) fetch(t, t);
    }

    // Keys are processed in chunks of at most 6 tiles with an online softmax
    // between chunks, which keeps only one chunk of scores in registers next
    // to the bias tiles.  The first chunk sets the row max exactly; a later
    // chunk exponentiates against the running max unless one of its scores
    // exceeds it by more than kLazyMargin (a wave-uniform test), in which
    // case the max is refreshed across the lane groups and O and the row
    // sums are rescaled first.  Softmax is invariant to the offset, so only
    // the rare refresh costs a cross-lane reduction.
    constexpr int kNumChunks = (NT + 5) / 6;
    constexpr int kChunk = (NT + kNumChunks - 1) / kNumChunks;
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 lacc = {0.0f, 0.0f, 0.0f, 0.0f};
    float lsum = 0.0f;  // fp32 path row sum (VALU)
    float m_run = -INFINITY;
    float mb_run = 0.0f;  // m_run * log2(e)
    // V^T fragments: transposed layout (fp32) or transpose reads of row-major V
    const T* vrow = v_row_major<T>() ? &vt_lds[(4 * g + (col >> 2)) * 16 + (col & 3) * 4]
                                     : &vt_lds[col * kVtStride + 4 * g];

#pragma unroll
    for (int c0 = 0; c0 < NT; c0 += kChunk) {
        // chunks must not interleave: that would keep two chunks of scores live
        __builtin_amdgcn_sched_barrier(0);
        // matrix sections run at raised wave priority, the softmax at the
        // normal one, so that a SIMD's waves tend to alternate between the
        // two pipes (1-2%)
        __builtin_amdgcn_s_setprio(1);
        const int cn = (NT - c0 < kChunk) ? NT - c0 : kChunk;
        f32x4 S[kChunk];
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            if (u >= cn) break;
            const int t = c0 + u;
            f32x4 c = bs[t];
            if constexpr (kUseMask) {
                const int slot = t % kPrefetch;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (kMask == kMaskF32) {
                        c[r] += __uint_as_float(mq[4 * slot + r]);
                    } else {
                        const uint32_t w = mq[2 * slot + (r >> 1)];
                        if constexpr (kMask == kMaskF16)
                            c[r] += static_cast<float>(
                                __builtin_bit_cast(_Float16, static_cast<uint16_t>(r & 1 ? w >> 16 : w)));
                        else
                            c[r] += __uint_as_float(r & 1 ? (w & 0xffff0000u) : (w << 16));
                    }
                }
                if (t + kPrefetch < NT) fetch(t + kPrefetch, slot);
            }
            if constexpr (sizeof(T) == 2) {
                const X4 kf = *reinterpret_cast<const X4*>(&k_lds[kidx<T>(16 * t + col, 4 * g)]);
                S[u] = Frag<T>::mma16(kf, qf, c);
            } else {
                const f32x4 kf = *reinterpret_cast<const f32x4*>(&k_lds[(16 * t + col) * 16 + 4 * g]);
                f32x4 acc = c;
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[kk], qf[kk], acc, 0, 0, 0);
                S[u] = acc;
            }
            if constexpr (kUseMask) __builtin_amdgcn_sched_barrier(0);  // keep the mask ring
        }

        __builtin_amdgcn_s_setprio(0);
        // lane-local chunk max: two 3-input maxes per tile on two chains
        float m0 = m_run, m1 = -INFINITY;
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            if (u >= cn) break;
            if (u & 1) {
                m1 = fmaxf(fmaxf(m1, S[u][0]), S[u][1]);
                m1 = fmaxf(fmaxf(m1, S[u][2]), S[u][3]);
            } else {
                m0 = fmaxf(fmaxf(m0, S[u][0]), S[u][1]);
                m0 = fmaxf(fmaxf(m0, S[u][2]), S[u][3]);
            }
        }
        const float lm = fmaxf(m0, m1);
        if (c0 == 0) {
            m_run = xmax32(xmax16(lm));
            mb_run = m_run * kLog2e;
        } else if (__builtin_amdgcn_ballot_w64(lm > m_run + kLazyMargin) != 0) {
            const float m = xmax32(xmax16(lm));
            const float mbn = m * kLog2e;
            const float alpha = __builtin_amdgcn_exp2f(mb_run - mbn);
            o *= alpha;
            lacc *= alpha;
            lsum *= alpha;
            m_run = m;
            mb_run = mbn;
        }
        const float mb = mb_run;

#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            if (u >= cn) break;
#pragma unroll
            for (int r = 0; r < 4; ++r) S[u][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(S[u][r], kLog2e, -mb));
        }

        __builtin_amdgcn_s_setprio(1);
        // O^T += V^T P^T; the row sums ride on the matrix pipe as ones^T P^T
        if constexpr (sizeof(T) == 2) {
            typedef typename Frag<T>::x8 X8;
            X8 ones8;
#pragma unroll
            for (int r = 0; r < 8; ++r) ones8[r] = T(1.0f);
#pragma unroll
            for (int u = 0; u + 1 < kChunk; u += 2) {
                if (u + 1 >= cn) break;
                const int t = c0 + u;
                X8 pb, va;
                const X4 v0 = lds_read_tr<T>(vrow + 256 * t);
                const X4 v1 = lds_read_tr<T>(vrow + 256 * (t + 1));
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    pb[r] = T(S[u][r]);
                    pb[r + 4] = T(S[u + 1][r]);
                    va[r] = v0[r];
                    va[r + 4] = v1[r];
                }
                o = Frag<T>::mma32(va, pb, o);
                lacc = Frag<T>::mma32(ones8, pb, lacc);
            }
            if (cn & 1) {
                // odd tile: the same 16x16x32 instruction with a zero upper
                // half, so each accumulator chain uses a single MFMA opcode
                const int u = cn - 1;
                X8 pb, va;
                const X4 v0 = lds_read_tr<T>(vrow + 256 * (c0 + u));
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    pb[r] = T(S[u][r]);
                    pb[r + 4] = T(0.0f);
                    va[r] = v0[r];
                    va[r + 4] = T(0.0f);
                }
                o = Frag<T>::mma32(va, pb, o);
                lacc = Frag<T>::mma32(ones8, pb, lacc);
            }
        } else {
#pragma unroll
            for (int u = 0; u < kChunk; ++u) {
                if (u >= cn) break;
                const f32x4 v0 = *reinterpret_cast<const f32x4*>(vrow + 16 * (c0 + u));
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    o = __builtin_amdgcn_mfma_f32_16x16x4f32(v0[r], S[u][r], o, 0, 0, 0);
                    lsum += S[u][r];
                }
            }
        }
    }
    __builtin_amdgcn_s_setprio(0);
    float l;
    if constexpr (sizeof(T) == 2) {
        l = lacc[0];  // every row of ones^T P^T holds the sum for query col
    } else {
        lsum += __shfl_xor(lsum, 16);
        l = lsum + __shfl_xor(lsum, 32);
    }

    // lane holds O[qi][4g + r], r = 0..3
    if (qi < N) {
        T* orow = static_cast<T*>(p.out) + b * p.os[0] + h * p.os[1] + qi * p.os[2];
        const float inv = 1.0f / l;
        X4 res;
#pragma unroll
        for (int r = 0; r < 4; ++r) res[r] = T(o[r] * inv);
        if constexpr (kVec) {
            *reinterpret_cast<X4*>(orow + 4 * g) = res;
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) orow[(4 * g + r) * p.os[3]] = res[r];
        }
    }
}

template <typename T, int NT, int kMask, bool kVec>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(waves_per_eu<T, NT, kMask, kVec>(), waves_per_eu<T, NT, kMask, kVec>())))
swin_attention_d16_kernel(const Params p) {
    typedef Stage<T, NT, kVec> St;
    constexpr int NP = St::NP;
    __shared__ __attribute__((aligned(16))) T q_lds[2][St::kQRows * 16];
    __shared__ __attribute__((aligned(16))) T k_lds[2][St::kRows * 16];
    __shared__ __attribute__((aligned(16))) T vt_lds[2][St::kVLds];
    __shared__ __attribute__((aligned(4))) uint8_t cls_lds[kMask == kMaskRegion ? NP : 4];

    uint32_t chunk;
    if (!xcd_chunk(blockIdx.x, p.launched, p.chunks, chunk)) return;
    // chunk = (range * H + h) * groups + group: the groups of one (range, head)
    // are consecutive, hence on one XCD, and share its L2 for K/V.
    const int grp = static_cast<int>(chunk % p.groups);
    const int rh = static_cast<int>(chunk / p.groups);
    const int h = rh % p.H;
    const int range = rh / p.H;
    // Tensor-mask modes take every ranges-th window (range, range + ranges,
    // ...): a window whose boundary flag is set costs more than one whose
    // flag is clear, and boundary windows come in runs (the last window
    // slab of a volume is a run of nWh * nWw), so contiguous ranges would
    // leave some workgroups with mostly masked windows (17% at config 3).
    constexpr bool kStrided = kMask == kMaskF16 || kMask == kMaskF32 || kMask == kMaskBF16;
    const int i0 = kStrided ? 0 : range * p.win_per_wg;
    const int i1 = kStrided ? (p.B - range + p.ranges - 1) / p.ranges : min(p.B, i0 + p.win_per_wg);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15;
    const int g = lane >> 4;
    const int strip = grp * kWaves + wave;
    const int qi = strip * 16 + col;
    const bool active = strip < p.strips;
    const int q0 = grp * kWaves * 16;  // first query row of this group

    if constexpr (kMask == kMaskRegion) {
        // shift-region class of every window token: one bit per axis, set at
        // or past ws - ss (covered by the prologue barrier below)
        for (int j = threadIdx.x; j < NP; j += kThreads) {
            int c = 0;
            if (j < p.N) {
                const int lw = j % p.ws[2];
                const int t = j / p.ws[2];
                const int lh = t % p.ws[1];
                const int ld = t / p.ws[1];
                c = ((ld >= p.ws[0] - p.ss[0]) ? 4 : 0) | ((lh >= p.ws[1] - p.ss[1]) ? 2 : 0) |
                    ((lw >= p.ws[2] - p.ss[2]) ? 1 : 0);
            }
            cls_lds[j] = static_cast<uint8_t>(c);
        }
    }

    St st;
    WindowIter<kMask> it;
    it.init(p, i0);
    if constexpr (kStrided) {
        it.base = range;
        it.stride = p.ranges;
    }
    int code_cur = -1;
    int code_next;
    int b_next = it.window(p, code_next);
    // tensor mode: the window's boundary flag is read before the next
    // window's rows are requested, so waiting for it never waits for them
    bool flag_next = true;
    if constexpr (kMask != kNoMask && kMask != kMaskRegion)
        flag_next = p.boundary == nullptr || p.boundary[b_next] != 0;
    st.load(p, b_next, h, q0, k_lds[0], vt_lds[0]);
    st.store(p.scale, q_lds[0], k_lds[0], vt_lds[0]);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // LDS-DMA rows have landed
    __syncthreads();

    f32x4 bs[NT];
    for (int i = i0; i < i1; ++i) {
        const int buf = (i - i0) & 1;
        const int b = b_next;
        const int code = code_next;
        const bool flag = flag_next;
        // New bias (+ region mask) tiles are built before the next window's
        // rows are requested: the vector-memory counter retires in order, so
        // waiting for the bias loads after that request would wait for the
        // rows as well.
        if (active && code != code_cur) {  // code is workgroup-uniform
            build_tiles<NT, kMask>(bs, p, h, qi, g, code, cls_lds);
            code_cur = code;
        }
        if (i + 1 < i1) {
            it.next(p);
            b_next = it.window(p, code_next);
            if constexpr (kMask != kNoMask && kMask != kMaskRegion)
                flag_next = p.boundary == nullptr || p.boundary[b_next] != 0;
            st.load(p, b_next, h, q0, k_lds[buf ^ 1], vt_lds[buf ^ 1]);
        }
        if (active) {
            bool use_mask = false;
            if constexpr (kMask != kNoMask && kMask != kMaskRegion) use_mask = flag;
            if (use_mask)
                attend<T, NT, kMask, (kMask != kNoMask && kMask != kMaskRegion), kVec>(
                    p, bs, q_lds[buf], k_lds[buf], vt_lds[buf], b, h, wave, qi, col, g);
            else
                attend<T, NT, kMask, false, kVec>(p, bs, q_lds[buf], k_lds[buf], vt_lds[buf], b,
                                                  h, wave, qi, col, g);
        }
        if (i + 1 < i1) st.store(p.scale, q_lds[buf ^ 1], k_lds[buf ^ 1], vt_lds[buf ^ 1]);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // LDS-DMA rows have landed
        __syncthreads();
    }
}

// Launch for element type T; NT from kTileCounts, kmask a MaskKind.
template <typename T>
void launch(const Params& p, int NT, int kmask, hipStream_t s) {
    const dim3 grid(p.launched), block(kThreads);
#define CRUMPET_ATTN_MASK(NTV, MK)                                                              \
    do {                                                                                        \
        if (p.vec_io)                                                                           \
            hipLaunchKernelGGL((swin_attention_d16_kernel<T, NTV, MK, true>), grid, block, 0, s,  \
                               p);                                                              \
        else                                                                                    \
            hipLaunchKernelGGL((swin_attention_d16_kernel<T, NTV, MK, false>), grid, block, 0, s, \
                               p);                                                              \
    } while (0)
#define CRUMPET_ATTN_NT(NTV)                                            \
    case NTV:                                                           \
        switch (kmask) {                                                \
            case kNoMask: CRUMPET_ATTN_MASK(NTV, kNoMask); break;       \
            case kMaskF16: CRUMPET_ATTN_MASK(NTV, kMaskF16); break;     \
            case kMaskF32: CRUMPET_ATTN_MASK(NTV, kMaskF32); break;     \
            case kMaskBF16: CRUMPET_ATTN_MASK(NTV, kMaskBF16); break;   \
            default: CRUMPET_ATTN_MASK(NTV, kMaskRegion); break;        \
        }                                                               \
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
