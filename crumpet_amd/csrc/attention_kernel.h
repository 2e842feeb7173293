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
//   registers instead of being re-read per window: a workgroup owns one head
//   (4 waves) or kHeadsPerWg heads (12 waves) and a group of 4 consecutive
//   16-query strips of each, and walks a range of windows (contiguous; with
//   a mask tensor every ranges-th window of a mask-major order, because
//   windows whose boundary flag is set cost more and come in runs, and the
//   windows that read one mask then run together on one XCD).  Each wave
//   builds the fp32 bias
//   tiles of its strip (NT tiles of 16 keys x 16 queries, 4 values per lane
//   each) once, straight from the caller's bias tensor (any float dtype and
//   strides), and uses them as the accumulator input of every window's
//   S^T = K Q^T MFMAs, so the bias add costs neither memory traffic nor VALU
//   work.
//
//   Q (the group's 64 rows per head, pre-scaled and rounded), K and V of a
//   window live in LDS, K and V double-buffered, one barrier per window.
//   While the waves compute window i, window i+1 is fetched into the other
//   buffer: for 2-byte types with unit d stride, K and V rows go straight
//   from memory to LDS (buffer loads with the lds flag, a few per wave from
//   inside the tile-pair loop) and only Q passes through registers; with
//   several heads per workgroup they arrive as token records (all heads' K
//   rows, then V rows, as they lie in memory), because a vector load moves
//   whole 128-byte lines.  Otherwise each thread holds its share in
//   registers and stores it after the compute (fp32 keeps V transposed;
//   2-byte types keep V row-major and read V^T with the LDS transpose read).
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
//   lane, which is one 8-byte store (two at head dim 32).
//
// Softmax (2-byte types, attend_offset)
//   Scores are produced in log2 units (Q carries scale * log2(e) as a hi/lo
//   pair in the 32-deep score product, the bias tiles log2(e)), so P = 2^S
//   costs one exp and half a conversion per score.  Instead of a row max, the
//   bias tiles carry a per-query offset, and the exact row sums that the same
//   pass produces check that every P stayed in the range where its rounding
//   is as good as with the exact max; a strip that misses it is redone with
//   the exact max, and its offsets move for the next window.  fp32
//   (attend_f32) keeps an online softmax over key chunks.
//
// Head dim 32 (D = 32; 2-byte types, vector IO, 14 or 22 tiles, one head per
//   workgroup)
//   The head dim fills the 32-deep score product, so Q_hi and Q_lo take one
//   product each per score tile over the same K fragment; V^T enters in two
//   16-dim halves with two output accumulators.  K and V take twice the LDS:
//   at 21-22 strips three strip groups of the head (12 waves, one workgroup
//   per CU) share double-buffered K and V; otherwise they are single-buffered
//   and three 4-wave workgroups per CU overlap each other's staging.
//
// Padding
//   Keys are padded to NP = 16*NT: padded key columns get a -inf bias
//   (probability exactly 0), padded query rows a 0 bias (never stored).  K, V
//   and Q rows past N are copies of row N-1 in LDS (zero on the register
//   path), harmless under those biases.  The kernel needs no workspace.
//
// Numerics follow torch-ext/crumpet/fused_attention.py:82-146: products
// accumulate in fp32, bias and mask are added in fp32, P is rounded (RNE) to
// the input type before the second product, and the output is acc / rowsum
// rounded to the output type.  The reference rounds q * scale to the input
// type; here q * scale * log2(e) enters as hi + lo, which carries it to
// about twice the input precision (for the default scale 16^-0.5 the
// reference's q * scale is exact, and so is this to within fp32).  The row
// sum is taken over the rounded P (the same values the numerator uses; the
// reference sums the unrounded fp32 P): both stay within the tolerance of
// the fp32 formula, and the difference is at most one rounding of P per key.
#pragma once

#include <hip/hip_runtime.h>

#include <math.h>
#include <type_traits>

#include "crumpet_common.h"
#include "crumpet_hip.h"

namespace crumpet {
namespace attn {

constexpr int kWaves = 4;  // waves (strips) per workgroup
constexpr int kThreads = 64 * kWaves;  // threads per head slot of a workgroup
// Heads per workgroup on the LDS-DMA path when H is a multiple of it and
// the heads of a token are adjacent (head stride 16, as in the usual
// [token][3][H][Dh] qkv layout): the workgroup runs the kWaves strips of
// each of its heads and stages their K and V together as token records
// (below), so that its loads read contiguous bytes.  With a mask tensor and
// boundary flags, one head per workgroup is faster (config 3: 186 against
// 237 us; with every window masked 270 against 238 us): those launches
// keep it, and so do fp32 masks (their loop needs more registers than 12
// waves per CU leave).
constexpr int kHeadsPerWg = 3;
// Tile counts with a kHeadsPerWg variant: the large windows, where K/V
// staging dominates and 3 heads' double-buffered K/V still fit one CU's LDS.
constexpr bool multi_head_tiles(int NT) { return NT == 14 || NT == 22; }
// LDS layout of a kHeadsPerWg workgroup: one record per token holding the
// K rows of its heads, then their V rows, as they lie in memory (head
// stride 16, V a fixed distance after K with the same strides), so that a
// 1 KB LDS-DMA load reads ~5 tokens' contiguous K+V bytes.  A vector load
// moves whole 128-byte lines from L2 at a fixed rate per CU, and K+V of a
// token is 2.25 lines; separate 32-byte rows would cost one line each.
// Record stride 104 elements (K 48, V 48, 8 of padding): 52 dwords, so the
// 16 lanes of a K fragment read (16 bytes of 16 consecutive rows) and the
// 4 rows of 32 bytes a 16-lane group of a V transpose read touches land on
// disjoint banks.
constexpr int kRecStride = 104;
constexpr int kRecV = 48;  // V rows' offset in a record
constexpr int kKRec = kRecStride;
constexpr int kVRec = kRecStride;
// Rows staged per window (a multiple of 32) and the loads of a window: 13
// 16-byte chunks per token (6 of K, 6 of V, a padding load), 64 per load.
constexpr int rec_rows(int NT) { return (NT * 16 + 31) / 32 * 32; }
constexpr int rec_loads(int NT) { return (rec_rows(NT) * 13 + 63) / 64; }
constexpr float kLog2e = 1.4426950408889634f;
// After the first key chunk of a strip, scores may exceed the running row
// max by this much (natural-log units) before the max is refreshed: the
// chunk's exps start right away with the running max, and P = exp(s - m)
// stays below e^8, well inside fp16 / bf16 range.
constexpr float kLazyMargin = 8.0f;

// Mask modes (template parameter kMask).  kMaskF16T / kMaskBF16T: a 16-bit
// mask tensor in the tiled layout of mask_tile.hip (one 8-byte word of 4
// keys per lane and key tile, a wave's tile contiguous), for the 2-byte
// tuned kernels at 14 and 22 tiles.
enum MaskKind {
    kNoMask = 0,
    kMaskF16 = 1,
    kMaskF32 = 2,
    kMaskBF16 = 3,
    kMaskRegion = 4,
    kMaskF16T = 5,
    kMaskBF16T = 6
};
constexpr bool mask_tensor(int kind) { return kind != kNoMask && kind != kMaskRegion; }
constexpr bool mask_tiled(int kind) { return kind == kMaskF16T || kind == kMaskBF16T; }
constexpr bool mask_f16(int kind) { return kind == kMaskF16 || kind == kMaskF16T; }

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
    int32_t hpw;             // heads per workgroup: 1, or kHeadsPerWg (H % 3 == 0, LDS-DMA path)
    int32_t kv_delta;        // hpw > 1: elements from a K row to the V row of the same token and head
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
// Head dim 32 on the tuned kernel (attention_d32.hip): 2-byte types, vector
// IO, 14 or 22 tiles (d32_tiles), one head per workgroup: 4 waves
// (p.hpw = 1), or kHeadsPerWg strip groups of 4 waves (p.hpw = kHeadsPerWg)
// at 22 tiles when the strips leave at most 3 of the 24 waves of a head's
// two workgroups idle, as many as the 4-wave form does (d32_group_slots).
void launch_d32(const Params& p, int NT, int kmask, int32_t dtype, hipStream_t s);
constexpr bool d32_tiles(int NT) { return NT == 14 || NT == 22; }
constexpr bool d32_group_slots(int NT, int strips) {
    return NT == 22 && strips % (kWaves * kHeadsPerWg) >= kWaves * kHeadsPerWg - 3;
}

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

// The first tile that can hold key N - 1 for an N that selects NT tiles
// (N > 16 * the previous tile count).
constexpr int first_last_tile(int NT) {
    int prev = 0;
    for (int c : kTileCounts) {
        if (c == NT) return prev;
        prev = c;
    }
    return 0;
}

// Whether lane keys k0 .. k0 + nk - 1 of row `row` include key N - 1 of row
// N - 1 (the fp32-operand kernel's mask reads those element by element).
__device__ __forceinline__ bool holds_last_key(int k0, int nk, int row, int N) {
    return row == N - 1 && k0 <= N - 1 && k0 + nk - 1 >= N - 1;
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
    typedef f32x4 x8;  // unused: fp32 operands take four 16x16x4 steps, no 8-element fragments
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

// Four dims d0 .. d0 + 3 of a Q row into LDS.  2-byte types store
// hi = q * scale rounded (scale includes log2(e)) and the remainder
// lo = q * scale - hi, rounded: hi + lo carries q * scale to about twice the
// input precision, so folding log2(e) into the operand adds no rounding of
// its own.  The row holds [hi 0-7 | lo 0-7 | hi 8-15 | lo 8-15] (the k-slices
// of the score product, q_slice).  fp32 stores q * scale.
template <typename T>
__device__ __forceinline__ void store_q4(T* row, int d0, typename Frag<T>::x4 v, float scale) {
    typedef typename Frag<T>::x4 X4;
    if constexpr (sizeof(T) == 2) {
        X4 hi, lo;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float x = static_cast<float>(v[e]) * scale;
            hi[e] = T(x);
            lo[e] = T(x - static_cast<float>(hi[e]));
        }
        *reinterpret_cast<X4*>(row + (d0 >> 3) * 16 + (d0 & 7)) = hi;
        *reinterpret_cast<X4*>(row + (d0 >> 3) * 16 + 8 + (d0 & 7)) = lo;
    } else {
        *reinterpret_cast<X4*>(row + d0) = scaled<T>(v, scale);
    }
}

// K layout in LDS.  2-byte types: each 16-row key tile stores the first 8
// dims of its 16 rows (16 B each), then the last 8, so a 16x16x32 key
// fragment (lane (col, g): row col, dims 8(g >> 1) .. + 7; the score product
// carries each 8 dims twice, for Q_hi and Q_lo, attend_offset) reads 256
// contiguous bytes with lanes 0-31 and the next 256 with lanes 32-63.  fp32:
// plain rows.
template <typename T>
__device__ __forceinline__ constexpr int kidx(int row, int d) {
    if constexpr (sizeof(T) == 2)
        return (row >> 4) * 256 + (d >> 3) * 128 + (row & 15) * 8 + (d & 7);
    else
        return row * 16 + d;
}

// Head dim 32 (2-byte types): a Q row holds 64 elements, hi = q * scale
// rounded (dims 0-31; scale includes log2(e)) and lo = the rounding
// remainder (32-63), the split store_q4 makes for head dim 16; each score tile then
// takes two 16x16x32 products over the same K fragment (Q_hi, then Q_lo),
// since the head dim fills the product's depth.  A key tile stores dims
// 8c .. 8c + 7 of its 16 rows as block c = 0..3 (16 B per row), so the lanes
// of lane group g that read one key fragment (row col, dims 8g .. 8g + 7)
// cover 256 contiguous bytes; V rows are plain (64 B).
template <typename T>
__device__ __forceinline__ void store_q8(T* row, int d0, typename Frag<T>::x8 v, float scale) {
    typename Frag<T>::x8 hi, lo;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float x = static_cast<float>(v[e]) * scale;
        hi[e] = T(x);
        lo[e] = T(x - static_cast<float>(hi[e]));
    }
    *reinterpret_cast<typename Frag<T>::x8*>(row + d0) = hi;
    *reinterpret_cast<typename Frag<T>::x8*>(row + 32 + d0) = lo;
}

// Elements per Q row in LDS: 2-byte types keep q * scale as a hi/lo pair
// (32 elements at head dim 16, 64 at head dim 32); fp32 keeps 16.
template <typename T, int D>
constexpr int q_row_len() {
    return sizeof(T) == 2 ? 2 * D : 16;
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
    // (an fp32 mask's prefetch needs a few more registers than 168 at 22
    // tiles)
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
            const int L = base + i * stride;
            if constexpr (kMask != kNoMask) {
                // mask-major order: the B / M windows that read mask m
                // (m, m + M, ...) are consecutive logical indices, hence
                // taken by consecutive ranges (consecutive workgroups, on one
                // XCD) at the same step, and share the mask rows in its L2
                const int M = p.mask_batch;
                if (M > 1 && M < p.B) {
                    const int copies = p.B / M;
                    const int m = L / copies;
                    return (L - m * copies) * M + m;
                }
            }
            return L;
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

// Buffer loads are range-checked per dword of the resource: an [N, N]
// extent of 16-bit values that ends in the middle of a dword would read the
// dword holding key N - 1 of row N - 1 as 0.  The bias and mask resources
// therefore start at the extent's base rounded down to 4 bytes (`lead`, 0
// or 2, is added to every offset) and span a whole number of dwords: every
// dword a lane loads is then a 4-aligned word holding at least one byte of
// the extent, so it lies in a mapped page, and its bytes past the extent
// (keys >= N) are masked by the -inf of the bias tiles.
struct AlignedRsrc {
    __amdgpu_buffer_rsrc_t rs;
    int lead;  // bytes from the resource base to the extent's first byte
};
__device__ __forceinline__ AlignedRsrc aligned_rsrc(const char* base, int64_t bytes) {
    char* ub = uniform_ptr(base);
    const int lead = static_cast<int>(reinterpret_cast<uintptr_t>(ub) & 3);
    const int extent = __builtin_amdgcn_readfirstlane(static_cast<int>((bytes + lead + 3) & ~int64_t(3)));
    return {__builtin_amdgcn_make_buffer_rsrc(ub - lead, 0, extent, 0x00020000), lead};
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

// Byte address of an LDS object, and a load of V from such an address
// (keeps the LDS address space where a pointer has to be made opaque).
template <typename T>
__device__ __forceinline__ uint32_t lds_byte_addr(const T* ptr) {
    typedef const __attribute__((address_space(3))) T LdsT;
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((LdsT*)ptr));
}
template <typename V>
__device__ __forceinline__ V lds_load(uint32_t addr) {
    typedef const __attribute__((address_space(3))) V LdsV;
    return *reinterpret_cast<LdsV*>(static_cast<uintptr_t>(addr));
}

// Staging of one window's Q (this group's rows), K and V into LDS.  Each
// thread owns chunks c = tid + k * kThreads of 4 elements; kQChunks Q chunks
// come first, then NP*4 K chunks, then NP*4 V chunks.
template <typename T, int NT, bool kVec, int D = 16>
struct Stage {
    static_assert(D == 16, "head dim 32 runs the LDS-DMA staging");
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
                store_q4<T>(&q_lds[(c >> 2) * q_row_len<T, 16>()], (c & 3) * 4, r[k], scale);
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
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

// Buffer descriptor words (base, stride 0, num_records, dword-3 flags) for a
// window's rows of `row` elements, workgroup-uniform.
template <typename T>
__device__ __forceinline__ u32x4 desc_words(const void* base, int64_t off, int64_t s2, int N, int row = 16) {
    const char* ub = uniform_ptr(static_cast<const char*>(base) + off * int64_t(sizeof(T)));
    const uint64_t a = reinterpret_cast<uint64_t>(ub);
    u32x4 d;
    d[0] = static_cast<uint32_t>(a);
    d[1] = static_cast<uint32_t>(a >> 32) & 0xffffu;
    d[2] = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
        static_cast<int>((int64_t(N - 1) * s2 + row) * int64_t(sizeof(T)))));
    d[3] = 0x00020000u;
    return d;
}

// 16 bytes per lane from buffer offset voff straight into LDS at
// lds_addr + 16 * lane (lds_addr wave-uniform).  Written as inline asm so
// that the compiler does not treat it as an LDS store it must wait for
// before unrelated LDS reads; the caller waits (vmcnt(0)) before the barrier
// that publishes the rows.  The LDS address enters as an operand bound to
// M0, so the compiler writes M0 itself and knows it is live (a clobber of
// the reserved M0 would not be honoured).  The compiler's hazard recognizer
// does not look inside inline asm, so the asm carries the wait states its
// load needs: one after an SALU write of M0, and five after a VALU write of
// an SGPR of the descriptor.  The second happens when the compiler restores
// a spilled descriptor with v_readlane right before the load: with one wait
// state the load read a stale descriptor word and fetched wrong rows (the
// head-dim-16 bf16 kernel at 14 tiles, which spills scalar registers).
__device__ __forceinline__ void dma16(u32x4 desc, uint32_t lds_addr, int voff) {
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(voff), "s"(desc), "{m0}"(lds_addr)
                 : "memory");
}

// s_waitcnt vmcnt(0) through the builtin: the compiler's wait insertion
// then knows that every vector-memory request issued before it, its own
// and the LDS-DMA loads it cannot see, has completed, and adds no wait of
// its own for registers loaded earlier.
__device__ __forceinline__ void wait_vmem() {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0) expcnt(7) lgkmcnt(15)
}

template <typename T, int D>
struct QVec {
    typedef typename Frag<T>::x4 type;
};
template <typename T>
struct QVec<T, 32> {
    typedef typename Frag<T>::x8 type;
};

template <typename T, int NT, int D>
struct Stage<T, NT, true, D> {
    static_assert(D == 16 || (D == 32 && sizeof(T) == 2), "head dim 32: 2-byte types");
    static constexpr int NP = NT * 16;
    static constexpr int kQRows = 16 * kWaves;
    static constexpr bool kDma = v_row_major<T>();
    static constexpr int kKC = (NP + 63) / 64;          // register path: rows per thread
    static constexpr int kRows = kDma ? (NP + 31) / 32 * 32 : kKC * 64;
    // DMA path: per round a wave loads 32 K rows and 32 V rows (head dim
    // 16), or 16 of each (head dim 32): 1 KB each
    static constexpr int kRounds = D == 16 ? (kRows + 127) / 128 : (kRows + 63) / 64;
    static constexpr int kVtStride = kRows + 4;
    static constexpr int kVLds = v_row_major<T>() ? kRows * D : 16 * kVtStride;
    typedef typename Frag<T>::x4 X4;
    // a thread's Q elements: 4 dims (head dim 16) or 8 (head dim 32)
    typedef typename QVec<T, D>::type QV;

    QV rq;
    X4 rk[kDma ? 1 : kKC], rv[kDma ? 1 : kKC];

    template <typename V = X4>
    static __device__ __forceinline__ V ld(__amdgpu_buffer_rsrc_t rs, int off) {
        if constexpr (sizeof(V) == 8)
            return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0));
        else
            return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }

    static __device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t off,
                                                                 int64_t s2, int N) {
        char* ub = uniform_ptr(static_cast<const char*>(base) + off * int64_t(sizeof(T)));
        const int extent = __builtin_amdgcn_readfirstlane(
            static_cast<int>((int64_t(N - 1) * s2 + D) * int64_t(sizeof(T))));
        return __builtin_amdgcn_make_buffer_rsrc(ub, 0, extent, 0x00020000);
    }

    __device__ __forceinline__ void load(const Params& p, int b, int h, int q0, T* k_dst, T* v_dst) {
        static_assert(D == 16, "head dim 32 stages through load_q and the DMA rounds");
        const int N = p.N;
        const int tid = threadIdx.x & (kThreads - 1);  // within the head slot
        const int n0 = tid >> 2;
        const int d0 = (tid & 3) * 4;
        const auto qr = rsrc(p.q, int64_t(b) * p.qs[0] + int64_t(h) * p.qs[1], p.qs[2], N);
        const auto kr = rsrc(p.k, int64_t(b) * p.ks[0] + int64_t(h) * p.ks[1], p.ks[2], N);
        const auto vr = rsrc(p.v, int64_t(b) * p.vs[0] + int64_t(h) * p.vs[1], p.vs[2], N);
        const int qs2 = static_cast<int>(p.qs[2]), ks2 = static_cast<int>(p.ks[2]),
                  vs2 = static_cast<int>(p.vs[2]);
        constexpr int es = sizeof(T);
        const int nq = min(q0 + n0, N - 1);
        rq = ld(qr, (nq * qs2 + d0) * es);
        if constexpr (kDma) {
#pragma unroll
            for (int r = 0; r < kRounds; ++r) dma_round<false>(p, window_desc<false>(p, b, h, h), k_dst, v_dst, r, 0);
        } else {
#pragma unroll
            for (int k = 0; k < kKC; ++k) {
                const int n = min(n0 + 64 * k, N - 1);
                rk[k] = ld(kr, (n * ks2 + d0) * es);
                rv[k] = ld(vr, (n * vs2 + d0) * es);
            }
        }
    }

    // The Q rows of head h for the next window (the register half of load()).
    __device__ __forceinline__ void load_q(const Params& p, int b, int h, int q0) {
        const int N = p.N;
        const int tid = threadIdx.x & (kThreads - 1);
        const int n0 = tid >> 2, d0 = (tid & 3) * (D / 4);
        constexpr int es = sizeof(T);
        const auto qr = rsrc(p.q, int64_t(b) * p.qs[0] + int64_t(h) * p.qs[1], p.qs[2], N);
        rq = ld<QV>(qr, (min(q0 + n0, N - 1) * static_cast<int>(p.qs[2]) + d0) * es);
    }

    // LDS-DMA rounds per wave for one window's K and V: kRounds with one
    // head per workgroup, one record load per round with kHeadsPerWg heads.
    // Head dim 32: kStageWaves waves share a window's key tiles (kWaves, or
    // all the waves of a workgroup of several strip groups).
    template <bool kRecs, int kStageWaves = kWaves>
    static constexpr int dma_rounds() {
        constexpr int kAllWaves = kWaves * kHeadsPerWg;
        if constexpr (kRecs) return (rec_loads(NT) + kAllWaves - 1) / kAllWaves;
        if constexpr (D == 32) return (kRows / 16 + kStageWaves - 1) / kStageWaves;
        return kRounds;
    }

    // Round r of this wave's LDS-DMA loads of window b's K and V.  16 bytes
    // per lane go straight into LDS at a wave-uniform address, lane l
    // writing 16-byte chunk l of the load's 1 KB; which bytes each lane
    // fetches sets the layout.
    //  - One head (h): round r of wave w fills rows 32*(4r + w) .. +31, K in
    //    the kidx tile layout, V as plain 32-byte rows (its transpose reads
    //    are conflict-free); row u holds key u.
    //  - kHeadsPerWg heads (h0 ..): token records (kRecStride elements),
    //    load j = wave + 4 * kHeadsPerWg * r of the workgroup's loads fills
    //    chunks 64j .. 64j + 63: chunk c is token c / 13, piece c % 13 (pieces
    //    0-5: the heads' K row bytes 16p .. 16p + 15, pieces 6-11 the same of
    //    V, which lies p.kv_delta elements after K; piece 12 pads the record
    //    and reloads piece 0).  The last load may run past the last record
    //    into the buffer's padding.
    // Buffer descriptors of one window's K and V rows (records: K and V
    // from K's base, V kv_delta elements after K), built once per window.
    struct WindowDesc {
        u32x4 k, v;
    };
    template <bool kRecs>
    static __device__ __forceinline__ WindowDesc window_desc(const Params& p, int b, int h, int h0) {
        const int N = p.N;
        if constexpr (!kRecs) {
            return {desc_words<T>(p.k, int64_t(b) * p.ks[0] + int64_t(h) * p.ks[1], p.ks[2], N, D),
                    desc_words<T>(p.v, int64_t(b) * p.vs[0] + int64_t(h) * p.vs[1], p.vs[2], N, D)};
        } else {
            const u32x4 d = desc_words<T>(p.k, int64_t(b) * p.ks[0] + int64_t(h0) * p.ks[1], p.ks[2], N,
                                          p.kv_delta + 16 * kHeadsPerWg);
            return {d, d};
        }
    }
    // Records: the lane's byte offset of round r's load, the same for every
    // window (it depends on the wave, the round and the lane only).
    static __device__ __forceinline__ int rec_voff(const Params& p, int r) {
        const int N = p.N;
        const int lane = threadIdx.x & 63;
        const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
        const int j = min(wave + kWaves * kHeadsPerWg * r, rec_loads(NT) - 1);  // (unused past the last)
        const int c = 64 * j + lane;
        const int n = c / 13;  // record n holds token n
        const int piece = c - 13 * n;
        const int part = piece < 6 ? 8 * piece : (piece < 12 ? p.kv_delta + 8 * (piece - 6) : 0);
        return (min(n, N - 1) * static_cast<int>(p.ks[2]) + part) * static_cast<int>(sizeof(T));
    }

    template <bool kRecs, int kStageWaves = kWaves>
    static __device__ __forceinline__ void dma_round(const Params& p, const WindowDesc& wd, T* k_dst, T* v_dst,
                                                     int r, int voff) {
        static_assert(kDma, "LDS-DMA staging");
        static_assert(kStageWaves == kWaves || D == 32, "shared staging: head dim 32");
        const int N = p.N;
        constexpr int es = sizeof(T);
        const int lane = threadIdx.x & 63;
        typedef __attribute__((address_space(3))) T LdsT;
        const uint32_t kl = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((LdsT*)k_dst));
        if constexpr (!kRecs && D == 32) {
            // round r of wave w (of the kStageWaves waves of the workgroup)
            // fills key tile kStageWaves * r + w: K as 4 blocks of 8 dims
            // (lane l: block l/16, row l%16), V as 16 plain 64-byte rows
            // (lane l: row l/4, dims 8*(l%4) ..)
            (void)voff;
            const uint32_t vl = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((LdsT*)v_dst));
            const int ks2 = static_cast<int>(p.ks[2]), vs2 = static_cast<int>(p.vs[2]);
            const int wave = __builtin_amdgcn_readfirstlane(
                kStageWaves == kWaves ? (threadIdx.x >> 6) & (kWaves - 1) : static_cast<int>(threadIdx.x >> 6));
            const int row0 = 16 * (kStageWaves * r + wave);
            if (row0 < kRows) {  // wave-uniform
                const int nk = min(row0 + (lane & 15), N - 1);
                dma16(wd.k, kl + row0 * 64, (nk * ks2 + 8 * (lane >> 4)) * es);
                const int nv = min(row0 + (lane >> 2), N - 1);
                dma16(wd.v, vl + row0 * 64, (nv * vs2 + 8 * (lane & 3)) * es);
            }
        } else if constexpr (!kRecs) {
            (void)voff;
            const uint32_t vl = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((LdsT*)v_dst));
            const int ks2 = static_cast<int>(p.ks[2]), vs2 = static_cast<int>(p.vs[2]);
            const int wave = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) & (kWaves - 1));
            const int row0 = 32 * (4 * r + wave);
            if (row0 < kRows) {  // wave-uniform
                // K: chunk l of these two tiles is (tile l/32, dims 8*((l/16)&1), row l&15)
                const int nk = min(row0 + ((lane >> 5) << 4) + (lane & 15), N - 1);
                const int hk = ((lane >> 4) & 1) * 8;
                dma16(wd.k, kl + row0 * 32, (nk * ks2 + hk) * es);
                const int nv = min(row0 + (lane >> 1), N - 1);
                dma16(wd.v, vl + row0 * 32, (nv * vs2 + (lane & 1) * 8) * es);
            }
        } else {
            static_assert(kRows == rec_rows(NT), "record rows");
            (void)v_dst;
            const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
            const int j = wave + kWaves * kHeadsPerWg * r;  // wave-uniform
            if (j < rec_loads(NT)) dma16(wd.k, kl + j * 1024, voff);
        }
    }

    __device__ __forceinline__ void store(float scale, T* q_lds, T* k_lds, T* vt_lds) const {
        const int tid = threadIdx.x & (kThreads - 1);  // within the head slot
        const int n0 = tid >> 2;
        if constexpr (D == 32)
            store_q8<T>(&q_lds[n0 * 64], (tid & 3) * 8, rq, scale);
        else
            store_q4<T>(&q_lds[n0 * q_row_len<T, 16>()], (tid & 3) * 4, rq, scale);
        if constexpr (!kDma) {
            const int d0 = (tid & 3) * 4;
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
// caller's bias tensor: lane (col, g) holds keys 16t + 4g + r of query
// qi.  The head's [N, N] bias is read through a buffer
// descriptor; keys past N read 0 or the next row and are replaced by -inf
// (probability exactly 0).  Padded query rows repeat row N - 1.  In
// region mode a key whose shift-region class differs from the query's on
// an axis that the window type `code` splits gets -100.  kLog2: the tiles
// are kept in log2 units (multiplied by log2(e)) plus the query's row offset
// `off`, for the offset softmax of the 2-byte types (attend_offset).  Runs
// when the window type changes (at most 8 times per workgroup) or the
// offsets move, never per window otherwise.
//
// A lane's 4 keys of a tile are consecutive in its bias row, so each tile
// is one load, and all of a wave's loads are issued before any is used (one
// memory round trip per build).  16-bit rows of an odd row stride start in the middle of
// a dword and unaligned loads are slow, so those lanes load the dwords
// around their keys from a dword-aligned offset and shift the halves into
// place (shift: 0 or 16 bits).  The resource is dword-aligned
// (aligned_rsrc).  (Bias rows never overlap: the host checks that the row
// stride is at least N.)
template <int NT, int kMask, bool kLog2, int kBiasDtype>
__device__ __forceinline__ void build_tiles_es(f32x4 (&bs)[NT], __amdgpu_buffer_rsrc_t rs, int lead, int N,
                                               int64_t bsd1, int qi, int g, int code, const uint8_t* cls,
                                               float off) {
    constexpr int kEs = kBiasDtype == CRUMPET_DTYPE_F32 ? 4 : 2;
    // Opaque copies of the lane's position and N: what the build derives from
    // them (per-key validity, offsets) is then computed here, each time,
    // instead of being hoisted out of the window loop and held in registers
    // that the attention loop needs.
    asm volatile("" : "+v"(qi), "+v"(g), "+s"(N));
    // Padded query rows (qi >= N) build row N - 1's tiles: their Q is row
    // N - 1's as well (the Q loads clamp the row), so they repeat that row's
    // scores; they are never stored and never enter the row-sum check.
    const int qr = qi < N ? qi : N - 1;
    const int rb = lead + static_cast<int>(int64_t(qr) * bsd1) * kEs;  // byte offset of the row
    const int shift = (rb & 2) * 8;                                     // 16-bit rows: 0 or 16
    const int rowb = rb & ~3;                                           // dword-aligned
    uint32_t cq = 0, cmask = 0;
    if constexpr (kMask == kMaskRegion) {
        cq = uint32_t(cls[qr]) * 0x01010101u;  // query class in every byte
        cmask = uint32_t(code) * 0x01010101u;
    }
    // a region-masked key adds -100 to its bias: in log2 units (kLog2) the
    // mask joins the row offset, so an unmasked key's value is exactly
    // bias * log2(e) + off
    constexpr float kMaskAdd = kLog2 ? -100.0f * kLog2e : -100.0f;
    // words per tile: 4 fp32 keys, or the 3 dwords around 4 16-bit keys
    constexpr int kWords = kEs == 4 ? 4 : 3;
    // Two halves of the tiles, each: all loads, then the conversions (the
    // raw words of every tile at once would not fit next to the tiles).
    constexpr int kHalf = (NT + 1) / 2;
#pragma unroll
    for (int u0 = 0; u0 < NT; u0 += kHalf) {
        __builtin_amdgcn_sched_barrier(0);
        uint32_t raw[kHalf][kWords];
#pragma unroll
        for (int u = 0; u < kHalf; ++u) {
            const int t = u0 + u;
            if (t >= NT) break;
            const int o = rowb + (16 * t + 4 * g) * kEs;
            if constexpr (kEs == 4) {
                const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) raw[u][i] = w[i];
            } else {
                const u32x3 w = __builtin_amdgcn_raw_buffer_load_b96(rs, o, 0, 0);
#pragma unroll
                for (int i = 0; i < 3; ++i) raw[u][i] = w[i];
            }
        }
#pragma unroll
        for (int u = 0; u < kHalf; ++u) {
            const int t = u0 + u;
            if (t >= NT) break;
            // one tile at a time: scheduled together, the per-key lane
            // masks of all tiles would not fit the scalar registers
            __builtin_amdgcn_sched_barrier(0);
            const int k4 = 16 * t + 4 * g;  // the tile's 4 keys
            uint32_t split = 0;  // byte r nonzero (0..7): key k4 + r is masked by the region rule
            if constexpr (kMask == kMaskRegion)
                split = (*reinterpret_cast<const uint32_t*>(&cls[k4]) ^ cq) & cmask;
            float v4[4];
            if constexpr (kEs == 4) {
#pragma unroll
                for (int r = 0; r < 4; ++r) v4[r] = __uint_as_float(raw[u][r]);
            } else {
                const uint32_t hw[2] = {__builtin_amdgcn_alignbit(raw[u][1], raw[u][0], shift),
                                        __builtin_amdgcn_alignbit(raw[u][2], raw[u][1], shift)};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t bits = (r & 1) ? hw[r >> 1] >> 16 : hw[r >> 1] & 0xffffu;
                    if constexpr (kBiasDtype == CRUMPET_DTYPE_BF16)
                        v4[r] = __uint_as_float(bits << 16);
                    else
                        v4[r] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float add = kLog2 ? off : 0.0f;
                if constexpr (kMask == kMaskRegion) {
                    // 1.0 if byte r of split is nonzero, else 0.0 (byte to
                    // float, clamped to [0, 1]: one instruction)
                    const float masked = __builtin_amdgcn_fmed3f(
                        static_cast<float>((split >> (8 * r)) & 0xffu), 0.0f, 1.0f);
                    add = __builtin_fmaf(masked, kMaskAdd, add);
                }
                bs[t][r] = kLog2 ? __builtin_fmaf(v4[r], kLog2e, add) : v4[r] + add;
            }
            // keys past N (only in the tile that holds key N - 1 and after
            // it): probability exactly 0
            if (16 * t + 16 > N) {
#pragma unroll
                for (int r = 0; r < 4; ++r) bs[t][r] = (k4 + r) < N ? bs[t][r] : -INFINITY;
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
}

// Region mode, tiles in log2 units: tiles built for window type `from` made
// those of type `to` without reading the bias again.  A key masked under one
// type and not the other gains or loses the mask's -100 * log2(e); keys past
// N stay -inf.  The sum is rounded once more than a fresh build's (a few
// ulps of 144, about 1e-5 in log2 units, i.e. 1e-5 relative in the key's
// probability) and a workgroup changes type at most 7 times.  Costs no
// memory round trip: a fresh build waits on a scattered gather of the bias
// rows (16 rows per load instruction), about 5 us per build at config 3.
template <int NT>
__device__ __forceinline__ void retype_tiles(f32x4 (&bs)[NT], int qi, int g, int N, int from, int to,
                                             const uint8_t* cls) {
    // opaque copies of the lane's position: the per-tile class addresses are
    // then computed here, not hoisted out of the window loop into registers
    asm volatile("" : "+v"(qi), "+v"(g));
    const int qr = qi < N ? qi : N - 1;
    const uint32_t cq = uint32_t(cls[qr]) * 0x01010101u;  // query class in every byte
    const uint32_t mf = uint32_t(from) * 0x01010101u, mt = uint32_t(to) * 0x01010101u;
    constexpr float kMaskAdd = -100.0f * kLog2e;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const uint32_t x = *reinterpret_cast<const uint32_t*>(&cls[16 * t + 4 * g]) ^ cq;
        const uint32_t sf = x & mf, st = x & mt;  // byte r nonzero: key masked under from / to
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float was = __builtin_amdgcn_fmed3f(static_cast<float>((sf >> (8 * r)) & 0xffu), 0.0f, 1.0f);
            const float now = __builtin_amdgcn_fmed3f(static_cast<float>((st >> (8 * r)) & 0xffu), 0.0f, 1.0f);
            bs[t][r] = __builtin_fmaf(now - was, kMaskAdd, bs[t][r]);
        }
    }
}

template <int NT, int kMask, bool kLog2>
__device__ __forceinline__ void build_tiles(f32x4 (&bs)[NT], const Params& prm, int h, int qi, int g,
                                            int code, const uint8_t* cls, float off) {
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
    const int es = bias_dtype == CRUMPET_DTYPE_F32 ? 4 : 2;
    // base and extent are workgroup-uniform; readfirstlane keeps the
    // descriptor in SGPRs (a VGPR descriptor costs a waterfall loop per load)
    const AlignedRsrc ar = aligned_rsrc(static_cast<const char*>(bias_ptr) + int64_t(h) * bsd0 * es,
                                        (int64_t(N - 1) * bsd1 + N) * es);
    // uniform: one dtype branch per build, none per tile or element
    if (bias_dtype == CRUMPET_DTYPE_F32)
        build_tiles_es<NT, kMask, kLog2, CRUMPET_DTYPE_F32>(bs, ar.rs, ar.lead, N, bsd1, qi, g, code, cls, off);
    else if (bias_dtype == CRUMPET_DTYPE_BF16)
        build_tiles_es<NT, kMask, kLog2, CRUMPET_DTYPE_BF16>(bs, ar.rs, ar.lead, N, bsd1, qi, g, code, cls, off);
    else
        build_tiles_es<NT, kMask, kLog2, CRUMPET_DTYPE_F16>(bs, ar.rs, ar.lead, N, bsd1, qi, g, code, cls, off);
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

// ---------------------------------------------------------------------------
// Offset softmax (2-byte types)
//
// Scores come out of the score product in log2 units, so that P = 2^S needs
// no multiply-add: the bias (+ region mask) tiles are kept multiplied by
// log2(e), and Q by scale * log2(e).  Q enters the 16x16x32 product as
// hi + lo (store_q4): its k-slices 8s .. 8s + 7 carry K . Q_hi (s even) and
// K . Q_lo (s odd) over dims 8(s >> 1) .. + 7, K repeated, so the folded
// log2(e) adds no rounding beyond fp32.
//
// No row max is taken.  The bias tiles carry a per-query offset instead
// (build_tiles), and softmax is invariant to it, so the offset only has to
// keep P inside the range where rounding to the input type costs no more
// than with the exact max: every P finite (in fp16 a P either rounds to at
// most 65504 or overflows to inf, and the row sum is the fp32 sum of the
// rounded P, so a finite row sum means finite P), a row sum of at most
// kRowSumMax = 2^64 (bf16 P can be finite far above that; the bound keeps
// the fp32 numerator P V finite for |v| below 2^64, and an fp16 row sum
// never reaches it) and of at least kRowSumMin = 2^-3 (with at most 512
// keys the largest P is then at least 2^-12, a normal fp16 number, and a P
// that is subnormal carries less than 2^-21 of the row's weight in rounding
// error).  The row sums come out of the same pass (ones^T P^T), so the check
// is exact: when a strip's row sums miss [2^-3, 2^64] (a bad first guess,
// or scores that moved from earlier windows), the wave redoes the strip
// with the exact row max subtracted in the fp32 accumulator, as the
// reference does, and moves its offsets so that a window like this one
// would have row sums near 2^kOffsetTarget; the caller rebuilds the wave's
// bias tiles with them before its next window (the tiles stay read-only
// here, which keeps them in registers).  In fp16 the range spans about
// 2^-3 .. 2^16 for the largest P, 9-10 octaves either side of the target,
// so a window whose scores jump from its predecessors' (a dominant
// diagonal, say) rarely costs the exact pass.
//
// Per score this leaves one exp and half a conversion on the VALU; with no
// max reduction between the score tiles, pair p+1's score MFMAs are issued
// next to pair p's exps, and K, V and mask fragments are requested one or
// two pairs ahead.
constexpr float kOffsetTarget = 7.0f;  // log2 of the row sum aimed at
constexpr float kRowSumMin = 0.125f;   // row sums outside [kRowSumMin, kRowSumMax] take
constexpr float kRowSumMax = 0x1p64f;  // the exact pass (NaN too)

// LDS-DMA rounds per wave with token records (1 otherwise: an array size).
template <typename St, bool kRecs>
constexpr int kRecRounds() {
    if constexpr (kRecs)
        return St::template dma_rounds<true>();
    else
        return 1;
}

// The next window's LDS-DMA rounds, issued from inside a window's compute:
// attend_offset spreads them over its tile pairs, so that a workgroup's
// loads reach the memory pipeline a few at a time while it computes instead
// of all at the window start (where every wave would stall on issue).
template <typename T, typename St, bool kRecs, int kStageWaves = kWaves>
struct DmaIssuer {
    static constexpr int kRounds = St::template dma_rounds<kRecs, kStageWaves>();
    const Params* p;
    typename St::WindowDesc wd;  // the next window's descriptors
    T* k_dst;
    T* v_dst;
    const int* voff;  // records: the lane's offset per round
    bool on;          // a next window exists (wave-uniform)
    __device__ __forceinline__ void operator()(int r) const {
        if (on) St::template dma_round<kRecs, kStageWaves>(*p, wd, k_dst, v_dst, r, kRecs ? voff[r] : 0);
    }
};
struct NoIssue {
    static constexpr int kRounds = 0;
    __device__ __forceinline__ void operator()(int) const {}
};

// One strip's normalised output, held back for a deferred store (vector IO,
// head dim 16): a wave writes window i's output after the wait on window
// i + 1's rows that ends window i.  The vector-memory counter retires stores
// with the loads, so a store issued before that wait would be waited for by
// it; issued after it, the store completes during window i + 1.
template <typename T>
struct PendingOut {
    typename Frag<T>::x4 r;  // O[qi][4g .. 4g + 3]
};

template <typename T>
__device__ __forceinline__ void store_out4(const Params& p, const typename Frag<T>::x4& r, int b, int h, int qi,
                                           int g) {
    // scalar base of the (window, head) block and a 32-bit lane offset
    char* ub = uniform_ptr(static_cast<char*>(p.out) + (int64_t(b) * p.os[0] + int64_t(h) * p.os[1]) *
                                                           int64_t(sizeof(T)));
    const int extent = __builtin_amdgcn_readfirstlane(
        static_cast<int>((int64_t(p.N - 1) * p.os[2] + 16) * int64_t(sizeof(T))));
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(ub, 0, extent, 0x00020000);
    if (qi < p.N)
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, r), rs,
                                              (qi * static_cast<int>(p.os[2]) + 4 * g) * static_cast<int>(sizeof(T)),
                                              0, 0);
}

// Head dim 16, LDS-DMA path: a wave's Q operand never passes through LDS.
// Lane (col, g) loads the 8 raw elements of dims 8(g >> 1) .. + 7 of its
// query row (clamped to N - 1; padded rows are never stored) from the
// window's Q rows, and q_operand turns them into the k-slice g of the score
// product: hi = q * scale rounded for even g, the remainder lo for odd g
// (store_q4 makes the same split).
template <typename T>
struct QRaw {
    u32x2 w[2];  // 8 elements of T
};

template <typename T>
__device__ __forceinline__ QRaw<T> load_qraw(const Params& p, int b, int h, int qi, int g) {
    const int N = p.N;
    char* ub = uniform_ptr(static_cast<const char*>(p.q) + (int64_t(b) * p.qs[0] + int64_t(h) * p.qs[1]) *
                                                            int64_t(sizeof(T)));
    const int extent = __builtin_amdgcn_readfirstlane(
        static_cast<int>((int64_t(N - 1) * p.qs[2] + 16) * int64_t(sizeof(T))));
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(ub, 0, extent, 0x00020000);
    const int off = (min(qi, N - 1) * static_cast<int>(p.qs[2]) + 8 * (g >> 1)) * static_cast<int>(sizeof(T));
    QRaw<T> r;
    r.w[0] = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
    r.w[1] = __builtin_amdgcn_raw_buffer_load_b64(rs, off + 8, 0, 0);
    return r;
}

template <typename T>
__device__ __forceinline__ typename Frag<T>::x8 q_operand(const QRaw<T>& raw, float scale, int g) {
    typedef typename Frag<T>::x4 X4;
    const X4 a = __builtin_bit_cast(X4, raw.w[0]);
    const X4 c = __builtin_bit_cast(X4, raw.w[1]);
    const bool lo = g & 1;
    typename Frag<T>::x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float x = static_cast<float>(e < 4 ? a[e] : c[e - 4]) * scale;
        const T hi = T(x);
        r[e] = lo ? T(x - static_cast<float>(hi)) : hi;
    }
    return r;
}

// Wave priority by progress through a window's tile pairs: 3 in the first
// quarter of the pairs down to 0 in the last.  The arbiter otherwise issues
// for the oldest wave of a SIMD first, so the three waves of a SIMD finished
// a window up to a third of its compute apart, and the youngest ran its last
// pairs alone, with its dependency stalls exposed; ranking by progress keeps
// the three in step (config 3 shifted: 119 -> 113 us).
__device__ __forceinline__ void set_wave_prio(int level) {
    switch (level) {  // the builtin takes a constant; level is one after unrolling
        case 0: __builtin_amdgcn_s_setprio(0); break;
        case 1: __builtin_amdgcn_s_setprio(1); break;
        case 2: __builtin_amdgcn_s_setprio(2); break;
        default: __builtin_amdgcn_s_setprio(3); break;
    }
}

template <typename T, int NT, int kMask, bool kUseMask, bool kVec, bool kRec, int D, bool kDefer, typename Issue>
__device__ __forceinline__ bool attend_offset(const Params& p, const f32x4 (&bs)[NT], const typename Frag<T>::x8& qf,
                                              const typename Frag<T>::x8& qf_lo, const T* __restrict__ k_lds,
                                              const T* __restrict__ v_lds, int b, int h, int qi, int col, int g,
                                              float& off, const Issue& issue, PendingOut<T>& pend) {
    static_assert(!kDefer || (kVec && D == 16), "deferred stores: vector IO, head dim 16");
    typedef typename Frag<T>::x4 X4;
    typedef typename Frag<T>::x8 X8;
    constexpr int kMaskBytes = (kMask == kMaskF32) ? 4 : 2;
    constexpr int kPairs = (NT + 1) / 2;
    const int N = p.N;

    static_assert(D == 16 || !kRec, "head dim 32: one head per workgroup");
    // Q^T operand of S^T = K Q^T (16x16x32): lane (col, g) holds elements
    // 8g..8g+7 of the k-slices of query col, i.e. Q_hi (g even) or Q_lo
    // (g odd) of dims 8(g >> 1) .. + 7 (head dim 16, store_q4, q_operand);
    // head dim 32: Q_hi dims 8g..8g+7 (qf) and Q_lo dims 8g..8g+7 (qf_lo),
    // two products per score tile.
    // S^T of one tile from its K fragment and accumulator input
    auto score = [&](const X8& kfr, const f32x4& c) -> f32x4 {
        const f32x4 s = Frag<T>::mma32(kfr, qf, c);
        if constexpr (D == 32)
            return Frag<T>::mma32(kfr, qf_lo, s);
        else
            return s;
    };

    // K operand: lane (col, g) reads row col of the tile, dims 8(g>>1)..+7
    // (head dim 16; kRec: k_lds and v_lds point at this head's row in the
    // first record) or dims 8g..+7 (head dim 32).  At head dim 16 lanes
    // 0-31 read the first 16 bytes of the 16 rows and lanes 32-63 the
    // second: a 16-byte LDS read serves lanes 0-31 in one pass, and with
    // lanes 16-31 on the second half of the same rows (dims 8(g&1)) the
    // 208-byte records had put two lanes on one bank (measured: 8.3 against
    // 4.5 cycles per read).
    constexpr int kKTile = kRec ? 16 * kKRec : 16 * D;  // elements from one K tile to the next
    constexpr int kVTile = kRec ? 16 * kVRec : 16 * D;
    const T* kbase = kRec ? k_lds + col * kKRec + (g >> 1) * 8
                          : k_lds + (D == 32 ? g : (g >> 1)) * 128 + col * 8;
    auto kfrag = [&](int t) -> X8 { return *reinterpret_cast<const X8*>(kbase + t * kKTile); };
    // V^T fragments by transpose reads of row-major V (lds_read_tr); head
    // dim 32 reads dims 16..31 at vrow + 16 for the second half of O
    const T* vrow = &v_lds[(4 * g + (col >> 2)) * (kRec ? kVRec : D) + (col & 3) * 4];

    // Tensor mask through a buffer descriptor spanning exactly the window's
    // [N, N] extent (see attend_f32 for the padding and end-of-extent rules).
    __amdgpu_buffer_rsrc_t mrsrc;
    int mvoff = 0;
    if constexpr (kUseMask && mask_tiled(kMask)) {
        // tiled layout (NT even): window m's block holds strips x NT/2 tile
        // pairs x 64 lanes x 2 tiles x 4 keys; lane (col, g) of strip s reads
        // its 4 keys of tiles 2p and 2p + 1 as 16 bytes at
        // ((s * NT/2 + p) * 64 + 16 g + col) * 16, a wave's pair being 1 KB
        // contiguous (p.ms[0]: elements per window block)
        static_assert(NT % 2 == 0, "tiled masks: an even tile count");
        const AlignedRsrc ar =
            aligned_rsrc(static_cast<const char*>(p.mask) + int64_t(b % p.mask_batch) * p.ms[0] * 2,
                         int64_t(p.strips) * NT * 512);
        mrsrc = ar.rs;
        mvoff = ar.lead + (((qi >> 4) * (NT / 2) * 64) + 16 * g + col) * 16;
    } else if constexpr (kUseMask) {
        const int qr = qi < N ? qi : N - 1;
        const AlignedRsrc ar =
            aligned_rsrc(static_cast<const char*>(p.mask) + int64_t(b % p.mask_batch) * p.ms[0] * kMaskBytes,
                         int64_t((N - 1) * p.ms[1] + N) * kMaskBytes);
        mrsrc = ar.rs;
        mvoff = ar.lead + static_cast<int>(qr * p.ms[1] * kMaskBytes);
    }
    // Mask values by tile, a lane's 4 keys of a tile consecutive in its row.
    // 2-byte masks: a row of an odd row stride starts in the middle of a
    // dword, and unaligned loads are slow.  Each lane therefore loads the
    // dwords around its keys from a dword-aligned offset (mvoff is the row's,
    // in a dword-aligned resource: aligned_rsrc) and shifts its halves into
    // place when it uses them (mshift: 0 or 16 bits).  Words per tile: 2-byte
    // 3, fp32 4.
    int mshift = 0;
    if constexpr (kUseMask && kMaskBytes == 2 && !mask_tiled(kMask)) {
        mshift = (mvoff & 2) * 8;
        mvoff &= ~3;
    }
    constexpr int kMWords = mask_tiled(kMask) ? 2 : (kMaskBytes == 2 ? 3 : 4);
    typedef uint32_t MaskWords[kMWords];
    // the words of tile t
    auto fetch = [&](int t, MaskWords& w) {
        if constexpr (kUseMask && mask_tiled(kMask)) {
            // the 4 keys in place (shift 0): hw[0] = w[0], hw[1] = w[1]
            const u32x2 v2 = __builtin_amdgcn_raw_buffer_load_b64(mrsrc, mvoff + (t >> 1) * 1024 + (t & 1) * 8, 0, 0);
            w[0] = v2[0];
            w[1] = v2[1];
        } else if constexpr (kUseMask) {
            const int o = mvoff + (16 * t + 4 * g) * kMaskBytes;
            if constexpr (kMaskBytes == 2) {
                const u32x3 v3 = __builtin_amdgcn_raw_buffer_load_b96(mrsrc, o, 0, 0);
#pragma unroll
                for (int r = 0; r < 3; ++r) w[r] = v3[r];
            } else {
                const u32x4 v4 = __builtin_amdgcn_raw_buffer_load_b128(mrsrc, o, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) w[r] = v4[r];
            }
        }
    };
    // tiled masks: the words of the tile pair (t, t + 1), t even, in one load
    auto fetch_pair = [&](int t, MaskWords& w0, MaskWords& w1) {
        if constexpr (kUseMask && mask_tiled(kMask)) {
            const u32x4 v4 = __builtin_amdgcn_raw_buffer_load_b128(mrsrc, mvoff + (t >> 1) * 1024, 0, 0);
            w0[0] = v4[0];
            w0[1] = v4[1];
            w1[0] = v4[2];
            w1[1] = v4[3];
        }
    };
    // accumulator input of tile t: bias (+ region mask) tile with the row
    // offset, plus the mask tensor's values in log2 units (w: tile t's words)
    auto cinit = [&](int t, const MaskWords& w) -> f32x4 {
        f32x4 c = bs[t];
        if constexpr (kUseMask) {
            uint32_t hw[2] = {0u, 0u};  // 2-byte masks: the 4 keys' halves in place
            if constexpr (mask_tiled(kMask)) {
                hw[0] = w[0];
                hw[1] = w[1];
            } else if constexpr (kMaskBytes == 2) {
                hw[0] = __builtin_amdgcn_alignbit(w[1], w[0], mshift);
                hw[1] = __builtin_amdgcn_alignbit(w[2], w[1], mshift);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float mv;
                if constexpr (kMask == kMaskF32)
                    mv = __uint_as_float(w[r]);
                else if constexpr (mask_f16(kMask))
                    mv = static_cast<float>(
                        __builtin_bit_cast(_Float16, static_cast<uint16_t>(r & 1 ? hw[r >> 1] >> 16 : hw[r >> 1])));
                else
                    mv = __uint_as_float(r & 1 ? (hw[r >> 1] & 0xffff0000u) : (hw[r >> 1] << 16));
                c[r] = __builtin_fmaf(mv, kLog2e, c[r]);
            }
        }
        return c;
    };

    X8 ones8;
#pragma unroll
    for (int r = 0; r < 8; ++r) ones8[r] = T(1.0f);
    // opaque: kept in registers for the window instead of rebuilt by moves
    // before every row-sum product
    asm volatile("" : "+v"(ones8));

    // P of the pair of tiles (t, t + 1), rounded to T: B operand of the
    // product below
    auto probs = [&](const f32x4& s0, const f32x4& s1, bool has1) -> X8 {
        X8 pb;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            pb[r] = T(__builtin_amdgcn_exp2f(s0[r]));
            pb[r + 4] = has1 ? T(__builtin_amdgcn_exp2f(s1[r])) : T(0.0f);
        }
        return pb;
    };
    // O^T += V^T P^T and the row sums (ones^T P^T) for the pair
    auto accumulate = [&](const X8& pb, const X4& v0, const X4& v1, bool has1, f32x4& o, f32x4& lacc) {
        X8 va;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            va[r] = v0[r];
            va[r + 4] = has1 ? v1[r] : T(0.0f);
        }
        o = Frag<T>::mma32(va, pb, o);
        lacc = Frag<T>::mma32(ones8, pb, lacc);
    };
    // head dim 32: O^T rows 16..31 += V^T (dims 16..31) P^T
    auto accumulate_hi = [&](const X8& pb, const X4& v0, const X4& v1, bool has1, f32x4& o) {
        X8 va;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            va[r] = v0[r];
            va[r + 4] = has1 ? v1[r] : T(0.0f);
        }
        o = Frag<T>::mma32(va, pb, o);
    };

    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 o2 = {0.0f, 0.0f, 0.0f, 0.0f};  // head dim 32: dims 16..31
    f32x4 lacc = {0.0f, 0.0f, 0.0f, 0.0f};
    {
        // Software pipeline over tile pairs.  Iteration pr requests the V
        // fragments of pair pr, the K fragments of pair pr + kKAhead and the
        // mask words of pair pr + kMaskAhead, issues the score MFMAs of pair
        // pr+1, and exponentiates pair pr and multiplies it into O (its V
        // reads are covered by the exps).  K is requested two pairs ahead
        // and pair pr+1's score MFMAs run during pair pr's exps, except with
        // a mask tensor at 3 waves per SIMD: there the mask words and the
        // accumulator inputs take the registers of the second K pair, so K
        // is requested one pair ahead and the score MFMAs follow the exps
        // that cover its LDS latency.  All indices are compile-time
        // constants, so the arrays live in registers.
        // register budget above 168 left after the bias tiles (not at 32 tiles)
        constexpr bool kWide = waves_per_eu<T, NT, kMask, kVec>() < 3 && NT <= 22;
        constexpr int kKAhead = (kUseMask && !kWide) ? 1 : 2;
        // the tiled mask copy (2 words per tile) at head dim 16, one head per
        // workgroup: two pairs ahead fits the registers (168) and hides more
        // of the loads (config 3: 153-154 -> 147-150 us)
        constexpr int kMaskAhead = (kWide || (mask_tiled(kMask) && !kRec && D == 16)) ? 2 : 1;  // pairs
        X8 kf[NT];
        f32x4 S[NT];
        MaskWords mw[kUseMask ? NT : 1];
#pragma unroll
        for (int t = 0; t < NT && t < 2 * kKAhead; ++t) kf[t] = kfrag(t);
        if constexpr (kUseMask) {
#pragma unroll
            for (int t = 0; t < NT && t < 2 * kMaskAhead; ++t) {
                if constexpr (mask_tiled(kMask)) {
                    if (t % 2 == 0) fetch_pair(t, mw[t], mw[t + 1]);
                } else {
                    fetch(t, mw[t]);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < NT && t < 2; ++t)
            S[t] = score(kf[t], cinit(t, mw[kUseMask ? t : 0]));
#pragma unroll
        for (int pr = 0; pr < kPairs; ++pr) {
            __builtin_amdgcn_sched_barrier(0);
            if ((pr * 4) % kPairs < 4) set_wave_prio(3 - (pr * 4) / kPairs);  // at each quarter
            // the next window's DMA rounds ceil(pr R / P) .. ceil((pr+1) R / P) - 1
#pragma unroll
            for (int k = (pr * Issue::kRounds + kPairs - 1) / kPairs;
                 k < ((pr + 1) * Issue::kRounds + kPairs - 1) / kPairs; ++k)
                issue(k);
            const int t0 = 2 * pr;
            const bool has1 = t0 + 1 < NT;
            const X4 v0 = lds_read_tr<T>(vrow + kVTile * t0);
            const X4 v1 = has1 ? lds_read_tr<T>(vrow + kVTile * (t0 + 1)) : v0;
            X4 w0 = v0, w1 = v1;
            if constexpr (D == 32) {
                w0 = lds_read_tr<T>(vrow + 16 + kVTile * t0);
                w1 = has1 ? lds_read_tr<T>(vrow + 16 + kVTile * (t0 + 1)) : w0;
            }
#pragma unroll
            for (int t = t0 + 2 * kKAhead; t < t0 + 2 * kKAhead + 2; ++t)
                if (t < NT) kf[t] = kfrag(t);
            if constexpr (kUseMask) {
#pragma unroll
                for (int t = t0 + 2 * kMaskAhead; t < t0 + 2 * kMaskAhead + 2; ++t)
                    if (t < NT) {
                        if constexpr (mask_tiled(kMask)) {
                            if (t % 2 == 0) fetch_pair(t, mw[t], mw[t + 1]);
                        } else {
                            fetch(t, mw[t]);
                        }
                    }
            }
            X8 pb;
            if constexpr (kKAhead == 1) {
                pb = probs(S[t0], S[has1 ? t0 + 1 : t0], has1);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int t = t0 + 2; t < t0 + 4; ++t)
                if (t < NT) S[t] = score(kf[t], cinit(t, mw[kUseMask ? t : 0]));
            if constexpr (kKAhead != 1) pb = probs(S[t0], S[has1 ? t0 + 1 : t0], has1);
            accumulate(pb, v0, v1, has1, o, lacc);
            asm volatile("" : "+v"(o));  // as in the exact pass below
            if constexpr (D == 32) {
                accumulate_hi(pb, w0, w1, has1, o2);
                asm volatile("" : "+v"(o2));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    set_wave_prio(0);

    float l = lacc[0];  // every row of ones^T P^T holds the sum of query col
    const bool bad = qi < N && !(l >= kRowSumMin && l <= kRowSumMax);  // also NaN and inf
    bool exact = false;  // the exact pass ran and moved the offsets (wave-uniform)
    if (__builtin_amdgcn_ballot_w64(bad) != 0) {
        // Exact pass: the row max of the scores, then the strip again with
        // the max subtracted in the fp32 accumulator.  Each pass reads K
        // (and the mask) through opaque copies of the fragment bases, so
        // that the compiler reads them again instead of keeping an earlier
        // pass's fragments live across the passes.
        uint32_t ka = lds_byte_addr(kbase);
        int mva = mvoff;
        asm volatile("" : "+v"(ka), "+v"(mva));
        mvoff = mva;
        float m0 = -INFINITY, m1 = -INFINITY;
        MaskWords w;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            __builtin_amdgcn_sched_barrier(0);
            fetch(t, w);
            const f32x4 sc = score(lds_load<X8>(ka + t * kKTile * sizeof(T)), cinit(t, w));
            m0 = fmaxf(fmaxf(m0, sc[0]), sc[1]);
            m1 = fmaxf(fmaxf(m1, sc[2]), sc[3]);
            // keeps each tile's max here (pure math may otherwise be sunk
            // below the loop, keeping every score tile live)
            asm volatile("" : "+v"(m0), "+v"(m1));
        }
        __builtin_amdgcn_sched_barrier(0);
        const float m = xmax32(xmax16(fmaxf(m0, m1)));
        o = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        o2 = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        lacc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        uint32_t kb = lds_byte_addr(kbase);
        int mvb = mvoff;
        asm volatile("" : "+v"(kb), "+v"(mvb));
        mvoff = mvb;
#pragma unroll
        for (int pr = 0; pr < kPairs; ++pr) {
            __builtin_amdgcn_sched_barrier(0);
            const int t0 = 2 * pr;
            const bool has1 = t0 + 1 < NT;
            MaskWords w0, w1;
            fetch(t0, w0);
            if (has1) fetch(t0 + 1, w1);
            const f32x4 s0 = score(lds_load<X8>(kb + t0 * kKTile * sizeof(T)), cinit(t0, w0) - m);
            f32x4 s1 = s0;
            if (has1)
                s1 = score(lds_load<X8>(kb + (t0 + 1) * kKTile * sizeof(T)), cinit(t0 + 1, w1) - m);
            const X4 v0 = lds_read_tr<T>(vrow + kVTile * t0);
            const X4 v1 = has1 ? lds_read_tr<T>(vrow + kVTile * (t0 + 1)) : v0;
            const X8 pb = probs(s0, s1, has1);
            accumulate(pb, v0, v1, has1, o, lacc);
            // keeps the O product in this iteration (it would otherwise be
            // sunk towards the store, keeping every V fragment live)
            asm volatile("" : "+v"(o));
            if constexpr (D == 32) {
                const X4 w0 = lds_read_tr<T>(vrow + 16 + kVTile * t0);
                const X4 w1 = has1 ? lds_read_tr<T>(vrow + 16 + kVTile * (t0 + 1)) : w0;
                accumulate_hi(pb, w0, w1, has1, o2);
                asm volatile("" : "+v"(o2));
            }
        }
        l = lacc[0];
        // move the offsets: a window like this one would have row sums
        // near 2^kOffsetTarget (rows whose scores are not finite keep theirs)
        const float delta = kOffsetTarget - m - __builtin_amdgcn_logf(l);
        off += (delta - delta == 0.0f) ? delta : 0.0f;  // 0 for NaN and infinities
        exact = true;
    }

    // lane holds O[qi][4g + r], r = 0..3 (head dim 32: and O[qi][16 + 4g + r])
    if constexpr (kDefer) {
        const float inv = 1.0f / l;
#pragma unroll
        for (int r = 0; r < 4; ++r) pend.r[r] = T(o[r] * inv);
    } else if (qi < N) {
        T* orow = static_cast<T*>(p.out) + b * p.os[0] + h * p.os[1] + qi * p.os[2];
        const float inv = 1.0f / l;
        X4 res;
#pragma unroll
        for (int r = 0; r < 4; ++r) res[r] = T(o[r] * inv);
        if constexpr (kVec) {
            *reinterpret_cast<X4*>(orow + 4 * g) = res;
            if constexpr (D == 32) {
                X4 res2;
#pragma unroll
                for (int r = 0; r < 4; ++r) res2[r] = T(o2[r] * inv);
                *reinterpret_cast<X4*>(orow + 16 + 4 * g) = res2;
            }
        } else {
            static_assert(D == 16, "head dim 32 runs vector IO");
#pragma unroll
            for (int r = 0; r < 4; ++r) orow[(4 * g + r) * p.os[3]] = res[r];
        }
    }
    return exact;
}

// One strip (16 queries, NT*16 keys) of one window, fp32 operands: the
// scores run on v_mfma_f32_16x16x4f32 (four steps over the head dim) and
// the softmax is online over key chunks of at most 6 tiles with a lazy
// rescale: the first chunk sets the row max exactly; a later chunk
// exponentiates against the running max unless one of its scores exceeds it
// by more than kLazyMargin (a wave-uniform test), in which case the max is
// refreshed across the lane groups and O and the row sum are rescaled
// first.  The row sum is taken on the VALU.
template <typename T, int NT, int kMask, bool kUseMask, bool kVec>
__device__ __forceinline__ void attend_f32(const Params& p, const f32x4 (&bs)[NT], const T* __restrict__ q_lds,
                                           const T* __restrict__ k_lds, const T* __restrict__ vt_lds, int b,
                                           int h, int wave, int qi, int col, int g) {
    static_assert(sizeof(T) == 4, "2-byte types run attend_offset");
    constexpr int kVtStride = Stage<T, NT, kVec>::kVtStride;
    constexpr int kPrefetch = NT < 6 ? NT : 6;
    const int N = p.N;

    // B operand of S^T = K Q^T: Q[qi][4g..4g+3] (pre-scaled in LDS)
    const f32x4 qf = *reinterpret_cast<const f32x4*>(&q_lds[(wave * 16 + col) * 16 + 4 * g]);

    // Tensor mask through a buffer descriptor spanning exactly the window's
    // [N, N] extent: offsets past it return 0, so no per-key test is needed;
    // padded keys read a finite neighbour (their bias is -inf) and padded
    // query rows read row N-1 (never stored).  A lane's 4 keys of a tile are
    // contiguous in the mask row: one 8-byte (16-bit masks) or 16-byte (fp32
    // masks) load per tile.  Only the last tile of row N-1 can reach past
    // the extent, and a range check at dword or access granularity would
    // then zero in-range keys sharing the load, so those lanes read that
    // tile again element by element.  Offsets are immediates.
    constexpr int kMaskBytes = (kMask == kMaskF32) ? 4 : 2;
    static_assert(!mask_tiled(kMask), "tiled masks: 2-byte tuned kernels only");
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
                const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(mrsrc, off, 0, 0);
                mq[2 * slot] = w[0];
                mq[2 * slot + 1] = w[1];
            } else {
                const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(mrsrc, off, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) mq[4 * slot + r] = w[r];
            }
            // the 16-bit keys of the last row holding key N - 1 are read again
            // element by element
            if (kMaskBytes == 2 && t >= first_last_tile(NT) && holds_last_key(16 * t + 4 * g, 4, qi, N)) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (kMaskBytes == 2) {
                        const uint32_t hv = __builtin_amdgcn_raw_buffer_load_b16(mrsrc, off + 2 * r, 0, 0);
                        if (r & 1)
                            mq[2 * slot + (r >> 1)] |= hv << 16;
                        else
                            mq[2 * slot + (r >> 1)] = hv;
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

    constexpr int kNumChunks = (NT + 5) / 6;
    constexpr int kChunk = (NT + kNumChunks - 1) / kNumChunks;
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
    float lsum = 0.0f;
    float m_run = -INFINITY;
    float mb_run = 0.0f;  // m_run * log2(e)
    const T* vrow = &vt_lds[col * kVtStride + 4 * g];  // transposed V

#pragma unroll
    for (int c0 = 0; c0 < NT; c0 += kChunk) {
        // chunks must not interleave: that would keep two chunks of scores live
        __builtin_amdgcn_sched_barrier(0);
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
            const f32x4 kf = *reinterpret_cast<const f32x4*>(&k_lds[(16 * t + col) * 16 + 4 * g]);
            f32x4 acc = c;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[kk], qf[kk], acc, 0, 0, 0);
            S[u] = acc;
            if constexpr (kUseMask) __builtin_amdgcn_sched_barrier(0);  // keep the mask ring
        }

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
        // O^T += V^T P^T
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
    lsum += __shfl_xor(lsum, 16);
    const float l = lsum + __shfl_xor(lsum, 32);

    // lane holds O[qi][4g + r], r = 0..3
    if (qi < N) {
        T* orow = static_cast<T*>(p.out) + b * p.os[0] + h * p.os[1] + qi * p.os[2];
        const float inv = 1.0f / l;
        f32x4 res;
#pragma unroll
        for (int r = 0; r < 4; ++r) res[r] = o[r] * inv;
        if constexpr (kVec) {
            *reinterpret_cast<f32x4*>(orow + 4 * g) = res;
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) orow[(4 * g + r) * p.os[3]] = res[r];
        }
    }
}

// HPW heads per workgroup (1, or kHeadsPerWg on the LDS-DMA path): head slot
// s = threadIdx.x / kThreads runs the kWaves strips of head h0 + s with its
// own K/V buffers; the slots share the window walk and the barriers.
// Head dim D = 32 (2-byte types, vector IO, one head): K and V take twice
// the LDS.  With HPW = 1 they are single-buffered (3 workgroups per CU,
// which overlap each other's staging): the next window's rows are requested
// after the barrier that ends a window's compute.  With HPW > 1 the slots
// are HPW strip groups of one head (12 waves, one workgroup per CU) that
// share double-buffered K and V, staged by all the waves during the compute.
template <typename T, int NT, int kMask, bool kVec, int HPW, int D = 16>
__global__ void __launch_bounds__(kThreads * HPW)
__attribute__((amdgpu_waves_per_eu(waves_per_eu<T, NT, kMask, kVec>(), waves_per_eu<T, NT, kMask, kVec>())))
swin_attention_tuned_kernel(const Params p) {
    typedef Stage<T, NT, kVec, D> St;
    constexpr int NP = St::NP;
    constexpr bool kGroupSlots = D == 32 && HPW > 1;  // the slots are strip groups of one head
    constexpr bool kSingle = D == 32 && HPW == 1;     // single-buffered K and V
    static_assert(D == 16 || (kVec && v_row_major<T>()), "head dim 32: LDS-DMA path");
    constexpr int kStageWaves = kGroupSlots ? kWaves * HPW : kWaves;  // waves sharing a window's DMA
    static_assert(!kGroupSlots || waves_per_eu<T, NT, kMask, kVec>() * 4 >= kWaves * HPW,
                  "the strip groups' waves must fit one CU's SIMDs together");
    // 2-byte LDS-DMA staging: K and V in DMA rounds (all at once for the
    // first window and for waves without a strip, spread over the compute of
    // the previous window otherwise); Q by register
    constexpr bool kSpread = kVec && v_row_major<T>();  // Stage<T, NT, true>::kDma
    // head dim 16 on that path keeps Q in registers (load_qraw, q_operand);
    // head dim 32 passes it through LDS, whose rows are wave-private there (a
    // wave stores and reads only its own 16 rows, in that order), so one
    // buffer serves
    constexpr bool kQReg = kSpread && D == 16;
    constexpr int kQBufs = HPW > 1 || kSingle ? 1 : 2;
    constexpr int kKVBufs = kSingle ? 1 : 2;
    static_assert(HPW == 1 || (kVec && v_row_major<T>()), "several heads per workgroup need the LDS-DMA path");
    constexpr bool kRecs = HPW > 1 && !kGroupSlots;  // token-record K/V layout shared by the head slots
    // (kRecs: K and V in one record array, k_lds; the last load's spill
    // lands in its padding)
    constexpr int kKLds = kRecs ? rec_loads(NT) * 512 : St::kRows * D;
    constexpr int kVLdsAll = kRecs ? 8 : St::kVLds;
    __shared__ __attribute__((aligned(16))) T q_lds[kQBufs][HPW][kQReg ? 8 : St::kQRows * q_row_len<T, D>()];
    __shared__ __attribute__((aligned(16))) T k_lds[kKVBufs][kKLds];
    __shared__ __attribute__((aligned(16))) T vt_lds[kKVBufs][kVLdsAll];
    __shared__ __attribute__((aligned(4))) uint8_t cls_lds[kMask == kMaskRegion ? NP : 4];
    static_assert(sizeof(q_lds) + sizeof(k_lds) + sizeof(vt_lds) + sizeof(cls_lds) <= 160 * 1024,
                  "LDS footprint exceeds the 160 KB of a gfx950 CU");

    // One word of every 64-byte line of the kernel arguments, all requested
    // before any is needed: the set-up below reads them in dependent chains
    // (behind branches, in the walk of the type table), and every workgroup
    // starting at once would otherwise wait for one scalar-cache miss after
    // another (about 2 us of set-up at config 3).
    if constexpr (kQReg) {
        typedef const __attribute__((address_space(4))) uint32_t KWord;
        KWord* kw = (KWord*)__builtin_amdgcn_kernarg_segment_ptr();
        constexpr int kLines = (sizeof(Params) + 63) / 64;
        static_assert(kLines <= 8, "kernel arguments beyond 8 lines");
        uint32_t w[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) w[l] = kw[16 * (l < kLines ? l : kLines - 1)];
        asm volatile("" ::"s"(w[0]), "s"(w[1]), "s"(w[2]), "s"(w[3]), "s"(w[4]), "s"(w[5]), "s"(w[6]), "s"(w[7]));
    }

    uint32_t chunk;
    if (!xcd_chunk(blockIdx.x, p.launched, p.chunks, chunk)) return;
    // chunk = (range * head blocks + head block) * groups + group: the groups
    // of one (range, head block) are consecutive, hence on one XCD, and
    // share its L2 for K/V.  A head block is HPW heads, or one head whose
    // strip groups HPW * group .. + HPW - 1 are the slots (kGroupSlots;
    // p.groups then counts blocks of HPW strip groups).
    const int slot = HPW > 1 ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kThreads) : 0;
    constexpr int kHeads = kGroupSlots ? 1 : HPW;  // heads per workgroup
    const int hb_count = p.H / kHeads;
    const int grp = kGroupSlots ? static_cast<int>(chunk % p.groups) * HPW + slot : static_cast<int>(chunk % p.groups);
    const int rh = static_cast<int>(chunk / p.groups);
    const int h0 = (rh % hb_count) * kHeads;  // first head of the workgroup
    const int h = kGroupSlots ? h0 : h0 + slot;
    const int range = rh / hb_count;
    // Tensor-mask modes take every ranges-th window (range, range + ranges,
    // ...): a window whose boundary flag is set costs more than one whose
    // flag is clear, and boundary windows come in runs (the last window
    // slab of a volume is a run of nWh * nWw), so contiguous ranges would
    // leave some workgroups with mostly masked windows (17% at config 3).
    constexpr bool kStrided = mask_tensor(kMask);
    const int i0 = kStrided ? 0 : range * p.win_per_wg;
    const int i1 = kStrided ? (p.B - range + p.ranges - 1) / p.ranges : min(p.B, i0 + p.win_per_wg);

    const int lane = threadIdx.x & 63;
    // wave-uniform, and provably so (scalar registers): the strip index, and
    // with it `active`, then steer branches the compiler keeps scalar, and
    // values assigned under them stay in scalar registers
    const int wave_id = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int wave = HPW > 1 ? wave_id & (kWaves - 1) : wave_id;  // strip within the group
    const int col = lane & 15;
    const int g = lane >> 4;
    const int strip = grp * kWaves + wave;
    const int qi = strip * 16 + col;
    const bool active = strip < p.strips;
    const int q0 = grp * kWaves * 16;  // first query row of this group

    if constexpr (kMask == kMaskRegion) {
        // shift-region class of every window token: one bit per axis, set at
        // or past ws - ss (covered by the prologue barrier below)
        for (int j = threadIdx.x; j < NP; j += kThreads * HPW) {
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

    // 2-byte types: scores in log2 units (attend_offset), so Q carries log2(e)
    const float qscale = sizeof(T) == 2 ? p.scale * kLog2e : p.scale;
    float off = 0.0f;  // row offset of the offset softmax (2-byte types, log2 units)

    // records: the lane's load offsets per round, the same for every window
    int rec_off[kRecs ? kRecRounds<St, kRecs>() : 1];
    if constexpr (kRecs) {
#pragma unroll
        for (int r = 0; r < kRecRounds<St, kRecs>(); ++r) rec_off[r] = St::rec_voff(p, r);
    }
    typedef typename Frag<T>::x8 X8;
    constexpr bool kTensor = mask_tensor(kMask);

    if constexpr (kQReg) {
        // Head dim 16 on the LDS-DMA path: while window i is computed, its DMA
        // rounds bring in window i + 1's K and V, and Q travels by register
        // (load_qraw a window ahead, q_operand after the end-of-window wait).
        // A window's output is stored after that wait (PendingOut).
        // the window being computed (b0, code0, flag0: tensor mode reads its
        // mask) and the next one (b1, ...), as plain scalars: a struct here
        // was kept in memory, which the compiler placed in LDS
        typedef typename St::WindowDesc WD;
        WindowIter<kMask> it;
        it.init(p, i0);
        if constexpr (kStrided) {
            it.base = range;
            it.stride = p.ranges;
        }
        auto window_flag = [&](int bw) {
            if constexpr (kTensor) return p.boundary == nullptr || p.boundary[bw] != 0;
            return true;
        };
        int code0;
        int b0 = it.window(p, code0);
        bool flag0 = window_flag(b0);
        QRaw<T> qraw;
        X8 qf = {};
        if constexpr (kMask == kMaskRegion) __syncthreads();  // the region classes, for the first build
        {
            const WD d0 = St::template window_desc<kRecs>(p, b0, h, h0);
#pragma unroll
            for (int r = 0; r < St::template dma_rounds<kRecs>(); ++r)
                St::template dma_round<kRecs>(p, d0, k_lds[0], vt_lds[0], r, kRecs ? rec_off[r] : 0);
        }
        if (active) qraw = load_qraw<T>(p, b0, h, qi, g);

        f32x4 bs[NT];
        PendingOut<T> pend;
        int code_cur = -1;
        bool rebuild = false;  // this wave's offsets moved: rebuild its tiles (wave-uniform)
        // The window after b0 (b1, ...) with its DMA descriptor, and its Q
        // rows requested, are prepared before the barrier that ends the
        // window before it: waves that finish their pair loop early do that
        // scalar work while the others compute, and the window top after the
        // barrier goes straight into the next pair loop.
        int b1 = b0, code1 = code0;
        bool flag1 = flag0;
        WD d1 = {};
        auto prepare_next = [&]() {
            it.next(p);
            b1 = it.window(p, code1);
            flag1 = window_flag(b1);
            d1 = St::template window_desc<kRecs>(p, b1, h, h0);
            if (active) qraw = load_qraw<T>(p, b1, h, qi, g);
        };
        for (int i = i0; i < i1; ++i) {
            const int buf = (i - i0) & 1;
            const bool more = i + 1 < i1;
            // New bias (+ region mask) tiles are built before the next
            // window's rows are requested: the vector-memory counter retires
            // in order, so waiting for the bias loads after that request
            // would wait for the rows as well.  The first window's tiles are
            // built while its rows arrive (one wait covers both).
            if (active && (code0 != code_cur || rebuild)) {  // code is workgroup-uniform
                if (kMask == kMaskRegion && !rebuild && code_cur >= 0)
                    retype_tiles<NT>(bs, qi, g, p.N, code_cur, code0, cls_lds);
                else
                    build_tiles<NT, kMask, true>(bs, p, h, qi, g, code0, cls_lds, off);
                code_cur = code0;
                rebuild = false;
            }
            if (i == i0) {
                wait_vmem();
                if (active) qf = q_operand<T>(qraw, qscale, g);
                if (more) prepare_next();
                __syncthreads();  // the first window's rows
            }
            const DmaIssuer<T, St, kRecs, kStageWaves> issue{&p, d1, k_lds[buf ^ 1], vt_lds[buf ^ 1], rec_off, more};
            T* const kw = k_lds[buf] + (kRecs ? 16 * slot : 0);  // this head's rows of each record
            T* const vw = kRecs ? k_lds[buf] + kRecV + 16 * slot : vt_lds[buf];
            if (active) {
                if (kTensor && flag0)
                    rebuild = attend_offset<T, NT, kMask, kTensor, kVec, kRecs, D, true>(
                        p, bs, qf, qf, kw, vw, b0, h, qi, col, g, off, issue, pend);
                else
                    rebuild = attend_offset<T, NT, kMask, false, kVec, kRecs, D, true>(
                        p, bs, qf, qf, kw, vw, b0, h, qi, col, g, off, issue, pend);
            } else {
#pragma unroll
                for (int r = 0; r < St::template dma_rounds<kRecs>(); ++r) issue(r);
            }
            wait_vmem();  // this wave's DMA rows (and its Q) have landed
            if (active) {
                if (more) qf = q_operand<T>(qraw, qscale, g);
                // after the wait: the store then retires during the next window
                store_out4<T>(p, pend.r, b0, h, qi, g);
            }
            b0 = b1;
            code0 = code1;
            flag0 = flag1;
            if (i + 2 < i1) prepare_next();
            __syncthreads();
        }
        return;
    }

    St st;
    WindowIter<kMask> it;
    it.init(p, i0);
    if constexpr (kStrided) {
        it.base = range;
        it.stride = p.ranges;
    }
    int code_cur = -1;
    bool rebuild = false;  // this wave's offsets moved: rebuild its tiles (wave-uniform)
    int code_next;
    int b_next = it.window(p, code_next);
    // tensor mode: the window's boundary flag is read before the next
    // window's rows are requested, so waiting for it never waits for them
    bool flag_next = true;
    if constexpr (kMask != kNoMask && kMask != kMaskRegion)
        flag_next = p.boundary == nullptr || p.boundary[b_next] != 0;
    auto stage_load = [&](int bw, int sb) {
        if constexpr (kSpread) {
            st.load_q(p, bw, h, q0);
            const auto wd = St::template window_desc<kRecs>(p, bw, h, h0);
#pragma unroll
            for (int r = 0; r < St::template dma_rounds<kRecs, kStageWaves>(); ++r)
                St::template dma_round<kRecs, kStageWaves>(p, wd, k_lds[sb], vt_lds[sb], r,
                                                           kRecs ? rec_off[r] : 0);
        } else {
            st.load(p, bw, h, q0, k_lds[sb], vt_lds[sb]);
        }
    };
    stage_load(b_next, 0);
    st.store(qscale, q_lds[0][slot], k_lds[0], vt_lds[0]);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // LDS-DMA rows have landed
    __syncthreads();

    f32x4 bs[NT];
    PendingOut<T> pend;  // unused: these paths store each strip's output at once
    for (int i = i0; i < i1; ++i) {
        const int buf = kKVBufs == 2 ? (i - i0) & 1 : 0;
        const int nbuf = kKVBufs == 2 ? buf ^ 1 : 0;  // the next window's K/V buffer
        const int b = b_next;
        const int code = code_next;
        const bool flag = flag_next;
        // New bias (+ region mask) tiles are built before the next window's
        // rows are requested: the vector-memory counter retires in order, so
        // waiting for the bias loads after that request would wait for the
        // rows as well.
        if (active && (code != code_cur || rebuild)) {  // code is workgroup-uniform
            if (kMask == kMaskRegion && sizeof(T) == 2 && !rebuild && code_cur >= 0)
                retype_tiles<NT>(bs, qi, g, p.N, code_cur, code, cls_lds);
            else
                build_tiles<NT, kMask, sizeof(T) == 2>(bs, p, h, qi, g, code, cls_lds, off);
            code_cur = code;
            rebuild = false;
        }
        if (i + 1 < i1) {
            it.next(p);
            b_next = it.window(p, code_next);
            if constexpr (kMask != kNoMask && kMask != kMaskRegion)
                flag_next = p.boundary == nullptr || p.boundary[b_next] != 0;
            if constexpr (kSpread) {
                if (active || kSingle)
                    st.load_q(p, b_next, h, q0);
                else
                    stage_load(b_next, nbuf);
            } else {
                stage_load(b_next, nbuf);
            }
        }
        const auto issue = [&]() {
            if constexpr (kSpread && !kSingle)
                return DmaIssuer<T, St, kRecs, kStageWaves>{&p, St::template window_desc<kRecs>(p, b_next, h, h0),
                                                            k_lds[nbuf], vt_lds[nbuf], rec_off, i + 1 < i1};
            else
                return NoIssue{};
        }();
        typedef std::decay_t<decltype(issue)> Issuer;
        const int qb = kQBufs == 2 ? buf : 0;
        T* const qw = q_lds[qb][slot];
        T* const kw = k_lds[buf] + (kRecs ? 16 * slot : 0);  // this head's rows of each record
        T* const vw = kRecs ? k_lds[buf] + kRecV + 16 * slot : vt_lds[buf];
        if (active) {
            bool use_mask = false;
            if constexpr (kTensor) use_mask = flag;
            if constexpr (sizeof(T) == 2) {
                // Q operands from the wave's LDS rows
                const X8 qa = *reinterpret_cast<const X8*>(&qw[(wave * 16 + col) * (2 * D) + 8 * g]);
                X8 qb = qa;
                if constexpr (D == 32) qb = *reinterpret_cast<const X8*>(&qw[(wave * 16 + col) * 64 + 32 + 8 * g]);
                if (use_mask)
                    rebuild = attend_offset<T, NT, kMask, kTensor, kVec, kRecs, D, false, Issuer>(
                        p, bs, qa, qb, kw, vw, b, h, qi, col, g, off, issue, pend);
                else
                    rebuild = attend_offset<T, NT, kMask, false, kVec, kRecs, D, false, Issuer>(
                        p, bs, qa, qb, kw, vw, b, h, qi, col, g, off, issue, pend);
            } else {
                if (use_mask)
                    attend_f32<T, NT, kMask, kTensor, kVec>(p, bs, qw, kw, vw, b, h, wave, qi, col, g);
                else
                    attend_f32<T, NT, kMask, false, kVec>(p, bs, qw, kw, vw, b, h, wave, qi, col, g);
            }
        }
        if constexpr (kSingle) {
            if (i + 1 < i1) {
                __syncthreads();  // every wave is done with this window's K and V
                const auto wd = St::template window_desc<false>(p, b_next, h, h0);
#pragma unroll
                for (int r = 0; r < St::template dma_rounds<false>(); ++r)
                    St::template dma_round<false>(p, wd, k_lds[0], vt_lds[0], r, 0);
            }
        }
        if (i + 1 < i1) st.store(qscale, q_lds[kQBufs == 2 ? buf ^ 1 : 0][slot], k_lds[nbuf], vt_lds[nbuf]);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // LDS-DMA rows have landed
        __syncthreads();
    }
}

// Launch for element type T; NT from kTileCounts, kmask a MaskKind.
template <typename T>
void launch(const Params& p, int NT, int kmask, hipStream_t s) {
    const dim3 grid(p.launched), block(kThreads * p.hpw);
#define CRUMPET_ATTN_MASK(NTV, MK)                                                                    \
    do {                                                                                              \
        if (p.vec_io) {                                                                               \
            if constexpr (v_row_major<T>() && multi_head_tiles(NTV) && MK != kMaskF32) {              \
                if (p.hpw == kHeadsPerWg) {                                                           \
                    hipLaunchKernelGGL((swin_attention_tuned_kernel<T, NTV, MK, true, kHeadsPerWg>), grid, \
                                       block, 0, s, p);                                               \
                    break;                                                                            \
                }                                                                                     \
            }                                                                                         \
            hipLaunchKernelGGL((swin_attention_tuned_kernel<T, NTV, MK, true, 1>), grid, block, 0, s, p); \
        } else {                                                                                      \
            hipLaunchKernelGGL((swin_attention_tuned_kernel<T, NTV, MK, false, 1>), grid, block, 0, s, p); \
        }                                                                                             \
    } while (0)
// tiled 16-bit masks: 2-byte types with vector IO at 14 and 22 tiles (the
// host selects them only there)
#define CRUMPET_ATTN_TILED(NTV, MK)                                                                   \
    do {                                                                                              \
        if constexpr (v_row_major<T>() && multi_head_tiles(NTV)) {                                    \
            if (p.vec_io) {                                                                           \
                if (p.hpw == kHeadsPerWg)                                                             \
                    hipLaunchKernelGGL((swin_attention_tuned_kernel<T, NTV, MK, true, kHeadsPerWg>), grid, \
                                       block, 0, s, p);                                               \
                else                                                                                  \
                    hipLaunchKernelGGL((swin_attention_tuned_kernel<T, NTV, MK, true, 1>), grid, block, 0, s, p); \
            }                                                                                         \
        }                                                                                             \
    } while (0)
#define CRUMPET_ATTN_NT(NTV)                                            \
    case NTV:                                                           \
        switch (kmask) {                                                \
            case kNoMask: CRUMPET_ATTN_MASK(NTV, kNoMask); break;       \
            case kMaskF16: CRUMPET_ATTN_MASK(NTV, kMaskF16); break;     \
            case kMaskF32: CRUMPET_ATTN_MASK(NTV, kMaskF32); break;     \
            case kMaskBF16: CRUMPET_ATTN_MASK(NTV, kMaskBF16); break;   \
            case kMaskF16T: CRUMPET_ATTN_TILED(NTV, kMaskF16T); break;  \
            case kMaskBF16T: CRUMPET_ATTN_TILED(NTV, kMaskBF16T); break; \
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
#undef CRUMPET_ATTN_TILED
#undef CRUMPET_ATTN_MASK
}

// Launch of the head-dim-32 kernel for element type T (2-byte) at NT tiles
// with HPW slots: one head of 4 waves (HPW = 1) or kHeadsPerWg strip groups
// of one head (no fp32 mask, d32_group_slots).
template <typename T, int NT, int HPW>
void launch32_slots(const Params& p, int kmask, hipStream_t s) {
    const dim3 grid(p.launched), block(kThreads * HPW);
    switch (kmask) {
        case kNoMask:
            hipLaunchKernelGGL((swin_attention_tuned_kernel<T, NT, kNoMask, true, HPW, 32>), grid, block, 0, s, p);
            break;
        case kMaskF16:
            hipLaunchKernelGGL((swin_attention_tuned_kernel<T, NT, kMaskF16, true, HPW, 32>), grid, block, 0, s, p);
            break;
        case kMaskF32:
            if constexpr (HPW == 1)
                hipLaunchKernelGGL((swin_attention_tuned_kernel<T, NT, kMaskF32, true, 1, 32>), grid, block, 0, s, p);
            break;
        case kMaskBF16:
            hipLaunchKernelGGL((swin_attention_tuned_kernel<T, NT, kMaskBF16, true, HPW, 32>), grid, block, 0, s, p);
            break;
        case kMaskF16T:
            hipLaunchKernelGGL((swin_attention_tuned_kernel<T, NT, kMaskF16T, true, HPW, 32>), grid, block, 0, s, p);
            break;
        case kMaskBF16T:
            hipLaunchKernelGGL((swin_attention_tuned_kernel<T, NT, kMaskBF16T, true, HPW, 32>), grid, block, 0, s, p);
            break;
        default:
            hipLaunchKernelGGL((swin_attention_tuned_kernel<T, NT, kMaskRegion, true, HPW, 32>), grid, block, 0, s,
                               p);
            break;
    }
}

// Launch of the head-dim-32 kernel for element type T (2-byte): p.hpw
// selects the slots (set by the host together with p.groups).
template <typename T>
void launch32(const Params& p, int NT, int kmask, hipStream_t s) {
    if (NT == 14) {
        launch32_slots<T, 14, 1>(p, kmask, s);
    } else if (NT == 22) {
        if (p.hpw == kHeadsPerWg && kmask != kMaskF32)
            launch32_slots<T, 22, kHeadsPerWg>(p, kmask, s);
        else
            launch32_slots<T, 22, 1>(p, kmask, s);
    }
}

}  // namespace
}  // namespace attn
}  // namespace crumpet
