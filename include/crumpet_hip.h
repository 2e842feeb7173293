/*
 * crumpet_hip.h - C ABI of the MI355X (gfx950) shifted-window kernels.
 *
 * libcrumpet_hip.so exports these entry points.  Every one of them is
 * stateless and re-entrant: the caller owns and preallocates every buffer,
 * passes raw device pointers plus sizes, and the work is enqueued
 * asynchronously on `stream` (a hipStream_t; NULL means the null stream).
 * Nothing here allocates device memory, synchronises the host or keeps
 * global device state.
 *
 * Each entry point returns CRUMPET_OK or a crumpet_status code.  The
 * human-readable reason of the last failure on the calling thread is
 * available from crumpet_last_error().
 *
 * The dispatcher ops of the reference that these entry points replace are
 * cited next to each declaration (file:line in chrisvoncsefalvay/crumpet).
 * The torch binding in crumpet_amd/csrc/torch_binding.cpp registers the same
 * op schemas under the `crumpet_ops` namespace and forwards to these calls.
 */
#ifndef CRUMPET_HIP_H_
#define CRUMPET_HIP_H_

#include <stddef.h>
#include <stdint.h>

/* Only these entry points are exported; everything else in the library is
 * built with hidden visibility. */
#if defined(__GNUC__)
#define CRUMPET_API __attribute__((visibility("default")))
#else
#define CRUMPET_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes returned by every entry point. */
enum crumpet_status {
    CRUMPET_OK = 0,
    CRUMPET_ERR_INVALID_ARGUMENT = 1, /* shape, shift, dtype, stride or pointer check failed */
    CRUMPET_ERR_UNSUPPORTED = 2,      /* valid request outside what the kernels implement */
    CRUMPET_ERR_HIP = 3               /* the HIP runtime reported an error at launch */
};

/* Element type codes. */
enum crumpet_dtype {
    CRUMPET_DTYPE_F32 = 0,
    CRUMPET_DTYPE_F16 = 1,
    CRUMPET_DTYPE_BF16 = 2,
    CRUMPET_DTYPE_U8 = 3 /* only for boundary flags */
};

/* Library version, e.g. "0.1.0". */
CRUMPET_API const char* crumpet_version(void);

/* Message describing the last non-OK status returned on this thread. */
CRUMPET_API const char* crumpet_last_error(void);

/* Static name of a status code. */
CRUMPET_API const char* crumpet_status_string(int status);

/*
 * Fused cyclic shift (torch.roll by -shift over D, H, W) plus 3D window
 * partition of a contiguous channels-last volume.
 *
 *   x   : [B, D, H, W, C]                      (elem_size bytes per element)
 *   out : [B * nW, ws_d * ws_h * ws_w, C]      nW = (D/ws_d)(H/ws_h)(W/ws_w)
 *
 *   out[(b*nW + win)*vol + loc, c] =
 *       x[b, (wd*ws_d+ld+ss_d) mod D, (wh*ws_h+lh+ss_h) mod H,
 *            (ww*ws_w+lw+ss_w) mod W, c]
 *
 * A pure byte copy: bit-exact for every element type.  D, H, W must be
 * divisible by the window and 0 <= ss < ws on every axis.
 *
 * Replaces op `fused_shift_partition_3d(Tensor! output, Tensor x, ...)`,
 * torch-ext/torch_binding.cpp:19-21, host entry
 * cuda/shift_partition_3d.cu:318-347.
 */
CRUMPET_API int crumpet_shift_partition_3d(void* out, const void* x,
                               int64_t B, int64_t D, int64_t H, int64_t W, int64_t C,
                               int64_t elem_size,
                               int64_t ws_d, int64_t ws_h, int64_t ws_w,
                               int64_t ss_d, int64_t ss_h, int64_t ss_w,
                               void* stream);

/*
 * Inverse of crumpet_shift_partition_3d: window reverse plus torch.roll by
 * +shift.
 *
 *   windows : [B * nW, vol, C]
 *   out     : [B, D, H, W, C]
 *
 * Replaces op `fused_unshift_unpartition_3d(Tensor! output, Tensor windows,
 * int B, int D, int H, int W, int C, ...)`, torch-ext/torch_binding.cpp:26-28,
 * host entry cuda/unshift_unpartition_3d.cu:284-318.
 */
CRUMPET_API int crumpet_unshift_unpartition_3d(void* out, const void* windows,
                                   int64_t B, int64_t D, int64_t H, int64_t W, int64_t C,
                                   int64_t elem_size,
                                   int64_t ws_d, int64_t ws_h, int64_t ws_w,
                                   int64_t ss_d, int64_t ss_h, int64_t ss_w,
                                   void* stream);

/*
 * Gradient of the shift-partition.  The adjoint of a permutation is its
 * inverse, so this is the unshift-unpartition gather applied to
 * grad_windows [B*nW, vol, C], writing grad_x [B, D, H, W, C].
 *
 * Replaces op `fused_shift_partition_3d_backward`, torch-ext/torch_binding.cpp:22-24,
 * host entry cuda/unshift_unpartition_3d.cu:320-348.
 */
CRUMPET_API int crumpet_shift_partition_3d_backward(void* grad_x, const void* grad_windows,
                                        int64_t B, int64_t D, int64_t H, int64_t W, int64_t C,
                                        int64_t elem_size,
                                        int64_t ws_d, int64_t ws_h, int64_t ws_w,
                                        int64_t ss_d, int64_t ss_h, int64_t ss_w,
                                        void* stream);

/*
 * Gradient of the unshift-unpartition: the shift-partition gather applied
 * to grad_x [B, D, H, W, C], writing grad_windows [B*nW, vol, C].
 *
 * Replaces op `fused_unshift_unpartition_3d_backward`,
 * torch-ext/torch_binding.cpp:29-31, host entry cuda/shift_partition_3d.cu:349-367.
 */
CRUMPET_API int crumpet_unshift_unpartition_3d_backward(void* grad_windows, const void* grad_x,
                                            int64_t B, int64_t D, int64_t H, int64_t W, int64_t C,
                                            int64_t elem_size,
                                            int64_t ws_d, int64_t ws_h, int64_t ws_w,
                                            int64_t ss_d, int64_t ss_h, int64_t ss_w,
                                            void* stream);

/*
 * Shifted-window additive attention mask, written densely.
 *
 *   out : [nW, vol, vol] of `dtype` (F32, F16 or BF16), contiguous
 *
 *   region(x, dim, ws, ss) = 0 if x < dim-ws; 1 if x < dim-ss; else 2
 *   label(p) = 9*region_d + 3*region_h + region_w, at unrolled window
 *              coordinates p = win*ws + loc (the shifted frame)
 *   out[win, i, j] = label(i) != label(j) ? -100 : 0
 *
 * All-zero shift gives an all-zero mask.  vol must not exceed 1024.
 *
 * Replaces op `compute_attn_mask_3d(Tensor! output, int D, int H, int W, ...)`,
 * torch-ext/torch_binding.cpp:16-18, host entry cuda/attn_mask_3d.cu:127-168.
 */
CRUMPET_API int crumpet_compute_attn_mask_3d(void* out, int32_t dtype,
                                 int64_t D, int64_t H, int64_t W,
                                 int64_t ws_d, int64_t ws_h, int64_t ws_w,
                                 int64_t ss_d, int64_t ss_h, int64_t ss_w,
                                 void* stream);

/*
 * Fused window attention, per window b and head h:
 *
 *   S = (q * scale) k^T + bias[h] + (boundary[b] ? mask[b mod mask_batch] : 0)
 *   out = softmax_rows(S) v
 *
 * q, k, v, out : [B, Hh, N, Dh] with arbitrary element strides (in elements,
 *                order b, h, n, d); dtype F16, BF16 or F32 (all four equal).
 * bias         : [Hh, N, N], strides (h, i, j) with unit j stride and a
 *                row stride i of at least N (rows do not overlap), dtype
 *                F32/F16/BF16.
 * mask         : [mask_batch, N, N] or NULL; strides (m, i, j) with unit j
 *                stride and a row stride of at least N; mask_batch
 *                must divide B (1 broadcasts, B is per window, nW repeats
 *                the per-window masks over an outer batch).
 * boundary     : [B] uint8 or NULL.  When NULL and mask != NULL every window
 *                reads its mask; a zero flag skips the mask for that window.
 * scale        : softmax scale.  fp32 operands: q is multiplied by it and
 *                rounded back.  2-byte operands: q * scale * log2(e) enters
 *                the product as a rounded value plus its rounded remainder,
 *                which is at least as precise as the rounded q * scale.
 *
 * Needs no workspace: every buffer is an input or the output.
 *
 * Supported: Dh = 16, 32, 64, 128 or 256 and any N >= 1.  Dh = 16 with N <= 512
 * (every Swin UNETR stage at feature size 48) runs the tuned kernel; other
 * shapes run the general kernel, whose shifted-window mode below takes
 * windows of up to 2048 tokens.
 *
 * Replaces the Triton launch of `_fused_swin_attention_kernel`,
 * torch-ext/crumpet/fused_attention.py:48-146 (wrapper :149-226).  The
 * reference had no dispatcher op for attention; the torch binding adds
 * `crumpet_ops::fused_swin_attention`.
 */
CRUMPET_API int crumpet_fused_swin_attention(void* out, const int64_t out_strides[4],
                                 const void* q, const int64_t q_strides[4],
                                 const void* k, const int64_t k_strides[4],
                                 const void* v, const int64_t v_strides[4],
                                 int32_t dtype,
                                 int64_t B, int64_t Hh, int64_t N, int64_t Dh,
                                 const void* bias, int32_t bias_dtype,
                                 const int64_t bias_strides[3],
                                 const void* mask, int32_t mask_dtype, int64_t mask_batch,
                                 const int64_t mask_strides[3],
                                 const uint8_t* boundary,
                                 float scale,
                                 void* stream);

/*
 * Tiled copy of a 16-bit mask [M, N, N] (strides in elements, unit key
 * stride) for crumpet_fused_swin_attention_tiled:
 *   tiles[m][s][p][16 g + c][j][r] = mask[m][min(16 s + c, N - 1)][16 (2p + j) + 4 g + r]
 * (0 for keys past N), s < ceil(N / 16), p < NT / 2 for the attention
 * kernel's tile count NT for N (2 where that is 1);
 * crumpet_attn_mask_tiles_elements(M, N) elements of the mask's dtype (-1
 * for N outside 1 .. 512), 8-byte aligned.  A lane's keys of a pair of key
 * tiles are then 16 contiguous bytes, a wave's 1 KB.  Bits are copied.
 *
 * No counterpart in the reference (it reads the mask in place,
 * torch-ext/crumpet/fused_attention.py:123-128); for callers that use one
 * mask tensor in many calls, as the MONAI layers do with their per-layer
 * mask (monai_patch.py:167-191).
 */
CRUMPET_API int64_t crumpet_attn_mask_tiles_elements(int64_t M, int64_t N);
CRUMPET_API int crumpet_attn_mask_tiles(void* out, const void* mask, int32_t mask_dtype, int64_t M,
                                        int64_t N, const int64_t mask_strides[3], void* stream);

/*
 * crumpet_fused_swin_attention with the mask also given as its tiled copy
 * (crumpet_attn_mask_tiles of the same mask, same M and N).  Results are
 * identical; the tuned kernels read the tiled copy where they run with
 * 2-byte q/k/v, vector IO and 129 <= N <= 352 (their 14- and 22-tile
 * forms), the mask itself otherwise.  mask and mask_tiles are required.
 *
 * No counterpart in the reference: a faster form of
 * crumpet_fused_swin_attention (torch-ext/crumpet/fused_attention.py:149-226)
 * for callers that keep the tiled copy with the mask.
 */
CRUMPET_API int crumpet_fused_swin_attention_tiled(void* out, const int64_t out_strides[4],
                                 const void* q, const int64_t q_strides[4],
                                 const void* k, const int64_t k_strides[4],
                                 const void* v, const int64_t v_strides[4],
                                 int32_t dtype,
                                 int64_t B, int64_t Hh, int64_t N, int64_t Dh,
                                 const void* bias, int32_t bias_dtype,
                                 const int64_t bias_strides[3],
                                 const void* mask, int32_t mask_dtype, int64_t mask_batch,
                                 const int64_t mask_strides[3],
                                 const void* mask_tiles,
                                 const uint8_t* boundary,
                                 float scale,
                                 void* stream);

/*
 * Fused window attention with the shifted-window mask of a [D, H, W] volume
 * (window ws, shift ss) instead of a mask tensor.  Bit-identical in meaning
 * to crumpet_fused_swin_attention with
 *   mask = crumpet_compute_attn_mask_3d(D, H, W, ws, ss)   ([nW, N, N]),
 *   mask_batch = nW, boundary = NULL,
 * for B a multiple of nW = (D/ws_d)(H/ws_h)(W/ws_w) and N = ws_d*ws_h*ws_w:
 * window b uses the mask of window b mod nW (the order MONAI tiles windows in).
 * The mask is never materialised or read: windows are processed grouped by
 * their boundary type and the kernel folds the type's mask into its bias
 * tiles.  Needs no workspace.
 *
 * Has no dispatcher-op counterpart in the reference; it replaces the
 * `mask.repeat` + `abs().amax` + masked Triton launch sequence of
 * torch-ext/crumpet/monai_patch.py:167-191 for the patched MONAI path.
 */
CRUMPET_API int crumpet_fused_swin_attention_shifted(
    void* out, const int64_t out_strides[4],
    const void* q, const int64_t q_strides[4],
    const void* k, const int64_t k_strides[4],
    const void* v, const int64_t v_strides[4],
    int32_t dtype,
    int64_t B, int64_t Hh, int64_t N, int64_t Dh,
    const void* bias, int32_t bias_dtype, const int64_t bias_strides[3],
    int64_t D, int64_t H, int64_t W,
    int64_t ws_d, int64_t ws_h, int64_t ws_w,
    int64_t ss_d, int64_t ss_h, int64_t ss_w,
    float scale,
    void* stream);

/*
 * Window-ordered qkv projection of a Swin window-attention block, with the
 * layout work before it fused into its operand gather:
 *
 *   out[t, :] = LN(xpad[src(t)]) @ weight^T + bias        out: [B*nW, N, n_out]
 *
 * x is the block input [B, D, H, W, C] (channels-last, contiguous, x_dtype).
 * xpad is x zero-padded at the end of each axis to multiples of the window
 * (padding applied after the LayerNorm, so padded tokens project to `bias`).
 * Token t = (b*nW + win)*N + loc runs in window order, and src(t) is the
 * position the cyclic shift by -ss and the window partition place at t
 * (the same order as crumpet_shift_partition_3d on xpad).
 *
 * normalize != 0 applies LayerNorm over C in fp32 (biased variance, eps);
 * ln_weight / ln_bias are optional (NULL = 1 / 0), fp32 or x_dtype
 * (ln_dtype).  weight [n_out, C] row-major and bias [n_out] (or NULL) are
 * in `dtype`, the compute and output type; the normalised input is rounded
 * to it once, products accumulate in fp32.  C and n_out are multiples of 16,
 * C <= 384 and 64*(C + 16/esize)*esize <= 64 KiB; every pointer 16-byte
 * aligned.
 *
 * No counterpart in the reference: it fuses the norm1 / F.pad / roll /
 * window_partition / qkv-Linear chain that torch-ext/crumpet/monai_patch.py
 * :79-97 and :153 run before the fused attention.
 */
CRUMPET_API int crumpet_window_qkv_3d(void* out, int32_t dtype,
                                      const void* x, int32_t x_dtype,
                                      int64_t B, int64_t D, int64_t H, int64_t W, int64_t C,
                                      int32_t normalize, const void* ln_weight,
                                      const void* ln_bias, int32_t ln_dtype, float eps,
                                      const void* weight, const void* bias, int64_t n_out,
                                      int64_t ws_d, int64_t ws_h, int64_t ws_w,
                                      int64_t ss_d, int64_t ss_h, int64_t ss_w,
                                      void* stream);

/*
 * Output projection of a Swin window-attention block, with the inverse
 * partition, reverse shift and crop fused into its store:
 *
 *   y[src(t), :] = windows[t, :] @ weight^T + bias       for src(t) inside y
 *
 * windows [B*nW, N, C] (window order over the volume padded to the window
 * grid, as crumpet_window_qkv_3d), y [B, D, H, W, n_out] (the caller's
 * unpadded volume; tokens in the padding are dropped).  windows, weight
 * [n_out, C], bias [n_out] (or NULL) and y share `dtype`; fp32 accumulation.
 * Same size and alignment rules as crumpet_window_qkv_3d.
 *
 * No counterpart in the reference: it fuses the proj-Linear / window_reverse
 * / roll / crop chain of torch-ext/crumpet/monai_patch.py:196-197 and
 * :98-111.
 */
CRUMPET_API int crumpet_window_proj_3d(void* y, const void* windows, int32_t dtype,
                                       int64_t B, int64_t D, int64_t H, int64_t W, int64_t C,
                                       const void* weight, const void* bias, int64_t n_out,
                                       int64_t ws_d, int64_t ws_h, int64_t ws_w,
                                       int64_t ss_d, int64_t ss_h, int64_t ss_w,
                                       void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CRUMPET_HIP_H_ */
