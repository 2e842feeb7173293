// Tiled layout of a 16-bit attention mask [M, N, N] for the tuned attention
// kernels (attention_kernel.h, mask kinds kMaskF16T / kMaskBF16T).
//
// In the score product a lane (col, g) of a wave holds keys 16 t + 4 g .. + 3
// of query 16 s + col for key tile t of query strip s.  Read from the
// row-major mask, one load instruction of a wave touches 16 rows; in this
// layout a lane's 4 keys of a pair of tiles (2p, 2p + 1) are 16 contiguous
// bytes and the 64 lanes' pair 1 KB:
//
//   tiles[m][s][p][16 g + col][j][r] = mask[m][min(16 s + col, N - 1)][16 (2p + j) + 4 g + r]
//
// with keys past N stored as 0 (the kernel's bias tiles carry -inf there)
// and padded query rows repeating row N - 1 (the kernels clamp those rows
// everywhere; they are never stored).  s < ceil(N / 16), p < NT / 2 for the
// kernel's tile count NT = select_tiles(N) (2 where that is 1).  The
// conversion reads the mask once and is meant to be kept with the mask by
// the caller (crumpet_amd.fused_attention keeps it per mask tensor).  The
// bits are copied, so fp16 and bf16 masks share the kernel.
#include <hip/hip_runtime.h>

#include "attention_kernel.h"
#include "crumpet_common.h"
#include "crumpet_hip.h"

namespace crumpet {
namespace {

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// One thread per (window, strip, tile, lane): 4 keys, 8 bytes of output at
// ((((m * strips + s) * NT/2 + t/2) * 64 + lane) * 2 + t % 2) * 8 bytes.
__global__ void __launch_bounds__(256)
mask_tile_kernel(u32x2_t* __restrict__ out, const uint16_t* __restrict__ mask, int64_t ms0, int64_t ms1,
                 int N, int strips, int NT, uint32_t total) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= total) return;
    // i enumerates (m, s, pair, lane, j): the output in order
    const uint32_t j = i & 1u;
    const uint32_t lane = (i >> 1) & 63u;
    uint32_t rest = i >> 7;
    const uint32_t pairs = static_cast<uint32_t>(NT) / 2u;
    const uint32_t t = 2u * (rest % pairs) + j;
    rest /= pairs;
    const uint32_t s = rest % static_cast<uint32_t>(strips);
    const uint32_t m = rest / static_cast<uint32_t>(strips);
    const int col = static_cast<int>(lane & 15u), g = static_cast<int>(lane >> 4);
    const int q = min(static_cast<int>(s) * 16 + col, N - 1);
    const int k0 = static_cast<int>(t) * 16 + 4 * g;
    const uint16_t* row = mask + int64_t(m) * ms0 + int64_t(q) * ms1;
    uint32_t h[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) h[r] = (k0 + r < N) ? row[k0 + r] : 0u;
    u32x2_t v;
    v.x = h[0] | (h[1] << 16);
    v.y = h[2] | (h[3] << 16);
    __builtin_nontemporal_store(v, out + i);
}

int tiles_shape(int64_t N, int64_t& strips, int64_t& NT) {
    if (N < 1 || N > 512) return -1;
    strips = (N + 15) / 16;
    NT = attn::select_tiles(N);
    if (NT % 2) ++NT;  // whole tile pairs (only NT = 1)
    return NT > 0 ? 0 : -1;
}

}  // namespace
}  // namespace crumpet

extern "C" int64_t crumpet_attn_mask_tiles_elements(int64_t M, int64_t N) {
    int64_t strips = 0, NT = 0;
    if (M < 0 || crumpet::tiles_shape(N, strips, NT) != 0) return -1;
    return M * strips * NT * 256;
}

extern "C" int crumpet_attn_mask_tiles(void* out, const void* mask, int32_t mask_dtype, int64_t M, int64_t N,
                                       const int64_t mask_strides[3], void* stream) {
    const char* what = "crumpet_attn_mask_tiles";
    if (mask_dtype != CRUMPET_DTYPE_F16 && mask_dtype != CRUMPET_DTYPE_BF16)
        return crumpet::fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: mask dtype must be float16 or bfloat16", what);
    int64_t strips = 0, NT = 0;
    if (M < 0 || crumpet::tiles_shape(N, strips, NT) != 0)
        return crumpet::fail(CRUMPET_ERR_UNSUPPORTED, "%s: N = %lld is outside 1 .. 512", what, (long long)N);
    if (M == 0) return CRUMPET_OK;
    if (!out || !mask || !mask_strides)
        return crumpet::fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: null pointer argument", what);
    if (mask_strides[2] != 1 || mask_strides[0] < 0 || mask_strides[1] < 0)
        return crumpet::fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: mask must have unit stride along keys", what);
    if (reinterpret_cast<uintptr_t>(out) % 8 != 0)
        return crumpet::fail(CRUMPET_ERR_INVALID_ARGUMENT, "%s: out must be 8-byte aligned", what);
    const int64_t total = M * strips * NT * 64;
    if (total > 0xffffff00LL)
        return crumpet::fail(CRUMPET_ERR_UNSUPPORTED, "%s: too many mask tiles", what);
    const uint32_t blocks = static_cast<uint32_t>((total + 255) / 256);
    hipLaunchKernelGGL(crumpet::mask_tile_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<crumpet::u32x2_t*>(out), static_cast<const uint16_t*>(mask), mask_strides[0],
                       mask_strides[1], static_cast<int>(N), static_cast<int>(strips), static_cast<int>(NT),
                       static_cast<uint32_t>(total));
    return crumpet::check_launch(what);
}
