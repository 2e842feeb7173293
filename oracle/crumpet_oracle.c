/*
 * crumpet_oracle.c - CPU restatement of the reference's shifted-window
 * index arithmetic, used ONLY as the checker by tests/, bench.py's
 * cpu_baseline leg and __graft_entry__.smoke().  The product path never
 * links or calls it.
 *
 * Every function is a scalar, closed-form statement of the reference's
 * eager semantics, written for byte/integer exactness:
 *
 *   oracle_shift_partition_3d    torch.roll(x, -ss, dims=(1,2,3)) then the
 *                                MONAI/Swin window partition view/permute
 *                                (torch-ext/crumpet/reference.py:101-118,141-160)
 *   oracle_unshift_unpartition_3d window reverse view/permute then
 *                                torch.roll(+ss) (reference.py:121-138,163-184)
 *   oracle_attn_mask_3d          region labels 9*r_d + 3*r_h + r_w compared
 *                                pairwise inside each window
 *                                (reference.py:50-98, cuda/attn_mask_3d.cu:42-50)
 *
 * These are pinned in tests/test_oracle.py against independent
 * constructions (numpy roll + reshape/transpose, MONAI slice assignment,
 * brute-force Python loops, bijectivity, hand-checked entries).
 */
#include <stdint.h>
#include <string.h>

static int64_t mod_pos(int64_t a, int64_t m) {
    int64_t r = a % m;
    return r < 0 ? r + m : r;
}

/* Source token of window token (b, win, loc) in the rolled-by-(-ss) frame. */
static int64_t partition_source(int64_t b, int64_t win, int64_t loc, int64_t D, int64_t H,
                                int64_t W, const int64_t ws[3], const int64_t ss[3]) {
    const int64_t nWh = H / ws[1], nWw = W / ws[2];
    const int64_t wd = win / (nWh * nWw), wh = (win / nWw) % nWh, ww = win % nWw;
    const int64_t ld = loc / (ws[1] * ws[2]), lh = (loc / ws[2]) % ws[1], lw = loc % ws[2];
    /* roll(x, -s)[p] = x[(p + s) mod dim] */
    const int64_t d = mod_pos(wd * ws[0] + ld + ss[0], D);
    const int64_t h = mod_pos(wh * ws[1] + lh + ss[1], H);
    const int64_t w = mod_pos(ww * ws[2] + lw + ss[2], W);
    return ((b * D + d) * H + h) * W + w;
}

void oracle_shift_partition_3d(void* out, const void* x, int64_t B, int64_t D, int64_t H,
                               int64_t W, int64_t C, int64_t esize, const int64_t ws[3],
                               const int64_t ss[3]) {
    const int64_t nW = (D / ws[0]) * (H / ws[1]) * (W / ws[2]);
    const int64_t vol = ws[0] * ws[1] * ws[2];
    const int64_t tb = C * esize;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t win = 0; win < nW; ++win)
            for (int64_t loc = 0; loc < vol; ++loc) {
                const int64_t dst = (b * nW + win) * vol + loc;
                const int64_t src = partition_source(b, win, loc, D, H, W, ws, ss);
                memcpy((char*)out + dst * tb, (const char*)x + src * tb, (size_t)tb);
            }
}

void oracle_unshift_unpartition_3d(void* out, const void* windows, int64_t B, int64_t D,
                                   int64_t H, int64_t W, int64_t C, int64_t esize,
                                   const int64_t ws[3], const int64_t ss[3]) {
    const int64_t nW = (D / ws[0]) * (H / ws[1]) * (W / ws[2]);
    const int64_t vol = ws[0] * ws[1] * ws[2];
    const int64_t tb = C * esize;
    /* the partition is a bijection: scatter each window token back */
    for (int64_t b = 0; b < B; ++b)
        for (int64_t win = 0; win < nW; ++win)
            for (int64_t loc = 0; loc < vol; ++loc) {
                const int64_t src = (b * nW + win) * vol + loc;
                const int64_t dst = partition_source(b, win, loc, D, H, W, ws, ss);
                memcpy((char*)out + dst * tb, (const char*)windows + src * tb, (size_t)tb);
            }
}

static int region(int64_t x, int64_t dim, int64_t window, int64_t shift) {
    if (x < dim - window) return 0;
    if (x < dim - shift) return 1;
    return 2;
}

/*
 * Writes the mask as raw element bits: `neg_bits` where labels differ and 0
 * elsewhere, in elements of `esize` bytes (2 or 4).  An all-zero shift gives
 * an all-zero mask, as the reference does (reference.py:76-77).
 */
void oracle_attn_mask_3d(void* out, int64_t esize, uint32_t neg_bits, int64_t D, int64_t H,
                         int64_t W, const int64_t ws[3], const int64_t ss[3]) {
    const int64_t nWh = H / ws[1], nWw = W / ws[2];
    const int64_t nW = (D / ws[0]) * nWh * nWw;
    const int64_t vol = ws[0] * ws[1] * ws[2];
    const int shifted = ss[0] || ss[1] || ss[2];
    int labels[4096];
    for (int64_t win = 0; win < nW; ++win) {
        const int64_t wd = win / (nWh * nWw), wh = (win / nWw) % nWh, ww = win % nWw;
        for (int64_t loc = 0; loc < vol; ++loc) {
            const int64_t ld = loc / (ws[1] * ws[2]), lh = (loc / ws[2]) % ws[1], lw = loc % ws[2];
            labels[loc] = 9 * region(wd * ws[0] + ld, D, ws[0], ss[0]) +
                          3 * region(wh * ws[1] + lh, H, ws[1], ss[1]) +
                          region(ww * ws[2] + lw, W, ws[2], ss[2]);
        }
        for (int64_t i = 0; i < vol; ++i)
            for (int64_t j = 0; j < vol; ++j) {
                const uint32_t v = (shifted && labels[i] != labels[j]) ? neg_bits : 0u;
                const int64_t idx = (win * vol + i) * vol + j;
                if (esize == 2)
                    ((uint16_t*)out)[idx] = (uint16_t)v;
                else
                    ((uint32_t*)out)[idx] = v;
            }
    }
}
