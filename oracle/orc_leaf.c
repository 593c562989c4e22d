/* orc_leaf.c -- the n x n int32*int32 -> int64 leaf products, the schoolbook
 * limb-plane convolution and the textbook big-integer product.
 * Test infrastructure only (see oracle.h). */
#include <stdlib.h>
#include <string.h>
#include "oracle.h"

/* ikj loop, src/kernel.c:39-53. */
void orc_mm_accum_ikj(int64_t *C, const int32_t *A, const int32_t *B,
                      int n, int sign)
{
    for (int i = 0; i < n; i++) {
        int64_t *crow = C + (size_t)i * n;
        for (int k = 0; k < n; k++) {
            int64_t a = (int64_t)A[(size_t)i * n + k] * sign;
            if (!a) continue;
            const int32_t *brow = B + (size_t)k * n;
            for (int j = 0; j < n; j++) crow[j] += a * brow[j];
        }
    }
}

/* Packed, cache-blocked GEMM with a register-tiled micro-kernel: the
 * reference's `packed` leaf, src/kernel.c:89-191.  Same blocking (128 rows
 * x 128 depth per A block, 256 columns per B panel, 6 x 2-vector int64
 * register tile, int32 operands widened to int64 lanes), so its throughput
 * stands for the reference's CPU path. */
#if defined(__AVX512F__)
#define VLANES 8
#else
#define VLANES 4
#endif
typedef int64_t lv_t __attribute__((vector_size(VLANES * 8)));
typedef int64_t lvu_t __attribute__((vector_size(VLANES * 8), aligned(8)));
typedef int32_t hv_t __attribute__((vector_size(VLANES * 4), aligned(4)));

enum { BLK_M = 128, BLK_K = 128, BLK_N = 256, TILE_M = 6, TILE_N = 2 * VLANES };

static void pack_rows(int32_t *dst, const int32_t *A, int n,
                      int r0, int mc, int k0, int kc)
{
    for (int s = 0; s * TILE_M < mc; s++) {
        int32_t *d = dst + (size_t)s * TILE_M * kc;
        for (int p = 0; p < kc; p++)
            for (int r = 0; r < TILE_M; r++) {
                int row = s * TILE_M + r;
                d[p * TILE_M + r] = row < mc ? A[(size_t)(r0 + row) * n + k0 + p] : 0;
            }
    }
}

static void pack_cols(int32_t *dst, const int32_t *B, int n,
                      int c0, int nc, int k0, int kc)
{
    for (int s = 0; s * TILE_N < nc; s++) {
        int32_t *d = dst + (size_t)s * TILE_N * kc;
        for (int p = 0; p < kc; p++)
            for (int c = 0; c < TILE_N; c++) {
                int col = s * TILE_N + c;
                d[p * TILE_N + c] = col < nc ? B[(size_t)(k0 + p) * n + c0 + col] : 0;
            }
    }
}

static void tile_kernel(const int32_t *restrict ap, const int32_t *restrict bp,
                        int64_t *C, int ldc, int kc, int mr, int nr, int sign)
{
    lv_t acc[TILE_M][2];
    for (int r = 0; r < TILE_M; r++) {
        acc[r][0] = (lv_t){0};
        acc[r][1] = (lv_t){0};
    }
    for (int p = 0; p < kc; p++) {
        lv_t b0 = __builtin_convertvector(*(const hv_t *)(bp + p * TILE_N), lv_t);
        lv_t b1 = __builtin_convertvector(*(const hv_t *)(bp + p * TILE_N + VLANES), lv_t);
        for (int r = 0; r < TILE_M; r++) {
            lv_t a = (lv_t){0} + (int64_t)ap[p * TILE_M + r];
            acc[r][0] += a * b0;
            acc[r][1] += a * b1;
        }
    }
    int64_t tile[TILE_M][TILE_N];
    for (int r = 0; r < TILE_M; r++) {
        *(lvu_t *)&tile[r][0] = acc[r][0];
        *(lvu_t *)&tile[r][VLANES] = acc[r][1];
    }
    for (int r = 0; r < mr; r++)
        for (int c = 0; c < nr; c++)
            C[(size_t)r * ldc + c] += sign > 0 ? tile[r][c] : -tile[r][c];
}

void orc_mm_accum_packed(int64_t *C, const int32_t *A, const int32_t *B,
                         int n, int sign)
{
    int32_t *pa = malloc(sizeof(int32_t) * (size_t)(BLK_M / TILE_M + 1) * TILE_M * BLK_K);
    int32_t *pb = malloc(sizeof(int32_t) * (size_t)(BLK_N / TILE_N + 1) * TILE_N * BLK_K);
    if (!pa || !pb) {
        free(pa); free(pb);
        orc_mm_accum_ikj(C, A, B, n, sign);
        return;
    }
    for (int c0 = 0; c0 < n; c0 += BLK_N) {
        int nc = n - c0 < BLK_N ? n - c0 : BLK_N;
        for (int k0 = 0; k0 < n; k0 += BLK_K) {
            int kc = n - k0 < BLK_K ? n - k0 : BLK_K;
            pack_cols(pb, B, n, c0, nc, k0, kc);
            for (int r0 = 0; r0 < n; r0 += BLK_M) {
                int mc = n - r0 < BLK_M ? n - r0 : BLK_M;
                pack_rows(pa, A, n, r0, mc, k0, kc);
                for (int c = 0; c < nc; c += TILE_N) {
                    int nr = nc - c < TILE_N ? nc - c : TILE_N;
                    for (int r = 0; r < mc; r += TILE_M) {
                        int mr = mc - r < TILE_M ? mc - r : TILE_M;
                        tile_kernel(pa + (size_t)(r / TILE_M) * TILE_M * kc,
                                    pb + (size_t)(c / TILE_N) * TILE_N * kc,
                                    C + (size_t)(r0 + r) * n + c0 + c,
                                    n, kc, mr, nr, sign);
                    }
                }
            }
        }
    }
    free(pa); free(pb);
}

static void leaf_accum(int64_t *C, const int32_t *A, const int32_t *B,
                       int n, int sign, int leaf)
{
    if (leaf == 2) orc_mm_accum_packed(C, A, B, n, sign);
    else           orc_mm_accum_ikj(C, A, B, n, sign);
}

/* src/methods.c:94-104: Cw[u+v] += A_u * B_v over all L^2 limb pairs. */
void orc_conv_limbplane(int64_t *Cw, const int32_t *A32, const int32_t *B32,
                        int n, int L, int leaf)
{
    size_t nn = (size_t)n * n;
    memset(Cw, 0, sizeof(int64_t) * (size_t)(2 * L - 1) * nn);
    for (int u = 0; u < L; u++)
        for (int v = 0; v < L; v++)
            leaf_accum(Cw + (size_t)(u + v) * nn, A32 + (size_t)u * nn,
                       B32 + (size_t)v * nn, n, 1, leaf);
}

/* src/methods.c:106-123 */
void orc_mm_limbplane(const uint16_t *Apl, const uint16_t *Bpl, int n, int L,
                      uint16_t *out, int RL, int leaf)
{
    size_t nn = (size_t)n * n, tot = (size_t)L * nn;
    int32_t *a = malloc(sizeof(int32_t) * tot);
    int32_t *b = malloc(sizeof(int32_t) * tot);
    int64_t *cw = malloc(sizeof(int64_t) * (size_t)(2 * L - 1) * nn);
    if (!a || !b || !cw) { free(a); free(b); free(cw); return; }
    for (size_t i = 0; i < tot; i++) { a[i] = Apl[i]; b[i] = Bpl[i]; }
    orc_conv_limbplane(cw, a, b, n, L, leaf);
    orc_normalize_planes(cw, 2 * L - 1, n, out, RL);
    free(a); free(b); free(cw);
}

/* src/methods.c:22-52: per output entry, schoolbook L x L limb products
 * summed over k into 2L uint64 columns, then one carry pass.  Inputs are
 * entry-major. */
void orc_mm_bigint_ijk(const uint16_t *Aem, const uint16_t *Bem, int n, int L,
                       uint16_t *out, int RL)
{
    int P = 2 * L;
    size_t nn = (size_t)n * n;
    uint64_t *col = malloc(sizeof(uint64_t) * (size_t)P);
    if (!col) return;
    for (int i = 0; i < n; i++)
        for (int j = 0; j < n; j++) {
            memset(col, 0, sizeof(uint64_t) * (size_t)P);
            for (int k = 0; k < n; k++) {
                const uint16_t *a = Aem + ((size_t)i * n + k) * L;
                const uint16_t *b = Bem + ((size_t)k * n + j) * L;
                for (int u = 0; u < L; u++) {
                    uint64_t au = a[u];
                    if (!au) continue;
                    for (int v = 0; v < L; v++) col[u + v] += au * b[v];
                }
            }
            uint64_t carry = 0;
            for (int w = 0; w < RL; w++) {
                uint64_t v = carry + (w < P ? col[w] : 0);
                out[(size_t)w * nn + (size_t)i * n + j] = (uint16_t)(v & 0xFFFF);
                carry = v >> ORC_LIMB_BITS;
            }
        }
    free(col);
}
