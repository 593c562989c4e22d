/* orc_fpx.c -- fp32 / fp64 <-> fixed-point limb planes (src/fpfixed.c).
 * Test infrastructure only (see oracle.h).
 *
 * Every finite nonzero fp32 x is mi * 2^e2 with mi in [2^23, 2^24) (fp64:
 * [2^52, 2^53)).  On a grid of scale 2^S the integer x * 2^S is mi shifted
 * left by e2 + S; that shifted significand is written straight into (at
 * most) three (fp64: five) signed base-2^16 limbs.  The exact product comes
 * back at scale 2^(SA+SB); the decoders gather the top <= 4 limbs of its
 * magnitude and round that window to 24 / 53 / 63 bits, half-even with a
 * sticky bit for everything below the window (a window that already has no
 * more bits than that is kept as it is). */
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include "oracle.h"

static int next_pow2(int x) { int r = 1; while (r < x) r <<= 1; return r; }

/* src/fpfixed.c:40-54 */
static void exp_range(const float *X, size_t cnt, int *lo, int *hi, int *any)
{
    int l = 1 << 30, h = -(1 << 30), seen = 0;
    for (size_t i = 0; i < cnt; i++) {
        float x = X[i];
        if (x == 0.0f || !isfinite(x)) continue;
        int e;
        frexpf(x, &e);
        if (e - 24 < l) l = e - 24;
        if (e - 24 > h) h = e - 24;
        seen = 1;
    }
    if (!seen) { l = 0; h = 0; }
    *lo = l; *hi = h; *any = seen;
}

/* src/fpfixed.c:115-129 */
static void exp_range_d(const double *X, size_t cnt, int *lo, int *hi, int *any)
{
    int l = 1 << 30, h = -(1 << 30), seen = 0;
    for (size_t i = 0; i < cnt; i++) {
        double x = X[i];
        if (x == 0.0 || !isfinite(x)) continue;
        int e;
        frexp(x, &e);
        if (e - 53 < l) l = e - 53;
        if (e - 53 > h) h = e - 53;
        seen = 1;
    }
    if (!seen) { l = 0; h = 0; }
    *lo = l; *hi = h; *any = seen;
}

static int setup(orc_fpx *c, int n, int loA, int hiA, int loB, int hiB,
                 int anyA, int anyB, int sig, int wr, int force_bits);

/* src/fpfixed.c:59-108 (fp32: 24-bit significand, touches <= 3 limbs). */
int orc_fpx_init(orc_fpx *c, const float *A, const float *B, int n,
                 int force_bits)
{
    size_t nn = (size_t)n * n;
    int loA, hiA, loB, hiB, anyA, anyB;
    exp_range(A, nn, &loA, &hiA, &anyA);
    exp_range(B, nn, &loB, &hiB, &anyB);
    return setup(c, n, loA, hiA, loB, hiB, anyA, anyB, 24, 3, force_bits);
}

/* src/fpfixed.c:131-142 (fp64: 53-bit significand, touches <= 5 limbs). */
int orc_fpx_init_d(orc_fpx *c, const double *A, const double *B, int n,
                   int force_bits)
{
    size_t nn = (size_t)n * n;
    int loA, hiA, loB, hiB, anyA, anyB;
    exp_range_d(A, nn, &loA, &hiA, &anyA);
    exp_range_d(B, nn, &loB, &hiB, &anyB);
    return setup(c, n, loA, hiA, loB, hiB, anyA, anyB, 53, 5, force_bits);
}

/* src/fpfixed.c:59-94 */
static int setup(orc_fpx *c, int n, int loA, int hiA, int loB, int hiB,
                 int anyA, int anyB, int sig, int wr, int force_bits)
{
    size_t nn = (size_t)n * n;
    memset(c, 0, sizeof *c);
    c->spreadA = anyA ? hiA - loA : 0;
    c->spreadB = anyB ? hiB - loB : 0;
    int L;
    if (force_bits > 0) {
        c->SA = c->SB = force_bits / 2;
        L = next_pow2(force_bits / ORC_LIMB_BITS);
    } else {
        c->SA = -loA;
        c->SB = -loB;
        int spread = c->spreadA > c->spreadB ? c->spreadA : c->spreadB;
        int bits = sig + spread + 1;
        int need = (bits + ORC_LIMB_BITS - 1) / ORC_LIMB_BITS;
        int need2 = spread / ORC_LIMB_BITS + wr;
        L = next_pow2(need > need2 ? need : need2);
        if (L < 2) L = 2;
    }
    c->n = n; c->L = L;
    /* src/fpfixed.c:84-88: refuse sizes whose int64 accumulators could
     * overflow. */
    if ((double)n * L * 65535.0 * 65535.0 > 4.0e18) return -1;
    c->A32 = calloc((size_t)L * nn, sizeof(int32_t));
    c->B32 = calloc((size_t)L * nn, sizeof(int32_t));
    c->Cw = calloc((size_t)(2 * L - 1) * nn, sizeof(int64_t));
    if (!c->A32 || !c->B32 || !c->Cw) { orc_fpx_free(c); return -1; }
    return 0;
}

/* src/fpfixed.c:175-193: zero, Inf and NaN are skipped; an offset below the
 * grid drops the value; limbs at or above L are dropped. */
static void encode_one(int32_t *planes, size_t nn, size_t idx, float x,
                       int L, int S)
{
    if (x == 0.0f || !isfinite(x)) return;
    int e;
    float m = frexpf(x, &e);
    int32_t mi = (int32_t)(fabsf(m) * 16777216.0f);
    int off = e - 24 + S;
    if (off < 0) return;
    int lo = off >> 4, sh = off & 15;
    uint64_t v = (uint64_t)mi << sh;
    int sgn = x < 0.0f ? -1 : 1;
    for (int t = 0; t < 3 && lo + t < L; t++)
        planes[(size_t)(lo + t) * nn + idx] = sgn * (int32_t)((v >> (16 * t)) & 0xFFFFu);
}

/* src/fpfixed.c:144-162: the 53-bit significand shifted by up to 15 bits
 * needs 68 bits, kept as a (high, low) pair of 64-bit words */
static void encode_one_d(int32_t *planes, size_t nn, size_t idx, double x,
                         int L, int S)
{
    if (x == 0.0 || !isfinite(x)) return;
    int e;
    double m = frexp(x, &e);
    uint64_t mi = (uint64_t)(fabs(m) * 9007199254740992.0);
    int off = e - 53 + S;
    if (off < 0) return;
    int lo = off >> 4, sh = off & 15;
    uint64_t w0 = mi << sh, w1 = sh ? mi >> (64 - sh) : 0;
    int sgn = x < 0.0 ? -1 : 1;
    for (int t = 0; t < 5 && lo + t < L; t++) {
        uint64_t part = t < 4 ? w0 >> (16 * t) : w1;
        planes[(size_t)(lo + t) * nn + idx] = sgn * (int32_t)(part & 0xFFFFu);
    }
}

/* src/fpfixed.c:164-173 */
void orc_fpx_encode_d(orc_fpx *c, const double *A, const double *B)
{
    size_t nn = (size_t)c->n * c->n;
    memset(c->A32, 0, sizeof(int32_t) * (size_t)c->L * nn);
    memset(c->B32, 0, sizeof(int32_t) * (size_t)c->L * nn);
    for (size_t i = 0; i < nn; i++) encode_one_d(c->A32, nn, i, A[i], c->L, c->SA);
    for (size_t i = 0; i < nn; i++) encode_one_d(c->B32, nn, i, B[i], c->L, c->SB);
}

void orc_fpx_encode(orc_fpx *c, const float *A, const float *B)
{
    size_t nn = (size_t)c->n * c->n;
    memset(c->A32, 0, sizeof(int32_t) * (size_t)c->L * nn);
    memset(c->B32, 0, sizeof(int32_t) * (size_t)c->L * nn);
    for (size_t i = 0; i < nn; i++) encode_one(c->A32, nn, i, A[i], c->L, c->SA);
    for (size_t i = 0; i < nn; i++) encode_one(c->B32, nn, i, B[i], c->L, c->SB);
}

/* src/fpfixed.c:212-251: carry over 2L+2 limbs with an arithmetic shift;
 * a negative result is negated in two's complement; then the top <= 4
 * nonzero limbs and a sticky bit for everything below. Returns the sign
 * (0 for an exact zero). */
static int extract(const int64_t *Cw, int L, size_t nn, size_t idx,
                   int32_t *limb, uint64_t *top, int *tb, int *shift,
                   int *sticky)
{
    int RL = 2 * L + 2, P = 2 * L - 1;
    int64_t carry = 0;
    for (int w = 0; w < RL; w++) {
        int64_t t = carry + (w < P ? Cw[(size_t)w * nn + idx] : 0);
        limb[w] = (int32_t)(t & 0xFFFF);
        carry = t >> ORC_LIMB_BITS;
    }
    int neg = carry < 0;
    if (neg) {
        int32_t borrow = 1;
        for (int w = 0; w < RL; w++) {
            int32_t t = (~limb[w] & 0xFFFF) + borrow;
            limb[w] = t & 0xFFFF;
            borrow = t >> ORC_LIMB_BITS;
        }
    }
    int h = -1;
    for (int w = RL - 1; w >= 0; w--) if (limb[w]) { h = w; break; }
    if (h < 0) return 0;
    int bl = 0;
    for (int32_t v = limb[h]; v; v >>= 1) bl++;
    int k = h + 1 < 4 ? h + 1 : 4;
    uint64_t acc = 0;
    for (int w = h; w > h - k; w--) acc = (acc << 16) | (uint64_t)limb[w];
    int base = 16 * (h - k + 1);
    int st = 0;
    for (int w = h - k; w >= 0; w--) if (limb[w]) { st = 1; break; }
    *top = acc; *tb = 16 * h + bl - base; *shift = base; *sticky = st;
    return neg ? -1 : 1;
}

/* src/fpfixed.c:253-267: round-half-even with a sticky bit. */
static uint64_t round_sig(uint64_t top, int tb, int bits, int sticky, int *shift)
{
    if (tb <= bits) return top;
    int drop = tb - bits;
    uint64_t sig = top >> drop;
    uint64_t rem = top & ((1ULL << drop) - 1);
    uint64_t half = 1ULL << (drop - 1);
    int up = rem > half ? 1 : rem < half ? 0 : (sticky ? 1 : (int)(sig & 1));
    sig += (uint64_t)up;
    if (sig >> bits) { sig >>= 1; drop++; }
    *shift += drop;
    return sig;
}

/* src/fpfixed.c:269-285: exact zero decodes to +0.0f. */
void orc_fpx_decode_f32_from(const orc_fpx *c, const int64_t *Cw, float *C)
{
    size_t nn = (size_t)c->n * c->n;
    int32_t *limb = malloc(sizeof(int32_t) * (size_t)(2 * c->L + 2));
    int S = c->SA + c->SB;
    if (!limb) return;
    for (size_t i = 0; i < nn; i++) {
        uint64_t top; int tb, shift, sticky;
        int sgn = extract(Cw, c->L, nn, i, limb, &top, &tb, &shift, &sticky);
        if (!sgn) { C[i] = 0.0f; continue; }
        uint64_t sig = round_sig(top, tb, 24, sticky, &shift);
        C[i] = (float)sgn * ldexpf((float)sig, shift - S);
    }
    free(limb);
}

void orc_fpx_decode_f32(const orc_fpx *c, float *C)
{
    orc_fpx_decode_f32_from(c, c->Cw, C);
}

/* src/fpfixed.c:308-322 */
void orc_fpx_decode_f64_from(const orc_fpx *c, const int64_t *Cw, double *C)
{
    size_t nn = (size_t)c->n * c->n;
    int32_t *limb = malloc(sizeof(int32_t) * (size_t)(2 * c->L + 2));
    int S = c->SA + c->SB;
    if (!limb) return;
    for (size_t i = 0; i < nn; i++) {
        uint64_t top; int tb, shift, sticky;
        int sgn = extract(Cw, c->L, nn, i, limb, &top, &tb, &shift, &sticky);
        if (!sgn) { C[i] = 0.0; continue; }
        uint64_t sig = round_sig(top, tb, 53, sticky, &shift);
        C[i] = (double)sgn * ldexp((double)sig, shift - S);
    }
    free(limb);
}

/* src/fpfixed.c:292-306, as a signed 63-bit significand and an exponent:
 * the reference's long double is sig * 2^ex (exact in x87 extended) */
void orc_fpx_decode_sig63_from(const orc_fpx *c, const int64_t *Cw, int64_t *sig,
                               int32_t *ex)
{
    size_t nn = (size_t)c->n * c->n;
    int32_t *limb = malloc(sizeof(int32_t) * (size_t)(2 * c->L + 2));
    int S = c->SA + c->SB;
    if (!limb) return;
    for (size_t i = 0; i < nn; i++) {
        uint64_t top; int tb, shift, sticky;
        int sgn = extract(Cw, c->L, nn, i, limb, &top, &tb, &shift, &sticky);
        if (!sgn) { sig[i] = 0; ex[i] = 0; continue; }
        uint64_t s63 = round_sig(top, tb, 63, sticky, &shift);
        sig[i] = sgn * (int64_t)s63;
        ex[i] = shift - S;
    }
    free(limb);
}

/* src/fpfixed.c:324-328 */
void orc_fpx_free(orc_fpx *c)
{
    free(c->A32); free(c->B32); free(c->Cw);
    c->A32 = NULL; c->B32 = NULL; c->Cw = NULL;
}

/* src/mlgemm.c:593-630 */
int orc_faithful_window(const orc_fpx *c, int max_keep, int *u0, int *hi)
{
    const size_t nn = (size_t)c->n * c->n;
    int top = -1;
    for (int w = c->L - 1; w >= 0 && top < 0; w--)
        for (size_t i = 0; i < nn; i++)
            if (c->A32[(size_t)w * nn + i] != 0 || c->B32[(size_t)w * nn + i] != 0) {
                top = w;
                break;
            }
    if (top < 0) top = c->L - 1;
    /* the largest power of two within max_keep, the live span and L; two
       limbs at least when both are allowed; one for max_keep <= 1 */
    int Lk = 1;
    if (max_keep >= 2) {
        while (2 * Lk <= max_keep && 2 * Lk <= top + 1 && 2 * Lk <= c->L) Lk *= 2;
        if (Lk == 1 && top >= 1 && c->L >= 2) Lk = 2;
    }
    *u0 = top - Lk + 1 < 0 ? 0 : top - Lk + 1;
    *hi = top;
    return Lk;
}

/* src/mlgemm.c:909-961, 1186-1250 */
int orc_faithful_cw(const orc_fpx *c, int max_keep, int64_t *Cw, int *u0)
{
    int hi;
    const int Lk = orc_faithful_window(c, max_keep, u0, &hi);
    const size_t nn = (size_t)c->n * c->n;
    memset(Cw, 0, (size_t)(2 * c->L - 1) * nn * sizeof(int64_t));
    orc_conv_limbplane(Cw + (size_t)(2 * *u0) * nn, c->A32 + (size_t)*u0 * nn,
                       c->B32 + (size_t)*u0 * nn, c->n, Lk, 2);
    return Lk;
}
