/* orc_mfft.c -- flat MFFT plan, ring transforms and conv_mfft / mm_mfft.
 * Test infrastructure only (see oracle.h).
 *
 * Ring R = Z[y]/(y^K + 1), elements stored in the power basis; multiplying
 * by y^e is a negacyclic shift of the coefficient vector.  The length-NB
 * transform uses omega = y^g with g = 2K/NB, so omega^(NB/2) = y^K = -1. */
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <time.h>
#include "oracle.h"

static double wall(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static int lg2(int x) { int r = 0; while ((1 << r) < x) r++; return r; }

/* src/mfft.c:77-95: sigma = floor(log2 L)/2 unless overridden, S = 2^sigma,
 * NB = 2L/S, K = 2S, g = 2K/NB; rejected unless L is a power of two and
 * NB divides 2K. */
int orc_plan_init(orc_plan *p, int L, int sigma_override)
{
    if (L < 2 || (L & (L - 1))) return -1;
    int l = lg2(L);
    int sigma = sigma_override > 0 ? sigma_override : l / 2;
    if (sigma < 1) sigma = 1;
    if (sigma > l) return -1;
    int S = 1 << sigma, NB = 2 * L / S, K = 2 * S;
    if (2 * S * S < L || (2 * K) % NB || NB < 2) return -1;
    p->L = L; p->S = S; p->NB = NB; p->K = K; p->g = 2 * K / NB;
    p->nprod = (long long)NB * K * K;
    return 0;
}

/* src/mfft.c:102-110: 3 log2 NB + log2 K + log2 n + 2*16. */
double orc_plan_maxbits(const orc_plan *p, int n)
{
    return 3.0 * log2((double)p->NB) + log2((double)p->K) + log2((double)n)
         + 2.0 * ORC_LIMB_BITS;
}

/* (y^e * x)[.] for one K-vector, e taken mod 2K. */
static void ring_shift_acc(int64_t *dst, const int64_t *x, int K, int e, int64_t scale)
{
    int m = 2 * K;
    e %= m; if (e < 0) e += m;
    for (int c = 0; c < K; c++) {
        int t = c + e, neg = 0;
        while (t >= K) { t -= K; neg ^= 1; }
        dst[t] += neg ? -scale * x[c] : scale * x[c];
    }
}

void orc_ring_dft(int64_t *X, const int64_t *x, int NB, int K, int g, int dir)
{
    memset(X, 0, sizeof(int64_t) * (size_t)NB * K);
    for (int j = 0; j < NB; j++)
        for (int b = 0; b < NB; b++) {
            long long e = (long long)dir * g * j * b;
            int m = 2 * K;
            int ee = (int)(((e % m) + m) % m);
            ring_shift_acc(X + (size_t)j * K, x + (size_t)b * K, K, ee, 1);
        }
}

/* Gentleman-Sande forward transform over planes, natural -> bit-reversed.
 * Butterfly (src/mfft.c:173-258): u' = u + v, v' = (u - v) * y^e with
 * e = g*t*(NB/len) mod 2K, stages len = NB, NB/2, ..., 2. */
void orc_fft_forward32(int32_t *X, int NB, int K, int g, size_t nn)
{
    int32_t *tmp = malloc(sizeof(int32_t) * (size_t)K * nn);
    if (!tmp) abort();
    for (int len = NB; len >= 2; len >>= 1) {
        int h = len / 2, step = NB / len;
        for (int j0 = 0; j0 < NB; j0 += len)
            for (int t = 0; t < h; t++) {
                int e = (int)(((long long)g * t * step) % (2 * K));
                int32_t *P = X + (size_t)(j0 + t) * K * nn;
                int32_t *Q = X + (size_t)(j0 + t + h) * K * nn;
                for (int c = 0; c < K; c++) {
                    int32_t *pc = P + (size_t)c * nn, *qc = Q + (size_t)c * nn;
                    int32_t *dc = tmp + (size_t)c * nn;
                    for (size_t i = 0; i < nn; i++) {
                        int32_t a = pc[i], b = qc[i];
                        pc[i] = a + b;
                        dc[i] = a - b;
                    }
                }
                for (int c = 0; c < K; c++) {
                    int tg = c + e, neg = 0;
                    while (tg >= K) { tg -= K; neg ^= 1; }
                    int32_t *qc = Q + (size_t)tg * nn;
                    const int32_t *dc = tmp + (size_t)c * nn;
                    if (neg) for (size_t i = 0; i < nn; i++) qc[i] = -dc[i];
                    else     for (size_t i = 0; i < nn; i++) qc[i] = dc[i];
                }
            }
    }
    free(tmp);
}

/* Cooley-Tukey inverse, bit-reversed -> natural, conjugate twiddles
 * (src/mfft.c:260-299): w = v * y^(-e); u' = u + w, v' = u - w; stages
 * len = 2, 4, ..., NB.  Result is NB times the inverse DFT. */
void orc_fft_inverse64(int64_t *X, int NB, int K, int g, size_t nn)
{
    int64_t *tmp = malloc(sizeof(int64_t) * (size_t)K * nn);
    if (!tmp) abort();
    int m = 2 * K;
    for (int len = 2; len <= NB; len <<= 1) {
        int h = len / 2, step = NB / len;
        for (int j0 = 0; j0 < NB; j0 += len)
            for (int t = 0; t < h; t++) {
                int e = (int)(((long long)g * t * step) % m);
                e = (m - e) % m;
                int64_t *P = X + (size_t)(j0 + t) * K * nn;
                int64_t *Q = X + (size_t)(j0 + t + h) * K * nn;
                for (int c = 0; c < K; c++) {
                    int tg = c + e, neg = 0;
                    while (tg >= K) { tg -= K; neg ^= 1; }
                    const int64_t *qc = Q + (size_t)c * nn;
                    int64_t *dc = tmp + (size_t)tg * nn;
                    if (neg) for (size_t i = 0; i < nn; i++) dc[i] = -qc[i];
                    else     for (size_t i = 0; i < nn; i++) dc[i] = qc[i];
                }
                for (int c = 0; c < K; c++) {
                    int64_t *pc = P + (size_t)c * nn, *qc = Q + (size_t)c * nn;
                    const int64_t *dc = tmp + (size_t)c * nn;
                    for (size_t i = 0; i < nn; i++) {
                        int64_t a = pc[i], w = dc[i];
                        pc[i] = a + w;
                        qc[i] = a - w;
                    }
                }
            }
    }
    free(tmp);
}

static void leaf(int64_t *C, const int32_t *A, const int32_t *B, int n,
                 int sign, int which)
{
    if (which == 2) orc_mm_accum_packed(C, A, B, n, sign);
    else            orc_mm_accum_ikj(C, A, B, n, sign);
}

/* One conv_mfft (src/mfft.c:302-422) with an optional cap on the pointwise
 * products run (-1 = all).  Stage seconds go to secs[0..2] if non-NULL. */
static long long conv_mfft_impl(int64_t *Cout, const int32_t *A32,
                                const int32_t *B32, int n, int L,
                                const orc_plan *p, int which,
                                long long cap, double *secs)
{
    size_t nn = (size_t)n * n;
    int NB = p->NB, K = p->K, S = p->S, g = p->g;
    size_t planes = (size_t)NB * K;
    int32_t *Ah = calloc(planes * nn, sizeof(int32_t));
    int32_t *Bh = calloc(planes * nn, sizeof(int32_t));
    int64_t *Ch = calloc(planes * nn, sizeof(int64_t));
    int64_t *Cw = calloc((size_t)(2 * L + S) * nn, sizeof(int64_t));
    long long ran = 0;
    if (!Ah || !Bh || !Ch || !Cw) goto out;

    double t0 = wall();
    /* pack: block b < L/S, ring coefficient c < S <- limb b*S + c
     * (mfft.c:322-336); the rest stays zero so the cyclic, negacyclic
     * convolution equals the linear one. */
    for (int b = 0; b < L / S; b++)
        for (int c = 0; c < S; c++) {
            size_t dst = ((size_t)b * K + c) * nn, src = (size_t)(b * S + c) * nn;
            memcpy(Ah + dst, A32 + src, sizeof(int32_t) * nn);
            memcpy(Bh + dst, B32 + src, sizeof(int32_t) * nn);
        }
    orc_fft_forward32(Ah, NB, K, g, nn);
    orc_fft_forward32(Bh, NB, K, g, nn);
    double t1 = wall();

    /* pointwise: Ch[b][(c1+c2) mod K] += +-Ah[b][c1] Bh[b][c2], minus on
     * wrap (mfft.c:383-395). */
    for (int b = 0; b < NB; b++)
        for (int c1 = 0; c1 < K; c1++)
            for (int c2 = 0; c2 < K; c2++) {
                if (cap >= 0 && ran >= cap) goto pw_done;
                int t = c1 + c2, sgn = 1;
                if (t >= K) { t -= K; sgn = -1; }
                leaf(Ch + ((size_t)b * K + t) * nn, Ah + ((size_t)b * K + c1) * nn,
                     Bh + ((size_t)b * K + c2) * nn, n, sgn, which);
                ran++;
            }
pw_done:;
    double t2 = wall();

    orc_fft_inverse64(Ch, NB, K, g, nn);
    /* fold: Cw[b*S + c] += Ch[b][c] / NB, exact (mfft.c:407-418) */
    for (int b = 0; b < NB; b++)
        for (int c = 0; c < K; c++) {
            int64_t *dst = Cw + (size_t)(b * S + c) * nn;
            const int64_t *src = Ch + ((size_t)b * K + c) * nn;
            for (size_t i = 0; i < nn; i++) dst[i] += src[i] / NB;
        }
    memcpy(Cout, Cw, sizeof(int64_t) * (size_t)(2 * L - 1) * nn);
    double t3 = wall();
    if (secs) { secs[0] = t1 - t0; secs[1] = t2 - t1; secs[2] = t3 - t2; }
out:
    free(Ah); free(Bh); free(Ch); free(Cw);
    return ran;
}

void orc_conv_mfft(int64_t *Cw, const int32_t *A32, const int32_t *B32,
                   int n, int L, const orc_plan *p, int which)
{
    conv_mfft_impl(Cw, A32, B32, n, L, p, which, -1, NULL);
}

/* src/mfft.c:424-438: widen u16 -> int32, conv, normalize 2L-1 planes. */
void orc_mm_mfft(const uint16_t *Apl, const uint16_t *Bpl, int n, int L,
                 const orc_plan *p, uint16_t *out, int RL, int which)
{
    size_t nn = (size_t)n * n, tot = (size_t)L * nn;
    int32_t *a = malloc(sizeof(int32_t) * tot);
    int32_t *b = malloc(sizeof(int32_t) * tot);
    int64_t *cw = calloc((size_t)(2 * L - 1) * nn, sizeof(int64_t));
    if (!a || !b || !cw) { free(a); free(b); free(cw); return; }
    for (size_t i = 0; i < tot; i++) { a[i] = Apl[i]; b[i] = Bpl[i]; }
    orc_conv_mfft(cw, a, b, n, L, p, which);
    orc_normalize_planes(cw, 2 * L - 1, n, out, RL);
    free(a); free(b); free(cw);
}

long long orc_mm_mfft_sampled(const uint16_t *Apl, const uint16_t *Bpl, int n,
                              int L, const orc_plan *p, uint16_t *out, int RL,
                              long long nprod_sample, double secs[4])
{
    size_t nn = (size_t)n * n, tot = (size_t)L * nn;
    int32_t *a = malloc(sizeof(int32_t) * tot);
    int32_t *b = malloc(sizeof(int32_t) * tot);
    int64_t *cw = calloc((size_t)(2 * L - 1) * nn, sizeof(int64_t));
    long long ran = -1;
    if (!a || !b || !cw) goto out;
    double t0 = wall();
    for (size_t i = 0; i < tot; i++) { a[i] = Apl[i]; b[i] = Bpl[i]; }
    double t1 = wall();
    ran = conv_mfft_impl(cw, a, b, n, L, p, 2, nprod_sample, secs);
    secs[0] += t1 - t0;
    double t2 = wall();
    orc_normalize_planes(cw, 2 * L - 1, n, out, RL);
    secs[3] = wall() - t2;
out:
    free(a); free(b); free(cw);
    return ran;
}
