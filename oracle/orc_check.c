/* orc_check.c -- checking helpers with no counterpart in the reference:
 * the fp32 input generator, exact single-entry products and Freivalds'
 * randomised check over Z_p.  Test infrastructure only (see oracle.h). */
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include "oracle.h"

void orc_fp32_rand(float *X, size_t count, uint64_t seed, int emin, int emax)
{
    uint64_t s = seed;
    unsigned span = (unsigned)(emax - emin + 1);
    for (size_t i = 0; i < count; i++) {
        uint64_t u = orc_sm64_next(&s);
        float m = 1.0f + (float)((u >> 40) & 0x7FFFFFu) * (1.0f / 8388608.0f);
        int e = emin + (int)(u % span);
        float x = ldexpf(m, e);
        X[i] = (u >> 63) ? -x : x;
    }
}

static int64_t limb_value(const uint16_t *Apl, size_t nn, int L, int u,
                          size_t e, int signed_top)
{
    uint16_t v = Apl[(size_t)u * nn + e];
    if (signed_top && u == L - 1) return (int16_t)v;
    return v;
}

void orc_entry_exact(const uint16_t *Apl, const uint16_t *Bpl, int n, int L,
                     int signed_top, int i, int j, uint16_t *limbs, int RL)
{
    size_t nn = (size_t)n * n;
    int P = 2 * L - 1;
    int64_t *col = calloc((size_t)P, sizeof(int64_t));
    if (!col) return;
    for (int k = 0; k < n; k++) {
        size_t ea = (size_t)i * n + k, eb = (size_t)k * n + j;
        for (int u = 0; u < L; u++) {
            int64_t a = limb_value(Apl, nn, L, u, ea, signed_top);
            if (!a) continue;
            for (int v = 0; v < L; v++)
                col[u + v] += a * limb_value(Bpl, nn, L, v, eb, signed_top);
        }
    }
    int64_t carry = 0;
    for (int w = 0; w < RL; w++) {
        int64_t t = carry + (w < P ? col[w] : 0);
        limbs[w] = (uint16_t)(t & 0xFFFF);
        carry = t >> 16;
    }
    free(col);
}

/* ---- arithmetic mod a 61-bit prime -------------------------------------- */
static const uint64_t PRIMES[4] = {
    2305843009213693951ULL, 2305843009213693921ULL,
    2305843009213693907ULL, 2305843009213693723ULL,
};

static inline uint64_t mulmod(uint64_t a, uint64_t b, uint64_t p)
{
    return (uint64_t)(((unsigned __int128)a * b) % p);
}
static inline uint64_t addmod(uint64_t a, uint64_t b, uint64_t p)
{
    uint64_t s = a + b;
    return s >= p ? s - p : s;
}
static inline uint64_t smod(int64_t v, uint64_t p)
{
    int64_t r = v % (int64_t)p;
    return (uint64_t)(r < 0 ? r + (int64_t)p : r);
}

/* value of every entry of a limb-plane matrix mod p (Horner from the top
 * limb; the top limb is signed when signed_top, or when `twos` the whole
 * RL-limb number is read as two's complement). */
static void entries_mod_u16(const uint16_t *pl, int n, int L, int signed_top,
                            int twos, uint64_t p, uint64_t *out)
{
    size_t nn = (size_t)n * n;
    uint64_t base = 65536 % p;
    uint64_t wrap = 1;  /* 2^(16 L) mod p */
    for (int u = 0; u < L; u++) wrap = mulmod(wrap, base, p);
    #pragma omp parallel for schedule(static)
    for (long long e = 0; e < (long long)nn; e++) {
        uint64_t acc = 0;
        for (int u = L - 1; u >= 0; u--) {
            uint16_t limb = pl[(size_t)u * nn + (size_t)e];
            int64_t v = limb;
            if (signed_top && u == L - 1) v = (int16_t)limb;
            acc = addmod(mulmod(acc, base, p), smod(v, p), p);
        }
        if (twos && (pl[(size_t)(L - 1) * nn + (size_t)e] & 0x8000))
            acc = addmod(acc, p - wrap, p);
        out[e] = acc;
    }
}

static void entries_mod_i32(const int32_t *pl, int n, int L, uint64_t p,
                            uint64_t *out)
{
    size_t nn = (size_t)n * n;
    uint64_t base = 65536 % p;
    #pragma omp parallel for schedule(static)
    for (long long e = 0; e < (long long)nn; e++) {
        uint64_t acc = 0;
        for (int u = L - 1; u >= 0; u--)
            acc = addmod(mulmod(acc, base, p), smod(pl[(size_t)u * nn + (size_t)e], p), p);
        out[e] = acc;
    }
}

static void entries_mod_i64(const int64_t *pl, int n, int P, uint64_t p,
                            uint64_t *out)
{
    size_t nn = (size_t)n * n;
    uint64_t base = 65536 % p;
    #pragma omp parallel for schedule(static)
    for (long long e = 0; e < (long long)nn; e++) {
        uint64_t acc = 0;
        for (int w = P - 1; w >= 0; w--)
            acc = addmod(mulmod(acc, base, p), smod(pl[(size_t)w * nn + (size_t)e], p), p);
        out[e] = acc;
    }
}

/* y = M r over Z_p for a dense n x n matrix of residues */
static void matvec(const uint64_t *M, const uint64_t *r, int n, uint64_t p,
                   uint64_t *y)
{
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < n; i++) {
        unsigned __int128 acc = 0;
        const uint64_t *row = M + (size_t)i * n;
        for (int k = 0; k < n; k++) {
            acc += (unsigned __int128)row[k] * r[k];
            if ((k & 31) == 31) acc %= p;
        }
        y[i] = (uint64_t)(acc % p);
    }
}

static int freivalds_core(const uint64_t *Am, const uint64_t *Bm,
                          const uint64_t *Cm, int n, uint64_t p, uint64_t seed)
{
    uint64_t *r = malloc(sizeof(uint64_t) * (size_t)n);
    uint64_t *y = malloc(sizeof(uint64_t) * (size_t)n);
    uint64_t *z = malloc(sizeof(uint64_t) * (size_t)n);
    uint64_t *w = malloc(sizeof(uint64_t) * (size_t)n);
    int ok = 0;
    if (!r || !y || !z || !w) goto out;
    uint64_t s = seed;
    for (int i = 0; i < n; i++) r[i] = orc_sm64_next(&s) % p;
    matvec(Bm, r, n, p, y);
    matvec(Am, y, n, p, z);
    matvec(Cm, r, n, p, w);
    ok = memcmp(z, w, sizeof(uint64_t) * (size_t)n) == 0;
out:
    free(r); free(y); free(z); free(w);
    return ok;
}

int orc_freivalds(const uint16_t *Apl, const uint16_t *Bpl, int n, int L,
                  int signed_top, const uint16_t *out, int RL,
                  int nprimes, uint64_t seed)
{
    size_t nn = (size_t)n * n;
    uint64_t *Am = malloc(sizeof(uint64_t) * nn);
    uint64_t *Bm = malloc(sizeof(uint64_t) * nn);
    uint64_t *Cm = malloc(sizeof(uint64_t) * nn);
    int ok = Am && Bm && Cm;
    for (int q = 0; ok && q < nprimes && q < 4; q++) {
        uint64_t p = PRIMES[q];
        entries_mod_u16(Apl, n, L, signed_top, 0, p, Am);
        entries_mod_u16(Bpl, n, L, signed_top, 0, p, Bm);
        entries_mod_u16(out, n, RL, 0, signed_top, p, Cm);
        ok = freivalds_core(Am, Bm, Cm, n, p, seed + (uint64_t)q);
    }
    free(Am); free(Bm); free(Cm);
    return ok;
}

int orc_freivalds_conv(const int32_t *A32, const int32_t *B32, int n, int L,
                       const int64_t *Cw, int nprimes, uint64_t seed)
{
    size_t nn = (size_t)n * n;
    uint64_t *Am = malloc(sizeof(uint64_t) * nn);
    uint64_t *Bm = malloc(sizeof(uint64_t) * nn);
    uint64_t *Cm = malloc(sizeof(uint64_t) * nn);
    int ok = Am && Bm && Cm;
    for (int q = 0; ok && q < nprimes && q < 4; q++) {
        uint64_t p = PRIMES[q];
        entries_mod_i32(A32, n, L, p, Am);
        entries_mod_i32(B32, n, L, p, Bm);
        entries_mod_i64(Cw, n, 2 * L - 1, p, Cm);
        ok = freivalds_core(Am, Bm, Cm, n, p, seed + (uint64_t)q);
    }
    free(Am); free(Bm); free(Cm);
    return ok;
}
