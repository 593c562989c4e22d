/* mfftbench_api.c -- the reference-named C API (include/mfftbench.h) over
 * the gfx950 shim (include/mfft_hip.h).
 *
 * Products run only on the device.  Errors follow the reference's
 * conventions (src/mfft.c:317-320, 432): a message on stderr and the output
 * left untouched; the code is kept for mfft_last_error().  Each call owns
 * nothing between calls except one cached device context per thread-free
 * process-wide slot (keyed by n, L and the plan), which saves re-allocating
 * the workspace when a caller repeats a shape. */
#define _GNU_SOURCE
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "mfft_hip.h"
#include "mfftbench.h"

static __thread int t_last_error;
static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;
static mfh_ctx *g_ctx;
static int g_key[4];

long long g_kernel_calls;
int g_mfft_profile;
mfft_profile_t g_mfft_prof;

void mfft_profile_reset(void) { memset(&g_mfft_prof, 0, sizeof g_mfft_prof); }

/* src/mfft.c:51-73: the same report */
void mfft_profile_print(const char *label)
{
    const mfft_profile_t *p = &g_mfft_prof;
    double tot = p->pack + p->build_ops + p->transform + p->pointwise + p->fold;
    if (tot <= 0) tot = 1e-30;
    printf("profile %s:\n"
           "  pack        %8.4f s  (%5.1f%%)\n"
           "  build_ops   %8.4f s  (%5.1f%%)  calls %lld\n"
           "  transform   %8.4f s  (%5.1f%%)  fft runs %lld\n"
           "  pointwise   %8.4f s  (%5.1f%%)\n"
           "  fold        %8.4f s  (%5.1f%%)\n"
           "  total       %8.4f s\n",
           label ? label : "mfft", p->pack, 100.0 * p->pack / tot, p->build_ops,
           100.0 * p->build_ops / tot, p->n_build, p->transform, 100.0 * p->transform / tot,
           p->n_fft, p->pointwise, 100.0 * p->pointwise / tot, p->fold,
           100.0 * p->fold / tot, tot);
}

/* stage times of the product just run on `c` into g_mfft_prof */
static void profile_add(mfh_ctx *c)
{
    float ms[5];
    if (mfh_stage_times(c, ms) != MFH_OK) return;
    g_mfft_prof.transform += (ms[0] + ms[2] + ms[3]) * 1e-3;
    g_mfft_prof.pointwise += ms[1] * 1e-3;
    g_mfft_prof.n_fft += 3;
}

int mfft_last_error(void) { return t_last_error; }
const char *mfft_strerror(int code) { return mfh_strerror(code); }

static int fail(const char *what, int code)
{
    t_last_error = code;
    fprintf(stderr, "mfft-hip: %s: %s\n", what, mfh_strerror(code));
    return code;
}

/* src/kernel.c:16-36 */
static const char *knames[KERNEL__COUNT] = {
    "ikj", "blocked", "packed", "strassen", "winograd", "bitplane",
    "convk", "convkara", "boolpack", "bitpack", "boolstrassen", "booltiled",
    "hip"};

const char *kernel_name(kernel_t k)
{
    if ((int)k < 0 || k >= KERNEL__COUNT) return "?";
    return knames[k];
}

int kernel_from_name(const char *s)
{
    for (int i = 0; i < KERNEL__COUNT; i++)
        if (strcmp(s, knames[i]) == 0) return i;
    return -1;
}

/* ---- src/bigmat.c ------------------------------------------------------ */
double now_sec(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

uint16_t *bigmat_alloc(int n, int L)
{
    return calloc((size_t)n * n * (size_t)L, sizeof(uint16_t));
}

/* SplitMix64 inputs, plane-major (src/bigmat.c:21-35).  Input generation,
 * not part of the product path. */
void bigmat_rand(uint16_t *m, int n, int L, uint64_t seed)
{
    uint64_t s = seed;
    size_t total = (size_t)n * n * (size_t)L;
    for (size_t i = 0; i < total; i++) {
        s += 0x9E3779B97F4A7C15ULL;
        uint64_t z = s;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        m[i] = (uint16_t)(z ^ (z >> 31));
    }
}

uint16_t *bigmat_to_entry_major(const uint16_t *plane, int n, int L)
{
    uint16_t *e = bigmat_alloc(n, L);
    if (!e) return NULL;
    size_t nn = (size_t)n * n;
    for (int u = 0; u < L; u++)
        for (size_t idx = 0; idx < nn; idx++) e[idx * L + u] = plane[(size_t)u * nn + idx];
    return e;
}

void normalize_planes(const int64_t *acc, int nplanes, int n, uint16_t *out, int RL)
{
    int rc = mfh_normalize(acc, nplanes, n, out, RL);
    t_last_error = rc;
    if (rc) fail("normalize_planes", rc);
}

int bigres_equal(const uint16_t *a, const uint16_t *b, int n, int RL,
                 int *bad_i, int *bad_j, int *bad_w)
{
    size_t nn = (size_t)n * n;
    for (int w = 0; w < RL; w++)
        for (size_t idx = 0; idx < nn; idx++)
            if (a[(size_t)w * nn + idx] != b[(size_t)w * nn + idx]) {
                if (bad_w) *bad_w = w;
                if (bad_i) *bad_i = (int)(idx / (size_t)n);
                if (bad_j) *bad_j = (int)(idx % (size_t)n);
                return 0;
            }
    return 1;
}

/* ---- plan (src/mfft.c:75-122) ------------------------------------------- */
static int ilog2i(int x) { int r = 0; while ((1 << r) < x) r++; return r; }

int mfft_plan_init(mfft_plan *p, int L, int sigma_override)
{
    if (L < 2 || (L & (L - 1))) return -1;
    int l = ilog2i(L);
    int sigma = sigma_override > 0 ? sigma_override : l / 2;
    if (sigma < 1) sigma = 1;
    if (sigma > l) return -1;
    int S = 1 << sigma, NB = 2 * L / S, K = 2 * S;
    if (2 * S * S < L || (2 * K) % NB || NB < 2) return -1;
    p->L = L; p->S = S; p->NB = NB; p->K = K; p->g = 2 * K / NB;
    p->rec = 0;
    p->nprod = (long long)NB * K * K;
    return 0;
}

long long mfft_plan_products(const mfft_plan *p)
{
    return p->nprod ? p->nprod : (long long)p->NB * p->K * p->K;
}

double mfft_plan_maxbits(const mfft_plan *p, int n)
{
    return 3.0 * log2((double)p->NB) + log2((double)p->K) + log2((double)n) +
           2.0 * LIMB_BITS;
}

void mfft_plan_describe(const mfft_plan *p, int n)
{
    printf("MFFT plan: L=%d limbs per entry (scalar width %d bits)  S=%d  "
           "NB=%d  K=%d  omega=I_%d^%d\n",
           p->L, p->L * LIMB_BITS, p->S, p->NB, p->K, ilog2i(p->K), p->g);
    printf("           n x n matrix products: MFFT %lld vs limb-plane %d "
           "(ratio %.2fx)  worst-case %.0f bits\n",
           mfft_plan_products(p), p->L * p->L,
           (double)(p->L * p->L) / (double)mfft_plan_products(p),
           mfft_plan_maxbits(p, n));
}

/* ---- recursive plan (src/mfft.c:474-527, 664-686) ------------------------
 * The reference's planner for the recursive pointwise step: a negacyclic
 * convolution of length 2^k over M_n(Z) with input magnitudes below 2^M
 * either bottoms out in Karatsuba (3^k products, intermediates of about
 * 2 + k + log2 n + 2M bits) or splits into 2^nu blocks (nu >= 2, 2 nu <=
 * k + 1), each a length-2^(k+1-nu) problem with M + nu bits; a split is
 * admissible while every intermediate stays within 62 bits.  The cheapest
 * admissible choice wins (ties keep the earlier one).  The table is local
 * to each call, so the planner is re-entrant. */
typedef struct { long long cost; int nu, outbits, maxbits, ok; } negplan;
#define NEG_K 26
#define NEG_M 74
typedef struct { negplan slot[NEG_K][NEG_M]; int done[NEG_K][NEG_M]; int ln; } negmemo;

static int ilog2c(int x) { int r = 0; while ((1 << r) < x) r++; return r; }

static negplan plan_neg(negmemo *m, int k, int M)
{
    negplan none = {0, 0, 0, 0, 0};
    if (k < 0 || k >= NEG_K || M < 0 || M >= NEG_M) return none;
    if (m->done[k][M]) return m->slot[k][M];
    negplan best = none;
    const int bbits = 2 + k + m->ln + 2 * M;
    if (bbits <= 62) {
        long long c = 1;
        for (int i = 0; i < k; i++) c *= 3;
        best = (negplan){c, 0, 1 + k + m->ln + 2 * M, bbits, 1};
    }
    for (int nu = 2; 2 * nu <= k + 1; nu++) {
        negplan ch = plan_neg(m, k + 1 - nu, M + nu);
        if (!ch.ok) continue;
        int mx = ch.maxbits > nu + ch.outbits ? ch.maxbits : nu + ch.outbits;
        if (mx > 62) continue;
        long long c = ((long long)1 << nu) * ch.cost;
        if (!best.ok || c < best.cost) best = (negplan){c, nu, ch.outbits + 1, mx, 1};
    }
    m->slot[k][M] = best;
    m->done[k][M] = 1;
    return best;
}

int mfft_plan_init_rec(mfft_plan *p, int L, int n, int sigma_override)
{
    if (L < 2 || (L & (L - 1)) || n < 1) return -1;
    negmemo *m = calloc(1, sizeof *m);
    if (!m) return -1;
    m->ln = ilog2c(n);
    int l = ilog2i(L), bs = 0;
    long long best = -1;
    for (int sigma = 1; sigma < l; sigma++) {
        int S = 1 << sigma, NB = 2 * L / S, K = 2 * S;
        if (2 * S * S < L || (2 * K) % NB || NB < 2) continue;
        if (sigma_override > 0 && sigma != sigma_override) continue;
        negplan pn = plan_neg(m, sigma + 1, LIMB_BITS + ilog2c(NB));
        if (!pn.ok) continue;
        long long c = (long long)NB * pn.cost;
        if (best < 0 || c < best) { best = c; bs = sigma; }
    }
    free(m);
    if (best < 0) return -1;
    p->L = L; p->S = 1 << bs; p->NB = 2 * L / p->S; p->K = 2 * p->S;
    p->g = 2 * p->K / p->NB;
    p->rec = 1;
    p->nprod = best;
    return 0;
}

/* src/mfft.c:560-662: C = A * B in M_n(Z)[t]/(t^K + 1), K int32 planes in,
 * K int64 planes out.  On the device: the linear convolution of the K
 * planes (integer-ALU schoolbook, exact mod 2^64) folded by t^K = -1, the
 * same result the reference's recursion and its Karatsuba base produce;
 * Mbits only steers the reference's planner and is not needed here. */
void ssa_negconv(int64_t *C, const int32_t *A, const int32_t *B, int K, int n, int Mbits,
                 kernel_t kern)
{
    (void)Mbits;
    t_last_error = 0;
    if (kern != KERNEL_HIP) { fail("ssa_negconv", MFH_E_UNSUPPORTED); return; }
    int rc = mfh_negconv(A, B, K, n, C);
    if (rc) fail("ssa_negconv", rc);
}

/* ---- device context cache ------------------------------------------------ */
/* A recursive plan (rec = 1) runs its outer transform as planned; its
 * pointwise negacyclic products are the device's matrix-core products
 * rather than a recursion, which gives the same exact result. */
static int get_ctx(int n, int L, const mfft_plan *p, mfh_ctx **out)
{
    if (!p) return MFH_E_ARG;
    int key[4] = {n, L, p->S, p->NB};
    if (g_ctx && memcmp(key, g_key, sizeof key) == 0) { *out = g_ctx; return 0; }
    if (g_ctx) { mfh_destroy(g_ctx); g_ctx = NULL; }
    mfh_plan hp = {p->L, p->S, p->NB, p->K, p->g, 0, (long long)p->NB * p->K * p->K};
    int rc = mfh_create(&g_ctx, n, L, &hp);
    if (rc) { g_ctx = NULL; return rc; }
    memcpy(g_key, key, sizeof key);
    *out = g_ctx;
    return 0;
}

static void mm_common(const uint16_t *Apl, const uint16_t *Bpl, int n, int L,
                      const mfft_plan *p, kernel_t k, uint16_t *out, int RL,
                      int kind, const char *name)
{
    t_last_error = 0;
    if (k != KERNEL_HIP) { fail(name, MFH_E_UNSUPPORTED); return; }
    if (!Apl || !Bpl || !out || !p || RL < 1 || n < 1) { fail(name, MFH_E_ARG); return; }
    pthread_mutex_lock(&g_lock);
    mfh_ctx *c = NULL;
    int rc = get_ctx(n, L, p, &c);
    if (!rc) {
        mfh_set_timing(c, g_mfft_profile != 0);
        rc = mfh_mm(c, kind, Apl, Bpl, out, RL);
        if (!rc && g_mfft_profile) profile_add(c);
    }
    pthread_mutex_unlock(&g_lock);
    if (rc) fail(name, rc);
}

void mm_mfft(const uint16_t *Apl, const uint16_t *Bpl, int n, int L,
             const mfft_plan *p, kernel_t k, uint16_t *out, int RL)
{
    mm_common(Apl, Bpl, n, L, p, k, out, RL, MFH_IN_U16, "mm_mfft");
}

void mm_mfft_signed(const uint16_t *Apl, const uint16_t *Bpl, int n, int L,
                    const mfft_plan *p, kernel_t k, uint16_t *out, int RL)
{
    mm_common(Apl, Bpl, n, L, p, k, out, RL, MFH_IN_U16_SIGNED, "mm_mfft_signed");
}

void conv_mfft(int64_t *Cw, const int32_t *A32, const int32_t *B32,
               int n, int L, const mfft_plan *p, kernel_t k)
{
    t_last_error = 0;
    if (k != KERNEL_HIP) { fail("conv_mfft", MFH_E_UNSUPPORTED); return; }
    if (!Cw || !A32 || !B32 || !p || n < 1) { fail("conv_mfft", MFH_E_ARG); return; }
    pthread_mutex_lock(&g_lock);
    mfh_ctx *c = NULL;
    int rc = get_ctx(n, L, p, &c);
    if (!rc) {
        mfh_set_timing(c, g_mfft_profile != 0);
        rc = mfh_conv(c, A32, B32, Cw);
        if (!rc && g_mfft_profile) profile_add(c);
    }
    pthread_mutex_unlock(&g_lock);
    if (rc) fail("conv_mfft", rc);
}

/* ---- schoolbook (src/kernel.c:1015-1033, src/methods.c:94-123) ---------- */
void mm_accum(int64_t *C, const int32_t *A, const int32_t *B, int n, int sign, kernel_t k)
{
    g_kernel_calls++;              /* src/kernel.c:1018 */
    t_last_error = 0;
    if (k != KERNEL_HIP) { fail("mm_accum", MFH_E_UNSUPPORTED); return; }
    int rc = mfh_mm_accum(C, A, B, n, sign);
    if (rc) fail("mm_accum", rc);
}

void conv_limbplane(int64_t *Cw, const int32_t *A32, const int32_t *B32, int n, int L,
                    kernel_t k)
{
    t_last_error = 0;
    if (k != KERNEL_HIP) { fail("conv_limbplane", MFH_E_UNSUPPORTED); return; }
    int rc = mfh_limbplane_conv(A32, B32, n, L, Cw);
    if (rc) fail("conv_limbplane", rc);
}

void mm_bigint_ijk(const uint16_t *Aem, const uint16_t *Bem, int n, int L, uint16_t *out, int RL)
{
    t_last_error = 0;
    int rc = mfh_bigint_mm(Aem, Bem, n, L, out, RL);
    if (rc) fail("mm_bigint_ijk", rc);
}

void mm_bigint_ikj(const uint16_t *Aem, const uint16_t *Bem, int n, int L, uint16_t *out, int RL)
{
    t_last_error = 0;
    int rc = mfh_bigint_mm(Aem, Bem, n, L, out, RL);
    if (rc) fail("mm_bigint_ikj", rc);
}

void mm_limbplane(const uint16_t *Apl, const uint16_t *Bpl, int n, int L, kernel_t k,
                  uint16_t *out, int RL)
{
    t_last_error = 0;
    if (k != KERNEL_HIP) { fail("mm_limbplane", MFH_E_UNSUPPORTED); return; }
    /* on the matrix cores where their partial-sum bound holds and their
     * workspace fits, else on the integer ALU (both exact; the ALU kernel
     * needs only the 2L-1 int64 coefficient planes) */
    int rc = RL >= 1 ? mfh_schoolbook(MFH_IN_U16, Apl, Bpl, n, L, out, RL) : MFH_E_ARG;
    if (rc == MFH_E_BOUND || rc == MFH_E_NOMEM) rc = mfh_limbplane_mm(Apl, Bpl, n, L, out, RL);
    if (rc) fail("mm_limbplane", rc);
}

/* ---- fp32 embedding (src/fpfixed.c) -------------------------------------- */
static int next_pow2(int x) { int r = 1; while (r < x) r <<= 1; return r; }

/* exponent range of finite nonzero entries: x = mi 2^e2 with mi an exact
 * sig-bit integer (src/fpfixed.c:40-54, 115-129); host-side sizing, as in the
 * reference */
static void scan(const float *X, size_t nn, int *lo, int *hi, int *any)
{
    int l = 1 << 30, h = -(1 << 30), seen = 0;
    for (size_t i = 0; i < nn; i++) {
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

static void scan_d(const double *X, size_t nn, int *lo, int *hi, int *any)
{
    int l = 1 << 30, h = -(1 << 30), seen = 0;
    for (size_t i = 0; i < nn; i++) {
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

/* What fpx_mm_f32 / fpx_mm_f64 need beyond the reference's fpx_ctx: device
 * copies of the matrices of the context's most recent encode, and a device
 * output buffer.  One entry per live context, keyed by its A32 planes
 * (unique while the context lives; a copied fpx_ctx finds the same entry),
 * removed by fpx_free.  Guarded by g_lock. */
typedef struct fpx_keep {
    const int32_t *key;
    int f64, n;
    void *dA, *dB, *dC;
    struct fpx_keep *next;
} fpx_keep;
static fpx_keep *g_keep;

static fpx_keep **keep_find(const int32_t *key)
{
    fpx_keep **k = &g_keep;
    while (*k && (*k)->key != key) k = &(*k)->next;
    return k;
}

static void keep_release(fpx_keep *k)
{
    if (k->dA) mfh_free(k->dA);
    if (k->dB) mfh_free(k->dB);
    if (k->dC) mfh_free(k->dC);
    free(k);
}

/* device copies of A and B for the context keyed by `key` (replacing
 * those of an earlier encode) */
static int keep_inputs(const int32_t *key, const void *A, const void *B, int n, int f64)
{
    const size_t bytes = (size_t)n * n * (f64 ? 8 : 4);
    fpx_keep *k = calloc(1, sizeof *k);
    if (!k) return MFH_E_NOMEM;
    k->key = key; k->f64 = f64; k->n = n;
    int rc = mfh_malloc(&k->dA, bytes);
    if (!rc) rc = mfh_malloc(&k->dB, bytes);
    if (!rc) rc = mfh_h2d(k->dA, A, bytes);
    if (!rc) rc = mfh_h2d(k->dB, B, bytes);
    if (rc) { keep_release(k); return rc; }
    pthread_mutex_lock(&g_lock);
    fpx_keep **slot = keep_find(key);
    if (*slot) { fpx_keep *old = *slot; k->next = old->next; keep_release(old); }
    *slot = k;
    pthread_mutex_unlock(&g_lock);
    return MFH_OK;
}

/* grid and limb count (src/fpfixed.c:59-78): `sig` significand bits, `wr`
 * limbs one shifted significand can touch; then the int64 guard and the host
 * planes (src/fpfixed.c:80-94) */
static int fpx_setup(fpx_ctx *c, int n, int loA, int hiA, int loB, int hiB,
                     int anyA, int anyB, int sig, int wr, int force_bits)
{
    size_t nn = (size_t)n * n;
    memset(c, 0, sizeof *c);
    c->sig = sig;
    c->spreadA = anyA ? hiA - loA : 0;
    c->spreadB = anyB ? hiB - loB : 0;
    int L;
    if (force_bits > 0) {
        c->SA = c->SB = force_bits / 2;
        L = next_pow2(force_bits / LIMB_BITS);
    } else {
        c->SA = -loA;
        c->SB = -loB;
        int spread = c->spreadA > c->spreadB ? c->spreadA : c->spreadB;
        int bits = sig + spread + 1;
        int need = (bits + LIMB_BITS - 1) / LIMB_BITS;
        int need2 = spread / LIMB_BITS + wr;
        L = next_pow2(need > need2 ? need : need2);
        if (L < 2) L = 2;
    }
    c->n = n; c->L = L;
    if ((double)n * L * 65535.0 * 65535.0 > 4.0e18) {
        fprintf(stderr, "fpx: n=%d L=%d would overflow int64 accumulators\n", n, L);
        t_last_error = MFH_E_BOUND;
        return -1;
    }
    c->A32 = calloc((size_t)L * nn, sizeof(int32_t));
    c->B32 = calloc((size_t)L * nn, sizeof(int32_t));
    c->Cw = calloc((size_t)(2 * L - 1) * nn, sizeof(int64_t));
    if (!c->A32 || !c->B32 || !c->Cw) { fpx_free(c); return -1; }
    return 0;
}

/* src/fpfixed.c:96-108: a 24-bit significand touches at most 3 limbs */
int fpx_init(fpx_ctx *c, const float *A, const float *B, int n, int force_bits)
{
    size_t nn = (size_t)n * n;
    int loA, hiA, loB, hiB, anyA, anyB;
    scan(A, nn, &loA, &hiA, &anyA);
    scan(B, nn, &loB, &hiB, &anyB);
    return fpx_setup(c, n, loA, hiA, loB, hiB, anyA, anyB, 24, 3, force_bits);
}

/* src/fpfixed.c:131-142: a 53-bit significand touches at most 5 limbs */
int fpx_init_d(fpx_ctx *c, const double *A, const double *B, int n, int force_bits)
{
    size_t nn = (size_t)n * n;
    int loA, hiA, loB, hiB, anyA, anyB;
    scan_d(A, nn, &loA, &hiA, &anyA);
    scan_d(B, nn, &loB, &hiB, &anyB);
    return fpx_setup(c, n, loA, hiA, loB, hiB, anyA, anyB, 53, 5, force_bits);
}

/* limb planes A32/B32 written on the device (the reference's encode, timed
 * into enc_secs as src/fpfixed.c:204 does); then device copies of A and B
 * are kept for fpx_mm_f32 / fpx_mm_f64 */
static void encode_common(fpx_ctx *c, const void *A, const void *B, int f64,
                          const char *name)
{
    t_last_error = 0;
    if (!c || !c->A32 || !c->B32 || !A || !B) { fail(name, MFH_E_ARG); return; }
    double t0 = now_sec();
    int rc = f64 ? mfh_fpx_encode_f64(A, c->n, c->L, c->SA, c->A32)
                 : mfh_fpx_encode(A, c->n, c->L, c->SA, c->A32);
    if (!rc)
        rc = f64 ? mfh_fpx_encode_f64(B, c->n, c->L, c->SB, c->B32)
                 : mfh_fpx_encode(B, c->n, c->L, c->SB, c->B32);
    if (rc) { fail(name, rc); return; }
    c->enc_secs = now_sec() - t0;
    if ((rc = keep_inputs(c->A32, A, B, c->n, f64))) fail(name, rc);
}

void fpx_encode(fpx_ctx *c, const float *A, const float *B)
{
    encode_common(c, A, B, 0, "fpx_encode");
}

void fpx_encode_d(fpx_ctx *c, const double *A, const double *B)
{
    encode_common(c, A, B, 1, "fpx_encode_d");
}

void fpx_decode_f32(fpx_ctx *c, float *C)
{
    double t0 = now_sec();
    t_last_error = 0;
    int rc = mfh_fpx_decode(c->Cw, c->n, c->L, c->SA + c->SB, C);
    if (rc) { fail("fpx_decode_f32", rc); return; }
    c->dec_secs = now_sec() - t0;
}

void fpx_decode_f64(fpx_ctx *c, double *C)
{
    t_last_error = 0;
    int rc = mfh_fpx_decode_f64(c->Cw, c->n, c->L, c->SA + c->SB, C);
    if (rc) fail("fpx_decode_f64", rc);
}

void fpx_decode_ld(fpx_ctx *c, long double *C)
{
    t_last_error = 0;
    int rc = mfh_fpx_decode_ld(c->Cw, c->n, c->L, c->SA + c->SB, C);
    if (rc) fail("fpx_decode_ld", rc);
}

/* the product of the kept device copies, decoded on the device into the
 * entry's output buffer, then copied to C */
static int fpx_mm_common(fpx_ctx *c, const mfft_plan *p, void *C, int f64, const char *name)
{
    t_last_error = 0;
    if (!c || !c->A32 || !p || !C) return fail(name, MFH_E_ARG);
    const size_t bytes = (size_t)c->n * c->n * (f64 ? 8 : 4);
    pthread_mutex_lock(&g_lock);
    fpx_keep *k = *keep_find(c->A32);
    int rc = (!k || k->f64 != (f64 != 0) || k->n != c->n) ? MFH_E_ARG : MFH_OK;
    if (!rc && !k->dC) rc = mfh_malloc(&k->dC, bytes);
    mfh_ctx *h = NULL;
    if (!rc) rc = get_ctx(c->n, c->L, p, &h);
    if (!rc)
        rc = f64 ? mfh_fpx_mm_f64_dev(h, k->dA, k->dB, c->SA, c->SB, k->dC)
                 : mfh_fpx_mm_dev(h, k->dA, k->dB, c->SA, c->SB, k->dC);
    if (!rc) rc = mfh_sync(h);
    if (!rc) rc = mfh_d2h(C, k->dC, bytes);
    pthread_mutex_unlock(&g_lock);
    if (rc) return fail(name, rc);
    return 0;
}

int fpx_mm_f32(fpx_ctx *c, const mfft_plan *p, float *C)
{
    return fpx_mm_common(c, p, C, 0, "fpx_mm_f32");
}

int fpx_mm_f64(fpx_ctx *c, const mfft_plan *p, double *C)
{
    return fpx_mm_common(c, p, C, 1, "fpx_mm_f64");
}

/* src/mlgemm.c:593-630: the window over the highest live limb planes */
int fpx_faithful_window(const fpx_ctx *c, int max_keep, int *u0_out, int *hi_out)
{
    const size_t nn = (size_t)c->n * c->n;
    int hi = -1;
    for (int w = 0; w < c->L; w++) {
        int any = 0;
        for (size_t i = 0; i < nn && !any; i++)
            if (c->A32[(size_t)w * nn + i] || c->B32[(size_t)w * nn + i]) any = 1;
        if (any) hi = w;
    }
    if (hi < 0) hi = c->L - 1;
    const int span = hi + 1;
    int Lk = 1;
    if (max_keep > 1) {
        const int keep = max_keep < c->L ? max_keep : c->L;
        while (Lk * 2 <= keep && Lk * 2 <= span && Lk * 2 <= c->L) Lk *= 2;
        if (Lk < 2 && keep >= 2 && span >= 2) Lk = 2;
    }
    if (Lk > span) Lk = span;
    if (Lk < 1) Lk = 1;
    int u0 = hi - Lk + 1;
    if (u0 < 0) u0 = 0;
    if (u0_out) *u0_out = u0;
    if (hi_out) *hi_out = hi;
    return Lk;
}

static int faithful_common(fpx_ctx *c, int max_keep, void *C, int f64, int *Lk_out,
                           int *u0_out, const char *name)
{
    t_last_error = 0;
    if (!c || !c->A32 || !c->B32 || !C || (c->sig == 53) != (f64 != 0))
        return fail(name, MFH_E_ARG);
    int u0, hi;
    const int Lk = fpx_faithful_window(c, max_keep, &u0, &hi);
    mfft_plan p;
    mfh_plan hp;
    if (Lk >= 2) {
        // src/mlgemm.c:1211-1213: the recursive plan from 4 limbs on
        const int ok = Lk >= 4 ? mfft_plan_init_rec(&p, Lk, c->n, 0) : mfft_plan_init(&p, Lk, 0);
        if (ok != 0) return fail(name, MFH_E_UNSUPPORTED);
        hp = (mfh_plan){p.L, p.S, p.NB, p.K, p.g, 0, (long long)p.NB * p.K * p.K};
    }
    const size_t nn = (size_t)c->n * c->n;
    int rc = mfh_fpx_faithful(c->A32 + (size_t)u0 * nn, c->B32 + (size_t)u0 * nn, c->n, c->L,
                              u0, Lk, Lk >= 2 ? &hp : NULL, c->SA + c->SB, f64, C);
    if (rc) return fail(name, rc);
    if (Lk_out) *Lk_out = Lk;
    if (u0_out) *u0_out = u0;
    return 0;
}

int fpx_faithful_f32(fpx_ctx *c, int max_keep, float *C, int *Lk, int *u0)
{
    return faithful_common(c, max_keep, C, 0, Lk, u0, "fpx_faithful_f32");
}

int fpx_faithful_f64(fpx_ctx *c, int max_keep, double *C, int *Lk, int *u0)
{
    return faithful_common(c, max_keep, C, 1, Lk, u0, "fpx_faithful_f64");
}

/* src/fpfixed.c:324-328, plus the device copies kept for the context */
void fpx_free(fpx_ctx *c)
{
    if (c->A32) {
        pthread_mutex_lock(&g_lock);
        fpx_keep **slot = keep_find(c->A32);
        fpx_keep *k = *slot;
        if (k) *slot = k->next;
        pthread_mutex_unlock(&g_lock);
        if (k) keep_release(k);
    }
    free(c->A32); free(c->B32); free(c->Cw);
    c->A32 = NULL; c->B32 = NULL; c->Cw = NULL;
}
