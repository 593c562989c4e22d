/* route2.c -- a C caller of include/mfftbench.h, compiled by gcc the way a
 * program written against the reference API would be (the calls of
 * src/main.c:94-135 and src/mlgemm.c:723-736 on the device path).  Test
 * infrastructure: the GPU tests load it in-process and hand it the golden
 * fixtures; every product goes through the reference-named C functions.
 *
 * The layouts below are those of the reference header on LP64
 * (src/mfftbench.h:59-67 mfft_profile_t, :139-143 mfft_plan, :182-189
 * fpx_ctx); a CPU test also compiles the reference header itself and
 * compares its sizeof/offsetof values with r2_layout(). */
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "mfft_hip.h"
#include "mfftbench.h"

_Static_assert(sizeof(fpx_ctx) == 72, "fpx_ctx: 7 ints, 3 pointers, 2 doubles");
_Static_assert(offsetof(fpx_ctx, n) == 0 && offsetof(fpx_ctx, L) == 4 &&
               offsetof(fpx_ctx, sig) == 8 && offsetof(fpx_ctx, SA) == 12 &&
               offsetof(fpx_ctx, SB) == 16 && offsetof(fpx_ctx, spreadA) == 20 &&
               offsetof(fpx_ctx, spreadB) == 24, "fpx_ctx int fields");
_Static_assert(offsetof(fpx_ctx, A32) == 32 && offsetof(fpx_ctx, B32) == 40 &&
               offsetof(fpx_ctx, Cw) == 48 && offsetof(fpx_ctx, enc_secs) == 56 &&
               offsetof(fpx_ctx, dec_secs) == 64, "fpx_ctx pointer/double fields");
_Static_assert(sizeof(mfft_plan) == 32 && offsetof(mfft_plan, g) == 16 &&
               offsetof(mfft_plan, rec) == 20 && offsetof(mfft_plan, nprod) == 24,
               "mfft_plan");
_Static_assert(sizeof(mfft_profile_t) == 56 && offsetof(mfft_profile_t, fold) == 32 &&
               offsetof(mfft_profile_t, n_build) == 40 &&
               offsetof(mfft_profile_t, n_fft) == 48, "mfft_profile_t");
_Static_assert(KERNEL_PACKED == 2 && KERNEL_BOOLTILED == 11 && KERNEL_HIP == 12,
               "kernel_t keeps the reference's numbering, KERNEL_HIP appended");

#define N_LAYOUT 19

/* sizeof / offsetof values, in the order the CPU test prints them for the
 * reference header */
int r2_layout(long *v, int cap)
{
    const long x[N_LAYOUT] = {
        (long)sizeof(fpx_ctx), (long)offsetof(fpx_ctx, sig), (long)offsetof(fpx_ctx, spreadB),
        (long)offsetof(fpx_ctx, A32), (long)offsetof(fpx_ctx, B32), (long)offsetof(fpx_ctx, Cw),
        (long)offsetof(fpx_ctx, enc_secs), (long)offsetof(fpx_ctx, dec_secs),
        (long)sizeof(mfft_plan), (long)offsetof(mfft_plan, rec), (long)offsetof(mfft_plan, nprod),
        (long)sizeof(mfft_profile_t), (long)offsetof(mfft_profile_t, pointwise),
        (long)offsetof(mfft_profile_t, fold), (long)offsetof(mfft_profile_t, n_fft),
        (long)KERNEL_PACKED, (long)KERNEL_BOOLTILED, (long)LIMB_BITS, (long)sizeof(kernel_t)};
    if (cap < N_LAYOUT) return -1;
    memcpy(v, x, sizeof x);
    return N_LAYOUT;
}

/* src/main.c:207-208, 111-134: seeded inputs, mm_mfft on the device,
 * bigres_equal against the expected limbs.  Returns 1 when equal, 0 with
 * bad = (i, j, w) of the first mismatch, or a negative error code (the
 * library's, -99 when the planner has no plan for L, as the recursive one
 * has none for L < 4, or -100 for an allocation failure). */
int r2_mm_mfft(int n, int L, uint64_t seed_a, uint64_t seed_b, int is_signed, int rec,
               const uint16_t *want, int RL, int *bad)
{
    mfft_plan p;
    if ((rec ? mfft_plan_init_rec(&p, L, n, 0) : mfft_plan_init(&p, L, 0)) != 0) return -99;
    uint16_t *A = bigmat_alloc(n, L), *B = bigmat_alloc(n, L);
    uint16_t *out = malloc((size_t)RL * n * n * sizeof(uint16_t));
    int rc = -100;
    if (A && B && out) {
        bigmat_rand(A, n, L, seed_a);
        bigmat_rand(B, n, L, seed_b);
        memset(out, 0xA5, (size_t)RL * n * n * sizeof(uint16_t));
        if (is_signed) mm_mfft_signed(A, B, n, L, &p, KERNEL_HIP, out, RL);
        else mm_mfft(A, B, n, L, &p, KERNEL_HIP, out, RL);
        rc = mfft_last_error();
        if (!rc) rc = bigres_equal(out, want, n, RL, &bad[0], &bad[1], &bad[2]);
    }
    free(A); free(B); free(out);
    return rc;
}

/* The multi-modular product (mfh_rns_*, include/mfft_hip.h; no reference
 * counterpart) from C on the same seeded inputs: create, one host-buffer
 * product, destroy, then bigres_equal against the expected limbs.  Returns 1
 * when equal, 0 with bad = the first mismatch, or a negative error code
 * (-100: allocation failure). */
int r2_rns_mm(int n, int L, uint64_t seed_a, uint64_t seed_b, int is_signed,
              const uint16_t *want, int RL, int *bad)
{
    uint16_t *A = bigmat_alloc(n, L), *B = bigmat_alloc(n, L);
    uint16_t *out = malloc((size_t)RL * n * n * sizeof(uint16_t));
    int rc = -100;
    if (A && B && out) {
        bigmat_rand(A, n, L, seed_a);
        bigmat_rand(B, n, L, seed_b);
        memset(out, 0xA5, (size_t)RL * n * n * sizeof(uint16_t));
        mfh_rns *r = NULL;
        rc = mfh_rns_create(&r, n, L);
        if (!rc) {
            rc = mfh_rns_mm(r, is_signed ? MFH_IN_U16_SIGNED : MFH_IN_U16, A, B, out, RL);
            mfh_rns_destroy(r);
        }
        if (!rc) rc = bigres_equal(out, want, n, RL, &bad[0], &bad[1], &bad[2]);
    }
    free(A); free(B); free(out);
    return rc;
}

/* g_mfft_profile / g_mfft_prof (src/mfftbench.h:69-71) around one product,
 * then one mm_accum: the pointwise seconds the caller sees in g_mfft_prof
 * and how far g_kernel_calls moved.  Returns 0 or a negative error code. */
int r2_instrumentation(int n, int L, double *pointwise_s, long long *kernel_calls)
{
    mfft_plan p;
    if (mfft_plan_init(&p, L, 0) != 0) return -100;
    uint16_t *A = bigmat_alloc(n, L), *B = bigmat_alloc(n, L);
    uint16_t *out = malloc((size_t)(2 * L + 1) * n * n * sizeof(uint16_t));
    int64_t *C = calloc((size_t)n * n, sizeof(int64_t));
    int32_t *a = calloc((size_t)n * n, sizeof(int32_t));
    int rc = -100;
    if (A && B && out && C && a) {
        bigmat_rand(A, n, L, 1);
        bigmat_rand(B, n, L, 2);
        mfft_profile_reset();
        g_mfft_profile = 1;
        mm_mfft(A, B, n, L, &p, KERNEL_HIP, out, 2 * L + 1);
        g_mfft_profile = 0;
        rc = mfft_last_error();
        *pointwise_s = g_mfft_prof.pointwise;
        const long long before = g_kernel_calls;
        if (!rc) {
            mm_accum(C, a, a, n, 1, KERNEL_HIP);
            rc = mfft_last_error();
        }
        *kernel_calls = g_kernel_calls - before;
    }
    free(A); free(B); free(out); free(C); free(a);
    return rc;
}

/* guard words after the context: a library that wrote past the reference's
 * 72-byte fpx_ctx would change them */
typedef struct {
    fpx_ctx f;
    uint64_t guard[4];
} guarded_ctx;
#define GUARD 0x5AFEC0DE5AFEC0DEull

static int guard_ok(const guarded_ctx *g)
{
    for (int i = 0; i < 4; i++)
        if (g->guard[i] != GUARD) return 0;
    return 1;
}

/* src/mlgemm.c:723-728 with conv_mfft in place of conv_limbplane: fpx_init,
 * fpx_encode, conv_mfft, fpx_decode_f32 (into C_conv), then the fused
 * fpx_mm_f32 (into C_fused) after the caller's encoded inputs have been
 * overwritten and freed.  Returns 0, a negative library code, -101 for an
 * init failure, -102 when the guard words after the context changed. */
int r2_fpx_f32(const float *A, const float *B, int n, int force_bits, float *C_conv,
               float *C_fused, int *L_out)
{
    guarded_ctx g;
    for (int i = 0; i < 4; i++) g.guard[i] = GUARD;
    const size_t nn = (size_t)n * n;
    float *Ac = malloc(nn * sizeof(float)), *Bc = malloc(nn * sizeof(float));
    if (!Ac || !Bc) { free(Ac); free(Bc); return -100; }
    memcpy(Ac, A, nn * sizeof(float));
    memcpy(Bc, B, nn * sizeof(float));
    if (fpx_init(&g.f, Ac, Bc, n, force_bits) != 0) { free(Ac); free(Bc); return -101; }
    fpx_encode(&g.f, Ac, Bc);
    int rc = mfft_last_error();
    memset(Ac, 0xFF, nn * sizeof(float));      /* NaNs, then gone */
    memset(Bc, 0xFF, nn * sizeof(float));
    free(Ac); free(Bc);
    *L_out = g.f.L;
    mfft_plan p;
    if (!rc && mfft_plan_init(&p, g.f.L, 0) != 0) rc = -100;
    if (!rc) {
        conv_mfft(g.f.Cw, g.f.A32, g.f.B32, n, g.f.L, &p, KERNEL_HIP);
        rc = mfft_last_error();
    }
    if (!rc) {
        fpx_decode_f32(&g.f, C_conv);
        rc = mfft_last_error();
    }
    if (!rc) rc = fpx_mm_f32(&g.f, &p, C_fused);
    fpx_free(&g.f);
    if (!rc && (!guard_ok(&g) || g.f.A32 || g.f.B32 || g.f.Cw)) rc = -102;
    return rc;
}

/* The fixed-point product by the multi-modular path from C: the grid of
 * fpx_init (L, SA, SB) on a context of L + 1 limbs, mfh_rns_fpx_mm on the
 * caller's host arrays.  Returns 0, a negative library code, or -101 for an
 * init failure. */
int r2_rns_fpx_f32(const float *A, const float *B, int n, int force_bits, float *C_out)
{
    fpx_ctx f;
    if (fpx_init(&f, A, B, n, force_bits) != 0) return -101;
    const int L = f.L, SA = f.SA, SB = f.SB;
    fpx_free(&f);
    mfh_rns *r = NULL;
    int rc = mfh_rns_create(&r, n, L + 1);
    if (!rc) {
        rc = mfh_rns_fpx_mm(r, A, B, SA, SB, C_out);
        mfh_rns_destroy(r);
    }
    return rc;
}

/* src/mlgemm.c:731-736 on the device: fpx_init_d, fpx_encode_d, conv_mfft,
 * fpx_decode_f64 and fpx_decode_ld, then the fused fpx_mm_f64 after the
 * inputs are gone. */
int r2_fpx_f64(const double *A, const double *B, int n, int force_bits, double *C_conv,
               double *C_fused, long double *C_ld, int *L_out)
{
    guarded_ctx g;
    for (int i = 0; i < 4; i++) g.guard[i] = GUARD;
    const size_t nn = (size_t)n * n;
    double *Ac = malloc(nn * sizeof(double)), *Bc = malloc(nn * sizeof(double));
    if (!Ac || !Bc) { free(Ac); free(Bc); return -100; }
    memcpy(Ac, A, nn * sizeof(double));
    memcpy(Bc, B, nn * sizeof(double));
    int rc = 0;
    if (fpx_init_d(&g.f, Ac, Bc, n, force_bits) != 0) rc = -101;
    if (!rc) {
        fpx_encode_d(&g.f, Ac, Bc);
        rc = mfft_last_error();
    }
    memset(Ac, 0xFF, nn * sizeof(double));
    memset(Bc, 0xFF, nn * sizeof(double));
    free(Ac); free(Bc);
    if (rc) return rc;
    *L_out = g.f.L;
    mfft_plan p;
    if (mfft_plan_init(&p, g.f.L, 0) != 0) rc = -100;
    if (!rc) {
        conv_mfft(g.f.Cw, g.f.A32, g.f.B32, n, g.f.L, &p, KERNEL_HIP);
        rc = mfft_last_error();
    }
    if (!rc) {
        fpx_decode_f64(&g.f, C_conv);
        rc = mfft_last_error();
    }
    if (!rc) {
        fpx_decode_ld(&g.f, C_ld);
        rc = mfft_last_error();
    }
    if (!rc) rc = fpx_mm_f64(&g.f, &p, C_fused);
    fpx_free(&g.f);
    if (!rc && (!guard_ok(&g) || g.f.A32 || g.f.B32 || g.f.Cw)) rc = -102;
    return rc;
}
