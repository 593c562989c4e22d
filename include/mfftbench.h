/* mfftbench.h -- C host API of the MI355X (gfx950) exact-integer MFFT
 * matrix multiply.
 *
 * Drop-in for the exact-integer path of hadilq/mfft-bench: the functions
 * below keep the names, signatures, layouts and error conventions of the
 * reference header src/mfftbench.h (cited per declaration).  The device path
 * is selected with the extra kernel_t value KERNEL_HIP, so a caller's method
 * table runs it exactly like the reference's `mfft` rows.  Products run
 * only on the GPU: this library has no CPU implementation of the product,
 * and a call that cannot run on the device fails (stderr message, output
 * untouched, mfft_last_error() < 0) instead of falling back.
 *
 * Layout (src/mfftbench.h:74-82): plane-major, p[u*n*n + i*n + j] is limb u
 * (base 2^16) of entry (i, j).  The exact product has RL = 2L+1 limbs.
 */
#ifndef MFFTBENCH_HIP_H
#define MFFTBENCH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LIMB_BITS 16
#define LIMB_MASK ((uint32_t)((1u << LIMB_BITS) - 1u))

/* src/mfftbench.h:33-47; KERNEL_HIP appended after the reference's twelve
 * CPU leaves so their numbering is unchanged. */
typedef enum {
    KERNEL_IKJ = 0,
    KERNEL_BLOCKED,
    KERNEL_PACKED,
    KERNEL_STRASSEN,
    KERNEL_WINOGRAD,
    KERNEL_BITPLANE,
    KERNEL_CONVK,
    KERNEL_CONVKARA,
    KERNEL_BOOLPACK,
    KERNEL_BITPACK,
    KERNEL_BOOLSTRASSEN,
    KERNEL_BOOLTILED,
    KERNEL_HIP,          /* gfx950: batched int8 MFMA pointwise GEMM */
    KERNEL__COUNT
} kernel_t;

const char *kernel_name(kernel_t k);                 /* src/kernel.c:21-25 */
int         kernel_from_name(const char *s);         /* src/kernel.c:31-36 */

/* ---- big-integer matrices (src/bigmat.c) -------------------------------- */
double    now_sec(void);                                         /* :8-13  */
uint16_t *bigmat_alloc(int n, int L);                            /* :15-18 */
void      bigmat_rand(uint16_t *m, int n, int L, uint64_t seed); /* :29-35 */
uint16_t *bigmat_to_entry_major(const uint16_t *plane, int n, int L); /* :37-46 */
/* :48-60 -- carry-propagates on the device */
void normalize_planes(const int64_t *acc, int nplanes, int n,
                      uint16_t *out, int RL);
int  bigres_equal(const uint16_t *a, const uint16_t *b, int n, int RL,
                  int *bad_i, int *bad_j, int *bad_w);           /* :62-75 */

/* ---- instrumentation the reference bench reads (src/mfftbench.h:56-71) --
 * g_kernel_calls counts mm_accum calls (the device MFFT path makes none).
 * With g_mfft_profile set, mm_mfft / conv_mfft add their device stage
 * times (HIP events) to g_mfft_prof: transform = forward transforms +
 * inverse (which also folds, and on the exact track carries), pointwise =
 * the batched MFMA step; packing and op lists are fused into the forward
 * kernel (pack = build_ops = 0), fold into the inverse (fold = 0). */
extern long long g_kernel_calls;
typedef struct {
    double pack;
    double build_ops;
    double transform;
    double pointwise;
    double fold;
    long long n_build;
    long long n_fft;
} mfft_profile_t;
extern int g_mfft_profile;
extern mfft_profile_t g_mfft_prof;
void mfft_profile_reset(void);
void mfft_profile_print(const char *label);

/* ---- the leaf operator and the limb-plane schoolbook ---------------------
 * k must be KERNEL_HIP: integer-ALU kernels on the device, exact modulo 2^64
 * for any int32 entries like the reference's int64 leaves. */
/* src/mfftbench.h:53-54: C += A*B if sign > 0, else C -= A*B */
void mm_accum(int64_t *C, const int32_t *A, const int32_t *B, int n, int sign,
              kernel_t k);
/* src/mfftbench.h:96-99: the textbook product on entry-major inputs
 * (bigmat_to_entry_major), plane-major output; these have no kernel_t and
 * always run on the device */
void mm_bigint_ijk(const uint16_t *Aem, const uint16_t *Bem, int n, int L,
                   uint16_t *out, int RL);
void mm_bigint_ikj(const uint16_t *Aem, const uint16_t *Bem, int n, int L,
                   uint16_t *out, int RL);
/* src/mfftbench.h:100-101: on the int8 matrix cores (mfh_schoolbook) where
 * the bound of its int32 partial sums holds (ceil(L/16) n <= 8224) and its
 * workspace fits in device memory, else on the integer ALU; exact either
 * way */
void mm_limbplane(const uint16_t *Apl, const uint16_t *Bpl, int n, int L,
                  kernel_t k, uint16_t *out, int RL);
/* src/mfftbench.h:105-106 */
void conv_limbplane(int64_t *Cw, const int32_t *A32, const int32_t *B32,
                    int n, int L, kernel_t k);

/* ---- flat MFFT plan (src/mfftbench.h:139-154, src/mfft.c:77-122) -------- */
typedef struct {
    int L, S, NB, K, g;
    int rec;
    long long nprod;
} mfft_plan;

int       mfft_plan_init(mfft_plan *p, int L, int sigma_override);
/* src/mfftbench.h:149, src/mfft.c:664-686: the plan whose pointwise step is
 * a recursive negacyclic convolution (rec = 1, nprod = the reference's
 * product count).  mm_mfft / conv_mfft accept it: the device runs its outer
 * transform and does the pointwise products on the matrix cores. */
int       mfft_plan_init_rec(mfft_plan *p, int L, int n, int sigma_override);
/* src/mfftbench.h:150-151, src/mfft.c:560-662: negacyclic convolution of K
 * int32 n x n planes into K int64 planes (k must be KERNEL_HIP) */
void      ssa_negconv(int64_t *C, const int32_t *A, const int32_t *B, int K, int n,
                      int Mbits, kernel_t k);
long long mfft_plan_products(const mfft_plan *p);
double    mfft_plan_maxbits(const mfft_plan *p, int n);
void      mfft_plan_describe(const mfft_plan *p, int n);

/* src/mfftbench.h:156-159, src/mfft.c:302-438.  k must be KERNEL_HIP. */
void mm_mfft(const uint16_t *Apl, const uint16_t *Bpl, int n, int L,
             const mfft_plan *p, kernel_t k, uint16_t *out, int RL);
void conv_mfft(int64_t *Cw, const int32_t *A32, const int32_t *B32,
               int n, int L, const mfft_plan *p, kernel_t k);

/* Two's complement entries (no reference counterpart: the reference's exact
 * track is unsigned, main.c:3-5, and its conv_mfft takes signed limbs):
 * limbs 0..L-2 unsigned, limb L-1 read as int16; `out` is the product mod
 * 2^(16*RL) in two's complement, exact when RL >= 2L+1. */
void mm_mfft_signed(const uint16_t *Apl, const uint16_t *Bpl, int n, int L,
                    const mfft_plan *p, kernel_t k, uint16_t *out, int RL);

/* ---- fp32/fp64 fixed-point embedding (src/mfftbench.h:182-199,
 *      src/fpfixed.c) ------------------------------------------------------
 * fpx_ctx has exactly the reference's fields and layout (72 bytes on
 * x86-64), so a caller built against either header may own it (on the
 * stack, as src/mlgemm.c:723 does).  What the fused fpx_mm_f32/_f64 need
 * beyond it is kept inside the library, keyed by the context's A32 planes,
 * and released by fpx_free. */
typedef struct {
    int n, L, sig;
    int SA, SB;
    int spreadA, spreadB;
    int32_t *A32, *B32;     /* signed limb planes, L*n*n each (host)      */
    int64_t *Cw;            /* exact product, 2L-1 int64 planes (host)    */
    double enc_secs, dec_secs;
} fpx_ctx;

int  fpx_init(fpx_ctx *c, const float *A, const float *B, int n,
              int force_bits);                                          /* :191 */
void fpx_encode(fpx_ctx *c, const float *A, const float *B);            /* :192 */
int  fpx_init_d(fpx_ctx *c, const double *A, const double *B, int n,
                int force_bits);                                        /* :193 */
void fpx_encode_d(fpx_ctx *c, const double *A, const double *B);        /* :195 */
void fpx_decode_ld(fpx_ctx *c, long double *C);                         /* :196 */
void fpx_decode_f32(fpx_ctx *c, float *C);                              /* :197 */
void fpx_decode_f64(fpx_ctx *c, double *C);                             /* :198 */
void fpx_free(fpx_ctx *c);                                              /* :199 */
/* encode -> MFFT product -> decode entirely on the device (no reference
 * counterpart; equals conv_mfft + fpx_decode_f32 bit for bit).  It
 * multiplies the matrices of the most recent fpx_encode on this context:
 * fpx_encode keeps a device copy of A and B for it, so the caller may free
 * or reuse its A and B as soon as fpx_encode returns.  The copy is
 * released by fpx_free.  Returns 0, or a negative MFH_E_* code (MFH_E_ARG
 * when the context has no fp32 encoding). */
int  fpx_mm_f32(fpx_ctx *c, const mfft_plan *p, float *C);
/* the same for the fp64 matrices of the most recent fpx_encode_d (equals
 * conv_mfft + fpx_decode_f64 bit for bit; no reference counterpart) */
int  fpx_mm_f64(fpx_ctx *c, const mfft_plan *p, double *C);

/* Faithful limb window (src/mlgemm.c:593-630, static there): hi = the
 * highest limb plane that is non-zero in A32 or B32 of an encoded context
 * (L-1 when all are zero); the window is the top limb (Lk = 1) for
 * max_keep <= 1, else the largest power of two Lk <= min(max_keep, hi+1, L)
 * (at least 2 when hi >= 1); *u0 = hi - Lk + 1.  Returns Lk. */
int  fpx_faithful_window(const fpx_ctx *c, int max_keep, int *u0, int *hi);
/* The fp32/64->mfft-faithful products (src/mlgemm.c:1186-1250 fp32,
 * :909-961 fp64) on the device, after fpx_encode / fpx_encode_d: the exact
 * product of the window's planes (one leaf GEMM for Lk = 1, else conv_mfft
 * under mfft_plan_init_rec for Lk >= 4 or mfft_plan_init, as there), placed
 * at plane 2 u0 of 2L-1 zero planes and rounded once by the reference's
 * decode into C (n x n).  Inexact by design: the planes below the window
 * are dropped.  The window is reported in *Lk and *u0 (either may be NULL).
 * c->Cw is not written.  Returns 0 or a negative MFH_E_* code (no reference
 * counterpart as a function: the reference inlines these steps). */
int  fpx_faithful_f32(fpx_ctx *c, int max_keep, float *C, int *Lk, int *u0);
int  fpx_faithful_f64(fpx_ctx *c, int max_keep, double *C, int *Lk, int *u0);

/* Status of the most recent call on this thread: 0, or a negative code
 * from mfft_hip.h (MFH_E_*). */
int         mfft_last_error(void);
const char *mfft_strerror(int code);

#ifdef __cplusplus
}
#endif
#endif
