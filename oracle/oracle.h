/* oracle.h -- CPU restatement of hadilq/mfft-bench's exact-integer MFFT
 * matrix multiply (flat plan, packed int32->int64 leaf), its limb-plane and
 * textbook oracles, the fp32/fp64 fixed-point embedding, and checking helpers.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load this library, and only as the checker or
 * the timed CPU baseline -- never as a product path.  Every function cites
 * the reference file:line whose semantics it restates (paths relative to the
 * reference repository root).
 *
 * Pinning (what checks each function beyond retyping it):
 *   orc_bigmat_rand        KAT against published SplitMix64 outputs and the
 *                          reference library built from source (oracle/_ref)
 *   orc_normalize_planes   Python big-integer fixtures (tests/golden)
 *   orc_conv_limbplane     brute-force big-integer products (tests/golden)
 *   orc_ring_dft           definition-level brute force; inverse(forward)=NB*id
 *   orc_conv_mfft          == orc_conv_limbplane, == reference conv_mfft
 *   orc_fpx_*              Python Fraction rounding fixtures + reference fpx
 *   orc_freivalds          planted-error detection on the CPU
 */
#ifndef MFFT_ORACLE_H
#define MFFT_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#define ORC_LIMB_BITS 16

/* ---- seeded inputs and limb-plane helpers (src/bigmat.c) ---------------- */
uint64_t orc_sm64_next(uint64_t *state);
void orc_bigmat_rand(uint16_t *m, int n, int L, uint64_t seed);
void orc_to_entry_major(const uint16_t *plane, int n, int L, uint16_t *em);
void orc_normalize_planes(const int64_t *acc, int nplanes, int n,
                          uint16_t *out, int RL);
int  orc_bigres_equal(const uint16_t *a, const uint16_t *b, int n, int RL,
                      int *bad_i, int *bad_j, int *bad_w);

/* ---- leaf n x n products: C += sign * A * B (src/kernel.c) --------------- */
void orc_mm_accum_packed(int64_t *C, const int32_t *A, const int32_t *B,
                         int n, int sign);
void orc_mm_accum_ikj(int64_t *C, const int32_t *A, const int32_t *B,
                      int n, int sign);

/* ---- schoolbook oracles (src/methods.c) --------------------------------- */
void orc_conv_limbplane(int64_t *Cw, const int32_t *A32, const int32_t *B32,
                        int n, int L, int leaf);
void orc_mm_limbplane(const uint16_t *Apl, const uint16_t *Bpl, int n, int L,
                      uint16_t *out, int RL, int leaf);
void orc_mm_bigint_ijk(const uint16_t *Aem, const uint16_t *Bem, int n, int L,
                       uint16_t *out, int RL);

/* ---- flat MFFT plan and convolution (src/mfft.c) ------------------------ */
typedef struct {
    int L, S, NB, K, g;
    long long nprod;
} orc_plan;

int    orc_plan_init(orc_plan *p, int L, int sigma_override);
double orc_plan_maxbits(const orc_plan *p, int n);

/* Brute-force length-NB DFT over R = Z[y]/(y^K+1), omega = y^g, natural
 * order in and out, for one matrix element:
 *     X[j] = sum_b omega^(dir * j * b) x[b],   dir = +1 forward, -1 inverse.
 * x, X: NB*K int64 values, block-major ([b][c]). */
void orc_ring_dft(int64_t *X, const int64_t *x, int NB, int K, int g, int dir);

/* Radix-2 transforms on NB*K planes of nn values (mfft.c:225-299 semantics):
 * forward = Gentleman-Sande, natural -> bit-reversed; inverse = Cooley-Tukey
 * with conjugate twiddles, bit-reversed -> natural (unscaled: NB * x). */
void orc_fft_forward32(int32_t *X, int NB, int K, int g, size_t nn);
void orc_fft_inverse64(int64_t *X, int NB, int K, int g, size_t nn);

/* leaf: 0 = ikj, 2 = packed (the reference's kernel_t numbering) */
void orc_conv_mfft(int64_t *Cw, const int32_t *A32, const int32_t *B32,
                   int n, int L, const orc_plan *p, int leaf);
void orc_mm_mfft(const uint16_t *Apl, const uint16_t *Bpl, int n, int L,
                 const orc_plan *p, uint16_t *out, int RL, int leaf);

/* Stage timings of one conv_mfft in which only `nprod_sample` of the
 * NB*K^2 pointwise products are run (in the reference's loop order); the
 * caller extrapolates.  secs[0]=pack+forward, [1]=pointwise sample,
 * [2]=inverse+fold, [3]=normalize.  Returns products actually run. */
long long orc_mm_mfft_sampled(const uint16_t *Apl, const uint16_t *Bpl, int n,
                              int L, const orc_plan *p, uint16_t *out, int RL,
                              long long nprod_sample, double secs[4]);

/* ---- fp32/fp64 fixed-point embedding (src/fpfixed.c) ------------------- */
typedef struct {
    int n, L;
    int SA, SB;
    int spreadA, spreadB;
    int32_t *A32, *B32;   /* L planes each */
    int64_t *Cw;          /* 2L-1 planes */
} orc_fpx;

int  orc_fpx_init(orc_fpx *c, const float *A, const float *B, int n,
                  int force_bits);
void orc_fpx_encode(orc_fpx *c, const float *A, const float *B);
void orc_fpx_decode_f32(const orc_fpx *c, float *C);
/* decode of a caller-provided Cw (2L-1 planes) with the context's scales */
void orc_fpx_decode_f32_from(const orc_fpx *c, const int64_t *Cw, float *C);
/* fp64 (src/fpfixed.c:115-173, 308-322) */
int  orc_fpx_init_d(orc_fpx *c, const double *A, const double *B, int n,
                    int force_bits);
void orc_fpx_encode_d(orc_fpx *c, const double *A, const double *B);
void orc_fpx_decode_f64_from(const orc_fpx *c, const int64_t *Cw, double *C);
/* long double decode (src/fpfixed.c:292-306) as sig * 2^ex, |sig| < 2^63 */
void orc_fpx_decode_sig63_from(const orc_fpx *c, const int64_t *Cw, int64_t *sig,
                               int32_t *ex);
void orc_fpx_free(orc_fpx *c);
/* The faithful limb window (src/mlgemm.c:593-630): returns Lk, sets *u0 and
 * *hi from the planes of an encoded context. */
int  orc_faithful_window(const orc_fpx *c, int max_keep, int *u0, int *hi);
/* The faithful product's coefficient planes (src/mlgemm.c:909-961 fp64 with
 * max_keep 2, :1186-1250 fp32): Cw (2L-1 planes) = 0 except the exact
 * convolution of the window planes at plane 2 u0 (the schoolbook, which
 * equals conv_mfft); returns Lk. */
int  orc_faithful_cw(const orc_fpx *c, int max_keep, int64_t *Cw, int *u0);

/* ---- checking helpers (not in the reference) ---------------------------- */
/* fp32 inputs +-m*2^e, m~U[1,2) with 23 random fraction bits, e~U{emin..emax},
 * one splitmix64 draw per value, in index order. */
void orc_fp32_rand(float *X, size_t count, uint64_t seed, int emin, int emax);

/* Exact value of one output entry C[i][j] = sum_k A[i][k]*B[k][j] as RL
 * base-2^16 limbs (two's complement mod 2^(16*RL)).  signed_top != 0 reads
 * the top input limb (u = L-1) as a signed int16. */
void orc_entry_exact(const uint16_t *Apl, const uint16_t *Bpl, int n, int L,
                     int signed_top, int i, int j, uint16_t *limbs, int RL);

/* Freivalds check of out == A*B over Z_p for `nprimes` 61-bit primes and a
 * seeded random vector: returns 1 if all agree, 0 if not.  Inputs and output
 * are plane-major u16 limbs; signed_top as above; the output is read as a
 * two's complement integer of RL limbs when signed_top != 0. */
int orc_freivalds(const uint16_t *Apl, const uint16_t *Bpl, int n, int L,
                  int signed_top, const uint16_t *out, int RL,
                  int nprimes, uint64_t seed);

/* Same check on raw int64 coefficient planes Cw (2L-1 of them) against int32
 * limb planes: sum_w Cw[w] 2^(16w) == (sum_u A32[u] 2^(16u)) (...)  mod p. */
int orc_freivalds_conv(const int32_t *A32, const int32_t *B32, int n, int L,
                       const int64_t *Cw, int nprimes, uint64_t seed);

#endif
