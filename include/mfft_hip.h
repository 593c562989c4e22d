/* mfft_hip.h -- C-ABI shim between the C host API (mfftbench.h) and the
 * gfx950 HIP kernels of the exact-integer MFFT matrix multiply.
 *
 * Plain C types only.  Every entry point returns 0 on success or a negative
 * MFH_E_* code; on error no output buffer has been written.  A context owns
 * the device workspace for one (n, L, plan) shape and one HIP stream; it may
 * be used by one host thread at a time.  Entry points taking host pointers
 * are synchronous.  Entry points ending in _dev take device pointers, are
 * ordered on the context's stream and return without synchronising
 * (mfh_sync() waits).
 *
 * Layouts follow the reference (src/mfftbench.h:74-82): a big-integer matrix
 * is L limb planes, plane u at p[u*n*n + i*n + j], each n x n row-major.
 * The exact product has RL = 2L+1 uint16 limb planes; the raw convolution
 * Cw has 2L-1 int64 planes.
 */
#ifndef MFFT_HIP_H
#define MFFT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    MFH_OK = 0,
    MFH_E_NODEV = -1,    /* no usable gfx950 device                        */
    MFH_E_NOMEM = -2,    /* device allocation failed                       */
    MFH_E_ARG = -3,      /* invalid argument (shape, plan, null pointer)   */
    MFH_E_BOUND = -4,    /* plan/size would overflow a stated accumulator  */
    MFH_E_RANGE = -5,    /* an input limb lies outside [-65535, 65535]     */
    MFH_E_HIP = -6,      /* HIP runtime error                              */
    MFH_E_UNSUPPORTED = -7,
    MFH_E_SCRATCH = -8   /* workspace larger than the fixed no-allocation
                            scratch (mfh_mm_dev_noalloc)                   */
};

/* Input forms accepted by the transform (the limb reader). */
enum {
    MFH_IN_U16 = 0,        /* unsigned limbs (the exact track)                */
    MFH_IN_U16_SIGNED = 1, /* limbs 0..L-2 unsigned, limb L-1 int16: a
                              two's complement W-bit integer               */
    MFH_IN_I32 = 2         /* signed int32 limbs, |limb| <= 65535 (conv_mfft) */
};

typedef struct mfh_ctx mfh_ctx;

/* Flat MFFT plan, the reference's mfft_plan (src/mfftbench.h:139-143). */
typedef struct {
    int L, S, NB, K, g;
    int rec;
    long long nprod;
} mfh_plan;

const char *mfh_strerror(int code);
int  mfh_device_count(void);
/* gfx arch name of device 0 (e.g. "gfx950"), or "" without a device */
const char *mfh_device_arch(void);

/* Workspace for products of n x n matrices with L limbs under `plan`.
 * Rejects plans whose worst case breaks the stated accumulator bounds
 * (int8 digits, int32 MFMA accumulators, int64 transform values).  The
 * int32 bound depends on the digit mode: sizes that only the 6-product mode
 * admits (n up to about 8128 at K = 16, against 2688 for the 9-product
 * mode) serve the exact-track products, while conv and fixed-point-float
 * products, which take the 9-product mode where plain 6-product digits do
 * not fit, return MFH_E_BOUND. */
int  mfh_create(mfh_ctx **ctx, int n, int L, const mfh_plan *plan);
void mfh_destroy(mfh_ctx *ctx);
/* device bytes held by the context */
size_t mfh_workspace_bytes(const mfh_ctx *ctx);
/* Row band height of the context's products (no reference counterpart: the
 * reference holds every transformed operand in host memory).  A's
 * transformed digits and the pointwise results are held for this many
 * padded rows at a time; it is n rounded up to a multiple of 64 (one band)
 * when the whole workspace fits in 90 % of the device memory free at
 * mfh_create, else the largest multiple of 64 rows that does, at least
 * 1/64 of the rows (MFH_E_NOMEM below that).  The environment variable
 * MFH_BAND_ROWS=<rows>, read at mfh_create, forces a height. */
int  mfh_band_rows(const mfh_ctx *ctx);

/* ---- host-buffer entry points (synchronous) ----------------------------- */
/* mm_mfft: exact product of unsigned (or, with MFH_IN_U16_SIGNED, two's
 * complement) limb matrices into RL >= 2L-1 uint16 planes. */
int mfh_mm(mfh_ctx *ctx, int in_kind, const uint16_t *A, const uint16_t *B,
           uint16_t *out, int RL);
/* conv_mfft: signed int32 limb planes -> 2L-1 int64 coefficient planes. */
int mfh_conv(mfh_ctx *ctx, const int32_t *A32, const int32_t *B32,
             int64_t *Cw);

/* Intermediate results of mfh_conv's device path, for inspection and
 * stage-level tests (no reference counterpart: the reference's stages are
 * static functions of src/mfft.c).  The product of A32 and B32 runs up to
 * `stage` for row band 0 and the raw device buffer is copied to out:
 *   MFH_STAGE_A: A's int8 digit planes, [NB][slots][planes] planes of
 *     rows x np entries in 16 x 64 tiles (tile (i/16, k/64) row-major, each
 *     tile row-major); point j is the transform's point j (omega^j), in
 *     natural order; slots are the K ring coefficients, or under the Gauss
 *     pointwise the 3K/2 slots [z0+z1 | z0 | z1] (z0, z1 the coefficient
 *     halves); planes are the digits of the digit mode;
 *   MFH_STAGE_B: the same for B^T (entry (j', k) = B[k][j']) over np rows,
 *     Gauss slots [z0 | z1-z0 | -(z0+z1)];
 *   MFH_STAGE_CLASSES: the int32 class results of the pointwise step,
 *     C[j][i][m][j'/16][t/4][j'%16][t%4], K np ints per (j, i, m).
 * info[0..4] = digit mode (0: three balanced base-2^8 digits, 5 classes of
 * 9 products; 1: three balanced base-2^7 digits and their pairwise sums, 6
 * Karatsuba products), pointwise algorithm (0 flat, 1 Gauss), band rows,
 * np, bytes of the stage; with out NULL only info is filled.  Returns 0,
 * or MFH_E_ARG when out_bytes is short. */
#define MFH_STAGE_A 0
#define MFH_STAGE_B 1
#define MFH_STAGE_CLASSES 2
int mfh_conv_stages(mfh_ctx *ctx, const int32_t *A32, const int32_t *B32, int stage,
                    void *out, size_t out_bytes, int64_t info[5]);

/* ---- device-buffer entry points (stream-ordered, no sync) --------------- */
/* dA and dB must be 16-byte aligned (the limbs are read 8 at a time; any
 * hipMalloc pointer is): MFH_E_ARG otherwise, before any kernel runs. */
int mfh_mm_dev(mfh_ctx *ctx, int in_kind, const void *dA, const void *dB,
               void *dOut, int RL);
int mfh_conv_dev(mfh_ctx *ctx, const void *dA32, const void *dB32, void *dCw);

/* mfh_mm_dev with no device allocation: no counterpart in the reference; for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  No context: the
 * workspace is one fixed device array of MFH_NOALLOC_BYTES per device, held
 * from the library's load until the process ends, and sizes whose workspace
 * exceeds it return MFH_E_SCRATCH before any kernel runs (n = 64 at 1024-bit
 * entries fits; n = 128 at 512 bits does not).  Same inputs, output and
 * checks as mfh_mm_dev, and the same kernels.  `stream` is a hipStream_t
 * passed as void * (NULL: the null stream); the call is ordered on it and
 * returns without synchronising.  Every call on a device shares that
 * device's array and leaves it holding its intermediates: calls that overlap
 * on one device (from two host threads, or on two streams not ordered
 * against each other) race. */
#define MFH_NOALLOC_BYTES (64u << 20)
int mfh_mm_dev_noalloc(int in_kind, const mfh_plan *plan, int n, int L, const void *dA,
                       const void *dB, void *dOut, int RL, void *stream);

/* fp32 fixed-point embedding on device (src/fpfixed.c semantics):
 * A, B fp32 n x n; scales 2^SA, 2^SB; product rounded once to fp32. */
int mfh_fpx_mm_dev(mfh_ctx *ctx, const void *dA, const void *dB, int SA,
                   int SB, void *dC);
int mfh_fpx_mm(mfh_ctx *ctx, const float *A, const float *B, int SA, int SB,
               float *C);
/* decode only: 2L-1 int64 planes -> fp32 with scale 2^-(SA+SB) (device) */
int mfh_fpx_decode_dev(mfh_ctx *ctx, const void *dCw, int SAB, void *dC);
/* fp64 on the same grid (src/fpfixed.c:131-173, 308-322): A, B fp64 n x n;
 * the product is rounded to 53 bits as fpx_decode_f64 does. */
int mfh_fpx_mm_f64_dev(mfh_ctx *ctx, const void *dA, const void *dB, int SA,
                       int SB, void *dC);
int mfh_fpx_mm_f64(mfh_ctx *ctx, const double *A, const double *B, int SA,
                   int SB, double *C);
int mfh_fpx_decode_f64_dev(mfh_ctx *ctx, const void *dCw, int SAB, void *dC);

/* ---- standalone host-buffer helpers (temporary device buffers) ---------- */
/* normalize_planes (src/bigmat.c:48-60) on the device */
int mfh_normalize(const int64_t *acc, int nplanes, int n, uint16_t *out, int RL);
/* fpx_encode (src/fpfixed.c:175-204) of one fp32 n x n matrix at scale 2^S
 * into L signed int32 limb planes */
int mfh_fpx_encode(const float *X, int n, int L, int S, int32_t *X32);
/* fpx_decode_f32 (src/fpfixed.c:269-285) of 2L-1 int64 planes */
int mfh_fpx_decode(const int64_t *Cw, int n, int L, int SAB, float *C);
/* fpx_encode_d (src/fpfixed.c:144-173): fp64 -> L signed limb planes */
int mfh_fpx_encode_f64(const double *X, int n, int L, int S, int32_t *X32);
/* fpx_decode_f64 (src/fpfixed.c:308-322) */
int mfh_fpx_decode_f64(const int64_t *Cw, int n, int L, int SAB, double *C);
/* fpx_decode_ld (src/fpfixed.c:292-306): rounding to 63 bits on the device,
 * C[i] = sig[i] * 2^ex[i] assembled on the host */
int mfh_fpx_decode_ld(const int64_t *Cw, int n, int L, int SAB, long double *C);
/* the device half of it: signed 63-bit significands and exponents */
int mfh_fpx_decode_sig63(const int64_t *Cw, int n, int L, int SAB, int64_t *sig,
                         int32_t *ex);

/* Faithful limb-window product of the fixed-point floats (the
 * fp32/64->mfft-faithful rows, src/mlgemm.c:909-961, 1186-1250): Aw, Bw are
 * the Lk window planes u0 .. u0+Lk-1 of two L-plane signed limb matrices
 * (host); their exact product, one leaf GEMM for Lk = 1 or the MFFT
 * convolution under `plan` (L = Lk) otherwise, is placed at plane 2 u0 of
 * 2L-1 zero planes and decoded on the device at scale 2^-SAB into C (fp32,
 * or fp64 when f64 != 0), n x n host. */
int mfh_fpx_faithful(const int32_t *Aw, const int32_t *Bw, int n, int L, int u0, int Lk,
                     const mfh_plan *plan, int SAB, int f64, void *C);

/* ---- schoolbook: the leaf operator and the limb-plane method ------------
 * Integer-ALU kernels, exact modulo 2^64 for any int32 entries (the
 * reference's int64 leaves wrap the same way); an independent second
 * computation of every product.  ctx may be NULL (null stream). */
/* mm_accum (src/kernel.c:1015-1033): C += A*B if sign > 0, else C -= A*B;
 * int64 C, int32 A, B, all n x n row-major */
int mfh_mm_accum(int64_t *C, const int32_t *A, const int32_t *B, int n, int sign);
int mfh_mm_accum_dev(mfh_ctx *ctx, void *dC, const void *dA, const void *dB, int n,
                     int sign);
/* conv_limbplane (src/methods.c:94-104): Cw[w] = sum_{u+v=w} A_u B_v over
 * L limb planes (in_kind MFH_IN_I32: int32; MFH_IN_U16: uint16;
 * MFH_IN_U16_SIGNED: uint16 with limb L-1 read as int16), 2L-1 int64 planes
 * out */
int mfh_limbplane_conv(const int32_t *A32, const int32_t *B32, int n, int L, int64_t *Cw);
int mfh_limbplane_conv_dev(mfh_ctx *ctx, int in_kind, const void *dA, const void *dB,
                           int n, int L, void *dCw);
/* mm_limbplane (src/methods.c:106-123): uint16 limb planes, the carry of
 * the convolution into RL uint16 limbs; dCw is 2L-1 int64 planes of scratch;
 * in_kind MFH_IN_U16 or MFH_IN_U16_SIGNED (two's complement entries, result
 * mod 2^(16 RL) in two's complement) */
int mfh_limbplane_mm(const uint16_t *A, const uint16_t *B, int n, int L, uint16_t *out,
                     int RL);
int mfh_limbplane_mm_dev(mfh_ctx *ctx, int in_kind, const void *dA, const void *dB, int n,
                         int L, void *dCw, void *dOut, int RL);

/* The same schoolbook on the int8 matrix cores (src/methods.c:94-123, the
 * products formed otherwise): every uint16 limb (the top one as int16 with
 * MFH_IN_U16_SIGNED) is split into the six int8 planes of its balanced
 * base-2^7 digits and pair sums, the planes of each Karatsuba class are
 * convolved over the limb axis with v_mfma_i32_16x16x64_i8 in blocks of 16
 * limbs (6 L^2 int8 n^3 GEMMs), and the classes are recombined and carried.
 * Out: RL > 0, RL uint16 limbs as mfh_limbplane_mm; RL = 0, the 2L-1 int64
 * coefficient planes as mfh_limbplane_conv.  The int32 partial sums are
 * exact modulo 2^32 and lie in a known range, which needs
 * 16 ceil(L/16) n 32640 < 2^32, i.e. ceil(L/16) n <= 8224 (MFH_E_BOUND
 * otherwise): n = 1024 at 2048 bits, 256 at 8192, 4096 at 512 bits
 * pass.  mfh_schoolbook_workspace gives the
 * bytes of device workspace mfh_schoolbook_dev needs; the host-buffer form
 * allocates its own. */
int mfh_schoolbook_workspace(int n, int L, size_t *bytes);
int mfh_schoolbook_dev(mfh_ctx *ctx, int in_kind, const void *dA, const void *dB, int n, int L,
                       void *dWork, size_t work_bytes, void *dOut, int RL);
int mfh_schoolbook(int in_kind, const uint16_t *A, const uint16_t *B, int n, int L, void *out,
                   int RL);

/* mm_bigint_ijk / mm_bigint_ikj (src/methods.c:22-86): entry-major uint16
 * inputs (Aem[(i*n + k)*L + u]), plane-major RL-limb output; on the device
 * the inputs are re-laid plane-major and multiplied by the schoolbook */
int mfh_bigint_mm(const uint16_t *Aem, const uint16_t *Bem, int n, int L, uint16_t *out,
                  int RL);
/* negacyclic convolution C = A*B mod (t^K + 1) of K int32 planes into K
 * int64 planes (ssa_negconv, src/mfft.c:560-662): the limb-plane
 * convolution folded by t^K = -1 */
int mfh_negconv(const int32_t *A, const int32_t *B, int K, int n, int64_t *C);

/* ---- multi-modular product ----------------------------------------------
 * No counterpart in the reference: the same exact product as mfh_mm /
 * mm_mfft (src/mfft.c:424-438) and mm_limbplane (src/methods.c:106-123),
 * computed by residue number system arithmetic instead of the MFFT, for
 * callers that want the product and not the transform.  The entries of A B
 * are reduced modulo nm primes p <= 65279 whose product exceeds 4 n 2^(2W)
 * (W = 16 L); per prime the product is four int8 GEMMs on the matrix cores,
 * and the Chinese remainder theorem, one more int8 GEMM per element, gives
 * the limbs.  Output as mfh_mm: RL >= 1 uint16 limb planes of the product
 * modulo 2^(16 RL) (two's complement for MFH_IN_U16_SIGNED), the limbs above
 * 2L+1 the sign extension.  Limits: n <= 32768, L <= 512 (MFH_E_BOUND). */
typedef struct mfh_rns mfh_rns;
/* plan only (host): the number of primes for n x n matrices of L limbs, the
 * first min(cap, count) of them (descending) written to primes */
int  mfh_rns_primes(int n, int L, int *primes, int cap);
int  mfh_rns_create(mfh_rns **ctx, int n, int L);
void mfh_rns_destroy(mfh_rns *ctx);
/* primes, padded size np (a multiple of 128), device bytes held */
int  mfh_rns_info(const mfh_rns *ctx, int *nprimes, int *np, size_t *bytes);
int  mfh_rns_mm_dev(mfh_rns *ctx, int in_kind, const void *dA, const void *dB, void *dOut,
                    int RL);
int  mfh_rns_mm(mfh_rns *ctx, int in_kind, const uint16_t *A, const uint16_t *B, uint16_t *out,
                int RL);
/* the residues of one operand read as rows r, inner index k (A, or B
 * transposed): dR gets nprimes planes of np x np uint16 digit pairs
 * lo | hi << 8 (r mod p = 256 (int8)hi + (int8)lo, |r| <= (p-1)/2), zero
 * outside n x n (a stage of mfh_rns_mm_dev, for tests) */
int  mfh_rns_residues_dev(mfh_rns *ctx, int in_kind, const void *dX, void *dR);
/* The fixed-point products of mfh_fpx_mm / mfh_fpx_mm_f64 (fpx_encode,
 * fpx_mm_f32, fpx_decode: src/fpfixed.c:144-322) by the multi-modular
 * product: on a grid of L limbs the context is created with L + 1 limbs
 * (mfh_rns_create(&ctx, n, L + 1); the limb above the grid carries the sign
 * of the two's complement operands).  Same inputs, scales and single
 * rounding as mfh_fpx_mm_dev on an L-limb context, so the same outputs bit
 * for bit.  The first call allocates the encoded operands and product
 * limbs ((8 L + 8) n^2 bytes, kept with the context). */
int  mfh_rns_fpx_mm_dev(mfh_rns *ctx, const void *dA, const void *dB, int SA, int SB,
                        void *dC);
int  mfh_rns_fpx_mm_f64_dev(mfh_rns *ctx, const void *dA, const void *dB, int SA, int SB,
                            void *dC);
int  mfh_rns_fpx_mm(mfh_rns *ctx, const float *A, const float *B, int SA, int SB, float *C);
int  mfh_rns_fpx_mm_f64(mfh_rns *ctx, const double *A, const double *B, int SA, int SB,
                        double *C);
int  mfh_rns_sync(mfh_rns *ctx);
/* stage times of the most recent product while timing is on: [0] B
 * transposed and the residues of both operands, [1] the per-prime GEMMs,
 * [2] CRT and carry, [3] total */
int  mfh_rns_set_timing(mfh_rns *ctx, int enable);
int  mfh_rns_stage_times(const mfh_rns *ctx, float ms[4]);
/* int8 MFMA ops the three stages issue (over the padded size np) */
int  mfh_rns_work(const mfh_rns *ctx, double *residue_ops, double *pointwise_ops,
                  double *crt_ops);

/* ---- device memory and timing helpers ----------------------------------- */
int  mfh_malloc(void **dptr, size_t bytes);
int  mfh_free(void *dptr);
int  mfh_h2d(void *dst, const void *src, size_t bytes);
int  mfh_d2h(void *dst, const void *src, size_t bytes);
int  mfh_sync(mfh_ctx *ctx);
/* bigmat_rand on device: plane-major uint16 limbs from splitmix64(seed),
 * identical to the host generator (src/bigmat.c:21-35). */
int  mfh_rand_u16_dev(mfh_ctx *ctx, void *dM, int n, int L, uint64_t seed);
/* fp32 inputs +-m*2^e (m in [1,2) with 23 random fraction bits, e uniform in
 * [emin, emax]) from splitmix64(seed), one draw per value. */
int  mfh_rand_f32_dev(mfh_ctx *ctx, void *dX, size_t count, uint64_t seed,
                      int emin, int emax);

/* Device-to-device copy by a plain streaming kernel (k_copy16), each byte
 * read once and written once; bytes and both pointers must be multiples of
 * 16.  No reference counterpart: it is the known-size kernel against which
 * hardware HBM byte counters are calibrated. */
int  mfh_copy_dev(mfh_ctx *ctx, void *dst, const void *src, size_t bytes);

/* Per-stage device times (ms) of the most recent product on this context,
 * measured with HIP events on the context's stream:
 *   [0] transforms in (both operands), [1] pointwise GEMM,
 *   [2] inverse transform + fold, [3] carry / decode, [4] total.
 * Timing is recorded only while enabled (it adds event records). */
int  mfh_set_timing(mfh_ctx *ctx, int enable);
int  mfh_stage_times(const mfh_ctx *ctx, float ms[5]);
/* Ops/bytes the kernels of the most recent product are designed to: int8
 * MFMA ops of the pointwise GEMM, the minimum HBM bytes of the forward
 * transforms, and those of the inverse + fold + carry (or decode) stages. */
int  mfh_work(const mfh_ctx *ctx, double *int8_ops, double *fwd_bytes,
              double *inv_bytes);
/* The pointwise step of the most recent product: ring products issued per
 * evaluation point (K^2, or 3 (K/2)^2 with the Gauss split of the ring
 * halves, the default where a Gauss kernel exists for K; MFH_POINTWISE=flat
 * at mfh_create forces K^2) and int8 digit products per ring product (6 or
 * 9).  No reference counterpart (the reference's plan counts its own n x n
 * products, mfft_plan.nprod). */
int  mfh_pointwise_info(const mfh_ctx *ctx, int *ring_products_per_point,
                        int *digit_products);

#ifdef __cplusplus
}
#endif
#endif
