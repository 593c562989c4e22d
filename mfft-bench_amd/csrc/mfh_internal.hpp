// mfh_internal.hpp -- shared definitions of the gfx950 MFFT kernels and the
// C-ABI shim (mfft_hip.h).  Not part of the public interface.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "mfft_hip.h"

// ---------------------------------------------------------------------------
// Number representation on the device
//
// Transformed values: the forward transform writes each ring coefficient of
// each evaluation point as a signed sum of one input limb from each of the
// L/S non-zero blocks, so |a^| <= (NB/2) * 65535.  Each is split into three
// balanced base-2^8 digits d0 + 2^8 d1 + 2^16 d2 with d_r in [-128, 127],
// which covers [-8421504, 8355711]: every plan with NB <= 254 fits
// (NB = 64 at n=256/W=8192 needs 2097120).
//
// Pointwise accumulators: one MFMA term is |d_A * d_B| <= 2^14.  A round
// (one 64-wide k block of one digit pair, all K ring coefficients) adds
// K*64 terms to an int32 accumulator, i.e. at most K * 2^20 in magnitude.
// A digit-weight class m = r+s has at most 3 digit pairs, so its int32
// result is bounded by 3 * (np/64) * K * 2^20, which must stay below 2^31.
// The pointwise step writes the int32 class results (five for B8, six for
// K7); the inverse transform recombines them into C^ in int64.
//
// int64: |C^| <= K * n * ((NB/2) * 65535)^2, and the inverse transform
// multiplies by at most NB more; both must stay below 2^62.
// ---------------------------------------------------------------------------
#define MFH_DIGITS 3
#define MFH_DIGIT_MAX 8355711LL   // 127 * (1 + 2^8 + 2^16)
#define MFH_DIGIT_MIN (-8421504LL) // -128 * (1 + 2^8 + 2^16)
#define MFH_KBLK 64               // k extent of one MFMA operand block

// Digit modes of the transformed values.
//  MFH_MODE_B8: three balanced base-2^8 digits d0, d1, d2 in [-128, 127];
//    9 digit products, accumulated in 5 weight classes m = r+s (2^(8m)).
//  MFH_MODE_K7: three balanced base-2^7 digits d0, d1 in [-64, 63] and d2 in
//    [-64, 64], plus the pairwise sums d0+d1, d0+d2, d1+d2 (in [-128, 127],
//    still int8; so is every product operand, and |product| <= 2^14):
//    Karatsuba's 6 products P0 = a0 b0, P1 = a1 b1, P2 = a2 b2,
//    P3 = (a0+a1)(b0+b1), P4 = (a0+a2)(b0+b2), P5 = (a1+a2)(b1+b2), one
//    class each, recombined as
//      c0 = P0, c1 = P3-P0-P1, c2 = P4-P0-P2+P1, c3 = P5-P1-P2, c4 = P2,
//      C^ = sum_m c_m 2^(7m).
//    Range: [-64 (1+2^7+2^14), 63 (1+2^7) + 64 2^14] = [-1056832, 1056703]:
//    the balanced digits of v are d0 = ((v+64) & 127) - 64,
//    v1 = (v+64) >> 7, d1 = ((v1+64) & 127) - 64, d2 = (v1+64) >> 7, and over
//    that range d2 reaches +64 but no further (it is 64 only for
//    v >= 2^20 - 64).
#define MFH_MODE_B8 0
#define MFH_MODE_K7 1
#define MFH_K7_MAX 1056703LL
#define MFH_PLANES_MAX 6          // digit planes per (point, coefficient)
#define MFH_CLASSES_MAX 6         // int32 class results per (point, element, t)
static inline int mfh_planes(int mode) { return mode == MFH_MODE_K7 ? 6 : 3; }
static inline int mfh_nclasses(int mode) { return mode == MFH_MODE_K7 ? 6 : 5; }

#define MFH_CLASSES (2 * MFH_DIGITS - 1)

// Layout of the pointwise step's int32 class results for a band of `rows`
// padded rows of A: for point j, element (i, j') with i the row within the
// band, class m and ring coefficient t = 4q + r, with j' = 16 jb + jl,
//     C5[j][i][m][jb][q][jl][r]       (q < K/4, r < 4, jl < 16)
// One wave's store of 4 consecutive t of 16 consecutive j' is then 256
// contiguous bytes, and the K values of 16 consecutive elements lie in one
// K*64-byte run.  Index of class 0 of (j, i, j', t); classes are
// mfh_c5_class_stride(np, K) ints apart.
__host__ __device__ inline size_t mfh_c5_index(int j, int i, int jj, int t, int np_, int ncl,
                                               int K, int rows)
{
    const size_t row = ((size_t)j * rows + i) * ncl;           // class 0 of (j, i)
    return ((row * (np_ / 16) + jj / 16) * (K / 4) + t / 4) * 64 + (jj & 15) * 4 + (t & 3);
}
// Layout of a digit plane (rows x np int8, rows a multiple of 16, np of
// 64): 16 x 64 tiles of 1 KB, row-major inside a tile, tiles row-major, so
// that one MFMA operand fragment (16 rows x 64 k) is one contiguous 1 KB.
__host__ __device__ inline size_t mfh_tile_off(int i, int k, int np_)
{
    return ((size_t)(i >> 4) * (np_ >> 6) + (k >> 6)) * 1024 + (i & 15) * 64 + (k & 63);
}
// inverse of mfh_tile_off: the element at offset e of a tiled plane
__host__ __device__ inline void mfh_tile_ik(size_t e, int np_, int &i, int &k)
{
    const size_t t = e >> 10;
    const int tpr = np_ >> 6;                      // tiles per tile row
    i = (int)(t / tpr) * 16 + (int)((e >> 6) & 15);
    k = (int)(t % tpr) * 64 + (int)(e & 63);
}
__host__ __device__ inline size_t mfh_c5_class_stride(int np_, int K)
{
    return (size_t)K * np_;
}

// class accumulators provably fit int32: a class has at most `pairs` digit
// products (3 for B8, 1 for K7) of np/64 rounds, each round at most
// K * 64 * 2^14
static inline bool mfh_class_bound_ok(int K, int np_, int pairs)
{
    return (long long)pairs * (np_ / MFH_KBLK) * ((long long)K << 20) <= 2147483647LL;
}

// at most this many row bands per product (the band height is at least
// np / MFH_BANDS_MAX rows)
#define MFH_BANDS_MAX 64

// Pointwise algorithm.  MFH_PW_FLAT: the K^2 products of each ring product
// (src/mfft.c:383-395).  MFH_PW_GAUSS: one Karatsuba level on the ring axis
// in Gauss's three-product form.  With u = y^(K/2) (u^2 = -1) and
// X = X0 + u X1 (X0, X1 of degree < H = K/2),
//     A B = (k1 - k3) + u (k1 + k2),
//     k1 = (A0 + A1) B0,  k2 = A0 (B1 - B0),  k3 = A1 (B0 + B1),
// three linear convolutions of length H (3 H^2 products instead of 4 H^2).
// The forward transform writes 3H operand slots per point: A's as
// [A0 + A1 | A0 | A1], B's as [B0 | B1 - B0 | -(B0 + B1)], so sub-product g
// multiplies slots gH .. gH+H-1 of both.  Every slot value obeys the bound
// of a single coefficient: block b contributes one limb to coefficient c
// and none to c + H or the other way round (its upper H coefficients are
// zero before the shift y^e), so X[c] +- X[c+H] is still a signed sum of
// one limb per non-zero block.
#define MFH_PW_FLAT 0
#define MFH_PW_GAUSS 1
// operand slots per evaluation point
static inline int mfh_slots(int K, int pw) { return pw == MFH_PW_GAUSS ? 3 * K / 2 : K; }

struct mfh_ctx {
    int n, np;            // matrix size, padded to a multiple of 64
    int L, S, NB, K, g;
    int dev;
    int use_fast;         // compile-time specialised kernels when available
    int pw;               // MFH_PW_GAUSS when the workspace holds Gauss slots
                          // (fixed at creation), else MFH_PW_FLAT
    int pwr;              // the current product's algorithm: Gauss needs pw and
                          // the 6-product digits (set with the digit mode)
    hipStream_t stream;
    // workspace
    int mode;             // digit mode of the current product (MFH_MODE_*)
    int recode;           // forward transform recodes limbs to signed form
    int offset;           // unsigned operands shifted by -2^(W-1) (with recode):
                          // the inverse adds back 2^(W-1) (r_i + s_j) + 2^(2W-2) n
    int64_t *dRow;        // offset mode: limb sums of A's rows [L][n] and of B's
    int64_t *dCol;        //   columns [L][n] (the shifted limbs)
    int k7_ok;            // plan admits MFH_MODE_K7 (workspace sized for it)
    int mode_ok;          // the selected digit setting keeps every bound
    int hb;               // row band height: A's digit planes and the class
                          // results hold hb padded rows at a time
    int8_t *dAh;          // A's digit planes [NB][slots][planes][hb][np]
    int8_t *dBh;          // B's digit planes [NB][slots][planes][np][np]
    int32_t *dC5;         // pointwise class results of a band (mfh_c5_index)
    int64_t *dCw;         // coefficient planes [2L-1][n][n]
    void *dBt;            // transposed B input, up to L*n*n int32
    int *dFlag;           // device error flags
    // staging for host-buffer entry points (allocated on first use), and two
    // pinned host chunks the caller's memory is copied through (pin[b] is
    // reusable once pev[b], recorded after its last transfer, has completed)
    void *dInA, *dInB, *dOut;
    size_t inBytes, outBytes;
    void *pin[2];
    hipEvent_t pev[2];
    size_t bytes;         // device bytes held
    // last product: output kind (0 limbs, 1 coefficient planes, 2 fp32),
    // output limbs, whether the carry ran inside the inverse kernel
    int last_out, last_RL, last_fused;
    // set by the float entry points around a product: the inverse kernels
    // that can decode into fp32 / fp64 (MFH_DEC_* + 1; 0 = none) do so,
    // writing dec_out with scale 2^-dec_SAB, instead of writing Cw
    int dec_req, dec_SAB;
    void *dec_out;
    // timing: ev[0] start, ev[4] end; per row band b, bev[b][0..3] before
    // A's forward transform, after it, after the pointwise step, after the
    // inverse (nbands of them)
    int timing;
    int nbands;
    hipEvent_t ev[5];
    hipEvent_t bev[MFH_BANDS_MAX][4];
    float stage_ms[5];
};

// kernel launchers (mfh_transform.hip, mfh_pointwise.hip)
int mfh_launch_transpose(const void *src, void *dst, int planes, int n,
                         int elem_bytes, hipStream_t st);
// Row bands: the forward transform of padded rows [r0, r0 + rows) of an
// operand (digit planes of rows x np), the pointwise products of A's band
// with all of B, and the inverse of the band's elements (rows r0.. below n,
// written at their places in the n x n outputs).  rows is a multiple of 64,
// or reaches np.
// side: 0 for A, 1 for B (the operand slots differ under MFH_PW_GAUSS)
int mfh_launch_forward(mfh_ctx *c, int in_kind, const void *src, int8_t *dst,
                       int scale_S, int r0, int rows, int side);
int mfh_launch_check_i32(mfh_ctx *c, const int32_t *src, int planes);
int mfh_launch_pointwise(mfh_ctx *c, int rows);
// ring sizes K with a Gauss pointwise kernel
bool mfh_gauss_supported(int K);
// out != nullptr asks for the carry into RL uint16 limbs to be fused;
// *carried tells whether it was (else Cw holds the coefficient planes)
int mfh_launch_inverse(mfh_ctx *c, int64_t *Cw, uint16_t *out, int RL, int *carried, int r0,
                       int rows);
int mfh_launch_carry(mfh_ctx *c, const int64_t *Cw, uint16_t *out, int RL);
// out[u][r] = sum_k limb_u(r, k) over the rows r of L uint16 planes of n x n,
// limb L-1 taken as x - 2^15 (offset mode)
int mfh_launch_offset_sums(const uint16_t *src, int64_t *out, int n, int L, hipStream_t st);
int mfh_launch_carry_planes(const int64_t *Cw, int P, size_t nn, uint16_t *out,
                            int RL, hipStream_t st);
// fp32 (is_f64 = 0) or fp64 matrix -> L signed limb planes at scale 2^S
int mfh_launch_encode(const void *X, int is_f64, int n, int L, int S, int32_t *out,
                      hipStream_t st);
// fp32 (is_f64 = 0) or fp64 matrix -> the L + 1 two's complement uint16 limb
// planes of the value mfh_launch_encode puts on an L-limb grid (the
// multi-modular product's input form)
int mfh_launch_encode_tc(const void *X, int is_f64, int n, int L, int S, uint16_t *out,
                         hipStream_t st);
// RLr carried two's complement limb planes -> floats at scale 2^-SAB, the
// decode of the coefficient planes of the same value (fmt: MFH_DEC_F32/F64)
int mfh_launch_decode_limbs(const uint16_t *limbs, size_t nn, int RLr, int SAB, int fmt,
                            void *out, int32_t *out2, hipStream_t st);
// 2L-1 coefficient planes -> floats at scale 2^-SAB (fmt: MFH_DEC_*)
int mfh_launch_decode(mfh_ctx *c, const int64_t *Cw, int SAB, int fmt, void *out,
                      int32_t *out2);
int mfh_launch_rand_u16(void *dst, size_t count, uint64_t seed, hipStream_t st);
// schoolbook (mfh_limbplane.hip): C += sign A B; Cw[w] = sum_{u+v=w} A_u B_v
// over limb planes of kind MFH_IN_U16, MFH_IN_U16_SIGNED or MFH_IN_I32
int mfh_launch_mm_accum(int64_t *C, const int32_t *A, const int32_t *B, int n, int sign,
                        hipStream_t st);
int mfh_launch_conv_limbplane(int64_t *Cw, const void *A, const void *B, int in_kind, int n,
                              int L, hipStream_t st);
// the schoolbook on the matrix cores: K7 digit planes of NLp >= L limbs
// (16 x 64 tiles over np x np), the int32 partials P[6][2NU-1][np][np][32]
// of the 16-limb block pairs (mfh_pointwise.hip), and their recombination
// into 2L-1 int64 planes (Cw) or RL carried uint16 limbs (out); lo: the
// lower end of every partial's range (width below 2^32)
int mfh_launch_sb_digits(const void *src, int in_kind, int8_t *out, int n, int np_, int L,
                         int NLp, hipStream_t st);
int mfh_launch_schoolbook(const int8_t *Ad, const int8_t *Bd, int32_t *P, int np_, int NU,
                          hipStream_t st);
int mfh_launch_sb_combine(const int32_t *P, int64_t *Cw, uint16_t *out, int RL, int n, int np_,
                          int L, int NU, long long lo, hipStream_t st);
// entry-major uint16 limbs (e[idx*L + u]) -> plane-major
int mfh_launch_entry_to_plane(const uint16_t *e, uint16_t *p, int n, int L, hipStream_t st);
// C[t] = lin[t] - lin[t+K], t < K (negacyclic fold of 2K-1 planes)
int mfh_launch_negfold(const int64_t *lin, int64_t *C, int n, int K, hipStream_t st);
int mfh_launch_copy16(void *dst, const void *src, size_t bytes, hipStream_t st);
int mfh_launch_rand_f32(void *dst, size_t count, uint64_t seed, int emin,
                        int emax, hipStream_t st);

// input kinds used internally for fixed-point float sources
#define MFH_IN_F32 100
#define MFH_IN_F64 101
// unsigned limbs read with 2^(16L-1) subtracted (the top limb as
// (int16)(x ^ 0x8000)); only the recoding forward transform takes it
#define MFH_IN_U16_OFFSET 102
// decode formats: fp32, fp64, 63-bit significand + exponent (long double)
#define MFH_DEC_F32 0
#define MFH_DEC_F64 1
#define MFH_DEC_SIG63 2

#define MFH_HIP(call)                                   \
    do {                                                \
        hipError_t e_ = (call);                         \
        if (e_ != hipSuccess) return MFH_E_HIP;         \
    } while (0)
