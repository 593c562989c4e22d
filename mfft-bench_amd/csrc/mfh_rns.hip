// mfh_rns.hip -- exact product of big-integer matrices by multi-modular
// (residue number system) arithmetic on the gfx950 int8 matrix cores.
//
// No counterpart in the reference: it computes the same function as
// mm_mfft / mm_limbplane (src/mfft.c:424-438, src/methods.c:106-123) -- the
// exact product of two n x n matrices of W = 16 L-bit integers, carried into
// RL uint16 limbs modulo 2^(16 RL) -- by another algorithm.  The MFFT issues
// NB K^2 small-integer GEMMs, about 8 L S of them (S ~ sqrt(L/2)); residues
// modulo 16-bit primes need about 2 (2W + log2 n) / 16 primes of 4 int8
// GEMMs each, linear in W.
//
// An entry of A B has at most 2W + log2(n) bits.  It is fixed by its
// residues modulo nm distinct primes p_m <= 65279 whose product M exceeds
// 4 n 2^(2W) (so |C| <= M/4 for unsigned and two's complement entries):
//   1. residues (k_rns_residue): an entry with bytes b_t (t < 2L) is
//        x = sum_t b_t 256^t  [- 2^W if it is a negative two's complement],
//      so x = sum_t (b_t - 128) w_{m,t} + 128 sum_t w_{m,t} [- 2^W]
//      (mod p_m) with w_{m,t} = 256^t mod p_m: an int8 GEMM of the shifted
//      bytes against the two balanced base-2^8 digits of the weights (two
//      int32 sums per prime, |sum| <= 2L 2^14), then reduced exactly in fp64.
//      A residue r is kept balanced, |r| <= (p-1)/2 <= 32639, as its two
//      balanced base-2^8 digits lo = ((r+128) & 255) - 128,
//      hi = (r - lo)/256, both int8: the uint16 "digit pair" lo | hi << 8;
//   2. pointwise (k_rns_pointwise): per prime, C_m = A_m B_m over the digit
//      pairs: four int8 GEMMs into three int32 classes hh, hl + lh, ll
//      (|class| <= 2 n 2^14), recombined exactly in fp64 as
//      65536 hh + 256 (hl+lh) + ll, reduced mod p_m, multiplied by
//      cinv_m = (M/p_m)^-1 mod p_m and reduced again: y_m, a digit pair;
//   3. CRT (k_rns_crt): C = sum_m y_m M/p_m - q M, q = round(sum_m y_m/p_m)
//      (exact: the fp64 sum errs by far less than the 1/4 margin).  The sum
//      is an int8 GEMM of the y digits against the balanced base-2^8 digits
//      of M/p_m (for lo) and of 256 M/p_m (for hi), one int32 column per
//      output byte (|column| <= 2 nm 2^14); q times the digits of M is
//      subtracted per column, groups of four columns are combined into int64
//      values of weight 2^(32 g), and the groups are carried into RL uint16
//      limbs by carry lookahead.  Everything is computed modulo
//      256^Jpad, Jpad >= 2 (2L+1) bytes: the RL <= 2L+1 output limbs are
//      exact; limbs beyond 2L+1 are the sign extension.  When 4L is a
//      multiple of 64 (L a multiple of 16) that would spend a whole 64-byte
//      chunk on the top limb's 2 bytes: then Jpad = 4L and limb 2L is
//      floor(C / 2^(32L)) mod 2^16, from C = M (t - q), t = sum_m y_m/p_m:
//      round(M 2^(-32L) (t - q) - low 2^(-32L)) with low = C mod 2^(32L)
//      (its top word suffices); the fp64 error, M 2^(-32L) nm^2 2^-53 with
//      t's summation, is checked on the host to be below 1/16.
//
// MFMA: v_mfma_i32_16x16x64_i8.  Operand fragments: lane l holds row l%16 and
// 16 k bytes 16 (l/16) .. +15 (A and B use the same k order); results: lane
// l, value v is row 4 (l/16) + v, column l%16.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <type_traits>
#include <vector>

#include "mfh_internal.hpp"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// per prime: p, the residue offsets k0 = 128 sum_t w_t and k1 = k0 - 2^W
// (mod p, in [0, p)), cinv = (M/p)^-1 mod p, 1/p, and the offsets of the
// scaled residues (B's, times cinv): k0b = k0 cinv, k1b = k1 cinv (mod p)
struct RnsMod {
    int p, k0, k1, cinv;
    double invp;
    int k0b, k1b;
};
static_assert(sizeof(RnsMod) == 32, "RnsMod layout");

constexpr int kPrimeMax = 65279;   // (p-1)/2 <= 32639 keeps the hi digit in int8
constexpr int kPrimeMin = 16411;   // smallest prime the plans draw on

// Balanced residue of an exact integer v held in a double, |v| <= 2^46:
// q = rint(v / p) computed as rint(v * fl(1/p)), r = v - q p (exact, the
// result is small).  v * fl(1/p) errs from v/p by at most 2^-22, while v/p
// (p odd) is at least 1/(2p) > 2^-17 from any half-integer, so q is the
// nearest integer and |r| <= (p-1)/2 with no correction step.
__device__ __forceinline__ int rns_reduce(double v, int p, double invp)
{
    const double q = rint(v * invp);
    return (int)fma(-q, (double)p, v);
}

// The same for an int32 v, with p given as a double: q as above,
// r = v - q p by one fma (exact: the result is small)
__device__ __forceinline__ int rns_reduce_i32(int v, double p, double invp)
{
    const double vd = (double)v;
    const double q = rint(vd * invp);
    return (int)fma(-q, p, vd);
}

// digit pair of a balanced residue r, |r| <= 32639: with t = r + 128,
// lo = (t & 255) - 128 and hi = t >> 8, so the pair lo | hi << 8 (as bytes)
// is t ^ 0x80 in the low 16 bits
__device__ __forceinline__ uint16_t rns_pair(int r)
{
    return (uint16_t)((r + 128) ^ 0x80);
}

__device__ __forceinline__ int rns_unpair(uint16_t w)
{
    return (int)(int8_t)(w >> 8) * 256 + (int)(int8_t)(w & 255);
}

// s_waitcnt vmcnt(V) lgkmcnt(0) (gfx9 encoding: vmcnt bits 3:0 and 15:14)
template <int V>
__device__ __forceinline__ void wait_vm_lgkm()
{
    __builtin_amdgcn_s_waitcnt((V & 15) | (7 << 4) | (0 << 8) | ((V >> 4) << 14));
}

// ---- 1. residues -----------------------------------------------------------
// X: L uint16 limb planes of an n x n matrix (plane u at X + u n^2), read as
// the GEMM operand "rows r, inner index k" (A, or B^T).  R: nm digit-pair
// planes of np x np (row stride np), zero outside n x n.  A wave owns EB
// blocks of 16 consecutive k of row r = blockIdx.y and keeps their byte
// fragments of all KB 64-byte k blocks in registers; W holds the weight
// fragments [ceil(nm/8)][KB][64 lanes][16 B]: fragment (ob, kb) row
// o = 16 ob + l%16 is digit o%2 (0: lo, 1: hi) of w_{8 ob + o/2, t},
// t = 64 kb + byte (zero past the last prime).
// scaled: W holds the weights times cinv (B's residues, so that the
// per-prime products come out already multiplied by cinv), with the offsets
// k0b / k1b
template <int KB, int EB>
__global__ __launch_bounds__(256) void k_rns_residue(const uint16_t *__restrict__ X, int n,
                                                     int np_, int L, int sgn, int scaled,
                                                     const v4i *__restrict__ W,
                                                     const RnsMod *__restrict__ mods, int nm,
                                                     uint16_t *__restrict__ R)
{
    constexpr int NE = 64 * EB;                  // elements of the workgroup
    constexpr int RS = NE + 4;                   // LDS row stride (u16): the 4 lane
                                                 // groups' rows fall in distinct banks
    __shared__ __align__(16) uint16_t stg[2][32][RS];
    // per wave: the digit pairs of 8 primes x 16 EB elements, rows padded so
    // that the four lane groups' writes fall in distinct banks
    __shared__ __align__(16) uint16_t tr[4][8][16 * EB + 8];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int r = blockIdx.y;
    const int kw0 = blockIdx.x * NE;             // first element of the workgroup
    const int k0 = kw0 + wave * 16 * EB;         // first element of this wave
    const size_t nn = (size_t)n * n, npp = (size_t)np_ * np_;
    // The limbs reach the registers through LDS, 32 limb planes at a time:
    // 16-byte loads of 8 consecutive elements of one plane (coalesced; NE/64
    // per thread and chunk), the next chunk's loads in flight while this
    // chunk's fragments are read (two LDS buffers).  Limbs at or past L,
    // rows at or past n and elements at or past n read as zero.
    const bool vec = (n & 7) == 0 && ((uintptr_t)X & 15) == 0;   // 16-byte aligned rows
    uint2 pre[EB][2];
    auto load_chunk = [&](int kb) {
#pragma unroll
        for (int i = 0; i < EB; ++i) {
            const int idx = threadIdx.x + 256 * i;
            const int pl = idx / (NE / 8), g8 = idx % (NE / 8);
            const int u = 32 * kb + pl, k = kw0 + 8 * g8;
            uint4 v = uint4{0, 0, 0, 0};
            if (r < n && u < L) {
                const uint16_t *src = X + (size_t)u * nn + (size_t)r * n + k;
                if (vec && k + 8 <= n) {
                    v = *(const uint4 *)src;
                } else {
                    uint32_t w[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) w[j] = k + j < n ? src[j] : 0;
                    v = uint4{w[0] | w[1] << 16, w[2] | w[3] << 16, w[4] | w[5] << 16,
                              w[6] | w[7] << 16};
                }
            }
            pre[i][0] = uint2{v.x, v.y};
            pre[i][1] = uint2{v.z, v.w};
        }
    };
    v4i ef[KB][EB];
    int sb[EB];
    bool ok[EB];
#pragma unroll
    for (int cb = 0; cb < EB; ++cb) {
        const int k = k0 + 16 * cb + col;
        ok[cb] = r < n && k < n;
        sb[cb] = 0;
    }
    load_chunk(0);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        uint16_t (*buf)[RS] = stg[kb & 1];
#pragma unroll
        for (int i = 0; i < EB; ++i) {
            const int idx = threadIdx.x + 256 * i;
            const int pl = idx / (NE / 8), g8 = idx % (NE / 8);
            *(uint2 *)&buf[pl][8 * g8] = pre[i][0];
            *(uint2 *)&buf[pl][8 * g8 + 4] = pre[i][1];
        }
        __syncthreads();
        if (kb + 1 < KB) load_chunk(kb + 1);
#pragma unroll
        for (int cb = 0; cb < EB; ++cb) {
            const int e = wave * 16 * EB + 16 * cb + col;
            uint32_t d[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int u = 8 * grp + 2 * q;
                d[q] = ((uint32_t)buf[u][e] | ((uint32_t)buf[u + 1][e] << 16)) ^ 0x80808080u;
            }
            ef[kb][cb] = v4i{(int)d[0], (int)d[1], (int)d[2], (int)d[3]};
            // the sign of a two's complement entry: bit 15 of limb L-1
            if (sgn && kb == (L - 1) / 32) sb[cb] = ok[cb] ? buf[(L - 1) % 32][e] >> 15 : 0;
        }
    }
    // Weight fragments of later blocks of 8 primes are in flight while
    // block ob is multiplied.  Up to 8 k blocks each wave prefetches block
    // ob + 1 into registers.  Beyond that (the registers hold the element
    // fragments) the workgroup copies each block once into LDS by
    // buffer-to-LDS copies, two blocks ahead into three buffers, and its
    // four waves read it there (when every wave loaded the block itself, the
    // weight stream from L2 bounded the kernel at 16 k blocks: 0.79 ms per
    // operand at 8192 bits, n = 256).  Each buffer is its own array, picked
    // at compile time (the loop runs in threes): with one array indexed by
    // the block the compiler waited for the copies just issued into the
    // next buffer before reading the current one.
    constexpr int PF = KB <= 8 ? KB : 0;
    constexpr int KL = PF ? 1 : KB;
    __shared__ __align__(16) v4i wl0[KL][64], wl1[PF ? 1 : KL][64], wl2[PF ? 1 : KL][64];
    const int nob = (nm + 7) / 8;            // blocks of 8 primes, the last partial
    // copies of block ob (KL / 4 per wave) into buffer B
    auto wcopy = [&](auto btag, int ob) {
        constexpr int B = decltype(btag)::value;
        v4i (*dst)[64] = B == 0 ? wl0 : B == 1 ? wl1 : wl2;
#pragma unroll
        for (int i = 0; i < KL / 4; ++i) {
            const int kb = wave + 4 * i;
            __builtin_amdgcn_global_load_lds((const void *)(W + ((size_t)ob * KB + kb) * 64 + lane),
                                             (void *)&dst[kb][0], 16, 0, 0);
        }
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    using B2 = std::integral_constant<int, 2>;
    v4i wn[PF > 0 ? PF : 1];
    // the constants of the lane's two primes of the next block load during
    // the current one (up to 2 k blocks, where registers are to spare, and
    // on the LDS path)
    constexpr bool MPF = KB <= 2 || !PF;
    RnsMod mdn[MPF ? 2 : 1];
    auto mload = [&](int ob) {
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
            const int m = 8 * ob + 2 * grp + mm;
            mdn[mm] = mods[m < nm ? m : 0];
        }
    };
    if constexpr (PF) {
        if (k0 >= np_) return;                   // past the padded row (after the barriers)
#pragma unroll
        for (int kb = 0; kb < PF; ++kb) wn[kb] = W[(size_t)kb * 64 + lane];
        if constexpr (MPF) mload(0);
    } else {
        mload(0);
        wcopy(B0{}, 0);
        wcopy(B1{}, nob > 1 ? 1 : 0);
    }
    // Block ob, its weights in buffer B (LDS path).  The prefetches are
    // unconditional (past the end the last block loads itself again): a
    // branch around them had made the compiler wait for every load where
    // the paths join.
    auto block = [&](auto btag, int ob) {
        constexpr int B = decltype(btag)::value;
        v4i acc[EB];
#pragma unroll
        for (int cb = 0; cb < EB; ++cb) acc[cb] = v4i{0, 0, 0, 0};
        const int obn = ob + 1 < nob ? ob + 1 : ob;
        RnsMod mdc[MPF ? 2 : 1];
        v4i wc[PF > 0 ? PF : 1];
        if constexpr (PF) {
            if constexpr (MPF) {
#pragma unroll
                for (int mm = 0; mm < 2; ++mm) mdc[mm] = mdn[mm];
                mload(obn);
            }
#pragma unroll
            for (int kb = 0; kb < PF; ++kb) {
                wc[kb] = wn[kb];
                wn[kb] = W[((size_t)obn * KB + kb) * 64 + lane];
            }
        } else {
            // Issue order per block: the constants of block ob + 1, then the
            // copies of block ob + 2.  Loads complete in order, so with only
            // the KL / 4 youngest loads (the copies of block ob + 1) left in
            // flight this wave's copies of block ob and the constants of
            // block ob have landed; after the barrier every wave's copies
            // have, and every wave has finished reading buffer (B + 2) % 3
            // (block ob - 1), which the copies of block ob + 2 then overwrite.
            // (A plain s_barrier: __syncthreads' fence would wait for every
            // copy in flight.)
            wait_vm_lgkm<KL / 4>();
            __builtin_amdgcn_s_barrier();
#pragma unroll
            for (int mm = 0; mm < 2; ++mm) mdc[mm] = mdn[mm];
            mload(obn);
            wcopy(std::integral_constant<int, (B + 2) % 3>{}, ob + 2 < nob ? ob + 2 : nob - 1);
        }
        v4i (*wb)[64] = B == 0 ? wl0 : B == 1 ? wl1 : wl2;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            const v4i w = PF ? wc[kb < PF ? kb : 0] : wb[PF ? 0 : kb][lane];
#pragma unroll
            for (int cb = 0; cb < EB; ++cb)
                acc[cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w, ef[kb][cb], acc[cb], 0, 0, 0);
        }
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
            const int m = 8 * ob + 2 * grp + mm;
            const RnsMod md = MPF ? mdc[MPF ? mm : 0] : mods[m < nm ? m : 0];
            const int off0 = scaled ? md.k0b : md.k0, off1 = scaled ? md.k1b : md.k1;
            const double pd = (double)md.p;
#pragma unroll
            for (int cb = 0; cb < EB; ++cb) {
                const int off = sb[cb] ? off1 : off0;
                int rr;
                if constexpr (KB <= 4) {
                    // |acc| <= 64 KB 2^14 <= 2^22: 256 acc_hi + acc_lo + off
                    // is below 2^31 in magnitude, exact in int32
                    rr = rns_reduce_i32(acc[cb][2 * mm + 1] * 256 + acc[cb][2 * mm] + off, pd,
                                        md.invp);
                } else {
                    const double v = (double)acc[cb][2 * mm + 1] * 256.0 +
                                     (double)acc[cb][2 * mm] + (double)off;
                    rr = rns_reduce(v, md.p, md.invp);
                }
                tr[wave][2 * grp + mm][16 * cb + col] = ok[cb] && m < nm ? rns_pair(rr) : 0;
            }
        }
        // the wave's 16 EB consecutive elements of 8 primes, 16 bytes per
        // lane: each store writes whole lines of the planes (none past the
        // padded row: without the early return the LDS path keeps every wave
        // in its barriers)
        if (lane < 16 * EB && k0 < np_) {
            const int pm = lane / (2 * EB), ch = lane % (2 * EB);
            const int m = 8 * ob + pm;
            const uint4 v = *(const uint4 *)&tr[wave][pm][8 * ch];
            if (m < nm) *(uint4 *)(R + (size_t)m * npp + (size_t)r * np_ + k0 + 8 * ch) = v;
        }
    };
    if constexpr (PF) {
#pragma unroll 1
        for (int ob = 0; ob < nob; ++ob) block(B0{}, ob);
    } else {
        int ob = 0;
#pragma unroll 1
        for (; ob + 3 <= nob; ob += 3) {
            block(B0{}, ob);
            block(B1{}, ob + 1);
            block(B2{}, ob + 2);
        }
        if (ob < nob) block(B0{}, ob);
        if (ob + 1 < nob) block(B1{}, ob + 1);
        // the copies still in flight land before the workgroup's LDS is
        // given to another
        wait_vm_lgkm<0>();
    }
}

// ---- 2. pointwise ----------------------------------------------------------
// Per prime m: the 128 x 128 output tile (ti, tj) of A_m B_m^T over the
// digit pairs (RA rows i, RB rows j, both k-contiguous, np x np), four
// waves of 64 x 64.  k blocks of 64 reach LDS by buffer-to-LDS copies, three
// stages deep (each stage its own array, so that the compiler does not wait
// for copies into one stage before reading another).  Stage layout per
// operand: 8 blocks of 16 rows; a block is 128 16-byte chunks, chunk
// (2 kq + h) 16 + r holding words 16 kq + 8 h .. +7 of row r, so lane l of a
// fragment reads chunks 32 (l/16) + l%16 and 32 (l/16) + 16 + l%16.
struct PwStage {
    v4i a[8][128];
    v4i b[8][128];
};

// NW waves issue the 32 copies of a stage (16 A, 16 B), 32 / NW each
template <int NW>
__device__ __forceinline__ void rns_issue(PwStage &st, const char *a0, const char *b0,
                                          size_t rowb, int kb, int wave, const uint32_t off[2])
{
#pragma unroll
    for (int ii = 0; ii < 32 / NW; ++ii) {
        const int idx = wave + NW * ii;              // 0..31
        const int opnd = idx >> 4, rb = (idx & 15) >> 1, sh = idx & 1;
        const char *src = (opnd ? b0 : a0) + (size_t)16 * rb * rowb + (size_t)kb * 128 + off[sh];
        v4i *dst = opnd ? &st.b[rb][64 * sh] : &st.a[rb][64 * sh];
        __builtin_amdgcn_global_load_lds((const void *)src, (void *)dst, 16, 0, 0);
    }
}

__device__ __forceinline__ void rns_split(const v4i d0, const v4i d1, v4i &lo, v4i &hi)
{
    // d0: words 0..7 (2 per dword), d1: words 8..15; word = lo byte | hi byte << 8
    lo = v4i{(int)__builtin_amdgcn_perm((uint32_t)d0.y, (uint32_t)d0.x, 0x06040200u),
             (int)__builtin_amdgcn_perm((uint32_t)d0.w, (uint32_t)d0.z, 0x06040200u),
             (int)__builtin_amdgcn_perm((uint32_t)d1.y, (uint32_t)d1.x, 0x06040200u),
             (int)__builtin_amdgcn_perm((uint32_t)d1.w, (uint32_t)d1.z, 0x06040200u)};
    hi = v4i{(int)__builtin_amdgcn_perm((uint32_t)d0.y, (uint32_t)d0.x, 0x07050301u),
             (int)__builtin_amdgcn_perm((uint32_t)d0.w, (uint32_t)d0.z, 0x07050301u),
             (int)__builtin_amdgcn_perm((uint32_t)d1.y, (uint32_t)d1.x, 0x07050301u),
             (int)__builtin_amdgcn_perm((uint32_t)d1.w, (uint32_t)d1.z, 0x07050301u)};
}

// a wave's accumulators: AB row blocks x 4 column blocks of 16 x 16, three
// classes each
template <int AB>
struct PwAcc {
    v4i hh[AB][4], md[AB][4], ll[AB][4];
};

template <int AB>
__device__ __forceinline__ void rns_compute(const PwStage &st, int wi, int wj, int lane,
                                            PwAcc<AB> &c)
{
    const int c0 = 32 * (lane >> 4) + (lane & 15);
    // every fragment read of the block issued before any is used (a fence
    // keeps the compiler from waiting for each pair before the next)
    v4i ra[AB][2], rb[4][2];
#pragma unroll
    for (int a = 0; a < AB; ++a) {
        ra[a][0] = st.a[AB * wi + a][c0];
        ra[a][1] = st.a[AB * wi + a][c0 + 16];
    }
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        rb[b][0] = st.b[4 * wj + b][c0];
        rb[b][1] = st.b[4 * wj + b][c0 + 16];
    }
    __builtin_amdgcn_sched_barrier(0);
    v4i alo[AB], ahi[AB], blo[4], bhi[4];
#pragma unroll
    for (int a = 0; a < AB; ++a) rns_split(ra[a][0], ra[a][1], alo[a], ahi[a]);
#pragma unroll
    for (int b = 0; b < 4; ++b) rns_split(rb[b][0], rb[b][1], blo[b], bhi[b]);
    // dependent MFMAs into md are 4 AB issues apart
#pragma unroll
    for (int a = 0; a < AB; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
            c.hh[a][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[a], bhi[b], c.hh[a][b], 0, 0, 0);
#pragma unroll
    for (int a = 0; a < AB; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
            c.md[a][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[a], blo[b], c.md[a][b], 0, 0, 0);
#pragma unroll
    for (int a = 0; a < AB; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
            c.ll[a][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[a], blo[b], c.ll[a][b], 0, 0, 0);
#pragma unroll
    for (int a = 0; a < AB; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
            c.md[a][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[a], bhi[b], c.md[a][b], 0, 0, 0);
}

// Persistent workgroups, one per CU: workgroup b runs on XCD b mod 8 and
// takes every wx-th (prime, tile) item of its XCD's range of the list (all
// tiles of one prime after another; XCD x gets the R items from x R, R a
// multiple of the BR x BC block), so the wx workgroups of an XCD run one
// block of BR x BC tiles of one prime at a time and share its operand panels
// in the XCD's L2, and the XCDs get equal shares of the work whatever the
// number of primes.  The copy pipeline runs across tile boundaries:
// the first k blocks of a workgroup's next tile load while it finishes the
// current one and writes its results.
struct TileMap {
    int tpr, BR, BC;
    __device__ void tile(int t, int &ti, int &tj) const
    {
        const int b = t / (BR * BC), w = t % (BR * BC), nbj = tpr / BC;
        ti = (b / nbj) * BR + w / BC;
        tj = (b % nbj) * BC + w % BC;
    }
};

template <int AB>
__global__ __launch_bounds__(64 * 2 * (8 / AB)) void k_rns_pointwise(
    const uint16_t *__restrict__ RA, const uint16_t *__restrict__ RB,
    const RnsMod *__restrict__ mods, int nm, int np_, uint16_t *__restrict__ Y, int wx,
    TileMap tm, int R)
{
    constexpr int NW = 2 * (8 / AB);
    __shared__ PwStage s0, s1, s2;
    // per wave: its 32 x 64 digit pairs of the finished tile, rows padded so
    // that the four lane groups' writes fall in distinct banks
    __shared__ __align__(16) uint16_t ytr[NW][16 * AB][72];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wi = wave >> 1, wj = wave & 1;
    const int T = tm.tpr * tm.tpr, nkb = np_ / 64;
    const int xcd = blockIdx.x & 7, k = blockIdx.x >> 3;
    // this XCD's items: [lo, hi) of the (prime, tile) list, prime-major
    const int N = nm * T, lo = min(xcd * R, N), hi = min(lo + R, N);
    const int items = hi - lo;
    const int mine = items > k ? (items - k + wx - 1) / wx : 0;
    const int G = mine * nkb;                // k-block steps of this workgroup
    if (G == 0) return;
    const size_t npp = (size_t)np_ * np_, rowb = (size_t)np_ * 2;
    uint32_t off[2];
#pragma unroll
    for (int sh = 0; sh < 2; ++sh) {
        const int c = 64 * sh + lane;
        off[sh] = (uint32_t)((c & 15) * rowb + (16 * (c >> 5) + 8 * ((c >> 4) & 1)) * 2);
    }
    // item it -> prime and output tile
    auto decode = [&](int it, int &m, int &ti, int &tj) {
        m = it / T;
        tm.tile(it % T, ti, tj);
    };
    // producer cursor: the next block to copy (item p_it, k block p_kb); the
    // divisions run once per item, not per block
    const int last_it = lo + k + wx * (mine - 1);
    int p_it = lo + k, p_kb = 0;
    const char *pa, *pb;
    auto panels = [&]() {
        int m, ti, tj;
        decode(p_it, m, ti, tj);
        pa = (const char *)(RA + m * npp + (size_t)ti * 128 * np_);
        pb = (const char *)(RB + m * npp + (size_t)tj * 128 * np_);
    };
    panels();
    // copy the cursor's block and advance it (past the last block it stays
    // there: the extra copies repeat the last block)
    auto issue = [&](PwStage &st) {
        rns_issue<NW>(st, pa, pb, rowb, p_kb, wave, off);
        if (++p_kb == nkb) {
            if (p_it < last_it) {
                p_kb = 0;
                p_it += wx;
                panels();
            } else {
                p_kb = nkb - 1;
            }
        }
    };
    PwAcc<AB> acc;
    auto zero = [&]() {
#pragma unroll
        for (int a = 0; a < AB; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b) acc.hh[a][b] = acc.md[a][b] = acc.ll[a][b] = v4i{0, 0, 0, 0};
    };
    int c_it = lo + k, c_kb = 0;         // consumer cursor
    auto epilogue = [&]() {
        int m, ti, tj;
        decode(c_it, m, ti, tj);
        c_it += wx;
        const RnsMod md = mods[m];
#pragma unroll
        for (int a = 0; a < AB; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const double cv = (double)acc.hh[a][b][v] * 65536.0 +
                                      (double)acc.md[a][b][v] * 256.0 + (double)acc.ll[a][b][v];
                    // B's residues carry the factor cinv: this is y_m
                    ytr[wave][16 * a + 4 * (lane >> 4) + v][16 * b + (lane & 15)] =
                        rns_pair(rns_reduce(cv, md.p, md.invp));
                }
        // 16 bytes per lane: each store writes whole 128-byte rows of Y
        uint16_t *y = Y + m * npp + (size_t)(ti * 128 + 16 * AB * wi) * np_ + tj * 128 + 64 * wj;
#pragma unroll
        for (int c = 0; c < 2 * AB; ++c) {
            const int row = 8 * c + (lane >> 3), ch = lane & 7;
            *(uint4 *)(y + (size_t)row * np_ + 8 * ch) = *(const uint4 *)&ytr[wave][row][8 * ch];
        }
        zero();
    };
    zero();
    // Three stages, two blocks in flight (a fourth stage measured no
    // faster).  Every step issues exactly 32 / NW copies per wave (past the
    // last step it copies the last block again, into the stage just
    // retired), so the outstanding copies are the same on every path: the
    // compiler's own waits then stay at vmcnt(32 / NW) (with a conditional
    // issue it waited for all copies, the ones just issued included, before
    // every block).  Stage g % 3 is complete once this wave's copies of g
    // are (only those of g + 1 may be outstanding after them) and every wave
    // has passed the barrier; the barrier also retires every read of stage
    // (g + 2) % 3 (step g - 1), which the copies of g + 2 then overwrite.
    issue(s0);
    issue(s1);
#define RNS_STEP(S, SN, GG)                                                    \
    {                                                                          \
        wait_vm_lgkm<32 / NW>();                                               \
        __builtin_amdgcn_s_barrier();                                          \
        issue(SN);                                                             \
        rns_compute<AB>(S, wi, wj, lane, acc);                                 \
        if (++c_kb == nkb) {                                                   \
            c_kb = 0;                                                          \
            epilogue();                                                        \
        }                                                                      \
    }
    // no exits inside the unrolled body: with them the accumulators were
    // copied at every exit and spilled
    int g = 0;
#pragma unroll 1
    for (; g + 3 <= G; g += 3) {
        RNS_STEP(s0, s2, g)
        RNS_STEP(s1, s0, g + 1)
        RNS_STEP(s2, s1, g + 2)
    }
    if (g < G) RNS_STEP(s0, s2, g)
    if (g + 1 < G) RNS_STEP(s1, s0, g + 1)
#undef RNS_STEP
}

TileMap tile_map(int tpr, int wx)
{
    TileMap tm;
    tm.tpr = tpr;
    tm.BC = 1;
    for (int d = 1; d <= 8 && d <= tpr; ++d)
        if (tpr % d == 0) tm.BC = d;
    tm.BR = 1;
    for (int d = 1; d <= wx / tm.BC && d <= tpr; ++d)
        if (tpr % d == 0) tm.BR = d;
    return tm;
}

// ---- 3. CRT and carry ------------------------------------------------------
// E = 16 EB elements (row i = blockIdx.y, columns j0 .. j0+E-1) per
// workgroup of NT / 64 waves.  LDS: the y digit pairs of the E elements as
// MFMA B fragments [KBc][EB][64 lanes][16 B] (fragment (kb, cb): element
// 16 cb + l%16, the digit pairs of primes 32 kb + 8 (l/16) .. +7), one
// pass's int64 groups [16 cpp][E], the carry lookahead's run data, q's
// partial fp64 sums, q, t - q and the carry into the pass per element.  T
// holds the A fragments [Jpad/16][KBc][64][16 B]: row j (output byte) of
// k = 2m + d is byte j of M/p_m (d = 0) or of 256 M/p_m (d = 1), zero for
// m >= nm.
// NT threads (512, or 256 for narrow outputs of at most four chunks);
// KBB: the T fragments of a chunk are loaded in batches of KBB k blocks,
// double-buffered (DBL), or all at once (KBB >= KBc, one wait per chunk).
// Wide outputs run in nh passes over ranges of cpp = ceil(nch / nh) output
// chunks, low to high: the LDS then holds one pass's int64 groups, which
// leaves room for more elements per workgroup (each T fragment serves E
// elements), and each pass carries into the next.  MP: compiled for more
// than one pass (otherwise nh = 1 and the pass loop folds away, which keeps
// the single-pass kernels' registers as they were).
template <int EB, int NT, int KBB, bool DBL, bool MP>
__global__ __launch_bounds__(NT) void k_rns_crt(
    const uint16_t *__restrict__ Y, int n, int np_, int nm, int KBc, int Jpad, int nh, double mtop,
    const v4i *__restrict__ T, const int8_t *__restrict__ mb, const RnsMod *__restrict__ mods,
    uint16_t *__restrict__ out, int RL, int RLc)
{
    constexpr int E = 16 * EB, SEGS = NT / E, NW = NT / 64;
    const int nch = Jpad / 64, cpp = MP ? (nch + nh - 1) / nh : nch;
    extern __shared__ __align__(16) unsigned char smem[];
    v4i *yl = (v4i *)smem;                                        // KBc*EB*64
    long long *grp = (long long *)(yl + (size_t)KBc * EB * 64);  // [16 cpp][E]
    long long *segc = grp + (size_t)16 * cpp * E;                 // [SEGS][E] x 4
    long long *seglo = segc + NT, *seghi = seglo + NT, *segin = seghi + NT;
    double *qs = (double *)(segin + NT);                          // [NT]
    long long *qv = (long long *)(qs + NT);                       // [E]
    long long *cin = qv + E;                                      // [E]: carry into the pass
    double *qf = (double *)(cin + E);                             // [E]: t - q

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i = blockIdx.y, j0 = blockIdx.x * E;
    const size_t npp = (size_t)np_ * np_, nn = (size_t)n * n;

    // 1. y digit pairs into LDS, and sum_m y_m / p_m.  A thread takes one
    //    element and groups of 8 primes: 8 loads of one digit pair each
    //    (each coalesced over the E consecutive elements of the workgroup),
    //    then one 16-byte write of its fragment slot (lane group pg % 4 of
    //    k block pg / 4, element e).  Columns at or beyond n hold y = 0
    //    (their operand rows were zero), so they need no check.
    {
        const int e = tid % E, mg = tid / E;
        const uint16_t *src = Y + (size_t)i * np_ + j0 + e;
        double qsum = 0;
        for (int pg = mg; pg < 4 * KBc; pg += SEGS) {
            uint32_t w[8];
            double ip[8];
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const int m = 8 * pg + b;
                w[b] = m < nm ? src[(size_t)m * npp] : 0;
                ip[b] = m < nm ? mods[m].invp : 0.0;
            }
#pragma unroll
            for (int b = 0; b < 8; ++b) qsum += (double)rns_unpair((uint16_t)w[b]) * ip[b];
            const int kb = pg >> 2, ln = (e & 15) + 16 * (pg & 3);
            yl[((size_t)kb * EB + (e >> 4)) * 64 + ln] =
                v4i{(int)(w[0] | w[1] << 16), (int)(w[2] | w[3] << 16), (int)(w[4] | w[5] << 16),
                    (int)(w[6] | w[7] << 16)};
        }
        qs[tid] = qsum;
    }
    __syncthreads();
    if (tid < E) {
        double t = 0;
        for (int r = 0; r < SEGS; ++r) t += qs[r * E + tid];
        qv[tid] = (long long)rint(t);
        qf[tid] = t - rint(t);
        if (MP) cin[tid] = 0;
    }
    __syncthreads();

    // one pass: output chunks c0 .. c1-1, their groups G0 = 16 c0 .. Gb-1
    // that hold output limbs
    auto pass = [&](const int c0, const int c1, const int G0, const int Gb) {
    // 2. byte columns: GEMM over the y digits, q M subtracted, groups of 4.
    //    The work is fragment rows of 16 output bytes (a chunk is 4).  Whole
    //    chunks are dealt to the waves in full rounds; after at least one
    //    full round the rows of the remaining chunks are split into one run
    //    of consecutive rows per wave, so that no SIMD gets a chunk more than
    //    another (2048 bits: 9 chunks over 8 waves, one row each of the
    //    ninth: CRT 1.22 -> 1.10 ms).  Fewer chunks than waves stay whole
    //    (512 bits: 3 chunks over 4 waves; split into runs of 3 rows they
    //    ran 2 % slower, the workgroups sharing a CU already filling it).
    //    Every T fragment of a row serves all EB element blocks, and every y
    //    fragment all rows of a run.  The T fragments stream in batches of KBB k blocks, the next
    //    batch loaded while the current one is multiplied (DBL), or arrive
    //    all at once.
    auto rows = [&](auto nrc, const int row0) {
        constexpr int NR = decltype(nrc)::value;
        v4i acc[NR][EB];
#pragma unroll
        for (int jj = 0; jj < NR; ++jj)
#pragma unroll
            for (int cb = 0; cb < EB; ++cb) acc[jj][cb] = v4i{0, 0, 0, 0};
        const v4i *tp = T + (size_t)row0 * KBc * 64 + lane;
        v4i ta[KBB][NR], tb[DBL ? KBB : 1][NR];
        auto load = [&](v4i (&t)[KBB][NR], int kb0) {
#pragma unroll
            for (int b = 0; b < KBB; ++b)
#pragma unroll
                for (int jj = 0; jj < NR; ++jj)
                    t[b][jj] = kb0 + b < KBc ? tp[((size_t)jj * KBc + kb0 + b) * 64]
                                             : v4i{0, 0, 0, 0};
        };
        auto mul = [&](const v4i (&t)[KBB][NR], int kb0) {
#pragma unroll
            for (int b = 0; b < KBB; ++b) {
                if (kb0 + b >= KBc) continue;
                v4i yf[EB];
#pragma unroll
                for (int cb = 0; cb < EB; ++cb)
                    yf[cb] = yl[((size_t)(kb0 + b) * EB + cb) * 64 + lane];
#pragma unroll
                for (int jj = 0; jj < NR; ++jj)
#pragma unroll
                    for (int cb = 0; cb < EB; ++cb)
                        acc[jj][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(t[b][jj], yf[cb],
                                                                             acc[jj][cb], 0, 0, 0);
            }
        };
        load(ta, 0);
        if constexpr (DBL) {
            for (int kb0 = 0; kb0 < KBc; kb0 += 2 * KBB) {
                load(tb, kb0 + KBB);
                mul(ta, kb0);
                load(ta, kb0 + 2 * KBB);
                mul(tb, kb0 + KBB);
            }
        } else {
            mul(ta, 0);
        }
#pragma unroll
        for (int jj = 0; jj < NR; ++jj)
#pragma unroll
            for (int cb = 0; cb < EB; ++cb) {
                const int el = 16 * cb + (lane & 15);
                const int gi = 4 * (row0 + jj) + (lane >> 4);
                const long long q = qv[el];
                long long g = 0;
#pragma unroll
                for (int v = 3; v >= 0; --v)
                    g = g * 256 + ((long long)acc[jj][cb][v] - q * (long long)mb[4 * gi + v]);
                grp[(size_t)(gi - G0) * E + el] = g;
            }
    };
    const int cfull = c1 - c0 >= NW ? c0 + (c1 - c0) / NW * NW : c1, R = 4 * (c1 - cfull);
    for (int ch = c0 + wave; ch < cfull; ch += NW) rows(std::integral_constant<int, 4>{}, 4 * ch);
    if (R > 0) {                        // R < 4 NW: runs of at most 4 rows
        const int rpw = (R + NW - 1) / NW, r0 = wave * rpw, cnt = min(rpw, R - r0);
        const int row0 = 4 * cfull + r0;
        if (cnt == 4) rows(std::integral_constant<int, 4>{}, row0);
        else if (cnt == 3) rows(std::integral_constant<int, 3>{}, row0);
        else if (cnt == 2) rows(std::integral_constant<int, 2>{}, row0);
        else if (cnt == 1) rows(std::integral_constant<int, 1>{}, row0);
    }
    __syncthreads();

    // 3. carry lookahead over this pass's groups G0 .. Gb-1 (of the Gc that
    // hold the RLc output limbs): SEGS runs of len >= 2 groups per element.
    // A run propagates with carry-in 0 (its 32-bit words Ls, carry-out c);
    // with the true carry-in X (|X| < 2^40) its carry-out is c + 1 when
    // X >= 2^(32 len) - Ls, c - 1 when X < -Ls, else c.  Ls's low 64 bits
    // and whether its higher words are all 0 or all 1 give both thresholds
    // whenever they are representable; otherwise the case cannot occur.  The
    // last run may be shorter and runs past it empty: their carry-outs are
    // not used; the carry into the next pass is the last run's exact one,
    // from its propagation with the true carry-in below.
    // the groups the GEMM covers (with the fp64 top limb, one fewer than
    // the output needs)
    const int Gc = min((RLc + 1) / 2, Jpad / 4);
    int len = (Gb - G0 + SEGS - 1) / SEGS;
    if (len < 2) len = 2;
    const int el = tid % E, sg = tid / E;
    const int g0 = G0 + sg * len, g1 = min(g0 + len, Gb);
    {
        long long cc = 0;
        uint64_t low = 0;
        bool zero_hi = true, ones_hi = true;
        for (int g = g0; g < g1; ++g) {
            const long long v = cc + grp[(size_t)(g - G0) * E + el];
            const uint64_t w = (uint64_t)v & 0xFFFFFFFFull;
            const int ix = g - g0;
            if (ix < 2) low |= w << (32 * ix);
            else {
                zero_hi &= w == 0;
                ones_hi &= w == 0xFFFFFFFFull;
            }
            cc = v >> 32;
        }
        const bool top_clear = (low >> 63) == 0;
        seglo[sg * E + el] = (zero_hi && top_clear) ? -(long long)low : INT64_MIN;
        seghi[sg * E + el] =
            (ones_hi && !top_clear && low != (1ull << 63)) ? (long long)(0 - low) : INT64_MAX;
        segc[sg * E + el] = cc;
    }
    __syncthreads();
    if (tid < E) {
        long long C = MP ? cin[tid] : 0;
        for (int r = 0; r < SEGS; ++r) {
            segin[r * E + tid] = C;
            C = segc[r * E + tid] + (C >= seghi[r * E + tid]) - (C < seglo[r * E + tid]);
        }
    }
    __syncthreads();
    if (j0 + el < n) {
        long long cc = segin[sg * E + el];
        uint16_t *o = out + (size_t)i * n + j0 + el;
        uint32_t top = 0, wl = 0;
        for (int g = g0; g < g1; ++g) {
            const long long v = cc + grp[(size_t)(g - G0) * E + el];
            const uint32_t w = (uint32_t)v;
            const int u = 2 * g;
            o[(size_t)u * nn] = (uint16_t)w;
            top = w & 0xFFFF;
            if (u + 1 < RLc) {
                o[(size_t)(u + 1) * nn] = (uint16_t)(w >> 16);
                top = w >> 16;
            }
            wl = w;
            cc = v >> 32;
        }
        // limb 2 Gc from fp64 (when the GEMM stops one limb short): C's
        // value above the Gc groups is an integer within 1/16 of the estimate
        if (mtop != 0.0 && 2 * Gc < RLc && g1 == Gc && g0 < g1) {
            const long long tl = llrint(mtop * qf[el] - (double)wl * 0x1p-32);
            top = (uint32_t)tl & 0xFFFF;
            o[(size_t)(2 * Gc) * nn] = (uint16_t)top;
        }
        // limbs above 2L+1: the sign extension of limb RLc-1
        if (g1 == Gc && g0 < g1 && RL > RLc) {
            const uint16_t ext = (top & 0x8000) ? 0xFFFF : 0;
            for (int u = RLc; u < RL; ++u) o[(size_t)u * nn] = ext;
        }
    }
    // the exact carry into group Gb (the next pass's carry-in): the last
    // non-empty run's, propagated above with its true carry-in (also for
    // columns at or past n, which write nothing)
    if (MP && g1 == Gb && g0 < g1) {
        long long cc = segin[sg * E + el];
        for (int g = g0; g < g1; ++g) cc = (cc + grp[(size_t)(g - G0) * E + el]) >> 32;
        cin[el] = cc;
    }
    };
    const int Gc = min((RLc + 1) / 2, Jpad / 4);   // groups that hold output limbs
    if constexpr (MP) {
        for (int c0 = 0; c0 < nch && 16 * c0 < Gc; c0 += cpp) {
            const int c1 = min(c0 + cpp, nch);
            pass(c0, c1, 16 * c0, min(16 * c1, Gc));
            __syncthreads();   // grp, the runs and cin are reused by the next pass
        }
    } else {
        pass(0, nch, 0, Gc);
    }
}

size_t crt_lds_bytes(int EB, int NT, int KBc, int Jpad, int nh)
{
    const int E = 16 * EB, cpp = (Jpad / 64 + nh - 1) / nh;
    return (size_t)KBc * EB * 1024 + (size_t)16 * cpp * E * 8 + 5 * NT * 8 + 3 * E * 8;
}

// ---- host planning ---------------------------------------------------------
// primes in [kPrimeMin, kPrimeMax], descending
const std::vector<int> &prime_list()
{
    static std::vector<int> pr;
    if (pr.empty()) {
        std::vector<char> comp(kPrimeMax + 1, 0);
        for (int a = 2; (long long)a * a <= kPrimeMax; ++a)
            if (!comp[a])
                for (int b = a * a; b <= kPrimeMax; b += a) comp[b] = 1;
        for (int p = kPrimeMax; p >= kPrimeMin; --p)
            if (!comp[p]) pr.push_back(p);
    }
    return pr;
}

// the primes of a plan: the largest ones until sum log2 p >= 2W + ceil(log2 n)
// + 3 (M > 4 n 2^(2W) with a bit to spare)
int plan_primes(int n, int L, std::vector<int> &ps)
{
    ps.clear();
    int lg = 0;
    while ((1LL << lg) < n) ++lg;
    const double need = 2.0 * 16 * L + lg + 3;
    const std::vector<int> &pr = prime_list();
    double bits = 0;
    size_t k = 0;
    while (k < pr.size() && bits < need) {
        ps.push_back(pr[k]);
        bits += log2((double)pr[k]);
        ++k;
    }
    if (bits < need) return MFH_E_BOUND;
    return MFH_OK;
}

long long modinv(long long a, long long p)
{
    long long t = 0, nt = 1, r = p, nr = ((a % p) + p) % p;
    while (nr) {
        const long long q = r / nr;
        long long x = t - q * nt; t = nt; nt = x;
        x = r - q * nr; r = nr; nr = x;
    }
    return t < 0 ? t + p : t;
}

// balanced base-256 digits d_j (j < J) of a non-negative integer held as
// little-endian 32-bit words: sum_j d_j 256^j = value mod 256^J
void balanced_bytes(const std::vector<uint32_t> &v, int J, int8_t *d)
{
    int carry = 0;
    for (int j = 0; j < J; ++j) {
        const size_t w = (size_t)j / 4;
        int b = w < v.size() ? (int)((v[w] >> (8 * (j % 4))) & 255) : 0;
        b += carry;
        if (b >= 128) { b -= 256; carry = 1; } else carry = 0;
        d[j] = (int8_t)b;
    }
}

int kres_blocks(int L)
{
    const int kb = (2 * L + 63) / 64;
    int b = 1;
    while (b < kb) b *= 2;
    return b;
}

}  // namespace

struct mfh_rns {
    int n, np, L, nm, nmk, KB, Jpad, crt_eb, crt_nh;
    double mtop;          // M / 2^(8 Jpad) when limb 2L comes from fp64, else 0
    int cus;              // compute units (8 XCDs of cus / 8)
    int dev;
    hipStream_t stream;
    RnsMod *dMod;
    v4i *dW, *dWb, *dT;
    int8_t *dMb;
    uint16_t *dRA, *dRB, *dY, *dBt;
    uint16_t *dFA, *dFB, *dFO;  // fixed-point products: operand and product limbs
    size_t bytes;
    int timing;
    hipEvent_t ev[4];
    std::vector<int> primes;
};

namespace {

int rns_alloc(mfh_rns *r, void **p, size_t bytes)
{
    *p = nullptr;
    if (!bytes) return MFH_OK;
    if (hipMalloc(p, bytes) != hipSuccess) { *p = nullptr; return MFH_E_NOMEM; }
    r->bytes += bytes;
    return MFH_OK;
}

// weight fragments of the residue GEMM (plain, and times cinv for B) and the
// CRT tables
int rns_tables(mfh_rns *r)
{
    const int nm = r->nm, L = r->L, KB = r->KB, Jpad = r->Jpad, nmk = r->nmk;
    const int KBc = nmk / 32;
    std::vector<RnsMod> mods(nm);
    // M and, per prime, cinv = (M/p_m)^-1 mod p_m, (M/p_m) mod p_m being
    // prod_{j != m} p_j mod p_m
    std::vector<uint32_t> M(1, 1);
    for (int m = 0; m < nm; ++m) {
        uint64_t c = 0;
        for (auto &x : M) {
            const uint64_t v = (uint64_t)x * (uint64_t)r->primes[m] + c;
            x = (uint32_t)v;
            c = v >> 32;
        }
        if (c) M.push_back((uint32_t)c);
    }
    for (int m = 0; m < nm; ++m) {
        const long long p = r->primes[m];
        long long pr = 1;
        for (int j = 0; j < nm; ++j)
            if (j != m) pr = pr * (r->primes[j] % p) % p;
        mods[m].cinv = (int)modinv(pr, p);
    }
    // residue weights: [ceil(nm/8)][KB][64][16], w_t = 256^t mod p (W) and
    // w_t cinv mod p (Wb), each as two balanced base-2^8 digits
    std::vector<int8_t> W((size_t)((nm + 7) / 8) * KB * 1024, 0), Wb(W.size(), 0);
    auto put = [&](std::vector<int8_t> &dst, int m, int t, long long w, long long p) {
        const long long wb = w > p / 2 ? w - p : w;
        const long long lo = ((wb + 128) & 255) - 128;
        const long long hi = (wb - lo) / 256;
        for (int d = 0; d < 2; ++d) {
            const int o = 2 * m + d, ob = o / 16, row = o % 16;
            const int kb = t / 64, g = (t % 64) / 16, b = t % 16;
            dst[(((size_t)ob * KB + kb) * 64 + row + 16 * g) * 16 + b] = (int8_t)(d ? hi : lo);
        }
    };
    for (int m = 0; m < nm; ++m) {
        const long long p = r->primes[m], ci = mods[m].cinv;
        long long w = 1, s1 = 0;
        for (int t = 0; t < 2 * L; ++t) {
            put(W, m, t, w, p);
            put(Wb, m, t, w * ci % p, p);
            s1 = (s1 + w) % p;
            w = w * 256 % p;
        }
        const long long k0 = 128 * s1 % p;              // 128 sum_t 256^t
        const long long k1 = ((k0 - w) % p + p) % p;    // w = 2^W mod p now
        mods[m].p = (int)p;
        mods[m].k0 = (int)k0;
        mods[m].k1 = (int)k1;
        mods[m].k0b = (int)(k0 * ci % p);
        mods[m].k1b = (int)(k1 * ci % p);
        mods[m].invp = 1.0 / (double)p;
    }
    // CRT: the balanced bytes of M and of each M/p_m
    std::vector<int8_t> mbh(Jpad);
    balanced_bytes(M, Jpad, mbh.data());
    if (r->mtop != 0.0) {
        // M / 2^(8 Jpad) from M's top three words (relative error 2^-64)
        const size_t k = M.size();
        double v = 0;
        for (size_t w = k; w-- > 0 && w + 3 >= k;) v = v * 4294967296.0 + (double)M[w];
        r->mtop = ldexp(v, 32 * (int)(k >= 3 ? k - 3 : 0) - 8 * Jpad);
    }
    std::vector<int8_t> T((size_t)(Jpad / 16) * KBc * 1024, 0);
    std::vector<int8_t> dm(Jpad);
    std::vector<uint32_t> Mm(M.size());
    for (int m = 0; m < nm; ++m) {
        const uint64_t p = (uint64_t)r->primes[m];
        uint64_t rem = 0;
        for (size_t w = M.size(); w-- > 0;) {
            const uint64_t cur = (rem << 32) | M[w];
            Mm[w] = (uint32_t)(cur / p);
            rem = cur % p;
        }
        balanced_bytes(Mm, Jpad, dm.data());
        for (int d = 0; d < 2; ++d) {
            const int k = 2 * m + d, kb = k / 64, g = (k % 64) / 16, b = k % 16;
            for (int j = 0; j < Jpad; ++j) {
                const int8_t v = d == 0 ? dm[j] : (j ? dm[j - 1] : (int8_t)0);
                const int jb = j / 16, ln = (j % 16) + 16 * g;
                T[(((size_t)jb * KBc + kb) * 64 + ln) * 16 + b] = v;
            }
        }
    }
    int rc = rns_alloc(r, (void **)&r->dMod, mods.size() * sizeof(RnsMod));
    if (!rc) rc = rns_alloc(r, (void **)&r->dW, W.size());
    if (!rc) rc = rns_alloc(r, (void **)&r->dWb, Wb.size());
    if (!rc) rc = rns_alloc(r, (void **)&r->dT, T.size());
    if (!rc) rc = rns_alloc(r, (void **)&r->dMb, mbh.size());
    if (rc) return rc;
    MFH_HIP(hipMemcpy(r->dMod, mods.data(), mods.size() * sizeof(RnsMod), hipMemcpyHostToDevice));
    MFH_HIP(hipMemcpy(r->dW, W.data(), W.size(), hipMemcpyHostToDevice));
    MFH_HIP(hipMemcpy(r->dWb, Wb.data(), Wb.size(), hipMemcpyHostToDevice));
    MFH_HIP(hipMemcpy(r->dT, T.data(), T.size(), hipMemcpyHostToDevice));
    MFH_HIP(hipMemcpy(r->dMb, mbh.data(), mbh.size(), hipMemcpyHostToDevice));
    return MFH_OK;
}

template <int KB, int EB>
void launch_residue(const mfh_rns *r, const uint16_t *X, int sgn, int scaled, uint16_t *R)
{
    // a workgroup covers 4 waves x 16 EB consecutive elements of one row
    dim3 grid((r->np + 64 * EB - 1) / (64 * EB), r->np);
    hipLaunchKernelGGL((k_rns_residue<KB, EB>), grid, dim3(256), 0, r->stream, X, r->n, r->np,
                       r->L, sgn, scaled, (const v4i *)(scaled ? r->dWb : r->dW),
                       (const RnsMod *)r->dMod, r->nm, R);
}

int run_residue(const mfh_rns *r, const uint16_t *X, int sgn, int scaled, uint16_t *R)
{
    switch (r->KB) {
    // EB = 4 element blocks per wave (EB = 8 for L <= 128 left one wave per
    // SIMD and ran 35 % slower: the limb loads need the occupancy)
    case 1: launch_residue<1, 4>(r, X, sgn, scaled, R); break;
    case 2: launch_residue<2, 4>(r, X, sgn, scaled, R); break;
    case 4: launch_residue<4, 4>(r, X, sgn, scaled, R); break;
    case 8: launch_residue<8, 4>(r, X, sgn, scaled, R); break;
    case 16: launch_residue<16, 2>(r, X, sgn, scaled, R); break;
    default: return MFH_E_BOUND;
    }
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

template <int EB, int NT, int KBB, bool DBL, bool MP = false>
int launch_crt(const mfh_rns *r, uint16_t *out, int RL, int RLc)
{
    const int KBc = r->nmk / 32;
    const size_t lds = crt_lds_bytes(EB, NT, KBc, r->Jpad, r->crt_nh);
    static bool attr_set = false;
    if (!attr_set) {
        MFH_HIP(hipFuncSetAttribute((const void *)k_rns_crt<EB, NT, KBB, DBL, MP>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        attr_set = true;
    }
    dim3 grid((r->n + 16 * EB - 1) / (16 * EB), r->n);
    hipLaunchKernelGGL((k_rns_crt<EB, NT, KBB, DBL, MP>), grid, dim3(NT), lds, r->stream, r->dY,
                       r->n, r->np, r->nm, KBc, r->Jpad, r->crt_nh, r->mtop, (const v4i *)r->dT,
                       r->dMb,
                       (const RnsMod *)r->dMod, out, RL, RLc);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

// the CRT kernel's shape: at most four output chunks: 4 waves; T fragments
// of at most 9 k blocks in one batch, else batches of 4, double-buffered
int run_crt(const mfh_rns *r, uint16_t *out, int RL, int RLc)
{
    const int KBc = r->nmk / 32, nch = r->Jpad / 64;
    const bool narrow = nch <= 4 && r->crt_nh == 1, one = KBc <= 9, mp = r->crt_nh > 1;
    switch (r->crt_eb) {
    case 4:
        // a batch sized to the k blocks: fewer registers, more workgroups
        if (narrow && KBc <= 4) return launch_crt<4, 256, 4, false>(r, out, RL, RLc);
        if (narrow) return one ? launch_crt<4, 256, 9, false>(r, out, RL, RLc)
                               : launch_crt<4, 256, 4, true>(r, out, RL, RLc);
        if (mp) return one ? launch_crt<4, 512, 9, false, true>(r, out, RL, RLc)
                           : launch_crt<4, 512, 4, true, true>(r, out, RL, RLc);
        return one ? launch_crt<4, 512, 9, false>(r, out, RL, RLc)
                   : launch_crt<4, 512, 4, true>(r, out, RL, RLc);
    case 2:
        if (mp) return one ? launch_crt<2, 512, 9, false, true>(r, out, RL, RLc)
                           : launch_crt<2, 512, 4, true, true>(r, out, RL, RLc);
        return one ? launch_crt<2, 512, 9, false>(r, out, RL, RLc)
                   : launch_crt<2, 512, 4, true>(r, out, RL, RLc);
    default:
        if (mp) return one ? launch_crt<1, 512, 9, false, true>(r, out, RL, RLc)
                           : launch_crt<1, 512, 4, true, true>(r, out, RL, RLc);
        return one ? launch_crt<1, 512, 9, false>(r, out, RL, RLc)
                   : launch_crt<1, 512, 4, true>(r, out, RL, RLc);
    }
}

void rns_mark(mfh_rns *r, int k)
{
    if (r->timing) (void)hipEventRecord(r->ev[k], r->stream);
}

// the product: B transposed, the residues of both operands, the per-prime
// GEMMs and the CRT into RL limbs at out
int rns_run(mfh_rns *r, int sgn, const void *dA, const void *dB, uint16_t *out, int RL)
{
    rns_mark(r, 0);
    int rc = mfh_launch_transpose(dB, r->dBt, r->L, r->n, 2, r->stream);
    if (!rc) rc = run_residue(r, (const uint16_t *)dA, sgn, 0, r->dRA);
    if (!rc) rc = run_residue(r, r->dBt, sgn, 1, r->dRB);
    if (rc) return rc;
    rns_mark(r, 1);
    const int wx = r->cus / 8;               // persistent workgroups per XCD
    // eight waves of 32 x 64 (two per SIMD); four waves of 64 x 64 spilled
    // and ran 1.8x slower
    const TileMap tm = tile_map(r->np / 128, wx);
    const int N = r->nm * tm.tpr * tm.tpr, blk = tm.BR * tm.BC;
    const int R = ((N + 7) / 8 + blk - 1) / blk * blk;
    hipLaunchKernelGGL(k_rns_pointwise<2>, dim3(8 * wx), dim3(512), 0, r->stream,
                       (const uint16_t *)r->dRA, (const uint16_t *)r->dRB,
                       (const RnsMod *)r->dMod, r->nm, r->np, r->dY, wx, tm, R);
    MFH_HIP(hipGetLastError());
    rns_mark(r, 2);
    const int RLc = std::min(RL, 2 * r->L + 1);
    rc = run_crt(r, out, RL, RLc);
    if (rc) return rc;
    rns_mark(r, 3);
    return MFH_OK;
}

}  // namespace

extern "C" {

int mfh_rns_primes(int n, int L, int *primes, int cap)
{
    if (n < 1 || L < 1) return MFH_E_ARG;
    std::vector<int> ps;
    const int rc = plan_primes(n, L, ps);
    if (rc) return rc;
    for (int k = 0; k < (int)ps.size() && k < cap && primes; ++k) primes[k] = ps[k];
    return (int)ps.size();
}

int mfh_rns_create(mfh_rns **out, int n, int L)
{
    if (!out) return MFH_E_ARG;
    *out = nullptr;
    // residue sums |2L 2^14| and the CRT columns |2 nmk 2^14| fit int32 far
    // beyond these limits; the pointwise classes need 2 n 2^14 < 2^31; the
    // CRT kernel holds 16 elements' int64 byte groups (2L+1 limbs) in LDS,
    // which caps L at 512
    if (n < 1 || n > 32768 || L < 1 || L > 512) return MFH_E_BOUND;
    int cnt = 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceCount(&cnt) != hipSuccess || cnt < 1) return MFH_E_NODEV;
    if (hipGetDeviceProperties(&prop, 0) != hipSuccess ||
        strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return MFH_E_NODEV;
    mfh_rns *r = new mfh_rns();
    r->cus = prop.multiProcessorCount >= 8 ? prop.multiProcessorCount / 8 * 8 : 8;
    r->n = n;
    r->L = L;
    r->np = (n + 127) / 128 * 128;
    int rc = plan_primes(n, L, r->primes);
    if (rc) { delete r; return rc; }
    r->nm = (int)r->primes.size();
    r->nmk = (r->nm + 31) / 32 * 32;
    r->KB = kres_blocks(L);
    // bytes of the CRT columns: 2 (2L+1), rounded up to 64-byte chunks;
    // when 4L fills whole chunks, 4L and limb 2L from fp64 (error bound
    // M 2^(-32L) nm^2 2^-53 below 1/16)
    {
        double lgM = 0;
        for (int p : r->primes) lgM += log2((double)p);
        const double err = exp2(lgM - 32.0 * L) * (double)r->nm * r->nm * 0x1p-53;
        const bool top = (4 * L) % 64 == 0 && err < 1.0 / 16;
        r->Jpad = top ? 4 * L : (2 * (2 * L + 1) + 63) / 64 * 64;
        r->mtop = top ? 1.0 : 0.0;          // the value is set with the tables
    }
    // the most elements per CRT workgroup whose LDS fits in at most four
    // passes over the output chunks
    r->crt_eb = r->crt_nh = 0;
    for (int eb : {4, 2, 1}) {
        for (int nh = 1; nh <= 4 && !r->crt_eb; ++nh)
            if (crt_lds_bytes(eb, 512, r->nmk / 32, r->Jpad, nh) <= 150 * 1024) {
                r->crt_eb = eb;
                r->crt_nh = nh;
            }
        if (r->crt_eb) break;
    }
    if (!r->crt_eb) { delete r; return MFH_E_BOUND; }
    r->dev = 0;
    if (hipSetDevice(0) != hipSuccess || hipStreamCreate(&r->stream) != hipSuccess) {
        delete r;
        return MFH_E_HIP;
    }
    for (auto &e : r->ev) (void)hipEventCreate(&e);
    const size_t res = (size_t)r->nm * r->np * r->np * 2;
    rc = rns_tables(r);
    if (!rc) rc = rns_alloc(r, (void **)&r->dRA, res);
    if (!rc) rc = rns_alloc(r, (void **)&r->dRB, res);
    if (!rc) rc = rns_alloc(r, (void **)&r->dY, res);
    if (!rc) rc = rns_alloc(r, (void **)&r->dBt, (size_t)L * n * n * 2);
    if (rc) { mfh_rns_destroy(r); return rc; }
    *out = r;
    return MFH_OK;
}

void mfh_rns_destroy(mfh_rns *r)
{
    if (!r) return;
    if (r->stream) (void)hipStreamSynchronize(r->stream);
    void *bufs[] = {r->dMod, r->dW, r->dWb, r->dT, r->dMb, r->dRA, r->dRB, r->dY, r->dBt,
                    r->dFA,  r->dFB, r->dFO};
    for (void *b : bufs)
        if (b) (void)hipFree(b);
    for (auto &e : r->ev)
        if (e) (void)hipEventDestroy(e);
    if (r->stream) (void)hipStreamDestroy(r->stream);
    delete r;
}

int mfh_rns_info(const mfh_rns *r, int *nmod, int *np_, size_t *bytes)
{
    if (!r) return MFH_E_ARG;
    if (nmod) *nmod = r->nm;
    if (np_) *np_ = r->np;
    if (bytes) *bytes = r->bytes;
    return MFH_OK;
}

int mfh_rns_residues_dev(mfh_rns *r, int in_kind, const void *dX, void *dR)
{
    if (!r || !dX || !dR) return MFH_E_ARG;
    if (in_kind != MFH_IN_U16 && in_kind != MFH_IN_U16_SIGNED) return MFH_E_ARG;
    return run_residue(r, (const uint16_t *)dX, in_kind == MFH_IN_U16_SIGNED, 0, (uint16_t *)dR);
}

int mfh_rns_mm_dev(mfh_rns *r, int in_kind, const void *dA, const void *dB, void *dOut, int RL)
{
    if (!r || !dA || !dB || !dOut || RL < 1) return MFH_E_ARG;
    if (in_kind != MFH_IN_U16 && in_kind != MFH_IN_U16_SIGNED) return MFH_E_ARG;
    return rns_run(r, in_kind == MFH_IN_U16_SIGNED, dA, dB, (uint16_t *)dOut, RL);
}

int mfh_rns_mm(mfh_rns *r, int in_kind, const uint16_t *A, const uint16_t *B, uint16_t *out,
               int RL)
{
    if (!r || !A || !B || !out || RL < 1) return MFH_E_ARG;
    const size_t in = (size_t)r->L * r->n * r->n * 2, ob = (size_t)RL * r->n * r->n * 2;
    void *dA = nullptr, *dB = nullptr, *dO = nullptr;
    int rc = MFH_OK;
    if (hipMalloc(&dA, in) != hipSuccess || hipMalloc(&dB, in) != hipSuccess ||
        hipMalloc(&dO, ob) != hipSuccess)
        rc = MFH_E_NOMEM;
    if (!rc && (hipMemcpyAsync(dA, A, in, hipMemcpyHostToDevice, r->stream) != hipSuccess ||
                hipMemcpyAsync(dB, B, in, hipMemcpyHostToDevice, r->stream) != hipSuccess))
        rc = MFH_E_HIP;
    if (!rc) rc = mfh_rns_mm_dev(r, in_kind, dA, dB, dO, RL);
    if (!rc && hipMemcpyAsync(out, dO, ob, hipMemcpyDeviceToHost, r->stream) != hipSuccess)
        rc = MFH_E_HIP;
    if (hipStreamSynchronize(r->stream) != hipSuccess && !rc) rc = MFH_E_HIP;
    for (void *p : {dA, dB, dO})
        if (p) (void)hipFree(p);
    return rc;
}

}  // extern "C"

namespace {
// fp32 (f64 = 0) or fp64 matrices on the fixed-point grid of L - 1 limbs (L
// the context's): both encoded as the L two's complement limbs of their grid
// values, multiplied exactly (2L limbs hold n 2^(32 (L-1)) with its sign),
// and decoded with the single rounding of the grid's decode
// (src/fpfixed.c:144-204, 212-322)
int rns_fpx(mfh_rns *r, int f64, const void *dA, const void *dB, int SA, int SB, void *dC)
{
    if (!r || !dA || !dB || !dC) return MFH_E_ARG;
    if (r->L < 2) return MFH_E_ARG;
    const int Lg = r->L - 1, RLr = 2 * r->L;
    const size_t nn = (size_t)r->n * r->n;
    // (a decode inside the CRT kernel, one thread per element from the
    // carried words in LDS, ran 2 % slower than this separate pass)
    int rc = MFH_OK;
    if (!r->dFO) {
        rc = rns_alloc(r, (void **)&r->dFA, (size_t)r->L * nn * 2);
        if (!rc) rc = rns_alloc(r, (void **)&r->dFB, (size_t)r->L * nn * 2);
        if (!rc) rc = rns_alloc(r, (void **)&r->dFO, (size_t)RLr * nn * 2);
        if (rc) return rc;
    }
    if ((rc = mfh_launch_encode_tc(dA, f64, r->n, Lg, SA, r->dFA, r->stream))) return rc;
    if ((rc = mfh_launch_encode_tc(dB, f64, r->n, Lg, SB, r->dFB, r->stream))) return rc;
    if ((rc = rns_run(r, 1, r->dFA, r->dFB, r->dFO, RLr))) return rc;
    return mfh_launch_decode_limbs(r->dFO, nn, RLr, SA + SB, f64 ? MFH_DEC_F64 : MFH_DEC_F32,
                                   dC, nullptr, r->stream);
}

int rns_fpx_host(mfh_rns *r, int f64, const void *A, const void *B, int SA, int SB, void *C)
{
    if (!r || !A || !B || !C) return MFH_E_ARG;
    const size_t bytes = (size_t)r->n * r->n * (f64 ? 8 : 4);
    void *dA = nullptr, *dB = nullptr, *dC = nullptr;
    int rc = MFH_OK;
    if (hipMalloc(&dA, bytes) != hipSuccess || hipMalloc(&dB, bytes) != hipSuccess ||
        hipMalloc(&dC, bytes) != hipSuccess)
        rc = MFH_E_NOMEM;
    if (!rc && (hipMemcpyAsync(dA, A, bytes, hipMemcpyHostToDevice, r->stream) != hipSuccess ||
                hipMemcpyAsync(dB, B, bytes, hipMemcpyHostToDevice, r->stream) != hipSuccess))
        rc = MFH_E_HIP;
    if (!rc) rc = rns_fpx(r, f64, dA, dB, SA, SB, dC);
    if (!rc && hipMemcpyAsync(C, dC, bytes, hipMemcpyDeviceToHost, r->stream) != hipSuccess)
        rc = MFH_E_HIP;
    if (hipStreamSynchronize(r->stream) != hipSuccess && !rc) rc = MFH_E_HIP;
    for (void *p : {dA, dB, dC})
        if (p) (void)hipFree(p);
    return rc;
}
}  // namespace

extern "C" {

int mfh_rns_fpx_mm_dev(mfh_rns *r, const void *dA, const void *dB, int SA, int SB, void *dC)
{
    return rns_fpx(r, 0, dA, dB, SA, SB, dC);
}

int mfh_rns_fpx_mm_f64_dev(mfh_rns *r, const void *dA, const void *dB, int SA, int SB,
                           void *dC)
{
    return rns_fpx(r, 1, dA, dB, SA, SB, dC);
}

int mfh_rns_fpx_mm(mfh_rns *r, const float *A, const float *B, int SA, int SB, float *C)
{
    return rns_fpx_host(r, 0, A, B, SA, SB, C);
}

int mfh_rns_fpx_mm_f64(mfh_rns *r, const double *A, const double *B, int SA, int SB,
                       double *C)
{
    return rns_fpx_host(r, 1, A, B, SA, SB, C);
}

int mfh_rns_sync(mfh_rns *r)
{
    if (!r) return MFH_E_ARG;
    MFH_HIP(hipStreamSynchronize(r->stream));
    return MFH_OK;
}

int mfh_rns_set_timing(mfh_rns *r, int enable)
{
    if (!r) return MFH_E_ARG;
    r->timing = enable ? 1 : 0;
    return MFH_OK;
}

int mfh_rns_stage_times(const mfh_rns *r, float ms[4])
{
    if (!r || !ms) return MFH_E_ARG;
    MFH_HIP(hipEventSynchronize(r->ev[3]));
    for (int k = 0; k < 3; ++k) MFH_HIP(hipEventElapsedTime(&ms[k], r->ev[k], r->ev[k + 1]));
    MFH_HIP(hipEventElapsedTime(&ms[3], r->ev[0], r->ev[3]));
    return MFH_OK;
}

int mfh_rns_work(const mfh_rns *r, double *res_ops, double *pw_ops, double *crt_ops)
{
    if (!r) return MFH_E_ARG;
    const double np3 = (double)r->np * r->np * r->np, np2 = (double)r->np * r->np;
    if (res_ops) *res_ops = 2.0 * 2 * np2 * (64.0 * r->KB) * (2.0 * r->nm);
    if (pw_ops) *pw_ops = (double)r->nm * 4 * 2 * np3;
    if (crt_ops) *crt_ops = 2.0 * r->n * r->n * (2.0 * r->nmk) * r->Jpad;
    return MFH_OK;
}

}  // extern "C"
