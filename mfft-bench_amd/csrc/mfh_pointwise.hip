// mfh_pointwise.hip -- the pointwise step of the MFFT matmul as one batched
// int8 MFMA GEMM on gfx950 (v_mfma_i32_16x16x64_i8).
//
// At every evaluation point j the product of two ring elements of
// R (x) M_n(Z), R = Z[y]/(y^K+1), is a length-K negacyclic convolution of
// n x n matrices (src/mfft.c:383-395):
//     C_j[t] = sum_{c1+c2 = t} A_j[c1] B_j[c2]  -  sum_{c1+c2 = t+K} A_j[c1] B_j[c2]
// i.e. [A_j[0] .. A_j[K-1]] times the block-negacyclic Toeplitz matrix of
// B_j.  The Toeplitz matrix is never formed: a wave owns one 16 x 16 output
// block for T consecutive t and streams the K B-planes past a sliding window
// of T+1 A-planes held in registers, so every operand fragment read from LDS
// feeds T (or more) MFMAs.
//
// Each transformed value is split into int8 digit planes (see
// mfh_internal.hpp: three balanced base-2^8 digits, or three base-2^7 digits
// and their pairwise sums for Karatsuba); the digit products are
// accumulated in int32 per weight class and stored per class; the inverse
// transform recombines the classes into the exact int64 C^_j[t].
//
// Signs: the negacyclic wrap (c1 + c2 >= K) subtracts.  An int8 operand
// cannot be negated (-(-128)), so the wave negates the int32 accumulator
// instead: within one k-block round, the terms of acc[t] are issued with all
// positive terms contiguous and all negative ones contiguous, and the
// accumulator is negated once between the two groups.  Rounds alternate
// between ascending and descending c2 so that one negation per round
// suffices; the orientation of the accumulator (+(P-N) or -(P-N)) is known
// from the direction of the last round and applied at the flush.
//
// Operands in HBM: digit plane (j, c, r) is an int8 matrix with the
// reduction index k along rows (A as A[i][k], B stored transposed as
// B^T[j'][k]), in 16 x 64 tiles (mfh_tile_off): one operand fragment is 1 KB
// contiguous.  B's planes hold all np rows, A's the `rows` rows of the
// current row band.  Each round stages, for all K ring
// coefficients, a (16*WBI) x 64 tile of A and a (16*WBJ) x 64 tile of B^T
// into LDS in MFMA operand order (lane l of a 16x64 fragment = row l%16,
// k bytes 16*(l/16) .. +15; A and B use the same k order, so the dot
// product is the same whatever order the hardware sums in).  The next
// round reaches LDS either through registers loaded a round ahead or by
// buffer-to-LDS copies issued while this round's MFMAs run (Cfg::DMA).
//
// Output: int32 class results in the layout of mfh_c5_index (4 consecutive
// ring coefficients of 16 consecutive columns are 256 contiguous bytes, so
// each wave store writes whole cache lines).
#include <type_traits>

#include "mfh_internal.hpp"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int pmod(int a, int m) { return ((a % m) + m) % m; }

// KB: 64-wide k blocks per LDS fill (1, or 2 for small rings, where one
// block alone gives too few MFMAs per barrier)
// WPE: waves per SIMD the kernel is compiled for (register budget 512/WPE).
// DMA: fill the round buffer with buffer-to-LDS copies after each round
// (no staging registers; the fill latency is hidden by the other
// workgroups on the CU) instead of from registers loaded a round ahead.
// BREG: (copy fills only) a wave reads all its B fragments of the round into
// registers up front, like the A fragments, so both tiles of the next round
// are copied in while this round's MFMAs run from registers.  BREG = 1: the
// barrier that frees the buffer and the copies come before the first MFMA;
// BREG = s + 2: after step s of the round's MFMAs.
// SHELL: (BREG >= 2 only) lookahead D > 0 selects the shell schedule of
// pw_round: fragment pairs are read D pairs ahead of the MFMAs that need
// them, and BREG - 2 counts shells instead of steps.
template <int K_, int T_, int WBI_, int WBJ_, int KB_ = 1, int WPE_ = 2, bool DMA_ = false,
          int BREG_ = 0, int SHELL_ = 0>
struct PwCfg {
    static constexpr int K = K_, T = T_, WBI = WBI_, WBJ = WBJ_, KB = KB_, WPE = WPE_;
    static constexpr bool DMA = DMA_;
    static constexpr int BREG = BREG_;
    static constexpr int SHELL = SHELL_;
    static_assert(!DMA || (KB == 1 && T == K), "copy fills: one k block, whole-ring waves");
    static_assert(!BREG || DMA, "B fragments in registers: copy fills only");
    // every LDS read of the round is issued before the barrier that frees
    // the buffer: the last pair is read at shell K-1-D
    static_assert(!SHELL || (BREG >= 2 && BREG - 2 >= K - 1 - SHELL && BREG - 2 < K),
                  "shell schedule: the barrier follows the round's last LDS read");
    static_assert(KB == 1 || KB == 2, "one or two k blocks per fill");
    static constexpr int G = K / T;                 // t-groups per block
    static constexpr int WAVES = WBI * WBJ * G;
    static constexpr int THREADS = WAVES * 64;
    static constexpr int BI = 16 * WBI, BJ = 16 * WBJ;
    static constexpr int A_CHUNKS = K * WBI * 64;   // 16-byte LDS chunks
    static constexpr int B_CHUNKS = K * WBJ * 64;
    static constexpr int SUB_CHUNKS = A_CHUNKS + B_CHUNKS;         // one k block
    static constexpr int LDS_BYTES = KB * SUB_CHUNKS * 16;          // one fill
    static constexpr int DYN_LDS = DMA ? 0 : LDS_BYTES;   // copy fills use static arrays
};

// One round: one 64-wide k block of one digit pair, all K values of c2.
// la points at this wave's A fragment of ring coefficient 0 (stride
// WBI*64 chunks per coefficient), lb likewise for B.
struct NoHook {
    __device__ __forceinline__ void operator()() const {}
};

// after_a runs once the wave's A fragments are in registers (T == K only)
template <class Cfg, bool ASC, int T0, class Issue, class AfterA = NoHook>
__device__ __forceinline__ void pw_round(v4i (&acc)[Cfg::T], const v4i *__restrict__ la,
                                         const v4i *__restrict__ lb, const Issue &issue,
                                         const AfterA &after_a = AfterA{})
{
    constexpr int K = Cfg::K, T = Cfg::T;
    constexpr int SA = Cfg::WBI * 64, SB = Cfg::WBJ * 64;
    if constexpr (T == K && Cfg::SHELL > 0) {
        // Shell schedule.  The K x K products (c1, c2) are issued in shells:
        // ascending rounds by m = max(c1, c2) = 0, 1, .., K-1, descending
        // rounds by m = min(c1, c2) = K-1, .., 0.  Shell m needs only the
        // fragment pairs (A_c, B_c) up to (down to) c = m, so a wave starts
        // its MFMAs once its first pair is in and reads the others D pairs
        // ahead (D*2 reads in flight: the LDS counter tracks at most 15).
        // Signs: ASC, the positive terms of acc[t] (c1 + c2 = t) all have
        // max <= t and its negative ones (c1 + c2 = t + K) max >=
        // ceil((t + K) / 2) >= t + 2 for t <= K-3, so acc[t] is flipped at
        // the start of shell min(t + 2, K - 1), and acc[K-1] (no negative
        // terms) after the round.  DESC: the negative terms of acc[t] have
        // min >= t + 1 and its positive ones min <= t / 2, so acc[t] is
        // flipped at the start of shell max(t - 1, 0).  One flip per
        // accumulator per round, as in the step schedule, each at least
        // one shell away from the MFMAs around it.
        constexpr int D = Cfg::SHELL;
        v4i af[K], bf[K];
#pragma unroll
        for (int s = 0; s < D && s < K; ++s) {
            const int c = ASC ? s : K - 1 - s;
            af[c] = la[c * SA];
            bf[c] = lb[c * SB];
        }
#pragma unroll
        for (int sh = 0; sh < K; ++sh) {
            const int m = ASC ? sh : K - 1 - sh;
            if (sh + D < K) {
                const int c = ASC ? sh + D : K - 1 - sh - D;
                af[c] = la[c * SA];
                bf[c] = lb[c * SB];
            }
            if (ASC) {
                if (m >= 2) acc[m - 2] = -acc[m - 2];
                if (m == K - 1) acc[K - 2] = -acc[K - 2];
#pragma unroll
                for (int c2 = 0; c2 <= m; ++c2) {
                    const int t = (m + c2) % K;
                    acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[m], bf[c2], acc[t], 0, 0, 0);
                }
#pragma unroll
                for (int c1 = 0; c1 < m; ++c1) {
                    const int t = (c1 + m) % K;
                    acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[c1], bf[m], acc[t], 0, 0, 0);
                }
            } else {
                if (m + 1 < K) acc[m + 1] = -acc[m + 1];
                if (m == 0) acc[0] = -acc[0];
#pragma unroll
                for (int c2 = K - 1; c2 >= m; --c2) {
                    const int t = (m + c2) % K;
                    acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[m], bf[c2], acc[t], 0, 0, 0);
                }
#pragma unroll
                for (int c1 = K - 1; c1 > m; --c1) {
                    const int t = (c1 + m) % K;
                    acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[c1], bf[m], acc[t], 0, 0, 0);
                }
            }
            issue(sh);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (ASC) acc[K - 1] = -acc[K - 1];
        return;
    }
    if constexpr (T == K) {
        // every A fragment is live at every step: hold all K of them.
        // Step st uses B fragment c2 (ascending or descending).  The
        // accumulator whose sign flips at the start of the next step is
        // issued first in this step (the flip then waits on nothing), B
        // fragments are read two steps ahead, and scheduling barriers keep
        // the compiler from hoisting a flip next to its producing MFMA.
        v4i af[K];
#pragma unroll
        for (int c1 = 0; c1 < K; ++c1) af[c1] = la[c1 * SA];
        if constexpr (Cfg::BREG) {
            v4i bf[K];
#pragma unroll
            for (int c2 = 0; c2 < K; ++c2) bf[c2] = lb[c2 * SB];
            after_a();
#pragma unroll
            for (int st = 0; st < K; ++st) {
                const int c2 = ASC ? st : K - 1 - st;
                if (ASC && c2 >= 1) acc[c2 - 1] = -acc[c2 - 1];
                if (!ASC) acc[c2] = -acc[c2];
                const int lead = ASC ? c2 : (c2 + K - 1) % K;
#pragma unroll
                for (int o = 0; o < T; ++o) {
                    const int t = (lead + o) % K;
                    acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[pmod(t - c2, K)], bf[c2],
                                                                   acc[t], 0, 0, 0);
                }
                issue(st);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (ASC) acc[K - 1] = -acc[K - 1];
            return;
        }
        after_a();
        v4i bq[3];
        bq[0] = lb[(ASC ? 0 : K - 1) * SB];
        if (K > 1) bq[1] = lb[(ASC ? 1 : K - 2) * SB];
#pragma unroll
        for (int st = 0; st < K; ++st) {
            const int c2 = ASC ? st : K - 1 - st;
            if (st + 2 < K) bq[(st + 2) % 3] = lb[(ASC ? st + 2 : K - 3 - st) * SB];
            // flips at this step: ASC flips t = c2-1 (after its last positive
            // term), DESC flips t = c2 (before its first positive term)
            if (ASC && c2 >= 1) acc[c2 - 1] = -acc[c2 - 1];
            if (!ASC) acc[c2] = -acc[c2];
            // first the accumulator flipped at the next step: ASC t = c2,
            // DESC t = c2-1; then the rest in cyclic order
            const int lead = ASC ? c2 : (c2 + K - 1) % K;
#pragma unroll
            for (int o = 0; o < T; ++o) {
                const int t = (lead + o) % K;
                acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[pmod(t - c2, K)], bq[st % 3],
                                                               acc[t], 0, 0, 0);
            }
            issue(st);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (ASC) acc[K - 1] = -acc[K - 1];
        return;
    }
    v4i win[T + 1];
    constexpr int first = ASC ? 0 : K - 1;
    // window key kk = tt - c2 holds A fragment c1 = (T0 + kk) mod K in slot
    // kk mod (T+1); the T live keys of a step never collide, and the key
    // entering at the next step takes the one free slot.
#pragma unroll
    for (int tt = 0; tt < T; ++tt)
        win[pmod(tt - first, T + 1)] = la[pmod(T0 + tt - first, K) * SA];
    // DESC: acc[t] for t = K-1 has no negative terms; its sign flip comes
    // before its first (positive) term.
#pragma unroll
    for (int st = 0; st < K; ++st) {
        const int c2 = ASC ? st : K - 1 - st;
        const v4i bf = lb[c2 * SB];
        issue(st);
        if (st + 1 < K) {
            const int c2n = ASC ? st + 1 : K - 2 - st;
            const int ttn = ASC ? 0 : T - 1;
            win[pmod(ttn - c2n, T + 1)] = la[pmod(T0 + ttn - c2n, K) * SA];
        }
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
            const int t = T0 + tt;
            // ASC: terms c2 <= t are positive, then negative; flip right
            // before the first negative one (c2 == t+1).
            // DESC: terms c2 > t are negative, then positive; flip right
            // before the first positive one (c2 == t).
            if ((ASC && c2 == t + 1) || (!ASC && c2 == t)) acc[tt] = -acc[tt];
            acc[tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(win[pmod(tt - c2, T + 1)], bf,
                                                            acc[tt], 0, 0, 0);
        }
    }
    if (ASC) {
        // t = K-1 never met c2 == t+1 inside the round
#pragma unroll
        for (int tt = 0; tt < T; ++tt)
            if (T0 + tt == K - 1) acc[tt] = -acc[tt];
    }
}

template <class Cfg, bool ASC, int TG = 0, class Issue>
__device__ __forceinline__ void pw_dispatch(int tg, v4i (&acc)[Cfg::T], const v4i *la,
                                            const v4i *lb, const Issue &issue)
{
    if constexpr (TG < Cfg::G) {
        if (tg == TG) pw_round<Cfg, ASC, TG * Cfg::T>(acc, la, lb, issue);
        else pw_dispatch<Cfg, ASC, TG + 1>(tg, acc, la, lb, issue);
    }
}

// Round index -> (digit pair, k block).  Pairs are ordered by weight class
// m = r + s so that each class's rounds are contiguous.
__device__ __forceinline__ void pair_of(int p, int &r, int &s, int &m)
{
    // (r,s): (0,0) | (0,1) (1,0) | (0,2) (1,1) (2,0) | (1,2) (2,1) | (2,2),
    // one nibble per pair index
    constexpr unsigned long long R = 0x221210100ULL, S = 0x212012010ULL;
    r = (int)((R >> (4 * p)) & 0xF);
    s = (int)((S >> (4 * p)) & 0xF);
    m = r + s;
}

// Direct-to-LDS loads of one round: for every ring coefficient, the
// (16*WBI) x 64 A tile and the (16*WBJ) x 64 B^T tile, i.e. FA + FB
// fragments of 16 x 64 bytes.  A fragment is one wave instruction: lane l
// fetches row l%16, k bytes 16*(l/16)..+15, and global_load_lds_dwordx4
// stores lane l's 16 bytes at fragment base + 16*l -- exactly the MFMA
// operand order.  Wave w loads fragments w, w+WAVES, ...; the per-lane
// offset is the same for all of them, so each load is a scalar base plus
// one vector offset.
template <class Cfg>
__device__ __forceinline__ void pw_load_round(v4i *buf, const int8_t *a0, const int8_t *b0,
                                              size_t da, size_t db, int fa, int fb,
                                              uint32_t lane_off)
{
    constexpr int W = Cfg::WAVES;
    constexpr int NA = Cfg::K * Cfg::WBI / W, NB = Cfg::K * Cfg::WBJ / W;
    static_assert((Cfg::K * Cfg::WBI) % W == 0 && (Cfg::K * Cfg::WBJ) % W == 0,
                  "fragments must split evenly over waves");
#pragma unroll
    for (int i = 0; i < NA; ++i)
        __builtin_amdgcn_global_load_lds((const void *)(a0 + i * da + lane_off),
                                         (void *)(buf + (fa + i * W) * 64), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < NB; ++i)
        __builtin_amdgcn_global_load_lds((const void *)(b0 + i * db + lane_off),
                                         (void *)(buf + Cfg::A_CHUNKS + (fb + i * W) * 64), 16,
                                         0, 0);
}

// workgroup barrier that waits only for this wave's LDS traffic
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// workgroup barrier after this wave's global loads (including copies into
// LDS) and LDS traffic have completed
__device__ __forceinline__ void round_barrier()
{
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Workgroup -> (row tile, column tile, point).  Workgroup w runs on XCD
// w mod 8, and about 512 consecutive workgroups are resident at once (two
// per CU).  When the tile grid allows, each such group of 512 covers a
// 16 x 32 block of tiles of one point and the 64 workgroups of one XCD an
// 8 x 8 sub-block of it, so that the operand tiles one XCD streams are
// shared by 8 of its workgroups.  Small points (at most 256 tiles, the
// point count a multiple of 8) go whole to one XCD: XCD x takes points x,
// x + 8, .., each in row order, so that its resident workgroups share the
// operand tiles of one point.  Otherwise tiles are taken in row order.
__device__ __forceinline__ void tile_of(int tiles_j, int &ti, int &tj, int &jp)
{
    const int per_point = gridDim.x, tiles_i = per_point / tiles_j;
    if (per_point <= 256 && gridDim.y % 8 == 0) {
        const int w = blockIdx.y * per_point + blockIdx.x;
        const int x = w & 7, q = w >> 3;
        jp = (q / per_point) * 8 + x;
        const int t = q % per_point;
        ti = t / tiles_j;
        tj = t % tiles_j;
    } else if (tiles_i % 16 == 0 && tiles_j % 32 == 0) {
        const int w = blockIdx.y * per_point + blockIdx.x;
        const int x = w & 7, q = w >> 3;
        const int g = q >> 6, ql = q & 63;            // group of 512, slot within XCD
        const int gpr = tiles_j / 32;                 // groups per 16-row band
        const int gpp = (tiles_i / 16) * gpr;         // groups per point
        jp = g / gpp;
        const int gp = g % gpp;
        ti = (gp / gpr) * 16 + (x >> 2) * 8 + (ql >> 3);
        tj = (gp % gpr) * 32 + (x & 3) * 8 + (ql & 7);
    } else {
        ti = blockIdx.x / tiles_j;
        tj = blockIdx.x % tiles_j;
        jp = blockIdx.y;
    }
}

struct NoIssue {
    __device__ __forceinline__ void operator()(int) const {}
};

// Round schedule of one workgroup: classes m = 0..4 in turn; within class m
// its digit pairs (r, m-r) and, for each, the np/64 k blocks.
struct RoundPos {
    int m, idx;            // class and round index inside the class
    int r, kb;             // its digit pair's A plane r and k block (idx = (r - rlo) * kblocks + kb)
};
// B8: class m holds the digit pairs (r, m-r); K7: class p is the single
// Karatsuba product of plane p with plane p.
template <int MODE>
__device__ __forceinline__ void class_pairs(int m, int &rlo, int &npairs)
{
    if constexpr (MODE == MFH_MODE_K7) {
        rlo = m;
        npairs = 1;
    } else {
        rlo = m > MFH_DIGITS - 1 ? m - (MFH_DIGITS - 1) : 0;
        const int rhi = m < MFH_DIGITS - 1 ? m : MFH_DIGITS - 1;
        npairs = rhi - rlo + 1;
    }
}

// One workgroup: a (16*WBI) x (16*WBJ) block of elements at one evaluation
// point, all K ring coefficients, all digit-weight classes in turn.  Each
// class's int32 result is stored as soon as the class is complete, so the
// only long-lived state is one int32 accumulator per (t, element).  Without
// Cfg::DMA rounds are double-buffered through registers: while a round's
// MFMAs read the LDS buffer, the next round's fragments stream from global
// memory into VGPRs; after the round they are written to LDS (one buffer
// per workgroup).  With Cfg::DMA the buffer is refilled by buffer-to-LDS
// copies: with Cfg::BREG every wave reads all its A and B fragments of the
// round into registers (up front, or with Cfg::SHELL a few pairs ahead of
// the MFMAs that use them), and once every wave has (a barrier, before the
// first MFMA or after an early step or shell) both tiles of the next round
// are copied in while the MFMAs run; without it the A tile is copied during the
// round and the B tile after it, while the other workgroups on the CU keep
// the MFMA units busy.
//
// Output: class m of (j, i, j', t) at mfh_c5_index + m * mfh_c5_class_stride.
// Accumulator bound: a class has at most 3 digit pairs x np/64 rounds of at
// most K * 2^20 each; mfh_create rejects sizes where that reaches 2^31 for
// every digit mode the plan admits, and a product in a mode whose bound
// fails is refused.
template <class Cfg, int MODE>
__global__ void __attribute__((amdgpu_flat_work_group_size(Cfg::THREADS, Cfg::THREADS),
                               amdgpu_waves_per_eu(Cfg::WPE, Cfg::WPE)))
k_pointwise(const int8_t *__restrict__ Ah, const int8_t *__restrict__ Bh,
            int32_t *__restrict__ C5, int np_, int rows, int tiles_j)
{
    constexpr int K = Cfg::K, T = Cfg::T, WBI = Cfg::WBI, WBJ = Cfg::WBJ, W = Cfg::WAVES;
    constexpr int NCLASS = MODE == MFH_MODE_K7 ? 6 : 2 * MFH_DIGITS - 1;
    constexpr int PL = MODE == MFH_MODE_K7 ? 6 : MFH_DIGITS;     // planes per coefficient
    constexpr int NA = K * WBI / W, NBF = K * WBJ / W;   // fragments per wave
    static_assert((K * WBI) % W == 0 && (K * WBJ) % W == 0, "fragments split evenly");
    extern __shared__ v4i lds[];
    // copy fills: A and B tiles in two distinct LDS objects, so that the
    // compiler can tell a copy into one from reads of the other
    __shared__ v4i sA[Cfg::DMA ? Cfg::A_CHUNKS : 1], sB[Cfg::DMA ? Cfg::B_CHUNKS : 1];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tg = wave / (WBI * WBJ);
    const int wb = wave % (WBI * WBJ);
    const int wbi = wb / WBJ, wbj = wb % WBJ;
    int ti, tj, jp;
    tile_of(tiles_j, ti, tj, jp);
    const int i0 = ti * Cfg::BI, j0 = tj * Cfg::BJ;
    const size_t plane = (size_t)np_ * np_;           // B: all np rows
    const size_t planeA = (size_t)rows * np_;         // A: the band's rows
    const int8_t *Aj = Ah + (size_t)jp * K * PL * planeA;
    const int8_t *Bj = Bh + (size_t)jp * K * PL * plane;

    // this wave's fragments f = wave + W*i:
    //   A: coefficient f / WBI, row block f % WBI
    //   B: coefficient f / WBJ, column block f % WBJ
    // planes in 16 x 64 tiles (mfh_tile_off): a fragment is 1 KB contiguous,
    // lane l's 16 bytes at row l % 16, k 16 (l / 16) of the tile
    const int8_t *a_blk = Aj + (size_t)(wave / WBI) * PL * planeA +
                          mfh_tile_off(i0 + (wave % WBI) * 16, 0, np_) + (lane & 15) * 64 +
                          (lane >> 4) * 16;
    const int8_t *b_blk = Bj + (size_t)(wave / WBJ) * PL * plane +
                          mfh_tile_off(j0 + (wave % WBJ) * 16, 0, np_) + (lane & 15) * 64 +
                          (lane >> 4) * 16;
    const size_t da = (size_t)(W / WBI) * PL * planeA;
    const size_t db = (size_t)(W / WBJ) * PL * plane;
    v4i *wa = lds + wave * 64 + lane;                     // this lane's A slot of fragment f=wave
    v4i *wbp = lds + Cfg::A_CHUNKS + wave * 64 + lane;
    const v4i *la = (Cfg::DMA ? sA : lds) + wbi * 64 + lane;
    const v4i *lb = (Cfg::DMA ? sB : lds + Cfg::A_CHUNKS) + wbj * 64 + lane;
    constexpr int KB = Cfg::KB, SUB = Cfg::SUB_CHUNKS, NF = NA + NBF;
    const int kblocks = np_ / (MFH_KBLK * KB);        // fills per digit pair
    const int col = j0 + wbj * 16 + (lane & 15);
    const int row0 = i0 + wbi * 16 + 4 * (lane >> 4);

    v4i R[Cfg::DMA ? 1 : KB * NF];
    // copy fills (DMA mode): the round's A or B tiles straight into LDS
    auto srcs = [&](RoundPos q, const int8_t *&a0, const int8_t *&b0) {
        const int s = MODE == MFH_MODE_K7 ? q.r : q.m - q.r;
        a0 = a_blk + (size_t)q.r * planeA + q.kb * 1024;        // next tile along k
        b0 = b_blk + (size_t)s * plane + q.kb * 1024;
    };
    auto dma_a = [&](RoundPos q) {
        const int8_t *a0, *b0;
        srcs(q, a0, b0);
#pragma unroll
        for (int i = 0; i < NA; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(a0 + i * da),
                                             (void *)(sA + (wave + i * W) * 64), 16, 0, 0);
    };
    auto dma_b = [&](RoundPos q) {
        const int8_t *a0, *b0;
        srcs(q, a0, b0);
#pragma unroll
        for (int i = 0; i < NBF; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(b0 + i * db),
                                             (void *)(sB + (wave + i * W) * 64), 16, 0, 0);
    };
    auto gload = [&](RoundPos q) {
        if constexpr (Cfg::DMA) return;
        const int r = q.r, kb = q.kb;
        const int s = MODE == MFH_MODE_K7 ? r : q.m - r;
#pragma unroll
        for (int sb = 0; sb < KB; ++sb) {
            const int8_t *a0 = a_blk + (size_t)r * planeA + (kb * KB + sb) * 1024;
            const int8_t *b0 = b_blk + (size_t)s * plane + (kb * KB + sb) * 1024;
#pragma unroll
            for (int i = 0; i < NA; ++i) R[sb * NF + i] = *(const v4i *)(a0 + i * da);
#pragma unroll
            for (int i = 0; i < NBF; ++i) R[sb * NF + NA + i] = *(const v4i *)(b0 + i * db);
        }
    };
    auto lwrite = [&]() {
        if constexpr (Cfg::DMA) return;
#pragma unroll
        for (int sb = 0; sb < KB; ++sb) {
#pragma unroll
            for (int i = 0; i < NA; ++i) wa[sb * SUB + i * W * 64] = R[sb * NF + i];
#pragma unroll
            for (int i = 0; i < NBF; ++i) wbp[sb * SUB + i * W * 64] = R[sb * NF + NA + i];
        }
    };
    auto next_of = [&](RoundPos q) {
        int rlo, np2;
        class_pairs<MODE>(q.m, rlo, np2);
        if (q.kb + 1 < kblocks) return RoundPos{q.m, q.idx + 1, q.r, q.kb + 1};
        if (q.idx + 1 < np2 * kblocks) return RoundPos{q.m, q.idx + 1, q.r + 1, 0};
        int rlo2, np3;
        class_pairs<MODE>(q.m + 1, rlo2, np3);
        return RoundPos{q.m + 1, 0, rlo2, 0};
    };

    // prologue: round (0,0) into LDS, round after it into registers
    RoundPos cur{0, 0, 0, 0};
    RoundPos nxt = next_of(cur);
    if constexpr (Cfg::DMA) {
        dma_a(cur);
        dma_b(cur);
    } else {
        gload(cur);
        lwrite();
        gload(nxt);
    }
    __syncthreads();

    v4i acc[T];
    // one round: MFMAs from LDS, then hand the registers' round to LDS and
    // start loading the one after
    // with two k blocks per fill the fill runs one ascending and one
    // descending pass, which leaves the accumulator's orientation unchanged
    auto step = [&](auto asc_tag) {
        constexpr bool ASC = decltype(asc_tag)::value;
        if constexpr (Cfg::DMA) {
            // Once every wave holds its A fragments, the next round's A tile
            // is copied in while this round's MFMAs run; the B tile follows
            // after the round.  The last barrier waits for both copies.
            const bool more = nxt.m < NCLASS;
            if constexpr (Cfg::BREG == 1) {
                // every wave holds its A and B fragments: copy both tiles
                pw_round<Cfg, ASC, 0>(acc, la, lb, NoIssue{}, [&]() {
                    lds_barrier();
                    if (more) {
                        dma_a(nxt);
                        dma_b(nxt);
                    }
                });
            } else if constexpr (Cfg::BREG >= 2) {
                // the same after step BREG-2 of the round's MFMAs
                pw_round<Cfg, ASC, 0>(acc, la, lb, [&](int st) {
                    if (st == Cfg::BREG - 2) {
                        lds_barrier();
                        if (more) {
                            dma_a(nxt);
                            dma_b(nxt);
                        }
                    }
                });
            } else {
                pw_round<Cfg, ASC, 0>(acc, la, lb, NoIssue{}, [&]() {
                    lds_barrier();
                    if (more) dma_a(nxt);
                });
                lds_barrier();
                if (more) dma_b(nxt);
            }
            round_barrier();
            cur = nxt;
            if (cur.m < NCLASS) nxt = next_of(cur);
            return;
        }
        if constexpr (KB == 1) {
            pw_dispatch<Cfg, ASC>(tg, acc, la, lb, NoIssue{});
        } else {
            pw_dispatch<Cfg, true>(tg, acc, la, lb, NoIssue{});
            pw_dispatch<Cfg, false>(tg, acc, la + SUB, lb + SUB, NoIssue{});
        }
        __syncthreads();                     // every wave is done reading LDS
        cur = nxt;
        if (cur.m < NCLASS) {
            lwrite();                        // waits for the registers' loads
            nxt = next_of(cur);
            if (nxt.m < NCLASS) gload(nxt);
        }
        __syncthreads();
    };
#pragma unroll 1
    for (int m = 0; m < NCLASS; ++m) {
#pragma unroll
        for (int tt = 0; tt < T; ++tt) acc[tt] = v4i{0, 0, 0, 0};
        int rlo, np2;
        class_pairs<MODE>(m, rlo, np2);
        const int rounds = np2 * kblocks;
        int rd = 0;
        bool flip = false;
        if constexpr (KB == 1) {
#pragma unroll 1
            for (; rd + 1 < rounds; rd += 2) {
                step(std::true_type{});
                step(std::false_type{});
            }
            // after an ascending round the accumulator holds -(P-N)
            flip = rd < rounds;
            if (flip) step(std::true_type{});
        } else {
#pragma unroll 1
            for (; rd < rounds; ++rd) step(std::true_type{});
        }
        // store this class: rows 4*(lane/16)+v, column lane%16, T values of t
#pragma unroll
        for (int v = 0; v < 4; ++v) {
#pragma unroll
            for (int tt = 0; tt < T; tt += 4) {
                int4 q;
                q.x = flip ? -acc[tt][v] : acc[tt][v];
                q.y = flip ? -acc[tt + 1][v] : acc[tt + 1][v];
                q.z = flip ? -acc[tt + 2][v] : acc[tt + 2][v];
                q.w = flip ? -acc[tt + 3][v] : acc[tt + 3][v];
                // read once, by the inverse transform: stream past the caches
                const v4i qv = {q.x, q.y, q.z, q.w};
                __builtin_nontemporal_store(
                    qv, (v4i *)(C5 + mfh_c5_index(jp, row0 + v, col, tg * T + tt, np_, NCLASS, K,
                                                 rows) +
                                (size_t)m * mfh_c5_class_stride(np_, K)));
            }
        }
    }
}

template <class Cfg>
int launch_cfg(mfh_ctx *c, int rows)
{
    if (c->np % (MFH_KBLK * Cfg::KB) || rows % Cfg::BI || c->np % Cfg::BJ || rows < 1 ||
        rows > c->np)
        return MFH_E_UNSUPPORTED;
    const int tiles_i = rows / Cfg::BI, tiles_j = c->np / Cfg::BJ;
    static bool attr_set = false;
    if (!attr_set) {
        MFH_HIP(hipFuncSetAttribute((const void *)k_pointwise<Cfg, MFH_MODE_B8>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    Cfg::DYN_LDS));
        MFH_HIP(hipFuncSetAttribute((const void *)k_pointwise<Cfg, MFH_MODE_K7>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    Cfg::DYN_LDS));
        attr_set = true;
    }
    dim3 grid((unsigned)(tiles_i * tiles_j), (unsigned)c->NB);
    if (c->mode == MFH_MODE_K7)
        hipLaunchKernelGGL((k_pointwise<Cfg, MFH_MODE_K7>), grid, dim3(Cfg::THREADS),
                           Cfg::DYN_LDS, c->stream, c->dAh, c->dBh, c->dC5, c->np, rows,
                           tiles_j);
    else
        hipLaunchKernelGGL((k_pointwise<Cfg, MFH_MODE_B8>), grid, dim3(Cfg::THREADS),
                           Cfg::DYN_LDS, c->stream, c->dAh, c->dBh, c->dC5, c->np, rows,
                           tiles_j);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

// ============================================================================
// Gauss pointwise (MFH_PW_GAUSS, mfh_internal.hpp).  At point j the ring
// product is Re + u Im with u = y^H, H = K/2, Re = k1 - k3, Im = k1 + k2:
// three linear convolutions of length H over the operand slots the forward
// transform wrote, sub-product g multiplying A slots gH .. gH+H-1 with B
// slots gH .. gH+H-1 (B's carry the signs of Re = k1 + A1 (-(B0+B1))).
// Folded by u^2 = -1, diagonal s of Re lands on C[s], and diagonal s of Im
// on C[s+H] (s < H) or, negated, on C[s-H] (s >= H).  A wave owns one
// 16 x 16 output block and accumulates
//   g = 2 (A1 x -(B0+B1), Re):  diagonal s into C[s]
//   g = 1 (A0 x (B1-B0), Im):   diagonal s < H into C[s+H], s >= H into
//                               ng[s-H] (subtracted at the end of the class)
//   g = 0 (A0+A1 x B0, both):   diagonal s into a temporary T, then
//                               C[s] += T and C[s+H] += T or C[s-H] -= T
// so that every term enters with a fixed sign.  Each accumulator sums at
// most K digit products per k (C[t], t < H-1: t+9 <= 2H-1), as a flat class
// accumulator does, so the flat kernel's int32 bound covers them; C is then
// stored like the flat kernel's class results and the inverse transform is
// the same.
//
// Sub-rounds: (digit pair, 64-wide k block, g), H fragments of A (WBI row
// blocks) and of B (WBJ column blocks) each.  A round is the three
// sub-rounds g = 0, 1, 2 of one (pair, k block), and sub-round g always
// lives in LDS slot g (distinct arrays, so the compiler can tell a copy into
// one slot from reads of another).  A wave reads its fragment pairs D ahead
// of the MFMAs that need them, in diagonal order (c1 + c2 = s, two
// diagonals interleaved so that no MFMA waits on the one before it); after
// the diagonal group BAR, when every read of the sub-round is done, it waits
// for its copies of the next sub-round, a barrier follows, and the copies of
// the same g of the next round go into this slot: they have two
// sub-rounds to land.  After the group PRE (>= BAR: the next slot is
// complete by then), the wave reads the first D pairs of the next
// sub-round, so that its first MFMAs do not wait for LDS.
// ============================================================================
//
// NSLOT = 2 (rings whose three slots do not fit in LDS): sub-round u lives
// in slot u mod 2, so the slot of sub-round g alternates with the parity of
// the round.  After the diagonal group BAR of sub-round u (its last read of
// the slot done) a barrier follows and the copies of sub-round u+2 go into
// the slot; after the group PRE > BAR the wave waits for its copies of
// sub-round u+1 (only the ones just issued may stay in flight), a second
// barrier follows, and the first pairs of sub-round u+1 are read.  Copies
// thus have one sub-round plus PRE - BAR diagonal groups to land.
template <int K_, int WBI_, int WBJ_, int WPE_, int D_, int BAR_, int PRE_, bool SPLIT_ = false,
          int NSLOT_ = 3>
struct GsCfg {
    static constexpr int K = K_, H = K_ / 2, WBI = WBI_, WBJ = WBJ_, WPE = WPE_;
    static constexpr int D = D_, BAR = BAR_, PRE = PRE_;
    static constexpr bool SPLIT = SPLIT_;
    static constexpr int NSLOT = NSLOT_;
    static constexpr int WAVES = WBI * WBJ, THREADS = WAVES * 64;
    static constexpr int BI = 16 * WBI, BJ = 16 * WBJ;
    static constexpr int A_CHUNKS = H * WBI * 64, B_CHUNKS = H * WBJ * 64;   // one sub-round
    static constexpr int NA = H * WBI / WAVES, NBF = H * WBJ / WAVES;        // copies per wave
    static constexpr int NPW = NA + NBF;
    static constexpr int ND = 2 * H - 1;             // diagonals of a length-H convolution
    // the diagonal group (even s0) in which pair H-1 is read
    static constexpr int LAST_READ = D >= H ? -1 : ((H - 1 - D) / 2) * 2;
    static_assert((H * WBI) % WAVES == 0 && (H * WBJ) % WAVES == 0 && WAVES % WBI == 0 &&
                      WAVES % WBJ == 0,
                  "copies split evenly over waves");
    static_assert(D >= 2 && D <= H, "diagonals 0 and 1 need pairs 0 and 1");
    static_assert(BAR % 2 == 0 && BAR > LAST_READ && BAR < ND, "barrier after the last read");
    static_assert(PRE % 2 == 0 && PRE >= BAR && PRE < ND, "prefetch after the barrier");
    static_assert(!SPLIT || PRE > BAR, "split barrier: arrive before waiting");
    static_assert(NSLOT == 2 || NPW < 16, "vmcnt immediate");
    static_assert(NSLOT == 2 || NSLOT == 3, "two or three LDS slots");
    static_assert(NSLOT * (A_CHUNKS + B_CHUNKS) * 16 <= 160 * 1024, "the slots fit in LDS");
};

// s_waitcnt vmcnt(V) lgkmcnt(0) (expcnt left alone)
template <int V>
__device__ __forceinline__ void vm_lgkm_wait()
{
    static_assert(V >= 0 && V < 16, "4-bit vmcnt field");
    __builtin_amdgcn_s_waitcnt((V & 15) | (7 << 4) | (0 << 8));
}
// s_waitcnt vmcnt(V) lgkmcnt(0) for V up to 63 (gfx9: vmcnt bits 3:0 and
// 15:14)
template <int V>
__device__ __forceinline__ void vm_lgkm_wait6()
{
    static_assert(V >= 0 && V < 64, "6-bit vmcnt");
    __builtin_amdgcn_s_waitcnt((V & 15) | (7 << 4) | (0 << 8) | ((V >> 4) << 14));
}
// the same, then a workgroup barrier
template <int V>
__device__ __forceinline__ void vm_lgkm_barrier()
{
    vm_lgkm_wait<V>();
    __builtin_amdgcn_s_barrier();
}
// Split barrier in LDS (gfx950 has no split s_barrier): a wave arrives by
// adding 1 to the counter once its own waits are done, goes on with work
// that needs no other wave, and waits only where it does, until every wave
// of the workgroup has arrived as often as it has (the counter is never
// reset; waves arrive in the same sequence).
// The counter is touched by inline asm: the compiler cannot tell it apart
// from the LDS slots that copies are still filling and would wait for every
// copy before each access.  An LDS operation it does not count only makes
// its own (in-order) lgkmcnt waits stricter.
__device__ __forceinline__ void split_arrive(int *ctr)
{
    const uint32_t a = (uint32_t)(uintptr_t)ctr, one = 1;
    if ((threadIdx.x & 63) == 0) asm volatile("ds_add_u32 %0, %1" ::"v"(a), "v"(one) : "memory");
}
__device__ __forceinline__ void split_wait(int *ctr, int target)
{
    const uint32_t a = (uint32_t)(uintptr_t)ctr;
    for (;;) {
        int v;
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
        if (__builtin_amdgcn_readfirstlane(v) >= target) break;
        __builtin_amdgcn_s_sleep(1);
    }
}

// One sub-round of one wave: the length-H linear convolution of its H A and
// H B fragments (la, lb: fragment of slot-coefficient 0, strides WBI*64 and
// WBJ*64 chunks) into acc / ng as G says.  pa / pb hold its first D pairs
// on entry and the next sub-round's (nla, nlb) on return.  hook(s0) runs
// after the MFMAs of each diagonal group.
template <class Cfg, int G, class Hook>
__device__ __forceinline__ void gs_sub(v4i (&acc)[Cfg::K], v4i (&ng)[Cfg::H - 1],
                                       v4i (&pa)[Cfg::D], v4i (&pb)[Cfg::D],
                                       const v4i *__restrict__ la, const v4i *__restrict__ lb,
                                       const v4i *__restrict__ nla, const v4i *__restrict__ nlb,
                                       const Hook &hook)
{
    constexpr int H = Cfg::H, D = Cfg::D, ND = Cfg::ND;
    constexpr int SA = Cfg::WBI * 64, SB = Cfg::WBJ * 64;
    v4i af[H], bf[H];
#pragma unroll
    for (int c = 0; c < D; ++c) {
        af[c] = pa[c];
        bf[c] = pb[c];
    }
    v4i tp[2];        // g = 0: the previous group's diagonal sums, folded one group late
    // g = 0: diagonal s's sum into C[s] and C[s+H] or -C[s-H]
    auto fold = [&](int s, const v4i &t) {
        acc[s] += t;
        if (s < H) acc[s + H] += t;
        else acc[s - H] -= t;
    };
#pragma unroll
    for (int s0 = 0; s0 < ND; s0 += 2) {
#pragma unroll
        for (int c = s0 + D; c < s0 + D + 2; ++c)
            if (c < H) {
                af[c] = la[c * SA];
                bf[c] = lb[c * SB];
            }
        v4i t[2];
#pragma unroll
        for (int q = 0; q < H; ++q) {
#pragma unroll
            for (int d = 0; d < 2; ++d) {
                const int s = s0 + d;
                const int lo = s - H + 1 > 0 ? s - H + 1 : 0;
                const int hi = s < H - 1 ? s : H - 1;
                const int c1 = lo + q;
                if (s < ND && c1 <= hi) {
                    const int c2 = s - c1;
                    if constexpr (G == 0) {
                        const v4i z = {0, 0, 0, 0};
                        t[d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[c1], bf[c2],
                                                                     q == 0 ? z : t[d], 0, 0, 0);
                    } else if constexpr (G == 1) {
                        if (s < H)
                            acc[s + H] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                                af[c1], bf[c2], acc[s + H], 0, 0, 0);
                        else
                            ng[s - H] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[c1], bf[c2],
                                                                              ng[s - H], 0, 0, 0);
                    } else {
                        acc[s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[c1], bf[c2], acc[s], 0,
                                                                       0, 0);
                    }
                }
            }
        }
        if constexpr (G == 0) {
            if (s0 >= 2) {
                fold(s0 - 2, tp[0]);
                fold(s0 - 1, tp[1]);
            }
            tp[0] = t[0];
            tp[1] = t[1];
        }
        hook(s0);
        if (s0 == Cfg::PRE) {
#pragma unroll
            for (int c = 0; c < D; ++c) {
                pa[c] = nla[c * SA];
                pb[c] = nlb[c * SB];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (G == 0) fold(ND - 1, tp[0]);   // the last group holds diagonal ND-1 only
}

template <class Cfg, int MODE>
__global__ void __attribute__((amdgpu_flat_work_group_size(Cfg::THREADS, Cfg::THREADS),
                               amdgpu_waves_per_eu(Cfg::WPE, Cfg::WPE)))
k_pointwise_gauss(const int8_t *__restrict__ Ah, const int8_t *__restrict__ Bh,
                  int32_t *__restrict__ C5, int np_, int rows, int tiles_j)
{
    constexpr int K = Cfg::K, H = Cfg::H, WBI = Cfg::WBI, WBJ = Cfg::WBJ, W = Cfg::WAVES;
    constexpr int NA = Cfg::NA, NBF = Cfg::NBF, NPW = Cfg::NPW;
    constexpr int NCLASS = MODE == MFH_MODE_K7 ? 6 : 2 * MFH_DIGITS - 1;
    constexpr int PL = MODE == MFH_MODE_K7 ? 6 : MFH_DIGITS;     // planes per slot
    constexpr int NSL = 3 * H;                                    // slots per point
    __shared__ v4i sA0[Cfg::A_CHUNKS], sA1[Cfg::A_CHUNKS], sA2[Cfg::A_CHUNKS];
    __shared__ v4i sB0[Cfg::B_CHUNKS], sB1[Cfg::B_CHUNKS], sB2[Cfg::B_CHUNKS];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wbi = wave / WBJ, wbj = wave % WBJ;
    int ti, tj, jp;
    tile_of(tiles_j, ti, tj, jp);
    const int i0 = ti * Cfg::BI, j0 = tj * Cfg::BJ;
    const size_t plane = (size_t)np_ * np_;           // B: all np rows
    const size_t planeA = (size_t)rows * np_;         // A: the band's rows
    const int8_t *Aj = Ah + (size_t)jp * NSL * PL * planeA;
    const int8_t *Bj = Bh + (size_t)jp * NSL * PL * plane;
    // copies: fragment f = wave + W i of a sub-round is A slot-coefficient
    // f / WBI at row block f % WBI (= wave % WBI), B likewise with WBJ; a
    // fragment is 1 KB contiguous in the tiled planes, lane l's 16 bytes at
    // row l % 16, k 16 (l / 16)
    const int8_t *a_blk = Aj + (size_t)(wave / WBI) * PL * planeA +
                          mfh_tile_off(i0 + (wave % WBI) * 16, 0, np_) + (lane & 15) * 64 +
                          (lane >> 4) * 16;
    const int8_t *b_blk = Bj + (size_t)(wave / WBJ) * PL * plane +
                          mfh_tile_off(j0 + (wave % WBJ) * 16, 0, np_) + (lane & 15) * 64 +
                          (lane >> 4) * 16;
    const size_t da = (size_t)(W / WBI) * PL * planeA;
    const size_t db = (size_t)(W / WBJ) * PL * plane;
    const int kblocks = np_ / MFH_KBLK;
    const int col = j0 + wbj * 16 + (lane & 15);
    const int row0 = i0 + wbi * 16 + 4 * (lane >> 4);

    // copies of sub-round g of round rd of class m into slot g
    auto copy = [&](auto gtag, int m, int rd) {
        constexpr int G = decltype(gtag)::value;
        v4i *dA = G == 0 ? sA0 : G == 1 ? sA1 : sA2;
        v4i *dB = G == 0 ? sB0 : G == 1 ? sB1 : sB2;
        int rlo, npr;
        class_pairs<MODE>(m, rlo, npr);
        const int r = rlo + rd / kblocks, kb = rd % kblocks;
        const int s = MODE == MFH_MODE_K7 ? r : m - r;
        const int8_t *a0 = a_blk + ((size_t)G * H * PL + r) * planeA + kb * 1024;
        const int8_t *b0 = b_blk + ((size_t)G * H * PL + s) * plane + kb * 1024;
#pragma unroll
        for (int i = 0; i < NA; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(a0 + i * da),
                                             (void *)(dA + (wave + i * W) * 64), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < NBF; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(b0 + i * db),
                                             (void *)(dB + (wave + i * W) * 64), 16, 0, 0);
    };
    using G0 = std::integral_constant<int, 0>;
    using G1 = std::integral_constant<int, 1>;
    using G2 = std::integral_constant<int, 2>;
    auto rounds_of = [&](int m) {
        int rlo, npr;
        class_pairs<MODE>(m, rlo, npr);
        return npr * kblocks;
    };

    // arrivals of the split barrier (Cfg::SPLIT)
    __shared__ int arrived;
    if (threadIdx.x == 0) arrived = 0;
    // prologue: the three sub-rounds of round 0 of class 0
    copy(G0{}, 0, 0);
    copy(G1{}, 0, 0);
    copy(G2{}, 0, 0);
    vm_lgkm_barrier<2 * NPW>();
    int u = 0;                 // sub-rounds begun

    v4i acc[K], ng[H - 1];
    constexpr int D = Cfg::D;
    v4i pa[D], pb[D];          // the first pairs of the next sub-round
#pragma unroll
    for (int c = 0; c < D; ++c) {
        pa[c] = sA0[(c * WBI + wbi) * 64 + lane];
        pb[c] = sB0[(c * WBJ + wbj) * 64 + lane];
    }
    // Round (m, rd) runs; (nm, nrd) is the round whose copies this one
    // issues: the next round, or the last round itself again (the slot is
    // done with and never read again), so that every sub-round issues
    // exactly NPW copies and the outstanding copies are known on every path.
    auto sub = [&](auto gtag, int nm, int nrd) {
        constexpr int G = decltype(gtag)::value;
        const v4i *la = (G == 0 ? sA0 : G == 1 ? sA1 : sA2) + wbi * 64 + lane;
        const v4i *lb = (G == 0 ? sB0 : G == 1 ? sB1 : sB2) + wbj * 64 + lane;
        const v4i *nla = (G == 0 ? sA1 : G == 1 ? sA2 : sA0) + wbi * 64 + lane;
        const v4i *nlb = (G == 0 ? sB1 : G == 1 ? sB2 : sB0) + wbj * 64 + lane;
        gs_sub<Cfg, G>(acc, ng, pa, pb, la, lb, nla, nlb, [&](int s0) {
            if constexpr (Cfg::SPLIT) {
                // arrive once this wave's copies of the next sub-round have
                // landed and its reads of this slot are done; before copying
                // into the slot and reading the next one, wait until every
                // wave has
                if (s0 == Cfg::BAR) {
                    vm_lgkm_wait<NPW>();
                    split_arrive(&arrived);
                } else if (s0 == Cfg::PRE) {
                    split_wait(&arrived, Cfg::WAVES * (u + 1));
                    copy(gtag, nm, nrd);
                }
            } else if (s0 == Cfg::BAR) {
                // this wave's copies of the next sub-round have landed (only
                // those of the one after it may still be in flight) and its
                // reads of this slot are done; after the barrier every
                // wave's are
                vm_lgkm_barrier<NPW>();
                copy(gtag, nm, nrd);
            }
        });
        ++u;
    };
#pragma unroll 1
    for (int m = 0; m < NCLASS; ++m) {
#pragma unroll
        for (int t = 0; t < K; ++t) acc[t] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < H - 1; ++t) ng[t] = v4i{0, 0, 0, 0};
        const int rounds = rounds_of(m);
#pragma unroll 1
        for (int rd = 0; rd < rounds; ++rd) {
            int nm = rd + 1 < rounds ? m : m + 1, nrd = rd + 1 < rounds ? rd + 1 : 0;
            if (nm == NCLASS) {
                nm = m;
                nrd = rd;
            }
            sub(G0{}, nm, nrd);
            sub(G1{}, nm, nrd);
            sub(G2{}, nm, nrd);
        }
#pragma unroll
        for (int t = 0; t < H - 1; ++t) acc[t] -= ng[t];
        // store this class: rows 4*(lane/16)+v, column lane%16, K values of t
#pragma unroll
        for (int v = 0; v < 4; ++v) {
#pragma unroll
            for (int tt = 0; tt < K; tt += 4) {
                const v4i qv = {acc[tt][v], acc[tt + 1][v], acc[tt + 2][v], acc[tt + 3][v]};
                __builtin_nontemporal_store(
                    qv, (v4i *)(C5 + mfh_c5_index(jp, row0 + v, col, tt, np_, NCLASS, K, rows) +
                                (size_t)m * mfh_c5_class_stride(np_, K)));
            }
        }
    }
    // the last round's copies into LDS complete before the workgroup ends
    __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8));
}

template <class Cfg>
int launch_gauss(mfh_ctx *c, int rows)
{
    if (c->np % MFH_KBLK || rows % Cfg::BI || c->np % Cfg::BJ || rows < 1 || rows > c->np)
        return MFH_E_UNSUPPORTED;
    const int tiles_i = rows / Cfg::BI, tiles_j = c->np / Cfg::BJ;
    dim3 grid((unsigned)(tiles_i * tiles_j), (unsigned)c->NB);
    if (c->mode == MFH_MODE_K7)
        hipLaunchKernelGGL((k_pointwise_gauss<Cfg, MFH_MODE_K7>), grid, dim3(Cfg::THREADS), 0,
                           c->stream, c->dAh, c->dBh, c->dC5, c->np, rows, tiles_j);
    else
        hipLaunchKernelGGL((k_pointwise_gauss<Cfg, MFH_MODE_B8>), grid, dim3(Cfg::THREADS), 0,
                           c->stream, c->dAh, c->dBh, c->dC5, c->np, rows, tiles_j);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

// Two-slot Gauss kernel (Cfg::NSLOT == 2): the three sub-rounds of a round
// of parity P live in slots P, 1-P, P.  Rounds run in one sequence over all
// classes; (m, rd) is the current round and (nm, nrd) the next one (the
// last round itself at the end, so that every sub-round issues the same
// copies: the slot they land in is never read again).
template <class Cfg, int MODE>
__global__ void __attribute__((amdgpu_flat_work_group_size(Cfg::THREADS, Cfg::THREADS),
                               amdgpu_waves_per_eu(Cfg::WPE, Cfg::WPE)))
k_pointwise_gauss2(const int8_t *__restrict__ Ah, const int8_t *__restrict__ Bh,
                   int32_t *__restrict__ C5, int np_, int rows, int tiles_j)
{
    static_assert(Cfg::NSLOT == 2, "two-slot schedule");
    static_assert(MODE == MFH_MODE_K7, "one digit pair per class");
    static_assert(Cfg::PRE > Cfg::BAR && !Cfg::SPLIT, "two barriers per sub-round");
    constexpr int K = Cfg::K, H = Cfg::H, WBI = Cfg::WBI, WBJ = Cfg::WBJ, W = Cfg::WAVES;
    constexpr int NA = Cfg::NA, NBF = Cfg::NBF;
    constexpr int NCLASS = MODE == MFH_MODE_K7 ? 6 : 2 * MFH_DIGITS - 1;
    constexpr int PL = MODE == MFH_MODE_K7 ? 6 : MFH_DIGITS;     // planes per slot
    constexpr int NSL = 3 * H;                                    // slots per point
    __shared__ v4i sA0[Cfg::A_CHUNKS], sA1[Cfg::A_CHUNKS];
    __shared__ v4i sB0[Cfg::B_CHUNKS], sB1[Cfg::B_CHUNKS];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wbi = wave / WBJ, wbj = wave % WBJ;
    int ti, tj, jp;
    tile_of(tiles_j, ti, tj, jp);
    const int i0 = ti * Cfg::BI, j0 = tj * Cfg::BJ;
    const size_t plane = (size_t)np_ * np_;
    const size_t planeA = (size_t)rows * np_;
    const int8_t *Aj = Ah + (size_t)jp * NSL * PL * planeA;
    const int8_t *Bj = Bh + (size_t)jp * NSL * PL * plane;
    const int8_t *a_blk = Aj + (size_t)(wave / WBI) * PL * planeA +
                          mfh_tile_off(i0 + (wave % WBI) * 16, 0, np_) + (lane & 15) * 64 +
                          (lane >> 4) * 16;
    const int8_t *b_blk = Bj + (size_t)(wave / WBJ) * PL * plane +
                          mfh_tile_off(j0 + (wave % WBJ) * 16, 0, np_) + (lane & 15) * 64 +
                          (lane >> 4) * 16;
    const size_t da = (size_t)(W / WBI) * PL * planeA;
    const size_t db = (size_t)(W / WBJ) * PL * plane;
    const int kblocks = np_ / MFH_KBLK;
    const int col = j0 + wbj * 16 + (lane & 15);
    const int row0 = i0 + wbi * 16 + 4 * (lane >> 4);

    // copies of sub-product G of round rd of class m into slot SL
    auto copy = [&](auto gtag, auto stag, int m, int rd) {
        constexpr int G = decltype(gtag)::value, SL = decltype(stag)::value;
        v4i *dA = SL == 0 ? sA0 : sA1;
        v4i *dB = SL == 0 ? sB0 : sB1;
        int rlo, npr;
        class_pairs<MODE>(m, rlo, npr);
        const int r = rlo + rd / kblocks, kb = rd % kblocks;
        const int s = MODE == MFH_MODE_K7 ? r : m - r;
        const int8_t *a0 = a_blk + ((size_t)G * H * PL + r) * planeA + kb * 1024;
        const int8_t *b0 = b_blk + ((size_t)G * H * PL + s) * plane + kb * 1024;
#pragma unroll
        for (int i = 0; i < NA; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(a0 + i * da),
                                             (void *)(dA + (wave + i * W) * 64), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < NBF; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(b0 + i * db),
                                             (void *)(dB + (wave + i * W) * 64), 16, 0, 0);
    };
    using G0 = std::integral_constant<int, 0>;
    using G1 = std::integral_constant<int, 1>;
    using G2 = std::integral_constant<int, 2>;
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;

    // prologue: sub-rounds 0 and 1 of round 0 of class 0 (slots 0 and 1)
    copy(G0{}, S0{}, 0, 0);
    copy(G1{}, S1{}, 0, 0);
    vm_lgkm_barrier<0>();

    v4i acc[K], ng[H - 1];
    constexpr int D = Cfg::D;
    v4i pa[D], pb[D];          // the first pairs of the next sub-round
#pragma unroll
    for (int c = 0; c < D; ++c) {
        pa[c] = sA0[(c * WBI + wbi) * 64 + lane];
        pb[c] = sB0[(c * WBJ + wbj) * 64 + lane];
    }
    // sub-round G in slot SL; its copies are sub-product TG of round
    // (tm, trd), into slot SL once every wave is done reading it
    auto sub = [&](auto gtag, auto stag, auto tgtag, int tm, int trd) {
        constexpr int G = decltype(gtag)::value, SL = decltype(stag)::value;
        const v4i *la = (SL == 0 ? sA0 : sA1) + wbi * 64 + lane;
        const v4i *lb = (SL == 0 ? sB0 : sB1) + wbj * 64 + lane;
        const v4i *nla = (SL == 0 ? sA1 : sA0) + wbi * 64 + lane;
        const v4i *nlb = (SL == 0 ? sB1 : sB0) + wbj * 64 + lane;
        gs_sub<Cfg, G>(acc, ng, pa, pb, la, lb, nla, nlb, [&](int s0) {
            if (s0 == Cfg::BAR) {
                // every wave has read its last pair of this slot: refill it
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                copy(tgtag, stag, tm, trd);
            } else if (s0 == Cfg::PRE) {
                // every wave's copies of the next sub-round have landed
                // (those just issued may still be in flight)
                vm_lgkm_wait6<Cfg::NPW>();
                __builtin_amdgcn_s_barrier();
            }
        });
    };
    // one round of parity P
    auto round = [&](auto ptag, int m, int rd, int nm, int nrd) {
        constexpr int P = decltype(ptag)::value;
        using SP = std::integral_constant<int, P>;
        using SQ = std::integral_constant<int, 1 - P>;
        sub(G0{}, SP{}, G2{}, m, rd);
        sub(G1{}, SQ{}, G0{}, nm, nrd);
        sub(G2{}, SP{}, G1{}, nm, nrd);
    };
    auto zero = [&]() {
#pragma unroll
        for (int t = 0; t < K; ++t) acc[t] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < H - 1; ++t) ng[t] = v4i{0, 0, 0, 0};
    };
    // after round R: a class that ends there is stored and C restarts
    auto finish = [&](int R) {
        if ((R + 1) % kblocks) return;
        const int m = R / kblocks;
#pragma unroll
        for (int t = 0; t < H - 1; ++t) acc[t] -= ng[t];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
#pragma unroll
            for (int tt = 0; tt < K; tt += 4) {
                const v4i qv = {acc[tt][v], acc[tt + 1][v], acc[tt + 2][v], acc[tt + 3][v]};
                __builtin_nontemporal_store(
                    qv, (v4i *)(C5 + mfh_c5_index(jp, row0 + v, col, tt, np_, NCLASS, K, rows) +
                                (size_t)m * mfh_c5_class_stride(np_, K)));
            }
        }
        zero();
    };
    // K7: one digit pair per class, so round R is k block R mod kblocks of
    // class R / kblocks, and the 6 kblocks rounds pair up into parities
    // 0, 1 with no branch between the two round bodies
    const int total = NCLASS * kblocks;
    zero();
#pragma unroll 1
    for (int R = 0; R < total; R += 2) {
        round(S0{}, R / kblocks, R % kblocks, (R + 1) / kblocks, (R + 1) % kblocks);
        finish(R);
        const int n1 = R + 2 < total ? R + 2 : R + 1;
        round(S1{}, (R + 1) / kblocks, (R + 1) % kblocks, n1 / kblocks, n1 % kblocks);
        finish(R + 1);
    }
    // the last round's copies into LDS complete before the workgroup ends
    __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8));
}

template <class Cfg>
int launch_gauss2(mfh_ctx *c, int rows)
{
    if (c->np % MFH_KBLK || rows % Cfg::BI || c->np % Cfg::BJ || rows < 1 || rows > c->np)
        return MFH_E_UNSUPPORTED;
    const int tiles_i = rows / Cfg::BI, tiles_j = c->np / Cfg::BJ;
    if (c->mode != MFH_MODE_K7) return MFH_E_UNSUPPORTED;
    dim3 grid((unsigned)(tiles_i * tiles_j), (unsigned)c->NB);
    hipLaunchKernelGGL((k_pointwise_gauss2<Cfg, MFH_MODE_K7>), grid, dim3(Cfg::THREADS), 0,
                       c->stream, c->dAh, c->dBh, c->dC5, c->np, rows, tiles_j);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

// ============================================================================
// Limb-plane schoolbook on the matrix cores (src/methods.c:94-104):
//     Cw[w] = sum_{u+v=w} A_u B_v
// with every limb split into the six int8 planes of its K7 digits (d0, d1,
// d2 and the pair sums): for each Karatsuba class m the int8 planes q_m of
// the limbs are convolved, Q_m[w] = sum_{u+v=w} q_m(A_u) q_m(B_v), and
// Cw = sum_m coef_m Q_m (mfh_launch_sb_combine).  Limbs are taken in blocks
// of 16: block pair (U, V) is a length-16 linear convolution of fragment
// sequences (one sub-round of gs_sub, every diagonal d = c1 + c2 into
// acc[d]), whose diagonals 0..15 fall on output block W = U + V and 16..30
// on block W + 1.  A workgroup owns one 32 x 32 tile, one class m and one
// W: it runs the block pairs (U, W - U) for every 64-wide k block and
// stores its 31 diagonal sums as the partial P[m][W][d] (int32; exact
// modulo 2^32, and the combine step knows each partial's range).
// Sub-round s (pair U = Ulo + s / kblocks, k block s % kblocks) lives in
// LDS slot s mod 2, with the two-barrier schedule of k_pointwise_gauss2.
//
// Digit planes (mfh_launch_sb_digits): [limb u < 16 NU][class plane][rows x
// np in 16 x 64 tiles], A by rows, B transposed (entry (j', k) = B[k][j']).
// P layout: mfh_c5_index with point m * NW + W, one class, K = 32.
template <class Cfg>
__global__ void __attribute__((amdgpu_flat_work_group_size(Cfg::THREADS, Cfg::THREADS),
                               amdgpu_waves_per_eu(Cfg::WPE, Cfg::WPE)))
k_schoolbook(const int8_t *__restrict__ Ad, const int8_t *__restrict__ Bd,
             int32_t *__restrict__ P, int np_, int NU, int tiles_j)
{
    static_assert(Cfg::NSLOT == 2 && Cfg::H == 16 && Cfg::PRE > Cfg::BAR, "two-slot schedule");
    constexpr int K = Cfg::K, H = Cfg::H, WBI = Cfg::WBI, WBJ = Cfg::WBJ, W = Cfg::WAVES;
    constexpr int NA = Cfg::NA, NBF = Cfg::NBF, PL = 6;
    __shared__ v4i sA0[Cfg::A_CHUNKS], sA1[Cfg::A_CHUNKS];
    __shared__ v4i sB0[Cfg::B_CHUNKS], sB1[Cfg::B_CHUNKS];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wbi = wave / WBJ, wbj = wave % WBJ;
    const int ti = blockIdx.x / tiles_j, tj = blockIdx.x % tiles_j;
    const int NW = 2 * NU - 1;
    const int Wb = blockIdx.y % NW, m = blockIdx.y / NW;
    const int i0 = ti * Cfg::BI, j0 = tj * Cfg::BJ;
    const size_t plane = (size_t)np_ * np_;
    const int8_t *a_blk = Ad + ((size_t)(wave / WBI) * PL + m) * plane +
                          mfh_tile_off(i0 + (wave % WBI) * 16, 0, np_) + (lane & 15) * 64 +
                          (lane >> 4) * 16;
    const int8_t *b_blk = Bd + ((size_t)(wave / WBJ) * PL + m) * plane +
                          mfh_tile_off(j0 + (wave % WBJ) * 16, 0, np_) + (lane & 15) * 64 +
                          (lane >> 4) * 16;
    const size_t da = (size_t)(W / WBI) * PL * plane, db = (size_t)(W / WBJ) * PL * plane;
    const int kblocks = np_ / MFH_KBLK;
    const int Ulo = Wb - NU + 1 > 0 ? Wb - NU + 1 : 0, Uhi = Wb < NU - 1 ? Wb : NU - 1;
    const int S = (Uhi - Ulo + 1) * kblocks;              // sub-rounds
    // copies of sub-round s (s >= S: the last one again) into slot SL
    auto copy = [&](auto stag, int s) {
        constexpr int SL = decltype(stag)::value;
        if (s >= S) s = S - 1;
        const int U = Ulo + s / kblocks, kb = s % kblocks, V = Wb - U;
        v4i *dA = SL == 0 ? sA0 : sA1;
        v4i *dB = SL == 0 ? sB0 : sB1;
        const int8_t *a0 = a_blk + (size_t)U * H * PL * plane + kb * 1024;
        const int8_t *b0 = b_blk + (size_t)V * H * PL * plane + kb * 1024;
#pragma unroll
        for (int i = 0; i < NA; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(a0 + i * da),
                                             (void *)(dA + (wave + i * W) * 64), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < NBF; ++i)
            __builtin_amdgcn_global_load_lds((const void *)(b0 + i * db),
                                             (void *)(dB + (wave + i * W) * 64), 16, 0, 0);
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using G2 = std::integral_constant<int, 2>;
    copy(S0{}, 0);
    copy(S1{}, 1);
    vm_lgkm_barrier<0>();
    v4i acc[K], ng[H - 1];
#pragma unroll
    for (int t = 0; t < K; ++t) acc[t] = v4i{0, 0, 0, 0};
    constexpr int D = Cfg::D;
    v4i pa[D], pb[D];
#pragma unroll
    for (int c = 0; c < D; ++c) {
        pa[c] = sA0[(c * WBI + wbi) * 64 + lane];
        pb[c] = sB0[(c * WBJ + wbj) * 64 + lane];
    }
    // sub-round s in slot SL; its copies are those of sub-round s + 2
    auto sub = [&](auto stag, int s) {
        constexpr int SL = decltype(stag)::value;
        const v4i *la = (SL == 0 ? sA0 : sA1) + wbi * 64 + lane;
        const v4i *lb = (SL == 0 ? sB0 : sB1) + wbj * 64 + lane;
        const v4i *nla = (SL == 0 ? sA1 : sA0) + wbi * 64 + lane;
        const v4i *nlb = (SL == 0 ? sB1 : sB0) + wbj * 64 + lane;
        gs_sub<Cfg, G2::value>(acc, ng, pa, pb, la, lb, nla, nlb, [&](int s0) {
            if (s0 == Cfg::BAR) {
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                copy(stag, s + 2);
            } else if (s0 == Cfg::PRE) {
                vm_lgkm_wait6<Cfg::NPW>();
                __builtin_amdgcn_s_barrier();
            }
        });
    };
#pragma unroll 1
    for (int s = 0; s < S; s += 2) {
        sub(S0{}, s);
        if (s + 1 < S) sub(S1{}, s + 1);
    }
    const int col = j0 + wbj * 16 + (lane & 15);
    const int row0 = i0 + wbi * 16 + 4 * (lane >> 4);
    const int jp = m * NW + Wb;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
#pragma unroll
        for (int tt = 0; tt < K; tt += 4) {
            const v4i qv = {acc[tt][v], acc[tt + 1][v], acc[tt + 2][v],
                            tt + 3 < K - 1 ? acc[tt + 3][v] : 0};
            __builtin_nontemporal_store(
                qv, (v4i *)(P + mfh_c5_index(jp, row0 + v, col, tt, np_, 1, K, np_)));
        }
    }
    __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8));
}

}  // namespace

// K values with a Gauss kernel (the forward transform writes Gauss slots
// only for these)
bool mfh_gauss_supported(int K) { return K == 8 || K == 16 || K == 32; }

int mfh_launch_schoolbook(const int8_t *Ad, const int8_t *Bd, int32_t *P, int np_, int NU,
                          hipStream_t st)
{
    using Cfg = GsCfg<32, 2, 2, 1, 4, 12, 24, false, 2>;
    if (np_ % MFH_KBLK || np_ % Cfg::BI || np_ % Cfg::BJ || NU < 1) return MFH_E_ARG;
    const int tiles_i = np_ / Cfg::BI, tiles_j = np_ / Cfg::BJ;
    dim3 grid((unsigned)(tiles_i * tiles_j), (unsigned)(6 * (2 * NU - 1)));
    hipLaunchKernelGGL(k_schoolbook<Cfg>, grid, dim3(Cfg::THREADS), 0, st, Ad, Bd, P, np_, NU,
                       tiles_j);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_pointwise(mfh_ctx *c, int rows)
{
    // the product's algorithm, set with its digit mode: the forward
    // transform wrote Gauss slots only when pwr says so
    if (c->pwr == MFH_PW_GAUSS) {
        switch (c->K) {
        // 64 x 32 tiles, 8 waves at 2 per SIMD, pairs read 4 ahead, barrier
        // after diagonal group 4, the next sub-round's first pairs read
        // after group 8
        case 16: return launch_gauss<GsCfg<16, 4, 2, 2, 4, 4, 8, true>>(c, rows);
        // 64 x 64 tiles, 16 waves at 4 per SIMD (96 KiB of slots), pairs
        // read 3 ahead, barrier after diagonal group 2, the next
        // sub-round's first pairs read after group 4 (512-bit n = 4096:
        // pointwise 262.8 -> 245.0 ms, product 277.7 -> 263.0 ms; fp32 on
        // the 512-bit grid at n = 2048 about equal)
        case 8: return launch_gauss<GsCfg<8, 4, 4, 4, 3, 2, 4, false>>(c, rows);
        // 32 x 32 tiles, 4 waves at 1 per SIMD, two 64 KiB slots, pairs
        // read 4 ahead, slot refilled after diagonal group 12, the next
        // sub-round's copies waited for after group 24 (4.30 -> 4.18 ms
        // at n = 256 with whole points per XCD, against 4.58 for the flat
        // kernel)
        case 32: return launch_gauss2<GsCfg<32, 2, 2, 1, 4, 12, 24, false, 2>>(c, rows);
        default: return MFH_E_UNSUPPORTED;
        }
    }
    switch (c->K) {
    case 4:  return launch_cfg<PwCfg<4, 4, 2, 2>>(c, rows);
    // K = 8 and K = 16: copy fills with the B fragments held in registers,
    // one workgroup per CU (64 x 64 tiles, 16 waves at 4 per SIMD, 116
    // VGPRs; 64 x 32 tiles, 8 waves at 2 per SIMD, 232 VGPRs): measured
    // 11-13 % (K = 8) and 5 % (K = 16) faster than two workgroups per CU
    // with half the tile.  Shell schedule with fragment pairs read 4 (K = 8)
    // or 7 (K = 16) pairs ahead; the barrier and the copies come after
    // shell 3 (K = 8) or 11 (K = 16), the earliest points at which every
    // read of the round has been issued.  Against the step schedule
    // (all A fragments before the first MFMA, barrier after step 1 or 2):
    // pointwise 1.2 % (K = 8, n = 4096) and 1.5-2 % (K = 16, n = 1024)
    // faster; barriers one to three shells later were 2-11 % slower.
    case 8:  return launch_cfg<PwCfg<8, 8, 4, 4, 1, 4, true, 5, 4>>(c, rows);
    case 16: return launch_cfg<PwCfg<16, 16, 4, 2, 1, 2, true, 13, 7>>(c, rows);
    // K = 32: the same with one 4-wave workgroup per CU at one wave per
    // SIMD (fragments and accumulators need 256 VGPRs + 234 AGPRs; 6 %
    // faster than 8-coefficient waves with a sliding A window); shell
    // schedule, 7 pairs ahead, barrier after shell 24 (2 % faster than the
    // barrier before the first MFMA with all fragments read up front)
    case 32: return launch_cfg<PwCfg<32, 32, 2, 2, 1, 1, true, 26, 7>>(c, rows);
    default: return MFH_E_UNSUPPORTED;
    }
}
