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
// shared by 8 of its workgroups; otherwise tiles are taken in row order.
__device__ __forceinline__ void tile_of(int tiles_j, int &ti, int &tj, int &jp)
{
    const int per_point = gridDim.x, tiles_i = per_point / tiles_j;
    if (tiles_i % 16 == 0 && tiles_j % 32 == 0) {
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

}  // namespace

int mfh_launch_pointwise(mfh_ctx *c, int rows)
{
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
