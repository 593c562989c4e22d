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
// Each transformed value is three balanced int8 digits (see
// mfh_internal.hpp); the products of digit r of A and digit s of B are
// accumulated in int32 per weight class m = r+s (2^(8m)) and flushed into
// int64 totals, which are the exact C^_j[t].
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
// Operands in HBM: digit plane (j, c, r) is an np x np int8 matrix,
// row-major with the reduction index k contiguous (A as A[i][k], B stored
// transposed as B^T[j'][k]).  Each round stages, for all K ring
// coefficients, a (16*WBI) x 64 tile of A and a (16*WBJ) x 64 tile of B^T
// into LDS in MFMA operand order (lane l of a 16x64 fragment = row l%16,
// k bytes 16*(l/16) .. +15; A and B use the same k order, so the dot
// product is the same whatever order the hardware sums in).
//
// Output C^[j][i][j'][t] int64: the K ring coefficients of one element are
// contiguous, which is the order the inverse transform reads.
#include <type_traits>

#include "mfh_internal.hpp"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int pmod(int a, int m) { return ((a % m) + m) % m; }

template <int K_, int T_, int WBI_, int WBJ_>
struct PwCfg {
    static constexpr int K = K_, T = T_, WBI = WBI_, WBJ = WBJ_;
    static constexpr int G = K / T;                 // t-groups per block
    static constexpr int WAVES = WBI * WBJ * G;
    static constexpr int THREADS = WAVES * 64;
    static constexpr int BI = 16 * WBI, BJ = 16 * WBJ;
    static constexpr int A_CHUNKS = K * WBI * 64;   // 16-byte LDS chunks
    static constexpr int B_CHUNKS = K * WBJ * 64;
    static constexpr int LDS_BYTES = 2 * (A_CHUNKS + B_CHUNKS) * 16;  // double-buffered
};

// One round: one 64-wide k block of one digit pair, all K values of c2.
// la points at this wave's A fragment of ring coefficient 0 (stride
// WBI*64 chunks per coefficient), lb likewise for B.
template <class Cfg, bool ASC, int T0, class Issue>
__device__ __forceinline__ void pw_round(v4i (&acc)[Cfg::T], const v4i *__restrict__ la,
                                         const v4i *__restrict__ lb, const Issue &issue)
{
    constexpr int K = Cfg::K, T = Cfg::T;
    constexpr int SA = Cfg::WBI * 64, SB = Cfg::WBJ * 64;
    if constexpr (T == K) {
        // every A fragment is live at every step: hold all K of them
        v4i af[K];
#pragma unroll
        for (int c1 = 0; c1 < K; ++c1) af[c1] = la[c1 * SA];
#pragma unroll
        for (int st = 0; st < K; ++st) {
            const int c2 = ASC ? st : K - 1 - st;
            const v4i bf = lb[c2 * SB];
            issue(st);
#pragma unroll
            for (int tt = 0; tt < T; ++tt) {
                const int t = tt;
                if ((ASC && c2 == t + 1) || (!ASC && c2 == t)) acc[tt] = -acc[tt];
                acc[tt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[pmod(t - c2, K)], bf,
                                                                acc[tt], 0, 0, 0);
            }
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
// one vector offset.  The loads of round r+1 are spread over the steps of
// round r (one or more per step) so they never stall the MFMA stream.
template <class Cfg>
struct RoundLoads {
    static constexpr int K = Cfg::K, WBI = Cfg::WBI, WBJ = Cfg::WBJ, W = Cfg::WAVES;
    static constexpr int FA = K * WBI, FB = K * WBJ;
    static constexpr int NA = FA / W, NB = FB / W;      // per wave
    static_assert(FA % W == 0 && FB % W == 0, "fragments must split evenly over waves");
    const int8_t *a0, *b0;      // this round's first A / B fragment of this wave
    size_t da, db;              // byte step between a wave's consecutive fragments
    v4i *lds_a, *lds_b;         // LDS destination of the first fragment
    uint32_t lane_off;          // row * np + 16 * quarter
    bool active;
    __device__ __forceinline__ void operator()(int st) const
    {
        if (!active) return;
        constexpr int N = NA + NB;
        // loads i with i*K/N == st, i.e. i in [ceil(st*N/K), ceil((st+1)*N/K))
#pragma unroll
        for (int i = 0; i < N; ++i) {
            if ((i * K) / N != st) continue;
            if (i < NA)
                __builtin_amdgcn_global_load_lds((const void *)(a0 + i * da + lane_off),
                                                 (void *)(lds_a + i * W * 64), 16, 0, 0);
            else
                __builtin_amdgcn_global_load_lds((const void *)(b0 + (i - NA) * db + lane_off),
                                                 (void *)(lds_b + (i - NA) * W * 64), 16, 0, 0);
        }
    }
};

template <class Cfg>
__global__ void __attribute__((amdgpu_flat_work_group_size(Cfg::THREADS, Cfg::THREADS),
                               amdgpu_waves_per_eu(1, 1)))
k_pointwise(const int8_t *__restrict__ Ah, const int8_t *__restrict__ Bh,
            int64_t *__restrict__ Ch, int np_, int tiles_j, int rounds_per_flush)
{
    constexpr int K = Cfg::K, T = Cfg::T, WBI = Cfg::WBI, WBJ = Cfg::WBJ;
    constexpr int BUF = Cfg::A_CHUNKS + Cfg::B_CHUNKS;   // 16-byte chunks per buffer
    using RL_ = RoundLoads<Cfg>;
    extern __shared__ v4i lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tg = wave / (WBI * WBJ);
    const int wb = wave % (WBI * WBJ);
    const int wbi = wb / WBJ, wbj = wb % WBJ;
    const int ti = blockIdx.x / tiles_j, tj = blockIdx.x % tiles_j;
    const int jp = blockIdx.y;
    const int i0 = ti * Cfg::BI, j0 = tj * Cfg::BJ;
    const size_t plane = (size_t)np_ * np_;
    const int8_t *Aj = Ah + (size_t)jp * K * MFH_DIGITS * plane;
    const int8_t *Bj = Bh + (size_t)jp * K * MFH_DIGITS * plane;

    // this wave's load slots: fragment f = wave + WAVES*i
    //   A: f < FA, coefficient f / WBI, row block f % WBI
    //   B: f - FA,  coefficient (f-FA) / WBJ, column block (f-FA) % WBJ
    const int fa = wave, fb = wave;              // first slot of each kind
    const int8_t *a_blk = Aj + (size_t)(fa / WBI) * MFH_DIGITS * plane +
                          (size_t)(i0 + (fa % WBI) * 16) * np_;
    const int8_t *b_blk = Bj + (size_t)(fb / WBJ) * MFH_DIGITS * plane +
                          (size_t)(j0 + (fb % WBJ) * 16) * np_;
    const size_t da = (size_t)(Cfg::WAVES / WBI) * MFH_DIGITS * plane;
    const size_t db = (size_t)(Cfg::WAVES / WBJ) * MFH_DIGITS * plane;
    const uint32_t lane_off = (uint32_t)((lane & 15) * np_ + (lane >> 4) * 16);

    long long tot[T][4];
    v4i acc[T];
#pragma unroll
    for (int tt = 0; tt < T; ++tt) {
        acc[tt] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int v = 0; v < 4; ++v) tot[tt][v] = 0;
    }

    const int kblocks = np_ / MFH_KBLK;
    const int rounds = MFH_DIGITS * MFH_DIGITS * kblocks;
    auto loads_for = [&](int rd) {
        RL_ q;
        int r, s, m;
        pair_of(rd / kblocks, r, s, m);
        const int kb = rd % kblocks;
        v4i *buf = lds + (rd & 1) * BUF;
        q.a0 = a_blk + (size_t)r * plane + kb * MFH_KBLK;
        q.b0 = b_blk + (size_t)s * plane + kb * MFH_KBLK;
        q.da = da;
        q.db = db;
        q.lds_a = buf + fa * 64;
        q.lds_b = buf + Cfg::A_CHUNKS + fb * 64;
        q.lane_off = lane_off;
        q.active = rd < rounds;
        return q;
    };
    // prologue: round 0, all at once
    {
        RL_ q0 = loads_for(0);
#pragma unroll
        for (int st = 0; st < K; ++st) q0(st);
    }
    int since = 0;
    auto one_round = [&](int rd, auto asc_tag) {
        constexpr bool ASC = decltype(asc_tag)::value;
        const v4i *cur = lds + (rd & 1) * BUF;
        // this round's tiles have landed (own loads), and every wave is done
        // with the buffer the next round's loads overwrite
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const RL_ q = loads_for(rd + 1);
        const v4i *la = cur + wbi * 64 + lane;
        const v4i *lb = cur + Cfg::A_CHUNKS + wbj * 64 + lane;
        pw_dispatch<Cfg, ASC>(tg, acc, la, lb, q);
        ++since;
        int r, s, m, rn, sn, mn;
        pair_of(rd / kblocks, r, s, m);
        const bool last = rd + 1 == rounds;
        mn = m;
        if (!last) pair_of((rd + 1) / kblocks, rn, sn, mn);
        if (last || mn != m || since == rounds_per_flush) {
            // after an ascending round acc = -(P-N), after a descending one +(P-N)
            const long long w = (ASC ? -1LL : 1LL) << (8 * m);
#pragma unroll
            for (int tt = 0; tt < T; ++tt) {
#pragma unroll
                for (int v = 0; v < 4; ++v) tot[tt][v] += (long long)acc[tt][v] * w;
                acc[tt] = v4i{0, 0, 0, 0};
            }
            since = 0;
        }
    };
    int rd = 0;
    for (; rd + 1 < rounds; rd += 2) {
        one_round(rd, std::true_type{});
        one_round(rd + 1, std::false_type{});
    }
    if (rd < rounds) one_round(rd, std::true_type{});

    // epilogue: lane holds rows 4*(lane/16)+v, column lane%16 of its block
    const int col = j0 + wbj * 16 + (lane & 15);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int row = i0 + wbi * 16 + 4 * (lane >> 4) + v;
        long long *dst = (long long *)Ch + (((size_t)jp * np_ + row) * np_ + col) * K + tg * T;
#pragma unroll
        for (int tt = 0; tt < T; tt += 2)
            *(longlong2 *)(dst + tt) = make_longlong2(tot[tt][v], tot[tt + 1][v]);
    }
}

template <class Cfg>
int launch_cfg(mfh_ctx *c)
{
    const int tiles_i = c->np / Cfg::BI, tiles_j = c->np / Cfg::BJ;
    static bool attr_set = false;
    if (!attr_set) {
        MFH_HIP(hipFuncSetAttribute((const void *)k_pointwise<Cfg>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    Cfg::LDS_BYTES));
        attr_set = true;
    }
    dim3 grid((unsigned)(tiles_i * tiles_j), (unsigned)c->NB);
    hipLaunchKernelGGL(k_pointwise<Cfg>, grid, dim3(Cfg::THREADS), Cfg::LDS_BYTES,
                       c->stream, c->dAh, c->dBh, c->dCh, c->np, tiles_j,
                       mfh_rounds_per_flush(c->K));
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

}  // namespace

int mfh_launch_pointwise(mfh_ctx *c)
{
    switch (c->K) {
    case 4:  return launch_cfg<PwCfg<4, 4, 2, 2>>(c);
    case 8:  return launch_cfg<PwCfg<8, 8, 2, 2>>(c);
    case 16: return launch_cfg<PwCfg<16, 16, 2, 2>>(c);
    case 32: return launch_cfg<PwCfg<32, 8, 1, 1>>(c);
    default: return MFH_E_UNSUPPORTED;
    }
}
