// mfh_limbplane.hip -- the schoolbook side of the library on gfx950: the leaf
// operator mm_accum (C += sign * A * B on int32 n x n matrices, int64 C) and
// the limb-plane convolution
//     Cw[w] = sum_{u+v=w} A_u B_v,   w = 0 .. 2L-2      (src/methods.c:94-104)
// as one batched launch.  Both are exact modulo 2^64, like the reference's
// int64 leaves (src/kernel.c:132-158): every product of two int32 values is
// formed exactly in 64 bits and the sums wrap, so the result does not
// depend on the order of summation.
//
// These run on the integer vector ALU (v_mad_i64_i32 class instructions),
// not on the int8 matrix cores: any int32 entry is accepted, which the
// digit-split MFMA path cannot do, so the schoolbook stays an independent
// second computation of every product the MFFT path makes.
//
// Tiling: a 256-thread workgroup owns a 64 x 64 output tile; each thread
// owns a 4 x 4 block (rows 4*(tid/16).., columns 4*(tid%16)..).  The k
// dimension is walked in slices of 32: the A slice is stored transposed in
// LDS (As[k][row]) and the B slice as is (Bs[k][col]), so a thread reads
// four consecutive rows and four consecutive columns with two 16-byte LDS
// loads per k and issues 16 multiply-adds.  Rows padded by 4 ints keep the
// transposed stores of A off a single bank.
#include "mfh_internal.hpp"

namespace {

constexpr int TI = 64, TK = 32, PADW = TI + 4;

// a limb; `sgn` reads a uint16 limb as int16 (the top limb of a two's
// complement entry)
template <class T>
__device__ __forceinline__ int load_in(const T *p, size_t off, bool sgn)
{
    if constexpr (sizeof(T) == 2) return sgn ? (int)(int16_t)p[off] : (int)p[off];
    else return (int)p[off];
}

// one k slice of A (rows i0.., cols k0..) and of B (rows k0.., cols j0..)
// into LDS; zero outside the n x n matrices
template <class T>
__device__ __forceinline__ void stage(int (*As)[PADW], int (*Bs)[PADW], const T *__restrict__ A,
                                      const T *__restrict__ B, int n, int i0, int j0, int k0,
                                      bool sgnA = false, bool sgnB = false)
{
    const int tid = threadIdx.x;
#pragma unroll
    for (int r = 0; r < (TI * TK) / 256; ++r) {
        const int idx = tid + 256 * r;
        // A: 32 consecutive k of one row per 32 threads (coalesced reads)
        const int ar = idx / TK, ak = idx % TK;
        const int gi = i0 + ar, gk = k0 + ak;
        As[ak][ar] = (gi < n && gk < n) ? load_in(A, (size_t)gi * n + gk, sgnA) : 0;
        // B: 64 consecutive columns of one k row per 64 threads
        const int bk = idx / TI, bc = idx % TI;
        const int gkb = k0 + bk, gj = j0 + bc;
        Bs[bk][bc] = (gkb < n && gj < n) ? load_in(B, (size_t)gkb * n + gj, sgnB) : 0;
    }
}

__device__ __forceinline__ void mac_slice(unsigned long long (&acc)[4][4], int (*As)[PADW],
                                          int (*Bs)[PADW], int r0, int c0)
{
#pragma unroll 8
    for (int kk = 0; kk < TK; ++kk) {
        const int4 a = *(const int4 *)&As[kk][r0];
        const int4 b = *(const int4 *)&Bs[kk][c0];
        const int av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int x = 0; x < 4; ++x)
#pragma unroll
            for (int y = 0; y < 4; ++y)
                acc[x][y] += (unsigned long long)((long long)av[x] * (long long)bv[y]);
    }
}

// C += sign * A * B (sign > 0 adds, otherwise subtracts: src/kernel.c:157)
__global__ __launch_bounds__(256) void k_mm_accum(long long *__restrict__ C,
                                                  const int32_t *__restrict__ A,
                                                  const int32_t *__restrict__ B, int n, int sign)
{
    __shared__ __align__(16) int As[TK][PADW];
    __shared__ __align__(16) int Bs[TK][PADW];
    const int i0 = blockIdx.y * TI, j0 = blockIdx.x * TI;
    const int r0 = 4 * (threadIdx.x / 16), c0 = 4 * (threadIdx.x % 16);
    unsigned long long acc[4][4] = {};
    for (int k0 = 0; k0 < n; k0 += TK) {
        stage(As, Bs, A, B, n, i0, j0, k0);
        __syncthreads();
        mac_slice(acc, As, Bs, r0, c0);
        __syncthreads();
    }
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y) {
            const int i = i0 + r0 + x, j = j0 + c0 + y;
            if (i < n && j < n) {
                unsigned long long *p = (unsigned long long *)&C[(size_t)i * n + j];
                *p = sign > 0 ? *p + acc[x][y] : *p - acc[x][y];
            }
        }
}

// Cw[w] for w = blockIdx.z: sum over the limb pairs (u, w-u) inside [0, L);
// signed_top reads limb L-1 of uint16 inputs as int16
template <class T>
__global__ __launch_bounds__(256) void k_conv_limbplane(long long *__restrict__ Cw,
                                                        const T *__restrict__ A,
                                                        const T *__restrict__ B, int n, int L,
                                                        int signed_top)
{
    __shared__ __align__(16) int As[TK][PADW];
    __shared__ __align__(16) int Bs[TK][PADW];
    const size_t nn = (size_t)n * n;
    const int w = blockIdx.z;
    const int i0 = blockIdx.y * TI, j0 = blockIdx.x * TI;
    const int r0 = 4 * (threadIdx.x / 16), c0 = 4 * (threadIdx.x % 16);
    const int ulo = w - L + 1 > 0 ? w - L + 1 : 0, uhi = w < L - 1 ? w : L - 1;
    unsigned long long acc[4][4] = {};
    for (int u = ulo; u <= uhi; ++u) {
        const T *Au = A + (size_t)u * nn, *Bv = B + (size_t)(w - u) * nn;
        for (int k0 = 0; k0 < n; k0 += TK) {
            stage(As, Bs, Au, Bv, n, i0, j0, k0, signed_top && u == L - 1,
                  signed_top && w - u == L - 1);
            __syncthreads();
            mac_slice(acc, As, Bs, r0, c0);
            __syncthreads();
        }
    }
    long long *Cout = Cw + (size_t)w * nn;
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y) {
            const int i = i0 + r0 + x, j = j0 + c0 + y;
            if (i < n && j < n) Cout[(size_t)i * n + j] = (long long)acc[x][y];
        }
}

// C[t] = lin[t] - lin[t+K] (t^K = -1) over the 2K-1 planes of a linear
// convolution, wrapping modulo 2^64
__global__ __launch_bounds__(256) void k_negfold(const long long *__restrict__ lin,
                                                 long long *__restrict__ C, size_t nn, int K)
{
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)K * nn) return;
    const int t = (int)(idx / nn);
    const size_t e = idx % nn;
    unsigned long long v = (unsigned long long)lin[idx];
    if (t + K < 2 * K - 1) v -= (unsigned long long)lin[(size_t)(t + K) * nn + e];
    C[idx] = (long long)v;
}

// entry-major limbs e[idx*L + u] -> plane-major p[u*nn + idx]
// (src/bigmat.c:37-46 inverted), through a 64 x 64 LDS tile: rows of the
// entry-major matrix are elements (blockIdx.x), columns limbs (blockIdx.y)
__global__ __launch_bounds__(256) void k_entry_to_plane(const uint16_t *__restrict__ e,
                                                        uint16_t *__restrict__ p, size_t nn,
                                                        int L)
{
    __shared__ uint16_t tile[64][66];
    const size_t r0 = (size_t)blockIdx.x * 64;
    const int c0 = blockIdx.y * 64;
    const int tx = threadIdx.x % 64, ty = threadIdx.x / 64;
    for (int r = ty; r < 64; r += 4) {
        const size_t rr = r0 + r;
        const int cc = c0 + tx;
        if (rr < nn && cc < L) tile[r][tx] = e[rr * L + cc];
    }
    __syncthreads();
    for (int c = ty; c < 64; c += 4) {
        const int cc = c0 + c;
        const size_t rr = r0 + tx;
        if (rr < nn && cc < L) p[(size_t)cc * nn + rr] = tile[tx][c];
    }
}

// ---- the schoolbook on the matrix cores (k_schoolbook, mfh_pointwise.hip) --
// K7 digit planes of uint16 limbs (the top one read as int16 for two's
// complement entries): out[u][p][tile order of (i, k)] for limbs
// u < NLp (zero from L on) and i, k < np (zero outside n x n); plane u of
// the source holds entry (i, k) at u*n*n + i*n + k (B is transposed first).
// One thread per 4 consecutive k of a row: one dword of each plane.
template <class T>
__global__ __launch_bounds__(256) void k_sb_digits(const T *__restrict__ src,
                                                   int8_t *__restrict__ out, int n, int np_,
                                                   int L, int NLp, int sgn_top)
{
    const size_t per_plane = (size_t)np_ * np_ / 4;
    const size_t q = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= (size_t)NLp * per_plane) return;
    const int u = (int)(q / per_plane);
    const size_t e4 = (q % per_plane) * 4;
    int i, k;
    mfh_tile_ik(e4, np_, i, k);
    const size_t nn = (size_t)n * n;
    uint32_t w[6] = {0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        int v = 0;
        if (u < L && i < n && k + d < n)
            v = load_in(src, (size_t)u * nn + (size_t)i * n + k + d, sgn_top && u == L - 1);
        const int d0 = ((v + 64) & 127) - 64;
        const int v1 = (v + 64) >> 7;
        const int d1 = ((v1 + 64) & 127) - 64;
        const int d2 = (v1 + 64) >> 7;
        const int dg[6] = {d0, d1, d2, d0 + d1, d0 + d2, d1 + d2};
#pragma unroll
        for (int p = 0; p < 6; ++p) w[p] |= (uint32_t)(uint8_t)(int8_t)dg[p] << (8 * d);
    }
    const size_t plane = (size_t)np_ * np_;
#pragma unroll
    for (int p = 0; p < 6; ++p) *(uint32_t *)(out + ((size_t)u * 6 + p) * plane + e4) = w[p];
}

// Cw[w] = sum_m coef_m Q_m[w], Q_m[w] = P[m][w/16][w%16] + P[m][w/16-1][w%16+16]
// (the Karatsuba recombination of the 6 classes is linear); each int32
// partial is the residue mod 2^32 of a value in [lo, lo + 2^32).  One
// thread per element walks w upwards: with Cw set it writes the 2L-1
// coefficient planes, else it carries them into RL uint16 limbs (the
// arithmetic-shift carry of normalize_planes, src/bigmat.c:48-60).
__global__ __launch_bounds__(256) void k_sb_combine(const int32_t *__restrict__ P,
                                                    long long *__restrict__ Cw,
                                                    uint16_t *__restrict__ out, int RL, int n,
                                                    int np_, int L, int NU, long long lo)
{
    const size_t nn = (size_t)n * n;
    const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= nn) return;
    const int i = (int)(e / n), j = (int)(e % n);
    const int NW = 2 * NU - 1, P2 = 2 * L - 1;
    const long long coef[6] = {1 - 128 - 16384, -128 + 16384 - 2097152,
                               -16384 - 2097152 + 268435456, 128, 16384, 2097152};
    long long prev[16], cc = 0;
#pragma unroll
    for (int c = 0; c < 16; ++c) prev[c] = 0;
    auto emit = [&](int w, long long v) {
        if (w >= P2) return;
        if (Cw) {
            Cw[(size_t)w * nn + e] = v;
        } else if (w < RL) {
            const long long x = cc + v;
            out[(size_t)w * nn + e] = (uint16_t)(x & 0xFFFF);
            cc = x >> 16;
        }
    };
#pragma unroll 1
    for (int wb = 0; wb < NW; ++wb) {
        long long cl[16], ch[16];
#pragma unroll
        for (int c = 0; c < 16; ++c) cl[c] = ch[c] = 0;
#pragma unroll
        for (int m = 0; m < 6; ++m) {
            const int32_t *p = P + mfh_c5_index(m * NW + wb, i, j, 0, np_, 1, 32, np_);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                typedef int v4i __attribute__((ext_vector_type(4)));
                const v4i v4 = __builtin_nontemporal_load((const v4i *)(p + q * 64));
                const int vv[4] = {v4[0], v4[1], v4[2], v4[3]};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = 4 * q + r;
                    if (t == 31) continue;
                    const long long val =
                        lo + (long long)(uint32_t)((uint32_t)vv[r] - (uint32_t)lo);
                    if (t < 16) cl[t] += coef[m] * val;
                    else ch[t - 16] += coef[m] * val;
                }
            }
        }
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            emit(16 * wb + c, cl[c] + prev[c]);
            prev[c] = ch[c];
        }
    }
#pragma unroll
    for (int c = 0; c < 16; ++c) emit(16 * NW + c, prev[c]);
    if (!Cw)
        for (int w = P2; w < RL; ++w) {
            out[(size_t)w * nn + e] = (uint16_t)(cc & 0xFFFF);
            cc >>= 16;
        }
}

}  // namespace

int mfh_launch_entry_to_plane(const uint16_t *e, uint16_t *p, int n, int L, hipStream_t st)
{
    const size_t nn = (size_t)n * n;
    const dim3 grid((unsigned)((nn + 63) / 64), (unsigned)((L + 63) / 64));
    hipLaunchKernelGGL(k_entry_to_plane, grid, dim3(256), 0, st, e, p, nn, L);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_negfold(const int64_t *lin, int64_t *C, int n, int K, hipStream_t st)
{
    const size_t nn = (size_t)n * n, cnt = (size_t)K * nn;
    hipLaunchKernelGGL(k_negfold, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, st,
                       (const long long *)lin, (long long *)C, nn, K);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_mm_accum(int64_t *C, const int32_t *A, const int32_t *B, int n, int sign,
                        hipStream_t st)
{
    const unsigned t = (unsigned)((n + TI - 1) / TI);
    hipLaunchKernelGGL(k_mm_accum, dim3(t, t), dim3(256), 0, st, (long long *)C, A, B, n, sign);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_conv_limbplane(int64_t *Cw, const void *A, const void *B, int in_kind, int n,
                              int L, hipStream_t st)
{
    const unsigned t = (unsigned)((n + TI - 1) / TI);
    const dim3 grid(t, t, (unsigned)(2 * L - 1));
    if (in_kind == MFH_IN_U16 || in_kind == MFH_IN_U16_SIGNED)
        hipLaunchKernelGGL(k_conv_limbplane<uint16_t>, grid, dim3(256), 0, st, (long long *)Cw,
                           (const uint16_t *)A, (const uint16_t *)B, n, L,
                           (int)(in_kind == MFH_IN_U16_SIGNED));
    else if (in_kind == MFH_IN_I32)
        hipLaunchKernelGGL(k_conv_limbplane<int32_t>, grid, dim3(256), 0, st, (long long *)Cw,
                           (const int32_t *)A, (const int32_t *)B, n, L, 0);
    else
        return MFH_E_ARG;
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_sb_digits(const void *src, int in_kind, int8_t *out, int n, int np_, int L,
                         int NLp, hipStream_t st)
{
    const size_t threads = (size_t)NLp * np_ * np_ / 4;
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (in_kind != MFH_IN_U16 && in_kind != MFH_IN_U16_SIGNED) return MFH_E_ARG;
    hipLaunchKernelGGL(k_sb_digits<uint16_t>, grid, dim3(256), 0, st, (const uint16_t *)src, out,
                       n, np_, L, NLp, (int)(in_kind == MFH_IN_U16_SIGNED));
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_sb_combine(const int32_t *P, int64_t *Cw, uint16_t *out, int RL, int n, int np_,
                          int L, int NU, long long lo, hipStream_t st)
{
    const size_t nn = (size_t)n * n;
    hipLaunchKernelGGL(k_sb_combine, dim3((unsigned)((nn + 255) / 256)), dim3(256), 0, st, P,
                       (long long *)Cw, out, RL, n, np_, L, NU, lo);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}
