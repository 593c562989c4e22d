// mfh_transform.hip -- bandwidth-side kernels of the gfx950 MFFT matmul:
// forward ring transform with digit split, inverse transform + fold, carry
// normalisation, fixed-point float encode/decode, plane transpose and seeded
// input generators.
//
// Ring R = Z[y]/(y^K + 1); omega = y^g is a primitive NB-th root of unity
// (g = 2K/NB).  A matrix element's L limbs form NB/2 non-zero blocks of S
// limbs (block b holds limbs b*S .. b*S+S-1 in ring coefficients 0..S-1,
// src/mfft.c:322-336); its transform is
//     X[j] = sum_b omega^(j*b) x_b,   j = 0 .. NB-1   (natural order).
// Multiplying by y^e is a negacyclic shift, so every output coefficient is
// a signed sum of input limbs: no multiplications anywhere.
#include <type_traits>
#include <utility>

#include "mfh_internal.hpp"
#include "mfh_decode.hpp"

namespace {

// ---- limb readers -----------------------------------------------------------
struct SrcU16 {
    const uint16_t *p;
    size_t nn;
    int n, L;
    __device__ int get(int u, int i, int k) const
    {
        return p[(size_t)u * nn + (size_t)i * n + k];
    }
};

// two's complement W-bit integers: the top limb is signed
struct SrcU16Signed {
    const uint16_t *p;
    size_t nn;
    int n, L;
    __device__ int get(int u, int i, int k) const
    {
        uint16_t v = p[(size_t)u * nn + (size_t)i * n + k];
        return u == L - 1 ? (int)(int16_t)v : (int)v;
    }
};

struct SrcI32 {
    const int32_t *p;
    size_t nn;
    int n, L;
    __device__ int get(int u, int i, int k) const
    {
        return p[(size_t)u * nn + (size_t)i * n + k];
    }
};

// fp32 on a fixed-point grid of scale 2^S (src/fpfixed.c:175-193): limb u
// of x * 2^S, as a signed limb.  frexp gives x = m 2^e, mi = |m| 2^24 is an
// exact 24-bit integer, and the value mi << (e - 24 + S) lands in limbs
// lo .. lo+2 with lo = (e-24+S) >> 4.
struct SrcF32 {
    static constexpr int NW = 3;   // limbs one entry can touch
    const float *p;
    size_t nn;
    int n, L, S;
    __device__ int get(int u, int i, int k) const
    {
        float x = p[(size_t)i * n + k];
        if (x == 0.0f || !isfinite(x)) return 0;
        int e;
        float m = frexpf(x, &e);
        int mi = (int)(fabsf(m) * 16777216.0f);
        int off = e - 24 + S;
        if (off < 0) return 0;
        int lo = off >> 4, t = u - lo;
        if (t < 0 || t > 2) return 0;
        unsigned long long v = (unsigned long long)mi << (off & 15);
        int limb = (int)((v >> (16 * t)) & 0xFFFFu);
        return x < 0.0f ? -limb : limb;
    }
    // the entry's limbs lo .. lo+2 (lo = L when it has none on the grid)
    __device__ void window(int i, int k, int &lo, int r[NW]) const
    {
        lo = L;
        for (int t = 0; t < NW; ++t) r[t] = 0;
        float x = p[(size_t)i * n + k];
        if (x == 0.0f || !isfinite(x)) return;
        int e;
        float m = frexpf(x, &e);
        int mi = (int)(fabsf(m) * 16777216.0f);
        int off = e - 24 + S;
        if (off < 0) return;
        lo = off >> 4;
        unsigned long long v = (unsigned long long)mi << (off & 15);
        for (int t = 0; t < NW; ++t) {
            int limb = (int)((v >> (16 * t)) & 0xFFFFu);
            r[t] = x < 0.0f ? -limb : limb;
        }
    }
};

// fp64 on the grid (src/fpfixed.c:144-162): mi = |m| 2^53 is an exact
// 53-bit integer; shifted by up to 15 it spans 68 bits, i.e. limbs
// lo .. lo+4.  The shift is done on a 128-bit pair (hi:lo words).
struct SrcF64 {
    static constexpr int NW = 5;
    const double *p;
    size_t nn;
    int n, L, S;
    __device__ void window(int i, int k, int &lo, int r[NW]) const
    {
        lo = L;
        for (int t = 0; t < NW; ++t) r[t] = 0;
        double x = p[(size_t)i * n + k];
        if (x == 0.0 || !isfinite(x)) return;
        int e;
        double m = frexp(x, &e);
        unsigned long long mi = (unsigned long long)(fabs(m) * 9007199254740992.0);
        int off = e - 53 + S;
        if (off < 0) return;
        lo = off >> 4;
        const int sh = off & 15;
        const unsigned long long w0 = mi << sh, w1 = sh ? mi >> (64 - sh) : 0ull;
        for (int t = 0; t < NW; ++t) {
            int limb = (int)((t < 4 ? w0 >> (16 * t) : w1) & 0xFFFFu);
            r[t] = x < 0.0 ? -limb : limb;
        }
    }
    __device__ int get(int u, int i, int k) const
    {
        int lo, r[NW];
        window(i, k, lo, r);
        int v = 0;
        for (int t = 0; t < NW; ++t) v = u == lo + t ? r[t] : v;
        return v;
    }
};


// C^ from the pointwise step's int32 class results (`cs` ints between
// classes): B8 sum_m class_m 2^(8m); K7 the Karatsuba recombination
// NT: stream the class values past the caches (each is read once)
template <bool NT = true>
__device__ __forceinline__ int ld_cls(const int32_t *p)
{
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}
template <bool NT = true>
__device__ __forceinline__ long long combine_classes(const int32_t *p, size_t cs, int mode)
{
    if (mode == MFH_MODE_K7) {
        const long long P0 = ld_cls<NT>(p), P1 = ld_cls<NT>(p + cs),
                        P2 = ld_cls<NT>(p + 2 * cs),
                        P3 = ld_cls<NT>(p + 3 * cs),
                        P4 = ld_cls<NT>(p + 4 * cs),
                        P5 = ld_cls<NT>(p + 5 * cs);
        const long long c1 = P3 - P0 - P1, c2 = P4 - P0 - P2 + P1, c3 = P5 - P1 - P2;
        return P0 + c1 * 128 + c2 * 16384 + c3 * 2097152 + P2 * 268435456;
    }
    long long v = 0;
#pragma unroll
    for (int m = MFH_CLASSES - 1; m >= 0; --m)
        v = v * 256 + (long long)ld_cls<NT>(p + m * cs);
    return v;
}

// The same from class values already in registers (MODE at compile time)
template <int MODE>
__device__ __forceinline__ long long combine_raw(const int *r)
{
    if constexpr (MODE == MFH_MODE_K7) {
        const long long P0 = r[0], P1 = r[1], P2 = r[2], P3 = r[3], P4 = r[4], P5 = r[5];
        const long long c1 = P3 - P0 - P1, c2 = P4 - P0 - P2 + P1, c3 = P5 - P1 - P2;
        return P0 + c1 * 128 + c2 * 16384 + c3 * 2097152 + P2 * 268435456;
    } else {
        long long v = 0;
#pragma unroll
        for (int m = MFH_CLASSES - 1; m >= 0; --m) v = v * 256 + (long long)r[m];
        return v;
    }
}

// Digit planes of one transformed value v (plane stride nnp):
//  B8: balanced base-2^8 digits, i.e. the low bytes of v, (v + 2^7) >> 8 and
//      (v + 2^15 + 2^7) >> 16 (each the floor that makes the lower digits
//      land in [-128, 127]).
//  K7: balanced base-2^7 digits d0, d1 in [-64, 63], d2 in [-64, 64] (for
//      |v| <= 1056703) and the sums d0+d1, d0+d2, d1+d2.
template <int MODE>
__device__ __forceinline__ void store_digits(int8_t *p, size_t nnp, int v)
{
    if constexpr (MODE == MFH_MODE_B8) {
        p[0] = (int8_t)v;
        p[nnp] = (int8_t)((v + 128) >> 8);
        p[2 * nnp] = (int8_t)((v + 32896) >> 16);
    } else {
        const int d0 = ((v + 64) & 127) - 64;
        const int v1 = (v + 64) >> 7;
        const int d1 = ((v1 + 64) & 127) - 64;
        const int d2 = (v1 + 64) >> 7;
        p[0] = (int8_t)d0;
        p[nnp] = (int8_t)d1;
        p[2 * nnp] = (int8_t)d2;
        p[3 * nnp] = (int8_t)(d0 + d1);
        p[4 * nnp] = (int8_t)(d0 + d2);
        p[5 * nnp] = (int8_t)(d1 + d2);
    }
}

// The digits store_digits writes, as values (plane order)
template <int MODE>
__device__ __forceinline__ void digit_vals(int v, int *d)
{
    if constexpr (MODE == MFH_MODE_B8) {
        d[0] = v;
        d[1] = (v + 128) >> 8;
        d[2] = (v + 32896) >> 16;
    } else {
        const int d0 = ((v + 64) & 127) - 64;
        const int v1 = (v + 64) >> 7;
        const int d1 = ((v1 + 64) & 127) - 64;
        const int d2 = (v1 + 64) >> 7;
        d[0] = d0;
        d[1] = d1;
        d[2] = d2;
        d[3] = d0 + d1;
        d[4] = d0 + d2;
        d[5] = d1 + d2;
    }
}

// Operand slot sl of a point whose K ring coefficients are z.  GS = 0: the
// coefficients themselves (K slots).  GS = 1 (operand A) / 2 (operand B):
// the 3H Gauss slots of MFH_PW_GAUSS (mfh_internal.hpp), H = K/2:
//   A: [z0 + z1 | z0 | z1],  B: [z0 | z1 - z0 | -(z0 + z1)]
// with z0 = z[0..H), z1 = z[H..K).
template <int GS, int K>
__device__ __forceinline__ int slot_val(const int *z, int sl)
{
    if constexpr (GS == 0) {
        return z[sl];
    } else {
        constexpr int H = K / 2;
        const int g = sl / H, c = sl % H;
        if constexpr (GS == 1) return g == 0 ? z[c] + z[c + H] : g == 1 ? z[c] : z[c + H];
        else return g == 0 ? z[c] : g == 1 ? z[c + H] - z[c] : -z[c] - z[c + H];
    }
}
// the same with the ring size and slot kind known at run time
__device__ __forceinline__ int slot_val_rt(const int *z, int sl, int K, int gs)
{
    if (gs == 0) return z[sl];
    const int H = K / 2, g = sl / H, c = sl % H;
    if (gs == 1) return g == 0 ? z[c] + z[c + H] : g == 1 ? z[c] : z[c + H];
    return g == 0 ? z[c] : g == 1 ? z[c + H] - z[c] : -z[c] - z[c + H];
}

// low bytes of a, b, c, d as one dword (a lowest)
__device__ __forceinline__ uint32_t pack4_lo(int a, int b, int c, int d)
{
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x04000c0cu);
    return lo | hi;
}

// 4 x 4 byte transpose: o[s] byte q = w[q] byte s
__device__ __forceinline__ void transpose4x4(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                             uint32_t *o)
{
    const uint32_t t0 = __builtin_amdgcn_perm(w1, w0, 0x05010400u);   // w0.0 w1.0 w0.1 w1.1
    const uint32_t t1 = __builtin_amdgcn_perm(w1, w0, 0x07030602u);   // w0.2 w1.2 w0.3 w1.3
    const uint32_t t2 = __builtin_amdgcn_perm(w3, w2, 0x05010400u);
    const uint32_t t3 = __builtin_amdgcn_perm(w3, w2, 0x07030602u);
    o[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
    o[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    o[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
    o[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

// Staged digit stores of the forward kernels with 256 elements per
// workgroup (which are 256 contiguous bytes of every digit plane).  A chunk
// is 48 consecutive planes (8 ring coefficients x 6 digits, or 16 x 3):
// every thread packs its element's 48 digit bytes into 12 dwords (group g =
// planes 4g .. 4g+3) and writes them to LDS; after a barrier, 192 threads
// each take one group and 16 consecutive elements, transpose the 16 x 4
// bytes in registers and write 16 bytes to each of the group's 4 planes.
// A wave store then covers 256 contiguous bytes of 4 planes (1 KB in 16-byte
// pieces) instead of 64 bytes of one plane, 16 times fewer store
// instructions.  LDS rows of 16 elements are padded to 20 dwords, so the 16
// readers of a group (80-byte stride) hit distinct banks.
// The same with NE = 64 elements staged by one wave in a private buffer
// (the 4096- and 8192-bit plans: 64 elements per workgroup, each wave
// computing a quarter of the output classes for all of them): 48 lanes
// store, no workgroup barrier.
constexpr int XCH_PLANES = 48, XCH_GROUPS = 12, XCH_ROW = 20;
constexpr int XCH_DWORDS = XCH_GROUPS * 16 * XCH_ROW;     // 256 elements: 15 KB

// t: this thread's element among the NE
template <int MODE, int NE>
__device__ __forceinline__ void xch_write(
    uint32_t *buf, const int (&z)[XCH_PLANES / (MODE == MFH_MODE_K7 ? 6 : 3)], int t)
{
    constexpr int PL = MODE == MFH_MODE_K7 ? 6 : 3;
    constexpr int CPC = XCH_PLANES / PL;
    constexpr int GSTRIDE = (NE / 16) * XCH_ROW;
    int d[XCH_PLANES];
#pragma unroll
    for (int c = 0; c < CPC; ++c) digit_vals<MODE>(z[c], d + c * PL);
    uint32_t *row = buf + (t >> 4) * XCH_ROW + (t & 15);
#pragma unroll
    for (int g = 0; g < XCH_GROUPS; ++g)
        row[g * GSTRIDE] = pack4_lo(d[4 * g], d[4 * g + 1], d[4 * g + 2], d[4 * g + 3]);
}

// o: the first byte of the NE elements in the chunk's first plane; only
// the first ngroups groups of 4 planes are stored (a point's last chunk may
// be partial)
template <int NE>
__device__ __forceinline__ void xch_store(const uint32_t *buf, int8_t *o, size_t nnp, int t,
                                          int ngroups = XCH_GROUPS)
{
    constexpr int EB = NE / 16, GSTRIDE = EB * XCH_ROW;
    if (t >= ngroups * EB) return;
    const int g = t / EB, eb = t % EB;
    const uint4 *src = (const uint4 *)(buf + g * GSTRIDE + eb * XCH_ROW);
    uint32_t w[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4 v = src[q];
        w[4 * q] = v.x;
        w[4 * q + 1] = v.y;
        w[4 * q + 2] = v.z;
        w[4 * q + 3] = v.w;
    }
    uint32_t p[4][4];          // p[s][q]: plane 4g+s, elements 4q .. 4q+3
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t o4[4];
        transpose4x4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3], o4);
#pragma unroll
        for (int s = 0; s < 4; ++s) p[s][q] = o4[s];
    }
    int8_t *dst = o + (size_t)(4 * g) * nnp + eb * 16;
#pragma unroll
    for (int s = 0; s < 4; ++s)
        *(uint4 *)(dst + (size_t)s * nnp) = make_uint4(p[s][0], p[s][1], p[s][2], p[s][3]);
}

// ---- forward transform, generic plan ---------------------------------------
// One thread per padded element (i, k) of a band of `rows` padded rows from
// row0 of an np x np operand; it writes the digit planes of every (point j,
// coefficient c).  Elements outside the n x n input are zero.  Output plane
// (j, c, r) holds digit r of X[j][c] as a rows x np int8 matrix in 16 x 64
// tiles (mfh_tile_off; the whole operand when row0 = 0, rows = np; the other
// forward kernels take the same band and layout).
// gs: operand slots as slot_val_rt (0: the K coefficients; 1, 2: the 3K/2
// Gauss slots of operand A, B).
template <class Src, int MODE>
__global__ __launch_bounds__(256) void k_forward_generic(
    Src src, int8_t *__restrict__ out, int np_, int LS, int S, int NB, int K,
    int g, int row0, int rows, int gs)
{
    const size_t nnp = (size_t)rows * np_;         // the band's elements (plane stride)
    const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= nnp) return;
    const int i = row0 + (int)(e / np_), k = (int)(e % np_);
    const bool valid = i < src.n && k < src.n;
    const size_t toff = mfh_tile_off(i - row0, k, np_);
    const int twoK = 2 * K, nsl = gs ? 3 * K / 2 : K;
    constexpr int PL = MODE == MFH_MODE_K7 ? 6 : 3;
    for (int j = 0; j < NB; ++j) {
        int z[32];
        for (int c = 0; c < K; ++c) {
            int acc = 0;
            if (valid) {
                for (int b = 0; b < LS; ++b) {
                    int ejb = (g * j * b) % twoK;
                    int s = c - ejb;
                    if (s < 0) s += twoK;
                    if (s < S) acc += src.get(b * S + s, i, k);
                    else if (s >= K && s < K + S) acc -= src.get(b * S + s - K, i, k);
                }
            }
            z[c] = acc;
        }
        for (int sl = 0; sl < nsl; ++sl)
            store_digits<MODE>(out + ((size_t)(j * nsl + sl) * PL) * nnp + toff, nnp,
                               slot_val_rt(z, sl, K, gs));
    }
}

// ---- forward transform of fixed-point floats, generic plan ---------------------
// An fp32/fp64 entry has at most NW non-zero limbs (a window lo .. lo+NW-1),
// so each output coefficient is a signed selection among NW values: limb
// u = b S + s lands, at point j, on ring position p = s + g j b (mod 2K),
// with a sign flip when p >= K.  Limbs at or above L are dropped, as the
// encoder drops them (src/fpfixed.c:155-156).
template <class Src, int MODE>
__global__ __launch_bounds__(256) void k_forward_window(Src src, int8_t *__restrict__ out,
                                                        int np_, int S, int NB, int K, int g,
                                                        int row0, int rows, int gs)
{
    constexpr int NW = Src::NW;
    const size_t nnp = (size_t)rows * np_;
    const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= nnp) return;
    const int i = row0 + (int)(e / np_), k = (int)(e % np_);
    const size_t toff = mfh_tile_off(i - row0, k, np_);
    int lo = src.L, r[NW];
    if (i < src.n && k < src.n) src.window(i, k, lo, r);
    int b[NW], s[NW];
#pragma unroll
    for (int t = 0; t < NW; ++t) {
        const int u = lo + t;
        if (u >= src.L) r[t] = 0;
        b[t] = u / S;
        s[t] = u % S;
    }
    const int twoK = 2 * K, nsl = gs ? 3 * K / 2 : K;
    constexpr int PL = MODE == MFH_MODE_K7 ? 6 : 3;
    for (int j = 0; j < NB; ++j) {
        int p[NW];
#pragma unroll
        for (int t = 0; t < NW; ++t) p[t] = (s[t] + (g * j * b[t]) % twoK) % twoK;
        int z[32];
        for (int c = 0; c < K; ++c) {
            int acc = 0;
#pragma unroll
            for (int t = 0; t < NW; ++t) acc += p[t] == c ? r[t] : p[t] == c + K ? -r[t] : 0;
            z[c] = acc;
        }
        for (int sl = 0; sl < nsl; ++sl)
            store_digits<MODE>(out + ((size_t)(j * nsl + sl) * PL) * nnp + toff, nnp,
                               slot_val_rt(z, sl, K, gs));
    }
}

// ---- forward transform, plan specialised at compile time ----------------------
// One thread per element; the element's L limbs are staged in LDS (u16
// pairs) for the workgroup's elements, or held in registers as int32 for
// fixed-point floats.  The NB output points are split into Q residue
// classes j = q + Q*j' (j' < P = NB/Q):
//     X[q + Q j'] = sum_{b' < P} w^(j' b') z_q[b'],   w = omega^Q,
//     z_q[b']     = sum_{b = b' mod P} omega^(q b) x_b
// (the twist omega^(q b) = y^(g q b) is a negacyclic shift, the fold adds
// the L/S non-zero blocks into P), and each class is a length-P radix-2
// DIF transform over K-vectors.  Every shift is a compile-time register
// renaming; only additions and negations remain.
template <int L>
struct LimbsI32 {
    int r[L];
    __device__ __forceinline__ int get(int u) const { return r[u]; }
};

// Packed limb pairs staged in LDS for the E elements of a workgroup: pair p
// of element slot t at lds[p * E + t] (consecutive threads read consecutive
// dwords: conflict-free).  Filled with 16-byte loads of 8 consecutive
// elements of planes 2p and 2p+1 (the input row length must be a multiple
// of 8, so such a run never straddles a row end).
template <int L, int E = 256>
struct LimbsLds {
    const uint32_t *base;      // lds + thread slot
    bool top_signed;
    bool recoded;              // pairs hold signed int16 limbs, top in `top`
    int top;
    __device__ __forceinline__ int get(int u) const
    {
        if (recoded && u == L - 1) return top;
        const uint32_t w = base[(u / 2) * E];
        if (recoded) return (u & 1) ? (int)(short)(w >> 16) : (int)(short)(w & 0xFFFFu);
        if (u == L - 1 && top_signed) return (int)(short)(w >> 16);
        return (u & 1) ? (int)(w >> 16) : (int)(w & 0xFFFFu);
    }
};

// e0: the first element in tile order (mfh_tile_ik); 8 consecutive
// elements in tile order are 8 consecutive columns of one row
template <int L, int E>
__device__ __forceinline__ void stage_limbs_u16(uint32_t *lds, const uint16_t *src, int n,
                                                size_t nn, int np_, size_t e0)
{
    constexpr int NP2 = L / 2, R8 = E / 8;      // 8-element runs per plane pair
    for (int t = threadIdx.x; t < NP2 * R8; t += 256) {
        const int p = t / R8, g8 = t % R8;
        const size_t e = e0 + 8 * g8;
        int i, k;
        mfh_tile_ik(e, np_, i, k);
        uint4 lo = {0, 0, 0, 0}, hi = {0, 0, 0, 0};
        if (i < n && k < n) {
            lo = *(const uint4 *)(src + (size_t)(2 * p) * nn + (size_t)i * n + k);
            hi = *(const uint4 *)(src + (size_t)(2 * p + 1) * nn + (size_t)i * n + k);
        }
        uint32_t w[8];
        const uint32_t l4[4] = {lo.x, lo.y, lo.z, lo.w}, h4[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            w[2 * d] = __builtin_amdgcn_perm(h4[d], l4[d], 0x05040100u);     // lo16(l)|lo16(h)<<16
            w[2 * d + 1] = __builtin_amdgcn_perm(h4[d], l4[d], 0x07060302u); // hi16(l)|hi16(h)<<16
        }
        uint4 *dst = (uint4 *)(lds + p * E + 8 * g8);
        dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
        dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    }
}

template <int L, class Src>
__device__ __forceinline__ void load_limbs(LimbsI32<L> &x, const Src &src, int i, int k,
                                           bool valid)
{
#pragma unroll
    for (int u = 0; u < L; ++u) x.r[u] = valid ? src.get(u, i, k) : 0;
}

// One output class q (compile time): twist + fold, length-P DIF, digits.
// XB = 0: each thread stores its element's digit bytes (o = its element in
// plane 0); XB = 1 or 2: staged stores through XB LDS buffers of
// XCH_DWORDS at xb (256 elements per workgroup, one thread each); XB = 3:
// staged per wave (64 elements per workgroup, wave w's buffer at
// xb + w * XCH_DWORDS / 4).
// GS: the operand slots written per point (slot_val: 0 the K coefficients,
// 1 / 2 the 3K/2 Gauss slots of operand A / B).
template <int S, int NB, int Q, int q, int MODE, class Limbs, int XB = 0, int GS = 0>
__device__ __forceinline__ void forward_class(const Limbs &x, int8_t *o, size_t nnp,
                                              uint32_t *xb = nullptr)
{
    constexpr int PL = MODE == MFH_MODE_K7 ? 6 : 3;
    constexpr int K = 2 * S, P = NB / Q, LS = NB / 2;
    constexpr int NSL = GS ? 3 * K / 2 : K;
    constexpr int g = 2 * K / NB, twoK = 2 * K;
    int z[P][K];
#pragma unroll
    for (int bp = 0; bp < P; ++bp)
#pragma unroll
        for (int c = 0; c < K; ++c) z[bp][c] = 0;
    // twist by omega^(q b) = y^(g q b) and fold the non-zero blocks
    // (ring coefficients c < S) of residue b mod P
#pragma unroll
    for (int b = 0; b < LS; ++b) {
#pragma unroll
        for (int c = 0; c < S; ++c) {
            const int pos = (c + (g * q * b) % twoK) % twoK;
            const int v = x.get(b * S + c);
            if (pos < K) z[b % P][pos] += v;
            else         z[b % P][pos - K] -= v;
        }
    }
    // length-P DIF with root w = y^(g Q): natural in, bit-reversed out;
    // butterfly u' = u + v, v' = (u - v) y^e
#pragma unroll
    for (int len = P; len >= 2; len >>= 1) {
#pragma unroll
        for (int j0 = 0; j0 < P; j0 += len) {
#pragma unroll
            for (int t = 0; t < len / 2; ++t) {
                const int ex = (g * Q * t * (P / len)) % twoK;
                int d[K];
#pragma unroll
                for (int c = 0; c < K; ++c) {
                    const int a = z[j0 + t][c], bb = z[j0 + t + len / 2][c];
                    z[j0 + t][c] = a + bb;
                    d[c] = a - bb;
                }
#pragma unroll
                for (int c = 0; c < K; ++c) {
                    const int pos = (c + ex) % twoK;
                    if (pos < K) z[j0 + t + len / 2][pos] = d[c];
                    else         z[j0 + t + len / 2][pos - K] = -d[c];
                }
            }
        }
    }
#pragma unroll
    for (int pos = 0; pos < P; ++pos) {
        int jp = 0;
#pragma unroll
        for (int bit = 1, rb = P >> 1; bit < P; bit <<= 1, rb >>= 1)
            if (pos & bit) jp |= rb;
        const int j = q + Q * jp;
        if constexpr (XB == 0) {
#pragma unroll
            for (int sl = 0; sl < NSL; ++sl)
                store_digits<MODE>(o + (size_t)((j * NSL + sl) * PL) * nnp, nnp,
                                   slot_val<GS, K>(z[pos], sl));
        } else if constexpr (XB == 3) {
            // the wave's own buffer: LDS operations of one wave complete in
            // order; the memory clobbers keep the compiler from moving the
            // other lanes' reads above the writes, or the next chunk's writes
            // above this chunk's reads
            constexpr int CPC = XCH_PLANES / PL;
            static_assert((NSL % CPC) * PL % 4 == 0, "whole groups of 4 planes per chunk");
            const int lane = threadIdx.x & 63;
            uint32_t *buf = xb + (threadIdx.x >> 6) * (XCH_DWORDS / 4);
            int8_t *wg = o - lane;
#pragma unroll
            for (int c0 = 0; c0 < NSL; c0 += CPC) {
                const int nv = NSL - c0 < CPC ? NSL - c0 : CPC;     // slots in this chunk
                int zc[CPC];
#pragma unroll
                for (int c = 0; c < CPC; ++c) zc[c] = c < nv ? slot_val<GS, K>(z[pos], c0 + c) : 0;
                asm volatile("" ::: "memory");
                xch_write<MODE, 64>(buf, zc, lane);
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                xch_store<64>(buf, wg + (size_t)((j * NSL + c0) * PL) * nnp, nnp, lane,
                              nv * PL / 4);
            }
        } else {
            // chunks of CPC coefficients; chunk k of the kernel uses buffer
            // k % XB.  One buffer: a barrier before each write (the previous
            // chunk's readers are done) and one before the reads.  Two: the
            // barrier before the reads of chunk k also orders every read of
            // chunk k-1 before the writes of chunk k+1 into its buffer.
            constexpr int CPC = XCH_PLANES / PL, NCH = (NSL + CPC - 1) / CPC;
            static_assert((NSL % CPC) * PL % 4 == 0, "whole groups of 4 planes per chunk");
            int8_t *wg = o - threadIdx.x;
#pragma unroll
            for (int c0 = 0; c0 < NSL; c0 += CPC) {
                const int k = (q * P + pos) * NCH + c0 / CPC;
                const int nv = NSL - c0 < CPC ? NSL - c0 : CPC;     // slots in this chunk
                uint32_t *buf = xb + (k % XB) * XCH_DWORDS;
                int zc[CPC];
#pragma unroll
                for (int c = 0; c < CPC; ++c) zc[c] = c < nv ? slot_val<GS, K>(z[pos], c0 + c) : 0;
                if (XB == 1 && k > 0) __syncthreads();
                xch_write<MODE, 256>(buf, zc, threadIdx.x);
                __syncthreads();
                xch_store<256>(buf, wg + (size_t)((j * NSL + c0) * PL) * nnp, nnp, threadIdx.x,
                               nv * PL / 4);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Threads of part p (p = thread / E, wave-uniform) produce the output
// classes q = p, p + TPE, ... of their element.
template <int S, int NB, int Q, int MODE, int TPE, int PART, class Limbs, int XB, int GS,
          int... is>
__device__ __forceinline__ void forward_part(const Limbs &x, int8_t *o, size_t nnp, uint32_t *xb,
                                             std::integer_sequence<int, is...>)
{
    // scheduling barriers between classes (and after each point's stores,
    // in forward_class): left free, the scheduler interleaves classes and
    // the S = 16 kernels need 256+ registers (140 with the barriers)
    ((forward_class<S, NB, Q, PART + TPE * is, MODE, Limbs, XB, GS>(x, o, nnp, xb),
      __builtin_amdgcn_sched_barrier(0)),
     ...);
}
template <int S, int NB, int Q, int MODE, int TPE, class Limbs, int XB, int GS, int PART = 0>
__device__ __forceinline__ void forward_parts(int part, const Limbs &x, int8_t *o, size_t nnp,
                                              uint32_t *xb)
{
    if constexpr (PART < TPE) {
        if (part == PART)
            forward_part<S, NB, Q, MODE, TPE, PART, Limbs, XB, GS>(
                x, o, nnp, xb, std::make_integer_sequence<int, Q / TPE>{});
        else
            forward_parts<S, NB, Q, MODE, TPE, Limbs, XB, GS, PART + 1>(part, x, o, nnp, xb);
    }
}

// E elements per workgroup of 256 threads, 256/E threads per element.
// Elements are enumerated in the digit planes' tile order (element e of the
// band is at offset e of every plane), so the 256 consecutive elements of a
// workgroup are 4 whole rows of one 16 x 64 tile: 256 contiguous bytes of
// each plane.
// top: limb L-1 is unsigned (0), int16 (1), or (int16)(x ^ 0x8000), i.e. the
// entry minus 2^(16L-1) (2, recoding only).
// XB > 0: staged digit stores through XB LDS buffers (E = 256 only; the
// band's element count must be a multiple of 256, so every thread of every
// workgroup has an element and reaches every barrier).
// At least two waves per SIMD: the W = 8192 kernels (81 KB of LDS, two
// workgroups per CU fit) otherwise take 256+ registers and run one wave per
// SIMD; capped at 256 they spill a few registers to scratch and write the
// 48 Gauss slots 1.29 -> 1.02 ms faster per product at n = 256 (no change
// for the 32 coefficient slots or the other plans, which fit already).
template <int S, int NB, int Q, int MODE, bool RECODE, class Limbs, class Src, int E = 256,
          int XB = 0, int GS = 0>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_forward_fast(
    Src src, int8_t *__restrict__ out, int np_,
                                                      int top_mode, int row0, int rows)
{
    constexpr int L = NB * S / 2;
    constexpr int TPE = 256 / E;
    static_assert(E * TPE == 256 && Q % TPE == 0, "threads split evenly over classes");
    static_assert(XB == 0 || (XB < 3 && E == 256) || (XB == 3 && (E == 64 || E == 256)),
                  "staged stores: 256 elements per workgroup, or 64 per wave");
    __shared__ uint32_t xbuf[XB == 3 ? XCH_DWORDS : XB > 0 ? XB * XCH_DWORDS : 1];
    const size_t nnp = (size_t)rows * np_;           // the band's elements (plane stride)
    const size_t eband = (size_t)row0 * np_;         // its first element in the operand
    const size_t e0 = (size_t)blockIdx.x * E;
    const int slot = threadIdx.x % E;
    const int part = __builtin_amdgcn_readfirstlane(threadIdx.x / E);
    const size_t e = e0 + slot;
    Limbs x;
    if constexpr (std::is_same_v<Limbs, LimbsLds<L, E>>) {
        __shared__ uint32_t stage[(L / 2) * E];
        stage_limbs_u16<L, E>(stage, src.p, src.n, src.nn, np_, eband + e0);
        __syncthreads();
        x.base = stage + slot;
        x.top_signed = top_mode != 0;
        x.recoded = RECODE;
        if constexpr (RECODE) {
            // Signed recoding y_u = x_u + c_u - 2^16 c_(u+1) with
            // c_(u+1) = [x_u + c_u >= 2^15]: the same integer, limbs below
            // the top in [-2^15, 2^15), the top limb (as `top` reads it) + c
            // unrecoded.  This halves the bound on the transformed values.
            // One thread per element rewrites the staged limbs; the others
            // of the element wait for it.
            __shared__ int top_s[TPE > 1 ? E : 1];
            if (part == 0) {
                uint32_t *sl = stage + slot;
                // padding outside the n x n entries stays 0 (not -2^(16L-1))
                int gi, gk;
                mfh_tile_ik(eband + e0 + slot, np_, gi, gk);
                const bool inside = gi < src.n && gk < src.n;
                int carry = 0;
#pragma unroll 8
                for (int p2 = 0; p2 < L / 2; ++p2) {
                    const uint32_t w = sl[p2 * E];
                    int lo = (int)(w & 0xFFFFu) + carry;
                    carry = lo >= 32768;
                    lo -= carry << 16;
                    int hi = (int)(w >> 16) + carry;
                    if (p2 + 1 < L / 2) {
                        carry = hi >= 32768;
                        hi -= carry << 16;
                    } else {
                        const uint32_t t = w >> 16;
                        x.top = top_mode == 1   ? (int)(short)t + carry
                                : top_mode == 2 ? (inside ? (int)(short)(t ^ 0x8000u) + carry : 0)
                                                : hi;
                        hi = 0;
                    }
                    sl[p2 * E] = ((uint32_t)lo & 0xFFFFu) | ((uint32_t)hi << 16);
                }
                if constexpr (TPE > 1) top_s[slot] = x.top;
            }
            if constexpr (TPE > 1) {
                __syncthreads();
                x.top = top_s[slot];
            }
        }
        if (XB == 0 && e >= nnp) return;
    } else {
        if (XB == 0 && e >= nnp) return;
        int i, k;
        mfh_tile_ik(e, np_, i, k);
        i += row0;
        const bool valid = i < src.n && k < src.n;
        load_limbs<L>(x, src, i, k, valid);
    }
    forward_parts<S, NB, Q, MODE, TPE, Limbs, XB, GS>(part, x, out + e, nnp, xbuf);
}

// |limb| <= 65535 for int32 inputs (the transform and digit bounds assume it)
__global__ __launch_bounds__(256) void k_check_i32(const int32_t *p, size_t count,
                                                   int *flag)
{
    size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    size_t stride = (size_t)gridDim.x * 256;
    bool bad = false;
    for (; idx < count; idx += stride) {
        int v = p[idx];
        bad |= (v > 65535) || (v < -65535);
    }
    if (bad) atomicOr(flag, 1);
}

// ---- inverse transform + /NB + fold -----------------------------------------
// One workgroup holds `epw` elements, each with NB*K int64 values, twice
// (ping-pong) in LDS; thread (le, c) owns ring coefficient c of element le.
// Input C^[j][i][j'][c] in natural point order is loaded bit-reversed, then
// Cooley-Tukey stages len = 2..NB with conjugate twiddles give NB * x_b in
// natural order (the semantics of src/mfft.c:260-299).  Fold:
//     Cw[b*S + c] = x_b[c] + x_(b-1)[c + S],  c < S   (src/mfft.c:407-418)
// The elements are those of rows r0.. of a row band ([eb0, eb1) of the n x n
// matrix); the class results hold the band's `rows` padded rows.
__global__ void k_inverse_fold(const int32_t *__restrict__ C5,
                               int64_t *__restrict__ Cw, int n, int np_,
                               int NB, int K, int S, int g, int lgNB, int P,
                               int epw, int mode, int ncl, size_t eb0, size_t eb1, int r0,
                               int rows)
{
    extern __shared__ int64_t sm[];
    const int tid = threadIdx.x;
    const int le = tid / K, c = tid % K;
    const size_t nn = (size_t)n * n;
    const size_t e = eb0 + (size_t)blockIdx.x * epw + le;
    const bool valid = le < epw && e < eb1;
    const int blk = NB * K;
    int64_t *X = sm + (size_t)le * blk;
    int64_t *Y = sm + (size_t)epw * blk + (size_t)le * blk;
    const int i = valid ? (int)(e / n) - r0 : 0, jj = valid ? (int)(e % n) : 0;
    if (valid) {
        for (int j = 0; j < NB; ++j) {
            const int r = lgNB ? (int)(__brev((unsigned)j) >> (32 - lgNB)) : 0;
            X[r * K + c] = combine_classes(C5 + mfh_c5_index(j, i, jj, c, np_, ncl, K, rows),
                                           mfh_c5_class_stride(np_, K), mode);
        }
    }
    __syncthreads();
    const int twoK = 2 * K;
    for (int len = 2; len <= NB; len <<= 1) {
        const int h = len >> 1, step = NB / len;
        if (valid) {
            for (int j0 = 0; j0 < NB; j0 += len)
                for (int t = 0; t < h; ++t) {
                    const int p = j0 + t, q = p + h;
                    const int ex = (g * t * step) % twoK;
                    int s = c + ex;                   // (y^-ex v)[c] = v[c+ex]
                    if (s >= twoK) s -= twoK;
                    int64_t w = s < K ? X[q * K + s] : -X[q * K + s - K];
                    int64_t u = X[p * K + c];
                    Y[p * K + c] = u + w;
                    Y[q * K + c] = u - w;
                }
        }
        __syncthreads();
        int64_t *tmp = X; X = Y; Y = tmp;
    }
    if (valid && c < S) {
        for (int b = 0; b < NB; ++b) {
            const int w = b * S + c;
            if (w >= P) break;
            int64_t v = X[b * K + c] >> lgNB;            // exact multiples of NB
            if (b > 0) v += X[(b - 1) * K + c + S] >> lgNB;
            Cw[(size_t)w * nn + e] = v;
        }
    }
}

// ---- inverse transform + /NB + fold, plan specialised ------------------------
// K lanes per element (lane c = ring coefficient c); each lane holds the NB
// values C^[j][c] of its element in registers, loaded in bit-reversed point
// order, and runs the Cooley-Tukey stages (conjugate twiddles) fully
// unrolled.  Multiplying the ring element in lanes c = 0..K-1 by y^-e is a
// lane rotation (ds_bpermute) plus a sign per lane:
//     (y^-e v)[c] = +-v[(c + e) mod K],  minus iff floor((c + e)/K) is odd.
// Fold: Cw[b*S + c] = x_b[c]/NB + x_(b-1)[c+S]/NB for the lanes c < S (the
// second term is one more rotation).  Cw goes through LDS so that each plane
// is written as one contiguous run of the workgroup's elements.
__device__ __forceinline__ long long bperm64(long long v, int addr)
{
    const int lo = __builtin_amdgcn_ds_bpermute(addr, (int)(unsigned long long)v);
    const int hi = __builtin_amdgcn_ds_bpermute(addr, (int)((unsigned long long)v >> 32));
    return (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}

//
// CARRY: instead of writing Cw, one thread per element (all in the first
// wave, E <= 64) propagates the carries through the element's 2L-1 planes
// straight from LDS and writes the RL uint16 output limbs (the semantics of
// k_carry), saving the int64 round trip through HBM.
//
// Offset mode (rowS != nullptr, CARRY only): the operands were A - hJ and
// B - hJ with h = 2^(16L-1) and J all ones, so
//     A B = (A-hJ)(B-hJ) + h (r_i + s_j) + h^2 n,
// r_i / s_j the sums of row i of A-hJ / column j of B-hJ.  With
// r_i = sum_u rowS[u][i] 2^(16u) (likewise s_j), h r_i adds
// rowS[u][i] 2^15 to plane L-1+u, and h^2 n adds n 2^14 to plane 2L-1.
// NT: class loads past the caches.  Plain loads measured faster only for
// the fused W = 2048 plan (NB = 32, K = 16: 3.07 -> 2.90 ms); elsewhere
// (fused NB = 16 K = 8 and NB = 64 K = 32, and without the fused carry)
// non-temporal loads were 3-4 % faster.
// DEC >= 0 (CARRY false): instead of writing Cw, one thread per element
// decodes the element's planes from LDS into fp32 / fp64 (MFH_DEC_*) at
// dec_out with scale 2^-SAB (the semantics of k_decode).
// PF: the K7 classes of the next point are loaded while the current one is
// combined (the W = 8192 fused plan: 1.55 -> 1.47 ms at n = 256; equal at
// W = 2048 and 512).
template <int NB, int K, bool CARRY, int NPASS = 2,
          bool NT = !(CARRY && NB == 32 && K == 16), int DEC = -1,
          bool PF = CARRY && NB == 64 && K == 32>
__global__ __launch_bounds__(256) void k_inverse_fast(const int32_t *__restrict__ C5,
                                                      int64_t *__restrict__ Cw,
                                                      uint16_t *__restrict__ out, int RL,
                                                      int n, int np_, int P, int mode, int ncl,
                                                      size_t eb0, size_t eb1, int r0, int rows,
                                                      const int64_t *__restrict__ rowS,
                                                      const int64_t *__restrict__ colS,
                                                      void *__restrict__ dec_out, int SAB)
{
    static_assert(DEC < 0 || !CARRY, "decode replaces the Cw output");
    constexpr int S = K / 2, g = 2 * K / NB, twoK = 2 * K;
    constexpr int PASS = 256 / K;            // elements per pass
    constexpr int E = NPASS * PASS;          // elements per workgroup
    constexpr int LG = __builtin_ctz(NB);
    extern __shared__ int64_t cwl[];         // [P][E]
    const int tid = threadIdx.x, lane = tid & 63;
    const int c = lane % K;
    const int gbase = (lane / K) * K;        // first lane of this element's group
    const size_t nn = (size_t)n * n;
    const size_t e0 = eb0 + (size_t)blockIdx.x * E;      // elements [eb0, eb1): a row band
#pragma unroll
    for (int pass = 0; pass < NPASS; ++pass) {
        const int el = pass * PASS + tid / K;
        const size_t e = e0 + el;
        const bool valid = e < eb1;
        const int i = valid ? (int)(e / n) - r0 : 0, jj = valid ? (int)(e % n) : 0;
        long long X[NB];
        if (PF && mode == MFH_MODE_K7) {
            // K7 classes of point j + 1 loaded while point j is combined
            // (an element outside the band reads element 0's and discards
            // them); the scheduling barriers keep the loads one point ahead
            const size_t cs = mfh_c5_class_stride(np_, K);
            const int32_t *p0 = C5 + mfh_c5_index(0, valid ? i : 0, valid ? jj : 0, c, np_, 6, K,
                                                  rows);
            const size_t js = mfh_c5_index(1, 0, 0, 0, np_, 6, K, rows);
            int cur[6], nx[6];
#pragma unroll
            for (int m = 0; m < 6; ++m) cur[m] = ld_cls<NT>(p0 + m * cs);
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                if (j + 1 < NB) {
#pragma unroll
                    for (int m = 0; m < 6; ++m) nx[m] = ld_cls<NT>(p0 + (j + 1) * js + m * cs);
                }
                int r = 0;
#pragma unroll
                for (int bit = 1, rb = NB >> 1; bit < NB; bit <<= 1, rb >>= 1)
                    if (j & bit) r |= rb;
                const long long v = combine_raw<MFH_MODE_K7>(cur);
                X[r] = valid ? v : 0;
#pragma unroll
                for (int m = 0; m < 6; ++m) cur[m] = nx[m];
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            int r = 0;
#pragma unroll
            for (int bit = 1, rb = NB >> 1; bit < NB; bit <<= 1, rb >>= 1)
                if (j & bit) r |= rb;
            X[r] = valid ? combine_classes<NT>(C5 + mfh_c5_index(j, i, jj, c, np_, ncl, K, rows),
                                           mfh_c5_class_stride(np_, K), mode)
                         : 0;
        }
        }
#pragma unroll
        for (int len = 2; len <= NB; len <<= 1) {
#pragma unroll
            for (int j0 = 0; j0 < NB; j0 += len) {
#pragma unroll
                for (int t = 0; t < len / 2; ++t) {
                    const int ex = (g * t * (NB / len)) % twoK;
                    const int p = j0 + t, q = p + len / 2;
                    long long w = X[q];
                    if (ex != 0) {
                        const int raw = c + ex;                   // < 3K
                        w = bperm64(w, (gbase + raw % K) * 4);
                        if ((raw / K) & 1) w = -w;
                    }
                    const long long u = X[p];
                    X[p] = u + w;
                    X[q] = u - w;
                }
            }
        }
        // fold and /NB (every value is an exact multiple of NB)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            long long hiw = 0;
            if (b > 0) hiw = bperm64(X[b - 1], (gbase + (c + S) % K) * 4) >> LG;
            const int w = b * S + c;
            if (c < S && w < P) cwl[(size_t)w * E + el] = (X[b] >> LG) + hiw;
        }
    }
    __syncthreads();
    const int ecount = (int)((eb1 - e0) < (size_t)E ? (eb1 - e0) : (size_t)E);
    if constexpr (CARRY) {
        // Carry over the RL output limbs by SEGS = 256/E threads per element,
        // each owning a run of `len` >= 4 consecutive limbs (carry lookahead):
        //  1. each run propagates its own planes with carry-in 0, giving its
        //     limbs (value Ls < 2^(16 len)) and carry-out c; with a true
        //     carry-in X (|X| < 2^47 < 2^(16 len)) the carry-out becomes
        //     c + floor((Ls + X) / 2^(16 len)), i.e. c + 1 when X >= 2^(16 len)
        //     - Ls, c - 1 when X < -Ls, else c: two thresholds per run, each
        //     representable only when Ls is within 2^63 of 0 or 2^(16 len);
        //  2. one lane per element chains the SEGS runs through them;
        //  3. each run propagates again from its true carry-in and writes.
        // Only the last run can be shorter than `len`; its carry-out is the
        // one discarded (limbs >= RL), so the thresholds never apply to it.
        constexpr int SEGS = 256 / E;
        int64_t *segc = cwl + (size_t)P * E;           // [SEGS][E] each
        int64_t *seglo = segc + SEGS * E, *seghi = seglo + SEGS * E, *segin = seghi + SEGS * E;
        const int el = tid % E, sg = tid / E;
        int len = (RL + SEGS - 1) / SEGS;
        if (len < 4) len = 4;
        const int w0 = sg * len, w1 = min(w0 + len, RL);
        // plane w of this element, with the offset-mode terms
        const int Lh = (P + 1) / 2;                    // L
        const size_t eg = e0 + el < eb1 ? e0 + el : eb0;
        const int gi = (int)(eg / n), gj = (int)(eg % n);
        auto plane = [&](int w) -> int64_t {
            int64_t v = w < P ? cwl[(size_t)w * E + el] : 0;
            if (rowS) {
                const int u = w - (Lh - 1);
                if (u >= 0 && u < Lh)
                    v += (rowS[(size_t)u * n + gi] + colS[(size_t)u * n + gj]) * 32768;
                if (w == 2 * Lh - 1) v += (int64_t)n * 16384;
            }
            return v;
        };
        {
            int64_t cc = 0;
            uint64_t low = 0;                          // limbs 0..3 of the run
            bool zero_hi = true, ones_hi = true;       // limbs 4.. all 0 / all 0xFFFF
            for (int w = w0; w < w1; ++w) {
                const int64_t v = cc + plane(w);
                const uint64_t limb = (uint64_t)(v & 0xFFFF);
                const int i = w - w0;
                if (i < 4) low |= limb << (16 * i);
                else {
                    zero_hi &= limb == 0;
                    ones_hi &= limb == 0xFFFF;
                }
                cc = v >> 16;
            }
            const bool top_clear = (low >> 63) == 0;
            seglo[sg * E + el] = (zero_hi && top_clear) ? -(int64_t)low : INT64_MIN;
            seghi[sg * E + el] = (ones_hi && !top_clear && low != (1ull << 63))
                                     ? (int64_t)(0 - low) : INT64_MAX;
            segc[sg * E + el] = cc;
        }
        __syncthreads();
        if (tid < E) {
            int64_t C = 0;
            for (int r = 0; r < SEGS; ++r) {
                segin[r * E + tid] = C;
                C = segc[r * E + tid] + (C >= seghi[r * E + tid]) - (C < seglo[r * E + tid]);
            }
        }
        __syncthreads();
        if (el < ecount) {
            int64_t cc = segin[sg * E + el];
            for (int w = w0; w < w1; ++w) {
                const int64_t v = cc + plane(w);
                __builtin_nontemporal_store((uint16_t)(v & 0xFFFF), out + (size_t)w * nn + e0 + el);
                cc = v >> 16;
            }
        }
    } else if constexpr (DEC >= 0) {
        if (tid < ecount)
            decode_value<DEC>([&](int w) { return cwl[(size_t)w * E + tid]; }, P, P + 3, SAB,
                              dec_out, nullptr, e0 + tid);
    } else {
        for (int idx = tid; idx < P * E; idx += 256) {
            const int w = idx / E, el = idx % E;
            if (el < ecount) Cw[(size_t)w * nn + e0 + el] = cwl[idx];
        }
    }
}

// ---- carry normalisation (src/bigmat.c:48-60) ------------------------------
__global__ __launch_bounds__(256) void k_carry(const int64_t *__restrict__ Cw,
                                               uint16_t *__restrict__ out,
                                               size_t nn, int P, int RL)
{
    const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= nn) return;
    int64_t carry = 0;
    for (int w = 0; w < RL; ++w) {
        int64_t v = carry + (w < P ? Cw[(size_t)w * nn + e] : 0);
        out[(size_t)w * nn + e] = (uint16_t)(v & 0xFFFF);
        carry = v >> 16;
    }
}

// ---- offset-mode limb sums ----------------------------------------------------
// out[u][r] = sum_k limb_u(r, k) over row r of plane u (n x n, row-major),
// the top limb (u = L-1) as x - 2^15.  One wave per (u, r); |sum| <= n 2^16.
__global__ __launch_bounds__(256) void k_offset_sums(const uint16_t *__restrict__ src,
                                                     int64_t *__restrict__ out, int n, int L)
{
    const int lane = threadIdx.x & 63;
    const size_t row = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);   // u * n + r
    if (row >= (size_t)L * n) return;
    const bool top = (int)(row / n) == L - 1;
    const uint16_t *p = src + row * n;
    long long acc = 0;
    for (int k = lane; k < n; k += 64) acc += top ? (int)p[k] - 32768 : (int)p[k];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
    if (lane == 0) out[row] = acc;
}


template <int FMT>
__global__ __launch_bounds__(256) void k_decode(const int64_t *__restrict__ Cw,
                                                void *__restrict__ out_,
                                                int32_t *__restrict__ out2,
                                                size_t nn, int P, int RL, int SAB)
{
    const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= nn) return;
    decode_value<FMT>([&](int w) { return Cw[(size_t)w * nn + e]; }, P, RL, SAB, out_, out2, e);
}

// ---- fp32 / fp64 encode into limb planes (src/fpfixed.c:144-204) ------------
// every one of the L planes is written (zero outside the entry's window)
template <class Src>
__global__ __launch_bounds__(256) void k_encode(Src src, int32_t *__restrict__ out)
{
    constexpr int NW = Src::NW;
    const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= src.nn) return;
    const int i = (int)(e / src.n), k = (int)(e % src.n);
    int lo, r[NW];
    src.window(i, k, lo, r);
    for (int u = 0; u < src.L; ++u) {
        int v = 0;
#pragma unroll
        for (int t = 0; t < NW; ++t) v = u == lo + t ? r[t] : v;
        out[(size_t)u * src.nn + e] = v;
    }
}

// fp32 / fp64 entries -> the two's complement uint16 limbs of the value
// k_encode puts on the grid (its limbs below src.L, i.e. x 2^S truncated to
// the grid) over src.L + 1 limbs: |value| < 2^(16 L), so the top limb holds
// the sign.  This is the multi-modular product's input form.
template <class Src>
__global__ __launch_bounds__(256) void k_encode_tc(Src src, uint16_t *__restrict__ out)
{
    const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= src.nn) return;
    const int i = (int)(e / src.n), k = (int)(e % src.n);
    int lo, r[Src::NW];
    src.window(i, k, lo, r);
    int carry = 0;
    for (int u = 0; u <= src.L; ++u) {
        int v = carry;
        if (u < src.L) {
#pragma unroll
            for (int t = 0; t < Src::NW; ++t) v += u == lo + t ? r[t] : 0;
        }
        out[(size_t)u * src.nn + e] = (uint16_t)(v & 0xFFFF);
        carry = v >> 16;
    }
}

// The fixed-point decode from RLr carried two's complement limbs
// (decode_carried: the same sign, window and rounding as the
// coefficient-plane decode of the same value, found from the top limb down)
template <int FMT>
__global__ __launch_bounds__(256) void k_decode_limbs(const uint16_t *__restrict__ limbs,
                                                      size_t nn, int RLr, int SAB,
                                                      void *__restrict__ out, int32_t *out2)
{
    const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= nn) return;
    decode_carried<FMT>([&](int w) -> uint32_t { return limbs[(size_t)w * nn + e]; }, RLr, SAB,
                        out, out2, e);
}

// ---- plane transpose (B operand) -----------------------------------------------
// uint16 planes with n a multiple of 64 (whole 64 x 64 tiles): 16-byte
// loads of 8 consecutive elements of a row, 16-byte stores of 8 consecutive
// elements of a column gathered from LDS (rows padded to 66 elements: the 8
// rows a lane gathers fall in distinct banks)
__global__ __launch_bounds__(256) void k_transpose_u16x8(const uint4 *__restrict__ src,
                                                        uint4 *__restrict__ dst, int n)
{
    __shared__ uint16_t tile[64][66];
    const size_t nn = (size_t)n * n;
    const uint16_t *s = (const uint16_t *)src + (size_t)blockIdx.z * nn;
    uint16_t *d = (uint16_t *)dst + (size_t)blockIdx.z * nn;
    const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int q = threadIdx.x + 256 * k;           // 512 chunks of 8
        const int r = q >> 3, c8 = (q & 7) * 8;
        const uint4 v = *(const uint4 *)(s + (size_t)(r0 + r) * n + c0 + c8);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            tile[r][c8 + 2 * e] = (uint16_t)(w[e] & 0xFFFFu);
            tile[r][c8 + 2 * e + 1] = (uint16_t)(w[e] >> 16);
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int q = threadIdx.x + 256 * k;
        const int c = q >> 3, r8 = (q & 7) * 8;       // dst row c0 + c, cols r0 + r8 ..
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w[e] = (uint32_t)tile[r8 + 2 * e][c] | ((uint32_t)tile[r8 + 2 * e + 1][c] << 16);
        *(uint4 *)(d + (size_t)(c0 + c) * n + r0 + r8) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

template <class T>
__global__ __launch_bounds__(256) void k_transpose(const T *__restrict__ src,
                                                   T *__restrict__ dst, int n)
{
    __shared__ T tile[64][65];
    const size_t nn = (size_t)n * n;
    const T *s = src + (size_t)blockIdx.z * nn;
    T *d = dst + (size_t)blockIdx.z * nn;
    const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
    const int tx = threadIdx.x % 64, ty = threadIdx.x / 64;
    for (int r = ty; r < 64; r += 4) {
        int rr = r0 + r, cc = c0 + tx;
        if (rr < n && cc < n) tile[r][tx] = s[(size_t)rr * n + cc];
    }
    __syncthreads();
    for (int r = ty; r < 64; r += 4) {
        int rr = c0 + r, cc = r0 + tx;     // dst row = src col
        if (rr < n && cc < n) d[(size_t)rr * n + cc] = tile[tx][r];
    }
}

// ---- seeded generators (splitmix64: output i is mix(seed + (i+1) gamma)) ----
__device__ __forceinline__ uint64_t sm64_mix(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void k_rand_u16(uint16_t *dst, size_t count,
                                                  uint64_t seed)
{
    size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    size_t stride = (size_t)gridDim.x * 256;
    for (; idx < count; idx += stride)
        dst[idx] = (uint16_t)sm64_mix(seed + (uint64_t)(idx + 1) * 0x9E3779B97F4A7C15ULL);
}

__global__ __launch_bounds__(256) void k_rand_f32(float *dst, size_t count,
                                                  uint64_t seed, int emin,
                                                  unsigned span)
{
    size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    size_t stride = (size_t)gridDim.x * 256;
    for (; idx < count; idx += stride) {
        uint64_t u = sm64_mix(seed + (uint64_t)(idx + 1) * 0x9E3779B97F4A7C15ULL);
        float m = 1.0f + (float)((u >> 40) & 0x7FFFFFu) * (1.0f / 8388608.0f);
        int e = emin + (int)(u % span);
        float x = ldexpf(m, e);
        dst[idx] = (u >> 63) ? -x : x;
    }
}

// plain 16-byte-vector copy: reads and writes each byte once, the yardstick
// that HBM byte counters are calibrated against
__global__ __launch_bounds__(256) void k_copy16(const uint4 *__restrict__ src,
                                                uint4 *__restrict__ dst, size_t count)
{
    size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    size_t stride = (size_t)gridDim.x * 256;
    for (; idx < count; idx += stride) dst[idx] = src[idx];
}

int lg2i(int x) { int r = 0; while ((1 << r) < x) ++r; return r; }

unsigned grid_for(size_t count, unsigned cap)
{
    size_t g = (count + 255) / 256;
    if (g > cap) g = cap;
    return g ? (unsigned)g : 1u;
}

}  // namespace

// ============================================================================
int mfh_launch_transpose(const void *src, void *dst, int planes, int n,
                         int elem_bytes, hipStream_t st)
{
    dim3 grid((n + 63) / 64, (n + 63) / 64, planes);
    if (elem_bytes == 2 && n % 64 == 0 && (uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0)
        hipLaunchKernelGGL(k_transpose_u16x8, grid, dim3(256), 0, st, (const uint4 *)src,
                           (uint4 *)dst, n);
    else if (elem_bytes == 2)
        hipLaunchKernelGGL(k_transpose<uint16_t>, grid, dim3(256), 0, st,
                           (const uint16_t *)src, (uint16_t *)dst, n);
    else if (elem_bytes == 4)
        hipLaunchKernelGGL(k_transpose<uint32_t>, grid, dim3(256), 0, st,
                           (const uint32_t *)src, (uint32_t *)dst, n);
    else if (elem_bytes == 8)
        hipLaunchKernelGGL(k_transpose<uint64_t>, grid, dim3(256), 0, st,
                           (const uint64_t *)src, (uint64_t *)dst, n);
    else
        return MFH_E_ARG;
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

namespace {
// compile-time plans: (S, NB) with Q output classes of length NB/Q
template <int S, int NB, int MODE, bool RECODE, class Src, class Limbs, int E = 256,
          int Q = NB / 4, int XB = 0, int GS = 0>
bool try_fast1(mfh_ctx *c, const Src &s, int8_t *dst, int top_mode, int row0, int rows)
{
    if (c->S != S || c->NB != NB || c->mode != MODE || (c->recode != 0) != RECODE) return false;
    if (top_mode == 2 && !RECODE) return false;
    const size_t nnp = (size_t)rows * c->np;
    if (XB > 0 && nnp % E) return false;     // staged stores need whole workgroups
    hipLaunchKernelGGL((k_forward_fast<S, NB, Q, MODE, RECODE, Limbs, Src, E, XB, GS>),
                       dim3((unsigned)((nnp + E - 1) / E)), dim3(256), 0, c->stream, s, dst,
                       c->np, top_mode, row0, rows);
    return true;
}
// gs: operand slots (slot_val); Gauss slots are compiled for the rings with
// a Gauss pointwise kernel, in the 6-product digit mode only
template <int S, int NB, int MODE, bool RECODE, class Src, class Limbs, int E = 256,
          int Q = NB / 4, int XB = 0>
bool try_fast(mfh_ctx *c, const Src &s, int8_t *dst, int top_mode, int row0, int rows, int gs)
{
    if (gs == 0)
        return try_fast1<S, NB, MODE, RECODE, Src, Limbs, E, Q, XB, 0>(c, s, dst, top_mode,
                                                                         row0, rows);
    if constexpr (MODE == MFH_MODE_K7 && (2 * S == 8 || 2 * S == 16 || 2 * S == 32)) {
        if (gs == 1)
            return try_fast1<S, NB, MODE, RECODE, Src, Limbs, E, Q, XB, 1>(c, s, dst, top_mode,
                                                                             row0, rows);
        return try_fast1<S, NB, MODE, RECODE, Src, Limbs, E, Q, XB, 2>(c, s, dst, top_mode,
                                                                         row0, rows);
    }
    return false;
}

// Plans with 256 elements per workgroup store their digits through LDS
// (XB = 1): forward 2.04 -> 1.77 ms at W = 2048 (both operands and the B
// transpose), 9.7 -> 6.2 ms at W = 512 and n = 4096, 1.71 -> 1.1 ms for
// fp32 at n = 2048; two buffers (one barrier per chunk) measured equal or
// slower.  Staging per wave with no workgroup barrier (XB = 3, 64-byte
// runs per plane) pays only at W = 1024 (0.081 -> 0.071 ms at n = 64;
// 2.53 -> 2.57 ms at W = 2048, n = 1024; 5.9 -> 7.9 ms at W = 512,
// n = 4096).
bool forward_fast_u16(mfh_ctx *c, const SrcU16 &s, int8_t *dst, int ts, int r0, int rows,
                      int gs)
{
    constexpr int K7 = MFH_MODE_K7, B8 = MFH_MODE_B8;
    if (c->n % 8) return false;   // staged 16-byte loads need rows of 8k limbs
    // W=2048: 4 output classes of 8 points (half the staged-limb reads of 8
    // classes of 4; 214 VGPRs, within the two waves per SIMD the LDS allows):
    // forward stage 2-3 % faster; 16 classes of 2 were 5 % slower
    return try_fast<8, 32, K7, true, SrcU16, LimbsLds<128>, 256, 4, 1>(c, s, dst, ts, r0,
                                                                       rows, gs) ||  // W=2048
           try_fast<8, 32, B8, false, SrcU16, LimbsLds<128>, 256, 8, 1>(c, s, dst, ts, r0, rows,
                                                                       gs) ||
           try_fast<8, 16, K7, false, SrcU16, LimbsLds<64>, 256, 4, 3>(c, s, dst, ts, r0,
                                                                       rows, gs) ||  // W=1024
           try_fast<16, 64, K7, true, SrcU16, LimbsLds<512, 64>, 64, 32, 3>(c, s, dst, ts, r0,
                                                                           rows, gs) ||  // W=8192
           try_fast<16, 64, B8, false, SrcU16, LimbsLds<512, 64>, 64, 32, 3>(c, s, dst, ts, r0,
                                                                            rows, gs) ||
           try_fast<4, 16, K7, false, SrcU16, LimbsLds<32>, 256, 4, 1>(c, s, dst, ts, r0,
                                                                       rows, gs) ||  // W=512
           try_fast<16, 32, K7, false, SrcU16, LimbsLds<256, 64>, 64, 16, 3>(c, s, dst, ts, r0,
                                                                            rows, gs);  // W=4096
}
}  // namespace

template <class Src>
void launch_generic(mfh_ctx *c, const Src &s, int8_t *dst, dim3 grid, int LS, int r0, int rows,
                    int gs)
{
    if (c->mode == MFH_MODE_K7)
        hipLaunchKernelGGL((k_forward_generic<Src, MFH_MODE_K7>), grid, dim3(256), 0, c->stream,
                           s, dst, c->np, LS, c->S, c->NB, c->K, c->g, r0, rows, gs);
    else
        hipLaunchKernelGGL((k_forward_generic<Src, MFH_MODE_B8>), grid, dim3(256), 0, c->stream,
                           s, dst, c->np, LS, c->S, c->NB, c->K, c->g, r0, rows, gs);
}

template <class Src>
void launch_window(mfh_ctx *c, const Src &s, int8_t *dst, dim3 grid, int r0, int rows, int gs)
{
    if (c->mode == MFH_MODE_K7)
        hipLaunchKernelGGL((k_forward_window<Src, MFH_MODE_K7>), grid, dim3(256), 0, c->stream,
                           s, dst, c->np, c->S, c->NB, c->K, c->g, r0, rows, gs);
    else
        hipLaunchKernelGGL((k_forward_window<Src, MFH_MODE_B8>), grid, dim3(256), 0, c->stream,
                           s, dst, c->np, c->S, c->NB, c->K, c->g, r0, rows, gs);
}

int mfh_launch_forward(mfh_ctx *c, int in_kind, const void *src, int8_t *dst,
                       int scale_S, int r0, int rows, int side)
{
    const size_t nnp = (size_t)rows * c->np;
    const size_t nn = (size_t)c->n * c->n;
    dim3 grid((unsigned)((nnp + 255) / 256));
    const int LS = c->L / c->S;
    const int gs = c->pwr == MFH_PW_GAUSS ? 1 + side : 0;
    if (c->use_fast) {
        bool done = false;
        if (in_kind == MFH_IN_U16 || in_kind == MFH_IN_U16_SIGNED ||
            in_kind == MFH_IN_U16_OFFSET) {
            SrcU16 s{(const uint16_t *)src, nn, c->n, c->L};
            const int top = in_kind == MFH_IN_U16 ? 0 : in_kind == MFH_IN_U16_SIGNED ? 1 : 2;
            done = forward_fast_u16(c, s, dst, top, r0, rows, gs);
        } else if (in_kind == MFH_IN_F32) {
            SrcF32 s{(const float *)src, nn, c->n, c->L, scale_S};
            done = try_fast<4, 16, MFH_MODE_K7, false, SrcF32, LimbsI32<32>, 256, 4, 1>(
                c, s, dst, 0, r0, rows, gs);
        }
        if (done) {
            MFH_HIP(hipGetLastError());
            return MFH_OK;
        }
    }
    switch (in_kind) {
    case MFH_IN_U16: {
        SrcU16 s{(const uint16_t *)src, nn, c->n, c->L};
        launch_generic<SrcU16>(c, s, dst, grid, LS, r0, rows, gs);
        break;
    }
    case MFH_IN_U16_SIGNED: {
        SrcU16Signed s{(const uint16_t *)src, nn, c->n, c->L};
        launch_generic<SrcU16Signed>(c, s, dst, grid, LS, r0, rows, gs);
        break;
    }
    case MFH_IN_I32: {
        SrcI32 s{(const int32_t *)src, nn, c->n, c->L};
        launch_generic<SrcI32>(c, s, dst, grid, LS, r0, rows, gs);
        break;
    }
    case MFH_IN_F32: {
        SrcF32 s{(const float *)src, nn, c->n, c->L, scale_S};
        launch_window<SrcF32>(c, s, dst, grid, r0, rows, gs);
        break;
    }
    case MFH_IN_F64: {
        SrcF64 s{(const double *)src, nn, c->n, c->L, scale_S};
        launch_window<SrcF64>(c, s, dst, grid, r0, rows, gs);
        break;
    }
    case MFH_IN_U16_OFFSET:
        return MFH_E_UNSUPPORTED;       // recoding kernels only
    default:
        return MFH_E_ARG;
    }
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_check_i32(mfh_ctx *c, const int32_t *src, int planes)
{
    size_t count = (size_t)planes * c->n * c->n;
    hipLaunchKernelGGL(k_check_i32, dim3(grid_for(count, 4096)), dim3(256), 0,
                       c->stream, src, count, c->dFlag);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

namespace {
template <int NB, int K, bool CARRY, int NPASS = 2, int DEC = -1>
bool try_inverse_fast_as(mfh_ctx *c, int64_t *Cw, uint16_t *out, int RL, size_t eb0,
                         size_t eb1, int r0, int rows)
{
    constexpr int E = NPASS * (256 / K);
    const int P = 2 * c->L - 1;
    // coefficient planes, plus four int64 per carry-run thread
    const size_t lds = ((size_t)P * E + (CARRY ? 4 * 256 : 0)) * sizeof(int64_t);
    if (lds > 160 * 1024) return false;
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void *)k_inverse_fast<NB, K, CARRY, NPASS,
                                                             !(CARRY && NB == 32 && K == 16), DEC>,
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024) != hipSuccess)
            return false;
        attr_set = true;
    }
    hipLaunchKernelGGL((k_inverse_fast<NB, K, CARRY, NPASS, !(CARRY && NB == 32 && K == 16),
                                       DEC>),
                       dim3((unsigned)((eb1 - eb0 + E - 1) / E)), dim3(256), lds, c->stream,
                       c->dC5, Cw, out, RL, c->n, c->np, P, c->mode, mfh_nclasses(c->mode), eb0,
                       eb1, r0, rows, c->offset ? c->dRow : nullptr,
                       c->offset ? c->dCol : nullptr, c->dec_out, c->dec_SAB);
    return true;
}
// out != nullptr: fused carry into RL uint16 limbs (Cw is not written).
// With the carry fused, one pass of 256/K elements per workgroup: half the
// LDS of two passes, so more workgroups per CU hide the class loads (with
// carry lookahead this also pays at K = 32, 8 elements per workgroup:
// inverse + carry 2.15 -> 1.19 ms at n=256, W=8192).
template <int NB, int K>
bool try_inverse_fast(mfh_ctx *c, int64_t *Cw, uint16_t *&out, int RL, size_t eb0, size_t eb1,
                      int r0, int rows)
{
    if (c->NB != NB || c->K != K) return false;
    if (out) return try_inverse_fast_as<NB, K, true, 1>(c, Cw, out, RL, eb0, eb1, r0, rows);
    out = nullptr;
    // decode fused: one pass of 256/K elements per workgroup, as with the
    // fused carry (fp32 n=2048: inverse 2.26 -> 1.93 ms against two passes)
    if (c->dec_req == MFH_DEC_F32 + 1)
        return try_inverse_fast_as<NB, K, false, 1, MFH_DEC_F32>(c, Cw, out, RL, eb0, eb1, r0,
                                                                 rows);
    if (c->dec_req == MFH_DEC_F64 + 1)
        return try_inverse_fast_as<NB, K, false, 1, MFH_DEC_F64>(c, Cw, out, RL, eb0, eb1, r0,
                                                                 rows);
    return try_inverse_fast_as<NB, K, false>(c, Cw, out, RL, eb0, eb1, r0, rows);
}
}  // namespace

int mfh_launch_inverse(mfh_ctx *c, int64_t *Cw, uint16_t *out, int RL, int *carried, int r0,
                       int rows)
{
    *carried = 0;
    if (r0 < 0 || r0 >= c->n || rows < 1 || r0 + rows > c->np) return MFH_E_ARG;
    const int r1 = r0 + rows < c->n ? r0 + rows : c->n;       // band rows inside the matrix
    const size_t eb0 = (size_t)r0 * c->n, eb1 = (size_t)r1 * c->n;
    // offset mode needs the fused carry (it adds the offset terms there)
    if (c->offset && (!c->use_fast || !out)) return MFH_E_UNSUPPORTED;
    if (c->use_fast &&
        (try_inverse_fast<32, 16>(c, Cw, out, RL, eb0, eb1, r0, rows) ||    // W=2048
         try_inverse_fast<16, 16>(c, Cw, out, RL, eb0, eb1, r0, rows) ||    // W=1024
         try_inverse_fast<16, 8>(c, Cw, out, RL, eb0, eb1, r0, rows) ||     // W=512
         try_inverse_fast<32, 32>(c, Cw, out, RL, eb0, eb1, r0, rows) ||    // W=4096
         try_inverse_fast<64, 32>(c, Cw, out, RL, eb0, eb1, r0, rows))) {   // W=8192
        // 1: carried into limbs; 2: decoded into floats (Cw not written)
        *carried = out ? 1 : c->dec_req ? 2 : 0;
        MFH_HIP(hipGetLastError());
        return MFH_OK;
    }
    if (c->offset) return MFH_E_UNSUPPORTED;
    const int blk = c->NB * c->K;
    int epw = 8192 / blk;              // 2 * epw * blk * 8 bytes <= 128 KiB
    if (epw > 64) epw = 64;
    if (epw < 1) return MFH_E_UNSUPPORTED;
    int threads = epw * c->K;
    if (threads > 1024) { epw = 1024 / c->K; threads = epw * c->K; }
    if (threads < 64) threads = 64;    // keep whole waves; extra threads idle
    const size_t lds = (size_t)2 * epw * blk * sizeof(int64_t);
    static bool attr_set = false;
    if (!attr_set) {
        MFH_HIP(hipFuncSetAttribute((const void *)k_inverse_fold,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 131072));
        attr_set = true;
    }
    dim3 grid((unsigned)((eb1 - eb0 + epw - 1) / epw));
    hipLaunchKernelGGL(k_inverse_fold, grid, dim3(threads), lds, c->stream,
                       c->dC5, Cw, c->n, c->np, c->NB, c->K, c->S, c->g,
                       lg2i(c->NB), 2 * c->L - 1, epw, c->mode, mfh_nclasses(c->mode), eb0, eb1,
                       r0, rows);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_offset_sums(const uint16_t *src, int64_t *out, int n, int L, hipStream_t st)
{
    const size_t rows = (size_t)L * n;
    hipLaunchKernelGGL(k_offset_sums, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, src,
                       out, n, L);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_carry(mfh_ctx *c, const int64_t *Cw, uint16_t *out, int RL)
{
    const size_t nn = (size_t)c->n * c->n;
    hipLaunchKernelGGL(k_carry, dim3((unsigned)((nn + 255) / 256)), dim3(256), 0,
                       c->stream, Cw, out, nn, 2 * c->L - 1, RL);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_carry_planes(const int64_t *Cw, int P, size_t nn, uint16_t *out,
                            int RL, hipStream_t st)
{
    hipLaunchKernelGGL(k_carry, dim3((unsigned)((nn + 255) / 256)), dim3(256), 0, st,
                       Cw, out, nn, P, RL);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_encode(const void *X, int is_f64, int n, int L, int S, int32_t *out,
                      hipStream_t st)
{
    const size_t nn = (size_t)n * n;
    const dim3 grid((unsigned)((nn + 255) / 256));
    if (is_f64)
        hipLaunchKernelGGL(k_encode<SrcF64>, grid, dim3(256), 0, st,
                           SrcF64{(const double *)X, nn, n, L, S}, out);
    else
        hipLaunchKernelGGL(k_encode<SrcF32>, grid, dim3(256), 0, st,
                           SrcF32{(const float *)X, nn, n, L, S}, out);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_encode_tc(const void *X, int is_f64, int n, int L, int S, uint16_t *out,
                         hipStream_t st)
{
    const size_t nn = (size_t)n * n;
    const dim3 grid((unsigned)((nn + 255) / 256));
    if (is_f64)
        hipLaunchKernelGGL(k_encode_tc<SrcF64>, grid, dim3(256), 0, st,
                           SrcF64{(const double *)X, nn, n, L, S}, out);
    else
        hipLaunchKernelGGL(k_encode_tc<SrcF32>, grid, dim3(256), 0, st,
                           SrcF32{(const float *)X, nn, n, L, S}, out);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_decode_limbs(const uint16_t *limbs, size_t nn, int RLr, int SAB, int fmt,
                            void *out, int32_t *out2, hipStream_t st)
{
    const dim3 grid((unsigned)((nn + 255) / 256));
    if (fmt == MFH_DEC_F32)
        hipLaunchKernelGGL(k_decode_limbs<MFH_DEC_F32>, grid, dim3(256), 0, st, limbs, nn, RLr,
                           SAB, out, out2);
    else if (fmt == MFH_DEC_F64)
        hipLaunchKernelGGL(k_decode_limbs<MFH_DEC_F64>, grid, dim3(256), 0, st, limbs, nn, RLr,
                           SAB, out, out2);
    else
        return MFH_E_ARG;
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_decode(mfh_ctx *c, const int64_t *Cw, int SAB, int fmt, void *out,
                      int32_t *out2)
{
    const size_t nn = (size_t)c->n * c->n;
    const dim3 grid((unsigned)((nn + 255) / 256));
    const int P = 2 * c->L - 1, RL = 2 * c->L + 2;
    if (fmt == MFH_DEC_F32)
        hipLaunchKernelGGL(k_decode<MFH_DEC_F32>, grid, dim3(256), 0, c->stream, Cw, out,
                           out2, nn, P, RL, SAB);
    else if (fmt == MFH_DEC_F64)
        hipLaunchKernelGGL(k_decode<MFH_DEC_F64>, grid, dim3(256), 0, c->stream, Cw, out,
                           out2, nn, P, RL, SAB);
    else if (fmt == MFH_DEC_SIG63 && out2)
        hipLaunchKernelGGL(k_decode<MFH_DEC_SIG63>, grid, dim3(256), 0, c->stream, Cw, out,
                           out2, nn, P, RL, SAB);
    else
        return MFH_E_ARG;
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_rand_u16(void *dst, size_t count, uint64_t seed, hipStream_t st)
{
    hipLaunchKernelGGL(k_rand_u16, dim3(grid_for(count, 65536)), dim3(256), 0, st,
                       (uint16_t *)dst, count, seed);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_copy16(void *dst, const void *src, size_t bytes, hipStream_t st)
{
    const size_t count = bytes / 16;
    hipLaunchKernelGGL(k_copy16, dim3(grid_for(count, 8192)), dim3(256), 0, st,
                       (const uint4 *)src, (uint4 *)dst, count);
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}

int mfh_launch_rand_f32(void *dst, size_t count, uint64_t seed, int emin,
                        int emax, hipStream_t st)
{
    if (emax < emin) return MFH_E_ARG;
    hipLaunchKernelGGL(k_rand_f32, dim3(grid_for(count, 65536)), dim3(256), 0, st,
                       (float *)dst, count, seed, emin, (unsigned)(emax - emin + 1));
    MFH_HIP(hipGetLastError());
    return MFH_OK;
}
