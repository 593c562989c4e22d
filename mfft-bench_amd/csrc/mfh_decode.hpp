// mfh_decode.hpp -- the fixed-point decode of one element from its carried
// planes (src/fpfixed.c:212-322), shared by the MFFT inverse, the standalone
// decode kernels and the multi-modular CRT.  Not part of the public
// interface.
#pragma once

#include "mfh_internal.hpp"

// ---- fixed-point decode (src/fpfixed.c:212-322) ------------------------------
// Carry over RL = 2L+2 limbs with an arithmetic shift, take the magnitude
// (two's complement negation when the final carry is negative), keep the
// top <= 4 limbs below the highest non-zero one plus a sticky bit, round to
// 24 bits half-even, and scale by 2^-(SA+SB).  Exact zero gives +0.0f.
// Streaming: both the value and its negation are tracked limb by limb, so no
// per-element limb array is needed.
struct TopTrack {
    int h;
    uint32_t hist[4];      // limbs w-3 .. w
    uint32_t win[4];       // limbs h-3 .. h when h was set
    uint32_t below;        // OR of limbs < w-3
    uint32_t sticky;       // OR of limbs < h-3 when h was set
    __device__ void init()
    {
        h = -1; below = 0; sticky = 0;
        for (int q = 0; q < 4; ++q) { hist[q] = 0; win[q] = 0; }
    }
    __device__ void push(int w, uint32_t limb)
    {
        below |= hist[0];
        hist[0] = hist[1]; hist[1] = hist[2]; hist[2] = hist[3]; hist[3] = limb;
        if (limb) {
            h = w;
            for (int q = 0; q < 4; ++q) win[q] = hist[q];
            sticky = below;
        }
    }
};

// FMT: MFH_DEC_F32 rounds to 24 bits and writes fp32, MFH_DEC_F64 to 53
// bits and fp64 (src/fpfixed.c:308-322), MFH_DEC_SIG63 to 63 bits and writes
// the signed significand and the exponent of the long double decode
// (src/fpfixed.c:292-306: int64 sig at out, int32 exponent at out2).
// The rounding of one element from its magnitude's highest non-zero limb h
// (h < 0: zero), the limbs h-3 .. h (win[0 .. 3], zero below limb 0), the OR
// of the limbs below h-3 (sticky) and the sign.
template <int FMT>
__device__ __forceinline__ void decode_round(bool isneg, int h, const uint32_t (&win)[4],
                                             uint32_t sticky, int SAB, void *__restrict__ out_,
                                             int32_t *__restrict__ out2, size_t e)
{
    constexpr int BITS = FMT == MFH_DEC_F32 ? 24 : FMT == MFH_DEC_F64 ? 53 : 63;
    if (h < 0) {
        if constexpr (FMT == MFH_DEC_F32) ((float *)out_)[e] = 0.0f;
        else if constexpr (FMT == MFH_DEC_F64) ((double *)out_)[e] = 0.0;
        else { ((long long *)out_)[e] = 0; out2[e] = 0; }
        return;
    }
    int bl = 32 - __clz(win[3]);
    const int k = h + 1 < 4 ? h + 1 : 4;
    unsigned long long top = 0;
#pragma unroll
    for (int q = 3; q >= 0; --q)
        if (q > 3 - k) top = (top << 16) | win[q];
    // limbs below the gathered ones: win[0 .. 3-k] (positions h-3 .. h-k)
    // only exist when k == 4, so sticky is the OR below h-3.
    const int base = 16 * (h - k + 1);
    int tb = 16 * h + bl - base;
    int shift = base;
    unsigned long long sig = top;
    // a window of at most BITS bits is returned as it stands (sticky unused)
    if (tb > BITS) {
        int drop = tb - BITS;
        sig = top >> drop;
        unsigned long long rem = top & ((1ULL << drop) - 1);
        unsigned long long half = 1ULL << (drop - 1);
        int up = rem > half ? 1 : rem < half ? 0 : (sticky ? 1 : (int)(sig & 1));
        sig += (unsigned long long)up;
        if (sig >> BITS) { sig >>= 1; drop++; }
        shift += drop;
    }
    if constexpr (FMT == MFH_DEC_F32) {
        float v = ldexpf((float)sig, shift - SAB);
        ((float *)out_)[e] = isneg ? -v : v;
    } else if constexpr (FMT == MFH_DEC_F64) {
        double v = ldexp((double)sig, shift - SAB);
        ((double *)out_)[e] = isneg ? -v : v;
    } else {
        ((long long *)out_)[e] = isneg ? -(long long)sig : (long long)sig;
        out2[e] = shift - SAB;
    }
}

// Decode of one element from its 2L-1 coefficient planes (plane(w), w < P)
// over RL limbs (src/fpfixed.c:212-322, see k_decode)
template <int FMT, class Plane>
__device__ __forceinline__ void decode_value(const Plane &plane, int P, int RL, int SAB,
                                             void *__restrict__ out_, int32_t *__restrict__ out2,
                                             size_t e)
{
    TopTrack pos, neg;
    pos.init(); neg.init();
    int64_t carry = 0;
    uint32_t borrow = 1;
    for (int w = 0; w < RL; ++w) {
        int64_t t = carry + (w < P ? plane(w) : 0);
        uint32_t limb = (uint32_t)(t & 0xFFFF);
        carry = t >> 16;
        uint32_t nl = ((~limb) & 0xFFFFu) + borrow;
        borrow = nl >> 16;
        nl &= 0xFFFFu;
        pos.push(w, limb);
        neg.push(w, nl);
    }
    const bool isneg = carry < 0;
    const int h = isneg ? neg.h : pos.h;
    uint32_t win[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) win[q] = isneg ? neg.win[q] : pos.win[q];
    decode_round<FMT>(isneg, h, win, isneg ? neg.sticky : pos.sticky, SAB, out_, out2, e);
}

// The same decode from P carried two's complement limbs (limb(w): uint16,
// w < P, the sign in bit 15 of limb P-1), scanned from the top: the highest
// limb that differs from the sign fill (0 or 0xFFFF) gives h, the window
// and, below it, the sticky OR (stopping at the first non-zero limb).  For a
// negative value the magnitude's limbs are ~x_w, plus 1 on the lowest
// non-zero one (x_w = 0 below it): the window takes that carry when every
// limb below the window is zero.  Same (sign, h, window, sticky) as
// decode_value on the same integer, hence the same bits.
template <int FMT, class Limb>
__device__ __forceinline__ void decode_carried(const Limb &limb, int P, int SAB,
                                               void *__restrict__ out_,
                                               int32_t *__restrict__ out2, size_t e)
{
    const bool isneg = (limb(P - 1) >> 15) & 1;
    const uint32_t fill = isneg ? 0xFFFFu : 0u;
    int w = P - 1;
    while (w >= 0 && limb(w) == fill) --w;
    uint32_t win[4] = {0, 0, 0, 0};
    if (w < 0) {                              // 0, or -2^(16 P) ... all ones: -1
        if (isneg) win[3] = 1;
        decode_round<FMT>(isneg, isneg ? 0 : -1, win, 0u, SAB, out_, out2, e);
        return;
    }
    uint32_t x[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) x[q] = w - 3 + q >= 0 ? limb(w - 3 + q) : 0u;
    uint32_t sticky = 0;
    for (int v = w - 4; v >= 0 && !sticky; --v) sticky = limb(v);
    if (!isneg) {
        decode_round<FMT>(false, w, x, sticky, SAB, out_, out2, e);
        return;
    }
    // negative: magnitude limbs over the window, the +1 entering at the
    // lowest non-zero limb when nothing below the window is non-zero
    uint32_t c = sticky ? 0u : 1u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t m = (~x[q] & 0xFFFFu) + c;
        c = m >> 16;
        win[q] = m & 0xFFFFu;
    }
    // every limb from the window down is zero: the value is -2^(16(w+1)) and
    // limbs w+1 .. P-1 are all ones, so the magnitude is 1 at limb w+1
    if (c) {
        uint32_t one[4] = {0, 0, 0, 1};
        decode_round<FMT>(true, w + 1, one, 0u, SAB, out_, out2, e);
        return;
    }
    decode_round<FMT>(true, w, win, sticky, SAB, out_, out2, e);
}

