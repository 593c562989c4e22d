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
// K*64 terms to an int32 accumulator, i.e. at most K * 2^20 in magnitude, so
// the int32 accumulators are flushed into int64 totals after at most
// floor((2^31 - 1) / (K * 2^20)) rounds.
//
// int64 totals: |C^| <= K * n * ((NB/2) * 65535)^2, and the inverse
// transform multiplies by at most NB more; both must stay below 2^62.
// ---------------------------------------------------------------------------
#define MFH_DIGITS 3
#define MFH_DIGIT_MAX 8355711LL   // 127 * (1 + 2^8 + 2^16)
#define MFH_DIGIT_MIN (-8421504LL) // -128 * (1 + 2^8 + 2^16)
#define MFH_KBLK 64               // k extent of one MFMA operand block

static inline int mfh_rounds_per_flush(int K)
{
    return (int)((2147483647LL) / ((long long)K << 20));
}

struct mfh_ctx {
    int n, np;            // matrix size, padded to a multiple of 64
    int L, S, NB, K, g;
    int dev;
    int use_fast;         // compile-time specialised kernels when available
    hipStream_t stream;
    // workspace
    int8_t *dAh, *dBh;    // digit planes [NB][K][3][np][np]
    int64_t *dCh;         // pointwise products [NB][np][np][K]
    int64_t *dCw;         // coefficient planes [2L-1][n][n]
    void *dBt;            // transposed B input, up to L*n*n int32
    int *dFlag;           // device error flags
    // staging for host-buffer entry points (allocated on first use)
    void *dInA, *dInB, *dOut;
    size_t inBytes, outBytes;
    size_t bytes;         // device bytes held
    // timing
    int timing;
    hipEvent_t ev[5];
    float stage_ms[5];
};

// kernel launchers (mfh_kernels.hip)
int mfh_launch_transpose(const void *src, void *dst, int planes, int n,
                         int elem_bytes, hipStream_t st);
int mfh_launch_forward(mfh_ctx *c, int in_kind, const void *src, int8_t *dst,
                       int scale_S);
int mfh_launch_check_i32(mfh_ctx *c, const int32_t *src, int planes);
int mfh_launch_pointwise(mfh_ctx *c);
int mfh_launch_inverse(mfh_ctx *c, int64_t *Cw);
int mfh_launch_carry(mfh_ctx *c, const int64_t *Cw, uint16_t *out, int RL);
int mfh_launch_carry_planes(const int64_t *Cw, int P, size_t nn, uint16_t *out,
                            int RL, hipStream_t st);
int mfh_launch_encode_f32(const float *X, int n, int L, int S, int32_t *out,
                          hipStream_t st);
int mfh_launch_decode_f32(mfh_ctx *c, const int64_t *Cw, int SAB, float *out);
int mfh_launch_rand_u16(void *dst, size_t count, uint64_t seed, hipStream_t st);
int mfh_launch_rand_f32(void *dst, size_t count, uint64_t seed, int emin,
                        int emax, hipStream_t st);

// input kind used internally for fp32 sources
#define MFH_IN_F32 100

#define MFH_HIP(call)                                   \
    do {                                                \
        hipError_t e_ = (call);                         \
        if (e_ != hipSuccess) return MFH_E_HIP;         \
    } while (0)
