// mfh_shim.hip -- extern "C" entry points of mfft_hip.h: device contexts,
// workspace, the product pipelines and timing.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <thread>

#include "mfh_internal.hpp"

// Workspace of mfh_mm_dev_noalloc: one fixed array per device, allocated by
// the runtime when the library's code object is loaded and held until the
// process ends.  Host code never uses this name as an address (on the host
// it is only a stand-in for the symbol): the device address comes from
// hipGetSymbolAddress, per device (noalloc_scratch below).
static __device__ __align__(256) unsigned char scratch[MFH_NOALLOC_BYTES];

namespace {

const char *kErr[] = {"ok",
                      "no usable gfx950 device",
                      "device out of memory",
                      "invalid argument",
                      "plan or size exceeds a stated accumulator bound",
                      "input limb outside [-65535, 65535]",
                      "HIP runtime error",
                      "unsupported plan",
                      "workspace exceeds the fixed no-allocation scratch"};

char g_arch[64];

int check_device()
{
    int cnt = 0;
    if (hipGetDeviceCount(&cnt) != hipSuccess || cnt < 1) return MFH_E_NODEV;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return MFH_E_NODEV;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return MFH_E_NODEV;
    return MFH_OK;
}

int dalloc(mfh_ctx *c, void **p, size_t bytes)
{
    *p = nullptr;
    if (!bytes) return MFH_OK;
    if (hipMalloc(p, bytes) != hipSuccess) { *p = nullptr; return MFH_E_NOMEM; }
    c->bytes += bytes;
    return MFH_OK;
}

int ensure_staging(mfh_ctx *c, size_t in_bytes, size_t out_bytes)
{
    if (c->inBytes < in_bytes) {
        if (c->dInA) { (void)hipFree(c->dInA); c->bytes -= c->inBytes; }
        if (c->dInB) { (void)hipFree(c->dInB); c->bytes -= c->inBytes; }
        c->dInA = c->dInB = nullptr;
        c->inBytes = 0;
        int rc = dalloc(c, &c->dInA, in_bytes);
        if (!rc) rc = dalloc(c, &c->dInB, in_bytes);
        if (rc) return rc;
        c->inBytes = in_bytes;
    }
    if (c->outBytes < out_bytes) {
        if (c->dOut) { (void)hipFree(c->dOut); c->bytes -= c->outBytes; }
        c->dOut = nullptr;
        c->outBytes = 0;
        int rc = dalloc(c, &c->dOut, out_bytes);
        if (rc) return rc;
        c->outBytes = out_bytes;
    }
    return MFH_OK;
}

// Digit mode of a product.  K7 (6 Karatsuba products instead of 9) needs
// every transformed value inside [-1056832, 1056703]; |a^| is at most the
// sum of NB/2 limb magnitudes (one limb per non-zero block):
//  * plain limbs: (NB/2) 65535;
//  * the exact track's forward transform can first recode limbs to
//    [-2^15, 2^15) with the top limb keeping its carry: up to 2^16 for
//    unsigned entries, (NB/2 - 1) 2^15 + 2^16; in [-2^15, 2^15] for two's
//    complement entries, or for unsigned ones shifted by -2^(W-1) (offset
//    mode, the inverse adds the shift's terms back): (NB/2) 2^15.
// Recoding runs in the plans the forward transform is specialised for
// (k7_recode_plan).  conv_mfft must return the convolution of the caller's
// limbs, so it never recodes.
//
// Each setting must also keep the int64 and int32 intermediates exact:
//  * int64: the inverse sees NB * K * n * |a^| |b^| (NB points of K-term
//    ring products over n), below 2^62;
//  * int32 classes: pairs * (np/64) * K * 2^20 (mfh_class_bound_ok), pairs =
//    1 for K7, 3 for B8.
bool k7_recode_plan(const mfh_ctx *c)
{
    return c->use_fast && c->n % 8 == 0 &&
           ((c->S == 8 && c->NB == 32) || (c->S == 16 && c->NB == 64));
}
bool fits(const mfh_ctx *c, long long amax, int pairs)
{
    const double bits = log2((double)c->NB) + log2((double)c->K) + log2((double)c->np) +
                        2.0 * log2((double)amax);
    return bits < 62.0 && mfh_class_bound_ok(c->K, c->np, pairs);
}
// kind: the input of an exact-track product (MFH_IN_U16 or
// MFH_IN_U16_SIGNED), or -1 for products of the caller's own limbs.  Sets
// mode / recode / offset to the first setting that fits, in the order
// recoded K7, plain K7, recoded K7 with symmetric limbs (signed entries, or
// unsigned ones in offset mode), B8; mode_ok = 0 when none does.
void select_mode(mfh_ctx *c, int kind)
{
    const bool exact = kind == MFH_IN_U16 || kind == MFH_IN_U16_SIGNED;
    const long long half = c->NB / 2;
    const long long a_plain = half * 65535, a_rec = (half + 1) * 32768, a_sym = half * 32768;
    const bool rec = exact && k7_recode_plan(c);
    struct { bool ok; int mode, recode, offset; } cand[] = {
        {rec && a_rec <= MFH_K7_MAX && fits(c, a_rec, 1), MFH_MODE_K7, 1, 0},
        {a_plain <= MFH_K7_MAX && fits(c, a_plain, 1), MFH_MODE_K7, 0, 0},
        {rec && a_sym <= MFH_K7_MAX && fits(c, a_sym, 1), MFH_MODE_K7, 1, kind == MFH_IN_U16},
        {a_plain <= MFH_DIGIT_MAX && fits(c, a_plain, 3), MFH_MODE_B8, 0, 0},
    };
    c->mode = MFH_MODE_B8;
    c->recode = c->offset = c->mode_ok = 0;
    c->pwr = MFH_PW_FLAT;
    for (const auto &k : cand)
        if (k.ok) {
            c->mode = k.mode;
            c->recode = k.recode;
            c->offset = k.offset;
            c->mode_ok = 1;
            // the Gauss kernels take the 6-product digits
            c->pwr = c->pw == MFH_PW_GAUSS && k.mode == MFH_MODE_K7 ? MFH_PW_GAUSS : MFH_PW_FLAT;
            return;
        }
}

void mark(mfh_ctx *c, int k)
{
    if (c->timing) (void)hipEventRecord(c->ev[k], c->stream);
}
void mark_band(mfh_ctx *c, int b, int k)
{
    if (c->timing) (void)hipEventRecord(c->bev[b][k], c->stream);
}

// transforms in, pointwise, inverse; leaves the coefficient planes in Cw,
// or, when out16 is given and the inverse kernel fuses the carry, the RL
// output limbs in out16 (*carried = 1).  B is transformed once; A goes
// through in row bands of c->hb padded rows (one band when the whole
// workspace fits), each transformed, multiplied by all of B and inverted
// into its rows of the output.
int run_conv(mfh_ctx *c, int kind, const void *dA, const void *dB, int64_t *Cw,
             int SA, int SB, uint16_t *out16 = nullptr, int RL = 0, int *carried = nullptr)
{
    int rc;
    if (!c->mode_ok) return MFH_E_BOUND;
    mark(c, 0);
    const int eb = (kind == MFH_IN_U16 || kind == MFH_IN_U16_SIGNED) ? 2
                   : kind == MFH_IN_F64 ? 8 : 4;
    const int planes = (kind == MFH_IN_F32 || kind == MFH_IN_F64) ? 1 : c->L;
    if ((rc = mfh_launch_transpose(dB, c->dBt, planes, c->n, eb, c->stream))) return rc;
    if (c->offset) {
        // shifted operands: row sums of A, column sums of B (rows of B^T)
        if (kind != MFH_IN_U16 || !out16) return MFH_E_UNSUPPORTED;
        kind = MFH_IN_U16_OFFSET;
        if ((rc = mfh_launch_offset_sums((const uint16_t *)dA, c->dRow, c->n, c->L, c->stream)) ||
            (rc = mfh_launch_offset_sums((const uint16_t *)c->dBt, c->dCol, c->n, c->L,
                                         c->stream)))
            return rc;
    }
    if ((rc = mfh_launch_forward(c, kind, c->dBt, c->dBh, SB, 0, c->np, 1))) return rc;
    int fused = 0, b = 0;
    for (int r0 = 0; r0 < c->n; r0 += c->hb, ++b) {
        const int rows = c->hb < c->np - r0 ? c->hb : c->np - r0;
        mark_band(c, b, 0);
        if ((rc = mfh_launch_forward(c, kind, dA, c->dAh, SA, r0, rows, 0))) return rc;
        mark_band(c, b, 1);
        if ((rc = mfh_launch_pointwise(c, rows))) return rc;
        mark_band(c, b, 2);
        if ((rc = mfh_launch_inverse(c, Cw, out16, RL, &fused, r0, rows))) return rc;
        mark_band(c, b, 3);
    }
    if (carried) *carried = fused;
    return MFH_OK;
}

// Row band height: all np rows when A's digit planes, B's, the class
// results and the fixed buffers fit in 90 % of the device memory free now,
// else the most multiples of 64 rows that do (at least np / MFH_BANDS_MAX).
// MFH_BAND_ROWS=<rows> forces a height (rounded up to a multiple of 64).
int band_rows(int np_, size_t per_row, size_t fixed, int *hb)
{
    const int min_rows = ((np_ + MFH_BANDS_MAX - 1) / MFH_BANDS_MAX + 63) / 64 * 64;
    if (const char *env = getenv("MFH_BAND_ROWS")) {
        long v = strtol(env, nullptr, 10);
        if (v > 0) {
            long r = (v + 63) / 64 * 64;
            if (r < min_rows) r = min_rows;
            *hb = r < np_ ? (int)r : np_;
            return MFH_OK;
        }
    }
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) return MFH_E_HIP;
    const double budget = 0.9 * (double)free_b - (double)fixed;
    if ((double)per_row * np_ <= budget) { *hb = np_; return MFH_OK; }
    const long fit = budget > 0 ? (long)(budget / (double)per_row) / 64 * 64 : 0;
    if (fit < min_rows) return MFH_E_NOMEM;
    *hb = (int)fit;
    return MFH_OK;
}

int read_flag(mfh_ctx *c, int *flag)
{
    MFH_HIP(hipMemcpyAsync(flag, c->dFlag, sizeof(int), hipMemcpyDeviceToHost, c->stream));
    MFH_HIP(hipStreamSynchronize(c->stream));
    return MFH_OK;
}

}  // namespace

extern "C" {

const char *mfh_strerror(int code)
{
    int k = -code;
    if (k < 0 || k >= (int)(sizeof kErr / sizeof kErr[0])) return "unknown error";
    return kErr[k];
}

int mfh_device_count(void)
{
    int cnt = 0;
    if (hipGetDeviceCount(&cnt) != hipSuccess) return 0;
    return cnt;
}

const char *mfh_device_arch(void)
{
    g_arch[0] = 0;
    int cnt = 0;
    if (hipGetDeviceCount(&cnt) == hipSuccess && cnt > 0) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, 0) == hipSuccess) {
            strncpy(g_arch, prop.gcnArchName, sizeof g_arch - 1);
            g_arch[sizeof g_arch - 1] = 0;
        }
    }
    return g_arch;
}

}  // extern "C"

namespace {
// Checks (n, L, plan) and fills the shape fields of a zeroed context: sizes,
// plan, kernel family and whether 6-product digits serve any of its
// products.  The int64 and int32 bounds must hold for some digit setting of
// the exact track (a superset of the others'); a size only some settings
// admit serves the products that use them (MFH_E_BOUND for the others, at
// call time).
int shape_init(mfh_ctx *c, int n, int L, const mfh_plan *p)
{
    if (n < 1 || L < 2 || (L & (L - 1))) return MFH_E_ARG;
    // the flat plan of src/mfft.c:77-95
    if (p->L != L || p->S < 1 || p->NB < 2 || p->K != 2 * p->S ||
        p->NB * p->S != 2 * L || (2 * p->K) % p->NB || p->g != 2 * p->K / p->NB)
        return MFH_E_ARG;
    if (p->K != 4 && p->K != 8 && p->K != 16 && p->K != 32) return MFH_E_UNSUPPORTED;
    // digit range: |a^| <= (NB/2) * 65535 must fit three balanced int8 digits
    if ((long long)(p->NB / 2) * 65535 > MFH_DIGIT_MAX) return MFH_E_BOUND;
    memset(c, 0, sizeof *c);
    c->n = n; c->np = (n + MFH_KBLK - 1) / MFH_KBLK * MFH_KBLK;
    c->L = L; c->S = p->S; c->NB = p->NB; c->K = p->K; c->g = p->g;
    c->use_fast = getenv("MFH_GENERIC_KERNELS") ? 0 : 1;
    // the Gauss pointwise where a kernel exists for K (MFH_POINTWISE=flat:
    // the K^2-product kernel throughout)
    const char *pwe = getenv("MFH_POINTWISE");
    c->pw = mfh_gauss_supported(c->K) && !(pwe && strcmp(pwe, "flat") == 0) ? MFH_PW_GAUSS
                                                                             : MFH_PW_FLAT;
    select_mode(c, MFH_IN_U16);
    if (!c->mode_ok) return MFH_E_BOUND;
    bool k7_ok = c->mode == MFH_MODE_K7;
    select_mode(c, -1);
    k7_ok |= c->mode_ok && c->mode == MFH_MODE_K7;
    c->k7_ok = k7_ok;
    select_mode(c, MFH_IN_U16);
    return MFH_OK;
}

// per padded row of A: its digit planes and its class results
size_t digit_row_bytes(const mfh_ctx *c)
{
    return (size_t)c->NB * mfh_slots(c->K, c->pw) * (c->k7_ok ? MFH_PLANES_MAX : MFH_DIGITS) *
           c->np;
}
size_t c5_row_bytes(const mfh_ctx *c)
{
    return (size_t)c->NB * (c->k7_ok ? MFH_CLASSES_MAX : MFH_CLASSES) * c->K * c->np *
           sizeof(int32_t);
}
}  // namespace

extern "C" {

int mfh_create(mfh_ctx **out, int n, int L, const mfh_plan *p)
{
    if (!out || !p) return MFH_E_ARG;
    *out = nullptr;
    mfh_ctx shape;
    int rc = shape_init(&shape, n, L, p);
    if (rc) return rc;
    if ((rc = check_device())) return rc;

    mfh_ctx *c = new mfh_ctx;
    *c = shape;
    c->dev = 0;
    if (hipSetDevice(0) != hipSuccess || hipStreamCreate(&c->stream) != hipSuccess) {
        delete c;
        return MFH_E_HIP;
    }
    for (int k = 0; k < 5; ++k) (void)hipEventCreate(&c->ev[k]);
    const int np_ = c->np;
    const size_t nn = (size_t)n * n;
    const size_t digit_row = digit_row_bytes(c), c5_row = c5_row_bytes(c);
    const size_t cw_bytes = (size_t)(2 * L - 1) * nn * sizeof(int64_t);
    const size_t bt_bytes = (size_t)L * nn * sizeof(int32_t);
    rc = band_rows(np_, digit_row + c5_row, digit_row * np_ + cw_bytes + bt_bytes, &c->hb);
    if (rc) { mfh_destroy(c); return rc; }
    c->nbands = (n + c->hb - 1) / c->hb;
    for (int b = 0; b < c->nbands; ++b)
        for (int k = 0; k < 4; ++k) (void)hipEventCreate(&c->bev[b][k]);
    rc = dalloc(c, (void **)&c->dAh, digit_row * c->hb);
    if (!rc) rc = dalloc(c, (void **)&c->dBh, digit_row * np_);
    if (!rc) rc = dalloc(c, (void **)&c->dC5, c5_row * c->hb);
    if (!rc) rc = dalloc(c, (void **)&c->dCw, cw_bytes);
    if (!rc) rc = dalloc(c, &c->dBt, bt_bytes);
    if (!rc) rc = dalloc(c, (void **)&c->dFlag, sizeof(int));
    if (!rc && k7_recode_plan(c)) {
        rc = dalloc(c, (void **)&c->dRow, (size_t)L * n * sizeof(int64_t));
        if (!rc) rc = dalloc(c, (void **)&c->dCol, (size_t)L * n * sizeof(int64_t));
    }
    if (rc) { mfh_destroy(c); return rc; }
    *out = c;
    return MFH_OK;
}

void mfh_destroy(mfh_ctx *c)
{
    if (!c) return;
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (int b = 0; b < 2; ++b) {
        if (c->pin[b]) (void)hipHostFree(c->pin[b]);
        if (c->pev[b]) (void)hipEventDestroy(c->pev[b]);
    }
    void *bufs[] = {c->dAh, c->dBh, c->dC5, c->dCw, c->dBt, c->dFlag,
                    c->dInA, c->dInB, c->dOut, c->dRow, c->dCol};
    for (void *b : bufs)
        if (b) (void)hipFree(b);
    for (int k = 0; k < 5; ++k)
        if (c->ev[k]) (void)hipEventDestroy(c->ev[k]);
    for (int b = 0; b < c->nbands; ++b)
        for (int k = 0; k < 4; ++k)
            if (c->bev[b][k]) (void)hipEventDestroy(c->bev[b][k]);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

size_t mfh_workspace_bytes(const mfh_ctx *c) { return c ? c->bytes : 0; }
int mfh_band_rows(const mfh_ctx *c) { return c ? c->hb : MFH_E_ARG; }

int mfh_mm_dev(mfh_ctx *c, int kind, const void *dA, const void *dB, void *dOut, int RL)
{
    if (!c || !dA || !dB || !dOut || RL < 1) return MFH_E_ARG;
    // the forward kernels stage limbs with 16-byte loads
    if (((uintptr_t)dA | (uintptr_t)dB) % 16) return MFH_E_ARG;
    if (kind != MFH_IN_U16 && kind != MFH_IN_U16_SIGNED) return MFH_E_ARG;
    select_mode(c, kind);
    int carried = 0;
    int rc = run_conv(c, kind, dA, dB, c->dCw, 0, 0, (uint16_t *)dOut, RL, &carried);
    if (rc) return rc;
    if (!carried && (rc = mfh_launch_carry(c, c->dCw, (uint16_t *)dOut, RL))) return rc;
    c->last_out = 0; c->last_RL = RL; c->last_fused = carried;
    mark(c, 4);
    return MFH_OK;
}

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch[kMaxDevices];   // device address of `scratch`, per device

// the device address of the current device's scratch array, looked up once
// per device with that device current
int noalloc_scratch(void **out)
{
    int dev = 0;
    MFH_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return MFH_E_UNSUPPORTED;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return MFH_E_HIP;
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return MFH_OK;
}
}  // namespace

// The buffers of mfh_create's workspace, for one band of all np rows, laid
// out in the scratch array at 256-byte boundaries (B's transposed limbs as
// uint16: only the exact-track product runs here).
int mfh_mm_dev_noalloc(int kind, const mfh_plan *plan, int n, int L, const void *dA,
                       const void *dB, void *dOut, int RL, void *stream)
{
    if (!plan || !dA || !dB || !dOut || RL < 1) return MFH_E_ARG;
    if (((uintptr_t)dA | (uintptr_t)dB) % 16) return MFH_E_ARG;
    if (kind != MFH_IN_U16 && kind != MFH_IN_U16_SIGNED) return MFH_E_ARG;
    mfh_ctx c;
    int rc = shape_init(&c, n, L, plan);
    if (rc) return rc;
    const size_t nn = (size_t)n * n;
    size_t off = 0;
    auto take = [&off](size_t bytes) {
        const size_t at = off;
        off += (bytes + 255) / 256 * 256;
        return at;
    };
    const size_t oAh = take(digit_row_bytes(&c) * c.np), oBh = take(digit_row_bytes(&c) * c.np);
    const size_t oC5 = take(c5_row_bytes(&c) * c.np);
    const size_t oCw = take((size_t)(2 * L - 1) * nn * sizeof(int64_t));
    const size_t oBt = take((size_t)L * nn * sizeof(uint16_t));
    const size_t oFlag = take(sizeof(int));
    const bool sums = k7_recode_plan(&c);
    const size_t oRow = sums ? take((size_t)L * n * sizeof(int64_t)) : 0;
    const size_t oCol = sums ? take((size_t)L * n * sizeof(int64_t)) : 0;
    if (off > (size_t)MFH_NOALLOC_BYTES) return MFH_E_SCRATCH;
    if ((rc = check_device())) return rc;
    void *base = nullptr;
    if ((rc = noalloc_scratch(&base))) return rc;
    unsigned char *b = (unsigned char *)base;
    c.dAh = (int8_t *)(b + oAh);
    c.dBh = (int8_t *)(b + oBh);
    c.dC5 = (int32_t *)(b + oC5);
    c.dCw = (int64_t *)(b + oCw);
    c.dBt = b + oBt;
    c.dFlag = (int *)(b + oFlag);
    if (sums) {
        c.dRow = (int64_t *)(b + oRow);
        c.dCol = (int64_t *)(b + oCol);
    }
    c.hb = c.np;
    c.nbands = 1;
    c.stream = (hipStream_t)stream;
    select_mode(&c, kind);
    int carried = 0;
    rc = run_conv(&c, kind, dA, dB, c.dCw, 0, 0, (uint16_t *)dOut, RL, &carried);
    if (rc) return rc;
    if (!carried) rc = mfh_launch_carry(&c, c.dCw, (uint16_t *)dOut, RL);
    return rc;
}

// products that return the caller's own limb convolution (conv_mfft, the
// fixed-point floats) never recode: plain K7 or B8, if either fits
static bool conv_size_ok(mfh_ctx *c)
{
    select_mode(c, -1);
    return c->mode_ok != 0;
}

int mfh_conv_dev(mfh_ctx *c, const void *dA32, const void *dB32, void *dCw)
{
    if (!c || !dA32 || !dB32 || !dCw) return MFH_E_ARG;
    if (!conv_size_ok(c)) return MFH_E_BOUND;
    int rc, flag = 0;
    MFH_HIP(hipMemsetAsync(c->dFlag, 0, sizeof(int), c->stream));
    if ((rc = mfh_launch_check_i32(c, (const int32_t *)dA32, c->L))) return rc;
    if ((rc = mfh_launch_check_i32(c, (const int32_t *)dB32, c->L))) return rc;
    if ((rc = read_flag(c, &flag))) return rc;
    if (flag) return MFH_E_RANGE;
    select_mode(c, -1);
    rc = run_conv(c, MFH_IN_I32, dA32, dB32, (int64_t *)dCw, 0, 0);
    if (rc) return rc;
    c->last_out = 1; c->last_fused = 0;
    mark(c, 4);
    return MFH_OK;
}

namespace {
// encode -> product -> decode of fp32 (f64 = 0) or fp64 matrices
int fpx_mm_dev(mfh_ctx *c, int f64, const void *dA, const void *dB, int SA, int SB, void *dC)
{
    if (!c || !dA || !dB || !dC) return MFH_E_ARG;
    if (!conv_size_ok(c)) return MFH_E_BOUND;
    select_mode(c, -1);
    // the specialised inverse kernels decode straight from their planes
    c->dec_req = (f64 ? MFH_DEC_F64 : MFH_DEC_F32) + 1;
    c->dec_out = dC;
    c->dec_SAB = SA + SB;
    int decoded = 0;
    int rc = run_conv(c, f64 ? MFH_IN_F64 : MFH_IN_F32, dA, dB, c->dCw, SA, SB, nullptr, 0,
                      &decoded);
    c->dec_req = 0;
    c->dec_out = nullptr;
    if (rc) return rc;
    if (decoded != 2 &&
        (rc = mfh_launch_decode(c, c->dCw, SA + SB, f64 ? MFH_DEC_F64 : MFH_DEC_F32, dC,
                                nullptr)))
        return rc;
    c->last_out = f64 ? 3 : 2; c->last_fused = decoded == 2;
    mark(c, 4);
    return MFH_OK;
}
}  // namespace

int mfh_fpx_mm_dev(mfh_ctx *c, const void *dA, const void *dB, int SA, int SB, void *dC)
{
    return fpx_mm_dev(c, 0, dA, dB, SA, SB, dC);
}

int mfh_fpx_mm_f64_dev(mfh_ctx *c, const void *dA, const void *dB, int SA, int SB, void *dC)
{
    return fpx_mm_dev(c, 1, dA, dB, SA, SB, dC);
}

int mfh_fpx_decode_dev(mfh_ctx *c, const void *dCw, int SAB, void *dC)
{
    if (!c || !dCw || !dC) return MFH_E_ARG;
    return mfh_launch_decode(c, (const int64_t *)dCw, SAB, MFH_DEC_F32, dC, nullptr);
}

int mfh_fpx_decode_f64_dev(mfh_ctx *c, const void *dCw, int SAB, void *dC)
{
    if (!c || !dCw || !dC) return MFH_E_ARG;
    return mfh_launch_decode(c, (const int64_t *)dCw, SAB, MFH_DEC_F64, dC, nullptr);
}

// ---- copies of the caller's (pageable) memory ------------------------------
// Through two pinned chunks: while one chunk's DMA runs, several host
// threads copy the next chunk between the caller's memory and the other
// (a plain hipMemcpy of pageable memory moved about 15 GB/s here).
namespace {
constexpr size_t PIN_CHUNK = (size_t)64 << 20;
constexpr int PIN_THREADS = 8;

void par_copy(void *dst, const void *src, size_t bytes)
{
    if (bytes < ((size_t)4 << 20)) {
        memcpy(dst, src, bytes);
        return;
    }
    const size_t part = (bytes / PIN_THREADS + 63) / 64 * 64;
    std::thread th[PIN_THREADS - 1];
    for (int t = 1; t < PIN_THREADS; ++t) {
        const size_t o = (size_t)t * part;
        if (o >= bytes) break;
        th[t - 1] = std::thread([=] { memcpy((char *)dst + o, (const char *)src + o,
                                             std::min(part, bytes - o)); });
    }
    memcpy(dst, src, std::min(part, bytes));
    for (auto &x : th)
        if (x.joinable()) x.join();
}

// the pinned chunks, on first use; false when they cannot be had (the
// copies then go straight from the caller's memory)
bool pin_ready(mfh_ctx *c)
{
    if (c->pin[1]) return true;
    for (int b = 0; b < 2; ++b) {
        if (hipHostMalloc(&c->pin[b], PIN_CHUNK, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&c->pev[b], hipEventDisableTiming) != hipSuccess ||
            hipEventRecord(c->pev[b], c->stream) != hipSuccess) {
            (void)hipGetLastError();
            for (int q = 0; q < 2; ++q) {
                if (c->pin[q]) (void)hipHostFree(c->pin[q]);
                if (c->pev[q]) (void)hipEventDestroy(c->pev[q]);
                c->pin[q] = nullptr;
                c->pev[q] = nullptr;
            }
            return false;
        }
    }
    return true;
}

// host -> device, stream-ordered; returns once the caller's memory has been
// read (it may be reused then)
int copy_in(mfh_ctx *c, void *dst, const void *src, size_t bytes)
{
    if (!pin_ready(c)) {
        MFH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
        MFH_HIP(hipStreamSynchronize(c->stream));
        return MFH_OK;
    }
    for (size_t off = 0, i = 0; off < bytes; off += PIN_CHUNK, ++i) {
        const int b = (int)(i & 1);
        const size_t len = std::min(PIN_CHUNK, bytes - off);
        MFH_HIP(hipEventSynchronize(c->pev[b]));
        par_copy(c->pin[b], (const char *)src + off, len);
        MFH_HIP(hipMemcpyAsync((char *)dst + off, c->pin[b], len, hipMemcpyHostToDevice,
                               c->stream));
        MFH_HIP(hipEventRecord(c->pev[b], c->stream));
    }
    return MFH_OK;
}

// device -> host after the work queued on the stream; returns with dst
// written
int copy_out(mfh_ctx *c, void *dst, const void *src, size_t bytes)
{
    if (!pin_ready(c)) {
        MFH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
        MFH_HIP(hipStreamSynchronize(c->stream));
        return MFH_OK;
    }
    const size_t nch = (bytes + PIN_CHUNK - 1) / PIN_CHUNK;
    auto issue = [&](size_t k) -> int {
        const int b = (int)(k & 1);
        const size_t off = k * PIN_CHUNK, len = std::min(PIN_CHUNK, bytes - off);
        MFH_HIP(hipMemcpyAsync(c->pin[b], (const char *)src + off, len, hipMemcpyDeviceToHost,
                               c->stream));
        MFH_HIP(hipEventRecord(c->pev[b], c->stream));
        return MFH_OK;
    };
    int rc;
    if (nch > 0 && (rc = issue(0))) return rc;
    for (size_t k = 0; k < nch; ++k) {
        // chunk k+1 goes into the other buffer, whose chunk k-1 is copied out
        if (k + 1 < nch && (rc = issue(k + 1))) return rc;
        const int b = (int)(k & 1);
        MFH_HIP(hipEventSynchronize(c->pev[b]));
        const size_t off = k * PIN_CHUNK;
        par_copy((char *)dst + off, c->pin[b], std::min(PIN_CHUNK, bytes - off));
    }
    return MFH_OK;
}
}  // namespace

int mfh_mm(mfh_ctx *c, int kind, const uint16_t *A, const uint16_t *B, uint16_t *out, int RL)
{
    if (!c || !A || !B || !out || RL < 1) return MFH_E_ARG;
    const size_t nn = (size_t)c->n * c->n;
    const size_t in_b = (size_t)c->L * nn * 2, out_b = (size_t)RL * nn * 2;
    int rc = ensure_staging(c, in_b, out_b);
    if (rc) return rc;
    if ((rc = copy_in(c, c->dInA, A, in_b)) || (rc = copy_in(c, c->dInB, B, in_b)) ||
        (rc = mfh_mm_dev(c, kind, c->dInA, c->dInB, c->dOut, RL)))
        return rc;
    return copy_out(c, out, c->dOut, out_b);
}

int mfh_conv(mfh_ctx *c, const int32_t *A32, const int32_t *B32, int64_t *Cw)
{
    if (!c || !A32 || !B32 || !Cw) return MFH_E_ARG;
    if (!conv_size_ok(c)) return MFH_E_BOUND;
    const size_t nn = (size_t)c->n * c->n;
    const size_t in_b = (size_t)c->L * nn * 4;
    const size_t out_b = (size_t)(2 * c->L - 1) * nn * 8;
    int rc = ensure_staging(c, in_b, 0);
    if (rc) return rc;
    if ((rc = copy_in(c, c->dInA, A32, in_b)) || (rc = copy_in(c, c->dInB, B32, in_b)) ||
        (rc = mfh_conv_dev(c, c->dInA, c->dInB, c->dCw)))
        return rc;
    return copy_out(c, Cw, c->dCw, out_b);
}

int mfh_conv_stages(mfh_ctx *c, const int32_t *A32, const int32_t *B32, int stage, void *out,
                    size_t out_bytes, int64_t *info)
{
    if (!c || !A32 || !B32 || !info || stage < MFH_STAGE_A || stage > MFH_STAGE_CLASSES)
        return MFH_E_ARG;
    if (!conv_size_ok(c)) return MFH_E_BOUND;
    const size_t nn = (size_t)c->n * c->n;
    const size_t in_b = (size_t)c->L * nn * 4;
    int rc = ensure_staging(c, in_b, 0), flag = 0;
    if (rc) return rc;
    const int rows = c->hb < c->np ? c->hb : c->np;        // row band 0
    const size_t planes = (size_t)c->NB * mfh_slots(c->K, c->pwr) * mfh_planes(c->mode);
    const size_t bytes = stage == MFH_STAGE_A   ? planes * rows * c->np
                         : stage == MFH_STAGE_B ? planes * c->np * c->np
                                                : (size_t)c->NB * rows * mfh_nclasses(c->mode) *
                                                      mfh_c5_class_stride(c->np, c->K) * 4;
    info[0] = c->mode;
    info[1] = c->pwr;
    info[2] = rows;
    info[3] = c->np;
    info[4] = (int64_t)bytes;
    if (!out) return MFH_OK;
    if (out_bytes < bytes) return MFH_E_ARG;
    MFH_HIP(hipMemcpyAsync(c->dInA, A32, in_b, hipMemcpyHostToDevice, c->stream));
    MFH_HIP(hipMemcpyAsync(c->dInB, B32, in_b, hipMemcpyHostToDevice, c->stream));
    MFH_HIP(hipMemsetAsync(c->dFlag, 0, sizeof(int), c->stream));
    if ((rc = mfh_launch_check_i32(c, (const int32_t *)c->dInA, c->L)) ||
        (rc = mfh_launch_check_i32(c, (const int32_t *)c->dInB, c->L)) ||
        (rc = read_flag(c, &flag)))
        return rc;
    if (flag) return MFH_E_RANGE;
    select_mode(c, -1);
    if ((rc = mfh_launch_transpose(c->dInB, c->dBt, c->L, c->n, 4, c->stream)) ||
        (rc = mfh_launch_forward(c, MFH_IN_I32, c->dBt, c->dBh, 0, 0, c->np, 1)) ||
        (rc = mfh_launch_forward(c, MFH_IN_I32, c->dInA, c->dAh, 0, 0, rows, 0)))
        return rc;
    if (stage == MFH_STAGE_CLASSES && (rc = mfh_launch_pointwise(c, rows))) return rc;
    const void *src = stage == MFH_STAGE_A ? (const void *)c->dAh
                      : stage == MFH_STAGE_B ? (const void *)c->dBh : (const void *)c->dC5;
    MFH_HIP(hipMemcpyAsync(out, src, bytes, hipMemcpyDeviceToHost, c->stream));
    MFH_HIP(hipStreamSynchronize(c->stream));
    return MFH_OK;
}

namespace {
int fpx_mm_host(mfh_ctx *c, int f64, const void *A, const void *B, int SA, int SB, void *C)
{
    if (!c || !A || !B || !C) return MFH_E_ARG;
    if (!conv_size_ok(c)) return MFH_E_BOUND;
    const size_t nn = (size_t)c->n * c->n, eb = f64 ? 8 : 4;
    int rc = ensure_staging(c, nn * eb, nn * eb);
    if (rc) return rc;
    MFH_HIP(hipMemcpyAsync(c->dInA, A, nn * eb, hipMemcpyHostToDevice, c->stream));
    MFH_HIP(hipMemcpyAsync(c->dInB, B, nn * eb, hipMemcpyHostToDevice, c->stream));
    if ((rc = fpx_mm_dev(c, f64, c->dInA, c->dInB, SA, SB, c->dOut))) return rc;
    MFH_HIP(hipMemcpyAsync(C, c->dOut, nn * eb, hipMemcpyDeviceToHost, c->stream));
    MFH_HIP(hipStreamSynchronize(c->stream));
    return MFH_OK;
}
}  // namespace

int mfh_fpx_mm(mfh_ctx *c, const float *A, const float *B, int SA, int SB, float *C)
{
    return fpx_mm_host(c, 0, A, B, SA, SB, C);
}

int mfh_fpx_mm_f64(mfh_ctx *c, const double *A, const double *B, int SA, int SB, double *C)
{
    return fpx_mm_host(c, 1, A, B, SA, SB, C);
}

int mfh_malloc(void **p, size_t bytes)
{
    if (!p) return MFH_E_ARG;
    int rc = check_device();
    if (rc) return rc;
    if (hipMalloc(p, bytes) != hipSuccess) { *p = nullptr; return MFH_E_NOMEM; }
    return MFH_OK;
}

int mfh_free(void *p)
{
    MFH_HIP(hipFree(p));
    return MFH_OK;
}

int mfh_h2d(void *dst, const void *src, size_t bytes)
{
    MFH_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return MFH_OK;
}

int mfh_d2h(void *dst, const void *src, size_t bytes)
{
    MFH_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return MFH_OK;
}

int mfh_sync(mfh_ctx *c)
{
    if (c) MFH_HIP(hipStreamSynchronize(c->stream));
    else MFH_HIP(hipDeviceSynchronize());
    return MFH_OK;
}

int mfh_rand_u16_dev(mfh_ctx *c, void *dM, int n, int L, uint64_t seed)
{
    if (!dM || n < 1 || L < 1) return MFH_E_ARG;
    return mfh_launch_rand_u16(dM, (size_t)L * n * n, seed, c ? c->stream : 0);
}

int mfh_rand_f32_dev(mfh_ctx *c, void *dX, size_t count, uint64_t seed, int emin, int emax)
{
    if (!dX) return MFH_E_ARG;
    return mfh_launch_rand_f32(dX, count, seed, emin, emax, c ? c->stream : 0);
}

int mfh_copy_dev(mfh_ctx *c, void *dst, const void *src, size_t bytes)
{
    if (!dst || !src || bytes % 16 || ((uintptr_t)dst | (uintptr_t)src) % 16)
        return MFH_E_ARG;
    if (!bytes) return MFH_OK;
    return mfh_launch_copy16(dst, src, bytes, c ? c->stream : 0);
}

int mfh_set_timing(mfh_ctx *c, int enable)
{
    if (!c) return MFH_E_ARG;
    c->timing = enable ? 1 : 0;
    return MFH_OK;
}

int mfh_stage_times(const mfh_ctx *c, float ms[5])
{
    if (!c || !ms) return MFH_E_ARG;
    MFH_HIP(hipEventSynchronize(c->ev[4]));
    // transforms in: B's (up to band 0) and every band's A; each band's
    // pointwise and inverse; carry/decode after the last band
    float t = 0;
    MFH_HIP(hipEventElapsedTime(&ms[0], c->ev[0], c->bev[0][0]));
    ms[1] = ms[2] = 0;
    for (int b = 0; b < c->nbands; ++b)
        for (int k = 0; k < 3; ++k) {
            MFH_HIP(hipEventElapsedTime(&t, c->bev[b][k], c->bev[b][k + 1]));
            ms[k] += t;
        }
    MFH_HIP(hipEventElapsedTime(&ms[3], c->bev[c->nbands - 1][3], c->ev[4]));
    MFH_HIP(hipEventElapsedTime(&ms[4], c->ev[0], c->ev[4]));
    return MFH_OK;
}

int mfh_pointwise_info(const mfh_ctx *c, int *ring, int *digit)
{
    if (!c) return MFH_E_ARG;
    if (ring) *ring = c->pwr == MFH_PW_GAUSS ? 3 * (c->K / 2) * (c->K / 2) : c->K * c->K;
    if (digit) *digit = c->mode == MFH_MODE_K7 ? 6 : 9;
    return MFH_OK;
}

int mfh_work(const mfh_ctx *c, double *ops, double *fwd, double *inv)
{
    if (!c) return MFH_E_ARG;
    const double nnp = (double)c->np * c->np, nn = (double)c->n * c->n;
    const double pts = (double)c->NB * c->K;
    const double products = c->mode == MFH_MODE_K7 ? 6.0 : 9.0;
    // ring products issued per point: K^2, or 3 (K/2)^2 with the Gauss split
    const double ring = c->pwr == MFH_PW_GAUSS ? 0.75 * c->K * c->K : (double)c->K * c->K;
    const double slots = (double)c->NB * mfh_slots(c->K, c->pwr);
    if (ops) *ops = 2.0 * products * c->NB * ring * nnp * c->np;
    if (fwd) *fwd = 2.0 * ((double)c->L * nn * 2.0 + slots * mfh_planes(c->mode) * nnp);
    if (inv) {
        // class results in; then the int64 coefficient planes (written, and
        // read back by the carry or decode) unless the carry ran inside the
        // inverse; then the product's output
        const double cw = (2.0 * c->L - 1.0) * nn * 8.0;
        double b = pts * nnp * 4.0 * mfh_nclasses(c->mode);
        if (c->last_out == 1) b += cw;
        else {
            if (!c->last_fused) b += 2.0 * cw;
            b += c->last_out == 2 ? nn * 4.0 : c->last_out == 3 ? nn * 8.0
                                                 : (double)c->last_RL * nn * 2.0;
        }
        *inv = b;
    }
    return MFH_OK;
}

}  // extern "C"

// standalone helpers: a throw-away context carrying only sizes and the null
// stream, with temporary device buffers
namespace {
struct TmpBufs {
    void *p[3] = {nullptr, nullptr, nullptr};
    ~TmpBufs() { for (void *q : p) if (q) (void)hipFree(q); }
};
void bare_ctx(mfh_ctx &c, int n, int L)
{
    memset(&c, 0, sizeof c);
    c.n = n; c.np = n; c.L = L; c.stream = 0;
}
}  // namespace

extern "C" {

int mfh_normalize(const int64_t *acc, int nplanes, int n, uint16_t *out, int RL)
{
    if (!acc || !out || n < 1 || nplanes < 0 || RL < 1) return MFH_E_ARG;
    int rc = check_device();
    if (rc) return rc;
    const size_t nn = (size_t)n * n;
    TmpBufs t;
    if (hipMalloc(&t.p[0], (size_t)(nplanes ? nplanes : 1) * nn * 8) != hipSuccess ||
        hipMalloc(&t.p[1], (size_t)RL * nn * 2) != hipSuccess)
        return MFH_E_NOMEM;
    MFH_HIP(hipMemcpy(t.p[0], acc, (size_t)nplanes * nn * 8, hipMemcpyHostToDevice));
    if ((rc = mfh_launch_carry_planes((const int64_t *)t.p[0], nplanes, nn,
                                      (uint16_t *)t.p[1], RL, 0)))
        return rc;
    MFH_HIP(hipMemcpy(out, t.p[1], (size_t)RL * nn * 2, hipMemcpyDeviceToHost));
    return MFH_OK;
}

namespace {
int encode_host(const void *X, int f64, int n, int L, int S, int32_t *X32)
{
    if (!X || !X32 || n < 1 || L < 1) return MFH_E_ARG;
    int rc = check_device();
    if (rc) return rc;
    const size_t nn = (size_t)n * n, eb = f64 ? 8 : 4;
    TmpBufs t;
    if (hipMalloc(&t.p[0], nn * eb) != hipSuccess ||
        hipMalloc(&t.p[1], (size_t)L * nn * 4) != hipSuccess)
        return MFH_E_NOMEM;
    MFH_HIP(hipMemcpy(t.p[0], X, nn * eb, hipMemcpyHostToDevice));
    if ((rc = mfh_launch_encode(t.p[0], f64, n, L, S, (int32_t *)t.p[1], 0))) return rc;
    MFH_HIP(hipMemcpy(X32, t.p[1], (size_t)L * nn * 4, hipMemcpyDeviceToHost));
    return MFH_OK;
}

// decode of host coefficient planes; out gets nn values of `out_bytes` each
// (SIG63: int64 significands, exponents to out2)
int decode_host(const int64_t *Cw, int n, int L, int SAB, int fmt, void *out,
                size_t out_bytes, int32_t *out2)
{
    if (!Cw || !out || n < 1 || L < 1) return MFH_E_ARG;
    int rc = check_device();
    if (rc) return rc;
    const size_t nn = (size_t)n * n;
    TmpBufs t;
    if (hipMalloc(&t.p[0], (size_t)(2 * L - 1) * nn * 8) != hipSuccess ||
        hipMalloc(&t.p[1], nn * out_bytes) != hipSuccess ||
        (out2 && hipMalloc(&t.p[2], nn * 4) != hipSuccess))
        return MFH_E_NOMEM;
    MFH_HIP(hipMemcpy(t.p[0], Cw, (size_t)(2 * L - 1) * nn * 8, hipMemcpyHostToDevice));
    mfh_ctx c;
    bare_ctx(c, n, L);
    if ((rc = mfh_launch_decode(&c, (const int64_t *)t.p[0], SAB, fmt, t.p[1],
                                (int32_t *)t.p[2])))
        return rc;
    MFH_HIP(hipDeviceSynchronize());
    MFH_HIP(hipMemcpy(out, t.p[1], nn * out_bytes, hipMemcpyDeviceToHost));
    if (out2) MFH_HIP(hipMemcpy(out2, t.p[2], nn * 4, hipMemcpyDeviceToHost));
    return MFH_OK;
}
}  // namespace

int mfh_mm_accum(int64_t *C, const int32_t *A, const int32_t *B, int n, int sign)
{
    if (!C || !A || !B || n < 1) return MFH_E_ARG;
    int rc = check_device();
    if (rc) return rc;
    const size_t nn = (size_t)n * n;
    TmpBufs t;
    if (hipMalloc(&t.p[0], nn * 8) != hipSuccess || hipMalloc(&t.p[1], nn * 4) != hipSuccess ||
        hipMalloc(&t.p[2], nn * 4) != hipSuccess)
        return MFH_E_NOMEM;
    MFH_HIP(hipMemcpy(t.p[0], C, nn * 8, hipMemcpyHostToDevice));
    MFH_HIP(hipMemcpy(t.p[1], A, nn * 4, hipMemcpyHostToDevice));
    MFH_HIP(hipMemcpy(t.p[2], B, nn * 4, hipMemcpyHostToDevice));
    if ((rc = mfh_launch_mm_accum((int64_t *)t.p[0], (const int32_t *)t.p[1],
                                  (const int32_t *)t.p[2], n, sign, 0)))
        return rc;
    MFH_HIP(hipDeviceSynchronize());
    MFH_HIP(hipMemcpy(C, t.p[0], nn * 8, hipMemcpyDeviceToHost));
    return MFH_OK;
}

int mfh_mm_accum_dev(mfh_ctx *c, void *dC, const void *dA, const void *dB, int n, int sign)
{
    if (!dC || !dA || !dB || n < 1) return MFH_E_ARG;
    return mfh_launch_mm_accum((int64_t *)dC, (const int32_t *)dA, (const int32_t *)dB, n, sign,
                               c ? c->stream : 0);
}

int mfh_limbplane_conv_dev(mfh_ctx *c, int in_kind, const void *dA, const void *dB, int n,
                           int L, void *dCw)
{
    if (!dA || !dB || !dCw || n < 1 || L < 1) return MFH_E_ARG;
    return mfh_launch_conv_limbplane((int64_t *)dCw, dA, dB, in_kind, n, L, c ? c->stream : 0);
}

int mfh_limbplane_mm_dev(mfh_ctx *c, int in_kind, const void *dA, const void *dB, int n, int L,
                         void *dCw, void *dOut, int RL)
{
    if (!dOut || RL < 1) return MFH_E_ARG;
    if (in_kind != MFH_IN_U16 && in_kind != MFH_IN_U16_SIGNED) return MFH_E_ARG;
    int rc = mfh_limbplane_conv_dev(c, in_kind, dA, dB, n, L, dCw);
    if (rc) return rc;
    return mfh_launch_carry_planes((const int64_t *)dCw, 2 * L - 1, (size_t)n * n,
                                   (uint16_t *)dOut, RL, c ? c->stream : 0);
}

// ---- the limb-plane schoolbook on the matrix cores -------------------------
namespace {
struct SbLayout {
    int np, NU;
    size_t bt, digits, partials;     // bytes: B^T limbs, one operand's digits, P
    long long lo;                    // lower end of every partial's range
};
// Every partial sums at most 16 NU digit products per k over n values of k,
// each in [-128 * 127, 128 * 128]: its range has width 16 NU n 32640, which
// must stay below 2^32 for the int32 residue to determine it.
int sb_layout(int n, int L, SbLayout &s)
{
    if (n < 1 || L < 1) return MFH_E_ARG;
    s.np = (n + MFH_KBLK - 1) / MFH_KBLK * MFH_KBLK;
    s.NU = (L + 15) / 16;
    const long long terms = 16LL * s.NU * n;
    if (terms * 32640 >= (1LL << 32)) return MFH_E_BOUND;
    s.lo = -terms * 16256;
    const size_t plane = (size_t)s.np * s.np;
    s.bt = ((size_t)L * n * n * 2 + 255) / 256 * 256;
    s.digits = (size_t)16 * s.NU * 6 * plane;
    s.partials = (size_t)6 * (2 * s.NU - 1) * plane * 32 * 4;
    return MFH_OK;
}
}  // namespace

int mfh_schoolbook_workspace(int n, int L, size_t *bytes)
{
    SbLayout s;
    if (!bytes) return MFH_E_ARG;
    const int rc = sb_layout(n, L, s);
    if (rc) return rc;
    *bytes = s.bt + 2 * s.digits + s.partials;
    return MFH_OK;
}

int mfh_schoolbook_dev(mfh_ctx *c, int in_kind, const void *dA, const void *dB, int n, int L,
                       void *dWork, size_t work_bytes, void *dOut, int RL)
{
    SbLayout s;
    if (!dA || !dB || !dWork || !dOut || RL < 0) return MFH_E_ARG;
    if (in_kind != MFH_IN_U16 && in_kind != MFH_IN_U16_SIGNED) return MFH_E_ARG;
    int rc = sb_layout(n, L, s);
    if (rc) return rc;
    if (work_bytes < s.bt + 2 * s.digits + s.partials) return MFH_E_ARG;
    hipStream_t st = c ? c->stream : 0;
    char *w = (char *)dWork;
    void *bt = w;
    int8_t *ad = (int8_t *)(w + s.bt), *bd = ad + s.digits;
    int32_t *P = (int32_t *)(bd + s.digits);
    if ((rc = mfh_launch_transpose(dB, bt, L, n, 2, st)) ||
        (rc = mfh_launch_sb_digits(dA, in_kind, ad, n, s.np, L, 16 * s.NU, st)) ||
        (rc = mfh_launch_sb_digits(bt, in_kind, bd, n, s.np, L, 16 * s.NU, st)) ||
        (rc = mfh_launch_schoolbook(ad, bd, P, s.np, s.NU, st)))
        return rc;
    return RL ? mfh_launch_sb_combine(P, nullptr, (uint16_t *)dOut, RL, n, s.np, L, s.NU, s.lo, st)
              : mfh_launch_sb_combine(P, (int64_t *)dOut, nullptr, 0, n, s.np, L, s.NU, s.lo, st);
}

int mfh_schoolbook(int in_kind, const uint16_t *A, const uint16_t *B, int n, int L, void *out,
                   int RL)
{
    if (!A || !B || !out || RL < 0) return MFH_E_ARG;
    size_t work = 0;
    int rc = mfh_schoolbook_workspace(n, L, &work);
    if (rc) return rc;
    if ((rc = check_device())) return rc;
    const size_t nn = (size_t)n * n, in_b = (size_t)L * nn * 2;
    const size_t out_b = RL ? (size_t)RL * nn * 2 : (size_t)(2 * L - 1) * nn * 8;
    TmpBufs t;
    if (hipMalloc(&t.p[0], 2 * in_b) != hipSuccess || hipMalloc(&t.p[1], work) != hipSuccess ||
        hipMalloc(&t.p[2], out_b) != hipSuccess) {
        (void)hipGetLastError();     // a caller may go on to a smaller method
        return MFH_E_NOMEM;
    }
    uint16_t *dA = (uint16_t *)t.p[0], *dB = dA + (size_t)L * nn;
    MFH_HIP(hipMemcpy(dA, A, in_b, hipMemcpyHostToDevice));
    MFH_HIP(hipMemcpy(dB, B, in_b, hipMemcpyHostToDevice));
    if ((rc = mfh_schoolbook_dev(nullptr, in_kind, dA, dB, n, L, t.p[1], work, t.p[2], RL)))
        return rc;
    MFH_HIP(hipDeviceSynchronize());
    MFH_HIP(hipMemcpy(out, t.p[2], out_b, hipMemcpyDeviceToHost));
    return MFH_OK;
}

namespace {
// conv_limbplane / mm_limbplane on host buffers: limb planes in, the 2L-1
// coefficient planes (out == nullptr) or RL carried limbs out
int limbplane_host(int in_kind, const void *A, const void *B, int n, int L, int64_t *Cw,
                   uint16_t *out, int RL)
{
    if (!A || !B || n < 1 || L < 1 || (!Cw && (!out || RL < 1))) return MFH_E_ARG;
    int rc = check_device();
    if (rc) return rc;
    const size_t nn = (size_t)n * n, eb = in_kind == MFH_IN_U16 ? 2 : 4;
    const size_t cw_b = (size_t)(2 * L - 1) * nn * 8;
    TmpBufs t;
    void *dOut = nullptr;
    if (hipMalloc(&t.p[0], (size_t)L * nn * eb) != hipSuccess ||
        hipMalloc(&t.p[1], (size_t)L * nn * eb) != hipSuccess ||
        hipMalloc(&t.p[2], cw_b + (out ? (size_t)RL * nn * 2 : 0)) != hipSuccess)
        return MFH_E_NOMEM;
    if (out) dOut = (char *)t.p[2] + cw_b;
    MFH_HIP(hipMemcpy(t.p[0], A, (size_t)L * nn * eb, hipMemcpyHostToDevice));
    MFH_HIP(hipMemcpy(t.p[1], B, (size_t)L * nn * eb, hipMemcpyHostToDevice));
    rc = out ? mfh_limbplane_mm_dev(nullptr, in_kind, t.p[0], t.p[1], n, L, t.p[2], dOut, RL)
             : mfh_limbplane_conv_dev(nullptr, in_kind, t.p[0], t.p[1], n, L, t.p[2]);
    if (rc) return rc;
    MFH_HIP(hipDeviceSynchronize());
    if (out) MFH_HIP(hipMemcpy(out, dOut, (size_t)RL * nn * 2, hipMemcpyDeviceToHost));
    else MFH_HIP(hipMemcpy(Cw, t.p[2], cw_b, hipMemcpyDeviceToHost));
    return MFH_OK;
}
}  // namespace

int mfh_limbplane_conv(const int32_t *A32, const int32_t *B32, int n, int L, int64_t *Cw)
{
    if (!Cw) return MFH_E_ARG;
    return limbplane_host(MFH_IN_I32, A32, B32, n, L, Cw, nullptr, 0);
}

int mfh_limbplane_mm(const uint16_t *A, const uint16_t *B, int n, int L, uint16_t *out, int RL)
{
    if (!out) return MFH_E_ARG;
    return limbplane_host(MFH_IN_U16, A, B, n, L, nullptr, out, RL);
}

int mfh_bigint_mm(const uint16_t *Aem, const uint16_t *Bem, int n, int L, uint16_t *out, int RL)
{
    if (!Aem || !Bem || !out || n < 1 || L < 1 || RL < 1) return MFH_E_ARG;
    int rc = check_device();
    if (rc) return rc;
    const size_t nn = (size_t)n * n, in_b = (size_t)L * nn * 2;
    const size_t cw_b = (size_t)(2 * L - 1) * nn * 8, out_b = (size_t)RL * nn * 2;
    TmpBufs t;
    if (hipMalloc(&t.p[0], 2 * in_b) != hipSuccess ||
        hipMalloc(&t.p[1], 2 * in_b) != hipSuccess ||
        hipMalloc(&t.p[2], cw_b + out_b) != hipSuccess)
        return MFH_E_NOMEM;
    uint16_t *eA = (uint16_t *)t.p[0], *eB = eA + (size_t)L * nn;
    uint16_t *pA = (uint16_t *)t.p[1], *pB = pA + (size_t)L * nn;
    void *dOut = (char *)t.p[2] + cw_b;
    MFH_HIP(hipMemcpy(eA, Aem, in_b, hipMemcpyHostToDevice));
    MFH_HIP(hipMemcpy(eB, Bem, in_b, hipMemcpyHostToDevice));
    if ((rc = mfh_launch_entry_to_plane(eA, pA, n, L, 0))) return rc;
    if ((rc = mfh_launch_entry_to_plane(eB, pB, n, L, 0))) return rc;
    if ((rc = mfh_limbplane_mm_dev(nullptr, MFH_IN_U16, pA, pB, n, L, t.p[2], dOut, RL)))
        return rc;
    MFH_HIP(hipDeviceSynchronize());
    MFH_HIP(hipMemcpy(out, dOut, out_b, hipMemcpyDeviceToHost));
    return MFH_OK;
}

int mfh_negconv(const int32_t *A, const int32_t *B, int K, int n, int64_t *C)
{
    if (!A || !B || !C || n < 1 || K < 1) return MFH_E_ARG;
    int rc = check_device();
    if (rc) return rc;
    const size_t nn = (size_t)n * n;
    TmpBufs t;
    if (hipMalloc(&t.p[0], (size_t)K * nn * 4) != hipSuccess ||
        hipMalloc(&t.p[1], (size_t)K * nn * 4) != hipSuccess ||
        hipMalloc(&t.p[2], (size_t)(3 * K - 1) * nn * 8) != hipSuccess)
        return MFH_E_NOMEM;
    int64_t *lin = (int64_t *)t.p[2], *dC = lin + (size_t)(2 * K - 1) * nn;
    MFH_HIP(hipMemcpy(t.p[0], A, (size_t)K * nn * 4, hipMemcpyHostToDevice));
    MFH_HIP(hipMemcpy(t.p[1], B, (size_t)K * nn * 4, hipMemcpyHostToDevice));
    if ((rc = mfh_launch_conv_limbplane(lin, t.p[0], t.p[1], MFH_IN_I32, n, K, 0))) return rc;
    if ((rc = mfh_launch_negfold(lin, dC, n, K, 0))) return rc;
    MFH_HIP(hipDeviceSynchronize());
    MFH_HIP(hipMemcpy(C, dC, (size_t)K * nn * 8, hipMemcpyDeviceToHost));
    return MFH_OK;
}

int mfh_fpx_faithful(const int32_t *Aw, const int32_t *Bw, int n, int L, int u0, int Lk,
                     const mfh_plan *plan, int SAB, int f64, void *C)
{
    if (!Aw || !Bw || !C || n < 1 || L < 1 || Lk < 1 || u0 < 0 || u0 + Lk > L)
        return MFH_E_ARG;
    if (Lk > 1 && (!plan || plan->L != Lk)) return MFH_E_ARG;
    int rc = check_device();
    if (rc) return rc;
    const size_t nn = (size_t)n * n, eb = f64 ? 8 : 4;
    const size_t cw_b = (size_t)(2 * L - 1) * nn * 8;
    TmpBufs t;
    if (hipMalloc(&t.p[0], 2 * (size_t)Lk * nn * 4) != hipSuccess ||
        hipMalloc(&t.p[1], cw_b) != hipSuccess || hipMalloc(&t.p[2], nn * eb) != hipSuccess)
        return MFH_E_NOMEM;
    int32_t *dA = (int32_t *)t.p[0], *dB = dA + (size_t)Lk * nn;
    int64_t *dCw = (int64_t *)t.p[1], *dWin = dCw + (size_t)(2 * u0) * nn;
    MFH_HIP(hipMemcpy(dA, Aw, (size_t)Lk * nn * 4, hipMemcpyHostToDevice));
    MFH_HIP(hipMemcpy(dB, Bw, (size_t)Lk * nn * 4, hipMemcpyHostToDevice));
    MFH_HIP(hipMemset(dCw, 0, cw_b));
    if (Lk == 1) {
        // the top planes' product, one leaf GEMM (src/mlgemm.c:1195-1197)
        if ((rc = mfh_launch_mm_accum(dWin, dA, dB, n, 1, 0))) return rc;
        MFH_HIP(hipDeviceSynchronize());
    } else {
        // the window's 2Lk-1 coefficient planes written in place at 2 u0
        mfh_ctx *c = nullptr;
        if ((rc = mfh_create(&c, n, Lk, plan))) return rc;
        rc = mfh_conv_dev(c, dA, dB, dWin);
        if (!rc) rc = mfh_sync(c);
        mfh_destroy(c);
        if (rc) return rc;
    }
    mfh_ctx bare;
    bare_ctx(bare, n, L);
    if ((rc = mfh_launch_decode(&bare, dCw, SAB, f64 ? MFH_DEC_F64 : MFH_DEC_F32, t.p[2],
                                nullptr)))
        return rc;
    MFH_HIP(hipDeviceSynchronize());
    MFH_HIP(hipMemcpy(C, t.p[2], nn * eb, hipMemcpyDeviceToHost));
    return MFH_OK;
}

int mfh_fpx_encode(const float *X, int n, int L, int S, int32_t *X32)
{
    return encode_host(X, 0, n, L, S, X32);
}

int mfh_fpx_encode_f64(const double *X, int n, int L, int S, int32_t *X32)
{
    return encode_host(X, 1, n, L, S, X32);
}

int mfh_fpx_decode(const int64_t *Cw, int n, int L, int SAB, float *C)
{
    return decode_host(Cw, n, L, SAB, MFH_DEC_F32, C, 4, nullptr);
}

int mfh_fpx_decode_f64(const int64_t *Cw, int n, int L, int SAB, double *C)
{
    return decode_host(Cw, n, L, SAB, MFH_DEC_F64, C, 8, nullptr);
}

int mfh_fpx_decode_sig63(const int64_t *Cw, int n, int L, int SAB, int64_t *sig, int32_t *ex)
{
    if (!ex) return MFH_E_ARG;
    return decode_host(Cw, n, L, SAB, MFH_DEC_SIG63, sig, 8, ex);
}

int mfh_fpx_decode_ld(const int64_t *Cw, int n, int L, int SAB, long double *C)
{
    if (!C || n < 1) return MFH_E_ARG;
    const size_t nn = (size_t)n * n;
    int64_t *sig = (int64_t *)malloc(nn * 8);
    int32_t *ex = (int32_t *)malloc(nn * 4);
    int rc = (sig && ex) ? mfh_fpx_decode_sig63(Cw, n, L, SAB, sig, ex) : MFH_E_NOMEM;
    // the significand has at most 63 bits and the scale stays far inside
    // the long double exponent range, so this conversion is exact
    if (!rc)
        for (size_t i = 0; i < nn; ++i) C[i] = sig[i] ? ldexpl((long double)sig[i], ex[i]) : 0.0L;
    free(sig);
    free(ex);
    return rc;
}

}  // extern "C"
