"""GPU parity of every entry point, through the C-ABI: conv_mfft on signed
limbs, two's complement products, the fp32 and fp64 embeddings and the long
double decode, device normalize /
encode / decode, the device input generator, the generic (runtime-plan)
kernels, and the full-size workloads checked by Freivalds' test plus exact
sampled entries."""
import ctypes as C
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SEED, SEED_B = 12345, 12345 ^ 0xABCDEF


def signed_limbs(orc, n, L, seed):
    A = orc.bigmat_rand(n, L, seed)
    top = slice((L - 1) * n * n, L * n * n)
    A32 = A.astype(np.int32)
    A32[top] = A[top].view(np.int16)
    return A, A32


# ---- conv_mfft: the convolution of the caller's limbs --------------------------
@pytest.mark.parametrize("n,L,sigma", [(6, 8, 0), (16, 32, 0), (9, 32, 3), (40, 64, 0),
                                       (24, 128, 0), (5, 512, 0)])
def test_conv_signed_limbs(gpu, orc, n, L, sigma):
    print(f"[conv] n={n} L={L}", flush=True)
    rng = np.random.default_rng(n * L)
    A = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    B = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    A[:n * n] = 65535                                   # worst-case magnitudes
    B[:n * n] = -65535
    want = orc.conv_limbplane(A, B, n, L)
    with gpu.Ctx(n, L, gpu.plan(L, sigma)) as ctx:
        got = ctx.conv(A, B)
    assert np.array_equal(got, want)


def test_conv_rejects_out_of_range_limb(gpu):
    n, L = 8, 16
    A = np.zeros(L * n * n, np.int32)
    A[5] = 65536
    with gpu.Ctx(n, L) as ctx:
        with pytest.raises(gpu.MfftError) as e:
            ctx.conv(A, A)
    assert e.value.code == -5


def test_mm_dev_rejects_unaligned_limbs(gpu, lib):
    """mfh_mm_dev reads limbs 8 at a time: a device pointer that is not
    16-byte aligned is refused before any kernel runs."""
    n, L = 8, 16
    with gpu.Ctx(n, L) as ctx:
        dA = gpu.DevBuf(L * n * n * 2 + 16)
        dO = gpu.DevBuf((2 * L + 1) * n * n * 2)
        off = C.c_void_p(dA.ptr.value + 2)
        rc = lib.mfh_mm_dev(ctx.h, 0, off, dA.ptr, dO.ptr, 2 * L + 1)
        for b in (dA, dO):
            b.free()
    assert rc == -3                      # MFH_E_ARG


def test_c_api_conv_mfft(gpu, orc):
    n, L = 12, 32
    rng = np.random.default_rng(1)
    A = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    B = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    cw, err = gpu.conv_mfft(A, B, n, L, gpu.plan(L))
    assert err == 0
    assert np.array_equal(cw, orc.conv_limbplane(A, B, n, L))


# ---- exact track -------------------------------------------------------------------
@pytest.mark.parametrize("case", range(13))
def test_products_fixture(gpu, orc, case):
    with open(os.path.join(GOLD, "products.json")) as f:
        c = json.load(f)[case]
    n, L, RL = c["n"], c["L"], c["RL"]
    A = orc.bigmat_rand(n, L, c["seed_a"])
    B = orc.bigmat_rand(n, L, c["seed_b"])
    with gpu.Ctx(n, L) as ctx:
        got = ctx.mm(A, B, RL, signed=c["signed"])
    assert np.array_equal(got, np.array(c["out"], dtype=np.uint16))


@pytest.mark.parametrize("n,L", [(8, 32), (48, 32), (24, 128), (10, 64), (7, 16), (16, 512)])
def test_signed_entries(gpu, orc, n, L):
    """Two's complement W-bit entries (top limb int16)."""
    A, A32 = signed_limbs(orc, n, L, SEED + 7)
    B, B32 = signed_limbs(orc, n, L, SEED_B + 7)
    RL = 2 * L + 1
    want = orc.normalize(orc.conv_limbplane(A32, B32, n, L), 2 * L - 1, n, RL)
    with gpu.Ctx(n, L) as ctx:
        got = ctx.mm(A, B, RL, signed=True)
    assert np.array_equal(got, want)
    out, err = gpu.mm_mfft(A, B, n, L, gpu.plan(L), signed=True)
    assert err == 0 and np.array_equal(out, want)


@pytest.mark.parametrize("L,RL", [(64, 1), (64, 5), (64, 64), (64, 129), (32, 3), (32, 70),
                                  (128, 2), (128, 100), (128, 262), (256, 3), (256, 300),
                                  (256, 515), (512, 1), (512, 37), (512, 1030)])
def test_short_and_long_outputs(gpu, orc, L, RL):
    """RL below 2L+1 truncates mod 2^(16 RL), above it zero-extends
    (src/bigmat.c:48-60); every ring size, so every fused-carry layout."""
    n = 16
    A = orc.bigmat_rand(n, L, 3)
    B = orc.bigmat_rand(n, L, 4)
    want = orc.normalize(orc.conv_limbplane(A.astype(np.int32), B.astype(np.int32), n, L),
                         2 * L - 1, n, RL)
    with gpu.Ctx(n, L) as ctx:
        assert np.array_equal(ctx.mm(A, B, RL), want)


def test_all_ones_worst_case(gpu, orc):
    """Every limb 0xFFFF: largest transformed values, longest carries."""
    for n, L in [(64, 128), (16, 64), (32, 32), (16, 512), (16, 256)]:
        A = np.full(L * n * n, 0xFFFF, np.uint16)
        RL = 2 * L + 1
        want = orc.mm_limbplane(A, A, n, L, RL)
        with gpu.Ctx(n, L) as ctx:
            assert np.array_equal(ctx.mm(A, A, RL), want), (n, L)


@pytest.mark.parametrize("n,L", [(16, 512), (8, 512), (24, 512)])
def test_offset_mode_extremes(gpu, orc, n, L):
    """8192-bit unsigned products run shifted by -2^(W-1) (the top limb read
    as (int16)(x ^ 0x8000)) with the shift's terms added back in the carry;
    entries at the shift's edges: 0, 2^(W-1) - 1, 2^(W-1), 2^W - 1, and
    random, mixed per entry.  Checked against the schoolbook oracle, and the
    two's complement products of the same limbs too."""
    rng = np.random.default_rng(n * L + 1)
    nn = n * n

    def pick(seed):
        A = orc.bigmat_rand(n, L, seed).reshape(L, nn)
        kind = rng.integers(0, 5, nn)
        A[:, kind == 0] = 0
        A[:, kind == 1] = 0xFFFF
        A[:, kind == 1] = 0xFFFF
        A[:L - 1, kind == 2] = 0xFFFF                     # 2^(W-1) - 1
        A[L - 1, kind == 2] = 0x7FFF
        A[:L - 1, kind == 3] = 0                          # 2^(W-1)
        A[L - 1, kind == 3] = 0x8000
        return A.reshape(-1).copy()

    A, B = pick(SEED), pick(SEED_B)
    RL = 2 * L + 1
    with gpu.Ctx(n, L) as ctx:
        got = ctx.mm(A, B, RL)
        got_s = ctx.mm(A, B, RL, signed=True)
    assert np.array_equal(got, orc.mm_limbplane(A, B, n, L, RL))
    A32, B32 = A.astype(np.int32), B.astype(np.int32)
    A32[(L - 1) * nn:] = A[(L - 1) * nn:].view(np.int16)
    B32[(L - 1) * nn:] = B[(L - 1) * nn:].view(np.int16)
    want_s = orc.normalize(orc.conv_limbplane(A32, B32, n, L), 2 * L - 1, n, RL)
    assert np.array_equal(got_s, want_s)


def test_carry_runs_of_ones_and_zeros(gpu):
    """Products whose limbs are long runs of 0xFFFF or 0x0000: the carry
    chains cross every carry-lookahead run boundary, in both directions.
    (-1)(1) summed over n is -n; (-1)(-1) is +n; (2^W - 1)(1) unsigned is
    n (2^W - 1).  Closed forms, so no oracle is needed."""
    for n, L in [(64, 128), (16, 64), (32, 32), (16, 512)]:
        RL = 2 * L + 1
        ones = np.full(L * n * n, 0xFFFF, np.uint16)             # -1 signed, 2^W-1 unsigned
        one = np.zeros(L * n * n, np.uint16)
        one[:n * n] = 1                                            # every entry 1
        mod = 1 << (16 * RL)
        cases = [(ones, one, True, (-n) % mod), (ones, ones, True, n),
                 (ones, one, False, n * ((1 << (16 * L)) - 1))]
        with gpu.Ctx(n, L) as ctx:
            for A, B, sgn, val in cases:
                got = ctx.mm(A, B, RL, signed=sgn).reshape(RL, n * n)
                want = np.array([(val >> (16 * w)) & 0xFFFF for w in range(RL)], np.uint16)
                assert np.array_equal(got, np.repeat(want[:, None], n * n, axis=1)), (n, L, sgn)


def test_generic_kernels_match(gpu, orc, monkeypatch):
    """The runtime-plan (generic) kernels, forced, give the same bits."""
    monkeypatch.setenv("MFH_GENERIC_KERNELS", "1")
    for n, L in [(64, 128), (40, 64), (96, 32)]:
        A = orc.bigmat_rand(n, L, SEED)
        B = orc.bigmat_rand(n, L, SEED_B)
        RL = 2 * L + 1
        want = orc.mm_mfft(A, B, n, L, orc.plan(L), RL)
        with gpu.Ctx(n, L) as ctx:
            assert np.array_equal(ctx.mm(A, B, RL), want), (n, L)


def test_fused_decode_matches_separate_decode(gpu, orc, monkeypatch):
    """fp32 and fp64 products: the specialised inverse kernels decode each
    element from their planes in LDS, the generic kernels write the int64
    planes and decode them in a separate pass; both give the same bits
    (n = 45: a ragged last workgroup in both)."""
    n = 45
    X = orc.fp32_rand(n * n, SEED, -30, 30)
    Y = orc.fp32_rand(n * n, SEED_B, -30, 30)
    rng = np.random.default_rng(11)
    Xd = rng.standard_normal(n * n) * np.exp2(rng.integers(-40, 40, n * n))
    Yd = rng.standard_normal(n * n) * np.exp2(rng.integers(-40, 40, n * n))
    res = []
    for generic in (False, True):
        if generic:
            monkeypatch.setenv("MFH_GENERIC_KERNELS", "1")
        with gpu.Ctx(n, 32) as ctx:
            f32 = ctx.fpx_mm(X, Y, 256, 256).view(np.uint32)
        with gpu.Ctx(n, 128) as ctx:
            f64 = ctx.fpx_mm_f64(Xd, Yd, 1024, 1024).view(np.uint64)
        res.append((f32, f64))
    assert np.count_nonzero(res[0][0]) > n * n // 2 and np.count_nonzero(res[0][1]) > n * n // 2
    assert np.array_equal(res[0][0], res[1][0])
    assert np.array_equal(res[0][1], res[1][1])


@pytest.mark.parametrize("force", [512, 1024, 2048, 4096, 8192])
def test_fused_decode_every_plan(gpu, orc, monkeypatch, force):
    """The fused fp64 decode of every specialised inverse plan ((NB, K) =
    (16, 8), (16, 16), (32, 16), (32, 32), (64, 32) at grids of 512 .. 8192
    bits), and the fp32 one where the grid takes fp32 entries, bit-equal to
    the generic kernels' separate decode and to the oracle (n = 45: a
    ragged last workgroup)."""
    n = 45
    print(f"[fused decode] force={force}", flush=True)
    rng = np.random.default_rng(force)
    A = np.ldexp(rng.uniform(1, 2, n * n) * rng.choice([-1, 1], n * n),
                 rng.integers(-60, 61, n * n))
    B = np.ldexp(rng.uniform(1, 2, n * n) * rng.choice([-1, 1], n * n),
                 rng.integers(-60, 61, n * n))
    oc = orc.fpx_d(A, B, n, force)
    oa, ob = orc.fpx_planes(oc)
    L, SA, SB = oc.L, oc.SA, oc.SB
    want = orc.fpx_decode_f64_from(oc, orc.conv_mfft(oa, ob, n, L, orc.plan(L)))
    orc.fpx_free(oc)
    X = orc.fp32_rand(n * n, force, -30, 30)
    Y = orc.fp32_rand(n * n, force + 1, -30, 30)
    oc = orc.fpx(X, Y, n, force)
    xa, xb = orc.fpx_planes(oc)
    want32 = orc.fpx_decode_from(oc, orc.conv_mfft(xa, xb, n, L, orc.plan(L)))
    orc.fpx_free(oc)
    for generic in (False, True):
        if generic:
            monkeypatch.setenv("MFH_GENERIC_KERNELS", "1")
        with gpu.Ctx(n, L) as ctx:
            got = ctx.fpx_mm_f64(A, B, SA, SB)
            got32 = ctx.fpx_mm(X, Y, SA, SB)
        assert np.array_equal(got.view(np.uint64), want.view(np.uint64)), generic
        assert np.array_equal(got32.view(np.uint32), want32.view(np.uint32)), generic
    assert np.count_nonzero(want) > n * n // 2


def test_device_generator_matches_host(gpu, orc, lib):
    n, L = 96, 32
    with gpu.Ctx(n, L) as ctx:
        d = gpu.DevBuf(L * n * n * 2)
        gpu.check(lib.mfh_rand_u16_dev(ctx.h, d.ptr, n, L, SEED))
        ctx.sync()
        got = d.download(np.uint16, L * n * n)
        d.free()
    assert np.array_equal(got, orc.bigmat_rand(n, L, SEED))
    x = gpu.DevBuf(4 * 1000)
    gpu.check(lib.mfh_rand_f32_dev(None, x.ptr, 1000, 77, -20, 20))
    gpu.check(lib.mfh_sync(None))
    assert np.array_equal(x.download(np.float32, 1000), orc.fp32_rand(1000, 77, -20, 20))
    x.free()


@pytest.mark.gpu
def test_copy_kernel(gpu, lib):
    nbytes = 3 * (1 << 20) + 4096
    src, dst = gpu.DevBuf(nbytes), gpu.DevBuf(nbytes)
    data = np.random.default_rng(3).integers(0, 256, nbytes, dtype=np.uint8)
    src.upload(data)
    gpu.check(lib.mfh_copy_dev(None, dst.ptr, src.ptr, nbytes))
    gpu.check(lib.mfh_sync(None))
    assert np.array_equal(dst.download(np.uint8, nbytes), data)
    assert lib.mfh_copy_dev(None, dst.ptr, src.ptr, nbytes - 8) == -3   # not a multiple of 16
    src.free()
    dst.free()


def test_device_normalize(gpu, orc):
    with open(os.path.join(GOLD, "normalize.json")) as f:
        for c in json.load(f):
            acc = np.array(c["acc"], dtype=np.int64)
            out, err = gpu.normalize_planes(acc, c["nplanes"], c["n"], c["RL"])
            assert err == 0
            assert np.array_equal(out, np.array(c["out"], dtype=np.uint16))


# ---- fp32 embedding -------------------------------------------------------------------
@pytest.mark.parametrize("case", range(3))
def test_fpx_fixture(gpu, orc, lib, case):
    with open(os.path.join(GOLD, "fpx.json")) as f:
        c = json.load(f)[case]
    n = c["n"]
    A = np.array(c["A_bits"], dtype=np.uint32).view(np.float32)
    B = np.array(c["B_bits"], dtype=np.uint32).view(np.float32)
    want = np.array(c["C_bits"], dtype=np.uint32)
    ctx = gpu.FpxCtx()
    assert lib.fpx_init(C.byref(ctx), A.ctypes.data, B.ctypes.data, n, 512) == 0
    lib.fpx_encode(C.byref(ctx), A.ctypes.data, B.ctypes.data)
    assert lib.mfft_last_error() == 0
    out = np.empty(n * n, np.float32)
    assert lib.fpx_mm_f32(C.byref(ctx), C.byref(gpu.plan(ctx.L)), out.ctypes.data) == 0
    assert np.array_equal(out.view(np.uint32), want)
    # reference-style call sequence: encode -> conv_mfft -> decode
    nn = n * n
    cw = np.ctypeslib.as_array(C.cast(ctx.Cw, C.POINTER(C.c_int64)), shape=((2 * ctx.L - 1) * nn,))
    a32 = np.ctypeslib.as_array(C.cast(ctx.A32, C.POINTER(C.c_int32)), shape=(ctx.L * nn,))
    b32 = np.ctypeslib.as_array(C.cast(ctx.B32, C.POINTER(C.c_int32)), shape=(ctx.L * nn,))
    oc = orc.fpx(A, B, n, 512)
    oa, ob = orc.fpx_planes(oc)
    orc.fpx_free(oc)
    assert np.array_equal(a32, oa) and np.array_equal(b32, ob)   # device encode
    lib.conv_mfft(ctx.Cw, ctx.A32, ctx.B32, n, ctx.L, C.byref(gpu.plan(ctx.L)), gpu.KERNEL_HIP)
    assert lib.mfft_last_error() == 0
    assert np.array_equal(cw, orc.conv_limbplane(oa, ob, n, ctx.L))
    out2 = np.empty(n * n, np.float32)
    lib.fpx_decode_f32(C.byref(ctx), out2.ctypes.data)
    assert np.array_equal(out2.view(np.uint32), want)
    lib.fpx_free(C.byref(ctx))


def test_fpx_zero_and_signs(gpu, orc, lib):
    n = 64
    A = orc.fp32_rand(n * n, 9, -20, 20)
    B = orc.fp32_rand(n * n, 10, -20, 20)
    A[: n] = 0.0                                          # row 0 of C is exactly zero
    with gpu.Ctx(n, 32) as ctx:
        got = ctx.fpx_mm(A, B, 256, 256)
    oc = orc.fpx(A, B, n, 512)
    oa, ob = orc.fpx_planes(oc)
    want = orc.fpx_decode_from(oc, orc.conv_limbplane(oa, ob, n, 32))
    orc.fpx_free(oc)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.all(got[:n].view(np.uint32) == 0)           # +0.0f


# ---- fp64 embedding and the long double decode -------------------------------------
def host_view(ptr, count, ctype):
    return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(ctype)), shape=(count,))


@pytest.mark.parametrize("case", range(4))
def test_fpx64_fixture(gpu, orc, lib, case):
    """fpx_init_d / fpx_encode_d / conv_mfft / fpx_decode_f64 / fpx_decode_ld
    and the fused fpx_mm_f64 against the Fraction fixtures (fpx64.json)."""
    with open(os.path.join(GOLD, "fpx64.json")) as f:
        c = json.load(f)[case]
    n, force = c["n"], c["force_bits"]
    print(f"[fpx64] {c['name']} n={n}", flush=True)
    A = np.array(c["A_bits"], dtype=np.uint64).view(np.float64)
    B = np.array(c["B_bits"], dtype=np.uint64).view(np.float64)
    want = np.array(c["C64_bits"], dtype=np.uint64)
    ctx = gpu.FpxCtx()
    assert lib.fpx_init_d(C.byref(ctx), A.ctypes.data, B.ctypes.data, n, force) == 0
    assert ctx.sig == 53
    lib.fpx_encode_d(C.byref(ctx), A.ctypes.data, B.ctypes.data)
    assert lib.mfft_last_error() == 0
    p = gpu.plan(ctx.L)
    out = np.empty(n * n, np.float64)
    assert lib.fpx_mm_f64(C.byref(ctx), C.byref(p), out.ctypes.data) == 0
    assert np.array_equal(out.view(np.uint64), want)
    nn = n * n
    oc = orc.fpx_d(A, B, n, force)
    oa, ob = orc.fpx_planes(oc)
    orc.fpx_free(oc)
    assert np.array_equal(host_view(ctx.A32, ctx.L * nn, C.c_int32), oa)   # device encode
    assert np.array_equal(host_view(ctx.B32, ctx.L * nn, C.c_int32), ob)
    lib.conv_mfft(ctx.Cw, ctx.A32, ctx.B32, n, ctx.L, C.byref(p), gpu.KERNEL_HIP)
    assert lib.mfft_last_error() == 0
    out2 = np.empty(n * n, np.float64)
    lib.fpx_decode_f64(C.byref(ctx), out2.ctypes.data)
    assert np.array_equal(out2.view(np.uint64), want)
    ld = np.empty(n * n, np.longdouble)
    lib.fpx_decode_ld(C.byref(ctx), ld.ctypes.data)
    assert lib.mfft_last_error() == 0
    want_ld = np.ldexp(np.array(c["ld_sig"], dtype=np.int64).astype(np.longdouble),
                       np.array(c["ld_ex"], dtype=np.int32))
    assert np.array_equal(ld, want_ld)
    lib.fpx_free(C.byref(ctx))


@pytest.mark.parametrize("n,force,emin,emax", [(64, 2048, -60, 60), (96, 0, -100, 100),
                                               (128, 0, -8, 8)])
def test_fpx64_random(gpu, orc, lib, n, force, emin, emax):
    """fpx_mm_f64 (device encode, product, decode) and the sig/exponent
    decode against the oracle on random fp64 matrices, padded and unpadded
    sizes, fixed and data-sized grids."""
    print(f"[fpx64] n={n} force={force}", flush=True)
    rng = np.random.default_rng(n + force)
    A = np.ldexp(rng.uniform(1, 2, n * n) * rng.choice([-1, 1], n * n),
                 rng.integers(emin, emax + 1, n * n))
    B = np.ldexp(rng.uniform(1, 2, n * n) * rng.choice([-1, 1], n * n),
                 rng.integers(emin, emax + 1, n * n))
    A[:n] = 0.0                                           # row 0 of C: +0.0
    oc = orc.fpx_d(A, B, n, force)
    oa, ob = orc.fpx_planes(oc)
    L, SA, SB = oc.L, oc.SA, oc.SB
    cw = orc.conv_mfft(oa, ob, n, L, orc.plan(L))
    want = orc.fpx_decode_f64_from(oc, cw)
    sig, ex = orc.fpx_decode_sig63_from(oc, cw)
    orc.fpx_free(oc)
    with gpu.Ctx(n, L) as ctx:
        got = ctx.fpx_mm_f64(A, B, SA, SB)
    assert np.array_equal(got.view(np.uint64), want.view(np.uint64))
    assert np.all(got[:n].view(np.uint64) == 0)
    dsig = np.empty(n * n, np.int64)
    dex = np.empty(n * n, np.int32)
    gpu.check(lib.mfh_fpx_decode_sig63(cw.ctypes.data, n, L, SA + SB, dsig.ctypes.data,
                                       dex.ctypes.data))
    assert np.array_equal(dsig, sig) and np.array_equal(dex, ex)


# ---- row bands ----------------------------------------------------------------------------
def banded(monkeypatch, rows):
    monkeypatch.setenv("MFH_BAND_ROWS", str(rows))


def test_row_bands_against_oracle(gpu, orc, monkeypatch):
    """A in bands of 64 padded rows: the last band holds the last 8 rows."""
    n, L = 72, 32
    banded(monkeypatch, 64)
    A, A32 = signed_limbs(orc, n, L, SEED + 3)
    B, B32 = signed_limbs(orc, n, L, SEED_B + 3)
    RL = 2 * L + 1
    with gpu.Ctx(n, L) as ctx:
        assert ctx.band_rows() == 64
        got_u = ctx.mm(A, B, RL)
        got_s = ctx.mm(A, B, RL, signed=True)
    assert np.array_equal(got_u, orc.mm_mfft(A, B, n, L, orc.plan(L), RL))
    want_s = orc.normalize(orc.conv_limbplane(A32, B32, n, L), 2 * L - 1, n, RL)
    assert np.array_equal(got_s, want_s)


@pytest.mark.parametrize("n,L,band", [(200, 128, 64), (100, 128, 64), (130, 32, 64),
                                      (96, 512, 64), (136, 64, 128), (100, 8, 64),
                                      (160, 16, 64), (136, 256, 64)])
def test_row_bands_same_bits(gpu, orc, monkeypatch, n, L, band):
    """Every ring size, fast (n % 8 == 0) and generic forward transforms,
    unsigned and signed: banded products equal the one-band products."""
    print(f"[bands] n={n} L={L} band={band}", flush=True)
    A = orc.bigmat_rand(n, L, SEED + n)
    B = orc.bigmat_rand(n, L, SEED_B + n)
    RL = 2 * L + 1
    with gpu.Ctx(n, L) as ctx:
        assert ctx.band_rows() >= n
        whole = [ctx.mm(A, B, RL), ctx.mm(A, B, RL, signed=True)]
        full_bytes = ctx.workspace_bytes()
    banded(monkeypatch, band)
    with gpu.Ctx(n, L) as ctx:
        assert ctx.band_rows() == band
        assert ctx.workspace_bytes() < full_bytes
        assert np.array_equal(ctx.mm(A, B, RL), whole[0])
        assert np.array_equal(ctx.mm(A, B, RL, signed=True), whole[1])


def test_row_bands_conv_and_floats(gpu, orc, monkeypatch):
    """Coefficient-plane outputs (conv, then the fp32 and fp64 decodes)."""
    n, L = 150, 64
    rng = np.random.default_rng(9)
    A32 = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    B32 = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    X = orc.fp32_rand(n * n, SEED, -30, 30)
    Y = orc.fp32_rand(n * n, SEED_B, -30, 30)
    rng = np.random.default_rng(10)
    Xd = rng.standard_normal(n * n) * np.exp2(rng.integers(-40, 40, n * n))
    Yd = rng.standard_normal(n * n) * np.exp2(rng.integers(-40, 40, n * n))
    res = []
    for band in (0, 64):
        if band:
            banded(monkeypatch, band)
        with gpu.Ctx(n, L) as ctx:
            assert (ctx.band_rows() == band) if band else ctx.band_rows() >= n
            res.append([ctx.conv(A32, B32)])
        with gpu.Ctx(n, 32) as ctx:
            res[-1].append(ctx.fpx_mm(X, Y, 256, 256).view(np.uint32))
        with gpu.Ctx(n, 128) as ctx:
            res[-1].append(ctx.fpx_mm_f64(Xd, Yd, 1024, 1024).view(np.uint64))
    for a, b in zip(*res):
        assert np.array_equal(a, b)


def test_row_bands_generic_kernels(gpu, orc, monkeypatch):
    """Runtime-plan kernels in bands against the oracle."""
    monkeypatch.setenv("MFH_GENERIC_KERNELS", "1")
    banded(monkeypatch, 64)
    n, L = 80, 32
    A = orc.bigmat_rand(n, L, SEED)
    B = orc.bigmat_rand(n, L, SEED_B)
    RL = 2 * L + 1
    with gpu.Ctx(n, L) as ctx:
        assert ctx.band_rows() == 64
        assert np.array_equal(ctx.mm(A, B, RL), orc.mm_mfft(A, B, n, L, orc.plan(L), RL))


# ---- full-size workloads ------------------------------------------------------------------
def check_large(gpu, orc, lib, n, W, signed, min_bands=1):
    L = W // 16
    RL = 2 * L + 1
    print(f"[large] n={n} W={W} signed={signed}", flush=True)
    with gpu.Ctx(n, L) as ctx:
        print(f"[large] band rows {ctx.band_rows()}, workspace {ctx.workspace_bytes() / 1e9:.1f} GB",
              flush=True)
        assert -(-n // ctx.band_rows()) >= min_bands
        dA, dB, dO = gpu.DevBuf(L * n * n * 2), gpu.DevBuf(L * n * n * 2), gpu.DevBuf(RL * n * n * 2)
        gpu.check(lib.mfh_rand_u16_dev(ctx.h, dA.ptr, n, L, SEED))
        gpu.check(lib.mfh_rand_u16_dev(ctx.h, dB.ptr, n, L, SEED_B))
        kind = gpu.MFH_IN_U16_SIGNED if signed else gpu.MFH_IN_U16
        gpu.check(lib.mfh_mm_dev(ctx.h, kind, dA.ptr, dB.ptr, dO.ptr, RL))
        ctx.sync()
        out = dO.download(np.uint16, RL * n * n)
        for b in (dA, dB, dO):
            b.free()
    A = orc.bigmat_rand(n, L, SEED)
    B = orc.bigmat_rand(n, L, SEED_B)
    assert orc.freivalds(A, B, n, L, out, RL, signed_top=signed, nprimes=2)
    rng = np.random.default_rng(n + W)
    picks = [(0, 0), (n - 1, n - 1)] + [tuple(int(v) for v in rng.integers(0, n, 2)) for _ in range(6)]
    for i, j in picks:
        want = orc.entry_exact(A, B, n, L, i, j, RL, signed_top=signed)
        assert np.array_equal(out.reshape(RL, n * n)[:, i * n + j], want), (i, j)


def test_c1_full_against_reference_path(gpu, orc):
    n, L = 64, 64
    A = orc.bigmat_rand(n, L, SEED)
    B = orc.bigmat_rand(n, L, SEED_B)
    want = orc.mm_mfft(A, B, n, L, orc.plan(L), 2 * L + 1)
    out, err = gpu.mm_mfft(A, B, n, L, gpu.plan(L))
    assert err == 0 and np.array_equal(out, want)


def test_c3_n1024_w2048(gpu, orc, lib):
    check_large(gpu, orc, lib, 1024, 2048, False)


def test_c2_n256_w8192(gpu, orc, lib):
    check_large(gpu, orc, lib, 256, 8192, False)


def test_c5_n4096_w512_signed(gpu, orc, lib):
    check_large(gpu, orc, lib, 4096, 512, True)


def test_n3072_w2048_beyond_the_9_product_bound(gpu, orc, lib):
    """n = 3072 at 2048 bits: 6-product digits keep the int32 classes in
    range (the 9-product mode would not)."""
    check_large(gpu, orc, lib, 3072, 2048, False)


def test_w8192_conv_refused_beyond_the_9_product_bound(gpu, lib):
    """n = 1408 at 8192 bits: the exact track (6-product digits in offset
    mode, |a^| <= 2^20) admits it; conv_mfft, whose plain limbs need
    9-product digits here (|a^| up to 2^21), would pass the int64 bound
    NB K n |a^|^2 < 2^62 only up to n = 512 and is refused at call time,
    before any kernel runs."""
    n, L = 1408, 512
    with gpu.Ctx(n, L) as ctx:
        dA, dB = gpu.DevBuf(L * n * n * 4), gpu.DevBuf(L * n * n * 4)
        dCw = gpu.DevBuf((2 * L - 1) * n * n * 8)
        rc = lib.mfh_conv_dev(ctx.h, dA.ptr, dB.ptr, dCw.ptr)
        for b in (dA, dB, dCw):
            b.free()
    assert rc == -4


def test_n4096_w2048_in_row_bands(gpu, orc, lib):
    """n = 4096 at 2048 bits: the one-band workspace (about 310 GB) exceeds
    the device, so A goes through in row bands."""
    check_large(gpu, orc, lib, 4096, 2048, False, min_bands=2)


def test_n1024_w4096(gpu, orc, lib):
    check_large(gpu, orc, lib, 1024, 4096, False)


def test_c4_fp32_n2048(gpu, orc):
    n = 2048
    A = orc.fp32_rand(n * n, SEED, -20, 20)
    B = orc.fp32_rand(n * n, SEED_B, -20, 20)
    with gpu.Ctx(n, 32) as ctx:
        got = ctx.fpx_mm(A, B, 256, 256)
        cw_dev = None
    oc = orc.fpx(A, B, n, 512)
    oa, ob = orc.fpx_planes(oc)
    # the exact product's planes from the GPU's own conv path, checked by
    # Freivalds, then decoded by the oracle and compared bit for bit
    with gpu.Ctx(n, 32) as ctx:
        cw_dev = ctx.conv(oa, ob)
    assert orc.freivalds_conv(oa, ob, n, 32, cw_dev, nprimes=2)
    want = orc.fpx_decode_from(oc, cw_dev)
    orc.fpx_free(oc)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
