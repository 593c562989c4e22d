"""GPU parity of the multi-modular fixed-point products (mfh_rns_fpx_mm*):
fp32 / fp64 matrices on an L-limb grid encoded as L + 1 two's complement
limbs, multiplied by residue arithmetic and decoded with the grid's single
rounding.  Every output must carry the bits of the oracle's fpx_encode ->
product -> fpx_decode (src/fpfixed.c:144-322 restated in oracle/), of the
Fraction fixtures, and at full size of the MFFT device path (mfh_fpx_mm_dev)."""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden")
SEED, SEED_B = 12345, 12345 ^ 0xABCDEF


def oracle_f32(orc, X, Y, n, force):
    oc = orc.fpx(X, Y, n, force)
    xa, xb = orc.fpx_planes(oc)
    L, SA, SB = oc.L, oc.SA, oc.SB
    want = orc.fpx_decode_from(oc, orc.conv_limbplane(xa, xb, n, L))
    orc.fpx_free(oc)
    return want, L, SA, SB


def oracle_f64(orc, A, B, n, force):
    oc = orc.fpx_d(A, B, n, force)
    oa, ob = orc.fpx_planes(oc)
    L, SA, SB = oc.L, oc.SA, oc.SB
    want = orc.fpx_decode_f64_from(oc, orc.conv_limbplane(oa, ob, n, L))
    orc.fpx_free(oc)
    return want, L, SA, SB


@pytest.mark.parametrize("case", range(3))
def test_rns_fpx_fixture(gpu, orc, case):
    """the Fraction fixtures of the fp32 track (products rounded once to
    nearest-even on a 512-bit grid)"""
    with open(os.path.join(GOLD, "fpx.json")) as f:
        c = json.load(f)[case]
    n = c["n"]
    A = np.array(c["A_bits"], dtype=np.uint32).view(np.float32)
    B = np.array(c["B_bits"], dtype=np.uint32).view(np.float32)
    want = np.array(c["C_bits"], dtype=np.uint32)
    print(f"[rns fpx fixture] {case} n={n}", flush=True)
    _, L, SA, SB = oracle_f32(orc, A, B, n, 512)
    with gpu.Rns(n, L + 1) as r:
        got = r.fpx_mm(A, B, SA, SB)
    assert np.array_equal(got.view(np.uint32), want)


@pytest.mark.parametrize("case", range(4))
def test_rns_fpx64_fixture(gpu, orc, case):
    with open(os.path.join(GOLD, "fpx64.json")) as f:
        c = json.load(f)[case]
    n, force = c["n"], c["force_bits"]
    A = np.array(c["A_bits"], dtype=np.uint64).view(np.float64)
    B = np.array(c["B_bits"], dtype=np.uint64).view(np.float64)
    want, L, SA, SB = oracle_f64(orc, A, B, n, force)
    print(f"[rns fpx64 fixture] {c['name']} n={n} L={L}", flush=True)
    assert np.array_equal(want.view(np.uint64), np.array(c["C64_bits"], dtype=np.uint64))
    with gpu.Rns(n, L + 1) as r:
        got = r.fpx_mm_f64(A, B, SA, SB)
    assert np.array_equal(got.view(np.uint64), want.view(np.uint64))


@pytest.mark.parametrize("force", [512, 1024, 2048, 4096])
@pytest.mark.parametrize("n", [1, 45, 130])
def test_rns_fpx_every_grid(gpu, orc, n, force):
    """fp32 and fp64 on grids of 512 .. 4096 bits, ragged n, exponents that
    put entries below the grid (truncated to zero) and at its top"""
    print(f"[rns fpx grid] n={n} force={force}", flush=True)
    rng = np.random.default_rng(force + n)
    A = np.ldexp(rng.uniform(1, 2, n * n) * rng.choice([-1, 1], n * n),
                 rng.integers(-60, 61, n * n))
    B = np.ldexp(rng.uniform(1, 2, n * n) * rng.choice([-1, 1], n * n),
                 rng.integers(-60, 61, n * n))
    want64, L, SA, SB = oracle_f64(orc, A, B, n, force)
    X = orc.fp32_rand(n * n, force, -30, 30)
    Y = orc.fp32_rand(n * n, force + 1, -30, 30)
    want32, L32, SA32, SB32 = oracle_f32(orc, X, Y, n, force)
    assert L32 == L
    with gpu.Rns(n, L + 1) as r:
        got64 = r.fpx_mm_f64(A, B, SA, SB)
        got32 = r.fpx_mm(X, Y, SA32, SB32)
    assert np.array_equal(got64.view(np.uint64), want64.view(np.uint64))
    assert np.array_equal(got32.view(np.uint32), want32.view(np.uint32))
    if n > 1:
        assert np.count_nonzero(want32) > n * n // 2


def test_rns_fpx_zero_signs_and_specials(gpu, orc):
    """a zero row (+0.0f out), a row below the grid (zero), a row of fp32
    magnitudes near the largest, infinities and NaN (encoded as zero, as the
    grid's encode does), and both signs"""
    n = 64
    A = orc.fp32_rand(n * n, 9, -20, 20)
    B = orc.fp32_rand(n * n, 10, -20, 20)
    A[:n] = 0.0
    A[n:2 * n] = np.float32(2.0 ** -300)          # below the grid: zero
    A[2 * n:3 * n] = -np.float32(3.4e38)          # top limbs of the grid
    B[5::7] = np.float32(np.inf)
    B[6::11] = -np.float32(np.inf)
    B[3::13] = np.float32(np.nan)
    want, L, SA, SB = oracle_f32(orc, A, B, n, 512)
    with gpu.Rns(n, L + 1) as r:
        got = r.fpx_mm(A, B, SA, SB)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.all(got[:2 * n].view(np.uint32) == 0)


def test_rns_fpx_context_limits(gpu):
    """an 8192-bit grid needs 513 limbs, past the multi-modular limit, and a
    one-limb context has no grid: both refused before any device work"""
    import ctypes as C
    lib = gpu.load()
    h = C.c_void_p()
    assert lib.mfh_rns_create(C.byref(h), 16, 513) == -4
    with gpu.Rns(4, 1) as r:
        d = gpu.DevBuf(64)
        assert lib.mfh_rns_fpx_mm_dev(r.h, d.ptr, d.ptr, 0, 0, d.ptr) == -3
        d.free()


@pytest.mark.parametrize("n,W,f64", [(2048, 512, False), (1024, 2048, True)])
def test_rns_fpx_full_size_equals_mfft(gpu, lib, n, W, f64):
    """the fp32 workload (n = 2048, 512-bit grid, e in [-20, 20]) and an fp64
    one: every output bit equal to the MFFT device path's on the same device
    inputs"""
    L = W // 16
    SA = SB = W // 2
    print(f"[rns fpx large] n={n} W={W} f64={f64}", flush=True)
    eb = 8 if f64 else 4
    dA, dB = gpu.DevBuf(n * n * eb), gpu.DevBuf(n * n * eb)
    d1, d2 = gpu.DevBuf(n * n * eb), gpu.DevBuf(n * n * eb)
    try:
        if f64:
            rng = np.random.default_rng(21)
            A = np.ldexp(rng.uniform(1, 2, n * n) * rng.choice([-1, 1], n * n),
                         rng.integers(-40, 41, n * n))
            B = np.ldexp(rng.uniform(1, 2, n * n) * rng.choice([-1, 1], n * n),
                         rng.integers(-40, 41, n * n))
            dA.upload(A)
            dB.upload(B)
        else:
            gpu.check(lib.mfh_rand_f32_dev(None, dA.ptr, n * n, SEED, -20, 20))
            gpu.check(lib.mfh_rand_f32_dev(None, dB.ptr, n * n, SEED_B, -20, 20))
            gpu.check(lib.mfh_sync(None))
        with gpu.Ctx(n, L) as ctx:
            fn = lib.mfh_fpx_mm_f64_dev if f64 else lib.mfh_fpx_mm_dev
            gpu.check(fn(ctx.h, dA.ptr, dB.ptr, SA, SB, d1.ptr))
            ctx.sync()
        with gpu.Rns(n, L + 1) as r:
            r.fpx_mm_dev(dA.ptr, dB.ptr, SA, SB, d2.ptr, f64=f64)
            r.sync()
        dt = np.uint64 if f64 else np.uint32
        want, got = d1.download(dt, n * n), d2.download(dt, n * n)
    finally:
        for b in (dA, dB, d1, d2):
            b.free()
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} outputs differ, first at {bad[:5]}"
    assert np.count_nonzero(want) > n * n // 2


def test_rns_fpx_limb_boundaries(gpu, orc):
    """Diagonal products +-2^k and +-(2 - 2^-23) 2^k for 64 consecutive
    exponents k (so every position modulo a 16-bit limb, whatever the
    grid's scale): the decode of carried limbs meets negative values whose
    magnitude is exactly a power of 2^16 (every limb below its window zero)
    and all-ones significands; the off-diagonal outputs are +0.0f."""
    n = 64
    A = np.zeros(n * n, np.float32)
    B = np.zeros(n * n, np.float32)
    for i in range(n):
        k, ea = -40 + i, i % 7 - 3
        ma = 1.0 if i % 4 else 2.0 - 2.0 ** -23
        A[i * n + i] = np.float32(np.ldexp(ma, ea) * (-1 if i % 2 else 1))
        B[i * n + i] = np.float32(np.ldexp(1.0, k - ea) * (-1 if i % 5 == 0 else 1))
    want, L, SA, SB = oracle_f32(orc, A, B, n, 512)
    with gpu.Rns(n, L + 1) as r:
        got = r.fpx_mm(A, B, SA, SB)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    d = np.arange(n) * (n + 1)
    assert np.count_nonzero(want[d]) == n
    off = np.ones(n * n, bool)
    off[d] = False
    assert np.all(got[off].view(np.uint32) == 0)
