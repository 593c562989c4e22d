"""The two pointwise algorithms at ring sizes K = 8 (W = 512 bits), K = 16
(W = 1024 and 2048 bits) and K = 32 (W = 4096 and 8192 bits, the two-slot
kernel): the Gauss
three-product split of the ring halves (the default there) and the
K^2-product kernel (MFH_POINTWISE=flat, read at context creation) must give
the same limbs, and both the oracle's.  Covers the exact track (unsigned and
two's complement, both forward-kernel families, ragged n, row bands), the
caller's own limbs (conv_mfft) and the fixed-point floats, and the issued
work each reports."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SEED, SEED_B = 12345, 12345 ^ 0xABCDEF


def _ctx(gpu, monkeypatch, flat, n, L, p=None):
    if flat:
        monkeypatch.setenv("MFH_POINTWISE", "flat")
    else:
        monkeypatch.delenv("MFH_POINTWISE", raising=False)
    ctx = gpu.Ctx(n, L, p)
    monkeypatch.delenv("MFH_POINTWISE", raising=False)
    return ctx


@pytest.mark.parametrize("n,L,signed", [(8, 64, False), (64, 64, False), (100, 64, False),
                                        (24, 128, False), (7, 128, False), (130, 128, False),
                                        (40, 64, True), (72, 128, True),
                                        (8, 32, False), (64, 32, False), (130, 32, False),
                                        (33, 32, True),
                                        (8, 256, False), (64, 256, False), (33, 256, True),
                                        (16, 512, False), (72, 512, False), (40, 512, True)])
def test_gauss_and_flat_products_agree(gpu, orc, monkeypatch, n, L, signed):
    print(f"[gauss] n={n} L={L} signed={signed}", flush=True)
    A = orc.bigmat_rand(n, L, SEED)
    B = orc.bigmat_rand(n, L, SEED_B)
    RL = 2 * L + 1
    outs, works = [], []
    for flat in (False, True):
        with _ctx(gpu, monkeypatch, flat, n, L) as ctx:
            outs.append(ctx.mm(A, B, RL, signed=signed))
            works.append(ctx.work()[0])
    assert np.array_equal(outs[0], outs[1])
    # issued int8 ops: 3 (K/2)^2 ring products per point against K^2
    assert works[0] == pytest.approx(0.75 * works[1])
    if signed:
        top = slice((L - 1) * n * n, L * n * n)
        A32, B32 = A.astype(np.int32), B.astype(np.int32)
        A32[top] = A[top].view(np.int16)
        B32[top] = B[top].view(np.int16)
        cw = orc.conv_limbplane(A32, B32, n, L)
        want = orc.normalize(cw, 2 * L - 1, n, RL)
    else:
        want = orc.mm_mfft(A, B, n, L, orc.plan(L), RL)
    assert np.array_equal(outs[0], want)


@pytest.mark.parametrize("n,L", [(150, 128), (136, 256)])
def test_gauss_row_bands_and_generic_kernels(gpu, orc, monkeypatch, n, L):
    """Row bands of 64 rows, and the runtime-plan forward kernel writing the
    Gauss slots (MFH_GENERIC_KERNELS), equal the oracle."""
    A = orc.bigmat_rand(n, L, 5)
    B = orc.bigmat_rand(n, L, 6)
    RL = 2 * L + 1
    want = orc.mm_mfft(A, B, n, L, orc.plan(L), RL)
    monkeypatch.setenv("MFH_BAND_ROWS", "64")
    with gpu.Ctx(n, L) as ctx:
        assert ctx.band_rows() == 64
        assert np.array_equal(ctx.mm(A, B, RL), want)
    monkeypatch.delenv("MFH_BAND_ROWS")
    monkeypatch.setenv("MFH_GENERIC_KERNELS", "1")
    with gpu.Ctx(n, L) as ctx:
        assert np.array_equal(ctx.mm(A, B, RL), want)
    monkeypatch.delenv("MFH_GENERIC_KERNELS")


@pytest.mark.parametrize("n,L", [(17, 32), (9, 64), (33, 128), (20, 256)])
def test_gauss_conv_signed_limbs(gpu, orc, monkeypatch, n, L):
    """conv_mfft on signed limbs at the extremes: Gauss slot values reach the
    same bound as single coefficients."""
    rng = np.random.default_rng(n + L)
    A = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    B = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    A[: (L // 2) * n * n] = 65535
    B[: (L // 2) * n * n] = -65535
    want = orc.conv_limbplane(A, B, n, L)
    for flat in (False, True):
        with _ctx(gpu, monkeypatch, flat, n, L) as ctx:
            assert np.array_equal(ctx.conv(A, B), want)


def test_gauss_fp64_product(gpu, orc, monkeypatch):
    """fp64 on a 2048-bit grid (L = 128, K = 16): the windowed forward kernel
    writing Gauss slots, with the fused decode, equals the flat kernel's and
    the oracle's result."""
    n = 48
    rng = np.random.default_rng(3)

    def draw():
        return ((rng.random(n * n) + 1.0) * np.exp2(rng.integers(-60, 61, n * n)) *
                np.where(rng.random(n * n) < 0.5, -1.0, 1.0))
    A, B = draw(), draw()
    A = np.ascontiguousarray(A, np.float64)
    B = np.ascontiguousarray(B, np.float64)
    oc = orc.fpx_d(A, B, n, 2048)
    oa, ob = orc.fpx_planes(oc)
    L = oa.size // (n * n)
    assert L == 128
    want = orc.fpx_decode_f64_from(oc, orc.conv_limbplane(oa, ob, n, L))
    orc.fpx_free(oc)
    for flat in (False, True):
        with _ctx(gpu, monkeypatch, flat, n, L) as ctx:
            got = ctx.fpx_mm_f64(A, B, 1024, 1024)
        assert np.array_equal(got.view(np.uint64), want.view(np.uint64))
