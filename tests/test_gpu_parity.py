"""GPU parity: the gfx950 path (through the C-ABI) against the CPU oracle on
the same seeded inputs.  Integer results must be bit-identical."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SEED = 12345
SEED_B = 12345 ^ 0xABCDEF

# (n, L, sigma): every ring size K in {4, 8, 16, 32}, padded and unpadded n
SMALL = [(1, 2, 0), (5, 4, 0), (8, 8, 0), (16, 16, 0), (8, 32, 3), (13, 32, 0),
         (8, 64, 0), (7, 128, 0), (3, 256, 0), (6, 512, 0), (64, 64, 0), (70, 32, 0),
         (100, 16, 0),
         # compile-time specialised transforms (n a multiple of 8)
         (24, 128, 0), (64, 128, 0), (40, 64, 0), (96, 32, 0), (136, 32, 0), (16, 512, 0),
         (24, 512, 0)]


@pytest.mark.parametrize("n,L,sigma", SMALL)
def test_mm_mfft_matches_oracle(gpu, orc, n, L, sigma):
    print(f"[mm] n={n} L={L} sigma={sigma}", flush=True)
    A = orc.bigmat_rand(n, L, SEED)
    B = orc.bigmat_rand(n, L, SEED_B)
    RL = 2 * L + 1
    p = gpu.plan(L, sigma)
    want = orc.mm_mfft(A, B, n, L, orc.plan(L, sigma), RL)
    with gpu.Ctx(n, L, p) as ctx:
        got = ctx.mm(A, B, RL)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} limbs differ, first at flat index {bad[:5]}"


def test_c_api_mm_mfft(gpu, orc):
    n, L = 12, 64
    A = orc.bigmat_rand(n, L, SEED)
    B = orc.bigmat_rand(n, L, SEED_B)
    want = orc.mm_limbplane(A, B, n, L, 2 * L + 1)
    got, err = gpu.mm_mfft(A, B, n, L, gpu.plan(L))
    assert err == 0
    assert np.array_equal(got, want)
