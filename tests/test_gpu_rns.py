"""GPU parity of the multi-modular product (mfh_rns_*): the same exact
product as mm_mfft / mm_limbplane, computed from residues modulo 16-bit
primes on the int8 matrix cores.  Every output limb must equal the oracle's
(src/methods.c:106-123 restated in oracle/), and at full size the MFFT
device path's."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SEED, SEED_B = 12345, 12345 ^ 0xABCDEF


def signed_limbs(orc, n, L, seed):
    A = orc.bigmat_rand(n, L, seed)
    top = slice((L - 1) * n * n, L * n * n)
    A32 = A.astype(np.int32)
    A32[top] = A[top].view(np.int16)
    return A, A32


def expected(orc, A, B, n, L, RL, signed):
    A32 = A.astype(np.int32)
    B32 = B.astype(np.int32)
    if signed:
        top = slice((L - 1) * n * n, L * n * n)
        A32[top] = A[top].view(np.int16)
        B32[top] = B[top].view(np.int16)
    return orc.normalize(orc.conv_limbplane(A32, B32, n, L), 2 * L - 1, n, RL)


# every residue-kernel instantiation (k blocks 1 .. 16), ragged n, odd L;
# at 16 k blocks the blocks of 8 primes run in threes (three LDS weight
# buffers): 129, 65 and 130 blocks at L = 511, 257 and 512 end on each
# buffer
SIZES = [(1, 1), (1, 2), (5, 4), (8, 8), (16, 16), (13, 32), (8, 64), (7, 128), (3, 256),
         (6, 512), (64, 64), (70, 32), (100, 16), (130, 8), (129, 33), (257, 3), (2, 512),
         (40, 100), (24, 200), (9, 300), (12, 511), (8, 257)]


@pytest.mark.parametrize("signed", [False, True])
@pytest.mark.parametrize("n,L", SIZES)
def test_rns_matches_oracle(gpu, orc, n, L, signed):
    print(f"[rns] n={n} L={L} signed={signed}", flush=True)
    A = orc.bigmat_rand(n, L, SEED + L)
    B = orc.bigmat_rand(n, L, SEED_B + n)
    RL = 2 * L + 1
    want = expected(orc, A, B, n, L, RL, signed)
    with gpu.Rns(n, L) as r:
        got = r.mm(A, B, RL, signed=signed)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} limbs differ, first at flat index {bad[:5]}"


def test_rns_unsigned_matches_mm_mfft_oracle(gpu, orc):
    """the oracle's own mm_mfft (src/mfft.c:424-438) on the 1024-bit workload"""
    n, L = 64, 64
    A = orc.bigmat_rand(n, L, SEED)
    B = orc.bigmat_rand(n, L, SEED_B)
    want = orc.mm_mfft(A, B, n, L, orc.plan(L), 2 * L + 1)
    with gpu.Rns(n, L) as r:
        assert np.array_equal(r.mm(A, B), want)


@pytest.mark.parametrize("L,RL", [(64, 1), (64, 5), (64, 128), (64, 129), (64, 200), (32, 3),
                                  (32, 70), (128, 2), (128, 256), (128, 300), (512, 37),
                                  (512, 1030), (7, 16), (7, 15)])
@pytest.mark.parametrize("signed", [False, True])
def test_rns_short_and_long_outputs(gpu, orc, L, RL, signed):
    """RL below 2L+1 truncates mod 2^(16 RL); above it the limbs are the sign
    extension (zero for unsigned entries), as normalize_planes gives
    (src/bigmat.c:48-60)."""
    n = 12
    A = orc.bigmat_rand(n, L, 3 + L)
    B = orc.bigmat_rand(n, L, 4 + RL)
    want = expected(orc, A, B, n, L, RL, signed)
    with gpu.Rns(n, L) as r:
        assert np.array_equal(r.mm(A, B, RL, signed=signed), want)


@pytest.mark.parametrize("n,L", [(64, 128), (16, 64), (32, 32), (16, 512), (5, 500), (128, 8)])
def test_rns_extremes(gpu, orc, n, L):
    """all limbs 0xFFFF (2^W - 1 unsigned: the largest product, n (2^W - 1)^2;
    -1 signed: +n), 0x8000 at the top and 0 below (-2^(W-1) signed: the most
    negative entries, product n 2^(2W-2)), and mixed signs per row"""
    RL = 2 * L + 1
    nn = n * n
    ones = np.full(L * nn, 0xFFFF, np.uint16)
    mostneg = np.zeros(L * nn, np.uint16)
    mostneg[(L - 1) * nn:] = 0x8000
    mixed = orc.bigmat_rand(n, L, 99)
    mixed[(L - 1) * nn:] = np.where(np.arange(nn) % 3 == 0, 0x8000, 0x7FFF).astype(np.uint16)
    with gpu.Rns(n, L) as r:
        for A, B in [(ones, ones), (mostneg, mostneg), (ones, mostneg), (mixed, ones),
                     (mixed, mostneg)]:
            for signed in (False, True):
                want = expected(orc, A, B, n, L, RL, signed)
                assert np.array_equal(r.mm(A, B, RL, signed=signed), want), signed


@pytest.mark.parametrize("n,L,signed", [(5, 8, False), (5, 8, True), (70, 3, True),
                                        (17, 64, False), (3, 512, True)])
def test_rns_residues_match_python_integers(gpu, orc, n, L, signed):
    """stage 1: the digit pairs of every entry's residues are the balanced
    residues of the entry (a Python integer) modulo each prime, and zero
    outside n x n"""
    X = orc.bigmat_rand(n, L, 7 + n)
    with gpu.Rns(n, L) as r:
        nm, np_, _ = r.info()
        R = r.residues(X, signed=signed)
    primes = [int(p) for p in gpu.rns_primes(n, L)]
    assert len(primes) == nm
    lo = R.astype(np.int64) & 255
    hi = R.astype(np.int64) >> 8
    val = np.where(hi >= 128, hi - 256, hi) * 256 + np.where(lo >= 128, lo - 256, lo)
    planes = X.reshape(L, n, n)
    for i in range(n):
        for k in range(n):
            x = 0
            for u in reversed(range(L)):
                x = (x << 16) | int(planes[u, i, k])
            if signed and x >> (16 * L - 1):
                x -= 1 << (16 * L)
            for m in range(0, nm, max(1, nm // 37)):
                p = primes[m]
                rr = x % p
                if rr > p // 2:
                    rr -= p
                assert val[m, i, k] == rr, (i, k, m)
    mask = np.ones((np_, np_), bool)
    mask[:n, :n] = False
    assert not R[:, mask].any()


def device_product(gpu, lib, n, L, signed, use_rns):
    RL = 2 * L + 1
    kind = gpu.MFH_IN_U16_SIGNED if signed else gpu.MFH_IN_U16
    dA, dB, dO = gpu.DevBuf(L * n * n * 2), gpu.DevBuf(L * n * n * 2), gpu.DevBuf(RL * n * n * 2)
    try:
        if use_rns:
            with gpu.Rns(n, L) as r:
                gpu.check(lib.mfh_rand_u16_dev(None, dA.ptr, n, L, SEED))
                gpu.check(lib.mfh_rand_u16_dev(None, dB.ptr, n, L, SEED_B))
                gpu.check(lib.mfh_sync(None))
                r.mm_dev(dA.ptr, dB.ptr, dO.ptr, RL, signed=signed)
                r.sync()
        else:
            with gpu.Ctx(n, L) as ctx:
                gpu.check(lib.mfh_rand_u16_dev(ctx.h, dA.ptr, n, L, SEED))
                gpu.check(lib.mfh_rand_u16_dev(ctx.h, dB.ptr, n, L, SEED_B))
                gpu.check(lib.mfh_mm_dev(ctx.h, kind, dA.ptr, dB.ptr, dO.ptr, RL))
                ctx.sync()
        return dO.download(np.uint16, RL * n * n)
    finally:
        for b in (dA, dB, dO):
            b.free()


@pytest.mark.parametrize("n,W,signed", [(1024, 2048, False), (256, 8192, False),
                                        (4096, 512, True), (2048, 1024, False)])
def test_rns_full_size_equals_mfft(gpu, orc, lib, n, W, signed):
    """the headline-size workloads: limb for limb equal to the MFFT device
    product, and Freivalds' check against the seeded inputs"""
    L = W // 16
    print(f"[rns large] n={n} W={W} signed={signed}", flush=True)
    got = device_product(gpu, lib, n, L, signed, True)
    want = device_product(gpu, lib, n, L, signed, False)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} limbs differ, first at {bad[:5]}"
    A = orc.bigmat_rand(n, L, SEED)
    B = orc.bigmat_rand(n, L, SEED_B)
    assert orc.freivalds(A, B, n, L, got, 2 * L + 1, signed_top=signed, nprimes=2)


@pytest.mark.parametrize("n,L", [(20, 300), (33, 512), (8, 8)])
def test_rns_crt_passes_repeat(gpu, orc, n, L):
    """The CRT of wide outputs runs in passes over output chunks, each
    carrying into the next (L = 300 and 512: four and three passes); a
    single-pass kernel must start from a zero carry whatever its LDS held.
    Two products in a row on one context, the second with a shorter output,
    both equal to the oracle."""
    print(f"[rns crt passes] n={n} L={L}", flush=True)
    A = orc.bigmat_rand(n, L, 71 + L)
    B = orc.bigmat_rand(n, L, 72 + n)
    with gpu.Rns(n, L) as r:
        for RL, signed in ((2 * L + 1, True), (L + 3, False)):
            want = expected(orc, A, B, n, L, RL, signed)
            assert np.array_equal(r.mm(A, B, RL, signed=signed), want), (RL, signed)
