"""CPU tests of the multi-modular product's plan (host logic, no device): the
primes are distinct primes that keep every residue digit pair in int8, and
their product leaves the reconstruction a margin of 4 over the largest
product entry."""
import math

import pytest


def is_prime(p):
    if p < 2:
        return False
    for d in range(2, math.isqrt(p) + 1):
        if p % d == 0:
            return False
    return True


@pytest.mark.parametrize("n,L", [(1, 1), (64, 64), (1024, 128), (256, 512), (4096, 32),
                                 (2048, 32), (3, 1024), (32768, 1), (100, 7)])
def test_rns_primes_bound(lib, n, L):
    import mfft_ctypes
    ps = [int(p) for p in mfft_ctypes.rns_primes(n, L)]
    assert len(set(ps)) == len(ps)
    assert ps == sorted(ps, reverse=True)
    assert all(is_prime(p) and p <= 65279 for p in ps)
    # balanced residues |r| <= (p-1)/2 <= 32639: both base-2^8 digits are int8
    assert max(ps) // 2 <= 32639
    M = math.prod(ps)
    W = 16 * L
    assert M > 4 * n * (1 << (2 * W)), "reconstruction margin"
    # no prime more than the bound needs: without the last one the product
    # falls below 2^(2W + ceil(log2 n) + 3)
    need = 2 * W + math.ceil(math.log2(n)) + 3 if n > 1 else 2 * W + 3
    assert sum(math.log2(p) for p in ps[:-1]) < need <= sum(math.log2(p) for p in ps)


def test_rns_primes_counts(lib):
    """the headline 2048-bit n = 1024 product needs 258 primes (4 n 2^4096 <
    M), i.e. 1032 int8 n^3 GEMMs, against the MFFT's 6 x 6144"""
    import mfft_ctypes
    assert len(mfft_ctypes.rns_primes(1024, 128)) == 258


def test_rns_limits(lib):
    import ctypes as C
    h = C.c_void_p()
    # beyond the stated limits the context is refused before any device work
    assert lib.mfh_rns_create(C.byref(h), 32769, 8) == -4
    assert lib.mfh_rns_create(C.byref(h), 16, 513) == -4
    assert lib.mfh_rns_primes(0, 8, None, 0) == -3


def test_digit_pair_packing():
    """the stored digit pair of a balanced residue r is (r + 128) ^ 0x80 in
    16 bits: low byte lo = ((r+128) & 255) - 128 and high byte
    hi = (r - lo) / 256, both int8, with r = 256 hi + lo"""
    import numpy as np
    r = np.arange(-32639, 32640, dtype=np.int64)
    w = ((r + 128) ^ 0x80) & 0xFFFF
    lo = (w & 255).astype(np.int64)
    hi = (w >> 8).astype(np.int64)
    lo = np.where(lo >= 128, lo - 256, lo)
    hi = np.where(hi >= 128, hi - 256, hi)
    assert np.array_equal(256 * hi + lo, r)
    assert hi.min() >= -128 and hi.max() <= 127


def test_fp64_reduction_needs_no_fixup(lib):
    """q = rint(v * fl(1/p)), r = v - q p (the kernels' reduction, in IEEE
    float64 as on the device) gives the balanced residue, |r| <= (p-1)/2,
    for |v| <= 2^46: v * fl(1/p) is within 2^-22 of v/p, and v/p is never
    closer than 1/(2p) to a half-integer.  Checked at the points closest to
    the half-integers (v = k p + (p-1)/2 and k p - (p-1)/2) and at random v,
    for the largest and smallest primes of the plans."""
    import numpy as np
    import mfft_ctypes
    ps = list(mfft_ctypes.rns_primes(256, 512))
    rng = np.random.default_rng(5)
    for p in (int(ps[0]), int(ps[-1]), 65269, 16411):
        h = (p - 1) // 2
        k = rng.integers(-(1 << 46) // p, (1 << 46) // p, size=20000, dtype=np.int64)
        v = np.concatenate([k * p + h, k * p - h, k * p,
                            rng.integers(-(1 << 46), 1 << 46, size=20000, dtype=np.int64)])
        v = v[np.abs(v) <= (1 << 46)]
        vd = v.astype(np.float64)
        assert np.array_equal(vd.astype(np.int64), v)            # exact in fp64
        q = np.rint(vd * (1.0 / p))
        r = (v - q.astype(np.int64) * p)
        assert np.abs(r).max() <= h, p
        assert np.array_equal(np.mod(r - v, p), np.zeros_like(r))


@pytest.mark.parametrize("n,L", [(1024, 128), (4096, 32), (256, 512), (64, 64), (16, 16)])
def test_fp64_top_limb(lib, n, L):
    """When 4L fills whole 64-byte chunks the CRT computes C mod 2^(32L) by
    the GEMM and the top limb as round(M 2^(-32L) (t - q) - w 2^-32), t =
    sum_m y_m fl(1/p_m) summed in fp64, q = rint(t), w the top 32-bit word
    of C mod 2^(32L).  Against Python integers: floor(C / 2^(32L)) for
    random and extreme signed products |C| <= n 2^(2W) (the kernel's error
    bound, M 2^(-32L) nm^2 2^-53, is far below 1/2 at these plans)."""
    import math
    import random
    from fractions import Fraction
    import mfft_ctypes
    ps = [int(p) for p in mfft_ctypes.rns_primes(n, L)]
    M = math.prod(ps)
    W = 16 * L
    mtop = float(Fraction(M, 1 << (32 * L)))
    cinv = [pow((M // p) % p, -1, p) for p in ps]
    lim = n * (1 << (2 * W))
    rnd = random.Random(n + L)
    cases = [lim, lim - 1, -lim, -lim + 1, 0, -1, 1, 1 << (32 * L), -(1 << (32 * L))]
    cases += [rnd.randrange(-lim, lim + 1) for _ in range(40)]
    for C in cases:
        t = 0.0
        for p, ci in zip(ps, cinv):
            r = C * ci % p
            if r > p // 2:
                r -= p
            t += float(r) * (1.0 / p)
        q = round(t)
        w = (C % (1 << (32 * L))) >> (32 * L - 32)
        est = mtop * (t - q) - w * 2.0 ** -32
        assert abs(est - (C >> (32 * L))) < 1e-3, (C, est)
