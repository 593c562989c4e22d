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
    assert len(ps) % 8 == 0
    assert len(set(ps)) == len(ps)
    assert ps == sorted(ps, reverse=True)
    assert all(is_prime(p) and p <= 65279 for p in ps)
    # balanced residues |r| <= (p-1)/2 <= 32639: both base-2^8 digits are int8
    assert max(ps) // 2 <= 32639
    M = math.prod(ps)
    W = 16 * L
    assert M > 4 * n * (1 << (2 * W)), "reconstruction margin"
    # no prime more than the bound and the rounding to 8 need
    assert math.prod(ps[:-8]) <= 4 * n * (1 << (2 * W)) * (1 << 24)


def test_rns_primes_counts(lib):
    """the headline 2048-bit n = 1024 product needs 264 primes (4 n 2^4096 <
    M), i.e. 1056 int8 n^3 GEMMs, against the MFFT's 6 x 6144"""
    import mfft_ctypes
    assert len(mfft_ctypes.rns_primes(1024, 128)) == 264
    assert len(mfft_ctypes.rns_primes(256, 512)) % 8 == 0


def test_rns_limits(lib):
    import ctypes as C
    h = C.c_void_p()
    # beyond the stated limits the context is refused before any device work
    assert lib.mfh_rns_create(C.byref(h), 32769, 8) == -4
    assert lib.mfh_rns_create(C.byref(h), 16, 513) == -4
    assert lib.mfh_rns_primes(0, 8, None, 0) == -3
