"""GPU parity of the schoolbook entry points through the C-ABI: the leaf
operator mm_accum (exact modulo 2^64 for any int32 entries), conv_limbplane,
mm_limbplane and ssa_negconv, against Python integers, the oracle and the
golden products; products under the recursive plan; and the MFFT products
of the full-size workloads checked against the schoolbook on the device."""
import ctypes as C
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SEED, SEED_B = 12345, 12345 ^ 0xABCDEF
M64 = (1 << 64) - 1


def exact_mm_mod64(C0, A, B, n, sign):
    """C0 +/- A B over Python integers, reduced to int64 two's complement."""
    P = A.reshape(n, n).astype(object).dot(B.reshape(n, n).astype(object))
    out = []
    for c, p in zip(C0.tolist(), P.reshape(-1).tolist()):
        v = (c + p if sign > 0 else c - p) & M64
        out.append(v - (1 << 64) if v >> 63 else v)
    return np.array(out, dtype=np.int64)


@pytest.mark.parametrize("n,sign", [(1, 1), (7, -1), (64, 1), (100, 0), (130, 1)])
def test_mm_accum_full_int32_range(gpu, lib, n, sign):
    rng = np.random.default_rng(n)
    A = rng.integers(-2 ** 31, 2 ** 31, size=n * n, dtype=np.int64).astype(np.int32)
    B = rng.integers(-2 ** 31, 2 ** 31, size=n * n, dtype=np.int64).astype(np.int32)
    A[0], B[0] = -2 ** 31, -2 ** 31                      # the one product of 2^62
    C0 = rng.integers(-2 ** 63, 2 ** 63 - 1, size=n * n, dtype=np.int64)
    want = exact_mm_mod64(C0, A, B, n, sign)
    got = C0.copy()
    lib.mm_accum(got.ctypes.data, A.ctypes.data, B.ctypes.data, n, sign, gpu.KERNEL_HIP)
    assert lib.mfft_last_error() == 0
    assert np.array_equal(got, want)


def test_mm_accum_matches_oracle_leaf(gpu, orc, lib):
    n = 192
    rng = np.random.default_rng(5)
    A = rng.integers(-65535, 65536, size=n * n).astype(np.int32)
    B = rng.integers(-65535, 65536, size=n * n).astype(np.int32)
    want = np.zeros(n * n, np.int64)
    orc.mm_accum(want, A, B, n, 1)
    orc.mm_accum(want, B, A, n, -1)
    got = np.zeros(n * n, np.int64)
    gpu.check(lib.mfh_mm_accum(got.ctypes.data, A.ctypes.data, B.ctypes.data, n, 1))
    gpu.check(lib.mfh_mm_accum(got.ctypes.data, B.ctypes.data, A.ctypes.data, n, -1))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n,L", [(5, 2), (16, 8), (33, 16), (64, 32), (20, 128)])
def test_conv_limbplane(gpu, orc, lib, n, L):
    print(f"[conv_limbplane] n={n} L={L}", flush=True)
    rng = np.random.default_rng(n * L)
    A = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    B = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    A[:7] = 2 ** 31 - 1                                  # outside the MFFT's limb range
    B[:7] = -2 ** 31
    want = orc.conv_limbplane(A, B, n, L)
    cw = np.zeros((2 * L - 1) * n * n, np.int64)
    lib.conv_limbplane(cw.ctypes.data, A.ctypes.data, B.ctypes.data, n, L, gpu.KERNEL_HIP)
    assert lib.mfft_last_error() == 0
    assert np.array_equal(cw, want)


def test_mm_limbplane_golden_products(gpu, orc, lib):
    with open(os.path.join(GOLD, "products.json")) as f:
        cases = [c for c in json.load(f) if not c["signed"]]
    assert cases
    for c in cases:
        n, L, RL = c["n"], c["L"], c["RL"]
        A = orc.bigmat_rand(n, L, c["seed_a"])       # the fixture's seeded inputs
        B = orc.bigmat_rand(n, L, c["seed_b"])
        out = np.zeros(RL * n * n, np.uint16)
        lib.mm_limbplane(A.ctypes.data, B.ctypes.data, n, L, gpu.KERNEL_HIP, out.ctypes.data, RL)
        assert lib.mfft_last_error() == 0
        assert np.array_equal(out, np.array(c["out"], dtype=np.uint16)), (n, L)


@pytest.mark.parametrize("n,L", [(48, 64), (64, 128)])
def test_mm_limbplane_matches_oracle(gpu, orc, lib, n, L):
    A = orc.bigmat_rand(n, L, SEED)
    B = orc.bigmat_rand(n, L, SEED_B)
    RL = 2 * L + 1
    out = np.zeros(RL * n * n, np.uint16)
    lib.mm_limbplane(A.ctypes.data, B.ctypes.data, n, L, gpu.KERNEL_HIP, out.ctypes.data, RL)
    assert lib.mfft_last_error() == 0
    assert np.array_equal(out, orc.mm_limbplane(A, B, n, L, RL))


@pytest.mark.parametrize("n,W,signed", [(1024, 2048, False), (256, 8192, False),
                                         (4096, 512, True)])
def test_mfft_equals_schoolbook_full_size(gpu, orc, lib, n, W, signed):
    """The full-size products computed twice on the device, by the MFFT path
    (int8 MFMA) and by the integer-ALU schoolbook, limb for limb."""
    L = W // 16
    RL = 2 * L + 1
    kind = gpu.MFH_IN_U16_SIGNED if signed else gpu.MFH_IN_U16
    print(f"[schoolbook] n={n} W={W} signed={signed}", flush=True)
    with gpu.Ctx(n, L) as ctx:
        dA, dB = gpu.DevBuf(L * n * n * 2), gpu.DevBuf(L * n * n * 2)
        dO1, dO2 = gpu.DevBuf(RL * n * n * 2), gpu.DevBuf(RL * n * n * 2)
        dCw = gpu.DevBuf((2 * L - 1) * n * n * 8)
        gpu.check(lib.mfh_rand_u16_dev(ctx.h, dA.ptr, n, L, SEED))
        gpu.check(lib.mfh_rand_u16_dev(ctx.h, dB.ptr, n, L, SEED_B))
        gpu.check(lib.mfh_mm_dev(ctx.h, kind, dA.ptr, dB.ptr, dO1.ptr, RL))
        gpu.check(lib.mfh_limbplane_mm_dev(ctx.h, kind, dA.ptr, dB.ptr, n, L, dCw.ptr,
                                            dO2.ptr, RL))
        ctx.sync()
        o1 = dO1.download(np.uint16, RL * n * n)
        o2 = dO2.download(np.uint16, RL * n * n)
        for b in (dA, dB, dO1, dO2, dCw):
            b.free()
    assert np.array_equal(o1, o2)
    A = orc.bigmat_rand(n, L, SEED)
    B = orc.bigmat_rand(n, L, SEED_B)
    assert orc.freivalds(A, B, n, L, o2, RL, signed_top=signed, nprimes=1)


@pytest.mark.parametrize("K,n", [(4, 8), (8, 33), (16, 64), (32, 17)])
def test_ssa_negconv(gpu, orc, lib, K, n):
    """C = A B mod (t^K + 1): the linear limb convolution folded by t^K = -1
    (src/mfft.c:529-557 is the reference's own base case)."""
    rng = np.random.default_rng(K * n)
    A = rng.integers(-2 ** 20, 2 ** 20, size=K * n * n).astype(np.int32)
    B = rng.integers(-2 ** 20, 2 ** 20, size=K * n * n).astype(np.int32)
    lin = orc.conv_limbplane(A, B, n, K).reshape(2 * K - 1, n * n)
    want = lin[:K].copy()
    want[:K - 1] -= lin[K:]
    got = np.zeros(K * n * n, np.int64)
    lib.ssa_negconv(got.ctypes.data, A.ctypes.data, B.ctypes.data, K, n, 36, gpu.KERNEL_HIP)
    assert lib.mfft_last_error() == 0
    assert np.array_equal(got.reshape(K, n * n), want)
    # t^K = -1 on a basis element: t^(K-1) * t = -1
    E1 = np.zeros(K * n * n, np.int32)
    E2 = np.zeros(K * n * n, np.int32)
    E1[(K - 1) * n * n:] = np.eye(n, dtype=np.int32).reshape(-1)
    E2[n * n:2 * n * n] = np.eye(n, dtype=np.int32).reshape(-1)
    lib.ssa_negconv(got.ctypes.data, E1.ctypes.data, E2.ctypes.data, K, n, 1, gpu.KERNEL_HIP)
    ref = np.zeros((K, n * n), np.int64)
    ref[0] = -np.eye(n, dtype=np.int64).reshape(-1)
    assert np.array_equal(got.reshape(K, n * n), ref)


@pytest.mark.parametrize("n,L", [(20, 8), (64, 64), (40, 128)])
def test_mm_mfft_recursive_plan(gpu, orc, n, L):
    """mm_mfft under mfft_plan_init_rec's plan gives the exact product."""
    p = gpu.plan_rec(L, n)
    assert p is not None and p.rec == 1
    A = orc.bigmat_rand(n, L, SEED)
    B = orc.bigmat_rand(n, L, SEED_B)
    out, err = gpu.mm_mfft(A, B, n, L, p)
    assert err == 0
    assert np.array_equal(out, orc.mm_limbplane(A, B, n, L, 2 * L + 1))


@pytest.mark.parametrize("n,L", [(3, 4), (17, 16), (64, 64), (7, 130)])
def test_mm_bigint_textbook_entry_major(gpu, orc, lib, n, L):
    """mm_bigint_ijk / mm_bigint_ikj take entry-major inputs
    (bigmat_to_entry_major, src/bigmat.c:37-46)."""
    A = orc.bigmat_rand(n, L, SEED)
    B = orc.bigmat_rand(n, L, SEED_B)
    Aem = A.reshape(L, n * n).T.copy()
    Bem = B.reshape(L, n * n).T.copy()
    RL = 2 * L + 1
    want = orc.mm_limbplane(A, B, n, L, RL)
    for f in (lib.mm_bigint_ijk, lib.mm_bigint_ikj):
        out = np.zeros(RL * n * n, np.uint16)
        f(Aem.ctypes.data, Bem.ctypes.data, n, L, out.ctypes.data, RL)
        assert lib.mfft_last_error() == 0
        assert np.array_equal(out, want)
    if n <= 17:
        assert np.array_equal(want, orc.mm_bigint_ijk(A, B, n, L, RL))


@pytest.mark.parametrize("n,L", [(9, 4), (40, 32)])
def test_limbplane_signed_top_limb(gpu, orc, lib, n, L):
    """Two's complement entries (limb L-1 read as int16) through the device
    schoolbook equal the MFFT path's signed product and the oracle's exact
    entries."""
    A = orc.bigmat_rand(n, L, SEED + 3)
    B = orc.bigmat_rand(n, L, SEED_B + 3)
    RL = 2 * L + 1
    dA, dB = gpu.DevBuf(A.nbytes), gpu.DevBuf(B.nbytes)
    dA.upload(A)
    dB.upload(B)
    dCw, dO = gpu.DevBuf((2 * L - 1) * n * n * 8), gpu.DevBuf(RL * n * n * 2)
    gpu.check(lib.mfh_limbplane_mm_dev(None, gpu.MFH_IN_U16_SIGNED, dA.ptr, dB.ptr, n, L,
                                       dCw.ptr, dO.ptr, RL))
    gpu.check(lib.mfh_sync(None))
    got = dO.download(np.uint16, RL * n * n)
    for b in (dA, dB, dCw, dO):
        b.free()
    want, err = gpu.mm_mfft(A, B, n, L, gpu.plan(L), signed=True)
    assert err == 0 and np.array_equal(got, want)
    for i, j in [(0, 0), (n - 1, 2), (3, n - 1)]:
        assert np.array_equal(got.reshape(RL, n * n)[:, i * n + j],
                              orc.entry_exact(A, B, n, L, i, j, RL, signed_top=True))


def test_profile_records_device_stages(gpu, orc, lib):
    """With g_mfft_profile set, mm_mfft adds its device stage times to
    g_mfft_prof the way the reference bench reads them (src/main.c:370)."""
    n, L = 64, 64
    flag = C.c_int.in_dll(lib, "g_mfft_profile")
    prof = gpu.ProfileT.in_dll(lib, "g_mfft_prof")
    lib.mfft_profile_reset()
    flag.value = 1
    try:
        A = orc.bigmat_rand(n, L, SEED)
        B = orc.bigmat_rand(n, L, SEED_B)
        out, err = gpu.mm_mfft(A, B, n, L, gpu.plan(L))
        out2, err2 = gpu.mm_mfft(A, B, n, L, gpu.plan(L))
    finally:
        flag.value = 0
    assert err == 0 and err2 == 0 and np.array_equal(out, out2)
    assert prof.n_fft == 6 and prof.transform > 0 and prof.pointwise > 0
    assert prof.pack == 0 and prof.build_ops == 0 and prof.fold == 0
    lib.mfft_profile_print(b"mfft-hip")
