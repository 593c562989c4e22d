"""The CPU oracle (oracle/) pinned against golden fixtures, known answers,
definitions and -- where it was built -- the reference's own C library.

A check here fails for the plausible mistakes: a dropped term, a wrong
sign, a transposed operand, a wrong twiddle or bit order."""
import json
import os
import struct

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SEED, SEED_B = 12345, 12345 ^ 0xABCDEF


def load(name):
    with open(os.path.join(GOLD, name)) as f:
        return json.load(f)


# ---- SplitMix64 inputs ---------------------------------------------------------
def test_splitmix_published_values(orc):
    # published SplitMix64 outputs for seed 0
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    assert load("splitmix.json")["seed0"][:3] == want
    m = orc.bigmat_rand(1, 3, 0)                       # low 16 bits, in order
    assert list(m) == [w & 0xFFFF for w in want]


def test_bigmat_rand_plane_major_order(orc):
    sm = load("splitmix.json")["seed12345"]
    m = orc.bigmat_rand(2, 1, SEED)                    # 4 limbs: one plane of 2x2
    assert list(m) == [w & 0xFFFF for w in sm]


def test_bigmat_rand_matches_reference(orc, ref):
    for n, L, s in [(3, 4, 1), (16, 8, SEED), (5, 128, SEED_B)]:
        assert np.array_equal(orc.bigmat_rand(n, L, s), ref.bigmat_rand(n, L, s))


# ---- exact products against Python big-integer fixtures ---------------------
@pytest.mark.parametrize("case", range(len(load("products.json"))))
def test_products_fixture(orc, case):
    c = load("products.json")[case]
    n, L, RL = c["n"], c["L"], c["RL"]
    A = orc.bigmat_rand(n, L, c["seed_a"])
    B = orc.bigmat_rand(n, L, c["seed_b"])
    want = np.array(c["out"], dtype=np.uint16)
    for i in range(n):
        for j in range(n):
            got = orc.entry_exact(A, B, n, L, i, j, RL, signed_top=c["signed"])
            assert np.array_equal(got, want.reshape(RL, n * n)[:, i * n + j])
    if c["signed"]:
        return
    assert np.array_equal(orc.mm_limbplane(A, B, n, L, RL), want)
    assert np.array_equal(orc.mm_bigint_ijk(A, B, n, L, RL), want)
    p = orc.plan(L)
    assert p is not None
    assert np.array_equal(orc.mm_mfft(A, B, n, L, p, RL), want)
    assert np.array_equal(orc.mm_mfft(A, B, n, L, p, RL, leaf=0), want)


def test_signed_products_via_conv(orc):
    """Two's complement entries: conv of the int32 limbs (top limb int16)
    normalised to 2L+1 limbs equals the fixture."""
    for c in load("products.json"):
        if not c["signed"]:
            continue
        n, L, RL = c["n"], c["L"], c["RL"]
        A = orc.bigmat_rand(n, L, c["seed_a"]).astype(np.int32)
        B = orc.bigmat_rand(n, L, c["seed_b"]).astype(np.int32)
        top = slice((L - 1) * n * n, L * n * n)
        A[top] = A[top].astype(np.uint16).view(np.int16)
        B[top] = B[top].astype(np.uint16).view(np.int16)
        cw = orc.conv_mfft(A, B, n, L, orc.plan(L))
        got = orc.normalize(cw, 2 * L - 1, n, RL)
        assert np.array_equal(got, np.array(c["out"], dtype=np.uint16))


def test_normalize_fixture(orc):
    for c in load("normalize.json"):
        acc = np.array(c["acc"], dtype=np.int64)
        got = orc.normalize(acc, c["nplanes"], c["n"], c["RL"])
        assert np.array_equal(got, np.array(c["out"], dtype=np.uint16))


# ---- ring transform -------------------------------------------------------------
def poly_eval_dft(x, NB, K, g, direction):
    """X[j] = sum_b (y^(g j b dir) * x_b) mod (y^K + 1), computed by explicit
    polynomial multiplication (not by shifting)."""
    X = np.zeros((NB, K), dtype=object)
    for j in range(NB):
        acc = [0] * (2 * K)
        for b in range(NB):
            e = (direction * g * j * b) % (2 * K)
            mono = [0] * (2 * K)
            mono[e] = 1                                  # y^e, e < 2K
            prod = [0] * (4 * K)
            for a in range(2 * K):
                for c in range(K):
                    prod[a + c] += mono[a] * int(x[b][c])
            for d in range(4 * K):                       # reduce: y^K = -1
                q, r = divmod(d, K)
                acc[r] += prod[d] * (-1) ** q
        X[j] = acc[:K]
    return X


@pytest.mark.parametrize("NB,K", [(4, 4), (8, 4), (8, 8), (4, 8), (16, 16)])
def test_ring_dft_definition(orc, NB, K):
    g = 2 * K // NB
    rng = np.random.default_rng(NB * 100 + K)
    x = rng.integers(-1000, 1000, size=(NB, K)).astype(np.int64)
    want = poly_eval_dft(x, NB, K, g, 1).astype(np.int64)
    got = orc.ring_dft(x.reshape(-1), NB, K, g, 1).reshape(NB, K)
    assert np.array_equal(got, want)
    back = orc.ring_dft(got.reshape(-1), NB, K, g, -1).reshape(NB, K)
    assert np.array_equal(back, NB * x)                 # inverse(forward) = NB id


@pytest.mark.parametrize("NB,K", [(8, 4), (16, 8), (32, 16)])
def test_radix2_transforms_are_the_dft(orc, NB, K):
    """orc_fft_forward32 = DFT in bit-reversed order; orc_fft_inverse64 of
    that = NB * input (mfft.c:225-299 semantics)."""
    g = 2 * K // NB
    nn = 3
    rng = np.random.default_rng(K)
    x = rng.integers(-5000, 5000, size=(NB, K, nn)).astype(np.int32)
    X = x.copy()
    orc.lib.orc_fft_forward32(X.ctypes.data, NB, K, g, nn)
    lg = NB.bit_length() - 1
    for e in range(nn):
        want = orc.ring_dft(x[:, :, e].astype(np.int64).reshape(-1), NB, K, g, 1).reshape(NB, K)
        for p in range(NB):
            j = int(format(p, f"0{lg}b")[::-1], 2)
            assert np.array_equal(X[p, :, e], want[j])
    Y = X.astype(np.int64)
    orc.lib.orc_fft_inverse64(Y.ctypes.data, NB, K, g, nn)
    assert np.array_equal(Y, NB * x.astype(np.int64))


# ---- convolution cores ------------------------------------------------------------
@pytest.mark.parametrize("n,L,sigma", [(5, 8, 0), (4, 32, 0), (3, 32, 3), (6, 64, 0), (2, 128, 0)])
def test_conv_mfft_equals_limbplane_signed_limbs(orc, n, L, sigma):
    rng = np.random.default_rng(L + n)
    A = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    B = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    p = orc.plan(L, sigma)
    assert np.array_equal(orc.conv_mfft(A, B, n, L, p), orc.conv_limbplane(A, B, n, L))


def test_plans(orc):
    # src/mfft.c:77-95: S = 2^(floor(log2 L)/2), NB = 2L/S, K = 2S
    for L, (S, NB, K) in {2: (2, 2, 4), 4: (2, 4, 4), 64: (8, 16, 16), 128: (8, 32, 16),
                          512: (16, 64, 32), 32: (4, 16, 8)}.items():
        p = orc.plan(L)
        assert (p.S, p.NB, p.K, p.g, p.nprod) == (S, NB, K, 2 * K // NB, NB * K * K)
    assert orc.plan(3) is None and orc.plan(1) is None
    assert orc.plan(32, 6) is None                     # sigma > log2 L


# ---- reference library, where built -----------------------------------------------
@pytest.mark.parametrize("n,L,sigma", [(8, 8, 0), (16, 16, 0), (8, 32, 3), (8, 64, 0),
                                       (6, 512, 0), (64, 64, 0), (7, 128, 0), (5, 1024, 0)])
def test_mm_mfft_matches_reference(orc, ref, n, L, sigma):
    A = orc.bigmat_rand(n, L, SEED)
    B = orc.bigmat_rand(n, L, SEED_B)
    RL = 2 * L + 1
    got = orc.mm_mfft(A, B, n, L, orc.plan(L, sigma), RL)
    want = ref.mm_mfft(A, B, n, L, ref.plan(L, sigma), RL)
    assert np.array_equal(got, want)


def test_conv_mfft_matches_reference(orc, ref):
    n, L = 6, 32
    rng = np.random.default_rng(3)
    A = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    B = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    assert np.array_equal(orc.conv_mfft(A, B, n, L, orc.plan(L)),
                          ref.conv_mfft(A, B, n, L, ref.plan(L)))


# ---- fp32 embedding ------------------------------------------------------------------
def bits_to_f32(bits):
    return np.array(bits, dtype=np.uint32).view(np.float32)


@pytest.mark.parametrize("case", range(3))
def test_fpx_roundtrip_fixture(orc, case):
    c = load("fpx.json")[case]
    n = c["n"]
    A, B = bits_to_f32(c["A_bits"]), bits_to_f32(c["B_bits"])
    assert np.array_equal(A, orc.fp32_rand(n * n, c["seed_a"], c["emin"], c["emax"]))
    ctx = orc.fpx(A, B, n, 512)
    A32, B32 = orc.fpx_planes(ctx)
    cw = orc.conv_limbplane(A32, B32, n, ctx.L)
    got = orc.fpx_decode_from(ctx, cw)
    orc.fpx_free(ctx)
    assert np.array_equal(got.view(np.uint32), np.array(c["C_bits"], dtype=np.uint32))


def test_fpx_rounding_edges(orc):
    """Ties to even, sticky bit, negative results and exact zero (+0.0)."""
    n = 2
    one = np.float32(1.0)
    # C[0][0] = 1 + 2^-24 (tie -> even: 1.0); C[0][1] = 1 + 3*2^-24 (tie -> up)
    A = np.array([one, np.float32(2.0 ** -24), np.float32(-1.0), np.float32(0)], np.float32)
    B = np.array([one, one, one, np.float32(3.0)], np.float32)
    ctx = orc.fpx(A, B, n, 512)
    A32, B32 = orc.fpx_planes(ctx)
    got = orc.fpx_decode_from(ctx, orc.conv_limbplane(A32, B32, n, ctx.L))
    orc.fpx_free(ctx)
    want = np.array([1.0, 1.0 + 3 * 2.0 ** -24, -1.0, -1.0], np.float64)
    # exact: row0 = [1 + 2^-24, 1 + 3*2^-24]; row1 = [-1, -1]
    assert got[0] == np.float32(1.0)
    assert got[1] == np.float32(1.0 + 2.0 ** -22)          # 1 + 3*2^-24 rounds up (tie, odd)
    assert got[2] == np.float32(-1.0) and got[3] == np.float32(-1.0)
    Z = np.zeros(4, np.float32)
    ctx = orc.fpx(Z, B, n, 512)
    A32, B32 = orc.fpx_planes(ctx)
    z = orc.fpx_decode_from(ctx, orc.conv_limbplane(A32, B32, n, ctx.L))
    orc.fpx_free(ctx)
    assert np.all(z.view(np.uint32) == 0)                  # +0.0f, not -0.0f
    del want


def test_fpx_matches_reference(orc, ref):
    n = 8
    A = orc.fp32_rand(n * n, 5, -20, 20)
    B = orc.fp32_rand(n * n, 6, -20, 20)
    want, L, SA, SB, cw_ref = ref.fpx_mfft_f32(A, B, n, 512)
    ctx = orc.fpx(A, B, n, 512)
    assert (ctx.L, ctx.SA, ctx.SB) == (L, SA, SB)
    A32, B32 = orc.fpx_planes(ctx)
    cw = orc.conv_mfft(A32, B32, n, L, orc.plan(L))
    assert np.array_equal(cw, cw_ref)
    got = orc.fpx_decode_from(ctx, cw)
    orc.fpx_free(ctx)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---- checkers -------------------------------------------------------------------------
def test_freivalds_accepts_and_rejects(orc):
    n, L = 12, 16
    RL = 2 * L + 1
    A = orc.bigmat_rand(n, L, SEED)
    B = orc.bigmat_rand(n, L, SEED_B)
    out = orc.mm_limbplane(A, B, n, L, RL)
    assert orc.freivalds(A, B, n, L, out, RL)
    for w, e in [(0, 0), (L, 7), (2 * L - 1, n * n - 1)]:
        bad = out.copy()
        bad[w * n * n + e] ^= 1                            # one wrong limb bit
        assert not orc.freivalds(A, B, n, L, bad, RL)
    # transposed product must fail
    assert not orc.freivalds(B, A, n, L, out, RL)


def test_freivalds_conv_rejects_planted_error(orc):
    n, L = 5, 8
    rng = np.random.default_rng(9)
    A = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    B = rng.integers(-65535, 65536, size=L * n * n).astype(np.int32)
    cw = orc.conv_limbplane(A, B, n, L)
    assert orc.freivalds_conv(A, B, n, L, cw)
    cw[3 * n * n + 2] += 1
    assert not orc.freivalds_conv(A, B, n, L, cw)


# ---- the post's roots of unity (the reference's only known-answer arrays) --------
def roots_build_H(s):
    """H_{s,k} recursion of the post, as restated in src/roots.c:32-55."""
    K, N, half = 1 << s, 1 << (s + 1), (1 << s) // 2
    H = [list(range(1, K + 1))]
    for _ in range(1, N):
        prev, cur = H[-1], []
        for j in range(1, K + 1):
            if j == 1:
                v = -prev[K - 1]
            elif j == 2:
                v = prev[K - 2]
            elif j <= half:
                v = prev[half + j - 3]
            else:
                v = prev[j - half - 1]
            cur.append(v)
        H.append(cur)
    return H


def h_matrix(row, K):
    M = np.zeros((K, K), dtype=np.int64)
    for j, v in enumerate(row):
        M[j, abs(v) - 1] = 1 if v > 0 else -1
    return M


def test_roots_post_arrays_and_order():
    # arrays printed in the post (src/roots.c:118-122)
    assert roots_build_H(1)[1] == [-2, 1]
    assert roots_build_H(2)[1] == [-4, 3, 1, 2]
    assert roots_build_H(2)[3] == [-3, -4, -2, 1]
    assert roots_build_H(3)[1] == [-8, 7, 5, 6, 1, 2, 3, 4]
    assert roots_build_H(3)[5] == [-7, -8, -6, 5, -2, 1, -4, 3]
    for s in range(1, 5):
        K = 1 << s
        H = roots_build_H(s)
        I = h_matrix(H[1], K)
        P = np.eye(K, dtype=np.int64)
        for k in range(1, 2 * K + 1):
            P = P @ I
            if k < 2 * K:
                assert np.array_equal(P, h_matrix(H[k], K))
            if k == K:
                assert np.array_equal(P, -np.eye(K, dtype=np.int64))   # I^K = -1
        assert np.array_equal(P, np.eye(K, dtype=np.int64))            # order 2K


# ---- fp64 embedding and the long double decode ---------------------------------
def bits_to_f64(bits):
    return np.array(bits, dtype=np.uint64).view(np.float64)


@pytest.mark.parametrize("case", range(4))
def test_fpx64_fixture(orc, case):
    """Encode, exact product and decode against Fraction arithmetic: rounding
    to nearest-even where the top 4-limb window is wider than the target,
    the window as it stands where it is not (fpx64.json)."""
    c = load("fpx64.json")[case]
    n = c["n"]
    A, B = bits_to_f64(c["A_bits"]), bits_to_f64(c["B_bits"])
    ctx = orc.fpx_d(A, B, n, c["force_bits"])
    A32, B32 = orc.fpx_planes(ctx)
    cw = orc.conv_limbplane(A32, B32, n, ctx.L)
    got = orc.fpx_decode_f64_from(ctx, cw)
    sig, ex = orc.fpx_decode_sig63_from(ctx, cw)
    orc.fpx_free(ctx)
    assert np.array_equal(got.view(np.uint64), np.array(c["C64_bits"], dtype=np.uint64))
    assert sig.tolist() == c["ld_sig"] and ex.tolist() == c["ld_ex"]


def test_fpx64_fixture_covers_both_regimes():
    cases = load("fpx64.json")
    assert all(c["truncated_f64"] > 0 for c in cases)
    edges = next(c for c in cases if c["name"] == "edges")
    C64 = bits_to_f64(edges["C64_bits"]).reshape(4, 4)
    assert C64[0, 0] == 64.0                       # window kept: not 64 + 2^-46
    assert C64[1, 0] == 1.0 and C64[1, 1] == 1.0 + 2.0 ** -51    # ties: even, up
    assert C64[3, 0] == -(1.0 + 2.0 ** -52) and C64[3, 1] == -(1.0 + 2.0 ** -51)
    assert C64[2, 2] == 2.0 ** -1073               # subnormal, ties to even
    assert np.all(C64[:, 3].view(np.uint64) == 0) and C64[2, 1].view(np.uint64) == 0


def test_fpx64_encode_limbs_sum_to_value(orc):
    """sum_u A32[u] 2^(16u) == x 2^SA exactly, for every entry on the grid."""
    from fractions import Fraction
    n = 5
    rng = np.random.default_rng(3)
    A = (rng.standard_normal(n * n) * 2.0 ** rng.integers(-40, 40, n * n)).astype(np.float64)
    A[3] = 0.0
    A[7] = -A[7]
    ctx = orc.fpx_d(A, A, n, 0)
    A32, _ = orc.fpx_planes(ctx)
    L, SA = ctx.L, ctx.SA
    orc.fpx_free(ctx)
    planes = A32.reshape(L, n * n)
    for e in range(n * n):
        v = sum(int(planes[u, e]) << (16 * u) for u in range(L))
        assert Fraction(v) == Fraction(float(A[e])) * Fraction(2) ** SA
        assert np.all(np.abs(planes[:, e]) <= 65535)
        assert np.count_nonzero(planes[:, e]) <= 5


def test_fpx64_matches_reference(orc, ref):
    for n, force, emin, emax in [(6, 0, -20, 20), (5, 2048, -60, 60), (4, 0, -500, 500)]:
        rng = np.random.default_rng(n + force)
        A = np.ldexp(rng.uniform(1, 2, n * n) * rng.choice([-1, 1], n * n),
                     rng.integers(emin, emax + 1, n * n))
        B = np.ldexp(rng.uniform(1, 2, n * n) * rng.choice([-1, 1], n * n),
                     rng.integers(emin, emax + 1, n * n))
        A[0] = 0.0
        want64, want_ld, L, SA, SB, rA, rB, rcw = ref.fpx_f64(A, B, n, force)
        ctx = orc.fpx_d(A, B, n, force)
        assert (ctx.L, ctx.SA, ctx.SB) == (L, SA, SB)
        A32, B32 = orc.fpx_planes(ctx)
        assert np.array_equal(A32, rA) and np.array_equal(B32, rB)
        cw = orc.conv_limbplane(A32, B32, n, L)
        assert np.array_equal(cw, rcw)
        got = orc.fpx_decode_f64_from(ctx, cw)
        sig, ex = orc.fpx_decode_sig63_from(ctx, cw)
        orc.fpx_free(ctx)
        assert np.array_equal(got.view(np.uint64), want64.view(np.uint64))
        ld = np.ldexp(sig.astype(np.longdouble), ex)
        assert np.array_equal(ld, want_ld)
