"""Stage-level parity of the device path, one size per ring size K, through
mfh_conv_stages (the product of the caller's own limbs, as conv_mfft, so the
limbs reach the transform unrecoded):

* forward: A's and B^T's int8 digit planes, recombined (K7: d0 + 2^7 d1 +
  2^14 d2, the pair-sum planes checked against their digits; B8: d0 + 2^8 d1
  + 2^16 d2), equal the oracle's forward transform (orc_fft_forward32,
  src/mfft.c:173-258) of the packed limbs (src/mfft.c:302-345), slot by slot:
  the K coefficients, or the Gauss slots [z0+z1 | z0 | z1] of A and
  [z0 | z1-z0 | -(z0+z1)] of B;
* pointwise: the int32 class results, recombined (K7: Karatsuba; B8: weights
  2^(8m)), equal the oracle's pointwise ring products of those transforms
  (src/mfft.c:383-395), C_j[t] = sum over c1+c2 = t of A_j[c1] B_j[c2] minus
  the sum over c1+c2 = t+K, as exact int64 matrix products.

A kernel regression then shows up at the stage that made it."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

STAGE_A, STAGE_B, STAGE_CLASSES = 0, 1, 2
MODE_B8, MODE_K7 = 0, 1


def bitrev(j, nbits):
    r = 0
    for _ in range(nbits):
        r = (r << 1) | (j & 1)
        j >>= 1
    return r


def tile_index(R, np_):
    """offset of entry (i, k) of an R x np plane in 16 x 64 tiles"""
    i = np.arange(R)[:, None]
    k = np.arange(np_)[None, :]
    return (((i >> 4) * (np_ >> 6) + (k >> 6)) * 1024 + (i & 15) * 64 + (k & 63)).astype(np.int64)


def digit_values(raw, NB, nslot, mode, R, np_):
    """the transformed values the digit planes encode: [NB][nslot][R][np]"""
    pl = 6 if mode == MODE_K7 else 3
    d = raw.view(np.int8).reshape(NB, nslot, pl, R * np_)[..., tile_index(R, np_)]
    d = d.astype(np.int64)
    if mode == MODE_K7:
        assert np.array_equal(d[:, :, 3], d[:, :, 0] + d[:, :, 1])
        assert np.array_equal(d[:, :, 4], d[:, :, 0] + d[:, :, 2])
        assert np.array_equal(d[:, :, 5], d[:, :, 1] + d[:, :, 2])
        assert d[:, :, :2].min() >= -64 and d[:, :, :2].max() <= 63
        return d[:, :, 0] + 128 * d[:, :, 1] + 16384 * d[:, :, 2]
    return d[:, :, 0] + 256 * d[:, :, 1] + 65536 * d[:, :, 2]


def oracle_transform(orc, X32, n, L, p):
    """[NB][K][n][n] int64: point j (natural order) of the transform of the
    limbs packed into NB blocks of K coefficients (S limbs each)"""
    nn = n * n
    X = np.zeros((p.NB, p.K, nn), np.int32)
    planes = X32.reshape(L, nn)
    for b in range(L // p.S):
        X[b, :p.S] = planes[b * p.S:(b + 1) * p.S]
    orc.fft_forward32(X, p.NB, p.K, p.g, nn)
    lg = p.NB.bit_length() - 1
    return np.stack([X[bitrev(j, lg)] for j in range(p.NB)]).astype(np.int64).reshape(
        p.NB, p.K, n, n)


def slots(z, gauss, side):
    """operand slots of a point's K coefficients z (axis 1)"""
    if not gauss:
        return z
    H = z.shape[1] // 2
    z0, z1 = z[:, :H], z[:, H:]
    if side == 0:
        return np.concatenate([z0 + z1, z0, z1], axis=1)
    return np.concatenate([z0, z1 - z0, -(z0 + z1)], axis=1)


def pad(v, R, np_):
    """[..][n][n] -> [..][R][np] with zeros outside"""
    out = np.zeros(v.shape[:-2] + (R, np_), np.int64)
    out[..., :v.shape[-2], :v.shape[-1]] = v
    return out


@pytest.mark.parametrize("n,L,full", [(20, 8, True), (20, 32, True), (24, 64, True),
                                      (24, 128, True), (20, 256, True), (20, 512, True),
                                      (36, 512, False)])
def test_forward_and_pointwise_stages(gpu, orc, n, L, full):
    p = gpu.plan(L)
    print(f"[stages] n={n} L={L} S={p.S} NB={p.NB} K={p.K} full={full}", flush=True)
    rng = np.random.default_rng(n * 1000 + L)
    lim = 65535 if full else 2000
    A32 = rng.integers(-lim, lim + 1, size=L * n * n).astype(np.int32)
    B32 = rng.integers(-lim, lim + 1, size=L * n * n).astype(np.int32)
    Ah = oracle_transform(orc, A32, n, L, p)
    Bh = oracle_transform(orc, B32, n, L, p)
    with gpu.Ctx(n, L, p) as ctx:
        (mode, pw, R, np_, _), rawA = ctx.stages(A32, B32, STAGE_A)
        info_b, rawB = ctx.stages(A32, B32, STAGE_B)
        info_c, rawC = ctx.stages(A32, B32, STAGE_CLASSES)
    assert info_b[:4] == info_c[:4] == (mode, pw, R, np_)
    assert R >= n and np_ >= n
    gauss = pw == 1
    nslot = 3 * p.K // 2 if gauss else p.K
    # forward: A and B^T
    va = digit_values(rawA, p.NB, nslot, mode, R, np_)
    assert np.array_equal(va, pad(slots(Ah, gauss, 0), R, np_))
    vb = digit_values(rawB, p.NB, nslot, mode, np_, np_)
    assert np.array_equal(vb, pad(np.swapaxes(slots(Bh, gauss, 1), -1, -2), np_, np_))
    # pointwise: the negacyclic ring product at every point
    K = p.K
    Ch = np.zeros((p.NB, K, n, n), np.int64)
    for c1 in range(K):
        prod = np.matmul(Ah[:, c1:c1 + 1], Bh)           # [NB][K][n][n], c2 along axis 1
        for c2 in range(K):
            t = c1 + c2
            if t < K:
                Ch[:, t] += prod[:, c2]
            else:
                Ch[:, t - K] -= prod[:, c2]
    ncl = 6 if mode == MODE_K7 else 5
    c5 = rawC.view(np.int32).reshape(p.NB, R, ncl, np_ // 16, K // 4, 16, 4).astype(np.int64)
    c5 = c5.transpose(0, 2, 1, 3, 5, 4, 6).reshape(p.NB, ncl, R, np_, K)   # [j][m][i][j'][t]
    cls = [c5[:, m] for m in range(ncl)]
    if mode == MODE_K7:
        P0, P1, P2, P3, P4, P5 = cls
        got = (P0 + (P3 - P0 - P1) * 128 + (P4 - P0 - P2 + P1) * 16384 +
               (P5 - P1 - P2) * 2097152 + P2 * 268435456)
    else:
        got = sum(cls[m] * (256 ** m) for m in range(ncl))
    want = pad(Ch, R, np_).transpose(0, 2, 3, 1)                          # [j][i][j'][t]
    assert np.array_equal(got, want)


def test_stage_info_without_output(gpu):
    """info alone (out NULL) reports the layout without running anything"""
    p = gpu.plan(128)
    n = 16
    A = np.zeros(128 * n * n, np.int32)
    with gpu.Ctx(n, 128, p) as ctx:
        info = (gpu.C.c_int64 * 5)()
        assert ctx.lib.mfh_conv_stages(ctx.h, A.ctypes.data, A.ctypes.data, 0, None, 0,
                                       info) == 0
        mode, pw, R, np_, nbytes = (int(v) for v in info)
        assert (mode, pw, np_) == (MODE_K7, 1, 64)
        assert nbytes == p.NB * 24 * 6 * R * np_
        assert ctx.lib.mfh_conv_stages(ctx.h, A.ctypes.data, A.ctypes.data, 3, None, 0,
                                       info) < 0
