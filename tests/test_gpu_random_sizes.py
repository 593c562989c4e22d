"""Seeded random sizes, all on the device and all through independent
computations: the MFFT product (every plan the planner gives for L, the
flat and the recursive one, Gauss or flat pointwise, whole or in row bands)
against the integer-ALU schoolbook, and the matrix-core schoolbook against
it too.  Widths from 128 to 8192 bits (every ring size K = 4 .. 32), ragged
n, unsigned and two's complement entries, random limbs or limbs at the
extremes (all 0x0000 / 0xFFFF / 0x8000 runs)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

N_CASES = 40


def _limbs(rng, n, L, style):
    if style == 0:
        return rng.integers(0, 65536, L * n * n, dtype=np.uint16)
    pick = np.array([0x0000, 0xFFFF, 0x8000, 0x7FFF, 0x0001], np.uint16)
    return pick[rng.integers(0, len(pick), L * n * n)]


def _cases():
    rng = np.random.default_rng(20261202)
    out = []
    for i in range(N_CASES):
        L = int(2 ** rng.integers(3, 10))                 # 8 .. 512 limbs
        n = int(rng.integers(1, 161 if L <= 128 else 97))
        out.append((i, n, L, bool(rng.integers(0, 2)), int(rng.integers(0, 2)),
                    bool(rng.integers(0, 4) == 0)))
    return out


@pytest.mark.parametrize("i,n,L,signed,style,band", _cases())
def test_random_size_against_schoolbook(gpu, monkeypatch, i, n, L, signed, style, band):
    print(f"[random] case {i}: n={n} L={L} signed={signed} style={style} band={band}", flush=True)
    lib = gpu.load()
    rng = np.random.default_rng(1000 + i)
    A, B = _limbs(rng, n, L, style), _limbs(rng, n, L, style)
    RL = 2 * L + 1
    kind = gpu.MFH_IN_U16_SIGNED if signed else gpu.MFH_IN_U16
    dA, dB = gpu.DevBuf(A.nbytes), gpu.DevBuf(B.nbytes)
    dA.upload(A)
    dB.upload(B)
    dCw, dRef = gpu.DevBuf((2 * L - 1) * n * n * 8), gpu.DevBuf(RL * n * n * 2)
    gpu.check(lib.mfh_limbplane_mm_dev(None, kind, dA.ptr, dB.ptr, n, L, dCw.ptr, dRef.ptr, RL))
    gpu.check(lib.mfh_sync(None))
    want = dRef.download(np.uint16, RL * n * n)
    if band:
        monkeypatch.setenv("MFH_BAND_ROWS", "64")
    for p in (gpu.plan(L), gpu.plan_rec(L, n)):
        if p is None:
            continue
        with gpu.Ctx(n, L, p) as ctx:
            got = ctx.mm(A, B, RL, signed=signed)
        assert np.array_equal(got, want), (i, n, L, p.S, p.NB, p.K)
    monkeypatch.delenv("MFH_BAND_ROWS", raising=False)
    out = np.empty(RL * n * n, np.uint16)
    rc = lib.mfh_schoolbook(kind, A.ctypes.data, B.ctypes.data, n, L, out.ctypes.data, RL)
    assert rc == 0
    assert np.array_equal(out, want), (i, n, L)
