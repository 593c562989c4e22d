"""mfh_mm_dev_noalloc (the entry point that allocates nothing) against
mfh_mm_dev, the existing entry point it varies, bit for bit: two calls in a
row, the second with a smaller input, so the second runs on a scratch array
that still holds the first call's intermediates; and the size check."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _product(gpu, lib, orc, n, L, kind, seed):
    RL = 2 * L + 1
    A = orc.bigmat_rand(n, L, seed)
    B = orc.bigmat_rand(n, L, seed ^ 0xABCDEF)
    dA, dB = gpu.DevBuf(A.nbytes), gpu.DevBuf(B.nbytes)
    dA.upload(A)
    dB.upload(B)
    out_bytes = RL * n * n * 2
    dRef, dGot = gpu.DevBuf(out_bytes), gpu.DevBuf(out_bytes)
    with gpu.Ctx(n, L) as ctx:
        gpu.check(lib.mfh_mm_dev(ctx.h, kind, dA.ptr, dB.ptr, dRef.ptr, RL), "mfh_mm_dev")
        ctx.sync()
    want = dRef.download(np.uint16, RL * n * n)
    p = gpu.plan(L)
    gpu.check(lib.mfh_mm_dev_noalloc(kind, C.byref(p), n, L, dA.ptr, dB.ptr, dGot.ptr, RL,
                                     None), "mfh_mm_dev_noalloc")
    gpu.check(lib.mfh_sync(None), "mfh_sync")
    got = dGot.download(np.uint16, RL * n * n)
    return A, B, want, got


def test_noalloc_matches_mm_dev_twice(gpu, lib, orc):
    # n=64 at 1024 bits (the largest of the three), then two smaller ones
    cases = [(64, 64, gpu.MFH_IN_U16, 12345), (40, 32, gpu.MFH_IN_U16_SIGNED, 7),
             (24, 16, gpu.MFH_IN_U16, 99)]
    for n, L, kind, seed in cases:
        print(f"[noalloc] n={n} L={L} kind={kind}", flush=True)
        A, B, want, got = _product(gpu, lib, orc, n, L, kind, seed)
        assert np.array_equal(got, want), f"n={n} L={L}: {(got != want).sum()} limbs differ"
        if kind == gpu.MFH_IN_U16:
            assert np.array_equal(got, orc.mm_mfft(A, B, n, L, orc.plan(L), 2 * L + 1))


def test_noalloc_rejects_sizes_beyond_scratch(gpu, lib):
    n, L = 128, 32                      # 512-bit entries at n=128: > 64 MiB of workspace
    RL = 2 * L + 1
    dA, dB = gpu.DevBuf(L * n * n * 2), gpu.DevBuf(L * n * n * 2)
    dO = gpu.DevBuf(RL * n * n * 2)
    marker = np.full(RL * n * n, 0x5A5A, np.uint16)
    dO.upload(marker)
    p = gpu.plan(L)
    rc = lib.mfh_mm_dev_noalloc(gpu.MFH_IN_U16, C.byref(p), n, L, dA.ptr, dB.ptr, dO.ptr, RL,
                                None)
    assert rc == -8
    assert np.array_equal(dO.download(np.uint16, RL * n * n), marker)   # output untouched
