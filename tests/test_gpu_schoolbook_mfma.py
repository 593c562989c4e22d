"""The limb-plane schoolbook on the matrix cores (mfh_schoolbook,
src/methods.c:94-123): K7 digit planes of the limbs convolved over the limb
axis with int8 MFMA in 16-limb blocks, the six Karatsuba classes recombined
and carried.  Checked against the oracle's schoolbook and the integer-ALU
device schoolbook, for unsigned and two's complement entries, ragged n and
L, short and long outputs, the coefficient planes (RL = 0), the class
partials at the edge of their int32 range (decoded from their residue), the
size bound, and mm_limbplane's routing."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

U16, U16_SIGNED = 0, 1


def sb(gpu, A, B, n, L, RL, kind=U16):
    lib = gpu.load()
    out = np.empty(RL * n * n if RL else (2 * L - 1) * n * n, np.uint16 if RL else np.int64)
    rc = lib.mfh_schoolbook(kind, A.ctypes.data, B.ctypes.data, n, L, out.ctypes.data, RL)
    assert rc == 0, rc
    return out


def signed_conv(orc, A, B, n, L):
    nn = n * n
    A32, B32 = A.astype(np.int32), B.astype(np.int32)
    A32[(L - 1) * nn:] = A[(L - 1) * nn:].view(np.int16)
    B32[(L - 1) * nn:] = B[(L - 1) * nn:].view(np.int16)
    return orc.conv_limbplane(A32, B32, n, L)


@pytest.mark.parametrize("n,L", [(8, 1), (8, 4), (20, 17), (64, 16), (33, 40), (100, 64),
                                  (70, 128), (16, 512), (130, 33)])
def test_schoolbook_matches_oracle(gpu, orc, n, L):
    print(f"[schoolbook] n={n} L={L}", flush=True)
    A = orc.bigmat_rand(n, L, 11 + L)
    B = orc.bigmat_rand(n, L, 12 + n)
    RL = 2 * L + 1
    assert np.array_equal(sb(gpu, A, B, n, L, RL), orc.mm_limbplane(A, B, n, L, RL))
    want_cw = orc.conv_limbplane(A.astype(np.int32), B.astype(np.int32), n, L)
    assert np.array_equal(sb(gpu, A, B, n, L, 0), want_cw)
    want_s = orc.normalize(signed_conv(orc, A, B, n, L), 2 * L - 1, n, RL)
    assert np.array_equal(sb(gpu, A, B, n, L, RL, U16_SIGNED), want_s)


@pytest.mark.parametrize("L,RL", [(16, 1), (16, 7), (40, 81), (40, 200), (128, 3)])
def test_schoolbook_short_and_long_outputs(gpu, orc, L, RL):
    n = 24
    A = orc.bigmat_rand(n, L, 5)
    B = orc.bigmat_rand(n, L, 6)
    want = orc.normalize(orc.conv_limbplane(A.astype(np.int32), B.astype(np.int32), n, L),
                         2 * L - 1, n, RL)
    assert np.array_equal(sb(gpu, A, B, n, L, RL), want)


def test_schoolbook_partials_at_their_range_edge(gpu):
    """Every limb 8128 = -64 - 64*128 + 2^14: digits (-64, -64, 1), so the
    class of (d0+d1)(d0+d1) multiplies -128 by -128 everywhere.  At n = 1024,
    L = 128 its partials for the middle limb blocks reach 2^31 (16 pairs x 8
    blocks x 1024 k x 2^14), one past the int32 maximum; the residue decode
    must still give the exact product, here n X^2 with X = 8128 sum 2^(16u)."""
    n, L = 1024, 128
    RL = 2 * L + 1
    A = np.full(L * n * n, 8128, np.uint16)
    out = sb(gpu, A, A, n, L, RL).reshape(RL, n * n)
    X = sum(8128 << (16 * u) for u in range(L))
    v = n * X * X
    want = np.array([(v >> (16 * w)) & 0xFFFF for w in range(RL)], np.uint16)
    assert np.array_equal(out[:, 0], want)
    assert (out == out[:, :1]).all()


def test_schoolbook_all_ones_and_alu_agree(gpu, orc):
    """0xFFFF limbs (unsigned: 2^W - 1; signed: -1) and random limbs at
    n = 256, 2048 bits: the matrix-core and the integer-ALU schoolbooks give
    the same limbs."""
    n, L = 256, 128
    RL = 2 * L + 1
    lib = gpu.load()
    for A in (np.full(L * n * n, 0xFFFF, np.uint16), orc.bigmat_rand(n, L, 9)):
        B = orc.bigmat_rand(n, L, 10)
        for kind in (U16, U16_SIGNED):
            alu = gpu.DevBuf((2 * L - 1) * n * n * 8)
            dA, dB, dO = gpu.DevBuf(A.nbytes), gpu.DevBuf(B.nbytes), gpu.DevBuf(RL * n * n * 2)
            dA.upload(A)
            dB.upload(B)
            assert lib.mfh_limbplane_mm_dev(None, kind, dA.ptr, dB.ptr, n, L, alu.ptr, dO.ptr,
                                            RL) == 0
            want = dO.download(np.uint16, RL * n * n)
            assert np.array_equal(sb(gpu, A, B, n, L, RL, kind), want)


def test_schoolbook_bound_and_routing(gpu, orc):
    """ceil(L/16) n above 8224 is refused with MFH_E_BOUND, and
    mm_limbplane then runs the integer-ALU schoolbook.  A's entries are 1,
    so C[i][j] is the column sum of B (limb w: sum_k B_w[k][j], then the
    carry): n = 128 (bound met: matrix cores) and n = 130 (ALU) at 16384
    bits both give it."""
    lib = gpu.load()
    bound = [k for k, v in gpu.ERRORS.items() if v == "MFH_E_BOUND"][0]
    b = C.c_size_t()
    assert lib.mfh_schoolbook_workspace(1024, 128, C.byref(b)) == 0
    assert lib.mfh_schoolbook_workspace(1040, 128, C.byref(b)) == bound
    L = 1024
    for n in (128, 130):
        nn = n * n
        A = np.zeros(L * nn, np.uint16)
        A[:nn] = 1
        B = orc.bigmat_rand(n, L, 23)
        RL = 2 * L + 1
        cw = np.zeros((2 * L - 1, n, n), np.int64)
        cw[:L] = B.reshape(L, n, n).astype(np.int64).sum(axis=1)[:, None, :]
        want = orc.normalize(cw.reshape(-1), 2 * L - 1, n, RL)
        out = np.empty(RL * nn, np.uint16)
        lib.mm_limbplane(A.ctypes.data, B.ctypes.data, n, L, gpu.KERNEL_HIP, out.ctypes.data, RL)
        assert lib.mfft_last_error() == 0
        assert np.array_equal(out, want), n
        got = np.empty(RL * nn, np.uint16)
        rc = lib.mfh_schoolbook(U16, A.ctypes.data, B.ctypes.data, n, L, got.ctypes.data, RL)
        assert rc == (0 if n == 128 else bound)
        if n == 128:
            assert np.array_equal(got, want)
