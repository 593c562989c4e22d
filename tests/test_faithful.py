"""The faithful limb-window products of the fixed-point floats (the
fp32->mfft-faithful and fp64->mfft-faithful rows, src/mlgemm.c:593-630,
909-961, 1186-1250).

CPU: the oracle's window and faithful product are pinned to the reference's
own ml_run (oracle/_ref, run in a subprocess): on the ML track's data,
reproduced here from its seeded generator (src/mlgemm.c:657-716), the window
the reference prints (L_keep, live hi, u0) and the relative error it prints
for each faithful row must equal the oracle's.  GPU: fpx_faithful_f32 /
fpx_faithful_f64 against the oracle, bit for bit."""
import ctypes as C
import os
import re
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ML_SEED = 987654321
M64 = (1 << 64) - 1


def ml_inputs(n, illcond):
    """fp32 data of the ML track, promoted to fp64 for the double rows
    (src/mlgemm.c:657-716, default data mode)"""
    s = ML_SEED

    def sm():
        nonlocal s
        s = (s + 0x9E3779B97F4A7C15) & M64
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        return z ^ (z >> 31)

    nn = n * n
    A = np.array([(sm() >> 11) / 9007199254740992.0 * 2.0 - 1.0 for _ in range(nn)])
    A = A.astype(np.float32)
    B = np.array([(sm() >> 11) / 9007199254740992.0 * 2.0 - 1.0 for _ in range(nn)])
    B = B.astype(np.float32)
    dA, dB = A.astype(np.float64), B.astype(np.float64)
    if illcond > 0:
        eA = np.array([sm() % (illcond + 1) - illcond // 2 for _ in range(nn)], np.int32)
        eB = np.array([sm() % (illcond + 1) - illcond // 2 for _ in range(nn)], np.int32)
        A, dA = np.ldexp(A, eA).astype(np.float32), np.ldexp(dA, eA)
        B, dB = np.ldexp(B, eB).astype(np.float32), np.ldexp(dB, eB)
    return A, B, dA, dB


def rel_err(Cv, R):
    """src/mlgemm.c:563-590, in long double"""
    d = Cv.astype(np.longdouble) - R.astype(np.longdouble)
    den = np.sum(R.astype(np.longdouble) ** 2)
    return float(np.sqrt(np.sum(d * d) / den)) if den > 0 else 0.0


def oracle_faithful(orc, A, B, dA, dB, n, fp_width):
    """(window, error) of the fp32 row (max_keep 1, fp_width grid) and of the
    fp64 row (max_keep 2, grid from the data), as ml_run computes them"""
    out = {}
    fx = orc.fpx(A, B, n, fp_width)
    a, b = orc.fpx_planes(fx)
    exact = orc.conv_limbplane(a, b, n, fx.L)
    sig, ex = orc.fpx_decode_sig63_from(fx, exact)
    R = np.ldexp(sig.astype(np.longdouble), ex)
    cw, Lk, u0 = orc.faithful_cw(fx, 1)
    _, _, hi = orc.faithful_window(fx, 1)
    out["fp32"] = ((Lk, fx.L, hi, u0), rel_err(orc.fpx_decode_from(fx, cw), R))
    orc.fpx_free(fx)
    dx = orc.fpx_d(dA, dB, n, 0)
    a, b = orc.fpx_planes(dx)
    Rd = orc.fpx_decode_f64_from(dx, orc.conv_limbplane(a, b, n, dx.L))
    cw, Lk, u0 = orc.faithful_cw(dx, 2)
    _, _, hi = orc.faithful_window(dx, 2)
    out["fp64"] = ((Lk, dx.L, hi, u0), rel_err(orc.fpx_decode_f64_from(dx, cw), Rd))
    orc.fpx_free(dx)
    return out


def reference_ml_run(n, fp_width, illcond):
    """the reference's ml_run (oracle/_ref) in a subprocess: the windows and
    errors it prints for the two faithful rows"""
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from oracle_ctypes import load_reference\n"
            "import ctypes as C\n"
            "r = load_reference()\n"
            "r.lib.ml_run.argtypes = [C.c_int] * 8\n"
            "sys.exit(r.lib.ml_run(%d, 1, 0, 0, %d, %d, 0, 0))\n"
            % (os.path.join(ROOT, "oracle"), n, fp_width, illcond))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                         timeout=300, cwd="/tmp").stdout
    got = {}
    for kind in ("fp32", "fp64"):
        m = re.search(kind + r"->mfft-faithful: L_keep=(\d+) of (\d+) \(live hi=(\d+) u0=(\d+)\)",
                      out)
        e = re.search(r"^" + kind + r"->mfft-faithful\s+\S+\s+\S+\s+\S+x\s+(\S+)\s+<-", out, re.M)
        if m and e:
            got[kind] = (tuple(int(x) for x in m.groups()), e.group(1))
    return got


@pytest.mark.parametrize("fp_width,illcond", [(0, 0), (0, 6), (0, 24), (512, 0), (256, 10)])
def test_faithful_rows_match_reference_ml_run(ref, orc, fp_width, illcond):
    n = 32
    want = reference_ml_run(n, fp_width, illcond)
    assert set(want) == {"fp32", "fp64"}, want
    A, B, dA, dB = ml_inputs(n, illcond)
    got = oracle_faithful(orc, A, B, dA, dB, n, fp_width)
    for kind in ("fp32", "fp64"):
        assert got[kind][0] == want[kind][0], (kind, got[kind][0], want[kind][0])
        assert "%.2e" % got[kind][1] == want[kind][1], (kind, got[kind][1], want[kind][1])


def test_faithful_window_rule_cases(orc):
    """The window on hand-made planes: the top live plane of A or B, the
    largest power of two that fits below it, max_keep and L, never less
    than two limbs when two are allowed and live."""
    n = 4
    A = np.zeros(n * n, np.float32)
    B = np.zeros(n * n, np.float32)
    A[0], B[3] = 1.0, 2.0 ** 40                      # B's entry sits 40 bits higher
    fx = orc.fpx(A, B, n, 512)
    hi = orc.faithful_window(fx, 1)[2]
    top = fx.SB + 40 + 1                              # bit length of 2^40 * 2^SB
    assert hi == (top - 1) // 16
    assert orc.faithful_window(fx, 1)[:2] == (1, hi)
    assert orc.faithful_window(fx, 2)[:2] == (2, hi - 1)
    assert orc.faithful_window(fx, 3)[:2] == (2, hi - 1)
    assert orc.faithful_window(fx, 8)[:2] == (8, hi - 7)
    assert orc.faithful_window(fx, 1000)[0] == min(fx.L, 1 << (hi + 1).bit_length() - 1)
    orc.fpx_free(fx)
    Z = np.zeros(n * n, np.float32)                  # nothing live: the top plane
    fz = orc.fpx(Z, Z, n, 512)
    assert orc.faithful_window(fz, 2) == (2, fz.L - 2, fz.L - 1)
    orc.fpx_free(fz)


# ---- on the device --------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("n,fp_width,illcond,keep", [(32, 0, 6, 1), (32, 512, 0, 2),
                                                     (100, 512, 0, 1), (100, 0, 12, 4),
                                                     (130, 256, 20, 2)])
def test_fpx_faithful_f32_device(gpu, orc, lib, n, fp_width, illcond, keep):
    A, B, _, _ = ml_inputs(n, illcond)
    print(f"[faithful f32] n={n} width={fp_width} illcond={illcond} keep={keep}", flush=True)
    fx = orc.fpx(A, B, n, fp_width)
    cw, Lk, u0 = orc.faithful_cw(fx, keep)
    want = orc.fpx_decode_from(fx, cw)
    orc.fpx_free(fx)
    ctx = gpu.FpxCtx()
    assert lib.fpx_init(C.byref(ctx), A.ctypes.data, B.ctypes.data, n, fp_width) == 0
    lib.fpx_encode(C.byref(ctx), A.ctypes.data, B.ctypes.data)
    out = np.full(n * n, np.nan, np.float32)
    gLk, gu0 = C.c_int(), C.c_int()
    assert lib.fpx_faithful_f32(C.byref(ctx), keep, out.ctypes.data, C.byref(gLk),
                                C.byref(gu0)) == 0
    lib.fpx_free(C.byref(ctx))
    assert (gLk.value, gu0.value) == (Lk, u0)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("n,force,illcond,keep", [(32, 0, 0, 2), (64, 0, 16, 2), (96, 2048, 4, 2),
                                                  (96, 0, 30, 8)])
def test_fpx_faithful_f64_device(gpu, orc, lib, n, force, illcond, keep):
    _, _, dA, dB = ml_inputs(n, illcond)
    print(f"[faithful f64] n={n} force={force} illcond={illcond} keep={keep}", flush=True)
    dx = orc.fpx_d(dA, dB, n, force)
    cw, Lk, u0 = orc.faithful_cw(dx, keep)
    want = orc.fpx_decode_f64_from(dx, cw)
    orc.fpx_free(dx)
    ctx = gpu.FpxCtx()
    assert lib.fpx_init_d(C.byref(ctx), dA.ctypes.data, dB.ctypes.data, n, force) == 0
    lib.fpx_encode_d(C.byref(ctx), dA.ctypes.data, dB.ctypes.data)
    out = np.full(n * n, np.nan)
    gLk, gu0 = C.c_int(), C.c_int()
    assert lib.fpx_faithful_f64(C.byref(ctx), keep, out.ctypes.data, C.byref(gLk),
                                C.byref(gu0)) == 0
    assert lib.fpx_faithful_window(C.byref(ctx), keep, None, None) == Lk
    lib.fpx_free(C.byref(ctx))
    assert (gLk.value, gu0.value) == (Lk, u0)
    assert np.array_equal(out.view(np.uint64), want.view(np.uint64))
