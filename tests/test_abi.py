"""The C-ABI library: it loads without a GPU, exports every function the
public headers declare, and its host-side logic (plan, sizing, argument and
bound checks, error conventions) matches the reference without any compute
call."""
import ctypes as C
import os
import re
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("mfftbench.h", "mfft_hip.h")]


def declared_functions(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"^\s*#[^\n]*", "", text, flags=re.M)      # preprocessor lines
    names = set()
    for m in re.finditer(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\(([^;{}]*)\)\s*;", text):
        name = m.group(1)
        if name in {"if", "while", "sizeof", "return"}:
            continue
        names.add(name)
    return names


def test_library_exports_every_declared_symbol(lib):
    import mfft_ctypes
    out = subprocess.run(["nm", "-D", "--defined-only", mfft_ctypes.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    declared = set()
    for h in HEADERS:
        declared |= declared_functions(h)
    assert len(declared) > 40
    missing = sorted(declared - exported)
    assert not missing, f"declared but not exported: {missing}"
    for name in declared:
        getattr(lib, name)                               # resolvable through ctypes


def test_no_internal_symbols_leak():
    import mfft_ctypes
    out = subprocess.run(["nm", "-D", "--defined-only", mfft_ctypes.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    names = [line.split()[-1] for line in out.splitlines() if " T " in line]
    assert not [n for n in names if n.startswith("_Z")], "C++ internals exported"


def test_loads_without_device(lib):
    assert lib.mfh_device_count() >= 0
    assert isinstance(lib.mfh_device_arch(), bytes)


def test_plan_matches_oracle(lib, orc):
    import mfft_ctypes as M
    for L in [2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 2048]:
        for sigma in [0, 1, 2, 3, 4, 5]:
            p = M.plan(L, sigma)
            q = orc.plan(L, sigma)
            assert (p is None) == (q is None), (L, sigma)
            if p is not None:
                assert (p.L, p.S, p.NB, p.K, p.g, p.nprod) == (q.L, q.S, q.NB, q.K, q.g, q.nprod)
                assert lib.mfft_plan_products(C.byref(p)) == q.nprod
                assert lib.mfft_plan_maxbits(C.byref(p), 64) == pytest.approx(
                    orc.lib.orc_plan_maxbits(C.byref(q), 64))
    assert M.plan(96) is None and M.plan(0) is None


def test_kernel_names(lib):
    assert lib.kernel_name(2) == b"packed" and lib.kernel_name(12) == b"hip"
    assert lib.kernel_from_name(b"hip") == 12 and lib.kernel_from_name(b"ikj") == 0
    assert lib.kernel_from_name(b"nope") == -1


def test_host_generator_and_compare(lib, orc):
    n, L = 7, 9
    m = np.empty(L * n * n, np.uint16)
    lib.bigmat_rand(m.ctypes.data, n, L, 4242)
    assert np.array_equal(m, orc.bigmat_rand(n, L, 4242))
    b = m.copy()
    bi, bj, bw = C.c_int(), C.c_int(), C.c_int()
    assert lib.bigres_equal(m.ctypes.data, b.ctypes.data, n, L, None, None, None) == 1
    b[3 * n * n + 2 * n + 5] ^= 1
    assert lib.bigres_equal(m.ctypes.data, b.ctypes.data, n, L,
                            C.byref(bi), C.byref(bj), C.byref(bw)) == 0
    assert (bi.value, bj.value, bw.value) == (2, 5, 3)


def test_cpu_leaf_is_refused_output_untouched(lib):
    """Only KERNEL_HIP runs: a CPU leaf is an error, never a fallback
    (src/mfft.c:432 convention: output left untouched)."""
    import mfft_ctypes as M
    n, L = 4, 8
    A = np.ones(L * n * n, np.uint16)
    out, err = M.mm_mfft(A, A, n, L, M.plan(L), kernel=M.KERNEL_PACKED)
    assert err == -7 and not out.any()
    cw, err = M.conv_mfft(A.astype(np.int32), A.astype(np.int32), n, L, M.plan(L),
                          kernel=M.KERNEL_PACKED)
    assert err == -7 and not cw.any()


def test_create_checks_arguments_and_bounds(lib):
    import mfft_ctypes as M
    h = C.c_void_p()
    p = M.plan(128)
    assert lib.mfh_create(C.byref(h), 0, 128, C.byref(p)) == -3          # n < 1
    bad = M.Plan(L=128, S=8, NB=32, K=16, g=2, rec=0, nprod=0)          # wrong g
    assert lib.mfh_create(C.byref(h), 64, 128, C.byref(bad)) == -3
    assert lib.mfh_create(C.byref(h), 64, 64, C.byref(p)) == -3         # L mismatch
    p1k = M.plan(1024)                                                  # K = 64
    assert lib.mfh_create(C.byref(h), 64, 1024, C.byref(p1k)) == -7
    # int32 class accumulators: pairs * (np/64) * K * 2^20 must stay below
    # 2^31 -- at K = 16 the 6-product mode (1 pair) admits n <= 8128
    assert lib.mfh_create(C.byref(h), 8192, 128, C.byref(p)) == -4
    p64 = M.plan(64)                                   # NB = 16: plain 6-product digits
    assert lib.mfh_create(C.byref(h), 8192, 64, C.byref(p64)) == -4
    # K = 32 (8192 bits): the int64 bound NB K n |a^|^2 < 2^62 binds first;
    # with |a^| <= 2^20 (6-product digits, offset mode) it admits n <= 1984
    p512 = M.plan(512)
    assert lib.mfh_create(C.byref(h), 2048, 512, C.byref(p512)) == -4
    if lib.mfh_device_count() == 0:
        assert lib.mfh_create(C.byref(h), 64, 128, C.byref(p)) == -1    # no device
        assert lib.mfh_create(C.byref(h), 3072, 128, C.byref(p)) == -1  # past the bounds
        assert lib.mfh_create(C.byref(h), 1984, 512, C.byref(p512)) == -1
        assert not h.value


def test_fpx_init_sizing_matches_reference_rules(lib, orc):
    import mfft_ctypes as M
    n = 6
    A = orc.fp32_rand(n * n, 1, -20, 20)
    B = orc.fp32_rand(n * n, 2, -5, 9)
    for force in (512, 0):
        ctx = M.FpxCtx()
        assert lib.fpx_init(C.byref(ctx), A.ctypes.data, B.ctypes.data, n, force) == 0
        oc = orc.fpx(A, B, n, force)
        assert (ctx.L, ctx.SA, ctx.SB, ctx.spreadA, ctx.spreadB) == \
               (oc.L, oc.SA, oc.SB, oc.spreadA, oc.spreadB)
        lib.fpx_free(C.byref(ctx))
        orc.fpx_free(oc)
    # fp64 sizing (src/fpfixed.c:131-142): 53-bit significands, 5-limb reach
    Ad = A.astype(np.float64) * 2.0 ** -700
    Bd = B.astype(np.float64) * (1.0 + 2.0 ** -40)
    for force in (2048, 0):
        ctx = M.FpxCtx()
        assert lib.fpx_init_d(C.byref(ctx), Ad.ctypes.data, Bd.ctypes.data, n, force) == 0
        oc = orc.fpx_d(Ad, Bd, n, force)
        assert (ctx.L, ctx.SA, ctx.SB, ctx.spreadA, ctx.spreadB, ctx.sig) == \
               (oc.L, oc.SA, oc.SB, oc.spreadA, oc.spreadB, 53)
        lib.fpx_free(C.byref(ctx))
        orc.fpx_free(oc)
    # src/fpfixed.c:84-88 overflow guard
    nb = 1024                                   # n * L * 65535^2 > 4e18 at L = 2^20
    big = np.ones(nb * nb, np.float32)
    ctx = M.FpxCtx()
    assert lib.fpx_init(C.byref(ctx), big.ctypes.data, big.ctypes.data, nb, 1 << 24) == -1


def test_schoolbook_rejects_cpu_leaves_and_leaves_outputs_untouched(lib):
    """mm_accum / conv_limbplane / mm_limbplane with a CPU kernel_t: error
    code, message, outputs untouched (no device call is made)."""
    import mfft_ctypes as M
    n, L = 4, 2
    A = np.ones(n * n, np.int32)
    Cm = np.full(n * n, 7, np.int64)
    lib.mm_accum(Cm.ctypes.data, A.ctypes.data, A.ctypes.data, n, 1, M.KERNEL_PACKED)
    assert lib.mfft_last_error() == -7 and np.all(Cm == 7)
    Cw = np.full((2 * L - 1) * n * n, 7, np.int64)
    A32 = np.ones(L * n * n, np.int32)
    lib.conv_limbplane(Cw.ctypes.data, A32.ctypes.data, A32.ctypes.data, n, L, M.KERNEL_IKJ)
    assert lib.mfft_last_error() == -7 and np.all(Cw == 7)
    A16 = np.ones(L * n * n, np.uint16)
    out = np.full((2 * L + 1) * n * n, 7, np.uint16)
    lib.mm_limbplane(A16.ctypes.data, A16.ctypes.data, n, L, M.KERNEL_PACKED, out.ctypes.data,
                     2 * L + 1)
    assert lib.mfft_last_error() == -7 and np.all(out == 7)


# ---- recursive plan (src/mfft.c:474-527, 664-686) ---------------------------------
def test_plan_rec_known_answers(lib):
    """Product counts the reference publishes for mfft-rec (README.md:319-324,
    measured at n = 32), and those of the workloads this library targets."""
    import mfft_ctypes as M
    for L, n, S, nprod in [(64, 32, 8, 1296), (512, 32, 16, 13824), (2048, 32, 32, 93312),
                           (4096, 32, 64, 279936), (512, 256, 16, 15552),
                           (128, 1024, 8, 2592), (32, 2048, 4, 432), (32, 4096, 4, 432)]:
        p = M.plan_rec(L, n)
        assert p is not None and p.rec == 1
        assert (p.S, p.nprod) == (S, nprod), (L, n)
        assert (p.NB, p.K, p.g) == (2 * L // S, 2 * S, 4 * S // (2 * L // S))
        assert lib.mfft_plan_products(C.byref(p)) == nprod
    assert M.plan_rec(2, 64) is None                   # no admissible block size
    assert M.plan_rec(96, 64) is None                  # L not a power of two


def test_plan_rec_matches_reference(lib, ref):
    import mfft_ctypes as M
    from oracle_ctypes import RefPlanStruct
    ref.lib.mfft_plan_init_rec.argtypes = [C.POINTER(RefPlanStruct), C.c_int, C.c_int, C.c_int]
    for L in [2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 2048, 4096]:
        for n in [1, 3, 32, 64, 256, 1000, 1024, 4096, 1 << 16]:
            for sigma in [0, 1, 2, 3, 5]:
                rp = RefPlanStruct()
                rrc = ref.lib.mfft_plan_init_rec(C.byref(rp), L, n, sigma)
                p = M.Plan()
                rc = lib.mfft_plan_init_rec(C.byref(p), L, n, sigma)
                assert rc == rrc, (L, n, sigma)
                if rc == 0:
                    assert (p.L, p.S, p.NB, p.K, p.g, p.rec, p.nprod) == \
                           (rp.L, rp.S, rp.NB, rp.K, rp.g, rp.rec, rp.nprod), (L, n, sigma)


def test_profile_globals_and_leaf_call_counter(lib):
    """g_kernel_calls / g_mfft_profile / g_mfft_prof (src/mfftbench.h:56-71)
    are exported with the reference's layout; mm_accum counts its calls."""
    import mfft_ctypes as M
    calls = C.c_longlong.in_dll(lib, "g_kernel_calls")
    prof = M.ProfileT.in_dll(lib, "g_mfft_prof")
    flag = C.c_int.in_dll(lib, "g_mfft_profile")
    assert flag.value == 0
    before = calls.value
    n = 2
    A = np.ones(n * n, np.int32)
    Cm = np.zeros(n * n, np.int64)
    lib.mm_accum(Cm.ctypes.data, A.ctypes.data, A.ctypes.data, n, 1, M.KERNEL_PACKED)
    assert calls.value == before + 1
    prof.pointwise = 1.0
    lib.mfft_profile_reset()
    assert (prof.pack, prof.transform, prof.pointwise, prof.n_fft) == (0.0, 0.0, 0.0, 0)
    assert C.sizeof(M.ProfileT) == 56


# ---- bench.py's argument contract (host logic, no GPU call) -------------------
def _bench(*args):
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    return subprocess.run([sys.executable, os.path.join(root, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120)


def test_bench_refuses_more_than_one_gpu():
    r = _bench("--gpus", "2")
    assert r.returncode == 2 and "one GPU only" in r.stderr


@pytest.mark.parametrize("args", [("--n", "100", "--bits", "48"), ("--n", "0", "--bits", "2048"),
                                  ("--n", "64", "--bits", "16")])
def test_bench_rejects_bad_sizes(args):
    r = _bench(*args)
    assert r.returncode == 2 and "power of two" in r.stderr


@pytest.mark.parametrize("args", [("--sweep-width", "--n", "-5"), ("--sweep-n", "--width", "48")])
def test_bench_sweeps_reject_bad_sizes(args):
    r = _bench(*args)
    assert r.returncode == 2 and "sweeps need" in r.stderr
