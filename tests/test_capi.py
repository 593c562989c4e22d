"""The reference API as a C program sees it.

tests/capi/route2.c is compiled by gcc against include/mfftbench.h and linked
with -lmfft_hip, the way a program written against src/mfftbench.h would be.
CPU tests: its struct layouts equal those of the reference header compiled
by gcc, and the library binds its own functions while leaving its data
symbols to the executable (-Bsymbolic-functions).  GPU tests: it runs the
reference's call sequences (src/main.c:111-134 mm_mfft + bigres_equal,
src/mlgemm.c:723-736 fpx_init / fpx_encode / conv_mfft / fpx_decode_*) on the
golden fixtures, in this process."""
import ctypes as C
import json
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CAPI = os.path.join(ROOT, "tests", "capi")
GOLD = os.path.join(ROOT, "tests", "golden")
INCLUDE = os.path.join(ROOT, "include")
LIBDIR = os.path.join(ROOT, "mfft-bench_amd", "lib")
REF_HEADER_DIR = "/root/reference/src"

LAYOUT_NAMES = ["sizeof(fpx_ctx)", "offsetof(fpx_ctx,sig)", "offsetof(fpx_ctx,spreadB)",
                "offsetof(fpx_ctx,A32)", "offsetof(fpx_ctx,B32)", "offsetof(fpx_ctx,Cw)",
                "offsetof(fpx_ctx,enc_secs)", "offsetof(fpx_ctx,dec_secs)",
                "sizeof(mfft_plan)", "offsetof(mfft_plan,rec)", "offsetof(mfft_plan,nprod)",
                "sizeof(mfft_profile_t)", "offsetof(mfft_profile_t,pointwise)",
                "offsetof(mfft_profile_t,fold)", "offsetof(mfft_profile_t,n_fft)",
                "KERNEL_PACKED", "KERNEL_BOOLTILED", "LIMB_BITS", "sizeof(kernel_t)"]


@pytest.fixture(scope="module")
def r2(lib):
    path = os.path.join(CAPI, "libroute2.so")
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} not built: run `make -C tests/capi`")
    d = C.CDLL(path)
    vp, i, u64 = C.c_void_p, C.c_int, C.c_uint64
    d.r2_layout.argtypes = [vp, i]
    d.r2_mm_mfft.argtypes = [i, i, u64, u64, i, i, vp, i, vp]
    d.r2_instrumentation.argtypes = [i, i, vp, vp]
    d.r2_fpx_f32.argtypes = [vp, vp, i, i, vp, vp, vp]
    d.r2_fpx_f64.argtypes = [vp, vp, i, i, vp, vp, vp, vp]
    d.r2_rns_mm.argtypes = [i, i, u64, u64, i, vp, i, vp]
    d.r2_rns_fpx_f32.argtypes = [vp, vp, i, i, vp]
    return d


def test_route2_layout(r2):
    v = np.zeros(32, np.int64)
    assert r2.r2_layout(v.ctypes.data, 32) == len(LAYOUT_NAMES)
    got = dict(zip(LAYOUT_NAMES, v[:len(LAYOUT_NAMES)].tolist()))
    assert got["sizeof(fpx_ctx)"] == 72 and got["sizeof(mfft_plan)"] == 32
    import mfft_ctypes as M
    assert C.sizeof(M.FpxCtx) == 72 and C.sizeof(M.Plan) == 32 and C.sizeof(M.ProfileT) == 56


def test_layout_matches_reference_header(r2, tmp_path):
    """sizeof/offsetof of fpx_ctx, mfft_plan and mfft_profile_t under
    include/mfftbench.h equal those of the reference's own header, both
    compiled by gcc (the reference header is read where it lies, when the
    reference checkout is present)."""
    if not os.path.exists(os.path.join(REF_HEADER_DIR, "mfftbench.h")):
        pytest.skip("reference header not present")
    exprs = []
    for name in LAYOUT_NAMES:
        if name.startswith("offsetof("):
            t, f = name[len("offsetof("):-1].split(",")
            exprs.append(f"(long)offsetof({t}, {f})")
        elif name.startswith("sizeof("):
            exprs.append(f"(long){name}")
        else:
            exprs.append(f"(long){name}")
    src = tmp_path / "layout.c"
    src.write_text("#include <stdio.h>\n#include <stddef.h>\n#include \"mfftbench.h\"\n"
                   "int main(void){\n" +
                   "".join(f'  printf("%ld\\n", {e});\n' for e in exprs) + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=gnu11", "-I", REF_HEADER_DIR, str(src), "-o", str(exe)],
                   check=True)
    want = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True,
                                           text=True).stdout.split()]
    v = np.zeros(32, np.int64)
    r2.r2_layout(v.ctypes.data, 32)
    got = v[:len(LAYOUT_NAMES)].tolist()
    assert dict(zip(LAYOUT_NAMES, got)) == dict(zip(LAYOUT_NAMES, want))


def test_library_binds_own_functions_not_data(tmp_path):
    """An executable that defines bigmat_alloc (as a program linking
    src/bigmat.c does) does not capture the library's own call inside
    bigmat_to_entry_major; and the executable's copy of g_kernel_calls is the
    one mm_accum counts in (no device needed: mm_accum counts, then rejects
    its null pointers)."""
    src = tmp_path / "interpose.c"
    src.write_text(r'''
#include <stdio.h>
#include "mfftbench.h"
static int mine;
uint16_t *bigmat_alloc(int n, int L) { (void)n; (void)L; mine++; return NULL; }
int main(void) {
    uint16_t p[8] = {1, 2, 3, 4, 5, 6, 7, 8};
    uint16_t *e = bigmat_to_entry_major(p, 2, 2);
    if (!e || mine) { printf("interposed %d\n", mine); return 1; }
    if (e[0] != 1 || e[1] != 5 || e[2] != 2 || e[7] != 8) return 2;
    long long before = g_kernel_calls;
    mm_accum(NULL, NULL, NULL, 4, 1, KERNEL_HIP);
    if (g_kernel_calls != before + 1) { printf("calls %lld\n", g_kernel_calls); return 3; }
    if (mfft_last_error() != -3) return 4;
    return 0;
}
''')
    exe = tmp_path / "interpose"
    subprocess.run(["gcc", "-std=gnu11", "-Wall", "-I", INCLUDE, str(src), "-o", str(exe),
                    "-L", LIBDIR, "-lmfft_hip", f"-Wl,-rpath,{LIBDIR}"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)


# ---- on the device --------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("rec", [0, 1])
def test_route2_mm_mfft_products(gpu, r2, rec):
    """src/main.c:207-208, 111-134 as C: bigmat_rand, mm_mfft(KERNEL_HIP)
    (mm_mfft_signed for the two's complement cases), bigres_equal against
    the Python big-integer products."""
    with open(os.path.join(GOLD, "products.json")) as f:
        cases = json.load(f)
    ran = 0
    for c in cases:
        n, L, RL = c["n"], c["L"], c["RL"]
        print(f"[route2] n={n} L={L} signed={c['signed']} rec={rec}", flush=True)
        want = np.array(c["out"], dtype=np.uint16)
        bad = np.zeros(3, np.int32)
        rc = r2.r2_mm_mfft(n, L, c["seed_a"], c["seed_b"], int(c["signed"]), rec,
                           want.ctypes.data, RL, bad.ctypes.data)
        if rc == -99:                       # no plan: only where the planner has none
            assert (gpu.plan_rec(L, n) if rec else gpu.plan(L)) is None
            continue
        assert rc == 1, (rc, bad.tolist())
        ran += 1
    assert ran >= len(cases) - 2


@pytest.mark.gpu
def test_route2_rns_products(gpu, r2):
    """the multi-modular product called from C (mfh_rns_create / mfh_rns_mm /
    mfh_rns_destroy) on the seeded inputs of every golden product, unsigned
    and two's complement, checked by bigres_equal in C"""
    with open(os.path.join(GOLD, "products.json")) as f:
        cases = json.load(f)
    for c in cases:
        n, L, RL = c["n"], c["L"], c["RL"]
        print(f"[route2 rns] n={n} L={L} signed={c['signed']}", flush=True)
        want = np.array(c["out"], dtype=np.uint16)
        bad = np.zeros(3, np.int32)
        rc = r2.r2_rns_mm(n, L, c["seed_a"], c["seed_b"], int(c["signed"]), want.ctypes.data,
                          RL, bad.ctypes.data)
        assert rc == 1, (n, L, c["signed"], rc, bad.tolist())


@pytest.mark.gpu
def test_route2_instrumentation(gpu, r2):
    pw = C.c_double(-1.0)
    calls = C.c_longlong(0)
    assert r2.r2_instrumentation(64, 64, C.byref(pw), C.byref(calls)) == 0
    assert pw.value > 0.0
    assert calls.value == 1


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(3))
def test_route2_fpx_f32_fixture(gpu, r2, case):
    """src/mlgemm.c:723-728 as C on the device (conv_mfft for the leaf), then
    fpx_mm_f32 after the caller freed its encoded inputs; both bit-equal to
    the Fraction fixtures; nothing written past the 72-byte context."""
    with open(os.path.join(GOLD, "fpx.json")) as f:
        c = json.load(f)[case]
    n = c["n"]
    A = np.array(c["A_bits"], dtype=np.uint32).view(np.float32)
    B = np.array(c["B_bits"], dtype=np.uint32).view(np.float32)
    want = np.array(c["C_bits"], dtype=np.uint32)
    conv = np.full(n * n, np.nan, np.float32)
    fused = np.full(n * n, np.nan, np.float32)
    L = C.c_int(0)
    assert r2.r2_fpx_f32(A.ctypes.data, B.ctypes.data, n, 512, conv.ctypes.data,
                         fused.ctypes.data, C.byref(L)) == 0
    assert L.value == 32
    assert np.array_equal(conv.view(np.uint32), want)
    assert np.array_equal(fused.view(np.uint32), want)


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(3))
def test_route2_rns_fpx_f32_fixture(gpu, r2, case):
    """the multi-modular fixed-point product called from C (fpx_init for the
    grid, mfh_rns_create with one limb more, mfh_rns_fpx_mm) against the
    Fraction fixtures"""
    with open(os.path.join(GOLD, "fpx.json")) as f:
        c = json.load(f)[case]
    n = c["n"]
    A = np.array(c["A_bits"], dtype=np.uint32).view(np.float32)
    B = np.array(c["B_bits"], dtype=np.uint32).view(np.float32)
    want = np.array(c["C_bits"], dtype=np.uint32)
    out = np.full(n * n, np.nan, np.float32)
    assert r2.r2_rns_fpx_f32(A.ctypes.data, B.ctypes.data, n, 512, out.ctypes.data) == 0
    assert np.array_equal(out.view(np.uint32), want)


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(4))
def test_route2_fpx_f64_fixture(gpu, r2, case):
    """src/mlgemm.c:731-736 as C on the device: fpx_decode_f64, fpx_decode_ld
    and the fused fpx_mm_f64 (inputs freed first) against fpx64.json."""
    with open(os.path.join(GOLD, "fpx64.json")) as f:
        c = json.load(f)[case]
    n, force = c["n"], c["force_bits"]
    print(f"[route2 fp64] {c['name']} n={n}", flush=True)
    A = np.array(c["A_bits"], dtype=np.uint64).view(np.float64)
    B = np.array(c["B_bits"], dtype=np.uint64).view(np.float64)
    want = np.array(c["C64_bits"], dtype=np.uint64)
    conv = np.full(n * n, np.nan)
    fused = np.full(n * n, np.nan)
    ld = np.zeros(n * n, np.longdouble)
    L = C.c_int(0)
    assert r2.r2_fpx_f64(A.ctypes.data, B.ctypes.data, n, force, conv.ctypes.data,
                         fused.ctypes.data, ld.ctypes.data, C.byref(L)) == 0
    assert np.array_equal(conv.view(np.uint64), want)
    assert np.array_equal(fused.view(np.uint64), want)
    want_ld = np.ldexp(np.array(c["ld_sig"], dtype=np.int64).astype(np.longdouble),
                       np.array(c["ld_ex"], dtype=np.int32))
    assert np.array_equal(ld, want_ld)
