"""ctypes binding of lib/libmfft_hip.so (include/mfftbench.h, include/mfft_hip.h).

Plumbing for the tests and bench.py: every product call goes through the
C-ABI into the gfx950 kernels.  Loading fails loudly when the library was not
built; there is no fallback.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libmfft_hip.so")

KERNEL_IKJ, KERNEL_PACKED, KERNEL_HIP = 0, 2, 12
MFH_IN_U16, MFH_IN_U16_SIGNED, MFH_IN_I32 = 0, 1, 2
ERRORS = {0: "MFH_OK", -1: "MFH_E_NODEV", -2: "MFH_E_NOMEM", -3: "MFH_E_ARG",
          -4: "MFH_E_BOUND", -5: "MFH_E_RANGE", -6: "MFH_E_HIP", -7: "MFH_E_UNSUPPORTED",
          -8: "MFH_E_SCRATCH"}


class MfftError(RuntimeError):
    def __init__(self, code, what=""):
        self.code = code
        super().__init__(f"{what}: {ERRORS.get(code, code)}")


class Plan(C.Structure):
    """mfft_plan / mfh_plan (identical layouts)."""
    _fields_ = [("L", C.c_int), ("S", C.c_int), ("NB", C.c_int), ("K", C.c_int),
                ("g", C.c_int), ("rec", C.c_int), ("nprod", C.c_longlong)]

    def __repr__(self):
        return f"Plan(L={self.L}, S={self.S}, NB={self.NB}, K={self.K}, g={self.g})"


class ProfileT(C.Structure):
    """mfft_profile_t (src/mfftbench.h:59-67)"""
    _fields_ = [("pack", C.c_double), ("build_ops", C.c_double), ("transform", C.c_double),
                ("pointwise", C.c_double), ("fold", C.c_double), ("n_build", C.c_longlong),
                ("n_fft", C.c_longlong)]


class FpxCtx(C.Structure):
    """fpx_ctx (src/mfftbench.h:182-189): the reference's fields, 72 bytes"""
    _fields_ = [("n", C.c_int), ("L", C.c_int), ("sig", C.c_int),
                ("SA", C.c_int), ("SB", C.c_int),
                ("spreadA", C.c_int), ("spreadB", C.c_int),
                ("A32", C.c_void_p), ("B32", C.c_void_p), ("Cw", C.c_void_p),
                ("enc_secs", C.c_double), ("dec_secs", C.c_double)]


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


_lib = None


def load(path=None):
    global _lib
    if _lib is not None and path is None:
        return _lib
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} not built: run `make -C mfft-bench_amd`")
    L = C.CDLL(path)
    vp, i, u64, sz = C.c_void_p, C.c_int, C.c_uint64, C.c_size_t
    pl = C.POINTER(Plan)
    sig = {
        "mfh_strerror": ([i], C.c_char_p), "mfh_device_count": ([], i),
        "mfh_device_arch": ([], C.c_char_p),
        "mfh_create": ([C.POINTER(vp), i, i, pl], i), "mfh_destroy": ([vp], None),
        "mfh_workspace_bytes": ([vp], sz), "mfh_band_rows": ([vp], i),
        "mfh_mm": ([vp, i, vp, vp, vp, i], i), "mfh_conv": ([vp, vp, vp, vp], i),
        "mfh_mm_dev": ([vp, i, vp, vp, vp, i], i), "mfh_conv_dev": ([vp, vp, vp, vp], i),
        "mfh_mm_dev_noalloc": ([i, pl, i, i, vp, vp, vp, i, vp], i),
        "mfh_fpx_mm_dev": ([vp, vp, vp, i, i, vp], i), "mfh_fpx_mm": ([vp, vp, vp, i, i, vp], i),
        "mfh_fpx_decode_dev": ([vp, vp, i, vp], i),
        "mfh_normalize": ([vp, i, i, vp, i], i), "mfh_fpx_encode": ([vp, i, i, i, vp], i),
        "mfh_fpx_decode": ([vp, i, i, i, vp], i),
        "mfh_fpx_mm_f64_dev": ([vp, vp, vp, i, i, vp], i),
        "mfh_fpx_mm_f64": ([vp, vp, vp, i, i, vp], i),
        "mfh_fpx_decode_f64_dev": ([vp, vp, i, vp], i),
        "mfh_fpx_encode_f64": ([vp, i, i, i, vp], i),
        "mfh_fpx_decode_f64": ([vp, i, i, i, vp], i),
        "mfh_fpx_decode_ld": ([vp, i, i, i, vp], i),
        "mfh_fpx_decode_sig63": ([vp, i, i, i, vp, vp], i),
        "mfh_mm_accum": ([vp, vp, vp, i, i], i),
        "mfh_mm_accum_dev": ([vp, vp, vp, vp, i, i], i),
        "mfh_limbplane_conv": ([vp, vp, i, i, vp], i),
        "mfh_limbplane_conv_dev": ([vp, i, vp, vp, i, i, vp], i),
        "mfh_limbplane_mm": ([vp, vp, i, i, vp, i], i),
        "mfh_limbplane_mm_dev": ([vp, i, vp, vp, i, i, vp, vp, i], i),
        "mfh_schoolbook_workspace": ([i, i, C.POINTER(sz)], i),
        "mfh_schoolbook_dev": ([vp, i, vp, vp, i, i, vp, sz, vp, i], i),
        "mfh_schoolbook": ([i, vp, vp, i, i, vp, i], i),
        "mm_accum": ([vp, vp, vp, i, i, i], None),
        "mm_limbplane": ([vp, vp, i, i, i, vp, i], None),
        "conv_limbplane": ([vp, vp, vp, i, i, i], None),
        "mfh_malloc": ([C.POINTER(vp), sz], i), "mfh_free": ([vp], i),
        "mfh_h2d": ([vp, vp, sz], i), "mfh_d2h": ([vp, vp, sz], i), "mfh_sync": ([vp], i),
        "mfh_rand_u16_dev": ([vp, vp, i, i, u64], i),
        "mfh_rand_f32_dev": ([vp, vp, sz, u64, i, i], i),
        "mfh_copy_dev": ([vp, vp, vp, sz], i),
        "mfh_set_timing": ([vp, i], i), "mfh_stage_times": ([vp, C.POINTER(C.c_float)], i),
        "mfh_work": ([vp, C.POINTER(C.c_double), C.POINTER(C.c_double), C.POINTER(C.c_double)], i),
        "mfh_pointwise_info": ([vp, C.POINTER(C.c_int), C.POINTER(C.c_int)], i),
        "mfh_conv_stages": ([vp, vp, vp, i, vp, sz, C.POINTER(C.c_int64)], i),
        "mfft_plan_init": ([pl, i, i], i), "mfft_plan_products": ([pl], C.c_longlong),
        "mfft_plan_init_rec": ([pl, i, i, i], i),
        "ssa_negconv": ([vp, vp, vp, i, i, i, i], None),
        "mfh_negconv": ([vp, vp, i, i, vp], i),
        "mfh_bigint_mm": ([vp, vp, i, i, vp, i], i),
        "mm_bigint_ijk": ([vp, vp, i, i, vp, i], None),
        "mm_bigint_ikj": ([vp, vp, i, i, vp, i], None),
        "bigmat_to_entry_major": ([vp, i, i], C.c_void_p),
        "mfft_plan_maxbits": ([pl, i], C.c_double),
        "mm_mfft": ([vp, vp, i, i, pl, i, vp, i], None),
        "mm_mfft_signed": ([vp, vp, i, i, pl, i, vp, i], None),
        "conv_mfft": ([vp, vp, vp, i, i, pl, i], None),
        "normalize_planes": ([vp, i, i, vp, i], None),
        "bigmat_rand": ([vp, i, i, u64], None),
        "bigres_equal": ([vp, vp, i, i, vp, vp, vp], i),
        "fpx_init": ([C.POINTER(FpxCtx), vp, vp, i, i], i),
        "fpx_encode": ([C.POINTER(FpxCtx), vp, vp], None),
        "fpx_decode_f32": ([C.POINTER(FpxCtx), vp], None),
        "fpx_free": ([C.POINTER(FpxCtx)], None),
        "fpx_mm_f32": ([C.POINTER(FpxCtx), pl, vp], i),
        "fpx_init_d": ([C.POINTER(FpxCtx), vp, vp, i, i], i),
        "fpx_encode_d": ([C.POINTER(FpxCtx), vp, vp], None),
        "fpx_decode_f64": ([C.POINTER(FpxCtx), vp], None),
        "fpx_decode_ld": ([C.POINTER(FpxCtx), vp], None),
        "fpx_mm_f64": ([C.POINTER(FpxCtx), pl, vp], i),
        "fpx_faithful_window": ([C.POINTER(FpxCtx), i, vp, vp], i),
        "fpx_faithful_f32": ([C.POINTER(FpxCtx), i, vp, vp, vp], i),
        "fpx_faithful_f64": ([C.POINTER(FpxCtx), i, vp, vp, vp], i),
        "mfh_fpx_faithful": ([vp, vp, i, i, i, i, pl, i, i, vp], i),
        "mfft_profile_reset": ([], None), "mfft_profile_print": ([C.c_char_p], None),
        "mfft_last_error": ([], i), "mfft_strerror": ([i], C.c_char_p),
        "kernel_name": ([i], C.c_char_p), "kernel_from_name": ([C.c_char_p], i),
        "now_sec": ([], C.c_double),
        "mfh_rns_primes": ([i, i, vp, i], i),
        "mfh_rns_create": ([C.POINTER(vp), i, i], i), "mfh_rns_destroy": ([vp], None),
        "mfh_rns_info": ([vp, C.POINTER(i), C.POINTER(i), C.POINTER(sz)], i),
        "mfh_rns_mm_dev": ([vp, i, vp, vp, vp, i], i),
        "mfh_rns_mm": ([vp, i, vp, vp, vp, i], i),
        "mfh_rns_residues_dev": ([vp, i, vp, vp], i),
        "mfh_rns_fpx_mm_dev": ([vp, vp, vp, i, i, vp], i),
        "mfh_rns_fpx_mm_f64_dev": ([vp, vp, vp, i, i, vp], i),
        "mfh_rns_fpx_mm": ([vp, vp, vp, i, i, vp], i),
        "mfh_rns_fpx_mm_f64": ([vp, vp, vp, i, i, vp], i),
        "mfh_rns_sync": ([vp], i), "mfh_rns_set_timing": ([vp, i], i),
        "mfh_rns_stage_times": ([vp, C.POINTER(C.c_float)], i),
        "mfh_rns_work": ([vp, C.POINTER(C.c_double), C.POINTER(C.c_double),
                          C.POINTER(C.c_double)], i),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    if path == LIB_PATH:
        _lib = L
    return L


def check(rc, what=""):
    if rc != 0:
        raise MfftError(rc, what)


def plan(L, sigma=0):
    p = Plan()
    if load().mfft_plan_init(C.byref(p), L, sigma) != 0:
        return None
    return p


def plan_rec(L, n, sigma=0):
    p = Plan()
    if load().mfft_plan_init_rec(C.byref(p), L, n, sigma) != 0:
        return None
    return p


def have_gpu():
    try:
        lib = load()
    except (OSError, FileNotFoundError):
        return False
    return lib.mfh_device_count() > 0 and lib.mfh_device_arch().startswith(b"gfx950")


class Ctx:
    """One device context (workspace for one n, L, plan)."""

    def __init__(self, n, L, p=None):
        self.lib = load()
        self.n, self.L = n, L
        self.plan = p or plan(L)
        h = C.c_void_p()
        check(self.lib.mfh_create(C.byref(h), n, L, C.byref(self.plan)), "mfh_create")
        self.h = h

    def close(self):
        if self.h:
            self.lib.mfh_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # host-buffer entry points
    def mm(self, A, B, RL=None, signed=False):
        RL = RL or 2 * self.L + 1
        out = np.empty(RL * self.n * self.n, dtype=np.uint16)
        kind = MFH_IN_U16_SIGNED if signed else MFH_IN_U16
        check(self.lib.mfh_mm(self.h, kind, _p(A), _p(B), _p(out), RL), "mfh_mm")
        return out

    def conv(self, A32, B32):
        cw = np.empty((2 * self.L - 1) * self.n * self.n, dtype=np.int64)
        check(self.lib.mfh_conv(self.h, _p(A32), _p(B32), _p(cw)), "mfh_conv")
        return cw

    def fpx_mm(self, A, B, SA, SB):
        out = np.empty(self.n * self.n, dtype=np.float32)
        check(self.lib.mfh_fpx_mm(self.h, _p(A), _p(B), SA, SB, _p(out)), "mfh_fpx_mm")
        return out

    def fpx_mm_f64(self, A, B, SA, SB):
        out = np.empty(self.n * self.n, dtype=np.float64)
        check(self.lib.mfh_fpx_mm_f64(self.h, _p(A), _p(B), SA, SB, _p(out)), "mfh_fpx_mm_f64")
        return out

    # device-level helpers
    def band_rows(self):
        return self.lib.mfh_band_rows(self.h)

    def workspace_bytes(self):
        return self.lib.mfh_workspace_bytes(self.h)

    def set_timing(self, on=True):
        check(self.lib.mfh_set_timing(self.h, int(on)))

    def stage_times(self):
        ms = (C.c_float * 5)()
        check(self.lib.mfh_stage_times(self.h, ms), "mfh_stage_times")
        return list(ms)

    def work(self):
        a, b, c = C.c_double(), C.c_double(), C.c_double()
        check(self.lib.mfh_work(self.h, C.byref(a), C.byref(b), C.byref(c)))
        return a.value, b.value, c.value

    def pointwise_info(self):
        """(ring products per point, int8 digit products per ring product) of
        the most recent product"""
        r, d = C.c_int(), C.c_int()
        check(self.lib.mfh_pointwise_info(self.h, C.byref(r), C.byref(d)))
        return r.value, d.value

    def sync(self):
        check(self.lib.mfh_sync(self.h), "mfh_sync")

    def stages(self, A32, B32, stage):
        """(info, raw bytes) of one stage of the conv product (mfh_conv_stages):
        info = (digit mode, pointwise algorithm, band rows, np, bytes)"""
        info = (C.c_int64 * 5)()
        check(self.lib.mfh_conv_stages(self.h, _p(A32), _p(B32), stage, None, 0, info),
              "mfh_conv_stages")
        out = np.empty(int(info[4]), dtype=np.uint8)
        check(self.lib.mfh_conv_stages(self.h, _p(A32), _p(B32), stage, _p(out), out.size,
                                       info), "mfh_conv_stages")
        return tuple(int(v) for v in info), out


def rns_primes(n, L):
    """the primes of the multi-modular product of n x n matrices of L limbs
    (host planning, no device needed)"""
    lib = load()
    cnt = lib.mfh_rns_primes(n, L, None, 0)
    check(min(cnt, 0), "mfh_rns_primes")
    out = np.zeros(cnt, dtype=np.int32)
    lib.mfh_rns_primes(n, L, _p(out), cnt)
    return out


class Rns:
    """One multi-modular product context (mfh_rns_*): tables and workspace for
    n x n matrices of L limbs."""

    def __init__(self, n, L):
        self.lib = load()
        self.n, self.L = n, L
        h = C.c_void_p()
        check(self.lib.mfh_rns_create(C.byref(h), n, L), "mfh_rns_create")
        self.h = h

    def close(self):
        if self.h:
            self.lib.mfh_rns_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self):
        """(primes, padded n, device bytes)"""
        nm, np_, b = C.c_int(), C.c_int(), C.c_size_t()
        check(self.lib.mfh_rns_info(self.h, C.byref(nm), C.byref(np_), C.byref(b)))
        return nm.value, np_.value, b.value

    def mm(self, A, B, RL=None, signed=False):
        RL = RL or 2 * self.L + 1
        out = np.empty(RL * self.n * self.n, dtype=np.uint16)
        kind = MFH_IN_U16_SIGNED if signed else MFH_IN_U16
        check(self.lib.mfh_rns_mm(self.h, kind, _p(A), _p(B), _p(out), RL), "mfh_rns_mm")
        return out

    def mm_dev(self, dA, dB, dOut, RL, signed=False):
        kind = MFH_IN_U16_SIGNED if signed else MFH_IN_U16
        check(self.lib.mfh_rns_mm_dev(self.h, kind, dA, dB, dOut, RL), "mfh_rns_mm_dev")

    def fpx_mm(self, A, B, SA, SB):
        """fp32 product on the grid of L - 1 limbs (the context has L)"""
        out = np.empty(self.n * self.n, dtype=np.float32)
        check(self.lib.mfh_rns_fpx_mm(self.h, _p(A), _p(B), SA, SB, _p(out)), "mfh_rns_fpx_mm")
        return out

    def fpx_mm_f64(self, A, B, SA, SB):
        out = np.empty(self.n * self.n, dtype=np.float64)
        check(self.lib.mfh_rns_fpx_mm_f64(self.h, _p(A), _p(B), SA, SB, _p(out)),
              "mfh_rns_fpx_mm_f64")
        return out

    def fpx_mm_dev(self, dA, dB, SA, SB, dC, f64=False):
        fn = self.lib.mfh_rns_fpx_mm_f64_dev if f64 else self.lib.mfh_rns_fpx_mm_dev
        check(fn(self.h, dA, dB, SA, SB, dC), "mfh_rns_fpx_mm_dev")

    def residues(self, X, signed=False):
        """digit-pair residues [primes][np][np] of one operand (rows r, inner k)"""
        nm, np_, _ = self.info()
        dX = DevBuf(max(X.nbytes, 16))
        dX.upload(X)
        dR = DevBuf(nm * np_ * np_ * 2)
        kind = MFH_IN_U16_SIGNED if signed else MFH_IN_U16
        check(self.lib.mfh_rns_residues_dev(self.h, kind, dX.ptr, dR.ptr), "mfh_rns_residues_dev")
        self.sync()
        return dR.download(np.uint16, nm * np_ * np_).reshape(nm, np_, np_)

    def sync(self):
        check(self.lib.mfh_rns_sync(self.h), "mfh_rns_sync")

    def set_timing(self, on=True):
        check(self.lib.mfh_rns_set_timing(self.h, int(on)))

    def stage_times(self):
        ms = (C.c_float * 4)()
        check(self.lib.mfh_rns_stage_times(self.h, ms), "mfh_rns_stage_times")
        return list(ms)

    def work(self):
        a, b, c = C.c_double(), C.c_double(), C.c_double()
        check(self.lib.mfh_rns_work(self.h, C.byref(a), C.byref(b), C.byref(c)))
        return a.value, b.value, c.value


class DevBuf:
    def __init__(self, nbytes):
        self.lib = load()
        p = C.c_void_p()
        check(self.lib.mfh_malloc(C.byref(p), nbytes), "mfh_malloc")
        self.ptr, self.nbytes = p, nbytes

    def upload(self, arr):
        assert arr.nbytes <= self.nbytes
        check(self.lib.mfh_h2d(self.ptr, _p(arr), arr.nbytes), "mfh_h2d")

    def download(self, dtype, count):
        out = np.empty(count, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(self.lib.mfh_d2h(_p(out), self.ptr, out.nbytes), "mfh_d2h")
        return out

    def free(self):
        if self.ptr:
            self.lib.mfh_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---- reference-named C API ---------------------------------------------------
def mm_mfft(A, B, n, L, p, RL=None, kernel=KERNEL_HIP, signed=False):
    lib = load()
    RL = RL or 2 * L + 1
    out = np.zeros(RL * n * n, dtype=np.uint16)
    f = lib.mm_mfft_signed if signed else lib.mm_mfft
    f(_p(A), _p(B), n, L, C.byref(p), kernel, _p(out), RL)
    return out, lib.mfft_last_error()


def conv_mfft(A32, B32, n, L, p, kernel=KERNEL_HIP):
    lib = load()
    cw = np.zeros((2 * L - 1) * n * n, dtype=np.int64)
    lib.conv_mfft(_p(cw), _p(A32), _p(B32), n, L, C.byref(p), kernel)
    return cw, lib.mfft_last_error()


def normalize_planes(acc, nplanes, n, RL):
    lib = load()
    out = np.zeros(RL * n * n, dtype=np.uint16)
    lib.normalize_planes(_p(np.ascontiguousarray(acc, np.int64)), nplanes, n, _p(out), RL)
    return out, lib.mfft_last_error()
