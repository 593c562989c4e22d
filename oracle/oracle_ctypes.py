"""ctypes bindings for the CPU oracle (oracle/build/liboracle_*.so) and, when
it was built, the reference's own C library (oracle/_ref/libmfftref_*.so).

Test infrastructure only: imported by tests/, by __graft_entry__.smoke() as
the checker, and by bench.py's cpu_baseline leg.  Never a product path.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def _cpu_has_avx512():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = line.split()
                    return "avx512f" in flags and "avx512dq" in flags and "avx512bw" in flags
    except OSError:
        pass
    return False


def _pick(dirname, stem):
    order = ["v4", "v3"] if _cpu_has_avx512() else ["v3"]
    for v in order:
        p = os.path.join(HERE, dirname, f"{stem}_{v}.so")
        if os.path.exists(p):
            return p
    return None


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


class PlanStruct(C.Structure):
    # orc_plan and the reference's mfft_plan differ: the reference has an
    # extra `rec` field before nprod (mfftbench.h:139-143).
    _fields_ = [("L", C.c_int), ("S", C.c_int), ("NB", C.c_int), ("K", C.c_int),
                ("g", C.c_int), ("nprod", C.c_longlong)]


class RefPlanStruct(C.Structure):
    _fields_ = [("L", C.c_int), ("S", C.c_int), ("NB", C.c_int), ("K", C.c_int),
                ("g", C.c_int), ("rec", C.c_int), ("nprod", C.c_longlong)]


class OrcFpx(C.Structure):
    _fields_ = [("n", C.c_int), ("L", C.c_int), ("SA", C.c_int), ("SB", C.c_int),
                ("spreadA", C.c_int), ("spreadB", C.c_int),
                ("A32", C.c_void_p), ("B32", C.c_void_p), ("Cw", C.c_void_p)]


class RefFpx(C.Structure):
    # mfftbench.h:182-189
    _fields_ = [("n", C.c_int), ("L", C.c_int), ("sig", C.c_int),
                ("SA", C.c_int), ("SB", C.c_int),
                ("spreadA", C.c_int), ("spreadB", C.c_int),
                ("A32", C.c_void_p), ("B32", C.c_void_p), ("Cw", C.c_void_p),
                ("enc_secs", C.c_double), ("dec_secs", C.c_double)]


class Oracle:
    """The C restatement (liboracle)."""

    def __init__(self, path=None):
        path = path or _pick("build", "liboracle")
        if path is None:
            raise FileNotFoundError("oracle library not built (make -C oracle)")
        self.path = path
        L = self.lib = C.CDLL(path)
        vp, i, u64 = C.c_void_p, C.c_int, C.c_uint64
        L.orc_bigmat_rand.argtypes = [vp, i, i, u64]
        L.orc_normalize_planes.argtypes = [vp, i, i, vp, i]
        L.orc_bigres_equal.argtypes = [vp, vp, i, i, vp, vp, vp]
        L.orc_mm_accum_packed.argtypes = [vp, vp, vp, i, i]
        L.orc_mm_accum_ikj.argtypes = [vp, vp, vp, i, i]
        L.orc_conv_limbplane.argtypes = [vp, vp, vp, i, i, i]
        L.orc_mm_limbplane.argtypes = [vp, vp, i, i, vp, i, i]
        L.orc_mm_bigint_ijk.argtypes = [vp, vp, i, i, vp, i]
        L.orc_to_entry_major.argtypes = [vp, i, i, vp]
        L.orc_plan_init.argtypes = [C.POINTER(PlanStruct), i, i]
        L.orc_plan_maxbits.argtypes = [C.POINTER(PlanStruct), i]
        L.orc_plan_maxbits.restype = C.c_double
        L.orc_ring_dft.argtypes = [vp, vp, i, i, i, i]
        L.orc_fft_forward32.argtypes = [vp, i, i, i, C.c_size_t]
        L.orc_fft_inverse64.argtypes = [vp, i, i, i, C.c_size_t]
        L.orc_conv_mfft.argtypes = [vp, vp, vp, i, i, C.POINTER(PlanStruct), i]
        L.orc_mm_mfft.argtypes = [vp, vp, i, i, C.POINTER(PlanStruct), vp, i, i]
        L.orc_mm_mfft_sampled.argtypes = [vp, vp, i, i, C.POINTER(PlanStruct), vp, i,
                                          C.c_longlong, vp]
        L.orc_mm_mfft_sampled.restype = C.c_longlong
        L.orc_fpx_init.argtypes = [C.POINTER(OrcFpx), vp, vp, i, i]
        L.orc_fpx_encode.argtypes = [C.POINTER(OrcFpx), vp, vp]
        L.orc_fpx_decode_f32.argtypes = [C.POINTER(OrcFpx), vp]
        L.orc_fpx_decode_f32_from.argtypes = [C.POINTER(OrcFpx), vp, vp]
        L.orc_fpx_free.argtypes = [C.POINTER(OrcFpx)]
        L.orc_fpx_init_d.argtypes = [C.POINTER(OrcFpx), vp, vp, i, i]
        L.orc_fpx_encode_d.argtypes = [C.POINTER(OrcFpx), vp, vp]
        L.orc_fpx_decode_f64_from.argtypes = [C.POINTER(OrcFpx), vp, vp]
        L.orc_fpx_decode_sig63_from.argtypes = [C.POINTER(OrcFpx), vp, vp, vp]
        L.orc_faithful_window.argtypes = [C.POINTER(OrcFpx), i, vp, vp]
        L.orc_faithful_cw.argtypes = [C.POINTER(OrcFpx), i, vp, vp]
        L.orc_fp32_rand.argtypes = [vp, C.c_size_t, u64, i, i]
        L.orc_entry_exact.argtypes = [vp, vp, i, i, i, i, i, vp, i]
        L.orc_freivalds.argtypes = [vp, vp, i, i, i, vp, i, i, u64]
        L.orc_freivalds_conv.argtypes = [vp, vp, i, i, vp, i, u64]

    # ---- inputs -----------------------------------------------------------
    def bigmat_rand(self, n, L, seed):
        m = np.empty(L * n * n, dtype=np.uint16)
        self.lib.orc_bigmat_rand(_p(m), n, L, seed)
        return m

    def fp32_rand(self, count, seed, emin=-20, emax=20):
        x = np.empty(count, dtype=np.float32)
        self.lib.orc_fp32_rand(_p(x), count, seed, emin, emax)
        return x

    # ---- plan ---------------------------------------------------------------
    def plan(self, L, sigma=0):
        p = PlanStruct()
        if self.lib.orc_plan_init(C.byref(p), L, sigma) != 0:
            return None
        return p

    # ---- products -------------------------------------------------------------
    def normalize(self, acc, nplanes, n, RL):
        out = np.empty(RL * n * n, dtype=np.uint16)
        self.lib.orc_normalize_planes(_p(np.ascontiguousarray(acc, np.int64)), nplanes, n, _p(out), RL)
        return out

    def mm_accum(self, Cacc, A, B, n, sign, packed=True):
        f = self.lib.orc_mm_accum_packed if packed else self.lib.orc_mm_accum_ikj
        f(_p(Cacc), _p(A), _p(B), n, sign)

    def conv_limbplane(self, A32, B32, n, L, leaf=2):
        cw = np.empty((2 * L - 1) * n * n, dtype=np.int64)
        self.lib.orc_conv_limbplane(_p(cw), _p(A32), _p(B32), n, L, leaf)
        return cw

    def mm_limbplane(self, A, B, n, L, RL, leaf=2):
        out = np.empty(RL * n * n, dtype=np.uint16)
        self.lib.orc_mm_limbplane(_p(A), _p(B), n, L, _p(out), RL, leaf)
        return out

    def mm_bigint_ijk(self, A, B, n, L, RL):
        Aem = np.empty_like(A)
        Bem = np.empty_like(B)
        self.lib.orc_to_entry_major(_p(A), n, L, _p(Aem))
        self.lib.orc_to_entry_major(_p(B), n, L, _p(Bem))
        out = np.empty(RL * n * n, dtype=np.uint16)
        self.lib.orc_mm_bigint_ijk(_p(Aem), _p(Bem), n, L, _p(out), RL)
        return out

    def conv_mfft(self, A32, B32, n, L, plan, leaf=2):
        cw = np.empty((2 * L - 1) * n * n, dtype=np.int64)
        self.lib.orc_conv_mfft(_p(cw), _p(A32), _p(B32), n, L, C.byref(plan), leaf)
        return cw

    def mm_mfft(self, A, B, n, L, plan, RL, leaf=2):
        out = np.empty(RL * n * n, dtype=np.uint16)
        self.lib.orc_mm_mfft(_p(A), _p(B), n, L, C.byref(plan), _p(out), RL, leaf)
        return out

    def ring_dft(self, x, NB, K, g, direction):
        x = np.ascontiguousarray(x, dtype=np.int64)
        X = np.empty(NB * K, dtype=np.int64)
        self.lib.orc_ring_dft(_p(X), _p(x), NB, K, g, direction)
        return X

    def fft_forward32(self, X, NB, K, g, nn):
        """in place: NB*K int32 planes of nn values, natural -> bit-reversed
        point order (src/mfft.c:173-258)"""
        assert X.dtype == np.int32 and X.flags.c_contiguous and X.size == NB * K * nn
        self.lib.orc_fft_forward32(_p(X), NB, K, g, nn)
        return X

    # ---- fp32 ----------------------------------------------------------------
    def fpx(self, A, B, n, force_bits):
        """encode A, B; returns (ctx, A32, B32) with numpy views of the planes"""
        ctx = OrcFpx()
        if self.lib.orc_fpx_init(C.byref(ctx), _p(A), _p(B), n, force_bits) != 0:
            return None
        self.lib.orc_fpx_encode(C.byref(ctx), _p(A), _p(B))
        return ctx

    def fpx_d(self, A, B, n, force_bits):
        """fp64 counterpart of fpx()"""
        ctx = OrcFpx()
        if self.lib.orc_fpx_init_d(C.byref(ctx), _p(A), _p(B), n, force_bits) != 0:
            return None
        self.lib.orc_fpx_encode_d(C.byref(ctx), _p(A), _p(B))
        return ctx

    def fpx_decode_f64_from(self, ctx, Cw):
        out = np.empty(ctx.n * ctx.n, dtype=np.float64)
        self.lib.orc_fpx_decode_f64_from(C.byref(ctx), _p(np.ascontiguousarray(Cw, np.int64)),
                                         _p(out))
        return out

    def fpx_decode_sig63_from(self, ctx, Cw):
        """long double decode as (sig, ex): value = sig * 2**ex"""
        sig = np.empty(ctx.n * ctx.n, dtype=np.int64)
        ex = np.empty(ctx.n * ctx.n, dtype=np.int32)
        self.lib.orc_fpx_decode_sig63_from(C.byref(ctx), _p(np.ascontiguousarray(Cw, np.int64)),
                                           _p(sig), _p(ex))
        return sig, ex

    def fpx_planes(self, ctx):
        nn = ctx.n * ctx.n
        buf = lambda ptr, cnt, ct: np.ctypeslib.as_array(C.cast(ptr, C.POINTER(ct)), shape=(cnt,))
        return (buf(ctx.A32, ctx.L * nn, C.c_int32).copy(),
                buf(ctx.B32, ctx.L * nn, C.c_int32).copy())

    def fpx_decode_from(self, ctx, Cw):
        out = np.empty(ctx.n * ctx.n, dtype=np.float32)
        self.lib.orc_fpx_decode_f32_from(C.byref(ctx), _p(np.ascontiguousarray(Cw, np.int64)), _p(out))
        return out

    def fpx_free(self, ctx):
        self.lib.orc_fpx_free(C.byref(ctx))

    def faithful_window(self, ctx, max_keep):
        """(Lk, u0, hi) of the faithful limb window (src/mlgemm.c:593-630)"""
        u0, hi = C.c_int(), C.c_int()
        Lk = self.lib.orc_faithful_window(C.byref(ctx), max_keep, C.byref(u0), C.byref(hi))
        return Lk, u0.value, hi.value

    def faithful_cw(self, ctx, max_keep):
        """the faithful product's 2L-1 coefficient planes, Lk, u0"""
        cw = np.empty((2 * ctx.L - 1) * ctx.n * ctx.n, dtype=np.int64)
        u0 = C.c_int()
        Lk = self.lib.orc_faithful_cw(C.byref(ctx), max_keep, _p(cw), C.byref(u0))
        return cw, Lk, u0.value

    # ---- checks -------------------------------------------------------------
    def entry_exact(self, A, B, n, L, i, j, RL, signed_top=False):
        limbs = np.empty(RL, dtype=np.uint16)
        self.lib.orc_entry_exact(_p(A), _p(B), n, L, int(signed_top), i, j, _p(limbs), RL)
        return limbs

    def freivalds(self, A, B, n, L, out, RL, signed_top=False, nprimes=2, seed=7):
        return bool(self.lib.orc_freivalds(_p(A), _p(B), n, L, int(signed_top), _p(out), RL,
                                           nprimes, seed))

    def freivalds_conv(self, A32, B32, n, L, Cw, nprimes=2, seed=7):
        return bool(self.lib.orc_freivalds_conv(_p(A32), _p(B32), n, L, _p(Cw), nprimes, seed))


class Reference:
    """The reference's own CPU library, built from its sources by
    oracle/ref.mk.  Absent on machines where it was not built."""

    KERNEL_IKJ, KERNEL_PACKED = 0, 2

    def __init__(self, path=None):
        path = path or _pick("_ref", "libmfftref")
        if path is None:
            raise FileNotFoundError("reference library not built (make -C oracle ref)")
        self.path = path
        L = self.lib = C.CDLL(path)
        vp, i, u64 = C.c_void_p, C.c_int, C.c_uint64
        L.bigmat_rand.argtypes = [vp, i, i, u64]
        L.normalize_planes.argtypes = [vp, i, i, vp, i]
        L.mm_accum.argtypes = [vp, vp, vp, i, i, i]
        L.mfft_plan_init.argtypes = [C.POINTER(RefPlanStruct), i, i]
        L.mfft_plan_maxbits.argtypes = [C.POINTER(RefPlanStruct), i]
        L.mfft_plan_maxbits.restype = C.c_double
        L.mm_mfft.argtypes = [vp, vp, i, i, C.POINTER(RefPlanStruct), i, vp, i]
        L.conv_mfft.argtypes = [vp, vp, vp, i, i, C.POINTER(RefPlanStruct), i]
        L.mm_limbplane.argtypes = [vp, vp, i, i, i, vp, i]
        L.conv_limbplane.argtypes = [vp, vp, vp, i, i, i]
        L.fpx_init.argtypes = [C.POINTER(RefFpx), vp, vp, i, i]
        L.fpx_encode.argtypes = [C.POINTER(RefFpx), vp, vp]
        L.fpx_decode_f32.argtypes = [C.POINTER(RefFpx), vp]
        L.fpx_free.argtypes = [C.POINTER(RefFpx)]
        L.fpx_init_d.argtypes = [C.POINTER(RefFpx), vp, vp, i, i]
        L.fpx_encode_d.argtypes = [C.POINTER(RefFpx), vp, vp]
        L.fpx_decode_f64.argtypes = [C.POINTER(RefFpx), vp]
        L.fpx_decode_ld.argtypes = [C.POINTER(RefFpx), vp]

    def bigmat_rand(self, n, L, seed):
        m = np.empty(L * n * n, dtype=np.uint16)
        self.lib.bigmat_rand(_p(m), n, L, seed)
        return m

    def plan(self, L, sigma=0):
        p = RefPlanStruct()
        if self.lib.mfft_plan_init(C.byref(p), L, sigma) != 0:
            return None
        return p

    def mm_mfft(self, A, B, n, L, plan, RL, kernel=2):
        out = np.zeros(RL * n * n, dtype=np.uint16)
        self.lib.mm_mfft(_p(A), _p(B), n, L, C.byref(plan), kernel, _p(out), RL)
        return out

    def conv_mfft(self, A32, B32, n, L, plan, kernel=2):
        cw = np.zeros((2 * L - 1) * n * n, dtype=np.int64)
        self.lib.conv_mfft(_p(cw), _p(A32), _p(B32), n, L, C.byref(plan), kernel)
        return cw

    def mm_limbplane(self, A, B, n, L, RL, kernel=2):
        out = np.zeros(RL * n * n, dtype=np.uint16)
        self.lib.mm_limbplane(_p(A), _p(B), n, L, kernel, _p(out), RL)
        return out

    def mm_accum(self, Cacc, A, B, n, sign, kernel=2):
        self.lib.mm_accum(_p(Cacc), _p(A), _p(B), n, sign, kernel)

    def fpx_mfft_f32(self, A, B, n, force_bits, plan_L_cb=None):
        """encode -> conv_mfft (flat plan, packed) -> decode_f32, all in the
        reference library.  Returns (C, L, SA, SB, Cw)."""
        ctx = RefFpx()
        if self.lib.fpx_init(C.byref(ctx), _p(A), _p(B), n, force_bits) != 0:
            return None
        try:
            self.lib.fpx_encode(C.byref(ctx), _p(A), _p(B))
            plan = self.plan(ctx.L)
            self.lib.conv_mfft(ctx.Cw, ctx.A32, ctx.B32, n, ctx.L, C.byref(plan), 2)
            out = np.empty(n * n, dtype=np.float32)
            self.lib.fpx_decode_f32(C.byref(ctx), _p(out))
            nn = n * n
            cw = np.ctypeslib.as_array(C.cast(ctx.Cw, C.POINTER(C.c_int64)),
                                       shape=((2 * ctx.L - 1) * nn,)).copy()
            return out, ctx.L, ctx.SA, ctx.SB, cw
        finally:
            self.lib.fpx_free(C.byref(ctx))


    def fpx_f64(self, A, B, n, force_bits):
        """fp64 encode -> conv_limbplane (ikj leaf) -> decode_f64 and
        decode_ld in the reference library.  Returns (C64, Cld, L, SA, SB,
        A32, B32, Cw) with Cld as numpy longdouble."""
        ctx = RefFpx()
        if self.lib.fpx_init_d(C.byref(ctx), _p(A), _p(B), n, force_bits) != 0:
            return None
        try:
            self.lib.fpx_encode_d(C.byref(ctx), _p(A), _p(B))
            self.lib.conv_limbplane(ctx.Cw, ctx.A32, ctx.B32, n, ctx.L, 0)
            out = np.empty(n * n, dtype=np.float64)
            self.lib.fpx_decode_f64(C.byref(ctx), _p(out))
            old = np.empty(n * n, dtype=np.longdouble)
            self.lib.fpx_decode_ld(C.byref(ctx), _p(old))
            nn = n * n
            arr = lambda ptr, cnt, ct: np.ctypeslib.as_array(C.cast(ptr, C.POINTER(ct)),
                                                             shape=(cnt,)).copy()
            return (out, old, ctx.L, ctx.SA, ctx.SB, arr(ctx.A32, ctx.L * nn, C.c_int32),
                    arr(ctx.B32, ctx.L * nn, C.c_int32),
                    arr(ctx.Cw, (2 * ctx.L - 1) * nn, C.c_int64))
        finally:
            self.lib.fpx_free(C.byref(ctx))


def load_oracle():
    return Oracle()


def load_reference():
    """Reference library or None when it was not built on this machine."""
    try:
        return Reference()
    except (FileNotFoundError, OSError):
        return None
