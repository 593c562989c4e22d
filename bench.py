"""Benchmark: exact 1024 x 1024 products of 2048-bit unsigned integers on one
MI355X (gfx950), through the C-ABI of mfft-bench_amd/lib/libmfft_hip.so.

One step = one exact MFFT matmul (forward transforms of both operands,
batched int8-MFMA pointwise GEMM, inverse transform + fold, carry) of
device-resident seeded inputs (splitmix64, seeds 12345 and 12345^0xABCDEF,
generated on the device bit-identically to the reference's bigmat_rand).

Prints ONE JSON line.  `value` is ms per product (lower is better); the line
also carries the issued int8 TOPS, the pointwise kernel's fraction of the
int8 MFMA peak (`roofline`), the reference CPU path timed on a bounded
sample on this host (`cpu_baseline`), and, in `multimodular`, the same
product computed by residue number system arithmetic (mfh_rns_mm_dev, no
reference counterpart) on the same inputs, with whether its limbs equal the
MFFT product's.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for sub in ("mfft-bench_amd", "oracle"):
    sys.path.insert(0, os.path.join(ROOT, sub))

METRIC = "ms per exact 1024² 2048-bit matmul; effective int8 TOPS; % MFMA peak"
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POP/s
HBM_PEAK_GBS = 8000.0

CONFIGS = {
    # name: (n, W bits, kind)
    "c1": (64, 1024, "unsigned"),
    "c2": (256, 8192, "unsigned"),
    "c3": (1024, 2048, "unsigned"),
    "c4": (2048, 512, "fp32"),       # fp32 entries on a shared 512-bit grid
    "c5": (4096, 512, "signed"),
}

# Freivalds primes below 2^24: residues times residues summed over n <= 4096
# terms stay below 2^63, so plain int64 numpy suffices
FREIVALDS_PRIMES = (16777213, 16777199)


def planes_mod(planes, n, nlimbs, p, twos):
    """value of every entry of a plane-major u16 matrix mod p; twos reads the
    whole number as two's complement of nlimbs limbs"""
    import numpy as np
    v = planes.reshape(nlimbs, n * n)
    acc = np.zeros(n * n, dtype=np.int64)
    for w in range(nlimbs - 1, -1, -1):
        acc = (acc * 65536 + v[w].astype(np.int64)) % p
    if twos:
        wrap = pow(2, 16 * nlimbs, p)
        acc = np.where(v[nlimbs - 1] >= 0x8000, (acc - wrap) % p, acc)
    return acc.reshape(n, n)


def entries_mod_signed_top(planes, n, L, p, signed):
    """inputs: limbs 0..L-2 unsigned, limb L-1 int16 when signed"""
    import numpy as np
    v = planes.reshape(L, n * n)
    acc = np.zeros(n * n, dtype=np.int64)
    for u in range(L - 1, -1, -1):
        limb = v[u].astype(np.int64)
        if signed and u == L - 1:
            limb = np.where(limb >= 0x8000, limb - 65536, limb)
        acc = (acc * 65536 + limb) % p
    return acc.reshape(n, n)


def freivalds_check(A, B, out, n, L, RL, signed, seed=7):
    """out == A*B over Z_p for the primes above and a seeded random vector"""
    import numpy as np
    rng = np.random.default_rng(seed)
    for p in FREIVALDS_PRIMES:
        Am = entries_mod_signed_top(A, n, L, p, signed)
        Bm = entries_mod_signed_top(B, n, L, p, signed)
        Cm = planes_mod(out, n, RL, p, signed)
        r = rng.integers(0, p, size=n, dtype=np.int64)
        y = (Bm @ r) % p
        if not np.array_equal((Am @ y) % p, (Cm @ r) % p):
            return False
    return True


def host_rand_u16(n, L, seed):
    """SplitMix64 limbs, plane-major (the reference's bigmat_rand), numpy"""
    import numpy as np
    i = np.arange(1, L * n * n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + i * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return (z & np.uint64(0xFFFF)).astype(np.uint16)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_cpu():
    """(CPU model, usable cores) of this host"""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 0
    return model, cores


def cpu_baseline(n, L, nprod_total):
    """Reference CPU path (oracle/_ref: the reference's own C sources,
    packed leaf), 1 thread.  When a whole mm_mfft fits in about 10 s (the
    1024-bit n=64 workload: ~0.2 s) it is timed whole, best of 3.  Otherwise
    a bounded sample: `s` of the NB*K^2 leaf products timed at full n and
    scaled, plus the reference's own phase profile (transform, pack, fold,
    normalize) of a whole mm_mfft at n/8 with the same plan, scaled by 64
    (those phases are O(n^2))."""
    from oracle_ctypes import load_reference
    import numpy as np
    ref = load_reference()
    kind = "reference"
    if ref is None:
        return None
    model, ncores = host_cpu()
    lib = ref.lib
    rp = ref.plan(L)
    A = np.random.default_rng(1).integers(0, 1 << 16, size=n * n).astype(np.int32)
    B = np.random.default_rng(2).integers(0, 1 << 16, size=n * n).astype(np.int32)
    Cacc = np.zeros(n * n, dtype=np.int64)
    t0 = time.perf_counter()
    ref.mm_accum(Cacc, A, B, n, 1, ref.KERNEL_PACKED)
    est = (time.perf_counter() - t0) * nprod_total
    base = {"unit": "ms", "cores": 1, "kind": kind, "cpu_model": model, "host_cores": ncores}
    if est < 10.0:
        As = ref.bigmat_rand(n, L, 12345)
        Bs = ref.bigmat_rand(n, L, 12345 ^ 0xABCDEF)
        best = None
        for _ in range(3):
            t0 = time.perf_counter()
            ref.mm_mfft(As, Bs, n, L, rp, 2 * L + 1)
            dt = time.perf_counter() - t0
            best = dt if best is None else min(best, dt)
        return dict(base, value=round(best * 1e3, 3),
                    sample=(f"reference src/ built from source, packed leaf, 1 thread: whole "
                            f"mm_mfft at n={n}, L={L} on the seeded inputs, best of 3 "
                            f"(not extrapolated)"))
    # transformed values at these plans are at most ~21 bits; the leaf's cost
    # does not depend on the values.  Time leaf products until ~10 s of work.
    times = []
    while sum(times) < 10.0 and len(times) < 1024:
        t0 = time.perf_counter()
        ref.mm_accum(Cacc, A, B, n, 1, ref.KERNEL_PACKED)
        times.append(time.perf_counter() - t0)
    s = len(times)
    t_leaf = float(np.median(times))
    # phase profile of a whole mm_mfft at n/8
    ns = min(256, max(8, n // 8))
    prof_on = C.c_int.in_dll(lib, "g_mfft_profile")

    class Prof(C.Structure):
        _fields_ = [("pack", C.c_double), ("build_ops", C.c_double),
                    ("transform", C.c_double), ("pointwise", C.c_double),
                    ("fold", C.c_double), ("n_build", C.c_longlong), ("n_fft", C.c_longlong)]
    prof = Prof.in_dll(lib, "g_mfft_prof")
    lib.mfft_profile_reset()
    prof_on.value = 1
    As = ref.bigmat_rand(ns, L, 12345)
    Bs = ref.bigmat_rand(ns, L, 12345 ^ 0xABCDEF)
    t0 = time.perf_counter()
    ref.mm_mfft(As, Bs, ns, L, rp, 2 * L + 1)
    wall = time.perf_counter() - t0
    prof_on.value = 0
    rest_small = wall - prof.pointwise   # widen, pack, build_ops, transforms, fold, normalize
    scale = (n / ns) ** 2
    total_s = nprod_total * t_leaf + rest_small * scale
    return dict(base, value=round(total_s * 1e3, 1),
                sample=(f"reference src/ built from source, packed leaf, 1 thread: {s} of "
                        f"{nprod_total} n={n} leaf products timed (median {t_leaf:.3f} s each) "
                        f"x {nprod_total}; other phases from the reference's own profile of one "
                        f"mm_mfft at n={ns} ({rest_small:.3f} s) x {scale:.0f}; extrapolated"))


def rns_measure(n, L, kind, dA, dB, steps, warmup, want=None, fpx_scale=None):
    """The multi-modular product (mfh_rns_*) of the same device-resident
    inputs: ms per product, stage times, the int8 GEMMs it issues, and
    whether its output equals `want` (the MFFT product's).  With
    fpx_scale = (SA, SB) the inputs are fp32 on an L-limb grid and the
    product is mfh_rns_fpx_mm_dev's (encode, L + 1 two's complement limbs
    multiplied, decode); the stage times cover its integer product."""
    import numpy as np
    import mfft_ctypes as M
    fp32 = fpx_scale is not None
    Lr = L + 1 if fp32 else L
    RL = 2 * L + 1
    lib = M.load()
    try:
        r = M.Rns(n, Lr)
    except M.MfftError as e:
        log(f"[bench] multi-modular n={n} L={Lr}: {e}")
        return None
    if fp32:
        SA, SB = fpx_scale
        dO = M.DevBuf(n * n * 4)
        step = lambda: M.check(lib.mfh_rns_fpx_mm_dev(r.h, dA.ptr, dB.ptr, SA, SB, dO.ptr),
                               "mfh_rns_fpx_mm_dev")
    else:
        dO = M.DevBuf(RL * n * n * 2)
        step = lambda: M.check(lib.mfh_rns_mm_dev(r.h, kind, dA.ptr, dB.ptr, dO.ptr, RL),
                               "mfh_rns_mm_dev")
    for _ in range(max(1, warmup)):
        step()
    r.sync()
    r.set_timing(True)
    stage = np.zeros(4)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
        stage += np.array(r.stage_times())
    r.sync()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    r.set_timing(False)
    st = stage / steps
    nm, np_, nbytes = r.info()
    res_ops, pw_ops, crt_ops = r.work()
    equal = None
    if want is not None:
        got = dO.download(np.uint32, n * n) if fp32 else dO.download(np.uint16, RL * n * n)
        equal = bool(np.array_equal(got, want))
    dO.free()
    r.close()
    log(f"[bench] multi-modular: {ms:.3f} ms/product, stages(ms) residues {st[0]:.3f} "
        f"per-prime GEMMs {st[1]:.3f} CRT+carry {st[2]:.3f}; {nm} primes; equal to MFFT: {equal}")
    return {"ms_per_step": round(ms, 3), "primes": nm,
            "int8_gemms_per_product": 4 * nm,
            "stage_ms": {"residues": round(st[0], 3), "per_prime_gemms": round(st[1], 3),
                         "crt_carry": round(st[2], 3)},
            "int8_ops": {"residues": res_ops, "per_prime_gemms": pw_ops, "crt": crt_ops},
            "per_prime_gemm_tops": round(pw_ops / (st[1] * 1e-3) / 1e12, 1),
            "per_prime_gemm_frac": round(pw_ops / (st[1] * 1e-3) / 5.0e15, 4),
            "device_bytes": nbytes, "equal_to_mfft": equal,
            "note": (("fp32 product on the same grid by residues mod 16-bit primes "
                      "(mfh_rns_fpx_mm_dev: encode to L+1 two's complement limbs, exact "
                      "product, decode), same inputs and output bits as the MFFT path"
                      if fp32 else
                      "exact product by residues mod 16-bit primes (mfh_rns_mm_dev), same "
                      "inputs and output limbs as the MFFT product") +
                     "; no counterpart in the reference")}


def method_table(args):
    """The reference bench's result table (src/main.c:137-165) for the device
    methods on one exact-track workload: the schoolbook (limbplane, the
    speedup baseline as in src/main.c:293-297), the flat MFFT plan and the
    recursive plan (and, at K = 16, the flat plan with the K^2-product
    pointwise kernel forced); limbplane-mma is the schoolbook on the int8
    matrix cores; rns is the multi-modular product (no reference
    counterpart: its `products` count the primes, each 4 int8 GEMMs).
    `products` is each method's n x n product
    count as the reference defines it (mfft_plan.nprod); `issued` is the
    ring products the device issued (NB times the per-point count of
    mfh_pointwise_info; each is 6 or 9 int8 digit GEMMs); `kernel_calls` is
    the reference's count of leaf mm_accum calls, which the device methods do
    not make (0); `exact` compares every limb with the schoolbook's result
    and checks it by Freivalds' test."""
    n, W, ekind = CONFIGS[args.config]
    if ekind == "fp32":
        log("bench.py --table: exact-track workloads only (c1, c2, c3, c5)")
        sys.exit(2)
    return method_table_for(n, W, ekind, args)


def method_table_for(n, W, ekind, args, header=True):
    import numpy as np
    import mfft_ctypes as M
    signed = ekind == "signed"
    L = W // 16
    RL = 2 * L + 1
    lib = M.load()
    kind = M.MFH_IN_U16_SIGNED if signed else M.MFH_IN_U16
    in_bytes = L * n * n * 2
    dA, dB = M.DevBuf(in_bytes), M.DevBuf(in_bytes)
    dRef, dO = M.DevBuf(RL * n * n * 2), M.DevBuf(RL * n * n * 2)
    dCw = M.DevBuf((2 * L - 1) * n * n * 8)
    M.check(lib.mfh_rand_u16_dev(None, dA.ptr, n, L, 12345))
    M.check(lib.mfh_rand_u16_dev(None, dB.ptr, n, L, 12345 ^ 0xABCDEF))
    M.check(lib.mfh_sync(None))

    def timed(fn, steps):
        fn()
        M.check(lib.mfh_sync(None))
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        M.check(lib.mfh_sync(None))
        return (time.perf_counter() - t0) / steps

    rows = []
    secs = timed(lambda: M.check(lib.mfh_limbplane_mm_dev(None, kind, dA.ptr, dB.ptr, n, L,
                                                          dCw.ptr, dRef.ptr, RL)), 2)
    ref_out = dRef.download(np.uint16, RL * n * n)
    rows.append(["limbplane", "hip", L * L, L * L, 0, secs, ref_out])
    # the same schoolbook on the matrix cores (limb pairs issued in blocks
    # of 16 limbs, each 6 int8 digit GEMMs)
    wbytes = M.C.c_size_t()
    if lib.mfh_schoolbook_workspace(n, L, M.C.byref(wbytes)) == 0:
        dW = M.DevBuf(wbytes.value)
        secs = timed(lambda: M.check(lib.mfh_schoolbook_dev(None, kind, dA.ptr, dB.ptr, n, L,
                                                            dW.ptr, wbytes.value, dO.ptr, RL)),
                     max(1, min(args.steps, 3)))
        dW.free()
        nu16 = (L + 15) // 16 * 16
        rows.append(["limbplane-mma", "hip", L * L, nu16 * nu16, 0, secs,
                     dO.download(np.uint16, RL * n * n)])
    else:
        log(f"[table] limbplane-mma n={n} W={W}: outside its partial-sum bound")
    variants = [("mfft", M.plan(L), False), ("mfft-rec", M.plan_rec(L, n), False)]
    if M.plan(L) is not None and M.plan(L).K == 16:
        # the K^2-product kernel beside the default Gauss one at this ring
        variants.insert(1, ("mfft-flatpw", M.plan(L), True))
    for name, p, flat in variants:
        if p is None:
            continue
        if flat:
            os.environ["MFH_POINTWISE"] = "flat"
        try:
            ctx = M.Ctx(n, L, p)
        except M.MfftError as e:
            # outside the stated bounds (MFH_E_BOUND) or ring sizes: no row
            log(f"[table] {name} n={n} W={W}: {e}")
            continue
        finally:
            os.environ.pop("MFH_POINTWISE", None)
        secs = timed(lambda: M.check(lib.mfh_mm_dev(ctx.h, kind, dA.ptr, dB.ptr, dO.ptr, RL)),
                     max(1, args.steps))
        ctx.sync()
        out = dO.download(np.uint16, RL * n * n)
        ring, _ = ctx.pointwise_info()
        rows.append([name, "hip", p.nprod, p.NB * ring, 0, secs, out])
        ctx.close()
    # the multi-modular product (no reference counterpart): `products` and
    # `issued` count its per-prime n x n products (4 int8 GEMMs each)
    try:
        rns = M.Rns(n, L)
        secs = timed(lambda: M.check(lib.mfh_rns_mm_dev(rns.h, kind, dA.ptr, dB.ptr, dO.ptr, RL)),
                     max(1, args.steps))
        rns.sync()
        nm = rns.info()[0]
        rows.append(["rns", "hip", nm, nm, 0, secs, dO.download(np.uint16, RL * n * n)])
        rns.close()
    except M.MfftError as e:
        log(f"[table] rns n={n} W={W}: {e}")
    A = host_rand_u16(n, L, 12345)
    B = host_rand_u16(n, L, 12345 ^ 0xABCDEF)
    base = rows[0][5]
    for r in rows:
        out = r[6]
        ok = freivalds_check(A, B, out, n, L, RL, signed)
        ok = ok and bool(np.array_equal(out, ref_out))
        r[6] = ok
    if args.csv:
        if header:
            print("n,bits,method,kernel,products,issued,kernel_calls,seconds,speedup,exact")
        for name, k, prod, issued, calls, secs, ok in rows:
            print(f"{n},{W},{name},{k},{prod},{issued},{calls},{secs:.6f},"
                  f"{(base / secs if base else 0.0):.3f},{'yes' if ok else 'NO'}")
    else:
        print(f"n={n} W={W} ({ekind}) on {lib.mfh_device_arch().decode()}")
        print(f"\n{'method':<14} {'kernel':<9} {'n*n products':>12} {'issued':>8} "
              f"{'seconds':>10} {'speedup':>9}  exact")
        print("-" * 82)
        for name, k, prod, issued, calls, secs, ok in rows:
            print(f"{name:<14} {k:<9} {prod:>12} {issued:>8} {secs:>10.4f} "
                  f"{(base / secs if base else 0.0):>8.2f}x  {'yes' if ok else 'NO!'}")
    for b in (dA, dB, dRef, dO, dCw):
        b.free()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS))
    ap.add_argument("--n", type=int, default=0,
                    help="with --bits: an exact-track workload of this size instead of --config "
                         "(the reference bench's --n / --bits, src/main.c:333-366)")
    ap.add_argument("--bits", "--width", type=int, default=0,
                    help="entry width W (a power of two >= 32)")
    ap.add_argument("--signed", action="store_true",
                    help="with --n/--bits: two's complement entries")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-verify", action="store_true")
    ap.add_argument("--no-rns", action="store_true",
                    help="skip the multi-modular product reported beside the MFFT one")
    ap.add_argument("--rns-only", action="store_true",
                    help="only the multi-modular product of the workload (--warmup untimed, "
                         "--steps timed; no MFFT kernels run), e.g. for counter passes")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run the plain copy kernel over MIB MiB, --steps times (the "
                         "known-size kernel that HBM byte counters are calibrated against)")
    ap.add_argument("--traffic-json", default=os.path.join(ROOT, "profiles", "traffic.json"),
                    help="HBM bytes per pointwise launch measured by rocprofv3 --pmc")
    ap.add_argument("--table", action="store_true",
                    help="instead of the JSON line: the reference bench's method table "
                         "(src/main.c:137-165) for the device methods on this workload")
    ap.add_argument("--csv", action="store_true", help="the same table as CSV")
    ap.add_argument("--sweep-width", "--sweep", action="store_true",
                    help="the method table at widths 128, 256, .., 8192 bits for --n "
                         "(default 64), as src/main.c:384-386")
    ap.add_argument("--sweep-n", action="store_true",
                    help="the method table at n = 32, 64, .. up to --n (default 64) for "
                         "--width (default 256), as src/main.c:387-389")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); products shard over GPUs by output tiles with no "
              f"exchange step, which this library does not implement",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import mfft_ctypes as M

    if args.copy_probe:
        lib = M.load()
        nbytes = args.copy_probe << 20
        src, dst = M.DevBuf(nbytes), M.DevBuf(nbytes)
        M.check(lib.mfh_rand_u16_dev(None, src.ptr, 1024, nbytes // (2 << 20), 1))
        M.check(lib.mfh_sync(None))
        t0 = time.perf_counter()
        for _ in range(args.steps):
            M.check(lib.mfh_copy_dev(None, dst.ptr, src.ptr, nbytes), "mfh_copy_dev")
        M.check(lib.mfh_sync(None))
        dt = (time.perf_counter() - t0) / args.steps
        log(f"[bench] copy {args.copy_probe} MiB: {dt * 1e3:.3f} ms, "
            f"{2 * nbytes / dt / 1e9:.1f} GB/s read+write")
        src.free()
        dst.free()
        return

    if args.sweep_width or args.sweep_n:
        ekind = "signed" if args.signed else "unsigned"
        nmax = args.n or 64
        W = args.bits or 256
        if nmax < 1 or W < 32 or W & (W - 1):
            log("bench.py: sweeps need --n >= 1 and --width a power of two >= 32")
            sys.exit(2)
        cases = ([(nmax, b) for b in (128, 256, 512, 1024, 2048, 4096, 8192)]
                 if args.sweep_width else
                 [(m, W) for m in (32 << i for i in range(16)) if m <= nmax])
        for i, (m, b) in enumerate(cases):
            if i and not args.csv:
                print()
            method_table_for(m, b, ekind, args, header=(i == 0))
        return

    if args.n or args.bits:
        if not (args.n > 0 and args.bits >= 32 and args.bits & (args.bits - 1) == 0):
            log("bench.py: --n N --bits W needs N >= 1 and W a power of two >= 32")
            sys.exit(2)
        CONFIGS["custom"] = (args.n, args.bits, "signed" if args.signed else "unsigned")
        args.config = "custom"

    if args.table or args.csv:
        method_table(args)
        return

    n, W, ekind = CONFIGS[args.config]
    signed = ekind == "signed"
    fp32 = ekind == "fp32"
    L = W // 16
    RL = 2 * L + 1
    lib = M.load()
    SA = SB = W // 2
    if args.rns_only:
        eb = 4 * n * n if fp32 else L * n * n * 2
        dA, dB = M.DevBuf(eb), M.DevBuf(eb)
        for d, seed in ((dA, 12345), (dB, 12345 ^ 0xABCDEF)):
            if fp32:
                M.check(lib.mfh_rand_f32_dev(None, d.ptr, n * n, seed, -20, 20))
            else:
                M.check(lib.mfh_rand_u16_dev(None, d.ptr, n, L, seed))
        M.check(lib.mfh_sync(None))
        kind = M.MFH_IN_U16_SIGNED if signed else M.MFH_IN_U16
        mm = rns_measure(n, L, kind, dA, dB, args.steps, args.warmup,
                         fpx_scale=(SA, SB) if fp32 else None)
        print(json.dumps({"workload": args.config, "n": n, "width_bits": W, "entries": ekind,
                          "multimodular": mm}), flush=True)
        return
    p = M.plan(L)
    ctx = M.Ctx(n, L, p)
    if fp32:
        dA, dB, dO = M.DevBuf(n * n * 4), M.DevBuf(n * n * 4), M.DevBuf(n * n * 4)
        M.check(lib.mfh_rand_f32_dev(ctx.h, dA.ptr, n * n, 12345, -20, 20))
        M.check(lib.mfh_rand_f32_dev(ctx.h, dB.ptr, n * n, 12345 ^ 0xABCDEF, -20, 20))
    else:
        in_bytes = L * n * n * 2
        dA, dB, dO = M.DevBuf(in_bytes), M.DevBuf(in_bytes), M.DevBuf(RL * n * n * 2)
        M.check(lib.mfh_rand_u16_dev(ctx.h, dA.ptr, n, L, 12345))
        M.check(lib.mfh_rand_u16_dev(ctx.h, dB.ptr, n, L, 12345 ^ 0xABCDEF))
    kind = M.MFH_IN_U16_SIGNED if signed else M.MFH_IN_U16
    ctx.sync()

    def step():
        if fp32:
            M.check(lib.mfh_fpx_mm_dev(ctx.h, dA.ptr, dB.ptr, SA, SB, dO.ptr), "mfh_fpx_mm_dev")
        else:
            M.check(lib.mfh_mm_dev(ctx.h, kind, dA.ptr, dB.ptr, dO.ptr, RL), "mfh_mm_dev")

    log(f"[bench] {args.config}: n={n} W={W} L={L} plan={p} warmup={args.warmup} steps={args.steps}"
        f" row band {ctx.band_rows()} of {-(-n // 64) * 64} padded rows")
    for _ in range(args.warmup):
        step()
    ctx.sync()
    ctx.set_timing(True)
    stage = np.zeros(5)
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
        # events are recorded around each stage on the context's stream; read
        # them back per step (the host waits only on the final event)
        stage += np.array(ctx.stage_times())
    ctx.sync()
    elapsed = time.perf_counter() - t0
    ctx.set_timing(False)
    ms = elapsed * 1e3 / args.steps
    st = stage / args.steps
    # int8 ops the pointwise kernel issued (over the np = 64-padded size: n
    # here is a multiple of 64 unless --n says otherwise), and the minimum
    # HBM bytes of the forward and inverse stages
    ops, fwd_b, inv_b = ctx.work()
    inv_bytes = inv_b          # inverse + fold + carry/decode, as the library ran them
    ring_pp, digit_pp = ctx.pointwise_info()
    nprod = p.NB * p.K * p.K
    # the effective rate on the 9-digit-product basis BASELINE.md defines
    # (9 NB K^2 2 n^3 int8 ops per product, whatever the kernels issue)
    ops9 = 9.0 * nprod * 2.0 * float(n) ** 3
    tops_issued = ops / (ms * 1e-3) / 1e12
    tops_pw = ops / (st[1] * 1e-3) / 1e12
    log(f"[bench] ms/product {ms:.3f}  stages(ms) fwd {st[0]:.3f} pw {st[1]:.3f} "
        f"inv {st[2]:.3f} carry {st[3]:.3f}  pointwise {tops_pw:.1f} TOPS")

    verified = None
    if not args.no_verify and not fp32:
        A = host_rand_u16(n, L, 12345)
        B = host_rand_u16(n, L, 12345 ^ 0xABCDEF)
        out = dO.download(np.uint16, RL * n * n)
        verified = freivalds_check(A, B, out, n, L, RL, signed)
        log(f"[bench] verification (Freivalds mod 2 primes): {verified}")

    traffic = None
    try:
        with open(args.traffic_json) as f:
            tj = json.load(f)
        traffic = tj.get(args.config, {}).get("pointwise_bytes")
    except (OSError, ValueError):
        pass

    mm = None
    if not args.no_rns:
        if fp32:
            mm = rns_measure(n, L, kind, dA, dB, args.steps, args.warmup,
                             dO.download(np.uint32, n * n), fpx_scale=(SA, SB))
        else:
            mm = rns_measure(n, L, kind, dA, dB, args.steps, args.warmup,
                             dO.download(np.uint16, RL * n * n))

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] timing the reference CPU path on a bounded sample ...")
        cpu = cpu_baseline(n, L, nprod)

    line = {
        "metric": METRIC,
        "value": round(ms, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 MFMA, int32/int64 accumulate",
        "data": "synthetic",
        "config": {"workload": (f"fp32 embedding on a {W}-bit grid, n={n}, entries +-m*2^e "
                                 f"(e in [-20, 20]), exact MFFT product rounded once to fp32"
                                 if fp32 else
                                 f"exact MFFT matmul, n={n}, W={W}-bit {ekind} entries "
                                 f"(L={L} limbs)") +
                               f", plan S={p.S} NB={p.NB} K={p.K}, seeds 12345/12345^0xABCDEF",
                   "n": n, "width_bits": W, "limbs": L, "S": p.S, "NB": p.NB, "K": p.K,
                   "parallelism": "single GPU"},
        "int8_tops_effective": round(ops9 / (ms * 1e-3) / 1e12, 1),
        "int8_tops_issued": round(tops_issued, 1),
        "int8_tops_basis": (f"effective: 9*NB*K^2*2n^3 = {ops9:.4g} int8 ops per product (9 "
                            f"digit products per ring product, K^2 ring products per point); "
                            f"issued: {ops:.4g} int8 ops the pointwise kernel ran ({digit_pp} "
                            f"digit products x {ring_pp} ring products per point)"),
        "pointwise": {"ring_products_per_point": ring_pp, "digit_products": digit_pp,
                      "algorithm": ("Gauss split of the ring halves (3 (K/2)^2)"
                                    if ring_pp != p.K * p.K else "K^2 ring products")},
        "mfma_pct_pointwise": round(100.0 * tops_pw / INT8_PEAK_TOPS, 2),
        "decomposition_independent_tops": round(nprod * 2.0 * n ** 3 / (ms * 1e-3) / 1e12, 2),
        "stage_ms": {"forward": round(st[0], 3), "pointwise": round(st[1], 3),
                     "inverse_fold": round(st[2], 3), "carry": round(st[3], 3)},
        "hbm_gbs": {"forward": round(fwd_b / (st[0] * 1e-3) / 1e9, 1),
                    "inverse_fold_carry": round(inv_bytes / ((st[2] + st[3]) * 1e-3) / 1e9, 1)},
        "verified": verified,
        "roofline": {"bound": "mfma", "achieved": round(tops_pw, 1), "peak": INT8_PEAK_TOPS,
                     "unit": "TOPS", "frac": round(tops_pw / INT8_PEAK_TOPS, 4),
                     "traffic": traffic,
                     "note": "int8 tera-operations per second issued by the pointwise kernel "
                             "(dense int8 MFMA peak 5.0 POP/s)"},
        "cpu_baseline": cpu,
        "multimodular": mm,
    }
    print(json.dumps(line), flush=True)
    for b in (dA, dB, dO):
        b.free()
    ctx.close()


if __name__ == "__main__":
    main()
