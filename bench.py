"""Benchmark: exact 1024 x 1024 products of 2048-bit unsigned integers on one
MI355X (gfx950), through the C-ABI of mfft-bench_amd/lib/libmfft_hip.so.

One step = one exact MFFT matmul (forward transforms of both operands,
batched int8-MFMA pointwise GEMM, inverse transform + fold, carry) of
device-resident seeded inputs (splitmix64, seeds 12345 and 12345^0xABCDEF,
generated on the device bit-identically to the reference's bigmat_rand).

Prints ONE JSON line.  `value` is ms per product (lower is better); the line
also carries the issued int8 TOPS, the pointwise kernel's fraction of the
int8 MFMA peak (`roofline`), and the reference CPU path timed on a bounded
sample on this host (`cpu_baseline`).
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
    # name: (n, W bits, signed)
    "c1": (64, 1024, False),
    "c2": (256, 8192, False),
    "c3": (1024, 2048, False),
    "c5": (4096, 512, True),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(n, L, nprod_total, plan_tuple):
    """Reference CPU path (oracle/_ref: the reference's own C sources,
    packed leaf) on a bounded sample, 1 thread.  Pointwise: `s` of the
    NB*K^2 leaf products timed at full n and scaled.  Transform, pack, fold
    and normalize: the reference's own phase profile of a whole mm_mfft at
    n/8 with the same plan, scaled by 64 (those phases are O(n^2))."""
    from oracle_ctypes import load_reference, Oracle, RefPlanStruct
    import numpy as np
    ref = load_reference()
    kind = "reference"
    if ref is None:
        return None
    lib = ref.lib
    s = 6
    A = np.random.default_rng(1).integers(0, 1 << 16, size=n * n).astype(np.int32)
    B = np.random.default_rng(2).integers(0, 1 << 16, size=n * n).astype(np.int32)
    # transformed values at the C3 plan are ~21-bit; the leaf's cost does not
    # depend on the values
    Cacc = np.zeros(n * n, dtype=np.int64)
    best = 1e30
    for _ in range(s):
        t0 = time.perf_counter()
        ref.mm_accum(Cacc, A, B, n, 1, ref.KERNEL_PACKED)
        best = min(best, time.perf_counter() - t0)
    t_leaf = best
    # phase profile of a whole mm_mfft at n/8
    ns = max(8, n // 8)
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
    rp = ref.plan(L)
    t0 = time.perf_counter()
    ref.mm_mfft(As, Bs, ns, L, rp, 2 * L + 1)
    wall = time.perf_counter() - t0
    prof_on.value = 0
    rest_small = wall - prof.pointwise   # widen, pack, build_ops, transforms, fold, normalize
    scale = (n / ns) ** 2
    total_s = nprod_total * t_leaf + rest_small * scale
    return {
        "value": round(total_s * 1e3, 1), "unit": "ms", "cores": 1, "kind": kind,
        "sample": (f"reference src/ built from source, packed leaf, 1 thread: {s} of "
                   f"{nprod_total} n={n} leaf products timed (best {t_leaf:.3f} s each) "
                   f"x {nprod_total}; other phases from the reference's own profile of one "
                   f"mm_mfft at n={ns} ({rest_small:.3f} s) x {scale:.0f}; extrapolated"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-verify", action="store_true")
    ap.add_argument("--traffic-json", default=os.path.join(ROOT, "profiles", "traffic.json"),
                    help="HBM bytes per pointwise launch measured by rocprofv3 --pmc")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); the multi-GPU sharding is described in DESIGN.md",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import mfft_ctypes as M

    n, W, signed = CONFIGS[args.config]
    L = W // 16
    RL = 2 * L + 1
    lib = M.load()
    p = M.plan(L)
    ctx = M.Ctx(n, L, p)
    in_bytes = L * n * n * 2
    dA, dB, dO = M.DevBuf(in_bytes), M.DevBuf(in_bytes), M.DevBuf(RL * n * n * 2)
    M.check(lib.mfh_rand_u16_dev(ctx.h, dA.ptr, n, L, 12345))
    M.check(lib.mfh_rand_u16_dev(ctx.h, dB.ptr, n, L, 12345 ^ 0xABCDEF))
    kind = M.MFH_IN_U16_SIGNED if signed else M.MFH_IN_U16
    ctx.sync()

    def step():
        M.check(lib.mfh_mm_dev(ctx.h, kind, dA.ptr, dB.ptr, dO.ptr, RL), "mfh_mm_dev")

    log(f"[bench] {args.config}: n={n} W={W} L={L} plan={p} warmup={args.warmup} steps={args.steps}")
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
    ops, fwd_b, inv_b = ctx.work()
    nprod = p.NB * p.K * p.K
    tops_issued = ops / (ms * 1e-3) / 1e12
    tops_pw = ops / (st[1] * 1e-3) / 1e12
    log(f"[bench] ms/product {ms:.3f}  stages(ms) fwd {st[0]:.3f} pw {st[1]:.3f} "
        f"inv {st[2]:.3f} carry {st[3]:.3f}  pointwise {tops_pw:.1f} TOPS")

    verified = None
    if not args.no_verify:
        from oracle_ctypes import Oracle
        orc = Oracle()
        A = orc.bigmat_rand(n, L, 12345)
        B = orc.bigmat_rand(n, L, 12345 ^ 0xABCDEF)
        out = dO.download(np.uint16, RL * n * n)
        verified = orc.freivalds(A, B, n, L, out, RL, signed_top=signed, nprimes=2)
        ok_entries = True
        rng = np.random.default_rng(5)
        for _ in range(4):
            i, j = (int(x) for x in rng.integers(0, n, size=2))
            want = orc.entry_exact(A, B, n, L, i, j, RL, signed_top=signed)
            got = out.reshape(RL, n * n)[:, i * n + j]
            ok_entries &= bool(np.array_equal(want, got))
        verified = bool(verified and ok_entries)
        log(f"[bench] verification (Freivalds mod 2 primes + 4 exact entries): {verified}")

    traffic = None
    try:
        with open(args.traffic_json) as f:
            tj = json.load(f)
        traffic = tj.get(args.config, {}).get("pointwise_bytes")
    except (OSError, ValueError):
        pass

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] timing the reference CPU path on a bounded sample ...")
        cpu = cpu_baseline(n, L, nprod, p)

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
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"exact MFFT matmul, n={n}, W={W}-bit "
                               f"{'signed' if signed else 'unsigned'} entries (L={L} limbs), "
                               f"plan S={p.S} NB={p.NB} K={p.K}, seeds 12345/12345^0xABCDEF",
                   "n": n, "width_bits": W, "limbs": L, "S": p.S, "NB": p.NB, "K": p.K,
                   "parallelism": "single GPU"},
        "int8_tops_effective": round(tops_issued, 1),
        "mfma_pct_pointwise": round(100.0 * tops_pw / INT8_PEAK_TOPS, 2),
        "decomposition_independent_tops": round(nprod * 2.0 * n ** 3 / (ms * 1e-3) / 1e12, 2),
        "stage_ms": {"forward": round(st[0], 3), "pointwise": round(st[1], 3),
                     "inverse_fold": round(st[2], 3), "carry": round(st[3], 3)},
        "hbm_gbs": {"forward": round(fwd_b / (st[0] * 1e-3) / 1e9, 1),
                    "inverse_fold_carry": round((inv_b + (2 * L - 1) * n * n * 8 + RL * n * n * 2)
                                                / ((st[2] + st[3]) * 1e-3) / 1e9, 1)},
        "verified": verified,
        "roofline": {"bound": "mfma", "achieved": round(tops_pw, 1), "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(tops_pw / INT8_PEAK_TOPS, 4),
                     "traffic": traffic},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    for b in (dA, dB, dO):
        b.free()
    ctx.close()


if __name__ == "__main__":
    main()
