"""bench.py's method table (src/main.c:137-165) and its sweeps
(src/main.c:381-390) on the device, in this process: every row's limbs
equal the schoolbook's and pass Freivalds' test."""
import argparse
import contextlib
import io
import os
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def _rows(n, W, signed=False):
    import bench
    args = argparse.Namespace(csv=True, steps=1)
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        bench.method_table_for(n, W, "signed" if signed else "unsigned", args, header=False)
    return [line.split(",") for line in buf.getvalue().splitlines() if line]


@pytest.mark.parametrize("W", [128, 256, 512, 1024, 2048, 4096, 8192])
def test_sweep_width_rows_exact(gpu, W):
    """--sweep-width at n = 32: limbplane, limbplane-mma (the schoolbook on
    the matrix cores), mfft (and mfft-flatpw at K = 16) and mfft-rec rows,
    all exact."""
    print(f"[table] n=32 W={W}", flush=True)
    rows = _rows(32, W)
    names = [r[2] for r in rows]
    assert names[:2] == ["limbplane", "limbplane-mma"] and "mfft" in names
    for r in rows:
        assert r[-1] == "yes", r
    mfft = next(r for r in rows if r[2] == "mfft")
    assert int(mfft[4]) > 0 and int(mfft[5]) > 0          # products, issued


@pytest.mark.parametrize("n", [32, 64, 96])
def test_sweep_n_rows_exact(gpu, n):
    rows = _rows(n, 256, signed=(n == 96))
    for r in rows:
        assert r[-1] == "yes", r


def _bench_json(argv):
    import json
    import bench
    buf = io.StringIO()
    old = sys.argv
    sys.argv = ["bench.py"] + argv
    try:
        with contextlib.redirect_stdout(buf):
            bench.main()
    finally:
        sys.argv = old
    return json.loads([line for line in buf.getvalue().splitlines() if line.startswith("{")][-1])


def test_bench_line_multimodular_equal(gpu):
    """bench.py's JSON line at the 1024-bit workload: the MFFT product and,
    beside it, the multi-modular product of the same device inputs with
    limbs equal to the MFFT's; --rns-only runs the latter alone"""
    d = _bench_json(["--config", "c1", "--steps", "2", "--warmup", "1", "--no-cpu-baseline"])
    assert d["value"] > 0 and d["n_gpus"] == 1
    mm = d["multimodular"]
    assert mm["equal_to_mfft"] is True and mm["primes"] == 129 and mm["ms_per_step"] > 0
    r = _bench_json(["--rns-only", "--config", "c1", "--steps", "2", "--warmup", "1"])
    assert r["multimodular"]["primes"] == 129 and r["multimodular"]["ms_per_step"] > 0


def test_bench_line_multimodular_fp32_equal(gpu, lib):
    """bench.py's multi-modular measurement on fp32 inputs (n = 256 on the
    512-bit grid, entries +-m 2^e, e in [-20, 20]): output bits equal to
    the MFFT path's on the same device inputs"""
    import numpy as np
    import bench
    n, L, S = 256, 32, 256
    dA, dB, dC = gpu.DevBuf(n * n * 4), gpu.DevBuf(n * n * 4), gpu.DevBuf(n * n * 4)
    try:
        gpu.check(lib.mfh_rand_f32_dev(None, dA.ptr, n * n, 12345, -20, 20))
        gpu.check(lib.mfh_rand_f32_dev(None, dB.ptr, n * n, 12345 ^ 0xABCDEF, -20, 20))
        gpu.check(lib.mfh_sync(None))
        with gpu.Ctx(n, L) as ctx:
            gpu.check(lib.mfh_fpx_mm_dev(ctx.h, dA.ptr, dB.ptr, S, S, dC.ptr))
            ctx.sync()
        want = dC.download(np.uint32, n * n)
        with contextlib.redirect_stderr(io.StringIO()):
            mm = bench.rns_measure(n, L, gpu.MFH_IN_U16, dA, dB, 2, 1, want, fpx_scale=(S, S))
    finally:
        for b in (dA, dB, dC):
            b.free()
    assert np.count_nonzero(want) > n * n // 2
    assert mm["equal_to_mfft"] is True and mm["primes"] == 67
