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
