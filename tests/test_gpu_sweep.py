"""A seeded sweep of product shapes through tmh_block_matmul, every format
and the reference's BlockMatMulMode values: each case's outputs bit for bit
against the oracle's Quant.matmul (quant.cr:155-182, pinned to
matmul_reference by the CPU tests), bias after the sum (host.cr:725-734).

The fixed-shape tests name the shapes the kernels were built around; this
sweep reaches the ones in between -- odd block counts, K that is not a
multiple of 64, 256 or 512, ragged outputs, activation rows with a padded
stride, a weight sliced by rows -- on every route AUTO and the explicit
modes take (one-row kernels, the few-rows kernels, the lanes and thread
kernels, the matrix cores).
"""
import sys

import numpy as np
import pytest

from oracle import oracle
import tensomite_hip as th

pytestmark = pytest.mark.gpu

FORMATS = ["Q8_0", "Q4_0", "Q4_1"]
MODES = ["auto", "thread", "lanes", "loads", "stream", "stream_activations", "matrix"]
CASES = 60  # per format
# AUTO, the mode tensomite's devices run by default, takes many routes by
# shape; the explicit modes one each
MODE_WEIGHTS = [0.4, 0.1, 0.1, 0.1, 0.1, 0.1, 0.1]


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    return th.HIPDevice(0)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def cases(fmt):
    """(rows, n, k, ldx, w_row, slice_rows, mode, with_bias), seeded per format."""
    rng = np.random.default_rng({"Q8_0": 71, "Q4_0": 72, "Q4_1": 73}[fmt])
    out = []
    for i in range(CASES):
        rows = int(rng.choice([1, 1, 2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 24, 31, 32, 33, 40]))
        blocks = int(rng.choice([1, 2, 3, 5, 8, 9, 16, 18, 24, 31, 48, 64, 72, 96, 128, 200, 256]))
        k = 32 * blocks
        # outputs: a few, many, past one tile; within ~4M weight values
        n = int(rng.integers(1, max(2, min(3000, (4 << 20) // k))))
        ldx = k + int(rng.choice([0, 0, 4, 32, 100]))
        slice_rows = int(rng.integers(0, 8))  # weight rows before the product's first
        mode = str(rng.choice(MODES, p=MODE_WEIGHTS))
        out.append((rows, n, k, ldx, slice_rows, mode, bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("fmt", FORMATS)
def test_random_shapes_bit_exact(dev, fmt):
    rng = np.random.default_rng(700)
    variant = oracle.best_variant()
    for i, (rows, n, k, ldx, w_row, mode, with_bias) in enumerate(cases(fmt)):
        say("sweep", fmt, i, "rows", rows, "n", n, "k", k, "ldx", ldx, "w_row", w_row, mode, "bias", with_bias)
        total = w_row + n
        wq = oracle.quantize(fmt, (rng.standard_normal(total * k, dtype=np.float32) * np.float32(0.02)))
        xs = rng.standard_normal(rows * ldx, dtype=np.float32)
        x = np.ascontiguousarray(xs.reshape(rows, ldx)[:, :k]).reshape(-1)
        bias = rng.uniform(-1, 1, n).astype(np.float32) if with_bias else None
        row_bytes = oracle.row_bytes(fmt, k)
        want = oracle.matmul(fmt, x, wq[w_row * row_bytes:], rows, n, k, variant)
        if bias is not None:
            want = oracle.add_bias(want, bias)
        wbuf = dev.from_array(wq)
        xbuf = dev.from_array(xs)
        bbuf = dev.from_array(bias) if bias is not None else None
        out = dev.block_matmul(fmt, wbuf, xbuf, rows, n, k, bias=bbuf, w_row=w_row, ldx=ldx, mode=mode)
        got = dev.to_array(out, np.float32, rows * n).reshape(rows, n)
        dev.sync()
        for buf in (wbuf, xbuf, bbuf, out):
            if buf is not None:
                buf.release()
        assert np.array_equal(bits(got), bits(want)), (fmt, i, rows, n, k, ldx, w_row, mode, with_bias)


def large_cases(fmt):
    """(rows, n, k) through AUTO: weights past the 4 MB one-row threshold and
    up to ~32 MB, rows from one to the matrix cores' range."""
    rng = np.random.default_rng({"Q8_0": 81, "Q4_0": 82, "Q4_1": 83}[fmt])
    out = []
    for _ in range(12):
        rows = int(rng.choice([1, 1, 2, 3, 8, 12, 16, 32, 48, 64]))
        k = 32 * int(rng.choice([64, 72, 128, 144, 256]))
        n = int(rng.integers(2048, max(2049, min(16384, (32 << 20) // k))))
        n = min(n, (256 << 20) // (rows * k))  # ~256 M weight values read by the CPU per case
        out.append((rows, n, k))
    return out


@pytest.mark.parametrize("fmt", FORMATS)
def test_random_large_shapes_bit_exact(dev, fmt):
    rng = np.random.default_rng(800)
    variant = oracle.best_variant()
    for i, (rows, n, k) in enumerate(large_cases(fmt)):
        say("large sweep", fmt, i, "rows", rows, "n", n, "k", k)
        wq = oracle.quantize(fmt, (rng.standard_normal(n * k, dtype=np.float32) * np.float32(0.02)))
        x = rng.standard_normal(rows * k, dtype=np.float32)
        want = oracle.matmul(fmt, x, wq, rows, n, k, variant)
        wbuf = dev.from_array(wq)
        xbuf = dev.from_array(x)
        out = dev.block_matmul(fmt, wbuf, xbuf, rows, n, k)
        got = dev.to_array(out, np.float32, rows * n).reshape(rows, n)
        dev.sync()
        for buf in (wbuf, xbuf, out):
            buf.release()
        assert np.array_equal(bits(got), bits(want)), (fmt, i, rows, n, k)
