"""tmh_block_matmul_fixed, the allocation-free form of tmh_block_matmul,
through the C ABI: its output equals tmh_block_matmul's bit for bit on two
calls in a row, the second smaller (the fixed array keeps the first call's
contents), for the matrix-core, lanes and one-row kernels and every format;
sizes past the fixed array are refused; and no call allocates (with every
library allocation made to fail, the calls still succeed)."""
import sys

import numpy as np
import pytest

import tensomite_hip as th
from oracle import oracle

pytestmark = pytest.mark.gpu


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    return th.HIPDevice(0)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def fixed(dev, kind, w, x, dst, bias, rows, n, k, ldx=None, mode="auto"):
    return dev.lib.tmh_block_matmul_fixed(th.kind_of(kind), w.pointer, 0, x.pointer, k if ldx is None else ldx,
                                          dst.pointer, bias.pointer if bias is not None else 0, rows, n, k,
                                          th.MODES[mode])


# (rows, n, k): the matrix cores (config 4's 512 x 2048 -> 2048), then 12
# rows (the quantise pass and the 9-16-row kernel): both through the static
# scratch, the second with a smaller input; then products that need no
# scratch: 8 rows (the few-rows kernel), one row over 4 MB (the one-row
# kernel with weights in LDS), one row the tiled one-row kernel takes
CALLS = [(512, 2048, 2048), (12, 1000, 4096), (8, 1000, 1024), (1, 4096, 2048), (1, 960, 576)]


@pytest.mark.parametrize("fmt", ["Q8_0", "Q4_0", "Q4_1"])
def test_fixed_equals_block_matmul_on_calls_in_a_row(dev, fmt):
    rng = np.random.default_rng(77)
    buffers = []
    for rows, n, k in CALLS:
        wq = oracle.quantize(fmt, rng.standard_normal(n * k, dtype=np.float32) * np.float32(0.02))
        x = rng.standard_normal(rows * k, dtype=np.float32)
        bias = rng.standard_normal(n, dtype=np.float32)
        w_buf, x_buf, b_buf = dev.from_array(wq), dev.from_array(x), dev.from_array(bias)
        want_buf = dev.alloc(4 * rows * n)
        got_buf = dev.alloc(4 * rows * n)
        buffers += [w_buf, x_buf, b_buf, want_buf, got_buf]
        dev.block_matmul(fmt, w_buf, x_buf, rows, n, k, dst=want_buf, bias=b_buf)
        say("fixed", fmt, rows, n, k)
        # every library allocation would fail meanwhile: the call makes none
        dev.lib.tmh_debug_fail_allocations(1 << 20)
        try:
            code = fixed(dev, fmt, w_buf, x_buf, got_buf, b_buf, rows, n, k)
        finally:
            dev.lib.tmh_debug_fail_allocations(0)
        th.check("tmh_block_matmul_fixed", code)
        dev.sync()
        want = dev.to_array(want_buf, np.float32, rows * n)
        got = dev.to_array(got_buf, np.float32, rows * n)
        assert np.array_equal(bits(got), bits(want)), (rows, n, k)
    for b in buffers:
        b.release()
    dev.sync()


def test_fixed_refuses_more_than_its_array(dev):
    # 512 rows of k = 16384: 8 MiB of int8 values plus the scales
    rows, n, k = 512, 64, 16384
    w = dev.alloc(n * k // 32 * 34)
    x = dev.alloc(4 * rows * k)
    y = dev.alloc(4 * rows * n)
    code = fixed(dev, "Q8_0", w, x, y, None, rows, n, k)
    assert code == th.ERROR_SCRATCH_LIMIT
    assert "fixed scratch" in th.error_text(code)
    # a shape error is still a shape error
    assert fixed(dev, "Q8_0", w, x, y, None, 4, n, 48) == th.ERROR_SHAPE
    for b in (w, x, y):
        b.release()
    dev.sync()
