"""HIP path against the oracle, bit for bit (tests/ only; runs on an MI355X).

Follows the reference's own checks for the path: spec/quant_spec.cr and
spec/block_matmul_spec.cr (device equals CPU bit for bit with a bias; every
mode; groups straddling rows; views; row slices; row alone == in batch;
gather), at the BASELINE configs' full shapes where the oracle's fast path
finishes in seconds, and through size-independent properties otherwise.
"""
import sys
import zlib

import numpy as np
import pytest

from oracle import oracle
import tensomite_hip as th

pytestmark = pytest.mark.gpu

FORMATS = ["Q8_0", "Q4_0", "Q4_1"]


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    return th.HIPDevice(0)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def weights(fmt, n, k, seed, scale=0.02):
    values = np.random.default_rng(seed).standard_normal(n * k, dtype=np.float32) * np.float32(scale)
    return oracle.quantize(fmt, values)


def acts(rows, k, seed, scale=1.0):
    return np.random.default_rng(seed).normal(0.0, scale, rows * k).astype(np.float32)


def run_product(dev, fmt, wq, x, rows, n, k, mode="auto", bias=None, w_row=0, ldx=None):
    wbuf = dev.from_array(wq)
    xbuf = dev.from_array(x)
    bbuf = dev.from_array(bias) if bias is not None else None
    out = dev.block_matmul(fmt, wbuf, xbuf, rows, n, k, bias=bbuf, w_row=w_row, ldx=ldx, mode=mode)
    got = dev.to_array(out, np.float32, rows * n).reshape(rows, n)
    dev.sync()
    return got


def test_device_is_gfx950(dev):
    say("device", dev.name, dev.arch, dev.compute_units)
    assert dev.arch.startswith("gfx950")


@pytest.mark.parametrize("k", [32, 64, 96, 576, 768, 1280, 2048, 8192])
def test_quantised_activations_bit_exact(dev, k):
    # quantize_rows_q8 == quantize_activations (quant.cr:424-442), bytes and
    # scales, for rows with zero blocks, the spike and the half-integer row.
    say("quantise k", k)
    rows = 5
    x = acts(rows, k, 100 + k)
    x[k:k + 32] = 0
    x[2 * k:2 * k + 32] = [127.0 if j == 0 else j - 15.5 for j in range(32)]
    x[3 * k + 3] = 50.0
    x[4 * k:5 * k] *= 1e-3
    xbuf = dev.from_array(x)
    scales, sums, totals, qs = dev.quantize_rows(xbuf, rows, k)
    nb = k // 32
    g_scales = dev.to_array(scales, np.float32, rows * nb)
    g_sums = dev.to_array(sums, np.float32, rows * nb)
    g_totals = dev.to_array(totals, np.int32, rows * nb)
    g_qs = dev.to_array(qs, np.int8, rows * k)
    for r in range(rows):
        s, m, q = oracle.quantize_activations(x[r * k:(r + 1) * k], with_sums=True)
        assert np.array_equal(g_qs[r * k:(r + 1) * k], q), r
        assert np.array_equal(bits(g_scales[r * nb:(r + 1) * nb]), bits(s)), r
        assert np.array_equal(bits(g_sums[r * nb:(r + 1) * nb]), bits(m)), r
        assert np.array_equal(g_totals[r * nb:(r + 1) * nb], q.reshape(nb, 32).astype(np.int32).sum(1)), r


@pytest.mark.parametrize("rows,k,ldx", [(600, 2048, 2048), (333, 3200, 3200), (400, 2080, 2081)])
def test_quantised_activations_large(dev, rows, k, ldx):
    # Prefill-sized inputs (tens of thousands of blocks, about a thousand
    # workgroups): the same bytes and scales as the oracle, with a ragged
    # last workgroup (333 x 100 blocks) and unaligned rows (ldx 2081).
    say("quantise large", rows, k, ldx)
    x = np.zeros(rows * ldx, np.float32)
    body = acts(rows, k, 7 + k).reshape(rows, k)
    body[1, :32] = 0
    body[2, 64:96] = [127.0 if j == 0 else j - 15.5 for j in range(32)]
    x.reshape(rows, ldx)[:, :k] = body
    xbuf = dev.from_array(x)
    scales, sums, totals, qs = dev.quantize_rows(xbuf, rows, k, ldx)
    nb = k // 32
    g_scales = dev.to_array(scales, np.float32, rows * nb).reshape(rows, nb)
    g_sums = dev.to_array(sums, np.float32, rows * nb).reshape(rows, nb)
    g_totals = dev.to_array(totals, np.int32, rows * nb).reshape(rows, nb)
    g_qs = dev.to_array(qs, np.int8, rows * k).reshape(rows, k)
    for r in range(rows):
        s, m, q = oracle.quantize_activations(body[r], with_sums=True)
        assert np.array_equal(g_qs[r], q), r
        assert np.array_equal(bits(g_scales[r]), bits(s)), r
        assert np.array_equal(bits(g_sums[r]), bits(m)), r
        assert np.array_equal(g_totals[r], q.reshape(nb, 32).astype(np.int32).sum(1)), r


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("mode", ["auto", "thread", "lanes", "unordered"])
def test_matches_cpu_with_bias_every_mode(dev, fmt, mode):
    # block_matmul_spec.cr:102-116 (rows 5, n 7, k 96: odd block count) and
    # 142-158 (3 x 37 over 1280-long rows: more blocks than lanes).
    rng = np.random.default_rng(1)
    for rows, n, k in ((5, 7, 96), (3, 37, 1280), (1, 37, 1280)):
        say("product", fmt, mode, rows, n, k)
        x = rng.uniform(-1, 1, rows * k).astype(np.float32)
        w = rng.uniform(-1, 1, n * k).astype(np.float32)
        bias = rng.uniform(-1, 1, n).astype(np.float32)
        wq = oracle.quantize(fmt, w)
        want = oracle.add_bias(oracle.matmul_reference(fmt, x, wq, rows, n, k), bias)
        got = run_product(dev, fmt, wq, x, rows, n, k, mode=mode, bias=bias)
        if mode == "unordered":  # the reference's spec checks closeness only (block_matmul_spec.cr:152-158)
            assert np.allclose(got, want, rtol=1e-4, atol=1e-5 * max(1.0, float(np.abs(want).max())))
        else:
            assert np.array_equal(bits(got), bits(want))


def close_not_same(got, want):
    """UNORDERED's results: within a few roundings of the host's sums, and
    (over many outputs) not all of the host's bits -- the fold order did change."""
    scale = max(1.0, float(np.abs(want).max()))
    return np.allclose(got, want, rtol=1e-4, atol=1e-5 * scale) and not np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("rows,n,k", [(1, 3000, 2048), (1, 8192, 2048), (2, 8192, 2048), (3, 2048, 8192),
                                      (4, 3000, 2048), (8, 2048, 8192), (12, 2048, 4096), (16, 3000, 2048)])
def test_unordered_below_matrix_rows(dev, fmt, rows, n, k):
    # Below 32 rows UNORDERED runs AUTO's kernels (the one-row kernels, the
    # few-rows kernels with weights in LDS, the lanes and 9-16-row kernels)
    # with each row's contributions summed in an order of their own: close to
    # the host's sums, not its bits (block_matmul_unordered_f32,
    # cuda/kernels.cu:1334-1375); AUTO on the same inputs stays exact.
    say("unordered", fmt, rows, n, k)
    wq = weights(fmt, n, k, 700 + rows)
    x = acts(rows, k, 701)
    want = oracle.matmul(fmt, x, wq, rows, n, k)
    got = run_product(dev, fmt, wq, x, rows, n, k, mode="unordered")
    assert close_not_same(got, want)
    assert np.array_equal(bits(run_product(dev, fmt, wq, x, rows, n, k)), bits(want))


@pytest.mark.parametrize("fmt", FORMATS)
def test_activation_row_groups(dev, fmt):
    # Every activation row count 1..17 (groups of 16, 8, 4, 2, 1), and each
    # row alone equals the row in the batch (block_matmul_spec.cr:118-123).
    n, k = 300, 576
    wq = weights(fmt, n, k, 7)
    x = acts(17, k, 8)
    want = oracle.matmul(fmt, x, wq, 17, n, k)
    for rows in list(range(1, 18)):
        say("rows", fmt, rows)
        got = run_product(dev, fmt, wq, x[:rows * k], rows, n, k)
        assert np.array_equal(bits(got), bits(want[:rows])), rows


@pytest.mark.parametrize("fmt", FORMATS)
def test_views_and_row_slices(dev, fmt):
    # block_matmul_spec.cr:197-205: activation rows read through a view
    # (rows ldx apart) and a weight sliced by rows (a merged projection).
    n, k, rows = 50, 1024, 3
    wq = weights(fmt, n, k, 9)
    x = acts(rows, k, 10)
    full = oracle.matmul_reference(fmt, x, wq, rows, n, k)
    say("slice", fmt)
    got = run_product(dev, fmt, wq, x, rows, 20, k, w_row=17)
    assert np.array_equal(bits(got), bits(full[:, 17:37]))
    ldx = k + 96
    strided = np.zeros(rows * ldx, np.float32)
    for r in range(rows):
        strided[r * ldx:r * ldx + k] = x[r * k:(r + 1) * k]
    say("view", fmt)
    wbuf, xbuf = dev.from_array(wq), dev.from_array(strided)
    out = dev.block_matmul(fmt, wbuf, xbuf, rows, n, k, ldx=ldx)
    got = dev.to_array(out, np.float32, rows * n).reshape(rows, n)
    assert np.array_equal(bits(got), bits(full))


CONFIG_SHAPES = {
    # config 1: GPT-2 c_attn, Q8_0
    "c_attn": ("Q8_0", 2304, 768, 1),
    # config 2: SmolLM2-135M Q4_0 set
    "qkv_135m": ("Q4_0", 960, 576, 1),
    "o_135m": ("Q4_0", 576, 576, 1),
    "gate_up_135m": ("Q4_0", 3072, 576, 1),
    "down_135m": ("Q4_0", 576, 1536, 1),
    "head_135m": ("Q4_0", 49152, 576, 1),
    # config 3: Q4_1 batched decode, every B the bench times on both shapes
    # (B = 5 besides: a group of 4 and one row)
    "q41_up_b1": ("Q4_1", 8192, 2048, 1),
    "q41_up_b2": ("Q4_1", 8192, 2048, 2),
    "q41_up_b4": ("Q4_1", 8192, 2048, 4),
    "q41_up_b8": ("Q4_1", 8192, 2048, 8),
    "q41_up_b16": ("Q4_1", 8192, 2048, 16),
    "q41_down_b1": ("Q4_1", 2048, 8192, 1),
    "q41_down_b2": ("Q4_1", 2048, 8192, 2),
    "q41_down_b4": ("Q4_1", 2048, 8192, 4),
    "q41_down_b5": ("Q4_1", 2048, 8192, 5),
    "q41_down_b8": ("Q4_1", 2048, 8192, 8),
    "q41_down_b16": ("Q4_1", 2048, 8192, 16),
    # config 5: 1.7B Q4_0 products at batch 1 and 8
    "qkv_1p7b": ("Q4_0", 6144, 2048, 1),
    "gate_up_1p7b_b8": ("Q4_0", 16384, 2048, 8),
    "down_1p7b": ("Q4_0", 2048, 8192, 1),
    "head_1p7b": ("Q4_0", 49152, 2048, 1),
}


@pytest.mark.parametrize("name", sorted(CONFIG_SHAPES))
def test_config_shapes_bit_exact(dev, name):
    fmt, n, k, rows = CONFIG_SHAPES[name]
    say("config", name, fmt, n, k, rows)
    wq = weights(fmt, n, k, zlib.crc32(name.encode()))
    x = acts(rows, k, 3)
    want = oracle.matmul(fmt, x, wq, rows, n, k)
    got = run_product(dev, fmt, wq, x, rows, n, k)
    assert np.array_equal(bits(got), bits(want))
    # run to run: the same bits again
    again = run_product(dev, fmt, wq, x, rows, n, k)
    assert np.array_equal(bits(again), bits(got))


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("n,k", [(4096, 2048), (1024, 8192), (2500, 4096)])
def test_one_row_over_4mb_with_bias(dev, fmt, n, k):
    # One-row products of more than 4 MB of weights, with a bias added after
    # each sum (host.cr:725-734), in every format, by both routes: AUTO's
    # one-row f32 kernel (weights staged into LDS, x quantised in every
    # workgroup's prologue), and the quantise pass followed by the lanes
    # product (the route of the reference's launch_blocks, cuda.cr:736-756).
    say("one row > 4 MB", fmt, n, k)
    wq = weights(fmt, n, k, n + k)
    assert wq.nbytes > 4 << 20
    x = acts(1, k, 5)
    bias = acts(1, n, 6)
    want = oracle.add_bias(oracle.matmul(fmt, x, wq, 1, n, k), bias)
    got = run_product(dev, fmt, wq, x, 1, n, k, bias=bias)
    assert np.array_equal(bits(got), bits(want))
    wbuf, xbuf, bbuf = dev.from_array(wq), dev.from_array(x), dev.from_array(bias)
    act = dev.quantize_rows(xbuf, 1, k)
    out = dev.block_matmul_quantised(fmt, wbuf, act, 1, n, k, bias=bbuf, mode="lanes")
    lanes = dev.to_array(out, np.float32, n).reshape(1, n)
    assert np.array_equal(bits(lanes), bits(want))


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("n,k", [(16384, 512), (1000, 4096), (1200, 8192), (2049, 8192), (8192, 2048)])
@pytest.mark.parametrize("rows", [1, 2])
def test_one_long_row_quantised_in_kernel(dev, fmt, n, k, rows):
    # One row over 4 MB of weights (and two rows, rows ldx apart): the
    # one-row kernel quantises x in its prologue (no norm). Whole blocks of
    # zeros (scale 0), a spike, exact halves (rounding ties), a ragged last
    # tile; the second row Gaussian. k = 512 stages x in one piece (its
    # halves would start a rotation group out of step); k = 2048..8192 in
    # two halves.
    wq = weights(fmt, n, k, n * 7 + k)
    if wq.nbytes <= 4 << 20:
        wq = np.concatenate([wq] * 2)
        n *= 2
    say("long rows", fmt, rows, n, k)
    x = acts(rows, k, k + 9)
    x[:256] = 0.0
    t = min(1024, x.size // 2)
    m = min(512, x.size - t)
    x[t:t + m] = (np.arange(m) % 255 - 127).astype(np.float32) * np.float32(0.5)
    x[300] = 1e4
    ldx = k + 32
    strided = np.zeros(rows * ldx, np.float32)
    for r in range(rows):
        strided[r * ldx:r * ldx + k] = x[r * k:(r + 1) * k]
    bias = acts(1, n, 8)
    want = oracle.add_bias(oracle.matmul(fmt, x, wq, rows, n, k), bias)
    got = run_product(dev, fmt, wq, strided, rows, n, k, bias=bias, ldx=ldx)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("k", [64, 512, 2048])
def test_few_rows_weights_in_lds(dev, fmt, k):
    # 1-8 rows (groups of 8, 4 and 2; one row above 4 MB) through the kernel
    # that quantises the rows in each workgroup's prologue: rows ldx apart,
    # a ragged last tile, a bias, and rows of zeros (scale 0), a spike and
    # exact halves (rounding ties) beside Gaussian ones.
    n = 1000 if k < 2048 else 4100
    wq = weights(fmt, n, k, k + 1)
    x = acts(8, k, k + 2)
    x[k:2 * k] = 0.0
    x[2 * k + 5] = 1e4
    x[3 * k:4 * k] = (np.arange(k) % 255 - 127).astype(np.float32) * np.float32(0.5)
    ldx = k + 32
    strided = np.zeros(8 * ldx, np.float32)
    for r in range(8):
        strided[r * ldx:r * ldx + k] = x[r * k:(r + 1) * k]
    bias = acts(1, n, 4)
    want = oracle.add_bias(oracle.matmul(fmt, x, wq, 8, n, k), bias)
    wbuf, xbuf, bbuf = dev.from_array(wq), dev.from_array(strided), dev.from_array(bias)
    for rows in range(1, 9):
        say("few rows", fmt, k, rows)
        out = dev.block_matmul(fmt, wbuf, xbuf, rows, n, k, bias=bbuf, ldx=ldx)
        got = dev.to_array(out, np.float32, rows * n).reshape(rows, n)
        assert np.array_equal(bits(got), bits(want[:rows])), rows


def same_or_both_nan(got, want):
    g, w = np.asarray(got, np.float32), np.asarray(want, np.float32)
    nan = np.isnan(w)
    return np.array_equal(np.isnan(g), nan) and np.array_equal(bits(g[~nan]), bits(w[~nan]))


@pytest.mark.parametrize("fmt", FORMATS)
def test_few_rows_nan_and_inf_blocks(dev, fmt):
    # The host's amax is taken in index order and skips a NaN unless it is the
    # block's first value (quant.cr:428-442); the few-rows kernel's lane-a-
    # block quantiser takes it as a tree. Blocks with a NaN first, a NaN in
    # the middle, and an inf, in every row count of the one-launch form.
    # A NaN first in a lane's 4 values (block index 4j, j >= 1) is inside
    # its block too: the 8-lane quantisers skip it like any other.
    n, k = 700, 512
    wq = weights(fmt, n, k, 41)
    x = acts(10, k, 42)
    for r in range(10):
        x[r * k + 32 * 9 + 5 + r] = np.nan  # inside a block: skipped by amax, quantised to 0
        x[r * k + 32 * 3 + 31 - r] = np.nan
        x[r * k + 32 * 5 + 4 * (1 + r % 7)] = np.nan  # first of lane 1 + r % 7's values
    x[4 * k + 32 * 6] = np.nan  # first in its block: the block's scale is NaN
    x[5 * k + 32 * 2] = np.nan
    x[6 * k + 32 * 12 + 6] = np.inf
    x[7 * k + 32 * 1] = -np.inf
    want = oracle.matmul(fmt, x, wq, 10, n, k)
    wbuf, xbuf = dev.from_array(wq), dev.from_array(x)
    for rows in range(1, 11):  # 9 and 10: the quantise pass and the 9-16-row kernel
        say("nan rows", fmt, rows)
        out = dev.block_matmul(fmt, wbuf, xbuf, rows, n, k)
        got = dev.to_array(out, np.float32, rows * n).reshape(rows, n)
        assert same_or_both_nan(got, want[:rows]), rows


def test_empty_calls_succeed_and_write_nothing(dev):
    # Empty work through the C ABI, as tensomite's empty tensors reach it:
    # products of no rows or no outputs (every mode, and the allocation-free
    # entry point), a quantise pass of no rows, a gather of no ids and a plan
    # of no products all return success, launch nothing, and leave the
    # output as it was; with nothing to do, null buffers are accepted too.
    wq = weights("Q4_0", 8, 64, 1)
    wbuf, xbuf = dev.from_array(wq), dev.from_array(acts(1, 64, 2))
    sentinel = np.full(16, 7.0, np.float32)
    out = dev.from_array(sentinel)
    say("empty calls")
    for entry in ("tmh_block_matmul", "tmh_block_matmul_fixed"):
        fn = getattr(dev.lib, entry)
        for rows, n in ((0, 8), (1, 0), (0, 0)):
            for mode in range(8):
                th.check(entry, fn(th.Q4_0, wbuf.pointer, 0, xbuf.pointer, 64, out.pointer, 0, rows, n, 64, mode))
        th.check(entry, fn(th.Q4_0, 0, 0, 0, 64, 0, 0, 0, 8, 64, 0))
    th.check("tmh_quantize_rows_q8", dev.lib.tmh_quantize_rows_q8(xbuf.pointer, 0, 64, 64, 0, 0, 0, 0))
    th.check("tmh_gather_blocks", dev.lib.tmh_gather_blocks(th.Q4_0, wbuf.pointer, 0, 8, 64, 0, 0, out.pointer))
    plan = dev.plan("Q4_0", [])
    plan.run()
    plan.destroy()
    dev.sync()
    assert np.array_equal(dev.to_array(out, np.float32, 16), sentinel)


@pytest.mark.parametrize("rows", [1, 2, 5, 8, 16, 40])
def test_zero_rows_fold_from_plus_zero(dev, rows):
    # Q4_0 with negative block scales and all-zero activation rows: every
    # contribution (0·d)·0 is -0.0, and the host's fold from 0.0f gives +0.0
    # (quant.cr:446-491); every route (one row, few rows, lanes, the
    # matrix-core kernel from 32 rows) must keep the +0.0 start.
    n, k = 3000, 512
    w = np.tile(np.array([1.0] + [0.25] * 31, np.float32), n * k // 32)
    wq = oracle.quantize("Q4_0", w)
    x = np.zeros(rows * k, np.float32)
    say("zero rows", rows)
    for mode in ("auto", "lanes", "thread", "matrix"):
        got = run_product(dev, "Q4_0", wq, x, rows, n, k, mode=mode)
        assert np.all(bits(got) == 0), mode


@pytest.mark.parametrize("fmt", FORMATS)
def test_special_rows(dev, fmt):
    # quant_spec.cr:30-48 on the device: zero first block, a spike of 50, a
    # zero activation block, the [127, j - 15.5] row, at {3, 5, 1280} and
    # {2, 9, 4096}.
    rng = np.random.default_rng(11)
    for count, n, k in ((1, 37, 64), (3, 5, 1280), (2, 9, 4096)):
        say("special", fmt, count, n, k)
        values = rng.uniform(-2.0, 2.0, n * k).astype(np.float32)
        values[:32] = 0
        values[32 * 3] = 50
        x = rng.uniform(-3.0, 3.0, count * k).astype(np.float32)
        if count > 1:
            x[k:k + 32] = 0
        if count > 2:
            x[2 * k:2 * k + 32] = [127.0 if j == 0 else j - 15.5 for j in range(32)]
        wq = oracle.quantize(fmt, values)
        want = oracle.matmul_reference(fmt, x, wq, count, n, k)
        for mode in ("auto", "thread"):
            got = run_product(dev, fmt, wq, x, count, n, k, mode=mode)
            assert np.array_equal(bits(got), bits(want)), mode


@pytest.mark.parametrize("fmt", FORMATS)
def test_gather(dev, fmt):
    # block_matmul_spec.cr:221-236: rows [4, 0, 4] of a 6 x 64 table, and a
    # row slice of it; the embedding shape of config 5.
    rng = np.random.default_rng(4)
    table = rng.uniform(-1, 1, 6 * 64).astype(np.float32)
    q = oracle.quantize(fmt, table)
    tbuf = dev.from_array(q)
    ids = dev.from_array(np.array([4, 0, 4], np.int32))
    say("gather", fmt)
    out = dev.gather(fmt, tbuf, 6, 64, ids, 3)
    got = dev.to_array(out, np.float32, 3 * 64).reshape(3, 64)
    dev.sync()
    assert np.array_equal(bits(got), bits(oracle.gather(fmt, q, 6, 64, [4, 0, 4])))
    ids2 = dev.from_array(np.array([2], np.int32))
    out = dev.gather(fmt, tbuf, 4, 64, ids2, 1, first_row=2)
    got = dev.to_array(out, np.float32, 64)
    dev.sync()
    assert np.array_equal(bits(got), bits(oracle.gather(fmt, q, 6, 64, [4])[0]))
    emb = weights(fmt, 49152, 2048, 21)
    ebuf = dev.from_array(emb)
    want_ids = np.array([0, 49151, 12345, 7, 7, 30000, 1, 2], np.int32)
    out = dev.gather(fmt, ebuf, 49152, 2048, dev.from_array(want_ids), 8)
    got = dev.to_array(out, np.float32, 8 * 2048).reshape(8, 2048)
    dev.sync()
    assert np.array_equal(bits(got), bits(oracle.gather(fmt, emb, 49152, 2048, want_ids)))


def test_gather_out_of_range_raises_at_sync(dev):
    # host.cr:652-654 raises ExecutionError; cuda.cr:972-983 at sync.
    q = oracle.quantize("Q4_0", np.ones(4 * 64, np.float32))
    tbuf = dev.from_array(q)
    for bad in (4, -1):
        say("gather bad id", bad)
        ids = dev.from_array(np.array([1, bad, 0], np.int32))
        out = dev.gather("Q4_0", tbuf, 4, 64, ids, 3)
        with pytest.raises(th.ExecutionError, match=f"index {bad} out of range for 4 rows"):
            dev.sync()
        got = dev.to_array(out, np.float32, 3 * 64)
        assert np.all(got[64:128] == 0)
    dev.sync()  # the report was cleared


def test_every_half_widens_exactly(dev):
    # F16#to_f32 (f16.cr:44-57) on the device, for all 65,536 halves: a Q8_0
    # table whose block b has d = half b and values (1, 0, ..., 0) gathers to
    # d itself.
    blocks = np.zeros((65536, 34), np.uint8)
    h = np.arange(65536, dtype=np.uint32)
    blocks[:, 0] = h & 0xFF
    blocks[:, 1] = h >> 8
    blocks[:, 2] = 1
    table = blocks.reshape(-1)
    rows, width = 65536 // 32, 32 * 32
    tbuf = dev.from_array(table)
    ids = dev.from_array(np.arange(rows, dtype=np.int32))
    say("halves")
    out = dev.gather("Q8_0", tbuf, rows, width, ids, rows)
    got = dev.to_array(out, np.float32, rows * width).reshape(65536, 32)[:, 0]
    dev.sync()
    want = oracle.f16_values_many(h.astype(np.uint16))
    finite = ~np.isnan(want)
    assert np.array_equal(bits(got[finite]), bits(want[finite]))
    assert np.all(np.isnan(got[~finite]))


def test_every_f32_rounds_to_half_exactly(dev):
    # F16.new (f16.cr:29-41) on the device, for all 2^32 f32 words: the
    # rounding the activation quantiser's scales and sums go through
    # (round_to_half), swept by tmh_debug_f16_words in chunks of 2^28 and
    # compared with the oracle's tmo_f16_bits on the same words.
    from concurrent.futures import ThreadPoolExecutor

    chunk = 1 << 28
    out = dev.alloc(2 * chunk)
    pool = ThreadPoolExecutor(4)
    host = np.empty(chunk, np.uint16)
    for c in range(1 << 32 >> 28):
        first = c * chunk
        say("f16 words", hex(first))
        th.check("tmh_debug_f16_words", dev.lib.tmh_debug_f16_words(first, chunk, out.pointer))
        dev.download(out, host)
        words = np.arange(chunk, dtype=np.uint32) + np.uint32(first)
        parts = np.array_split(words.view(np.float32), 4)
        want = np.concatenate(list(pool.map(oracle.f16_bits_many, parts)))
        bad = np.nonzero(host != want)[0]
        assert bad.size == 0, (hex(first + int(bad[0])), hex(int(host[bad[0]])), hex(int(want[bad[0]])))
    pool.shutdown()
    out.release()


def test_buffer_pool_reuse_and_counters(dev):
    # CUDA#alloc from the pool after retire + sync (cuda.cr:339-353, 439-454).
    say("pool")
    before = dev.counters()
    b = dev.alloc(123457)
    b.release()
    dev.sync()
    c = dev.alloc(123457)
    after = dev.counters()
    assert after["pool_hits"] >= before["pool_hits"] + 1
    c.release()
    assert after["pool_limit"] >= 1 << 30


def test_async_upload_round_trip(dev):
    # tmh_upload_async: the caller's memory may change right after the call.
    rng = np.random.default_rng(5)
    data = rng.integers(0, 256, (40 << 20) + 13, dtype=np.uint8)
    buf = dev.alloc(data.nbytes)
    say("async upload")
    scratch = data.copy()
    dev.upload(buf, scratch, asynchronous=True)
    scratch[:] = 0  # reused at once
    got = dev.to_array(buf, np.uint8, data.nbytes)
    assert np.array_equal(got, data)


def test_errors_are_typed(dev):
    say("errors")
    w = dev.from_array(np.zeros(34 * 4, np.uint8))
    x = dev.from_array(np.zeros(64, np.float32))
    with pytest.raises(th.ShapeError):
        th.check("tmh_block_matmul", dev.lib.tmh_block_matmul(0, w.pointer, 0, x.pointer, 48, x.pointer, 0, 1, 2,
                                                               48, 0))
    with pytest.raises(th.DTypeError):
        th.check("tmh_block_matmul", dev.lib.tmh_block_matmul(5, w.pointer, 0, x.pointer, 64, x.pointer, 0, 1, 2,
                                                               64, 0))
    dev.lib.tmh_debug_fail_allocations(1)
    try:
        with pytest.raises(th.DeviceError, match="OUT_OF_MEMORY"):
            dev.alloc(77777777)
    finally:
        dev.lib.tmh_debug_fail_allocations(0)
    dev.lib.tmh_debug_disable_kernels(1)
    try:
        with pytest.raises(th.NoKernels):
            dev.block_matmul("Q8_0", w, x, 1, 2, 64)
    finally:
        dev.lib.tmh_debug_disable_kernels(0)
    dev.sync()


@pytest.mark.parametrize("kernel", ["stream", "rows"])
@pytest.mark.parametrize("fmt", FORMATS)
def test_plan_equals_products_one_by_one(dev, fmt, kernel, monkeypatch):
    # tmh_plan_*: many one-row products in one launch give each product's
    # bits, in the streamed kernel (the default; x of k = 8192 too long to
    # stage) and in the tiled one (TMH_PLAN_KERNEL=rows).
    monkeypatch.setenv("TMH_PLAN_KERNEL", kernel)
    shapes = [(960, 576), (576, 576), (3072, 576), (576, 1536), (300, 2048), (7, 64), (2304, 768), (100, 8192),
              (1, 4096), (130, 128)]
    ws, xs, wants = [], [], []
    for i, (n, k) in enumerate(shapes):
        wq = weights(fmt, n, k, 500 + i)
        x = acts(1, k, 600 + i)
        ws.append(dev.from_array(wq))
        xs.append(dev.from_array(x))
        wants.append(oracle.matmul(fmt, x, wq, 1, n, k)[0])
    ys = [dev.alloc(4 * n) for n, _ in shapes]
    bias = dev.from_array(np.arange(3072, dtype=np.float32) * 0.25)
    items = [(ws[i], 0, xs[i], ys[i], bias if i == 2 else None, n, k) for i, (n, k) in enumerate(shapes)]
    say("plan", fmt)
    plan = dev.plan(fmt, items)
    for _ in range(3):
        plan.run()
    dev.sync()
    for i, (n, k) in enumerate(shapes):
        got = dev.to_array(ys[i], np.float32, n)
        want = wants[i] + (np.arange(3072, dtype=np.float32)[:n] * 0.25 if i == 2 else 0)
        assert np.array_equal(bits(got), bits(want.astype(np.float32))), shapes[i]
    plan.destroy()


class View:
    """A slice of a device buffer, as the plan API takes it (pointer, bytes)."""

    def __init__(self, buffer, byte_offset, bytesize):
        self.buffer = buffer  # keeps the allocation alive
        self.pointer = buffer.pointer + byte_offset
        self.bytesize = bytesize


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("wgs,ring", [("1", "2"), ("1", "5"), ("6", "2")])
def test_stream_plan_many_small_products(dev, fmt, wgs, ring, monkeypatch):
    # The streamed kernel where one workgroup's steps span many products (a
    # third and later product quantised in turn), rows shorter than a step,
    # biases on some products, x only 4-byte aligned for some, ragged last
    # steps.
    monkeypatch.setenv("TMH_PLAN_KERNEL", "stream")
    monkeypatch.setenv("TMH_STREAM_WGS", wgs)
    monkeypatch.setenv("TMH_STREAM_RING", ring)
    rng = np.random.default_rng(900)
    ks = [64, 128, 576, 192, 1536, 64, 256]
    shapes = [(int(rng.integers(1, 300)), ks[i % len(ks)]) for i in range(700)]
    xs = [acts(1, k, 2000 + i) for i, (_, k) in enumerate(shapes)]
    offsets, packed = [], []
    at = 0
    for i, x in enumerate(xs):
        at += 1 if i % 3 == 0 else 4  # every third x starts one float past 16 bytes
        offsets.append(at)
        at += len(x)
    host = np.zeros(at + 4, np.float32)
    for o, x in zip(offsets, xs):
        host[o:o + len(x)] = x
    xbuf = dev.from_array(host)
    items, wants, ys = [], [], []
    for i, (n, k) in enumerate(shapes):
        wq = weights(fmt, n, k, 1000 + i)
        b = rng.uniform(-1, 1, n).astype(np.float32) if i % 4 == 1 else None
        y = dev.alloc(4 * n)
        ys.append(y)
        items.append((dev.from_array(wq), 0, View(xbuf, 4 * offsets[i], 4 * k), y,
                      dev.from_array(b) if b is not None else None, n, k))
        want = oracle.matmul(fmt, xs[i], wq, 1, n, k)[0]
        wants.append(want if b is None else oracle.add_bias(want[None, :], b)[0])
    say("stream plan", fmt, wgs, ring, len(shapes))
    plan = dev.plan(fmt, items)
    for _ in range(2):
        plan.run()
    dev.sync()
    for i, (n, k) in enumerate(shapes):
        got = dev.to_array(ys[i], np.float32, n)
        assert np.array_equal(bits(got), bits(wants[i])), (i, shapes[i])
    plan.destroy()


def plan_input(dev, mode, x, k, seed):
    """A plan product's activation row in input mode `mode` (0 f32, 1 RMSNorm, 2
    quantised beforehand) and the f32 row the product should see."""
    if mode == 0:
        return dev.from_array(x), None, x
    if mode == 1:
        w = np.random.default_rng(seed).normal(1.0, 0.3, k).astype(np.float32)
        return dev.from_array(x), th.RMSNormInput(dev.from_array(w), 1e-5), oracle.rmsnorm(x[None, :], w, 1e-5)[0]
    scales, sums, totals, qs = dev.quantize_rows(dev.from_array(x), 1, k)
    return qs, th.QuantisedInput(scales, sums, totals), x


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("wgs,ring,rows", [("1", "2", "short"), ("6", "2", "short"), ("2", "3", "short"),
                                           ("6", "2", "long")])
def test_stream_plan_input_modes(dev, fmt, wgs, ring, rows, monkeypatch):
    # Products whose x comes in each input mode in one plan: f32, f32 under
    # an RMSNorm (normalised by every workgroup that takes part of it), and
    # already quantised -- staged before the loop for a workgroup's first
    # product, prepared in the loop for the later ones ("long": an f32 row of
    # 8192 is past the staging budget, so every product is prepared from
    # global memory); the bits of the oracle's RMSNorm then product, or of
    # the product of x.
    monkeypatch.setenv("TMH_PLAN_KERNEL", "stream")
    if rows == "long" and fmt == "Q8_0":
        # A Q8_0 row of 8192 values (8704 bytes) is longer than a step of
        # the streamed kernel, and the tiled kernel takes f32 x only: a plan
        # with such a product in another input mode is refused.
        wq = weights(fmt, 16, 8192, 3000)
        x = acts(1, 8192, 4000)
        for mode in (1, 2):
            xbuf, xin, _ = plan_input(dev, mode, x, 8192, 5000)
            with pytest.raises(th.ShapeError):
                dev.plan(fmt, [(dev.from_array(wq), 0, xbuf, dev.alloc(64), None, 16, 8192, xin)])
        return
    monkeypatch.setenv("TMH_STREAM_WGS", wgs)
    monkeypatch.setenv("TMH_STREAM_RING", ring)
    rng = np.random.default_rng(950)
    ks = [64, 576, 2048, 128, 1536, 256] if rows == "short" else [64, 576, 8192, 2048]
    # k cycles independently of the mode (i % 3), so every mode meets every k
    shapes = [(int(rng.integers(1, 200)) if i % 9 else 2048, ks[(i // 3) % len(ks)]) for i in range(160)]
    items, wants, ys = [], [], []
    for i, (n, k) in enumerate(shapes):
        mode = i % 3
        wq = weights(fmt, n, k, 3000 + i)
        x = acts(1, k, 4000 + i)
        xbuf, xin, seen = plan_input(dev, mode, x, k, 5000 + i)
        b = rng.uniform(-1, 1, n).astype(np.float32) if i % 4 == 1 else None
        y = dev.alloc(4 * n)
        ys.append(y)
        items.append((dev.from_array(wq), 0, xbuf, y, dev.from_array(b) if b is not None else None, n, k, xin))
        want = oracle.matmul(fmt, seen, wq, 1, n, k)[0]
        wants.append(want if b is None else oracle.add_bias(want[None, :], b)[0])
    say("stream plan modes", fmt, wgs, ring, len(shapes))
    plan = dev.plan(fmt, items)
    for _ in range(2):
        plan.run()
    dev.sync()
    for i, (n, k) in enumerate(shapes):
        got = dev.to_array(ys[i], np.float32, n)
        assert np.array_equal(bits(got), bits(wants[i])), (i, shapes[i], i % 3)
    plan.destroy()


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("mode,n,k", [(1, 6144, 2048), (1, 16384, 2048), (2, 2048, 8192), (2, 2048, 2048),
                                      (1, 49152, 576), (2, 32, 64), (1, 100, 64), (2, 96, 128)])
def test_stream_plan_one_product_input_modes(dev, fmt, mode, n, k):
    # The decode step's single-product plans: the qkv, gate_up and head
    # products over an RMSNorm of the residual row, and the o and down
    # products over an already quantised row with the residual as bias.
    say("one-product plan", fmt, mode, n, k)
    wq = weights(fmt, n, k, 6000 + n + k)
    x = acts(1, k, 7000 + k)
    xbuf, xin, seen = plan_input(dev, mode, x, k, 8000 + k)
    b = acts(1, n, 9000 + n) if mode == 2 else None
    y = dev.alloc(4 * n)
    item = (dev.from_array(wq), 0, xbuf, y, dev.from_array(b) if b is not None else None, n, k, xin)
    if fmt == "Q8_0" and k == 8192:
        # a Q8_0 row of 8192 values is longer than a step of the streamed kernel
        with pytest.raises(th.ShapeError):
            dev.plan(fmt, [item])
        return
    plan = dev.plan(fmt, [item])
    plan.run()
    got = dev.to_array(y, np.float32, n)
    dev.sync()
    want = oracle.matmul(fmt, seen, wq, 1, n, k)[0]
    if b is not None:
        want = oracle.add_bias(want[None, :], b)[0]
    assert np.array_equal(bits(got), bits(want))
    plan.destroy()


def test_plan_input_modes_need_the_streamed_kernel(dev, monkeypatch):
    # The tiled kernel takes f32 x only: a plan with another input mode is
    # refused when it is asked for.
    monkeypatch.setenv("TMH_PLAN_KERNEL", "rows")
    wq = weights("Q4_0", 64, 256, 1)
    x = acts(1, 256, 2)
    xbuf, xin, _ = plan_input(dev, 1, x, 256, 3)
    with pytest.raises(th.ShapeError):
        dev.plan("Q4_0", [(dev.from_array(wq), 0, xbuf, dev.alloc(256), None, 64, 256, xin)])


MATRIX_SHAPES = [
    # (rows, n, k): config 4 prefill, ragged edges, short k, the 1.7B MLP
    (512, 2048, 2048), (512, 8192, 2048), (33, 100, 576), (64, 64, 64), (100, 130, 1024), (128, 8192, 2048),
    (40, 2048, 8192),
    # more tiles than compute units (several rounds of workgroups): a tile
    # count that is a multiple of 8 (ids regrouped by XCD) with ragged rows
    # and outputs and tiles of one stage (k = 256); a count that is not (516);
    # an odd count
    (250, 8300, 256), (100, 16500, 512), (520, 2100, 256),
]


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("shape", MATRIX_SHAPES)
def test_matrix_cores_bit_exact(dev, fmt, shape):
    # The MFMA path (mode matrix, and auto from 32 rows) gives the host's bits.
    rows, n, k = shape
    say("matrix", fmt, rows, n, k)
    wq = weights(fmt, n, k, 700 + rows + n)
    x = acts(rows, k, 800 + rows)
    want = oracle.matmul(fmt, x, wq, rows, n, k)
    for mode in ("matrix", "auto"):
        got = run_product(dev, fmt, wq, x, rows, n, k, mode=mode)
        assert np.array_equal(bits(got), bits(want)), mode


FEW_SHAPES = [
    # (rows, n, k): AUTO takes the few-rows matrix-core kernel for 9-16 rows
    # where k is a multiple of 512: ragged outputs, config 3's two shapes at
    # B = 16, one row short of a tile
    (9, 100, 512), (12, 37, 1024), (10, 2048, 1024), (15, 130, 512), (16, 8192, 2048), (16, 2048, 8192),
]


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("shape", FEW_SHAPES)
def test_few_rows_bit_exact(dev, fmt, shape):
    rows, n, k = shape
    say("few rows", fmt, rows, n, k)
    rng = np.random.default_rng(930 + rows)
    wq = weights(fmt, n, k, 931 + n)
    x = acts(rows, k, 932 + rows)
    bias = rng.uniform(-1, 1, n).astype(np.float32)
    want = oracle.add_bias(oracle.matmul(fmt, x, wq, rows, n, k), bias)
    got = run_product(dev, fmt, wq, x, rows, n, k, mode="auto", bias=bias)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", FORMATS)
def test_matrix_cores_subnormal_scales(dev, fmt):
    # Weights and activations small enough that the block scales d, the
    # activation scales and the Q4_1 sums are subnormal halves: the f16
    # products of the matrix-core kernel must keep them, not flush them.
    rows, n, k = 64, 128, 512
    say("matrix subnormal", fmt)
    wq = weights(fmt, n, k, 920, scale=1e-4)
    x = acts(rows, k, 921, scale=1e-3)
    want = oracle.matmul(fmt, x, wq, rows, n, k)
    got = run_product(dev, fmt, wq, x, rows, n, k, mode="matrix")
    assert np.array_equal(bits(got), bits(want))
    size = {"Q8_0": 34, "Q4_0": 18, "Q4_1": 20}[fmt]
    d_bits = np.asarray(wq, np.uint8).reshape(-1, size)[:, :2].copy().view(np.uint16)
    assert ((d_bits & 0x7c00) == 0).mean() > 0.5  # most weight scales are subnormal halves
    s, _, _ = oracle.quantize_activations(x[:k], with_sums=True)
    assert (np.abs(s) < 6.1e-5).any() and (np.abs(s) > 0).all()


@pytest.mark.parametrize("fmt", FORMATS)
def test_matrix_cores_with_bias_and_slice(dev, fmt):
    rows, n, k = 70, 96, 1280
    rng = np.random.default_rng(5)
    wq = oracle.quantize(fmt, rng.uniform(-1, 1, n * k).astype(np.float32))
    x = rng.uniform(-3, 3, rows * k).astype(np.float32)
    bias = rng.uniform(-1, 1, 40).astype(np.float32)
    full = oracle.matmul_reference(fmt, x, wq, rows, n, k)
    want = oracle.add_bias(np.ascontiguousarray(full[:, 30:70]), bias)
    say("matrix slice", fmt)
    got = run_product(dev, fmt, wq, x, rows, 40, k, mode="matrix", bias=bias, w_row=30)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("rows,n,k", [(64, 192, 1024), (64, 16448, 1024)])
def test_unordered_matrix_close(dev, fmt, rows, n, k):
    # UNORDERED from 32 rows runs the matrix-core kernel with each block's
    # contribution added by one fused multiply-add: the host's sums to within
    # the rounding of 32 products and sums (k = 1024), not its bits (257
    # tiles: more than one round of workgroups).
    say("unordered matrix", fmt, rows, n, k)
    wq = weights(fmt, n, k, 910)
    x = acts(rows, k, 911)
    want = oracle.matmul(fmt, x, wq, rows, n, k)
    got = run_product(dev, fmt, wq, x, rows, n, k, mode="unordered")
    scale = float(np.abs(want).max())
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5 * scale)


def test_plan_unordered_mode(dev):
    # A plan set to UNORDERED (tmh_plan_set_mode): the streamed kernel folds
    # each row its own way, close to the host's sums; set back to AUTO, the
    # host's bits again.
    import bench

    c2 = bench.build_config2(dev, copies=1)
    plan = c2["plans"][0]
    prods = c2["prods"]
    want = [oracle.matmul("Q4_0", c2["xs"][i], c2["weights"][i], 1, n, k)[0] for i, (_, n, k) in enumerate(prods)]
    plan.set_mode("unordered")
    plan.run()
    got = [dev.to_array(y, np.float32, n) for y, (_, n, _) in zip(c2["ybufs"], prods)]
    assert close_not_same(np.concatenate(got), np.concatenate(want))
    plan.set_mode("auto")
    plan.run()
    got = [dev.to_array(y, np.float32, n) for y, (_, n, _) in zip(c2["ybufs"], prods)]
    assert np.array_equal(bits(np.concatenate(got)), bits(np.concatenate(want)))
    with pytest.raises(th.Error):
        plan.set_mode("thread")
    for p in c2["plans"]:
        p.destroy()


def test_bench_config2_plan_bit_exact(dev):
    # bench.py's timed launch exactly as it builds it (config 2: the 121
    # products of a SmolLM2-135M token, the 49152 x 576 head included, packed
    # at 256-byte offsets in one weight buffer, one k_matvec_stream plan),
    # run twice: every product's bits equal the oracle's.
    import bench

    c2 = bench.build_config2(dev, copies=1)
    plan = c2["plans"][0]
    say("bench plan", plan.describe())
    assert "stream" in plan.describe()
    for _ in range(2):
        plan.run()
    dev.sync()
    for i, (name, n, k) in enumerate(c2["prods"]):
        got = dev.to_array(c2["ybufs"][i], np.float32, n)
        want = oracle.matmul("Q4_0", c2["xs"][i], c2["weights"][i], 1, n, k)[0]
        assert np.array_equal(bits(got), bits(want)), name
    plan.destroy()
