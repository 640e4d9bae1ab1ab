"""The oracle's quantised products (Quant.matmul_reference, quant.cr:122-142)
and fast path (Quant.matmul, quant.cr:155-413), pinned without retyping them:

* a float64 product of the values each side's quantisation keeps, within the
  per-output bound of spec/block_matmul_spec.cr:11-31;
* closed forms: zero blocks, exact single blocks, sign and index probes
  (a plausible slip -- a nibble half swapped, a dropped -8, a transposed
  operand -- fails them);
* expression order: inputs where the reference's association gives
  different f32 bits from the alternatives;
* the reference's invariants: fast == reference bit for bit at the shapes of
  quant_spec.cr:30-48, on 1, 8 and 3 threads (50-72), products of few and
  many spans alternating (74-98), and each row alone == in a batch
  (block_matmul_spec.cr:118-123).
"""
import numpy as np
import pytest

from oracle import oracle

FORMATS = ["Q8_0", "Q4_0", "Q4_1"]


def f64_reference(x, rows, wq, fmt, n, k):
    """block_matmul_spec.cr:11-31: float64 sums of dequantised weights times
    Q8_0-kept activations, and each output's bound."""
    weights = oracle.dequantize(fmt, wq, n * k).reshape(n, k).astype(np.float64)
    kept = oracle.dequantize("Q8_0", oracle.quantize("Q8_0", x), rows * k).reshape(rows, k).astype(np.float64)
    sums = kept @ weights.T
    bounds = 1e-5 * np.maximum(1.0, np.abs(sums))
    if fmt == "Q4_1":
        for b in range(k // 32):
            minimum = np.abs(weights[:, b * 32:(b + 1) * 32].min(axis=1))
            bounds += minimum[None, :] * np.abs(kept[:, b * 32:(b + 1) * 32].sum(axis=1))[:, None] / 1024
    return sums, bounds


def spec_values(n, seed):
    """random_values of spec_helper.cr:42-45: uniform in [-1, 1) (numpy's generator, not Crystal's)."""
    return np.random.default_rng(seed).uniform(-1.0, 1.0, n).astype(np.float32)


@pytest.mark.parametrize("fmt", FORMATS)
def test_sums_integer_block_products_within_f64_bound(fmt):
    # block_matmul_spec.cr:94-100, rows 5, n 7, k 96, and a longer case.
    for rows, n, k, seed in ((5, 7, 96, 1), (3, 37, 1280, 4), (2, 64, 2048, 9)):
        x = spec_values(rows * k, seed)
        w = spec_values(n * k, seed + 1)
        wq = oracle.quantize(fmt, w)
        got = oracle.matmul_reference(fmt, x, wq, rows, n, k).astype(np.float64)
        sums, bounds = f64_reference(x, rows, wq, fmt, n, k)
        assert np.all(np.abs(got - sums) <= bounds), np.max(np.abs(got - sums) - bounds)


@pytest.mark.parametrize("fmt", FORMATS)
def test_zero_blocks_and_zero_rows(fmt):
    k, n = 128, 5
    w = spec_values(n * k, 3)
    w[:32] = 0  # first block of the first weight row
    x = spec_values(2 * k, 4)
    x[k:] = 0  # second activation row all zero
    wq = oracle.quantize(fmt, w)
    got = oracle.matmul_reference(fmt, x, wq, 2, n, k)
    assert np.all(got[1].view(np.uint32) == 0)  # +0.0: the fold starts at 0.0f
    # dropping the first (zero) block changes nothing
    got_tail = oracle.matmul_reference(fmt, x[:k].reshape(1, k)[:, 32:].copy(),
                                       oracle.quantize(fmt, w.reshape(n, k)[:, 32:].copy()), 1, n, k - 32)
    assert got_tail[0, 0].view(np.uint32) == got[0, 0].view(np.uint32)


def test_single_block_exact_values():
    # Weights and activations chosen so every quantised value is exact and
    # every product exact: y = Σ w·x exactly. Element j pairs with element j;
    # the nibble layout (low = j, high = j + 16) and the -8 of Q4_0 matter.
    j = np.arange(32)
    x = np.where(j == 0, 127.0, (j % 7) - 3.0).astype(np.float32)  # amax 127 -> d = 1, q = x
    # Q8_0: amax 127 -> d = 1, q = w
    w8 = np.where(j == 5, -127.0, (j % 5) - 2.0).astype(np.float32)
    got = oracle.matmul_reference("Q8_0", x, oracle.quantize("Q8_0", w8), 1, 1, 32)[0, 0]
    assert got == np.float32(np.dot(w8.astype(np.float64), x.astype(np.float64)))
    # Q4_0: max |w| = 8 with sign -> d = 1 (d = m / -8 with m = -8): q - 8 = w for w in [-8, 7]
    w4 = np.where(j == 3, -8.0, (j % 16) - 8.0).astype(np.float32)
    w4[3] = -8.0
    got = oracle.matmul_reference("Q4_0", x, oracle.quantize("Q4_0", w4), 1, 1, 32)[0, 0]
    assert got == np.float32(np.dot(w4.astype(np.float64), x.astype(np.float64)))
    # Q4_1: min 0, max 15 -> d = 1, m = 0, q = w
    w41 = (j % 16).astype(np.float32)
    got = oracle.matmul_reference("Q4_1", x, oracle.quantize("Q4_1", w41), 1, 1, 32)[0, 0]
    # Q4_1 adds m·(d·Σq) with m = 0: exact
    assert got == np.float32(np.dot(w41.astype(np.float64), x.astype(np.float64)))


@pytest.mark.parametrize("fmt", FORMATS)
def test_element_pairing_probe(fmt):
    # A one-hot activation at element e picks weight element e alone, for
    # every e: catches a swapped nibble half, an offset block or a transposed
    # operand.
    rng = np.random.default_rng(7)
    k, n = 64, 3
    w = rng.uniform(-1, 1, n * k).astype(np.float32)
    wq = oracle.quantize(fmt, w)
    deq = oracle.dequantize(fmt, wq, n * k).reshape(n, k)
    for e in range(k):
        x = np.zeros(k, np.float32)
        x[e] = 1.0  # activation block: d = 1/127, q[e] = 127, others 0
        got = oracle.matmul_reference(fmt, x, wq, 1, n, k)[0]
        sx = np.float32(np.float16(np.float32(1.0) / np.float32(127.0)))
        for col in range(n):
            want = np.float64(deq[col, e]) * 127.0 * np.float64(sx)
            if fmt == "Q4_1":
                # plus m · F16(127 · d) over the block that holds e
                b = e // 32
                m = np.float32(np.frombuffer(wq[col * (k // 32) * 20 + b * 20 + 2:][:2].tobytes(), np.float16)[0])
                want = (np.float64(deq[col, e]) - np.float64(m)) * 127.0 * np.float64(sx) \
                    + np.float64(m) * np.float64(np.float32(np.float16(np.float32(127.0) * (np.float32(1.0) / np.float32(127.0)))))
            assert abs(np.float64(got[col]) - want) <= 1e-6 * max(1.0, abs(want)), (e, col)


def contributions_with_order(fmt, x, wq, k, order):
    """One output's block contributions folded left to right from +0.0, each
    written in a stated association, from the oracle's own activation
    quantisation."""
    return fold_sequential(block_contributions(fmt, x, wq, k, order))


def fold_sequential(values):
    """sum = 0f32, then sum += value in index order (quant.cr:446-491)."""
    total = np.float32(0.0)
    for v in values:
        total = np.float32(total + v)
    return total


def fold_reversed(values):
    return fold_sequential(values[::-1])


def fold_pairwise(values):
    """A balanced tree of f32 adds (what a parallel reduction computes)."""
    v = list(values)
    while len(v) > 1:
        nxt = [np.float32(v[i] + v[i + 1]) for i in range(0, len(v) - 1, 2)]
        if len(v) % 2:
            nxt.append(v[-1])
        v = nxt
    return np.float32(v[0])


def block_contributions(fmt, x, wq, k, order):
    """One output's per-block contributions (Appendix A's expressions), each
    written in a stated association, as a list in block order."""
    scales, sums, qs = oracle.quantize_activations(x, with_sums=(fmt == "Q4_1"))
    bb = oracle.BLOCK_BYTES[oracle.kind_of(fmt)]
    f32 = np.float32
    out = []
    for b in range(k // 32):
        blk = wq[b * bb:(b + 1) * bb]
        d = f32(np.frombuffer(blk[:2].tobytes(), np.float16)[0])
        qb = qs[b * 32:(b + 1) * 32].astype(np.int64)
        if fmt == "Q8_0":
            t = int((blk[2:].view(np.int8).astype(np.int64) * qb).sum())
        else:
            base = 2 if fmt == "Q4_0" else 4
            lo = (blk[base:base + 16] & 0x0F).astype(np.int64)
            hi = (blk[base:base + 16] >> 4).astype(np.int64)
            off = 8 if fmt == "Q4_0" else 0
            t = int(((lo - off) * qb[:16]).sum() + ((hi - off) * qb[16:]).sum())
        tf, sx = f32(t), scales[b]
        if fmt == "Q4_1":
            m = f32(np.frombuffer(blk[2:4].tobytes(), np.float16)[0])
            c = order(tf, d, sx) + f32(m * sums[b])
        else:
            c = order(tf, d, sx)
        out.append(f32(c))
    return out


ORDERS = {
    "(t*d)*s": lambda t, d, s: np.float32(np.float32(t * d) * s),
    "t*(d*s)": lambda t, d, s: np.float32(t * np.float32(d * s)),
    "(d*s)*t": lambda t, d, s: np.float32(np.float32(d * s) * t),
}
# The association each format's fold uses: quant.cr:454, 471, 488.
REFERENCE_ORDER = {"Q8_0": "t*(d*s)", "Q4_0": "(t*d)*s", "Q4_1": "(d*s)*t"}


@pytest.mark.parametrize("fmt", FORMATS)
def test_expression_order(fmt):
    # Over many random rows, the reference's association must reproduce the
    # oracle's bits every time, and the alternative must differ somewhere
    # (so the check has teeth).
    rng = np.random.default_rng(11)
    k = 64
    differs = 0
    for trial in range(300):
        w = rng.uniform(-2, 2, k).astype(np.float32)
        # activations correlated with the weights give large block integers,
        # where t*d is no longer exact in f32 and the associations part
        x = (w * 1.5 + rng.uniform(-0.3, 0.3, k)).astype(np.float32)
        wq = oracle.quantize(fmt, w)
        got = oracle.matmul_reference(fmt, x, wq, 1, 1, k)[0, 0]
        want = contributions_with_order(fmt, x, wq, k, ORDERS[REFERENCE_ORDER[fmt]])
        assert got.view(np.uint32) == want.view(np.uint32), trial
        other = "(t*d)*s" if REFERENCE_ORDER[fmt] != "(t*d)*s" else "t*(d*s)"
        alt = contributions_with_order(fmt, x, wq, k, ORDERS[other])
        differs += int(alt.view(np.uint32) != got.view(np.uint32))
    assert differs > 0


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("k", [128, 256, 2048])
def test_blocks_fold_in_block_order(fmt, k):
    # quant.cr:446-491 folds the block contributions left to right from
    # 0.0f. At k >= 128 (4 blocks or more) the order shows in the bits: the
    # sequential fold must reproduce the oracle every time, while a reversed
    # fold and a pairwise tree must each differ somewhere. Blocks of x are
    # scaled by 2^u, u in [-6, 6], so partial sums cross binades.
    rng = np.random.default_rng(k + len(fmt))
    order = ORDERS[REFERENCE_ORDER[fmt]]
    reversed_differs = pairwise_differs = 0
    trials = 120 if k < 2048 else 30
    for trial in range(trials):
        w = rng.uniform(-2, 2, k).astype(np.float32)
        scale = np.repeat(2.0 ** rng.uniform(-6, 6, k // 32), 32)
        x = (rng.uniform(-1, 1, k) * scale).astype(np.float32)
        wq = oracle.quantize(fmt, w)
        got = oracle.matmul_reference(fmt, x, wq, 1, 1, k)[0, 0]
        c = block_contributions(fmt, x, wq, k, order)
        assert got.view(np.uint32) == fold_sequential(c).view(np.uint32), trial
        reversed_differs += int(fold_reversed(c).view(np.uint32) != got.view(np.uint32))
        pairwise_differs += int(fold_pairwise(c).view(np.uint32) != got.view(np.uint32))
    assert reversed_differs > 0 and pairwise_differs > 0, (reversed_differs, pairwise_differs)


def test_fold_starts_from_plus_zero():
    # Q4_0 with a negative scale d and an all-zero activation row: every
    # contribution (0·d)·0 is -0.0, and a fold from +0.0 gives +0.0 (a fold
    # that starts from the first contribution would give -0.0).
    k, n = 256, 4
    w = np.tile(np.array([1.0] + [0.25] * 31, np.float32), n * k // 32)  # m = +1: d = -1/8
    wq = oracle.quantize("Q4_0", w)
    x = np.zeros(k, np.float32)
    c = block_contributions("Q4_0", x, wq[:k // 32 * 18], k, ORDERS[REFERENCE_ORDER["Q4_0"]])
    assert all(v.view(np.uint32) == 0x80000000 for v in c)  # -0.0 each
    for fn in (oracle.matmul_reference, oracle.matmul):
        got = fn("Q4_0", x, wq, 1, n, k)
        assert np.all(got.view(np.uint32) == 0), fn


VARIANTS = [v for v in ("portable", "v3", "v4", "vnni") if oracle.variant_runs(v)]


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("fmt", FORMATS)
def test_fast_path_equals_reference_bit_for_bit(fmt, variant):
    # quant_spec.cr:30-48: shapes {1,37,64}, {3,5,1280}, {2,9,4096}, with a
    # zero first block, a spike of 50, a zero activation block and the
    # [127, j - 15.5] row; on every build the host runs (the vnni build
    # computes the block dots with vpdpbusd).
    rng = np.random.default_rng(11)
    for count, n, k in ((1, 37, 64), (3, 5, 1280), (2, 9, 4096)):
        values = rng.uniform(-2.0, 2.0, n * k).astype(np.float32)
        values[:32] = 0
        values[32 * 3] = 50
        x = rng.uniform(-3.0, 3.0, count * k).astype(np.float32)
        if count > 1:
            x[k:k + 32] = 0
        if count > 2:
            x[2 * k:2 * k + 32] = [127.0 if j == 0 else j - 15.5 for j in range(32)]
        wq = oracle.quantize(fmt, values)
        fast = oracle.matmul(fmt, x, wq, count, n, k, variant)
        ref = oracle.matmul_reference(fmt, x, wq, count, n, k)
        assert np.array_equal(fast.view(np.uint32), ref.view(np.uint32)), (count, n, k)


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("fmt", FORMATS)
def test_fast_path_on_every_byte_value(fmt, variant):
    # Raw weight bytes over the whole byte range (Q8_0 values down to -128,
    # every nibble) under finite half scales, and activations with the
    # extreme +-127 and 0: the fast path's integer dots against the
    # reference's, bit for bit.
    rng = np.random.default_rng(21)
    count, n, k = 3, 19, 1024
    blocks = n * k // 32
    size = oracle.row_bytes(fmt, k) // (k // 32)
    raw = rng.integers(0, 256, (blocks, size), dtype=np.uint8)
    halves = rng.uniform(-4.0, 4.0, (blocks, 2)).astype(np.float16).view(np.uint8).reshape(blocks, 4)
    raw[:, :2] = halves[:, :2]
    if fmt == "Q4_1":
        raw[:, 2:4] = halves[:, 2:]
    x = rng.uniform(-3.0, 3.0, count * k).astype(np.float32)
    x[:32] = [127.0 if j % 2 else -127.0 for j in range(32)]
    x[k:k + 64] = 0
    wq = raw.reshape(-1)
    fast = oracle.matmul(fmt, x, wq, count, n, k, variant)
    ref = oracle.matmul_reference(fmt, x, wq, count, n, k)
    assert np.array_equal(fast.view(np.uint32), ref.view(np.uint32))


def test_same_bits_on_any_number_of_threads():
    # quant_spec.cr:50-72
    rng = np.random.default_rng(12)
    n, k = 301, 2048
    values = rng.uniform(-2.0, 2.0, n * k).astype(np.float32)
    x = rng.uniform(-3.0, 3.0, k).astype(np.float32)
    saved = oracle.threads()
    try:
        for fmt in FORMATS:
            wq = oracle.quantize(fmt, values)
            ref = oracle.matmul_reference(fmt, x, wq, 1, n, k)
            for t in (1, 8, 3):
                oracle.set_threads(t)
                got = oracle.matmul(fmt, x, wq, 1, n, k)
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (fmt, t)
    finally:
        oracle.set_threads(saved)


def test_alternating_products_keep_their_spans():
    # quant_spec.cr:74-98 (fewer repetitions)
    rng = np.random.default_rng(13)
    k = 2048
    x = rng.uniform(-3.0, 3.0, k).astype(np.float32)
    products = []
    for outputs in (61, 1201):
        wq = oracle.quantize("Q8_0", rng.uniform(-2.0, 2.0, outputs * k).astype(np.float32))
        products.append((outputs, wq, oracle.matmul_reference("Q8_0", x, wq, 1, outputs, k)))
    saved = oracle.threads()
    try:
        oracle.set_threads(8)
        for i in range(200):
            n, wq, ref = products[i % 2]
            got = oracle.matmul("Q8_0", x, wq, 1, n, k)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), i
    finally:
        oracle.set_threads(saved)


@pytest.mark.parametrize("fmt", FORMATS)
def test_row_alone_equals_row_in_batch(fmt):
    # block_matmul_spec.cr:118-123
    rows, n, k = 5, 7, 96
    x = spec_values(rows * k, 1)
    wq = oracle.quantize(fmt, spec_values(n * k, 2))
    batched = oracle.matmul_reference(fmt, x, wq, rows, n, k)
    single = np.concatenate([oracle.matmul_reference(fmt, x[r * k:(r + 1) * k], wq, 1, n, k) for r in range(rows)])
    assert np.array_equal(batched.view(np.uint32), single.view(np.uint32))


def test_bias_is_a_separate_rounding():
    # host.cr:725-734
    rng = np.random.default_rng(3)
    dst = rng.normal(0, 1, (4, 7)).astype(np.float32)
    bias = rng.normal(0, 1, 7).astype(np.float32)
    got = oracle.add_bias(dst, bias)
    assert np.array_equal(got.view(np.uint32), (dst + bias[None, :]).view(np.uint32))
