"""The oracle's Llama forward (oracle/tmq_llama.c), pinned by the reference's
own model-level fixtures and invariants:

* Maths.exp (maths.cr:36-54) within 2 ulp of the correctly rounded exp over
  its range, with the special values its spec states (spec/maths_spec.cr);
  its range reduction and 2^n scaling bit for bit by an identity they
  imply (exp(k·LN2_HI + y) == 2^k · exp(r)); the order of its last sums by
  the rounding profile that order gives near zero. The polynomial's
  coefficients are pinned by the bound only;
* the tiny_llama quantised GGUFs against the F32 PyTorch logits of
  logits.json: Q8_0 strays less than a quarter of Q4_0's error
  (block_matmul_spec.cr:275-284), and both stay close;
* prefill gives the bits of one-by-one decode (block_matmul_spec.cr:253-260);
* forward_last's row equals the full forward's last row;
* RMSNorm, SwiGLU and the RoPE tables against float64 restatements of their
  definitions (bounds, not retyped bits);
* the order of every sequential f32 fold of the decode graph -- RMSNorm's
  sum of squares (host.cr:374-386), attention's dot products, softmax
  total and value fold (host.cr:408-440) -- against plain f32 loops in index
  order, where a reversed fold and a pairwise tree must each give other bits
  on the same inputs.
"""
import json
import os

import numpy as np
import pytest

from llama_fixtures import random_llama, tiny_llama, tiny_llama_from_safetensors
from oracle import oracle


def ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def test_exp_within_two_ulp_and_special_values():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-87.0, 88.7, 1 << 20), rng.uniform(-1, 1, 1 << 16),
                        np.linspace(-87.3, 88.7, 100001)]).astype(np.float32)
    got = oracle.exp_many(x)
    want = np.exp(x.astype(np.float64)).astype(np.float32)
    normal = want >= np.float32(1.1754944e-38)
    assert ulp_distance(got[normal], want[normal]).max() <= 2
    special = np.array([0.0, -0.0, np.inf, -np.inf, 89.0, -88.0, np.nan], np.float32)
    s = oracle.exp_many(special)
    assert s[0] == 1 and s[1] == 1 and np.isinf(s[2]) and s[3] == 0 and np.isinf(s[4]) and s[5] == 0
    assert np.isnan(s[6])


def test_exp_range_reduction_identity():
    # Maths.exp (maths.cr:36-54) reduces x to r = (x - n·LN2_HI) - n·LN2_LO
    # with n = round(x·log2 e), evaluates one polynomial at r and scales it
    # by 2^⌊n/2⌋ · 2^(n - ⌊n/2⌋). For x = k·LN2_HI + y (LN2_HI = 355/512, so
    # k·LN2_HI is exact for |k| <= 128, and y a multiple of 2^-17 keeps x
    # exact) n is k, x - k·LN2_HI is y exactly, and the polynomial is taken at
    # r = f32(y - f32(k·LN2_LO)) -- the r that exp(r) itself reduces to with
    # n = 0. Powers of two scale exactly, so exp(x) == 2^k · exp(r) bit for
    # bit. A one-constant reduction, a floor for the rounding, a dropped low
    # part or a single 2^n (which overflows at k = 128) each break it; the
    # polynomial itself is pinned only by the 2 ulp bound above.
    LN2_HI, LN2_LO = np.float32(0.693359375), np.float32(-2.12194440e-4)
    rng = np.random.default_rng(5)
    ks, ys = [], []
    for k in range(-125, 128):
        for y in rng.integers(-13107, 13108, 40):  # |y| <= 0.1
            ks.append(k), ys.append(np.float32(y) * np.float32(2.0 ** -17))
    for y in rng.integers(-45875, -3932, 400):  # k = 128: x in [88.40, 88.72]
        ks.append(128), ys.append(np.float32(y) * np.float32(2.0 ** -17))
    k = np.array(ks, np.int64)
    y = np.array(ys, np.float32)
    x = (k.astype(np.float32) * LN2_HI + y).astype(np.float32)
    assert np.all(x.astype(np.float64) == k * 0.693359375 + y.astype(np.float64))  # x exact
    r = (y - (k.astype(np.float32) * LN2_LO).astype(np.float32)).astype(np.float32)
    got = oracle.exp_many(x).astype(np.float64)
    scaled = np.ldexp(oracle.exp_many(r).astype(np.float64), k)
    assert np.all(np.isfinite(got))
    assert np.array_equal(got, scaled), np.flatnonzero(got != scaled)[:5]


def test_exp_assembly_order_near_zero():
    # For |x| <= 2^-8, n = 0 and Maths.exp returns f32(1 + f32(r + f32(p·r²)))
    # (maths.cr:46-47): the inner sum is within 2^-24·|r| of r + p·r², so the
    # one rounding at the end misses the correctly rounded exp only where
    # exp(x) lies that close to a rounding boundary, a share of about |x| of
    # the inputs (<= 0.4% here). Rounding 1 + r first and adding p·r² after
    # (two roundings of comparable size) misrounds about a quarter of them.
    rng = np.random.default_rng(9)
    x = rng.uniform(-2.0 ** -8, 2.0 ** -8, 1 << 18).astype(np.float32)
    got = oracle.exp_many(x)
    want = np.exp(x.astype(np.float64)).astype(np.float32)
    d = ulp_distance(got, want)
    assert d.max() <= 1
    assert (d == 0).mean() >= 0.99, (d == 0).mean()


def test_rmsnorm_swiglu_against_definitions():
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (3, 2048)).astype(np.float32)
    w = rng.normal(1, 0.1, 2048).astype(np.float32)
    got = oracle.rmsnorm(x, w, 1e-5).astype(np.float64)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-5) * w
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
    # a row of equal values: Σx²/n exact, root exact -> x / root exact
    ones = np.full((1, 64), 2.0, np.float32)
    assert np.all(oracle.rmsnorm(ones, None, 0.0) == 1.0)
    g = rng.normal(0, 3, 10000).astype(np.float32)
    v = rng.normal(0, 1, 10000).astype(np.float32)
    gd = g.astype(np.float64)
    want = gd / (np.exp(-gd) + 1) * v
    assert np.allclose(oracle.swiglu(g, v), want, rtol=2e-6, atol=1e-7)


def test_rope_tables_against_definition():
    cos, sin = oracle.rope_tables(64, 2048, 10000.0)
    p = np.arange(2048)[:, None].astype(np.float64)
    i = np.arange(64)[None, :] % 32
    freq = 1.0 / 10000.0 ** (2 * i / 64)
    assert np.allclose(cos, np.cos(p * freq), atol=2e-4)  # angles are rounded to f32 first
    assert np.allclose(sin, np.sin(p * freq), atol=2e-4)
    assert np.all(cos[0] == 1) and np.all(sin[0] == 0)


@pytest.fixture(scope="module")
def fixture_logits(golden):
    with open(os.path.join(golden, "tiny_llama", "logits.json")) as f:
        return json.load(f)


def test_tiny_llama_q8_0_strays_less_than_q4_0(golden, fixture_logits):
    # block_matmul_spec.cr:275-284 on the oracle's forward.
    prompt = fixture_logits["prompt_ids"]
    reference = np.array(fixture_logits["logits"], np.float64)
    errors = {}
    for fmt in ("Q8_0", "Q4_0"):
        config, weights = tiny_llama(golden, fmt)
        model = oracle.Llama(config, weights)
        logits = model.forward(prompt)
        errors[fmt] = np.abs(logits - reference).mean()
    assert errors["Q8_0"] < errors["Q4_0"] / 4
    # and Q8_0 stays near the F32 model: a sign or index slip anywhere in the
    # forward sends the error to the logits' own scale (mean |logit| ~1.4)
    assert errors["Q8_0"] < 0.15


@pytest.mark.parametrize("fmt", ["Q8_0", "Q4_0"])
def test_gguf_equals_safetensors_quantised(golden, fixture_logits, fmt):
    # block_matmul_spec.cr:243-250: the llama.cpp-permuted GGUF, unpermuted on
    # load, equals the F32 model quantised here, in every weight byte and in
    # the forward's bits; this pins the q/k row order.
    config, from_gguf = tiny_llama(golden, fmt)
    _, quantised = tiny_llama_from_safetensors(golden, fmt)
    for name in ("embed", "head", "norm"):
        assert np.array_equal(from_gguf[name], quantised[name]), name
    for name in ("qkv", "o", "gate_up", "down", "attn_norm", "ffn_norm"):
        for a, b in zip(from_gguf[name], quantised[name]):
            assert np.array_equal(a, b), name
    prompt = fixture_logits["prompt_ids"]
    got = oracle.Llama(config, from_gguf).forward(prompt)
    want = oracle.Llama(config, quantised).forward(prompt)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt", ["Q8_0", "Q4_0"])
def test_prefill_equals_one_by_one_decode(golden, fixture_logits, fmt):
    # block_matmul_spec.cr:253-260
    prompt = fixture_logits["prompt_ids"]
    config, weights = tiny_llama(golden, fmt)
    model = oracle.Llama(config, weights)
    prefill = model.forward(prompt)
    model.reset()
    one_by_one = np.concatenate([model.forward([i]) for i in prompt])
    assert np.array_equal(prefill.view(np.uint32), one_by_one.view(np.uint32))
    model.reset()
    last = model.forward(prompt, last_only=True)
    assert np.array_equal(last[0].view(np.uint32), prefill[-1].view(np.uint32))


def test_random_model_generates_deterministically():
    config = dict(layers=2, width=128, heads=4, kv_heads=2, head_width=32, hidden=256, vocab=512, context=64,
                  eps=1e-5, theta=10000.0, kind="Q4_0")
    weights = random_llama(config, seed=3)
    model = oracle.Llama(config, weights)
    prompt = list(np.random.default_rng(4).integers(0, 512, 12))
    a = model.generate(prompt, 20)
    b = model.generate(prompt, 20)
    assert a == b and len(a) == 20


def test_attention_against_float64_definition():
    # host.cr:408-440 against softmax(q·kᵀ·scale + mask)·v in float64, over
    # grouped heads, several cache rows and causal masks; a transposed
    # operand, a wrong kv head or a mask off by one fails the bound.
    rng = np.random.default_rng(5)
    heads, kv_heads, width, capacity, rows = 4, 2, 8, 40, 3
    q = rng.normal(0, 1, (6, heads, width)).astype(np.float32)
    k = rng.normal(0, 1, (rows, kv_heads, capacity, width)).astype(np.float32)
    v = rng.normal(0, 1, (rows, kv_heads, capacity, width)).astype(np.float32)
    table = [[0, 4, 10], [1, 39, 40], [2, 0, 1], [0, 9, 10], [1, 20, 30], [2, 7, 8]]
    got = oracle.attention(q, k, v, table, 0.35)
    for t, (r, last, n) in enumerate(table):
        for h in range(heads):
            kv = h // (heads // kv_heads)
            s = k[r, kv, :n].astype(np.float64) @ q[t, h].astype(np.float64) * 0.35
            s[np.arange(n) > last] = -np.inf
            e = np.exp(s - s.max())
            want = (e / e.sum()) @ v[r, kv, :n].astype(np.float64)
            assert np.allclose(got[t, h], want, atol=2e-6), (t, h)


def test_rope_against_definition():
    # host.cr:448-466: x·cos + rotate_half(x)·sin, rotate_half = [-x2, x1]
    rng = np.random.default_rng(6)
    cos, sin = oracle.rope_tables(8, 32, 10000.0)
    x = rng.normal(0, 1, (5, 3 * 8)).astype(np.float32)
    pos = [0, 3, 31, 7, 7]
    got = oracle.rope(x, 3, 8, cos, sin, pos)
    xd = x.reshape(5, 3, 8).astype(np.float64)
    rot = np.concatenate([-xd[..., 4:], xd[..., :4]], -1)
    want = xd * cos[pos][:, None, :] + rot * sin[pos][:, None, :]
    assert np.allclose(got, want, atol=1e-6)
    assert np.array_equal(got[0], x[0].reshape(3, 8))  # position 0: cos 1, sin 0


def fold_sequential(values):
    total = np.float32(0.0)
    for v in values:
        total = np.float32(total + np.float32(v))
    return total


def fold_reversed(values):
    return fold_sequential(list(values)[::-1])


def fold_pairwise(values):
    v = [np.float32(a) for a in values]
    while len(v) > 1:
        nxt = [np.float32(v[i] + v[i + 1]) for i in range(0, len(v) - 1, 2)]
        if len(v) % 2:
            nxt.append(v[-1])
        v = nxt
    return v[0]


def rmsnorm_with_fold(x, w, eps, fold):
    """host.cr:374-386 with the squares' sum taken by `fold`: squares rounded
    one by one, root = sqrt(Σ/n + eps) rounded, then x / root · w."""
    f32 = np.float32
    n = x.size
    total = fold([f32(v * v) for v in x])
    root = np.sqrt(f32(f32(total / f32(n)) + f32(eps)))
    out = x / root
    return out * w if w is not None else out


def test_rmsnorm_sums_squares_in_index_order():
    # Rows whose Σx² crosses many binades (values scaled by 2^u) or adds many
    # near-equal terms: the index-order fold gives the oracle's bits on every
    # row; reversed and pairwise folds differ on some.
    rng = np.random.default_rng(2)
    rows = []
    for n in (5, 64, 100, 1000):
        for _ in range(6):
            rows.append((rng.normal(0, 1, n) * 2.0 ** rng.uniform(-8, 8, n)).astype(np.float32))
        rows.append(rng.normal(0, 1, n).astype(np.float32))
        rows.append(np.sort(np.abs(rng.normal(0, 1, n))).astype(np.float32))
    rev = pair = 0
    for x in rows:
        w = rng.normal(1, 0.1, x.size).astype(np.float32)
        got = oracle.rmsnorm(x[None, :], w, 1e-5)[0]
        want = rmsnorm_with_fold(x, w, 1e-5, fold_sequential)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), x.size
        rev += int(not np.array_equal(rmsnorm_with_fold(x, w, 1e-5, fold_reversed).view(np.uint32), got.view(np.uint32)))
        pair += int(not np.array_equal(rmsnorm_with_fold(x, w, 1e-5, fold_pairwise).view(np.uint32), got.view(np.uint32)))
    assert rev > 0 and pair > 0, (rev, pair)


def attention_with_folds(q, k, v, last, n, scale, total_fold, value_fold):
    """host.cr:408-440 for one query head: scores q·k in column order, · scale,
    + the causal mask (0 up to `last`, -inf after), the first highest score,
    Maths.exp(score - top), the total by `total_fold`, then per column the
    fold by `value_fold` of (e_p / total) · v_p[col]."""
    f32 = np.float32
    scores = np.empty(n, np.float32)
    top = f32(0.0)
    for p in range(n):
        x = f32(fold_sequential([f32(q[c] * k[p, c]) for c in range(q.size)]) * f32(scale))
        x = f32(x + (f32(-np.inf) if p > last else f32(0.0)))
        scores[p] = x
        if p == 0 or x > top:
            top = x
    e = oracle.exp_many((scores - top).astype(np.float32))
    total = total_fold(list(e))
    out = np.empty(v.shape[1], np.float32)
    for c in range(v.shape[1]):
        out[c] = value_fold([f32(f32(e[p] / total) * v[p, c]) for p in range(n)])
    return out


def test_attention_folds_in_position_order():
    # The softmax total and each output column's value fold are sums in
    # position order from 0f32: the index-order loops give the oracle's bits
    # for every head; a pairwise total, or a reversed value fold, differs on
    # some heads. Grouped heads, a causal mask past `last`, several lengths.
    rng = np.random.default_rng(7)
    heads, kv_heads, width, capacity = 4, 2, 8, 72
    table = [[0, 3, 4], [0, 40, 41], [1, 70, 72], [1, 20, 33], [0, 63, 64]]
    q = rng.normal(0, 2, (len(table), heads, width)).astype(np.float32)
    keys = rng.normal(0, 1, (2, kv_heads, capacity, width)).astype(np.float32)
    values = (rng.normal(0, 1, (2, kv_heads, capacity, width)) *
              2.0 ** rng.uniform(-6, 6, (2, kv_heads, capacity, 1))).astype(np.float32)
    got = oracle.attention(q, keys, values, table, 0.35)
    total_differs = value_differs = 0
    for t, (r, last, n) in enumerate(table):
        for h in range(heads):
            kv = h // (heads // kv_heads)
            args = (q[t, h], keys[r, kv, :n], values[r, kv, :n], last, n, 0.35)
            want = attention_with_folds(*args, fold_sequential, fold_sequential)
            assert np.array_equal(got[t, h].view(np.uint32), want.view(np.uint32)), (t, h)
            a = attention_with_folds(*args, fold_pairwise, fold_sequential)
            b = attention_with_folds(*args, fold_sequential, fold_reversed)
            total_differs += int(not np.array_equal(a.view(np.uint32), want.view(np.uint32)))
            value_differs += int(not np.array_equal(b.view(np.uint32), want.view(np.uint32)))
    assert total_differs > 0 and value_differs > 0, (total_differs, value_differs)
