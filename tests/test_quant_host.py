"""The library's host quantiser (tmh_quantize_weights, through
tensomite.cr_amd/quant_host.py; no GPU needed) equals the oracle's
Quant.quantize byte for byte: on the reference's fixture rows, on N(0, 0.02)
matrices as the BASELINE configs use, on edge values (signed zeros, ties,
subnormal scales, constant blocks), whatever the thread count; and the
synthetic weights do not depend on the thread count either."""
import json
import os

import numpy as np
import pytest

import quant_host
from oracle import oracle

FORMATS = ["Q8_0", "Q4_0", "Q4_1"]


@pytest.mark.parametrize("fmt", FORMATS)
def test_fixture_rows(golden, fmt):
    with open(os.path.join(golden, "quant", "expected.json")) as f:
        expected = json.load(f)
    for i, row in enumerate(expected["rows"]):
        got = quant_host.quantize(fmt, np.array(row, dtype=np.float32))
        assert got.tobytes().hex() == expected[fmt]["bytes"][i], i


@pytest.mark.parametrize("fmt", FORMATS)
def test_random_matrices_equal_oracle(fmt):
    rng = np.random.default_rng(42)
    for std in (0.02, 1.0, 1e-4, 300.0):
        v = rng.normal(0, std, 64 * 2048).astype(np.float32)
        assert np.array_equal(quant_host.quantize(fmt, v), oracle.quantize(fmt, v)), std


@pytest.mark.parametrize("fmt", FORMATS)
def test_edge_values_equal_oracle(fmt):
    rng = np.random.default_rng(3)
    blocks = [
        np.zeros(32), -np.zeros(32), np.concatenate([[-0.0, 0.0], np.zeros(30)]),
        np.concatenate([[0.0, -0.0], np.ones(30)]), np.full(32, 0.25), np.full(32, -3.0),
        np.array([(i - 16) / 2 for i in range(32)]), np.array([127.0] + [j - 15.5 for j in range(1, 32)]),
        np.array([1e-8 * (i - 7) for i in range(32)]), np.array([6e-5 * ((-1) ** i) for i in range(32)]),
        rng.uniform(-1, 1, 32) * 1e-30, np.array([65504.0, -65504.0] + [1.0] * 30),
        np.array([-5.0] + [5.0] * 31), np.array([5.0] + [-5.0] * 31),
    ]
    v = np.concatenate([np.asarray(b, dtype=np.float32) for b in blocks])
    assert np.array_equal(quant_host.quantize(fmt, v), oracle.quantize(fmt, v))


@pytest.mark.parametrize("fmt", FORMATS)
def test_nan_and_infinities_equal_oracle(fmt):
    # A NaN or an infinity at each position of a block (and whole blocks of
    # them): the host quantiser's bytes equal the oracle's. Q8_0's scale is
    # x.max_of(&.abs) (quant.cr:499-500): the first value's magnitude,
    # replaced only by a larger one, so a NaN first makes the scale NaN
    # while a NaN later is skipped.
    rng = np.random.default_rng(17)
    blocks = []
    for special in (np.nan, np.inf, -np.inf):
        for pos in range(32):
            b = rng.uniform(-1, 1, 32).astype(np.float32)
            b[pos] = special
            blocks.append(b)
        blocks.append(np.full(32, special, np.float32))
    v = np.concatenate(blocks)
    assert np.array_equal(quant_host.quantize(fmt, v), oracle.quantize(fmt, v))


def test_q8_0_nan_first_value():
    # scale NaN/127 = NaN -> half 0x7E00 (f16.cr: NaN keeps its sign; |NaN|
    # has none); every value NaN·(1/NaN) rounds to NaN, and to_i8! of NaN is
    # 0 as x86-64 converts it (cvttss2si's integer indefinite, low byte 0)
    b = np.linspace(-1, 1, 32).astype(np.float32)
    b[0] = np.nan
    want = np.array([0x00, 0x7E] + [0] * 32, np.uint8)
    assert np.array_equal(oracle.quantize("Q8_0", b), want)
    assert np.array_equal(quant_host.quantize("Q8_0", b), want)


def test_f16_bits_match_oracle():
    rng = np.random.default_rng(9)
    words = rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    values = words.view(np.float32)
    values = values[~np.isnan(values)]
    assert np.array_equal(quant_host.f16_bits(values), oracle.f16_bits_many(values))
    nan = np.array([np.nan, -np.nan], dtype=np.float32)
    assert quant_host.f16_bits(nan).tolist() == [0x7E00, 0xFE00]


@pytest.mark.parametrize("fmt", FORMATS)
def test_threads_do_not_change_bytes(fmt):
    v = np.random.default_rng(17).normal(0, 0.5, 32 * 70001).astype(np.float32)
    want = oracle.quantize(fmt, v)
    for threads in (1, 2, 3, 8, 0):
        assert np.array_equal(quant_host.quantize(fmt, v, threads=threads), want), threads


def test_synthetic_weights_are_chunked_by_seed_only(monkeypatch):
    # chunk c of a matrix comes from default_rng([seed, c]), N(0,1) f32 times
    # f32(0.02), quantised -- however many workers make them
    n, k = 300, 32 * 1024  # 9.8M values: three chunks
    got = quant_host.synthetic_weights("Q4_0", n, k, seed=[7, 1])
    monkeypatch.setattr(quant_host, "_cores", lambda: 1)
    assert np.array_equal(quant_host.synthetic_weights("Q4_0", n, k, seed=[7, 1]), got)
    c = quant_host.CHUNK_VALUES
    first = np.random.default_rng([7, 1, 1]).standard_normal(c, dtype=np.float32) * np.float32(0.02)
    assert np.array_equal(got[c // 32 * 18:2 * c // 32 * 18], oracle.quantize("Q4_0", first))


def test_quantiser_refuses_bad_input():
    import tensomite_hip as th
    with pytest.raises(th.DTypeError):
        quant_host.quantize(3, np.zeros(32, np.float32))
    with pytest.raises(ValueError):
        quant_host.quantize("Q8_0", np.zeros(33, np.float32))
