"""The oracle's quantisers against the data the reference's own tests hold.

Mirrors spec/quant_spec.cr:12-28 and 110-135 (fixtures copied verbatim into
tests/golden/quant/) and block_matmul_spec.cr:244-251, which asserts that the
tiny_llama GGUFs (gguf-py quantisations, scripts/make_fixtures.py:298-357)
equal tensomite's own quantisation: here byte for byte, matrix by matrix.
"""
import json
import os

import numpy as np
import pytest
from safetensors.numpy import load_file

from gguf_io import GGUF
from oracle import oracle

FORMATS = ["Q8_0", "Q4_0", "Q4_1"]


@pytest.fixture(scope="module")
def expected(golden):
    with open(os.path.join(golden, "quant", "expected.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("fmt", FORMATS)
def test_quantises_as_ggml_byte_for_byte(expected, fmt):
    # quant_spec.cr:15-19
    for i, row in enumerate(expected["rows"]):
        got = oracle.quantize(fmt, np.array(row, dtype=np.float32))
        assert got.tobytes().hex() == expected[fmt]["bytes"][i], f"row {i}"


@pytest.mark.parametrize("fmt", FORMATS)
def test_dequantises_as_ggml(expected, fmt):
    # quant_spec.cr:21-27
    for i, hexed in enumerate(expected[fmt]["bytes"]):
        data = np.frombuffer(bytes.fromhex(hexed), dtype=np.uint8)
        count = len(expected["rows"][i])
        got = oracle.dequantize(fmt, data, count)
        want = np.array(expected[fmt]["values"][i], dtype=np.float32)
        assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist(), f"row {i}"


@pytest.mark.parametrize("fmt", FORMATS)
def test_table_round_trip_and_blocks_gguf(expected, golden, fmt):
    # quant_spec.cr:115-134: the 3x64 table quantised here, and as stored in
    # blocks.gguf, both dequantise to the expected values.
    table = np.array(expected["table"], dtype=np.float32)
    want = np.array(expected[fmt]["table"], dtype=np.float32).reshape(-1)
    ours = oracle.quantize(fmt, table)
    stored = GGUF(os.path.join(golden, "quant", "blocks.gguf"))
    assert stored.kind(fmt.lower()) == fmt and stored.shape(fmt.lower()) == [3, 64]
    assert ours.tobytes() == stored.raw(fmt.lower()).tobytes()
    got = oracle.dequantize(fmt, ours, table.size)
    assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist()


def gguf_permute(weights: np.ndarray, heads: int) -> np.ndarray:
    """llama.cpp's rotary row order for q/k, as scripts/make_fixtures.py:290-293 applies it."""
    return weights.reshape(heads, 2, weights.shape[0] // heads // 2, *weights.shape[1:]).swapaxes(1, 2).reshape(weights.shape)


GGUF_NAMES = {
    "input_layernorm": "attn_norm", "post_attention_layernorm": "ffn_norm",
    "self_attn.q_proj": "attn_q", "self_attn.k_proj": "attn_k", "self_attn.v_proj": "attn_v",
    "self_attn.o_proj": "attn_output", "mlp.gate_proj": "ffn_gate", "mlp.up_proj": "ffn_up",
    "mlp.down_proj": "ffn_down",
}


@pytest.mark.parametrize("fmt", ["Q8_0", "Q4_0"])
def test_tiny_llama_gguf_bytes(golden, fmt):
    # block_matmul_spec.cr:244-251, at the byte level: every quantised matrix
    # of model-<fmt>.gguf is the restated quantiser's output on the F32
    # safetensors weights, in llama.cpp's q/k row order.
    base = os.path.join(golden, "tiny_llama")
    with open(os.path.join(base, "config.json")) as f:
        config = json.load(f)
    weights = load_file(os.path.join(base, "model.safetensors"))
    gguf = GGUF(os.path.join(base, f"model-{fmt.lower()}.gguf"))
    checked = 0
    for name, tensor in weights.items():
        if name.startswith("model.layers."):
            _, _, layer, rest = name.split(".", 3)
            part, last = rest.rsplit(".", 1)
            key = f"blk.{layer}.{GGUF_NAMES[part]}.{last}"
            if part == "self_attn.q_proj":
                tensor = gguf_permute(tensor, config["num_attention_heads"])
            elif part == "self_attn.k_proj":
                tensor = gguf_permute(tensor, config["num_key_value_heads"])
        else:
            key = {"model.embed_tokens.weight": "token_embd.weight", "model.norm.weight": "output_norm.weight",
                   "lm_head.weight": "output.weight"}[name]
        if tensor.ndim == 1:
            assert gguf.kind(key) == "F32"
            continue
        assert gguf.kind(key) == fmt, key
        assert gguf.shape(key) == list(tensor.shape), key
        ours = oracle.quantize(fmt, np.ascontiguousarray(tensor, dtype=np.float32))
        assert ours.tobytes() == gguf.raw(key).tobytes(), key
        checked += 1
    assert checked == 2 * 7 + 2


def test_activation_quantiser_equals_weight_q8_0(expected):
    # quant.cr:428-442 against quant.cr:499-505: the same d, id and rounding,
    # so the activation scales and values equal Q8_0's stored bytes.
    for i, row in enumerate(expected["rows"]):
        values = np.array(row, dtype=np.float32)
        scales, sums, qs = oracle.quantize_activations(values, with_sums=True)
        stored = bytes.fromhex(expected["Q8_0"]["bytes"][i])
        for b in range(values.size // 32):
            block = stored[b * 34:(b + 1) * 34]
            d = np.frombuffer(block[:2], dtype=np.float16)[0].astype(np.float32)
            assert scales[b].view(np.uint32) == d.view(np.uint32), (i, b)
            assert qs[b * 32:(b + 1) * 32].tobytes() == block[2:], (i, b)


def test_q8_1_sum_closed_form(expected):
    # quant.cr:440: sums = F16(float(Σq) · d) with d = amax/127 unrounded, not
    # the F16 scale: checked with numpy's IEEE float16 rounding.
    rng = np.random.default_rng(5)
    rows = [np.array(r, dtype=np.float32) for r in expected["rows"]] + [
        rng.normal(0, s, 32 * 16).astype(np.float32) for s in (1e-3, 1.0, 300.0)]
    for values in rows:
        scales, sums, qs = oracle.quantize_activations(values, with_sums=True)
        for b in range(values.size // 32):
            block = values[b * 32:(b + 1) * 32]
            d = np.float32(np.max(np.abs(block))) / np.float32(127.0)
            total = np.float32(int(qs[b * 32:(b + 1) * 32].astype(np.int32).sum()))
            want = np.float32(np.float16(total * d))
            assert sums[b].view(np.uint32) == want.view(np.uint32)
            assert scales[b].view(np.uint32) == np.float32(np.float16(d)).view(np.uint32)


@pytest.mark.parametrize("fmt", FORMATS)
def test_gather_dequantises_rows(expected, fmt):
    # block_matmul_spec.cr:221-236 with quant_spec.cr's table: rows 2, 0, 2.
    table = np.array(expected["table"], dtype=np.float32)
    q = oracle.quantize(fmt, table)
    whole = np.array(expected[fmt]["table"], dtype=np.float32).reshape(3, 64)
    got = oracle.gather(fmt, q, 3, 64, [2, 0, 2])
    assert np.array_equal(got.view(np.uint32), whole[[2, 0, 2]].view(np.uint32))
    with pytest.raises(IndexError):
        oracle.gather(fmt, q, 3, 64, [3])
    with pytest.raises(IndexError):
        oracle.gather(fmt, q, 3, 64, [-1])


@pytest.mark.parametrize("fmt", FORMATS)
def test_dequantised_values_within_half_a_step(expected, fmt):
    # quant_spec.cr:144-158
    table = np.array(expected["table"], dtype=np.float32).reshape(-1)
    got = oracle.dequantize(fmt, oracle.quantize(fmt, table), table.size)
    for b in range(table.size // 32):
        block = table[b * 32:(b + 1) * 32]
        amax, span = np.abs(block).max(), block.max() - block.min()
        bound = {"Q8_0": amax / 254, "Q4_0": amax / 8, "Q4_1": span / 30}[fmt]
        assert np.all(np.abs(got[b * 32:(b + 1) * 32] - block) <= bound + amax / 1024 + 1e-7)
