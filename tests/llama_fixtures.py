"""Llama weights for the decode tests: the reference's tiny_llama GGUF
fixtures, loaded as Llama.load(GGUF) loads them (llama.cr:184-235), and a
random-init SmolLM2-shaped model built with the
package's host quantiser."""
import json
import os

import numpy as np

from gguf_io import GGUF

BLOCK_BYTES = {"Q8_0": 34, "Q4_0": 18, "Q4_1": 20}


def unpermute_order(rows: int, heads: int):
    """Llama.unpermute's row order for block weights (llama.cr:226-235): each
    head's rows from llama.cpp's rotary pairing (2i, 2i+1) back to (i, i + half)."""
    half = rows // heads // 2
    order = []
    for head in range(heads):
        for pair in range(2):
            for i in range(half):
                order.append(head * 2 * half + 2 * i + pair)
    return order


def take_rows(data: np.ndarray, row_bytes: int, order) -> np.ndarray:
    """Tensor#take_rows on block bytes (tensor/quantised.cr:32-43)."""
    rows = data.reshape(-1, row_bytes)
    return np.ascontiguousarray(rows[order]).reshape(-1)


def tiny_llama(golden: str, fmt: str):
    """(config, weights) of tiny_llama/model-<fmt>.gguf, q/k unpermuted and
    the projections merged (Linear.merge, modules.cr:36-56)."""
    base = os.path.join(golden, "tiny_llama")
    with open(os.path.join(base, "config.json")) as f:
        hf = json.load(f)
    g = GGUF(os.path.join(base, f"model-{fmt.lower()}.gguf"))
    width, heads, kv = hf["hidden_size"], hf["num_attention_heads"], hf["num_key_value_heads"]
    hw = hf.get("head_dim", width // heads)
    rb = width // 32 * BLOCK_BYTES[fmt]
    config = dict(layers=hf["num_hidden_layers"], width=width, heads=heads, kv_heads=kv, head_width=hw,
                  hidden=hf["intermediate_size"], vocab=hf["vocab_size"],
                  context=hf["max_position_embeddings"], eps=hf["rms_norm_eps"],
                  theta=hf["rope_parameters"]["rope_theta"], kind=fmt)
    w = dict(embed=g.raw("token_embd.weight"), head=g.raw("output.weight"), norm=g.f32("output_norm.weight"),
             attn_norm=[], ffn_norm=[], qkv=[], o=[], gate_up=[], down=[])
    for layer in range(config["layers"]):
        p = f"blk.{layer}."
        q = take_rows(g.raw(p + "attn_q.weight"), rb, unpermute_order(heads * hw, heads))
        k = take_rows(g.raw(p + "attn_k.weight"), rb, unpermute_order(kv * hw, kv))
        v = g.raw(p + "attn_v.weight")
        w["qkv"].append(np.concatenate([q, k, v]))
        w["o"].append(g.raw(p + "attn_output.weight"))
        w["gate_up"].append(np.concatenate([g.raw(p + "ffn_gate.weight"), g.raw(p + "ffn_up.weight")]))
        w["down"].append(g.raw(p + "ffn_down.weight"))
        w["attn_norm"].append(g.f32(p + "attn_norm.weight"))
        w["ffn_norm"].append(g.f32(p + "ffn_norm.weight"))
    return config, w


from quant_host import SMOLLM2_1P7B  # noqa: E402,F401


def random_llama(config: dict, seed: int, std: float = 0.02, norm_jitter: float = 0.0):
    """A random-init Llama of `config`'s shape (tied head): every matrix
    ~N(0, std) quantised by the package's host quantiser; RMSNorm weights 1
    (as initialised, modules.cr:316-318), optionally jittered."""
    import quant_host

    c = config
    fmt = c["kind"]
    rng = np.random.default_rng(seed)
    qn, kvn = c["heads"] * c["head_width"], c["kv_heads"] * c["head_width"]
    s = [0]

    def matrix(n, k):
        s[0] += 1
        return quant_host.synthetic_weights(fmt, n, k, seed * 1000 + s[0], std)

    def norm():
        v = np.ones(c["width"], np.float32)
        if norm_jitter:
            v += rng.normal(0, norm_jitter, c["width"]).astype(np.float32)
        return v

    w = dict(embed=matrix(c["vocab"], c["width"]), head=None, norm=norm(),
             attn_norm=[], ffn_norm=[], qkv=[], o=[], gate_up=[], down=[])
    for _ in range(c["layers"]):
        w["qkv"].append(matrix(qn + 2 * kvn, c["width"]))
        w["o"].append(matrix(c["width"], qn))
        w["gate_up"].append(matrix(2 * c["hidden"], c["width"]))
        w["down"].append(matrix(c["width"], c["hidden"]))
        w["attn_norm"].append(norm())
        w["ffn_norm"].append(norm())
    return w


def tiny_llama_from_safetensors(golden: str, fmt: str):
    """The F32 tiny_llama quantised by the oracle's quantiser, as
    Llama.load(dir).quantize(dtype, embeddings: true) builds it
    (module.cr:268-277, llama.cr:218-221): Hugging Face row order, no unpermute."""
    from safetensors.numpy import load_file
    from oracle import oracle

    base = os.path.join(golden, "tiny_llama")
    config, _ = tiny_llama(golden, fmt)
    t = load_file(os.path.join(base, "model.safetensors"))

    def q(name):
        return oracle.quantize(fmt, np.ascontiguousarray(t[name], np.float32).reshape(-1))

    w = dict(embed=q("model.embed_tokens.weight"), head=q("lm_head.weight"), norm=t["model.norm.weight"],
             attn_norm=[], ffn_norm=[], qkv=[], o=[], gate_up=[], down=[])
    for layer in range(config["layers"]):
        p = f"model.layers.{layer}."
        w["qkv"].append(np.concatenate([q(p + "self_attn.q_proj.weight"), q(p + "self_attn.k_proj.weight"),
                                        q(p + "self_attn.v_proj.weight")]))
        w["o"].append(q(p + "self_attn.o_proj.weight"))
        w["gate_up"].append(np.concatenate([q(p + "mlp.gate_proj.weight"), q(p + "mlp.up_proj.weight")]))
        w["down"].append(q(p + "mlp.down_proj.weight"))
        w["attn_norm"].append(t[p + "input_layernorm.weight"])
        w["ffn_norm"].append(t[p + "post_attention_layernorm.weight"])
    return config, w


# Model-sized synthetic weights come from the package (quant_host), so bench.py
# measures the same models the tests check.
from quant_host import random_block_llama, random_blocks  # noqa: E402,F401


def write_llama_gguf(path: str, config: dict, weights: dict, norm_kind: str = "F32") -> None:
    """Writes `weights` (the decoder's layout, q/k in Hugging Face order) as a
    llama.cpp GGUF, by the package's exporter (gguf_export.write_llama)."""
    import gguf_export

    gguf_export.write_llama(path, config, weights, norm_kind)
