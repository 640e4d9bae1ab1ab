"""Writes GGUF files the reference loads, so the same weight bytes can be
timed by tensomite.cr itself wherever Crystal is installed.

`write_gguf` follows GGUF.write (src/tensomite/gguf.cr:156-191): version 3,
typed metadata, tensor directory (dimensions innermost first, ggml kind,
offset), data aligned to 32 bytes, written under a temporary name and renamed
into place. `write_llama` writes a decoder's weights in llama.cpp's layout
(the one Llama.load reads, llama.cr:184-235): q and k rows permuted to
llama.cpp's rotary pairing (the inverse of Llama.unpermute, llama.cr:226-235),
the merged projections split, the llama.* metadata Llama.config reads
(llama.cr:57-77). `export_configs` writes the BASELINE configs' weights, the
same bytes bench.py measures.
"""
from __future__ import annotations

import os
import struct

import numpy as np

MAGIC = 0x46554747
ALIGNMENT = 32
KINDS = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q8_0": 8, "BF16": 30}
BLOCK_BYTES = {"Q8_0": 34, "Q4_0": 18, "Q4_1": 20}


def _string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(v) -> bytes:
    if isinstance(v, bool):
        return struct.pack("<IB", 7, v)
    if isinstance(v, int):
        return struct.pack("<II", 4, v) if 0 <= v < 1 << 32 else struct.pack("<Iq", 11, v)
    if isinstance(v, float):
        return struct.pack("<If", 6, v)
    return struct.pack("<I", 8) + _string(str(v))


def _bytes_for(kind: str, shape) -> int:
    count = int(np.prod(shape))
    if kind in BLOCK_BYTES:
        return count // 32 * BLOCK_BYTES[kind]
    return count * (4 if kind == "F32" else 2)


def write_gguf(path: str, metadata, tensors) -> None:
    """metadata: (key, value) pairs; tensors: (name, kind, shape outermost
    first, bytes) in file order. Each tensor's data is written as it comes, so
    a model need not be held twice."""
    header = bytearray(struct.pack("<IIQQ", MAGIC, 3, len(tensors), len(metadata)))
    for key, value in metadata:
        header += _string(key) + _value(value)
    offset = 0
    for name, kind, shape, data in tensors:
        if _bytes_for(kind, shape) != np.asarray(data).nbytes:
            raise ValueError(f"{name}: {np.asarray(data).nbytes} bytes for {kind} {shape}")
        header += _string(name) + struct.pack("<I", len(shape))
        for d in reversed(shape):
            header += struct.pack("<Q", d)
        header += struct.pack("<IQ", KINDS[kind], offset)
        offset += (np.asarray(data).nbytes + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT
    header += b"\0" * (-len(header) % ALIGNMENT)
    temp = f"{path}.{os.getpid()}.tmp"
    try:
        with open(temp, "wb") as f:
            f.write(header)
            for _, _, _, data in tensors:
                raw = np.ascontiguousarray(data).view(np.uint8)
                f.write(raw.tobytes())
                f.write(b"\0" * (-raw.nbytes % ALIGNMENT))
        os.replace(temp, path)
    finally:
        if os.path.exists(temp):
            os.remove(temp)


def llama_cpp_order(rows: int, heads: int) -> np.ndarray:
    """For each Hugging Face row i (head h, half j, index t: i = h·w + j·w/2 + t),
    the llama.cpp row it is stored at: h·w + 2t + j (rotary pairs interleaved)."""
    width = rows // heads
    half = width // 2
    i = np.arange(rows)
    h, r = i // width, i % width
    j, t = r // half, r % half
    return h * width + 2 * t + j


def write_llama(path: str, config: dict, weights: dict, norm_kind: str = "F32") -> None:
    """A decoder's weights (embed, head or None when tied, norm, per-layer
    attn_norm, ffn_norm, merged qkv with q/k in Hugging Face order, o, merged
    gate_up, down) as a llama.cpp GGUF with norms as F32, F16 or BF16."""
    c = config
    fmt = c["kind"]
    rb = c["width"] // 32 * BLOCK_BYTES[fmt]
    qn, kvn = c["heads"] * c["head_width"], c["kv_heads"] * c["head_width"]

    def permuted(data, heads):
        rows = np.asarray(data).reshape(-1, rb)
        out = np.empty_like(rows)
        out[llama_cpp_order(rows.shape[0], heads)] = rows
        return out.reshape(-1)

    def norm(v):
        v = np.asarray(v, np.float32)
        if norm_kind == "F16":
            return v.astype(np.float16).view(np.uint8)
        if norm_kind == "BF16":
            return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
        return v.view(np.uint8)

    meta = [("general.architecture", "llama"), ("llama.block_count", c["layers"]),
            ("llama.embedding_length", c["width"]), ("llama.attention.head_count", c["heads"]),
            ("llama.attention.head_count_kv", c["kv_heads"]), ("llama.feed_forward_length", c["hidden"]),
            ("llama.context_length", c["context"]), ("llama.attention.layer_norm_rms_epsilon", float(c["eps"])),
            ("llama.rope.freq_base", float(c["theta"]))]
    W, H = c["width"], c["hidden"]
    tensors = [("token_embd.weight", fmt, [c["vocab"], W], weights["embed"]),
               ("output_norm.weight", norm_kind, [W], norm(weights["norm"]))]
    if weights.get("head") is not None:
        tensors.append(("output.weight", fmt, [c["vocab"], W], weights["head"]))
    for l in range(c["layers"]):
        b = f"blk.{l}."
        qkv = np.asarray(weights["qkv"][l])
        q, k, v = qkv[:qn * rb], qkv[qn * rb:(qn + kvn) * rb], qkv[(qn + kvn) * rb:]
        gu = np.asarray(weights["gate_up"][l])
        tensors += [(b + "attn_norm.weight", norm_kind, [W], norm(weights["attn_norm"][l])),
                    (b + "attn_q.weight", fmt, [qn, W], permuted(q, c["heads"])),
                    (b + "attn_k.weight", fmt, [kvn, W], permuted(k, c["kv_heads"])),
                    (b + "attn_v.weight", fmt, [kvn, W], v),
                    (b + "attn_output.weight", fmt, [W, qn], weights["o"][l]),
                    (b + "ffn_norm.weight", norm_kind, [W], norm(weights["ffn_norm"][l])),
                    (b + "ffn_gate.weight", fmt, [H, W], gu[:gu.size // 2]),
                    (b + "ffn_up.weight", fmt, [H, W], gu[gu.size // 2:]),
                    (b + "ffn_down.weight", fmt, [W, H], weights["down"][l])]
    write_gguf(path, meta, tensors)


def export_configs(directory: str, configs=(1, 2, 3, 4, 5)) -> list:
    """The BASELINE configs' weights as GGUF files in `directory`, the bytes
    bench.py measures: config1.gguf (c_attn Q8_0), config2.gguf (the 121
    SmolLM2-135M products), config3.gguf and config4.gguf (the Q4_1 and Q8_0
    matrices), config5.gguf (the 1.7B-shape Llama, loadable by Llama.load).
    Returns the paths written."""
    import quant_host

    os.makedirs(directory, exist_ok=True)
    out = []

    def path(name):
        out.append(os.path.join(directory, name))
        return out[-1]

    if 1 in configs:
        w = quant_host.synthetic_weights("Q8_0", 2304, 768, seed=0x5EED0001)
        write_gguf(path("config1.gguf"), [("general.name", "config1 c_attn")],
                   [("c_attn.weight", "Q8_0", [2304, 768], w)])
    if 2 in configs:
        shapes = [(f"{name}.{layer}", n, k) for layer in range(30)
                  for name, n, k in (("qkv", 960, 576), ("o", 576, 576), ("gate_up", 3072, 576), ("down", 576, 1536))]
        shapes.append(("head", 49152, 576))
        write_gguf(path("config2.gguf"), [("general.name", "config2 SmolLM2-135M Q4_0 set")],
                   [(name + ".weight", "Q4_0", [n, k], quant_host.synthetic_weights("Q4_0", n, k, seed=0x5EED0002 + i))
                    for i, (name, n, k) in enumerate(shapes)])
    if 3 in configs:
        write_gguf(path("config3.gguf"), [("general.name", "config3 Q4_1")],
                   [(f"w{n}x{k}", "Q4_1", [n, k], quant_host.synthetic_weights("Q4_1", n, k, seed=0x5EED0003 + n))
                    for n, k in ((8192, 2048), (2048, 8192))])
    if 4 in configs:
        write_gguf(path("config4.gguf"), [("general.name", "config4 Q8_0")],
                   [(f"w{n}x2048", "Q8_0", [n, 2048], quant_host.synthetic_weights("Q8_0", n, 2048, seed=0x5EED0004 + n))
                    for n in (2048, 8192)])
    if 5 in configs:
        config = dict(quant_host.SMOLLM2_1P7B)
        write_llama(path("config5.gguf"), config, quant_host.synthetic_llama(config, seed=0x5EED0005))
    return out
