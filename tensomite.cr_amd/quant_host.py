"""Host-side weight quantisation for the HIP device.

`Tensor#quantize` runs on the host even for a GPU device: it reads the values
back, quantises them with `Quant.quantize` and uploads the blocks
(src/tensomite/tensor/quantised.cr:11-19). `quantize` is that host step,
done by the library's native quantiser (tmh_quantize_weights, over all host
cores; quant.cr:77-90, 497-535):

  Q8_0  d = amax / 127; id = 1/d (0 when d is 0); q = round-half-away(x·id)
  Q4_0  m = the first value of largest magnitude; d = m / -8;
        q = min(15, trunc(x·id + 8.5))
  Q4_1  d = (max - min) / 15; q = min(15, trunc((x - min)·id + 0.5))

with d (and min) stored as F16, rounded to nearest even (F16.new, f16.cr:29-41).

`synthetic_weights` and `synthetic_llama` make the BASELINE configs' weights,
W ~ N(0, 0.02) quantised, deterministically from a seed: values come in
fixed chunks, each from its own numpy generator seeded by (seed, chunk), so
the bytes do not depend on how many threads make them.
"""
from __future__ import annotations

import ctypes
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

Q8_0, Q4_0, Q4_1 = 0, 1, 2
KINDS = {"Q8_0": Q8_0, "Q4_0": Q4_0, "Q4_1": Q4_1}
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18, Q4_1: 20}

CHUNK_VALUES = 1 << 22  # values per generator chunk (a whole number of blocks)


def _kind(kind) -> int:
    return KINDS[kind] if isinstance(kind, str) else int(kind)


def _cores() -> int:
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:
        return max(1, os.cpu_count() or 1)


def f16_bits(values: np.ndarray) -> np.ndarray:
    """F16.new(value).bits for an f32 array (f16.cr:29-41)."""
    v = np.asarray(values, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        h = v.astype(np.float16).view(np.uint16)
    nan = np.isnan(v)
    if nan.any():
        sign = (v.view(np.uint32) >> 16).astype(np.uint16) & np.uint16(0x8000)
        h = np.where(nan, sign | np.uint16(0x7E00), h)
    return h


def quantize(kind, values: np.ndarray, threads: int = 0) -> np.ndarray:
    """Quant.quantize: f32 values, a whole number of blocks of 32, to block
    bytes, by the library's host quantiser on `threads` threads (0: all)."""
    import tensomite_hip as th

    k = _kind(kind)
    if k not in BLOCK_BYTES:
        raise th.DTypeError(f"kind {kind} is not a block format")
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    if v.size % 32:
        raise ValueError(f"{v.size} values are not whole blocks of 32")
    out = np.empty(v.size // 32 * BLOCK_BYTES[k], dtype=np.uint8)
    th.check("tmh_quantize_weights", th.library().tmh_quantize_weights(
        k, v.ctypes.data_as(ctypes.c_void_p), v.size, out.ctypes.data_as(ctypes.c_void_p), int(threads)))
    return out


def synthetic_weights(kind, n: int, k: int, seed, std: float = 0.02) -> np.ndarray:
    """W[n, k] ~ N(0, std) in f32, quantised: the BASELINE configs' weights.
    Chunk c of CHUNK_VALUES values comes from default_rng([*seed, c]) as
    standard normals in f32 times f32(std); chunks are made and quantised on
    all host cores."""
    kk = _kind(kind)
    bb = BLOCK_BYTES[kk]
    total = n * k
    if total % 32:
        raise ValueError(f"{n} x {k} values are not whole blocks of 32")
    entropy = list(seed) if isinstance(seed, (list, tuple)) else [int(seed)]
    out = np.empty(total // 32 * bb, dtype=np.uint8)
    scale = np.float32(std)

    def chunk(c):
        lo = c * CHUNK_VALUES
        hi = min(total, lo + CHUNK_VALUES)
        v = np.random.default_rng(entropy + [c]).standard_normal(hi - lo, dtype=np.float32)
        v *= scale
        out[lo // 32 * bb:hi // 32 * bb] = quantize(kk, v, threads=1)

    chunks = (total + CHUNK_VALUES - 1) // CHUNK_VALUES
    with ThreadPoolExecutor(max_workers=min(_cores(), chunks)) as pool:
        list(pool.map(chunk, range(chunks)))
    return out


def synthetic_llama(config: dict, seed: int, std: float = 0.02) -> dict:
    """BASELINE config 5's weights at `config`'s shape: every matrix and the
    embedding table (the tied head) W ~ N(0, std) quantised to config["kind"],
    the RMSNorm weights 1 (Llama's initial norms), in the decoder's layout
    (embed, head None, norm, per-layer attn_norm, ffn_norm, merged qkv, o,
    merged gate_up, down). Matrix m of layer l comes from seed [seed, l, m]."""
    c = config
    fmt = c["kind"]
    qn, kvn = c["heads"] * c["head_width"], c["kv_heads"] * c["head_width"]
    ones = np.ones(c["width"], np.float32)
    w = dict(embed=synthetic_weights(fmt, c["vocab"], c["width"], [seed, 1 << 20, 0], std), head=None,
             norm=ones.copy(), attn_norm=[], ffn_norm=[], qkv=[], o=[], gate_up=[], down=[])
    for layer in range(c["layers"]):
        w["qkv"].append(synthetic_weights(fmt, qn + 2 * kvn, c["width"], [seed, layer, 0], std))
        w["o"].append(synthetic_weights(fmt, c["width"], qn, [seed, layer, 1], std))
        w["gate_up"].append(synthetic_weights(fmt, 2 * c["hidden"], c["width"], [seed, layer, 2], std))
        w["down"].append(synthetic_weights(fmt, c["width"], c["hidden"], [seed, layer, 3], std))
        w["attn_norm"].append(ones.copy())
        w["ffn_norm"].append(ones.copy())
    return w


def random_blocks(fmt: str, n: int, k: int, rng, std: float = 0.02) -> np.ndarray:
    """[n, k] weights as random block bytes: uniform quants with F16 scales
    (and Q4_1 minimums) drawn so the values have about `std` spread. Valid
    blocks of the format, made without a float pass, for model-sized tests."""
    bb = {"Q8_0": 34, "Q4_0": 18, "Q4_1": 20}[fmt]
    blocks = n * k // 32
    data = np.frombuffer(rng.bytes(blocks * bb), np.uint8).copy().reshape(blocks, bb)
    # centre the quants (no shared offset in every dot product)
    if fmt == "Q8_0":
        q = data[:, 2:]
        q[q == 0x80] = 0
    elif fmt == "Q4_0":
        q = data[:, 2:]
        lo, hi = q & 15, q >> 4
        q[...] = np.where(lo == 0, 8, lo) | (np.where(hi == 0, 8, hi) << 4)
    spread = {"Q8_0": 73.9, "Q4_0": 4.6, "Q4_1": 4.6}[fmt]
    d = (rng.uniform(0.5, 1.5, blocks) * std / spread).astype(np.float16)
    data[:, 0:2] = d.view(np.uint8).reshape(blocks, 2)
    if fmt == "Q4_1":
        m = (-7.5 * d.astype(np.float32)).astype(np.float16)
        data[:, 2:4] = m.view(np.uint8).reshape(blocks, 2)
    return data.reshape(-1)


def random_block_llama(config: dict, seed: int, norm_jitter: float = 0.05, std: float = 0.05,
                       embed_std: float = 0.02):
    """A Llama of `config`'s shape (tied head) with random_blocks matrices and
    jittered RMSNorm weights, as a dict of the decoder's weight layout (embed,
    head None, norm, per-layer attn_norm, ffn_norm, merged qkv, o, merged
    gate_up, down); quick to make at the 1.7B shape.
    The default spreads make layers matter against the embedding, so greedy
    tokens vary from step to step."""
    c = config
    fmt = c["kind"]
    rng = np.random.default_rng(seed)
    qn, kvn = c["heads"] * c["head_width"], c["kv_heads"] * c["head_width"]

    def norm():
        return (1.0 + rng.normal(0, norm_jitter, c["width"])).astype(np.float32)

    w = dict(embed=random_blocks(fmt, c["vocab"], c["width"], rng, std=embed_std), head=None, norm=norm(),
             attn_norm=[], ffn_norm=[], qkv=[], o=[], gate_up=[], down=[])
    for _ in range(c["layers"]):
        w["qkv"].append(random_blocks(fmt, qn + 2 * kvn, c["width"], rng, std))
        w["o"].append(random_blocks(fmt, c["width"], qn, rng, std))
        w["gate_up"].append(random_blocks(fmt, 2 * c["hidden"], c["width"], rng, std))
        w["down"].append(random_blocks(fmt, c["width"], c["hidden"], rng, std))
        w["attn_norm"].append(norm())
        w["ffn_norm"].append(norm())
    return w


# SmolLM2-1.7B's shape (Llama, tied head), in the decoder's config keys.
SMOLLM2_1P7B = dict(layers=24, width=2048, heads=32, kv_heads=32, head_width=64, hidden=8192, vocab=49152,
                    context=2048, eps=1e-5, theta=10000.0, kind="Q4_0")
