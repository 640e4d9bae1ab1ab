"""Host-side weight quantisation for the HIP device, vectorised with numpy.

`Tensor#quantize` runs on the host even for a GPU device: it reads the values
back, quantises them with `Quant.quantize` and uploads the blocks
(src/tensomite/tensor/quantised.cr:11-19). This is that host step, whole
matrices at a time: the bytes equal `Quant.quantize`'s (quant.cr:77-90,
497-535) for every finite input, because every step is one IEEE f32
operation in the reference's order:

  Q8_0  d = amax / 127; id = 1/d (0 when d is 0); q = round-half-away(x·id)
  Q4_0  m = the first value of largest magnitude; d = m / -8;
        q = min(15, trunc(x·id + 8.5))
  Q4_1  d = (max - min) / 15; q = min(15, trunc((x - min)·id + 0.5))

and d (and min) are stored as F16, rounded to nearest even (numpy's f32 ->
f16 conversion is IEEE's; a NaN is stored as 0x7e00 with its sign, as
F16.new does, f16.cr:33-35).
"""
from __future__ import annotations

import numpy as np

Q8_0, Q4_0, Q4_1 = 0, 1, 2
KINDS = {"Q8_0": Q8_0, "Q4_0": Q4_0, "Q4_1": Q4_1}
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18, Q4_1: 20}


def _kind(kind) -> int:
    return KINDS[kind] if isinstance(kind, str) else int(kind)


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


def _round_away(v: np.ndarray) -> np.ndarray:
    """round(:ties_away) for |v| < 2^31 (quant.cr:309-313): truncate, then step
    away from zero when the dropped fraction is at least a half."""
    whole = np.trunc(v)
    fraction = v - whole
    return whole + (fraction >= np.float32(0.5)) - (fraction <= np.float32(-0.5))


def quantize(kind, values: np.ndarray) -> np.ndarray:
    """Quant.quantize: f32 values, a whole number of blocks of 32, to block bytes."""
    k = _kind(kind)
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    if v.size % 32:
        raise ValueError(f"{v.size} values are not whole blocks of 32")
    blocks = v.reshape(-1, 32)
    nb = blocks.shape[0]
    out = np.empty((nb, BLOCK_BYTES[k]), dtype=np.uint8)
    f32 = np.float32
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        if k == Q8_0:
            amax = np.abs(blocks).max(axis=1)
            d = amax / f32(127.0)
            idv = np.where(d == 0, f32(0.0), f32(1.0) / d).astype(np.float32)
            q = _round_away(blocks * idv[:, None]).astype(np.int32).astype(np.int8)
            out[:, 0:2] = f16_bits(d).view(np.uint8).reshape(nb, 2)
            out[:, 2:] = q.view(np.uint8)
        elif k == Q4_0:
            first = np.argmax(np.abs(blocks), axis=1)  # first index of the largest magnitude
            m = blocks[np.arange(nb), first]
            d = m / f32(-8.0)
            idv = np.where(d == 0, f32(0.0), f32(1.0) / d).astype(np.float32)
            t = (blocks * idv[:, None]) + f32(8.5)
            q = np.minimum(np.trunc(t).astype(np.int32).astype(np.int8), 15).astype(np.uint8)
            out[:, 0:2] = f16_bits(d).view(np.uint8).reshape(nb, 2)
            out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
        elif k == Q4_1:
            mn = blocks.min(axis=1)
            mx = blocks.max(axis=1)
            # Enumerable#min keeps the first of equal values: for a zero
            # minimum, the sign is the first zero's.
            zero = mn == 0
            if zero.any():
                rows = np.nonzero(zero)[0]
                mn[rows] = blocks[rows, np.argmax(blocks[rows] == 0, axis=1)]
            d = (mx - mn) / f32(15.0)
            idv = np.where(d == 0, f32(0.0), f32(1.0) / d).astype(np.float32)
            t = ((blocks - mn[:, None]) * idv[:, None]) + f32(0.5)
            q = np.minimum(np.trunc(t).astype(np.int32).astype(np.int8), 15).astype(np.uint8)
            out[:, 0:2] = f16_bits(d).view(np.uint8).reshape(nb, 2)
            out[:, 2:4] = f16_bits(mn).view(np.uint8).reshape(nb, 2)
            out[:, 4:] = q[:, :16] | (q[:, 16:] << 4)
        else:
            raise ValueError(f"kind {kind} is not a block format")
    return out.reshape(-1)


def synthetic_weights(kind, n: int, k: int, seed: int, std: float = 0.02, chunk_rows: int = 4096) -> np.ndarray:
    """W[n, k] ~ N(0, std) in f32, quantised: the BASELINE configs' weights,
    generated and quantised in row chunks to bound host memory."""
    rng = np.random.default_rng(seed)
    parts = []
    for r0 in range(0, n, chunk_rows):
        rows = min(chunk_rows, n - r0)
        parts.append(quantize(kind, rng.normal(0.0, std, rows * k).astype(np.float32)))
    return np.concatenate(parts)


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
