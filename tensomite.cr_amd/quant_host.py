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
