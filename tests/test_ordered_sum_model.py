"""A CPU model of the device's speculative ordered sum (ordered_sum_wave in
tensomite.cr_amd/csrc/tmh_device.h), checked against the sequential f32
fold it must reproduce bit for bit.

The device folds n values (RMSNorm's squares, attention's weights) as 64
chunks, one per lane of a wave: each lane folds its chunk in order from a
guessed start; when every start equals the previous lane's end the result
is the sequential fold's (induction from lane 0, which starts at +0.0);
otherwise starts are re-guessed from the previous end plus a prefix sum
(in the DPP tree order: row_shr 1/2/4/8, row_bcast 15/31) of the
mismatches. The first mismatching lane always gets its predecessor's end
unchanged, so 64 passes bound the loop.

The model uses the same steps in float32 numpy (IEEE round-to-nearest
adds, one rounding each), vectorised over many inputs, so a flaw in the
scheme -- a wrong correction, a lost lane, a pass bound that can be hit --
shows here without a GPU. The reference for each input is
np.add.accumulate in float32: a strictly sequential left-to-right fold,
the host's `sum += v` loop (host.cr:374-386 for RMSNorm's squares).
"""
import numpy as np
import pytest

LANES = 64


def dpp_prefix(x):
    """Inclusive prefix sum over the lane axis in the device's DPP order."""
    x = x.copy()
    lane = np.arange(LANES)
    for sh in (1, 2, 4, 8):
        src = np.zeros_like(x)
        ok = (lane % 16) >= sh
        src[..., ok] = x[..., lane[ok] - sh]
        x = x + src
    src = np.zeros_like(x)
    rows13 = (lane // 16 == 1) | (lane // 16 == 3)
    src[..., rows13] = x[..., (lane[rows13] // 16) * 16 - 1]
    x = x + src
    src = np.zeros_like(x)
    rows23 = lane // 16 >= 2
    src[..., rows23] = x[..., [31]]
    return x + src


def shift_up(x):
    out = np.zeros_like(x)
    out[..., 1:] = x[..., :-1]
    return out


def speculative_sum(v):
    """v: [T, n] float32 -> (sums [T], passes [T]) by the device's scheme."""
    t, n = v.shape
    m = -(-n // LANES)
    chunks = np.zeros((t, LANES * m), np.float32)
    chunks[:, :n] = v
    chunks = chunks.reshape(t, LANES, m)
    start = np.zeros((t, LANES), np.float32)
    end = np.zeros((t, LANES), np.float32)
    done = np.zeros(t, bool)
    passes = np.zeros(t, np.int32)
    lane0 = np.arange(LANES) == 0
    for p in range(LANES + 1):
        e = start.copy()
        with np.errstate(invalid="ignore", over="ignore"):
            for i in range(m):
                e = e + chunks[:, :, i]
        prev = shift_up(e)
        ok = lane0 | (prev.view(np.uint32) == start.view(np.uint32))
        now = ~done & ok.all(axis=1)
        end[now] = e[now]
        passes[now] = p + 1
        done |= now
        if done.all():
            break
        with np.errstate(invalid="ignore", over="ignore"):
            miss = np.where(ok, np.float32(0), prev - start).astype(np.float32)
            before = shift_up(dpp_prefix(miss))
            guess = np.where(before == 0, prev, prev + before).astype(np.float32)
        start = np.where(lane0, np.float32(0), guess).astype(np.float32)
    assert done.all(), "the pass bound was reached"
    return end[:, -1], passes


def rows(rng, t, n):
    out = np.empty((t, n), np.float32)
    for r in range(t):
        kind = r % 7
        if kind == 0:
            x = rng.normal(0, 1, n)
        elif kind == 1:
            x = rng.normal(0, 1, n) * 2.0 ** rng.uniform(-10, 10)
        elif kind == 2:
            x = np.where(rng.random(n) < 0.01, rng.normal(0, 100, n), rng.normal(0, 0.01, n))
        elif kind == 3:
            x = np.trunc(rng.normal(0, 8, n))        # small integers: exact ties
        elif kind == 4:
            x = rng.choice([-1.0, 1.0], n) * 2.0 ** rng.uniform(-40, 40, n)
        elif kind == 5:
            x = np.sort(np.abs(rng.normal(0, 1, n)) * 2.0 ** rng.uniform(-8, 8, n))
        else:
            x = rng.normal(0, 1, n) * np.exp(-np.arange(n) / 200.0)
        out[r] = x.astype(np.float32)
    return out * out  # squares, each rounded to f32 as the device squares them


@pytest.mark.parametrize("n,trials", [(2048, 700), (576, 700), (100, 700), (8192, 140), (1000, 350)])
def test_speculative_sum_equals_sequential_fold(n, trials):
    rng = np.random.default_rng(n)
    v = rows(rng, trials, n)
    got, passes = speculative_sum(v)
    want = np.add.accumulate(v, axis=1, dtype=np.float32)[:, -1]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert passes.max() <= LANES + 1


def test_speculative_sum_signed_values_and_specials():
    # the scheme does not rely on the values' signs; NaN and inf runs too
    rng = np.random.default_rng(7)
    v = rng.normal(0, 1, (500, 2048)).astype(np.float32)
    v[1, 77] = np.nan
    v[2, 1000] = np.inf
    v[3, 5] = -np.inf
    v[3, 6] = np.inf
    got, _ = speculative_sum(v)
    with np.errstate(invalid="ignore"):
        want = np.add.accumulate(v, axis=1, dtype=np.float32)[:, -1]
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()
