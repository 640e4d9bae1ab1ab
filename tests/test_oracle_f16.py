"""The oracle's F16 conversions (src/tensomite/f16.cr:29-57), pinned by the
reference's spec (spec/f16_spec.cr) and by numpy's IEEE half conversion."""
import numpy as np

from oracle import oracle


def all_halves():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    widened = oracle.f16_values_many(bits)
    return bits, widened


def test_widens_every_half_to_its_value():
    # f16_spec.cr:12-23: the value the bits define, exactly; NaN payloads kept.
    bits, widened = all_halves()
    sign = np.where(bits >> 15 == 1, -1.0, 1.0)
    exponent = (bits.astype(np.int64) >> 10) & 0x1F
    fraction = bits.astype(np.int64) & 0x3FF
    for e in range(32):
        sel = exponent == e
        got = widened[sel].astype(np.float64)
        if e == 0:
            want = sign[sel] * fraction[sel] * 2.0 ** -24
            assert np.array_equal(got, want)
            assert np.array_equal(np.signbit(widened[sel]), bits[sel] >> 15 == 1)
        elif e == 31:
            words = widened[sel].view(np.uint32)
            want = ((bits[sel].astype(np.uint32) & 0x8000) << 16) | 0x7F800000 | (fraction[sel].astype(np.uint32) << 13)
            assert np.array_equal(words, want)
        else:
            want = sign[sel] * (1 + fraction[sel] / 1024) * 2.0 ** (e - 15)
            assert np.array_equal(got, want)
    # and numpy's own widening agrees wherever it is not a NaN
    ok = ~np.isnan(widened)
    assert np.array_equal(widened[ok].view(np.uint32), bits.view(np.float16)[ok].astype(np.float32).view(np.uint32))


def test_round_trips_every_half_that_is_not_a_nan():
    # f16_spec.cr:4-10
    bits, widened = all_halves()
    ok = ~np.isnan(widened)
    back = oracle.f16_bits_many(widened[ok])
    assert np.array_equal(back, bits[ok])


def test_known_values():
    # f16_spec.cr:25-42
    assert oracle.f16_bits(1.0) == 0x3C00
    assert oracle.f16_bits(-2.0) == 0xC000
    assert oracle.f16_bits(65504.0) == 0x7BFF
    assert np.float32(oracle.f16_value(0x0001)) == np.float32(5.9604645e-8)
    assert np.float32(oracle.f16_value(0x03FF)) == np.float32(6.097555e-5)
    assert oracle.f16_bits(1.00048828125) == 0x3C00
    assert oracle.f16_bits(1.00146484375) == 0x3C02
    assert oracle.f16_bits(65519.0) == 0x7BFF
    assert oracle.f16_bits(65520.0) == 0x7C00
    assert oracle.f16_bits(np.float32(2.9802322e-8)) == 0x0000
    assert oracle.f16_bits(np.float32(8.940697e-8)) == 0x0002
    assert np.isnan(oracle.f16_value(oracle.f16_bits(float("nan"))))
    assert oracle.f16_bits(float("nan")) == 0x7E00
    assert oracle.f16_bits(float("-inf")) == 0xFC00


def test_rounds_as_ieee_for_every_exponent():
    # f32 -> f16 against numpy's IEEE round-to-nearest-even conversion, for
    # every sign and exponent: all 2^13 patterns of the 13 bits rounding drops
    # (where ties and carries live), under several upper fractions, plus
    # random words. NaNs are left out: the reference makes every NaN 0x7e00.
    rng = np.random.default_rng(1)
    low = np.arange(1 << 13, dtype=np.uint32)
    uppers = np.array([0, 1, 0x1FF, 0x200, 0x3FE, 0x3FF], dtype=np.uint32)
    words = []
    for se in range(512):
        head = np.uint32(se) << np.uint32(23)
        for up in uppers:
            words.append(head | (up << np.uint32(13)) | low)
        words.append(head | rng.integers(0, 1 << 23, 4096, dtype=np.uint32))
    words = np.concatenate(words)
    values = words.view(np.float32)
    values = values[~np.isnan(values)]
    got = oracle.f16_bits_many(values)
    want = values.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
