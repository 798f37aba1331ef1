"""Pins the oracle's fp8 e4m3fn and bf16 codecs against torch's own casts (the
conversions the reference harness performs) and against the format definition."""

import numpy as np
import pytest
import torch

from oracle import fp8


def _probe_floats(n=300_000, seed=0):
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    return np.concatenate(
        [
            bits.view(np.float32),
            np.linspace(-600, 600, 120_001, dtype=np.float32),
            (rng.standard_normal(100_000) * 50).astype(np.float32),
            # every e4m3 value, its neighbours and the midpoints between values
            np.nextafter(fp8.E4M3_DECODE[np.isfinite(fp8.E4M3_DECODE)], np.float32(np.inf)),
            np.nextafter(fp8.E4M3_DECODE[np.isfinite(fp8.E4M3_DECODE)], np.float32(-np.inf)),
            fp8.E4M3_DECODE[np.isfinite(fp8.E4M3_DECODE)],
            np.array([0.0, -0.0, 448.0, 464.0, 464.00003, 480.0, np.inf, -np.inf, np.nan, 2**-10, 3 * 2**-11], np.float32),
        ]
    ).astype(np.float32)


def test_e4m3_decode_table_matches_torch():
    t = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(t, fp8.E4M3_DECODE, equal_nan=True)


def test_e4m3_decode_format_points():
    d = fp8.E4M3_DECODE
    assert d[0x7E] == 448.0 and d[0xFE] == -448.0  # largest finite
    assert d[0x08] == 2.0**-6  # smallest normal
    assert d[0x01] == 2.0**-9  # smallest subnormal
    assert d[0x38] == 1.0
    assert np.isnan(d[0x7F]) and np.isnan(d[0xFF])
    assert np.isfinite(d).sum() == 254


def test_e4m3_encode_matches_torch():
    x = _probe_floats()
    ours = fp8.e4m3_encode(x)
    theirs = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    bad = np.nonzero(ours != theirs)[0]
    assert bad.size == 0, (x[bad[:5]], ours[bad[:5]], theirs[bad[:5]])


def test_e4m3_round_trip_and_ties():
    codes = np.arange(256, dtype=np.uint8)
    vals = fp8.E4M3_DECODE[codes]
    fin = np.isfinite(vals)
    back = fp8.e4m3_encode(vals[fin])
    # +0 and -0 both decode to 0; everything else must round-trip exactly
    assert np.array_equal(fp8.E4M3_DECODE[back], vals[fin])
    # ties go to the even code: 1 + 1/16 lies between 1 (0x38) and 1.125 (0x39)
    assert fp8.e4m3_encode(np.array([1.0625], np.float32))[0] == 0x38
    assert fp8.e4m3_encode(np.array([1.1875], np.float32))[0] == 0x3A


def test_bf16_matches_torch():
    x = _probe_floats(seed=1)
    ours = fp8.f32_to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], theirs[~nan])
    # NaN maps to a NaN (payload bits are not part of the contract)
    assert np.all(np.isnan(fp8.bf16_bits_to_f32(ours[nan])))


@pytest.mark.parametrize("v,bits", [(1.0, 0x3F80), (1.00390625, 0x3F80), (1.01171875, 0x3F82), (-2.0, 0xC000)])
def test_bf16_known_points(v, bits):
    assert int(fp8.f32_to_bf16_bits(np.array([v], np.float32))[0]) == bits
