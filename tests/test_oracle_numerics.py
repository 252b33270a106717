"""Pins the oracle's number formats against torch's CPU casts and known answers."""
import numpy as np
import pytest
import torch

from oracle.numerics import bf16_round, e4m3_decode, e4m3_encode


def _torch_e4m3(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _structured_values():
    vals = []
    codes = np.arange(256, dtype=np.uint8)
    dec = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    dec = dec[np.isfinite(dec)]
    srt = np.unique(dec)
    mids = (srt[1:].astype(np.float64) + srt[:-1]) / 2
    for v in np.concatenate([srt.astype(np.float64), mids]):
        f = np.float32(v)
        vals += [f, np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))]
    return np.array(vals, np.float32)


def test_e4m3_known_answers():
    # round-to-nearest-even known answers (ties go to the even mantissa)
    cases = {1.0625: 0x38, 1.1875: 0x3A, 0.0087890625: 0x04, 447.9: 0x7E, 448.0: 0x7E,
             -448.0: 0xFE, 1.0: 0x38, 2.0 ** -6: 0x08, 2.0 ** -9: 0x01, 2.0 ** -10: 0x00,
             0.0: 0x00}
    for x, code in cases.items():
        assert int(e4m3_encode(np.float32(x))) == code, x
    assert int(e4m3_encode(np.float32(-0.0))) == 0x80


def test_e4m3_encode_matches_torch_structured():
    x = _structured_values()
    x = x[np.abs(x) <= 448]
    np.testing.assert_array_equal(e4m3_encode(x), _torch_e4m3(x))


def test_e4m3_encode_matches_torch_random():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.uniform(-448, 448, 200000),
        rng.standard_normal(200000) * np.exp2(rng.integers(-14, 8, 200000)),
    ]).astype(np.float32)
    np.testing.assert_array_equal(e4m3_encode(x), _torch_e4m3(x))


def test_e4m3_overflow_to_nan_like_torch():
    x = np.array([464.0, 464.00003, 470.0, 1e6, -500.0], np.float32)
    np.testing.assert_array_equal(e4m3_encode(x), _torch_e4m3(x))


def test_e4m3_decode_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = e4m3_decode(codes)
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(got[fin], ref[fin])
    assert np.all(np.isnan(got[~fin]))


def test_e4m3_roundtrip_exact():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    np.testing.assert_array_equal(e4m3_encode(e4m3_decode(codes)), codes)


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32),
        (rng.standard_normal(100000) * 1e30).astype(np.float32),
        np.array([1.00390625, 1.01171875, -1.00390625, 0.0, -0.0], np.float32),  # exact ties
    ])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(bf16_round(x), ref)
