"""Pins torch's float8_e4m3fn conversion (used by every oracle function) with an
independent codec written from the format definition (oracle/e4m3.py)."""

import numpy as np
import torch

from oracle import e4m3


def _torch_codes(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_table_known_values():
    t = e4m3.decode_table()
    assert t[0x00] == 0.0 and t[0x80] == 0.0
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0
    assert t[0x01] == 2.0 ** -9  # smallest subnormal
    assert t[0x08] == 2.0 ** -6  # smallest normal
    assert t[0x38] == 1.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    # torch decodes every code to the same value
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    tv = codes.view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(np.isnan(tv), np.isnan(t))
    np.testing.assert_array_equal(tv[~np.isnan(tv)], t[~np.isnan(t)])


def test_known_answers():
    vals = np.array([448.0, 460.0, 464.0, 465.0, 480.0, 1e9, np.inf, np.nan, -465.0, 2 ** -9,
                     2 ** -10, 1.5 * 2 ** -10, 1.0, -0.0, 1.0625, 1.1875], dtype=np.float32)
    want = [0x7E, 0x7E, 0x7E, 0x7F, 0x7F, 0x7F, 0x7F, 0x7F, 0xFF, 0x01, 0x00, 0x01, 0x38, 0x80,
            0x38, 0x3A]
    assert e4m3.encode(vals).tolist() == want
    assert _torch_codes(torch.from_numpy(vals)).tolist() == want


def test_every_bf16_pattern_matches_torch():
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    x = bits.view(torch.bfloat16)
    ours = e4m3.encode(x.float().numpy())
    np.testing.assert_array_equal(ours, _torch_codes(x))


def test_random_fp32_and_ties_match_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(1_000_000).astype(np.float32) * 50,
        (rng.standard_normal(200_000) * 2.0 ** -8).astype(np.float32),  # subnormal range
        # exact midpoints between adjacent e4m3 values (ties to even)
        ((e4m3.decode_table()[1:0x7E] + e4m3.decode_table()[2:0x7F]) / 2).astype(np.float32),
        np.float32(np.nextafter(np.float32(464.0), np.float32(0))).reshape(1),
        np.float32(np.nextafter(np.float32(464.0), np.float32(1e9))).reshape(1),
    ])
    np.testing.assert_array_equal(e4m3.encode(x), _torch_codes(torch.from_numpy(x)))
