"""Pins the oracle's fp16 conversions: fp16 -> fp32 over all 65536 bit patterns
and fp32 -> fp16 (round-to-nearest-even) against numpy's IEEE conversions.
ggml stores every q4_0/q8_0 scale through this conversion (f16_to_f32 of
tests/kernel_verify.rs:253-268 in the reference)."""
import numpy as np


def test_fp16_to_fp32_all_patterns(orc):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = orc.fp16_bits_to_fp32(bits)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))


def test_fp32_to_fp16_rne(orc):
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 5, 20000),
        # every fp16 value, its midpoints to the next value and a hair either side
        (np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float64)),
    ]).astype(np.float64)
    h = np.arange(0, 0x7bff, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (h + np.arange(1, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float64)) / 2
    x = np.concatenate([x, mids, np.nextafter(mids, 0), np.nextafter(mids, 1e9), -mids,
                        [0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -25, 2.0 ** -24,
                         3 * 2.0 ** -26, 2.0 ** -14, 1e-40]])
    x = x.astype(np.float32)
    want = x.astype(np.float16).view(np.uint16)
    got = orc.fp32_to_fp16_bits(x)
    assert np.array_equal(got, want)
