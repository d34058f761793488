"""Pins the oracle's q4_0 quantizer (ggml quantize_row_q4_0_ref, which the
reference's tests call through ggml_quantize_chunk, tests/attn_test.rs:210-229)
and its dequantizer (tests/kernel_verify.rs:270-292)."""
import numpy as np
import pytest

from tests.q4_ref import pack_blocks, quantize_blocks_np


def block_bytes(orc, x):
    return orc.quantize_q4_0(np.asarray(x, dtype=np.float32).reshape(1, 32))[0]


def test_zero_block_kat(orc):
    # max = +0.0 so d = 0/-8 = -0.0: fp16 0x8000; id = 0 so every code is 8.
    got = block_bytes(orc, np.zeros(32))
    assert list(got[:2]) == [0x00, 0x80]
    assert all(b == 0x88 for b in got[2:])


def test_ramp_block_kat(orc):
    # x_j = j - 16: max = -16 (j=0), d = 2.0 (fp16 0x4000), id = 0.5,
    # code_j = trunc(j/2 + 0.5), clamped to 15 at j = 31.
    got = block_bytes(orc, np.arange(32) - 16)
    codes = [min(15, (j + 1) // 2) for j in range(32)]
    assert list(got[:2]) == [0x00, 0x40]
    assert list(got[2:]) == [codes[j] | (codes[j + 16] << 4) for j in range(16)]


@pytest.mark.parametrize("first_pos,first_sign", [(5, 1.0), (3, -1.0)])
def test_signed_max_first_occurrence_kat(orc, first_pos, first_sign):
    # Two elements of magnitude 3 with opposite signs: the FIRST one sets max.
    x = np.ones(32, dtype=np.float32)
    other = 9
    x[first_pos] = 3.0 * first_sign
    x[other] = -3.0 * first_sign
    got = block_bytes(orc, x)
    codes = np.zeros(32, dtype=np.int32)
    for j in range(32):
        codes[j] = (got[2 + j] & 15) if j < 16 else (got[2 + j - 16] >> 4)
    d = np.frombuffer(got[:2].tobytes(), dtype=np.float16)[0]
    assert d == np.float16(-0.375 * first_sign)
    assert codes[first_pos] == 0       # x = max maps to -8
    assert codes[other] == 15          # x = -max maps to +8, clamped to 7
    rest = 5 if first_sign > 0 else 11  # 1 * (-8/3) + 8.5 -> 5 ; 1 * (8/3) + 8.5 -> 11
    assert all(codes[j] == rest for j in range(32) if j not in (first_pos, other))


def test_reference_roundtrip_invariants(orc):
    # attn_test.rs:790-833: every value lands within one grid step |d| of x,
    # and the mean error sits near half a step.
    rng = np.random.default_rng(7)
    data = (rng.standard_normal(32 * 8) * 0.5).astype(np.float32)
    deq = orc.dequantize_q4_0(orc.quantize_q4_0(data), 32 * 8)
    worst, tot, n = 0.0, 0.0, 0
    for b in range(8):
        blk, dq = data[32 * b:32 * b + 32], deq[32 * b:32 * b + 32]
        d = np.abs(dq).max() / 8
        e = np.abs(dq - blk) / d
        worst, tot, n = max(worst, e.max()), tot + e.sum(), n + 32
    assert worst <= 1 + 1e-3
    assert 0.1 < tot / n < 0.4


def test_random_blocks_match_numpy_restatement(orc):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((20000, 32)).astype(np.float32)
    x[::7] *= np.float32(1e-3)
    x[::11] *= np.float32(300.0)
    x[5::13, 4] = x[5::13, 20] = 2.5  # ties in |x|
    x[6::13, 4] = 2.5
    x[6::13, 20] = -2.5
    x[::17] = np.round(x[::17] * 4) / 4  # values on binary grid points: exact products
    want = pack_blocks(*quantize_blocks_np(x))
    got = orc.quantize_q4_0(x.reshape(-1)).reshape(-1, 18)
    assert np.array_equal(got, want)


def test_dequant_formula_and_bounds(orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((500, 32)).astype(np.float32)
    q = orc.quantize_q4_0(x.reshape(-1)).reshape(-1, 18)
    deq = orc.dequantize_q4_0(q.reshape(-1), x.size).reshape(-1, 32)
    d = q[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    codes = np.concatenate([q[:, 2:] & 15, q[:, 2:] >> 4], axis=1).astype(np.int32)
    assert codes.min() >= 0 and codes.max() <= 15
    assert np.array_equal(deq, ((codes - 8) * d[:, None]).astype(np.float32))
    # the element of largest magnitude always gets code 0 (x = max -> x/d = -8)
    assert np.all(codes[np.arange(500), np.abs(x).argmax(axis=1)] == 0)
