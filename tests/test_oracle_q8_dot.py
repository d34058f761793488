"""Pins the oracle's q8_0 rounding of Q and the q4_0 x q8_0 block dot that
ggml's CPU flash_attn_ext uses for the K side (the mechanism the reference
describes for its quantized mul_mat at tests/kernel_verify.rs:332-361)."""
import numpy as np


def q8_parts(qb):
    qb = qb.reshape(-1, 34)
    d = qb[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    return d, qb[:, 2:].view(np.int8).astype(np.int32)


def test_q8_known_answers(orc):
    x = np.zeros(64, dtype=np.float32)
    x[32:] = np.linspace(-2.0, 1.0, 32)
    d, q = q8_parts(orc.quantize_q8_0(x))
    assert d[0] == 0 and np.all(q[0] == 0)          # zero block
    assert q[1][0] == -127 and q[1][-1] == 64        # amax element -> -127; 1.0 -> 63.5 -> 64 (even)
    assert d[1] == np.float16(2.0 / 127)


def test_q8_variants_differ_only_at_ties(orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4000, 32)).astype(np.float32)
    _, a = q8_parts(orc.quantize_q8_0(x.reshape(-1), orc.Q8_X86))
    _, b = q8_parts(orc.quantize_q8_0(x.reshape(-1), orc.Q8_SCALAR))
    diff = np.abs(a - b)
    assert diff.max() <= 1 and (diff > 0).mean() < 1e-3
    amax = np.abs(x).max(axis=1, keepdims=True)
    assert np.all(np.abs(a - x * 127 / amax) <= 0.5 + 1e-4)


def test_vec_dot_matches_integer_math(orc):
    rng = np.random.default_rng(9)
    for n in (32, 256):
        k = rng.standard_normal(n).astype(np.float32)
        qv = rng.standard_normal(n).astype(np.float32)
        kq = orc.quantize_q4_0(k)
        qq = orc.quantize_q8_0(qv)
        dk = kq.reshape(-1, 18)[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1)
        codes = np.concatenate([kq.reshape(-1, 18)[:, 2:] & 15, kq.reshape(-1, 18)[:, 2:] >> 4], axis=1)
        dq, q8 = q8_parts(qq)
        exact = sum(float(((codes[b].astype(np.int64) - 8) * q8[b]).sum()) * dk[b] * dq[b]
                    for b in range(n // 32))
        got = orc.vec_dot_q4_0_q8_0(kq, qq, n)
        assert abs(got - exact) <= 1e-6 * max(1.0, abs(exact))
