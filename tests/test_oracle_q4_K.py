"""The oracle's Q4_K dequantizer and W_o projection (reference: the W_o
mul_mat of src/model/attn.rs:285 over attn_output.weight, src/model/weights.rs:438;
Q4_K is the model's main weight type, tests/kernel_verify.rs:553-557).

The reference holds no Q4_K vectors (its test quantizes through the ggml
library at run time), so the dequantizer is pinned by constructed blocks:
every one of the 96 scale bits is set alone and the (scale, min) it moves is
read back through the values; distinct sub-block scales show which values each
sub-block owns. The projection is pinned by a plain triple loop on small sizes
and by the pinned sigmoid_mul for the gate."""
import numpy as np
import pytest

pytestmark = pytest.mark.filterwarnings("ignore")

K1 = 256


def _block(d, dmin, scales12, qs128):
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    b[4:16] = scales12
    b[16:144] = qs128
    return b


def _field_of_bit(byte, bit):
    """ggml's documented packing of the 12 scale bytes: which sub-block field
    (scale 'sc' or min 'm') and which bit of that 6-bit field a scale bit feeds."""
    if byte < 4:
        return ("sc", byte, bit) if bit < 6 else ("sc", byte + 4, bit - 2)
    if byte < 8:
        return ("m", byte - 4, bit) if bit < 6 else ("m", byte, bit - 2)
    return ("sc", byte - 4, bit) if bit < 4 else ("m", byte - 4, bit - 4)


def test_every_scale_bit_lands_in_its_documented_field(orc):
    ones = np.full(128, 0x11, np.uint8)  # every code is 1
    for byte in range(12):
        for bit in range(8):
            sc = np.zeros(12, np.uint8)
            sc[byte] = 1 << bit
            # d = 1, dmin = 0: value = scale of its sub-block; d = 0, dmin = 1: value = -min
            vs = orc.dequantize_q4_K(_block(1.0, 0.0, sc, ones), K1)[0].reshape(8, 32)
            vm = -orc.dequantize_q4_K(_block(0.0, 1.0, sc, ones), K1)[0].reshape(8, 32)
            field, sub, fbit = _field_of_bit(byte, bit)
            want_s = np.zeros(8)
            want_m = np.zeros(8)
            (want_s if field == "sc" else want_m)[sub] = 1 << fbit
            assert np.array_equal(vs, np.repeat(want_s[:, None], 32, 1)), (byte, bit)
            assert np.array_equal(vm, np.repeat(want_m[:, None], 32, 1)), (byte, bit)


def test_code_nibbles_feed_values_in_group_order(orc):
    # sub-block s gets scale s + 1 (s < 4 use the low 6 bits of bytes 0-3; s >= 4
    # the low nibbles of bytes 8-11), min 0, so value / (s + 1) is the code
    sc = np.zeros(12, np.uint8)
    for s in range(4):
        sc[s] = s + 1
        sc[8 + s] = s + 5
    rng = np.random.default_rng(4)
    qs = rng.integers(0, 256, 128, dtype=np.uint8)
    v = orc.dequantize_q4_K(_block(1.0, 0.0, sc, qs), K1)[0]
    codes = np.rint(v.reshape(8, 32) / np.arange(1, 9)[:, None]).astype(int)
    assert np.allclose(codes * np.arange(1, 9)[:, None], v.reshape(8, 32))
    for j in range(4):  # 32-byte group j feeds sub-blocks 2j (low nibbles) and 2j + 1 (high)
        assert np.array_equal(codes[2 * j], qs[32 * j:32 * j + 32] & 15)
        assert np.array_equal(codes[2 * j + 1], qs[32 * j:32 * j + 32] >> 4)


def test_scales_times_codes_minus_mins(orc):
    sc = np.zeros(12, np.uint8)
    sc[0:4] = [3, 63, 17, 40]
    sc[4:8] = [5, 0, 63, 9]
    qs = np.full(128, 0xF7, np.uint8)  # low code 7, high code 15
    v = orc.dequantize_q4_K(_block(0.5, 0.25, sc, qs), K1)[0].reshape(8, 32)
    # sub-blocks 0, 2 take the low code 7, sub-blocks 1, 3 the high code 15
    assert np.all(v[0] == np.float32(0.5 * 3 * 7 - 0.25 * 5))
    assert np.all(v[1] == np.float32(0.5 * 63 * 15 - 0.25 * 0))
    assert np.all(v[2] == np.float32(0.5 * 17 * 7 - 0.25 * 63))
    assert np.all(v[3] == np.float32(0.5 * 40 * 15 - 0.25 * 9))


def _random_q4k(rng, n, k):
    w = rng.integers(0, 256, (n, k // 256 * 144), dtype=np.uint8)
    for r in range(n):
        for b in range(k // 256):
            w[r, 144 * b:144 * b + 2] = np.frombuffer(np.float16(rng.uniform(1e-3, 2e-2)).tobytes(), np.uint8)
            w[r, 144 * b + 2:144 * b + 4] = np.frombuffer(np.float16(rng.uniform(0, 1e-2)).tobytes(), np.uint8)
    return w


def test_out_proj_matches_a_plain_loop(orc):
    rng = np.random.default_rng(5)
    N, K, M = 3, 512, 2
    w = _random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    wd = orc.dequantize_q4_K(w, K)
    want = np.zeros((M, N))
    for t in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                acc += float(wd[n, k]) * float(x[t, k])
            want[t, n] = acc
    got = orc.out_proj(w, x)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)


def test_out_proj_gate_is_the_pinned_sigmoid_mul(orc):
    rng = np.random.default_rng(6)
    N, K, M = 4, 256, 3
    w = _random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    g = rng.standard_normal((M, K)).astype(np.float32)
    gated = orc.sigmoid_mul(x, g)
    assert np.array_equal(orc.out_proj(w, x, g), orc.out_proj(w, gated))
