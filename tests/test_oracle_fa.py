"""Pins the oracle's flash_attn_ext (ggml CPU one-chunk online softmax) against
float64 brute force and against special cases with closed-form answers."""
import numpy as np
import pytest

from tests.fa_ref import attention_f64, cache_dequant, q8_dequant, rel_err


def make(orc, rng, n_q, H, Hkv, n_kv, D=256, outliers=0):
    q = rng.standard_normal((n_q, H, D)).astype(np.float32)
    k = rng.standard_normal((n_kv, Hkv * D)).astype(np.float32)
    v = rng.standard_normal((n_kv, Hkv * D)).astype(np.float32)
    if outliers:
        ch = rng.choice(Hkv * D, outliers, replace=False)
        k[:, ch] *= 8
        v[:, ch] *= 8
    kq = orc.quantize_q4_0(k).reshape(n_kv, Hkv, -1)
    vq = orc.quantize_q4_0(v).reshape(n_kv, Hkv, -1)
    return q, kq, vq


@pytest.mark.parametrize("n_q,H,Hkv,n_kv,start", [(1, 16, 2, 512, 511), (2, 16, 2, 768, 700),
                                                  (5, 4, 1, 300, 100), (3, 8, 8, 64, 60)])
def test_fa_matches_f64_bruteforce(orc, n_q, H, Hkv, n_kv, start):
    rng = np.random.default_rng(n_kv + n_q)
    q, kq, vq = make(orc, rng, n_q, H, Hkv, n_kv, outliers=3)
    mask = orc.causal_mask(n_q, n_kv, start)
    got = orc.flash_attn_ext(q, kq, vq, mask, scale=1 / 16)
    ref = attention_f64(q8_dequant(orc, q), cache_dequant(orc, kq), cache_dequant(orc, vq), 1 / 16, mask)
    assert rel_err(got, ref) < 2e-5


def test_gqa_block_map_is_pinned(orc):
    # A kernel that used h % Hkv instead of h // (H/Hkv) would match this instead.
    rng = np.random.default_rng(2)
    q, kq, vq = make(orc, rng, 1, 8, 2, 256)
    got = orc.flash_attn_ext(q, kq, vq, None)
    qd, kd, vd = q8_dequant(orc, q), cache_dequant(orc, kq), cache_dequant(orc, vq)
    assert rel_err(got, attention_f64(qd, kd, vd, 1 / 16)) < 2e-5
    assert rel_err(got, attention_f64(qd, kd, vd, 1 / 16, head_map=lambda h: h % 2)) > 0.1


def test_single_key_returns_v(orc):
    rng = np.random.default_rng(3)
    q, kq, vq = make(orc, rng, 2, 16, 2, 1)
    got = orc.flash_attn_ext(q, kq, vq, None)
    vd = cache_dequant(orc, vq)
    for h in range(16):
        assert np.array_equal(got[:, h, :], np.broadcast_to(vd[0, h // 8], (2, 256)).astype(np.float32))


def test_uniform_scores_give_mean_of_v(orc):
    rng = np.random.default_rng(4)
    q, _, vq = make(orc, rng, 1, 16, 2, 200)
    kq = orc.quantize_q4_0(np.zeros((200, 512), dtype=np.float32)).reshape(200, 2, -1)
    got = orc.flash_attn_ext(q, kq, vq, None)
    vd = cache_dequant(orc, vq)
    want = np.stack([vd[:, h // 8].mean(axis=0) for h in range(16)])[None]
    assert np.abs(got - want).max() < 1e-5


def test_one_visible_key_and_all_masked(orc):
    rng = np.random.default_rng(5)
    q, kq, vq = make(orc, rng, 2, 16, 2, 256)
    mask = np.full((2, 256), -np.inf, dtype=np.float16)
    mask[0, 77] = 0
    got = orc.flash_attn_ext(q, kq, vq, mask)
    vd = cache_dequant(orc, vq)
    for h in range(16):
        assert np.array_equal(got[0, h], vd[77, h // 8].astype(np.float32))
    assert np.all(got[1] == 0)  # every key masked: S = 0 -> output 0


def test_causal_variant_equals_mask_and_gate(orc):
    rng = np.random.default_rng(6)
    q, kq, vq = make(orc, rng, 2, 16, 2, 512)
    mask = orc.causal_mask(2, 512, 300)
    a = orc.flash_attn_ext(q, kq, vq, mask)
    b = orc.flash_attn_ext_causal(q, kq, vq, 300)
    assert np.array_equal(a, b)
    gate = rng.standard_normal(q.shape).astype(np.float32)
    c = orc.flash_attn_ext_causal(q, kq, vq, 300, gate=gate)
    d = orc.sigmoid_mul(a.reshape(2, -1), gate.reshape(2, -1)).reshape(a.shape)
    assert np.array_equal(c, d)


def test_q8_variant_effect_within_tolerance(orc):
    rng = np.random.default_rng(8)
    q, kq, vq = make(orc, rng, 1, 16, 2, 1024)
    a = orc.flash_attn_ext(q, kq, vq, None, variant=orc.Q8_X86)
    b = orc.flash_attn_ext(q, kq, vq, None, variant=orc.Q8_SCALAR)
    assert rel_err(b, a) < 2e-3
