"""Pins the oracle's K/Q producer restatement (RMSNorm, IMROPE, quantize-on-write)
with closed forms and hand-derived tables, not with its own formula:
  * position 0 rotates nothing; a rotation keeps each pair's norm;
  * text positions (t = h = w = e = p, the engine's case) reduce IMROPE to
    plain NEOX rope, whose angle p * base^(-2ic/n_rot) is computed here in
    float64;
  * the IMROPE sector table for two section vectors, worked out by hand from the
    rule of rope_ref (reference tests/attn_test.rs:175-186);
  * RMSNorm of a constant row, and agreement with the reference test's own
    restatement rms_norm_row (tests/attn_test.rs:278-283) to fp32 rounding.
"""
import numpy as np
import pytest

from oracle import oracle as orc


def test_position_zero_is_identity():
    r = orc.rope_params(16, [3, 3, 2, 0], 1e7)
    x = np.random.default_rng(1).standard_normal(64).astype(np.float32)
    cache = orc.imrope_cache(r, (0, 0, 0, 0))
    assert np.array_equal(cache[0::2], np.ones(8, np.float32))
    assert np.array_equal(cache[1::2], np.zeros(8, np.float32))
    assert np.array_equal(orc.rope_row(x, r, cache), x)


def test_rotation_keeps_pair_norms_and_passes_tail_dims():
    r = orc.rope_params(64, [11, 11, 10, 0], 1e7)
    x = np.random.default_rng(2).standard_normal(256).astype(np.float32)
    y = orc.rope_row(x, r, orc.imrope_cache(r, (171999, 171999, 171999, 171999)))
    n0 = x[:32].astype(np.float64) ** 2 + x[32:64].astype(np.float64) ** 2
    n1 = y[:32].astype(np.float64) ** 2 + y[32:64].astype(np.float64) ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5)
    assert np.array_equal(y[64:], x[64:])


@pytest.mark.parametrize("p", [1, 37, 4095, 131071])
def test_text_positions_are_neox_rope(p):
    n_rot, base = 64, 1e4
    r = orc.rope_params(n_rot, [11, 11, 10, 0], base)
    cache = orc.imrope_cache(r, (p, p, p, p))
    ic = np.arange(32, dtype=np.float64)
    ang = p * base ** (-2.0 * ic / n_rot)
    # the oracle forms the angle as ic fp32 multiplies: relative error ~ ic * 2^-24
    tol = (ic + 2) * 2.0 ** -23 * ang + 1e-6
    got = np.arctan2(cache[1::2].astype(np.float64), cache[0::2].astype(np.float64))
    err = np.abs(np.angle(np.exp(1j * (got - ang))))
    assert np.all(err <= tol), (err - tol).max()


def _component_table(sections, n_pairs):
    """Which position component (t h w e = 0 1 2 3) pair ic uses, read back by
    giving every component a different position."""
    r = orc.rope_params(2 * n_pairs, sections, 10.0)
    pos = (3, 5, 7, 11)
    c = orc.imrope_cache(r, pos)
    ang = np.arctan2(c[1::2].astype(np.float64), c[0::2].astype(np.float64))
    out = []
    for i in range(n_pairs):
        cand = [pk * 10.0 ** (-2.0 * i / (2 * n_pairs)) for pk in pos]
        d = [abs(np.angle(np.exp(1j * (ang[i] - a)))) for a in cand]
        out.append(int(np.argmin(d)))
    return out


def test_imrope_sector_tables():
    # sections (3, 3, 2, 0), 8 pairs: sector = ic; t when %3 == 0 and < 9, h when
    # %3 == 1 and < 9, w when %3 == 2 and < 6 -> t h w t h w t h
    assert _component_table([3, 3, 2, 0], 8) == [0, 1, 2, 0, 1, 2, 0, 1]
    # sections (2, 1, 1, 4): t needs < 6, h < 3, w < 3 -> t h w t e e e e
    assert _component_table([2, 1, 1, 4], 8) == [0, 1, 2, 0, 3, 3, 3, 3]


def test_rms_norm_constant_row_and_reference_restatement():
    eps = 1e-6
    y = orc.rms_norm_mul_row(np.full(256, 0.5, np.float32), None, eps)
    np.testing.assert_allclose(y, 0.5 / np.sqrt(0.25 + eps), rtol=1e-7)
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(256) * 3).astype(np.float32)
    w = rng.standard_normal(256).astype(np.float32)
    ms = np.float32(np.sum(x * x, dtype=np.float32) / np.float32(256))
    ref = (x / np.sqrt(ms + np.float32(eps))) * w  # rms_norm_row of the reference test
    np.testing.assert_allclose(orc.rms_norm_mul_row(x, w, eps), ref, rtol=3e-6, atol=1e-7)


def test_fused_q4_0_matches_composition_and_step_bound():
    rng = np.random.default_rng(4)
    n_tok, n_head, D = 5, 2, 256
    r = orc.rope_params(64, [11, 11, 10, 0], 1e7)
    src = rng.standard_normal((n_tok, n_head, D)).astype(np.float32)
    w = rng.standard_normal(D).astype(np.float32)
    pos = np.tile(np.arange(100, 100 + n_tok, dtype=np.int32), 4)
    idx = np.array([7, 0, 3, 9, 1], dtype=np.int64)
    cache = np.zeros((10, n_head * D // 32 * 18), np.uint8)
    orc.rope_norm_set_rows_q4_0(cache, src, w, 1e-6, pos, r, idx)
    f = orc.rope_norm_f32(src, w, 1e-6, pos, r)
    for t in range(n_tok):
        row = cache[idx[t]].reshape(n_head, -1)
        assert np.array_equal(row, orc.quantize_q4_0(f[t]))
        deq = orc.dequantize_q4_0(row, D)
        d = np.abs(orc.fp16_bits_to_fp32(row.reshape(n_head, 8, 18)[:, :, :2].copy().view(np.uint16).ravel()))
        assert np.all(np.abs(deq - f[t]).reshape(n_head, 8, 32) <= d.reshape(n_head, 8, 1) * 1.0000001)
    untouched = [i for i in range(10) if i not in idx]
    assert not cache[untouched].any()
