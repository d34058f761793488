"""The fused K/Q producer (per-head RMSNorm, IMROPE, q4_0 quantize-on-write) on
the GPU against the oracle's restatement of ggml's rms_norm -> mul ->
rope_multi(IMROPE) -> set_rows chain (reference src/model/attn.rs:166-200,
src/engine/kv.rs:313-399).

Bar: the float stage (norm and rotation) agrees to a few fp32 ulps. The kernel's
square root and cos/sin are correctly rounded; the C library's cosf/sinf are not
for about 1% of arguments, so there the rotated value may differ in the last
bit, and a q4_0 code may flip where the scaled value sits on a rounding boundary.
Where two values of a block tie in magnitude to the last bit with opposite
signs, the block maximum (the first of the largest, as ggml picks it) may be the
other one: d changes sign and the codes mirror, which dequantises to the same
values but the extreme one, a code step away. Hence for the q4_0 output: |d|
(fp16) equal or one ulp apart, at least 99.9% of the codes equal, every
dequantised value within one code step of the oracle's, and rows outside idx
untouched. The quantizer itself is bit-exact (test_gpu_set_rows.py)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

EPS = 1e-6
# the engine's geometry with plausible model values, the reference test's own
# small configuration (tests/attn_test.rs:23-31), and sections that use e
CASES = [
    # D, n_head, n_tok, n_rot, sections, freq_base, pos0
    (256, 2, 512, 64, (11, 11, 10, 0), 1e7, 16384),
    (256, 2, 7, 64, (11, 11, 10, 0), 1e7, 171990),
    (64, 1, 40, 16, (3, 3, 2, 0), 1e7, 0),
    (128, 4, 33, 32, (2, 1, 1, 4), 1e4, 900),
    (256, 16, 20, 256, (43, 43, 42, 0), 1e6, 5000),
]


def _inputs(rng, D, n_head, n_tok, pos0, distinct):
    src = (rng.standard_normal((n_tok, n_head, D)) * 2).astype(np.float32)
    w = (1 + 0.3 * rng.standard_normal(D)).astype(np.float32)
    t = np.arange(pos0, pos0 + n_tok, dtype=np.int32)
    pos = np.concatenate([t, t + 3, t + 7, t + 11]) if distinct else np.tile(t, 4)
    return src, w, pos.astype(np.int32)


def _fp16_ulps(a, b):
    return np.abs(a.astype(np.int32) - b.astype(np.int32))


def _compare_q4(got, want, D):
    g = got.reshape(-1, 18)
    w = want.reshape(-1, 18)
    dg = g[:, :2].copy().view(np.uint16).ravel()
    dw = w[:, :2].copy().view(np.uint16).ravel()
    assert _fp16_ulps(dg & 0x7FFF, dw & 0x7FFF).max() <= 1
    cg = np.concatenate([g[:, 2:] & 15, g[:, 2:] >> 4], axis=1)
    cw = np.concatenate([w[:, 2:] & 15, w[:, 2:] >> 4], axis=1)
    same = (cg == cw).mean()
    assert same >= 0.999, same
    d = np.abs(dw.view(np.float16).astype(np.float32))
    vg = (cg.astype(np.float32) - 8) * dg.view(np.float16).astype(np.float32)[:, None]
    vw = (cw.astype(np.float32) - 8) * dw.view(np.float16).astype(np.float32)[:, None]
    assert np.all(np.abs(vg - vw) <= d[:, None] * 1.001 + 1e-30)


@pytest.mark.parametrize("D,n_head,n_tok,n_rot,sections,base,pos0", CASES)
def test_rope_norm_f32(sqa, orc, dev, D, n_head, n_tok, n_rot, sections, base, pos0):
    rng = np.random.default_rng(D + n_tok)
    src, w, pos = _inputs(rng, D, n_head, n_tok, pos0, distinct=sections[3] > 0)
    rp = orc.rope_params(n_rot, sections, base)
    want = orc.rope_norm_f32(src, w, EPS, pos, rp)
    out = torch.empty((n_tok, n_head, D), dtype=torch.float32, device=dev)
    sqa.rope_norm_f32(out, torch.from_numpy(src).to(dev), torch.from_numpy(w).to(dev), EPS,
                      torch.from_numpy(pos).to(dev), sqa.rope_params(n_rot, sections, base))
    got = out.cpu().numpy()
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= 2e-6 * scale


@pytest.mark.parametrize("D,n_head,n_tok,n_rot,sections,base,pos0", CASES[:4])
def test_rope_norm_set_rows_q4_0(sqa, orc, dev, D, n_head, n_tok, n_rot, sections, base, pos0):
    rng = np.random.default_rng(7 * D + n_tok)
    src, w, pos = _inputs(rng, D, n_head, n_tok, pos0, distinct=sections[3] > 0)
    rows = n_tok + 9
    idx = rng.permutation(rows)[:n_tok].astype(np.int64)
    rb = n_head * D // 32 * 18
    init = rng.integers(0, 256, (rows, rb), dtype=np.uint8)
    rp = orc.rope_params(n_rot, sections, base)
    want = orc.rope_norm_set_rows_q4_0(init.copy(), src, w, EPS, pos, rp, idx)
    cache = torch.from_numpy(init.copy()).to(dev)
    sqa.rope_norm_set_rows_q4_0(cache, torch.from_numpy(src).to(dev), torch.from_numpy(w).to(dev), EPS,
                                torch.from_numpy(pos).to(dev), sqa.rope_params(n_rot, sections, base),
                                torch.from_numpy(idx).to(dev))
    got = cache.cpu().numpy()
    others = np.setdiff1d(np.arange(rows), idx)
    assert np.array_equal(got[others], init[others])
    _compare_q4(got[idx], want[idx], D)


def test_no_norm_and_strided_source(sqa, orc, dev):
    """norm_w = NULL skips the normalisation; the source is the q half of an
    interleaved [q | gate] projection (head stride 2*D, reference attn.rs:131-164)."""
    rng = np.random.default_rng(11)
    D, n_head, n_tok = 256, 16, 9
    full = rng.standard_normal((n_tok, n_head, 2 * D)).astype(np.float32)
    pos = np.tile(np.arange(50, 50 + n_tok, dtype=np.int32), 4)
    rp = orc.rope_params(64, (11, 11, 10, 0), 1e7)
    want = orc.rope_norm_f32(np.ascontiguousarray(full[:, :, :D]), None, EPS, pos, rp)
    t_full = torch.from_numpy(full).to(dev)
    out = torch.empty((n_tok, n_head, D), dtype=torch.float32, device=dev)
    sqa.rope_norm_f32(out, t_full[:, :, :D], None, EPS, torch.from_numpy(pos).to(dev),
                      sqa.rope_params(64, (11, 11, 10, 0), 1e7))
    assert np.abs(out.cpu().numpy() - want).max() <= 2e-6 * np.abs(want).max()


def test_cache_written_by_producer_feeds_attention(sqa, orc, dev):
    """K written by the producer and read back by flash_attn_ext gives the
    oracle's attention over the oracle's cache (the layer's own data flow)."""
    rng = np.random.default_rng(12)
    D, Hkv, n_kv = 256, 2, 300
    src, w, pos = _inputs(rng, D, Hkv, n_kv, 0, distinct=False)
    rp = orc.rope_params(64, (11, 11, 10, 0), 1e7)
    idx = np.arange(n_kv, dtype=np.int64)
    kc = orc.rope_norm_set_rows_q4_0(np.zeros((n_kv, Hkv * D // 32 * 18), np.uint8), src, w, EPS, pos, rp, idx)
    vsrc = rng.standard_normal((n_kv, Hkv * D)).astype(np.float32)
    vc = orc.set_rows_q4_0(np.zeros((n_kv, Hkv * D // 32 * 18), np.uint8), vsrc, idx)
    q = rng.standard_normal((1, 16, D)).astype(np.float32)
    want = orc.flash_attn_ext(q, kc.reshape(n_kv, Hkv, -1), vc.reshape(n_kv, Hkv, -1))
    kdev = torch.zeros((n_kv, Hkv, D // 32 * 18), dtype=torch.uint8, device=dev)
    sqa.rope_norm_set_rows_q4_0(kdev, torch.from_numpy(src).to(dev), torch.from_numpy(w).to(dev), EPS,
                                torch.from_numpy(pos).to(dev), sqa.rope_params(64, (11, 11, 10, 0), 1e7),
                                torch.from_numpy(idx).to(dev))
    vdev = torch.from_numpy(vc.reshape(n_kv, Hkv, -1)).to(dev)
    out = torch.empty((1, 16, D), dtype=torch.float32, device=dev)
    ws = torch.empty(sqa.flash_attn_workspace_size(torch.from_numpy(q).to(dev), kdev, n_kv), dtype=torch.uint8,
                     device=dev)
    sqa.flash_attn_ext(torch.from_numpy(q).to(dev), kdev, vdev, n_kv, out=out, workspace=ws)
    got = out.cpu().numpy()
    rms = np.sqrt((want.astype(np.float64) ** 2).mean())
    assert np.abs(got - want).max() <= 2e-3 * rms
