"""The allocation-free decode entry point (sqa_flash_attn_ext_static) against
the workspace entry point (sqa_flash_attn_ext) through the C ABI: same kernels,
so the outputs must be identical bit for bit. Two calls in a row, the second
with a smaller input, so the second reuses scratch the first left behind; then
its error paths (prefill shapes, scratch above its maximum), and its use under
HIP graph capture."""
import numpy as np
import pytest
import torch

from tests.gen import qkv, rel_err

pytestmark = pytest.mark.gpu


def _run_both(sqa, dev, q, kq, vq, mask):
    qt = torch.from_numpy(q).to(dev)
    kt = torch.from_numpy(np.ascontiguousarray(kq)).to(dev)
    vt = torch.from_numpy(np.ascontiguousarray(vq)).to(dev)
    mt = torch.from_numpy(mask).to(dev) if mask is not None else None
    n_kv = kq.shape[0]
    ref = sqa.flash_attn_ext(qt, kt, vt, n_kv, mask=mt)
    out = torch.full_like(ref, float("nan"))
    sqa.flash_attn_ext_static(qt, kt, vt, n_kv, mask=mt, out=out)
    torch.cuda.synchronize()
    return out.cpu().numpy(), ref.cpu().numpy()


def test_static_entry_matches_workspace_entry(sqa, orc, dev):
    # first call: verify, n_q = 2 over 40000 keys with an unaligned mask (packed copy in scratch)
    q, kq, vq = qkv(orc, 61, 2, 40001)
    mask = orc.causal_mask(2, 40001, 39999)
    got, ref = _run_both(sqa, dev, q, kq, vq, mask)
    assert np.array_equal(got, ref)
    assert rel_err(got, orc.flash_attn_ext(q, kq, vq, mask)) <= 2e-3
    # second call, smaller: decode over 3000 keys, fewer splits, no mask
    q, kq, vq = qkv(orc, 62, 1, 3000)
    got, ref = _run_both(sqa, dev, q, kq, vq, None)
    assert np.array_equal(got, ref)
    assert rel_err(got, orc.flash_attn_ext(q, kq, vq, None)) <= 2e-3


@pytest.mark.parametrize("Hkv,H,n_q,n_kv", [(1, 16, 1, 20000), (8, 16, 2, 5000)])
def test_static_entry_other_kv_head_counts(sqa, orc, dev, Hkv, H, n_q, n_kv):
    """Other KV-head counts: more splits per head at one KV head, fewer at eight."""
    q, kq, vq = qkv(orc, 64 + Hkv, n_q, n_kv, H=H, Hkv=Hkv)
    mask = orc.causal_mask(n_q, n_kv, n_kv - n_q)
    got, ref = _run_both(sqa, dev, q, kq, vq, mask)
    assert np.array_equal(got, ref)
    assert rel_err(got, orc.flash_attn_ext(q, kq, vq, mask)) <= 2e-3


def test_static_entry_rejects_what_it_cannot_run(sqa, orc, dev):
    q, kq, vq = qkv(orc, 63, 8, 1024)  # 8 positions: a prefill chunk
    qt, kt, vt = (torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in (q, kq, vq))
    with pytest.raises(sqa.SqaError) as e:
        sqa.flash_attn_ext_static(qt, kt, vt, 1024)
    assert e.value.status == 2  # unsupported: only decode/verify shapes
    # 4 positions x 4 heads per KV head over 2M keys: a mask copy past the scratch maximum
    n_kv = 2_000_001
    kt = torch.zeros((n_kv, 2, 144), dtype=torch.uint8, device=dev)
    qt = torch.zeros((4, 8, 256), device=dev)
    mt = torch.zeros((4, n_kv), dtype=torch.float16, device=dev)
    with pytest.raises(sqa.SqaError) as e:
        sqa.flash_attn_ext_static(qt, kt, kt, n_kv, mask=mt)
    assert e.value.status == 3 and "maximum" in str(e.value)


def test_static_entry_graph_replay(sqa, orc, dev):
    """The static entry captured once in a HIP graph (the use it exists for) with
    an unaligned mask (n_kv odd: the packed copy runs inside the graph too) and
    replayed at two positions, new Q and a new mask filled eagerly before each
    replay; every replay is checked against the oracle."""
    n_kv = 3001
    _, kq, vq = qkv(orc, 71, 1, n_kv)
    kt = torch.from_numpy(np.ascontiguousarray(kq)).to(dev)
    vt = torch.from_numpy(np.ascontiguousarray(vq)).to(dev)
    qt = torch.empty((1, 16, 256), device=dev)
    mt = torch.empty((1, n_kv), dtype=torch.float16, device=dev)
    out = torch.empty((1, 16, 256), device=dev)
    rng = np.random.default_rng(72)
    qt.copy_(torch.from_numpy(rng.standard_normal((1, 16, 256), dtype=np.float32)))
    sqa.fill_causal_mask(mt, 2000)
    sqa.flash_attn_ext_static(qt, kt, vt, n_kv, mask=mt, out=out)  # eager first call, outside the capture
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            sqa.flash_attn_ext_static(qt, kt, vt, n_kv, mask=mt, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for pos in (2500, 3000, 1234):
        q = rng.standard_normal((1, 16, 256), dtype=np.float32)
        qt.copy_(torch.from_numpy(q))
        sqa.fill_causal_mask(mt, pos)
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        ref = orc.flash_attn_ext(q, kq, vq, orc.causal_mask(1, n_kv, pos))
        err = rel_err(out.cpu().numpy(), ref)
        print(f"static entry graph replay at position {pos}: max err / rms = {err:.3e}")
        assert err <= 2e-3, pos
