"""Elementwise kernels beside the attention op: the sigmoid output gate
(src/model/attn.rs:282-283) and the device-built causal mask
(src/model/graph.rs:534-576)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [(2048, 4096), (3, 4099)])
def test_sigmoid_mul(sqa, orc, dev, shape):
    rng = np.random.default_rng(shape[1])
    x = rng.standard_normal(shape).astype(np.float32)
    g = (rng.standard_normal(shape) * 4).astype(np.float32)
    want = orc.sigmoid_mul(x, g)
    got = sqa.sigmoid_mul(torch.from_numpy(x).to(dev), torch.from_numpy(g).to(dev)).cpu().numpy()
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()


@pytest.mark.parametrize("n_q,n_kv,start", [(1, 4096, 4095), (512, 16896, 16384), (7, 300, 10)])
def test_fill_causal_mask(sqa, orc, dev, n_q, n_kv, start):
    want = orc.causal_mask(n_q, n_kv, start)
    m = torch.empty((n_q, n_kv), dtype=torch.float16, device=dev)
    sqa.fill_causal_mask(m, start)
    assert np.array_equal(m.cpu().numpy().view(np.uint16), want.view(np.uint16))
