"""The HIP path against the committed golden fixtures (tests/golden/):
set_rows bit-exact on the quantizer edge blocks, flash_attn_ext within
max |gpu - fixture| <= 2e-3 * rms(fixture)."""
import os

import numpy as np
import pytest
import torch

from tests.gen import rel_err
from tests.test_golden import FA_CASES, load

pytestmark = pytest.mark.gpu
TOL = 2e-3


def test_set_rows_edge_blocks_bit_exact(sqa, dev):
    g = load("q4_0_blocks")
    x, want = g["x"], g["q4_0"]
    n = x.shape[0] // 8 * 8  # rows of 8 blocks (256 values, one KV head row)
    src = torch.from_numpy(np.ascontiguousarray(x[:n].reshape(-1, 256))).to(dev)
    rows = src.shape[0]
    cache = torch.zeros((rows + 3, 1, 144), dtype=torch.uint8, device=dev)
    idx = torch.arange(rows, dtype=torch.int64, device=dev) + 2
    sqa.set_rows_q4_0(cache, src, idx)
    got = cache.cpu().numpy()[2:2 + rows].reshape(-1, 18)
    assert np.array_equal(got, want[:n])


@pytest.mark.parametrize("name", FA_CASES)
def test_fa_fixture(sqa, dev, name):
    g = load(name)
    q = torch.from_numpy(g["q"]).to(dev)
    k = torch.from_numpy(g["k"]).to(dev)
    v = torch.from_numpy(g["v"]).to(dev)
    mask = torch.from_numpy(g["mask"]).to(dev)
    n_kv = g["k"].shape[0]
    out = sqa.flash_attn_ext(q, k, v, n_kv, mask=mask, scale=float(g["scale"]))
    if "gate" in g:
        n_q = out.shape[0]
        out = sqa.sigmoid_mul(out.view(n_q, -1), torch.from_numpy(g["gate"]).to(dev).view(n_q, -1)).view(out.shape)
    torch.cuda.synchronize()
    err = rel_err(out.cpu().numpy(), g["out"])
    print(f"{name}: max err / rms = {err:.3e}")
    assert err <= TOL
