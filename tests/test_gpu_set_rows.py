"""q4_0 set_rows on the GPU is bit-exact with the oracle's ggml
quantize_row_q4_0 (quantize-on-write of src/engine/kv.rs:356-396)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def edge_rows(rng, n, ne0=512):
    x = rng.standard_normal((max(n, 8), ne0)).astype(np.float32)
    x[0] = 0                                          # all-zero blocks: d = -0.0
    x[1] = np.tile(np.arange(32) - 16, ne0 // 32)     # ramp KAT
    x[2, ::32] = 3.0                                  # +max first
    x[2, 9::32] = -3.0
    x[3] *= np.float32(1e-30)                         # tiny values, subnormal-range d
    x[4] *= np.float32(3e4)                           # large values near fp16 range
    x[5] = np.round(x[5] * 8) / 8                     # grid values: exact products, rounding ties
    x[6, 5::32] = x[6, 20::32] = -2.0                 # magnitude ties
    x[7] = np.float32(1e-45)                          # denormal floats
    return x[np.argsort(rng.random(x.shape[0]))][:n] if n < 8 else x


@pytest.mark.parametrize("ne0,n,rows", [(512, 300, 1024), (256, 7, 16), (256, 8, 16), (4096, 33, 40)])
def test_set_rows_bit_exact(sqa, orc, dev, ne0, n, rows):
    rng = np.random.default_rng(ne0 + n)
    src = edge_rows(rng, n, ne0)
    idx = rng.permutation(rows)[:n].astype(np.int64)
    init = rng.integers(0, 256, (rows, ne0 // 32 * 18), dtype=np.uint8)
    want = orc.set_rows_q4_0(init.copy(), src, idx)
    cache = torch.from_numpy(init.copy()).to(dev)
    sqa.set_rows_q4_0(cache, torch.from_numpy(src).to(dev), torch.from_numpy(idx).to(dev))
    got = cache.cpu().numpy()
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} bytes differ, first at {bad[:4].tolist()}"


def fused_split_values(M, n_each=4):
    """Values x of a block whose maximum is M where ggml's x*id + 8.5f, rounded
    twice, and a fused multiply-add truncate to different codes: x*id within half
    an ulp below a half-integer (id = 1/(M/-8) as ggml forms it)."""
    d = np.float32(M) / np.float32(-8)
    idv = np.float32(1) / d
    out = []
    for h in np.arange(-8, 8) + 0.5:
        x0 = np.float32(h / np.float64(idv))
        cand = (x0.view(np.int32) + np.arange(-64, 65, dtype=np.int32)).view(np.float32)
        cand = cand[np.abs(cand) < M]
        sep = (cand * idv).astype(np.float32) + np.float32(8.5)
        fused = (cand.astype(np.float64) * np.float64(idv) + 8.5).astype(np.float32)
        diff = cand[np.minimum(sep.astype(np.int32), 15) != np.minimum(fused.astype(np.int32), 15)]
        out.extend(diff[:n_each].tolist())
    return np.array(out, np.float32)


def test_set_rows_multiply_add_not_fused(sqa, orc, dev):
    """Blocks of values where a fused x*id + 8.5f (one rounding) truncates to
    another code than ggml's two roundings: bit-exact only without the fusion."""
    rng = np.random.default_rng(21)
    rows, ne0 = [], 512
    for M in (0.9, 1.7, 2.3, 5.1, 13.7, 0.031):
        vals = fused_split_values(M)
        assert len(vals) >= 4
        for _ in range(2):
            r = rng.choice(vals, (ne0 // 32, 32)).astype(np.float32)
            r[:, 0] = np.float32(M)  # the block maximum, first
            rows.append(r.reshape(ne0))
    src = np.stack(rows)
    n = src.shape[0]
    idx = np.arange(n, dtype=np.int64)
    init = np.zeros((n, ne0 // 32 * 18), np.uint8)
    want = orc.set_rows_q4_0(init.copy(), src, idx)
    # the data has teeth: a fused multiply-add would change codes here
    blocks = src.reshape(-1, 32)
    idv = np.float32(1) / (blocks[:, :1] / np.float32(-8))
    fused = np.minimum((blocks.astype(np.float64) * idv.astype(np.float64) + 8.5).astype(np.float32).astype(np.int32), 15)
    codes = want.reshape(-1, 18)[:, 2:]
    codes = np.concatenate([codes & 15, codes >> 4], axis=1)
    assert (fused != codes).sum() > 100
    cache = torch.from_numpy(init.copy()).to(dev)
    sqa.set_rows_q4_0(cache, torch.from_numpy(src).to(dev), torch.from_numpy(idx).to(dev))
    got = cache.cpu().numpy()
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} bytes differ, first at {bad[:4].tolist()}"


def test_set_rows_unaligned_source_and_out_of_range_index(sqa, orc, dev):
    rng = np.random.default_rng(3)
    n, ne0, rows = 40, 512, 64
    big = rng.standard_normal(n * ne0 + 1).astype(np.float32)
    src = big[1:].reshape(n, ne0)                      # 4-byte offset: scalar-load path
    idx = rng.permutation(rows)[:n].astype(np.int64)
    idx[3], idx[7] = -1, rows                          # skipped, never written
    init = rng.integers(0, 256, (rows, ne0 // 32 * 18), dtype=np.uint8)
    want = orc.set_rows_q4_0(init.copy(), src, idx)
    big_t = torch.from_numpy(big).to(dev)
    src_t = big_t[1:].view(n, ne0)
    assert src_t.data_ptr() % 16 != 0
    cache = torch.from_numpy(init.copy()).to(dev)
    sqa.set_rows_q4_0(cache, src_t, torch.from_numpy(idx).to(dev))
    assert np.array_equal(cache.cpu().numpy(), want)


def test_set_rows_large_random(sqa, orc, dev):
    rng = np.random.default_rng(99)
    n, ne0 = 2048, 512
    src = (rng.standard_normal((n, ne0)) * rng.uniform(1e-3, 1e3, (n, 1))).astype(np.float32)
    idx = np.arange(n, dtype=np.int64)
    want = orc.set_rows_q4_0(np.zeros((n, 288), np.uint8), src, idx)
    cache = torch.zeros((n, 288), dtype=torch.uint8, device=dev)
    sqa.set_rows_q4_0(cache, torch.from_numpy(src).to(dev), torch.from_numpy(idx).to(dev))
    assert np.array_equal(cache.cpu().numpy(), want)
