"""Seeded random shapes through the attention kernels against a float64 brute
force, and through the K/Q producer against the oracle: KV heads 1-8, group
sizes 1-16, decode / verify / prefill chunk sizes, causal-from-positions,
causal and holed F16 masks, the fused sigmoid gate, V scales over three
decades, outlier channels.

The float64 reference runs on the same dequantised operands (q8_0 Q, q4_0 K
and V), so the bound measures the kernels' own arithmetic rather than ggml's
fp32 path, which itself lands up to ~1e-3 x RMS from the exact result on such
inputs. Bound: half the 2e-3 x RMS tolerance of this path."""
import numpy as np
import pytest
import torch

from tests import fa_ref
from tests.gen import qkv, rel_err
from tests.test_gpu_rope import EPS, _compare_q4, _inputs

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _attention_case(orc, rng):
    Hkv = int(rng.choice([1, 2, 3, 4, 8]))
    G = int(rng.choice([1, 2, 4, 8, 16]))
    kind = rng.choice(["decode", "decode", "prefill"])
    if kind == "decode":
        n_q = int(rng.integers(1, 5))
        while n_q * G > 16:
            n_q -= 1
        n_kv = int(np.exp(rng.uniform(0, np.log(20000 // Hkv))))
    else:
        if 16 % G:
            G = 8
        n_q = int(rng.integers(5, 120))
        n_kv = int(rng.integers(n_q, 4000))
    n_kv = max(n_kv, n_q)
    H = Hkv * G
    outl = int(rng.choice([0, 3, 8]))
    sv = float(np.exp(rng.uniform(np.log(1e-1), np.log(1e2))))
    q, kq, vq = qkv(orc, int(rng.integers(1 << 30)), n_q, n_kv, H=H, Hkv=Hkv, outliers=outl, scale_v=sv)
    form = str(rng.choice(["causal_mask", "causal_pos", "holes"]))
    mask = orc.causal_mask(n_q, n_kv, n_kv - n_q)
    if form == "holes":
        m = mask.astype(np.float32)
        m[rng.random(m.shape) < 0.2] = -np.inf
        fin = (rng.random(m.shape) < 0.1) & np.isfinite(m)
        m[fin] = -rng.uniform(0, 4, size=int(fin.sum()))
        mask = m.astype(np.float16)
    return q, kq, vq, mask, form, f"Hkv={Hkv} H={H} n_q={n_q} n_kv={n_kv} outliers={outl} V x{sv:.3g} {form}"


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_random_attention_shapes_against_f64(sqa, orc, dev, seed):
    rng = np.random.default_rng(1000 + seed)
    worst = 0.0
    for _ in range(60):
        q, kq, vq, mask, form, label = _attention_case(orc, rng)
        n_q, n_kv = q.shape[0], kq.shape[0]
        qt = torch.from_numpy(q).to(dev)
        kt = torch.from_numpy(np.ascontiguousarray(kq)).to(dev)
        vt = torch.from_numpy(np.ascontiguousarray(vq)).to(dev)
        gate = None
        if form == "causal_pos":
            # half of these with the sigmoid gate fused (split merge or prefill epilogue)
            gate = rng.standard_normal(q.shape).astype(np.float32) if rng.random() < 0.5 else None
            gt = torch.from_numpy(gate).to(dev) if gate is not None else None
            out = sqa.flash_attn_ext_causal(qt, kt, vt, n_kv, n_kv - n_q, gate=gt, scale=1 / 16)
        else:
            out = sqa.flash_attn_ext(qt, kt, vt, n_kv, mask=torch.from_numpy(mask).to(dev), scale=1 / 16)
        got = out.cpu().numpy()
        exact = fa_ref.attention_f64(fa_ref.q8_dequant(orc, q), fa_ref.cache_dequant(orc, kq),
                                     fa_ref.cache_dequant(orc, vq), 1 / 16, mask)
        if gate is not None:
            exact = exact / (1.0 + np.exp(-gate.astype(np.float64)))
            label += " gate"
        err = rel_err(got, exact)
        worst = max(worst, err)
        assert np.all(np.isfinite(got)), label
        assert err <= TOL / 2, f"{label}: {err:.3e}"
    print(f"seed {seed}: worst gpu vs f64 {worst:.3e}")


@pytest.mark.parametrize("seed", [1, 2])
def test_random_producer_shapes(sqa, orc, dev, seed):
    rng = np.random.default_rng(2000 + seed)
    for _ in range(80):
        D = int(rng.choice([64, 128, 256]))
        n_head = int(rng.integers(1, 17))
        n_tok = int(rng.integers(1, 300))
        n_rot = 8 * int(rng.integers(1, D // 8 + 1))
        sec = [int(x) for x in rng.integers(0, 17, 4)]
        if sum(sec) == 0:
            sec[0] = 1
        base = float(rng.choice([1e4, 1e6, 1e7]))
        pos0 = int(rng.integers(0, 1 << 18))
        use_w = bool(rng.random() < 0.8)
        r2 = np.random.default_rng(int(rng.integers(1 << 30)))
        src, w, pos = _inputs(r2, D, n_head, n_tok, pos0, distinct=bool(rng.random() < 0.5))
        rp = orc.rope_params(n_rot, sec, base)
        wt = torch.from_numpy(w).to(dev) if use_w else None
        label = f"D={D} heads={n_head} tokens={n_tok} n_rot={n_rot} sections={tuple(sec)} base={base:g} pos0={pos0}"
        want = orc.rope_norm_f32(src, w if use_w else None, EPS, pos, rp)
        out = torch.empty((n_tok, n_head, D), dtype=torch.float32, device=dev)
        sqa.rope_norm_f32(out, torch.from_numpy(src).to(dev), wt, EPS, torch.from_numpy(pos).to(dev),
                          sqa.rope_params(n_rot, sec, base))
        assert np.abs(out.cpu().numpy() - want).max() <= 2e-6 * np.abs(want).max(), label
        rows = n_tok + 5
        idx = r2.permutation(rows)[:n_tok].astype(np.int64)
        init = r2.integers(0, 256, (rows, n_head * D // 32 * 18), dtype=np.uint8)
        wq = orc.rope_norm_set_rows_q4_0(init.copy(), src, w if use_w else None, EPS, pos, rp, idx)
        cache = torch.from_numpy(init.copy()).to(dev)
        sqa.rope_norm_set_rows_q4_0(cache, torch.from_numpy(src).to(dev), wt, EPS, torch.from_numpy(pos).to(dev),
                                    sqa.rope_params(n_rot, sec, base), torch.from_numpy(idx).to(dev))
        got = cache.cpu().numpy()
        others = np.setdiff1d(np.arange(rows), idx)
        assert np.array_equal(got[others], init[others]), label
        _compare_q4(got[idx], wq[idx], D)
