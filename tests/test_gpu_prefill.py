"""MFMA prefill flash_attn_ext on the GPU against the oracle's ggml CPU
flash_attn_ext on identical inputs (ubatch chunks appended after a cached
prefix, src/engine/runner.rs:1104-1108 in the reference). Tolerance:
max |gpu - oracle| <= 2e-3 * rms(oracle)."""
import numpy as np
import pytest
import torch

from tests import fa_ref
from tests.gen import qkv, rel_err
from tests.test_gpu_decode import run_gpu

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.mark.parametrize("n_q,n_kv,start", [(3, 256, 200), (64, 1024, 960), (100, 777, 600), (512, 4096, 3584)])
def test_prefill_causal_mask(sqa, orc, dev, n_q, n_kv, start):
    q, kq, vq = qkv(orc, n_q + n_kv, n_q, n_kv)
    mask = orc.causal_mask(n_q, n_kv, start)
    ref = orc.flash_attn_ext(q, kq, vq, mask)
    got = run_gpu(sqa, dev, q, kq, vq, mask)
    err = rel_err(got, ref)
    print(f"prefill n_q={n_q} n_kv={n_kv}: max err / rms = {err:.3e}")
    assert err <= TOL


def test_prefill_pp512_after_16k(sqa, orc, dev):
    """ubatch 512 appended after 16384 cached tokens: 16896 keys, causal."""
    q, kq, vq = qkv(orc, 4, 512, 16896)
    mask = orc.causal_mask(512, 16896, 16384)
    ref = orc.flash_attn_ext(q, kq, vq, mask)
    got = run_gpu(sqa, dev, q, kq, vq, mask)
    err = rel_err(got, ref)
    print(f"pp512 @16384: max err / rms = {err:.3e}")
    assert err <= TOL


def test_prefill_causal_positions_gate(sqa, orc, dev):
    q, kq, vq = qkv(orc, 5, 200, 2048)
    gate = np.random.default_rng(6).standard_normal(q.shape).astype(np.float32)
    ref = orc.flash_attn_ext_causal(q, kq, vq, 1848, gate=gate)
    got = run_gpu(sqa, dev, q, kq, vq, causal=1848, gate=gate)
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("H,Hkv,n_q", [(4, 1, 40), (16, 16, 40), (8, 4, 40), (16, 16, 200), (4, 2, 150)])
def test_prefill_other_gqa_ratios(sqa, orc, dev, H, Hkv, n_q):
    """G = 1 puts 128 query positions in one workgroup (the mask staging of
    every position is exercised with n_q = 200)."""
    q, kq, vq = qkv(orc, H + n_q, n_q, 600, H=H, Hkv=Hkv)
    mask = orc.causal_mask(n_q, 600, 600 - n_q)
    ref = orc.flash_attn_ext(q, kq, vq, mask)
    got = run_gpu(sqa, dev, q, kq, vq, mask)
    assert rel_err(got, ref) <= TOL


def test_prefill_fully_masked_rows_are_zero(sqa, orc, dev):
    q, kq, vq = qkv(orc, 9, 32, 512)
    mask = orc.causal_mask(32, 512, 400)
    mask[5] = -np.inf
    ref = orc.flash_attn_ext(q, kq, vq, mask)
    got = run_gpu(sqa, dev, q, kq, vq, mask)
    assert np.all(got[5] == 0)
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("n_q", [2, 64])
def test_rising_logits_force_rescales(sqa, orc, dev, n_q):
    """A mask rising by 0.05 per key (natural-log units) lifts the running
    maximum every few tiles, so the online softmax rescales its accumulator
    many times (the decode kernel for n_q = 2, the prefill kernel for 64)."""
    n_kv = 3000
    q, kq, vq = qkv(orc, 77 + n_q, n_q, n_kv)
    causal = orc.causal_mask(n_q, n_kv, n_kv - n_q).astype(np.float32)
    ramp = np.arange(n_kv, dtype=np.float32) * np.float32(0.05)
    mask = (causal + ramp[None, :]).astype(np.float16)
    ref = orc.flash_attn_ext(q, kq, vq, mask)
    got = run_gpu(sqa, dev, q, kq, vq, mask)
    err = rel_err(got, ref)
    print(f"rising logits n_q={n_q}: max err / rms = {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("H,Hkv,n_q", [(4, 2, 6), (4, 1, 1), (8, 4, 3), (16, 2, 5)])
def test_small_chunks_at_other_gqa_ratios(sqa, orc, dev, H, Hkv, n_q):
    """Up to 4 positions with at most 16 query rows per KV head run on the
    split-KV decode kernel whatever n_head_kv is ((4, 1, 1), (8, 4, 3)); more
    positions run as prefill chunks whatever their row count."""
    q, kq, vq = qkv(orc, 31 + n_q, n_q, 700, H=H, Hkv=Hkv)
    mask = orc.causal_mask(n_q, 700, 700 - n_q)
    ref = orc.flash_attn_ext(q, kq, vq, mask)
    got = run_gpu(sqa, dev, q, kq, vq, mask)
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("n_q,n_kv,start", [(64, 64, 0), (300, 512, 0), (494, 512, 17)])
def test_chunk_at_context_start_with_outliers(sqa, orc, dev, n_q, n_kv, start):
    """The first ubatch of a prompt: early rows see a few keys, so their outputs
    are a handful of V rows at full size next to rows averaging hundreds of
    keys (1% of the channels x8): an fp16 rounding of P d_v would show."""
    q, kq, vq = qkv(orc, 500 + n_q, n_q, n_kv, outliers=5)
    mask = orc.causal_mask(n_q, n_kv, start)
    ref = orc.flash_attn_ext(q, kq, vq, mask)
    got = run_gpu(sqa, dev, q, kq, vq, mask)
    err = rel_err(got, ref)
    print(f"prefill chunk n_q={n_q} start={start} outliers: max err / rms = {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("scale_v", [1e-4, 3e-2, 500.0, 2000.0, 8000.0])
def test_prefill_v_scale_range(sqa, orc, dev, scale_v):
    """V of any finite size: the softmax weights carry 2^ep and the lazy rescale
    a slack of ks binades, both from the largest |d_v| of the head, so that
    P d_v keeps 22 bits without overflow. 1e-4 reaches ep = 7; 500 (largest
    |d_v| about 1800, on the outlier channels) a slack of 4 with ep = 0; 2000
    and 8000 (|d_v| about 7400 and 29500) ep = -1 and -3 with a slack of 3."""
    q, kq, vq = qkv(orc, 77, 300, 512, outliers=5, scale_v=scale_v)
    mask = orc.causal_mask(300, 512, 212)
    ref = orc.flash_attn_ext(q, kq, vq, mask)
    got = run_gpu(sqa, dev, q, kq, vq, mask)
    err = rel_err(got, ref)
    dv = np.abs(vq.reshape(-1, 18)[:, :2].copy().view(np.float16)).max()
    print(f"prefill V x{scale_v} (max |d_v| {dv:.3g}): max err / rms = {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("seed", [100, 101])
def test_prefill_large_v_outliers_against_f64(sqa, orc, dev, seed):
    """Large V (x17.7, 8 outlier channels x8: max |d_v| about 50) over 3 KV
    heads of 16 query heads. The weight of P on 2^ep must not push the P of keys
    a few binades below the row maximum into the fp16 subnormals (ep = e2 did:
    3e-4 to 1.1e-3 x RMS from the exact result over these seeds); measured
    against a float64 brute force on the dequantized operands, as ggml's fp32
    CPU path is itself ~1e-3 off here."""
    n_q, n_kv = 40, 2807
    q, kq, vq = qkv(orc, seed, n_q, n_kv, H=48, Hkv=3, outliers=8, scale_v=17.7)
    mask = orc.causal_mask(n_q, n_kv, n_kv - n_q)
    got = run_gpu(sqa, dev, q, kq, vq, mask)
    exact = fa_ref.attention_f64(fa_ref.q8_dequant(orc, q), fa_ref.cache_dequant(orc, kq),
                                 fa_ref.cache_dequant(orc, vq), 1 / 16, mask)
    err = rel_err(got, exact)
    print(f"large V seed {seed}: gpu vs f64 {err:.3e}")
    assert err <= TOL / 10


def test_prefill_masked_rows_with_garbage_bytes(sqa, orc, dev):
    """Masked cache rows holding 0xFF bytes (NaN block scales, what an unzeroed
    buffer may hold) or stale rows of other data (a rewound draft) do not change
    the output (ggml's CPU loop never reads them)."""
    n_q, n_kv = 40, 1200
    q, kq, vq = qkv(orc, 43, n_q, n_kv)
    rng = np.random.default_rng(44)
    dead = rng.choice(n_kv - n_q, 400, replace=False)
    _, k_old, v_old = qkv(orc, 45, 1, len(dead) - 200)
    kq, vq = kq.copy(), vq.copy()
    kq[dead[:200]] = 0xFF
    vq[dead[:200]] = 0xFF
    kq[dead[200:]] = k_old
    vq[dead[200:]] = v_old
    mask = orc.causal_mask(n_q, n_kv, n_kv - n_q)
    mask[:, dead] = -np.inf
    ref = orc.flash_attn_ext(q, kq, vq, mask)
    assert np.all(np.isfinite(ref))
    got = run_gpu(sqa, dev, q, kq, vq, mask)
    assert np.all(np.isfinite(got))
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("n_q,n_kv,unaligned", [(200, 3000, False), (300, 1500, True), (64, 4096, False)])
def test_prefill_mask_trim_with_irregular_masks(sqa, orc, dev, n_q, n_kv, unaligned):
    """The mask path stops each query tile at the last key any of its rows
    leaves visible. Rows here end their visible keys at random places (not a
    causal staircase), some have -inf holes before that end, one row is fully
    masked, and masked keys hold 0xFF bytes: the trimmed kernel must match the
    oracle. unaligned: n_kv % 8 != 0 and an odd row stride (the packed copy is
    what gets scanned)."""
    if unaligned:
        n_kv += 3
    rng = np.random.default_rng(n_q + n_kv)
    q, kq, vq = qkv(orc, 2000 + n_q, n_q, n_kv)
    mask = np.zeros((n_q, n_kv), dtype=np.float16)
    ends = rng.integers(1, n_kv + 1, n_q)
    for r in range(n_q):
        mask[r, ends[r]:] = -np.inf
        holes = rng.choice(ends[r], min(ends[r] - 1, 5), replace=False) if ends[r] > 1 else []
        mask[r, holes] = -np.inf
    mask[n_q // 3] = -np.inf
    kq, vq = kq.copy(), vq.copy()
    dead = np.where(np.all(np.isinf(mask), axis=0))[0]
    kq[dead] = 0xFF
    vq[dead] = 0xFF
    ref = orc.flash_attn_ext(q, kq, vq, mask)
    if unaligned:  # rows with a stride of n_kv + 1 halfs
        buf = np.full((n_q, n_kv + 1), -np.inf, dtype=np.float16)
        buf[:, :n_kv] = mask
        qt = torch.from_numpy(q).to(dev)
        kt = torch.from_numpy(np.ascontiguousarray(kq)).to(dev)
        vt = torch.from_numpy(np.ascontiguousarray(vq)).to(dev)
        mt = torch.from_numpy(buf).to(dev)[:, :n_kv]
        got = sqa.flash_attn_ext(qt, kt, vt, n_kv, mask=mt, scale=1 / 16)
        torch.cuda.synchronize()
        got = got.cpu().numpy()
    else:
        got = run_gpu(sqa, dev, q, kq, vq, mask)
    assert np.all(np.isfinite(got))
    err = rel_err(got, ref)
    print(f"irregular mask n_q={n_q} n_kv={n_kv}: max err / rms = {err:.3e}")
    assert err <= TOL


def test_mask_form_start_chunk_costs_what_the_causal_form_does(sqa, orc, dev):
    """The first chunk of a prompt (512 queries at positions 0..511) through the
    engine's F16 mask: half of its key tiles are masked in every row of their
    query tile and must be skipped as the causal-from-positions form skips them.
    Parity first, then the main kernel's time (HIP events, median of 7 rounds of
    10 calls, the two forms alternating) within 10% of the causal form's."""
    n_q = n_kv = 512
    q, kq, vq = qkv(orc, 4242, n_q, n_kv, outliers=5)
    mask = orc.causal_mask(n_q, n_kv, 0)
    ref = orc.flash_attn_ext(q, kq, vq, mask)
    qt = torch.from_numpy(q).to(dev)
    kt = torch.from_numpy(np.ascontiguousarray(kq)).to(dev)
    vt = torch.from_numpy(np.ascontiguousarray(vq)).to(dev)
    mt = torch.from_numpy(mask).to(dev)
    out = torch.empty((n_q, 16, 256), device=dev)
    ws = torch.empty(sqa.flash_attn_workspace_size(qt, kt, n_kv), dtype=torch.uint8, device=dev)
    sqa.flash_attn_ext(qt, kt, vt, n_kv, mask=mt, scale=1 / 16, out=out, workspace=ws)
    torch.cuda.synchronize()
    assert rel_err(out.cpu().numpy(), ref) <= TOL
    forms = {"mask": lambda: sqa.flash_attn_ext(qt, kt, vt, n_kv, mask=mt, scale=1 / 16, out=out, workspace=ws),
             "causal": lambda: sqa.flash_attn_ext_causal(qt, kt, vt, n_kv, 0, scale=1 / 16, out=out, workspace=ws)}
    times = {k: [] for k in forms}
    for r in range(7):
        for name in (("mask", "causal") if r % 2 == 0 else ("causal", "mask")):
            sqa.profile_begin(64)
            for _ in range(10):
                forms[name]()
            torch.cuda.synchronize()
            sqa.profile_end()
            t, c = sqa.profile_get("fa_prefill")
            times[name].append(t / c)
    med = {k: sorted(v)[len(v) // 2] for k, v in times.items()}
    print(f"start chunk 512x512: fa_prefill mask form {1e3 * med['mask']:.2f} us, "
          f"causal form {1e3 * med['causal']:.2f} us")
    assert med["mask"] <= 1.10 * med["causal"]
