"""The long-prefill attention stack at its real shape: ubatch 2048 appended after
131072 cached tokens (133120 keys), 16q/2kv heads, hd256, q4_0 K/V. One layer
of the stack runs set_rows (the 2048 new K/V rows quantized on write) ->
flash_attn_ext -> sigmoid output gate (reference: src/engine/kv.rs:313-399,
src/model/attn.rs:238-251, :282-283), in both forms the library offers:

  mask  : the engine's F16 causal mask through flash_attn_ext, then the
          separate sigmoid_mul kernel;
  fused : causal-from-positions through flash_attn_ext_causal with the gate
          applied in the attention kernel's own epilogue (one key split at this
          shape, so no split merge runs).

The oracle runs on 16 sampled query positions (first, last and interior) with
all 16 heads, each against its own mask row: max |gpu - oracle| <= 2e-3 *
rms(oracle) over those rows."""
import numpy as np
import pytest
import torch

from tests.gen import rel_err
from tests.test_gpu_decode import run_gpu

pytestmark = pytest.mark.gpu
TOL = 2e-3
H, HKV, D = 16, 2, 256
RB = D // 32 * 18


def _fill_cache(sqa, dev, gen, n_rows, n_total):
    """q4_0 cache of n_total rows; rows [0, n_rows) from N(0,1) by set_rows."""
    cache = torch.zeros((n_total, HKV, RB), dtype=torch.uint8, device=dev)
    chunk = 16384
    for r0 in range(0, n_rows, chunk):
        n = min(chunk, n_rows - r0)
        src = torch.randn((n, HKV * D), generator=gen, device=dev)
        sqa.set_rows_q4_0(cache, src, torch.arange(r0, r0 + n, device=dev, dtype=torch.int64))
    return cache


def _sample_positions(n_q, count, seed):
    rng = np.random.default_rng(seed)
    inner = rng.choice(np.arange(1, n_q - 1), count - 2, replace=False)
    return np.sort(np.concatenate([[0, n_q - 1], inner])).astype(np.int64)


def test_stack_layer_ub2048_at_131072(sqa, orc, dev):
    n_q, start = 2048, 131072
    n_kv = start + n_q
    gen = torch.Generator(device=dev)
    gen.manual_seed(2048)
    kc = _fill_cache(sqa, dev, gen, start, n_kv)
    vc = _fill_cache(sqa, dev, gen, start, n_kv)
    # the layer's 2048 new K/V rows, quantized on write at 131072..133119
    k_new = torch.randn((n_q, HKV * D), generator=gen, device=dev)
    v_new = torch.randn((n_q, HKV * D), generator=gen, device=dev)
    idx = torch.arange(start, n_kv, device=dev, dtype=torch.int64)
    sqa.set_rows_q4_0(kc, k_new, idx)
    sqa.set_rows_q4_0(vc, v_new, idx)
    q = torch.randn((n_q, H, D), generator=gen, device=dev)
    gate = torch.randn((n_q, H, D), generator=gen, device=dev)

    # form 1: F16 mask + unfused gate
    mask = torch.empty((n_q, n_kv), dtype=torch.float16, device=dev)
    sqa.fill_causal_mask(mask, start)
    attn = sqa.flash_attn_ext(q, kc, vc, n_kv, mask=mask)
    out_mask = sqa.sigmoid_mul(attn.view(n_q, H * D), gate.view(n_q, H * D)).view(n_q, H, D)
    # form 2: causal from positions, gate fused into the attention epilogue
    sqa.profile_begin(64)
    try:
        out_fused = sqa.flash_attn_ext_causal(q, kc, vc, n_kv, start, gate=gate)
        torch.cuda.synchronize()
    finally:
        sqa.profile_end()
    assert sqa.profile_get("fa_prefill")[1] == 1
    assert sqa.profile_get("fa_combine")[1] == 0, "expected one key split (gate in the kernel epilogue)"

    rows = _sample_positions(n_q, 16, 5)
    kh, vh = kc.cpu().numpy(), vc.cpu().numpy()
    # the new rows landed bit-exact where set_rows put them
    assert np.array_equal(kh[start:], orc.quantize_q4_0(k_new.cpu().numpy()).reshape(n_q, HKV, RB))
    assert np.array_equal(vh[start:], orc.quantize_q4_0(v_new.cpu().numpy()).reshape(n_q, HKV, RB))
    qh = q.cpu().numpy()[rows]
    gh = gate.cpu().numpy()[rows]
    mh = mask[torch.from_numpy(rows).to(dev)].cpu().numpy()
    assert np.array_equal(mh, orc.causal_mask(n_q, n_kv, start)[rows])
    ref_attn = orc.flash_attn_ext(qh, kh, vh, mh)
    ref = orc.sigmoid_mul(ref_attn.reshape(len(rows), H * D), gh.reshape(len(rows), H * D)).reshape(ref_attn.shape)
    ref_causal = np.concatenate([orc.flash_attn_ext_causal(qh[i:i + 1], kh, vh, start + int(r), gate=gh[i:i + 1])
                                 for i, r in enumerate(rows)])
    assert rel_err(ref_causal, ref) <= 1e-6  # the two oracle forms agree
    e_mask = rel_err(out_mask.cpu().numpy()[rows], ref)
    e_fused = rel_err(out_fused.cpu().numpy()[rows], ref)
    print(f"ub2048 @131072, 16 sampled positions x 16 heads: mask form {e_mask:.3e}, fused form {e_fused:.3e}")
    assert e_mask <= TOL and e_fused <= TOL


@pytest.mark.parametrize("n_q,n_kv,q_pos0", [(64, 500, 436), (300, 512, 212)])
def test_prefill_gate_in_kernel_epilogue(sqa, orc, dev, n_q, n_kv, q_pos0):
    """Short key ranges get one split, so the gate runs in the attention kernel's
    epilogue rather than in the split merge."""
    from tests.gen import qkv

    q, kq, vq = qkv(orc, n_q + q_pos0, n_q, n_kv)
    gate = np.random.default_rng(n_kv).standard_normal(q.shape).astype(np.float32)
    ref = orc.flash_attn_ext_causal(q, kq, vq, q_pos0, gate=gate)
    sqa.profile_begin(16)
    try:
        got = run_gpu(sqa, dev, q, kq, vq, causal=q_pos0, gate=gate)
    finally:
        sqa.profile_end()
    assert sqa.profile_get("fa_prefill")[1] == 1
    assert sqa.profile_get("fa_combine")[1] == 0
    err = rel_err(got, ref)
    print(f"gate epilogue n_q={n_q} n_kv={n_kv}: max err / rms = {err:.3e}")
    assert err <= TOL
