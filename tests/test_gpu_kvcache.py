"""The engine's KV-cache call sequence on the GPU, checked against the oracle at
every step (reference: tests/attn_test.rs:517-587 run_steps_full and :742-779
attn_decode_after_prefill_matches_cpu; src/engine/kv.rs:150-170, 211-297,
313-447; mask fill src/model/graph.rs:486-576).

Per step: KvCache.begin_step(n) reserves rows [step_start, step_start + n);
each layer quantizes its n new K and V rows into the cache through
sqa_kv_cache_append at idx = step_start + j; the F16 causal mask is filled on
the device over n_kv_padded keys; flash_attn_ext runs over the library's own
k_view/v_view of [0, n_kv_padded). The oracle runs on a host copy of the same
cache rows with the same mask. The caches start as 0xFF bytes (NaN scales) and
are zeroed once, as the engine does at load: the padded rows past n_used are
then exact zeros and are masked. A rewind (MTP rejecting drafted tokens) leaves
stale rows past the cursor, which stay masked. One decode step is captured in a
HIP graph and replayed at three positions, each replay checked against the
oracle."""
import numpy as np
import pytest
import torch

from tests.gen import rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-3
H, HKV, D = 16, 2, 256
RB = D // 32 * 18
N_LAYERS, CAP = 2, 3000


def _host(kv, slot, n_pad):
    return kv.k[slot][:n_pad].cpu().numpy(), kv.v[slot][:n_pad].cpu().numpy()


def _check_layer(kv, orc, slot, q, mask, out, k_cur, v_cur, s0, label):
    n_pad = kv.n_kv_padded()
    kh, vh = _host(kv, slot, n_pad)
    n = k_cur.shape[0]
    # quantize-on-write landed at rows s0..s0+n, bit-exact
    assert np.array_equal(kh[s0:s0 + n], orc.quantize_q4_0(k_cur.cpu().numpy()).reshape(n, HKV, RB)), label
    assert np.array_equal(vh[s0:s0 + n], orc.quantize_q4_0(v_cur.cpu().numpy()).reshape(n, HKV, RB)), label
    mh = mask.cpu().numpy()
    assert np.array_equal(mh, orc.causal_mask(n, n_pad, s0)), label
    ref = orc.flash_attn_ext(q.cpu().numpy(), kh, vh, mh)
    got = out.cpu().numpy()
    assert np.all(np.isfinite(got)), label
    err = rel_err(got, ref)
    print(f"{label} layer {slot}: n_used={kv.n_used} n_kv_padded={n_pad} max err / rms = {err:.3e}")
    assert err <= TOL, label


def _step(sqa, kv, orc, gen, dev, n, label, n_layers=N_LAYERS):
    kv.begin_step(n)
    s0 = kv.step_start
    n_pad = kv.n_kv_padded()
    assert n_pad == (kv.n_used + 255) // 256 * 256
    idx = torch.arange(s0, s0 + n, device=dev, dtype=torch.int64)
    mask = torch.empty((n, n_pad), dtype=torch.float16, device=dev)
    sqa.fill_causal_mask(mask, s0)
    for slot in range(n_layers):
        k_cur = torch.randn((n, HKV * D), generator=gen, device=dev)
        v_cur = torch.randn((n, HKV * D), generator=gen, device=dev)
        q = torch.randn((n, H, D), generator=gen, device=dev)
        kv.append(slot, k_cur, v_cur, idx)
        out = kv.attend(slot, q, mask=mask)
        torch.cuda.synchronize()
        _check_layer(kv, orc, slot, q, mask, out, k_cur, v_cur, s0, label)
    return s0


def test_prefill_then_decode_through_kv_cache(sqa, orc, dev):
    gen = torch.Generator(device=dev)
    gen.manual_seed(517)
    kv = sqa.KvCache(N_LAYERS, D, HKV, CAP, device=dev)
    assert kv.kv_cap_alloc == 3072
    for t in kv.k + kv.v:
        t.fill_(0xFF)  # what uninitialised memory may hold: NaN block scales
    kv.zero_caches()
    # a 16-token prefill chunk, then one decode step (attn_test.rs:742-779)
    _step(sqa, kv, orc, gen, dev, 16, "prefill 16")
    _step(sqa, kv, orc, gen, dev, 1, "decode after prefill")
    # a longer chunk that crosses the first 256-row padding boundary
    _step(sqa, kv, orc, gen, dev, 494, "prefill 494")
    assert kv.n_used == 511 and kv.n_kv_padded() == 512
    for i in range(3):  # 511 -> 512 -> 513: n_kv_padded moves from 512 to 768
        _step(sqa, kv, orc, gen, dev, 1, f"decode {i}")
    assert kv.n_used == 514 and kv.n_kv_padded() == 768
    # rows past the cursor are still the zeros written at load
    for slot in range(N_LAYERS):
        kh, vh = _host(kv, slot, 768)
        assert not kh[514:].any() and not vh[514:].any()

    # MTP verify of two tokens, then reject the draft: rewind by one and re-decode
    _step(sqa, kv, orc, gen, dev, 2, "verify n_q=2")
    kv.rewind_to(kv.n_used - 1)
    s0 = _step(sqa, kv, orc, gen, dev, 1, "decode after rewind")
    assert s0 == 515 and kv.n_used == 516


def test_mtp_head_cache_beside_the_trunk(sqa, orc, dev):
    """The MTP head runs the same full-attention layer over a KV cache of its own
    (reference: src/model/mtp.rs:78 KvCache::new(.., 1 layer, ..) and :186-199
    build_attn_layer on st.kv): a catch-up over the committed tokens (n >= 1),
    then one draft position at a time (n = 1), interleaved with the trunk's
    decode and verify steps and its rewind after a rejected draft. Both caches
    go through the same library calls; every attention output is checked
    against the oracle on a host copy of its own cache."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(193)
    trunk = sqa.KvCache(N_LAYERS, D, HKV, CAP, device=dev)
    mtp = sqa.KvCache(1, D, HKV, 1000, device=dev)
    for kv in (trunk, mtp):
        for t in kv.k + kv.v:
            t.fill_(0xFF)
        kv.zero_caches()
    _step(sqa, trunk, orc, gen, dev, 16, "trunk prefill 16")
    _step(sqa, mtp, orc, gen, dev, 16, "mtp catch-up 16", n_layers=1)
    for i in range(3):
        _step(sqa, mtp, orc, gen, dev, 1, f"mtp draft {i}", n_layers=1)
        _step(sqa, trunk, orc, gen, dev, 2, f"trunk verify {i}")
        if i % 2 == 0:  # draft rejected: both caches drop it
            trunk.rewind_to(trunk.n_used - 1)
            mtp.rewind_to(mtp.n_used - 1)
            _step(sqa, mtp, orc, gen, dev, 1, f"mtp catch-up {i}", n_layers=1)
    assert trunk.n_used == 16 + 2 * 3 - 2 and mtp.n_used == 16 + 3


def test_graph_replayed_decode_step_matches_oracle(sqa, orc, dev):
    gen = torch.Generator(device=dev)
    gen.manual_seed(779)
    kv = sqa.KvCache(1, D, HKV, CAP, device=dev)
    kv.zero_caches()
    _step(sqa, kv, orc, gen, dev, 600, "prefill 600", 1)  # n_used 600, n_kv_padded 768 for the next steps
    _step(sqa, kv, orc, gen, dev, 1, "eager decode", 1)   # kernel attributes are set outside the capture

    # the step's fixed buffers (graph replay needs stable pointers, kv.rs:299-311)
    idx = torch.empty((1,), dtype=torch.int64, device=dev)
    k_cur = torch.empty((1, HKV * D), device=dev)
    v_cur = torch.empty((1, HKV * D), device=dev)
    q = torch.empty((1, H, D), device=dev)
    out = torch.empty((1, H, D), device=dev)
    n_pad = kv.n_kv_padded_after(1)
    mask = torch.empty((1, n_pad), dtype=torch.float16, device=dev)
    kv.begin_step(1)
    ws = torch.empty(max(kv.workspace_size(0, q), 1), dtype=torch.uint8, device=dev)

    def body():
        kv.append(0, k_cur, v_cur, idx)
        kv.attend(0, q, mask=mask, out=out, workspace=ws)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            body()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    for r in range(3):
        if r > 0:
            kv.begin_step(1)
        s0 = kv.step_start
        assert kv.n_kv_padded() == n_pad
        idx.fill_(s0)
        k_cur.copy_(torch.randn((1, HKV * D), generator=gen, device=dev))
        v_cur.copy_(torch.randn((1, HKV * D), generator=gen, device=dev))
        q.copy_(torch.randn((1, H, D), generator=gen, device=dev))
        sqa.fill_causal_mask(mask, s0)  # filled outside the graph, as the engine fills it
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        _check_layer(kv, orc, 0, q, mask, out, k_cur, v_cur, s0, f"graph replay {r}")
