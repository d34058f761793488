"""A decode step captured once in a HIP graph and replayed (the reference keeps
the cache pointers fixed so that ggml-cuda can replay the step's graph,
src/engine/kv.rs:299-311): the K producer into the cache row, V set_rows, the Q
producer, and flash_attn_ext over the cache with the step's F16 mask. Every
replay, with new contents in the input buffers (rows, positions, Q/K/V) and
eager work between replays, must equal the same calls run eagerly, byte for byte.
The mask is filled eagerly before each replay, as the engine fills it."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

D, HKV, H, N_KV, EPS = 256, 2, 16, 2048, 1e-6


def test_decode_step_graph_replay_matches_eager(sqa, dev):
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    rope = sqa.rope_params(64, (11, 11, 10, 0), 1e7)
    rb = D // 32 * 18
    kc = torch.zeros((N_KV, HKV, rb), dtype=torch.uint8, device=dev)
    vc = torch.zeros_like(kc)
    n0 = 1500
    idx0 = torch.arange(n0, device=dev, dtype=torch.int64)
    pos0 = torch.arange(n0, device=dev, dtype=torch.int32).repeat(4)
    kw = 1 + 0.1 * torch.randn((D,), generator=gen, device=dev)
    qw = 1 + 0.1 * torch.randn((D,), generator=gen, device=dev)
    sqa.rope_norm_set_rows_q4_0(kc, torch.randn((n0, HKV, D), generator=gen, device=dev), kw, EPS, pos0, rope, idx0)
    sqa.set_rows_q4_0(vc, torch.randn((n0, HKV * D), generator=gen, device=dev), idx0)

    # static buffers of the step
    k_src = torch.empty((1, HKV, D), device=dev)
    v_src = torch.empty((1, HKV * D), device=dev)
    q_src = torch.empty((1, H, D), device=dev)
    q = torch.empty((1, H, D), device=dev)
    idx = torch.empty((1,), dtype=torch.int64, device=dev)
    pos = torch.empty((4,), dtype=torch.int32, device=dev)
    mask = torch.empty((1, N_KV), dtype=torch.float16, device=dev)
    out = torch.empty((1, H, D), device=dev)
    ws = torch.empty(sqa.flash_attn_workspace_size(q, kc, N_KV), dtype=torch.uint8, device=dev)

    def step():
        sqa.rope_norm_set_rows_q4_0(kc, k_src, kw, EPS, pos, rope, idx)
        sqa.set_rows_q4_0(vc, v_src, idx)
        sqa.rope_norm_f32(q, q_src, qw, EPS, pos, rope)
        sqa.flash_attn_ext(q, kc, vc, N_KV, mask=mask, out=out, workspace=ws)

    def load_inputs(t):
        k_src.copy_(torch.randn((1, HKV, D), generator=gen, device=dev))
        v_src.copy_(torch.randn((1, HKV * D), generator=gen, device=dev))
        q_src.copy_(torch.randn((1, H, D), generator=gen, device=dev))
        idx.fill_(t)
        pos.fill_(t)
        sqa.fill_causal_mask(mask, t)

    load_inputs(n0)
    step()  # eager first call: one-time kernel attributes are set outside the capture
    torch.cuda.synchronize()

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    for t in range(n0, n0 + 5):
        load_inputs(t)
        k_before, v_before = kc.clone(), vc.clone()
        g.replay()
        torch.cuda.synchronize()
        got_out, got_k, got_v = out.clone(), kc.clone(), vc.clone()
        kc.copy_(k_before)
        vc.copy_(v_before)
        out.zero_()
        step()
        torch.cuda.synchronize()
        assert torch.equal(got_k, kc), t
        assert torch.equal(got_v, vc), t
        assert torch.equal(got_out, out), t
        assert torch.isfinite(out).all()
        # the replay wrote row t and nothing else
        changed = (got_k != k_before).flatten(1).any(1).nonzero().flatten().tolist()
        assert changed == [t], changed
