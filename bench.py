"""Benchmark of the full-attention hot path on one MI355X.

Workload (the headline shape): long-context decode, n_q = 1, 16 query heads /
2 KV heads, head_dim 256, q4_0 K and V, KV length 172032, over 10 independent
full-attention layers (990.9 MB of cache, larger than the 256 MB MALL, so the
layers cannot be served from cache). A step is one decode token through the
10 layers: per layer one flash_attn_ext call (split-KV kernel + combine) with
the engine's F16 mask. K/V ~ N(0,1) are quantized on the GPU by the q4_0
set_rows kernel; Q ~ N(0,1). Synthetic data, seeded.

Metric: achieved HBM GB/s = algorithmic bytes / time, where the algorithmic
bytes of one layer are n_kv*576 (K+V) + 2*16*256*4 (Q, O) + n_kv*2 (mask).

Prints ONE JSON line (rank 0). Extra fields: per-layer microseconds, the
roofline of the dominant kernel (fa_decode), the CPU oracle timed on this
host, the MTP verify (n_q = 2) marginal cost, the decode time split into a
per-byte and a fixed part over KV lengths at one split count, and the prefill leg:
pp512 = a 512-token ubatch appended after 16384 cached tokens (n_kv = 16896,
causal F16 mask), 10 layers, reported as attention TFLOP/s against the fp16
MFMA peak. Its FLOPs count QK^T and PV over the keys each query may see:
4 * head_dim * n_head * sum_i (16384 + i + 1).

--copy-ref appends a plain 256 MiB device copy so that hardware counters of
the same run can be scaled by a kernel of known traffic.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA, MI355X
PP_N_Q, PP_START = 512, 16384
STACK_N_Q, STACK_START = 2048, 131072
# HBM bytes per fa_decode launch at 172K (n_q = 1), from rocprofv3 counter
# passes over this script: 2.0 x FETCH_SIZE + 1.0 x WRITE_SIZE (KiB x 1024),
# the factors taken from a plain 256 MiB copy in the same run
# (profiles/fa_decode_verify_172k_pp512_out_proj_hbm_traffic.txt).
DECODE_TRAFFIC_BYTES = int((2.0 * 48758.8 + 4160.0) * 1024)
H, HKV, D = 16, 2, 256
N_LAYERS = 10
N_KV = 172032
ROW = 576  # K + V bytes per token per layer (2 kv heads x 144 B x 2)


def layer_bytes(n_kv, n_q, with_mask=True):
    return n_kv * ROW + 2 * n_q * H * D * 4 + (n_kv * n_q * 2 if with_mask else 0)


def fill_caches(sqa, torch, dev, n_layers, n_kv, seed):
    """Quantize N(0,1) rows into q4_0 caches with the set_rows kernel."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    ks, vs = [], []
    chunk = 16384
    for _ in range(n_layers):
        pair = []
        for _ in range(2):
            cache = torch.empty((n_kv, HKV, D // 32 * 18), dtype=torch.uint8, device=dev)
            for r0 in range(0, n_kv, chunk):
                n = min(chunk, n_kv - r0)
                src = torch.randn((n, HKV * D), generator=gen, device=dev, dtype=torch.float32)
                idx = torch.arange(r0, r0 + n, device=dev, dtype=torch.int64)
                sqa.set_rows_q4_0(cache, src, idx)
            pair.append(cache)
        ks.append(pair[0])
        vs.append(pair[1])
    torch.cuda.synchronize()
    return ks, vs


def time_steps(torch, fn, steps):
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b)  # ms


def capture(torch, fn):
    """fn captured once in a HIP graph (on a side stream, after one eager call)."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    return g


def verify_leg(sqa, torch, dev, ks, vs, steps, lengths=(32768, 131072, N_KV), graphs=True):
    """MTP verify (n_q = 2: the current token plus one draft, causal across the
    two rows) against plain decode (n_q = 1) over the first n_kv rows of the 10
    layers' caches, at each KV length in lengths (32768, 131072 and 172032
    keys by default). Each 10-layer step is
    captured in a HIP graph and replayed, so the figures are GPU time (at 32K a
    layer takes less GPU time than the Python wrapper takes to launch it, and
    eager launches would time the host); the two step kinds alternate within
    one loop, each bracketed by its own events, so the marginal cost of the
    draft row is a difference of neighbouring steps. Kernel times come from one
    more eager pass with the library's event hooks; roofline = algorithmic
    bytes / fa_decode time. graphs=False times eager launches instead (for
    counter collection, which serialises every dispatch)."""
    out = {}
    for n_kv in lengths:
        q1 = torch.randn((1, H, D), device=dev)
        q2 = torch.randn((2, H, D), device=dev)
        m1 = torch.empty((1, n_kv), dtype=torch.float16, device=dev)
        m2 = torch.empty((2, n_kv), dtype=torch.float16, device=dev)
        sqa.fill_causal_mask(m1, n_kv - 1)
        sqa.fill_causal_mask(m2, n_kv - 2)
        o1 = torch.empty((1, H, D), device=dev)
        o2 = torch.empty((2, H, D), device=dev)
        w1 = torch.empty(sqa.flash_attn_workspace_size(q1, ks[0], n_kv), dtype=torch.uint8, device=dev)
        w2 = torch.empty(sqa.flash_attn_workspace_size(q2, ks[0], n_kv), dtype=torch.uint8, device=dev)

        def run(q, m, o, w):
            for li in range(N_LAYERS):
                sqa.flash_attn_ext(q, ks[li], vs[li], n_kv, mask=m, out=o, workspace=w)

        run1 = lambda: run(q1, m1, o1, w1)
        run2 = lambda: run(q2, m2, o2, w2)
        if graphs:
            g1, g2 = capture(torch, run1), capture(torch, run2)
            rep1, rep2 = g1.replay, g2.replay
        else:
            g1 = g2 = None
            rep1, rep2 = run1, run2
        for _ in range(3):
            rep1()
            rep2()
        rounds = max(10, steps)
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(rounds)]
        torch.cuda.synchronize()
        for r in range(rounds):
            ev[r][0].record()
            rep1()
            ev[r][1].record()
            rep2()
            ev[r][2].record()
        torch.cuda.synchronize()
        t1 = sorted(e[0].elapsed_time(e[1]) for e in ev)
        t2 = sorted(e[1].elapsed_time(e[2]) for e in ev)
        marg = sorted(e[1].elapsed_time(e[2]) / e[0].elapsed_time(e[1]) - 1 for e in ev)
        med = lambda xs: xs[len(xs) // 2]
        kern = {}
        for name, fn in (("nq1", run1), ("nq2", run2)):
            sqa.profile_begin(3 * N_LAYERS * 4 + 16)
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            sqa.profile_end()
            for kn in ("fa_decode", "fa_combine"):
                t, c = sqa.profile_get(kn)
                if c:
                    kern[f"{name}_{kn}"] = round(t / c * 1e3, 2)
        frac = {name: round(layer_bytes(n_kv, nq) / (kern[f"{name}_fa_decode"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
                for name, nq in (("nq1", 1), ("nq2", 2))}
        out[f"n_kv_{n_kv}"] = {
            "nq1_per_layer_us": round(med(t1) * 1e3 / N_LAYERS, 2),
            "nq2_per_layer_us": round(med(t2) * 1e3 / N_LAYERS, 2),
            "nq2_GB/s": round(N_LAYERS * layer_bytes(n_kv, 2) / (med(t2) * 1e-3) / 1e9, 1),
            "draft_row_marginal_pct": round(100 * med(marg), 1),
            "marginal_pct_iqr": [round(100 * marg[len(marg) // 4], 1), round(100 * marg[3 * len(marg) // 4], 1)],
            "kernels_us": kern,
            "fa_decode_roofline_frac": frac,
            "timing": ("HIP graph replay of the 10-layer step (GPU time)" if graphs else "eager launches")
                      + "; kernels from events, eager",
            "rounds": rounds}
        del g1, g2, rep1, rep2
    return out


def length_curve_leg(sqa, torch, dev, ks, vs, rounds, lengths=(65536, 98304, 131072, N_KV)):
    """Decode (n_q = 1, every key visible, as the main leg) at several KV lengths
    that all run the same split count (256 splits x 2 KV heads on 256 CUs: the
    split rule reaches its cap from 65536 keys on), so the splits differ only in
    their number of 64-key tiles. Each 10-layer step is captured in a HIP graph
    and replayed. A least-squares line through (bytes per layer, time) splits the
    time into a per-byte part (marginal = the rate at which a longer context
    streams) and a fixed part (the value at zero bytes: the launches, the first
    loads' latency, the pipeline fill and drain, the partial stores and the split
    merge), for the whole layer (graph replay) and for the decode kernel alone
    (events on eager launches)."""
    pts = []
    for n_kv in lengths:
        q = torch.randn((1, H, D), device=dev)
        m = torch.zeros((1, n_kv), dtype=torch.float16, device=dev)
        o = torch.empty((1, H, D), device=dev)
        wsz = sqa.flash_attn_workspace_size(q, ks[0], n_kv)
        w = torch.empty(wsz, dtype=torch.uint8, device=dev)

        def run(q=q, m=m, o=o, w=w, n_kv=n_kv):
            for li in range(N_LAYERS):
                sqa.flash_attn_ext(q, ks[li], vs[li], n_kv, mask=m, out=o, workspace=w)

        g = capture(torch, run)
        for _ in range(3):
            g.replay()
        t = sorted(time_steps(torch, g.replay, 1) for _ in range(rounds))
        layer_us = t[len(t) // 2] * 1e3 / N_LAYERS
        sqa.profile_begin(3 * N_LAYERS * 4 + 16)
        for _ in range(3):
            run()
        torch.cuda.synchronize()
        sqa.profile_end()
        dt, dc = sqa.profile_get("fa_decode")
        # workspace = partials (splits x 16 rows x (1 KiB + 8 B)) + room for a packed mask copy + 256
        splits = (wsz - 256 - (2 * ((n_kv + 7) // 8 * 8) + 255) // 256 * 256) // (H * D * 4 + H * 2 * 4)
        pts.append((n_kv, layer_bytes(n_kv, 1), layer_us, dt / dc * 1e3, splits))
        del g

    def fit(ys):
        xs = [p[1] for p in pts]
        n = len(xs)
        mx, my = sum(xs) / n, sum(ys) / n
        b = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
        return b, my - b * mx  # us per byte, us at zero bytes

    bl, al = fit([p[2] for p in pts])
    bk, ak = fit([p[3] for p in pts])
    return {
        "points": [{"n_kv": p[0], "splits": p[4], "per_layer_us": round(p[2], 2), "fa_decode_us": round(p[3], 2)}
                   for p in pts],
        "layer_marginal_GB/s": round(1e-3 / bl, 1),
        "layer_fixed_us": round(al, 2),
        "fa_decode_marginal_GB/s": round(1e-3 / bk, 1),
        "fa_decode_marginal_frac_of_peak": round(1e-3 / bk / HBM_PEAK_GBS, 4),
        "fa_decode_fixed_us": round(ak, 2),
        "timing": "per layer: HIP graph replay of the 10-layer step; fa_decode: events, eager; "
                  "least-squares line over the points",
        "rounds": rounds}


def prefill_flops(n_q, start, heads=H, head_dim=D):
    """QK^T + PV multiply-adds (2 flops each) over the visible keys."""
    keys = n_q * (start + 1) + n_q * (n_q - 1) // 2
    return 4 * head_dim * heads * keys


def prefill_leg(sqa, torch, dev, steps, warmup):
    """pp512 per layer: set_rows of the 512 new K and V rows into the q4_0
    cache (positions 16384..16895), then flash_attn_ext over 16896 keys with
    the causal F16 mask."""
    n_kv = PP_START + PP_N_Q
    ks, vs = fill_caches(sqa, torch, dev, N_LAYERS, n_kv, seed=7)
    qs = [torch.randn((PP_N_Q, H, D), device=dev, dtype=torch.float32) for _ in range(N_LAYERS)]
    knew = [torch.randn((PP_N_Q, HKV * D), device=dev, dtype=torch.float32) for _ in range(N_LAYERS)]
    vnew = [torch.randn((PP_N_Q, HKV * D), device=dev, dtype=torch.float32) for _ in range(N_LAYERS)]
    idx = torch.arange(PP_START, n_kv, device=dev, dtype=torch.int64)
    mask = torch.empty((PP_N_Q, n_kv), dtype=torch.float16, device=dev)
    sqa.fill_causal_mask(mask, PP_START)
    out = torch.empty((PP_N_Q, H, D), dtype=torch.float32, device=dev)
    ws = torch.empty(sqa.flash_attn_workspace_size(qs[0], ks[0], n_kv), dtype=torch.uint8, device=dev)

    def step():
        for li in range(N_LAYERS):
            sqa.set_rows_q4_0(ks[li], knew[li], idx)
            sqa.set_rows_q4_0(vs[li], vnew[li], idx)
            sqa.flash_attn_ext(qs[li], ks[li], vs[li], n_kv, mask=mask, out=out, workspace=ws)

    for _ in range(warmup):
        step()
    ms = time_steps(torch, step, steps) / steps
    sqa.profile_begin(steps * N_LAYERS * 4 + 16)
    time_steps(torch, step, steps)
    sqa.profile_end()
    kern = {}
    for name in ("set_rows_q4_0", "fa_prefill_prep", "fa_prefill", "fa_combine"):
        t, c = sqa.profile_get(name)
        if c:
            kern[name] = round(t / c * 1e3, 2)
    flops = prefill_flops(PP_N_Q, PP_START)
    tflops = N_LAYERS * flops / (ms * 1e-3) / 1e12
    main_tf = flops / (kern["fa_prefill"] * 1e-6) / 1e12
    del ks, vs, qs, ws, knew, vnew
    return {"workload": f"pp512: n_q={PP_N_Q} after {PP_START} cached (n_kv={n_kv}), 16q/2kv, hd256, "
                        f"q4_0 K/V (512 new rows quantized on write), causal F16 mask, {N_LAYERS} layers",
            "per_layer_us": round(ms * 1e3 / N_LAYERS, 2), "TFLOP/s": round(tflops, 1),
            "pct_of_mfma_f16_peak": round(100 * tflops / MFMA_F16_PEAK_TFLOPS, 1),
            "kernels_us": kern,
            "roofline": {"kernel": "fa_prefill", "bound": "mfma", "achieved": round(main_tf, 1),
                         "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(main_tf / MFMA_F16_PEAK_TFLOPS, 4), "flops_per_launch": flops}}


def stack_leg(sqa, torch, dev, steps, warmup):
    """The 10-layer attention stack of a long prefill: ubatch 2048 at prior
    context 131072 (n_kv = 133120). Per layer: set_rows of the 2048 new K and
    V rows, causal flash attention over 133120 keys, sigmoid output gate.
    Two forms: 'mask' = the engine's F16 mask + separate sigmoid_mul kernel;
    'fused' = causal-from-positions + the gate fused into the epilogue."""
    n_kv = STACK_START + STACK_N_Q
    ks, vs = [], []
    for li in range(N_LAYERS):  # caches filled in-place to keep peak memory low
        k, v = fill_caches(sqa, torch, dev, 1, n_kv, seed=100 + li)
        ks += k
        vs += v
    q = torch.randn((STACK_N_Q, H, D), device=dev, dtype=torch.float32)
    gate = torch.randn((STACK_N_Q, H, D), device=dev, dtype=torch.float32)
    knew = torch.randn((STACK_N_Q, HKV * D), device=dev, dtype=torch.float32)
    vnew = torch.randn((STACK_N_Q, HKV * D), device=dev, dtype=torch.float32)
    idx = torch.arange(STACK_START, n_kv, device=dev, dtype=torch.int64)
    mask = torch.empty((STACK_N_Q, n_kv), dtype=torch.float16, device=dev)
    sqa.fill_causal_mask(mask, STACK_START)
    attn = torch.empty((STACK_N_Q, H, D), dtype=torch.float32, device=dev)
    out = torch.empty((STACK_N_Q, H, D), dtype=torch.float32, device=dev)
    ws = torch.empty(sqa.flash_attn_workspace_size(q, ks[0], n_kv), dtype=torch.uint8, device=dev)

    def step_mask():
        for li in range(N_LAYERS):
            sqa.set_rows_q4_0(ks[li], knew, idx)
            sqa.set_rows_q4_0(vs[li], vnew, idx)
            sqa.flash_attn_ext(q, ks[li], vs[li], n_kv, mask=mask, out=attn, workspace=ws)
            sqa.sigmoid_mul(attn.view(STACK_N_Q, H * D), gate.view(STACK_N_Q, H * D),
                            out=out.view(STACK_N_Q, H * D))

    def step_fused():
        for li in range(N_LAYERS):
            sqa.set_rows_q4_0(ks[li], knew, idx)
            sqa.set_rows_q4_0(vs[li], vnew, idx)
            sqa.flash_attn_ext_causal(q, ks[li], vs[li], n_kv, STACK_START, gate=gate, out=out, workspace=ws)

    res = {"workload": f"{N_LAYERS}-layer stack: ubatch {STACK_N_Q} at prior context {STACK_START} "
                       f"(n_kv={n_kv}), 16q/2kv, hd256, q4_0 K/V; set_rows -> FA -> sigmoid gate"}
    flops = prefill_flops(STACK_N_Q, STACK_START)
    for name, fn in (("mask", step_mask), ("fused", step_fused)):
        for _ in range(warmup):
            fn()
        ms = time_steps(torch, fn, steps) / steps
        sqa.profile_begin(steps * N_LAYERS * 8 + 16)
        time_steps(torch, fn, steps)
        sqa.profile_end()
        kern = {}
        for kn in ("set_rows_q4_0", "fa_prefill_prep", "fa_prefill", "fa_combine", "sigmoid_mul"):
            t, c = sqa.profile_get(kn)
            if c:
                kern[kn] = round(t / c * 1e3, 2)
        res[name] = {"ms_per_stack": round(ms, 3),
                     "attn_TFLOP/s": round(N_LAYERS * flops / (ms * 1e-3) / 1e12, 1),
                     "kernels_us": kern,
                     "fa_prefill_frac_of_mfma_peak": round(flops / (kern["fa_prefill"] * 1e-6) / 1e12
                                                           / MFMA_F16_PEAK_TFLOPS, 4)}
    del ks, vs, mask, ws
    return res


def producer_leg(sqa, torch, dev, steps, warmup, graphs=True):
    """K/Q producer per layer: RMSNorm + IMROPE + q4_0 quantize-on-write of the new
    K rows (2 KV heads), and RMSNorm + IMROPE of Q (16 heads, F32 out), for a
    512-token and a 2048-token ubatch. n_rot 64, sections (11, 11, 10, 0),
    freq_base 1e7 (plausible model values; the kernel takes them as parameters).
    Kernel times from the event hooks around eager launches include the host's
    launch gap when the host is the slower side (small kernels); with graphs,
    the K and Q launches of 10 layers are also captured apart and replayed, which
    times them on the GPU alone."""
    rope = sqa.rope_params(64, (11, 11, 10, 0), 1e7)
    out = {}
    for n_tok, start in ((PP_N_Q, PP_START), (2048, 131072)):
        gen = torch.Generator(device=dev)
        gen.manual_seed(n_tok)
        k_src = torch.randn((n_tok, HKV, D), generator=gen, device=dev)
        q_src = torch.randn((n_tok, H, D), generator=gen, device=dev)
        kw = torch.randn((D,), generator=gen, device=dev)
        qw = torch.randn((D,), generator=gen, device=dev)
        t = torch.arange(start, start + n_tok, device=dev, dtype=torch.int32)
        pos = t.repeat(4)
        idx = t.to(torch.int64)
        cache = torch.zeros((start + n_tok, HKV, D // 32 * 18), dtype=torch.uint8, device=dev)
        q_out = torch.empty_like(q_src)

        def step():
            for _ in range(N_LAYERS):
                sqa.rope_norm_set_rows_q4_0(cache, k_src, kw, 1e-6, pos, rope, idx)
                sqa.rope_norm_f32(q_out, q_src, qw, 1e-6, pos, rope)

        for _ in range(warmup):
            step()
        ms = time_steps(torch, step, steps) / steps
        sqa.profile_begin(steps * N_LAYERS * 2 + 8)
        time_steps(torch, step, steps)
        sqa.profile_end()
        kern = {}
        for name in ("rope_norm_set_rows_q4_0", "rope_norm_f32"):
            tt, c = sqa.profile_get(name)
            kern[name] = round(tt / c * 1e3, 2)
        k_bytes = n_tok * HKV * (D * 4 + 288 // HKV) + n_tok * (16 + 8)
        q_bytes = n_tok * H * D * 8 + n_tok * 16
        out[f"ubatch{n_tok}"] = {
            "per_layer_us": round(ms * 1e3 / N_LAYERS, 2), "kernels_us": kern,
            "k_GB/s": round(k_bytes / (kern["rope_norm_set_rows_q4_0"] * 1e-6) / 1e9, 1),
            "q_GB/s": round(q_bytes / (kern["rope_norm_f32"] * 1e-6) / 1e9, 1),
            "bytes": {"k": k_bytes, "q": q_bytes}}
        if graphs:
            def kstep():
                for _ in range(N_LAYERS):
                    sqa.rope_norm_set_rows_q4_0(cache, k_src, kw, 1e-6, pos, rope, idx)

            def qstep():
                for _ in range(N_LAYERS):
                    sqa.rope_norm_f32(q_out, q_src, qw, 1e-6, pos, rope)

            gk, gq = capture(torch, kstep), capture(torch, qstep)
            for _ in range(2):
                gk.replay()
                gq.replay()
            k_us = time_steps(torch, gk.replay, steps) / steps * 1e3 / N_LAYERS
            q_us = time_steps(torch, gq.replay, steps) / steps * 1e3 / N_LAYERS
            del gk, gq
            out[f"ubatch{n_tok}"]["graph_kernels_us"] = {"rope_norm_set_rows_q4_0": round(k_us, 2),
                                                         "rope_norm_f32": round(q_us, 2)}
            out[f"ubatch{n_tok}"]["graph_q_GB/s"] = round(q_bytes / (q_us * 1e-6) / 1e9, 1)
        del k_src, q_src, cache, q_out
    return out


def out_proj_leg(sqa, torch, dev, np, steps, warmup, graphs=True):
    """W_o projection per layer (attn.rs:281-285): dst = W . (x * sigmoid(gate)) with
    W a Q4_K [4096, 2048] weight (n_head 16 x head_dim 256 in, n_embd 2048 out) of
    random codes and scales, for a decode token, a 2-token verify and the 512-token
    ubatch. Decode is bound by the weight bytes; the ubatch by the MFMA work.
    graph_launch_floor_us: what one launch of a one-element add costs in the
    same kind of replayed graph, the floor under any kernel's figure here."""
    K, N = H * D, 2048
    rng = np.random.default_rng(7)
    out = {}
    ws_w = []
    for _ in range(N_LAYERS):
        w = rng.integers(0, 256, (N, K // 256, 144), dtype=np.uint8)
        w[:, :, 0:2] = rng.uniform(2e-4, 4e-3, (N, K // 256)).astype(np.float16).view(np.uint8).reshape(N, -1, 2)
        w[:, :, 2:4] = rng.uniform(0, 4e-3, (N, K // 256)).astype(np.float16).view(np.uint8).reshape(N, -1, 2)
        ws_w.append(torch.from_numpy(w.reshape(N, -1)).to(dev))
    w_bytes = N * K // 256 * 144
    for M in (1, 2, PP_N_Q):
        x = torch.randn((M, K), device=dev)
        g = torch.randn((M, K), device=dev)
        o = torch.empty((M, N), device=dev)
        need = sqa.out_proj_workspace_size(ws_w[0], x)
        wsp = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)

        def step():
            for w in ws_w:
                sqa.out_proj(w, x, g, out=o, workspace=wsp)

        for _ in range(warmup):
            step()
        ms = time_steps(torch, step, steps) / steps
        sqa.profile_begin(steps * N_LAYERS + 8)
        time_steps(torch, step, steps)
        sqa.profile_end()
        tt, c = sqa.profile_get("out_proj")
        us = tt / c * 1e3
        out[f"m{M}"] = {"per_layer_us": round(ms * 1e3 / N_LAYERS, 2), "kernels_us": round(us, 2),
                        "weight_GB/s": round(w_bytes / (us * 1e-6) / 1e9, 1),
                        "TFLOP/s": round(2 * N * K * M / (us * 1e-6) / 1e12, 2)}
        if graphs:
            g = capture(torch, step)  # the same 10 layers without the Python launch cost
            for _ in range(2):
                g.replay()
            ms_g = time_steps(torch, g.replay, steps) / steps
            del g
            gl = ms_g * 1e3 / N_LAYERS
            out[f"m{M}"]["graph_per_layer_us"] = round(gl, 2)
            out[f"m{M}"]["graph_weight_GB/s"] = round(w_bytes / (gl * 1e-6) / 1e9, 1)
    out["shape"] = {"K": K, "N": N, "weight": "Q4_K", "weight_bytes": w_bytes}
    if graphs:
        # the floor of any launch in a replayed graph: 10 one-element adds
        one = torch.zeros(1, device=dev)

        def trivial():
            for _ in range(N_LAYERS):
                one.add_(1.0)

        g = capture(torch, trivial)
        for _ in range(2):
            g.replay()
        out["graph_launch_floor_us"] = round(time_steps(torch, g.replay, steps) / steps * 1e3 / N_LAYERS, 2)
        del g
    return out


def host_cpu():
    """(CPU model, logical CPUs usable by this process)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return model, n


def cpu_threads(rows):
    """Threads for the oracle: one (query, head) row per task as ggml partitions
    its FA work, capped at the 16 host cores a one-GPU share of the box holds."""
    return max(1, min(host_cpu()[1], 16, rows))


def cpu_baseline(orc, kq, vq, q, mask, budget_s=8.0):
    """The oracle (C restatement of ggml's CPU flash_attn_ext) on this host."""
    threads = cpu_threads(q.shape[0] * q.shape[1])
    orc.flash_attn_ext(q, kq, vq, mask, threads=threads)  # warm
    t0 = time.perf_counter()
    reps = 0
    while True:
        orc.flash_attn_ext(q, kq, vq, mask, threads=threads)
        reps += 1
        if time.perf_counter() - t0 > budget_s / threads or reps >= 20:
            break
    dt = (time.perf_counter() - t0) / reps
    return dt, threads, reps


def cpu_prefill_baseline(orc, np, n_pos=16, seed=11):
    """The oracle on a bounded sample of the pp512 workload: n_pos of the 512
    query positions (evenly spaced, all 16 heads) over the 16896-key cache with
    their causal mask rows, timed and scaled by the visible keys of all 512
    positions over those of the sample."""
    n_kv = PP_START + PP_N_Q
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((n_kv, HKV * D), dtype=np.float32)
    v = rng.standard_normal((n_kv, HKV * D), dtype=np.float32)
    kq = orc.quantize_q4_0(k).reshape(n_kv, HKV, -1)
    vq = orc.quantize_q4_0(v).reshape(n_kv, HKV, -1)
    pos = np.linspace(0, PP_N_Q - 1, n_pos).astype(np.int64)
    q = rng.standard_normal((n_pos, H, D), dtype=np.float32)
    mask = orc.causal_mask(PP_N_Q, n_kv, PP_START)[pos]
    threads = cpu_threads(n_pos * H)
    orc.flash_attn_ext(q, kq, vq, mask, threads=threads)  # warm
    reps, t0 = 0, time.perf_counter()
    while reps < 3:
        orc.flash_attn_ext(q, kq, vq, mask, threads=threads)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    sample_keys = int(sum(PP_START + p + 1 for p in pos))
    full_keys = PP_N_Q * (PP_START + 1) + PP_N_Q * (PP_N_Q - 1) // 2
    layer_s = dt * full_keys / sample_keys
    return {"value": round(prefill_flops(PP_N_Q, PP_START) / layer_s / 1e12, 5), "unit": "TFLOP/s",
            "cores": threads, "kind": "port",
            "sample": f"{n_pos} of the 512 pp512 query positions x 16 heads over {n_kv} keys with their "
                      f"causal mask rows, {reps} runs of {dt * 1e3:.1f} ms, scaled by visible keys to "
                      f"{layer_s * 1e3:.0f} ms per layer"}


def _trace_key(r):
    name = r["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0]
    name = name.replace("void ", "").replace("sqa::", "")
    def total(prefix):  # work-items over all dimensions (traces list X, Y and Z apart)
        if r.get(prefix):
            return r[prefix]
        dims = [r.get(f"{prefix}_{a}") for a in "XYZ"]
        return str(int(dims[0]) * int(dims[1] or 1) * int(dims[2] or 1)) if dims[0] else "?"
    return name, total("Grid_Size"), total("Workgroup_Size")


def summarize_trace(trace_dir):
    """One row per (kernel, grid, workgroup size) of the rocprofv3 kernel traces
    (*kernel_trace.csv) under trace_dir: launches and the median, mean and
    minimum duration. Kernels of one name launched at different grids (the
    decode kernel at different KV lengths) fall in different rows; shapes that
    share a grid are profiled in separate runs (--main-nkv, --verify-nkv).
    Counter collections (*counter_collection.csv) under trace_dir give one row
    per (kernel, grid, workgroup size, counter): the mean value per dispatch."""
    import csv
    import glob
    import statistics
    groups = {}
    for f in sorted(glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True)):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
                groups.setdefault(_trace_key(r), []).append(d)
    if groups:
        print(f"{'kernel':48s} {'grid':>8s} {'wg':>5s} {'launches':>8s} {'median us':>10s} {'mean us':>9s} "
              f"{'min us':>8s}")
    for (name, grid, wg), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        print(f"{name[:48]:48s} {grid:>8s} {wg:>5s} {len(d):8d} {statistics.median(d):10.2f} "
              f"{statistics.mean(d):9.2f} {min(d):8.2f}")
    per_dispatch = {}
    for f in sorted(glob.glob(os.path.join(trace_dir, "**", "*counter_collection.csv"), recursive=True)):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                key = _trace_key(r) + (r["Counter_Name"],)
                disp = (f, r.get("Dispatch_Id") or r.get("Correlation_Id"))
                slot = per_dispatch.setdefault(key, {})
                slot[disp] = slot.get(disp, 0.0) + float(r["Counter_Value"])
    if per_dispatch:
        print(f"{'kernel':48s} {'grid':>8s} {'wg':>5s} {'counter':24s} {'dispatches':>10s} {'mean per dispatch':>18s}")
    for (name, grid, wg, counter), v in sorted(per_dispatch.items()):
        print(f"{name[:48]:48s} {grid:>8s} {wg:>5s} {counter:24s} {len(v):10d} "
              f"{statistics.mean(v.values()):18.1f}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # ~10 ms of untimed decode steps: the GPU reaches its steady clock after a few
    # ms of load, and a decode server runs continuously.
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-verify", action="store_true", help="skip the n_q=2 verify leg")
    ap.add_argument("--no-prefill", action="store_true", help="skip the pp512 prefill leg")
    ap.add_argument("--no-stack", action="store_true", help="skip the 10-layer ubatch-2048 stack leg")
    ap.add_argument("--no-producer", action="store_true", help="skip the K/Q producer (norm + rope) leg")
    ap.add_argument("--no-graph", action="store_true", help="no HIP graphs: skip the graph-replay decode timing; the verify and W_o legs "
                         "time eager launches (for counter collection)")
    ap.add_argument("--no-out-proj", action="store_true", help="skip the W_o projection leg")
    ap.add_argument("--copy-ref", action="store_true",
                    help="run a plain 256 MiB device copy at the end (counter calibration)")
    ap.add_argument("--main-nkv", type=int, default=N_KV,
                    help="KV length of the main decode leg (profiling aid; the headline is 172032)")
    ap.add_argument("--verify-nkv", type=int, nargs="+", default=[32768, 131072, N_KV],
                    help="KV lengths of the verify leg (profiling aid: one length per run gives one trace row each)")
    ap.add_argument("--summarize-trace", metavar="DIR",
                    help="print per-(kernel, grid) durations (kernel traces) and counter means (counter "
                         "collections) of the rocprofv3 output under DIR and exit")
    args = ap.parse_args()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU's share of this single-GPU path; --gpus {args.gpus} is not "
              "supported: the path runs on one GPU and has no multi-GPU mode", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import __graft_entry__ as ge

    sqa = ge.load_package()
    dev = torch.device("cuda:0")
    torch.manual_seed(0)

    ks, vs = fill_caches(sqa, torch, dev, N_LAYERS, N_KV, seed=1)
    n_main = min(args.main_nkv, N_KV)
    qs = [torch.randn((1, H, D), device=dev, dtype=torch.float32) for _ in range(N_LAYERS)]
    mask = torch.zeros((1, n_main), dtype=torch.float16, device=dev)  # decode: every key visible
    out = torch.empty((1, H, D), dtype=torch.float32, device=dev)
    ws = torch.empty(sqa.flash_attn_workspace_size(qs[0], ks[0], n_main), dtype=torch.uint8, device=dev)

    def step():
        for li in range(N_LAYERS):
            sqa.flash_attn_ext(qs[li], ks[li], vs[li], n_main, mask=mask, out=out, workspace=ws)

    for _ in range(args.warmup):
        step()
    ms = time_steps(torch, step, args.steps)
    ms_per_step = ms / args.steps
    bytes_step = N_LAYERS * layer_bytes(n_main, 1)
    value = bytes_step / (ms_per_step * 1e-3) / 1e9

    # Per-kernel durations with HIP events on the launch stream (same steps again).
    sqa.profile_begin(args.steps * N_LAYERS * 4 + 16)
    time_steps(torch, step, args.steps)
    sqa.profile_end()
    dec_ms, dec_n = sqa.profile_get("fa_decode")
    comb_ms, comb_n = sqa.profile_get("fa_combine")  # absent when the split merge is fused
    dec_avg_us = dec_ms / dec_n * 1e3
    kernels = {"fa_decode": round(dec_avg_us, 2)}
    if comb_n:
        kernels["fa_combine"] = round(comb_ms / comb_n * 1e3, 2)
    achieved = layer_bytes(n_main, 1) / (dec_avg_us * 1e-6) / 1e9

    result = {
        "metric": "q4_0 FA decode HBM GB/s @172K ctx (% peak); pp512 attn TFLOP/s (% MFMA)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 KV, q8_0 Q: int8 MFMA (QK) + fp16 MFMA (PV), fp32 accumulate",
        "data": "synthetic (seeded N(0,1) Q/K/V; K/V quantized on the GPU)",
        "config": {"workload": f"decode n_q=1, 16q/2kv heads, hd256, q4_0 K/V, n_kv={n_main}, "
                               "10 independent layers, F16 mask", "n_kv": n_main, "layers": N_LAYERS,
                   "n_q": 1, "heads": H, "kv_heads": HKV, "head_dim": D},
        "per_layer_us": round(ms_per_step * 1e3 / N_LAYERS, 2),
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
        "kernels_us": kernels,
        "roofline": {"kernel": "fa_decode", "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": DECODE_TRAFFIC_BYTES if n_main == N_KV else None,
                     "bytes_per_launch": layer_bytes(n_main, 1)},
    }

    # The same 10-layer step captured once in a HIP graph and replayed: the
    # reference keeps the step's pointers fixed so that ggml-cuda replays its
    # graph. Reported beside the eager figure; `value` stays the eager one.
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                step()
        torch.cuda.current_stream().wait_stream(side)
        for _ in range(3):
            graph.replay()
        ms_g = time_steps(torch, graph.replay, args.steps) / args.steps
        result["decode_graph_replay"] = {"per_layer_us": round(ms_g * 1e3 / N_LAYERS, 2),
                                         "GB/s": round(bytes_step / (ms_g * 1e-3) / 1e9, 1)}
        del graph
        if n_main == N_KV:
            result["decode_length_curve"] = length_curve_leg(sqa, torch, dev, ks, vs, max(10, args.steps))

    if not args.no_verify:
        result["verify_nq2"] = verify_leg(sqa, torch, dev, ks, vs, args.steps,
                                             tuple(min(n, N_KV) for n in args.verify_nkv),
                                             graphs=not args.no_graph)

    if not args.no_prefill:
        result["prefill_pp512"] = prefill_leg(sqa, torch, dev, max(2, args.steps // 2), 2)
        torch.cuda.empty_cache()
    if not args.no_stack:
        result["stack_ub2048_131k"] = stack_leg(sqa, torch, dev, 2, 1)
        torch.cuda.empty_cache()
    if not args.no_producer:
        result["producer_rope_norm"] = producer_leg(sqa, torch, dev, max(2, args.steps // 2), 2,
                                                    graphs=not args.no_graph)
        torch.cuda.empty_cache()
    if not args.no_out_proj:
        result["out_proj_wo"] = out_proj_leg(sqa, torch, dev, np, max(2, args.steps // 2), 2,
                                             graphs=not args.no_graph)
        torch.cuda.empty_cache()

    if not args.no_cpu:
        from oracle import oracle as orc

        kq = ks[0][:n_main].cpu().numpy()
        vq = vs[0][:n_main].cpu().numpy()
        qh = qs[0].cpu().numpy()
        mh = mask.cpu().numpy()
        dt, threads, reps = cpu_baseline(orc, kq, vq, qh, mh)
        model, ncpu = host_cpu()
        result["cpu_baseline"] = {"value": round(layer_bytes(n_main, 1) / dt / 1e9, 3), "unit": "GB/s",
                                  "cores": threads, "kind": "port",
                                  "sample": f"{reps} runs of one {n_main}-key decode layer (n_q=1, 16 rows); "
                                            f"{dt * 1e3:.1f} ms per layer",
                                  "host_cpu": model, "host_logical_cpus": ncpu,
                                  "build": "gcc -O3 -march=x86-64-v3 -fopenmp, one (query, head) row per thread"}
        if not args.no_prefill:
            result["cpu_baseline_prefill_pp512"] = cpu_prefill_baseline(orc, np)
        # Check the timed GPU output of that layer against the oracle.
        o_gpu = sqa.flash_attn_ext(qs[0], ks[0], vs[0], n_main, mask=mask).cpu().numpy()
        o_ref = orc.flash_attn_ext(qh, kq, vq, mh, threads=threads)
        rms = float(np.sqrt(np.mean(o_ref.astype(np.float64) ** 2)))
        result["parity_max_err_over_rms"] = float(np.abs(o_gpu - o_ref).max() / rms)

    if args.copy_ref:
        a = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()

    print(json.dumps(result))


if __name__ == "__main__":
    main()
