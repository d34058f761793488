"""Writes the committed golden fixtures of this directory from the oracle
(the C restatement of ggml's CPU quantize_row_q4_0 and flash_attn_ext).

The reference ships no golden vectors for this path: its only tests at the
ggml boundary need the external ggml library (tests/attn_test.rs:790, 845).
These fixtures freeze the oracle's answers on small seeded inputs, so that
(1) the oracle cannot drift unnoticed (tests/test_golden.py re-derives them on
the CPU) and (2) the GPU parity tests compare the HIP path against fixed data.

Usage (from the repository root):  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle as orc  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def q4_0_edge_blocks():
    """Hand-picked 32-value blocks covering the quantizer's edge cases:
    zeros, signed-max ties (first occurrence wins), negative max, rounding
    boundaries of x*id + 8.5, fp16-subnormal scales, huge values, and the
    closed-form ramp x_j = j - 16 (tests/attn_test.rs:783-788 rule d = max/-8)."""
    rng = np.random.default_rng(20240601)
    blocks = []
    blocks.append(np.zeros(32, np.float32))                       # d = -0, bytes 0x88
    blocks.append(np.arange(32, dtype=np.float32) - 16)            # ramp, max |x| = -16
    b = np.zeros(32, np.float32); b[3] = 5.0; b[9] = -5.0          # tie: first (+5) wins
    blocks.append(b)
    b = np.zeros(32, np.float32); b[9] = -5.0; b[3] = 5.0; b[1] = -5.0
    blocks.append(b)                                               # tie: first (-5) wins
    blocks.append(np.full(32, 1.0, np.float32))                    # constant block
    blocks.append(np.full(32, -3.25, np.float32))
    b = np.linspace(-1, 1, 32, dtype=np.float32); blocks.append(b)
    # values exactly on x*id + 8.5 == integer boundaries for d = -1 (max = 8)
    b = np.array([8.0] + [(k + 0.5) for k in range(-8, 7)] * 2 + [0.5], np.float32)[:32]
    blocks.append(b)
    blocks.append((rng.standard_normal(32) * 1e-6).astype(np.float32))   # subnormal fp16 scale
    blocks.append((rng.standard_normal(32) * 6e4).astype(np.float32))    # near fp16 max scale
    blocks.append((rng.standard_normal(32) * 1e-9).astype(np.float32))   # scale flushes to 0 in fp16
    b = rng.standard_normal(32).astype(np.float32); b[17] = 40.0; blocks.append(b)  # outlier
    for _ in range(20):
        blocks.append(rng.standard_normal(32).astype(np.float32) * np.float32(rng.uniform(0.01, 100)))
    x = np.stack(blocks).astype(np.float32)
    return x, orc.quantize_q4_0(x.reshape(1, -1)).reshape(len(blocks), 18)


def fa_case(seed, n_q, n_kv, mask_kind, H=16, Hkv=2, outliers=0, gate=False, scale=1.0 / 16):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n_q, H, 256), dtype=np.float32)
    k = rng.standard_normal((n_kv, Hkv * 256), dtype=np.float32)
    v = rng.standard_normal((n_kv, Hkv * 256), dtype=np.float32)
    if outliers:
        ch = rng.choice(Hkv * 256, outliers, replace=False)
        k[:, ch] *= 8
        v[:, ch] *= 8
    kq = orc.quantize_q4_0(k).reshape(n_kv, Hkv, 144)
    vq = orc.quantize_q4_0(v).reshape(n_kv, Hkv, 144)
    if mask_kind == "zero":
        mask = np.zeros((n_q, n_kv), np.float16)
    else:  # causal: query t sees keys <= n_kv - n_q + t
        mask = orc.causal_mask(n_q, n_kv, n_kv - n_q)
    g = rng.standard_normal((n_q, H, 256), dtype=np.float32) if gate else None
    out = orc.flash_attn_ext(q, kq, vq, mask, scale=scale)
    if gate:
        out = orc.sigmoid_mul(out.reshape(n_q, -1), g.reshape(n_q, -1)).reshape(out.shape)
    d = dict(q=q, k=kq, v=vq, mask=mask, scale=np.float32(scale), out=out)
    if gate:
        d["gate"] = g
    return d


CASES = {
    # decode, one query, 1% outlier channels (5 of 512) as in the CPU-runnable decode shape
    "fa_decode_outliers": dict(seed=11, n_q=1, n_kv=160, mask_kind="zero", outliers=5),
    # MTP verify: two rows with the causal mask across them
    "fa_verify_causal": dict(seed=12, n_q=2, n_kv=129, mask_kind="causal"),
    # prefill chunk with the fused output gate
    "fa_prefill_gate": dict(seed=13, n_q=4, n_kv=96, mask_kind="causal", gate=True),
    # other GQA ratio (4 q heads per kv head)
    "fa_prefill_g4": dict(seed=14, n_q=6, n_kv=70, mask_kind="causal", H=8, Hkv=2),
}


def main():
    x, qb = q4_0_edge_blocks()
    np.savez_compressed(os.path.join(HERE, "q4_0_blocks.npz"), x=x, q4_0=qb)
    for name, kw in CASES.items():
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **fa_case(**kw))
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
