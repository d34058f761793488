"""Seeded synthetic inputs shared by the parity tests: Q, K, V ~ N(0,1) float32,
optional outlier channels (x8), K/V quantized to q4_0 by the oracle."""
import numpy as np


def qkv(orc, seed, n_q, n_kv, H=16, Hkv=2, D=256, outliers=0, scale_k=1.0, scale_v=1.0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n_q, H, D), dtype=np.float32)
    k = rng.standard_normal((n_kv, Hkv * D), dtype=np.float32) * np.float32(scale_k)
    v = rng.standard_normal((n_kv, Hkv * D), dtype=np.float32) * np.float32(scale_v)
    if outliers:
        ch = rng.choice(Hkv * D, outliers, replace=False)
        k[:, ch] *= 8
        v[:, ch] *= 8
    kq = orc.quantize_q4_0(k).reshape(n_kv, Hkv, -1)
    vq = orc.quantize_q4_0(v).reshape(n_kv, Hkv, -1)
    return q, kq, vq


def rel_err(got, ref):
    ref = np.asarray(ref, dtype=np.float64)
    rms = np.sqrt(np.mean(ref ** 2))
    return float(np.abs(np.asarray(got, dtype=np.float64) - ref).max() / rms)
