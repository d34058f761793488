"""Float64 brute-force attention on dequantized operands, the two-pass
textbook form of the op the reference builds at src/model/attn.rs:228-251
(softmax over keys of scale * Q.K + mask, times V; GQA head h reads KV head
h // (H/Hkv), the block map of tests/attn_test.rs:306-312)."""
import numpy as np


def q8_dequant(orc, q):
    """q float32 (n_q, H, D) -> the q8_0-rounded values ggml's CPU FA multiplies with."""
    n_q, H, D = q.shape
    qb = orc.quantize_q8_0(q.reshape(-1)).reshape(-1, 34)
    d = qb[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1)
    v = qb[:, 2:].view(np.int8).astype(np.float64)
    return (v * d[:, None]).reshape(n_q, H, D)


def cache_dequant(orc, cache):
    n_kv, Hkv, rb = cache.shape
    D = rb // 18 * 32
    return orc.dequantize_q4_0(cache.reshape(-1), n_kv * Hkv * D).reshape(n_kv, Hkv, D).astype(np.float64)


def attention_f64(qd, kd, vd, scale, mask=None, head_map=None):
    """qd (n_q,H,D), kd/vd (n_kv,Hkv,D) float64; mask (n_q, n_kv) or None."""
    n_q, H, D = qd.shape
    Hkv = kd.shape[1]
    G = H // Hkv
    out = np.zeros((n_q, H, D))
    for h in range(H):
        kh = head_map(h) if head_map else h // G
        s = scale * qd[:, h, :] @ kd[:, kh, :].T
        if mask is not None:
            s = s + mask.astype(np.float64)[:n_q]
        m = s.max(axis=1, keepdims=True)
        with np.errstate(invalid="ignore"):
            p = np.where(np.isfinite(s), np.exp(s - np.where(np.isfinite(m), m, 0)), 0.0)
        den = p.sum(axis=1, keepdims=True)
        out[:, h, :] = np.where(den > 0, (p @ vd[:, kh, :]) / np.where(den > 0, den, 1), 0.0)
    return out


def rel_err(got, ref):
    ref = np.asarray(ref, dtype=np.float64)
    rms = np.sqrt(np.mean(ref ** 2))
    return float(np.abs(np.asarray(got, dtype=np.float64) - ref).max() / rms)
