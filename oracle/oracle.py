"""ctypes front end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, never by the product package. It exposes the C
restatement of ggml's CPU semantics (see ggml_cpu_ref.h for the reference
call sites each function follows) on numpy arrays.

Array conventions (numpy shapes, C order):
  q      float32 (n_q, H, D)            ggml view [D, n_q, H] of the engine's [D, H, n_q]
  cache  uint8   (n_kv, Hkv, D//32*18)  q4_0 rows: the engine's K/V cache layout
  mask   float16 (n_q_pad, n_kv)        0 / -inf entries
  out    float32 (n_q, H, D)
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q4_K, TYPE_I32, TYPE_I64 = 0, 1, 2, 12, 26, 27
Q8_X86, Q8_SCALAR = 0, 1
QK = 32
Q4_BLOCK = 18
Q8_BLOCK = 34


class Tensor(ctypes.Structure):
    """Same layout as sqa_tensor in include/sqattn.h."""

    _fields_ = [
        ("type", ctypes.c_int32),
        ("pad_", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_uint64 * 4),
        ("data", ctypes.c_void_p),
    ]


class Rope(ctypes.Structure):
    """Same layout as sqa_rope in include/sqattn.h."""

    _fields_ = [
        ("n_rot", ctypes.c_int32),
        ("sections", ctypes.c_int32 * 4),
        ("freq_base", ctypes.c_float),
        ("freq_scale", ctypes.c_float),
        ("ext_factor", ctypes.c_float),
        ("attn_factor", ctypes.c_float),
    ]


def rope_params(n_rot, sections, freq_base, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0):
    r = Rope()
    r.n_rot = n_rot
    for i in range(4):
        r.sections[i] = sections[i]
    r.freq_base, r.freq_scale, r.ext_factor, r.attn_factor = freq_base, freq_scale, ext_factor, attn_factor
    return r


def build(force=False):
    """Compile liboracle.so with its Makefile (gcc only, no GPU)."""
    args = ["make", "-C", HERE] + (["-B"] if force else [])
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER(Tensor)
        L.orc_fp32_to_fp16.restype = ctypes.c_uint16
        L.orc_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.orc_fp16_to_fp32.restype = ctypes.c_float
        L.orc_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        for name in ("orc_quantize_row_q4_0", "orc_dequantize_row_q4_0"):
            getattr(L, name).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.orc_quantize_row_q8_0.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int]
        L.orc_vec_dot_q4_0_q8_0.restype = ctypes.c_float
        L.orc_vec_dot_q4_0_q8_0.argtypes = [ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
        L.orc_set_rows_q4_0.argtypes = [P, P, P]
        L.orc_flash_attn_ext.argtypes = [P, P, P, P, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                         P, ctypes.c_int, ctypes.c_int]
        L.orc_flash_attn_ext_causal.argtypes = [P, P, P, ctypes.c_int64, P, ctypes.c_float, P,
                                                ctypes.c_int, ctypes.c_int]
        L.orc_sigmoid_mul.argtypes = [P, P, P]
        R = ctypes.POINTER(Rope)
        L.orc_rms_norm_mul_row.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float, ctypes.c_int64,
                                           ctypes.c_void_p]
        L.orc_imrope_cache.argtypes = [ctypes.c_int32, ctypes.c_void_p, ctypes.c_float, ctypes.c_float,
                                       ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p]
        L.orc_rope_row.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p,
                                   ctypes.c_void_p]
        L.orc_rope_theta_scale.restype = ctypes.c_float
        L.orc_rope_theta_scale.argtypes = [R]
        L.orc_rope_norm_set_rows_q4_0.argtypes = [P, P, P, ctypes.c_float, P, R, P]
        L.orc_rope_norm_f32.argtypes = [P, P, P, ctypes.c_float, P, R]
        L.orc_dequantize_row_q4_K.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.orc_out_proj.argtypes = [P, P, P, P]
        L.orc_max_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def tensor(ttype, ne, nb, arr):
    t = Tensor()
    t.type = ttype
    for i in range(4):
        t.ne[i] = ne[i] if i < len(ne) else 1
    last = nb[-1] * (ne[len(nb) - 1] if len(nb) else 1)
    for i in range(4):
        t.nb[i] = nb[i] if i < len(nb) else last
    t.data = arr.ctypes.data
    return t


# ------------------------------------------------------------------ scalars --

def fp32_to_fp16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    L = lib()
    return np.array([L.orc_fp32_to_fp16(float(v)) for v in x], dtype=np.uint16)


def fp16_bits_to_fp32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    L = lib()
    return np.array([L.orc_fp16_to_fp32(int(v)) for v in h], dtype=np.float32)


def quantize_q4_0(x):
    """float32 (..., k) -> uint8 (..., k//32*18) via orc_quantize_row_q4_0."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    assert k % QK == 0
    out = np.zeros(x.shape[:-1] + (k // QK * Q4_BLOCK,), dtype=np.uint8)
    lib().orc_quantize_row_q4_0(_ptr(x), _ptr(out), x.size)
    return out


def dequantize_q4_0(q, k):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    n = q.size // Q4_BLOCK * QK
    out = np.zeros(q.shape[:-1] + (k,), dtype=np.float32)
    assert out.size == n
    lib().orc_dequantize_row_q4_0(_ptr(q), _ptr(out), n)
    return out


def quantize_q8_0(x, variant=Q8_X86):
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    out = np.zeros(x.shape[:-1] + (k // QK * Q8_BLOCK,), dtype=np.uint8)
    lib().orc_quantize_row_q8_0(_ptr(x), _ptr(out), x.size, variant)
    return out


def vec_dot_q4_0_q8_0(xq4, yq8, n):
    return float(lib().orc_vec_dot_q4_0_q8_0(n, _ptr(np.ascontiguousarray(xq4)), _ptr(np.ascontiguousarray(yq8))))


# ---------------------------------------------------------------------- ops --

def set_rows_q4_0(dst, src, idx):
    """dst uint8 (rows, ne0//32*18) updated in place; src f32 (n, ne0); idx int64 (n,)."""
    src = np.ascontiguousarray(src, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    ne0 = src.shape[1]
    rb = ne0 // QK * Q4_BLOCK
    assert dst.flags.c_contiguous and dst.dtype == np.uint8 and dst.shape[1] == rb
    td = tensor(TYPE_Q4_0, [ne0, dst.shape[0]], [Q4_BLOCK, rb], dst)
    ts = tensor(TYPE_F32, [ne0, src.shape[0]], [4, ne0 * 4], src)
    ti = tensor(TYPE_I64, [idx.shape[0]], [8], idx)
    rc = lib().orc_set_rows_q4_0(ctypes.byref(td), ctypes.byref(ts), ctypes.byref(ti))
    assert rc == 0, rc
    return dst


def _fa_tensors(q, kc, vc, D):
    q = np.ascontiguousarray(q, dtype=np.float32)
    n_q, H, _ = q.shape
    n_kv, Hkv, rb = kc.shape
    assert rb == D // QK * Q4_BLOCK
    tq = tensor(TYPE_F32, [D, n_q, H, 1], [4, H * D * 4, D * 4], q)
    tk = tensor(TYPE_Q4_0, [D, n_kv, Hkv, 1], [Q4_BLOCK, Hkv * rb, rb], kc)
    tv = tensor(TYPE_Q4_0, [D, n_kv, Hkv, 1], [Q4_BLOCK, Hkv * rb, rb], vc)
    out = np.zeros((n_q, H, D), dtype=np.float32)
    to = tensor(TYPE_F32, [D, H, n_q, 1], [4, D * 4, H * D * 4], out)
    return q, tq, tk, tv, out, to


def flash_attn_ext(q, kc, vc, mask=None, scale=None, max_bias=0.0, softcap=0.0,
                   threads=None, variant=Q8_X86):
    """ggml CPU flash_attn_ext over q4_0 K/V (see module docstring for shapes)."""
    kc = np.ascontiguousarray(kc, dtype=np.uint8)
    vc = np.ascontiguousarray(vc, dtype=np.uint8)
    D = q.shape[2]
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    q, tq, tk, tv, out, to = _fa_tensors(q, kc, vc, D)
    tm = None
    if mask is not None:
        mask = np.ascontiguousarray(mask, dtype=np.float16)
        tm = tensor(TYPE_F16, [mask.shape[1], mask.shape[0], 1, 1], [2, mask.shape[1] * 2], mask)
    threads = threads or lib().orc_max_threads()
    rc = lib().orc_flash_attn_ext(ctypes.byref(tq), ctypes.byref(tk), ctypes.byref(tv),
                                  ctypes.byref(tm) if tm is not None else None,
                                  scale, max_bias, softcap, ctypes.byref(to), threads, variant)
    assert rc == 0, rc
    return out


def flash_attn_ext_causal(q, kc, vc, q_pos0, gate=None, scale=None, threads=None, variant=Q8_X86):
    kc = np.ascontiguousarray(kc, dtype=np.uint8)
    vc = np.ascontiguousarray(vc, dtype=np.uint8)
    D = q.shape[2]
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    q, tq, tk, tv, out, to = _fa_tensors(q, kc, vc, D)
    tg = None
    if gate is not None:
        gate = np.ascontiguousarray(gate, dtype=np.float32)
        n_q, H, _ = gate.shape
        tg = tensor(TYPE_F32, [D, H, n_q, 1], [4, D * 4, H * D * 4], gate)
    threads = threads or lib().orc_max_threads()
    rc = lib().orc_flash_attn_ext_causal(ctypes.byref(tq), ctypes.byref(tk), ctypes.byref(tv),
                                         q_pos0, ctypes.byref(tg) if tg is not None else None,
                                         scale, ctypes.byref(to), threads, variant)
    assert rc == 0, rc
    return out


def sigmoid_mul(x, gate):
    x = np.ascontiguousarray(x, dtype=np.float32)
    gate = np.ascontiguousarray(gate, dtype=np.float32)
    out = np.zeros_like(x)
    n1, n0 = x.shape
    tx = tensor(TYPE_F32, [n0, n1], [4, n0 * 4], x)
    tg = tensor(TYPE_F32, [n0, n1], [4, n0 * 4], gate)
    to = tensor(TYPE_F32, [n0, n1], [4, n0 * 4], out)
    assert lib().orc_sigmoid_mul(ctypes.byref(to), ctypes.byref(tx), ctypes.byref(tg)) == 0
    return out


def causal_mask(n_q, n_kv, step_start):
    """F16 mask (n_q, n_kv): row t allows keys <= step_start + t (graph.rs:534-576)."""
    m = np.full((n_q, n_kv), -np.inf, dtype=np.float16)
    for t in range(n_q):
        m[t, : min(step_start + t + 1, n_kv)] = 0
    return m


# ----------------------------------------------------- K/Q producer (norm+rope) --

def rms_norm_mul_row(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros_like(x)
    wa = None if w is None else np.ascontiguousarray(w, dtype=np.float32)
    lib().orc_rms_norm_mul_row(_ptr(x), None if wa is None else _ptr(wa), eps, x.size, _ptr(y))
    return y


def imrope_cache(rope, p4):
    """cos/sin pairs (n_rot,) of one token with positions p4 = (t, h, w, e)."""
    sec = np.array(list(rope.sections), dtype=np.int32)
    p = np.array(p4, dtype=np.int32)
    cache = np.zeros(rope.n_rot, dtype=np.float32)
    ts = lib().orc_rope_theta_scale(ctypes.byref(rope))
    lib().orc_imrope_cache(rope.n_rot, _ptr(sec), ts, rope.freq_scale, rope.attn_factor, _ptr(p), _ptr(cache))
    return cache


def rope_row(x, rope, cache):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros_like(x)
    lib().orc_rope_row(_ptr(x), x.size, rope.n_rot, _ptr(cache), _ptr(y))
    return y


def _producer_tensors(src, norm_w, pos):
    src = np.ascontiguousarray(src, dtype=np.float32)
    n_tok, n_head, D = src.shape
    ts = tensor(TYPE_F32, [D, n_head, n_tok], [4, D * 4, n_head * D * 4], src)
    tw = None
    if norm_w is not None:
        norm_w = np.ascontiguousarray(norm_w, dtype=np.float32)
        tw = tensor(TYPE_F32, [D], [4], norm_w)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    assert pos.shape == (4 * n_tok,)
    tp = tensor(TYPE_I32, [4 * n_tok], [4], pos)
    return (src, norm_w, pos), ts, tw, tp


def rope_norm_set_rows_q4_0(cache, src, norm_w, eps, pos, rope, idx):
    """cache uint8 (rows, n_head*D//32*18) updated in place; src f32 (n_tok, n_head, D);
    pos int32 (4*n_tok,) t/h/w/e positions; idx int64 (n_tok,)."""
    keep, ts, tw, tp = _producer_tensors(src, norm_w, pos)
    n_tok, n_head, D = keep[0].shape
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    rb = n_head * D // QK * Q4_BLOCK
    assert cache.flags.c_contiguous and cache.dtype == np.uint8 and cache.shape[1] == rb
    td = tensor(TYPE_Q4_0, [n_head * D, cache.shape[0]], [Q4_BLOCK, rb], cache)
    ti = tensor(TYPE_I64, [n_tok], [8], idx)
    rc = lib().orc_rope_norm_set_rows_q4_0(ctypes.byref(td), ctypes.byref(ts),
                                           ctypes.byref(tw) if tw is not None else None, eps,
                                           ctypes.byref(tp), ctypes.byref(rope), ctypes.byref(ti))
    assert rc == 0, rc
    return cache


def rope_norm_f32(src, norm_w, eps, pos, rope):
    keep, ts, tw, tp = _producer_tensors(src, norm_w, pos)
    out = np.zeros_like(keep[0])
    n_tok, n_head, D = out.shape
    to = tensor(TYPE_F32, [D, n_head, n_tok], [4, D * 4, n_head * D * 4], out)
    rc = lib().orc_rope_norm_f32(ctypes.byref(to), ctypes.byref(ts), ctypes.byref(tw) if tw is not None else None,
                                 eps, ctypes.byref(tp), ctypes.byref(rope))
    assert rc == 0, rc
    return out


Q4K_BLOCK = 144  # bytes per 256-value Q4_K super-block


def dequantize_q4_K(wq, k):
    """Rows of Q4_K bytes (n, k // 256 * 144) -> float32 (n, k), ggml's dequantize_row_q4_K."""
    wq = np.ascontiguousarray(wq, dtype=np.uint8).reshape(-1, k // 256 * Q4K_BLOCK)
    out = np.empty((wq.shape[0], k), np.float32)
    for i in range(wq.shape[0]):
        lib().orc_dequantize_row_q4_K(_ptr(wq[i]), _ptr(out[i]), k)
    return out


def out_proj(wq, x, gate=None):
    """W_o projection (src/model/attn.rs:281-285): wq Q4_K rows (N, K // 256 * 144),
    x (M, K) float32 attention output, gate (M, K) or None -> (M, N) float32 =
    (x * sigmoid(gate)) @ dequant(W)^T accumulated in double."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    wq = np.ascontiguousarray(wq, dtype=np.uint8).reshape(-1, K // 256 * Q4K_BLOCK)
    N = wq.shape[0]
    out = np.empty((M, N), np.float32)
    tw = tensor(TYPE_Q4_K, [K, N], [Q4K_BLOCK, K // 256 * Q4K_BLOCK], wq)
    tx = tensor(TYPE_F32, [K, M], [4, K * 4], x)
    to = tensor(TYPE_F32, [N, M], [4, N * 4], out)
    tg = None
    if gate is not None:
        gate = np.ascontiguousarray(gate, dtype=np.float32)
        assert gate.shape == x.shape
        tg = tensor(TYPE_F32, [K, M], [4, K * 4], gate)
    rc = lib().orc_out_proj(ctypes.byref(to), ctypes.byref(tw), ctypes.byref(tx),
                            ctypes.byref(tg) if tg is not None else None)
    assert rc == 0, rc
    return out
