"""MI355X (gfx950) full-attention hot path of the qwen35moe engine.

Python host mirror of the C ABI in include/sqattn.h, named after the ggml ops
and the engine objects it stands in for (reference: src/backend/ffi.rs:363-405,
src/engine/kv.rs). Device memory and streams come from PyTorch; every kernel
runs from libsqattn.so, which sits next to this file. If the library is
missing the import fails: there is no CPU fallback.

Tensor conventions (torch shapes, C order, all on the GPU):
  q       float32 (n_q, H, D)             the engine's [D, H, n_q] Q
  cache   uint8   (rows, Hkv, D//32*18)   one q4_0 K or V cache (kv.rs:95-148)
  mask    float16 (n_q_pad, n_kv)         0 / -inf, or None
  out     float32 (n_q, H, D)             [D, H, n_q] attention output
"""
import ctypes
import struct
import os

import torch

__all__ = [
    "Tensor", "lib", "last_error", "SqaError", "set_rows_q4_0", "flash_attn_ext",
    "flash_attn_ext_causal", "flash_attn_ext_static", "sigmoid_mul", "fill_causal_mask", "supports_flash_attn_ext",
    "flash_attn_workspace_size", "out_proj", "out_proj_workspace_size", "KvCache", "cache_view", "row_bytes", "profile_begin", "profile_end",
    "profile_get", "Rope", "rope_params", "rope_norm_set_rows_q4_0", "rope_norm_f32",
]

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsqattn.so")

TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q4_K, TYPE_I32, TYPE_I64 = 0, 1, 2, 12, 26, 27
Q4_K_BLOCK = 144  # bytes per 256-value Q4_K super-block
QK4_0 = 32
Q4_0_BLOCK = 18
KV_PAD = 256
STATUS = {0: "ok", 1: "invalid argument", 2: "unsupported configuration", 3: "workspace too small",
          4: "HIP runtime error", 5: "KV cache overflow", 6: "argument out of range"}


class SqaError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"{STATUS.get(status, status)}: {msg}")
        self.status = status


_TENSOR_LAYOUT = struct.Struct("<ii4q4QQ")  # type, pad_, ne[4], nb[4], data


class Tensor(ctypes.Structure):
    """sqa_tensor: ggml's {type, ne[4], nb[4], data} (reference ffi.rs:22-39)."""

    _fields_ = [
        ("type", ctypes.c_int32),
        ("pad_", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_uint64 * 4),
        ("data", ctypes.c_void_p),
    ]

    @staticmethod
    def make(ttype, ne, nb, ptr):
        """Fields packed in one go: a decode step builds five of these per call."""
        ne = tuple(ne) + (1,) * (4 - len(ne))
        nb = list(nb)
        while len(nb) < 4:
            nb.append(nb[-1] * ne[len(nb) - 1])
        return Tensor.from_buffer_copy(_TENSOR_LAYOUT.pack(ttype, 0, *ne, *nb, ptr))


class Rope(ctypes.Structure):
    """sqa_rope: the ggml_rope_multi parameters of RopeParams (reference attn.rs:30-65)."""

    _fields_ = [
        ("n_rot", ctypes.c_int32),
        ("sections", ctypes.c_int32 * 4),
        ("freq_base", ctypes.c_float),
        ("freq_scale", ctypes.c_float),
        ("ext_factor", ctypes.c_float),
        ("attn_factor", ctypes.c_float),
    ]


def rope_params(n_rot, sections, freq_base, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0):
    """RopeParams::text (reference attn.rs:46-64): no YaRN ramp, attn_factor 1."""
    r = Rope()
    r.n_rot = int(n_rot)
    for i in range(4):
        r.sections[i] = int(sections[i])
    r.freq_base, r.freq_scale, r.ext_factor, r.attn_factor = freq_base, freq_scale, ext_factor, attn_factor
    return r


_lib = None


def lib():
    """The loaded libsqattn.so (raises if it was never built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER(Tensor)
        vp, sz, i64, f32, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int64, ctypes.c_float, ctypes.c_int32
        sigs = {
            "sqa_version": (ctypes.c_char_p, []),
            "sqa_last_error": (ctypes.c_char_p, []),
            "sqa_status_string": (ctypes.c_char_p, [ctypes.c_int]),
            "sqa_set_rows_q4_0": (ctypes.c_int, [P, P, P, vp]),
            "sqa_supports_set_rows": (ctypes.c_int, [P, P, P]),
            "sqa_rope_norm_set_rows_q4_0": (ctypes.c_int, [P, P, P, f32, P, ctypes.POINTER(Rope), P, vp]),
            "sqa_rope_norm_f32": (ctypes.c_int, [P, P, P, f32, P, ctypes.POINTER(Rope), vp]),
            "sqa_supports_rope_norm": (ctypes.c_int, [P, P, P, P, ctypes.POINTER(Rope), P]),
            "sqa_flash_attn_ext": (ctypes.c_int, [P, P, P, P, f32, f32, f32, P, vp, sz, vp]),
            "sqa_flash_attn_ext_workspace_size": (sz, [P, P, P, P]),
            "sqa_supports_flash_attn_ext": (ctypes.c_int, [P, P, P, P, f32, f32, f32, P]),
            "sqa_flash_attn_ext_causal": (ctypes.c_int, [P, P, P, i64, P, f32, P, vp, sz, vp]),
            "sqa_flash_attn_ext_static": (ctypes.c_int, [P, P, P, P, f32, f32, f32, P, vp]),
            "sqa_sigmoid_mul": (ctypes.c_int, [P, P, P, vp]),
            "sqa_out_proj_workspace_size": (sz, [P, P]),
            "sqa_supports_out_proj": (ctypes.c_int, [P, P, P, P]),
            "sqa_out_proj": (ctypes.c_int, [P, P, P, P, vp, sz, vp]),
            "sqa_fill_causal_mask": (ctypes.c_int, [P, i64, vp]),
            "sqa_kv_cache_layer_bytes": (sz, [i64, i64, i64]),
            "sqa_kv_cache_create": (vp, [i32, i64, i64, i64, ctypes.POINTER(vp), ctypes.POINTER(vp)]),
            "sqa_kv_cache_destroy": (None, [vp]),
            "sqa_kv_cache_n_used": (i64, [vp]),
            "sqa_kv_cache_step_start": (i64, [vp]),
            "sqa_kv_cache_n_kv_padded": (i64, [vp]),
            "sqa_kv_cache_n_kv_padded_after": (i64, [vp, i64]),
            "sqa_kv_cache_begin_step": (ctypes.c_int, [vp, i64]),
            "sqa_kv_cache_rewind_to": (ctypes.c_int, [vp, i64]),
            "sqa_kv_cache_reset": (None, [vp]),
            "sqa_kv_cache_k_view": (ctypes.c_int, [vp, i32, P]),
            "sqa_kv_cache_v_view": (ctypes.c_int, [vp, i32, P]),
            "sqa_kv_cache_append": (ctypes.c_int, [vp, i32, P, P, P, vp]),
            "sqa_profile_begin": (ctypes.c_int, [i32]),
            "sqa_profile_end": (ctypes.c_int, []),
            "sqa_profile_get": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                               ctypes.POINTER(i64)]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error():
    return lib().sqa_last_error().decode()


def _check(rc):
    if rc != 0:
        raise SqaError(rc, last_error())


def _stream(stream):
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return getattr(stream, "cuda_stream", stream)


def _ref(t):
    return ctypes.byref(t) if t is not None else None


def row_bytes(D, Hkv=1):
    return D // QK4_0 * Q4_0_BLOCK * Hkv


# ------------------------------------------------------------ descriptors ---

def q_desc(q):
    """(n_q, H, D) float32 -> ggml view [D, n_q, H] (the permute of attn.rs:232)."""
    n_q, H, D = q.shape
    s = q.stride()
    return Tensor.make(TYPE_F32, [D, n_q, H, 1], [4, s[0] * 4, s[1] * 4], q.data_ptr())


def cache_view(cache, n_kv):
    """(rows, Hkv, D//32*18) uint8 -> q4_0 view [D, n_kv, Hkv] (kv.rs:401-447 permuted)."""
    rows, Hkv, rb = cache.shape
    D = rb // Q4_0_BLOCK * QK4_0
    assert cache.dtype == torch.uint8 and cache.is_contiguous() and n_kv <= rows
    return Tensor.make(TYPE_Q4_0, [D, n_kv, Hkv, 1], [Q4_0_BLOCK, Hkv * rb, rb], cache.data_ptr())


def out_desc(out):
    n_q, H, D = out.shape
    assert out.is_contiguous()
    return Tensor.make(TYPE_F32, [D, H, n_q, 1], [4, D * 4, H * D * 4], out.data_ptr())


def mask_desc(mask):
    if mask is None:
        return None
    n_rows, n_kv = mask.shape
    assert mask.dtype == torch.float16 and mask.stride(1) == 1
    return Tensor.make(TYPE_F16, [n_kv, n_rows, 1, 1], [2, mask.stride(0) * 2], mask.data_ptr())


# ---------------------------------------------------------------------- ops --

def set_rows_q4_0(cache, src, idx, stream=None):
    """cache[idx[i]] = quantize_row_q4_0(src[i]) (GGML_OP_SET_ROWS, kv.rs:356-396).

    cache: uint8 (rows, ..., row_bytes) contiguous; src: float32 (n, ne0); idx: int64 (n,)."""
    rows = cache.shape[0]
    rb = cache[0].numel()
    ne0 = src.shape[1]
    assert rb == ne0 // QK4_0 * Q4_0_BLOCK, "row length mismatch"
    td = Tensor.make(TYPE_Q4_0, [ne0, rows], [Q4_0_BLOCK, rb], cache.data_ptr())
    ts = Tensor.make(TYPE_F32, [ne0, src.shape[0]], [4, src.stride(0) * 4], src.data_ptr())
    ti = Tensor.make(TYPE_I64, [idx.shape[0]], [idx.stride(0) * 8], idx.data_ptr())
    _check(lib().sqa_set_rows_q4_0(ctypes.byref(td), ctypes.byref(ts), ctypes.byref(ti), _stream(stream)))
    return cache


def _producer_descs(src, norm_w, pos):
    n_tok, n_head, D = src.shape
    ts = Tensor.make(TYPE_F32, [D, n_head, n_tok], [4, src.stride(1) * 4, src.stride(0) * 4], src.data_ptr())
    tw = None if norm_w is None else Tensor.make(TYPE_F32, [D], [4], norm_w.data_ptr())
    tp = Tensor.make(TYPE_I32, [pos.shape[0]], [4], pos.data_ptr())
    return ts, tw, tp


def rope_norm_set_rows_q4_0(cache, src, norm_w, eps, pos, rope, idx, stream=None):
    """K producer (reference attn.rs:166-200 + kv.rs:313-399): per-head RMSNorm times
    norm_w, IMROPE with positions pos, q4_0 quantize-on-write into cache rows idx.

    cache: uint8 (rows, ..., n_head*D//32*18) contiguous; src: float32 (n_tok, n_head, D)
    with contiguous rows; norm_w: float32 (D,) or None; pos: int32 (4*n_tok,);
    idx: int64 (n_tok,)."""
    n_tok, n_head, D = src.shape
    rows = cache.shape[0]
    rb = cache[0].numel()
    assert rb == n_head * D // QK4_0 * Q4_0_BLOCK, "row length mismatch"
    ts, tw, tp = _producer_descs(src, norm_w, pos)
    td = Tensor.make(TYPE_Q4_0, [n_head * D, rows], [Q4_0_BLOCK, rb], cache.data_ptr())
    ti = Tensor.make(TYPE_I64, [idx.shape[0]], [idx.stride(0) * 8], idx.data_ptr())
    _check(lib().sqa_rope_norm_set_rows_q4_0(ctypes.byref(td), ctypes.byref(ts), _ref(tw), eps, ctypes.byref(tp),
                                             ctypes.byref(rope), ctypes.byref(ti), _stream(stream)))
    return cache


def rope_norm_f32(out, src, norm_w, eps, pos, rope, stream=None):
    """Q producer (reference attn.rs:166-199): out float32 (n_tok, n_head, D) contiguous."""
    n_tok, n_head, D = src.shape
    ts, tw, tp = _producer_descs(src, norm_w, pos)
    to = Tensor.make(TYPE_F32, [D, n_head, n_tok], [4, D * 4, n_head * D * 4], out.data_ptr())
    _check(lib().sqa_rope_norm_f32(ctypes.byref(to), ctypes.byref(ts), _ref(tw), eps, ctypes.byref(tp),
                                   ctypes.byref(rope), _stream(stream)))
    return out


def flash_attn_workspace_size(q, k_cache, n_kv):
    n_q, H, D = q.shape
    tq, tk = q_desc(q), cache_view(k_cache, n_kv)
    to = Tensor.make(TYPE_F32, [D, H, n_q, 1], [4, D * 4, H * D * 4], 16)
    return int(lib().sqa_flash_attn_ext_workspace_size(ctypes.byref(tq), ctypes.byref(tk), ctypes.byref(tk),
                                                       ctypes.byref(to)))


def supports_flash_attn_ext(q, k_cache, n_kv, mask=None, scale=None, max_bias=0.0, softcap=0.0):
    n_q, H, D = q.shape
    scale = D ** -0.5 if scale is None else scale
    tq, tk = q_desc(q), cache_view(k_cache, n_kv)
    to = Tensor.make(TYPE_F32, [D, H, n_q, 1], [4, D * 4, H * D * 4], 16)
    tm = mask_desc(mask)
    return bool(lib().sqa_supports_flash_attn_ext(ctypes.byref(tq), ctypes.byref(tk), ctypes.byref(tk),
                                                  _ref(tm), scale, max_bias, softcap, ctypes.byref(to)))


def _workspace(nbytes, device):
    if nbytes == 0:
        return None, 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    return ws, nbytes


def flash_attn_ext(q, k_cache, v_cache, n_kv, mask=None, scale=None, max_bias=0.0, softcap=0.0,
                   out=None, workspace=None, stream=None):
    """ggml_flash_attn_ext(q, k, v, mask, scale, max_bias, softcap) over q4_0 caches."""
    n_q, H, D = q.shape
    scale = D ** -0.5 if scale is None else scale
    if out is None:
        out = torch.empty((n_q, H, D), dtype=torch.float32, device=q.device)
    tq, tk, tv = q_desc(q), cache_view(k_cache, n_kv), cache_view(v_cache, n_kv)
    to, tm = out_desc(out), mask_desc(mask)
    if workspace is None:  # a given workspace is checked by the library
        need = int(lib().sqa_flash_attn_ext_workspace_size(ctypes.byref(tq), ctypes.byref(tk), ctypes.byref(tv),
                                                           ctypes.byref(to)))
        workspace, _ = _workspace(need, q.device)
    wptr = workspace.data_ptr() if workspace is not None else None
    wbytes = workspace.numel() if workspace is not None else 0
    _check(lib().sqa_flash_attn_ext(ctypes.byref(tq), ctypes.byref(tk), ctypes.byref(tv), _ref(tm), scale,
                                    max_bias, softcap, ctypes.byref(to), wptr, wbytes, _stream(stream)))
    return out


def flash_attn_ext_static(q, k_cache, v_cache, n_kv, mask=None, scale=None, max_bias=0.0, softcap=0.0,
                          out=None, stream=None):
    """flash_attn_ext for decode/verify shapes with the library's own device scratch:
    no workspace, no allocation inside the call (out must be given for that)."""
    n_q, H, D = q.shape
    scale = D ** -0.5 if scale is None else scale
    if out is None:
        out = torch.empty((n_q, H, D), dtype=torch.float32, device=q.device)
    tq, tk, tv = q_desc(q), cache_view(k_cache, n_kv), cache_view(v_cache, n_kv)
    to, tm = out_desc(out), mask_desc(mask)
    _check(lib().sqa_flash_attn_ext_static(ctypes.byref(tq), ctypes.byref(tk), ctypes.byref(tv), _ref(tm), scale,
                                           max_bias, softcap, ctypes.byref(to), _stream(stream)))
    return out


def flash_attn_ext_causal(q, k_cache, v_cache, n_kv, q_pos0, gate=None, scale=None, out=None,
                          workspace=None, stream=None):
    """Mask-free causal FA (query t at position q_pos0 + t) with optional fused sigmoid gate."""
    n_q, H, D = q.shape
    scale = D ** -0.5 if scale is None else scale
    if out is None:
        out = torch.empty((n_q, H, D), dtype=torch.float32, device=q.device)
    tq, tk, tv = q_desc(q), cache_view(k_cache, n_kv), cache_view(v_cache, n_kv)
    to = out_desc(out)
    tg = None
    if gate is not None:
        s = gate.stride()
        tg = Tensor.make(TYPE_F32, [D, H, n_q, 1], [4, s[1] * 4, s[0] * 4], gate.data_ptr())
    if workspace is None:  # a given workspace is checked by the library
        need = int(lib().sqa_flash_attn_ext_workspace_size(ctypes.byref(tq), ctypes.byref(tk), ctypes.byref(tv),
                                                           ctypes.byref(to)))
        workspace, _ = _workspace(need, q.device)
    wptr = workspace.data_ptr() if workspace is not None else None
    wbytes = workspace.numel() if workspace is not None else 0
    _check(lib().sqa_flash_attn_ext_causal(ctypes.byref(tq), ctypes.byref(tk), ctypes.byref(tv), q_pos0,
                                           _ref(tg), scale, ctypes.byref(to), wptr, wbytes, _stream(stream)))
    return out


def sigmoid_mul(x, gate, out=None, stream=None):
    """out = x * sigmoid(gate) over 2-D float32 [n_tok, n] (attn.rs:282-283)."""
    if out is None:
        out = torch.empty_like(x)
    n1, n0 = x.shape
    d = [Tensor.make(TYPE_F32, [n0, n1], [4, t.stride(0) * 4], t.data_ptr()) for t in (out, x, gate)]
    _check(lib().sqa_sigmoid_mul(ctypes.byref(d[0]), ctypes.byref(d[1]), ctypes.byref(d[2]), _stream(stream)))
    return out


def _out_proj_descs(w, x, gate, out):
    """w: uint8 (N, K // 256 * 144) Q4_K rows; x, gate: float32 (M, K); out: float32 (M, N)."""
    M, K = x.shape
    N = w.shape[0]
    tw = Tensor.make(TYPE_Q4_K, [K, N], [Q4_K_BLOCK, w.stride(0)], w.data_ptr())
    tx = Tensor.make(TYPE_F32, [K, M], [4, x.stride(0) * 4], x.data_ptr())
    tg = None if gate is None else Tensor.make(TYPE_F32, [K, M], [4, gate.stride(0) * 4], gate.data_ptr())
    to = None if out is None else Tensor.make(TYPE_F32, [N, M], [4, out.stride(0) * 4], out.data_ptr())
    return tw, tx, tg, to


def out_proj_workspace_size(w, x):
    tw, tx, _, _ = _out_proj_descs(w, x, None, None)
    return int(lib().sqa_out_proj_workspace_size(ctypes.byref(tw), ctypes.byref(tx)))


def out_proj(w, x, gate=None, out=None, workspace=None, stream=None):
    """W_o projection (attn.rs:281-285): out (M, N) = (x * sigmoid(gate)) @ W^T with
    W the Q4_K weight rows w (N, K // 256 * 144) and x, gate (M, K) float32."""
    M, K = x.shape
    if out is None:
        out = torch.empty((M, w.shape[0]), dtype=torch.float32, device=x.device)
    tw, tx, tg, to = _out_proj_descs(w, x, gate, out)
    need = int(lib().sqa_out_proj_workspace_size(ctypes.byref(tw), ctypes.byref(tx)))
    if workspace is None:
        workspace, _ = _workspace(need, x.device)
    _check(lib().sqa_out_proj(ctypes.byref(tw), ctypes.byref(tx), _ref(tg), ctypes.byref(to),
                              workspace.data_ptr() if workspace is not None else None,
                              workspace.numel() if workspace is not None else 0, _stream(stream)))
    return out


def fill_causal_mask(mask, step_start, stream=None):
    """Device fill of the F16 mask (n_q, n_kv): row t allows keys <= step_start + t."""
    tm = mask_desc(mask)
    _check(lib().sqa_fill_causal_mask(ctypes.byref(tm), step_start, _stream(stream)))
    return mask


def profile_begin(max_records=4096):
    """Bracket every kernel launch with HIP events until profile_end()."""
    _check(lib().sqa_profile_begin(max_records))


def profile_end():
    lib().sqa_profile_end()


def profile_get(kernel):
    """(total_ms, launches) recorded for one kernel since profile_begin()."""
    ms, n = ctypes.c_double(), ctypes.c_int64()
    _check(lib().sqa_profile_get(kernel.encode(), ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value


# ---------------------------------------------------------------- KvCache ---

class KvCache:
    """Single-sequence append-only q4_0 KV cache (mirror of kv.rs:67-448).

    Owns one K and one V uint8 buffer per full-attention layer, each of shape
    (cap_alloc, Hkv, D//32*18); bookkeeping runs in the C++ library."""

    def __init__(self, n_layers, head_dim, n_head_kv, kv_cap, device="cuda"):
        L = lib()
        self.head_dim, self.n_head_kv, self.kv_cap = head_dim, n_head_kv, kv_cap
        nbytes = int(L.sqa_kv_cache_layer_bytes(head_dim, n_head_kv, kv_cap))
        if nbytes == 0:
            raise SqaError(1, "invalid KV cache geometry")
        self.kv_cap_alloc = (kv_cap + KV_PAD - 1) // KV_PAD * KV_PAD
        shape = (self.kv_cap_alloc, n_head_kv, row_bytes(head_dim))
        self.k = [torch.empty(shape, dtype=torch.uint8, device=device) for _ in range(n_layers)]
        self.v = [torch.empty(shape, dtype=torch.uint8, device=device) for _ in range(n_layers)]
        kp = (ctypes.c_void_p * n_layers)(*[t.data_ptr() for t in self.k])
        vp = (ctypes.c_void_p * n_layers)(*[t.data_ptr() for t in self.v])
        self._h = L.sqa_kv_cache_create(n_layers, head_dim, n_head_kv, kv_cap, kp, vp)
        if not self._h:
            raise SqaError(1, last_error())

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().sqa_kv_cache_destroy(h)
            self._h = None

    def zero_caches(self):
        """Zero every layer once at load (kv.rs:150-170): padded rows then contribute 0."""
        for t in self.k + self.v:
            t.zero_()

    @property
    def n_used(self):
        return int(lib().sqa_kv_cache_n_used(self._h))

    @property
    def step_start(self):
        return int(lib().sqa_kv_cache_step_start(self._h))

    def n_kv_padded(self):
        return int(lib().sqa_kv_cache_n_kv_padded(self._h))

    def n_kv_padded_after(self, n_tokens):
        return int(lib().sqa_kv_cache_n_kv_padded_after(self._h, n_tokens))

    def begin_step(self, n_tokens):
        _check(lib().sqa_kv_cache_begin_step(self._h, n_tokens))

    def rewind_to(self, pos):
        _check(lib().sqa_kv_cache_rewind_to(self._h, pos))

    def reset(self):
        lib().sqa_kv_cache_reset(self._h)

    def view(self, slot, which="k"):
        t = Tensor()
        fn = lib().sqa_kv_cache_k_view if which == "k" else lib().sqa_kv_cache_v_view
        _check(fn(self._h, slot, ctypes.byref(t)))
        return t

    def append(self, slot, k_cur, v_cur, idx, stream=None):
        """Quantize this step's K/V rows, float32 (n_tokens, Hkv*D), into layer `slot`."""
        n_tok, ne0 = k_cur.shape
        tk = Tensor.make(TYPE_F32, [ne0, n_tok], [4, k_cur.stride(0) * 4], k_cur.data_ptr())
        tv = Tensor.make(TYPE_F32, [ne0, n_tok], [4, v_cur.stride(0) * 4], v_cur.data_ptr())
        ti = Tensor.make(TYPE_I64, [n_tok], [8], idx.data_ptr())
        _check(lib().sqa_kv_cache_append(self._h, slot, ctypes.byref(tk), ctypes.byref(tv), ctypes.byref(ti),
                                         _stream(stream)))

    def workspace_size(self, slot, q):
        """Workspace bytes of attend() for q over the current [0, n_kv_padded) views."""
        n_q, H, D = q.shape
        tq, tk, tv = q_desc(q), self.view(slot, "k"), self.view(slot, "v")
        to = Tensor.make(TYPE_F32, [D, H, n_q, 1], [4, D * 4, H * D * 4], 16)
        return int(lib().sqa_flash_attn_ext_workspace_size(ctypes.byref(tq), ctypes.byref(tk), ctypes.byref(tv),
                                                           ctypes.byref(to)))

    def attend(self, slot, q, mask=None, scale=None, out=None, workspace=None, stream=None):
        """flash_attn_ext over this layer's [0, n_kv_padded) views, taken from the
        library's k_view/v_view (the permuted views of kv.rs:401-447 that
        attn.rs:228-251 hands to ggml_flash_attn_ext)."""
        n_q, H, D = q.shape
        scale = D ** -0.5 if scale is None else scale
        if out is None:
            out = torch.empty((n_q, H, D), dtype=torch.float32, device=q.device)
        tq, tk, tv = q_desc(q), self.view(slot, "k"), self.view(slot, "v")
        to, tm = out_desc(out), mask_desc(mask)
        if workspace is None:
            workspace, _ = _workspace(self.workspace_size(slot, q), q.device)
        wptr = workspace.data_ptr() if workspace is not None else None
        wbytes = workspace.numel() if workspace is not None else 0
        _check(lib().sqa_flash_attn_ext(ctypes.byref(tq), ctypes.byref(tk), ctypes.byref(tv), _ref(tm), scale,
                                        0.0, 0.0, ctypes.byref(to), wptr, wbytes, _stream(stream)))
        return out
