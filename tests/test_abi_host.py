"""Host-side checks of the C ABI (no GPU needed): every symbol declared in
include/sqattn.h is exported, argument validation rejects what ggml would
reject, support queries answer like probe_flash_attn (src/engine/runner.rs:
509-559 of the reference), and the KvCache bookkeeping follows kv.rs."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "sqattn.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sqa_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(sqa):
    L = sqa.lib()
    syms = declared_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(L, s), s
    assert sqa.lib().sqa_version().startswith(b"sqattn")


def fa_descs(sqa, n_q=1, H=16, Hkv=2, D=256, n_kv=4096, qtype=0, ktype=2, nb2=144):
    T = sqa.Tensor.make
    q = T(qtype, [D, n_q, H, 1], [4, H * D * 4, D * 4], 4096)
    rb = D // 32 * 18
    k = T(ktype, [D, n_kv, Hkv, 1], [18, Hkv * rb, nb2], 8192)
    o = T(0, [D, H, n_q, 1], [4, D * 4, H * D * 4], 16384)
    return q, k, o


def supports(sqa, q, k, o, mask=None, scale=0.0625, mb=0.0, sc=0.0):
    L = sqa.lib()
    return L.sqa_supports_flash_attn_ext(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k),
                                         ctypes.byref(mask) if mask else None, scale, mb, sc, ctypes.byref(o))


def test_supports_matches_engine_probe(sqa):
    q, k, o = fa_descs(sqa)
    m = sqa.Tensor.make(1, [4096, 1, 1, 1], [2, 8192], 32768)
    assert supports(sqa, q, k, o, m) == 1                      # the probe shape (runner.rs:544-556)
    assert supports(sqa, q, k, o, None) == 1
    assert supports(sqa, q, k, o, m, mb=8.0) == 0              # ALiBi
    assert supports(sqa, q, k, o, m, sc=30.0) == 0             # softcap
    q2, k2, o2 = fa_descs(sqa, ktype=1)                        # f16 K
    assert supports(sqa, q2, k2, o2) == 0
    q3, k3, o3 = fa_descs(sqa, D=128)                          # head_dim 128
    assert supports(sqa, q3, k3, o3) == 0
    bad_mask = sqa.Tensor.make(1, [4000, 1, 1, 1], [2, 8000], 32768)  # ne[0] != n_kv
    assert supports(sqa, q, k, o, bad_mask) == 0


def test_invalid_calls_return_errors_before_any_launch(sqa):
    L = sqa.lib()
    q, k, o = fa_descs(sqa)
    rc = L.sqa_flash_attn_ext(None, ctypes.byref(k), ctypes.byref(k), None, 0.0625, 0.0, 0.0,
                              ctypes.byref(o), None, 0, None)
    assert rc == 1 and "null" in sqa.last_error()
    rc = L.sqa_flash_attn_ext(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k), None, 0.0625, 1.0, 0.0,
                              ctypes.byref(o), None, 0, None)
    assert rc == 2 and "ALiBi" in sqa.last_error()
    rc = L.sqa_flash_attn_ext(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k), None, 0.0625, 0.0, 0.0,
                              ctypes.byref(o), None, 0, None)
    assert rc == 3  # workspace missing
    rc = L.sqa_flash_attn_ext_causal(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k), -1, None, 0.0625,
                                     ctypes.byref(o), None, 0, None)
    assert rc == 6
    T = sqa.Tensor.make
    src = T(0, [500, 4], [4, 2000], 4096)
    dst = T(2, [500, 64], [18, 288], 8192)
    idx = T(27, [4], [8], 16384)
    assert L.sqa_set_rows_q4_0(ctypes.byref(dst), ctypes.byref(src), ctypes.byref(idx), None) == 1
    assert "multiple of 32" in sqa.last_error()
    assert L.sqa_supports_set_rows(ctypes.byref(dst), ctypes.byref(src), ctypes.byref(idx)) == 0


def test_workspace_size_scales_with_splits(sqa):
    L = sqa.lib()
    q, k, o = fa_descs(sqa, n_kv=172032)
    big = L.sqa_flash_attn_ext_workspace_size(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k), ctypes.byref(o))
    q, k, o = fa_descs(sqa, n_kv=256)
    small = L.sqa_flash_attn_ext_workspace_size(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k), ctypes.byref(o))
    assert big > small > 0
    # at most one split per CU of 16 rows x (256 + 2) floats, plus room for an
    # aligned copy of an F16 mask row of 172032 keys, plus 256-byte alignment slack
    assert big <= 256 * 16 * 258 * 4 + 172032 * 2 + 4 * 256


class FakeKv:
    """KvCache bookkeeping with dummy (never dereferenced) buffer addresses."""

    def __init__(self, sqa, n_layers=10, D=256, Hkv=2, cap=172032):
        L = sqa.lib()
        self.L, self.sqa = L, sqa
        kp = (ctypes.c_void_p * n_layers)(*[0x10000 * (i + 1) for i in range(n_layers)])
        vp = (ctypes.c_void_p * n_layers)(*[0x90000000 + 0x10000 * i for i in range(n_layers)])
        self.h = L.sqa_kv_cache_create(n_layers, D, Hkv, cap, kp, vp)
        assert self.h


def test_kv_cache_bookkeeping_follows_kv_rs(sqa):
    L = sqa.lib()
    assert L.sqa_kv_cache_layer_bytes(256, 2, 172032) == 172032 * 576 // 2  # 99 MB per K or V
    assert L.sqa_kv_cache_layer_bytes(256, 2, 1000) == 1024 * 288             # padded to 256
    kv = FakeKv(sqa, cap=1000).h
    assert L.sqa_kv_cache_n_kv_padded(kv) == 0
    assert L.sqa_kv_cache_begin_step(kv, 300) == 0
    assert (L.sqa_kv_cache_step_start(kv), L.sqa_kv_cache_n_used(kv)) == (0, 300)
    assert L.sqa_kv_cache_n_kv_padded(kv) == 512
    assert L.sqa_kv_cache_n_kv_padded_after(kv, 213) == 768
    assert L.sqa_kv_cache_begin_step(kv, 1) == 0 and L.sqa_kv_cache_step_start(kv) == 300
    assert L.sqa_kv_cache_begin_step(kv, 700) == 5                  # overflow (kv.rs:239-253)
    assert "overflow" in sqa.last_error()
    assert L.sqa_kv_cache_n_used(kv) == 301                          # unchanged by the failure
    assert L.sqa_kv_cache_rewind_to(kv, 400) == 6                    # past written
    assert L.sqa_kv_cache_rewind_to(kv, 100) == 0
    assert (L.sqa_kv_cache_step_start(kv), L.sqa_kv_cache_n_used(kv)) == (100, 100)
    t = sqa.Tensor()
    assert L.sqa_kv_cache_k_view(kv, 3, ctypes.byref(t)) == 0
    assert list(t.ne) == [256, 256, 2, 1] and list(t.nb)[:3] == [18, 288, 144]
    assert t.data == 0x10000 * 4 and t.type == 2
    assert L.sqa_kv_cache_v_view(kv, 10, ctypes.byref(t)) == 6
    L.sqa_kv_cache_reset(kv)
    assert L.sqa_kv_cache_n_used(kv) == 0
    L.sqa_kv_cache_destroy(kv)


def test_kv_cache_create_rejects_bad_geometry(sqa):
    L = sqa.lib()
    bufs = (ctypes.c_void_p * 1)(0x1000)
    assert not L.sqa_kv_cache_create(1, 100, 2, 256, bufs, bufs)    # head_dim % 32
    assert "multiple of 32" in sqa.last_error()
    nul = (ctypes.c_void_p * 1)(None)
    assert not L.sqa_kv_cache_create(1, 256, 2, 256, bufs, nul)


def test_producer_argument_checks_before_any_launch(sqa):
    """rope_norm entry points reject what they do not run (YaRN ramp, odd n_rot,
    head dims outside {64, 128, 256}, short pos, mismatched dst) with a status
    and a message, without touching the device (fake non-null pointers)."""
    L = sqa.lib()
    T = sqa.Tensor.make
    D, n_head, n_tok = 256, 2, 8
    src = T(0, [D, n_head, n_tok], [4, D * 4, n_head * D * 4], 4096)
    w = T(0, [D], [4], 8192)
    pos = T(26, [4 * n_tok], [4], 12288)
    idx = T(27, [n_tok], [8], 16384)
    dst = T(2, [n_head * D, 64], [18, n_head * D // 32 * 18], 32768)
    by = ctypes.byref

    def call(rope, s=src, p=pos, d=dst, i=idx, ww=w):
        return L.sqa_rope_norm_set_rows_q4_0(by(d), by(s), by(ww) if ww else None, 1e-6, by(p), by(rope),
                                             by(i), None)

    good = sqa.rope_params(64, (11, 11, 10, 0), 1e7)
    yarn = sqa.rope_params(64, (11, 11, 10, 0), 1e7, ext_factor=1.0)
    assert call(yarn) == 2 and b"ext_factor" in L.sqa_last_error()
    assert call(sqa.rope_params(12, (3, 3, 0, 0), 1e7)) == 2           # n_rot % 8
    assert call(sqa.rope_params(64, (0, 0, 0, 0), 1e7)) == 1            # empty sections
    assert call(good, p=T(26, [4 * n_tok - 1], [4], 12288)) == 1        # short pos
    assert call(good, d=T(2, [D, 64], [18, 144], 32768)) == 1           # dst row of one head
    assert call(good, s=T(0, [96, n_head, n_tok], [4, 384, 768], 4096),
                d=T(2, [96 * n_head, 64], [18, 108], 32768)) == 2        # head dim 96
    assert call(good, ww=T(0, [D], [4], 8196)) == 1                     # unaligned weight
    out = T(0, [D, n_head, n_tok], [4, D * 4, n_head * D * 4], 65536)
    assert L.sqa_rope_norm_f32(by(out), by(src), by(w), 1e-6, by(pos), by(yarn), None) == 2
    # the support query answers without launching, for both forms
    assert L.sqa_supports_rope_norm(by(dst), by(src), by(w), by(pos), by(good), by(idx)) == 1
    assert L.sqa_supports_rope_norm(by(dst), by(src), by(w), by(pos), by(yarn), by(idx)) == 0
    assert L.sqa_supports_rope_norm(by(out), by(src), None, by(pos), by(good), None) == 1
    assert L.sqa_supports_rope_norm(by(out), by(src), by(w), by(pos), by(sqa.rope_params(12, (3, 3, 0, 0), 1e7)),
                                    None) == 0
