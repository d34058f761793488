// abi.cpp - the extern "C" entry points of include/sqattn.h: argument
// validation, support queries, error reporting and kernel dispatch.
//
// Validation mirrors what ggml checks when the engine builds these nodes
// (src/backend/ffi.rs:363-405 of the reference): anything ggml itself would
// reject is SQA_ERR_INVALID; a valid op this library has no kernel for is
// SQA_ERR_UNSUPPORTED (where ggml-cuda would abort, runner.rs:509-513).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "common.hpp"

namespace sqa {

static thread_local char g_err[512] = "";

int set_error(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return status;
}

int hip_status(hipError_t e, const char *what) {
    if (e == hipSuccess) return SQA_OK;
    return set_error(SQA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int device_cu_count() {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
    if (cache[dev] == 0) {
        int cu = 0;
        if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0)
            cu = 256;
        cache[dev] = cu;
    }
    return cache[dev];
}

namespace {

bool is_contig_rows(const sqa_tensor &t, int64_t esize) { return t.nb[0] == (uint64_t)esize; }

// Checks shared by sqa_flash_attn_ext and the causal variant.
int check_fa(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
             const sqa_tensor *dst, bool *decode) {
    if (!q || !k || !v || !dst) return set_error(SQA_ERR_INVALID, "flash_attn_ext: null tensor");
    if (!q->data || !k->data || !v->data || !dst->data)
        return set_error(SQA_ERR_INVALID, "flash_attn_ext: null data pointer");
    if (q->type != SQA_TYPE_F32 || dst->type != SQA_TYPE_F32)
        return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext: q and dst must be F32");
    if (k->type != SQA_TYPE_Q4_0 || v->type != SQA_TYPE_Q4_0)
        return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext: K and V must be q4_0");
    if (q->ne[0] != k->ne[0] || k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2])
        return set_error(SQA_ERR_INVALID, "flash_attn_ext: q/k/v shape mismatch");
    if (k->ne[2] <= 0 || q->ne[2] % k->ne[2] != 0)
        return set_error(SQA_ERR_INVALID, "flash_attn_ext: n_head %% n_head_kv != 0");
    if (dst->ne[0] != v->ne[0] || dst->ne[1] != q->ne[2] || dst->ne[2] != q->ne[1] || dst->ne[3] != 1)
        return set_error(SQA_ERR_INVALID, "flash_attn_ext: dst must be [D, H, n_q, 1]");
    if (q->ne[3] != 1 || k->ne[3] != 1 || v->ne[3] != 1)
        return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext: ne[3] > 1 (batched sequences)");
    if (q->ne[0] != kHeadDim || v->ne[0] != kHeadDim)
        return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext: head_dim %lld (only 256)",
                         (long long)q->ne[0]);
    if (q->ne[1] < 1 || k->ne[1] < 1)
        return set_error(SQA_ERR_INVALID, "flash_attn_ext: empty q or KV");
    if (!is_contig_rows(*q, 4) || q->nb[1] % 4 || q->nb[2] % 4)
        return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext: q rows must have unit element stride");
    const uint64_t head_row = kHeadRowBytes;
    const uint64_t row = head_row * (uint64_t)k->ne[2];
    for (const sqa_tensor *t : {k, v}) {
        if (t->nb[0] != SQA_Q4_0_BLOCK_BYTES || t->nb[2] != head_row || t->nb[1] != row)
            return set_error(SQA_ERR_UNSUPPORTED,
                             "flash_attn_ext: K/V must use the cache layout (nb = 18, %llu, %llu)",
                             (unsigned long long)row, (unsigned long long)head_row);
        if ((uintptr_t)t->data % 16)
            return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext: K/V data must be 16-byte aligned");
    }
    const uint64_t dst_row = 4ull * kHeadDim;
    if (dst->nb[0] != 4 || dst->nb[1] != dst_row || dst->nb[2] != dst_row * (uint64_t)dst->ne[1])
        return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext: dst must be contiguous");
    if ((uintptr_t)dst->data % 16)
        return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext: dst data must be 16-byte aligned");
    const int64_t G = q->ne[2] / k->ne[2];
    const bool q_aligned = (uintptr_t)q->data % 16 == 0 && q->nb[1] % 16 == 0 && q->nb[2] % 16 == 0;
    // the split-KV decode kernel: up to 4 positions and 16 query rows per KV head,
    // 16-byte aligned q rows; everything else runs as a prefill chunk
    *decode = q->ne[1] <= 4 && q->ne[1] * G <= 16 && q_aligned;
    if (!*decode && 16 % G != 0)
        return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext: prefill needs n_head/n_head_kv to divide 16");
    return SQA_OK;
}

int check_mask(const sqa_tensor *mask, const sqa_tensor *q, const sqa_tensor *k) {
    if (!mask) return SQA_OK;
    if (!mask->data) return set_error(SQA_ERR_INVALID, "flash_attn_ext: mask has no data");
    if (mask->type != SQA_TYPE_F16)
        return set_error(SQA_ERR_INVALID, "flash_attn_ext: mask must be F16");
    if (mask->ne[0] != k->ne[1])
        return set_error(SQA_ERR_INVALID, "flash_attn_ext: mask->ne[0] (%lld) != n_kv (%lld)",
                         (long long)mask->ne[0], (long long)k->ne[1]);
    if (mask->ne[1] < q->ne[1])
        return set_error(SQA_ERR_INVALID, "flash_attn_ext: mask has fewer rows than queries");
    if (mask->nb[0] != 2 || mask->nb[1] % 2)
        return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext: mask rows must be contiguous");
    if (mask->ne[2] != 1 || mask->ne[3] != 1)
        return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext: per-head masks not supported");

    return SQA_OK;
}

size_t fa_workspace(const sqa_tensor *q, const sqa_tensor *k, bool decode) {
    const int64_t n_q = q->ne[1], H = q->ne[2], n_kv = k->ne[1], Hkv = k->ne[2];
    return decode ? fa_decode_workspace(n_q, H, Hkv, n_kv) : fa_prefill_workspace(n_q, H, Hkv, n_kv);
}

int run_fa(const FaArgs &a, bool decode, hipStream_t s) {
    return decode ? launch_fa_decode(a, s) : launch_fa_prefill(a, s);
}

}  // namespace
}  // namespace sqa

using namespace sqa;

extern "C" {

const char *sqa_version(void) { return "sqattn-gfx950 0.1.0"; }
const char *sqa_last_error(void) { return g_err; }

const char *sqa_status_string(int status) {
    switch (status) {
        case SQA_OK: return "ok";
        case SQA_ERR_INVALID: return "invalid argument";
        case SQA_ERR_UNSUPPORTED: return "unsupported configuration";
        case SQA_ERR_WORKSPACE: return "workspace too small";
        case SQA_ERR_HIP: return "HIP runtime error";
        case SQA_ERR_OVERFLOW: return "KV cache overflow";
        case SQA_ERR_RANGE: return "argument out of range";
        default: return "unknown status";
    }
}

int sqa_supports_set_rows(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *idx) {
    if (!dst || !src || !idx) return 0;
    if (dst->type != SQA_TYPE_Q4_0 || src->type != SQA_TYPE_F32 || idx->type != SQA_TYPE_I64) return 0;
    if (src->ne[0] != dst->ne[0] || src->ne[0] % SQA_QK4_0 || idx->ne[0] != src->ne[1]) return 0;
    if (src->ne[2] != 1 || src->ne[3] != 1 || dst->ne[2] != 1 || dst->ne[3] != 1) return 0;
    if (src->nb[0] != 4 || dst->nb[0] != SQA_Q4_0_BLOCK_BYTES || idx->nb[0] % 8) return 0;
    if ((uintptr_t)dst->data % 2 || dst->nb[1] % 2 || (uintptr_t)src->data % 4 || src->nb[1] % 4) return 0;
    return 1;
}

int sqa_set_rows_q4_0(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *idx,
                      void *stream) {
    if (!dst || !src || !idx) return set_error(SQA_ERR_INVALID, "set_rows: null tensor");
    if (src->ne[1] > 0 && (!dst->data || !src->data || !idx->data))
        return set_error(SQA_ERR_INVALID, "set_rows: null data pointer");
    if (dst->type != SQA_TYPE_Q4_0 || src->type != SQA_TYPE_F32 || idx->type != SQA_TYPE_I64)
        return set_error(SQA_ERR_INVALID, "set_rows: types must be q4_0 <- F32 at I64");
    if (src->ne[0] != dst->ne[0] || idx->ne[0] != src->ne[1])
        return set_error(SQA_ERR_INVALID, "set_rows: shape mismatch");
    if (src->ne[0] % SQA_QK4_0)
        return set_error(SQA_ERR_INVALID, "set_rows: row length %lld not a multiple of 32",
                         (long long)src->ne[0]);
    if (!sqa_supports_set_rows(dst, src, idx))
        return set_error(SQA_ERR_UNSUPPORTED, "set_rows: strides/alignment not supported");
    return launch_set_rows_q4_0(*dst, *src, *idx, (hipStream_t)stream);
}

// ---- K/Q producer: norm + IMROPE (+ q4_0 set_rows) ----------------------------

static int check_producer(const sqa_tensor *src, const sqa_tensor *norm_w, const sqa_tensor *pos,
                          const sqa_rope *rope, const char *what) {
    if (!src || !pos || !rope) return set_error(SQA_ERR_INVALID, "%s: null argument", what);
    if (src->type != SQA_TYPE_F32 || pos->type != SQA_TYPE_I32)
        return set_error(SQA_ERR_INVALID, "%s: src must be F32 and pos I32", what);
    const int64_t D = src->ne[0], n_tok = src->ne[2];
    if (src->ne[3] != 1 || pos->ne[0] != 4 * n_tok || pos->nb[0] != 4)
        return set_error(SQA_ERR_INVALID, "%s: pos must be I32 [4 * n_tok] contiguous", what);
    if (n_tok > 0 && (!src->data || !pos->data)) return set_error(SQA_ERR_INVALID, "%s: null data pointer", what);
    if (D != 64 && D != 128 && D != 256)
        return set_error(SQA_ERR_UNSUPPORTED, "%s: head dim %lld not in {64, 128, 256}", what, (long long)D);
    if (src->nb[0] != 4 || src->nb[1] % 4 || src->nb[2] % 4 || (uintptr_t)src->data % 4)
        return set_error(SQA_ERR_UNSUPPORTED, "%s: src elements must be contiguous F32", what);
    if (norm_w && (norm_w->type != SQA_TYPE_F32 || norm_w->ne[0] != D || norm_w->nb[0] != 4 ||
                   (uintptr_t)norm_w->data % 16))
        return set_error(SQA_ERR_INVALID, "%s: norm weight must be F32 [D], contiguous, 16-byte aligned", what);
    if (rope->n_rot <= 0 || rope->n_rot % 8 || rope->n_rot > D)
        return set_error(SQA_ERR_UNSUPPORTED, "%s: n_rot %d must be a positive multiple of 8 <= D", what,
                         rope->n_rot);
    int sect = 0;
    for (int k = 0; k < 4; ++k) {
        if (rope->sections[k] < 0) return set_error(SQA_ERR_INVALID, "%s: negative rope section", what);
        sect += rope->sections[k];
    }
    if (sect <= 0) return set_error(SQA_ERR_INVALID, "%s: rope sections sum to zero", what);
    if (rope->ext_factor != 0.0f)
        return set_error(SQA_ERR_UNSUPPORTED, "%s: ext_factor != 0 (YaRN ramp) is not supported", what);
    if (!std::isfinite(rope->freq_base) || rope->freq_base <= 0.0f)
        return set_error(SQA_ERR_INVALID, "%s: freq_base must be positive", what);
    return SQA_OK;
}

static int check_producer_q4(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *norm_w,
                             const sqa_tensor *pos, const sqa_rope *rope, const sqa_tensor *idx) {
    const char *what = "rope_norm_set_rows_q4_0";
    int st = check_producer(src, norm_w, pos, rope, what);
    if (st != SQA_OK) return st;
    if (!dst || !idx) return set_error(SQA_ERR_INVALID, "%s: null dst or idx", what);
    if (dst->type != SQA_TYPE_Q4_0 || idx->type != SQA_TYPE_I64)
        return set_error(SQA_ERR_INVALID, "%s: dst must be Q4_0 and idx I64", what);
    const int64_t D = src->ne[0], n_head = src->ne[1], n_tok = src->ne[2];
    if (dst->ne[0] != D * n_head || idx->ne[0] != n_tok)
        return set_error(SQA_ERR_INVALID, "%s: dst row must hold n_head * D values, idx n_tok entries", what);
    if (dst->nb[0] != SQA_Q4_0_BLOCK_BYTES || dst->nb[1] % 2 || (uintptr_t)dst->data % 2 || idx->nb[0] % 8)
        return set_error(SQA_ERR_UNSUPPORTED, "%s: dst/idx strides not supported", what);
    if (n_tok > 0 && (!dst->data || !idx->data)) return set_error(SQA_ERR_INVALID, "%s: null data pointer", what);
    return SQA_OK;
}

int sqa_supports_rope_norm(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *norm_w,
                           const sqa_tensor *pos, const sqa_rope *rope, const sqa_tensor *idx) {
    if (idx) return check_producer_q4(dst, src, norm_w, pos, rope, idx) == SQA_OK;
    if (check_producer(src, norm_w, pos, rope, "rope_norm_f32") != SQA_OK) return 0;
    if (!dst || dst->type != SQA_TYPE_F32 || dst->ne[0] != src->ne[0] || dst->ne[1] != src->ne[1] ||
        dst->ne[2] != src->ne[2] || dst->nb[0] != 4 || dst->nb[1] != (uint64_t)(4 * src->ne[0]) ||
        dst->nb[2] != (uint64_t)(4 * src->ne[0] * src->ne[1]) || (uintptr_t)dst->data % 16)
        return 0;
    return 1;
}

int sqa_rope_norm_set_rows_q4_0(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *norm_w,
                                float eps, const sqa_tensor *pos, const sqa_rope *rope,
                                const sqa_tensor *idx, void *stream) {
    const int st = check_producer_q4(dst, src, norm_w, pos, rope, idx);
    if (st != SQA_OK) return st;
    const float ts = powf(rope->freq_base, -2.0f / (float)rope->n_rot);
    return launch_rope_norm(dst, *src, norm_w, eps, *pos, *rope, ts, idx, (hipStream_t)stream);
}

int sqa_rope_norm_f32(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *norm_w, float eps,
                      const sqa_tensor *pos, const sqa_rope *rope, void *stream) {
    const char *what = "rope_norm_f32";
    int st = check_producer(src, norm_w, pos, rope, what);
    if (st != SQA_OK) return st;
    if (!dst || dst->type != SQA_TYPE_F32) return set_error(SQA_ERR_INVALID, "%s: dst must be F32", what);
    const int64_t D = src->ne[0], n_head = src->ne[1], n_tok = src->ne[2];
    if (dst->ne[0] != D || dst->ne[1] != n_head || dst->ne[2] != n_tok || dst->nb[0] != 4 ||
        dst->nb[1] != (uint64_t)(4 * D) || dst->nb[2] != (uint64_t)(4 * D * n_head) || (uintptr_t)dst->data % 16)
        return set_error(SQA_ERR_INVALID, "%s: dst must be F32 [D, n_head, n_tok] contiguous, 16-byte aligned",
                         what);
    const float ts = powf(rope->freq_base, -2.0f / (float)rope->n_rot);
    return launch_rope_norm(dst, *src, norm_w, eps, *pos, *rope, ts, nullptr, (hipStream_t)stream);
}

size_t sqa_flash_attn_ext_workspace_size(const sqa_tensor *q, const sqa_tensor *k,
                                         const sqa_tensor *v, const sqa_tensor *dst) {
    bool decode = false;
    if (check_fa(q, k, v, dst, &decode) != SQA_OK) return 0;
    return fa_workspace(q, k, decode);
}

int sqa_supports_flash_attn_ext(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                                const sqa_tensor *mask, float scale, float max_bias,
                                float logit_softcap, const sqa_tensor *dst) {
    bool decode = false;
    if (check_fa(q, k, v, dst, &decode) != SQA_OK) return 0;
    if (check_mask(mask, q, k) != SQA_OK) return 0;
    if (!isfinite(scale) || max_bias != 0.0f || logit_softcap != 0.0f) return 0;
    return 1;
}

int sqa_flash_attn_ext(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                       const sqa_tensor *mask, float scale, float max_bias, float logit_softcap,
                       const sqa_tensor *dst, void *workspace, size_t workspace_bytes,
                       void *stream) {
    bool decode = false;
    int rc = check_fa(q, k, v, dst, &decode);
    if (rc) return rc;
    rc = check_mask(mask, q, k);
    if (rc) return rc;
    if (!isfinite(scale)) return set_error(SQA_ERR_INVALID, "flash_attn_ext: scale not finite");
    if (max_bias != 0.0f)
        return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext: ALiBi (max_bias != 0) not supported");
    if (logit_softcap != 0.0f)
        return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext: logit_softcap not supported");
    FaArgs a{q, k, v, mask, nullptr, dst, scale, -1, workspace, workspace_bytes};
    return run_fa(a, decode, (hipStream_t)stream);
}

int sqa_flash_attn_ext_static(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                              const sqa_tensor *mask, float scale, float max_bias, float logit_softcap,
                              const sqa_tensor *dst, void *stream) {
    bool decode = false;
    int rc = check_fa(q, k, v, dst, &decode);
    if (rc) return rc;
    rc = check_mask(mask, q, k);
    if (rc) return rc;
    if (!isfinite(scale)) return set_error(SQA_ERR_INVALID, "flash_attn_ext_static: scale not finite");
    if (max_bias != 0.0f)
        return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext_static: ALiBi (max_bias != 0) not supported");
    if (logit_softcap != 0.0f)
        return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext_static: logit_softcap not supported");
    if (!decode)
        return set_error(SQA_ERR_UNSUPPORTED,
                         "flash_attn_ext_static: only decode/verify shapes (up to 4 positions and 16 query "
                         "rows per KV head, 16-byte aligned q rows); use sqa_flash_attn_ext");
    const size_t need = fa_decode_workspace(q->ne[1], q->ne[2], k->ne[2], k->ne[1],
                                            decode_mask_needs_copy(mask, k->ne[1]));
    if (need > kStaticScratchBytes)
        return set_error(SQA_ERR_WORKSPACE,
                         "flash_attn_ext_static: these shapes need %zu bytes of scratch, above its %zu-byte "
                         "maximum; use sqa_flash_attn_ext with a workspace",
                         need, kStaticScratchBytes);
    void *ws = nullptr;
    rc = static_scratch(&ws);
    if (rc) return rc;
    FaArgs a{q, k, v, mask, nullptr, dst, scale, -1, ws, kStaticScratchBytes};
    return launch_fa_decode(a, (hipStream_t)stream);
}

int sqa_flash_attn_ext_causal(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                              int64_t q_pos0, const sqa_tensor *gate, float scale,
                              const sqa_tensor *dst, void *workspace, size_t workspace_bytes,
                              void *stream) {
    bool decode = false;
    int rc = check_fa(q, k, v, dst, &decode);
    if (rc) return rc;
    if (q_pos0 < 0) return set_error(SQA_ERR_RANGE, "flash_attn_ext_causal: q_pos0 < 0");
    if (!isfinite(scale)) return set_error(SQA_ERR_INVALID, "flash_attn_ext: scale not finite");
    if (gate) {
        if (!gate->data || gate->type != SQA_TYPE_F32 || gate->ne[0] != dst->ne[0] ||
            gate->ne[1] != dst->ne[1] || gate->ne[2] != dst->ne[2] || gate->nb[0] != 4 ||
            gate->nb[1] % 4 || gate->nb[2] % 4)
            return set_error(SQA_ERR_INVALID, "flash_attn_ext_causal: gate must be F32 [D, H, n_q]");
    }
    FaArgs a{q, k, v, nullptr, gate, dst, scale, q_pos0, workspace, workspace_bytes};
    return run_fa(a, decode, (hipStream_t)stream);
}

int sqa_sigmoid_mul(const sqa_tensor *dst, const sqa_tensor *x, const sqa_tensor *gate,
                    void *stream) {
    if (!dst || !x || !gate) return set_error(SQA_ERR_INVALID, "sigmoid_mul: null tensor");
    for (const sqa_tensor *t : {dst, x, gate}) {
        if (t->type != SQA_TYPE_F32 || t->nb[0] != 4 || t->ne[2] != 1 || t->ne[3] != 1)
            return set_error(SQA_ERR_INVALID, "sigmoid_mul: tensors must be 2-D F32 with unit stride");
        if (t->ne[0] != x->ne[0] || t->ne[1] != x->ne[1])
            return set_error(SQA_ERR_INVALID, "sigmoid_mul: shape mismatch");
        if (x->ne[0] * x->ne[1] > 0 && !t->data)
            return set_error(SQA_ERR_INVALID, "sigmoid_mul: null data pointer");
    }
    return launch_sigmoid_mul(*dst, *x, *gate, (hipStream_t)stream);
}

static int check_out_proj(const sqa_tensor *w, const sqa_tensor *x, const sqa_tensor *gate,
                          const sqa_tensor *dst) {
    if (!w || !x) return set_error(SQA_ERR_INVALID, "out_proj: null tensor");
    const int64_t K = w->ne[0], N = w->ne[1], M = x->ne[1];
    if (w->type != SQA_TYPE_Q4_K || w->ne[2] != 1 || w->ne[3] != 1)
        return set_error(SQA_ERR_UNSUPPORTED, "out_proj: weight must be a 2-D Q4_K tensor");
    if (K <= 0 || K % 256 || N % 16)
        return set_error(SQA_ERR_UNSUPPORTED, "out_proj: need K %% 256 == 0 and N %% 16 == 0 (K=%lld, N=%lld)",
                         (long long)K, (long long)N);
    if (w->nb[1] % 16 || (uintptr_t)w->data % 16)
        return set_error(SQA_ERR_UNSUPPORTED, "out_proj: weight rows must be 16-byte aligned");
    if (x->type != SQA_TYPE_F32 || x->nb[0] != 4 || x->nb[1] % 4 || x->ne[0] != K || x->ne[2] != 1 || x->ne[3] != 1)
        return set_error(SQA_ERR_INVALID, "out_proj: x must be F32 [K, M] with unit element stride");
    if (gate && (gate->type != SQA_TYPE_F32 || gate->nb[0] != 4 || gate->nb[1] % 4 || gate->ne[0] != K ||
                 gate->ne[1] != M || gate->ne[2] != 1 || gate->ne[3] != 1))
        return set_error(SQA_ERR_INVALID, "out_proj: gate must be F32 [K, M] with unit element stride");
    if (dst) {
        if (dst->type != SQA_TYPE_F32 || dst->nb[0] != 4 || dst->ne[0] != N || dst->ne[1] != M ||
            dst->ne[2] != 1 || dst->ne[3] != 1)
            return set_error(SQA_ERR_INVALID, "out_proj: dst must be F32 [N, M]");
        if (dst->nb[1] % 16 || (uintptr_t)dst->data % 16)
            return set_error(SQA_ERR_UNSUPPORTED, "out_proj: dst rows must be 16-byte aligned");
    }
    if (M > 0 && N > 0 && (!w->data || !x->data || (gate && !gate->data) || (dst && !dst->data)))
        return set_error(SQA_ERR_INVALID, "out_proj: null data pointer");
    return SQA_OK;
}

size_t sqa_out_proj_workspace_size(const sqa_tensor *w, const sqa_tensor *x) {
    if (!w || !x) return 0;
    return out_proj_workspace(w->ne[0], x->ne[1]);
}

int sqa_supports_out_proj(const sqa_tensor *w, const sqa_tensor *x, const sqa_tensor *gate,
                          const sqa_tensor *dst) {
    return check_out_proj(w, x, gate, dst) == SQA_OK ? 1 : 0;
}

int sqa_out_proj(const sqa_tensor *w, const sqa_tensor *x, const sqa_tensor *gate, const sqa_tensor *dst,
                 void *workspace, size_t workspace_bytes, void *stream) {
    if (!dst) return set_error(SQA_ERR_INVALID, "out_proj: null dst");
    const int rc = check_out_proj(w, x, gate, dst);
    if (rc != SQA_OK) return rc;
    return launch_out_proj(*w, *x, gate, *dst, workspace, workspace_bytes, (hipStream_t)stream);
}

int sqa_fill_causal_mask(const sqa_tensor *mask, int64_t step_start, void *stream) {
    if (!mask || (mask->ne[0] * mask->ne[1] > 0 && !mask->data))
        return set_error(SQA_ERR_INVALID, "fill_causal_mask: null tensor");
    if (mask->type != SQA_TYPE_F16 || mask->nb[0] != 2 || mask->nb[1] % 2)
        return set_error(SQA_ERR_INVALID, "fill_causal_mask: mask must be F16 with contiguous rows");
    if (step_start < 0) return set_error(SQA_ERR_RANGE, "fill_causal_mask: step_start < 0");
    return launch_fill_causal_mask(*mask, step_start, (hipStream_t)stream);
}

}  // extern "C"
