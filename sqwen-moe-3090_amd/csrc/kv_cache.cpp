// kv_cache.cpp - host-side mirror of the engine's KvCache bookkeeping
// (reference: src/engine/kv.rs:67-448): capacity padding, the shared write
// cursor, overflow and rewind errors, the FA-order K/V views, and append
// through the q4_0 set_rows kernel. No device memory is allocated here: the
// caller hands in one K and one V buffer per layer (kv.rs keeps them in a
// persistent backend buffer, src/backend/ctx.rs:455-570).
#include <new>
#include <vector>

#include "common.hpp"

struct sqa_kv_cache {
    int32_t n_layers;
    int64_t head_dim, n_head_kv, kv_cap, kv_cap_alloc;
    int64_t n_used, step_start;
    std::vector<void *> k, v;
};

using namespace sqa;

namespace {
int64_t cap_alloc(int64_t cap) { return (cap + SQA_KV_PAD - 1) / SQA_KV_PAD * SQA_KV_PAD; }
int64_t row_bytes_head(int64_t head_dim) { return head_dim / SQA_QK4_0 * SQA_Q4_0_BLOCK_BYTES; }

int make_view(const sqa_kv_cache *kv, int32_t slot, bool is_k, sqa_tensor *out) {
    if (!kv || !out) return set_error(SQA_ERR_INVALID, "kv_cache view: null argument");
    if (slot < 0 || slot >= kv->n_layers)
        return set_error(SQA_ERR_RANGE, "kv_cache view: slot %d of %d", slot, kv->n_layers);
    const int64_t rh = row_bytes_head(kv->head_dim);
    const int64_t rg = rh * kv->n_head_kv;
    const int64_t n_kv = sqa_kv_cache_n_kv_padded(kv);
    out->type = SQA_TYPE_Q4_0;
    out->pad_ = 0;
    out->ne[0] = kv->head_dim;
    out->ne[1] = n_kv;
    out->ne[2] = kv->n_head_kv;
    out->ne[3] = 1;
    out->nb[0] = SQA_Q4_0_BLOCK_BYTES;
    out->nb[1] = (uint64_t)rg;
    out->nb[2] = (uint64_t)rh;
    out->nb[3] = (uint64_t)(rg * kv->kv_cap_alloc);
    out->data = is_k ? kv->k[slot] : kv->v[slot];
    return SQA_OK;
}
}  // namespace

extern "C" {

size_t sqa_kv_cache_layer_bytes(int64_t head_dim, int64_t n_head_kv, int64_t kv_cap) {
    if (head_dim <= 0 || head_dim % SQA_QK4_0 || n_head_kv <= 0 || kv_cap <= 0) return 0;
    return (size_t)(cap_alloc(kv_cap) * n_head_kv * row_bytes_head(head_dim));
}

sqa_kv_cache *sqa_kv_cache_create(int32_t n_layers, int64_t head_dim, int64_t n_head_kv,
                                  int64_t kv_cap, void *const *k_bufs, void *const *v_bufs) {
    if (n_layers <= 0 || head_dim <= 0 || n_head_kv <= 0 || kv_cap <= 0) {
        set_error(SQA_ERR_INVALID, "kv_cache_create: non-positive size");
        return nullptr;
    }
    if (head_dim % SQA_QK4_0) {
        set_error(SQA_ERR_INVALID, "kv_cache_create: head_dim %lld not a multiple of 32",
                  (long long)head_dim);
        return nullptr;
    }
    if (!k_bufs || !v_bufs) {
        set_error(SQA_ERR_INVALID, "kv_cache_create: null buffer list");
        return nullptr;
    }
    for (int32_t i = 0; i < n_layers; ++i) {
        if (!k_bufs[i] || !v_bufs[i]) {
            set_error(SQA_ERR_INVALID, "kv_cache_create: null buffer for layer %d", i);
            return nullptr;
        }
    }
    sqa_kv_cache *kv = new (std::nothrow) sqa_kv_cache;
    if (!kv) {
        set_error(SQA_ERR_INVALID, "kv_cache_create: out of host memory");
        return nullptr;
    }
    kv->n_layers = n_layers;
    kv->head_dim = head_dim;
    kv->n_head_kv = n_head_kv;
    kv->kv_cap = kv_cap;
    kv->kv_cap_alloc = cap_alloc(kv_cap);
    kv->n_used = 0;
    kv->step_start = 0;
    kv->k.assign(k_bufs, k_bufs + n_layers);
    kv->v.assign(v_bufs, v_bufs + n_layers);
    return kv;
}

void sqa_kv_cache_destroy(sqa_kv_cache *kv) { delete kv; }

int64_t sqa_kv_cache_n_used(const sqa_kv_cache *kv) { return kv ? kv->n_used : -1; }
int64_t sqa_kv_cache_step_start(const sqa_kv_cache *kv) { return kv ? kv->step_start : -1; }

int64_t sqa_kv_cache_n_kv_padded(const sqa_kv_cache *kv) {
    return kv ? cap_alloc(kv->n_used) : -1;
}

int64_t sqa_kv_cache_n_kv_padded_after(const sqa_kv_cache *kv, int64_t n_tokens) {
    return kv ? cap_alloc(kv->n_used + n_tokens) : -1;
}

int sqa_kv_cache_begin_step(sqa_kv_cache *kv, int64_t n_tokens) {
    if (!kv) return set_error(SQA_ERR_INVALID, "kv_cache_begin_step: null cache");
    if (n_tokens < 0) return set_error(SQA_ERR_RANGE, "kv_cache_begin_step: n_tokens < 0");
    if (kv->n_used + n_tokens > kv->kv_cap)
        return set_error(SQA_ERR_OVERFLOW, "KV cache overflow: n_used=%lld + n_tokens=%lld > kv_cap=%lld",
                         (long long)kv->n_used, (long long)n_tokens, (long long)kv->kv_cap);
    kv->step_start = kv->n_used;
    kv->n_used += n_tokens;
    return SQA_OK;
}

int sqa_kv_cache_rewind_to(sqa_kv_cache *kv, int64_t pos) {
    if (!kv) return set_error(SQA_ERR_INVALID, "kv_cache_rewind_to: null cache");
    if (pos < 0 || pos > kv->n_used)
        return set_error(SQA_ERR_RANGE, "KV rewind out of range: pos=%lld > written %lld",
                         (long long)pos, (long long)kv->n_used);
    if (pos > kv->kv_cap)
        return set_error(SQA_ERR_RANGE, "KV rewind out of range: pos=%lld > capacity %lld",
                         (long long)pos, (long long)kv->kv_cap);
    kv->n_used = pos;
    kv->step_start = pos;
    return SQA_OK;
}

void sqa_kv_cache_reset(sqa_kv_cache *kv) {
    if (kv) {
        kv->n_used = 0;
        kv->step_start = 0;
    }
}

int sqa_kv_cache_k_view(const sqa_kv_cache *kv, int32_t slot, sqa_tensor *out) {
    return make_view(kv, slot, true, out);
}

int sqa_kv_cache_v_view(const sqa_kv_cache *kv, int32_t slot, sqa_tensor *out) {
    return make_view(kv, slot, false, out);
}

int sqa_kv_cache_append(sqa_kv_cache *kv, int32_t slot, const sqa_tensor *k_cur,
                        const sqa_tensor *v_cur, const sqa_tensor *idx, void *stream) {
    if (!kv || !k_cur || !v_cur || !idx) return set_error(SQA_ERR_INVALID, "kv_cache_append: null argument");
    if (slot < 0 || slot >= kv->n_layers)
        return set_error(SQA_ERR_RANGE, "kv_cache_append: slot %d of %d", slot, kv->n_layers);
    const int64_t n_embd = kv->head_dim * kv->n_head_kv;
    const int64_t n_tok = k_cur->ne[1];
    for (const sqa_tensor *t : {k_cur, v_cur}) {
        if (t->type != SQA_TYPE_F32 || t->ne[0] != n_embd || t->ne[1] != n_tok || t->nb[0] != 4 ||
            t->nb[1] != (uint64_t)(n_embd * 4))
            return set_error(SQA_ERR_INVALID,
                             "kv_cache_append: K/V must be F32 [%lld, n_tokens] with one contiguous row per token",
                             (long long)n_embd);
    }
    if (idx->type != SQA_TYPE_I64 || idx->ne[0] != n_tok)
        return set_error(SQA_ERR_INVALID, "kv_cache_append: idx must be I64 [n_tokens]");
    if (kv->step_start + n_tok != kv->n_used)
        return set_error(SQA_ERR_INVALID, "kv_cache_append: n_tokens %lld does not match begin_step",
                         (long long)n_tok);
    const int64_t rg = row_bytes_head(kv->head_dim) * kv->n_head_kv;
    sqa_tensor dst{};
    dst.type = SQA_TYPE_Q4_0;
    dst.ne[0] = n_embd;
    dst.ne[1] = kv->kv_cap_alloc;
    dst.ne[2] = dst.ne[3] = 1;
    dst.nb[0] = SQA_Q4_0_BLOCK_BYTES;
    dst.nb[1] = (uint64_t)rg;
    dst.nb[2] = dst.nb[3] = (uint64_t)(rg * kv->kv_cap_alloc);
    dst.data = kv->k[slot];
    int rc = sqa_set_rows_q4_0(&dst, k_cur, idx, stream);
    if (rc) return rc;
    dst.data = kv->v[slot];
    return sqa_set_rows_q4_0(&dst, v_cur, idx, stream);
}

}  // extern "C"
