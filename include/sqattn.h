/*
 * sqattn.h - C ABI of the MI355X (gfx950) full-attention hot path:
 *   q4_0 quantize-on-write (set_rows), FlashAttention over a q4_0 K/V cache
 *   (split-KV decode/verify and MFMA prefill), and the sigmoid output gate.
 *
 * Every entry point takes plain pointers and sizes. Tensors are described with
 * sqa_tensor, which carries the same {type, ne[4], nb[4], data} fields as
 * ggml's tensor struct (reference: src/backend/ffi.rs:22-39), so a caller that
 * already holds ggml tensors fills one by copying four fields. Views may be
 * non-contiguous (permuted q, strided K/V cache views) exactly as ggml allows.
 *
 * Status convention (reference: src/backend/ctx.rs:689-697): 0 means success.
 * Where ggml aborts on an unsupported op (src/engine/runner.rs:509-513) these
 * functions return SQA_ERR_UNSUPPORTED instead; sqa_last_error() returns a
 * thread-local message describing the most recent failure.
 *
 * Ownership (reference: src/backend/ctx.rs:455-650): the caller owns every
 * buffer. No entry point allocates device memory; split-KV scratch comes in
 * through (workspace, workspace_bytes), sized by *_workspace_size().
 * Streams are passed as `void *` (a hipStream_t; NULL = default stream).
 * All launches are asynchronous on that stream.
 */
#ifndef SQATTN_H
#define SQATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Type codes are ggml's enum ggml_type values (reference: src/backend/ffi.rs:48-64). */
#define SQA_TYPE_F32 0
#define SQA_TYPE_F16 1
#define SQA_TYPE_Q4_0 2
#define SQA_TYPE_Q4_K 12
#define SQA_TYPE_I32 26
#define SQA_TYPE_I64 27

/* q4_0 block: fp16 scale d + 16 bytes of nibbles, 32 values, 18 bytes
 * (reference: src/engine/kv.rs:33, :181-182; tests/kernel_verify.rs:270-292). */
#define SQA_QK4_0 32
#define SQA_Q4_0_BLOCK_BYTES 18

/* KV length granularity the cache is padded to (reference: src/engine/kv.rs:35-37). */
#define SQA_KV_PAD 256

enum sqa_status {
    SQA_OK = 0,
    SQA_ERR_INVALID = 1,     /* null pointer, shape/stride/type mismatch */
    SQA_ERR_UNSUPPORTED = 2, /* valid ggml op, but not a configuration this library runs */
    SQA_ERR_WORKSPACE = 3,   /* workspace missing or smaller than *_workspace_size() */
    SQA_ERR_HIP = 4,         /* a HIP runtime call failed (launch error, bad device) */
    SQA_ERR_OVERFLOW = 5,    /* KV cache cursor would pass its capacity */
    SQA_ERR_RANGE = 6        /* a position/index argument is out of range */
};

typedef struct sqa_tensor {
    int32_t type;   /* SQA_TYPE_* */
    int32_t pad_;   /* keeps ne[] 8-byte aligned; ignored */
    int64_t ne[4];  /* elements per dimension, ne[0] fastest */
    uint64_t nb[4]; /* byte strides; nb[0] is the element (or q4_0 block) size */
    void *data;     /* device pointer */
} sqa_tensor;

/* Library version and the last error message of the calling thread. */
const char *sqa_version(void);
const char *sqa_last_error(void);
const char *sqa_status_string(int status);

/* ------------------------------------------------------------------------ */
/* set_rows: quantize-on-write into a q4_0 cache.                            */
/* ------------------------------------------------------------------------ */

/*
 * dst[idx[i], :] = quantize_row_q4_0(src[i, :]) for i in [0, src->ne[1]).
 * Replaces GGML_OP_SET_ROWS with a q4_0 destination as issued by
 * KvCache::append (reference: src/engine/kv.rs:313-399, the ggml_set_rows
 * declaration at src/backend/ffi.rs:394-405).
 *   src: F32 [ne0, n_rows] (row stride src->nb[1], elements contiguous)
 *   idx: I64 [n_rows] (element stride idx->nb[0])
 *   dst: Q4_0 [ne0, dst_rows] (row stride dst->nb[1]); ne0 % 32 == 0
 * Bit-exact with ggml's quantize_row_q4_0 (scalar reference semantics).
 * Rows whose index lies outside [0, dst->ne[1]) are not written; where ggml's
 * CPU backend asserts, the kernel skips them, since a device-side index cannot
 * be checked on the host without a copy.
 */
int sqa_set_rows_q4_0(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *idx,
                      void *stream);

/* Support query for set_rows, mirroring ggml_backend_supports_op
 * (reference: src/backend/ffi.rs:361-362). Returns 1 if supported. */
int sqa_supports_set_rows(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *idx);

/* ------------------------------------------------------------------------ */
/* K/Q producer: per-head RMSNorm, IMROPE, q4_0 quantize-on-write            */
/* ------------------------------------------------------------------------ */

/*
 * Rotary parameters of ggml_rope_multi (reference: declaration at
 * src/backend/ffi.rs:417-432; values from RopeParams, src/model/attn.rs:30-65).
 * Only the text-mode settings the engine uses are supported: ext_factor must be
 * 0 (no YaRN ramp, so n_ctx_orig, beta_fast and beta_slow play no part).
 */
typedef struct sqa_rope {
    int32_t n_rot;       /* rotated leading dims of each head row; n_rot % 8 == 0, <= D */
    int32_t sections[4]; /* IMROPE sections (t, h, w, e), sum > 0 (the engine: n_rot / 2) */
    float freq_base;
    float freq_scale;
    float ext_factor; /* must be 0 */
    float attn_factor;
} sqa_rope;

/*
 * The K producer chain of one full-attention layer in one kernel:
 *   y = rms_norm(x, eps) * norm_w          (ggml_rms_norm + ggml_mul per head row,
 *                                           reference: head_rms_norm, src/model/attn.rs:68-84)
 *   y = rope_multi(y, pos, IMROPE, rope)   (src/model/attn.rs:180-200)
 *   dst[idx[t], head h] = quantize_row_q4_0(y)   (set_rows of KvCache::append,
 *                                           src/engine/kv.rs:313-399)
 *   src    F32  [D, n_head, n_tok] (element stride 4, head stride nb[1], token stride nb[2])
 *   norm_w F32  [D] contiguous, or NULL for no normalisation (then eps is unused)
 *   pos    I32  [4 * n_tok] contiguous: t, h, w, e positions (ggml's rope_multi layout)
 *   idx    I64  [n_tok] destination rows
 *   dst    Q4_0 [D * n_head, dst_rows] (row stride nb[1]); token t's head h lands at
 *          blocks h*D/32 .. (h+1)*D/32 - 1 of row idx[t]
 * D is 64, 128 or 256. Rows whose index lies outside [0, dst_rows) are skipped,
 * as in sqa_set_rows_q4_0.
 */
int sqa_rope_norm_set_rows_q4_0(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *norm_w,
                                float eps, const sqa_tensor *pos, const sqa_rope *rope,
                                const sqa_tensor *idx, void *stream);

/* The same normalisation and rotation with an F32 result, the Q side of the
 * layer (src/model/attn.rs:166-199): dst F32 [D, n_head, n_tok] contiguous. */
int sqa_rope_norm_f32(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *norm_w, float eps,
                      const sqa_tensor *pos, const sqa_rope *rope, void *stream);

/* Support query for both producer forms (idx != NULL: the q4_0 one, else the
 * F32 one), mirroring ggml_backend_supports_op (reference: src/backend/ffi.rs:
 * 361-362). Returns 1 if the call with these operands would run. */
int sqa_supports_rope_norm(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *norm_w,
                           const sqa_tensor *pos, const sqa_rope *rope, const sqa_tensor *idx);

/* ------------------------------------------------------------------------ */
/* flash_attn_ext                                                            */
/* ------------------------------------------------------------------------ */

/*
 * GGML_OP_FLASH_ATTN_EXT (reference: ggml_flash_attn_ext declaration at
 * src/backend/ffi.rs:363-377, called from src/model/attn.rs:238-249):
 *   q    F32  [D, n_q, H, 1]     any strides (the engine passes a permuted view)
 *   k    Q4_0 [D, n_kv, Hkv, 1]  row stride nb[1], head stride nb[2]
 *   v    Q4_0 [D, n_kv, Hkv, 1]
 *   mask F16  [n_kv, >=n_q, 1, 1] or NULL; -inf entries exclude a key
 *   dst  F32  [D, H, n_q, 1]     contiguous
 *   out[d,h,t] = sum_k softmax_k(scale * q8_0(Q[h,t]) . K[h/g,k] + mask[k,t]) * V[h/g,k,d]
 * with g = H/Hkv (block GQA map h -> h/g). Q is rounded to q8_0 per 32-value
 * block before the K dot, as ggml's CPU backend does for a q4_0 K.
 * Supported: D == 256, H % Hkv == 0, q4_0 K and V, max_bias == 0,
 * logit_softcap == 0. Decode/verify (n_q * H/Hkv <= 16) uses the split-KV
 * kernel; larger n_q uses the MFMA prefill kernel.
 * Inputs: a key that -inf excludes from every row of the call contributes 0
 * whatever its bytes hold (stale or unwritten cache rows may be anything);
 * V block scales of any finite size. A row with no visible key returns 0.
 */
int sqa_flash_attn_ext(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                       const sqa_tensor *mask, float scale, float max_bias, float logit_softcap,
                       const sqa_tensor *dst, void *workspace, size_t workspace_bytes,
                       void *stream);

/* Workspace bytes sqa_flash_attn_ext / sqa_flash_attn_ext_causal need for
 * these shapes (0 is a valid answer). */
size_t sqa_flash_attn_ext_workspace_size(const sqa_tensor *q, const sqa_tensor *k,
                                         const sqa_tensor *v, const sqa_tensor *dst);

/* Support query mirroring probe_flash_attn (reference: src/engine/runner.rs:509-559).
 * Returns 1 if sqa_flash_attn_ext would run these shapes and parameters. */
int sqa_supports_flash_attn_ext(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                                const sqa_tensor *mask, float scale, float max_bias,
                                float logit_softcap, const sqa_tensor *dst);

/*
 * Allocation-free form of sqa_flash_attn_ext for decode/verify shapes (up to 4
 * positions and 16 query rows per KV head, any number of KV heads, 16-byte
 * aligned q rows).
 * It has no counterpart in the reference: it is for callers that cannot
 * allocate or pass a workspace (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Its scratch is a device array of
 * SQA_STATIC_SCRATCH_BYTES inside the library, one per GPU, held until the
 * process ends; no call allocates or frees memory. Every call on one GPU
 * shares that GPU's array, so calls that overlap on one GPU (two streams, two
 * threads) race. Shapes whose scratch exceeds the maximum return
 * SQA_ERR_WORKSPACE, other shapes SQA_ERR_UNSUPPORTED. Same arguments, result
 * and errors as sqa_flash_attn_ext otherwise.
 */
#define SQA_STATIC_SCRATCH_BYTES (16u << 20)
int sqa_flash_attn_ext_static(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                              const sqa_tensor *mask, float scale, float max_bias, float logit_softcap,
                              const sqa_tensor *dst, void *stream);

/*
 * Mask-free causal variant with an optional fused output gate. Query t sits at
 * absolute position q_pos0 + t and sees keys 0..q_pos0+t, the rule the engine
 * encodes in its host-built F16 mask (reference: src/model/graph.rs:486-576,
 * mask row q allows keys < step_start + q + 1). Keys at or past n_kv are never
 * read. If gate is non-NULL (F32, same [D, H, n_q] layout as dst, any row
 * stride nb[2]) the result is multiplied by sigmoid(gate), which fuses the
 * ggml_sigmoid + ggml_mul pair of src/model/attn.rs:282-283.
 */
int sqa_flash_attn_ext_causal(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                              int64_t q_pos0, const sqa_tensor *gate, float scale,
                              const sqa_tensor *dst, void *workspace, size_t workspace_bytes,
                              void *stream);

/* ------------------------------------------------------------------------ */
/* Output gate and causal mask                                               */
/* ------------------------------------------------------------------------ */

/* dst = x * sigmoid(gate), elementwise over F32 [n, n_tok] tensors with
 * contiguous rows: the unfused gate of src/model/attn.rs:282-283. dst may alias x. */
int sqa_sigmoid_mul(const sqa_tensor *dst, const sqa_tensor *x, const sqa_tensor *gate,
                    void *stream);

/* Fill an F16 mask [n_kv, n_q] on the device: row t allows keys <= step_start + t
 * (0x0000) and masks the rest (0xFC00 = -inf); same contents as
 * fill_mask_rows (reference: src/model/graph.rs:534-576) without the host pass. */
int sqa_fill_causal_mask(const sqa_tensor *mask, int64_t step_start, void *stream);

/* ------------------------------------------------------------------------ */
/* W_o output projection                                                     */
/* ------------------------------------------------------------------------ */

/*
 * dst = W . (x * sigmoid(gate)): the gate and W_o projection that end the
 * full-attention layer (reference: ggml_sigmoid, ggml_mul and
 * ggml_mul_mat(attn_output, gated) at src/model/attn.rs:281-285; attn_output
 * declared at src/model/weights.rs:438).
 *   w    Q4_K [K, N]  ggml's block_q4_K rows (K % 256 == 0, N % 16 == 0,
 *                     16-byte aligned rows), K = n_head * head_dim, N = n_embd
 *   x    F32  [K, M]  the attention output of M tokens (unit element stride)
 *   gate F32  [K, M]  or NULL (then dst = W . x)
 *   dst  F32  [N, M]  16-byte aligned rows
 * The weights enter as exact codes and (scale, min) pairs; products
 * accumulate in fp32. The gated activations xg = x * sigmoid(gate):
 *   up to 4 tokens: fp32 throughout, any finite size;
 *   more tokens: an fp16 hi + lo pair. Each value is carried to about 22 bits
 *     where |xg| >= 2^-3 and to an absolute 2^-25 below that (the fp16
 *     subnormal spacing of the lo part), so activations of RMS >= 1e-2 keep
 *     the result within 1e-4 of its RMS; |xg| < 65504, and above 64 tokens
 *     every 32-value sum of xg (a Q4_K sub-block) must also stay below 65504.
 * ggml's CPU path instead rounds the activations to 8 bits (its q8_K vec_dot
 * type): this result is the closer of the two to the exact W . x.
 */
size_t sqa_out_proj_workspace_size(const sqa_tensor *w, const sqa_tensor *x);
int sqa_supports_out_proj(const sqa_tensor *w, const sqa_tensor *x, const sqa_tensor *gate,
                          const sqa_tensor *dst);
int sqa_out_proj(const sqa_tensor *w, const sqa_tensor *x, const sqa_tensor *gate, const sqa_tensor *dst,
                 void *workspace, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------------------ */
/* KV cache bookkeeping (host only: no device calls)                         */
/* ------------------------------------------------------------------------ */

/*
 * Host-side mirror of KvCache (reference: src/engine/kv.rs:67-448): per layer
 * a q4_0 K cache [Hkv*D, cap_alloc] and a q4_0 V cache [D, Hkv, cap_alloc] in
 * caller-owned device buffers, cap_alloc = ceil(cap / 256) * 256, one write
 * cursor shared by all layers.
 */
typedef struct sqa_kv_cache sqa_kv_cache;

/* Bytes one layer's K (or V) buffer needs: cap_alloc * Hkv * D / 32 * 18. */
size_t sqa_kv_cache_layer_bytes(int64_t head_dim, int64_t n_head_kv, int64_t kv_cap);

/* k_bufs/v_bufs: n_layers device pointers each of sqa_kv_cache_layer_bytes().
 * Returns NULL (and sets sqa_last_error) on invalid arguments. */
sqa_kv_cache *sqa_kv_cache_create(int32_t n_layers, int64_t head_dim, int64_t n_head_kv,
                                  int64_t kv_cap, void *const *k_bufs, void *const *v_bufs);
void sqa_kv_cache_destroy(sqa_kv_cache *kv);

int64_t sqa_kv_cache_n_used(const sqa_kv_cache *kv);
int64_t sqa_kv_cache_step_start(const sqa_kv_cache *kv);
/* ceil(n_used / 256) * 256 (reference: src/engine/kv.rs:224-226). */
int64_t sqa_kv_cache_n_kv_padded(const sqa_kv_cache *kv);
int64_t sqa_kv_cache_n_kv_padded_after(const sqa_kv_cache *kv, int64_t n_tokens);
/* Reserve [n_used, n_used + n_tokens); SQA_ERR_OVERFLOW past kv_cap (kv.rs:239-253). */
int sqa_kv_cache_begin_step(sqa_kv_cache *kv, int64_t n_tokens);
/* Move the cursor back to pos without touching data (kv.rs:280-297). */
int sqa_kv_cache_rewind_to(sqa_kv_cache *kv, int64_t pos);
void sqa_kv_cache_reset(sqa_kv_cache *kv);
/* Views over [0, n_kv_padded) of layer `slot` in flash_attn_ext order
 * [D, n_kv_padded, Hkv, 1] (the permuted k_view/v_view of kv.rs:401-447). */
int sqa_kv_cache_k_view(const sqa_kv_cache *kv, int32_t slot, sqa_tensor *out);
int sqa_kv_cache_v_view(const sqa_kv_cache *kv, int32_t slot, sqa_tensor *out);
/* Quantize n_tokens new K and V rows (F32 [Hkv*D, n_tokens], contiguous per token)
 * into layer `slot` at rows idx[0..n_tokens) (kv.rs:313-399). */
int sqa_kv_cache_append(sqa_kv_cache *kv, int32_t slot, const sqa_tensor *k_cur,
                        const sqa_tensor *v_cur, const sqa_tensor *idx, void *stream);


/* ------------------------------------------------------------------------ */
/* Per-kernel device timing (profiling aid)                                  */
/* ------------------------------------------------------------------------ */

/* Start bracketing kernel launches with HIP events (up to max_records
 * launches); the device-side counterpart of the engine's SQWEN_PROFILE host
 * timers (reference: src/engine/runner.rs:1602-1705). */
int sqa_profile_begin(int32_t max_records);
int sqa_profile_end(void);
/* Synchronise and sum the recorded durations of one kernel: "fa_decode",
 * "fa_combine", "fa_prefill", "set_rows_q4_0", "sigmoid_mul". */
int sqa_profile_get(const char *kernel, double *total_ms, int64_t *count);

#ifdef __cplusplus
}
#endif

#endif /* SQATTN_H */
