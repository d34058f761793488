/*
 * ggml_cpu_ref.c - CPU oracle (test infrastructure; see ggml_cpu_ref.h).
 *
 * Built with -ffp-contract=off so that every multiply and add rounds on its
 * own, as ggml's scalar reference code does; where ggml's x86 kernels use a
 * fused multiply-add (ggml_vec_mad_f32) the code calls fmaf explicitly.
 */
#include "ggml_cpu_ref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- fp16 --- */

uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu)); /* NaN */
    if (ax >= 0x47800000u) return (uint16_t)(sign | 0x7c00u); /* >= 65536: inf */
    if (ax >= 0x38800000u) {                                  /* normal in fp16 */
        const uint32_t e = (ax >> 23) - 127 + 15;
        const uint32_t m = ax & 0x7fffffu;
        uint32_t r = (e << 10) | (m >> 13);
        const uint32_t rem = m & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r += 1; /* may carry into inf */
        return (uint16_t)(sign | r);
    }
    if (ax <= 0x33000000u) return (uint16_t)sign; /* <= 2^-25 rounds to zero (tie -> even 0) */
    /* fp16 subnormal: value / 2^-24 rounded to nearest even */
    const uint32_t E = ax >> 23;
    const uint32_t M = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t s = 126 - E; /* 14..24 */
    uint32_t r = M >> s;
    const uint32_t rem = M & ((1u << s) - 1u);
    const uint32_t half = 1u << (s - 1);
    if (rem > half || (rem == half && (r & 1u))) r += 1;
    return (uint16_t)(sign | r);
}

float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: normalise */
            float v = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ---------------------------------------------------------------- q4_0 --- */

/* ggml quantize_row_q4_0_ref: d = max / -8 where max is the signed value of
 * largest magnitude (first occurrence wins: strict `<`), id = 1/d, code =
 * min(15, (int8_t)(x*id + 8.5f)) with the product and the add rounded
 * separately; d is stored as fp16 but the codes use the fp32 d. */
void orc_quantize_row_q4_0(const float *x, uint8_t *y, int64_t k) {
    const int qk = SQA_QK4_0;
    const int64_t nb = k / qk;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        float max = 0.0f;
        for (int j = 0; j < qk; j++) {
            const float v = x[i * qk + j];
            if (amax < fabsf(v)) {
                amax = fabsf(v);
                max = v;
            }
        }
        const float d = max / -8;
        const float id = d ? 1.0f / d : 0.0f;
        uint8_t *blk = y + i * SQA_Q4_0_BLOCK_BYTES;
        const uint16_t dh = orc_fp32_to_fp16(d);
        memcpy(blk, &dh, 2);
        for (int j = 0; j < qk / 2; ++j) {
            const float x0 = x[i * qk + 0 + j] * id;
            const float x1 = x[i * qk + qk / 2 + j] * id;
            const int8_t t0 = (int8_t)(x0 + 8.5f);
            const int8_t t1 = (int8_t)(x1 + 8.5f);
            const uint8_t xi0 = (uint8_t)(t0 < 15 ? t0 : 15);
            const uint8_t xi1 = (uint8_t)(t1 < 15 ? t1 : 15);
            blk[2 + j] = (uint8_t)(xi0 | (xi1 << 4));
        }
    }
}

void orc_dequantize_row_q4_0(const uint8_t *x, float *y, int64_t k) {
    const int qk = SQA_QK4_0;
    const int64_t nb = k / qk;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *blk = x + i * SQA_Q4_0_BLOCK_BYTES;
        uint16_t dh;
        memcpy(&dh, blk, 2);
        const float d = orc_fp16_to_fp32(dh);
        for (int j = 0; j < qk / 2; ++j) {
            const int x0 = (blk[2 + j] & 0x0F) - 8;
            const int x1 = (blk[2 + j] >> 4) - 8;
            y[i * qk + j + 0] = x0 * d;
            y[i * qk + j + qk / 2] = x1 * d;
        }
    }
}

/* ---------------------------------------------------------------- q8_0 --- */

void orc_quantize_row_q8_0(const float *x, uint8_t *y, int64_t k, int variant) {
    const int qk = 32;
    const int64_t nb = k / qk;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < qk; j++) {
            const float a = fabsf(x[i * qk + j]);
            amax = amax > a ? amax : a;
        }
        uint8_t *blk = y + i * ORC_Q8_0_BLOCK_BYTES;
        int8_t *qs = (int8_t *)(blk + 2);
        const float d = amax / 127.f;
        const uint16_t dh = orc_fp32_to_fp16(d);
        memcpy(blk, &dh, 2);
        if (variant == ORC_Q8_X86) {
            const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
            for (int j = 0; j < qk; j++) qs[j] = (int8_t)nearbyintf(x[i * qk + j] * id);
        } else {
            const float id = d ? 1.0f / d : 0.0f;
            for (int j = 0; j < qk; j++) qs[j] = (int8_t)roundf(x[i * qk + j] * id);
        }
    }
}

/* q4_0 . q8_0: per block the exact integer sum of (nib-8)*q8, scaled by
 * d4 * d8 and accumulated in fp32 (ggml's scalar vec_dot order). */
float orc_vec_dot_q4_0_q8_0(int64_t n, const uint8_t *x, const uint8_t *y) {
    const int64_t nb = n / 32;
    float sumf = 0.0f;
    for (int64_t ib = 0; ib < nb; ++ib) {
        const uint8_t *bx = x + ib * SQA_Q4_0_BLOCK_BYTES;
        const uint8_t *by = y + ib * ORC_Q8_0_BLOCK_BYTES;
        const int8_t *qy = (const int8_t *)(by + 2);
        int sumi0 = 0, sumi1 = 0;
        for (int j = 0; j < 16; ++j) {
            const int v0 = (bx[2 + j] & 0x0F) - 8;
            const int v1 = (bx[2 + j] >> 4) - 8;
            sumi0 += v0 * qy[j];
            sumi1 += v1 * qy[j + 16];
        }
        const int sumi = sumi0 + sumi1;
        uint16_t dx, dy;
        memcpy(&dx, bx, 2);
        memcpy(&dy, by, 2);
        sumf += (float)sumi * orc_fp16_to_fp32(dx) * orc_fp16_to_fp32(dy);
    }
    return sumf;
}

/* ------------------------------------------------------------ set_rows --- */

int orc_set_rows_q4_0(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *idx) {
    if (!dst || !src || !idx) return SQA_ERR_INVALID;
    if (dst->type != SQA_TYPE_Q4_0 || src->type != SQA_TYPE_F32 || idx->type != SQA_TYPE_I64)
        return SQA_ERR_INVALID;
    const int64_t ne0 = src->ne[0];
    const int64_t n_rows = src->ne[1];
    if (dst->ne[0] != ne0 || ne0 % SQA_QK4_0 != 0 || idx->ne[0] != n_rows) return SQA_ERR_INVALID;
    for (int64_t i = 0; i < n_rows; ++i) {
        const int64_t r = *(const int64_t *)((const char *)idx->data + i * idx->nb[0]);
        if (r < 0 || r >= dst->ne[1]) continue; /* ggml asserts; the device kernel skips */
        orc_quantize_row_q4_0((const float *)((const char *)src->data + i * src->nb[1]),
                              (uint8_t *)dst->data + r * dst->nb[1], ne0);
    }
    return SQA_OK;
}

/* -------------------------------------------------------- flash attention --- */

/* One (query, head) row of ggml's CPU flash_attn_ext: Q row -> q8_0, then for
 * every key with a mask value other than -inf: s = scale * (q4_0 . q8_0) (+
 * softcap) + slope*mask; online softmax with expf; V dequantised to fp32 and
 * accumulated with a fused multiply-add; finally divided by the sum (0 if the
 * sum is 0, i.e. every key masked). causal_limit >= 0 replaces the mask with
 * "key <= causal_limit". */
static void fa_row(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                   const sqa_tensor *mask, int64_t causal_limit, float scale, float slope,
                   float logit_softcap, int64_t iq1, int64_t iq2, float *out, float *vkq,
                   float *v32, uint8_t *q_q, int q8_variant) {
    const int64_t DK = k->ne[0];
    const int64_t DV = v->ne[0];
    const int64_t n_kv = k->ne[1];
    const int64_t rk2 = q->ne[2] / k->ne[2];
    const int64_t rv2 = q->ne[2] / v->ne[2];
    const int64_t ik2 = iq2 / rk2;
    const int64_t iv2 = iq2 / rv2;

    const float *pq = (const float *)((const char *)q->data + iq1 * q->nb[1] + iq2 * q->nb[2]);
    orc_quantize_row_q8_0(pq, q_q, DK, q8_variant);
    const uint16_t *mp =
        mask ? (const uint16_t *)((const char *)mask->data + iq1 * mask->nb[1]) : NULL;

    float S = 0.0f;
    float M = -INFINITY;
    memset(vkq, 0, DV * sizeof(float));
    for (int64_t ic = 0; ic < n_kv; ++ic) {
        float mv;
        if (causal_limit >= 0) {
            mv = ic <= causal_limit ? 0.0f : -INFINITY;
        } else {
            mv = mp ? slope * orc_fp16_to_fp32(mp[ic]) : 0.0f;
        }
        if (mv == -INFINITY) continue;

        const uint8_t *kd = (const uint8_t *)k->data + ic * k->nb[1] + ik2 * k->nb[2];
        float s = orc_vec_dot_q4_0_q8_0(DK, kd, q_q);
        s = s * scale;
        if (logit_softcap != 0.0f) s = logit_softcap * tanhf(s);
        s += mv;

        const float Mold = M;
        float ms = 1.0f;
        float vs = 1.0f;
        if (s > M) {
            M = s;
            ms = expf(Mold - M);
            for (int64_t d = 0; d < DV; ++d) vkq[d] *= ms;
        } else {
            vs = expf(s - M);
        }
        const uint8_t *vd = (const uint8_t *)v->data + ic * v->nb[1] + iv2 * v->nb[2];
        orc_dequantize_row_q4_0(vd, v32, DV);
        for (int64_t d = 0; d < DV; ++d) vkq[d] = fmaf(v32[d], vs, vkq[d]);
        S = S * ms + vs;
    }
    const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
    for (int64_t d = 0; d < DV; ++d) out[d] = vkq[d] * S_inv;
}

static int fa_check(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                    const sqa_tensor *mask, const sqa_tensor *dst) {
    if (!q || !k || !v || !dst) return SQA_ERR_INVALID;
    if (q->type != SQA_TYPE_F32 || k->type != SQA_TYPE_Q4_0 || v->type != SQA_TYPE_Q4_0 ||
        dst->type != SQA_TYPE_F32)
        return SQA_ERR_INVALID;
    if (q->ne[0] != k->ne[0] || k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2]) return SQA_ERR_INVALID;
    if (q->ne[0] % SQA_QK4_0 || v->ne[0] % SQA_QK4_0) return SQA_ERR_INVALID;
    if (k->ne[2] <= 0 || q->ne[2] % k->ne[2]) return SQA_ERR_INVALID;
    if (dst->ne[0] != v->ne[0] || dst->ne[1] != q->ne[2] || dst->ne[2] != q->ne[1])
        return SQA_ERR_INVALID;
    if (q->ne[3] != 1 || k->ne[3] != 1) return SQA_ERR_UNSUPPORTED;
    if (mask) {
        if (mask->type != SQA_TYPE_F16 || mask->ne[0] != k->ne[1] || mask->ne[1] < q->ne[1])
            return SQA_ERR_INVALID;
    }
    return SQA_OK;
}

static int fa_run(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                  const sqa_tensor *mask, int64_t q_pos0, const sqa_tensor *gate, float scale,
                  float max_bias, float logit_softcap, const sqa_tensor *dst, int n_threads,
                  int q8_variant) {
    const int64_t n_q = q->ne[1];
    const int64_t H = q->ne[2];
    const int64_t DK = k->ne[0];
    const int64_t DV = v->ne[0];
    const int64_t n_rows = n_q * H;
    if (logit_softcap != 0.0f) scale /= logit_softcap;
    const uint32_t n_head_log2 = 1u << (uint32_t)floor(log2((double)H));
    const float m0 = powf(2.0f, -(max_bias) / n_head_log2);
    const float m1 = powf(2.0f, -(max_bias / 2.0f) / n_head_log2);
    if (n_threads < 1) n_threads = 1;

#pragma omp parallel num_threads(n_threads)
    {
        float *vkq = (float *)malloc(DV * sizeof(float));
        float *v32 = (float *)malloc(DV * sizeof(float));
        uint8_t *q_q = (uint8_t *)malloc((DK / 32) * ORC_Q8_0_BLOCK_BYTES);
#pragma omp for schedule(dynamic, 1)
        for (int64_t ir = 0; ir < n_rows; ++ir) {
            const int64_t iq2 = ir / n_q; /* head */
            const int64_t iq1 = ir % n_q; /* query */
            const uint32_t h = (uint32_t)iq2;
            const float slope = (max_bias > 0.0f)
                                    ? (h < n_head_log2 ? powf(m0, h + 1)
                                                       : powf(m1, 2 * (h - n_head_log2) + 1))
                                    : 1.0f;
            float *out = (float *)((char *)dst->data + (iq1 * H + iq2) * DV * sizeof(float));
            const int64_t climit = q_pos0 >= 0 ? q_pos0 + iq1 : -1;
            fa_row(q, k, v, mask, climit, scale, slope, logit_softcap, iq1, iq2, out, vkq, v32,
                   q_q, q8_variant);
            if (gate) {
                const float *g =
                    (const float *)((const char *)gate->data + iq1 * gate->nb[2] + iq2 * gate->nb[1]);
                for (int64_t d = 0; d < DV; ++d) out[d] = out[d] * (1.f / (1.f + expf(-g[d])));
            }
        }
        free(vkq);
        free(v32);
        free(q_q);
    }
    return SQA_OK;
}

int orc_flash_attn_ext(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                       const sqa_tensor *mask, float scale, float max_bias, float logit_softcap,
                       const sqa_tensor *dst, int n_threads, int q8_variant) {
    const int rc = fa_check(q, k, v, mask, dst);
    if (rc) return rc;
    return fa_run(q, k, v, mask, -1, NULL, scale, max_bias, logit_softcap, dst, n_threads,
                  q8_variant);
}

int orc_flash_attn_ext_causal(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                              int64_t q_pos0, const sqa_tensor *gate, float scale,
                              const sqa_tensor *dst, int n_threads, int q8_variant) {
    const int rc = fa_check(q, k, v, NULL, dst);
    if (rc) return rc;
    if (q_pos0 < 0) return SQA_ERR_RANGE;
    return fa_run(q, k, v, NULL, q_pos0, gate, scale, 0.0f, 0.0f, dst, n_threads, q8_variant);
}

/* ggml_vec_sigmoid_f32 (1/(1+expf(-x))) followed by ggml_mul. */
int orc_sigmoid_mul(const sqa_tensor *dst, const sqa_tensor *x, const sqa_tensor *gate) {
    if (!dst || !x || !gate) return SQA_ERR_INVALID;
    const int64_t n0 = x->ne[0], n1 = x->ne[1];
    for (int64_t j = 0; j < n1; ++j) {
        const float *xr = (const float *)((const char *)x->data + j * x->nb[1]);
        const float *gr = (const float *)((const char *)gate->data + j * gate->nb[1]);
        float *dr = (float *)((char *)dst->data + j * dst->nb[1]);
        for (int64_t i = 0; i < n0; ++i) dr[i] = xr[i] * (1.f / (1.f + expf(-gr[i])));
    }
    return SQA_OK;
}

/* -------------------------------------------- K/Q producer: norm + rope --- */

/* ggml_rms_norm (CPU): the squares summed in double, mean and scale in float,
 * y = x * scale; then ggml_mul by the [n] weight when w is given. The reference
 * test restates it at tests/attn_test.rs:278-283 (float sum, division by the
 * root); ggml's own order is followed here. */
void orc_rms_norm_mul_row(const float *x, const float *w, float eps, int64_t n, float *y) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; ++i) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < n; ++i) {
        y[i] = x[i] * scale;
        if (w) y[i] = y[i] * w[i];
    }
}

/* IMROPE cos/sin of the n_rot/2 rotation pairs of one token: ggml's
 * mrope cache with the interleaved sector rule, restated at
 * tests/attn_test.rs:153-193 (rope_ref). The four angles start at the token's
 * positions and are multiplied by theta_scale = freq_base^(-2/n_rot) once per
 * pair, in float, as ggml does; pair ic takes the angle of its sector:
 * h when ic%S%3 == 1 and ic%S < 3*s1, w when 2 and < 3*s2, t when 0 and < 3*s0,
 * else e (S = s0+s1+s2+s3). With ext_factor 0 (rope_yarn without ramp):
 * cos = cosf(freq_scale*theta)*attn_factor, sin likewise. */
void orc_imrope_cache(int32_t n_rot, const int32_t sections[4], float theta_scale, float freq_scale,
                      float attn_factor, const int32_t p[4], float *cache) {
    const int32_t sect = sections[0] + sections[1] + sections[2] + sections[3];
    float th_t = (float)p[0], th_h = (float)p[1], th_w = (float)p[2], th_e = (float)p[3];
    for (int32_t i0 = 0; i0 < n_rot; i0 += 2) {
        const int32_t sector = (i0 / 2) % sect;
        float theta;
        if (sector % 3 == 1 && sector < 3 * sections[1]) theta = th_h;
        else if (sector % 3 == 2 && sector < 3 * sections[2]) theta = th_w;
        else if (sector % 3 == 0 && sector < 3 * sections[0]) theta = th_t;
        else theta = th_e;
        const float th = freq_scale * theta;
        cache[i0] = cosf(th) * attn_factor;
        cache[i0 + 1] = sinf(th) * attn_factor;
        th_t *= theta_scale;
        th_h *= theta_scale;
        th_w *= theta_scale;
        th_e *= theta_scale;
    }
}

/* Rotation of one head row: pairs (ic, ic + n_rot/2) for ic < n_rot/2 (the
 * NEOX-style pairing of mrope), dims >= n_rot copied (attn_test.rs:195-205). */
void orc_rope_row(const float *x, int64_t n, int32_t n_rot, const float *cache, float *y) {
    const int32_t half = n_rot / 2;
    for (int64_t i = n_rot; i < n; ++i) y[i] = x[i];
    for (int32_t ic = 0; ic < half; ++ic) {
        const float ct = cache[2 * ic], st = cache[2 * ic + 1];
        const float x0 = x[ic], x1 = x[ic + half];
        y[ic] = x0 * ct - x1 * st;
        y[ic + half] = x0 * st + x1 * ct;
    }
}

static int producer_check(const sqa_tensor *src, const sqa_tensor *norm_w, const sqa_tensor *pos,
                          const sqa_rope *rope) {
    if (!src || !pos || !rope || src->type != SQA_TYPE_F32 || pos->type != SQA_TYPE_I32) return SQA_ERR_INVALID;
    if (norm_w && (norm_w->type != SQA_TYPE_F32 || norm_w->ne[0] != src->ne[0])) return SQA_ERR_INVALID;
    if (pos->ne[0] != 4 * src->ne[2] || rope->n_rot <= 0 || rope->n_rot % 2 || rope->n_rot > src->ne[0])
        return SQA_ERR_INVALID;
    if (rope->sections[0] + rope->sections[1] + rope->sections[2] + rope->sections[3] <= 0) return SQA_ERR_INVALID;
    if (rope->ext_factor != 0.0f) return SQA_ERR_UNSUPPORTED;
    return SQA_OK;
}

/* One token-head row through norm and rope into y (n floats). */
static void producer_row(const sqa_tensor *src, const sqa_tensor *norm_w, float eps, const sqa_tensor *pos,
                         const sqa_rope *rope, float theta_scale, int64_t t, int64_t h, float *y) {
    const int64_t n = src->ne[0], n_tok = src->ne[2];
    const float *x = (const float *)((const char *)src->data + h * src->nb[1] + t * src->nb[2]);
    float *tmp = (float *)malloc((size_t)n * sizeof(float));
    float *cache = (float *)malloc((size_t)rope->n_rot * sizeof(float));
    if (norm_w) orc_rms_norm_mul_row(x, (const float *)norm_w->data, eps, n, tmp);
    else memcpy(tmp, x, (size_t)n * sizeof(float));
    const int32_t *pp = (const int32_t *)pos->data;
    const int32_t p[4] = {pp[t], pp[t + n_tok], pp[t + 2 * n_tok], pp[t + 3 * n_tok]};
    orc_imrope_cache(rope->n_rot, rope->sections, theta_scale, rope->freq_scale, rope->attn_factor, p, cache);
    orc_rope_row(tmp, n, rope->n_rot, cache, y);
    free(cache);
    free(tmp);
}

float orc_rope_theta_scale(const sqa_rope *rope) { return powf(rope->freq_base, -2.0f / (float)rope->n_rot); }

int orc_rope_norm_set_rows_q4_0(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *norm_w,
                                float eps, const sqa_tensor *pos, const sqa_rope *rope, const sqa_tensor *idx) {
    const int st = producer_check(src, norm_w, pos, rope);
    if (st != SQA_OK) return st;
    if (!dst || !idx || dst->type != SQA_TYPE_Q4_0 || idx->type != SQA_TYPE_I64) return SQA_ERR_INVALID;
    const int64_t n = src->ne[0], n_head = src->ne[1], n_tok = src->ne[2];
    if (n % SQA_QK4_0 || dst->ne[0] != n * n_head || idx->ne[0] != n_tok) return SQA_ERR_INVALID;
    const float ts = orc_rope_theta_scale(rope);
    float *y = (float *)malloc((size_t)n * sizeof(float));
    for (int64_t t = 0; t < n_tok; ++t) {
        const int64_t r = *(const int64_t *)((const char *)idx->data + t * idx->nb[0]);
        if (r < 0 || r >= dst->ne[1]) continue;
        for (int64_t h = 0; h < n_head; ++h) {
            producer_row(src, norm_w, eps, pos, rope, ts, t, h, y);
            orc_quantize_row_q4_0(y, (uint8_t *)dst->data + r * dst->nb[1] + h * (n / SQA_QK4_0) * SQA_Q4_0_BLOCK_BYTES,
                                  n);
        }
    }
    free(y);
    return SQA_OK;
}

int orc_rope_norm_f32(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *norm_w, float eps,
                      const sqa_tensor *pos, const sqa_rope *rope) {
    const int st = producer_check(src, norm_w, pos, rope);
    if (st != SQA_OK) return st;
    if (!dst || dst->type != SQA_TYPE_F32) return SQA_ERR_INVALID;
    const int64_t n = src->ne[0], n_head = src->ne[1], n_tok = src->ne[2];
    const float ts = orc_rope_theta_scale(rope);
    for (int64_t t = 0; t < n_tok; ++t)
        for (int64_t h = 0; h < n_head; ++h)
            producer_row(src, norm_w, eps, pos, rope, ts, t, h, (float *)dst->data + (t * n_head + h) * n);
    return SQA_OK;
}

/* -------------------------------------------- W_o projection: Q4_K x F32 --- */

/* Q4_K super-block (ggml block_q4_K, 256 values, 144 bytes):
 *   bytes 0-1   d     fp16, scale of the sub-block scales
 *   bytes 2-3   dmin  fp16, scale of the sub-block mins
 *   bytes 4-15  12 bytes of 6-bit (scale, min) pairs for the 8 sub-blocks of 32:
 *               sub-block s < 4: scale = b[s] & 63,           min = b[s+4] & 63
 *               sub-block s >= 4: scale = (b[s+4] & 15) | (b[s-4] >> 6) << 4,
 *                                 min   = (b[s+4] >> 4) | (b[s]   >> 6) << 4
 *   bytes 16-143 codes: byte l of 32-byte group j holds value 64j + l in its
 *               low nibble and value 64j + 32 + l in its high nibble
 * value = (d * scale) * code - (dmin * min), each product in fp32 (both exact:
 * 11 + 6 significant bits), one rounding at the subtraction. */
static void q4k_scale_min(const uint8_t *b, int s, int *sc, int *mn) {
    if (s < 4) {
        *sc = b[s] & 63;
        *mn = b[s + 4] & 63;
    } else {
        *sc = (b[s + 4] & 15) | ((b[s - 4] >> 6) << 4);
        *mn = (b[s + 4] >> 4) | ((b[s] >> 6) << 4);
    }
}

void orc_dequantize_row_q4_K(const uint8_t *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / 256; ++i) {
        const uint8_t *blk = x + 144 * i;
        const float d = orc_fp16_to_fp32((uint16_t)(blk[0] | (blk[1] << 8)));
        const float dmin = orc_fp16_to_fp32((uint16_t)(blk[2] | (blk[3] << 8)));
        const uint8_t *sc = blk + 4, *qs = blk + 16;
        for (int j = 0; j < 4; ++j) {
            int s0, m0, s1, m1;
            q4k_scale_min(sc, 2 * j, &s0, &m0);
            q4k_scale_min(sc, 2 * j + 1, &s1, &m1);
            const float dl = d * (float)s0, ml = dmin * (float)m0;
            const float dh = d * (float)s1, mh = dmin * (float)m1;
            float *yo = y + 256 * i + 64 * j;
            for (int l = 0; l < 32; ++l) {
                yo[l] = dl * (float)(qs[32 * j + l] & 15) - ml;
                yo[32 + l] = dh * (float)(qs[32 * j + l] >> 4) - mh;
            }
        }
    }
}

/* dst[N, M] = W[K, N]^T . xg[K, M] (ggml_mul_mat(W, xg) with ne = [K, N] and
 * [K, M]), xg = x * sigmoid(gate) in fp32 as ggml_sigmoid + ggml_mul compute it
 * (or x when gate is NULL). The weights are dequantized to fp32 as above and
 * every row dot is accumulated in double: the exact product of what ggml's
 * CPU path would multiply before it rounds the activations to 8 bits. */
int orc_out_proj(const sqa_tensor *dst, const sqa_tensor *w, const sqa_tensor *x, const sqa_tensor *gate) {
    if (!dst || !w || !x) return SQA_ERR_INVALID;
    const int64_t K = w->ne[0], N = w->ne[1], M = x->ne[1];
    if (w->type != SQA_TYPE_Q4_K || K % 256 || x->ne[0] != K || dst->ne[0] != N || dst->ne[1] != M)
        return SQA_ERR_INVALID;
    float *xg = (float *)malloc((size_t)(K * M) * sizeof(float));
    float *wd = (float *)malloc((size_t)(K * N) * sizeof(float));
    if (!xg || !wd) {
        free(xg);
        free(wd);
        return SQA_ERR_INVALID;
    }
    for (int64_t t = 0; t < M; ++t) {
        const float *xr = (const float *)((const char *)x->data + t * x->nb[1]);
        const float *gr = gate ? (const float *)((const char *)gate->data + t * gate->nb[1]) : NULL;
        for (int64_t k = 0; k < K; ++k) xg[t * K + k] = gr ? xr[k] * (1.f / (1.f + expf(-gr[k]))) : xr[k];
    }
    for (int64_t n = 0; n < N; ++n)
        orc_dequantize_row_q4_K((const uint8_t *)w->data + n * w->nb[1], wd + n * K, K);
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t t = 0; t < M; ++t) {
            double acc = 0.0;
            for (int64_t k = 0; k < K; ++k) acc += (double)wd[n * K + k] * (double)xg[t * K + k];
            ((float *)((char *)dst->data + t * dst->nb[1]))[n] = (float)acc;
        }
    }
    free(xg);
    free(wd);
    return SQA_OK;
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
