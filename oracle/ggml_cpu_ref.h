/*
 * ggml_cpu_ref.h - CPU oracle for the full-attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is the reference the HIP kernels are compared
 * against: only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
 * leg may load it. The product library never links or calls it.
 *
 * It restates, from the published algorithm, ggml's CPU-backend semantics for
 * the ops the engine issues on this path. ggml itself is an external
 * dependency of the reference (llama.cpp commit ed7ac35e1, named at
 * src/backend/ffi.rs:1 of the reference), not vendored and not present here.
 * Functions and the reference call sites they follow:
 *   orc_fp32_to_fp16 / orc_fp16_to_fp32  - IEEE binary16, round-to-nearest-even
 *                                          (f16_to_f32 of tests/kernel_verify.rs:253-268)
 *   orc_quantize_row_q4_0                - ggml quantize_row_q4_0_ref (the quantizer the
 *                                          tests call through ggml_quantize_chunk,
 *                                          tests/attn_test.rs:210-229; rules at :781-788)
 *   orc_dequantize_row_q4_0              - tests/kernel_verify.rs:270-292, attn_test.rs:257-276
 *   orc_quantize_row_q8_0                - ggml's q8_0 from_float, the vec_dot type of q4_0
 *   orc_vec_dot_q4_0_q8_0                - ggml's q4_0 x q8_0 block dot
 *   orc_set_rows_q4_0                    - GGML_OP_SET_ROWS CPU loop (src/engine/kv.rs:313-399)
 *   orc_flash_attn_ext                   - ggml CPU flash_attn_ext one-chunk online softmax,
 *                                          the op built at src/model/attn.rs:228-251
 *   orc_flash_attn_ext_causal            - the same with the causal rule of
 *                                          src/model/graph.rs:486-576 and the gate of
 *                                          src/model/attn.rs:282-283
 *   orc_sigmoid_mul                      - ggml_sigmoid + ggml_mul (src/model/attn.rs:282-283)
 *   orc_rms_norm_mul_row                 - ggml_rms_norm + ggml_mul of head_rms_norm
 *                                          (src/model/attn.rs:68-84; test restatement
 *                                          tests/attn_test.rs:278-283)
 *   orc_imrope_cache / orc_rope_row      - ggml_rope_multi with GGML_ROPE_TYPE_IMROPE
 *                                          (src/model/attn.rs:180-200; test restatement
 *                                          rope_ref, tests/attn_test.rs:148-208)
 *   orc_rope_norm_set_rows_q4_0          - norm -> rope -> set_rows for K, and
 *   orc_rope_norm_f32                      norm -> rope for Q (src/model/attn.rs:166-200)
 *   orc_dequantize_row_q4_K              - ggml dequantize_row_q4_K: the Q4_K weight format
 *                                          (the model's main quant type, tests/kernel_verify.rs:
 *                                          553-557) of attn_output.weight (src/model/weights.rs:438)
 *   orc_out_proj                         - ggml_mul_mat(attn_output, attn_out * sigmoid(gate)),
 *                                          the W_o projection of src/model/attn.rs:281-285, as
 *                                          an fp64 GEMM over the fp32 dequantized weights
 */
#ifndef GGML_CPU_REF_H
#define GGML_CPU_REF_H

#include <stdint.h>
#include "../include/sqattn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_Q8_0_BLOCK_BYTES 34

/* Q -> q8_0 rounding variants: ggml's x86 (AVX2) from_float uses id = 127/amax
 * and round-to-nearest-even; its portable scalar reference uses id = 1/d and
 * roundf (ties away from zero). */
#define ORC_Q8_X86 0
#define ORC_Q8_SCALAR 1

uint16_t orc_fp32_to_fp16(float f);
float orc_fp16_to_fp32(uint16_t h);

void orc_quantize_row_q4_0(const float *x, uint8_t *y, int64_t k);
void orc_dequantize_row_q4_0(const uint8_t *x, float *y, int64_t k);
void orc_quantize_row_q8_0(const float *x, uint8_t *y, int64_t k, int variant);
float orc_vec_dot_q4_0_q8_0(int64_t n, const uint8_t *x, const uint8_t *y);

/* Host-memory versions of the C-ABI ops (same descriptors, host pointers). */
int orc_set_rows_q4_0(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *idx);
int orc_flash_attn_ext(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                       const sqa_tensor *mask, float scale, float max_bias, float logit_softcap,
                       const sqa_tensor *dst, int n_threads, int q8_variant);
int orc_flash_attn_ext_causal(const sqa_tensor *q, const sqa_tensor *k, const sqa_tensor *v,
                              int64_t q_pos0, const sqa_tensor *gate, float scale,
                              const sqa_tensor *dst, int n_threads, int q8_variant);
int orc_sigmoid_mul(const sqa_tensor *dst, const sqa_tensor *x, const sqa_tensor *gate);
void orc_rms_norm_mul_row(const float *x, const float *w, float eps, int64_t n, float *y);
void orc_imrope_cache(int32_t n_rot, const int32_t sections[4], float theta_scale, float freq_scale,
                      float attn_factor, const int32_t p[4], float *cache);
void orc_rope_row(const float *x, int64_t n, int32_t n_rot, const float *cache, float *y);
float orc_rope_theta_scale(const sqa_rope *rope);
int orc_rope_norm_set_rows_q4_0(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *norm_w,
                                float eps, const sqa_tensor *pos, const sqa_rope *rope, const sqa_tensor *idx);
int orc_rope_norm_f32(const sqa_tensor *dst, const sqa_tensor *src, const sqa_tensor *norm_w, float eps,
                      const sqa_tensor *pos, const sqa_rope *rope);

void orc_dequantize_row_q4_K(const uint8_t *x, float *y, int64_t k);
int orc_out_proj(const sqa_tensor *dst, const sqa_tensor *w, const sqa_tensor *x, const sqa_tensor *gate);

int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
