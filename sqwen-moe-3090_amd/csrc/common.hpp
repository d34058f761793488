// common.hpp - shared definitions of the gfx950 attention library.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/sqattn.h"

namespace sqa {

// Head dimension and q4_0 geometry of the path (qwen35moe full attention:
// head_dim 256 enforced at src/model/arch.rs:156-160 of the reference).
constexpr int kHeadDim = 256;
constexpr int kBlocksPerHead = kHeadDim / SQA_QK4_0;            // 8
constexpr int kHeadRowBytes = kBlocksPerHead * SQA_Q4_0_BLOCK_BYTES;  // 144

// Store of an attention kernel's result or split partial, written through to
// memory at once (an agent-scope relaxed store: a vector store with sc1). The
// next kernel reads it from memory anyway (the L2 of another XCD cannot serve
// it), and a plain store leaves a dirty L2 line that the end of the kernel must
// write back, after the last workgroup's stores, on the critical path.
__device__ __forceinline__ void store_through(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Records a message for sqa_last_error() and returns the status.
int set_error(int status, const char *fmt, ...);
int hip_status(hipError_t e, const char *what);

// Device count of compute units (cached per device).
int device_cu_count();

// Optional event timing around launches (profile.cpp).
bool profile_on();
int profile_start(const char *name, hipStream_t s);
void profile_stop(int slot, hipStream_t s);

// Kernel launchers (defined next to their kernels).
int launch_set_rows_q4_0(const sqa_tensor &dst, const sqa_tensor &src, const sqa_tensor &idx,
                         hipStream_t s);
// Norm + IMROPE producer; idx != null: q4_0 quantize-on-write into dst rows,
// else F32 output (rope_norm_q4_0.hip). theta_scale = powf(freq_base, -2/n_rot).
int launch_rope_norm(const sqa_tensor *dst, const sqa_tensor &src, const sqa_tensor *norm_w, float eps,
                     const sqa_tensor &pos, const sqa_rope &rope, float theta_scale, const sqa_tensor *idx,
                     hipStream_t s);
int launch_sigmoid_mul(const sqa_tensor &dst, const sqa_tensor &x, const sqa_tensor &gate,
                       hipStream_t s);
int launch_fill_causal_mask(const sqa_tensor &mask, int64_t step_start, hipStream_t s);

struct FaArgs {
    const sqa_tensor *q, *k, *v, *mask, *gate, *dst;
    float scale;
    int64_t q_pos0;  // >= 0: causal from positions, mask ignored
    void *ws;
    size_t ws_bytes;
};
// Decode workspace bytes; mask_copy: the F16 mask needs the packed copy (its
// rows are not 16-byte aligned or n_kv % 8 != 0, see decode_mask_needs_copy).
size_t fa_decode_workspace(int64_t n_q, int64_t H, int64_t n_kvh, int64_t n_kv, bool mask_copy = true);
bool decode_mask_needs_copy(const sqa_tensor *mask, int64_t n_kv);
// Device scratch of the allocation-free decode entry point: its size, and its
// address on the current device (looked up once per device).
constexpr size_t kStaticScratchBytes = SQA_STATIC_SCRATCH_BYTES;
int static_scratch(void **out);
// Merges split partials [n_splits][rows][256] + [n_splits][rows][2] into dst;
// n_splits <= kMaxSplits (the split planners cap there).
constexpr int kMaxSplits = 256;
int launch_fa_combine(const float *part_acc, const float *part_ml, int n_splits, int rows_total,
                      float *dst, const sqa_tensor *gate, int H, hipStream_t s);
int launch_fa_decode(const FaArgs &a, hipStream_t s);
// W_o projection dst[N, M] = W[K, N] (Q4_K) . (x * sigmoid(gate)) (gate may be null)
size_t out_proj_workspace(int64_t K, int64_t M);
int launch_out_proj(const sqa_tensor &w, const sqa_tensor &x, const sqa_tensor *gate, const sqa_tensor &dst,
                    void *ws, size_t ws_bytes, hipStream_t s);
size_t fa_prefill_workspace(int64_t n_q, int64_t H, int64_t Hkv, int64_t n_kv);
int launch_fa_prefill(const FaArgs &a, hipStream_t s);

}  // namespace sqa
