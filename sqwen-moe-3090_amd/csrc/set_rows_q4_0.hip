// set_rows_q4_0.hip - quantize-on-write of F32 rows into a q4_0 cache.
//
// Device counterpart of the GGML_OP_SET_ROWS nodes KvCache::append emits
// (reference: src/engine/kv.rs:356-396). Each q4_0 block of 32 values is
// handled by 8 lanes holding 4 consecutive floats each, so one wavefront reads
// 8 blocks = 1 KiB of contiguous source per load instruction.
//
// The arithmetic is ggml's quantize_row_q4_0_ref, bit for bit:
//   max  = value of largest |x| in the block, first occurrence on ties
//   d    = max / -8            (stored as fp16, round-to-nearest-even)
//   id   = d != 0 ? 1/d : 0    (correctly rounded fp32 division)
//   code = min(15, (int8_t)(x*id + 8.5f)) with the multiply and the add each
//          rounded on their own (no fused multiply-add)
// An all-zero block therefore stores d = -0.0 (fp16 0x8000) and codes 8.
#include "common.hpp"

namespace sqa {
namespace {

constexpr int kThreads = 256;

template <bool kVec>
__global__ __launch_bounds__(kThreads) void set_rows_q4_0_kernel(
    uint8_t *__restrict__ dst, int64_t dst_nb1, int64_t dst_rows, const char *__restrict__ src,
    int64_t src_nb1, const char *__restrict__ idx, int64_t idx_nb0, int64_t n_rows,
    int blocks_per_row) {
    const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t blk = gid >> 3;
    const int t = threadIdx.x & 7;
    if (blk >= n_rows * blocks_per_row) return;  // whole 8-lane groups exit together
    const int64_t row = blk / blocks_per_row;
    const int b = (int)(blk - row * blocks_per_row);
    const int64_t r = *reinterpret_cast<const int64_t *>(idx + row * idx_nb0);
    if (r < 0 || r >= dst_rows) return;  // same row for all 8 lanes of the group

    const float *x = reinterpret_cast<const float *>(src + row * src_nb1) + b * SQA_QK4_0 + 4 * t;
    float v[4];
    if constexpr (kVec) {
        const float4 f = *reinterpret_cast<const float4 *>(x);
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = x[j];
    }

    // Lane-local first-occurrence maximum of |x|; index 32 marks "none".
    float amax = 0.0f, mx = 0.0f;
    int im = 32;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float a = fabsf(v[j]);
        if (amax < a) { amax = a; mx = v[j]; im = 4 * t + j; }
    }
#pragma unroll
    for (int off = 4; off >= 1; off >>= 1) {
        const float a2 = __shfl_xor(amax, off, 8);
        const float m2 = __shfl_xor(mx, off, 8);
        const int i2 = __shfl_xor(im, off, 8);
        if (a2 > amax || (a2 == amax && i2 < im)) { amax = a2; mx = m2; im = i2; }
    }

    const float d = mx / -8.0f;
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float y = __fadd_rn(__fmul_rn(v[j], id), 8.5f);
        int c = (int)y;  // truncation toward zero, y in [0.5, 16.5] for finite input
        c = c < 15 ? c : 15;
        word |= (uint32_t)(c & 0xff) << (8 * j);
    }
    // qs[j] = code[j] | code[j+16] << 4: lanes 0..3 take the high nibbles from lanes 4..7.
    const uint32_t hi = __shfl_down(word, 4, 8);
    uint8_t *blkp = dst + r * dst_nb1 + (int64_t)b * SQA_Q4_0_BLOCK_BYTES;
    if (t < 4) {
        const uint32_t qs = word | (hi << 4);
        uint16_t *p = reinterpret_cast<uint16_t *>(blkp + 2 + 4 * t);
        p[0] = (uint16_t)(qs & 0xffff);
        p[1] = (uint16_t)(qs >> 16);
    } else if (t == 4) {
        const _Float16 dh = (_Float16)d;
        *reinterpret_cast<_Float16 *>(blkp) = dh;
    }
}

}  // namespace

int launch_set_rows_q4_0(const sqa_tensor &dst, const sqa_tensor &src, const sqa_tensor &idx,
                         hipStream_t s) {
    const int64_t n_rows = src.ne[1];
    const int bpr = (int)(src.ne[0] / SQA_QK4_0);
    if (n_rows == 0) return SQA_OK;
    const int64_t total_lanes = n_rows * bpr * 8;
    const int64_t grid = (total_lanes + kThreads - 1) / kThreads;
    const bool vec = ((uintptr_t)src.data % 16 == 0) && (src.nb[1] % 16 == 0);
    const int prof = profile_start("set_rows_q4_0", s);
    if (vec) {
        set_rows_q4_0_kernel<true><<<dim3((unsigned)grid), dim3(kThreads), 0, s>>>(
            (uint8_t *)dst.data, (int64_t)dst.nb[1], dst.ne[1], (const char *)src.data,
            (int64_t)src.nb[1], (const char *)idx.data, (int64_t)idx.nb[0], n_rows, bpr);
    } else {
        set_rows_q4_0_kernel<false><<<dim3((unsigned)grid), dim3(kThreads), 0, s>>>(
            (uint8_t *)dst.data, (int64_t)dst.nb[1], dst.ne[1], (const char *)src.data,
            (int64_t)src.nb[1], (const char *)idx.data, (int64_t)idx.nb[0], n_rows, bpr);
    }
    profile_stop(prof, s);
    return hip_status(hipGetLastError(), "set_rows_q4_0 launch");
}

}  // namespace sqa
