// set_rows_q4_0.hip - quantize-on-write of F32 rows into a q4_0 cache.
//
// Device counterpart of the GGML_OP_SET_ROWS nodes KvCache::append emits
// (reference: src/engine/kv.rs:356-396). Each q4_0 block of 32 values is
// handled by 8 lanes holding 4 consecutive floats each, so one wavefront reads
// 8 blocks = 1 KiB of contiguous source per load instruction.
//
// The arithmetic is ggml's quantize_row_q4_0_ref, bit for bit (q4_0_block.hpp).
#include "q4_0_block.hpp"

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

    quantize_q4_0_block8(v, t, dst + r * dst_nb1 + (int64_t)b * SQA_Q4_0_BLOCK_BYTES);
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
