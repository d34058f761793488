// fa_combine.hip - merges the split-KV partials of the decode and prefill
// attention kernels: out = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M), with
// M = max_s m_s (the log-sum-exp rule), optionally times sigmoid(gate) (the
// output gate of src/model/attn.rs:282-283 in the reference). The weights
// e^(m_s - M) <= 1 come from the hardware exp2 (about 1 ulp; a weight below
// 2^-126, negligible beside the largest one of 1, may read as 0). Partials:
// acc [n_splits][rows][256] unnormalised, ml [n_splits][rows][2] = (m, l) with m
// in natural-log units of the scaled logits.
#include "common.hpp"

namespace sqa {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

// x of lane ^ 16 and of lane ^ 32 through gfx950's row swaps (VALU, no LDS
// round trip): a swap of x with itself leaves x in one result and the
// partner's x in the other
__device__ __forceinline__ float lane_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// Merge of up to kMaxSplits (256) split partials with one memory latency on the
// path. Grid: (rows, 16 chunks of 16 dims); 256 threads = 16 dims x 16 split
// groups. Each thread issues the loads of its 16 splits' acc values and (m, l)
// pairs at once; the maximum, the weights and the sums then follow from
// registers, with cross-lane reductions inside a wavefront and one LDS exchange
// per quantity across the 4 wavefronts.
static_assert(kMaxSplits == 256, "16 split groups x 16 splits per thread");
__global__ __launch_bounds__(256) void fa_combine_kernel(const float *__restrict__ part_acc,
                                                              const float *__restrict__ part_ml,
                                                              int n_splits, int rows_total,
                                                              float *__restrict__ dst, const char *gate,
                                                              int64_t gate_nb1, int64_t gate_nb2, int H) {
    __shared__ float xm[4], xo[4][16], xl[4];
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const int dl = tid & 15, sg = tid >> 4, wv = tid >> 6;
    const int d = blockIdx.y * 16 + dl;
    const int64_t sstride = (int64_t)rows_total * 256;
    const float *pa = part_acc + (int64_t)row * 256 + d;
    const float2 *pm = reinterpret_cast<const float2 *>(part_ml) + row;
    float acc[16];
    float2 ml[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int sp = sg + 16 * j;
        const bool ok = sp < n_splits;
        acc[j] = ok ? pa[sp * sstride] : 0.0f;
        ml[j] = ok ? pm[(int64_t)sp * rows_total] : make_float2(-INFINITY, 0.0f);
    }
    // M: maximum over all splits (lanes 16 apart hold other split groups)
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < 16; ++j) m = fmaxf(m, ml[j].x);
    m = fmaxf(m, lane_xor16(m));
    m = fmaxf(m, lane_xor32(m));
    if ((tid & 63) == 0) xm[wv] = m;
    __syncthreads();
    const float M = fmaxf(fmaxf(xm[0], xm[1]), fmaxf(xm[2], xm[3]));
    float o = 0.0f, l = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float w = (M == -INFINITY || ml[j].x == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f((ml[j].x - M) * kLog2e);
        o = fmaf(acc[j], w, o);
        l = fmaf(ml[j].y, w, l);
    }
    o += lane_xor16(o);
    o += lane_xor32(o);
    l += lane_xor16(l);
    l += lane_xor32(l);
    if ((tid & 63) < 16) xo[wv][dl] = o;
    if ((tid & 63) == 0) xl[wv] = l;
    __syncthreads();
    if (tid < 16) {
        const float ot = (xo[0][dl] + xo[1][dl]) + (xo[2][dl] + xo[3][dl]);
        const float L = (xl[0] + xl[1]) + (xl[2] + xl[3]);
        float r = (L == 0.0f) ? 0.0f : ot * (1.0f / L);
        if (gate) {
            const int t = row / H, h = row % H;
            const float gv = reinterpret_cast<const float *>(gate + t * gate_nb2 + h * gate_nb1)[d];
            r = r * (1.0f / (1.0f + expf(-gv)));
        }
        dst[(int64_t)row * 256 + d] = r;
    }
}

// The same merge for many rows and few splits (prefill): 64 threads per row,
// one float4 of the row each, 4 rows per block; every thread walks the splits
// itself (the (m, l) pairs are the same for the 64 threads of a row and come
// from the cache).
constexpr int kRowsMaxSplits = 32;
__global__ __launch_bounds__(256) void fa_combine_rows_kernel(const float *__restrict__ part_acc,
                                                              const float *__restrict__ part_ml,
                                                              int n_splits, int rows_total,
                                                              float *__restrict__ dst, const char *gate,
                                                              int64_t gate_nb1, int64_t gate_nb2, int H) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int c = threadIdx.x & 63;
    if (row >= rows_total) return;
    float ms[kRowsMaxSplits];
    float M = -INFINITY;
#pragma unroll
    for (int sp = 0; sp < kRowsMaxSplits; ++sp) {
        ms[sp] = sp < n_splits ? part_ml[((int64_t)sp * rows_total + row) * 2] : -INFINITY;
        M = fmaxf(M, ms[sp]);
    }
    const int64_t sstride = (int64_t)rows_total * 256;
    const float *pa = part_acc + (int64_t)row * 256 + 4 * c;
    float L = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int sp = 0; sp < kRowsMaxSplits; ++sp) {
        if (sp >= n_splits) break;
        const float w = (M == -INFINITY || ms[sp] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f((ms[sp] - M) * kLog2e);
        L = fmaf(part_ml[((int64_t)sp * rows_total + row) * 2 + 1], w, L);
        const float4 a = *reinterpret_cast<const float4 *>(pa + sp * sstride);
        o.x = fmaf(a.x, w, o.x);
        o.y = fmaf(a.y, w, o.y);
        o.z = fmaf(a.z, w, o.z);
        o.w = fmaf(a.w, w, o.w);
    }
    const float inv = L == 0.0f ? 0.0f : 1.0f / L;
    float r[4] = {o.x * inv, o.y * inv, o.z * inv, o.w * inv};
    if (gate) {
        const int t = row / H, h = row % H;
        const float *gp = reinterpret_cast<const float *>(gate + t * gate_nb2 + h * gate_nb1) + 4 * c;
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = r[j] * (1.0f / (1.0f + expf(-gp[j])));
    }
    *reinterpret_cast<float4 *>(dst + (int64_t)row * 256 + 4 * c) = make_float4(r[0], r[1], r[2], r[3]);
}

}  // namespace

int launch_fa_combine(const float *part_acc, const float *part_ml, int n_splits, int rows_total,
                      float *dst, const sqa_tensor *gate, int H, hipStream_t s) {
    const char *g = gate ? (const char *)gate->data : nullptr;
    const int64_t g1 = gate ? (int64_t)gate->nb[1] : 0, g2 = gate ? (int64_t)gate->nb[2] : 0;
    if (n_splits > kMaxSplits)
        return set_error(SQA_ERR_UNSUPPORTED, "fa_combine: %d splits > %d", n_splits, kMaxSplits);
    const int prof = profile_start("fa_combine", s);
    if (n_splits <= kRowsMaxSplits && rows_total >= 64) {
        fa_combine_rows_kernel<<<dim3((unsigned)((rows_total + 3) / 4)), dim3(256), 0, s>>>(
            part_acc, part_ml, n_splits, rows_total, dst, g, g1, g2, H);
    } else {
        fa_combine_kernel<<<dim3((unsigned)rows_total, 16), dim3(256), 0, s>>>(part_acc, part_ml, n_splits,
                                                                            rows_total, dst, g, g1, g2, H);
    }
    profile_stop(prof, s);
    return hip_status(hipGetLastError(), "fa_combine launch");
}

}  // namespace sqa
