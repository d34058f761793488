// gate_mask.hip - the elementwise pieces beside the attention op:
//   sigmoid_mul       out = x * sigmoid(gate)   (ggml_sigmoid + ggml_mul of
//                     src/model/attn.rs:282-283 in the reference)
//   fill_causal_mask  F16 [n_kv, n_q] causal mask built on the device
//                     (src/model/graph.rs:534-576 builds it on the host)
// Both are HBM-bound streaming kernels: 16-byte accesses, one grid-stride loop.
#include "common.hpp"

namespace sqa {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float sigmoid_ref(float g) { return 1.0f / (1.0f + expf(-g)); }

// Rows of n0 floats; row strides in bytes. n0 % 4 == 0 and 16-byte alignment
// are checked on the host for the vector path.
template <bool kVec>
__global__ __launch_bounds__(kThreads) void sigmoid_mul_kernel(
    char *__restrict__ dst, int64_t dst_nb1, const char *__restrict__ x, int64_t x_nb1,
    const char *__restrict__ gate, int64_t g_nb1, int64_t n0, int64_t n1) {
    const int64_t per_row = kVec ? n0 / 4 : n0;
    const int64_t total = per_row * n1;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        const int64_t row = i / per_row;
        const int64_t col = i - row * per_row;
        if constexpr (kVec) {
            const float4 a = reinterpret_cast<const float4 *>(x + row * x_nb1)[col];
            const float4 g = reinterpret_cast<const float4 *>(gate + row * g_nb1)[col];
            float4 o;
            o.x = a.x * sigmoid_ref(g.x);
            o.y = a.y * sigmoid_ref(g.y);
            o.z = a.z * sigmoid_ref(g.z);
            o.w = a.w * sigmoid_ref(g.w);
            reinterpret_cast<float4 *>(dst + row * dst_nb1)[col] = o;
        } else {
            const float a = reinterpret_cast<const float *>(x + row * x_nb1)[col];
            const float g = reinterpret_cast<const float *>(gate + row * g_nb1)[col];
            reinterpret_cast<float *>(dst + row * dst_nb1)[col] = a * sigmoid_ref(g);
        }
    }
}

// One lane writes 8 consecutive keys of one query row.
__global__ __launch_bounds__(kThreads) void fill_causal_mask_kernel(
    char *__restrict__ mask, int64_t nb1, int64_t n_kv, int64_t n_q, int64_t step_start) {
    const int64_t groups = (n_kv + 7) / 8;
    const int64_t total = groups * n_q;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        const int64_t t = i / groups;
        const int64_t k0 = (i - t * groups) * 8;
        const int64_t limit = step_start + t;  // keys <= limit are visible
        uint16_t *row = reinterpret_cast<uint16_t *>(mask + t * nb1);
        if (k0 + 8 <= n_kv && ((uintptr_t)(row + k0) % 16) == 0) {
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t lo = (k0 + 2 * j <= limit) ? 0x0000u : 0xFC00u;
                const uint32_t hi = (k0 + 2 * j + 1 <= limit) ? 0x0000u : 0xFC00u;
                w[j] = lo | (hi << 16);
            }
            *reinterpret_cast<uint4 *>(row + k0) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            for (int64_t k = k0; k < k0 + 8 && k < n_kv; ++k) row[k] = (k <= limit) ? 0x0000 : 0xFC00;
        }
    }
}

int64_t grid_for(int64_t work) {
    int64_t g = (work + kThreads - 1) / kThreads;
    const int64_t cap = (int64_t)device_cu_count() * 16;
    return g < 1 ? 1 : (g > cap ? cap : g);
}

}  // namespace

int launch_sigmoid_mul(const sqa_tensor &dst, const sqa_tensor &x, const sqa_tensor &gate,
                       hipStream_t s) {
    const int64_t n0 = x.ne[0], n1 = x.ne[1];
    if (n0 * n1 == 0) return SQA_OK;
    const bool vec = n0 % 4 == 0 && (uintptr_t)dst.data % 16 == 0 && (uintptr_t)x.data % 16 == 0 &&
                     (uintptr_t)gate.data % 16 == 0 && dst.nb[1] % 16 == 0 && x.nb[1] % 16 == 0 &&
                     gate.nb[1] % 16 == 0;
    const int64_t grid = grid_for(vec ? n0 / 4 * n1 : n0 * n1);
    const int prof = profile_start("sigmoid_mul", s);
    if (vec) {
        sigmoid_mul_kernel<true><<<dim3((unsigned)grid), dim3(kThreads), 0, s>>>(
            (char *)dst.data, (int64_t)dst.nb[1], (const char *)x.data, (int64_t)x.nb[1],
            (const char *)gate.data, (int64_t)gate.nb[1], n0, n1);
    } else {
        sigmoid_mul_kernel<false><<<dim3((unsigned)grid), dim3(kThreads), 0, s>>>(
            (char *)dst.data, (int64_t)dst.nb[1], (const char *)x.data, (int64_t)x.nb[1],
            (const char *)gate.data, (int64_t)gate.nb[1], n0, n1);
    }
    profile_stop(prof, s);
    return hip_status(hipGetLastError(), "sigmoid_mul launch");
}

int launch_fill_causal_mask(const sqa_tensor &mask, int64_t step_start, hipStream_t s) {
    const int64_t n_kv = mask.ne[0], n_q = mask.ne[1];
    if (n_kv * n_q == 0) return SQA_OK;
    const int64_t grid = grid_for((n_kv + 7) / 8 * n_q);
    fill_causal_mask_kernel<<<dim3((unsigned)grid), dim3(kThreads), 0, s>>>(
        (char *)mask.data, (int64_t)mask.nb[1], n_kv, n_q, step_start);
    return hip_status(hipGetLastError(), "fill_causal_mask launch");
}

}  // namespace sqa
