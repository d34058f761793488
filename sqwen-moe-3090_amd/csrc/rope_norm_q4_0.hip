// rope_norm_q4_0.hip - the K (and Q) producer of a full-attention layer in one
// pass over the projected rows: per-head RMSNorm times its weight, IMROPE, and
// for K the q4_0 quantize-on-write into the cache row of the token. It replaces
// the ggml_rms_norm -> ggml_mul -> ggml_rope_multi(IMROPE) -> ggml_set_rows
// chain of src/model/attn.rs:166-200 and src/engine/kv.rs:313-399 in the
// reference (head_rms_norm at attn.rs:68-84), which ggml runs as separate
// kernels with the rows round-tripping through memory between them.
//
// Arithmetic follows ggml's CPU kernels step by step, each operation rounded on
// its own (contraction off in the kernel):
//   norm: sum of x*x in double, mean = (float)(sum / D), scale =
//         1/sqrtf(mean + eps) (the root correctly rounded), y = x*scale, then y*w;
//   rope: the angle of rotation pair ic is the token's position of the pair's
//         IMROPE sector times theta_scale^ic, formed as ic successive fp32
//         multiplies (theta_scale = powf(freq_base, -2/n_rot) is computed once on
//         the host with the C library, as ggml does); cos/sin of freq_scale*angle
//         (correctly rounded) times attn_factor; (x0, x1) = (y[ic], y[ic + n_rot/2]) ->
//         (x0*c - x1*s, x0*s + x1*c); dims >= n_rot pass through;
//   q4_0: ggml's quantize_row_q4_0_ref (q4_0_block.hpp).
//
// Layout: one workgroup per token. Its first n_rot/2 threads form the token's
// cos/sin table in LDS (as ggml forms one cache per token), then the heads stream
// through D/4 lanes per head row, 4 consecutive dims each, so the 8 lanes of a
// 32-value block hold it as the quantizer wants. The rotation partner of dim d
// sits in the same register of the lane n_rot/8 away (n_rot % 8 == 0).
#include "q4_0_block.hpp"

namespace sqa {
namespace {

constexpr int kThreads = 256;

struct ProducerParams {
    const char *src;
    int64_t src_nb1, src_nb2;  // head, token strides in bytes
    const float *norm_w;       // [D] or null
    float eps;
    const int32_t *pos;        // [4 * n_tok]
    int64_t n_tok;
    int n_head;
    int n_rot;
    int sections[4];
    int sect;  // sum of the sections
    float theta_scale, freq_scale, attn_factor;
    // q4_0 output
    uint8_t *dst;
    int64_t dst_nb1, dst_rows;
    const char *idx;
    int64_t idx_nb0;
    // F32 output ([D, n_head, n_tok] contiguous)
    float *dst_f32;
};

template <int D, bool kQ4, bool kVec>
__global__ __launch_bounds__(kThreads) void rope_norm_kernel(ProducerParams p) {
    // every multiply and add rounded on its own, as ggml's C: with contraction on
    // (hipcc's default, and inside HIP's __fmul_rn / __fadd_rn, which are plain
    // * and +) the rotation x0*c - x1*s became an fma, an ulp off in a quarter
    // of the values
#pragma clang fp contract(off)
    constexpr int kLanes = D / 4;                  // lanes per head row
    constexpr int kRowsPerPass = kThreads / kLanes;  // head rows in flight
    __shared__ float2 cs[D / 2];                   // (cos, sin) of rotation pair ic
    const int tid = threadIdx.x;
    const int64_t t = blockIdx.x;
    const int half = p.n_rot >> 1;

    // ---- the token's rotation table: pair ic, angle pos[sector] * theta_scale^ic
    if (tid < half) {
        const int ic = tid;
        const int sector = ic % p.sect;
        int c;  // position component: 0 t, 1 h, 2 w, 3 e
        if (sector % 3 == 1 && sector < 3 * p.sections[1]) c = 1;
        else if (sector % 3 == 2 && sector < 3 * p.sections[2]) c = 2;
        else if (sector % 3 == 0 && sector < 3 * p.sections[0]) c = 0;
        else c = 3;
        float th = (float)p.pos[t + c * p.n_tok];
        for (int k = 0; k < ic; ++k) th = th * p.theta_scale;
        const float ang = p.freq_scale * th;
        // cos and sin in double, rounded once to float: the correctly rounded
        // values, which the C library's cosf/sinf also return but for about 1% of
        // arguments (the fp32 device sincosf differs from them in the last bit far
        // more often)
        double sd, cd;
        sincos((double)ang, &sd, &cd);
        cs[ic] = make_float2((float)cd * p.attn_factor, (float)sd * p.attn_factor);
    }
    __syncthreads();

    int64_t r = 0;
    if constexpr (kQ4) {
        r = *reinterpret_cast<const int64_t *>(p.idx + t * p.idx_nb0);
        if (r < 0 || r >= p.dst_rows) return;  // whole workgroup, past its only barrier
    }
    const int l = tid % kLanes;
    const int sh = half >> 2;  // lanes between the two dims of a pair
    const int lp = 4 * l < half ? l + sh : (4 * l < p.n_rot ? l - sh : l);
    for (int h = tid / kLanes; h < p.n_head; h += kRowsPerPass) {  // uniform per row group
        const float *x = reinterpret_cast<const float *>(p.src + h * p.src_nb1 + t * p.src_nb2) + 4 * l;
        float v[4];
        if constexpr (kVec) {
            const float4 f = *reinterpret_cast<const float4 *>(x);
            v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = x[j];
        }

        if (p.norm_w) {
            double s = 0.0;
#pragma unroll
            for (int j = 0; j < 4; ++j) s += (double)(v[j] * v[j]);
#pragma unroll
            for (int off = kLanes / 2; off >= 1; off >>= 1) s += __shfl_xor(s, off, kLanes);
            const float mean = (float)(s / (double)D);
            // sqrtf correctly rounded, as the C library's: the root in double rounded
            // once to float (the fp32 square root compiles to v_sqrt_f32 alone,
            // up to an ulp off, which moved the scale of about 10% of rows)
            const float root = (float)__builtin_sqrt((double)(mean + p.eps));
            const float scale = __fdiv_rn(1.0f, root);
            const float4 w = *reinterpret_cast<const float4 *>(p.norm_w + 4 * l);
            const float wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = v[j] * scale * wv[j];
        }

        float out[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float pv = __shfl(v[j], lp, kLanes);  // every lane takes part
            const int d = 4 * l + j;
            if (d >= p.n_rot) {
                out[j] = v[j];
            } else if (d < half) {
                const float2 c = cs[d];  // x0 = v, x1 = partner: x0*c - x1*s
                out[j] = v[j] * c.x - pv * c.y;
            } else {
                const float2 c = cs[d - half];  // x0 = partner, x1 = v: x0*s + x1*c
                out[j] = pv * c.y + v[j] * c.x;
            }
        }

        if constexpr (kQ4) {
            const int b = l >> 3;  // block of this lane's dims within the head row
            quantize_q4_0_block8(out, l & 7,
                                 p.dst + r * p.dst_nb1 + (int64_t)(h * (D / SQA_QK4_0) + b) * SQA_Q4_0_BLOCK_BYTES);
        } else {
            *reinterpret_cast<float4 *>(p.dst_f32 + (t * p.n_head + h) * D + 4 * l) =
                make_float4(out[0], out[1], out[2], out[3]);
        }
    }
}

template <int D, bool kQ4>
void launch_d(const ProducerParams &p, bool vec, hipStream_t s) {
    const int64_t grid = p.n_tok;  // one workgroup per token
    if (vec)
        rope_norm_kernel<D, kQ4, true><<<dim3((unsigned)grid), dim3(kThreads), 0, s>>>(p);
    else
        rope_norm_kernel<D, kQ4, false><<<dim3((unsigned)grid), dim3(kThreads), 0, s>>>(p);
}

template <bool kQ4>
int launch_any(const ProducerParams &p, int D, bool vec, hipStream_t s) {
    switch (D) {
        case 64: launch_d<64, kQ4>(p, vec, s); break;
        case 128: launch_d<128, kQ4>(p, vec, s); break;
        case 256: launch_d<256, kQ4>(p, vec, s); break;
        default: return set_error(SQA_ERR_UNSUPPORTED, "rope_norm: head dim %d not in {64, 128, 256}", D);
    }
    return SQA_OK;
}

}  // namespace

int launch_rope_norm(const sqa_tensor *dst, const sqa_tensor &src, const sqa_tensor *norm_w, float eps,
                     const sqa_tensor &pos, const sqa_rope &rope, float theta_scale, const sqa_tensor *idx,
                     hipStream_t s) {
    ProducerParams p{};
    const int D = (int)src.ne[0];
    p.src = (const char *)src.data;
    p.src_nb1 = (int64_t)src.nb[1];
    p.src_nb2 = (int64_t)src.nb[2];
    p.norm_w = norm_w ? (const float *)norm_w->data : nullptr;
    p.eps = eps;
    p.pos = (const int32_t *)pos.data;
    p.n_tok = src.ne[2];
    p.n_head = (int)src.ne[1];
    p.n_rot = rope.n_rot;
    p.sect = 0;
    for (int k = 0; k < 4; ++k) {
        p.sections[k] = rope.sections[k];
        p.sect += rope.sections[k];
    }
    p.theta_scale = theta_scale;
    p.freq_scale = rope.freq_scale;
    p.attn_factor = rope.attn_factor;
    if (p.n_tok == 0) return SQA_OK;
    const bool vec = (uintptr_t)src.data % 16 == 0 && src.nb[1] % 16 == 0 && src.nb[2] % 16 == 0;
    const bool q4 = idx != nullptr;
    if (q4) {
        p.dst = (uint8_t *)dst->data;
        p.dst_nb1 = (int64_t)dst->nb[1];
        p.dst_rows = dst->ne[1];
        p.idx = (const char *)idx->data;
        p.idx_nb0 = (int64_t)idx->nb[0];
    } else {
        p.dst_f32 = (float *)dst->data;
    }
    const int prof = profile_start(q4 ? "rope_norm_set_rows_q4_0" : "rope_norm_f32", s);
    const int rc = q4 ? launch_any<true>(p, D, vec, s) : launch_any<false>(p, D, vec, s);
    profile_stop(prof, s);
    if (rc != SQA_OK) return rc;
    return hip_status(hipGetLastError(), "rope_norm launch");
}

}  // namespace sqa
