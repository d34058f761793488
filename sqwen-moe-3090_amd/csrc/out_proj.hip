// out_proj.hip - the W_o projection that closes the full-attention layer:
//   dst = W . (x * sigmoid(gate))        (src/model/attn.rs:281-285 in the
// reference: ggml_sigmoid + ggml_mul, then ggml_mul_mat(attn_output, gated))
// with W = attn_output.weight in ggml's Q4_K format, ne = [K, N] (K = n_head *
// head_dim = 4096 here, N = n_embd), x and gate F32 [K, M] (M tokens), dst F32
// [N, M].
//
// Q4_K super-block (256 values, 144 bytes): fp16 d and dmin, twelve bytes of
// 6-bit (scale, min) pairs for the 8 sub-blocks of 32, then 128 bytes of 4-bit
// codes (byte l of 32-byte group j: value 64j + l in the low nibble, value
// 64j + 32 + l in the high one). A value is d*scale*code - dmin*min.
//
// Up to 4 tokens (decode, verify) one kernel, op_gemv (below); more tokens two:
//   op_prep  one thread per (token, 32-value sub-block): xg = x * sigmoid(gate)
//            in fp32, written as an fp16 hi + lo pair (xg = hi + lo to ~22
//            bits) [M16][K], plus the sub-block sum S = sum xg [M16][K/32];
//            tokens M..M16-1 (M16 = M rounded up to 16) are zeros
//   op_gemm  16x16x32 f16 MFMAs over the raw codes: per sub-block the A operand
//            is the 4-bit codes as fp16 subnormals (code * 2^-24 for low
//            nibbles, code * 2^-20 for high ones: exact, one v_perm and one
//            v_and per two codes), B = xg hi and lo, so C = sum code * xg has
//            every product exact; the wave then adds (d*scale*2^24 or 2^20) * C
//            - dmin*min * S per (row, token). Rows of W are read once per token
//            tile straight from the weight bytes.
// A workgroup owns 16 rows (decode: 16 wavefronts) or 64 rows (4 wavefronts)
// and one tile of 16 tokens; its wavefronts split K by super-block and add
// their partial sums through LDS.
//
// MFMA operand layouts (lane = 16*g + n):
//   16x16x32 f16: A[n][8g..8g+7]   B[8g..8g+7][n]   C[4g..4g+3][n]
#include <mutex>

#include "common.hpp"

namespace sqa {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

constexpr int kQK = 256;           // values per Q4_K super-block
constexpr int kBlockBytes = 144;   // bytes per super-block
constexpr int kSubs = kQK / 32;    // sub-blocks per super-block
constexpr int kGemvTokens = 4;     // token counts up to this take op_gemv
constexpr int kGemvMaxLds = 160 * 1024;
constexpr int kGemvSbStride = kQK + 4;  // floats per super-block of activations in LDS

__device__ __forceinline__ float h2f(uint32_t bits) {
    _Float16 h;
    const uint16_t b = (uint16_t)bits;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// ---------------------------------------------------------------- op_prep
// x (and gate) rows: 16-byte aligned when VEC (checked on the host)
template <bool GATE, bool VEC>
__global__ __launch_bounds__(256) void op_prep_kernel(const char *__restrict__ x, int64_t x_nb1,
                                                      const char *__restrict__ gate, int64_t g_nb1, int K, int M,
                                                      int M16, uint16_t *__restrict__ xh, uint16_t *__restrict__ xl,
                                                      float *__restrict__ S) {
    const int subs = K / 32;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)subs * M16) return;
    const int t = (int)(idx / subs), s = (int)(idx - (int64_t)t * subs);
    float v[32], gv[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = gv[j] = 0.0f;
    if (t < M) {
        const float *xr = reinterpret_cast<const float *>(x + t * x_nb1) + 32 * s;
        const float *gr = GATE ? reinterpret_cast<const float *>(gate + t * g_nb1) + 32 * s : nullptr;
        if (VEC) {
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const float4 a = reinterpret_cast<const float4 *>(xr)[c];
                v[4 * c] = a.x, v[4 * c + 1] = a.y, v[4 * c + 2] = a.z, v[4 * c + 3] = a.w;
                if (GATE) {
                    const float4 b = reinterpret_cast<const float4 *>(gr)[c];
                    gv[4 * c] = b.x, gv[4 * c + 1] = b.y, gv[4 * c + 2] = b.z, gv[4 * c + 3] = b.w;
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 32; ++j) {
                v[j] = xr[j];
                if (GATE) gv[j] = gr[j];
            }
        }
        if (GATE) {
#pragma unroll
            for (int j = 0; j < 32; ++j) v[j] = v[j] * (1.0f / (1.0f + expf(-gv[j])));
        }
    }
    float sum = 0.0f;
    uint16_t hb[32], lb[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        sum += v[j];
        float a = v[j];
        // opaque: one fp32 value feeds both the stored hi and the hi subtracted for lo
        asm volatile("" : "+v"(a));
        const _Float16 h = (_Float16)a;
        const _Float16 l = (_Float16)(a - (float)h);
        __builtin_memcpy(&hb[j], &h, 2);
        __builtin_memcpy(&lb[j], &l, 2);
    }
    uint4 *ho = reinterpret_cast<uint4 *>(xh + (int64_t)t * K + 32 * s);
    uint4 *lo = reinterpret_cast<uint4 *>(xl + (int64_t)t * K + 32 * s);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        uint4 a, b;
        __builtin_memcpy(&a, hb + 8 * c, 16);
        __builtin_memcpy(&b, lb + 8 * c, 16);
        ho[c] = a;
        lo[c] = b;
    }
    S[idx] = sum;  // [token][sub-block]
}

// ---------------------------------------------------------------- op_gemm
struct GemmParams {
    const uint8_t *w;
    int64_t w_nb1;
    const uint16_t *xh, *xl;
    const float *S;
    int K, N, M, M16;
    float *dst;
    int64_t d_nb1;
};

// (scale, min) of sub-block s from the 12 scale bytes b[0..11], held as three
// dwords q0 = b[0..3], q1 = b[4..7], q2 = b[8..11]
__device__ __forceinline__ void scale_min(uint32_t q0, uint32_t q1, uint32_t q2, int s, int &sc, int &mn) {
    if (s < 4) {
        sc = (q0 >> (8 * s)) & 63;
        mn = (q1 >> (8 * s)) & 63;
    } else {
        const int r = 8 * (s - 4);
        sc = ((q2 >> r) & 15) | (((q0 >> (r + 6)) & 3) << 4);
        mn = ((q2 >> (r + 4)) & 15) | (((q1 >> (r + 6)) & 3) << 4);
    }
}

// A workgroup of KS wavefronts owns 16*RT rows of W and one tile of 16 tokens;
// wavefront w takes super-blocks w, w + KS, ... of K, and the KS partial sums
// meet in LDS at the end. Each wavefront loads all operands of a super-block
// (scales, codes, activations) before it computes on them.
template <int KS, int RT>
__global__ __launch_bounds__(64 * KS) void op_gemm_kernel(GemmParams p) {
    __shared__ float sc_lds[KS][RT][kSubs][2][16];  // per wave: scaled d*scale and dmin*min per sub-block, row
    __shared__ float red[KS][RT][4][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    const int r0 = blockIdx.x * 16 * RT;
    const int t0 = blockIdx.y * 16;
    const int nsb = p.K / kQK;

    floatx4 acc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt] = floatx4{0.f, 0.f, 0.f, 0.f};
    // a column past the M tokens reads token t0's data (one broadcast row for
    // decode) and masks it to zero
    const int tok = t0 + n < p.M ? t0 + n : t0;
    const uint32_t tok_mask = t0 + n < p.M ? 0xFFFFFFFFu : 0u;
    const uint16_t *xh_t = p.xh + (int64_t)tok * p.K + 8 * g;
    const uint16_t *xl_t = p.xl + (int64_t)tok * p.K + 8 * g;
    const float *srow = p.S + (int64_t)tok * (p.K / 32);
    float(*my_sc)[kSubs][2][16] = sc_lds[wave];
    const uint8_t *wrow[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) wrow[rt] = p.w + (int64_t)(r0 + 16 * rt + n) * p.w_nb1;

    for (int sb = wave; sb < nsb; sb += KS) {
        // ---- every load of the super-block first ----
        uint4 hdr[RT];  // d, dmin, scales[0..11] of row tile-row n
        uint2 q[RT][4];  // codes 8g..8g+7 of both sub-blocks of group j
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const uint8_t *blk = wrow[rt] + (int64_t)sb * kBlockBytes;
            hdr[rt] = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
            for (int j = 0; j < 4; ++j) q[rt][j] = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * j + 8 * g);
        }
        uint4 xb[4][4];  // [j][hi lo, hi lo of the high sub-block]; zeros past the M tokens
        float sv[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k0 = sb * kQK + 64 * j;
            xb[j][0] = *reinterpret_cast<const uint4 *>(xh_t + k0);
            xb[j][1] = *reinterpret_cast<const uint4 *>(xl_t + k0);
            xb[j][2] = *reinterpret_cast<const uint4 *>(xh_t + k0 + 32);
            xb[j][3] = *reinterpret_cast<const uint4 *>(xl_t + k0 + 32);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                xb[j][c].x &= tok_mask, xb[j][c].y &= tok_mask, xb[j][c].z &= tok_mask, xb[j][c].w &= tok_mask;
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) sv[e] = __uint_as_float(__float_as_uint(srow[sb * kSubs + e]) & tok_mask);
        // ---- scales of the wave's rows: lane (g, n) decodes sub-blocks 2g, 2g+1 of
        // tile-row n of every row tile and publishes them by row (the LDS accesses
        // of one wavefront complete in order: no barrier) ----
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const float d = h2f(hdr[rt].x & 0xffffu), dmin = h2f(hdr[rt].x >> 16);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int s = 2 * g + e;
                int sc, mn;
                scale_min(hdr[rt].y, hdr[rt].z, hdr[rt].w, s, sc, mn);
                // even sub-blocks read low nibbles (code * 2^-24), odd ones high (2^-20)
                my_sc[rt][s][0][n] = d * (float)sc * (e == 0 ? 16777216.0f : 1048576.0f);
                my_sc[rt][s][1][n] = dmin * (float)mn;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            half8 bh0, bl0, bh1, bl1;
            __builtin_memcpy(&bh0, &xb[j][0], 16);
            __builtin_memcpy(&bl0, &xb[j][1], 16);
            __builtin_memcpy(&bh1, &xb[j][2], 16);
            __builtin_memcpy(&bl1, &xb[j][3], 16);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                uint32_t sp[4];  // bytes 2m, 2m+1 spread to the two halves of dword m
                sp[0] = __builtin_amdgcn_perm(0u, q[rt][j].x, 0x0c010c00u);
                sp[1] = __builtin_amdgcn_perm(0u, q[rt][j].x, 0x0c030c02u);
                sp[2] = __builtin_amdgcn_perm(0u, q[rt][j].y, 0x0c010c00u);
                sp[3] = __builtin_amdgcn_perm(0u, q[rt][j].y, 0x0c030c02u);
                uint32_t lo[4], hi[4];
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    lo[m] = sp[m] & 0x000F000Fu;
                    hi[m] = sp[m] & 0x00F000F0u;
                }
                half8 alo, ahi;
                __builtin_memcpy(&alo, lo, 16);
                __builtin_memcpy(&ahi, hi, 16);
                floatx4 cl = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bh0, floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                cl = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bl0, cl, 0, 0, 0);
                floatx4 ch = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bh1, floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                ch = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bl1, ch, 0, 0, 0);
                const floatx4 dl = *reinterpret_cast<const floatx4 *>(&my_sc[rt][2 * j][0][4 * g]);
                const floatx4 ml = *reinterpret_cast<const floatx4 *>(&my_sc[rt][2 * j][1][4 * g]);
                const floatx4 dh = *reinterpret_cast<const floatx4 *>(&my_sc[rt][2 * j + 1][0][4 * g]);
                const floatx4 mh = *reinterpret_cast<const floatx4 *>(&my_sc[rt][2 * j + 1][1][4 * g]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float a = fmaf(cl[i], dl[i], acc[rt][i]);
                    a = fmaf(-ml[i], sv[2 * j], a);
                    a = fmaf(ch[i], dh[i], a);
                    acc[rt][i] = fmaf(-mh[i], sv[2 * j + 1], a);
                }
            }
        }
    }

    // ---- the KS partial sums through LDS ----
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][rt][i][lane] = acc[rt][i];
    __syncthreads();
    // wavefront w finishes row tiles w, w + KS, ...
    const int t = t0 + n;
    float *drow = reinterpret_cast<float *>(reinterpret_cast<char *>(p.dst) + (int64_t)t * p.d_nb1);
    for (int rt = wave; rt < RT; rt += KS) {
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float a = 0.0f;
#pragma unroll
            for (int w = 0; w < KS; ++w) a += red[w][rt][i][lane];
            o[i] = a;
        }
        if (t < p.M)
            *reinterpret_cast<float4 *>(drow + r0 + 16 * rt + 4 * g) = make_float4(o[0], o[1], o[2], o[3]);
    }
}

// ---------------------------------------------------------------- op_gemv
// Decode and verify (M <= 4 tokens, MT = 1, 2 or 4 slots): one workgroup of 256
// threads takes 8 rows of W; thread (row, l32) takes half h = l32 & 1 (code
// groups 2h, 2h+1) of super-blocks l32 / 2, l32 / 2 + 16, ... of its row, so a
// row's bytes are read by 32 consecutive threads. Each code is dequantized in
// fp32 and the thread accumulates sum(code * xg) and sum(xg) per sub-block:
// out += d*scale * sum(code * xg) - dmin*min * sum(xg). The gated activations
// and their sub-block sums are built in LDS by the workgroup itself (no
// separate pass), while the thread's first weights are already in flight.
template <int MT>
__global__ __launch_bounds__(256) void op_gemv_kernel(const uint8_t *__restrict__ w, int64_t w_nb1,
                                                      const char *__restrict__ x, int64_t x_nb1,
                                                      const char *__restrict__ gate, int64_t g_nb1, int K, int N,
                                                      int M, float *__restrict__ dst, int64_t d_nb1) {
    // [MT][K/256][kGemvSbStride] gated activations (a super-block's 256 values
    // padded to 260 floats, so the super-blocks a wavefront reads at once sit on
    // different bank quads), then [MT][K/32] sub-block sums
    extern __shared__ __align__(16) float xs[];
    const int tid = threadIdx.x;
    const int nsb = K / kQK;
    const int tstride = nsb * kGemvSbStride;
    float *ssum = xs + MT * tstride;
    const int row = blockIdx.x * 8 + (tid >> 5), l32 = tid & 31, hj = l32 & 1;
    const uint8_t *wr = w + (int64_t)row * w_nb1;
    // header (d, dmin, scales) and the 64 code bytes of groups 2h, 2h+1
    uint4 hdr, qb[4];
    auto load_w = [&](int sb) {
        const uint4 *blk = reinterpret_cast<const uint4 *>(wr + (int64_t)sb * kBlockBytes);
        hdr = blk[0];
#pragma unroll
        for (int c = 0; c < 4; ++c) qb[c] = blk[1 + 4 * hj + c];
    };
    if ((l32 >> 1) < nsb) load_w(l32 >> 1);  // in flight while the activations load
    // 16 values per thread per round, all loads of a round issued before any use
    for (int i0 = 0; i0 < MT * K; i0 += 256 * 16) {
        float v[16], gv[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int i = i0 + 256 * u + tid;
            const int t = i / K, k = i - t * K;
            const bool ok = i < MT * K && t < M;
            v[u] = ok ? reinterpret_cast<const float *>(x + t * x_nb1)[k] : 0.0f;
            gv[u] = ok && gate ? reinterpret_cast<const float *>(gate + t * g_nb1)[k] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int i = i0 + 256 * u + tid;
            const int t = i / K, k = i - t * K;
            if (i < MT * K)
                xs[t * tstride + (k >> 8) * kGemvSbStride + (k & 255)] =
                    gate ? v[u] * (1.0f / (1.0f + expf(-gv[u]))) : v[u];
        }
    }
    __syncthreads();
    for (int i = tid; i < MT * (K / 32); i += 256) {
        const int t = i / (K / 32), sub = i - t * (K / 32);
        const float *src = xs + t * tstride + (sub >> 3) * kGemvSbStride + 32 * (sub & 7);
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) a += src[j];
        ssum[i] = a;
    }
    __syncthreads();
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
    for (int sb = l32 >> 1; sb < nsb; sb += 16) {
        if (sb != (l32 >> 1)) load_w(sb);
        const float d = h2f(hdr.x & 0xffffu), dmin = h2f(hdr.x >> 16);
        const uint32_t *qw = &qb[0].x;  // 16 dwords: code bytes of groups 2h, 2h+1
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int j = 2 * hj + jj;  // sub-blocks 2j (low nibbles) and 2j+1 (high)
            int sc0, mn0, sc1, mn1;
            scale_min(hdr.y, hdr.z, hdr.w, 2 * j, sc0, mn0);
            scale_min(hdr.y, hdr.z, hdr.w, 2 * j + 1, sc1, mn1);
            float dl[MT], dh[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t) dl[t] = dh[t] = 0.0f;
            const float *xl = xs + sb * kGemvSbStride + 64 * j;
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                const uint32_t q = qw[8 * jj + m];  // code bytes 32j + 4m .. +3
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const float4 xa = *reinterpret_cast<const float4 *>(xl + t * tstride + 4 * m);
                    const float4 xb = *reinterpret_cast<const float4 *>(xl + t * tstride + 32 + 4 * m);
                    dl[t] = fmaf((float)(q & 15), xa.x, dl[t]);
                    dl[t] = fmaf((float)((q >> 8) & 15), xa.y, dl[t]);
                    dl[t] = fmaf((float)((q >> 16) & 15), xa.z, dl[t]);
                    dl[t] = fmaf((float)((q >> 24) & 15), xa.w, dl[t]);
                    dh[t] = fmaf((float)((q >> 4) & 15), xb.x, dh[t]);
                    dh[t] = fmaf((float)((q >> 12) & 15), xb.y, dh[t]);
                    dh[t] = fmaf((float)((q >> 20) & 15), xb.z, dh[t]);
                    dh[t] = fmaf((float)(q >> 28), xb.w, dh[t]);
                }
            }
            const float s0 = d * (float)sc0, m0 = dmin * (float)mn0;
            const float s1 = d * (float)sc1, m1 = dmin * (float)mn1;
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const float *st = ssum + t * (K / 32) + sb * kSubs + 2 * j;
                float a = fmaf(s0, dl[t], acc[t]);
                a = fmaf(-m0, st[0], a);
                a = fmaf(s1, dh[t], a);
                acc[t] = fmaf(-m1, st[1], a);
            }
        }
    }
    // the 32 threads of a row are 32 consecutive lanes
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) acc[t] += __shfl_xor(acc[t], o);
    }
    if (l32 == 0 && row < N) {
#pragma unroll
        for (int t = 0; t < MT; ++t)
            if (t < M) reinterpret_cast<float *>(reinterpret_cast<char *>(dst) + t * d_nb1)[row] = acc[t];
    }
}

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

size_t out_proj_workspace(int64_t K, int64_t M) {
    if (M <= kGemvTokens) return 0;  // the decode path keeps its operands in LDS
    const int64_t M16 = (M + 15) / 16 * 16;
    return 2 * al256((size_t)(M16 * K) * 2) + al256((size_t)(K / 32 * M16) * 4) + 256;
}

int launch_out_proj(const sqa_tensor &w, const sqa_tensor &x, const sqa_tensor *gate, const sqa_tensor &dst,
                    void *ws, size_t ws_bytes, hipStream_t s) {
    const int64_t K = w.ne[0], N = w.ne[1], M = x.ne[1];
    if (M == 0 || N == 0) return SQA_OK;
    if (M <= kGemvTokens) {
        static std::once_flag lds_once;  // up to 4 x 16K floats of activations
        static hipError_t lds_err = hipSuccess;
        std::call_once(lds_once, [] {
            for (const void *f : {(const void *)op_gemv_kernel<1>, (const void *)op_gemv_kernel<2>,
                                  (const void *)op_gemv_kernel<4>})
                if (lds_err == hipSuccess)
                    lds_err = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kGemvMaxLds);
        });
        if (lds_err != hipSuccess) return hip_status(lds_err, "out_proj LDS attribute");
        const int mt = M == 1 ? 1 : (M == 2 ? 2 : 4);
        const size_t lds = (size_t)mt * (K / kQK * kGemvSbStride + K / 32) * sizeof(float);
        if (lds > (size_t)kGemvMaxLds)
            return set_error(SQA_ERR_UNSUPPORTED, "out_proj: K = %lld too large for %d tokens", (long long)K, (int)M);
        const int prof = profile_start("out_proj", s);
        const uint8_t *wd = (const uint8_t *)w.data;
        const char *xd = (const char *)x.data, *gd = gate ? (const char *)gate->data : nullptr;
        const int64_t wn = (int64_t)w.nb[1], xn = (int64_t)x.nb[1], gn = gate ? (int64_t)gate->nb[1] : 0;
        float *dd = (float *)dst.data;
        const int64_t dn = (int64_t)dst.nb[1];
        const dim3 grid((unsigned)(N / 8));
        if (mt == 1)
            op_gemv_kernel<1><<<grid, dim3(256), lds, s>>>(wd, wn, xd, xn, gd, gn, (int)K, (int)N, (int)M, dd, dn);
        else if (mt == 2)
            op_gemv_kernel<2><<<grid, dim3(256), lds, s>>>(wd, wn, xd, xn, gd, gn, (int)K, (int)N, (int)M, dd, dn);
        else
            op_gemv_kernel<4><<<grid, dim3(256), lds, s>>>(wd, wn, xd, xn, gd, gn, (int)K, (int)N, (int)M, dd, dn);
        profile_stop(prof, s);
        return hip_status(hipGetLastError(), "out_proj launch");
    }
    const int64_t M16 = (M + 15) / 16 * 16;
    const size_t need = out_proj_workspace(K, M);
    if (!ws || ws_bytes < need)
        return set_error(SQA_ERR_WORKSPACE, "out_proj: workspace %zu bytes < %zu needed", ws_bytes, need);
    uint8_t *base = reinterpret_cast<uint8_t *>(((uintptr_t)ws + 255) & ~(uintptr_t)255);
    uint16_t *xh = reinterpret_cast<uint16_t *>(base);
    uint16_t *xl = reinterpret_cast<uint16_t *>(base + al256((size_t)(M16 * K) * 2));
    float *S = reinterpret_cast<float *>(base + 2 * al256((size_t)(M16 * K) * 2));

    const int prof = profile_start("out_proj", s);
    const int64_t nprep = K / 32 * M16;
    const bool vec = (uintptr_t)x.data % 16 == 0 && x.nb[1] % 16 == 0 &&
                     (!gate || ((uintptr_t)gate->data % 16 == 0 && gate->nb[1] % 16 == 0));
    const dim3 pg((unsigned)((nprep + 255) / 256));
    const char *xd = (const char *)x.data, *gd = gate ? (const char *)gate->data : nullptr;
    const int64_t xn = (int64_t)x.nb[1], gn = gate ? (int64_t)gate->nb[1] : 0;
    if (gate && vec)
        op_prep_kernel<true, true><<<pg, dim3(256), 0, s>>>(xd, xn, gd, gn, (int)K, (int)M, (int)M16, xh, xl, S);
    else if (gate)
        op_prep_kernel<true, false><<<pg, dim3(256), 0, s>>>(xd, xn, gd, gn, (int)K, (int)M, (int)M16, xh, xl, S);
    else if (vec)
        op_prep_kernel<false, true><<<pg, dim3(256), 0, s>>>(xd, xn, gd, gn, (int)K, (int)M, (int)M16, xh, xl, S);
    else
        op_prep_kernel<false, false><<<pg, dim3(256), 0, s>>>(xd, xn, gd, gn, (int)K, (int)M, (int)M16, xh, xl, S);
    GemmParams p;
    p.w = (const uint8_t *)w.data;
    p.w_nb1 = (int64_t)w.nb[1];
    p.xh = xh;
    p.xl = xl;
    p.S = S;
    p.K = (int)K;
    p.N = (int)N;
    p.M = (int)M;
    p.M16 = (int)M16;
    p.dst = (float *)dst.data;
    p.d_nb1 = (int64_t)dst.nb[1];
    // one 16-token tile per workgroup; for decode (one token tile) 16 rows and 16
    // wavefronts that take one super-block each, else 64 rows and 4 wavefronts
    if (M16 == 16 || N % 64 != 0)
        op_gemm_kernel<16, 1><<<dim3((unsigned)(N / 16), (unsigned)(M16 / 16)), dim3(1024), 0, s>>>(p);
    else
        op_gemm_kernel<4, 4><<<dim3((unsigned)(N / 64), (unsigned)(M16 / 16)), dim3(256), 0, s>>>(p);
    profile_stop(prof, s);
    return hip_status(hipGetLastError(), "out_proj launch");
}

}  // namespace sqa
