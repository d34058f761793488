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

__device__ __forceinline__ float h2f(uint32_t bits) {
    _Float16 h;
    const uint16_t b = (uint16_t)bits;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// ---------------------------------------------------------------- op_prep
// One thread per 8 values (a quarter sub-block) of one token: xg = x *
// sigmoid(gate) as an fp16 hi + lo pair, and through the lane quad the
// sub-block sum S (f32) and its hi + lo slots for the min MFMA of op_gemm2.
// Tokens M..Mp-1 and the sub-blocks that pad K to whole groups of four
// super-blocks are zeros. x (and gate) rows are 16-byte aligned when VEC.
template <bool GATE, bool VEC>
__global__ __launch_bounds__(256) void op_prep_kernel(const char *__restrict__ x, int64_t x_nb1,
                                                      const char *__restrict__ gate, int64_t g_nb1, int K, int M,
                                                      int Mp, int nq, uint16_t *__restrict__ xh,
                                                      uint16_t *__restrict__ xl, float *__restrict__ S,
                                                      uint16_t *__restrict__ sp) {
    const int subs = K / 32, psubs = 32 * nq;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)Mp * psubs * 4) return;  // whole quads: the total is a multiple of 4
    const int qtr = (int)(idx & 3);
    const int64_t ts = idx >> 2;
    const int t = (int)(ts / psubs), s = (int)(ts - (int64_t)t * psubs);
    float v[8], gv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = gv[j] = 0.0f;
    if (t < M && s < subs) {
        const float *xr = reinterpret_cast<const float *>(x + t * x_nb1) + 32 * s + 8 * qtr;
        const float *gr = GATE ? reinterpret_cast<const float *>(gate + t * g_nb1) + 32 * s + 8 * qtr : nullptr;
        if (VEC) {
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const float4 a = reinterpret_cast<const float4 *>(xr)[c];
                v[4 * c] = a.x, v[4 * c + 1] = a.y, v[4 * c + 2] = a.z, v[4 * c + 3] = a.w;
                if (GATE) {
                    const float4 b = reinterpret_cast<const float4 *>(gr)[c];
                    gv[4 * c] = b.x, gv[4 * c + 1] = b.y, gv[4 * c + 2] = b.z, gv[4 * c + 3] = b.w;
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                v[j] = xr[j];
                if (GATE) gv[j] = gr[j];
            }
        }
        if (GATE) {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = v[j] * (1.0f / (1.0f + expf(-gv[j])));
        }
    }
    float sum = 0.0f;
    uint16_t hb[8], lb[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        sum += v[j];
        float a = v[j];
        // opaque: one fp32 value feeds both the stored hi and the hi subtracted for lo
        asm volatile("" : "+v"(a));
        const _Float16 h = (_Float16)a;
        const _Float16 l = (_Float16)(a - (float)h);
        __builtin_memcpy(&hb[j], &h, 2);
        __builtin_memcpy(&lb[j], &l, 2);
    }
    // sum over the quad (quad_perm [1,0,3,2], then [2,3,0,1])
    sum += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(sum), 0xB1, 0xf, 0xf, false));
    sum += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(sum), 0x4E, 0xf, 0xf, false));
    if (qtr == 0) {
        // S hi + lo in the slot order of the min MFMA: group q of 4 super-blocks,
        // slot 8g + e = sub-block 2g + (e & 1) of super-block 4q + (e >> 1)
        const int sb = s >> 3, sub = s & 7;
        const int slot = 8 * (sub >> 1) + 2 * (sb & 3) + (sub & 1);
        float a = sum;
        asm volatile("" : "+v"(a));
        const _Float16 h = (_Float16)a;
        const _Float16 l = (_Float16)(a - (float)h);
        uint16_t *o = sp + ((int64_t)t * nq + (sb >> 2)) * 64 + slot;
        __builtin_memcpy(o, &h, 2);
        __builtin_memcpy(o + 32, &l, 2);
        if (s < subs) S[(int64_t)t * subs + s] = sum;  // [token][sub-block]
    }
    if (s >= subs) return;
    uint4 a, b;
    __builtin_memcpy(&a, hb, 16);
    __builtin_memcpy(&b, lb, 16);
    *reinterpret_cast<uint4 *>(xh + (int64_t)t * K + 32 * s + 8 * qtr) = a;
    *reinterpret_cast<uint4 *>(xl + (int64_t)t * K + 32 * s + 8 * qtr) = b;
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

// ---------------------------------------------------------------- op_gemm2
// Larger token counts: a workgroup of 8 wavefronts owns 128 rows of W
// (wavefront w: rows 16w..16w+15) and 32 tokens (two token tiles of 16).
//   * Per super-block and row tile, the A operand of sub-block s is code *
//     scale_s as an fp16 subnormal: an integer of at most 15 * 63 = 945, i.e.
//     exactly code * scale * 2^-24 (one v_mul_u32_u24 scales the two codes of a
//     dword, as the halves cannot carry into each other). The 8 sub-blocks then
//     accumulate into one MFMA chain C = 2^-24 sum_k scale * code * x against x
//     hi and lo, and acc += d 2^24 C once per super-block.
//   * The min term sum_sb dmin * sum_s min_s * S_s runs on the MFMA as well:
//     A = dmin * min as an fp16 hi + lo pair (17 bits) against B = S hi + lo,
//     where k slot 8g + e of a group of four super-blocks holds sub-block
//     2g + (e & 1) of super-block 4q + (e >> 1), so that each lane fills its
//     two slots from the super-block it already holds.
//   * Everything comes HBM -> LDS by DMA, double buffered: half a super-block
//     of activations (128 values x 32 tokens, hi and lo: 16 KB, chunk c of
//     token row t at c ^ (t & 15)), the 128 weight rows' super-block (18 KB)
//     and, one group of four super-blocks ahead, the S hi/lo slots (4 KB).
//     Each wait counts the wavefront's younger DMAs, so the stages in flight
//     are not waited for.
constexpr int kG2Rows = 128;
constexpr int kG2Tok = 32;
constexpr int kG2RT = 1;                            // row tiles of 16 per wavefront
constexpr int kG2Waves = kG2Rows / (16 * kG2RT);   // 8: two wavefronts per SIMD
constexpr int kG2XInst = 16 / kG2Waves;             // activation DMA instructions per wavefront
constexpr int kG2Half = kG2Tok * 512;        // activation bytes of half a super-block
constexpr int kG2WBytes = kG2Rows * kBlockBytes;  // 18432
constexpr int kG2WInst = kG2WBytes / 1024;   // 18 DMA instructions
constexpr int kG2WPer = (kG2WInst + kG2Waves - 1) / kG2Waves;
constexpr int kG2SBytes = kG2Tok * 128;      // S slots of one group: [32 tokens][hi 64 B | lo 64 B]
constexpr int kG2XAhead = 1;                  // activation halves in flight ahead of the one in use
constexpr int kG2WAhead = 1;                  // weight super-blocks in flight ahead of the one in use
constexpr int kG2XBufs = kG2XAhead + 1;
constexpr int kG2WBufs = kG2WAhead + 1;
static_assert(2 * kG2WAhead >= kG2XAhead, "a weight stage is issued no later than the activations of its first half");
static_assert(kG2XAhead == 1, "the per-half wait drains every DMA: the activations of the next half are issued last");
static_assert(kG2WBytes % 1024 == 0, "weight stage in whole DMA instructions");

// 16 bytes per lane from sbase + voff into LDS at m0 + 16 * lane, asynchronously
// (the caller waits with s_waitcnt vmcnt); sbase and m0 are wave-uniform.
__device__ __forceinline__ void dma16(uint32_t voff, const void *sbase, uint32_t m0v) {
    const uint64_t b = (uint64_t)(uintptr_t)sbase;
    const uint64_t bs = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(b >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    const uint32_t ms = (uint32_t)__builtin_amdgcn_readfirstlane((int)m0v);
    // m0 as an operand: the compiler writes it and knows it holds the LDS base
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(bs), "{m0}"(ms) : "memory");
}

struct Gemm2Params {
    const uint8_t *w;
    int64_t w_nb1;
    const uint16_t *x;  // xh [Mp][K]; xl starts xl_off bytes later
    uint32_t xl_off;
    const uint16_t *sp;  // [Mp][nq][64] fp16 S hi (32 slots) then lo (32 slots)
    int K, N, M, Mp, nq;
    float *dst;
    int64_t d_nb1;
};

// 77824 bytes of dynamic LDS: two workgroups per CU (deeper rings measured slower,
// 48 vs 36 us at 512 tokens, as they halve the workgroups a CU holds)
constexpr int kG2Lds = kG2XBufs * kG2Half + kG2WBufs * kG2WBytes + 2 * kG2SBytes;

__global__ __launch_bounds__(64 * kG2Waves) void op_gemm2_kernel(Gemm2Params p) {
    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t(*xs)[kG2Half] = reinterpret_cast<uint8_t(*)[kG2Half]>(lds);
    uint8_t(*wb)[kG2WBytes] = reinterpret_cast<uint8_t(*)[kG2WBytes]>(lds + kG2XBufs * kG2Half);
    uint8_t *sb_lds = lds + kG2XBufs * kG2Half + kG2WBufs * kG2WBytes;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    // workgroups go round-robin to the 8 XCDs: give each XCD whole token tiles
    // (every row block of them), so an XCD's L2 serves its activations to all
    // its row blocks
    int bx = (int)blockIdx.x, by = (int)blockIdx.y;
    {
        const int nx = (int)gridDim.x, ny = (int)gridDim.y;
        if (ny % 8 == 0) {
            const int id = bx + nx * by, k = id / 8;
            by = (id % 8) * (ny / 8) + k / nx;
            bx = k % nx;
        }
    }
    const int row0 = bx * kG2Rows;
    const int t0 = by * kG2Tok;
    const int nsb = p.K / kQK;
    const uint32_t xs0 = (uint32_t)(uintptr_t)&xs[0][0], wb0 = (uint32_t)(uintptr_t)&wb[0][0];
    const uint32_t sb0 = (uint32_t)(uintptr_t)&sb_lds[0];

    // ---- DMA plans (wave-uniform bases, per-lane offsets) ----
    // activations: instruction i = kG2XInst * wave + r covers tokens 2i, 2i+1: lane ->
    // token 2i + (lane >> 5), hi/lo (lane >> 4) & 1, LDS chunk lane & 15
    auto issue_x = [&](int h, int buf) {
#pragma unroll
        for (int r = 0; r < kG2XInst; ++r) {
            const int i = kG2XInst * wave + r;
            const int t = 2 * i + (lane >> 5);
            const uint32_t off = (uint32_t)((lane >> 4) & 1) * p.xl_off +
                                 (uint32_t)((t0 + t) * p.K + 128 * h) * 2u + 16u * (uint32_t)((lane & 15) ^ (t & 15));
            dma16(off, p.x, xs0 + (uint32_t)(buf * kG2Half + 1024 * i));
        }
    };
    // weights: chunk id = 64 * i + lane -> row id / 9, chunk id % 9 (rows past N
    // read row 0 and are never stored)
    uint32_t woff[kG2WPer];
#pragma unroll
    for (int r = 0; r < kG2WPer; ++r) {
        const int i = kG2Waves * r + wave;
        const int id = 64 * (i < kG2WInst ? i : 0) + lane;
        const int row = id / 9, ch = id - 9 * (id / 9);
        const int grow = row0 + row < p.N ? row0 + row : 0;
        woff[r] = (uint32_t)((int64_t)grow * p.w_nb1) + 16u * (uint32_t)ch;
    }
    auto issue_w = [&](int sb, int buf) {
#pragma unroll
        for (int r = 0; r < kG2WPer; ++r) {
            const int i = kG2Waves * r + wave;
            if (i < kG2WInst) dma16(woff[r], p.w + (int64_t)sb * kBlockBytes, wb0 + (uint32_t)(buf * kG2WBytes + 1024 * i));
        }
    };
    // S slots of group q into buffer q & 1: wavefront w < 4 copies tokens
    // 8w..8w+7 (128 bytes each)
    auto issue_s = [&](int q) {
        if (wave >= kG2Tok / 8) return;
        const int t = 8 * wave + (lane >> 3);
        const uint32_t off = (uint32_t)(((t0 + t) * p.nq + q) * 128 + 16 * (lane & 7));
        dma16(off, p.sp, sb0 + (uint32_t)((q & 1) * kG2SBytes + 1024 * wave));
    };

    floatx4 acc[kG2RT][2], accm[kG2RT][2];
#pragma unroll
    for (int rt = 0; rt < kG2RT; ++rt)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) acc[rt][tt] = accm[rt][tt] = floatx4{0.f, 0.f, 0.f, 0.f};
    uint32_t amh[kG2RT][4], aml[kG2RT][4];  // A of the min MFMA per row tile: slots 2u, 2u+1 in dword u
#pragma unroll
    for (int rt = 0; rt < kG2RT; ++rt)
#pragma unroll
        for (int u = 0; u < 4; ++u) amh[rt][u] = aml[rt][u] = 0u;

    // Issue order: weights of super-blocks 0..kG2WAhead-1, S of group 0 and
    // activation halves 0..kG2XAhead-1 first; then at the start of half k the
    // weights of super-block k/2 + kG2WAhead (even k), the S of group k/8 + 1 (k a
    // multiple of 8) and activation half k + kG2XAhead. A stage is read only after
    // the wait for activation half h, and every DMA it needs was issued no later
    // than that half's.
    const int nh = 2 * nsb, ngrp = (nsb + 3) / 4;
    for (int sb = 0; sb < kG2WAhead && sb < nsb; ++sb) issue_w(sb, sb);
    issue_s(0);
    for (int k = 0; k < kG2XAhead && k < nh; ++k) issue_x(k, k);
    for (int sb = 0; sb < nsb; ++sb) {
        const int u = sb & 3;
        const uint8_t *wcur = &wb[sb % kG2WBufs][0];
        int sc[kG2RT][8];
        floatx4 dq[kG2RT];  // d 2^24 of C rows 4g..4g+3
        floatx4 C[kG2RT][2];
#pragma unroll
        for (int rt = 0; rt < kG2RT; ++rt)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) C[rt][tt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int h = 2 * sb + hh;
            // this wavefront's DMAs for half h have landed; the barrier publishes
            // every wavefront's and retires the buffers the next DMAs overwrite.
            // Half h's activations were the last DMA issued (at the start of half
            // h - 1, after that half's weights and S slots), so the wait drains all.
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (hh == 0 && sb + kG2WAhead < nsb) issue_w(sb + kG2WAhead, (sb + kG2WAhead) % kG2WBufs);
            if (hh == 0 && u == 0 && (sb >> 2) + 1 < ngrp) issue_s((sb >> 2) + 1);
            if (h + kG2XAhead < nh) issue_x(h + kG2XAhead, (h + kG2XAhead) % kG2XBufs);
            if (hh == 0) {
                // scales of A row n (every sub-block), d of C rows 4g..4g+3, and
                // this lane's two min slots (sub-blocks 2g, 2g+1)
#pragma unroll
                for (int rt = 0; rt < kG2RT; ++rt) {
                    const uint8_t *hrow = wcur + (16 * kG2RT * wave + 16 * rt + n) * kBlockBytes;
                    const uint4 hd = *reinterpret_cast<const uint4 *>(hrow);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        int mn;
                        scale_min(hd.y, hd.z, hd.w, e, sc[rt][e], mn);
                    }
                    int m0, m1, unused;
                    scale_min(hd.y, hd.z, hd.w, 2 * g, unused, m0);
                    scale_min(hd.y, hd.z, hd.w, 2 * g + 1, unused, m1);
                    const float dmin = h2f(hd.x >> 16);
                    float a0 = dmin * (float)m0, a1 = dmin * (float)m1;  // exact: 11 x 6 bits
                    asm volatile("" : "+v"(a0), "+v"(a1));
                    const _Float16 h0 = (_Float16)a0, h1 = (_Float16)a1;
                    const _Float16 l0 = (_Float16)(a0 - (float)h0), l1 = (_Float16)(a1 - (float)h1);
                    uint16_t b[4];
                    __builtin_memcpy(&b[0], &h0, 2);
                    __builtin_memcpy(&b[1], &h1, 2);
                    __builtin_memcpy(&b[2], &l0, 2);
                    __builtin_memcpy(&b[3], &l1, 2);
                    const uint32_t hw = (uint32_t)b[0] | ((uint32_t)b[1] << 16);
                    const uint32_t lw = (uint32_t)b[2] | ((uint32_t)b[3] << 16);
#pragma unroll
                    for (int uu = 0; uu < 4; ++uu) {
                        amh[rt][uu] = u == uu ? hw : amh[rt][uu];
                        aml[rt][uu] = u == uu ? lw : aml[rt][uu];
                    }
                    float dv[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        dv[i] = h2f(*reinterpret_cast<const uint16_t *>(wcur + (16 * kG2RT * wave + 16 * rt + 4 * g + i) * kBlockBytes));
                    dq[rt] = floatx4{dv[0], dv[1], dv[2], dv[3]} * 16777216.0f;
                }
            }
            const uint8_t *xb = &xs[h % kG2XBufs][0];
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int j = 2 * hh + jj;  // code group: sub-blocks 2j (low nibbles), 2j+1 (high)
                half8 alo[kG2RT], ahi[kG2RT];
#pragma unroll
                for (int rt = 0; rt < kG2RT; ++rt) {
                    const uint2 qv = *reinterpret_cast<const uint2 *>(wcur + (16 * kG2RT * wave + 16 * rt + n) * kBlockBytes +
                                                                      16 + 32 * j + 8 * g);
                    uint32_t sp4[4];  // bytes 2m, 2m+1 spread to the two halves of dword m
                    sp4[0] = __builtin_amdgcn_perm(0u, qv.x, 0x0c010c00u);
                    sp4[1] = __builtin_amdgcn_perm(0u, qv.x, 0x0c030c02u);
                    sp4[2] = __builtin_amdgcn_perm(0u, qv.y, 0x0c010c00u);
                    sp4[3] = __builtin_amdgcn_perm(0u, qv.y, 0x0c030c02u);
                    uint32_t lo[4], hi[4];
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        lo[m] = __umul24(sp4[m] & 0x000F000Fu, (uint32_t)sc[rt][2 * j]);
                        hi[m] = __umul24((sp4[m] >> 4) & 0x000F000Fu, (uint32_t)sc[rt][2 * j + 1]);
                    }
                    __builtin_memcpy(&alo[rt], lo, 16);
                    __builtin_memcpy(&ahi[rt], hi, 16);
                }
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    const int tr = 16 * tt + n;
                    const uint8_t *row = xb + 512 * tr;
                    const int c0 = 8 * jj + g, c1 = 8 * jj + 4 + g;
                    half8 bh0, bl0, bh1, bl1;
                    {
                        const uint4 a = *reinterpret_cast<const uint4 *>(row + 16 * (c0 ^ (tr & 15)));
                        const uint4 b = *reinterpret_cast<const uint4 *>(row + 256 + 16 * (c0 ^ (tr & 15)));
                        const uint4 c = *reinterpret_cast<const uint4 *>(row + 16 * (c1 ^ (tr & 15)));
                        const uint4 d = *reinterpret_cast<const uint4 *>(row + 256 + 16 * (c1 ^ (tr & 15)));
                        __builtin_memcpy(&bh0, &a, 16);
                        __builtin_memcpy(&bl0, &b, 16);
                        __builtin_memcpy(&bh1, &c, 16);
                        __builtin_memcpy(&bl1, &d, 16);
                    }
#pragma unroll
                    for (int rt = 0; rt < kG2RT; ++rt) {
                        C[rt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[rt], bh0, C[rt][tt], 0, 0, 0);
                        C[rt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[rt], bl0, C[rt][tt], 0, 0, 0);
                        C[rt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[rt], bh1, C[rt][tt], 0, 0, 0);
                        C[rt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[rt], bl1, C[rt][tt], 0, 0, 0);
                    }
                }
            }
        }
#pragma unroll
        for (int rt = 0; rt < kG2RT; ++rt)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[rt][tt][i] = fmaf(dq[rt][i], C[rt][tt][i], acc[rt][tt][i]);
        // min MFMA at the end of a group of four super-blocks (or of K)
        if (u == 3 || sb == nsb - 1) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const uint8_t *srow = sb_lds + ((sb >> 2) & 1) * kG2SBytes + 128 * (16 * tt + n);
                const uint4 bhv = *reinterpret_cast<const uint4 *>(srow + 16 * g);
                const uint4 blv = *reinterpret_cast<const uint4 *>(srow + 64 + 16 * g);
                half8 bh, bl;
                __builtin_memcpy(&bh, &bhv, 16);
                __builtin_memcpy(&bl, &blv, 16);
#pragma unroll
                for (int rt = 0; rt < kG2RT; ++rt) {
                    half8 ah, al;
                    __builtin_memcpy(&ah, amh[rt], 16);
                    __builtin_memcpy(&al, aml[rt], 16);
                    accm[rt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, accm[rt][tt], 0, 0, 0);
                    accm[rt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl, accm[rt][tt], 0, 0, 0);
                    accm[rt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh, accm[rt][tt], 0, 0, 0);
                }
            }
#pragma unroll
            for (int rt = 0; rt < kG2RT; ++rt)
#pragma unroll
                for (int uu = 0; uu < 4; ++uu) amh[rt][uu] = aml[rt][uu] = 0u;
        }
    }
    // ---- out[token][rows 4g..4g+3] = acc - accm ----
#pragma unroll
    for (int rt = 0; rt < kG2RT; ++rt) {
        const int r = row0 + 16 * kG2RT * wave + 16 * rt;
        if (r >= p.N) continue;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int t = t0 + 16 * tt + n;
            if (t >= p.M) continue;
            float *drow = reinterpret_cast<float *>(reinterpret_cast<char *>(p.dst) + (int64_t)t * p.d_nb1);
            const floatx4 o = acc[rt][tt] - accm[rt][tt];
            *reinterpret_cast<float4 *>(drow + r + 4 * g) = make_float4(o[0], o[1], o[2], o[3]);
        }
    }
}

// ---------------------------------------------------------------- op_gemv
// Decode and verify (M <= 4 tokens, MT = 1, 2 or 4 slots): one workgroup of
// kGemvThreads threads takes kGemvRows rows of W. Thread t owns the 8
// activations k = 8t .. 8t + 7 (and the same slice of every further
// 8 * kGemvThreads values of K) for all of those rows, so it loads its slice of
// x and gate once and, for each row, the slice's 8 code bytes, all before it
// uses any of them: one memory latency, then arithmetic, then one reduction.
// The four threads of a lane quad share one 32-value sub-block: each loads and
// unpacks the super-block headers of two of the 8 rows, and the quad
// broadcasts the rows' scales.
//   Value 64j + 16h2 + i of a super-block sits in byte 32j + 16(h2 & 1) + i of
//   its codes, low nibble for h2 < 2, high for h2 >= 2; sub-block 2j + (h2 >> 1).
// Per row and token: out += d * scale * sum(code * xg) - dmin * min * sum(xg).
// The codes enter v_fma_mix as fp16 subnormals, two per v_and, against the
// fp32 activations, so every product is exact: a low nibble left in bits 0-3
// of an fp16 is code * 2^-24, a high nibble left in bits 4-7 is code * 2^-20,
// and the 2^24 or 2^20 goes into the scale. The gate's sigmoid is 1/(1 + 2^(-g
// log2 e)) from the hardware exp2 and reciprocal (about 2 ulp). The partial
// sums of the (row, token) pairs are added by recursive halving inside each
// wavefront (lane swaps and DPP moves, each lane ending with one pair's sum),
// then across the wavefronts through LDS. VEC: x (and gate) rows are 16-byte
// aligned and read four floats at a time.
// Lane K of each quad's x in all four lanes of the quad (quad_perm [K,K,K,K]).
template <int K>
__device__ __forceinline__ float quad_bcast(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), K * 0x55, 0xf, 0xf, false));
}

// One halving step of the GEMV's wavefront sum (below): values a[0 .. 2N) to
// a[0 .. N), the lane with `up` clear keeping the lower half, plus the
// partner's copy of the kept half moved by the DPP control CTRL.
template <int N, int CTRL>
__device__ __forceinline__ void halve_dpp(float *a, bool up) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
        const float keep = up ? a[N + j] : a[j];
        const float give = up ? a[j] : a[N + j];
        a[j] = keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(give), CTRL, 0xf, 0xf, false));
    }
}

constexpr int kGemvRows = 8;
constexpr int kGemvThreads = 512;
template <int MT, bool VEC>
__global__ __launch_bounds__(kGemvThreads) void op_gemv_kernel(const uint8_t *__restrict__ w, int64_t w_nb1,
                                                               const char *__restrict__ x, int64_t x_nb1,
                                                               const char *__restrict__ gate, int64_t g_nb1, int K,
                                                               int N, int M, float *__restrict__ dst, int64_t d_nb1) {
    constexpr int R = kGemvRows, W = kGemvThreads / 64;
    __shared__ float red[W][R * MT];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = blockIdx.x * R;
    float acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[r][t] = 0.0f;
    // x * code + acc, the code in the low (SEL 0) or high (SEL 1) fp16 half of c
#define SQA_MIX(ACC, X, C, SEL)                                                                           \
    asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[0," #SEL ",0] op_sel_hi:[0,1,0]" : "+v"(ACC) : "v"(X), "v"(C))
    for (int k0 = 8 * tid; k0 < K; k0 += 8 * kGemvThreads) {
        const int sb = k0 >> 8, v = k0 & 255, j = v >> 6, h2 = (v >> 4) & 3;
        const bool hi_nib = h2 >= 2;
        const uint32_t nib = hi_nib ? 0x00F000F0u : 0x000F000Fu;  // codes of bytes 0, 2 of a dword
        const float cscale = hi_nib ? 1048576.0f : 16777216.0f;     // 2^20 or 2^24
        const int s = 2 * j + (h2 >> 1);                            // sub-block
        const int cb = 16 + 32 * j + 16 * (h2 & 1) + (v & 8);       // the slice's first code byte
        // weights first (8 code bytes of every row; the super-block headers of
        // rows 2 qd and 2 qd + 1 only, see below), then the activations
        const int qd = lane & 3;  // the lane quad shares one sub-block (32 values)
        uint4 hdr[2];
        uint2 q[R];
#pragma unroll
        for (int u = 0; u < 2; ++u)
            hdr[u] = *reinterpret_cast<const uint4 *>(w + (int64_t)(row0 + 2 * qd + u) * w_nb1 +
                                                      (int64_t)sb * kBlockBytes);
#pragma unroll
        for (int r = 0; r < R; ++r)
            q[r] = *reinterpret_cast<const uint2 *>(w + (int64_t)(row0 + r) * w_nb1 + (int64_t)sb * kBlockBytes + cb);
        float xg[MT][8];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const bool ok = t < M;
            const float *xr = reinterpret_cast<const float *>(x + (ok ? t : 0) * x_nb1) + k0;
            const float *gr = gate ? reinterpret_cast<const float *>(gate + (ok ? t : 0) * g_nb1) + k0 : nullptr;
            float gv[8];
            if (VEC) {
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const float4 a = reinterpret_cast<const float4 *>(xr)[c];
                    xg[t][4 * c] = a.x, xg[t][4 * c + 1] = a.y, xg[t][4 * c + 2] = a.z, xg[t][4 * c + 3] = a.w;
                    if (gr) {
                        const float4 b = reinterpret_cast<const float4 *>(gr)[c];
                        gv[4 * c] = b.x, gv[4 * c + 1] = b.y, gv[4 * c + 2] = b.z, gv[4 * c + 3] = b.w;
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    xg[t][i] = xr[i];
                    if (gr) gv[i] = gr[i];
                }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (gr)
                    xg[t][i] *= __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * gv[i]));
                xg[t][i] = ok ? xg[t][i] : 0.0f;
            }
        }
        // d * scale * 2^24 (or 2^20) and dmin * min of sub-block s for the 8 rows:
        // the four lanes of a quad share s, so lane qd unpacks rows 2 qd and
        // 2 qd + 1 (ggml's get_scale_min_k4, branch-free) and the quad
        // broadcasts them (quad_perm [k,k,k,k])
        float dsu[2], dmu[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const uint32_t q0 = hdr[u].y, q1 = hdr[u].z, q2 = hdr[u].w;
            const uint32_t lo_sh = 8u * (uint32_t)(s & 3);
            const uint32_t sc_lo = (q0 >> lo_sh) & 63u, mn_lo = (q1 >> lo_sh) & 63u;
            const uint32_t sc_hi = ((q2 >> lo_sh) & 15u) | (((q0 >> (lo_sh + 6u)) & 3u) << 4);
            const uint32_t mn_hi = ((q2 >> (lo_sh + 4u)) & 15u) | (((q1 >> (lo_sh + 6u)) & 3u) << 4);
            const uint32_t sc = s < 4 ? sc_lo : sc_hi, mn = s < 4 ? mn_lo : mn_hi;
            dsu[u] = h2f(hdr[u].x & 0xffffu) * (float)sc * cscale;
            dmu[u] = h2f(hdr[u].x >> 16) * (float)mn;
        }
        float ds[R], dm[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int k = r >> 1;
            ds[r] = k == 0 ? quad_bcast<0>(dsu[r & 1]) : k == 1 ? quad_bcast<1>(dsu[r & 1])
                  : k == 2 ? quad_bcast<2>(dsu[r & 1]) : quad_bcast<3>(dsu[r & 1]);
            dm[r] = k == 0 ? quad_bcast<0>(dmu[r & 1]) : k == 1 ? quad_bcast<1>(dmu[r & 1])
                  : k == 2 ? quad_bcast<2>(dmu[r & 1]) : quad_bcast<3>(dmu[r & 1]);
        }
        float sx[MT];  // sum of this slice's activations (the min term)
#pragma unroll
        for (int t = 0; t < MT; ++t)
            sx[t] = ((xg[t][0] + xg[t][1]) + (xg[t][2] + xg[t][3])) + ((xg[t][4] + xg[t][5]) + (xg[t][6] + xg[t][7]));
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t qw[2] = {q[r].x, q[r].y};
            float dot[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t) dot[t] = 0.0f;
#pragma unroll
            for (int m = 0; m < 2; ++m) {  // bytes 4m .. 4m+3 of the slice: values 4m .. 4m+3
                const uint32_t c02 = qw[m] & nib;         // values 4m, 4m + 2
                const uint32_t c13 = (qw[m] >> 8) & nib;  // values 4m + 1, 4m + 3
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    SQA_MIX(dot[t], xg[t][4 * m], c02, 0);
                    SQA_MIX(dot[t], xg[t][4 * m + 1], c13, 0);
                    SQA_MIX(dot[t], xg[t][4 * m + 2], c02, 1);
                    SQA_MIX(dot[t], xg[t][4 * m + 3], c13, 1);
                }
            }
#pragma unroll
            for (int t = 0; t < MT; ++t) acc[r][t] = fmaf(-dm[r], sx[t], fmaf(ds[r], dot[t], acc[r][t]));
        }
    }
#undef SQA_MIX
    // Sum of the V = R * MT values (index r * MT + t) over the wavefront by
    // recursive halving: each step pairs lanes that differ in one bit; the lane
    // with the bit clear keeps the lower half of its values, the other the
    // upper half, each adding its partner's copy of the half it keeps. Lane bits
    // 5 and 4 swap halves between rows (permlane32 / permlane16 swaps, which
    // exchange the upper 32 lanes of the first operand with the lower 32 of the
    // second and the odd rows of the first with the even rows of the second: a
    // swap and an add per pair), bit 3 pairs lane ^ 8 (row_ror:8), bit 2 lane ^ 7
    // (row_half_mirror: the same bits above 2), bit 1 lane ^ 2 (quad_perm), and
    // the bits left over are summed in place. Lane l then holds the full sum of
    // index l >> (6 - log2 V): V - 1 swaps or DPP moves instead of 6 V.
    constexpr int V = R * MT;
    static_assert(V == 8 || V == 16 || V == 32, "halving steps below");
    float a[V];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) a[r * MT + t] = acc[r][t];
#pragma unroll
    for (int j = 0; j < V / 2; ++j) {  // bit 5
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[j]), __float_as_uint(a[V / 2 + j]), false, false);
        a[j] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
#pragma unroll
    for (int j = 0; j < V / 4; ++j) {  // bit 4
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[j]), __float_as_uint(a[V / 4 + j]), false, false);
        a[j] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    halve_dpp<V / 8, 0x128>(a, (lane & 8) != 0);                   // bit 3, lane ^ 8 (row_ror:8)
    if constexpr (V >= 16) halve_dpp<V / 16, 0x141>(a, (lane & 4) != 0);  // bit 2, lane ^ 7 (row_half_mirror)
    if constexpr (V >= 32) halve_dpp<V / 32, 0x4e>(a, (lane & 2) != 0);   // bit 1, lane ^ 2 (quad_perm [2,3,0,1])
    float s = a[0];
    s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0xb1, 0xf, 0xf, false));  // lane ^ 1
    if constexpr (V <= 16) s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x4e, 0xf, 0xf, false));
    if constexpr (V <= 8) s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x141, 0xf, 0xf, false));
    constexpr int kSpan = 64 / V;  // lanes that share an index
    if ((lane & (kSpan - 1)) == 0) red[wave][lane / kSpan] = s;
    __syncthreads();
    if (tid < R * MT) {
        const int r = tid / MT, t = tid - r * MT;
        float o = 0.0f;
#pragma unroll
        for (int wv = 0; wv < W; ++wv) o += red[wv][tid];
        if (t < M && row0 + r < N) reinterpret_cast<float *>(reinterpret_cast<char *>(dst) + t * d_nb1)[row0 + r] = o;
    }
}

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workspace of the GEMM path: tokens padded to Mp (a multiple of 32), xh and xl
// [Mp][K] fp16, S [Mp][K/32] f32, the S hi/lo slots [Mp][nq][64] fp16.
struct OpLayout {
    int64_t Mp, nq;
    size_t xl, s, sp, total;
};
OpLayout op_layout(int64_t K, int64_t M) {
    OpLayout l;
    l.Mp = (M + kG2Tok - 1) / kG2Tok * kG2Tok;
    l.nq = (K / kQK + 3) / 4;
    l.xl = al256((size_t)(l.Mp * K) * 2);
    l.s = 2 * l.xl;
    l.sp = l.s + al256((size_t)(l.Mp * (K / 32)) * 4);
    l.total = l.sp + al256((size_t)(l.Mp * l.nq * 64) * 2) + 256;
    return l;
}

}  // namespace

size_t out_proj_workspace(int64_t K, int64_t M) {
    if (M <= kGemvTokens) return 0;  // the decode path keeps its operands in registers
    return op_layout(K, M).total;
}

int launch_out_proj(const sqa_tensor &w, const sqa_tensor &x, const sqa_tensor *gate, const sqa_tensor &dst,
                    void *ws, size_t ws_bytes, hipStream_t s) {
    const int64_t K = w.ne[0], N = w.ne[1], M = x.ne[1];
    if (M == 0 || N == 0) return SQA_OK;
    if (M <= kGemvTokens) {
        const int mt = M == 1 ? 1 : (M == 2 ? 2 : 4);
        const int prof = profile_start("out_proj", s);
        const uint8_t *wd = (const uint8_t *)w.data;
        const char *xd = (const char *)x.data, *gd = gate ? (const char *)gate->data : nullptr;
        const int64_t wn = (int64_t)w.nb[1], xn = (int64_t)x.nb[1], gn = gate ? (int64_t)gate->nb[1] : 0;
        float *dd = (float *)dst.data;
        const int64_t dn = (int64_t)dst.nb[1];
        const dim3 grid((unsigned)(N / kGemvRows));
        const bool vec = (uintptr_t)xd % 16 == 0 && xn % 16 == 0 && (!gd || ((uintptr_t)gd % 16 == 0 && gn % 16 == 0));
#define SQA_GEMV(MTV)                                                                                          \
    (vec ? op_gemv_kernel<MTV, true> : op_gemv_kernel<MTV, false>)<<<grid, dim3(kGemvThreads), 0, s>>>(        \
        wd, wn, xd, xn, gd, gn, (int)K, (int)N, (int)M, dd, dn)
        if (mt == 1)
            SQA_GEMV(1);
        else if (mt == 2)
            SQA_GEMV(2);
        else
            SQA_GEMV(4);
#undef SQA_GEMV
        profile_stop(prof, s);
        return hip_status(hipGetLastError(), "out_proj launch");
    }
    const OpLayout L = op_layout(K, M);
    const size_t need = L.total;
    if (!ws || ws_bytes < need)
        return set_error(SQA_ERR_WORKSPACE, "out_proj: workspace %zu bytes < %zu needed", ws_bytes, need);
    uint8_t *base = reinterpret_cast<uint8_t *>(((uintptr_t)ws + 255) & ~(uintptr_t)255);
    uint16_t *xh = reinterpret_cast<uint16_t *>(base);
    uint16_t *xl = reinterpret_cast<uint16_t *>(base + L.xl);
    float *S = reinterpret_cast<float *>(base + L.s);
    uint16_t *sp = reinterpret_cast<uint16_t *>(base + L.sp);
    // op_gemm2 once there are enough 32-token tiles to fill the chip; its DMA
    // offsets are 32-bit
    const bool big = M > 64 && (uint64_t)L.xl * 2 < (1ull << 32) && (uint64_t)N * w.nb[1] < (1ull << 32);
    if (big) {
        static std::once_flag g2_once;
        static hipError_t g2_err = hipSuccess;
        std::call_once(g2_once, [] {
            g2_err = hipFuncSetAttribute((const void *)op_gemm2_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         kG2Lds);
        });
        if (g2_err != hipSuccess) return hip_status(g2_err, "out_proj LDS attribute");
    }

    const int prof = profile_start("out_proj", s);
    const int64_t nprep = 4 * 32 * L.nq * L.Mp;
    const bool vec = (uintptr_t)x.data % 16 == 0 && x.nb[1] % 16 == 0 &&
                     (!gate || ((uintptr_t)gate->data % 16 == 0 && gate->nb[1] % 16 == 0));
    const dim3 pg((unsigned)((nprep + 255) / 256));
    const char *xd = (const char *)x.data, *gd = gate ? (const char *)gate->data : nullptr;
    const int64_t xn = (int64_t)x.nb[1], gn = gate ? (int64_t)gate->nb[1] : 0;
    const int Ki = (int)K, Mi = (int)M, Mpi = (int)L.Mp, nqi = (int)L.nq;
    if (gate && vec)
        op_prep_kernel<true, true><<<pg, dim3(256), 0, s>>>(xd, xn, gd, gn, Ki, Mi, Mpi, nqi, xh, xl, S, sp);
    else if (gate)
        op_prep_kernel<true, false><<<pg, dim3(256), 0, s>>>(xd, xn, gd, gn, Ki, Mi, Mpi, nqi, xh, xl, S, sp);
    else if (vec)
        op_prep_kernel<false, true><<<pg, dim3(256), 0, s>>>(xd, xn, gd, gn, Ki, Mi, Mpi, nqi, xh, xl, S, sp);
    else
        op_prep_kernel<false, false><<<pg, dim3(256), 0, s>>>(xd, xn, gd, gn, Ki, Mi, Mpi, nqi, xh, xl, S, sp);
    if (big) {
        Gemm2Params q;
        q.w = (const uint8_t *)w.data;
        q.w_nb1 = (int64_t)w.nb[1];
        q.x = xh;
        q.xl_off = (uint32_t)L.xl;
        q.sp = sp;
        q.K = Ki;
        q.N = (int)N;
        q.M = Mi;
        q.Mp = Mpi;
        q.nq = nqi;
        q.dst = (float *)dst.data;
        q.d_nb1 = (int64_t)dst.nb[1];
        op_gemm2_kernel<<<dim3((unsigned)((N + kG2Rows - 1) / kG2Rows), (unsigned)(L.Mp / kG2Tok)), dim3(64 * kG2Waves), kG2Lds,
                          s>>>(q);
    } else {
        const int64_t M16 = (M + 15) / 16 * 16;
        GemmParams p;
        p.w = (const uint8_t *)w.data;
        p.w_nb1 = (int64_t)w.nb[1];
        p.xh = xh;
        p.xl = xl;
        p.S = S;
        p.K = Ki;
        p.N = (int)N;
        p.M = Mi;
        p.M16 = (int)M16;
        p.dst = (float *)dst.data;
        p.d_nb1 = (int64_t)dst.nb[1];
        // one 16-token tile per workgroup; for decode (one token tile) 16 rows and
        // 16 wavefronts that take one super-block each, else 64 rows and 4 wavefronts
        if (M16 == 16 || N % 64 != 0)
            op_gemm_kernel<16, 1><<<dim3((unsigned)(N / 16), (unsigned)(M16 / 16)), dim3(1024), 0, s>>>(p);
        else
            op_gemm_kernel<4, 4><<<dim3((unsigned)(N / 64), (unsigned)(M16 / 16)), dim3(256), 0, s>>>(p);
    }
    profile_stop(prof, s);
    return hip_status(hipGetLastError(), "out_proj launch");
}

}  // namespace sqa
