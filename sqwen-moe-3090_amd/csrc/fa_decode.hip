// fa_decode.hip - split-KV FlashAttention over a q4_0 K/V cache for decode and
// speculative verify (n_q * H/Hkv <= 16 query rows per KV head).
//
// Replaces the ggml FLASH_ATTN_EXT node built at src/model/attn.rs:228-251 of
// the reference for n_q = 1..2 (decode step, MTP verify of runner.rs:1263-1270).
//
// Work split
//   A workgroup owns a contiguous key range (a "split") for ALL KV heads, so it
//   streams whole 288-byte cache rows (2 heads x 144 B): every HBM line it
//   touches is used by it alone. Tiles of 128 keys are staged through LDS with
//   16-byte loads; 4 wavefronts (one per SIMD) work on a tile, 2 per KV head,
//   64 keys each in two steps of 32.
//   Each split writes unnormalised (acc, max, sum) partials; fa_combine merges
//   them with the usual log-sum-exp rescaling.
//
// Arithmetic (matches ggml's CPU flash_attn_ext within fp32 rounding)
//   * Q is rounded to q8_0 per 32-value block exactly as ggml's x86 from_float
//     does (d = amax/127, codes = rint(x * 127/amax)), so the K dot is the exact
//     integer sum of (nib-8)*q8 per block. It runs on v_mfma_i32_16x16x32_i8
//     (one q4_0 block = one K=32 step); the -8 offset enters through the
//     accumulator input (-8 * sum(q8)), and each block's integer result is
//     scaled by d_q * d_k in fp32.
//   * P*V runs on v_mfma_f32_16x16x32_f16 with fp32 accumulation: V is
//     dequantised to fp16 ((nib-8) exact, times d_v rounded once), and P is
//     split into fp16 hi + lo parts so the probabilities keep ~22 bits.
//   * Online softmax in fp32 with exp2.
//
// MFMA operand layout used throughout (16x16xK, 64 lanes, lane = 16*g + n):
//   A: lane holds A[row n][k = 8g .. 8g+7]      B: lane holds B[k = 8g .. 8g+7][col n]
//   C: lane holds C[rows 4g .. 4g+3][col n]
#include "common.hpp"

namespace sqa {
namespace {

typedef int int32x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int kWavesPerHead = 2;
constexpr int kKeysPerWave = 64;   // per tile, processed as 2 steps of 32 keys
constexpr int kTileKeys = kWavesPerHead * kKeysPerWave;  // 128
constexpr int kLdsRow = 304;  // 288-byte cache row + 16 bytes of padding (bank spread)
constexpr float kLog2e = 1.4426950408889634f;

template <int HKV>
struct Geo {
    static constexpr int kWaves = kWavesPerHead * HKV;
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kRowBytes = HKV * kHeadRowBytes;             // 288 for 2 KV heads
    static constexpr int kChunksPerRow = kRowBytes / 16;              // 18
    static constexpr int kChunksPerTensor = kTileKeys * kChunksPerRow;
    static constexpr int kChunksPerThread = 2 * kChunksPerTensor / kThreads;  // 18
    static constexpr int kLdsTensor = kTileKeys * kLdsRow;
    // Compact scale tables: d_k as fp32 [HKV][8 blocks][128 keys], d_v as fp16 bits.
    static constexpr int kLdsDk = HKV * kBlocksPerHead * kTileKeys * 4;
    static constexpr int kLdsDv = HKV * kBlocksPerHead * kTileKeys * 2;
    static constexpr int kLdsBytes = 2 * kLdsTensor + kLdsDk + kLdsDv;
    static_assert(kRowBytes % 16 == 0, "cache rows must be whole 16-byte chunks");
    static_assert((2 * kChunksPerTensor) % kThreads == 0, "tile must split evenly");
};

__device__ __forceinline__ uint32_t lds_u32(const uint8_t *p) {
    return *reinterpret_cast<const uint32_t *>(p);
}
// Four bytes at a 2-byte aligned LDS address.
__device__ __forceinline__ uint32_t lds_u32_a2(const uint8_t *base, int off) {
    const int a4 = off & ~3;
    const uint32_t w0 = lds_u32(base + a4);
    const uint32_t w1 = lds_u32(base + a4 + 4);
    return __builtin_amdgcn_alignbyte(w1, w0, (uint32_t)(off & 3));
}
__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    const uint16_t b = (uint16_t)h;
    _Float16 f;
    __builtin_memcpy(&f, &b, 2);
    return (float)f;
}

struct DecodeParams {
    const char *q;
    int64_t q_nb1, q_nb2;  // bytes per query, per head
    const uint8_t *k, *v;  // cache views, rows of HKV*144 bytes
    const char *mask;      // F16 [n_kv, >= n_q] or null
    int64_t mask_nb1;
    int64_t q_pos0;        // >= 0: causal from positions (mask ignored)
    int n_q, H, G;
    int64_t n_kv;
    float scale;
    int n_splits;
    int64_t units;         // ceil(n_kv / 16)
    float *part_acc;       // [n_splits][n_q*H][256]
    float *part_ml;        // [n_splits][n_q*H][2]
};

// Query rows of one KV head: row r (0..15) is query r / G, head kvh*G + r % G.
// QK^T runs as C[key][row] = K . Q^T so each lane ends up holding 8 logits of
// ONE row, laid out exactly as the A operand of the following P*V MFMA.
template <int HKV>
__global__ __launch_bounds__(Geo<HKV>::kThreads, 1) void fa_decode_kernel(DecodeParams p) {
    using GE = Geo<HKV>;
    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t *sK = smem;
    uint8_t *sV = smem + GE::kLdsTensor;
    float *sDk = reinterpret_cast<float *>(smem + 2 * GE::kLdsTensor);
    uint16_t *sDv = reinterpret_cast<uint16_t *>(smem + 2 * GE::kLdsTensor + GE::kLdsDk);

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int g = lane >> 4;
    const int n = lane & 15;
    const int kvh = wave / kWavesPerHead;
    const int wq = wave % kWavesPerHead;

    // Key range of this split, in 16-key units.
    const int split = blockIdx.x;
    const int64_t u0 = (p.units * split) / p.n_splits;
    const int64_t u1 = (p.units * (split + 1)) / p.n_splits;
    const int64_t k_begin = u0 * 16;
    const int64_t k_end = (u1 * 16 < p.n_kv) ? u1 * 16 : p.n_kv;

    // ---------------- Q -> q8_0, B operand of row n -------------------------
    const int my_t = n / p.G;
    const int my_h = kvh * p.G + n % p.G;
    const bool row_ok = my_t < p.n_q;
    const float *qrow = reinterpret_cast<const float *>(p.q + (int64_t)my_t * p.q_nb1 +
                                                        (int64_t)my_h * p.q_nb2);
    int64_t bq[kBlocksPerHead];  // 8 int8 per block: elements 4g..4g+3, 16+4g..16+4g+3
    float dq[kBlocksPerHead];    // fp16-rounded q8_0 scale of row n
    int cinit[kBlocksPerHead];   // -8 * sum(q8) of row n
#pragma unroll
    for (int b = 0; b < kBlocksPerHead; ++b) {
        float x[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[j] = row_ok ? qrow[32 * b + 4 * g + j] : 0.0f;
            x[4 + j] = row_ok ? qrow[32 * b + 16 + 4 * g + j] : 0.0f;
        }
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(x[j]));
        amax = fmaxf(amax, __shfl_xor(amax, 16));
        amax = fmaxf(amax, __shfl_xor(amax, 32));
        const float d = amax / 127.f;
        const float id = amax != 0.0f ? 127.f / amax : 0.0f;
        uint32_t lo = 0, hi = 0;
        int sumq = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int qv = (int)rintf(x[j] * id);
            sumq += qv;
            if (j < 4) lo |= (uint32_t)(qv & 0xff) << (8 * j);
            else hi |= (uint32_t)(qv & 0xff) << (8 * (j - 4));
        }
        sumq += __shfl_xor(sumq, 16);
        sumq += __shfl_xor(sumq, 32);
        bq[b] = (int64_t)(((uint64_t)hi << 32) | lo);
        dq[b] = (float)(_Float16)d;
        cinit[b] = -8 * sumq;
    }
    const int t_of_n = my_t;  // query of this lane's row (column of C)

    // ---------------- running softmax state ----------------------------------
    floatx4 acc[16];  // O[row 4g+i][dim of virtual tile T, column n]
#pragma unroll
    for (int T = 0; T < 16; ++T) acc[T] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;  // of row n
    float l_part = 0.0f;      // this lane's share of row n's sum

    // ---------------- tile pipeline -----------------------------------------
    uint4 pre[GE::kChunksPerThread];
    auto load_tile = [&](int64_t kt, int nvalid) {
#pragma unroll
        for (int i = 0; i < GE::kChunksPerThread; ++i) {
            const int c = tid + GE::kThreads * i;
            const int tens = c / GE::kChunksPerTensor;
            const int cc = c - tens * GE::kChunksPerTensor;
            const int key = cc / GE::kChunksPerRow;
            const int j = cc - key * GE::kChunksPerRow;
            const uint8_t *base = tens ? p.v : p.k;
            if (key < nvalid) {
                pre[i] = *reinterpret_cast<const uint4 *>(base + (kt + key) * GE::kRowBytes + 16 * j);
            } else {
                pre[i] = make_uint4(0, 0, 0, 0);
            }
        }
    };
    // Raw rows to LDS; the chunk holding the start of block m (byte 18m of the
    // row, m = head*8 + block) also files that block's scale in sDk / sDv.
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < GE::kChunksPerThread; ++i) {
            const int c = tid + GE::kThreads * i;
            const int tens = c / GE::kChunksPerTensor;
            const int cc = c - tens * GE::kChunksPerTensor;
            const int key = cc / GE::kChunksPerRow;
            const int j = cc - key * GE::kChunksPerRow;
            uint8_t *dstp = (tens ? sV : sK) + key * kLdsRow + 16 * j;
            *reinterpret_cast<uint4 *>(dstp) = pre[i];
            // 18m lies in chunk j = (18m)/16 = m + m/8 at byte (2m) % 16.
            const int m = j - j / 9;
            if (j % 9 != 8) {
                const int byte = (2 * m) & 15;
                const uint32_t wsel = byte < 4 ? pre[i].x : byte < 8 ? pre[i].y : byte < 12 ? pre[i].z : pre[i].w;
                const uint32_t bits = (byte & 2) ? (wsel >> 16) : (wsel & 0xffff);
                const int slot = (m >> 3) * kBlocksPerHead + (m & 7);  // head*8 + block
                if (tens) sDv[slot * kTileKeys + key] = (uint16_t)bits;
                else sDk[slot * kTileKeys + key] = half_bits_to_float(bits);
            }
        }
    };

    const int64_t n_tiles = (k_end - k_begin + kTileKeys - 1) / kTileKeys;
    if (n_tiles > 0) {
        load_tile(k_begin, (int)((k_end - k_begin) < kTileKeys ? (k_end - k_begin) : kTileKeys));
        store_tile();
    }
    __syncthreads();

    const float* dk_head = sDk + kvh * kBlocksPerHead * kTileKeys;
    const uint16_t* dv_head = sDv + kvh * kBlocksPerHead * kTileKeys;
    for (int64_t it = 0; it < n_tiles; ++it) {
        const int64_t kt = k_begin + it * kTileKeys;
        const int nvalid = (int)((k_end - kt) < kTileKeys ? (k_end - kt) : kTileKeys);
        if (it + 1 < n_tiles) {
            const int64_t kn = kt + kTileKeys;
            load_tile(kn, (int)((k_end - kn) < kTileKeys ? (k_end - kn) : kTileKeys));
        }
#pragma unroll 1
        for (int ks = 0; ks < kKeysPerWave / 32; ++ks) {
        const int wkey0 = wq * kKeysPerWave + 32 * ks;  // first key of this step inside the tile
        if (wkey0 < nvalid) {
            // ---- logits: s[st][i] = S[key wkey0+16st+4g+i][row n] -------------
            float s[2][4];
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const int ka = wkey0 + 16 * st + n;       // A row (key) this lane feeds
                const int kc = wkey0 + 16 * st + 4 * g;   // first of the 4 C-row keys it receives
                const uint8_t *krow = sK + ka * kLdsRow + kvh * kHeadRowBytes;
                float sacc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int b = 0; b < kBlocksPerHead; ++b) {
                    const uint32_t x = lds_u32_a2(krow, 18 * b + 2 + 4 * g);
                    const uint32_t alo = x & 0x0F0F0F0Fu;
                    const uint32_t ahi = (x >> 4) & 0x0F0F0F0Fu;
                    const int64_t aop = (int64_t)(((uint64_t)ahi << 32) | alo);
                    const int32x4 cin = {cinit[b], cinit[b], cinit[b], cinit[b]};
                    const int32x4 c = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bq[b], cin, 0, 0, 0);
                    const floatx4 dk = *reinterpret_cast<const floatx4 *>(dk_head + b * kTileKeys + kc);
#pragma unroll
                    for (int i = 0; i < 4; ++i) sacc[i] = fmaf((float)c[i], dq[b] * dk[i], sacc[i]);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int kl = kc + i;
                    const int64_t kabs = kt + kl;
                    float sv = sacc[i] * p.scale;
                    if (kl >= nvalid) {
                        sv = -INFINITY;
                    } else if (p.q_pos0 >= 0) {
                        if (kabs > p.q_pos0 + t_of_n) sv = -INFINITY;
                    } else if (p.mask && row_ok) {
                        const uint16_t mb = *reinterpret_cast<const uint16_t *>(
                            p.mask + (int64_t)t_of_n * p.mask_nb1 + kabs * 2);
                        const float mv = half_bits_to_float(mb);
                        sv = (mv == -INFINITY) ? -INFINITY : sv + mv;
                    }
                    s[st][i] = sv;
                }
            }
            // ---- online softmax for row n over the wave's 32 keys --------------
            float mt = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                             fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
            mt = fmaxf(mt, __shfl_xor(mt, 16));
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float m_new = fmaxf(m_run, mt);
            const float mref = (m_new == -INFINITY) ? 0.0f : m_new;
            const float alpha = exp2f((m_run - mref) * kLog2e);
            float pr[2][4];
            float psum = 0.0f;
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pr[st][i] = exp2f((s[st][i] - mref) * kLog2e);
                    psum += pr[st][i];
                }
            l_part = l_part * alpha + psum;
            m_run = m_new;
            if (__any(alpha != 1.0f)) {
                float ar[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) ar[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
                for (int T = 0; T < 16; ++T)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[T][i] *= ar[i];
            }
            // ---- A operand: P[row n][k = 8g+jj], jj<4 -> key 4g+jj, else 16+4g+jj-4
            half8 pa_hi, pa_lo;
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const float pv = pr[jj >> 2][jj & 3];
                const _Float16 h = (_Float16)pv;
                pa_hi[jj] = h;
                pa_lo[jj] = (_Float16)(pv - (float)h);
            }

            // ---- O += P V ------------------------------------------------------
#pragma unroll
            for (int rr = 0; rr < 2; ++rr) {
                const int beta = 4 * rr + (n >> 2);
                const int omega = n & 3;
                uint32_t w[8];
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const int key = wkey0 + (jj < 4 ? 4 * g + jj : 16 + 4 * g + jj - 4);
                    const uint8_t *vrow = sV + key * kLdsRow + kvh * kHeadRowBytes;
                    w[jj] = lds_u32_a2(vrow, 18 * beta + 2 + 4 * omega);
                }
                // d_v of the 8 keys: two runs of 4 consecutive keys.
                const uint16_t *dvb = dv_head + beta * kTileKeys + wkey0 + 4 * g;
                const uint2 dv0 = *reinterpret_cast<const uint2 *>(dvb);
                const uint2 dv1 = *reinterpret_cast<const uint2 *>(dvb + 16);
                const uint32_t dvw[4] = {dv0.x, dv0.y, dv1.x, dv1.y};
                half2v dvp[4];
#pragma unroll
                for (int pp = 0; pp < 4; ++pp) __builtin_memcpy(&dvp[pp], &dvw[pp], 4);
#pragma unroll
                for (int jb = 0; jb < 4; ++jb) {
                    const uint32_t sel = (uint32_t)jb | (0x0cu << 8) | ((uint32_t)(4 + jb) << 16) | (0x0cu << 24);
                    uint32_t blo[4], bhi[4];
#pragma unroll
                    for (int pp = 0; pp < 4; ++pp) {
                        const uint32_t t = __builtin_amdgcn_perm(w[2 * pp + 1], w[2 * pp], sel);
                        uint32_t lo16 = (t & 0x000F000Fu) | 0x64006400u;
                        uint32_t hi16 = ((t >> 4) & 0x000F000Fu) | 0x64006400u;
                        half2v hl, hh;
                        __builtin_memcpy(&hl, &lo16, 4);
                        __builtin_memcpy(&hh, &hi16, 4);
                        const half2v off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
                        hl = (hl + off) * dvp[pp];
                        hh = (hh + off) * dvp[pp];
                        __builtin_memcpy(&blo[pp], &hl, 4);
                        __builtin_memcpy(&bhi[pp], &hh, 4);
                    }
                    half8 bl, bh;
                    __builtin_memcpy(&bl, blo, 16);
                    __builtin_memcpy(&bh, bhi, 16);
                    const int Tl = rr * 8 + jb;
                    const int Th = rr * 8 + 4 + jb;
                    acc[Tl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa_hi, bl, acc[Tl], 0, 0, 0);
                    acc[Tl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa_lo, bl, acc[Tl], 0, 0, 0);
                    acc[Th] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa_hi, bh, acc[Th], 0, 0, 0);
                    acc[Th] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa_lo, bh, acc[Th], 0, 0, 0);
                }
            }
        }
        }
        __syncthreads();
        if (it + 1 < n_tiles) store_tile();
        __syncthreads();
    }

    // ---------------- merge the 4 waves of each KV head ------------------------
    l_part += __shfl_xor(l_part, 16);
    l_part += __shfl_xor(l_part, 32);

    float *sML = reinterpret_cast<float *>(smem + 2 * GE::kLdsTensor);  // [HKV][waves per head][16][2]
    float *sAcc = reinterpret_cast<float *>(smem);                        // [HKV][16][256]
    if (g == 0) {
        sML[((kvh * kWavesPerHead + wq) * 16 + n) * 2 + 0] = m_run;
        sML[((kvh * kWavesPerHead + wq) * 16 + n) * 2 + 1] = l_part;
    }
    __syncthreads();
    float fac[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = 4 * g + i;
        float M = -INFINITY;
        for (int w2 = 0; w2 < kWavesPerHead; ++w2)
            M = fmaxf(M, sML[((kvh * kWavesPerHead + w2) * 16 + row) * 2]);
        const float mw = sML[((kvh * kWavesPerHead + wq) * 16 + row) * 2];
        fac[i] = (mw == -INFINITY) ? 0.0f : exp2f((mw - M) * kLog2e);
    }
    float *myAcc = sAcc + kvh * 16 * 256;
    for (int w2 = 0; w2 < kWavesPerHead; ++w2) {
        if (wq == w2) {
#pragma unroll
            for (int T = 0; T < 16; ++T) {
                const int rr = T >> 3, i8 = T & 7;
                const int dim = 32 * (4 * rr + (n >> 2)) +
                                (i8 < 4 ? 4 * (n & 3) + i8 : 16 + 4 * (n & 3) + (i8 - 4));
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = 4 * g + i;
                    const float vv = acc[T][i] * fac[i];
                    float *dstp = myAcc + row * 256 + dim;
                    *dstp = (w2 == 0) ? vv : (*dstp + vv);
                }
            }
        }
        __syncthreads();
    }
    // ---------------- write this split's partials ----------------------------
    const int rows_total = p.n_q * p.H;
    for (int e = tid; e < HKV * 16 * 256; e += GE::kThreads) {
        const int kh = e / (16 * 256);
        const int row = (e / 256) % 16;
        const int dim = e % 256;
        const int t = row / p.G;
        const int h = kh * p.G + row % p.G;
        if (t < p.n_q) {
            const int64_t ridx = (int64_t)t * p.H + h;
            p.part_acc[((int64_t)split * rows_total + ridx) * 256 + dim] = sAcc[e];
        }
    }
    for (int e = tid; e < HKV * 16; e += GE::kThreads) {
        const int kh = e / 16;
        const int row = e % 16;
        const int t = row / p.G;
        const int h = kh * p.G + row % p.G;
        if (t < p.n_q) {
            float M = -INFINITY, L = 0.0f;
            for (int w2 = 0; w2 < kWavesPerHead; ++w2)
                M = fmaxf(M, sML[((kh * kWavesPerHead + w2) * 16 + row) * 2]);
            for (int w2 = 0; w2 < kWavesPerHead; ++w2) {
                const float mw = sML[((kh * kWavesPerHead + w2) * 16 + row) * 2];
                const float lw = sML[((kh * kWavesPerHead + w2) * 16 + row) * 2 + 1];
                if (mw != -INFINITY) L += lw * exp2f((mw - M) * kLog2e);
            }
            const int64_t ridx = (int64_t)t * p.H + h;
            p.part_ml[((int64_t)split * rows_total + ridx) * 2 + 0] = M;
            p.part_ml[((int64_t)split * rows_total + ridx) * 2 + 1] = L;
        }
    }
}

// Merge split partials: out = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M),
// optionally times sigmoid(gate). Grid: (rows, 4 dim chunks of 64); 256 threads
// = 64 dims x 4 interleaved split subsets reduced through LDS.
__global__ __launch_bounds__(256) void fa_combine_kernel(const float *__restrict__ part_acc,
                                                         const float *__restrict__ part_ml,
                                                         int n_splits, int rows_total,
                                                         float *__restrict__ dst, const char *gate,
                                                         int64_t gate_nb1, int64_t gate_nb2, int H) {
    __shared__ float red[4][64];
    __shared__ float redl[4];
    const int row = blockIdx.x;
    const int d = blockIdx.y * 64 + (threadIdx.x & 63);
    const int sub = threadIdx.x >> 6;
    float M = -INFINITY;
    for (int s = 0; s < n_splits; ++s) M = fmaxf(M, part_ml[((int64_t)s * rows_total + row) * 2]);
    float o = 0.0f, L = 0.0f;
    if (M != -INFINITY) {
        for (int s = sub; s < n_splits; s += 4) {
            const float ms = part_ml[((int64_t)s * rows_total + row) * 2];
            if (ms == -INFINITY) continue;
            const float f = exp2f((ms - M) * kLog2e);
            L += part_ml[((int64_t)s * rows_total + row) * 2 + 1] * f;
            o += part_acc[((int64_t)s * rows_total + row) * 256 + d] * f;
        }
    }
    red[sub][threadIdx.x & 63] = o;
    if ((threadIdx.x & 63) == 0) redl[sub] = L;
    __syncthreads();
    if (sub == 0) {
        const float ot = red[0][d & 63] + red[1][d & 63] + red[2][d & 63] + red[3][d & 63];
        const float Lt = redl[0] + redl[1] + redl[2] + redl[3];
        float r = (Lt == 0.0f) ? 0.0f : ot * (1.0f / Lt);
        if (gate) {
            const int t = row / H, h = row % H;
            const float gv = reinterpret_cast<const float *>(gate + t * gate_nb2 + h * gate_nb1)[d];
            r = r * (1.0f / (1.0f + expf(-gv)));
        }
        dst[(int64_t)row * 256 + d] = r;
    }
}

int decode_splits(int64_t n_kv) {
    const int64_t units = (n_kv + 15) / 16;
    int64_t s = (units + 7) / 8;  // at least 128 keys per split
    const int64_t cap = device_cu_count();
    if (s > cap) s = cap;
    if (s < 1) s = 1;
    return (int)s;
}

}  // namespace

size_t fa_decode_workspace(int64_t n_q, int64_t H, int64_t n_kv) {
    const int64_t splits = decode_splits(n_kv);
    return (size_t)(splits * n_q * H * (256 + 2) * sizeof(float)) + 256;
}

int launch_fa_decode(const FaArgs &a, hipStream_t s) {
    const sqa_tensor &q = *a.q, &k = *a.k;
    const int64_t n_q = q.ne[1], H = q.ne[2], n_kv = k.ne[1], Hkv = k.ne[2];
    const int G = (int)(H / Hkv);
    DecodeParams p;
    p.q = (const char *)q.data;
    p.q_nb1 = (int64_t)q.nb[1];
    p.q_nb2 = (int64_t)q.nb[2];
    p.k = (const uint8_t *)k.data;
    p.v = (const uint8_t *)a.v->data;
    p.mask = (a.q_pos0 < 0 && a.mask) ? (const char *)a.mask->data : nullptr;
    p.mask_nb1 = a.mask ? (int64_t)a.mask->nb[1] : 0;
    p.q_pos0 = a.q_pos0;
    p.n_q = (int)n_q;
    p.H = (int)H;
    p.G = G;
    p.n_kv = n_kv;
    p.scale = a.scale;
    p.n_splits = decode_splits(n_kv);
    p.units = (n_kv + 15) / 16;
    const size_t need = fa_decode_workspace(n_q, H, n_kv);
    if (!a.ws || a.ws_bytes < need)
        return set_error(SQA_ERR_WORKSPACE, "flash_attn_ext: workspace %zu bytes < %zu needed",
                         a.ws_bytes, need);
    uintptr_t wsb = ((uintptr_t)a.ws + 255) & ~(uintptr_t)255;
    p.part_acc = reinterpret_cast<float *>(wsb);
    p.part_ml = p.part_acc + (int64_t)p.n_splits * n_q * H * 256;
    if (Hkv != 2) return set_error(SQA_ERR_UNSUPPORTED, "decode kernel built for 2 KV heads");
    using GE = Geo<2>;
    static bool lds_ok = false;  // raise the dynamic-LDS limit once per process
    if (!lds_ok) {
        hipError_t e0 = hipFuncSetAttribute((const void *)fa_decode_kernel<2>,
                                            hipFuncAttributeMaxDynamicSharedMemorySize, GE::kLdsBytes);
        if (e0 != hipSuccess) return hip_status(e0, "fa_decode LDS attribute");
        lds_ok = true;
    }
    int prof = profile_start("fa_decode", s);
    fa_decode_kernel<2><<<dim3(p.n_splits), dim3(GE::kThreads), GE::kLdsBytes, s>>>(p);
    profile_stop(prof, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_status(e, "fa_decode launch");
    const char *gate = a.gate ? (const char *)a.gate->data : nullptr;
    prof = profile_start("fa_combine", s);
    fa_combine_kernel<<<dim3((unsigned)(n_q * H), 4), dim3(256), 0, s>>>(
        p.part_acc, p.part_ml, p.n_splits, (int)(n_q * H), (float *)a.dst->data, gate,
        a.gate ? (int64_t)a.gate->nb[1] : 0, a.gate ? (int64_t)a.gate->nb[2] : 0, (int)H);
    profile_stop(prof, s);
    return hip_status(hipGetLastError(), "fa_combine launch");
}

}  // namespace sqa
