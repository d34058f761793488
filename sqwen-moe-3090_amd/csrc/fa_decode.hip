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
//   16-byte loads; 8 wavefronts (two per SIMD) work on a tile, 4 per KV head,
//   32 keys each.
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

constexpr int kWavesPerHead = 4;
constexpr int kKeysPerWave = 32;
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
    static constexpr int kChunksPerThread = 2 * kChunksPerTensor / kThreads;  // 9
    static constexpr int kLdsTensor = kTileKeys * kLdsRow;
    static constexpr int kLdsMask = 16 * kTileKeys * 2;  // up to 16 query rows of F16 mask
    static constexpr int kLdsBytes = 2 * kLdsTensor + kLdsMask;
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
    int mask_vec;          // mask rows 16-byte aligned: one 16-byte load per 8 keys
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
//
// BD (block-diagonal) variant, used when a KV head has at most 8 query rows
// (decode, n_q = 1): C columns 0..7 carry the rows' dot with the even q4_0 block
// of a block pair and columns 8..15 the same rows with the odd block, so no
// column of the i8 MFMA is padding. Each block pair takes two MFMAs (the two
// 16-value halves of each block, k-slots 0-1 for the even block and 2-3 for the
// odd one, the other slots zero); a DPP rotate by 8 lanes then adds the even
// and odd halves of every logit.
template <int HKV, bool BD>
__global__ __launch_bounds__(Geo<HKV>::kThreads, 1) void fa_decode_kernel(DecodeParams p) {
    using GE = Geo<HKV>;
    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t *sK = smem;
    uint8_t *sV = smem + GE::kLdsTensor;
    uint16_t *sMask = reinterpret_cast<uint16_t *>(smem + 2 * GE::kLdsTensor);

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


    // ---------------- running softmax state ----------------------------------
    floatx4 acc[16];  // O[row 4g+i][dim of virtual tile T, column n]
#pragma unroll
    for (int T = 0; T < 16; ++T) acc[T] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;  // of row n
    float l_part = 0.0f;      // this lane's share of row n's sum

    // ---------------- tile pipeline -----------------------------------------
    // Chunk i of this thread is number c = tid + kThreads*i of the tile's K|V
    // chunks: K if c < kChunksPerTensor, else V chunk cc = c - kChunksPerTensor,
    // i.e. bytes [16cc, 16cc+16) of the tile's contiguous rows: key cc/18,
    // 16-byte column cc%18. The K/V split falls on a wave boundary, so the
    // tensor of every chunk is wave-uniform.
    // Loads never sit behind a divergent branch and their values are not
    // touched until store_tile, so all of them stay in flight during compute.
    // Full tiles use plain base + 16*tid + constant addressing; the one partial
    // tile a split can end with reads key 0 for rows past the valid range and
    // zeroes them at store time.
    uint4 pre[GE::kChunksPerThread];
    uint4 pre_mask = make_uint4(0, 0, 0, 0);
    int pre_nvalid = 0;
    int64_t pre_kt = 0;
    const bool mask_loader = p.mask && tid < 16 * p.n_q;  // 16 lanes x 8 keys per query row
    const int mrow = mask_loader ? (tid >> 4) : 0;         // clamped to a valid row otherwise
    const int mc8 = (tid & 15) * 8;
    auto chunk_src = [&](int i, const uint8_t *kb, const uint8_t *vb) {
        const int c = tid + GE::kThreads * i;
        return c < GE::kChunksPerTensor ? kb + 16 * c : vb + 16 * (c - GE::kChunksPerTensor);
    };
    auto load_tile = [&](int64_t kt, int nvalid) {
        const uint8_t *kb = p.k + kt * GE::kRowBytes;
        const uint8_t *vb = p.v + kt * GE::kRowBytes;
        if (nvalid == kTileKeys) {
#pragma unroll
            for (int i = 0; i < GE::kChunksPerThread; ++i)
                pre[i] = *reinterpret_cast<const uint4 *>(chunk_src(i, kb, vb));
        } else {
#pragma unroll
            for (int i = 0; i < GE::kChunksPerThread; ++i) {
                const int c = tid + GE::kThreads * i;
                const int cc = c < GE::kChunksPerTensor ? c : c - GE::kChunksPerTensor;
                const bool ok = cc / GE::kChunksPerRow < nvalid;
                pre[i] = *reinterpret_cast<const uint4 *>(ok ? chunk_src(i, kb, vb) : kb);
            }
        }
        if (p.mask && p.mask_vec && wave * 64 < 16 * p.n_q) {  // wave-uniform: mask-loading waves
            const int cm = mc8 + 8 <= nvalid ? mc8 : 0;  // keys past nvalid are never used
            pre_mask = *reinterpret_cast<const uint4 *>(p.mask + (int64_t)mrow * p.mask_nb1 + (kt + cm) * 2);
        }
        pre_nvalid = nvalid;
        pre_kt = kt;
    };
    // Raw rows to LDS, row stride kLdsRow = 288 + 16 bytes.
    auto store_tile = [&]() {
        const uint4 z = make_uint4(0, 0, 0, 0);
        const bool full = pre_nvalid == kTileKeys;
#pragma unroll
        for (int i = 0; i < GE::kChunksPerThread; ++i) {
            const int c = tid + GE::kThreads * i;
            const bool isv = c >= GE::kChunksPerTensor;
            const int cc = isv ? c - GE::kChunksPerTensor : c;
            const int key = cc / GE::kChunksPerRow;
            const uint4 ch = (full || key < pre_nvalid) ? pre[i] : z;
            *reinterpret_cast<uint4 *>((isv ? sV : sK) + 16 * cc + 16 * key) = ch;  // key*kLdsRow + 16j
        }
        if (mask_loader) {
            if (!p.mask_vec) {  // unaligned mask rows (ragged n_kv): element loads, slow path
                const uint16_t *mp = reinterpret_cast<const uint16_t *>(p.mask + (int64_t)mrow * p.mask_nb1) + pre_kt;
                uint16_t e[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) e[j] = mp[mc8 + j < pre_nvalid ? mc8 + j : 0];
                __builtin_memcpy(&pre_mask, e, 16);
            }
            *reinterpret_cast<uint4 *>(sMask + mrow * kTileKeys + mc8) = pre_mask;
        }
    };

    const int64_t n_tiles = (k_end - k_begin + kTileKeys - 1) / kTileKeys;
    if (n_tiles > 0) load_tile(k_begin, (int)((k_end - k_begin) < kTileKeys ? (k_end - k_begin) : kTileKeys));

    // ---------------- Q -> q8_0, B operand of row n -------------------------
    // Row of C column n: query r / G, head kvh*G + r % G, r = n (or n & 7 in BD).
    const int my_r = BD ? (n & 7) : n;
    const int my_t = my_r / p.G;
    const int my_h = kvh * p.G + my_r % p.G;
    const bool row_ok = my_t < p.n_q;
    // Rows past n_q read row 0 (always valid) and are zeroed: no branch around the
    // loads, so they issue back to back.
    const float *qrow = reinterpret_cast<const float *>(
        p.q + (row_ok ? (int64_t)my_t * p.q_nb1 + (int64_t)my_h * p.q_nb2 : 0));
    constexpr int kQB = BD ? kBlocksPerHead / 2 : kBlocksPerHead;  // B operands per subtile
    constexpr int kQH = BD ? 2 : 1;                                  // MFMAs per B operand group
    int64_t bq[kQB][kQH];  // int8 B operands
    float dq[kQB];         // fp16-rounded q8_0 scale of (row, block) of column n
    int cinit[kQB];        // -8 * sum(q8) of that block
    float4 qv4[2 * kBlocksPerHead];  // all 16 loads issue before any arithmetic
    // Lane (g, n) loads the values of k-slot s of block beta, i.e. elements
    // 4s..4s+3 and 16+4s..16+4s+3 (the low and high nibbles of qs[4s..4s+3]).
    // Plain: beta = b, s = g. BD: beta = 2bp + (n >> 3), s = 2hf + (g & 1),
    // active only when (g >> 1) == (n >> 3).
    const bool q_active = BD ? ((g >> 1) == (n >> 3)) : true;
#pragma unroll
    for (int b = 0; b < kBlocksPerHead; ++b) {
        const int beta = BD ? 2 * (b >> 1) + (n >> 3) : b;
        const int slot = BD ? 2 * (b & 1) + (g & 1) : g;
        qv4[2 * b] = *reinterpret_cast<const float4 *>(qrow + 32 * beta + 4 * slot);
        qv4[2 * b + 1] = *reinterpret_cast<const float4 *>(qrow + 32 * beta + 16 + 4 * slot);
    }
    const bool use = row_ok && q_active;
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
        float x[kQH][8];
#pragma unroll
        for (int hf = 0; hf < kQH; ++hf) {
            const float4 a0 = qv4[2 * (qb * kQH + hf)], a1 = qv4[2 * (qb * kQH + hf) + 1];
            const float v8[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) x[hf][j] = use ? v8[j] : 0.0f;
        }
        float amax = 0.0f;
#pragma unroll
        for (int hf = 0; hf < kQH; ++hf)
#pragma unroll
            for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(x[hf][j]));
        // the block's 32 values sit in lanes g^1 (BD) or all four g (plain)
        amax = fmaxf(amax, __shfl_xor(amax, 16));
        if (!BD) amax = fmaxf(amax, __shfl_xor(amax, 32));
        const float d = amax / 127.f;
        const float id = amax != 0.0f ? 127.f / amax : 0.0f;
        int sumq = 0;
#pragma unroll
        for (int hf = 0; hf < kQH; ++hf) {
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int qv = (int)rintf(x[hf][j] * id);
                sumq += qv;
                if (j < 4) lo |= (uint32_t)(qv & 0xff) << (8 * j);
                else hi |= (uint32_t)(qv & 0xff) << (8 * (j - 4));
            }
            bq[qb][hf] = (int64_t)(((uint64_t)hi << 32) | lo);
        }
        sumq += __shfl_xor(sumq, 16);
        if (!BD) sumq += __shfl_xor(sumq, 32);
        float dqv = (float)(_Float16)d;
        int civ = -8 * sumq;
        if (BD) {  // inactive lanes of column n take the values from lane g ^ 2
            const float dq2 = __shfl_xor(dqv, 32);
            const int ci2 = __shfl_xor(civ, 32);
            dqv = q_active ? dqv : dq2;
            civ = q_active ? civ : ci2;
        }
        dq[qb] = dqv;
        cinit[qb] = civ;
    }
    const int t_of_n = my_t;  // query of this lane's row (column of C)

    if (n_tiles > 0) store_tile();
    __syncthreads();

    // fp16 magic 0x6400 (= 1024) in a VGPR so (t & mask) | magic is one v_and_or_b32
    // (VOP3 on this target cannot take two literal operands).
    uint32_t magic;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
    const half2v off_lo = {(_Float16)-1032.0f, (_Float16)-1032.0f};  // 1024 + 8
    const half2v off_hi = {(_Float16)-1152.0f, (_Float16)-1152.0f};  // 1024 + 16*8
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
                for (int qb = 0; qb < kQB; ++qb) {
                    int32x4 c = {cinit[qb], cinit[qb], cinit[qb], cinit[qb]};
#pragma unroll
                    for (int hf = 0; hf < kQH; ++hf) {
                        // A: key ka, block beta_a, k-slot of this lane (see the Q layout)
                        const int beta_a = BD ? 2 * qb + (g >> 1) : qb;
                        const int slot = BD ? 2 * hf + (g & 1) : g;
                        const uint32_t x = lds_u32_a2(krow, 18 * beta_a + 2 + 4 * slot);
                        const uint32_t alo = x & 0x0F0F0F0Fu;
                        const uint32_t ahi = (x >> 4) & 0x0F0F0F0Fu;
                        const int64_t aop = (int64_t)(((uint64_t)ahi << 32) | alo);
                        c = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bq[qb][hf], c, 0, 0, 0);
                    }
                    const int beta_c = BD ? 2 * qb + (n >> 3) : qb;  // block of column n
                    // d_k of the 4 C-row keys kc..kc+3: fp16 at byte 18*beta of each row
                    const uint8_t *dkp = sK + kc * kLdsRow + kvh * kHeadRowBytes + 18 * beta_c;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float dk = half_bits_to_float(*reinterpret_cast<const uint16_t *>(dkp + i * kLdsRow));
                        sacc[i] = fmaf((float)c[i], dq[qb] * dk, sacc[i]);
                    }
                }
                if (BD) {  // even-block half (columns 0-7) + odd-block half (8-15)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int other = __builtin_amdgcn_mov_dpp(__float_as_int(sacc[i]), 0x128, 0xf, 0xf, false);
                        sacc[i] += __int_as_float(other);
                    }
                }
                uint2 mraw = make_uint2(0, 0);
                if (p.mask) mraw = *reinterpret_cast<const uint2 *>(sMask + (row_ok ? t_of_n : 0) * kTileKeys + kc);
                const uint32_t mw[2] = {mraw.x, mraw.y};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int kl = kc + i;
                    const int64_t kabs = kt + kl;
                    float sv = sacc[i] * p.scale;
                    const float mv = half_bits_to_float((mw[i >> 1] >> (16 * (i & 1))) & 0xffff);
                    bool dead = kl >= nvalid;
                    if (p.q_pos0 >= 0) {
                        dead = dead || (kabs > p.q_pos0 + t_of_n);
                    } else if (p.mask && row_ok) {
                        dead = dead || (mv == -INFINITY);
                        sv += mv;
                    }
                    s[st][i] = dead ? -INFINITY : sv;
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
                const float pv = (BD && n >= 8) ? 0.0f : pr[jj >> 2][jj & 3];  // BD: rows 8-15 unused
                const _Float16 h = (_Float16)pv;
                pa_hi[jj] = h;
                pa_lo[jj] = (_Float16)(pv - (float)h);
            }

            // ---- O += P V ------------------------------------------------------
#pragma unroll
            for (int rr = 0; rr < 2; ++rr) {
                const int beta = 4 * rr + (n >> 2);
                const int omega = n & 3;
                uint32_t w[8], dvh[8];
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const int key = wkey0 + (jj < 4 ? 4 * g + jj : 16 + 4 * g + jj - 4);
                    const uint8_t *vrow = sV + key * kLdsRow + kvh * kHeadRowBytes;
                    w[jj] = lds_u32_a2(vrow, 18 * beta + 2 + 4 * omega);
                    dvh[jj] = *reinterpret_cast<const uint16_t *>(vrow + 18 * beta);  // d_v (fp16 bits)
                }
                half2v dvp[4];
#pragma unroll
                for (int pp = 0; pp < 4; ++pp) {
                    const uint32_t pk = dvh[2 * pp] | (dvh[2 * pp + 1] << 16);
                    __builtin_memcpy(&dvp[pp], &pk, 4);
                }
#pragma unroll
                for (int jb = 0; jb < 4; ++jb) {
                    const uint32_t sel = (uint32_t)jb | (0x0cu << 8) | ((uint32_t)(4 + jb) << 16) | (0x0cu << 24);
                    uint32_t blo[4], bhi[4];
#pragma unroll
                    for (int pp = 0; pp < 4; ++pp) {
                        // bytes jb of keys 2pp, 2pp+1 -> halves; low nibble n gives fp16
                        // 1024 + n, the high nibble in place gives 1024 + 16n (both exact)
                        const uint32_t t = __builtin_amdgcn_perm(w[2 * pp + 1], w[2 * pp], sel);
                        const uint32_t lo16 = (t & 0x000F000Fu) | magic;
                        const uint32_t hi16 = (t & 0x00F000F0u) | magic;
                        half2v hl, hh;
                        __builtin_memcpy(&hl, &lo16, 4);
                        __builtin_memcpy(&hh, &hi16, 4);
                        hl = (hl + off_lo) * dvp[pp];  // (n - 8) * d_v
                        hh = (hh + off_hi) * dvp[pp];  // 16 (n - 8) * d_v, the 16 leaves at the end
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

    float *sML = reinterpret_cast<float *>(smem + GE::kLdsTensor + HKV * 16 * 256 * 4);  // [HKV][waves][16][2]
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
                    const float vv = acc[T][i] * (i8 < 4 ? fac[i] : fac[i] * 0.0625f);  // hi tiles carry x16
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
// optionally times sigmoid(gate). Grid: (rows, 16 chunks of 16 dims); 256
// threads = 16 dims x 16 split groups, each thread summing every 16th split
// with all its loads in flight; the split weights are computed once per block.
constexpr int kMaxSplits = 1024;
__global__ __launch_bounds__(256) void fa_combine_kernel(const float *__restrict__ part_acc,
                                                         const float *__restrict__ part_ml,
                                                         int n_splits, int rows_total,
                                                         float *__restrict__ dst, const char *gate,
                                                         int64_t gate_nb1, int64_t gate_nb2, int H) {
    __shared__ float wts[kMaxSplits];
    __shared__ float red[16][17];
    __shared__ float redm[256];
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const int dl = tid & 15;
    const int sg = tid >> 4;
    const int d = blockIdx.y * 16 + dl;
    float mloc = -INFINITY;
    for (int s = tid; s < n_splits; s += 256) mloc = fmaxf(mloc, part_ml[((int64_t)s * rows_total + row) * 2]);
    redm[tid] = mloc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) redm[tid] = fmaxf(redm[tid], redm[tid + w]);
        __syncthreads();
    }
    const float M = redm[0];
    __syncthreads();
    float lloc = 0.0f;
    for (int s = tid; s < n_splits; s += 256) {
        const float ms = part_ml[((int64_t)s * rows_total + row) * 2];
        const float ls = part_ml[((int64_t)s * rows_total + row) * 2 + 1];
        const float w = (M == -INFINITY || ms == -INFINITY) ? 0.0f : exp2f((ms - M) * kLog2e);
        wts[s] = w;
        lloc += ls * w;
    }
    redm[tid] = lloc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (tid < w) redm[tid] += redm[tid + w];
        __syncthreads();
    }
    const float L = redm[0];
    const float *pa = part_acc + (int64_t)row * 256 + d;
    const int64_t sstride = (int64_t)rows_total * 256;
    float o = 0.0f;
#pragma unroll 16
    for (int s = sg; s < n_splits; s += 16) o = fmaf(pa[s * sstride], wts[s], o);
    red[sg][dl] = o;
    __syncthreads();
    if (tid < 16) {
        float ot = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) ot += red[j][tid];
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
        const float w = (M == -INFINITY || ms[sp] == -INFINITY) ? 0.0f : exp2f((ms[sp] - M) * kLog2e);
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

namespace {

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
    p.mask_vec = p.mask && (uintptr_t)p.mask % 16 == 0 && p.mask_nb1 % 16 == 0;
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
        for (const void *fn : {(const void *)fa_decode_kernel<2, true>, (const void *)fa_decode_kernel<2, false>}) {
            hipError_t e0 = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, GE::kLdsBytes);
            if (e0 != hipSuccess) return hip_status(e0, "fa_decode LDS attribute");
        }
        lds_ok = true;
    }
    int prof = profile_start("fa_decode", s);
    if (n_q * G <= 8)
        fa_decode_kernel<2, true><<<dim3(p.n_splits), dim3(GE::kThreads), GE::kLdsBytes, s>>>(p);
    else
        fa_decode_kernel<2, false><<<dim3(p.n_splits), dim3(GE::kThreads), GE::kLdsBytes, s>>>(p);
    profile_stop(prof, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_status(e, "fa_decode launch");
    return launch_fa_combine(p.part_acc, p.part_ml, p.n_splits, (int)(n_q * H), (float *)a.dst->data, a.gate,
                             (int)H, s);
}

}  // namespace sqa
