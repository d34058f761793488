// fa_decode.hip - split-KV FlashAttention over a q4_0 K/V cache for decode and
// speculative verify (n_q <= 4 positions, n_q * H/Hkv <= 16 query rows per KV
// head, 2 KV heads).
//
// Replaces the ggml FLASH_ATTN_EXT node built at src/model/attn.rs:228-251 of
// the reference for n_q = 1..2 (decode step, MTP verify of runner.rs:1263-1270).
//
// Memory pipeline
//   A workgroup (8 wavefronts, one per CU) owns a contiguous key range (a
//   "split") for both KV heads and streams it in 64-key tiles: 64 cache rows of
//   K and of V (288 B each) plus the tile's F16 mask rows. Tiles move from HBM
//   to LDS with global_load_lds_dwordx4 (16 bytes per lane, no registers), into
//   a ring of 4 stages, so three tiles are in flight while one is computed. Each
//   row lands with a 16-byte pad (304-byte LDS rows, a duplicate chunk is
//   fetched into the pad) so that the 16 rows a wavefront reads together fall
//   on different banks. One barrier per tile: after it the tile has landed for
//   every wavefront and the stage computed last is free for the next DMA.
//
// Arithmetic (ggml's CPU flash_attn_ext within fp32 rounding)
//   * QK: Q is rounded to q8_0 per 32-value block as ggml's x86 from_float does
//     (d = amax/127, codes = rint(x * 127/amax)); each q4_0 x q8_0 block dot is
//     the exact integer of ggml's vec_dot, computed on v_mfma_i32_16x16x64_i8:
//     K = 64 covers a block pair, and the B operand is block-diagonal (columns
//     0-7: 8 query rows x even block, columns 8-15: the same rows x odd block),
//     so one MFMA yields both blocks' integers for 16 keys x 8 rows. The 4-bit
//     codes enter unbiased (0..15) and the -8 offset through the accumulator
//     input (-8 * sum(q8)). Each integer is scaled by d_k * d_q in fp32; the
//     softmax scale and log2(e) ride in d_q.
//   * PV: v_mfma_f32_16x16x16_f16 with fp32 accumulation. V is dequantised in
//     registers to the exact (nib - 8) (fp16 integer via 0x6400 | nib) times d_v,
//     rounded once to fp16; P is split into fp16 hi + lo parts (~22 bits).
//   * Online softmax in fp32, base 2.
//   * The four wavefronts of a KV head merge through LDS; splits are merged by
//     fa_combine (fa_combine.hip).
//
// MFMA operand layouts (lane = 16*g + n):
//   16x16x64 i8 : A[n][16g..16g+15]  B[16g..16g+15][n]  C[4g..4g+3][n]
//   16x16x16 f16: A[n][4g..4g+3]     B[4g..4g+3][n]     C[4g..4g+3][n]
#include "common.hpp"

namespace sqa {
namespace {

typedef int int32x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kTileKeys = 64;
constexpr int kStages = 4;
constexpr int kRowBytes = 2 * kHeadRowBytes;          // 288: one cache row, both KV heads
constexpr int kLdsRow = kRowBytes + 16;               // 304
constexpr int kSlotsPerRow = kLdsRow / 16;            // 19 (18 data chunks + pad)
constexpr int kTensorBytes = kTileKeys * kLdsRow;     // 19456
constexpr int kTensorInsts = kTensorBytes / 1024;     // 19 DMA instructions of 64 x 16 B
constexpr int kStageBytes = 2 * kTensorBytes;         // K then V
constexpr int kMaxMaskRows = 4;                       // query positions
constexpr int kMaskStageBytes = kMaxMaskRows * kTileKeys * 2;
constexpr int kMaskOff = kStages * kStageBytes;
constexpr int kCompOff = kMaskOff + kStages * kMaskStageBytes;
constexpr int kCompWaveBytes = 2 * 8 * 16 * 2;        // [K|V][8 blocks][16 keys] fp16 scales
constexpr int kLdsBytes = kCompOff + kWaves * kCompWaveBytes;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kSlack = 8.0f;  // log2 of the largest P the lazy rescale admits
static_assert(kTensorBytes % 1024 == 0, "a tile tensor must be whole DMA instructions");
static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
static_assert(32 * 1024 <= kStageBytes, "Q staging must fit in one stage");

// 16 bytes per lane from sbase + voff into LDS at m0 + 16 * lane. The data
// arrives asynchronously; the caller waits with s_waitcnt vmcnt.
__device__ __forceinline__ void dma16(uint32_t voff, const void *sbase, uint32_t m0v) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(m0v)
                 : "memory");
}

// Wait until at most n vector-memory loads of this wavefront are outstanding
// and its LDS accesses are done, then synchronise the workgroup. n is
// wave-uniform and small.
__device__ __forceinline__ void wait_vm_barrier(int n) {
    switch (n) {
#define SQA_WAIT_CASE(N) \
    case N: asm volatile("s_waitcnt vmcnt(" #N ") lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
        SQA_WAIT_CASE(0) SQA_WAIT_CASE(1) SQA_WAIT_CASE(2) SQA_WAIT_CASE(3) SQA_WAIT_CASE(4)
        SQA_WAIT_CASE(5) SQA_WAIT_CASE(6) SQA_WAIT_CASE(7) SQA_WAIT_CASE(8) SQA_WAIT_CASE(9)
        SQA_WAIT_CASE(10) SQA_WAIT_CASE(11) SQA_WAIT_CASE(12) SQA_WAIT_CASE(13) SQA_WAIT_CASE(14)
        SQA_WAIT_CASE(15) SQA_WAIT_CASE(16) SQA_WAIT_CASE(17) SQA_WAIT_CASE(18) SQA_WAIT_CASE(19)
#undef SQA_WAIT_CASE
        default: asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    }
}

__device__ __forceinline__ uint32_t lds32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }

struct DecodeParams {
    const uint8_t *k, *v;   // cache rows of 288 bytes (both KV heads), row stride 288
    const char *q;          // F32, row (t, h) at q + t*q_nb1 + h*q_nb2, 16-byte aligned
    int64_t q_nb1, q_nb2;
    const char *mask;       // F16 [n_kv] per query row, 16-byte aligned rows, or null
    int64_t mask_nb1;
    int64_t mask_len;       // readable keys per mask row (multiple of 8, >= n_kv)
    int64_t q_pos0;         // >= 0: causal from positions (mask ignored)
    int n_q, H, G, rows;    // rows = n_q * G query rows per KV head
    int64_t n_kv;
    float qscale;           // softmax scale * log2(e)
    int n_splits;
    float *part_acc;        // [n_splits][n_q*H][256]
    float *part_ml;         // [n_splits][n_q*H][2]
};

// Per-lane byte offsets of the tile DMA: slot s = 64*j + lane of instruction j
// holds chunk min(s % 19, 17) of row s / 19 (chunk 18 is the pad).
__device__ __forceinline__ uint32_t tile_slot_offset(int j, int lane) {
    const int s = 64 * j + lane;
    const int row = s / kSlotsPerRow;
    const int col = s - row * kSlotsPerRow;
    return (uint32_t)(row * kRowBytes + (col < 17 ? col : 17) * 16);
}

// TWO = false: up to 8 query rows per KV head (one block-diagonal B set).
// TWO = true : 9..16 rows (rows 0-7 and 8-15 as two B sets, one A operand).
template <bool TWO>
__global__ __launch_bounds__(kThreads, 1) void fa_decode_kernel(DecodeParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in an SGPR
    const int lane = tid & 63;
    const int g = lane >> 4;
    const int n = lane & 15;
    const int kvh = wave >> 2;  // KV head of this wavefront
    const int wq = wave & 3;    // its 16-key quarter of every tile
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

    // ---------------- key range of this split --------------------------------
    const int split = blockIdx.x;
    int64_t k0 = (p.n_kv * split / p.n_splits) & ~(int64_t)7;
    int64_t k1 = split + 1 == p.n_splits ? p.n_kv : ((p.n_kv * (split + 1) / p.n_splits) & ~(int64_t)7);
    if (p.q_pos0 >= 0 && k1 > p.q_pos0 + p.n_q) k1 = p.q_pos0 + p.n_q;  // no row sees past this
    const int n_tiles = k1 > k0 ? (int)((k1 - k0 + kTileKeys - 1) / kTileKeys) : 0;

    // ---------------- DMA plan of this wavefront -----------------------------
    // 19 K + 19 V instructions per tile: K j -> wave j % 8, V j -> wave (j + 3) % 8
    // (waves 0-5 issue 5, waves 6-7 issue 4), the mask rows -> wave 6.
    uint32_t koff[3], voff[3];
    int nk = 0, nv = 0;
#pragma unroll
    for (int r = 0; r < 3; ++r) {
        const int jk = wave + 8 * r;
        const int jv = ((wave + 5) & 7) + 8 * r;
        koff[r] = tile_slot_offset(jk < kTensorInsts ? jk : 0, lane);
        voff[r] = tile_slot_offset(jv < kTensorInsts ? jv : 0, lane);
        nk += jk < kTensorInsts;
        nv += jv < kTensorInsts;
    }
    const bool mask_dma = p.mask && wave == 6;
    const int mrow_l = lane >> 3;  // mask DMA lane -> query row, 16-byte segment
    const uint32_t moff = (uint32_t)((int64_t)(mrow_l < p.n_q ? mrow_l : 0) * p.mask_nb1 + 16 * (lane & 7));
    const int per_tile = nk + nv + (mask_dma ? 1 : 0);  // DMA instructions per tile (wave-uniform)

    auto issue_tile = [&](int t) {
        const int64_t kt = k0 + (int64_t)t * kTileKeys;
        const int st = t & (kStages - 1);
        // keys past the cache end re-read its last row (they are masked off)
        const uint32_t lim = p.n_kv - kt >= kTileKeys ? 0xFFFFFFFFu : (uint32_t)((p.n_kv - kt) * kRowBytes - 16);
        const uint8_t *kb = p.k + kt * kRowBytes;
        const uint8_t *vb = p.v + kt * kRowBytes;
        const uint32_t kbase = lds0 + st * kStageBytes;
        const uint32_t vbase = kbase + kTensorBytes;
#pragma unroll
        for (int r = 0; r < 3; ++r) {
            if (r < nk) dma16(koff[r] < lim ? koff[r] : lim, kb, kbase + 1024u * (wave + 8 * r));
            if (r < nv) dma16(voff[r] < lim ? voff[r] : lim, vb, vbase + 1024u * (((wave + 5) & 7) + 8 * r));
        }
        if (mask_dma) {
            const uint32_t mlim =
                p.mask_len - kt >= kTileKeys + 8 ? 0xFFFFFFFFu : (uint32_t)((p.mask_len - 8 - kt) * 2);
            const uint32_t mo = moff - 16 * (lane & 7) + ((16u * (lane & 7)) < mlim ? 16u * (lane & 7) : mlim);
            if (mrow_l < p.n_q)
                dma16(mo, p.mask + kt * 2, lds0 + kMaskOff + st * kMaskStageBytes);
        }
    };

    // ---------------- Q rows to LDS (stage 3), then the first 3 tiles --------
    const int q_rows = p.n_q * p.H;
    const uint32_t qlds = lds0 + 3 * kStageBytes;
    int q_issued = 0;
    for (int r = wave; r < q_rows; r += kWaves) {
        const int t = r / p.H, h = r - t * p.H;
        dma16(16u * lane, p.q + t * p.q_nb1 + h * p.q_nb2, qlds + 1024u * r);
        ++q_issued;
    }
    const int pre = n_tiles < kStages - 1 ? n_tiles : kStages - 1;
    for (int t = 0; t < pre; ++t) issue_tile(t);
    wait_vm_barrier(per_tile * pre);  // Q landed (tiles may still be in flight)
    (void)q_issued;

    // ---------------- Q -> q8_0 block-diagonal B operands --------------------
    // Column n of C: row r = (n & 7) [+ 8 for the second set], block 2*pair +
    // (n >> 3). Lane (g, n) supplies k = 16g..16g+15, i.e. values 16*(g&1).. of
    // the column's block when (g >> 1) == (n >> 3), zeros otherwise.
    // The four wavefronts of a KV head each quantise one block pair (pair = wq)
    // and exchange the operands through LDS (where the Q rows were).
    constexpr int kSets = TWO ? 2 : 1;
    constexpr int kOpndBytes = 32;  // per lane: 16 code bytes, d_q, -8*sum(q8)
    int32x4 bq[kSets][4];
    float dqs[kSets][4];
    int cinit[kSets][4];
    const bool q_active = (g >> 1) == (n >> 3);
    uint8_t *qs_lds = smem + 3 * kStageBytes;
    {
        int32x4 my_bq[kSets];
        float my_dq[kSets];
        int my_ci[kSets];
        const int pr = wq;
#pragma unroll
        for (int set = 0; set < kSets; ++set) {
            const int r = 8 * set + (n & 7);
            const bool row_ok = r < p.rows;
            const int t = r / p.G;
            const int hq = kvh * p.G + (r - t * p.G);
            const float *qrow = reinterpret_cast<const float *>(qs_lds + (row_ok ? (t * p.H + hq) : 0) * 1024);
            const int blk = 2 * pr + (n >> 3);
            float x[16];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 v4 = *reinterpret_cast<const float4 *>(qrow + 32 * blk + 16 * (g & 1) + 4 * j);
                x[4 * j] = v4.x;
                x[4 * j + 1] = v4.y;
                x[4 * j + 2] = v4.z;
                x[4 * j + 3] = v4.w;
            }
            const bool use = row_ok && q_active;
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                x[j] = use ? x[j] : 0.0f;
                amax = fmaxf(amax, fabsf(x[j]));
            }
            amax = fmaxf(amax, __shfl_xor(amax, 16));  // the other 16 values of the block
            const float d = amax / 127.f;
            const float id = amax != 0.0f ? 127.f / amax : 0.0f;
            int sumq = 0;
            uint32_t w4[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t w = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int qv = (int)rintf(x[4 * j + e] * id);
                    sumq += qv;
                    w |= (uint32_t)(qv & 0xff) << (8 * e);
                }
                w4[j] = w;
            }
            __builtin_memcpy(&my_bq[set], w4, 16);
            sumq += __shfl_xor(sumq, 16);
            const float dqv = (float)(_Float16)d * p.qscale;
            const int civ = -8 * sumq;
            const float dq2 = __shfl_xor(dqv, 32);  // inactive lanes: column n lives in lane ^ 32
            const int ci2 = __shfl_xor(civ, 32);
            my_dq[set] = q_active ? dqv : dq2;
            my_ci[set] = q_active ? civ : ci2;
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // every Q row read
#pragma unroll
        for (int set = 0; set < kSets; ++set) {
            uint8_t *o = qs_lds + (((kvh * 4 + pr) * kSets + set) * 64 + lane) * kOpndBytes;
            *reinterpret_cast<int32x4 *>(o) = my_bq[set];
            *reinterpret_cast<float2 *>(o + 16) = make_float2(my_dq[set], __int_as_float(my_ci[set]));
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // operands published
#pragma unroll
        for (int pp = 0; pp < 4; ++pp)
#pragma unroll
            for (int set = 0; set < kSets; ++set) {
                const uint8_t *o = qs_lds + (((kvh * 4 + pp) * kSets + set) * 64 + lane) * kOpndBytes;
                bq[set][pp] = *reinterpret_cast<const int32x4 *>(o);
                const float2 dc = *reinterpret_cast<const float2 *>(o + 16);
                dqs[set][pp] = dc.x;
                cinit[set][pp] = __float_as_int(dc.y);
            }
    }
    // This lane's logit row (column n of the combined C): query position and validity.
    const int my_r = TWO ? n : (n & 7);
    const bool my_ok = my_r < p.rows;
    const int my_t = my_ok ? my_r / p.G : 0;

    // ---------------- per-lane constants --------------------------------------
    uint32_t magic;  // fp16 0x6400 = 1024 in both halves; in a VGPR so v_and_or_b32 takes it
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
    const half2v off8 = {(_Float16)-1032.0f, (_Float16)-1032.0f};  // 1024 + 8
    // K operand: lane (g, n) reads key n's block 2*pair + (g >> 1), nibbles of half g & 1.
    // qs of block b sits at 18b + 2 in the head row: 4-aligned for odd b, 2 mod 4 for even b.
    const int ka_blk_par = g >> 1;
    const uint32_t ka_shift = (ka_blk_par ? 0u : 16u) + 4u * (uint32_t)(g & 1);
    // V operand: byte n of a block's qs; dword at (18b + 2 + n) & ~3, byte (18b + 2 + n) & 3.
    const uint32_t vsel_e = (uint32_t)((2 + n) & 3);  // even b
    const uint32_t vsel_o = (uint32_t)((0 + n) & 3);  // odd b (18b + 2 = 0 mod 4)
    const uint32_t psel_e = vsel_e | (0x0cu << 8) | ((4u + vsel_e) << 16) | (0x0cu << 24);
    const uint32_t psel_o = vsel_o | (0x0cu << 8) | ((4u + vsel_o) << 16) | (0x0cu << 24);
    uint8_t *comp = smem + kCompOff + wave * kCompWaveBytes;  // [K|V][8][16] fp16

    floatx4 acc[16];  // O[row 4g+i][dim 16T + n]
#pragma unroll
    for (int T = 0; T < 16; ++T) acc[T] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;  // base-2 running max of row my_r
    float l_part = 0.0f;      // this lane's share of the row's sum

    for (int t = 0; t < n_tiles; ++t) {
        // tile t landed for this wavefront once only the younger tiles are pending
        const int younger = (n_tiles - 1 - t) < (kStages - 2) ? (n_tiles - 1 - t) : (kStages - 2);
        wait_vm_barrier(per_tile * younger);
        if (t + kStages - 1 < n_tiles) issue_tile(t + kStages - 1);

        const int64_t kt = k0 + (int64_t)t * kTileKeys;
        const int st = t & (kStages - 1);
        const uint8_t *sK = smem + st * kStageBytes + kvh * kHeadRowBytes;
        const uint8_t *sV = sK + kTensorBytes;
        const int key0 = 16 * wq;  // first key of this wavefront in the tile

        // a tile holding keys past the range end or past a causal limit
        const bool tail = kt + kTileKeys > k1 || (p.q_pos0 >= 0 && kt + kTileKeys - 1 > p.q_pos0);

        // The wavefront's 16 keys enter the MFMAs permuted: row r of the QK A
        // operand (and k index r of the PV operands) is key key0 + (r >> 2) + 4*(r & 3),
        // so lane group g holds keys key0 + g + 4i (i = 0..3) and the four groups
        // read V from consecutive LDS rows (distinct banks).
        // -- compact d_k and d_v of those keys, [K|V][block][4g + i] ------------
        {
            const int tensor = lane >> 5, blk = (lane >> 2) & 7, gg = lane & 3;
            const uint8_t *src = (tensor ? sV : sK) + (key0 + gg) * kLdsRow + 18 * blk;
            uint32_t d0 = *reinterpret_cast<const uint16_t *>(src);
            uint32_t d1 = *reinterpret_cast<const uint16_t *>(src + 4 * kLdsRow);
            uint32_t d2 = *reinterpret_cast<const uint16_t *>(src + 8 * kLdsRow);
            uint32_t d3 = *reinterpret_cast<const uint16_t *>(src + 12 * kLdsRow);
            if (tail) {  // rows past the range may hold any bytes: zero scales keep P*V finite
                const int64_t kq = kt + key0 + gg;
                d0 = kq < k1 ? d0 : 0u;
                d1 = kq + 4 < k1 ? d1 : 0u;
                d2 = kq + 8 < k1 ? d2 : 0u;
                d3 = kq + 12 < k1 ? d3 : 0u;
            }
            *reinterpret_cast<uint2 *>(comp + ((tensor * 8 + blk) * 16 + 4 * gg) * 2) =
                make_uint2(d0 | (d1 << 16), d2 | (d3 << 16));
        }

        // -- QK: xs[i] = S[key key0+g+4i][row of column n] --------------------
        float xs[kSets][4];
#pragma unroll
        for (int set = 0; set < kSets; ++set)
#pragma unroll
            for (int i = 0; i < 4; ++i) xs[set][i] = 0.0f;
        const uint8_t *krow = sK + (key0 + (n >> 2) + 4 * (n & 3)) * kLdsRow;
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
            // key of A row n, block 2*pair + (g >> 1): five dwords from the aligned
            // address below its 16 qs bytes, shifted to the nibble half g & 1
            const uint8_t *ap = krow + ((18 * (2 * pr + ka_blk_par) + 2) & ~3);
            const uint32_t w0 = lds32(ap), w1 = lds32(ap + 4), w2 = lds32(ap + 8), w3 = lds32(ap + 12),
                           w4 = lds32(ap + 16);
            uint32_t aw[4];
            aw[0] = __builtin_amdgcn_alignbit(w1, w0, ka_shift) & 0x0F0F0F0Fu;
            aw[1] = __builtin_amdgcn_alignbit(w2, w1, ka_shift) & 0x0F0F0F0Fu;
            aw[2] = __builtin_amdgcn_alignbit(w3, w2, ka_shift) & 0x0F0F0F0Fu;
            aw[3] = __builtin_amdgcn_alignbit(w4, w3, ka_shift) & 0x0F0F0F0Fu;
            int32x4 aop;
            __builtin_memcpy(&aop, aw, 16);
            const uint2 dk2 = *reinterpret_cast<const uint2 *>(comp + ((2 * pr + (n >> 3)) * 16 + 4 * g) * 2);
            half4 dkh;  // d_k of keys key0+g+4i, block of column n
            __builtin_memcpy(&dkh, &dk2, 8);
#pragma unroll
            for (int set = 0; set < kSets; ++set) {
                const int ci = cinit[set][pr];
                int32x4 c = {ci, ci, ci, ci};
                c = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop, bq[set][pr], c, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) xs[set][i] = fmaf((float)c[i] * dqs[set][pr], (float)dkh[i], xs[set][i]);
            }
        }
        // even-block half (columns 0-7) + odd-block half (columns 8-15) of each logit
        float s[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (TWO) {  // lanes n < 8 take rows 0-7 (set 0), lanes n >= 8 rows 8-15 (set 1)
                const float u = n < 8 ? xs[0][i] : xs[1][i];
                const float w = n < 8 ? xs[1][i] : xs[0][i];
                s[i] = u + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(w), 0x128, 0xf, 0xf, false));
            } else {
                s[i] = xs[0][i] +
                       __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(xs[0][i]), 0x128, 0xf, 0xf, false));
            }
        }
        // mask (F16, base-e units) and the ragged / causal tail
        if (p.mask) {
            const uint16_t *mrow = reinterpret_cast<const uint16_t *>(smem + kMaskOff + st * kMaskStageBytes) +
                                   my_t * kTileKeys + key0 + g;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint16_t mb = mrow[4 * i];
                _Float16 mh;
                __builtin_memcpy(&mh, &mb, 2);
                s[i] = fmaf((float)mh, kLog2e, s[i]);
            }
        }
        if (tail) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t key = kt + key0 + g + 4 * i;
                bool dead = key >= k1;
                if (p.q_pos0 >= 0) dead = dead || key > p.q_pos0 + my_t;
                s[i] = dead ? -INFINITY : s[i];
            }
        }
        // -- online softmax of row my_r over the wavefront's 16 keys ------------
        // The reference max m_run moves only when a logit exceeds it by more than
        // kSlack (base 2): the common path needs no cross-lane max and no rescale;
        // P stays below 2^kSlack, which the fp16 hi/lo split and fp32 sums carry.
        const float lim = m_run + kSlack;
        if (__any((s[0] > lim) | (s[1] > lim) | (s[2] > lim) | (s[3] > lim))) {
            float mt = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
            mt = fmaxf(mt, __shfl_xor(mt, 16));
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float m_new = fmaxf(m_run, mt);
            const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            l_part *= alpha;
            m_run = m_new;
            float ar[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) ar[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
            for (int T = 0; T < 16; ++T)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[T][i] *= ar[i];
        }
        const float mref = m_run == -INFINITY ? 0.0f : m_run;
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pv[i] = __builtin_amdgcn_exp2f(s[i] - mref);
        l_part += (pv[0] + pv[1]) + (pv[2] + pv[3]);
        half4 pa_hi, pa_lo;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const _Float16 h = (_Float16)pv[i];
            pa_hi[i] = h;
            pa_lo[i] = (_Float16)(pv[i] - (float)h);
        }
        // -- O += P V, two blocks (four 16-dim tiles) at a time ----------------
        const uint8_t *vr0 = sV + (key0 + g) * kLdsRow;  // keys key0+g+4i at +4i rows
#pragma unroll
        for (int bb = 0; bb < 8; bb += 2) {
            half4 bv[4];
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int b = bb + h2;
                const int vo = (18 * b + 2 + n) & ~3;  // this lane's dword of block b's qs
                const uint32_t x0 = lds32(vr0 + vo), x1 = lds32(vr0 + 4 * kLdsRow + vo),
                               x2 = lds32(vr0 + 8 * kLdsRow + vo), x3 = lds32(vr0 + 12 * kLdsRow + vo);
                const uint32_t sel = (b & 1) ? psel_o : psel_e;
                const uint32_t t01 = __builtin_amdgcn_perm(x1, x0, sel);  // keys i=0,1 -> bits 0-7, 16-23
                const uint32_t t23 = __builtin_amdgcn_perm(x3, x2, sel);
                const uint2 dv2 = *reinterpret_cast<const uint2 *>(comp + ((8 + b) * 16 + 4 * g) * 2);
                half2v dv01, dv23;
                __builtin_memcpy(&dv01, &dv2.x, 4);
                __builtin_memcpy(&dv23, &dv2.y, 4);
                const uint32_t l01 = (t01 & 0x000F000Fu) | magic, l23 = (t23 & 0x000F000Fu) | magic;
                const uint32_t h01 = ((t01 >> 4) & 0x000F000Fu) | magic, h23 = ((t23 >> 4) & 0x000F000Fu) | magic;
                half2v a, c, e, f;
                __builtin_memcpy(&a, &l01, 4);
                __builtin_memcpy(&c, &l23, 4);
                __builtin_memcpy(&e, &h01, 4);
                __builtin_memcpy(&f, &h23, 4);
                a = (a + off8) * dv01;  // (nib - 8) * d_v
                c = (c + off8) * dv23;
                e = (e + off8) * dv01;
                f = (f + off8) * dv23;
                bv[2 * h2] = half4{a[0], a[1], c[0], c[1]};
                bv[2 * h2 + 1] = half4{e[0], e[1], f[0], f[1]};
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[2 * bb + j] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa_hi, bv[j], acc[2 * bb + j], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[2 * bb + j] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa_lo, bv[j], acc[2 * bb + j], 0, 0, 0);
        }
    }

    // ---------------- merge the 4 wavefronts of each KV head -------------------
    l_part += __shfl_xor(l_part, 16);
    l_part += __shfl_xor(l_part, 32);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");  // ring free for reuse
    constexpr int kRowsUsed = TWO ? 16 : 8;
    float *sML = reinterpret_cast<float *>(smem + kMaskOff);  // [2][4][16][2]
    if (g == 0) {
        sML[((kvh * 4 + wq) * 16 + n) * 2 + 0] = m_run;
        sML[((kvh * 4 + wq) * 16 + n) * 2 + 1] = l_part;
    }
    __syncthreads();
    // sAcc[kvh][wq][T][n][quad]: float4 of rows 4q..4q+3 per (T, n), the quad
    // index XOR-swizzled with (n >> 1) & 3 so that 8 consecutive n of one quad
    // hit 8 distinct bank groups (conflict-free 16-byte accesses).
    float *sAcc = reinterpret_cast<float *>(smem);
    if (4 * g < kRowsUsed) {
        float fac[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 4 * g + i;
            float M = -INFINITY;
#pragma unroll
            for (int w2 = 0; w2 < 4; ++w2) M = fmaxf(M, sML[((kvh * 4 + w2) * 16 + row) * 2]);
            const float mw = sML[((kvh * 4 + wq) * 16 + row) * 2];
            fac[i] = mw == -INFINITY ? 0.0f : exp2f(mw - M);
        }
#pragma unroll
        for (int T = 0; T < 16; ++T) {
            const float4 o = make_float4(acc[T][0] * fac[0], acc[T][1] * fac[1], acc[T][2] * fac[2], acc[T][3] * fac[3]);
            *reinterpret_cast<float4 *>(sAcc + ((((kvh * 4 + wq) * 16 + T) * 16 + n) * 16 + 4 * (g ^ ((n >> 1) & 3)))) = o;
        }
    }
    __syncthreads();
    // ---------------- this split's partials ------------------------------------
    const int rows_total = p.n_q * p.H;
    constexpr int kQuads = kRowsUsed / 4;
    for (int e = tid; e < 2 * 16 * 16 * kQuads; e += kThreads) {
        const int nn = e % 16;  // consecutive threads: consecutive dims of one row
        const int rq = (e / 16) % kQuads;
        const int T = (e / (16 * kQuads)) % 16;
        const int kh = e / (kQuads * 256);
        float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) {
            const float4 v4 = *reinterpret_cast<const float4 *>(
                sAcc + ((((kh * 4 + w2) * 16 + T) * 16 + nn) * 16 + 4 * (rq ^ ((nn >> 1) & 3))));
            sum.x += v4.x;
            sum.y += v4.y;
            sum.z += v4.z;
            sum.w += v4.w;
        }
        const float sv[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 4 * rq + i;
            if (row < p.rows) {
                const int tq = row / p.G, hq = kh * p.G + row % p.G;
                p.part_acc[((int64_t)split * rows_total + (int64_t)tq * p.H + hq) * 256 + 16 * T + nn] = sv[i];
            }
        }
    }
    if (tid < 2 * 16) {
        const int kh = tid >> 4, row = tid & 15;
        if (row < p.rows) {
            float M = -INFINITY, L = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < 4; ++w2) M = fmaxf(M, sML[((kh * 4 + w2) * 16 + row) * 2]);
#pragma unroll
            for (int w2 = 0; w2 < 4; ++w2) {
                const float mw = sML[((kh * 4 + w2) * 16 + row) * 2];
                if (mw != -INFINITY) L += sML[((kh * 4 + w2) * 16 + row) * 2 + 1] * exp2f(mw - M);
            }
            const int tq = row / p.G, hq = kh * p.G + row % p.G;
            const int64_t ridx = (int64_t)split * rows_total + (int64_t)tq * p.H + hq;
            p.part_ml[ridx * 2 + 0] = M == -INFINITY ? M : M * kLn2;  // combine works in base e
            p.part_ml[ridx * 2 + 1] = L;
        }
    }
}

// Copies an F16 mask whose rows are unaligned or whose length is not a
// multiple of 8 into [n_q][len8] rows (len8 = n_kv rounded up to 8, -inf pad).
__global__ __launch_bounds__(256) void mask_pack_kernel(const char *__restrict__ src, int64_t nb1, int64_t n_kv,
                                                        int n_q, int64_t len8, uint16_t *__restrict__ dst) {
    const int64_t total = len8 * n_q;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t t = i / len8, k = i - t * len8;
        dst[i] = k < n_kv ? reinterpret_cast<const uint16_t *>(src + t * nb1)[k] : (uint16_t)0xFC00;
    }
}

int decode_splits(int64_t n_kv) {
    int64_t s = (n_kv + 255) / 256;  // at least ~4 tiles per split
    const int64_t cap = device_cu_count();
    if (s > cap) s = cap;
    if (s < 1) s = 1;
    return (int)s;
}

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

size_t fa_decode_workspace(int64_t n_q, int64_t H, int64_t n_kv) {
    const int64_t splits = decode_splits(n_kv);
    const size_t acc = al256((size_t)(splits * n_q * H * 256) * sizeof(float));
    const size_t ml = al256((size_t)(splits * n_q * H * 2) * sizeof(float));
    const size_t mask = al256((size_t)(n_q * ((n_kv + 7) / 8 * 8)) * 2);
    return acc + ml + mask + 256;
}

int launch_fa_decode(const FaArgs &a, hipStream_t s) {
    const sqa_tensor &q = *a.q, &k = *a.k;
    const int64_t n_q = q.ne[1], H = q.ne[2], n_kv = k.ne[1], Hkv = k.ne[2];
    if (Hkv != 2) return set_error(SQA_ERR_UNSUPPORTED, "decode kernel built for 2 KV heads");
    if (n_q > kMaxMaskRows) return set_error(SQA_ERR_UNSUPPORTED, "decode kernel takes at most 4 query positions");
    DecodeParams p;
    p.k = (const uint8_t *)k.data;
    p.v = (const uint8_t *)a.v->data;
    p.q = (const char *)q.data;
    p.q_nb1 = (int64_t)q.nb[1];
    p.q_nb2 = (int64_t)q.nb[2];
    p.q_pos0 = a.q_pos0;
    p.n_q = (int)n_q;
    p.H = (int)H;
    p.G = (int)(H / Hkv);
    p.rows = (int)(n_q * p.G);
    p.n_kv = n_kv;
    p.qscale = a.scale * kLog2e;
    p.n_splits = decode_splits(n_kv);
    const size_t need = fa_decode_workspace(n_q, H, n_kv);
    if (!a.ws || a.ws_bytes < need)
        return set_error(SQA_ERR_WORKSPACE, "flash_attn_ext: workspace %zu bytes < %zu needed", a.ws_bytes, need);
    uint8_t *wsb = reinterpret_cast<uint8_t *>(((uintptr_t)a.ws + 255) & ~(uintptr_t)255);
    p.part_acc = reinterpret_cast<float *>(wsb);
    p.part_ml = reinterpret_cast<float *>(wsb + al256((size_t)(p.n_splits * n_q * H * 256) * sizeof(float)));
    uint16_t *mask_copy = reinterpret_cast<uint16_t *>(reinterpret_cast<uint8_t *>(p.part_ml) +
                                                       al256((size_t)(p.n_splits * n_q * H * 2) * sizeof(float)));
    p.mask = nullptr;
    p.mask_nb1 = 0;
    p.mask_len = 0;
    if (a.q_pos0 < 0 && a.mask) {
        const char *m = (const char *)a.mask->data;
        const int64_t nb1 = (int64_t)a.mask->nb[1];
        if ((uintptr_t)m % 16 == 0 && nb1 % 16 == 0 && n_kv % 8 == 0) {
            p.mask = m;
            p.mask_nb1 = nb1;
            p.mask_len = n_kv;
        } else {
            const int64_t len8 = (n_kv + 7) / 8 * 8;
            const int64_t total = len8 * n_q;
            int64_t grid = (total + 255) / 256;
            if (grid > 1024) grid = 1024;
            mask_pack_kernel<<<dim3((unsigned)grid), dim3(256), 0, s>>>(m, nb1, n_kv, (int)n_q, len8, mask_copy);
            p.mask = (const char *)mask_copy;
            p.mask_nb1 = len8 * 2;
            p.mask_len = len8;
        }
    }
    static bool lds_ok = false;
    if (!lds_ok) {
        hipError_t e = hipFuncSetAttribute((const void *)fa_decode_kernel<false>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void *)fa_decode_kernel<true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    kLdsBytes);
        if (e != hipSuccess) return hip_status(e, "fa_decode LDS attribute");
        lds_ok = true;
    }
    const int prof = profile_start("fa_decode", s);
    if (p.rows <= 8)
        fa_decode_kernel<false><<<dim3((unsigned)p.n_splits), dim3(kThreads), kLdsBytes, s>>>(p);
    else
        fa_decode_kernel<true><<<dim3((unsigned)p.n_splits), dim3(kThreads), kLdsBytes, s>>>(p);
    profile_stop(prof, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_status(e, "fa_decode launch");
    return launch_fa_combine(p.part_acc, p.part_ml, p.n_splits, (int)(n_q * H), (float *)a.dst->data, a.gate,
                             (int)H, s);
}

}  // namespace sqa
