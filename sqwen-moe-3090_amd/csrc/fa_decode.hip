// fa_decode.hip - split-KV FlashAttention over a q4_0 K/V cache for decode and
// speculative verify (n_q <= 4 positions, n_q * H/Hkv <= 16 query rows per KV
// head, any number of KV heads).
//
// Replaces the ggml FLASH_ATTN_EXT node built at src/model/attn.rs:228-251 of
// the reference for n_q = 1..2 (decode step, MTP verify of runner.rs:1263-1270).
//
// Work split
//   The key range is cut into splits, about two workgroups per CU in all. Each
//   split is served by one workgroup per KV head, all placed by the dispatcher
//   on the same XCD (so the cache lines the heads share in a cache row of
//   Hkv x 144 bytes are fetched from HBM once and served to the other heads'
//   workgroups by that XCD's L2); two workgroups fit on a CU, so one's
//   wavefronts can issue while the other's wait at their barrier. Of the two
//   workgroups on a CU the one dispatched first wins the issue arbitration
//   (older wavefronts go first) and runs about twice as fast while both are
//   resident, so the splits of the first dispatch round take twice the tiles
//   of the second: both rounds then end together (measured at 172K keys: 27.0
//   us against 28.6 us for equal splits, whose second round runs on alone for
//   the last tiles). A workgroup (8 wavefronts) walks its split
//   in 64-key tiles: four score wavefronts (16-key quarter w of every tile)
//   compute the logits and the softmax weights P of tile t; four value
//   wavefronts (64-dim slice v of the output) accumulate P V of tile t-1 over
//   all 64 keys of that tile. P crosses from score to value wavefronts through
//   LDS, one tile behind, so one barrier per tile serves both. A value
//   wavefront owns its output dims outright: there is no merge of O.
//
// Memory pipeline
//   Tiles move from HBM to LDS with global_load_lds_dwordx4 (16 bytes per lane,
//   no registers): the head's 144 bytes of each 288-byte cache row land in a
//   144-byte LDS row (nine chunks, 36 dwords: one column of 32 rows spans 8
//   bank positions, a 160-byte row only 4). K (and the tile's F16
//   mask rows) go into a ring of 3 stages, issued 2 tiles ahead of the QK that
//   reads them; V into a ring of 3 stages, issued 1 tile ahead of its tile's QK,
//   i.e. 2 ahead of the PV that reads it. LDS rows rotate their chunks so that
//   the rows a wavefront reads together sit on different banks: K rows 8-15 of
//   each 16-row group by one chunk, V rows by two chunks per 8-row group.
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
//   * Softmax: base 2, fp32. The reference max of a row moves only when a logit
//     exceeds it by more than kSlack, so P <= 2^kSlack and the common tile needs
//     no rescale. A score wavefront that sees such a logit uses the larger max
//     for its own P and raises a flag; on the next tile every wavefront of the
//     workgroup reads the four maxima used, takes their maximum, and rescales
//     its share (l, O, and the P values of that tile) onto it. In the form of
//     up to 8 rows, the four score wavefronts exchange their row maxima on a
//     split's first tile (one more barrier), so that tile starts from the
//     common maximum and nothing is rescaled; the 16-row form has no registers
//     to spare for it (two workgroups per CU need <= 128 VGPRs).
//   * PV: v_mfma_f32_16x16x32_f16 with fp32 accumulation, d_v on the A side:
//     A = P d_v 2^E of the block as an exact fp16 hi + lo pair (P arrives as an
//     fp16 hi + lo pair, ~22 bits), B = the nibbles: one v_and per two keys
//     leaves the fp16 subnormal nib * 2^-24 for the low nibble, which one packed
//     multiply by 2^14 lifts to nib * 2^-10 (as a subnormal 2^-24 deep, the
//     MFMA's fp32 sums lost up to ~2^-12 of the output at long contexts), and nib
//     * 2^-20 for the high nibble; the -8 offset comes in as -8 * sum A from one
//     more MFMA against ones. Every product is exact in fp32, so a row
//     that a few keys dominate carries no fp16
//     rounding of V or P into its output (ggml's CPU path dequantizes V to fp32
//     exactly). P is kept at 2^-4 of its value (<= 16); 2^E is one power of
//     two per value wavefront that puts the largest |d_v| it has seen near 2^8
//     (lowered, with O rescaled, when a larger one comes), so A stays finite
//     and clear of fp16 subnormals for V of any size. With up to 8 query rows,
//     A rows 8-15 carry the lo parts of rows 0-7, so one set of three MFMAs
//     per half tile and block serves both parts (C rows r and r + 8 are added
//     at the end).
//   * A key that no row of the call sees (masked in every row, past the split
//     or past the cache end) contributes exactly 0 whatever its bytes, as in
//     ggml's CPU loop, which skips masked keys: a -inf mask entry replaces the
//     logit, and the score wavefronts publish which keys have P != 0 in some
//     row, so the value wavefronts zero the others' V scales.
//   * Splits are merged by fa_combine (fa_combine.hip). The partials are
//     written through to memory (store_through), so the end of the kernel has
//     no dirty L2 lines of them to write back.
//
// MFMA operand layouts (lane = 16*g + n):
//   16x16x64 i8 : A[n][16g..16g+15]  B[16g..16g+15][n]  C[4g..4g+3][n]
//   16x16x32 f16: A[n][8g..8g+7]     B[8g..8g+7][n]     C[4g..4g+3][n]
#include <mutex>
#include <vector>

#include "common.hpp"

namespace sqa {
namespace {

typedef int int32x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int kScoreWaves = 4;
constexpr int kValueWaves = 4;
constexpr int kWaves = kScoreWaves + kValueWaves;
constexpr int kThreads = 64 * kWaves;
constexpr int kTileKeys = 64;
constexpr int kKStages = 3;
constexpr int kVStages = 3;
constexpr int kSlotsPerRow = 9;                       // the head row's 9 chunks
constexpr int kLdsRow = 16 * kSlotsPerRow;            // 144
constexpr int kTensorBytes = kTileKeys * kLdsRow;     // 9216
constexpr int kTensorInsts = kTensorBytes / 1024;     // 9 DMA instructions of 64 x 16 B
constexpr int kMaxMaskRows = 4;                       // query positions
constexpr int kMaskStageBytes = kMaxMaskRows * kTileKeys * 2;
constexpr int kPRow = 136;                            // fp16 P row: 64 keys hi, 64 keys lo, 8 pad
// LDS map
constexpr int kOffV = kKStages * kTensorBytes;
constexpr int kOffMask = kOffV + kVStages * kTensorBytes;
constexpr int kOffDk = kOffMask + kKStages * kMaskStageBytes;  // per score wave [8 blocks][16 keys] fp16
constexpr int kOffDv = kOffDk + kScoreWaves * 256;             // per value wave [2 blocks][2 halves][4][8] fp16
constexpr int kOffP = kOffDv + kValueWaves * 256;              // [2 tiles][16 rows][kPRow] fp16 hi|lo
constexpr int kOffM = kOffP + 2 * 16 * kPRow * 2;              // [2 tiles][4 waves][16 rows] f32
constexpr int kOffFlag = kOffM + 2 * 4 * 16 * 4;               // [2 tiles][4 waves] u32
constexpr int kOffL = kOffFlag + 2 * 4 * 4;                    // [4 waves][16 rows] f32
constexpr int kLdsBytes = kOffL + 4 * 16 * 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kSlack = 8.0f;  // log2 of the largest P the lazy rescale admits
// P is stored as P 2^-kPShift (<= 2^(kSlack - kPShift) = 16) and l summed from the
// same values; with |d_v 2^E| < 2^11, A = P d_v 2^E stays below 2^15.
constexpr float kPShift = 4.0f;
// Largest d_v exponent E of the value wavefronts (d_v enters A as d_v 2^E): V
// scales below 2^-20 lose low bits of A; 2^E stays two fp16 powers of two.
constexpr int kMaxDvExp = 28;
// Tile shares of a first-round and a second-round split when two workgroups
// share each CU (see launch_fa_decode).
constexpr int kFirstRoundWeight = 2;
constexpr int kSecondRoundWeight = 1;
static_assert(kTensorBytes % 1024 == 0, "a tile tensor must be whole DMA instructions");
static_assert(2 * kLdsBytes <= 160 * 1024, "two workgroups per CU");
static_assert(4 * 2 * 64 * 32 <= (kVStages - 1) * kTensorBytes, "Q operands must fit in V stages 1..2");

// 16 bytes per lane from sbase + voff into LDS at m0 + 16 * lane. The data
// arrives asynchronously; the caller waits with s_waitcnt vmcnt.
// sbase and m0v are wave-uniform; readfirstlane keeps them in SGPRs even where
// the compiler has placed them in VGPRs.
__device__ __forceinline__ void dma16(uint32_t voff, const void *sbase, uint32_t m0v) {
    const uint64_t b = (uint64_t)(uintptr_t)sbase;
    const uint64_t bs = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(b >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    const uint32_t ms = (uint32_t)__builtin_amdgcn_readfirstlane((int)m0v);
    // m0 as an operand: the compiler writes it and knows it holds the LDS base
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(bs), "{m0}"(ms) : "memory");
}

typedef const __attribute__((address_space(3))) uint32_t lds_u32;  // LDS dword from a raw LDS address

__device__ __forceinline__ uint32_t lds32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }
__device__ __forceinline__ uint32_t lds16(const uint8_t *p) { return *reinterpret_cast<const uint16_t *>(p); }

// Largest of a non-negative value over the 64 lanes, in a scalar register: DPP
// row shifts fold each row of 16 into its last lane, row broadcasts fold rows
// into lane 63 (lanes without a source keep their own value).
__device__ __forceinline__ int wave_max_u16(uint32_t v) {
    int x = (int)v;
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x111, 0xf, 0xf, false));  // row_shr:1
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x112, 0xf, 0xf, false));  // row_shr:2
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x114, 0xf, 0xf, false));  // row_shr:4
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x118, 0xf, 0xf, false));  // row_shr:8
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x142, 0xa, 0xf, false));  // row_bcast:15
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x143, 0xc, 0xf, false));  // row_bcast:31
    return __builtin_amdgcn_readlane(x, 63);
}

// Exchanges with lane ^ 16 and lane ^ 32 through gfx950's row swaps (VALU, no
// LDS round trip): a swap of x with itself returns x and the partner's x in the
// two halves of its result, in an order that depends on the lane.
__device__ __forceinline__ float xmax16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xmax32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xsum16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xsum32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ int xsum16(int x) {
    const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)x, (uint32_t)x, false, false);
    return (int)(r[0] + r[1]);
}
__device__ __forceinline__ uint32_t or16(uint32_t x) {  // x | x of lane ^ 16
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return r[0] | r[1];
}
__device__ __forceinline__ uint32_t or32(uint32_t x) {  // x | x of lane ^ 32
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return r[0] | r[1];
}
// x of lane ^ 32: lanes 0-31 find it in the swapped source, lanes 32-63 in the
// swapped destination
__device__ __forceinline__ int xother32(int x) {
    const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)x, (uint32_t)x, false, false);
    return (int)((threadIdx.x & 32) ? r[0] : r[1]);
}

// a * b - c in packed fp16, the negation as an operand modifier (written as
// -c in C, the backend lowers the negation of the first pair as three VALU)
__device__ __forceinline__ half8 fma_minus(half8 a, half8 b, half8 c) {
    uint32_t x[4], y[4], z[4], r[4];
    __builtin_memcpy(x, &a, 16);
    __builtin_memcpy(y, &b, 16);
    __builtin_memcpy(z, &c, 16);
#pragma unroll
    for (int m = 0; m < 4; ++m)
        asm("v_pk_fma_f16 %0, %1, %2, %3 neg_lo:[0,0,1] neg_hi:[0,0,1]" : "=v"(r[m]) : "v"(x[m]), "v"(y[m]), "v"(z[m]));
    half8 o;
    __builtin_memcpy(&o, r, 16);
    return o;
}

__device__ __forceinline__ float exp2_or_zero(float a, float b) {  // 2^(a-b), 0 when a = -inf
    return a == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(a - b);
}

struct DecodeParams {
    const uint8_t *k, *v;   // cache rows of row_bytes = n_kvh x 144 bytes (all KV heads)
    int64_t row_bytes;
    int n_kvh;              // KV heads
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
    // Split s covers tiles [c(s) * tiles / cw_total, c(s + 1) * tiles / cw_total)
    // with c(s) = w_first * s for s < n_first, else w_first * n_first +
    // w_second * (s - n_first): a split of the first dispatch round weighs w_first.
    int64_t tiles, cw_total;
    int n_first, w_first, w_second;
    float *part_acc;        // [n_splits][n_q*H][256]
    float *part_ml;         // [n_splits][n_q*H][2]
};

// Chunk rotation of an LDS row: K rows 8-15 of every 16-row group start one
// slot later, V rows two slots later per 8-row group (mod kSlotsPerRow).
__device__ __forceinline__ int k_rot(int row) { return (row >> 3) & 1; }
__device__ __forceinline__ int v_rot(int row) { return 2 * ((row >> 3) & 3); }

// Per-lane source offset of DMA instruction j of a tile stage: slot s = 64*j +
// lane lands at LDS byte 16*s, i.e. slot s % 9 of row s / 9, and holds chunk
// (slot - rot) mod 9 of that row's head half.
template <bool V>
__device__ __forceinline__ uint32_t slot_offset(int j, int lane, int kvh, uint32_t row_bytes) {
    const int s = 64 * j + lane;
    const int row = s / kSlotsPerRow;
    const int slot = s - row * kSlotsPerRow;
    int c = slot - (V ? v_rot(row) : k_rot(row));
    c = c < 0 ? c + kSlotsPerRow : c;
    return (uint32_t)row * row_bytes + (uint32_t)(kvh * kHeadRowBytes + c * 16);
}
// LDS byte of head-row byte c (0..143) of row `row` inside a tile stage
template <bool V>
__device__ __forceinline__ int lds_byte(int row, int c) {
    int slot = (c >> 4) + (V ? v_rot(row) : k_rot(row));
    slot = slot >= kSlotsPerRow ? slot - kSlotsPerRow : slot;
    return row * kLdsRow + slot * 16 + (c & 15);
}

// TWO = false: up to 8 query rows per KV head (one block-diagonal B set).
// TWO = true : 9..16 rows (rows 0-7 and 8-15 as two B sets, one A operand).
// Both forms must stay within 128 VGPRs so that two workgroups share a CU: the
// 8-row form is held there by its bound (4 waves per SIMD); the 16-row form
// allocates 127 by itself and spills if it is bound the same way.
template <bool TWO>
__global__ __launch_bounds__(kThreads, TWO ? 2 : 4) void fa_decode_kernel(DecodeParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, in an SGPR
    const int lane = tid & 63;
    const int g = lane >> 4;
    const int n = lane & 15;
    const bool score = wave < kScoreWaves;
    const int wq = wave & 3;  // score: 16-key quarter of every tile; value: 64-dim slice
    // LDS byte address of smem, computed once: the cast carries a null check the
    // compiler would otherwise repeat at every use
    uint32_t lds0 = (uint32_t)(uintptr_t)smem;
    asm volatile("" : "+s"(lds0));
    constexpr int kRowMask = TWO ? 15 : 7;  // rows 8-15 mirror rows 0-7 when only 8 exist

    // ---------------- split and KV head of this workgroup ---------------------
    // Workgroups go round-robin to the 8 XCDs: ids 8 Hkv a + 8h + x (x < 8) are
    // split 8a + x, head h, so all heads of a split share an XCD (and its L2).
    const int id = blockIdx.x;
    const int hb = id >> 3;
    const int sa = hb / p.n_kvh;
    const int kvh = hb - sa * p.n_kvh;
    const int split = (sa << 3) | (id & 7);
    auto cw = [&](int s) -> int64_t {
        return s < p.n_first ? (int64_t)p.w_first * s
                             : (int64_t)p.w_first * p.n_first + (int64_t)p.w_second * (s - p.n_first);
    };
    const int64_t t_begin = cw(split) * p.tiles / p.cw_total;
    const int64_t t_end = cw(split + 1) * p.tiles / p.cw_total;
    const int64_t k0 = t_begin * kTileKeys;
    int64_t k1 = t_end * kTileKeys;
    if (k1 > p.n_kv) k1 = p.n_kv;
    if (p.q_pos0 >= 0 && k1 > p.q_pos0 + p.n_q) k1 = p.q_pos0 + p.n_q;  // no row sees past this
    const int n_tiles = k1 > k0 ? (int)((k1 - k0 + kTileKeys - 1) / kTileKeys) : 0;

    uint8_t *qs_lds = smem + kOffV + kTensorBytes;  // Q operands (V stages 1-2, free until V(1) is issued)
    // Per-tile exchange areas
    _Float16 *pbuf = reinterpret_cast<_Float16 *>(smem + kOffP);
    float *mbuf = reinterpret_cast<float *>(smem + kOffM);
    uint32_t *fbuf = reinterpret_cast<uint32_t *>(smem + kOffFlag);
    float *lbuf = reinterpret_cast<float *>(smem + kOffL);
    const int rows_total = p.n_q * p.H;

    if (score) {
        // ============ score wavefronts: QK and softmax weights =================
        // Q -> q8_0 block-diagonal B operands. Column n of C: row r = (n & 7)
        // [+ 8 for the second set], block 2*pair + (n >> 3). Lane (g, n) supplies
        // k = 16g..16g+15, i.e. values 16*(g&1).. of the column's block when
        // (g >> 1) == (n >> 3), zeros otherwise. The four wavefronts each load
        // their block pair (pair = wq) of the Q rows straight from global memory
        // at entry, quantise it and exchange the operands through LDS.
        constexpr int kSets = TWO ? 2 : 1;
        constexpr int kOpndBytes = 32;  // per lane: 16 code bytes, d_q, -8*sum(q8)
        int32x4 bq[kSets][4];
        float dqs[kSets][4];
        int cinit[kSets][4];
        const bool q_active = (g >> 1) == (n >> 3);
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
                const float *qrow = reinterpret_cast<const float *>(p.q + (row_ok ? t * p.q_nb1 + hq * p.q_nb2 : 0));
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
                amax = xmax16(amax);  // the other 16 values of the block
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
                sumq = xsum16(sumq);
                const float dqv = (float)(_Float16)d * p.qscale;
                const int civ = -8 * sumq;
                const float dq2 = __int_as_float(xother32(__float_as_int(dqv)));  // inactive lanes: column n lives in lane ^ 32
                const int ci2 = xother32(civ);
                my_dq[set] = q_active ? dqv : dq2;
                my_ci[set] = q_active ? civ : ci2;
            }
#pragma unroll
            for (int set = 0; set < kSets; ++set) {
                uint8_t *o = qs_lds + ((pr * kSets + set) * 64 + lane) * kOpndBytes;
                *reinterpret_cast<int32x4 *>(o) = my_bq[set];
                *reinterpret_cast<float2 *>(o + 16) = make_float2(my_dq[set], __int_as_float(my_ci[set]));
            }
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // operands published
#pragma unroll
            for (int pp = 0; pp < 4; ++pp)
#pragma unroll
                for (int set = 0; set < kSets; ++set) {
                    const uint8_t *o = qs_lds + ((pp * kSets + set) * 64 + lane) * kOpndBytes;
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
        const bool row_writer = TWO || n < 8;  // lanes n >= 8 mirror rows 0-7 when only 8 exist
        // K operand: lane (g, n) reads key n's block 2*pair + (g >> 1), nibbles of half g & 1.
        // qs of block b sits at 18b + 2 in the head row: 4-aligned for odd b, 2 mod 4 for
        // even b. The five dwords from the aligned address below it stay inside two
        // adjacent slots of the row (block 7 spills one unused dword into the next).
        const int ka_blk_par = g >> 1;
        const uint32_t ka_shift = (ka_blk_par ? 0u : 16u) + 4u * (uint32_t)(g & 1);
        uint8_t *dk_comp = smem + kOffDk + wave * 256;  // [8 blocks][16 keys] fp16
        const int key0 = 16 * wq;                       // first key of this wavefront in a tile
        // P is stored in key order: this lane's four keys key0 + 4g + i
        const int p_col = key0 + 4 * g;
        int ka_off[4];  // LDS offsets of this lane's K windows (block pair pr), within a stage
#pragma unroll
        for (int pr = 0; pr < 4; ++pr)
            ka_off[pr] = lds_byte<false>(key0 + n, (18 * (2 * pr + ka_blk_par) + 2) & ~3);
        // d_k compaction: lane -> block lane >> 3, keys key0 + 4gg + 2hh and the next one
        const int dk_blk = lane >> 3, dk_gg = lane & 3, dk_hh = (lane >> 2) & 1;
        const int dk_src = lds_byte<false>(key0 + 4 * dk_gg + 2 * dk_hh, 18 * dk_blk);
        const int dk_dst = (dk_blk * 16 + 4 * dk_gg + 2 * dk_hh) * 2;

        // first tile holding keys past the range end (k1) or past a causal limit
        // (key > q_pos0 for the first position): tile t ends at key k0 + 64t + 63
        int t_tail = (int)((k1 - k0) / kTileKeys);
        if (p.q_pos0 >= 0) {
            const int64_t x = p.q_pos0 - k0 - (kTileKeys - 1);  // tail when 64t > x
            if (x < 0)
                t_tail = 0;
            else if (x / kTileKeys < t_tail)
                t_tail = (int)(x / kTileKeys) + 1;
        }
        float m_ref = -INFINITY;   // base-2 reference max of row my_r (common to the workgroup)
        float m_used = -INFINITY;  // reference this wavefront used for the last tile's P
        float l_acc = 0.0f;        // this lane's share of the row's sum, relative to m_ref
        float l_prev = 0.0f;       // the last tile's share, relative to m_used
        // K stage of the tile (t mod kKStages, carried through the loop: LDS
        // addresses are then one add of a wave-uniform offset) and this lane's P
        // row in tile buffer 0
        int st = 0;
        _Float16 *const prow0 = pbuf + my_r * kPRow + p_col;

        for (int tt = 0; tt <= n_tiles; ++tt) {
            // the tile index is wave-uniform; with 16 rows the compiler loses track of that
            const int t = TWO ? __builtin_amdgcn_readfirstlane(tt) : tt;
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // K(t) and P(t-1) readable

            // -- fold the last tile's sum into l under the workgroup's common max --
            if (t > 0) {
                const int pb = (t - 1) & 1;
                const uint4 fl = *reinterpret_cast<const uint4 *>(fbuf + pb * 4);
                if ((fl.x | fl.y | fl.z | fl.w) & 1u) {
                    const float *mr = mbuf + pb * 64;
                    const float mn = fmaxf(fmaxf(mr[my_r], mr[16 + my_r]), fmaxf(mr[32 + my_r], mr[48 + my_r]));
                    l_acc = l_acc * exp2_or_zero(m_ref, mn) + l_prev * exp2_or_zero(m_used, mn);
                    m_ref = mn;
                } else {
                    l_acc += l_prev;
                }
            }
            if (t == n_tiles) break;

            const int64_t kt = k0 + (int64_t)t * kTileKeys;
            const uint8_t *sK = smem + st * kTensorBytes;
            // a tile holding keys past the range end or past a causal limit
            const bool tail = t >= t_tail;

            // A row r of QK is key key0 + r, so lane group g holds keys key0 + 4g + i.
            // -- compact d_k of those keys, [block][4g + i] ------------------------
            *reinterpret_cast<uint32_t *>(dk_comp + dk_dst) =
                lds16(sK + dk_src) | (lds16(sK + dk_src + kLdsRow) << 16);

            // -- QK: xs[i] = S[key key0+4g+i][row of column n] --------------------
            float xs[kSets][4];
#pragma unroll
            for (int set = 0; set < kSets; ++set)
#pragma unroll
                for (int i = 0; i < 4; ++i) xs[set][i] = 0.0f;
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) {
                // key of A row n, block 2*pair + (g >> 1): five dwords from the aligned
                // address below its 16 qs bytes, shifted to the nibble half g & 1
                const uint8_t *ap = sK + ka_off[pr];
                const uint32_t w0 = lds32(ap), w1 = lds32(ap + 4), w2 = lds32(ap + 8), w3 = lds32(ap + 12),
                               w4 = lds32(ap + 16);
                uint32_t aw[4];
                aw[0] = __builtin_amdgcn_alignbit(w1, w0, ka_shift) & 0x0F0F0F0Fu;
                aw[1] = __builtin_amdgcn_alignbit(w2, w1, ka_shift) & 0x0F0F0F0Fu;
                aw[2] = __builtin_amdgcn_alignbit(w3, w2, ka_shift) & 0x0F0F0F0Fu;
                aw[3] = __builtin_amdgcn_alignbit(w4, w3, ka_shift) & 0x0F0F0F0Fu;
                int32x4 aop;
                __builtin_memcpy(&aop, aw, 16);
                const uint2 dk2 = *reinterpret_cast<const uint2 *>(dk_comp + ((2 * pr + (n >> 3)) * 16 + 4 * g) * 2);
                half4 dkh;  // d_k of keys key0+4g+i, block of column n
                __builtin_memcpy(&dkh, &dk2, 8);
#pragma unroll
                for (int set = 0; set < kSets; ++set) {
                    const int ci = cinit[set][pr];
                    int32x4 c = {ci, ci, ci, ci};
                    c = __builtin_amdgcn_mfma_i32_16x16x64_i8(aop, bq[set][pr], c, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        xs[set][i] = fmaf((float)c[i] * dqs[set][pr], (float)dkh[i], xs[set][i]);
                }
            }
            // even-block half (columns 0-7) + odd-block half (columns 8-15) of each logit
            float s[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (TWO) {  // lanes n < 8 take rows 0-7 (set 0), lanes n >= 8 rows 8-15 (set 1)
                    const float u = n < 8 ? xs[0][i] : xs[1][i];
                    const float w = n < 8 ? xs[1][i] : xs[0][i];
                    s[i] = u + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(w), 0x128, 0xf, 0xf, true));
                } else {
                    s[i] = xs[0][i] +
                           __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(xs[0][i]), 0x128, 0xf, 0xf, true));
                }
            }
            // mask (F16, base-e units) and the ragged / causal tail
            if (p.mask) {
                const uint16_t *mrow = reinterpret_cast<const uint16_t *>(smem + kOffMask + st * kMaskStageBytes) +
                                       my_t * kTileKeys + key0 + 4 * g;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint16_t mb = mrow[i];
                    _Float16 mh;
                    __builtin_memcpy(&mh, &mb, 2);
                    // a -inf entry excludes the key whatever its logit (even NaN from a
                    // garbage scale): ggml's CPU loop skips such keys
                    s[i] = mb == 0xFC00u ? -INFINITY : fmaf((float)mh, kLog2e, s[i]);
                }
            }
            if (tail) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int64_t key = kt + key0 + 4 * g + i;
                    bool dead = key >= k1;
                    if (p.q_pos0 >= 0) dead = dead || key > p.q_pos0 + my_t;
                    s[i] = dead ? -INFINITY : s[i];
                }
            }
            // -- softmax weights under the reference max (lazy, see the header) ---
            const float lim = m_ref + kSlack;
            bool need = __any((s[0] > lim) | (s[1] > lim) | (s[2] > lim) | (s[3] > lim));
            float mu = m_ref;
            if (need) {
                float mt = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
                mt = xmax32(xmax16(mt));
                mu = fmaxf(m_ref, mt);
            }
            if (!TWO && t == 0) {
                // The split's first tile (m_ref = -inf, so mu is this wavefront's
                // row maximum), up to 8 rows: the four score wavefronts agree on
                // each row's maximum over all 64 keys (through lbuf, free until the
                // statistics, and one more barrier, which the value wavefronts
                // match) and start from it, so the tile's P needs no rescale by the
                // value wavefronts and no maximum has moved.
                if (g == 0 && row_writer) lbuf[wq * 16 + my_r] = mu;
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // first-tile maxima
                mu = fmaxf(fmaxf(lbuf[my_r], lbuf[16 + my_r]), fmaxf(lbuf[32 + my_r], lbuf[48 + my_r]));
                m_ref = mu;
                need = false;
            }
            m_used = mu;
            // the reference plus the P shift: exact while |mu| < 2^21
            const float mb = (mu == -INFINITY ? 0.0f : mu) + kPShift;
            float pv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) pv[i] = __builtin_amdgcn_exp2f(s[i] - mb);
            l_prev = (pv[0] + pv[1]) + (pv[2] + pv[3]);
            const int buf = t & 1;
            if (row_writer) {
                half4 ph, pl;
                ph = half4{(_Float16)pv[0], (_Float16)pv[1], (_Float16)pv[2], (_Float16)pv[3]};
                uint32_t hw[2];
                __builtin_memcpy(hw, &ph, 8);
                float r[4];  // exact residual p - hi, read from the packed fp16 halves by v_fma_mix
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (i & 1)
                        asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "=v"(r[i]) : "v"(pv[i]), "v"(hw[i >> 1]));
                    else
                        asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel:[0,0,0] op_sel_hi:[0,0,1]" : "=v"(r[i]) : "v"(pv[i]), "v"(hw[i >> 1]));
                }
                pl = half4{(_Float16)r[0], (_Float16)r[1], (_Float16)r[2], (_Float16)r[3]};
                _Float16 *prow = prow0 + buf * (16 * kPRow);
                *reinterpret_cast<half4 *>(prow) = ph;
                *reinterpret_cast<half4 *>(prow + 64) = pl;
                if (g == 0) mbuf[(buf * 4 + wq) * 16 + my_r] = mu;
            }
            // keys of this wavefront that some row sees: bit 4g + i of the 16. P >= 0
            // (or NaN), so P != 0 is a nonzero bit pattern; the 16 lanes of group g
            // (one DPP row) OR their nibbles, the four groups then OR theirs.
            uint32_t alive = min(__float_as_uint(pv[0]), 1u) | (min(__float_as_uint(pv[1]), 1u) << 1) |
                             (min(__float_as_uint(pv[2]), 1u) << 2) | (min(__float_as_uint(pv[3]), 1u) << 3);
            alive |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)alive, 0x121, 0xf, 0xf, false);  // row_ror:1
            alive |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)alive, 0x122, 0xf, 0xf, false);  // row_ror:2
            alive |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)alive, 0x124, 0xf, 0xf, false);  // row_ror:4
            alive |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)alive, 0x128, 0xf, 0xf, false);  // row_ror:8
            alive = or16(alive << (4 * g));
            alive = or32(alive);
            if (lane == 0) fbuf[buf * 4 + wq] = (need ? 1u : 0u) | (alive << 16);
            st = st == kKStages - 1 ? 0 : st + 1;
        }

        // ---------------- this split's softmax statistics ------------------------
        l_acc = xsum32(xsum16(l_acc));
        if (g == 0 && row_writer) lbuf[wq * 16 + my_r] = l_acc;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (wq == 0 && g == 0 && row_writer && my_ok) {
            const float L = (lbuf[my_r] + lbuf[16 + my_r]) + (lbuf[32 + my_r] + lbuf[48 + my_r]);
            const int tq = my_r / p.G, hq = kvh * p.G + my_r % p.G;
            const int64_t ridx = (int64_t)split * rows_total + (int64_t)tq * p.H + hq;
            store_through(p.part_ml + ridx * 2 + 0, m_ref == -INFINITY ? m_ref : m_ref * kLn2);  // combine works in base e
            store_through(p.part_ml + ridx * 2 + 1, L);
        }
    } else {
        // ============ value wavefronts: O[rows][64 dims] += P V =================
        // ---------------- DMA plan of this wavefront ---------------------------
        // Value wavefronts issue every DMA (score wavefronts carry no DMA state):
        // 9 K + 9 V instructions per tile, K j -> value wave j % 4, V j -> value
        // wave (j + 2) % 4, the mask rows -> value wave 3 (4 or 5 per wavefront).
        const int vw = wave - kScoreWaves;
        uint32_t koff[3], voff[3];
        int nk = 0, nv = 0;
#pragma unroll
        for (int r = 0; r < 3; ++r) {
            const int jk = vw + 4 * r;
            const int jv = ((vw + 2) & 3) + 4 * r;
            koff[r] = slot_offset<false>(jk < kTensorInsts ? jk : 0, lane, kvh, (uint32_t)p.row_bytes);
            voff[r] = slot_offset<true>(jv < kTensorInsts ? jv : 0, lane, kvh, (uint32_t)p.row_bytes);
            nk += jk < kTensorInsts;
            nv += jv < kTensorInsts;
        }
        const bool mask_dma = p.mask && vw == kValueWaves - 1;
        const int mrow_l = lane >> 3;  // mask DMA lane -> query row, 16-byte segment
        const uint32_t moff = (uint32_t)((int64_t)(mrow_l < p.n_q ? mrow_l : 0) * p.mask_nb1 + 16 * (lane & 7));
        // every wavefront issues 2 or 3 of the 9 K and of the 9 V instructions
        static_assert(kTensorInsts == 9 && kValueWaves == 4, "2 or 3 instructions per wavefront and tensor");
        const bool k3 = nk == 3, v3 = nv == 3;

        // keys past the cache end re-read its last row (they are masked off); mask
        // segments past the readable length re-read its last 16 bytes
        auto lim_of = [&](int64_t kt) -> uint32_t {
            return p.n_kv - kt >= kTileKeys ? 0xFFFFFFFFu : (uint32_t)((p.n_kv - kt) * p.row_bytes - 16);
        };
        auto mlim_of = [&](int64_t kt) -> uint32_t {
            return p.mask_len - kt >= kTileKeys + 8 ? 0xFFFFFFFFu : (uint32_t)((p.mask_len - 8 - kt) * 2);
        };
        // Tiles below t_fast need neither limit: tile t starts at key k0 + 64t, and
        // lim_of / mlim_of are unlimited while 64t <= n_kv - k0 - 64 and
        // 64t <= mask_len - k0 - 72.
        int t_fast = (int)min((int64_t)n_tiles, (p.n_kv - k0) / kTileKeys);
        if (mask_dma) {
            const int64_t y = p.mask_len - k0 - (kTileKeys + 8);
            t_fast = y < 0 ? 0 : (int)min((int64_t)t_fast, y / kTileKeys + 1);
        }
        const uint8_t *kb0 = p.k + k0 * p.row_bytes;
        const uint8_t *vb0 = p.v + k0 * p.row_bytes;
        const int64_t tile_bytes = kTileKeys * p.row_bytes;
        const char *mb0 = p.mask ? p.mask + k0 * 2 : nullptr;
        const bool mask_lane = mask_dma && mrow_l < p.n_q;
        // kb, vb: the tile's first cache row (the loop carries them, one add per tile)
        auto issue_k = [&](int t, int st, const uint8_t *kb) {  // st = t mod kKStages
            const uint32_t kbase = lds0 + st * kTensorBytes;
            const uint32_t mdst = lds0 + kOffMask + st * kMaskStageBytes;
            if (t < t_fast) {
                dma16(koff[0], kb, kbase + 1024u * vw);
                dma16(koff[1], kb, kbase + 1024u * (vw + 4));
                if (k3) dma16(koff[2], kb, kbase + 1024u * (vw + 8));
                if (mask_lane) dma16(moff, mb0 + (int64_t)t * (kTileKeys * 2), mdst);
            } else {
                const int64_t kt = k0 + (int64_t)t * kTileKeys;
                const uint32_t lim = lim_of(kt);
                dma16(koff[0] < lim ? koff[0] : lim, kb, kbase + 1024u * vw);
                dma16(koff[1] < lim ? koff[1] : lim, kb, kbase + 1024u * (vw + 4));
                if (k3) dma16(koff[2] < lim ? koff[2] : lim, kb, kbase + 1024u * (vw + 8));
                if (mask_dma) {
                    const uint32_t mlim = mlim_of(kt);
                    const uint32_t mo = moff - 16 * (lane & 7) + ((16u * (lane & 7)) < mlim ? 16u * (lane & 7) : mlim);
                    if (mrow_l < p.n_q) dma16(mo, mb0 + (int64_t)t * (kTileKeys * 2), mdst);
                }
            }
        };
        auto issue_v = [&](int t, int st, const uint8_t *vb) {  // st = t mod kVStages
            const uint32_t vbase = lds0 + kOffV + st * kTensorBytes;
            const int j0 = (vw + 2) & 3;
            if (t < t_fast) {
                dma16(voff[0], vb, vbase + 1024u * j0);
                dma16(voff[1], vb, vbase + 1024u * (j0 + 4));
                if (v3) dma16(voff[2], vb, vbase + 1024u * (j0 + 8));
            } else {
                const uint32_t lim = lim_of(k0 + (int64_t)t * kTileKeys);
                dma16(voff[0] < lim ? voff[0] : lim, vb, vbase + 1024u * j0);
                dma16(voff[1] < lim ? voff[1] : lim, vb, vbase + 1024u * (j0 + 4));
                if (v3) dma16(voff[2] < lim ? voff[2] : lim, vb, vbase + 1024u * (j0 + 8));
            }
        };
        // The wait at interval t: K of tile t and V of tile t-1 must have landed.
        // The loop issues K(t+2) and V(t+1) at interval t, after K 0, K 1 and V 0
        // before the loop, so the younger DMAs at interval t are K(t+1) and V(t):
        // at least 2 + 2 = 4 instructions while t + 1 < n_tiles (value wavefront 1
        // has 2 K and 2 V per tile; 0 and 2 have a third of K or of V, 3 the mask
        // row when there is a mask), at least 2 (V(t)) when t + 1 == n_tiles, none
        // at the end. Waiting down to that lower bound is exact for the wavefronts
        // with 4 and, for those with 5, also waits for the oldest of K(t+1), issued
        // an interval earlier.
        auto wait_interval = [&](int t) {
            if (t + 1 < n_tiles)
                asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            else if (t < n_tiles)
                asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            else
                asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        };

        // ---------------- K 0-1 and V 0 ------------------------------------------
        // (V stages 1-2 hold the Q operands until the loop's first barrier)
        static_assert(kKStages == 3 && kVStages == 3, "the stage counter below");
        if (n_tiles > 0) issue_k(0, 0, kb0);
        if (n_tiles > 1) issue_k(1, 1, kb0 + tile_bytes);
        if (n_tiles > 0) issue_v(0, 0, vb0);
        if (!TWO) {
            // rows 8-15 of both P buffers (never written with 8 rows) hold zeros: the
            // residual operand of the lanes that carry hi parts (see the PV below)
            const int zi = vw * 64 + lane;  // 256 lanes x 4 fp16 = 2 buffers x 8 rows x 64 hi
            *reinterpret_cast<half4 *>(pbuf + ((zi >> 7) * 16 + 8 + ((zi >> 4) & 7)) * kPRow + 4 * (zi & 15)) =
                half4{0, 0, 0, 0};
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // Q operands published
        const int dq = wq;  // dims 64dq..64dq+63: blocks 2dq, 2dq+1
        // B operand from the nibbles: a nibble in the low bits of an fp16 is the
        // subnormal nib * 2^-24 (low nibble), which one packed multiply by 2^14
        // makes nib * 2^-10, exact and normal; left in bits 4-7, the high nibble
        // is nib * 2^-20 and enters as it is.
        const half8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
        const half8 kLoToNormal = {16384, 16384, 16384, 16384, 16384, 16384, 16384, 16384};  // 2^14
        uint8_t *dv_comp = smem + kOffDv + vw * 256;  // [bl][half][g][j] fp16
        const int ra = n & kRowMask;  // P row of this lane's A operand
        // d_v compaction: lane -> block bl, half h, key group gg, pair jj: keys
        // 32h + 8gg + 2jj and the next one (B k-slots 8gg + 2jj, +1)
        const int cbl = lane >> 5, ch = (lane >> 4) & 1, cgg = (lane >> 2) & 3, cjj = lane & 3;
        const int ckey = 32 * ch + 8 * cgg + 2 * cjj;
        const int cdst = ((cbl * 2 + ch) * 4 + cgg) * 16 + 4 * cjj;  // bytes
        const uint32_t csrc = (uint32_t)lds_byte<true>(ckey, 18 * (2 * dq + cbl));
        // V bytes of this lane: B k-slot 8g + j is key 32h + 8g + j; its byte n of block
        // 2dq + bl sits at byte c = 2 + 18*(2dq + bl) + n of the head row, rotated by
        // v_rot = 2g slots for every row the lane reads; the dword holding it carries
        // it as byte c & 3.
        uint32_t vlane[2], vsel[2];  // v_perm selector: byte c&3 of the lower key's dword -> bits 0-7, of the upper -> 16-23
#pragma unroll
        for (int bl = 0; bl < 2; ++bl) {
            const int c = 2 + 18 * (2 * dq + bl) + n;
            vlane[bl] = (uint32_t)(lds_byte<true>(8 * g, c) & ~3);
            const uint32_t b = (uint32_t)(c & 3);
            vsel[bl] = b | (0x0cu << 8) | ((4u + b) << 16) | (0x0cu << 24);
        }

        // acc[2bl] = 2^-10 sum_k A nib_lo, acc[2bl + 1] = 2^-20 sum_k A nib_hi, and
        // cor[bl] = sum_k A, with A = P d_v of block 2dq + bl, so that
        // O[row 4g+i][dim 64dq + 32bl + n] = 2^10 acc - 8 cor (2^20 acc for the
        // high nibble, dim + 16).
        floatx4 acc[4], cor[2];
#pragma unroll
        for (int T = 0; T < 4; ++T) acc[T] = floatx4{0.f, 0.f, 0.f, 0.f};
        cor[0] = cor[1] = floatx4{0.f, 0.f, 0.f, 0.f};
        // d_v enters A as d_v 2^E (E per wavefront, only ever lowered): P 2^-4 <= 16
        // times |d_v 2^E| < 2^11 keeps A below 2^15, and the largest d_v near 2^8
        // keeps A clear of fp16 subnormals, whatever the size of V. The partial O
        // is scaled back by 2^-E; l does not carry E.
        int e_dv = kMaxDvExp;
        uint32_t dv_thr = 0;  // fp16 magnitude bits of 2^(11 - E)
        half2v dv_s1, dv_s2;  // 2^floor(E/2), 2^(E - floor(E/2))
        auto set_dv_scale = [&](int e) {
            e_dv = e;
            const int x = 11 - e;
            dv_thr = x >= 16 ? 0x7C00u : (x >= -14 ? (uint32_t)(x + 15) << 10 : 1u << (x + 24));
            const int e1 = e >> 1, e2 = e - e1;
            const uint16_t b1 = (uint16_t)((e1 + 15) << 10), b2 = (uint16_t)((e2 + 15) << 10);
            _Float16 h1, h2;
            __builtin_memcpy(&h1, &b1, 2);
            __builtin_memcpy(&h2, &b2, 2);
            dv_s1 = half2v{h1, h1};
            dv_s2 = half2v{h2, h2};
        };
        set_dv_scale(kMaxDvExp);
        float m_acc[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};  // reference max of rows 4g+i
        // P rows of this lane in tile buffer 0 (see the PV below)
        const _Float16 *const arow0 = pbuf + ra * kPRow + 8 * g + (TWO || n < 8 ? 0 : 64);
        const _Float16 *const lrow0 = TWO ? arow0 + 64 : pbuf + (n ^ 8) * kPRow + 8 * g;

        int c = 0;  // t mod 3, carried through the loop (3 K and 3 V stages)
        const uint8_t *kn = kb0 + 2 * tile_bytes, *vn = vb0 + tile_bytes;  // K(t+2), V(t+1)
        for (int tt = 0; tt <= n_tiles; ++tt) {
            const int t = TWO ? __builtin_amdgcn_readfirstlane(tt) : tt;  // wave-uniform tile index
            const int c1 = c == 2 ? 0 : c + 1, c2 = c == 0 ? 2 : c - 1;  // (t + 1) mod 3, (t + 2) mod 3
            wait_interval(t);
            if (t + 2 < n_tiles) issue_k(t + 2, c2, kn);
            if (t + 1 < n_tiles) issue_v(t + 1, c1, vn);
            kn += tile_bytes;
            vn += tile_bytes;
            c = c1;
            if (t == 0) {
                // the score wavefronts' first-tile maxima exchange (no tile, no barrier)
                if (!TWO && n_tiles > 0) asm volatile("s_barrier" ::: "memory");
                continue;
            }

            const int tv = t - 1;  // PV of the tile whose P the score wavefronts wrote last
            const int pb = tv & 1;
            const uint32_t sv_off = (uint32_t)(kOffV + c2 * kTensorBytes);  // stage of V(t - 1), wave-uniform

            // flags of the score wavefronts: bit 0 = maximum moved, bits 16-31 = their
            // 16 keys that some row of the call can see (P != 0)
            const uint4 fl = *reinterpret_cast<const uint4 *>(fbuf + pb * 4);

            // -- P rows (k-slot order), read first: their latency runs under the
            // d_v compaction below. 16 rows: pa, pl = hi and lo of row n. Up to 8 rows:
            // A row n < 8 carries the hi part of P d_v of row n and A row n + 8 its lo
            // part (C rows r and r + 8 are summed at the end), so one set of MFMAs
            // serves both: pa = the P part the lane multiplies (hi of row n, lo of row
            // n - 8), pl = the hi part whose rounding residual the lane adds (zero row
            // n + 8, hi of row n - 8).
            half8 pa[2], pl[2];  // tile halves 0, 1
            {
                const _Float16 *arow = arow0 + pb * (16 * kPRow);
                const _Float16 *lrow = lrow0 + pb * (16 * kPRow);
                pa[0] = *reinterpret_cast<const half8 *>(arow);
                pa[1] = *reinterpret_cast<const half8 *>(arow + 32);
                pl[0] = *reinterpret_cast<const half8 *>(lrow);
                pl[1] = *reinterpret_cast<const half8 *>(lrow + 32);
            }

            // -- d_v of the slice's two blocks for all 64 keys, in B k-slot order --
            // A key no row sees (masked, past the range or past the cache end) gets
            // d_v = 0, so its bytes, whatever they hold, add exactly 0 as ggml's CPU
            // loop skips such keys.
            {
                const uint8_t *src = smem + sv_off + csrc;
                uint32_t da = lds16(src), db = lds16(src + kLdsRow);
                const uint64_t alive = (uint64_t)((fl.x >> 16) | (fl.y & 0xFFFF0000u)) |
                                       ((uint64_t)((fl.z >> 16) | (fl.w & 0xFFFF0000u)) << 32);
                da = (alive >> ckey) & 1 ? da : 0u;
                db = (alive >> (ckey + 1)) & 1 ? db : 0u;
                auto store_scaled = [&]() {  // d_v 2^E in two exact steps (2^E may exceed fp16)
                    uint32_t w = da | (db << 16);
                    half2v wh;
                    __builtin_memcpy(&wh, &w, 4);
                    wh = wh * dv_s1 * dv_s2;
                    __builtin_memcpy(&w, &wh, 4);
                    *reinterpret_cast<uint32_t *>(dv_comp + cdst) = w;
                };
                // a d_v at or above 2^(11 - E) lowers E so that the largest |d_v| of
                // the tile lands in [2^8, 2^9); O is rescaled by the exact power of
                // two and the tile's d_v are stored again. On the split's first tile
                // O is still zero: E comes straight from the tile's largest |d_v|.
                const uint32_t mag = max(da & 0x7FFFu, db & 0x7FFFu);
                if (!TWO && tv == 0) {
                    const int mx = wave_max_u16(mag);
                    if (mx != 0) {
                        const int ex = mx >> 10;
                        const int lg = ex ? ex - 15 : (31 - __clz(mx)) - 24;  // floor(log2 max |d_v|)
                        set_dv_scale(min(8 - lg, kMaxDvExp));
                    }
                    store_scaled();
                } else {
                store_scaled();
                if (__any(mag >= dv_thr)) {
                    const int mx = wave_max_u16(mag);
                    const int ex = mx >> 10;
                    const int lg = ex ? ex - 15 : (31 - __clz(mx)) - 24;  // floor(log2 max |d_v|)
                    const int e_new = 8 - lg;
                    if (e_new < e_dv) {
                        const float f = __builtin_amdgcn_ldexpf(1.0f, e_new - e_dv);
#pragma unroll
                        for (int T = 0; T < 4; ++T) acc[T] *= f;
                        cor[0] *= f;
                        cor[1] *= f;
                        set_dv_scale(e_new);
                        store_scaled();
                    }
                }
                }
            }

            // -- the split's first tile: P is relative to the rows' common maxima
            if (!TWO && tv == 0) {
                const float *mr = mbuf + pb * 64;
#pragma unroll
                for (int i = 0; i < 4; ++i) m_acc[i] = mr[(4 * g + i) & kRowMask];
            }
            // -- a possible move of the reference max ---------------------------------
            if ((fl.x | fl.y | fl.z | fl.w) & 1u) {
                const float *mr = mbuf + pb * 64;
                float fac[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = (4 * g + i) & kRowMask;
                    const float mn = fmaxf(fmaxf(mr[r], mr[16 + r]), fmaxf(mr[32 + r], mr[48 + r]));
                    fac[i] = exp2_or_zero(m_acc[i], mn);
                    m_acc[i] = mn;
                }
                const floatx4 f4 = {fac[0], fac[1], fac[2], fac[3]};
#pragma unroll
                for (int T = 0; T < 4; ++T) acc[T] *= f4;
                cor[0] *= f4;
                cor[1] *= f4;
                // P of score wavefront w (keys 16w..16w+15: this lane's half-h slots 8g..8g+7
                // come from wavefront 2h + (g >> 1)) onto the new max
                float mw[4];
#pragma unroll
                for (int w = 0; w < 4; ++w) mw[w] = mr[16 * w + ra];
                const float mna = fmaxf(fmaxf(mw[0], mw[1]), fmaxf(mw[2], mw[3]));
                const _Float16 *prow = pbuf + (pb * 16 + ra) * kPRow + 8 * g;  // hi | lo of row ra
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const half8 ph = *reinterpret_cast<const half8 *>(prow + 32 * h);
                    const half8 plo = *reinterpret_cast<const half8 *>(prow + 64 + 32 * h);
                    // P alpha as hi = fp16(P alpha) and lo = fp16(P alpha - hi), both
                    // rounded once from the exact product by v_fma_mixlo_f16. Left to
                    // the compiler, the stored hi came from the fp32 product (rounded
                    // twice) and the hi subtracted for lo from the exact one, and where
                    // the product sat near an fp16 rounding midpoint the two differed:
                    // hi + lo one fp16 ulp of hi off.
                    const float al = exp2_or_zero(mw[2 * h + (g >> 1)], mna);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float sv = (float)ph[e] + (float)plo[e];  // exact: lo is below hi's ulp
                        uint32_t hw, lw;
                        asm("v_fma_mixlo_f16 %0, %1, %2, 0" : "=v"(hw) : "v"(sv), "v"(al));
                        asm("v_fma_mixlo_f16 %0, %1, %2, -%3 op_sel_hi:[0,0,1]" : "=v"(lw) : "v"(sv), "v"(al), "v"(hw));
                        const _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)hw);
                        const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)lw);
                        pa[h][e] = TWO || n < 8 ? hi : lo;
                        pl[h][e] = TWO ? lo : (n < 8 ? (_Float16)0 : hi);
                    }
                }
            }

            // -- O += P V over the two halves of the tile and the slice's blocks ---
            // A = P d_v exactly as Ah + Al in packed fp16: Ph d_v has at most 22
            // significant bits, so its residual after rounding to fp16 (at most 11) is
            // exact in one fma; Pl d_v is 2^-11 of it and rounds once. Every MFMA
            // product is then exact in fp32, and V's -8 offset comes in as -8 sum A.
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                // the slice's V bytes for the 32 keys of this half, two keys per register:
                // x[4*bl + m] holds keys 32h + 8g + 2m (bits 0-7) and 32h + 8g + 2m + 1
                // (bits 16-23), byte n of block 2dq + bl's qs: adjacent rows, one
                // ds_read2_b32 each. A base per two pairs keeps both dword offsets within
                // ds_read2's 8 bits.
                uint32_t x[8];
#pragma unroll
                for (int bl = 0; bl < 2; ++bl)
#pragma unroll
                    for (int mp = 0; mp < 2; ++mp) {
                        uint32_t va = lds0 + sv_off + vlane[bl] + (uint32_t)((32 * h + 4 * mp) * kLdsRow);
                        const lds_u32 *r0 = reinterpret_cast<const lds_u32 *>((uintptr_t)va);
#pragma unroll
                        for (int m2 = 0; m2 < 2; ++m2)
                            x[4 * bl + 2 * mp + m2] = __builtin_amdgcn_perm(r0[(2 * m2 + 1) * (kLdsRow / 4)],
                                                                             r0[2 * m2 * (kLdsRow / 4)], vsel[bl]);
                    }
#pragma unroll
                for (int bl = 0; bl < 2; ++bl) {
                    const uint4 dv4 = *reinterpret_cast<const uint4 *>(dv_comp + ((bl * 2 + h) * 4 + g) * 16);
                    half8 dv8;
                    __builtin_memcpy(&dv8, &dv4, 16);
                    uint32_t wlo[4], whi[4];
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        wlo[m] = x[4 * bl + m] & 0x000F000Fu;
                        whi[m] = x[4 * bl + m] & 0x00F000F0u;
                    }
                    half8 blo, bhi;
                    __builtin_memcpy(&blo, wlo, 16);
                    __builtin_memcpy(&bhi, whi, 16);
                    // nib 2^-24 times 2^14: nib 2^-10 exactly, in the normal range (with
                    // the low nibbles as subnormals 2^-24 deep, the MFMA's sums lost up
                    // to ~2^-12 of the output at long contexts; the high nibbles' nib
                    // 2^-20 cost nothing measurable)
                    blo = blo * kLoToNormal;
                    if (TWO) {
                        const half8 ah = pa[h] * dv8;
                        const half8 ar = __builtin_elementwise_fma(pa[h], dv8, -ah);
                        const half8 al = __builtin_elementwise_fma(pl[h], dv8, ar);
                        acc[2 * bl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, blo, acc[2 * bl], 0, 0, 0);
                        acc[2 * bl + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bhi, acc[2 * bl + 1], 0, 0, 0);
                        cor[bl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, ones, cor[bl], 0, 0, 0);
                        acc[2 * bl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, blo, acc[2 * bl], 0, 0, 0);
                        acc[2 * bl + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bhi, acc[2 * bl + 1], 0, 0, 0);
                        cor[bl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, ones, cor[bl], 0, 0, 0);
                    } else {
                        // hi lanes: pl = 0, so a = round(pa d_v); lo lanes: a = pl_lo d_v plus the
                        // exact residual of the hi part, rounded once
                        const half8 th = pl[h] * dv8;
                        const half8 tr = fma_minus(pl[h], dv8, th);
                        const half8 a = __builtin_elementwise_fma(pa[h], dv8, tr);
                        acc[2 * bl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, blo, acc[2 * bl], 0, 0, 0);
                        acc[2 * bl + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bhi, acc[2 * bl + 1], 0, 0, 0);
                        cor[bl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ones, cor[bl], 0, 0, 0);
                    }
                }
            }
        }

        // ---------------- this split's partial O (un-normalised) -----------------
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // pairs the statistics barrier
        const float o_scale = __builtin_amdgcn_ldexpf(1.0f, -e_dv);
        auto store_row = [&](int row, int i) {
            const int tq = row / p.G, hq = kvh * p.G + row % p.G;
            float *dst = p.part_acc + ((int64_t)split * rows_total + (int64_t)tq * p.H + hq) * 256 + 64 * dq + n;
#pragma unroll
            for (int bl = 0; bl < 2; ++bl) {
                store_through(dst + 32 * bl, fmaf(acc[2 * bl][i], 1024.0f, -8.0f * cor[bl][i]) * o_scale);
                store_through(dst + 32 * bl + 16, fmaf(acc[2 * bl + 1][i], 1048576.0f, -8.0f * cor[bl][i]) * o_scale);
            }
        };
        if (!TWO) {
            // C row r + 8 (lanes of group g + 2, lane ^ 32) holds the lo part of row
            // r: one lane swap per pair of C values adds them, lanes 0-31 keeping
            // i = 0, 1 (rows 4g + i) and lanes 32-63 i = 2, 3 (rows 4(g - 2) + i),
            // so every lane stores two rows
            const bool up = lane >= 32;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                auto fold = [&](floatx4 &x) {
                    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[i]), __float_as_uint(x[i + 2]),
                                                                    false, false);
                    x[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
                };
#pragma unroll
                for (int T = 0; T < 4; ++T) fold(acc[T]);
                fold(cor[0]);
                fold(cor[1]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = up ? 4 * (g - 2) + i + 2 : 4 * g + i;
                if (row < p.rows) store_row(row, i);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 4 * g + i;
                if (row < p.rows) store_row(row, i);
            }
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

// About two workgroups per CU over all KV heads (one split per CU at 2 KV
// heads), a multiple of 8 so that the workgroup numbering above holds (at most
// kMaxSplits); at least ~4 tiles per split, unless that leaves CUs idle: then
// up to one workgroup per CU, down to one tile per split. Graph-replayed
// 10-layer decode, us per layer (4-tile rule / this rule): 8K keys 13.3 /
// 10.9, 16K 13.6 / 11.9; from 32K on the 4-tile rule already fills the CUs
// (two workgroups per CU with 2-tile splits ran 16.4 against 14.0 at 32K).
int decode_splits(int64_t n_kv, int64_t n_kvh) {
    const int64_t tiles = (n_kv + kTileKeys - 1) / kTileKeys;
    const int64_t cus = device_cu_count();
    int64_t cap = 2 * cus / n_kvh / 8 * 8;
    if (cap > kMaxSplits) cap = kMaxSplits;
    if (cap < 8) cap = 8;
    int64_t s = (tiles + 3) / 4;
    const int64_t fill = tiles < cus / n_kvh ? tiles : cus / n_kvh;  // one workgroup per CU
    if (s < fill) s = fill;
    s = (s + 7) / 8 * 8;
    if (s > cap) s = cap;
    return (int)s;
}

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

// Scratch of the allocation-free decode entry point (sqa_flash_attn_ext_static):
// split partials and, for an unaligned mask, its packed copy. A file-scope
// device array: every GPU the library runs on holds its own copy at its own
// address until the process ends, and every call on that GPU shares it, so
// calls that overlap on one GPU race. Host code takes its address per device
// from hipGetSymbolAddress and never uses the array's name as a device pointer.
__device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

int static_scratch(void **out) {
    static std::mutex mu;
    static std::vector<void *> ptrs;  // per device
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "flash_attn_ext_static: hipGetDevice");
    std::lock_guard<std::mutex> lock(mu);
    if ((int)ptrs.size() <= dev) ptrs.resize(dev + 1, nullptr);
    if (!ptrs[dev]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e, "flash_attn_ext_static: hipGetSymbolAddress(scratch)");
        ptrs[dev] = ptr;
    }
    *out = ptrs[dev];
    return SQA_OK;
}

size_t fa_decode_workspace(int64_t n_q, int64_t H, int64_t n_kvh, int64_t n_kv, bool mask_copy) {
    const int64_t splits = decode_splits(n_kv, n_kvh);
    const size_t acc = al256((size_t)(splits * n_q * H * 256) * sizeof(float));
    const size_t ml = al256((size_t)(splits * n_q * H * 2) * sizeof(float));
    const size_t mask = mask_copy ? al256((size_t)(n_q * ((n_kv + 7) / 8 * 8)) * 2) : 0;
    return acc + ml + mask + 256;
}

bool decode_mask_needs_copy(const sqa_tensor *mask, int64_t n_kv) {
    return mask && !((uintptr_t)mask->data % 16 == 0 && mask->nb[1] % 16 == 0 && n_kv % 8 == 0);
}

int launch_fa_decode(const FaArgs &a, hipStream_t s) {
    const sqa_tensor &q = *a.q, &k = *a.k;
    const int64_t n_q = q.ne[1], H = q.ne[2], n_kv = k.ne[1], Hkv = k.ne[2];
    if (n_q > kMaxMaskRows) return set_error(SQA_ERR_UNSUPPORTED, "decode kernel takes at most 4 query positions");
    DecodeParams p;
    p.k = (const uint8_t *)k.data;
    p.v = (const uint8_t *)a.v->data;
    p.row_bytes = (int64_t)k.nb[1];  // n_kvh x 144, checked by the caller
    p.n_kvh = (int)Hkv;
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
    p.n_splits = decode_splits(n_kv, Hkv);
    // whole 64-key tiles per split: no tile is read by two splits. With two
    // workgroups per CU, the ones dispatched first (ids below the CU count, i.e.
    // splits below CUs / Hkv) issue ahead of the second round on the same CU
    // (the older wavefront wins the arbitration) and run faster: they take the
    // larger share, kFirstRoundWeight : kSecondRoundWeight, so that both rounds
    // end together instead of the second running on alone.
    p.tiles = (n_kv + kTileKeys - 1) / kTileKeys;
    const int cus = device_cu_count();
    p.n_first = Hkv * p.n_splits > cus ? (int)(cus / Hkv) : p.n_splits;
    if (p.n_first > p.n_splits) p.n_first = p.n_splits;
    p.w_first = p.n_first < p.n_splits ? kFirstRoundWeight : 1;
    p.w_second = p.n_first < p.n_splits ? kSecondRoundWeight : 1;
    p.cw_total = (int64_t)p.w_first * p.n_first + (int64_t)p.w_second * (p.n_splits - p.n_first);
    const bool pack_mask = a.q_pos0 < 0 && decode_mask_needs_copy(a.mask, n_kv);
    const size_t need = fa_decode_workspace(n_q, H, Hkv, n_kv, pack_mask);
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
        if (!pack_mask) {
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
    static std::once_flag lds_once;  // the LDS limit is raised once per process
    static hipError_t lds_err = hipSuccess;
    std::call_once(lds_once, [] {
        lds_err = hipFuncSetAttribute((const void *)fa_decode_kernel<false>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      kLdsBytes);
        if (lds_err == hipSuccess)
            lds_err = hipFuncSetAttribute((const void *)fa_decode_kernel<true>,
                                          hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    });
    if (lds_err != hipSuccess) return hip_status(lds_err, "fa_decode LDS attribute");
    const unsigned grid = (unsigned)(Hkv * p.n_splits);  // (split, KV head) pairs
    const int prof = profile_start("fa_decode", s);
    if (p.rows <= 8)
        fa_decode_kernel<false><<<dim3(grid), dim3(kThreads), kLdsBytes, s>>>(p);
    else
        fa_decode_kernel<true><<<dim3(grid), dim3(kThreads), kLdsBytes, s>>>(p);
    profile_stop(prof, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_status(e, "fa_decode launch");
    return launch_fa_combine(p.part_acc, p.part_ml, p.n_splits, (int)(n_q * H), (float *)a.dst->data, a.gate,
                             (int)H, s);
}

}  // namespace sqa
