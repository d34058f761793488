// fa_prefill.hip - FlashAttention for prefill chunks (more than 16 query rows
// per KV head, or more than 4 positions): the ubatch node of
// src/model/attn.rs:228-251 in the reference (n_q = 512 or 2048 over a q4_0
// cache of 16K-133K keys).
//
// Two short pre-passes, then one MFMA kernel:
//   kvprep K, V q4_0 -> per 32-key tile and KV head: Kc fp16 codes (nib - 8)
//                 [32 keys][256] and Dk fp16 scales [8 blocks][32 keys]; Vc
//                 fp16 codes [256 dims][32 keys] and Dv fp16 scales [8 blocks]
//                 [32 keys]; per KV head the largest |d_v|
//   qprep  Q f32 -> q8_0 with ggml's x86 rounding (d = amax/127, codes =
//                 rint(x * 127/amax)), then Q' = code * fp16(d) * scale *
//                 log2(e) as an fp16 hi + lo pair [n_q*H][256] each (Q' has at
//                 most 7 + 24 significant bits; hi + lo hold 22 of them)
// A tile of one KV head is a contiguous 33792-byte record [Kc | Dk | Vc | Dv]
// laid out exactly as the main kernel wants it in LDS (rows permuted, chunks
// swizzled, see below), so its K and V halves move HBM -> LDS as straight
// copies. Keys past n_kv are zero.
//
// fa_prefill_kernel: a workgroup takes 128 query rows of ONE KV head (GQA
// packed: row r is position r / G, head kvh*G + r % G) and streams 32-key
// tiles. Its 8 wavefronts (2 per SIMD) split the work by kind:
//   score wave w (0..3), rows 32w..32w+31, holds their Q' hi and lo (128
//     registers): S^T = sum over q4_0 blocks b of d_k[b] * (Kc_b.Q'h_b +
//     Kc_b.Q'l_b), the products on v_mfma_f32_16x16x32_f16 (all exact in
//     fp32: a code has at most 3 significant bits) and the d_k scaling as an
//     fp32 FMA with the fp16 scale as operand; then the mask and the
//     online softmax in fp32 (base 2, with a lazy reference maximum that moves
//     only when a logit passes it by more than a slack of ks binades, so
//     P <= 2^ks and most tiles need no rescale of O; ks = 8 unless V is large,
//     below). P (as an fp16 hi + lo pair) and the rescale factors go to LDS.
//   value wave 4 + w, the same 32 rows, holds their O (128 registers) one tile
//     behind: O = alpha O + P V per block b (alpha only when a maximum moved)
//     with A = P d_v as an fp16 hi + lo pair built by packed fp16 ops (two
//     MFMAs, ~22 bits) and B = the exact V codes, so every product is exact in
//     fp32. P carries 2^ep, one power of two per KV head, and l, summed from
//     the same P, carries the same factor. ep and ks follow the largest |d_v|
//     of the head so that A = P 2^ep d_v stays below 2^15 for every finite V
//     while P 2^ep stays as far from the fp16 subnormals as that allows.
//     The d_v and V operands of a tile are read ahead of the MFMAs that use them.
//   A masked key contributes exactly 0 even over NaN/Inf block scales (as ggml's
//   CPU loop, which skips it): a -inf mask entry replaces the logit, and the
//   pre-pass reads NaN/Inf V scales as 0.
// Computing S^T (keys as rows) leaves each lane with 8 logits of one query row
// in the A-operand layout of the P*V MFMA. K rows sit in LDS in the order
// r -> key sigma(r) = 8*((r>>2)&3) + 4*(r>>4) + (r&3), which makes a lane's 8
// logits keys 8g..8g+7, so its V operand is one 16-byte run of a Vc row.
//
// LDS reads are ds_read_b64 (16 lanes a pass). To keep them conflict free,
// 16-byte chunk c of K row r is stored at chunk c ^ (r & 7) with its 8-byte
// halves swapped when r & 8, and chunk c of Vc row d at c ^ ((d >> 1) & 3),
// halves swapped when d & 8.
//
// Tiles move HBM -> LDS with global_load_lds_dwordx4: in iteration t the K half
// (and mask rows) of tile t + 1 and the V half of tile t are in flight while
// the score waves work on tile t and the value waves on tile t - 1; one
// barrier per iteration.
//
// Operand layout of the 16x16x32 MFMAs (64 lanes, lane = 16*g + n):
//   A: A[row n][k = 8g..8g+7]   B: B[k = 8g..8g+7][col n]   C: C[rows 4g..4g+3][col n]
#include <mutex>

#include "common.hpp"

namespace sqa {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

constexpr int kPK = 32;                  // keys per tile
constexpr int kScoreWaves = 4;           // 32 rows each
constexpr int kValueWaves = 4;           // 32 rows each
constexpr int kWaves = kScoreWaves + kValueWaves;
constexpr int kThreads = 64 * kWaves;
constexpr int kRG = 2;                   // 16-row groups per score wave
constexpr int kRowsPerWG = kScoreWaves * kRG * 16;  // 128 query rows
constexpr int kOffDk = kPK * 512;        // inside the K half: Dk after Kc
constexpr int kKHalf = kOffDk + 8 * kPK * 2;  // Kc + Dk: 16896 bytes
constexpr int kOffDv = kHeadDim * kPK * 2;  // inside the V half: Dv after Vc
constexpr int kVHalf = kOffDv + 8 * kPK * 2;  // Vc + Dv: 16896 bytes
constexpr int kTileBytes = kKHalf + kVHalf;   // one tile record
constexpr int kKInst = (kKHalf + 1023) / 1024;  // 17 DMA instructions, the last one 512 bytes
constexpr int kVInst = (kVHalf + 1023) / 1024;  // 17, the last one 512 bytes
constexpr int kKStage = kKInst * 1024, kVStage = kVInst * 1024;
// LDS map: 2 K stages | 2 V stages | 2 P buffers | 2 rescale buffers | 2 mask stages
constexpr int kLdsV = 2 * kKStage;
constexpr int kLdsP = kLdsV + 2 * kVStage;        // [4 waves][2 rg][2 halves][64 lanes][16 B]
constexpr int kPBuf = kScoreWaves * kRG * 2 * 1024;
constexpr int kLdsA = kLdsP + 2 * kPBuf;          // [4 waves][2 rg][16 rows] f32
constexpr int kABuf = kScoreWaves * kRG * 16 * 4;
constexpr int kLdsMask = kLdsA + 2 * kABuf;       // [qb positions][32 keys] f16
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kSlack = 8;  // log2 of the largest P the lazy rescale admits (V not large)
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

static_assert(kTileBytes == 33792 && kTileBytes % 256 == 0, "tile record");
static_assert(kKHalf == kVHalf && kKInst == 17 && kVInst == 17, "both halves: 16 DMA instructions and a half");
constexpr int kLdsMaxBytes = kLdsMask + 2 * 128 * kPK * 2;  // with the mask stages of G = 1
static_assert(kLdsMaxBytes <= 160 * 1024, "LDS budget");

__device__ __forceinline__ float h2f(uint32_t bits) {
    const uint16_t b = (uint16_t)bits;
    _Float16 f;
    __builtin_memcpy(&f, &b, 2);
    return (float)f;
}

__device__ __forceinline__ uint4 swap_halves(uint4 v, bool swap) {
    return swap ? make_uint4(v.z, v.w, v.x, v.y) : v;
}

// max(x, x of lane ^ 16) and max(x, x of lane ^ 32) with gfx950's row swaps (no
// LDS round trip): each swap returns the two halves of a lane pair's values.
__device__ __forceinline__ float xmax16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xmax32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// LDS/record row of key k (0..31) of a tile: the inverse of sigma.
__device__ __forceinline__ int key_row(int k) { return 16 * ((k >> 2) & 1) + 4 * (k >> 3) + (k & 3); }

// ---------------------------------------------------------------- pre-passes

// One workgroup per (64 keys, KV head): the 64 q4_0 rows of K and of V are
// staged in LDS with 16-byte loads (zeros past n_kv), then
//   K: thread t takes blocks (key, b) = t and t + 256 (key = idx / 8, b = idx % 8):
//      its 32 codes as fp16 (4 swizzled 16-byte chunks of the key's row) and its
//      scale into the Dk row of block b;
//   V: thread t writes the Vc row of dim t (32 codes, 64 bytes) of both tiles;
//      threads 0..15 write the Dv rows and fold the largest |d_v| into
//      dvmax[head] (fp16 magnitude bits, cleared by qprep_kernel, which runs
//      first).
// N dwords of a q4_0 block's qs bytes starting at byte off (2 mod 4 for even
// blocks, 0 mod 4 for odd ones) of an LDS row: aligned reads, shifted by
// alignbit. Every read stays inside the row's 144 bytes.
template <int N = 4>
__device__ __forceinline__ void qs_dwords(const uint8_t *row, int off, uint32_t *q) {
    const uint32_t *p = reinterpret_cast<const uint32_t *>(row + (off & ~3));
    const uint32_t sh = 8u * (uint32_t)(off & 3);
    uint32_t a = p[0];
#pragma unroll
    for (int m = 0; m < N; ++m) {
        const uint32_t b = p[sh ? m + 1 : (m + 1 < N ? m + 1 : m)];
        q[m] = __builtin_amdgcn_alignbit(b, a, sh);
        a = b;
    }
}

// Two 4-bit codes n (bits 0-3 and 16-19 of x) as the packed fp16 pair n - 8:
// 0x6400 | n is exactly 1024 + n, and 1024 + n - 1032 is exact.
__device__ __forceinline__ uint32_t codes_f16(uint32_t x) {
    const uint32_t y = (x & 0x000F000Fu) | 0x64006400u;
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 v;
    __builtin_memcpy(&v, &y, 4);
    const h2 d = v + h2{(_Float16)-1032.0f, (_Float16)-1032.0f};
    uint32_t r;
    __builtin_memcpy(&r, &d, 4);
    return r;
}

__global__ __launch_bounds__(256) void kvprep_kernel(const uint8_t *__restrict__ k, int64_t k_nb1, int64_t k_nb2,
                                                     const uint8_t *__restrict__ v, int64_t v_nb1, int64_t v_nb2,
                                                     int64_t n_kv, int64_t kv_tiles, uint8_t *__restrict__ kv,
                                                     uint32_t *__restrict__ dvmax) {
    __shared__ __align__(16) uint8_t sk[64 * kHeadRowBytes], sv[64 * kHeadRowBytes];
    const int t = threadIdx.x;
    const int h = blockIdx.y;
    const int64_t k0 = (int64_t)blockIdx.x * 64;
    for (int idx = t; idx < 64 * 9; idx += 256) {  // 9 x 16 bytes per 144-byte row
        const int key = idx / 9, c = idx - 9 * key;
        uint4 a = make_uint4(0, 0, 0, 0), b = make_uint4(0, 0, 0, 0);
        if (k0 + key < n_kv) {
            a = *reinterpret_cast<const uint4 *>(k + (k0 + key) * k_nb1 + h * k_nb2 + 16 * c);
            b = *reinterpret_cast<const uint4 *>(v + (k0 + key) * v_nb1 + h * v_nb2 + 16 * c);
        }
        *reinterpret_cast<uint4 *>(sk + kHeadRowBytes * key + 16 * c) = a;
        *reinterpret_cast<uint4 *>(sv + kHeadRowBytes * key + 16 * c) = b;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int idx = t + 256 * i;
        const int key = idx >> 3, b = idx & 7;
        const uint16_t *src = reinterpret_cast<const uint16_t *>(sk + kHeadRowBytes * key + 18 * b);
        // the block's 16 qs bytes as 4 dwords (they start 2 bytes off a dword for
        // even b); codes 2j, 2j+1 (low nibbles) and 16 + 2j, 17 + 2j (high) as fp16
        uint32_t q[4];
        qs_dwords(sk + kHeadRowBytes * key, 18 * b + 2, q);
        uint32_t out[16];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t x0 = __builtin_amdgcn_perm(0u, q[m], 0x0c010c00u);  // bytes 4m, 4m+1
            const uint32_t x1 = __builtin_amdgcn_perm(0u, q[m], 0x0c030c02u);  // bytes 4m+2, 4m+3
            out[2 * m] = codes_f16(x0);
            out[2 * m + 1] = codes_f16(x1);
            out[8 + 2 * m] = codes_f16(x0 >> 4);
            out[8 + 2 * m + 1] = codes_f16(x1 >> 4);
        }
        const int64_t gkey = k0 + key;
        const int r = key_row((int)(gkey & (kPK - 1)));
        uint8_t *rec = kv + ((int64_t)h * kv_tiles + (gkey >> 5)) * kTileBytes;
        uint8_t *row = rec + r * 512;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int pos = (4 * b + j) ^ (r & 7);
            const uint4 x = make_uint4(out[4 * j], out[4 * j + 1], out[4 * j + 2], out[4 * j + 3]);
            *reinterpret_cast<uint4 *>(row + 16 * pos) = swap_halves(x, r & 8);
        }
        *reinterpret_cast<uint16_t *>(rec + kOffDk + (b * kPK + r) * 2) = src[0];
    }
    // V: thread t takes dword m of block beta's qs (dims 32 beta + 4m + i from the
    // low nibbles, 32 beta + 16 + 4m + i from the high ones, i < 4) for the 8 keys
    // 8 kg .. 8 kg + 7 and writes those keys' 16-byte chunk of each of its 8 Vc
    // rows (tile kg >> 2, chunk kg & 3); the first wavefront also writes the Dv
    // rows (below)
    {
        const int beta = (t >> 2) & 7, m = t & 3, kg = t >> 5;
        uint32_t w[8];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            uint32_t q1[1];
            qs_dwords<1>(sv + kHeadRowBytes * (8 * kg + kk), 18 * beta + 2 + 4 * m, q1);
            w[kk] = q1[0];
        }
        uint8_t *vrec = kv + ((int64_t)h * kv_tiles + ((k0 >> 5) + (kg >> 2))) * kTileBytes + kKHalf;
        const int c = kg & 3;  // keys 8c..8c+7 of the tile
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // byte i of keys 2j (bits 0-7) and 2j + 1 (bits 16-23)
            const uint32_t sel = (uint32_t)i | 0x0c00u | ((uint32_t)(4 + i) << 16) | 0x0c000000u;
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t x = __builtin_amdgcn_perm(w[2 * j + 1], w[2 * j], sel);
                lo[j] = codes_f16(x);
                hi[j] = codes_f16(x >> 4);
            }
            // chunk c of dim d at c ^ ((d >> 1) & 3), halves swapped when d & 8
            const int dl = 32 * beta + 4 * m + i, dh = dl + 16;
            *reinterpret_cast<uint4 *>(vrec + 64 * dl + 16 * (c ^ ((dl >> 1) & 3))) =
                swap_halves(make_uint4(lo[0], lo[1], lo[2], lo[3]), dl & 8);
            *reinterpret_cast<uint4 *>(vrec + 64 * dh + 16 * (c ^ ((dh >> 1) & 3))) =
                swap_halves(make_uint4(hi[0], hi[1], hi[2], hi[3]), dh & 8);
        }
        // Dv rows: thread t < 64 takes tile u, block b, keys 8q..8q+7 of the tile
        uint32_t dmax = 0;
        if (t < 64) {
            const int u = t >> 5, b = (t >> 2) & 7, q = t & 3;
            uint16_t dd[8];
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                dd[kk] = *reinterpret_cast<const uint16_t *>(sv + kHeadRowBytes * (32 * u + 8 * q + kk) + 18 * b);
                // a NaN/Inf scale (bytes that are not q4_0) reads as 0: such a key, if
                // masked, adds exactly 0 (P d_v is formed in fp16, where 0 * NaN = NaN)
                dd[kk] = (dd[kk] & 0x7C00u) == 0x7C00u ? (uint16_t)0 : dd[kk];
                const uint32_t mag = dd[kk] & 0x7fffu;
                dmax = mag > dmax ? mag : dmax;
            }
            uint8_t *vrec = kv + ((int64_t)h * kv_tiles + ((k0 >> 5) + u)) * kTileBytes + kKHalf;
            uint4 x;
            __builtin_memcpy(&x, dd, 16);
            *reinterpret_cast<uint4 *>(vrec + kOffDv + 64 * b + 16 * q) = x;
        }
        if (t < 64) {
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                const uint32_t other = (uint32_t)__shfl_xor((int)dmax, o);
                dmax = other > dmax ? other : dmax;
            }
            if (t == 0) atomicMax(dvmax + h, dmax);
        }
    }
}

// A quad of threads per 32-value block of one (query, head) row, 8 values each:
// q8_0 with ggml's x86 rounding (d = amax/127 over the block, codes =
// rint(x * 127/amax)), then Q' = code * qd with qd = fp16(d) * scale * log2(e) in
// fp32, written as fp16 hi = fp16(Q') and lo = fp16(Q' - hi).
// Exclusive key limit of query tile `tile` under an F16 mask: 1 + the last
// key any of its qb rows leaves visible (an entry other than -inf), 0 if none.
// Keys past it are masked in every row of the tile, so the main kernel stops
// there, as it does at the causal limit of the position form. Run by one
// 256-thread workgroup: each wavefront takes 4 rows at a time and reads them
// backwards 1024 keys per step (a lane takes two 8-key 16-byte loads per
// row, all 8 loads in flight at once) until a step holds a visible key, so a
// causal row costs its masked tail only: one step at pp512 (tails up to 511
// keys), two for a 2048-token ubatch. Rows are 16-byte aligned with len (a
// multiple of 8) readable keys. Every thread of the workgroup must call it.
__device__ __forceinline__ void mask_tile_limit(const char *__restrict__ mask, int64_t nb1, int64_t len, int n_q, int qb, int tile,
                                int32_t *__restrict__ lim) {
    __shared__ int32_t best[4];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int q0 = tile * qb;
    const int64_t c_top = (len - 1) / 1024 * 1024;
    const uint4 none = make_uint4(0xFC00FC00u, 0xFC00FC00u, 0xFC00FC00u, 0xFC00FC00u);
    auto last_of = [&](uint4 a, uint4 b, int64_t c0) {  // the wavefront's last visible key in one step, or -1
        int last = -1;
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 16; ++e)
            if (((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) != 0xFC00u)
                last = (int)(c0 + 512 * (e >> 3) + 8 * lane + (e & 7));
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) last = max(last, __shfl_xor(last, o));
        return last;
    };
    auto load = [&](const uint16_t *row, int64_t k) {
        return k < len ? *reinterpret_cast<const uint4 *>(row + k) : none;
    };
    int32_t mine = -1;  // wave-uniform
    for (int r0 = 4 * wave; r0 < qb; r0 += 16) {
        uint4 a[4], b[4];
        const uint16_t *rows[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {  // the first step of four rows at once
            const bool ok = r0 + j < qb && q0 + r0 + j < n_q;
            rows[j] = ok ? reinterpret_cast<const uint16_t *>(mask + (int64_t)(q0 + r0 + j) * nb1) : nullptr;
            a[j] = ok ? load(rows[j], c_top + 8 * lane) : none;
            b[j] = ok ? load(rows[j], c_top + 512 + 8 * lane) : none;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int last = last_of(a[j], b[j], c_top);
            for (int64_t c0 = c_top - 1024; last < 0 && rows[j] && c0 >= 0; c0 -= 1024)  // longer tails
                last = last_of(load(rows[j], c0 + 8 * lane), load(rows[j], c0 + 512 + 8 * lane), c0);
            mine = max(mine, last);
        }
    }
    if (lane == 0) best[wave] = mine;
    __syncthreads();
    if (threadIdx.x == 0) lim[tile] = max(max(best[0], best[1]), max(best[2], best[3])) + 1;
}

// The same as a kernel of its own, for a packed mask copy (written after the
// Q pre-pass): one workgroup per query tile.
__global__ __launch_bounds__(256) void mask_tile_limit_kernel(const char *__restrict__ mask, int64_t nb1, int64_t len,
                                                              int n_q, int qb, int32_t *__restrict__ lim) {
    mask_tile_limit(mask, nb1, len, n_q, qb, blockIdx.x, lim);
}

// Workgroups from n_qblocks on are the mask scan (mask_tile_limit) of query
// tile blockIdx.x - n_qblocks, when the kernel reads the caller's mask in place.
struct MaskScan {
    const char *mask;  // null: no scan here
    int64_t nb1, len;
    int qb, n_qblocks;
    int32_t *lim;
};

__global__ __launch_bounds__(256) void qprep_kernel(const char *__restrict__ q, int64_t nb1, int64_t nb2,
                                                    int n_q, int H, float qscale, uint16_t *__restrict__ qh,
                                                    uint16_t *__restrict__ ql, uint32_t *__restrict__ dvmax, int hkv,
                                                    bool aligned, MaskScan ms) {
    if (ms.mask && (int)blockIdx.x >= ms.n_qblocks) {
        mask_tile_limit(ms.mask, ms.nb1, ms.len, n_q, ms.qb, (int)blockIdx.x - ms.n_qblocks, ms.lim);
        return;
    }
    // one thread per 8 values: a quad of lanes owns a 32-value block
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid < hkv) dvmax[gid] = 0;  // for kvprep_kernel, launched next
    if (gid >= (int64_t)n_q * H * kBlocksPerHead * 4) return;  // whole quads: the total is a multiple of 4
    const int qtr = (int)(gid & 3);
    const int64_t bid = gid >> 2;
    const int b = (int)(bid % kBlocksPerHead);
    const int64_t row = bid / kBlocksPerHead;  // t * H + h
    const int h = (int)(row % H);
    const int64_t t = row / H;
    const float *x = reinterpret_cast<const float *>(q + t * nb1 + h * nb2) + 32 * b + 8 * qtr;
    float v[8];
    if (aligned) {  // 16-byte aligned rows: vector loads
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float4 f = reinterpret_cast<const float4 *>(x)[j];
            v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = x[j];
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    // the block's amax over the quad (quad_perm [1,0,3,2], then [2,3,0,1])
    amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0xB1, 0xf, 0xf, false)));
    amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(amax), 0x4E, 0xf, 0xf, false)));
    const float d = amax / 127.f;
    const float id = amax != 0.0f ? 127.f / amax : 0.0f;
    const float qd = (float)(_Float16)d * qscale;
    uint16_t oh[8], ol[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        // x opaque: left visible, the compiler may round code * qd to fp16 twice
        // (once from the fp32 product for hi, once from the exact product for the
        // hi it subtracts), and a hi + lo off by one fp16 ulp of hi
        float xx = rintf(v[j] * id) * qd;
        asm volatile("" : "+v"(xx));
        const _Float16 hh = (_Float16)xx;
        const _Float16 ll = (_Float16)(xx - (float)hh);
        __builtin_memcpy(&oh[j], &hh, 2);
        __builtin_memcpy(&ol[j], &ll, 2);
    }
    uint4 a, c;
    __builtin_memcpy(&a, oh, 16);
    __builtin_memcpy(&c, ol, 16);
    *reinterpret_cast<uint4 *>(qh + row * kHeadDim + 32 * b + 8 * qtr) = a;
    *reinterpret_cast<uint4 *>(ql + row * kHeadDim + 32 * b + 8 * qtr) = c;
}

// Copies an F16 mask whose rows are unaligned or whose length is not a
// multiple of 8 into [n_q][len8] rows (len8 = n_kv rounded up to 8, -inf pad).
__global__ __launch_bounds__(256) void pf_mask_pack_kernel(const char *__restrict__ src, int64_t nb1, int64_t n_kv,
                                                           int n_q, int64_t len8, uint16_t *__restrict__ dst) {
    const int64_t total = len8 * n_q;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t t = i / len8, kk = i - t * len8;
        dst[i] = kk < n_kv ? reinterpret_cast<const uint16_t *>(src + t * nb1)[kk] : (uint16_t)0xFC00;
    }
}

// ------------------------------------------------------------ main kernel

// 16 bytes per lane from sbase + voff into LDS at m0 + 16 * lane (asynchronous;
// the caller waits with s_waitcnt vmcnt).
__device__ __forceinline__ void dma16(uint32_t voff, const void *sbase, uint32_t m0v) {
    // m0 as an operand: the compiler writes it and knows it holds the LDS base
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0v) : "memory");
}

// Two 8-byte LDS reads into one MFMA operand. volatile keeps them two single
// ds_read_b64 straight into the operand's registers: merged into ds_read2 pairs
// they would bring halves of different operands and need register moves.
__device__ __forceinline__ half8 lds_half8(const uint8_t *base, int off_lo, int off_hi) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    typedef const volatile __attribute__((address_space(3))) u32x2 lds_u32x2;
    const u32x2 a = *(lds_u32x2 *)(base + off_lo);
    const u32x2 b = *(lds_u32x2 *)(base + off_hi);
    const uint4 u = make_uint4(a.x, a.y, b.x, b.y);
    half8 h;
    __builtin_memcpy(&h, &u, 16);
    return h;
}


struct PrefillParams {
    const uint8_t *kv;        // [Hkv][kv_tiles] tile records
    const uint32_t *dvmax;    // [Hkv] fp16 magnitude bits
    const uint16_t *qh, *ql;  // [n_q*H][256] fp16 Q' hi and lo
    int64_t n_kv, kv_tiles;
    int n_q, H, G, Hkv;
    const char *mask;  // F16 rows 16-byte aligned, mask_len (a multiple of 8) keys each, or null
    int64_t mask_nb1, mask_len;
    int64_t q_pos0;    // >= 0: causal from positions (mask ignored)
    const int32_t *tile_lim;  // with a mask: [q_tiles] exclusive key limit of each query tile
    int n_splits;
    int q_tiles;        // workgroups per (KV head, split)
    int64_t split_len;  // keys per split, a multiple of kPK
    int qb;             // query positions per workgroup (128 / G)
    int mask_stage;     // LDS bytes per mask stage (qb x 64)
    float *part_acc, *part_ml;  // n_splits > 1
    float *dst;                 // n_splits == 1: [n_q][H][256]
    const char *gate;
    int64_t gate_nb1, gate_nb2;
};

__global__ __launch_bounds__(kThreads, 1) void fa_prefill_kernel(PrefillParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, g = lane >> 4, n = lane & 15;
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

    // Workgroups are dealt round-robin to the 8 XCDs (each with its own L2).
    // Renumber so that each XCD gets a contiguous run of ids, i.e. the query
    // tiles of the same (KV head, split): they stream the same K/V range, which
    // that XCD's L2 then serves to all of them.
    const int nb = (int)gridDim.x;
    const int lin = (int)blockIdx.x;
    const int id = nb % 8 == 0 ? (lin % 8) * (nb / 8) + lin / 8 : lin;
    const int q_tile = id % p.q_tiles;
    const int grp = id / p.q_tiles;
    const int kvh = grp / p.n_splits, split = grp % p.n_splits;
    const int q_base = q_tile * p.qb;

    // Key range: the split, cut at the last key any query of the workgroup sees.
    const int64_t k_begin = (int64_t)split * p.split_len;
    int64_t k_end = k_begin + p.split_len < p.n_kv ? k_begin + p.split_len : p.n_kv;
    if (p.q_pos0 >= 0) {
        const int64_t q_last = (q_base + p.qb < p.n_q ? q_base + p.qb : p.n_q) - 1;
        const int64_t lim = p.q_pos0 + q_last + 1;
        if (k_end > lim) k_end = lim;
    } else if (p.tile_lim) {  // the mask's last visible key over the tile's rows
        const int64_t lim = p.tile_lim[q_tile];
        if (k_end > lim) k_end = lim;
    }
    const int n_tiles = k_end > k_begin ? (int)((k_end - k_begin + kPK - 1) / kPK) : 0;

    // ---------------- DMA: 1 KB per instruction, a fixed share per wave ---------
    // Iteration t: K half + mask of tile t + 1, V half of tile t (stage = tile & 1).
    // K instruction jj (0..16, the last one 512 bytes) goes to wave jj % 8, V
    // instruction jj to wave (jj + 4) % 8, mask instruction jm (< 8) to wave
    // (jm + 2) % 8.
    const int n_mask_inst = p.mask ? (p.qb + 15) / 16 : 0;
    const uint8_t *kv_h = p.kv + (int64_t)kvh * p.kv_tiles * kTileBytes;
    const int jk0 = wave, jv0 = (wave + 4) % kWaves, jm = (wave + kWaves - 2) % kWaves;
    const bool has_m = jm < n_mask_inst;
    static_assert(kKInst == 2 * kWaves + 1 && kVInst == 2 * kWaves + 1, "two full DMA instructions per wave and half");
    const bool k_half = jk0 == 0, v_half = jv0 == 0;  // the wave that issues the 512-byte instruction
    // mask row of this lane's slot in instruction jm: position q_base + r (clamped
    // to n_q - 1), chunk c = (s & 3) ^ ((r >> 1) & 3) of the row's 32 keys
    const int m_r = (64 * jm + lane) >> 2;
    const int m_c = ((64 * jm + lane) & 3) ^ ((m_r >> 1) & 3);
    const uint32_t m_row =
        has_m ? (uint32_t)((int64_t)(q_base + m_r < p.n_q ? q_base + m_r : p.n_q - 1) * p.mask_nb1) : 0u;
    const bool m_lane = m_r < p.qb;
    // record of the split's first tile (k_begin is a multiple of kPK); tile t's
    // record is t records further on
    const uint8_t *rec0 = kv_h + (k_begin / kPK) * kTileBytes;
    auto issue = [&](int t_k, int t_v) {  // tile indices or -1
        if (t_k >= 0) {
            const uint8_t *rec = rec0 + (int64_t)t_k * kTileBytes;
            const uint32_t st = lds0 + (uint32_t)((t_k & 1) * kKStage);
            // instructions jk0 and jk0 + 8 (full), and 16 (512 bytes) on wave 0
            dma16(1024u * jk0 + 16u * lane, rec, st + 1024u * jk0);
            dma16(1024u * (jk0 + kWaves) + 16u * lane, rec, st + 1024u * (jk0 + kWaves));
            if (k_half && lane < 32) dma16(1024u * (kKInst - 1) + 16u * lane, rec, st + 1024u * (kKInst - 1));
            if (has_m) {
                const int64_t kt = k_begin + (int64_t)t_k * kPK;
                const int64_t col = kt + 8 * m_c < p.mask_len ? kt + 8 * m_c : p.mask_len - 8;
                const uint32_t sm = lds0 + (uint32_t)(kLdsMask + (t_k & 1) * p.mask_stage + 1024 * jm);
                if (m_lane) dma16(m_row + (uint32_t)(2 * col), p.mask, sm);
            }
        }
        if (t_v >= 0) {
            const uint8_t *rec = rec0 + (int64_t)t_v * kTileBytes + kKHalf;
            const uint32_t st = lds0 + (uint32_t)(kLdsV + (t_v & 1) * kVStage);
            dma16(1024u * jv0 + 16u * lane, rec, st + 1024u * jv0);
            dma16(1024u * (jv0 + kWaves) + 16u * lane, rec, st + 1024u * (jv0 + kWaves));
            if (v_half && lane < 32) dma16(1024u * (kVInst - 1) + 16u * lane, rec, st + 1024u * (kVInst - 1));
        }
    };
    if (n_tiles > 0) issue(0, -1);

    // e2 with max |d_v| * 2^e2 in [1, 2) (at most 15)
    int e2 = 0;
    {
        const float dm = h2f(p.dvmax[kvh]);
        if (dm > 0.0f) {
            int e;
            (void)frexpf(dm, &e);
            e2 = 1 - e < 15 ? 1 - e : 15;
        }
    }
    // 2^ep rides on P (the score waves' exp2 argument); O and l both carry it,
    // so it cancels in O / l. The lazy rescale keeps P 2^ep <= 2^(ks + ep), and
    // |d_v| < 2^(1 - e2), so A = P 2^ep d_v < 2^(ks + ep + 1 - e2):
    //   e2 >= 0: ep = e2 (at most 7), ks = 8: A < 2^9, P 2^ep <= 2^15;
    //   e2 < 0: ks + ep = 14 + e2 (A < 2^15), ep = 0 while ks can give way
    //     (down to 3), then ep < 0 (to -4 at fp16's largest d_v).
    // Lowering ep instead (ep = e2 for large V, max |d_v| >= 2) put the P of keys
    // a few binades below the row maximum into the fp16 subnormals, where its
    // lo half vanishes: outputs up to 3e-3 x RMS from the exact result. A smaller
    // slack only moves the reference maximum more often.
    int ep = e2 > 7 ? 7 : e2, ks = kSlack;
    if (e2 < 0) {
        const int top = 14 + e2;  // log2 of the largest P 2^ep that A's range admits
        ks = top >= kSlack ? kSlack : (top >= 3 ? top : 3);
        ep = top >= 3 ? 0 : top - 3;
    }
    const float lim_top = (float)(ks + ep);  // the lazy test's bound on s'
    const int nh = (n >> 3) & 1;

    // The two kinds of wave run separate code with the same barrier count:
    // n_tiles + 1 in the loop, then two for the hand-over of m and l.
    if (wave < kScoreWaves) {
        const int w = wave;
        float *ml = reinterpret_cast<float *>(smem + kLdsP) + w * (kRG * 32);  // [rg][row][m, l]
        // Q' hi and lo of rows r = 32w + 16rg + n (position q_base + r / G, head
        // kvh*G + r % G) as B operands, dims 32b + 8g..+7
        half8 bqh[kRG][8], bql[kRG][8];
        int my_pos[kRG], m_off[kRG];
        float m_run[kRG], l_part[kRG];
        // The logits are accumulated relative to the row's P reference mref =
        // (m_run, or 0 before the first visible key) - ep: s' = s - mref, so that
        // P = 2^s' needs no subtraction, and the lazy-maximum test s > m_run +
        // ks reads s' > lim_s (ks + ep, or -inf before the first visible key).
        // Both change only when the maximum moves.
        float mref[kRG], lim_s[kRG];
#pragma unroll
        for (int rg = 0; rg < kRG; ++rg) {
            const int r = 32 * w + 16 * rg + n;
            const int pos = q_base + r / p.G;
            my_pos[rg] = pos;
            const bool ok = pos < p.n_q;
            const uint32_t m = ok ? 0xffffffffu : 0u;
            const int64_t row = (int64_t)(ok ? pos : 0) * p.H + kvh * p.G + r % p.G;
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                uint4 u = *reinterpret_cast<const uint4 *>(p.qh + row * kHeadDim + 32 * b + 8 * g);
                uint4 v = *reinterpret_cast<const uint4 *>(p.ql + row * kHeadDim + 32 * b + 8 * g);
                u = make_uint4(u.x & m, u.y & m, u.z & m, u.w & m);
                v = make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
                __builtin_memcpy(&bqh[rg][b], &u, 16);
                __builtin_memcpy(&bql[rg][b], &v, 16);
            }
            const int pl = r / p.G;  // mask row of the position, keys 8g..8g+7
            m_off[rg] = kLdsMask + 64 * pl + 16 * (g ^ ((pl >> 1) & 3));
            m_run[rg] = -INFINITY;
            l_part[rg] = 0.0f;
            mref[rg] = -(float)ep;
            lim_s[rg] = -INFINITY;
        }
        // K operand of key row 16kg + n, dims 32b + 8g..+7: chunk (4b + g) ^ (n & 7),
        // halves swapped when n & 8; the XOR touches bit 2 of 4b + g, so even and odd
        // b use two bases and b >> 1 adds 128 bytes.
        int k_off[2][2];  // [b & 1][half]
#pragma unroll
        for (int bp = 0; bp < 2; ++bp)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) k_off[bp][hf] = n * 512 + 16 * ((4 * bp + g) ^ (n & 7)) + 8 * (hf ^ nh);
        const int p_off = w * (kRG * 2048) + 16 * lane;  // P slots [w][rg][half][lane]

        for (int t = 0; t <= n_tiles && n_tiles > 0; ++t) {
            // this wave's DMAs landed; the barrier makes every wave's visible and
            // retires the buffers the new DMAs overwrite
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            issue(t + 1 < n_tiles ? t + 1 : -1, t < n_tiles ? t : -1);
            if (t == n_tiles) break;
            const int64_t kt = k_begin + (int64_t)t * kPK;
            const int nvalid = (int)(k_end - kt < kPK ? k_end - kt : kPK);
            // this tile's four per-lane K bases, opaque to the compiler: every K read
            // is then one of them plus an immediate offset (hoisting all 64
            // base + offset sums out of the loop would need 64 more registers)
            int kb[2][2];
#pragma unroll
            for (int bp = 0; bp < 2; ++bp)
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    kb[bp][hf] = (t & 1) * kKStage + k_off[bp][hf];
                    asm volatile("" : "+v"(kb[bp][hf]));
                }
            // mask rows of the tile, read now so that their latency hides behind QK
            uint4 mrow[kRG];
            if (p.mask) {
#pragma unroll
                for (int rg = 0; rg < kRG; ++rg)
                    mrow[rg] = *reinterpret_cast<const uint4 *>(smem + m_off[rg] + (t & 1) * p.mask_stage);
            }
            // ---- S^T: sa[rg][kg][i] = S[key kt + 8g + 4kg + i][row n of group rg] ----
            floatx4 sa[kRG][2];
#pragma unroll
            for (int rg = 0; rg < kRG; ++rg) sa[rg][0] = sa[rg][1] = -mref[rg];
            // d_k of the lane's four C rows 16kg + 4g + i, block b: 8 bytes at
            // Dk[b][16kg + 4g]
            const uint8_t *dkb = smem + (t & 1) * kKStage + kOffDk + 8 * g;
            // Software-pipelined by one step: step j = (block j >> 1, key group j & 1)
            // issues its MFMAs, then the d_k scaling of step j - 1 runs while they
            // execute. The scheduling barrier keeps the compiler from pulling the
            // scaling back next to the MFMAs it reads (it did, leaving 4-12
            // instructions between an MFMA and its consumer). The sum into sa keeps
            // the block order of the plain loop.
            floatx4 cp[kRG];
            uint2 dkp;
#pragma unroll
            for (int j = 0; j <= 16; ++j) {
                floatx4 cn[kRG];
                uint2 dkn;
                if (j < 16) {
                    const int b = j >> 1, kg = j & 1;
                    const int o = kg * 8192 + 128 * (b >> 1);
                    const half8 ak = lds_half8(smem, kb[b & 1][0] + o, kb[b & 1][1] + o);
                    dkn = *reinterpret_cast<const uint2 *>(dkb + 64 * b + 32 * kg);
#pragma unroll
                    for (int rg = 0; rg < kRG; ++rg) {
                        const floatx4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, bqh[rg][b],
                                                                                 floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        cn[rg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, bql[rg][b], c, 0, 0, 0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                if (j > 0) {
                    const int kg = (j - 1) & 1;
                    _Float16 dk[4];
                    __builtin_memcpy(dk, &dkp, 8);
#pragma unroll
                    for (int rg = 0; rg < kRG; ++rg)
#pragma unroll
                        for (int i = 0; i < 4; ++i) sa[rg][kg][i] = fmaf(cp[rg][i], (float)dk[i], sa[rg][kg][i]);
                }
                if (j < 16) {
                    dkp = dkn;
#pragma unroll
                    for (int rg = 0; rg < kRG; ++rg) cp[rg] = cn[rg];
                }
            }
            float s[kRG][8];  // keys 8g + jj, base-2 logits
#pragma unroll
            for (int rg = 0; rg < kRG; ++rg)
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) s[rg][jj] = sa[rg][jj >> 2][jj & 3];
            // ---- mask / causal / ragged tail ----------------------------------------
            // a block of the mask that is +0 for all of this wave's rows and keys (every
            // fully visible tile of a causal mask) changes no logit: skip it
            bool mask_live = false;
            if (p.mask) {
                uint32_t any = 0;
#pragma unroll
                for (int rg = 0; rg < kRG; ++rg) any |= mrow[rg].x | mrow[rg].y | mrow[rg].z | mrow[rg].w;
                mask_live = __any(any != 0u);
            }
            if (mask_live) {
#pragma unroll
                for (int rg = 0; rg < kRG; ++rg) {
                    const uint32_t mw[4] = {mrow[rg].x, mrow[rg].y, mrow[rg].z, mrow[rg].w};
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        // a -inf entry excludes the key whatever its logit (even NaN from
                        // a garbage scale): ggml's CPU loop skips such keys
                        const uint32_t mb = (mw[jj >> 1] >> (16 * (jj & 1))) & 0xffff;
                        s[rg][jj] = mb == 0xFC00u ? -INFINITY : fmaf(h2f(mb), kLog2e, s[rg][jj]);
                    }
                }
            }
            if (nvalid < kPK || (p.q_pos0 >= 0 && kt + kPK - 1 > p.q_pos0 + q_base)) {
#pragma unroll
                for (int rg = 0; rg < kRG; ++rg) {
                    int64_t lim = nvalid;  // keys at or past lim are dead for this row
                    if (p.q_pos0 >= 0 && p.q_pos0 + my_pos[rg] + 1 - kt < lim) lim = p.q_pos0 + my_pos[rg] + 1 - kt;
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) s[rg][jj] = 8 * g + jj < lim ? s[rg][jj] : -INFINITY;
                }
            }
            // ---- online softmax (base 2); P and the rescale factors to LDS -----------
            uint8_t *pb = smem + kLdsP + (t & 1) * kPBuf + p_off;
            float *ab = reinterpret_cast<float *>(smem + kLdsA + (t & 1) * kABuf) + w * (kRG * 16);
#pragma unroll
            for (int rg = 0; rg < kRG; ++rg) {
                // lazy maximum: the reference moves only when a logit passes it by more
                // than ks, so P <= 2^ks and most tiles need no rescale of O
                float alpha = 1.0f;
                bool over = false;
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) over |= s[rg][jj] > lim_s[rg];
                if (__any(over)) {
                    float mt = fmaxf(fmaxf(fmaxf(s[rg][0], s[rg][1]), fmaxf(s[rg][2], s[rg][3])),
                                     fmaxf(fmaxf(s[rg][4], s[rg][5]), fmaxf(s[rg][6], s[rg][7])));
                    mt = xmax16(mt);
                    mt = xmax32(mt);
                    const float m_new = fmaxf(m_run[rg], mt + mref[rg]);
                    alpha = m_run[rg] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run[rg] - m_new);
                    l_part[rg] *= alpha;
                    m_run[rg] = m_new;
                    // onto the new reference: s - mref_new = s' + (mref - mref_new)
                    const float mref_new = (m_new == -INFINITY ? 0.0f : m_new) - (float)ep;
                    const float d = mref[rg] - mref_new;
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) s[rg][jj] += d;
                    mref[rg] = mref_new;
                    lim_s[rg] = m_new == -INFINITY ? -INFINITY : lim_top;
                }
                float pf[8], psum = 0.0f;
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    pf[jj] = __builtin_amdgcn_exp2f(s[rg][jj]);
                    psum += pf[jj];
                }
                l_part[rg] += psum;
                // P as an fp16 hi + lo pair (22 bits): the value waves form P d_v from it
                half8 ph, pl;
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) ph[jj] = (_Float16)pf[jj];
                // the exact residual p - hi, with hi read from its packed fp16 half by
                // v_fma_mix (no conversion of hi back to fp32)
                uint32_t hw[4];
                __builtin_memcpy(hw, &ph, 16);
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    float r;
                    if (jj & 1)
                        asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "=v"(r) : "v"(pf[jj]), "v"(hw[jj >> 1]));
                    else
                        asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel:[0,0,0] op_sel_hi:[0,0,1]" : "=v"(r) : "v"(pf[jj]), "v"(hw[jj >> 1]));
                    pl[jj] = (_Float16)r;
                }
                *reinterpret_cast<half8 *>(pb + rg * 2048) = ph;
                *reinterpret_cast<half8 *>(pb + rg * 2048 + 1024) = pl;
                if (g == 0) ab[rg * 16 + n] = alpha;
            }
        }
        // ---- hand m and l of the rows to the value waves ----------------------------
        __syncthreads();
        if (n_tiles > 0) {
#pragma unroll
            for (int rg = 0; rg < kRG; ++rg) {
                float lp = l_part[rg];
                lp += __shfl_xor(lp, 16);
                lp += __shfl_xor(lp, 32);
                if (g == 0) {
                    ml[rg * 32 + 2 * n] = m_run[rg];
                    ml[rg * 32 + 2 * n + 1] = lp;
                }
            }
        }
        __syncthreads();
        return;
    }

    // ---- value waves: O[row 32w + 16rg + 4g + i][dim 16T + n] ----------------
    const int w = wave - kScoreWaves;
    const float *ml = reinterpret_cast<const float *>(smem + kLdsP) + w * (kRG * 32);  // [rg][row][m, l]
    // V operand of dim 16T + n, keys 8g..8g+7: chunk g ^ ((n >> 1) & 3), halves swapped when n & 8.
    const int v_off0 = 64 * n + 16 * (g ^ ((n >> 1) & 3)) + 8 * nh;
    const int v_off1 = v_off0 ^ 8;
    const int p_off = w * (kRG * 2048) + 16 * lane;
    floatx4 acc[kRG][16];
#pragma unroll
    for (int rg = 0; rg < kRG; ++rg)
#pragma unroll
        for (int T = 0; T < 16; ++T) acc[rg][T] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int t = 0; t <= n_tiles && n_tiles > 0; ++t) {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        issue(t + 1 < n_tiles ? t + 1 : -1, t < n_tiles ? t : -1);
        if (t == 0) continue;
        const int tp = t - 1;
        const uint8_t *vs = smem + kLdsV + (tp & 1) * kVStage;
        // this tile's two per-lane V bases, opaque to the compiler (see the K reads)
        int vb0 = kLdsV + (tp & 1) * kVStage + v_off0, vb1 = kLdsV + (tp & 1) * kVStage + v_off1;
        asm volatile("" : "+v"(vb0), "+v"(vb1));
        const uint8_t *pb = smem + kLdsP + (tp & 1) * kPBuf + p_off;
        const float *ab = reinterpret_cast<const float *>(smem + kLdsA + (tp & 1) * kABuf) + w * (kRG * 16);
        half8 ph[kRG], pl[kRG];
        bool resc = false;
#pragma unroll
        for (int rg = 0; rg < kRG; ++rg) {
            // rescale factors of rows 4g..4g+3: exactly 1 unless a maximum moved
            const floatx4 a4 = *reinterpret_cast<const floatx4 *>(ab + rg * 16 + 4 * g);
            resc |= (a4[0] != 1.0f) | (a4[1] != 1.0f) | (a4[2] != 1.0f) | (a4[3] != 1.0f);
            ph[rg] = *reinterpret_cast<const half8 *>(pb + rg * 2048);
            pl[rg] = *reinterpret_cast<const half8 *>(pb + rg * 2048 + 1024);
        }
        if (__any(resc)) {  // rare with the lazy maximum: O = alpha O
#pragma unroll
            for (int rg = 0; rg < kRG; ++rg) {
                const floatx4 a4 = *reinterpret_cast<const floatx4 *>(ab + rg * 16 + 4 * g);
#pragma unroll
                for (int T = 0; T < 16; ++T) acc[rg][T] *= a4;
            }
        }
        // d_v of the 8 blocks and V of block 0 first, then V of block b + 1 while
        // block b computes: the LDS latency stays off the MFMA chain
        uint4 dvr[8];
#pragma unroll
        for (int b = 0; b < 8; ++b) dvr[b] = *reinterpret_cast<const uint4 *>(vs + kOffDv + 64 * b + 16 * g);
        half8 bvn[2];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) bvn[hf] = lds_half8(smem, vb0 + 1024 * hf, vb1 + 1024 * hf);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const half8 bv[2] = {bvn[0], bvn[1]};
            if (b < 7) {
#pragma unroll
                for (int hf = 0; hf < 2; ++hf)
                    bvn[hf] = lds_half8(smem, vb0 + 1024 * (2 * b + 2 + hf), vb1 + 1024 * (2 * b + 2 + hf));
            }
            half8 dvb;
            __builtin_memcpy(&dvb, &dvr[b], 16);
            // A = P 2^ep d_v as an fp16 hi + lo pair (22 bits): the products with the
            // exact V codes are then exact in fp32, so a row that a few keys
            // dominate carries no fp16 rounding of P d_v into its output. Ph d_v has
            // at most 22 significant bits, so its residual after rounding to fp16
            // (at most 11 bits) is exact in one fma; Pl d_v is 2^-11 of it and
            // rounds once.
            half8 ah[kRG], al[kRG];
#pragma unroll
            for (int rg = 0; rg < kRG; ++rg) {
                ah[rg] = ph[rg] * dvb;
                const half8 r = __builtin_elementwise_fma(ph[rg], dvb, -ah[rg]);
                al[rg] = __builtin_elementwise_fma(pl[rg], dvb, r);
            }
#pragma unroll
            for (int rg = 0; rg < kRG; ++rg)
#pragma unroll
                for (int hf = 0; hf < 2; ++hf)
                    acc[rg][2 * b + hf] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[rg], bv[hf], acc[rg][2 * b + hf], 0, 0, 0);
#pragma unroll
            for (int rg = 0; rg < kRG; ++rg)
#pragma unroll
                for (int hf = 0; hf < 2; ++hf)
                    acc[rg][2 * b + hf] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[rg], bv[hf], acc[rg][2 * b + hf], 0, 0, 0);
        }
    }
    __syncthreads();  // m and l of the rows ...
    __syncthreads();  // ... are in LDS
    const int rows_total = p.n_q * p.H;
#pragma unroll
    for (int rg = 0; rg < kRG; ++rg) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 32 * w + 16 * rg + 4 * g + i;
            const int qrow = q_base + r / p.G, hrow = kvh * p.G + r % p.G;
            if (qrow >= p.n_q) continue;
            const float mrow = n_tiles > 0 ? ml[rg * 32 + 2 * (4 * g + i)] : -INFINITY;
            const float lrow = n_tiles > 0 ? ml[rg * 32 + 2 * (4 * g + i) + 1] : 0.0f;
            const int64_t ridx = (int64_t)qrow * p.H + hrow;
            if (p.n_splits == 1) {
                const float inv = lrow == 0.0f ? 0.0f : 1.0f / lrow;
#pragma unroll
                for (int T = 0; T < 16; ++T) {
                    float o = acc[rg][T][i] * inv;
                    if (p.gate) {
                        const float gv = reinterpret_cast<const float *>(p.gate + qrow * p.gate_nb2 +
                                                                         hrow * p.gate_nb1)[16 * T + n];
                        o = o * (1.0f / (1.0f + expf(-gv)));
                    }
                    store_through(p.dst + ridx * kHeadDim + 16 * T + n, o);
                }
            } else {
                float *pa_out = p.part_acc + ((int64_t)split * rows_total + ridx) * kHeadDim;
#pragma unroll
                for (int T = 0; T < 16; ++T) store_through(pa_out + 16 * T + n, acc[rg][T][i]);
                if (n == 0) {
                    // the combine works in base e: m * ln 2 (acc and l of every split
                    // carry the same 2^ep, which cancels in the merge)
                    store_through(p.part_ml + ((int64_t)split * rows_total + ridx) * 2,
                                  mrow == -INFINITY ? mrow : mrow * 0.6931471805599453f);
                    store_through(p.part_ml + ((int64_t)split * rows_total + ridx) * 2 + 1, lrow);
                }
            }
        }
    }
}

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

struct PrefillPlan {
    int64_t kv_tiles;
    int qb, q_tiles, n_splits, mask_stage;
    int64_t split_len;
    size_t off_kv, off_dvmax, off_qh, off_ql, off_mask, off_lim, off_pa, off_pm, total;
};

PrefillPlan plan(int64_t n_q, int64_t H, int64_t Hkv, int64_t n_kv) {
    PrefillPlan pl{};
    const int G = (int)(H / Hkv);
    pl.qb = kRowsPerWG / G;
    pl.mask_stage = pl.qb * kPK * 2;
    pl.kv_tiles = (n_kv + 63) / 64 * 2;  // vdeq writes 64-key groups
    pl.q_tiles = (int)((n_q + pl.qb - 1) / pl.qb);
    const int64_t wgs = (int64_t)pl.q_tiles * Hkv;
    const int64_t cus = device_cu_count();
    int64_t splits = (cus + wgs - 1) / wgs;
    const int64_t max_by_len = (n_kv + 511) / 512;  // at least ~512 keys per split
    if (splits > max_by_len) splits = max_by_len;
    if (splits > kMaxSplits) splits = kMaxSplits;
    if (splits < 1) splits = 1;
    pl.split_len = ((n_kv + splits - 1) / splits + kPK - 1) / kPK * kPK;
    pl.n_splits = (int)((n_kv + pl.split_len - 1) / pl.split_len);
    size_t o = 0;
    pl.off_kv = o; o = al256(o + (size_t)Hkv * pl.kv_tiles * kTileBytes);
    pl.off_dvmax = o; o = al256(o + (size_t)Hkv * 4);
    pl.off_qh = o; o = al256(o + (size_t)n_q * H * kHeadDim * 2);
    pl.off_ql = o; o = al256(o + (size_t)n_q * H * kHeadDim * 2);
    pl.off_mask = o; o = al256(o + (size_t)n_q * ((n_kv + 7) / 8 * 8) * 2);
    pl.off_lim = o; o = al256(o + (size_t)pl.q_tiles * 4);
    pl.off_pa = o;
    pl.off_pm = o;
    if (pl.n_splits > 1) {
        o = al256(o + (size_t)pl.n_splits * n_q * H * kHeadDim * 4);
        pl.off_pm = o;
        o = al256(o + (size_t)pl.n_splits * n_q * H * 2 * 4);
    }
    pl.total = o + 256;
    return pl;
}

}  // namespace

size_t fa_prefill_workspace(int64_t n_q, int64_t H, int64_t Hkv, int64_t n_kv) {
    return plan(n_q, H, Hkv, n_kv).total;
}

int launch_fa_prefill(const FaArgs &a, hipStream_t s) {
    const sqa_tensor &q = *a.q, &k = *a.k, &v = *a.v;
    const int64_t n_q = q.ne[1], H = q.ne[2], n_kv = k.ne[1], Hkv = k.ne[2];
    const int G = (int)(H / Hkv);
    if (16 % G != 0) return set_error(SQA_ERR_UNSUPPORTED, "prefill: n_head/n_head_kv must divide 16");
    const PrefillPlan pl = plan(n_q, H, Hkv, n_kv);
    if (!a.ws || a.ws_bytes < pl.total)
        return set_error(SQA_ERR_WORKSPACE, "flash_attn_ext: workspace %zu bytes < %zu needed", a.ws_bytes,
                         pl.total);
    uint8_t *base = reinterpret_cast<uint8_t *>(((uintptr_t)a.ws + 255) & ~(uintptr_t)255);
    uint8_t *kv = base + pl.off_kv;
    uint32_t *dvmax = reinterpret_cast<uint32_t *>(base + pl.off_dvmax);
    uint16_t *qh = reinterpret_cast<uint16_t *>(base + pl.off_qh);
    uint16_t *ql = reinterpret_cast<uint16_t *>(base + pl.off_ql);

    PrefillParams p;
    p.mask = nullptr;
    p.mask_nb1 = 0;
    p.mask_len = 0;
    const char *mask_src = nullptr;
    int64_t mask_src_nb1 = 0;
    if (a.q_pos0 < 0 && a.mask) {
        mask_src = (const char *)a.mask->data;
        mask_src_nb1 = (int64_t)a.mask->nb[1];
        if ((uintptr_t)mask_src % 16 == 0 && mask_src_nb1 % 16 == 0 && n_kv % 8 == 0) {
            p.mask = mask_src;
            p.mask_nb1 = mask_src_nb1;
            p.mask_len = n_kv;
            mask_src = nullptr;
        } else {
            const int64_t len8 = (n_kv + 7) / 8 * 8;
            p.mask = (const char *)(base + pl.off_mask);
            p.mask_nb1 = len8 * 2;
            p.mask_len = len8;
        }
        // the mask DMA addresses rows with 32-bit offsets
        if ((n_q - 1) * p.mask_nb1 + p.mask_len * 2 > (int64_t)UINT32_MAX)
            return set_error(SQA_ERR_UNSUPPORTED, "prefill: mask of %lld rows x %lld bytes exceeds 4 GiB",
                             (long long)n_q, (long long)p.mask_nb1);
    }

    int prof = profile_start("fa_prefill_prep", s);
    {
        const int64_t nqb = n_q * H * kBlocksPerHead;
        const int qblocks = (int)((4 * nqb + 255) / 256);
        int32_t *lim = reinterpret_cast<int32_t *>(base + pl.off_lim);
        // an in-place mask is scanned by extra workgroups of the Q pre-pass, a
        // packed copy by a kernel of its own once it is written
        const MaskScan ms{p.mask && !mask_src ? p.mask : nullptr, p.mask_nb1, p.mask_len, pl.qb, qblocks, lim};
        qprep_kernel<<<dim3((unsigned)(qblocks + (ms.mask ? pl.q_tiles : 0))), dim3(256), 0, s>>>(
            (const char *)q.data, (int64_t)q.nb[1], (int64_t)q.nb[2], (int)n_q, (int)H, a.scale * kLog2e, qh, ql,
            dvmax, (int)Hkv, (uintptr_t)q.data % 16 == 0 && q.nb[1] % 16 == 0 && q.nb[2] % 16 == 0, ms);
        kvprep_kernel<<<dim3((unsigned)(pl.kv_tiles / 2), (unsigned)Hkv), dim3(256), 0, s>>>(
            (const uint8_t *)k.data, (int64_t)k.nb[1], (int64_t)k.nb[2], (const uint8_t *)v.data, (int64_t)v.nb[1],
            (int64_t)v.nb[2], n_kv, pl.kv_tiles, kv, dvmax);
        if (mask_src) {
            int64_t grid = (p.mask_len * n_q + 255) / 256;
            if (grid > 2048) grid = 2048;
            pf_mask_pack_kernel<<<dim3((unsigned)grid), dim3(256), 0, s>>>(
                mask_src, mask_src_nb1, n_kv, (int)n_q, p.mask_len, (uint16_t *)(base + pl.off_mask));
        }
        if (mask_src)  // the packed copy, just written
            mask_tile_limit_kernel<<<dim3((unsigned)pl.q_tiles), dim3(256), 0, s>>>(
                p.mask, p.mask_nb1, p.mask_len, (int)n_q, pl.qb, reinterpret_cast<int32_t *>(base + pl.off_lim));
    }
    profile_stop(prof, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_status(e, "prefill pre-pass launch");

    p.tile_lim = p.mask ? reinterpret_cast<const int32_t *>(base + pl.off_lim) : nullptr;
    p.kv = kv;
    p.dvmax = dvmax;
    p.qh = qh;
    p.ql = ql;
    p.n_kv = n_kv;
    p.kv_tiles = pl.kv_tiles;
    p.n_q = (int)n_q;
    p.H = (int)H;
    p.G = G;
    p.Hkv = (int)Hkv;
    p.q_pos0 = a.q_pos0;
    p.n_splits = pl.n_splits;
    p.q_tiles = pl.q_tiles;
    p.split_len = pl.split_len;
    p.qb = pl.qb;
    p.mask_stage = pl.mask_stage;
    p.part_acc = reinterpret_cast<float *>(base + pl.off_pa);
    p.part_ml = reinterpret_cast<float *>(base + pl.off_pm);
    p.dst = (float *)a.dst->data;
    p.gate = (pl.n_splits == 1 && a.gate) ? (const char *)a.gate->data : nullptr;
    p.gate_nb1 = a.gate ? (int64_t)a.gate->nb[1] : 0;
    p.gate_nb2 = a.gate ? (int64_t)a.gate->nb[2] : 0;

    const int lds_bytes = kLdsMask + (p.mask ? 2 * pl.mask_stage : 0);
    // The function's LDS limit is raised once per process to the largest size
    // any launch uses, so concurrent first calls cannot leave a smaller one set.
    static std::once_flag lds_once;
    static hipError_t lds_err = hipSuccess;
    std::call_once(lds_once, [] {
        lds_err = hipFuncSetAttribute((const void *)fa_prefill_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      kLdsMaxBytes);
    });
    if (lds_err != hipSuccess) return hip_status(lds_err, "fa_prefill LDS attribute");
    prof = profile_start("fa_prefill", s);
    fa_prefill_kernel<<<dim3((unsigned)(pl.q_tiles * Hkv * pl.n_splits)), dim3(kThreads), lds_bytes, s>>>(p);
    profile_stop(prof, s);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_status(e, "fa_prefill launch");
    if (pl.n_splits > 1)
        return launch_fa_combine(p.part_acc, p.part_ml, pl.n_splits, (int)(n_q * H), p.dst, a.gate, (int)H, s);
    return SQA_OK;
}

}  // namespace sqa
