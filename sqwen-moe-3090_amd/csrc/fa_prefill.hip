// fa_prefill.hip - FlashAttention for prefill chunks (n_q * H/Hkv > 16 query
// rows per KV head): the ubatch node of src/model/attn.rs:228-251 in the
// reference (n_q = 512 or 2048 over a q4_0 cache of 16K-133K keys).
//
// Three short pre-passes, then one MFMA kernel:
//   kdeq  K q4_0 -> Kf  fp16 hi, lo [Hkv][n_kv][256]
//   vdeq  V q4_0 -> Vt  fp16 hi, lo [Hkv][256][n_kv_pad]  (transposed: keys contiguous)
//   qprep Q f32  -> q8_0 (ggml's x86 rounding) -> Q' = q8*d
// Every dequantized value x = (nib-8)*d or q8*d is split as hi = fp16(x),
// lo = fp16(x - hi); x needs at most 18 significant bits and hi + lo hold 22,
// so Q', K and V enter the MFMAs exactly. Only P is rounded to fp16 once.
// K/V are dequantized once per call instead of once per query tile.
//
// fa_prefill_kernel: a workgroup takes 16 query rows per wave x 8 waves of
// ONE KV head (GQA packing: with 8 q heads per KV head that is 16 positions x
// 8 heads), streams 32-key tiles of Kf and Vt through LDS and runs
//   S^T = K Q'^T  on v_mfma_f32_16x16x32_f16: Kh.Qh + Kh.Ql + Kl.Qh (the
//                 Kl.Ql term is below 2^-22 relative and dropped),
//   online softmax in fp32,
//   O  += P V     on v_mfma_f32_16x16x32_f16: P.Vh + P.Vl (P rounded to fp16).
// Computing S^T (keys as rows) leaves each lane with 8 logits of one query
// row, which is exactly the A-operand layout of the P*V MFMA. Long key ranges
// with few query tiles are split across workgroups and merged by fa_combine.
//
// Operand layout of the 16x16x32 MFMAs (64 lanes, lane = 16*g + n):
//   A: A[row n][k = 8g..8g+7]   B: B[k = 8g..8g+7][col n]   C: C[rows 4g..4g+3][col n]
#include "common.hpp"

namespace sqa {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));

constexpr int kPK = 32;           // keys per tile
constexpr int kWaves = 8;         // 16 query rows each
constexpr int kThreads = 64 * kWaves;
constexpr int kKRow = 512 + 16;   // LDS bytes per fp16 K row (padded against bank conflicts)
constexpr int kVRow = 64 + 16;    // LDS bytes per transposed V row (32 keys, padded)
constexpr int kMaxQ = 16 * kWaves;  // query positions per workgroup when G = 1
constexpr float kLog2e = 1.4426950408889634f;

// v if keep, else zeros; a per-component AND keeps the operand in registers
// (a select between two uint4 objects can be lowered to a select of their
// addresses, which forces both onto the scratch stack).
__device__ __forceinline__ uint4 keep_if(uint4 v, bool keep) {
    const uint32_t m = keep ? 0xffffffffu : 0u;
    return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
}

__device__ __forceinline__ float h2f(uint32_t bits) {
    const uint16_t b = (uint16_t)bits;
    _Float16 f;
    __builtin_memcpy(&f, &b, 2);
    return (float)f;
}

// ---------------------------------------------------------------- pre-passes

// x -> (hi, lo) fp16 bit patterns with hi + lo == x for x of <= 22 significant bits.
__device__ __forceinline__ void split_hl(float x, uint16_t &hi, uint16_t &lo) {
    const _Float16 h = (_Float16)x;
    const _Float16 l = (_Float16)(x - (float)h);
    __builtin_memcpy(&hi, &h, 2);
    __builtin_memcpy(&lo, &l, 2);
}

// One thread per q4_0 block of K: 18 bytes in, 32 fp16 hi + 32 fp16 lo out.
__global__ __launch_bounds__(256) void kdeq_kernel(const uint8_t *__restrict__ k, int64_t nb1, int64_t nb2,
                                                   int64_t n_kv, int hkv, uint16_t *__restrict__ kf,
                                                   uint16_t *__restrict__ kfl) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = n_kv * hkv * kBlocksPerHead;
    if (gid >= total) return;
    const int b = (int)(gid % kBlocksPerHead);
    const int64_t kh = gid / kBlocksPerHead;  // key * hkv + head
    const int h = (int)(kh % hkv);
    const int64_t key = kh / hkv;
    const uint16_t *src = reinterpret_cast<const uint16_t *>(k + key * nb1 + h * nb2 + 18 * b);
    const float d = h2f(src[0]);
    uint16_t out[32], outl[32];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t two = src[1 + j];  // qs[2j], qs[2j+1]
        const int b0 = two & 0xff, b1 = two >> 8;
        split_hl((float)((b0 & 15) - 8) * d, out[2 * j], outl[2 * j]);
        split_hl((float)((b1 & 15) - 8) * d, out[2 * j + 1], outl[2 * j + 1]);
        split_hl((float)((b0 >> 4) - 8) * d, out[16 + 2 * j], outl[16 + 2 * j]);
        split_hl((float)((b1 >> 4) - 8) * d, out[16 + 2 * j + 1], outl[16 + 2 * j + 1]);
    }
    const int64_t off = ((int64_t)h * n_kv + key) * kHeadDim + 32 * b;
    uint4 *dst = reinterpret_cast<uint4 *>(kf + off);
    uint4 *dstl = reinterpret_cast<uint4 *>(kfl + off);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint4 v, w;
        __builtin_memcpy(&v, out + 8 * j, 16);
        __builtin_memcpy(&w, outl + 8 * j, 16);
        dst[j] = v;
        dstl[j] = w;
    }
}

// One workgroup per (64 keys, head): thread t handles keys 8*(t%8)..+7 of the
// 8 dims {32beta + 4w + j, 32beta + 16 + 4w + j} (beta = t/32, w = (t/8)%4), and
// writes each dim's 8 keys as one 16-byte row segment of Vt. Keys past n_kv
// are written as zeros, so the padded tail of Vt is finite.
__global__ __launch_bounds__(256) void vdeq_kernel(const uint8_t *__restrict__ v, int64_t nb1, int64_t nb2,
                                                   int64_t n_kv, int64_t n_kv_pad, uint16_t *__restrict__ vt,
                                                   uint16_t *__restrict__ vtl) {
    const int t = threadIdx.x;
    const int h = blockIdx.y;
    const int64_t k0 = (int64_t)blockIdx.x * 64 + 8 * (t & 7);
    const int beta = t >> 5;
    const int w = (t >> 3) & 3;
    uint16_t lo[8][4], hi[8][4], lol[8][4], hil[8][4];  // [key][j], hi/lo parts
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
        const int64_t key = k0 + kk;
        const bool ok = key < n_kv;
        const uint16_t *blk = reinterpret_cast<const uint16_t *>(v + (ok ? key : 0) * nb1 + h * nb2 + 18 * beta);
        const float d = ok ? h2f(blk[0]) : 0.0f;
        const uint32_t q01 = blk[1 + 2 * w], q23 = blk[2 + 2 * w];
        const uint32_t x = q01 | (q23 << 16);  // qs[4w..4w+3]
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int byte = (x >> (8 * j)) & 0xff;
            split_hl((float)((byte & 15) - 8) * d, lo[kk][j], lol[kk][j]);
            split_hl((float)((byte >> 4) - 8) * d, hi[kk][j], hil[kk][j]);
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint16_t row_lo[8], row_hi[8], row_lol[8], row_hil[8];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            row_lo[kk] = lo[kk][j];
            row_hi[kk] = hi[kk][j];
            row_lol[kk] = lol[kk][j];
            row_hil[kk] = hil[kk][j];
        }
        const int dlo = 32 * beta + 4 * w + j;
        uint4 a, b, c, e;
        __builtin_memcpy(&a, row_lo, 16);
        __builtin_memcpy(&b, row_hi, 16);
        __builtin_memcpy(&c, row_lol, 16);
        __builtin_memcpy(&e, row_hil, 16);
        const int64_t o0 = ((int64_t)h * kHeadDim + dlo) * n_kv_pad + k0;
        const int64_t o1 = ((int64_t)h * kHeadDim + dlo + 16) * n_kv_pad + k0;
        *reinterpret_cast<uint4 *>(vt + o0) = a;
        *reinterpret_cast<uint4 *>(vt + o1) = b;
        *reinterpret_cast<uint4 *>(vtl + o0) = c;
        *reinterpret_cast<uint4 *>(vtl + o1) = e;
    }
}

// One thread per 32-value block of one (query, head) row: q8_0 with ggml's x86
// rounding (d = amax/127, codes = rint(x * 127/amax)), then Q' = code * fp16(d)
// (exact in fp32) split as hi = fp16(Q'), lo = fp16(Q' - hi) (exact).
__global__ __launch_bounds__(256) void qprep_kernel(const char *__restrict__ q, int64_t nb1, int64_t nb2,
                                                    int n_q, int H, uint16_t *__restrict__ qhi,
                                                    uint16_t *__restrict__ qlo) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (int64_t)n_q * H * kBlocksPerHead) return;
    const int b = (int)(gid % kBlocksPerHead);
    const int64_t row = gid / kBlocksPerHead;  // t * H + h
    const int h = (int)(row % H);
    const int64_t t = row / H;
    const float *x = reinterpret_cast<const float *>(q + t * nb1 + h * nb2) + 32 * b;
    float v[32];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        v[j] = x[j];
        amax = fmaxf(amax, fabsf(v[j]));
    }
    const float d = amax / 127.f;
    const float id = amax != 0.0f ? 127.f / amax : 0.0f;
    const float dh = (float)(_Float16)d;
    uint16_t oh[32], ol[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float qq = rintf(v[j] * id) * dh;  // exact: 7-bit code x 11-bit scale
        const _Float16 hh = (_Float16)qq;
        const _Float16 ll = (_Float16)(qq - (float)hh);
        __builtin_memcpy(&oh[j], &hh, 2);
        __builtin_memcpy(&ol[j], &ll, 2);
    }
    uint4 *dh4 = reinterpret_cast<uint4 *>(qhi + row * kHeadDim + 32 * b);
    uint4 *dl4 = reinterpret_cast<uint4 *>(qlo + row * kHeadDim + 32 * b);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint4 a, c;
        __builtin_memcpy(&a, oh + 8 * j, 16);
        __builtin_memcpy(&c, ol + 8 * j, 16);
        dh4[j] = a;
        dl4[j] = c;
    }
}

// ------------------------------------------------------------ main kernel

struct PrefillParams {
    const uint16_t *kf, *kfl, *vt, *vtl, *qhi, *qlo;
    int64_t n_kv, n_kv_pad;
    int n_q, H, G, Hkv;
    const char *mask;  // F16 [n_kv, >= n_q] or null
    int64_t mask_nb1;
    int64_t q_pos0;    // >= 0: causal from positions
    float scale;
    int n_splits;
    int q_tiles;        // workgroups per (KV head, split)
    int64_t split_len;  // keys per split, a multiple of kPK
    float *part_acc, *part_ml;  // n_splits > 1
    float *dst;                 // n_splits == 1: [n_q][H][256]
    const char *gate;
    int64_t gate_nb1, gate_nb2;
};

__global__ __launch_bounds__(kThreads, 1) void fa_prefill_kernel(PrefillParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t *sK = smem;                          // hi: [32 keys][kKRow]
    uint8_t *sKl = smem + kPK * kKRow;           // lo
    uint8_t *sV = smem + 2 * kPK * kKRow;        // hi: [256 dims][kVRow]
    uint8_t *sVl = sV + kHeadDim * kVRow;        // lo
    uint16_t *sM = reinterpret_cast<uint16_t *>(sVl + kHeadDim * kVRow);  // [queries][32]

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, n = lane & 15;
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
    const int QW = 16 / p.G;           // query positions per wave
    const int QB = QW * kWaves;        // query positions per workgroup
    const int q_base = q_tile * QB;

    // This lane's query row (column n of S^T and row n of the P*V A operand).
    const int my_q = q_base + wave * QW + n / p.G;
    const int my_h = kvh * p.G + n % p.G;
    const bool row_ok = my_q < p.n_q;
    const int my_ql = wave * QW + n / p.G;  // query index inside the workgroup

    // Key range: the split, cut at the last key any query of the workgroup sees.
    int64_t k_begin = (int64_t)split * p.split_len;
    int64_t k_end = k_begin + p.split_len < p.n_kv ? k_begin + p.split_len : p.n_kv;
    if (p.q_pos0 >= 0) {
        const int64_t q_last = (q_base + QB < p.n_q ? q_base + QB : p.n_q) - 1;
        const int64_t lim = p.q_pos0 + q_last + 1;
        if (k_end > lim) k_end = lim;
    }

    // Q' (hi, lo) as B operands: lane holds row n, dims 32ks + 8g .. +7.
    half8 bqh[8], bql[8];
    {
        const int64_t roff = ((int64_t)(row_ok ? my_q : 0) * p.H + my_h) * kHeadDim;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const uint4 a = *reinterpret_cast<const uint4 *>(p.qhi + roff + 32 * ks + 8 * g);
            const uint4 b = *reinterpret_cast<const uint4 *>(p.qlo + roff + 32 * ks + 8 * g);
            __builtin_memcpy(&bqh[ks], &a, 16);
            __builtin_memcpy(&bql[ks], &b, 16);
        }
    }

    floatx4 acc[16];  // O[row 4g+i][dim 16T + n]
#pragma unroll
    for (int T = 0; T < 16; ++T) acc[T] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_part = 0.0f;

    // Tile staging through registers: per thread 2 chunks (16 B) of each of
    // Kh, Kl (32 keys x 512 B) and Vh, Vl (256 dims x 64 B).
    uint4 pk[2], pkl[2], pv[2], pvl[2];
    uint4 pmsk = make_uint4(0, 0, 0, 0);
    int pre_nvalid = 0;
    const bool mask_loader = p.mask && tid < QB * 4;  // 4 lanes x 8 keys per query position
    const int mq = tid >> 2, mc = (tid & 3) * 8;
    const bool mask_aligned = ((uintptr_t)p.mask % 16 == 0) && (p.mask_nb1 % 16 == 0);
    const uint16_t *kf_h = p.kf + (int64_t)kvh * p.n_kv * kHeadDim;
    const uint16_t *kfl_h = p.kfl + (int64_t)kvh * p.n_kv * kHeadDim;
    const uint16_t *vt_h = p.vt + (int64_t)kvh * kHeadDim * p.n_kv_pad;
    const uint16_t *vtl_h = p.vtl + (int64_t)kvh * kHeadDim * p.n_kv_pad;
    auto load_tile = [&](int64_t kt, int nvalid) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = tid + kThreads * i;  // 0..1023
            const int key = c >> 5, col = c & 31;
            const int64_t ko = (kt + (key < nvalid ? key : 0)) * kHeadDim + 8 * col;
            pk[i] = *reinterpret_cast<const uint4 *>(kf_h + ko);
            pkl[i] = *reinterpret_cast<const uint4 *>(kfl_h + ko);
            const int dim = c >> 2, seg = c & 3;
            const int64_t vo = (int64_t)dim * p.n_kv_pad + kt + 8 * seg;
            pv[i] = *reinterpret_cast<const uint4 *>(vt_h + vo);
            pvl[i] = *reinterpret_cast<const uint4 *>(vtl_h + vo);
        }
        if (p.mask && wave * 64 < QB * 4) {  // wave-uniform
            const int qq = q_base + (mask_loader ? mq : 0);
            const int64_t mrow = qq < p.n_q ? qq : 0;
            const uint16_t *mp = reinterpret_cast<const uint16_t *>(p.mask + mrow * p.mask_nb1) + kt;
            if (mask_aligned && nvalid == kPK) {  // uniform; stays in flight
                pmsk = *reinterpret_cast<const uint4 *>(mp + mc);
            } else {  // last tile of a range or unaligned rows: waits here
                uint16_t e[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) e[j] = mp[mc + j < nvalid ? mc + j : 0];
                __builtin_memcpy(&pmsk, e, 16);
            }
        }
        pre_nvalid = nvalid;
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = tid + kThreads * i;
            const int key = c >> 5, col = c & 31;
            const bool ok = key < pre_nvalid;
            *reinterpret_cast<uint4 *>(sK + key * kKRow + 16 * col) = keep_if(pk[i], ok);
            *reinterpret_cast<uint4 *>(sKl + key * kKRow + 16 * col) = keep_if(pkl[i], ok);
            const int dim = c >> 2, seg = c & 3;
            *reinterpret_cast<uint4 *>(sV + dim * kVRow + 16 * seg) = keep_if(pv[i], true);
            *reinterpret_cast<uint4 *>(sVl + dim * kVRow + 16 * seg) = keep_if(pvl[i], true);
        }
        if (mask_loader) *reinterpret_cast<uint4 *>(sM + mq * kPK + mc) = pmsk;
    };

    const int64_t n_tiles = k_end > k_begin ? (k_end - k_begin + kPK - 1) / kPK : 0;
    if (n_tiles > 0) {
        load_tile(k_begin, (int)(k_end - k_begin < kPK ? k_end - k_begin : kPK));
        store_tile();
    }
    __syncthreads();

    for (int64_t it = 0; it < n_tiles; ++it) {
        const int64_t kt = k_begin + it * kPK;
        const int nvalid = (int)(k_end - kt < kPK ? k_end - kt : kPK);
        if (it + 1 < n_tiles) {
            const int64_t kn = kt + kPK;
            load_tile(kn, (int)(k_end - kn < kPK ? k_end - kn : kPK));
        }
        {
            const int k0 = 0;
            float s[2][4];
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                floatx4 c = {0.f, 0.f, 0.f, 0.f};
                const int koff = (k0 + 16 * st + n) * kKRow + 16 * g;
#pragma unroll
                for (int ks = 0; ks < 8; ++ks) {
                    const half8 a = *reinterpret_cast<const half8 *>(sK + koff + 64 * ks);
                    const half8 al = *reinterpret_cast<const half8 *>(sKl + koff + 64 * ks);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bqh[ks], c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bql[ks], c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bqh[ks], c, 0, 0, 0);
                }
                const int kc = k0 + 16 * st + 4 * g;
                uint2 mraw = make_uint2(0, 0);
                if (p.mask) mraw = *reinterpret_cast<const uint2 *>(sM + my_ql * kPK + kc);
                const uint32_t mw[2] = {mraw.x, mraw.y};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int kl = kc + i;
                    float sv = c[i] * p.scale;
                    bool dead = kl >= nvalid;
                    if (p.q_pos0 >= 0) {
                        dead = dead || (kt + kl > p.q_pos0 + my_q);
                    } else if (p.mask && row_ok) {
                        const float mv = h2f((mw[i >> 1] >> (16 * (i & 1))) & 0xffff);
                        dead = dead || (mv == -INFINITY);
                        sv += mv;
                    }
                    s[st][i] = dead ? -INFINITY : sv;
                }
            }
            float mt = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                             fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
            mt = fmaxf(mt, __shfl_xor(mt, 16));
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float m_new = fmaxf(m_run, mt);
            const float mref = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = exp2f((m_run - mref) * kLog2e);
            half8 pa;
            float psum = 0.0f;
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const float pr = exp2f((s[jj >> 2][jj & 3] - mref) * kLog2e);
                psum += pr;
                pa[jj] = (_Float16)pr;
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
            // O += P V: B[k][dim 16T+n], k = 8g+jj -> key 4g + jj (jj<4), 16 + 4g + jj-4
#pragma unroll
            for (int T = 0; T < 16; ++T) {
                const int vo = (16 * T + n) * kVRow + 2 * (k0 + 4 * g);
                const uint2 b0 = *reinterpret_cast<const uint2 *>(sV + vo);
                const uint2 b1 = *reinterpret_cast<const uint2 *>(sV + vo + 32);
                const uint2 c0 = *reinterpret_cast<const uint2 *>(sVl + vo);
                const uint2 c1 = *reinterpret_cast<const uint2 *>(sVl + vo + 32);
                const uint4 bb = make_uint4(b0.x, b0.y, b1.x, b1.y);
                const uint4 cc = make_uint4(c0.x, c0.y, c1.x, c1.y);
                half8 bv, bvl;
                __builtin_memcpy(&bv, &bb, 16);
                __builtin_memcpy(&bvl, &cc, 16);
                acc[T] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, bv, acc[T], 0, 0, 0);
                acc[T] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, bvl, acc[T], 0, 0, 0);
            }
        }
        __syncthreads();
        if (it + 1 < n_tiles) store_tile();
        __syncthreads();
    }

    // ---- epilogue: each wave owns its 16 rows
    l_part += __shfl_xor(l_part, 16);
    l_part += __shfl_xor(l_part, 32);
    float lrow[4], mrow[4];
    int qrow[4], hrow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        lrow[i] = __shfl(l_part, 4 * g + i);
        mrow[i] = __shfl(m_run, 4 * g + i);
        qrow[i] = q_base + wave * QW + (4 * g + i) / p.G;
        hrow[i] = kvh * p.G + (4 * g + i) % p.G;
    }
    const int rows_total = p.n_q * p.H;
    if (p.n_splits == 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (qrow[i] >= p.n_q) continue;
            const int64_t r = (int64_t)qrow[i] * p.H + hrow[i];
            const float inv = lrow[i] == 0.0f ? 0.0f : 1.0f / lrow[i];
#pragma unroll
            for (int T = 0; T < 16; ++T) {
                float o = acc[T][i] * inv;
                if (p.gate) {
                    const float gv = reinterpret_cast<const float *>(p.gate + qrow[i] * p.gate_nb2 +
                                                                     hrow[i] * p.gate_nb1)[16 * T + n];
                    o = o * (1.0f / (1.0f + expf(-gv)));
                }
                p.dst[r * kHeadDim + 16 * T + n] = o;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (qrow[i] >= p.n_q) continue;
            const int64_t r = (int64_t)qrow[i] * p.H + hrow[i];
            float *pa = p.part_acc + ((int64_t)split * rows_total + r) * kHeadDim;
#pragma unroll
            for (int T = 0; T < 16; ++T) pa[16 * T + n] = acc[T][i];
            if (n == 0) {
                p.part_ml[((int64_t)split * rows_total + r) * 2] = mrow[i];
                p.part_ml[((int64_t)split * rows_total + r) * 2 + 1] = lrow[i];
            }
        }
    }
}

constexpr size_t kLdsBytes = 2 * (size_t)kPK * kKRow + 2 * (size_t)kHeadDim * kVRow + (size_t)kMaxQ * kPK * 2;

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

struct PrefillPlan {
    int64_t n_kv_pad;
    int q_tiles, n_splits;
    int64_t split_len;
    size_t off_kf, off_kfl, off_vt, off_vtl, off_qh, off_ql, off_pa, off_pm, total;
};

PrefillPlan plan(int64_t n_q, int64_t H, int64_t Hkv, int64_t n_kv) {
    PrefillPlan pl{};
    const int G = (int)(H / Hkv);
    const int QB = (16 / G) * kWaves;
    pl.n_kv_pad = (n_kv + 63) / 64 * 64;  // vdeq writes 64-key groups
    pl.q_tiles = (int)((n_q + QB - 1) / QB);
    const int64_t wgs = (int64_t)pl.q_tiles * Hkv;
    const int64_t cus = device_cu_count();
    int64_t splits = (cus + wgs - 1) / wgs;
    const int64_t max_by_len = (n_kv + 1023) / 1024;  // at least ~1024 keys per split
    if (splits > max_by_len) splits = max_by_len;
    if (splits < 1) splits = 1;
    pl.split_len = ((n_kv + splits - 1) / splits + kPK - 1) / kPK * kPK;
    pl.n_splits = (int)((n_kv + pl.split_len - 1) / pl.split_len);
    size_t o = 0;
    pl.off_kf = o; o = al256(o + (size_t)Hkv * n_kv * kHeadDim * 2);
    pl.off_kfl = o; o = al256(o + (size_t)Hkv * n_kv * kHeadDim * 2);
    pl.off_vt = o; o = al256(o + (size_t)Hkv * kHeadDim * pl.n_kv_pad * 2);
    pl.off_vtl = o; o = al256(o + (size_t)Hkv * kHeadDim * pl.n_kv_pad * 2);
    pl.off_qh = o; o = al256(o + (size_t)n_q * H * kHeadDim * 2);
    pl.off_ql = o; o = al256(o + (size_t)n_q * H * kHeadDim * 2);
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
    uint16_t *kf = reinterpret_cast<uint16_t *>(base + pl.off_kf);
    uint16_t *kfl = reinterpret_cast<uint16_t *>(base + pl.off_kfl);
    uint16_t *vt = reinterpret_cast<uint16_t *>(base + pl.off_vt);
    uint16_t *vtl = reinterpret_cast<uint16_t *>(base + pl.off_vtl);
    uint16_t *qh = reinterpret_cast<uint16_t *>(base + pl.off_qh);
    uint16_t *ql = reinterpret_cast<uint16_t *>(base + pl.off_ql);

    int prof = profile_start("fa_prefill_prep", s);
    {
        const int64_t nk = n_kv * Hkv * kBlocksPerHead;
        kdeq_kernel<<<dim3((unsigned)((nk + 255) / 256)), dim3(256), 0, s>>>(
            (const uint8_t *)k.data, (int64_t)k.nb[1], (int64_t)k.nb[2], n_kv, (int)Hkv, kf, kfl);
        vdeq_kernel<<<dim3((unsigned)(pl.n_kv_pad / 64), (unsigned)Hkv), dim3(256), 0, s>>>(
            (const uint8_t *)v.data, (int64_t)v.nb[1], (int64_t)v.nb[2], n_kv, pl.n_kv_pad, vt, vtl);
        const int64_t nqb = n_q * H * kBlocksPerHead;
        qprep_kernel<<<dim3((unsigned)((nqb + 255) / 256)), dim3(256), 0, s>>>(
            (const char *)q.data, (int64_t)q.nb[1], (int64_t)q.nb[2], (int)n_q, (int)H, qh, ql);
    }
    profile_stop(prof, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_status(e, "prefill pre-pass launch");

    PrefillParams p;
    p.kf = kf;
    p.kfl = kfl;
    p.vt = vt;
    p.vtl = vtl;
    p.qhi = qh;
    p.qlo = ql;
    p.n_kv = n_kv;
    p.n_kv_pad = pl.n_kv_pad;
    p.n_q = (int)n_q;
    p.H = (int)H;
    p.G = G;
    p.Hkv = (int)Hkv;
    p.mask = (a.q_pos0 < 0 && a.mask) ? (const char *)a.mask->data : nullptr;
    p.mask_nb1 = a.mask ? (int64_t)a.mask->nb[1] : 0;
    p.q_pos0 = a.q_pos0;
    p.scale = a.scale;
    p.n_splits = pl.n_splits;
    p.q_tiles = pl.q_tiles;
    p.split_len = pl.split_len;
    p.part_acc = reinterpret_cast<float *>(base + pl.off_pa);
    p.part_ml = reinterpret_cast<float *>(base + pl.off_pm);
    p.dst = (float *)a.dst->data;
    p.gate = (pl.n_splits == 1 && a.gate) ? (const char *)a.gate->data : nullptr;
    p.gate_nb1 = a.gate ? (int64_t)a.gate->nb[1] : 0;
    p.gate_nb2 = a.gate ? (int64_t)a.gate->nb[2] : 0;

    static bool lds_ok = false;
    if (!lds_ok) {
        e = hipFuncSetAttribute((const void *)fa_prefill_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)kLdsBytes);
        if (e != hipSuccess) return hip_status(e, "fa_prefill LDS attribute");
        lds_ok = true;
    }
    prof = profile_start("fa_prefill", s);
    fa_prefill_kernel<<<dim3((unsigned)(pl.q_tiles * Hkv * pl.n_splits)), dim3(kThreads), kLdsBytes, s>>>(p);
    profile_stop(prof, s);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_status(e, "fa_prefill launch");
    if (pl.n_splits > 1)
        return launch_fa_combine(p.part_acc, p.part_ml, pl.n_splits, (int)(n_q * H), p.dst, a.gate, (int)H, s);
    return SQA_OK;
}

}  // namespace sqa
