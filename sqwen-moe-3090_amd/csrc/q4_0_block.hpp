// q4_0_block.hpp - ggml's quantize_row_q4_0_ref for one 32-value block held by
// 8 consecutive lanes (4 consecutive values each), bit for bit:
//   max  = value of largest |x| in the block, first occurrence on ties
//   d    = max / -8            (stored as fp16, round-to-nearest-even)
//   id   = d != 0 ? 1/d : 0    (correctly rounded fp32 division)
//   code = min(15, (int8_t)(x*id + 8.5f)) with the multiply and the add each
//          rounded on their own (contraction off: no fused multiply-add)
// An all-zero block therefore stores d = -0.0 (fp16 0x8000) and codes 8.
#pragma once
#include "common.hpp"

namespace sqa {

// v: this lane's 4 values (block elements 4t..4t+3, t = lane & 7); blk: the
// 18-byte block. All 8 lanes of the group must call it together.
__device__ __forceinline__ void quantize_q4_0_block8(const float v[4], int t, uint8_t *blk) {
    // x*id + 8.5f as two roundings: with contraction on (hipcc's default, and
    // inside HIP's __fmul_rn / __fadd_rn, which are plain * and +) it became one
    // fma (v_fmaak_f32), and a value whose x*id lies within half an ulp below a
    // half-integer then truncated to the code below ggml's
#pragma clang fp contract(off)
    // Lane-local first-occurrence maximum of |x|; index 32 marks "none".
    float amax = 0.0f, mx = 0.0f;
    int im = 32;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float a = fabsf(v[j]);
        if (amax < a) { amax = a; mx = v[j]; im = 4 * t + j; }
    }
#pragma unroll
    for (int off = 4; off >= 1; off >>= 1) {
        const float a2 = __shfl_xor(amax, off, 8);
        const float m2 = __shfl_xor(mx, off, 8);
        const int i2 = __shfl_xor(im, off, 8);
        if (a2 > amax || (a2 == amax && i2 < im)) { amax = a2; mx = m2; im = i2; }
    }

    const float d = mx / -8.0f;
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float y = v[j] * id + 8.5f;
        int c = (int)y;  // truncation toward zero, y in [0.5, 16.5] for finite input
        c = c < 15 ? c : 15;
        word |= (uint32_t)(c & 0xff) << (8 * j);
    }
    // qs[j] = code[j] | code[j+16] << 4: lanes 0..3 take the high nibbles from lanes 4..7.
    const uint32_t hi = __shfl_down(word, 4, 8);
    if (t < 4) {
        const uint32_t qs = word | (hi << 4);
        uint16_t *p = reinterpret_cast<uint16_t *>(blk + 2 + 4 * t);
        p[0] = (uint16_t)(qs & 0xffff);
        p[1] = (uint16_t)(qs >> 16);
    } else if (t == 4) {
        const _Float16 dh = (_Float16)d;
        *reinterpret_cast<_Float16 *>(blk) = dh;
    }
}

}  // namespace sqa
