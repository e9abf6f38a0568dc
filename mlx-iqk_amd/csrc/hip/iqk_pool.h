// fp16 weights from 2-bit codes through a four-entry v_perm table: shared by
// the dequant producer and the fused prefill GEMM.
//
// Bit-exactness: a sub-block's four weights are the CPU dequantizer's f32
// chain dl = d * float(index), y = dl * float(value) (each product exact),
// rounded once to fp16 (make_pool).  They are formed once per sub-block, and
// each pair of output weights is one v_perm_b32 from that 8-byte table.
#ifndef IQK_POOL_H
#define IQK_POOL_H

#include "iqk_device.h"

namespace iqk {

// Four fp16 values as a v_perm pool: low bytes in slots 0-3, high bytes in
// slots 4-7, so the selector for a code c is (c, 4+c).
struct Pool {
    uint32_t lo, hi;
};

// The four entries are dl * v_c rounded once to fp16.  The products pass
// through an empty asm so they reach v_cvt_f16_f32 as f32 values: folded into
// v_fma_mix(dl, v, +0.0) instead, a -0.0 product (a negative scale times a
// zero index) would come out +0.0, one fp16 bit off the CPU chain.
__device__ __forceinline__ float opaque(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ Pool make_pool(float dl, float v0, float v1, float v2, float v3) {
    const float y0 = opaque(dl * v0), y1 = opaque(dl * v1), y2 = opaque(dl * v2), y3 = opaque(dl * v3);
    const uint32_t p01 = float_to_half_bits(y0) | (float_to_half_bits(y1) << 16);
    const uint32_t p23 = float_to_half_bits(y2) | (float_to_half_bits(y3) << 16);
    return {perm(p23, p01, 0x06040200u), perm(p23, p01, 0x07050301u)};
}

__device__ __forceinline__ _Float16 half_of_bits(uint32_t bits) { return __builtin_bit_cast(_Float16, uint16_t(bits)); }

// 16 codes of one word -> 8 dwords of fp16 pairs in k order.  Weight k's
// code sits in byte k/4 of e[k%4]; output dword 2b pairs weights (4b, 4b+1),
// dword 2b+1 pairs (4b+2, 4b+3).  A first perm spreads the two codes to
// (ca, ca, cb, cb), the or makes it the lookup selector (ca, 4+ca, cb, 4+cb).
__device__ __forceinline__ void expand_word(uint32_t qw, Pool p, uint32_t *out) {
    const uint32_t e0 = qw & 0x03030303u;
    const uint32_t e1 = (qw >> 2) & 0x03030303u;
    const uint32_t e2 = (qw >> 4) & 0x03030303u;
    const uint32_t e3 = (qw >> 6) & 0x03030303u;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const uint32_t spread = uint32_t(b) * 0x00000101u + uint32_t(b + 4) * 0x01010000u;
        const uint32_t s01 = perm(e1, e0, spread) | 0x04000400u;
        const uint32_t s23 = perm(e3, e2, spread) | 0x04000400u;
        out[2 * b] = perm(p.hi, p.lo, s01);
        out[2 * b + 1] = perm(p.hi, p.lo, s23);
    }
}

// 16 codes of one word -> 8 dwords of fp16 pairs in the order a GEMM operand
// may take when its other operand is permuted to match: dword 2j holds weights
// (j, j+4), dword 2j+1 weights (j+8, j+12), j = 0..3.  One perm looks up the
// low bytes of four weights, one the high bytes, two more interleave them:
// 23 VALU per 16 weights (expand_word's natural order takes 31).
__device__ __forceinline__ void expand_word_paired(uint32_t qw, Pool p, uint32_t *out) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t e = (qw >> (2 * j)) & 0x03030303u;  // codes j, j+4, j+8, j+12
        const uint32_t lo = perm(p.lo, p.lo, e), hi = perm(p.hi, p.hi, e);
        out[2 * j] = perm(hi, lo, 0x05010400u);
        out[2 * j + 1] = perm(hi, lo, 0x07030602u);
    }
}

}  // namespace iqk

#endif  // IQK_POOL_H
