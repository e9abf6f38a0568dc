// Decode GEMV on int8 MFMA (gfx950) for the three members: the routed
// decode's fast path.
//
// Reference: the Metal decode GEMV (src/mlx_iqk/kernels.py:286-401) computes
// out[m, r] = half(sum_sb dl_sb * sum_{j in sb} w_j x_j) with an f32 fma
// chain per lane.  Here the multiply-accumulate runs on
// v_mfma_i32_16x16x64_i8.
//
// * Weights as int8.  IQ2_KS/IQ2_K: both alphabets (-31,-13,1,17) and
//   (-26,-8,6,22) fit int8.  IQ1_S_R4: 8 * (g + shift) with g in {-1,0,1}
//   and shift +-1/8 is one of (-7,1,9) or (-9,-1,7).  Either way one
//   v_perm_b32 maps four packed 2-bit codes to four int8 weights, from a
//   4-byte pool chosen by the sub-block's alphabet / shift-sign bit.
//   IQ1_S_R4 looks its eight weights per grid index up in the grid expanded
//   to int8 (8g + 1) in LDS; the negative shift's 8g - 1 is the exact
//   correction -2 sum(f) of the block's integer activations.  Each workgroup
//   expands the grid from its 4 KiB of 2-bit codes (a quarter of the bytes
//   of the expanded grid), each entry's weights in the paired order
//   0,4,1,5,2,6,3,7, which the staged activations follow.
// * Activations as integers.  x is converted once per workgroup with a
//   per-32-element power-of-two scale, f = rint(x * 2^E), |f| <= 2^20, and
//   split into balanced bytes f = b0 + 2^8 b1 + 2^16 b2 (each b in
//   [-128, 127]: the bytes of f + 0x808080, each minus 128): the A operand.
//   The MFMA's integer sums are exact, so each sub-block's sum(w x) is exact
//   up to the rounding of x to 2^-20 of its 32-element block's maximum
//   (exact for every element within 2^9 of that maximum).  A block holding
//   an inf or NaN gets a NaN scale, so the rows that read it come back NaN.
// * Layout.  A wavefront owns 16 rows (the MFMA's N) and 1024 of the
//   reduction axis; a workgroup owns 32 rows and all of it (N/1024
//   wavefronts per 16 rows), so a wavefront's compute after its last byte
//   arrives stays short.  Lane (n, g) = (l%16, l/16).  In MFMA number m
//   lane group g holds the 16 weights at k = base(g) + imm(m) of row n:
//     2-bit members: base = 64g, imm = 256s + 16j (m = 4s + j), so the four
//       lanes of row n read 64 contiguous code bytes per super-block s;
//     IQ1_S_R4:      base = 128g, imm = 512i + 16t (m = 8i + t), so they
//       read 64 contiguous index bytes per i.
//   A-rows 4g..4g+2 carry the byte planes of lane group g's 16 activations
//   and zero elsewhere, so D rows 4g..4g+2 -- which the MFMA places in lane
//   group g -- collect exactly that lane's weights, one byte plane each:
//   sum(w x) = 2^-E (D0 + 2^8 D1 + 2^16 D2).  Each lane folds its own
//   (row, sub-block) sums with the sub-block's scale.  Every lane reads its
//   A operands from LDS, the 52 lanes whose A rows carry no activations from
//   a zero span (reading only in the 12 data lanes, behind a branch, with
//   zeros held in registers, measured 0.3-2% slower at 1 token).  The
//   partial sums of a row's lanes and wavefronts meet in LDS.
// * Two row blocks.  Large IQ1_S_R4 dispatches, and the IQ2 members' large
//   2048-wide ones, give each wavefront 32 rows (two 16-row blocks, R = 2)
//   that share every A read, so a workgroup stages its activations once for
//   64 rows; the per-row arithmetic is the same as with one block, so
//   results are identical bit for bit.
// * Several pairs a workgroup.  Other large dispatches in pairs mode serve
//   three (or two) consecutive pairs of one activation row in one workgroup
//   (gemv_mfma_pairs_kernel): the activations are staged once for the
//   pairs' experts, again with each row's arithmetic unchanged.
//
// The floor variants keep every global load and delete the decode.

#include <type_traits>

#include "iqk_device.h"
#include "iqk_host.h"

#define IQK_GRID_STORAGE __constant__ static const __attribute__((aligned(16)))
#include "../iq1s_grid.h"

namespace iqk {

typedef int int4_t __attribute__((ext_vector_type(4)));
typedef unsigned short ushort2_t __attribute__((ext_vector_type(2)));

struct Gemv2Args {
    const uint32_t *x;
    const void *s0, *s1, *s2, *s3, *s4;
    const uint32_t *sel;
    const uint32_t *toks;  // sorted/union modes: activation row of each pair
    uint32_t pairs_per_row;
    uint32_t mats;
    uint32_t n_x_rows;
    uint32_t num_experts;
    uint32_t out_features;
    uint16_t *y;
};

constexpr uint32_t kV8Base = 0x1101F3E1u;   // int8 -31, -13, 1, 17
constexpr uint32_t kV8Shift = 0x1606F8E6u;  // int8 -26, -8, 6, 22
constexpr uint32_t kG8Plus = 0x000901F9u;   // int8 8(g + 1/8), g = -1, 0, 1
constexpr int kWaveK = 1024;                // reduction elements per wavefront (default)
constexpr int kGroupRows = 32;              // rows per workgroup

// Byte planes sit 16 bytes more than N apart, so one lane group's three
// plane reads fall in different LDS banks.
template <int N>
constexpr int kPlaneStride = N + 16;

// Work split of one workgroup: 32 rows, KS wavefronts of WK reduction
// elements per 16 rows.  IQ1_S_R4's 2048-wide down projection uses 512-wide
// slices, so its workgroups are eight wavefronts like the others and a CU
// holds three copies of the LDS grid instead of six.
template <int MEMBER, int N>
struct Gemv2Shape {
    static constexpr int WK = MEMBER == IQ1_S_R4 && N == 2048 ? 512 : kWaveK;
    static constexpr int KS = N / WK;      // wavefronts per 16 rows
    static constexpr int THREADS = 64 * 2 * KS;
    static constexpr int UNITS = N / 8;    // activation staging units of 8 elements
    static_assert(THREADS >= UNITS && UNITS % 64 == 0, "whole wavefronts stage the activations");
};

// The 16 int8 weights of 16 packed 2-bit codes (code j at bit 2j); operand
// dword s holds codes s, 4+s, 8+s, 12+s (byte t = code 4t+s).
__device__ __forceinline__ int4_t codes_to_i8(uint32_t q, uint32_t pool) {
    int4_t b;
    b.x = int(perm(pool, pool, q & 0x03030303u));
    b.y = int(perm(pool, pool, (q >> 2) & 0x03030303u));
    b.z = int(perm(pool, pool, (q >> 4) & 0x03030303u));
    b.w = int(perm(pool, pool, (q >> 6) & 0x03030303u));
    return b;
}

// Plane k, operand dword: bytes k of u[0..3], each minus 128.
__device__ __forceinline__ void byte_planes(const uint32_t *u, uint32_t &p0, uint32_t &p1, uint32_t &p2) {
    const uint32_t a01 = perm(u[1], u[0], 0x05010400u), a23 = perm(u[3], u[2], 0x05010400u);
    p0 = perm(a23, a01, 0x05040100u) ^ 0x80808080u;
    p1 = perm(a23, a01, 0x07060302u) ^ 0x80808080u;
    p2 = (perm(u[1], u[0], 0x0c0c0602u) | perm(u[3], u[2], 0x06020c0cu)) ^ 0x80808080u;
}

// Byte view of a stream; offsets are 32-bit (the dispatcher checks every
// stream and the activations fit 4 GiB), so loads take a uniform base and a
// 32-bit lane offset.
__device__ __forceinline__ const uint8_t *bytes(const void *p) { return static_cast<const uint8_t *>(p); }

// The value of lane (l ^ X) within l's quad (X = 1, 2), by a DPP quad permute.
template <int X>
__device__ __forceinline__ uint32_t quad_xor(uint32_t v) {
    constexpr int ctrl = X == 1 ? 0xB1 : 0x4E;  // quad_perm [1,0,3,2] / [2,3,0,1]
    return uint32_t(__builtin_amdgcn_mov_dpp(int(v), ctrl, 0xF, 0xF, false));
}

// The value of lane 7 - (l % 8) of l's half-row of 8 lanes (DPP row_half_mirror).
__device__ __forceinline__ uint32_t half_row_mirror(uint32_t v) {
    return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x141, 0xF, 0xF, false));
}

__device__ __forceinline__ int digits_sum(int4_t d) { return (((d.z << 8) + d.y) << 8) + d.x; }

// The three plane sums of an IQ2_K super-block as a float: d.x + 2^8 d.y is
// exact in int32 (|d.x|, |d.y| < 2^20), so converting it rounds that value
// once, as fma(float(d.y), 256, float(d.x)) does; the 2^16 plane is added by
// an fma (the whole sum can pass 2^31).
__device__ __forceinline__ float planes_sum(int4_t d) {
    return fmaf(float(d.z), 65536.f, float(d.x + (d.y << 8)));
}

// 8 x the low / high 16 bits of v.  Plain code, not inline asm: the
// compiler must see every instruction that writes a register, because a
// register whose last writer was an MFMA still in flight (an unused dword of
// its result) may be handed to the next value, and only the compiler's
// hazard pass inserts the wait that keeps the MFMA's late write from landing
// on top of it.
__device__ __forceinline__ uint32_t lo16_x8(uint32_t v) { return (v & 0xffffu) << 3; }
__device__ __forceinline__ uint32_t hi16_x8(uint32_t v) { return (v >> 16) << 3; }

// Keeps a value computed where it stands: without a use in its own
// super-block each fold could be sunk behind the last stream word, into every
// wavefront's tail.
__device__ __forceinline__ void pin(float &v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(uint32_t &v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(int &v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(uint2_t &v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(uint4_t &v) { asm volatile("" : "+v"(v)); }

// Two IQ1_S_R4 grid entries (the low and high 16 bits of e; 2-bit code c
// at bit 2k for weight k, g = c - 1) as int8 weights 8g + 1, eight bytes an
// entry in the paired order 0,4,1,5,2,6,3,7: word j of the code pattern
// gathers weights j and 4+j of both entries, one v_perm each from the pool,
// and two v_perm per 4 bytes regroup them by entry.
__device__ __forceinline__ void expand_grid_pair(uint32_t e, uint4_t &out) {
    uint32_t d[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) d[j] = perm(kG8Plus, kG8Plus, (e >> (2 * j)) & 0x03030303u);
    out = uint4_t{perm(d[1], d[0], 0x05040100u), perm(d[3], d[2], 0x05040100u),   // first entry
                  perm(d[1], d[0], 0x07060302u), perm(d[3], d[2], 0x07060302u)};  // second entry
}

__device__ __forceinline__ int4_t mfma(int4_t a, int4_t b, int4_t c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// The A operands of K MFMAs, 16 bytes each from p (lanes without
// activations point into a zero span).
template <int K>
__device__ __forceinline__ void read_a(int4_t (&a)[K], const uint8_t *p) {
#pragma unroll
    for (int j = 0; j < K; ++j) a[j] = __builtin_bit_cast(int4_t, *reinterpret_cast<const uint4_t *>(p + 16 * j));
}

// One A operand read by every lane (non-data lanes point into a zero span).
__device__ __forceinline__ int4_t read_a_all(const uint8_t *p) {
    return __builtin_bit_cast(int4_t, *reinterpret_cast<const uint4_t *>(p));
}

// Bytes of zeros after the byte planes: a wavefront's reduction span, what a
// lane without activations reads.
template <int MEMBER, int N>
constexpr int kZeroSpan = Gemv2Shape<MEMBER, N>::WK;

// Shared memory of one workgroup: the activations' three byte planes and a
// zero span, 2^-E per 32-element block, the
// wavefronts' partial row sums (32 R rows of each of its P pairs), and for
// IQ1_S_R4 the expanded grid and each block's integer 2 sum(f).
template <int MEMBER, int N, int R, int P>
struct Gemv2Smem {
    static constexpr bool IQ1 = MEMBER == IQ1_S_R4;
    uint8_t dig[3 * kPlaneStride<N> + kZeroSpan<MEMBER, N>] __attribute__((aligned(16)));
    float sbs[N / 32] __attribute__((aligned(16)));
    float nsbs[MEMBER == IQ2_KS ? N / 32 : 4] __attribute__((aligned(16)));  // -16 x 2^-E (IQ2_KS)
    float part[P][Gemv2Shape<MEMBER, N>::KS][4][kGroupRows * R];
    int fsum[IQ1 ? N / 32 : 4] __attribute__((aligned(16)));
    uint2_t b8[IQ1 ? IQK_IQ1S_GRID_SIZE : 1];
    uint2_t ktab[MEMBER == IQ2_K ? 32 : 1];
    float fw[MEMBER == IQ2_K ? N / 16 : 4] __attribute__((aligned(16)));
};

// Activation exponent block: 64 elements for IQ2_K (a lane group's span of
// a super-block, so its four words share one exponent), 32 otherwise.
template <int MEMBER>
constexpr int kExpBlock = MEMBER == IQ2_K ? 64 : 32;

// Activations (fp16) -> balanced byte planes of 16-element words, in the
// byte order the member's B operand uses.  Thread tid = 2wd + hp holds xv,
// fp16 pairs 4hp..4hp+3 of word wd (its own 16 bytes: each byte of x is
// loaded once), and converts 8 activations, operand dwords 2hp and 2hp+1:
//   TRANSPOSED (2-bit members): dword s byte t is element 4t+s, so the
//     thread takes elements 4t+2hp (low halves) and 4t+2hp+1 (high halves)
//     of the fp16 pairs 2t+hp, two of them from the word's other thread;
//   paired (IQ1_S_R4): the 8-element group hp holds its elements in the
//     order 0,4,1,5,2,6,3,7 of the grid expansion, so the thread takes
//     elements 8hp..8hp+7, the pairs 4hp..4hp+3 it holds.
// One exponent E covers BLOCK (32 or 64) consecutive elements, 2^-E lands in
// sbs[element / BLOCK] (and -16 x 2^-E in nsbs, when given).  With `fsum`,
// each 32-element block's 2 sum(f) lands there too, with `fword` each
// 16-element word's sum(f); the ZERO_BYTES after the planes are cleared.
template <int N, bool TRANSPOSED, int ZERO_BYTES, int BLOCK>
__device__ __forceinline__ void stage_activations(uint8_t *dig, float *sbs, float *nsbs, int *fsum, float *fword, int tid,
                                                  uint4_t xv) {
    static_assert(BLOCK == 32 || BLOCK == 64, "4 or 8 threads per exponent block");
    const uint32_t wd = uint32_t(tid) >> 1, hp = uint32_t(tid) & 1u;
    if (tid < ZERO_BYTES / 16)
        *reinterpret_cast<uint4_t *>(dig + 3 * kPlaneStride<N> + 16 * tid) = uint4_t{0u, 0u, 0u, 0u};
    uint32_t xp[4] = {xv.x, xv.y, xv.z, xv.w};
    if constexpr (TRANSPOSED) {  // hp 0 keeps pairs 0, 2 and takes 4, 6; hp 1 keeps 5, 7 and takes 1, 3
        const uint32_t r0 = quad_xor<1>(hp ? xv.x : xv.y), r1 = quad_xor<1>(hp ? xv.z : xv.w);
        xp[0] = hp ? r0 : xv.x;
        xp[1] = hp ? r1 : xv.z;
        xp[2] = hp ? xv.y : r0;
        xp[3] = hp ? xv.w : r1;
    }
    // max |x| on the fp16 bits (magnitude order is integer order)
    ushort2_t m2 = __builtin_bit_cast(ushort2_t, xp[0] & 0x7fff7fffu);
#pragma unroll
    for (int t = 1; t < 4; ++t) m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(ushort2_t, xp[t] & 0x7fff7fffu));
    uint32_t mx = max(uint32_t(m2.x), uint32_t(m2.y));
    mx = max(mx, quad_xor<1>(mx));  // the 4 threads of a 32-element block
    mx = max(mx, quad_xor<2>(mx));
    if constexpr (BLOCK == 64) mx = max(mx, half_row_mirror(mx));  // the 8 of a 64-element block
    const bool finite = mx < 0x7c00u;
    // E so that max|x| * 2^E lies in [2^19, 2^20)
    const float amax = finite ? half_bits_to_float(mx) : 0.f;
    const int ex = amax > 0.f ? int((__float_as_uint(amax) >> 23) & 0xffu) - 127 : 0;
    const int E = 19 - ex;
    const float up = finite ? __uint_as_float(uint32_t(E + 127) << 23) : 0.f;
    // x * 2^E + 1.5 * 2^23 rounds x * 2^E to an integer f: the sum stays in
    // [2^23, 2^24), where the ulp is 1, and its bits are 0x4B400000 + f.
    // Re-biased, the bits' bytes 0-2 are the bytes of f + 0x808080.
    constexpr uint32_t kMagicBits = 0x4B400000u;
    constexpr uint32_t kRebias = 0x808080u - kMagicBits;  // mod 2^32
    const float magic = __uint_as_float(kMagicBits);
    uint32_t blo[4], bhi[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        blo[t] = __float_as_uint(fmaf(half_bits_to_float(xp[t] & 0xffffu), up, magic)) + kRebias;
        bhi[t] = __float_as_uint(fmaf(half_bits_to_float(xp[t] >> 16), up, magic)) + kRebias;
    }
    // operand dwords 2hp (u0) and 2hp+1 (u1)
    uint32_t u0[4], u1[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        if constexpr (TRANSPOSED) {
            u0[t] = blo[t];
            u1[t] = bhi[t];
        } else {  // elements 2t, 2t+1 at positions 2(2t % 4) + 2t / 4 and that + 2
            const int pos = 4 * (t & 1) + (t >> 1);
            (pos < 4 ? u0 : u1)[pos & 3] = blo[t];
            (pos < 4 ? u0 : u1)[(pos & 3) + 2] = bhi[t];
        }
    }
    if (fsum || fword) {  // sums of f (mod 2^32, exact: |sum| < 2^26)
        uint32_t f = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) f += blo[t] + bhi[t];
        f -= 8u * 0x808080u;
        f += quad_xor<1>(f);  // the 16-element word
        if (fword && (tid & 1) == 0) fword[tid >> 1] = float(int(f));
        f += quad_xor<2>(f);  // the 32-element block
        if (fsum && (tid & 3) == 0) fsum[tid >> 2] = 2 * int(f);
    }
    uint32_t l0, l1, l2, h0, h1, h2;
    byte_planes(u0, l0, l1, l2);
    byte_planes(u1, h0, h1, h2);
    const uint32_t off = 16 * wd + 8 * hp;
    *reinterpret_cast<uint2_t *>(dig + 0 * kPlaneStride<N> + off) = uint2_t{l0, h0};
    *reinterpret_cast<uint2_t *>(dig + 1 * kPlaneStride<N> + off) = uint2_t{l1, h1};
    *reinterpret_cast<uint2_t *>(dig + 2 * kPlaneStride<N> + off) = uint2_t{l2, h2};
    if ((tid & (BLOCK / 8 - 1)) == 0) {
        sbs[tid / (BLOCK / 8)] = finite ? __uint_as_float(uint32_t(127 - E) << 23) : __builtin_nanf("");
        if (nsbs) nsbs[tid / (BLOCK / 8)] = finite ? __uint_as_float(0x80000000u | (uint32_t(131 - E) << 23))
                                                   : __builtin_nanf("");
    }
}

// -- per-member lane state: loads, floor hash, and the decode ---------------------

// IQ2_KS streams: qs u32 [N/16], scl u8 [N/64], sch u8 [N/256], sex u8 [N/256], dv f16.
template <int N>
struct LaneIq2ks {
    uint4_t sc, q[4];
    uint32_t hb, ab, dvb;

    __device__ __forceinline__ void load(const Gemv2Args &a, uint32_t row, uint32_t kq, uint32_t g) {
        sc = load_u4(bytes(a.s1) + (row * (N / 64) + 16 * kq));
        hb = *reinterpret_cast<const uint32_t *>(bytes(a.s2) + (row * (N / 256) + 4 * kq));
        ab = *reinterpret_cast<const uint32_t *>(bytes(a.s3) + (row * (N / 256) + 4 * kq));
        dvb = *reinterpret_cast<const uint16_t *>(bytes(a.s4) + 2 * row);
#pragma unroll
        for (uint32_t s = 0; s < 4; ++s) q[s] = load_u4(bytes(a.s0) + (row * (N / 4) + 256 * kq + 64 * s + 16 * g));
    }

    __device__ __forceinline__ uint32_t hash() const {
        uint32_t h = 59u * (sc.x + sc.y + sc.z + sc.w) + 61u * hb + 71u * ab + 67u * dvb;
#pragma unroll
        for (int s = 0; s < 4; ++s) h += q[s].x + 3u * q[s].y + 5u * q[s].z + 7u * q[s].w;
        return h;
    }

    // Sub-blocks 8s+2g+h (32 weights, words 2h, 2h+1 of q[s]) of R rows, one
    // lane instance each, which share every A read; sbs / nsbs: 2^-E and
    // -16 x 2^-E of each 32-element block.
    template <int R, bool EARLY>
    __device__ __forceinline__ static void decode(const LaneIq2ks (&ln)[R], const uint8_t *abase, const float *sbs,
                                                  const float *nsbs, int g, float (&out)[R]) {
        // Scale index x 2^-E and alphabet pool of sub-blocks 8s+2g+h, formed
        // from the scale bytes alone (left to the scheduler: pinning them
        // here measured slower), so the code words meet only their expansion,
        // the MFMAs and the folds.  The 5-bit indices of super-blocks 2p and
        // 2p+1 are packed one a byte, byte 2h + (s - 2p): a v_perm takes
        // byte g of both scale words as (s0, s1, s0, s1), masks keep the
        // nibble h of each, two masked shifts add the high bits; then each
        // factor is (idx - 16) 2^-E = fma(float(byte), 2^-E, -16 x 2^-E),
        // exact as before.  The pool is a bit-select on the alphabet bit.
        const uint32_t g2 = uint32_t(g) | (uint32_t(g) << 8);
        const uint32_t selg = (g2 | (g2 << 16)) + 0x04000400u;  // bytes g, 4+g, g, 4+g
        float fac[R][4][2];
        uint32_t pool[R][4][2], idx4[R];
        // Super-block s's factors and pools: all before the first code word
        // (EARLY), or each just before its MFMAs (the registers of all four
        // would cost a wavefront per SIMD).
        const auto prep = [&](int s) {
            const int sp = s >> 1, t = s & 1;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t hbg = ln[r].hb >> (2 * g), abg = ln[r].ab >> (2 * g);
                if (t == 0) {
                    const uint32_t pb = perm(ln[r].sc[2 * sp + 1], ln[r].sc[2 * sp], selg);
                    const uint32_t u = hbg >> (16 * sp);  // high bits: super-block 2sp at bits h, 2sp+1 at 8+h
                    idx4[r] = (pb & 0x00000F0Fu) | ((pb >> 4) & 0x0F0F0000u) | ((u & 0x101u) << 4) |
                              ((u & 0x202u) << 19);
                }
                const float2 up = *reinterpret_cast<const float2 *>(sbs + 8 * s + 2 * g);
                const float2 nup = *reinterpret_cast<const float2 *>(nsbs + 8 * s + 2 * g);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float idx5 = float((idx4[r] >> (8 * (2 * h + t))) & 0xffu);
                    fac[r][s][h] = fmaf(idx5, h ? up.y : up.x, h ? nup.y : nup.x);
                    const uint32_t m = uint32_t(int32_t(abg << (31 - (8 * s + h))) >> 31);
                    pool[r][s][h] = (m & kV8Shift) | (~m & kV8Base);
                }
            }
        };
        if constexpr (EARLY) {
#pragma unroll
            for (int s = 0; s < 4; ++s) prep(s);
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.f;
        int4_t Dp[R][2], A[4] = {};
#pragma unroll
        for (int s = 0; s <= 4; ++s) {
            int4_t D[R][2];
            if (s < 4) {
                if constexpr (!EARLY) prep(s);
                read_a(A, abase + 256 * s);
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        D[r][h] = mfma(A[2 * h], codes_to_i8(ln[r].q[s][2 * h], pool[r][s][h]), int4_t{0, 0, 0, 0});
                        D[r][h] = mfma(A[2 * h + 1], codes_to_i8(ln[r].q[s][2 * h + 1], pool[r][s][h]), D[r][h]);
                    }
            }
            if (s > 0) {  // fold the previous super-block while this one's MFMAs run
                const int sp = s - 1;
#pragma unroll
                for (int r = 0; r < R; ++r) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) acc[r] = fmaf(float(digits_sum(Dp[r][h])), fac[r][sp][h], acc[r]);
                    pin(acc[r]);
                }
            }
            if (s < 4) {
#pragma unroll
                for (int r = 0; r < R; ++r) { Dp[r][0] = D[r][0]; Dp[r][1] = D[r][1]; }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) out[r] = acc[r] * half_bits_to_float(ln[r].dvb);
    }

    // Pairs 0 .. np-1 (np <= PM, uniform per workgroup) of this lane's expert
    // rows, each with its own activations (abase[p], sbs[p], nsbs[p] as for
    // decode): each super-block's factors, pools and B operands are formed once
    // and serve every pair, and each pair's MFMAs and folds are decode<1,
    // true>'s in its order, so each pair's result is decode's bit for bit.
    template <int PM>
    __device__ __forceinline__ void decode_pairs(const uint8_t *const (&abase)[PM], const float *const (&sbs)[PM],
                                                 const float *const (&nsbs)[PM], int np, int g,
                                                 float (&out)[PM]) const {
        const uint32_t g2 = uint32_t(g) | (uint32_t(g) << 8);
        const uint32_t selg = (g2 | (g2 << 16)) + 0x04000400u;
        const uint32_t hbg = hb >> (2 * g), abg = ab >> (2 * g);
        float acc[PM];
#pragma unroll
        for (int p = 0; p < PM; ++p) acc[p] = 0.f;
        uint32_t idx4 = 0;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int sp = s >> 1, t = s & 1;
            if (t == 0) {
                const uint32_t pb = perm(sc[2 * sp + 1], sc[2 * sp], selg);
                const uint32_t u = hbg >> (16 * sp);
                idx4 = (pb & 0x00000F0Fu) | ((pb >> 4) & 0x0F0F0000u) | ((u & 0x101u) << 4) | ((u & 0x202u) << 19);
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {  // sub-block 8s + 2g + h: words 2h, 2h+1 of q[s]
                const float idx5 = float((idx4 >> (8 * (2 * h + t))) & 0xffu);
                const uint32_t m = uint32_t(int32_t(abg << (31 - (8 * s + h))) >> 31);
                const uint32_t pool = (m & kV8Shift) | (~m & kV8Base);
                const int4_t B0 = codes_to_i8(q[s][2 * h], pool), B1 = codes_to_i8(q[s][2 * h + 1], pool);
#pragma unroll
                for (int p = 0; p < PM; ++p) {
                    if (p < np) {
                        const float fac = fmaf(idx5, sbs[p][8 * s + 2 * g + h], nsbs[p][8 * s + 2 * g + h]);
                        const uint8_t *ap = abase[p] + 256 * s + 32 * h;
                        int4_t D = mfma(read_a_all(ap), B0, int4_t{0, 0, 0, 0});
                        D = mfma(read_a_all(ap + 16), B1, D);
                        acc[p] = fmaf(float(digits_sum(D)), fac, acc[p]);
                    }
                }
            }
        }
#pragma unroll
        for (int p = 0; p < PM; ++p) out[p] = acc[p] * half_bits_to_float(dvb);
    }
};

// IQ2_K streams: qs u32 [N/16], scl u16 [N/64], sex u8 [N/128], dv f16 [N/256].
template <int N>
struct LaneIq2k {
    uint4_t sc0, sc1, q[4];
    uint2_t ex, dv;

    __device__ __forceinline__ void load(const Gemv2Args &a, uint32_t row, uint32_t kq, uint32_t g) {
        sc0 = load_u4(bytes(a.s1) + (row * (N / 32) + 32 * kq));
        sc1 = load_u4(bytes(a.s1) + (row * (N / 32) + 32 * kq + 16));
        ex = *reinterpret_cast<const uint2_t *>(bytes(a.s2) + (row * (N / 128) + 8 * kq));
        dv = *reinterpret_cast<const uint2_t *>(bytes(a.s3) + (row * (N / 128) + 8 * kq));
#pragma unroll
        for (uint32_t s = 0; s < 4; ++s) q[s] = load_u4(bytes(a.s0) + (row * (N / 4) + 256 * kq + 64 * s + 16 * g));
    }

    __device__ __forceinline__ uint32_t hash() const {
        uint32_t h = 59u * (sc0.x + sc0.y + sc0.z + sc0.w + sc1.x + sc1.y + sc1.z + sc1.w) +
                     71u * (ex.x + ex.y) + 67u * (dv.x + dv.y);
#pragma unroll
        for (int s = 0; s < 4; ++s) h += q[s].x + 3u * q[s].y + 5u * q[s].z + 7u * q[s].w;
        return h;
    }

    // sub-blocks 16s+4g+j (16 weights, word j of q[s]); d per super-block s.
    // The scale index goes into the weights: with v = 2u + off,
    // u in (-12, -3, 4, 12) and off = -7 (base alphabet) or -2 (shifted),
    // idx * v = 2 (idx u) + idx off, and idx u fits int8, so the MFMA's B is a
    // per-word pool idx * u and its D accumulates over the lane's four words
    // of a super-block, which share one activation exponent.  The constant
    // part idx * off * sum(f) takes one fma per word from the word's integer
    // activation sum fw.  A lane folds once per super-block.
    // R rows, one lane instance each, share every A read.
    template <int R, bool EARLY>
    __device__ __forceinline__ static void decode(const LaneIq2k (&ln)[R], const uint8_t *abase, const float *sbs,
                                                  const float *fw, const uint2_t *ktab, int g, float (&out)[R]) {
        // This lane's scale word of super-block s is u16 g of the pair
        // (sc.y:sc.x) or (sc.w:sc.z); one v_perm spreads its two bytes to
        // (b0, b0, b1, b1), and shifts put nibble j at bits 3-6 of byte j.
        const uint32_t selg = 0x01010000u + uint32_t(2 * g) * 0x01010101u;
        // alphabet bits of super-block s: byte 2s + g/2 of ex, bits 4(g%2) + j
        const int exs = 8 * (g >> 1) + 4 * (g & 1);
        // Before any code word is needed: each super-block's d x 2^-E, its
        // constant part sum_j (idx off)_j fw_j, and its four word pools.
        float dfac[R][4], offs[R][4];
        uint32_t pools[R][4][4], scp[R][4], exg[R][2];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            scp[r][0] = perm(ln[r].sc0.y, ln[r].sc0.x, selg);
            scp[r][1] = perm(ln[r].sc0.w, ln[r].sc0.z, selg);
            scp[r][2] = perm(ln[r].sc1.y, ln[r].sc1.x, selg);
            scp[r][3] = perm(ln[r].sc1.w, ln[r].sc1.z, selg);
            exg[r][0] = ln[r].ex.x >> exs;
            exg[r][1] = ln[r].ex.y >> exs;
        }
        // Super-block s's factors and pools: all before the first code word
        // (EARLY), or each just before its MFMAs (the registers of all four
        // would cost a wavefront per SIMD).
        const auto prep = [&](int s) {
            const float4 fwv = *reinterpret_cast<const float4 *>(fw + 16 * s + 4 * g);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                dfac[r][s] = half_bits_to_float((ln[r].dv[s >> 1] >> (16 * (s & 1))) & 0xffffu) * sbs[4 * s + g];
                offs[r][s] = 0.f;
                // byte j: the table's byte offset 8 (alpha_j << 4 | nib_j) of
                // word j; the multiply copies alphabet bit j to bit 8j (no two
                // copies meet, so no carries; pinned, or it becomes a
                // quarter-rate 32-bit multiply by the shifted constant)
                uint32_t a8 = __umul24((exg[r][s >> 1] >> (16 * (s & 1))) & 15u, 0x204081u);
                pin(a8);
                const uint32_t kofs = ((scp[r][s] << 3) & 0x00780078u) | ((scp[r][s] >> 1) & 0x78007800u) |
                                      ((a8 & 0x01010101u) << 7);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint2_t e = *reinterpret_cast<const uint2_t *>(reinterpret_cast<const uint8_t *>(ktab) +
                                                                         ((kofs >> (8 * j)) & 0xffu));
                    pools[r][s][j] = e.x;
                    offs[r][s] = fmaf(__uint_as_float(e.y), fwv[j], offs[r][s]);
                }
            }
        };
        if constexpr (EARLY) {
#pragma unroll
            for (int s = 0; s < 4; ++s) prep(s);
        }
        float acc[R];
        int4_t Wp[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
        for (int s = 0; s <= 4; ++s) {
            int4_t W[R];
#pragma unroll
            for (int r = 0; r < R; ++r) W[r] = int4_t{0, 0, 0, 0};
            if (s < 4) {
                if constexpr (!EARLY) prep(s);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int4_t a = read_a_all(abase + 256 * s + 16 * j);
#pragma unroll
                    for (int r = 0; r < R; ++r) W[r] = mfma(a, codes_to_i8(ln[r].q[s][j], pools[r][s][j]), W[r]);
                }
            }
            if (s > 0) {  // fold the previous super-block while this one's MFMAs run
                const int sp = s - 1;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float sum = planes_sum(Wp[r]);
                    acc[r] = fmaf(fmaf(2.f, sum, offs[r][sp]), dfac[r][sp], acc[r]);
                    pin(acc[r]);
                }
            }
            if (s < 4) {
#pragma unroll
                for (int r = 0; r < R; ++r) Wp[r] = W[r];
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) out[r] = acc[r];
    }

    // One row block, streamed: each super-block's factors and pools formed
    // just before its MFMAs and folded right after them -- decode<1, true>'s
    // operations in its order, so bit-identical, with fewer values live at
    // once (64 VGPRs against 74: eight wavefronts a SIMD).  The sorted
    // dispatch uses it: 1-2.5% faster there (IQ2_K [2048 x 4096], 256
    // experts, 8 and 32 tokens); in the pair dispatches it measured the same.
    __device__ __forceinline__ float decode_streamed(const uint8_t *abase, const float *sbs, const float *fw,
                                                     const uint2_t *ktab, int g) const {
        const uint32_t selg = 0x01010000u + uint32_t(2 * g) * 0x01010101u;
        const int exs = 8 * (g >> 1) + 4 * (g & 1);
        const uint32_t scp[4] = {perm(sc0.y, sc0.x, selg), perm(sc0.w, sc0.z, selg), perm(sc1.y, sc1.x, selg),
                                 perm(sc1.w, sc1.z, selg)};
        const uint32_t exg[2] = {ex.x >> exs, ex.y >> exs};
        float acc = 0.f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float dfac = half_bits_to_float((dv[s >> 1] >> (16 * (s & 1))) & 0xffffu) * sbs[4 * s + g];
            uint32_t a8 = __umul24((exg[s >> 1] >> (16 * (s & 1))) & 15u, 0x204081u);
            pin(a8);
            const uint32_t kofs =
                ((scp[s] << 3) & 0x00780078u) | ((scp[s] >> 1) & 0x78007800u) | ((a8 & 0x01010101u) << 7);
            const float4 fwv = *reinterpret_cast<const float4 *>(fw + 16 * s + 4 * g);
            int4_t B[4];
            float offs = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint2_t e = *reinterpret_cast<const uint2_t *>(reinterpret_cast<const uint8_t *>(ktab) +
                                                                     ((kofs >> (8 * j)) & 0xffu));
                B[j] = codes_to_i8(q[s][j], e.x);
                offs = fmaf(__uint_as_float(e.y), fwv[j], offs);
            }
            int4_t W = int4_t{0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 4; ++j) W = mfma(read_a_all(abase + 256 * s + 16 * j), B[j], W);
            const float sum = planes_sum(W);
            acc = fmaf(fmaf(2.f, sum, offs), dfac, acc);
        }
        return acc;
    }

    // Pairs 0 .. np-1 (np <= PM, uniform per workgroup) of this lane's expert
    // rows, each with its own activations (abase[p], sbs[p], fw[p] as for
    // decode): each super-block's pools and B operands are formed once and
    // serve every pair, and each pair's factors, MFMAs and fold are
    // decode<1, true>'s in its order, so each pair's result is decode's bit
    // for bit.
    template <int PM>
    __device__ __forceinline__ void decode_pairs(const uint8_t *const (&abase)[PM], const float *const (&sbs)[PM],
                                                 const float *const (&fw)[PM], const uint2_t *ktab, int np, int g,
                                                 float (&out)[PM]) const {
        const uint32_t selg = 0x01010000u + uint32_t(2 * g) * 0x01010101u;
        const int exs = 8 * (g >> 1) + 4 * (g & 1);
        const uint32_t scp[4] = {perm(sc0.y, sc0.x, selg), perm(sc0.w, sc0.z, selg), perm(sc1.y, sc1.x, selg),
                                 perm(sc1.w, sc1.z, selg)};
        const uint32_t exg[2] = {ex.x >> exs, ex.y >> exs};
        float acc[PM];
#pragma unroll
        for (int p = 0; p < PM; ++p) acc[p] = 0.f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float dvs = half_bits_to_float((dv[s >> 1] >> (16 * (s & 1))) & 0xffffu);
            const uint32_t a8 = __umul24((exg[s >> 1] >> (16 * (s & 1))) & 15u, 0x204081u);
            const uint32_t kofs =
                ((scp[s] << 3) & 0x00780078u) | ((scp[s] >> 1) & 0x78007800u) | ((a8 & 0x01010101u) << 7);
            int4_t B[4];
            float ey[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint2_t e = *reinterpret_cast<const uint2_t *>(reinterpret_cast<const uint8_t *>(ktab) +
                                                                     ((kofs >> (8 * j)) & 0xffu));
                B[j] = codes_to_i8(q[s][j], e.x);
                ey[j] = __uint_as_float(e.y);
            }
#pragma unroll
            for (int p = 0; p < PM; ++p) {
                if (p < np) {
                    const float4 fwv = *reinterpret_cast<const float4 *>(fw[p] + 16 * s + 4 * g);
                    const float dfac = dvs * sbs[p][4 * s + g];
                    float offs = 0.f;
#pragma unroll
                    for (int j = 0; j < 4; ++j) offs = fmaf(ey[j], fwv[j], offs);
                    int4_t W = int4_t{0, 0, 0, 0};
#pragma unroll
                    for (int j = 0; j < 4; ++j) W = mfma(read_a_all(abase[p] + 256 * s + 16 * j), B[j], W);
                    const float sum = planes_sum(W);
                    acc[p] = fmaf(fmaf(2.f, sum, offs), dfac, acc[p]);
                }
            }
        }
#pragma unroll
        for (int p = 0; p < PM; ++p) out[p] = acc[p];
    }
};

// IQ2_K's per-word factors, by (alphabet << 4 | scale nibble): the int8 pool
// idx * u_c (u = -12, -3, 4, 12) and the float idx * off, with idx =
// nibble - 8 and off = -7 (base alphabet) or -2 (shifted).
struct Iq2kTable {
    uint32_t w[2 * 32];
};

constexpr Iq2kTable make_iq2k_table() {
    Iq2kTable t{};
    constexpr int u[4] = {-12, -3, 4, 12};
    for (int alpha = 0; alpha < 2; ++alpha)
        for (int nib = 0; nib < 16; ++nib) {
            const int idx = nib - 8, off = alpha ? -2 : -7, e = alpha * 16 + nib;
            for (int c = 0; c < 4; ++c) t.w[2 * e] |= uint32_t(uint8_t(int8_t(idx * u[c]))) << (8 * c);
            t.w[2 * e + 1] = __builtin_bit_cast(uint32_t, float(idx * off));
        }
    return t;
}

__constant__ const Iq2kTable kIq2kTab = make_iq2k_table();

// IQ1_S_R4 streams: qs u32 [N/32] (4 index bytes per 32-weight block),
// qh u16 [N/32], dv f16.
template <int N, int WK>
struct LaneIq1s {
    static constexpr int NI = WK / 512;  // 512-weight spans per wavefront
    uint4_t qv[NI];
    uint2_t qh[NI];
    uint32_t dvb;

    __device__ __forceinline__ void load(const Gemv2Args &a, uint32_t row, uint32_t kq, uint32_t g) {
        const uint32_t qo = row * (N / 8) + (WK / 8) * kq + 16 * g, ho = row * (N / 16) + (WK / 16) * kq + 8 * g;
#pragma unroll
        for (int i = 0; i < NI; ++i) qh[i] = *reinterpret_cast<const uint2_t *>(bytes(a.s1) + (ho + 32 * i));
        dvb = *reinterpret_cast<const uint16_t *>(bytes(a.s2) + 2 * row);
#pragma unroll
        for (int i = 0; i < NI; ++i) qv[i] = load_u4(bytes(a.s0) + (qo + 64 * i));
    }

    __device__ __forceinline__ uint32_t hash() const {
        uint32_t h = 67u * dvb;
#pragma unroll
        for (int i = 0; i < NI; ++i)
            h += (2 * i + 3) * (qv[i].x + 3u * qv[i].y + 5u * qv[i].z + 7u * qv[i].w) + 59u * (qh[i].x + 7u * qh[i].y);
        return h;
    }

    // Grid indices of the four 8-weight groups of block 4i + b, as the 16-bit
    // halves of ix[0] (groups 0, 1) and ix[1] (groups 2, 3): low bytes of the
    // index word placed by a v_perm, the 3-bit high fields of the qh word by
    // one multiply that copies them to two places (bits 8 and 21 up; for
    // groups 2, 3: 2 and 15 up): the copies do not overlap, so no carries,
    // and the mask keeps exactly the wanted fields at bits 8-10 and 24-26.
    __device__ __forceinline__ void grid_indices(int i, int b, uint32_t (&ix)[2]) const {
        const uint32_t qw = qv[i][b];
        const uint32_t hw = (qh[i][b >> 1] >> (16 * (b & 1))) & 0xfffu;  // four 3-bit high fields
        ix[0] = (__umul24(hw, 0x200100u) & 0x07000700u) | perm(qw, qw, 0x0c010c00u);
        ix[1] = (__umul24(hw, 0x008004u) & 0x07000700u) | perm(qw, qw, 0x0c030c02u);
    }

    // The decode's grid lookups without the decode: every entry its blocks
    // index (two 8-byte LDS reads per 16 weights, the decode's addresses),
    // folded into a hash.
    __device__ __forceinline__ uint32_t grid_hash(const uint2_t *b8) const {
        const uint8_t *b8b = reinterpret_cast<const uint8_t *>(b8);
        uint32_t h = 0;
#pragma unroll
        for (int c = 0; c < 4 * NI; ++c) {
            uint32_t ix[2];
            grid_indices(c >> 2, c & 3, ix);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const uint2_t w0 = *reinterpret_cast<const uint2_t *>(b8b + lo16_x8(ix[t]));
                const uint2_t w1 = *reinterpret_cast<const uint2_t *>(b8b + hi16_x8(ix[t]));
                h += (2u * c + 5u) * (w0.x + 3u * w0.y) + (2u * c + 7u) * (w1.x + 5u * w1.y);
            }
        }
        return h;
    }

    // blocks 16i+4g+b (32 weights: index bytes of dword b of qv[i], qh word b
    // of qh[i]).  The table holds 8g + 1; a block with a negative shift uses
    // 8g - 1, which takes 2 sum(f) off its digit sum.  fsum2: 2 sum(f) of
    // each 32-element block.
    // R rows, one lane instance each, share every A read.
    template <int R, bool EARLY>
    __device__ __forceinline__ static void decode(const LaneIq1s (&ln)[R], const uint8_t *abase, const float *sbs,
                                                  const int *fsum2, const uint2_t *b8, int g, float (&out)[R]) {
        // Each block's scale x 2^-E and its negative-shift correction
        // 2 sum(f) (or 0); 2s + 1 of the two blocks of a qh dword lands in
        // its bytes 0 and 2 in two ops.  All are formed before the first
        // index byte (EARLY), or each pair of blocks just before its MFMAs
        // (the registers of all would cost a wavefront per SIMD).
        float fac[R][4 * NI];
        int corr[R][4 * NI];
        const auto prep = [&](int i, int bp) {  // blocks 4i + 2bp, +1
            const float2 upv = *reinterpret_cast<const float2 *>(sbs + 16 * i + 4 * g + 2 * bp);
            const int2 fsv = *reinterpret_cast<const int2 *>(fsum2 + 16 * i + 4 * g + 2 * bp);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t qh = ln[r].qh[i][bp];
                const uint32_t odd = ((qh >> 11) & 0x000E000Eu) | 0x00010001u;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int c = 4 * i + 2 * bp + h;
                    fac[r][c] = float((odd >> (16 * h)) & 0xffu) * (h ? upv.y : upv.x);
                    corr[r][c] = (h ? fsv.y : fsv.x) & (int32_t(qh << (16 - 16 * h)) >> 31);
                    pin(fac[r][c]);
                    pin(corr[r][c]);
                }
            }
        };
        if constexpr (EARLY) {
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                prep(i, 0);
                prep(i, 1);
            }
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.f;
        const uint8_t *b8b = reinterpret_cast<const uint8_t *>(b8);
        int4_t Dp[R], A[4] = {};
#pragma unroll
        for (int c = 0; c <= 4 * NI; ++c) {  // block c = 4i + b
            int4_t D[R];
            if (c < 4 * NI) {
                const int i = c >> 2, b = c & 3;
                if ((b & 1) == 0) {  // blocks b, b+1
                    if constexpr (!EARLY) prep(i, b >> 1);
                    read_a(A, abase + 512 * i + 32 * b);
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    uint32_t ix[2];
                    ln[r].grid_indices(i, b, ix);
#pragma unroll
                    for (int t = 0; t < 2; ++t) {  // 8-weight groups 2t, 2t+1 of the block
                        const uint2_t w0 = *reinterpret_cast<const uint2_t *>(b8b + lo16_x8(ix[t]));
                        const uint2_t w1 = *reinterpret_cast<const uint2_t *>(b8b + hi16_x8(ix[t]));
                        D[r] = mfma(A[2 * (b & 1) + t], int4_t{int(w0.x), int(w0.y), int(w1.x), int(w1.y)},
                                    t ? D[r] : int4_t{0, 0, 0, 0});
                    }
                }
            }
            if (c > 0) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    acc[r] = fmaf(float(digits_sum(Dp[r]) - corr[r][c - 1]), fac[r][c - 1], acc[r]);
                    pin(acc[r]);
                }
            }
            if (c < 4 * NI) {
#pragma unroll
                for (int r = 0; r < R; ++r) Dp[r] = D[r];
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) out[r] = acc[r] * (0.125f * half_bits_to_float(ln[r].dvb));
    }
};

template <int MEMBER, int N>
using LaneOf = std::conditional_t<MEMBER == IQ2_KS, LaneIq2ks<N>,
                                  std::conditional_t<MEMBER == IQ2_K, LaneIq2k<N>,
                                                     LaneIq1s<N, Gemv2Shape<MEMBER, N>::WK>>>;

// What a launch computes: the decode, or one of its floors -- the decode's
// loads with the decode deleted (kFloor), and for IQ1_S_R4 also that floor
// with the decode's grid staging and lookups kept (kFloorGrid).
enum GemvKind : int { kDecode = 0, kFloor = 1, kFloorGrid = 2 };

// How a launch maps pairs to activation rows and stream reads.
// Either way one workgroup serves one (row tile, pair).  Pairs sorted by
// expert put a run's workgroups next to each other in the grid, so the run's
// later reads of its expert's rows mostly hit L2; the union form
// (gemv_mfma_union_kernel) decodes a run's pairs together instead.
enum GemvMode : int {
    kPairs = 0,   // pair m reads x[m / pairs_per_row]
    kSorted = 1,  // pair m reads x[toks[m]]
};

// R = 1: six wavefronts per SIMD, three workgroups of eight (N = 4096) or
// six of four (N = 2048) per CU, so a 1-token routed decode's 768
// workgroups are resident at once.  R = 2 (dispatches of many workgroups:
// IQ1_S_R4, and the IQ2 members at 2048 wide): each wavefront takes 32 rows, two MFMA column blocks that
// share every A read, so a workgroup stages its activations for 64 rows;
// five wavefronts per SIMD.
// T: 16-row tiles a workgroup (2: 32 rows; 1: 16 rows, for dispatches too
// small to give every CU the same number of 32-row workgroups, such as one
// token's gate alone: 384 of them on 256 CUs).  With T = 1 each thread
// stages two activation units (N = 4096) and expands twice the grid entries.
template <int MEMBER, int N, int FLOOR, int MODE, int R, int T = 2>
__global__ __launch_bounds__((64 * T * Gemv2Shape<MEMBER, N>::KS))
__attribute__((amdgpu_waves_per_eu(R == 2 ? 5 : 6)))
void gemv_mfma_kernel(Gemv2Args a) {
    using S = Gemv2Shape<MEMBER, N>;
    constexpr int KS = S::KS;
    constexpr int THREADS = 64 * T * KS;
    constexpr int ROWS = 16 * T * R;  // rows per workgroup
    constexpr int XU = S::UNITS > THREADS ? S::UNITS / THREADS : 1;  // activation units a thread stages
    static_assert(T == 1 || T == 2, "one or two 16-row tiles");
    static_assert(S::UNITS <= THREADS || S::UNITS == XU * THREADS, "whole staging passes");
    __shared__ Gemv2Smem<MEMBER, N, R, 1> sm;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, l = tid & 63;
    const int n = l & 15, g = l >> 4;
    const int kq = wave % KS, tile = wave / KS;
    const uint32_t m0 = MODE == kPairs ? blockIdx.z * a.pairs_per_row + blockIdx.y : blockIdx.z;
    const uint32_t rowg = blockIdx.x * ROWS;

    // Activation row of the pair; a row beyond x reads row 0 and yields NaN.
    const uint32_t tok = MODE == kPairs ? blockIdx.z : a.toks[m0];
    const bool x_ok = MODE == kPairs || tok < a.n_x_rows;

    // Activation (and IQ1_S_R4 grid) loads first: they do not wait for the
    // expert id, and vector loads retire in order, so staging them waits for
    // none of the stream bytes issued after them.
    const bool stager = tid < S::UNITS;  // uniform per wavefront
    uint4_t xv[XU];                        // fp16 pairs 4u .. 4u+3 of the pair's row, unit u = tid + THREADS i
#pragma unroll
    for (int i = 0; i < XU; ++i) {
        xv[i] = uint4_t{0u, 0u, 0u, 0u};
        if (stager)
            xv[i] = load_u4(bytes(a.x) + ((x_ok ? tok : 0u) * (2 * N) + 16 * uint32_t(tid + THREADS * i)));
    }
    constexpr bool IQ1 = MEMBER == IQ1_S_R4;
    // IQ1_S_R4: the codes of grid entries 4u .. 4u+3, u = tid + THREADS i
    constexpr bool GRID = IQ1 && FLOOR != kFloor;
    constexpr int GU = IQK_IQ1S_GRID_SIZE / (4 * THREADS);  // four-entry units a thread expands
    static_assert(!IQ1 || IQK_IQ1S_GRID_SIZE == 4 * GU * THREADS, "whole grid units per thread");
    uint2_t gridc[IQ1 ? GU : 1] = {};
    if constexpr (GRID) {
#pragma unroll
        for (int i = 0; i < GU; ++i) gridc[i] = reinterpret_cast<const uint2_t *>(iqk_iq1s_grid_codes)[tid + THREADS * i];
    }
    const auto stage_grid = [&]() {
#pragma unroll
        for (int i = 0; i < (IQ1 ? GU : 1); ++i) {
            uint4_t g0, g1;
            expand_grid_pair(gridc[i].x, g0);
            expand_grid_pair(gridc[i].y, g1);
            reinterpret_cast<uint4_t *>(sm.b8)[2 * (tid + THREADS * i)] = g0;
            reinterpret_cast<uint4_t *>(sm.b8)[2 * (tid + THREADS * i) + 1] = g1;
        }
    };
    constexpr bool KTAB = MEMBER == IQ2_K && FLOOR == kDecode;
    uint2_t ktv = {0u, 0u};
    if (KTAB && tid < 32) ktv = reinterpret_cast<const uint2_t *>(kIq2kTab.w)[tid];

    // An id beyond the stack reads expert 0 (in bounds) and writes NaN rows.
    // No early exit: a branch here would let the compiler sink the loads
    // above behind the wait for the id.
    const uint32_t e_raw = a.sel[m0];
    const bool valid = e_raw < a.num_experts;  // uniform per workgroup
    const uint32_t e = valid ? e_raw : 0u;
    LaneOf<MEMBER, N> lane[R];  // rows rowg + 16 (R tile + r) + n
#pragma unroll
    for (int r = 0; r < R; ++r) lane[r].load(a, e * a.out_features + rowg + 16 * (R * tile + r) + n, kq, g);

    // The pair's contraction, straight-line code.
    {
        float acc[R];
        if constexpr (FLOOR != kDecode) {
            uint32_t h = 0;
#pragma unroll
            for (int i = 0; i < XU; ++i) h += xv[i].x + 3u * xv[i].y + 5u * xv[i].z + 7u * xv[i].w;
#pragma unroll
            for (int r = 0; r < R; ++r) h += lane[r].hash();
            if constexpr (GRID) {  // kFloorGrid: the grid staging and every lookup
                stage_grid();
                __syncthreads();
#pragma unroll
                for (int r = 0; r < R; ++r) h += lane[r].grid_hash(sm.b8);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = float((h >> r) & 0xffu);
        } else {
            {
                if constexpr (GRID) stage_grid();
                if (KTAB && tid < 32) sm.ktab[tid] = ktv;
            }
            if (stager) {
                stage_activations<N, !IQ1, kZeroSpan<MEMBER, N>, kExpBlock<MEMBER>>(
                    sm.dig, sm.sbs, MEMBER == IQ2_KS ? sm.nsbs : nullptr, IQ1 ? sm.fsum : nullptr,
                    MEMBER == IQ2_K ? sm.fw : nullptr, tid, xv[0]);
#pragma unroll
                for (int i = 1; i < XU; ++i)  // a quad's threads take units of one quad, so the DPP stays in it
                    stage_activations<N, !IQ1, 0, kExpBlock<MEMBER>>(
                        sm.dig, sm.sbs, MEMBER == IQ2_KS ? sm.nsbs : nullptr, IQ1 ? sm.fsum : nullptr,
                        MEMBER == IQ2_K ? sm.fw : nullptr, tid + THREADS * i, xv[i]);
            }
            __syncthreads();
            const int ai = l & 15;  // this lane's A row
            const bool data = (ai >> 2) == g && (ai & 3) < 3;
            constexpr int LANE_K = IQ1 ? 128 : 64;
            const uint8_t *abase = sm.dig + (data ? (ai & 3) * kPlaneStride<N> + S::WK * kq + LANE_K * g
                                                  : 3 * kPlaneStride<N>);
            const float *sbs = sm.sbs + (S::WK / 32) * kq;
            using Lane = LaneOf<MEMBER, N>;
            // the prologue of every super-block before the first code word,
            // or (two row blocks) each just before its MFMAs: registers for a
            // wavefront per SIMD
            constexpr bool EARLY = R == 1;
            if constexpr (IQ1)
                Lane::template decode<R, EARLY>(lane, abase, sbs, sm.fsum + (S::WK / 32) * kq, sm.b8, g, acc);
            else if constexpr (MEMBER == IQ2_KS)
                Lane::template decode<R, EARLY>(lane, abase, sbs, sm.nsbs + (S::WK / 32) * kq, g, acc);
            else if constexpr (MODE == kSorted && R == 1)
                acc[0] = lane[0].decode_streamed(abase, sm.sbs + (S::WK / 64) * kq, sm.fw + (S::WK / 16) * kq,
                                                 sm.ktab, g);
            else
                Lane::template decode<R, EARLY>(lane, abase, sm.sbs + (S::WK / 64) * kq, sm.fw + (S::WK / 16) * kq,
                                         sm.ktab, g, acc);
        }
        // Partials of the row's lanes and wavefronts: wave 0 sums them after
        // the barrier.
#pragma unroll
        for (int r = 0; r < R; ++r) sm.part[0][kq][g][16 * (R * tile + r) + n] = acc[r];
        __syncthreads();
        if (tid < ROWS) {
            float sum = 0.f;
#pragma unroll
            for (int k = 0; k < KS; ++k)
                sum += (sm.part[0][k][0][tid] + sm.part[0][k][1][tid]) + (sm.part[0][k][2][tid] + sm.part[0][k][3][tid]);
            a.y[size_t(m0) * a.out_features + rowg + tid] = valid && x_ok ? uint16_t(float_to_half_bits(sum)) : kHalfNaN;
        }
    }
}

// P consecutive pairs of one activation row (pairs mode, one row block a
// wavefront; P = 1 is gemv_mfma_kernel): the workgroup stages the
// activations once and serves the same 32 rows of each pair's expert in
// turn, so the staging's VALU work (a quarter of a single pair's) is shared
// P ways.  That pays in dispatches of many tokens, where back-to-back
// workgroups are bound by VALU issue rather than by HBM.
template <int MEMBER, int N, int FLOOR, int P>
__global__ __launch_bounds__((Gemv2Shape<MEMBER, N>::THREADS))
__attribute__((amdgpu_waves_per_eu(6)))
void gemv_mfma_pairs_kernel(Gemv2Args a) {
    using S = Gemv2Shape<MEMBER, N>;
    constexpr int KS = S::KS;
    constexpr int ROWS = kGroupRows;  // rows per workgroup
    __shared__ Gemv2Smem<MEMBER, N, 1, P> sm;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, l = tid & 63;
    const int n = l & 15, g = l >> 4;
    const int kq = wave % KS, tile = wave / KS;
    // pairs m0 .. m0 + P - 1, all reading activation row blockIdx.z
    const uint32_t m0 = blockIdx.z * a.pairs_per_row + blockIdx.y * P;
    const uint32_t rowg = blockIdx.x * ROWS;

    // Activation (and IQ1_S_R4 grid) loads first: they do not wait for the
    // expert id, and vector loads retire in order, so staging them waits for
    // none of the stream bytes issued after them.
    const bool stager = tid < S::UNITS;  // uniform per wavefront
    uint4_t xv = {0u, 0u, 0u, 0u};         // fp16 pairs 4tid .. 4tid+3 of the pair's row
    if (stager) xv = load_u4(bytes(a.x) + (blockIdx.z * (2 * N) + 16 * uint32_t(tid)));
    constexpr bool IQ1 = MEMBER == IQ1_S_R4;
    // IQ1_S_R4: the codes of grid entries 4tid .. 4tid+3
    constexpr bool GRID = IQ1 && FLOOR != kFloor;
    static_assert(!IQ1 || IQK_IQ1S_GRID_SIZE == 4 * S::THREADS, "four grid entries per thread");
    uint2_t gridc = {0u, 0u};
    if constexpr (GRID) gridc = reinterpret_cast<const uint2_t *>(iqk_iq1s_grid_codes)[tid];
    constexpr bool KTAB = MEMBER == IQ2_K && FLOOR == kDecode;
    uint2_t ktv = {0u, 0u};
    if (KTAB && tid < 32) ktv = reinterpret_cast<const uint2_t *>(kIq2kTab.w)[tid];

    // An id beyond the stack reads expert 0 (in bounds) and writes NaN rows.
    // No early exit: a branch here would let the compiler sink the loads
    // above behind the wait for the id.
    uint32_t e[P];
    bool valid[P];  // uniform per workgroup
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t e_raw = a.sel[m0 + p];
        valid[p] = e_raw < a.num_experts;
        e[p] = valid[p] ? e_raw : 0u;
    }
    using Lane = LaneOf<MEMBER, N>;
    // this wavefront's 16 rows of pair p's expert
    const auto row_of = [&](int p) { return e[p] * a.out_features + rowg + 16 * tile + n; };
    Lane lane[1];
    lane[0].load(a, row_of(0), kq, g);

    if constexpr (GRID) {  // the grid expanded to int8 in LDS, once for all P pairs
        uint4_t g0, g1;
        expand_grid_pair(gridc.x, g0);
        expand_grid_pair(gridc.y, g1);
        reinterpret_cast<uint4_t *>(sm.b8)[2 * tid] = g0;
        reinterpret_cast<uint4_t *>(sm.b8)[2 * tid + 1] = g1;
    }
    if constexpr (FLOOR == kDecode) {
        if (KTAB && tid < 32) sm.ktab[tid] = ktv;
        if (stager)
            stage_activations<N, !IQ1, kZeroSpan<MEMBER, N>, kExpBlock<MEMBER>>(
                sm.dig, sm.sbs, MEMBER == IQ2_KS ? sm.nsbs : nullptr, IQ1 ? sm.fsum : nullptr,
                MEMBER == IQ2_K ? sm.fw : nullptr, tid, xv);
    }
    if constexpr (FLOOR == kDecode || GRID) __syncthreads();
    const int ai = l & 15;  // this lane's A row
    const bool data = (ai >> 2) == g && (ai & 3) < 3;
    constexpr int LANE_K = IQ1 ? 128 : 64;
    const uint8_t *abase = sm.dig + (data ? (ai & 3) * kPlaneStride<N> + S::WK * kq + LANE_K * g
                                          : 3 * kPlaneStride<N>);
    const float *sbs = sm.sbs + (S::WK / 32) * kq;

    // Each pair's contraction in turn, straight-line code; its partial row
    // sums (of the row's lanes and wavefronts) meet in LDS.  A pair's stream
    // loads go out once the previous pair's decode is done with its registers:
    // loading them a pair ahead needs ~100 VGPRs, four wavefronts per SIMD
    // instead of six, and measured slower.
#pragma unroll
    for (int p = 0; p < P; ++p) {
        if (p > 0) lane[0].load(a, row_of(p), kq, g);
        float acc[1];
        if constexpr (FLOOR != kDecode) {
            uint32_t h = xv.x + 3u * xv.y + 5u * xv.z + 7u * xv.w + lane[0].hash();
            if constexpr (GRID) h += lane[0].grid_hash(sm.b8);  // kFloorGrid: every lookup of the decode
            acc[0] = float(h & 0xffu);
        } else if constexpr (IQ1) {
            Lane::template decode<1, true>(lane, abase, sbs, sm.fsum + (S::WK / 32) * kq, sm.b8, g, acc);
        } else if constexpr (MEMBER == IQ2_KS) {
            Lane::template decode<1, true>(lane, abase, sbs, sm.nsbs + (S::WK / 32) * kq, g, acc);
        } else {
            Lane::template decode<1, true>(lane, abase, sm.sbs + (S::WK / 64) * kq, sm.fw + (S::WK / 16) * kq,
                                           sm.ktab, g, acc);
        }
        // the row index again from an opaque copy of the thread index: held
        // across the decode it costs a register the decode needs
        int t2 = tid;
        asm volatile("" : "+v"(t2));
        sm.part[p][(t2 >> 6) % KS][(t2 >> 4) & 3][16 * ((t2 >> 6) / KS) + (t2 & 15)] = acc[0];
    }
    // The first P x 32 threads sum the partials after the barrier.
    __syncthreads();
    if (tid < ROWS * P) {
        const int p = tid / ROWS, row = tid % ROWS;
        float sum = 0.f;
#pragma unroll
        for (int k = 0; k < KS; ++k)
            sum += (sm.part[p][k][0][row] + sm.part[p][k][1][row]) + (sm.part[p][k][2][row] + sm.part[p][k][3][row]);
        bool ok = true;
#pragma unroll
        for (int q = 0; q < P; ++q)
            if (q == p) ok = ok && valid[q];
        a.y[size_t(m0 + uint32_t(p)) * a.out_features + rowg + uint32_t(row)] =
            ok ? uint16_t(float_to_half_bits(sum)) : kHalfNaN;
    }
}

// The union form (sorted pairs, IQ2 members; reference: the first pair of a
// run of equal ids computes the run, src/mlx_iqk/kernels.py:484-572): a
// workgroup serves PM adjacent pairs, m0 = PM z .. m0 + PM - 1, and within
// them each run of equal ids together.  It stages every pair's activation row
// (a run's pairs are different tokens), then for each run loads the expert's
// rows once and expands its B operands once for all the run's pairs; the
// runs of a chunk follow one another, a run's loads issued once the previous
// run's decode is done with its registers.  Every pair's output is the pair
// GEMV's, bit for bit.
template <int MEMBER, int N, int PM>
struct GemvUnionSmem {
    uint8_t dig[PM][3 * kPlaneStride<N>] __attribute__((aligned(16)));
    uint8_t zero[kZeroSpan<MEMBER, N>] __attribute__((aligned(16)));  // what lanes without activations read
    float sbs[PM][N / 32] __attribute__((aligned(16)));
    float aux[PM][MEMBER == IQ2_KS ? N / 32 : N / 16] __attribute__((aligned(16)));  // nsbs (IQ2_KS), fw (IQ2_K)
    float part[PM][Gemv2Shape<MEMBER, N>::KS][4][kGroupRows];
    uint2_t ktab[MEMBER == IQ2_K ? 32 : 1];
};

template <int MEMBER, int N, int PM>
__global__ __launch_bounds__((Gemv2Shape<MEMBER, N>::THREADS))
__attribute__((amdgpu_waves_per_eu(6)))
void gemv_mfma_union_kernel(Gemv2Args a) {
    static_assert(MEMBER != IQ1_S_R4, "no union form for IQ1_S_R4");
    using S = Gemv2Shape<MEMBER, N>;
    constexpr int KS = S::KS;
    constexpr int ROWS = kGroupRows;
    __shared__ GemvUnionSmem<MEMBER, N, PM> sm;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, l = tid & 63;
    const int n = l & 15, g = l >> 4;
    const int kq = wave % KS, tile = wave / KS;
    const uint32_t m0 = blockIdx.z * PM;
    const uint32_t rowg = blockIdx.x * ROWS;
    const int cnt = a.mats - m0 < uint32_t(PM) ? int(a.mats - m0) : PM;  // uniform, >= 1

    uint32_t id[PM], tok[PM];
#pragma unroll
    for (int p = 0; p < PM; ++p) {
        id[p] = p < cnt ? a.sel[m0 + uint32_t(p)] : 0xffffffffu;
        tok[p] = p < cnt ? a.toks[m0 + uint32_t(p)] : 0u;
    }
    const bool stager = tid < S::UNITS;  // uniform per wavefront
    uint4_t xv[PM];
#pragma unroll
    for (int p = 0; p < PM; ++p) {
        xv[p] = uint4_t{0u, 0u, 0u, 0u};
        if (p < cnt && stager)
            xv[p] = load_u4(bytes(a.x) + ((tok[p] < a.n_x_rows ? tok[p] : 0u) * (2 * N) + 16 * uint32_t(tid)));
    }
    constexpr bool KTAB = MEMBER == IQ2_K;
    uint2_t ktv = {0u, 0u};
    if (KTAB && tid < 32) ktv = reinterpret_cast<const uint2_t *>(kIq2kTab.w)[tid];
    const auto expert = [&](int p) { return id[p] < a.num_experts ? id[p] : 0u; };
    LaneOf<MEMBER, N> lane;
    lane.load(a, expert(0) * a.out_features + rowg + 16 * tile + n, kq, g);

    if (KTAB && tid < 32) sm.ktab[tid] = ktv;
    if (tid < kZeroSpan<MEMBER, N> / 16) reinterpret_cast<uint4_t *>(sm.zero)[tid] = uint4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int p = 0; p < PM; ++p)
        if (p < cnt && stager)
            stage_activations<N, true, 0, kExpBlock<MEMBER>>(sm.dig[p], sm.sbs[p],
                                                             MEMBER == IQ2_KS ? sm.aux[p] : nullptr, nullptr,
                                                             MEMBER == IQ2_K ? sm.aux[p] : nullptr, tid, xv[p]);
    __syncthreads();
    const int ai = l & 15;
    const bool data = (ai >> 2) == g && (ai & 3) < 3;
#pragma unroll
    for (int st = 0; st < PM; ++st) {
        if (st < cnt && (st == 0 || id[st] != id[st - 1])) {
            int np = 1;
#pragma unroll
            for (int p = 1; p < PM - st; ++p)
                if (np == p && st + p < cnt && id[st + p] == id[st]) np = p + 1;
            if (st > 0) lane.load(a, expert(st) * a.out_features + rowg + 16 * tile + n, kq, g);
            const uint8_t *abase[PM];
            const float *sbs[PM], *aux[PM];
#pragma unroll
            for (int p = 0; p < PM; ++p) {
                const int q = st + p < PM ? st + p : PM - 1;
                abase[p] = data ? sm.dig[q] + (ai & 3) * kPlaneStride<N> + S::WK * kq + 64 * g : sm.zero;
                sbs[p] = sm.sbs[q] + (S::WK / kExpBlock<MEMBER>) * kq;
                aux[p] = sm.aux[q] + (S::WK / (MEMBER == IQ2_KS ? 32 : 16)) * kq;
            }
            float acc[PM];
            if constexpr (MEMBER == IQ2_KS)
                lane.template decode_pairs<PM>(abase, sbs, aux, np, g, acc);
            else
                lane.template decode_pairs<PM>(abase, sbs, aux, sm.ktab, np, g, acc);
#pragma unroll
            for (int p = 0; p < PM - st; ++p)
                if (p < np) sm.part[st + p][kq][g][16 * tile + n] = acc[p];
        }
    }
    __syncthreads();
    if (tid < ROWS * cnt) {
        const int p = tid / ROWS, row = tid % ROWS;
        float sum = 0.f;
#pragma unroll
        for (int k = 0; k < KS; ++k)
            sum += (sm.part[p][k][0][row] + sm.part[p][k][1][row]) + (sm.part[p][k][2][row] + sm.part[p][k][3][row]);
        bool ok = false;
#pragma unroll
        for (int q = 0; q < PM; ++q)
            if (q == p) ok = id[q] < a.num_experts && tok[q] < a.n_x_rows;
        a.y[size_t(m0 + uint32_t(p)) * a.out_features + rowg + uint32_t(row)] =
            ok ? uint16_t(float_to_half_bits(sum)) : kHalfNaN;
    }
}

// Pairs a union workgroup serves.  A pair's staged activations take 12.3 KB
// of LDS (4096 wide), so three pairs keep three workgroups a CU.
constexpr int kUnionPairs = 3;

template <int MEMBER>
int launch_union(int64_t n, const Gemv2Args &a, uint32_t mats, hipStream_t st) {
    const dim3 grid{a.out_features / kGroupRows, 1u, (mats + kUnionPairs - 1) / kUnionPairs};
    if (n == 4096)
        hipLaunchKernelGGL((gemv_mfma_union_kernel<MEMBER, 4096, kUnionPairs>), grid,
                           dim3{uint32_t(Gemv2Shape<MEMBER, 4096>::THREADS)}, 0, st, a);
    else
        hipLaunchKernelGGL((gemv_mfma_union_kernel<MEMBER, 2048, kUnionPairs>), grid,
                           dim3{uint32_t(Gemv2Shape<MEMBER, 2048>::THREADS)}, 0, st, a);
    return record_launch(hipGetLastError());
}

template <int MEMBER, int FLOOR, int MODE, int R, int P, int T = 2>
int launch_gemv_mfma(int64_t n, const Gemv2Args &a, uint32_t mats, hipStream_t st) {
    const uint32_t groups = a.out_features / (16 * T * R);
    const dim3 grid = MODE == kPairs ? dim3{groups, a.pairs_per_row / P, mats / a.pairs_per_row} : dim3{groups, 1u, mats};
    const dim3 block4096{uint32_t(64 * T * Gemv2Shape<MEMBER, 4096>::KS)},
        block2048{uint32_t(64 * T * Gemv2Shape<MEMBER, 2048>::KS)};
    static_assert(P == 1 || (MODE == kPairs && R == 1 && T == 2), "several pairs a workgroup: pairs mode, one row block");
    if constexpr (P > 1) {
        if (n == 4096)
            hipLaunchKernelGGL((gemv_mfma_pairs_kernel<MEMBER, 4096, FLOOR, P>), grid, block4096, 0, st, a);
        else
            hipLaunchKernelGGL((gemv_mfma_pairs_kernel<MEMBER, 2048, FLOOR, P>), grid, block2048, 0, st, a);
    } else if (n == 4096) {
        hipLaunchKernelGGL((gemv_mfma_kernel<MEMBER, 4096, FLOOR, MODE, R, T>), grid, block4096, 0, st, a);
    } else {
        hipLaunchKernelGGL((gemv_mfma_kernel<MEMBER, 2048, FLOOR, MODE, R, T>), grid, block2048, 0, st, a);
    }
    return record_launch(hipGetLastError());
}

template <int FLOOR, int MODE, int R, int P = 1, int T = 2>
int launch_member(int member, int64_t n, const Gemv2Args &a, uint32_t mats, hipStream_t st) {
    switch (member) {
        case IQK_MEMBER_IQ2_KS: return launch_gemv_mfma<IQ2_KS, FLOOR, MODE, R, P, T>(n, a, mats, st);
        case IQK_MEMBER_IQ2_K: return launch_gemv_mfma<IQ2_K, FLOOR, MODE, R, P, T>(n, a, mats, st);
        default:
            if constexpr (MODE == kPairs) return launch_gemv_mfma<IQ1_S_R4, FLOOR, MODE, R, P, T>(n, a, mats, st);
            return IQK_ERR_MEMBER;  // no sorted or union form for IQ1_S_R4
    }
}

// A decode launch in pairs mode: R row blocks a wavefront, P pairs a
// workgroup; pairs == 0 asks for 16-row workgroups (one pair, one row block).
template <int FLOOR, int R>
int launch_pairs(int member, int64_t n, const Gemv2Args &a, uint32_t mats, int pairs, hipStream_t st) {
    if constexpr (R != 1) {
        return launch_member<FLOOR, kPairs, R, 1>(member, n, a, mats, st);
    } else {
        switch (pairs) {
            case 3: return launch_member<FLOOR, kPairs, 1, 3>(member, n, a, mats, st);
            case 2: return launch_member<FLOOR, kPairs, 1, 2>(member, n, a, mats, st);
            case 0: return launch_member<FLOOR, kPairs, 1, 1, 1>(member, n, a, mats, st);
            default: return launch_member<FLOOR, kPairs, 1, 1>(member, n, a, mats, st);
        }
    }
}

// Dispatches of many 32-row workgroups take two row blocks per wavefront:
// IQ1_S_R4 at either width from twice the 768 of a 1-token decode (top-6
// measured 5-10% faster with two blocks at 2 and 3 tokens, 13% slower at 1),
// the IQ2 members at 2048 wide (the down projection) from eight times (top-6
// down measured 2-4% slower with two blocks at 4 tokens, 2-4% faster at 8 and
// 6-7% at 32).  The IQ2 members' 4096-wide dispatches keep one block (1-2%
// slower with two).
constexpr uint64_t kTwoRowMinGroups = 2 * 768;
constexpr uint64_t kTwoRowMinGroupsIq2 = 8 * 768;

// Pairs a workgroup (pairs mode, one row block a wavefront): three pairs of
// one activation row share its staging once a dispatch has two rounds of the
// chip's 768 resident workgroups.  Measured (256 experts, top-6 gate and up
// as one dispatch, back to back): IQ2_K 48.7 -> 45.7 us at 8 tokens, 188 ->
// 176-178 us at 32, 13.9 -> 13.3 us at 2; IQ2_KS 44.8 -> 42.5 us at 8.  Six
// pairs a workgroup measured the same or slower.
constexpr uint64_t kSharedStagingMinGroups = 2 * 768;

// Dispatches of fewer 32-row workgroups than this (one round of three a CU)
// run 16-row workgroups instead, so the CUs share the work evenly: one
// token's gate alone (the switch module's own dispatch, 384 workgroups of 32
// rows) gives 256 CUs one or two workgroups each.
constexpr uint64_t kHalfTileMaxGroups = 768;

// Pairs a workgroup: 3 or 2 (shared staging), 1, or 0 (one pair in 16-row
// workgroups).
int pairs_per_group(uint64_t workgroups, uint32_t pairs_per_row) {
    if (workgroups < kHalfTileMaxGroups) return 0;
    if (workgroups < kSharedStagingMinGroups) return 1;
    return pairs_per_row % 3 == 0 ? 3 : pairs_per_row % 2 == 0 ? 2 : 1;
}

// Called by the GEMV entry points (after their argument checks) when
// out_features is a multiple of the workgroup's 32 rows; returns -1 when this
// path does not apply.  `toks` NULL = pairs mode (x row m / pairs_per_row);
// else x row toks[m] of n_x_rows: the sorted entry point (see GemvMode), or
// with union_runs the union kernel.
int gemv_mfma_dispatch(int floor, int member, int64_t n, int64_t out, int64_t num_experts, const void *x,
                       int64_t n_x_rows, const void *const *streams, int n_streams, const uint32_t *sel,
                       const uint32_t *toks, bool union_runs, uint32_t pairs_per_row, uint32_t mats, void *y,
                       hipStream_t st) {
    if (out % kGroupRows) return -1;
    // 32-bit offsets: every stream (the code plane is the largest, N/4 bytes a
    // row) and the activations stay below 4 GiB
    const uint64_t lim = uint64_t(1) << 32;
    if (uint64_t(num_experts) * uint64_t(out) * uint64_t(n / 4) >= lim) return -1;
    if (uint64_t(n_x_rows) * uint64_t(2 * n) >= lim) return -1;
    Gemv2Args a;
    a.x = static_cast<const uint32_t *>(x);
    a.s0 = streams[0]; a.s1 = streams[1]; a.s2 = streams[2];
    a.s3 = n_streams > 3 ? streams[3] : nullptr;
    a.s4 = n_streams > 4 ? streams[4] : nullptr;
    a.sel = sel;
    a.toks = toks;
    a.pairs_per_row = pairs_per_row;
    a.mats = mats;
    a.n_x_rows = uint32_t(n_x_rows);
    a.num_experts = uint32_t(num_experts);
    a.out_features = uint32_t(out);
    a.y = static_cast<uint16_t *>(y);
    if (!toks) {
        const uint64_t groups = uint64_t(mats) * uint64_t(out / kGroupRows);
        const bool two = out % (2 * kGroupRows) == 0 &&
                         (member == IQK_MEMBER_IQ1_S_R4 ? groups >= kTwoRowMinGroups
                                                        : n == 2048 && groups >= kTwoRowMinGroupsIq2);
        // only IQ1_S_R4 has grid lookups to keep; the others' kFloorGrid is kFloor
        const int kind = floor == kFloorGrid && member != IQK_MEMBER_IQ1_S_R4 ? kFloor : floor;
        const int pairs = two ? 1 : pairs_per_group(groups, pairs_per_row);
        if (two) {
            switch (kind) {
                case kFloor: return launch_pairs<kFloor, 2>(member, n, a, mats, pairs, st);
                case kFloorGrid: return launch_pairs<kFloorGrid, 2>(member, n, a, mats, pairs, st);
                default: return launch_pairs<kDecode, 2>(member, n, a, mats, pairs, st);
            }
        }
        switch (kind) {
            case kFloor: return launch_pairs<kFloor, 1>(member, n, a, mats, pairs, st);
            case kFloorGrid: return launch_pairs<kFloorGrid, 1>(member, n, a, mats, pairs, st);
            default: return launch_pairs<kDecode, 1>(member, n, a, mats, pairs, st);
        }
    }
    if (floor != kDecode) return IQK_ERR_ARGUMENT;
    if (union_runs) {
        switch (member) {
            case IQK_MEMBER_IQ2_KS: return launch_union<IQ2_KS>(n, a, mats, st);
            case IQK_MEMBER_IQ2_K: return launch_union<IQ2_K>(n, a, mats, st);
            default: return IQK_ERR_MEMBER;  // no union form for IQ1_S_R4
        }
    }
    return launch_member<kDecode, kSorted, 1>(member, n, a, mats, st);
}

}  // namespace iqk
