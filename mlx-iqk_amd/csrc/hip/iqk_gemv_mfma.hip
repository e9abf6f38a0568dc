// Decode GEMV on int8 MFMA (gfx950), IQ2_KS: the routed decode's fast path.
//
// Reference: the Metal decode GEMV (src/mlx_iqk/kernels.py:332-401) computes
// out[m, r] = half(sum_sb dl_sb * sum_{j in sb} v_j x_j) with an f32 fma chain
// per lane.  Here the multiply-accumulate runs on v_mfma_i32_16x16x64_i8:
//
// * Weights.  Both alphabets are v = 2w + off, w in {-16, -7, 0, 8},
//   off in {1, 6}.  One v_perm_b32 maps four packed 2-bit codes to four int8
//   w values, so a 16-code word becomes the 16-byte B operand of one lane in
//   11 VALU ops.
// * Activations.  x is converted once per workgroup into an integer with a
//   per-sub-block power-of-two scale, x ~ f * 2^-E, |f| < 2^20, split into
//   three int8 digits f = d0 * 2^14 + d1 * 2^7 + d2 (d1, d2 in [0,127]).  The
//   digits are the A operand; the MFMA's integer sums are exact, so a
//   sub-block's sum(w x) is exact up to the rounding of x to 20 bits relative
//   to its sub-block maximum (below fp16's resolution for every element
//   within 2^9 of that maximum).  The conversion runs while the code loads
//   are in flight.
// * Layout.  A wavefront owns 16 rows (the MFMA's N); lane (n, g) = (l%16,
//   l/16).  For super-block s the four lanes of row n read its 64 contiguous
//   code bytes, lane group g taking words 16s+4g..16s+4g+3, i.e. sub-blocks
//   8s+2g and 8s+2g+1.  A-rows 4g..4g+2 carry the digits of lane group g's
//   k-range and zero elsewhere, so D rows 4g..4g+2 -- which the MFMA places in
//   lane group g -- collect exactly that lane's sub-block, one digit each.
//   Two MFMAs complete a sub-block; each lane then folds one (row, sub-block):
//   sum(v x) = 2^(1-E) * (D0 2^14 + D1 2^7 + D2) + off * sum(x), scaled by the
//   sub-block's index.  A-operand reads come from LDS; lanes whose A row is
//   zero read a zero region at the same offsets.
//
// The floor variant keeps every global load and deletes the decode.

#include "iqk_device.h"
#include "iqk_host.h"

namespace iqk {

typedef int int4_t __attribute__((ext_vector_type(4)));

struct Gemv2Args {
    const uint32_t *x;
    const void *qs, *scl, *sch, *sex, *dv;
    const uint32_t *sel;
    uint32_t pairs_per_row;
    uint32_t num_experts;
    uint32_t out_features;
    uint16_t *y;
};

constexpr uint32_t kW8Pool = 0x0800F9F0u;  // int8 w for codes 0..3: -16, -7, 0, 8
constexpr int kWaves = 4;                   // wavefronts per workgroup (16 rows each)

// The 16 int8 weights of one code word, in the byte order the digits use:
// operand dword s holds codes s, 4+s, 8+s, 12+s.
__device__ __forceinline__ int4_t word_to_w8(uint32_t q) {
    int4_t b;
    b.x = int(perm(kW8Pool, kW8Pool, q & 0x03030303u));
    b.y = int(perm(kW8Pool, kW8Pool, (q >> 2) & 0x03030303u));
    b.z = int(perm(kW8Pool, kW8Pool, (q >> 4) & 0x03030303u));
    b.w = int(perm(kW8Pool, kW8Pool, (q >> 6) & 0x03030303u));
    return b;
}

template <int N, bool FLOOR>
__global__ __launch_bounds__(64 * kWaves) void gemv_mfma_iq2ks(Gemv2Args a) {
    constexpr int SB = N / 256;   // super-blocks per row
    constexpr int NSUB = N / 32;  // sub-blocks per row
    constexpr int WORDS = N / 16;
    // LDS: digit planes [3][N], a zero plane [N], per-sub-block (sum x, 2^(1-E))
    __shared__ __attribute__((aligned(16))) uint8_t lds[4 * N];
    __shared__ float2 sbt[NSUB];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, l = tid & 63;
    const int n = l & 15, g = l >> 4;
    const uint32_t m = blockIdx.y;
    const uint32_t row0 = blockIdx.x * (16 * kWaves) + 16 * wave;
    const uint32_t e = a.sel[m];
    uint16_t *ytile = a.y + size_t(m) * a.out_features + row0;
    if (e >= a.num_experts) {  // uniform per workgroup
        if (l < 16) ytile[l] = kHalfNaN;
        return;
    }
    const size_t row = size_t(e) * a.out_features + row0 + n;

    // -- issue every stream load of this lane's row first -----------------------
    uint4_t q[SB];
#pragma unroll
    for (int s = 0; s < SB; ++s)
        q[s] = load_u4(static_cast<const uint32_t *>(a.qs) + row * WORDS + 16 * s + 4 * g);
    uint4_t sc[SB / 4 > 0 ? SB / 4 : 1];  // the row's N/64 scale bytes
#pragma unroll
    for (int i = 0; i < SB / 4; ++i) sc[i] = load_u4(static_cast<const uint8_t *>(a.scl) + row * (N / 64) + 16 * i);
    uint4_t hb, ab;  // the row's N/256 bytes of high-bit and alphabet planes
    if constexpr (SB == 16) {
        hb = load_u4(static_cast<const uint8_t *>(a.sch) + row * SB);
        ab = load_u4(static_cast<const uint8_t *>(a.sex) + row * SB);
    } else {
        const uint2_t h2 = *reinterpret_cast<const uint2_t *>(static_cast<const uint8_t *>(a.sch) + row * SB);
        const uint2_t a2 = *reinterpret_cast<const uint2_t *>(static_cast<const uint8_t *>(a.sex) + row * SB);
        hb = uint4_t{h2.x, h2.y, 0u, 0u};
        ab = uint4_t{a2.x, a2.y, 0u, 0u};
    }
    const uint32_t dvb = static_cast<const uint16_t *>(a.dv)[row];
    const uint32_t tok = m / a.pairs_per_row;
    const uint32_t *xrow = a.x + size_t(tok) * (N / 2);

    if constexpr (FLOOR) {
        uint32_t iacc = 0;
        if (tid < WORDS) {  // the activation loads of the decode's conversion
            const uint4_t x0 = load_u4(xrow + 8 * tid), x1 = load_u4(xrow + 8 * tid + 4);
            iacc += x0.x + 3u * x0.y + 5u * x0.z + 7u * x0.w + 11u * x1.x + 13u * x1.y + 17u * x1.z + 19u * x1.w;
        }
#pragma unroll
        for (int s = 0; s < SB; ++s) iacc += q[s].x + 3u * q[s].y + 5u * q[s].z + 7u * q[s].w;
#pragma unroll
        for (int i = 0; i < SB / 4; ++i) iacc += 59u * (sc[i].x + sc[i].y + sc[i].z + sc[i].w);
        iacc += 61u * (hb.x + hb.y + hb.z + hb.w) + 71u * (ab.x + ab.y + ab.z + ab.w) + 67u * dvb;
        float acc = float(iacc & 0xffu);
        acc += __shfl_xor(acc, 16);
        acc += __shfl_xor(acc, 32);
        if (g == 0) ytile[n] = uint16_t(float_to_half_bits(acc));
        return;
    } else {
        // -- activations -> LDS digits (one code word of x per thread) ----------
        for (int i = tid; i < N / 16; i += 64 * kWaves)  // the zero plane
            *reinterpret_cast<uint4_t *>(lds + 3 * N + 16 * i) = uint4_t{0u, 0u, 0u, 0u};
        if (tid < WORDS) {
            const uint4_t x0 = load_u4(xrow + 8 * tid), x1 = load_u4(xrow + 8 * tid + 4);
            const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            float xf[16];
            float amax = 0.f, xsum = 0.f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                xf[j] = half_bits_to_float((xw[j / 2] >> (16 * (j & 1))) & 0xffffu);
                amax = fmaxf(amax, fabsf(xf[j]));
                xsum += xf[j];
            }
            amax = fmaxf(amax, __shfl_xor(amax, 1));  // the two words of a sub-block
            xsum += __shfl_xor(xsum, 1);
            // E so that max|x| * 2^E lies in [2^19, 2^20): |f| < 2^20, d0 in [-64, 63]
            const int ex = amax > 0.f ? int((__float_as_uint(amax) >> 23) & 0xffu) - 127 : 0;
            const int E = 19 - ex;
            uint32_t d0[4] = {0, 0, 0, 0}, d1[4] = {0, 0, 0, 0}, d2[4] = {0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int f = int(__builtin_rintf(__builtin_ldexpf(xf[j], E)));
                const int s = j & 3, t = j >> 2;  // operand dword s, byte t holds element 4t+s
                d2[s] |= uint32_t(f & 127) << (8 * t);
                d1[s] |= uint32_t((f >> 7) & 127) << (8 * t);
                d0[s] |= uint32_t((f >> 14) & 255) << (8 * t);
            }
            *reinterpret_cast<uint4_t *>(lds + 0 * N + 16 * tid) = uint4_t{d0[0], d0[1], d0[2], d0[3]};
            *reinterpret_cast<uint4_t *>(lds + 1 * N + 16 * tid) = uint4_t{d1[0], d1[1], d1[2], d1[3]};
            *reinterpret_cast<uint4_t *>(lds + 2 * N + 16 * tid) = uint4_t{d2[0], d2[1], d2[2], d2[3]};
            if ((tid & 1) == 0) sbt[tid >> 1] = float2{xsum, __builtin_ldexpf(1.f, 1 - E)};
        }
        __syncthreads();

        // -- MFMA over the row tile ----------------------------------------------
        const int ai = l & 15;  // this lane's A row
        const bool data = (ai >> 2) == g && (ai & 3) < 3;
        const uint8_t *abase = lds + (data ? (ai & 3) * N + 64 * g : 3 * N);
        const float d = half_bits_to_float(dvb);
        float acc = 0.f;
#pragma unroll
        for (int s = 0; s < SB; ++s) {
            const uint32_t scb = (sc[s / 4][s % 4] >> (8 * g)) & 0xffu;  // byte 4s+g
            const uint32_t hib = (hb[s / 4] >> (8 * (s % 4) + 2 * g)) & 3u;
            const uint32_t alb = (ab[s / 4] >> (8 * (s % 4) + 2 * g)) & 3u;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                int4_t D = {0, 0, 0, 0};
#pragma unroll
                for (int j = 2 * h; j < 2 * h + 2; ++j) {
                    const int4_t A = __builtin_bit_cast(int4_t, *reinterpret_cast<const uint4_t *>(abase + (16 * s + j) * 16));
                    D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, word_to_w8(q[s][j]), D, 0, 0, 0);
                }
                const int sint = (D.x << 14) + (D.y << 7) + D.z;
                const float2 t = sbt[8 * s + 2 * g + h];
                const float off = ((alb >> h) & 1u) ? 6.f : 1.f;
                const float S = fmaf(float(sint), t.y, off * t.x);
                const int idx = int(((scb >> (4 * h)) & 15u) | (((hib >> h) & 1u) << 4)) - 16;
                acc = fmaf(float(idx), S, acc);
            }
        }
        acc *= d;
        acc += __shfl_xor(acc, 16);
        acc += __shfl_xor(acc, 32);
        if (g == 0) ytile[n] = uint16_t(float_to_half_bits(acc));
    }
}

template <bool FLOOR>
int launch_gemv_mfma(int64_t n, const Gemv2Args &a, uint32_t mats, hipStream_t st) {
    const dim3 grid{a.out_features / (16 * kWaves), mats}, block{64 * kWaves};
    if (n == 4096)
        hipLaunchKernelGGL((gemv_mfma_iq2ks<4096, FLOOR>), grid, block, 0, st, a);
    else
        hipLaunchKernelGGL((gemv_mfma_iq2ks<2048, FLOOR>), grid, block, 0, st, a);
    return record_launch(hipGetLastError());
}

// Called by the GEMV entry points for IQ2_KS when out_features is a multiple
// of 64 (the workgroup tile); returns -1 when this path does not apply.
int gemv_mfma_dispatch(bool floor, int member, int64_t n, int64_t out, int64_t num_experts, const void *x,
                       const void *const *streams, const uint32_t *sel, uint32_t pairs_per_row, uint32_t mats,
                       void *y, hipStream_t st) {
    if (member != IQK_MEMBER_IQ2_KS || out % (16 * kWaves)) return -1;
    Gemv2Args a;
    a.x = static_cast<const uint32_t *>(x);
    a.qs = streams[0]; a.scl = streams[1]; a.sch = streams[2]; a.sex = streams[3]; a.dv = streams[4];
    a.sel = sel;
    a.pairs_per_row = pairs_per_row;
    a.num_experts = uint32_t(num_experts);
    a.out_features = uint32_t(out);
    a.y = static_cast<uint16_t *>(y);
    return floor ? launch_gemv_mfma<true>(n, a, mats, st) : launch_gemv_mfma<false>(n, a, mats, st);
}

}  // namespace iqk
