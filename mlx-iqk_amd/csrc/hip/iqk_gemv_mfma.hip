// Decode GEMV on int8 MFMA (gfx950), IQ2_KS: the routed decode's fast path.
//
// Reference: the Metal decode GEMV (src/mlx_iqk/kernels.py:332-401) computes
// out[m, r] = half(sum_sb dl_sb * sum_{j in sb} v_j x_j) with an f32 fma chain
// per lane.  Here the multiply-accumulate runs on v_mfma_i32_16x16x64_i8.
//
// * Weights.  The two alphabets (-31,-13,1,17) and (-26,-8,6,22) fit int8, so
//   one v_perm_b32 maps four packed 2-bit codes to four int8 values v, from
//   a 4-byte pool chosen by the sub-block's alphabet bit.
// * Activations.  x is converted once per workgroup into an integer with a
//   per-sub-block power-of-two scale, f = rint(x * 2^E) with |f| <= 2^20,
//   and split into balanced bytes f = b0 + 2^8 b1 + 2^16 b2 (each b in
//   [-128, 127]: the bytes of f + 0x808080, each minus 128).  The bytes are
//   the A operand.  The MFMA's integer sums are exact, so a sub-block's
//   sum(v x) is exact up to the rounding of x to 2^-20 of its sub-block
//   maximum (exact for every element within 2^9 of that maximum).  A
//   sub-block holding an inf or NaN gets a NaN scale, so the rows that read
//   it come back NaN.
// * Layout.  A wavefront owns 16 rows (the MFMA's N) and 1024 of the
//   reduction axis; a workgroup owns 32 rows and all of it, N/1024
//   wavefronts per 16 rows, so a whole wavefront's compute after its last
//   byte arrives stays short.  Lane (n, g) = (l%16, l/16).  For super-block
//   s the four lanes of row n read its 64 contiguous code bytes, lane group g
//   taking words 16s+4g..16s+4g+3, i.e. sub-blocks 8s+2g and 8s+2g+1.
//   A-rows 4g..4g+2 carry the byte planes of lane group g's k-range and zero
//   elsewhere, so D rows 4g..4g+2 -- which the MFMA places in lane group g --
//   collect exactly that lane's sub-block, one byte plane each.  Two MFMAs
//   complete a sub-block; each lane then folds one (row, sub-block):
//   sum(v x) = 2^-E (D0 + 2^8 D1 + 2^16 D2), times the sub-block's index.
//   Lanes whose A row is zero read a zero span of LDS at the same offsets.
//   The partial sums of a row's wavefronts meet in LDS.
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

constexpr uint32_t kV8Base = 0x1101F3E1u;   // int8 -31, -13, 1, 17
constexpr uint32_t kV8Shift = 0x1606F8E6u;  // int8 -26, -8, 6, 22
constexpr int kWaveK = 1024;                // reduction elements per wavefront
constexpr int kGroupRows = 32;              // rows per workgroup

template <int N>
struct Gemv2Shape {
    static constexpr int KS = N / kWaveK;     // wavefronts per 16 rows
    static constexpr int THREADS = 64 * 2 * KS;
    static constexpr int SBW = kWaveK / 256;  // super-blocks per wavefront
    static_assert(N / 8 == THREADS, "one thread per 8 activations");
};

// The 16 int8 weights of one code word; operand dword s holds codes s, 4+s,
// 8+s, 12+s (byte t = code 4t+s).
__device__ __forceinline__ int4_t word_to_v8(uint32_t q, uint32_t pool) {
    int4_t b;
    b.x = int(perm(pool, pool, q & 0x03030303u));
    b.y = int(perm(pool, pool, (q >> 2) & 0x03030303u));
    b.z = int(perm(pool, pool, (q >> 4) & 0x03030303u));
    b.w = int(perm(pool, pool, (q >> 6) & 0x03030303u));
    return b;
}

// Bit `pos` of w as an all-ones / all-zeros mask.
__device__ __forceinline__ uint32_t bit_mask(uint32_t w, int pos) {
    return uint32_t(int32_t(w << (31 - pos)) >> 31);
}

// Plane k, operand dword: bytes k of u[0..3], each minus 128.
__device__ __forceinline__ void byte_planes(const uint32_t *u, uint32_t &p0, uint32_t &p1, uint32_t &p2) {
    const uint32_t a01 = perm(u[1], u[0], 0x05010400u), a23 = perm(u[3], u[2], 0x05010400u);
    p0 = perm(a23, a01, 0x05040100u) ^ 0x80808080u;
    p1 = perm(a23, a01, 0x07060302u) ^ 0x80808080u;
    p2 = (perm(u[1], u[0], 0x0c0c0602u) | perm(u[3], u[2], 0x06020c0cu)) ^ 0x80808080u;
}

template <int N, bool FLOOR>
__global__ __launch_bounds__(Gemv2Shape<N>::THREADS) void gemv_mfma_iq2ks(Gemv2Args a) {
    using S = Gemv2Shape<N>;
    constexpr int KS = S::KS, SBW = S::SBW;
    // LDS: byte planes [3][N], a zero span [kWaveK], 2^-E per sub-block, partials
    __shared__ __attribute__((aligned(16))) uint8_t dig[3 * N + kWaveK];
    __shared__ float sbs[N / 32];
    __shared__ float part[KS][kGroupRows];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, l = tid & 63;
    const int n = l & 15, g = l >> 4;
    const int kq = wave % KS, tile = wave / KS;
    const uint32_t m = blockIdx.y;
    const uint32_t rowg = blockIdx.x * kGroupRows;

    // -- activation loads first: they do not wait for the expert id -------------
    const uint32_t tok = m / a.pairs_per_row;
    const uint32_t wd = uint32_t(tid) >> 1, hp = uint32_t(tid) & 1u;  // code word of x, half of it
    const uint32_t *xw = a.x + size_t(tok) * (N / 2) + 8 * wd;
    const uint4_t x0 = load_u4(xw), x1 = load_u4(xw + 4);

    const uint32_t e = a.sel[m];
    uint16_t *ygroup = a.y + size_t(m) * a.out_features + rowg;
    if (e >= a.num_experts) {  // uniform per workgroup
        if (tid < kGroupRows) ygroup[tid] = kHalfNaN;
        return;
    }
    const size_t row = size_t(e) * a.out_features + rowg + 16 * tile + n;

    // -- this lane's stream bytes: planes first, then the code words -------------
    const uint4_t scv = load_u4(static_cast<const uint8_t *>(a.scl) + row * (N / 64) + 16 * kq);
    const uint32_t hbw = *reinterpret_cast<const uint32_t *>(static_cast<const uint8_t *>(a.sch) + row * (N / 256) + 4 * kq);
    const uint32_t abw = *reinterpret_cast<const uint32_t *>(static_cast<const uint8_t *>(a.sex) + row * (N / 256) + 4 * kq);
    const uint32_t dvb = static_cast<const uint16_t *>(a.dv)[row];
    uint4_t q[SBW];
#pragma unroll
    for (int s = 0; s < SBW; ++s)
        q[s] = load_u4(static_cast<const uint32_t *>(a.qs) + row * (N / 16) + 64 * kq + 16 * s + 4 * g);

    float acc;
    if constexpr (FLOOR) {
        uint32_t iacc = x0.x + 3u * x0.y + 5u * x0.z + 7u * x0.w + 11u * x1.x + 13u * x1.y + 17u * x1.z + 19u * x1.w;
#pragma unroll
        for (int s = 0; s < SBW; ++s) iacc += q[s].x + 3u * q[s].y + 5u * q[s].z + 7u * q[s].w;
        iacc += 59u * (scv.x + scv.y + scv.z + scv.w) + 61u * hbw + 71u * abw + 67u * dvb;
        acc = float(iacc & 0xffu);
    } else {
        // -- activations -> balanced byte planes in LDS ---------------------------
        if (tid < kWaveK / 16)
            *reinterpret_cast<uint4_t *>(dig + 3 * N + 16 * tid) = uint4_t{0u, 0u, 0u, 0u};
        {
            // This thread's 8 activations: operand dwords 2hp and 2hp+1 of word
            // wd, i.e. elements 4t + 2hp (low halves) and 4t + 2hp + 1 (high
            // halves) of the fp16 pairs xp[t] = pair 2t + hp.
            const uint32_t xp[4] = {hp ? x0.y : x0.x, hp ? x0.w : x0.z, hp ? x1.y : x1.x, hp ? x1.w : x1.z};
            // max |x| on the fp16 bits (magnitude order is integer order)
            uint32_t mx = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) mx = max(mx, max(xp[t] & 0x7fffu, (xp[t] >> 16) & 0x7fffu));
            mx = max(mx, uint32_t(__shfl_xor(int(mx), 1)));  // the 4 threads of a 32-element sub-block
            mx = max(mx, uint32_t(__shfl_xor(int(mx), 2)));
            const bool finite = mx < 0x7c00u;
            // E so that max|x| * 2^E lies in [2^19, 2^20)
            const float amax = finite ? half_bits_to_float(mx) : 0.f;
            const int ex = amax > 0.f ? int((__float_as_uint(amax) >> 23) & 0xffu) - 127 : 0;
            const int E = 19 - ex;
            const float up = finite ? __uint_as_float(uint32_t(E + 127) << 23) : 0.f;
            uint32_t ulo[4], uhi[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                ulo[t] = uint32_t(int(__builtin_rintf(half_bits_to_float(xp[t] & 0xffffu) * up)) + 0x808080);
                uhi[t] = uint32_t(int(__builtin_rintf(half_bits_to_float(xp[t] >> 16) * up)) + 0x808080);
            }
            uint32_t l0, l1, l2, h0, h1, h2;
            byte_planes(ulo, l0, l1, l2);
            byte_planes(uhi, h0, h1, h2);
            const uint32_t off = 16 * wd + 8 * hp;
            *reinterpret_cast<uint2_t *>(dig + 0 * N + off) = uint2_t{l0, h0};
            *reinterpret_cast<uint2_t *>(dig + 1 * N + off) = uint2_t{l1, h1};
            *reinterpret_cast<uint2_t *>(dig + 2 * N + off) = uint2_t{l2, h2};
            if ((tid & 3) == 0)
                sbs[tid >> 2] = finite ? __uint_as_float(uint32_t(127 - E) << 23) : __builtin_nanf("");
        }
        __syncthreads();

        // -- MFMA over the wavefront's 16 rows x 1024 ------------------------------
        const int ai = l & 15;  // this lane's A row
        const bool data = (ai >> 2) == g && (ai & 3) < 3;
        const uint8_t *abase = dig + (data ? (ai & 3) * N + kWaveK * kq + 64 * g : 3 * N);
        const uint32_t hbg = hbw >> (2 * g), abg = abw >> (2 * g);
        const uint32_t scg[4] = {scv.x >> (8 * g), scv.y >> (8 * g), scv.z >> (8 * g), scv.w >> (8 * g)};
        acc = 0.f;
        int4_t Dp[2];
#pragma unroll
        for (int s = 0; s <= SBW; ++s) {
            int4_t D[2];
            if (s < SBW) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t pool = (bit_mask(abg, 8 * s + h) & (kV8Shift ^ kV8Base)) ^ kV8Base;
                    D[h] = int4_t{0, 0, 0, 0};
#pragma unroll
                    for (int j = 2 * h; j < 2 * h + 2; ++j) {
                        const int4_t A =
                            __builtin_bit_cast(int4_t, *reinterpret_cast<const uint4_t *>(abase + 256 * s + 16 * j));
                        D[h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, word_to_v8(q[s][j], pool), D[h], 0, 0, 0);
                    }
                }
            }
            if (s > 0) {  // fold the previous super-block while this one's MFMAs run
                const int sp = s - 1;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int sint = Dp[h].x + (Dp[h].y << 8) + (Dp[h].z << 16);
                    const float up = sbs[8 * (SBW * kq + sp) + 2 * g + h];
                    const int idx = int(((scg[sp] >> (4 * h)) & 15u) | (((hbg >> (8 * sp + h)) & 1u) << 4)) - 16;
                    acc = fmaf(float(sint), float(idx) * up, acc);
                }
            }
            if (s < SBW) { Dp[0] = D[0]; Dp[1] = D[1]; }
        }
        acc *= half_bits_to_float(dvb);
    }
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    if (g == 0) part[kq][16 * tile + n] = acc;
    __syncthreads();
    if (tid < kGroupRows) {
        float sum = 0.f;
#pragma unroll
        for (int k = 0; k < KS; ++k) sum += part[k][tid];
        ygroup[tid] = uint16_t(float_to_half_bits(sum));
    }
}

template <bool FLOOR>
int launch_gemv_mfma(int64_t n, const Gemv2Args &a, uint32_t mats, hipStream_t st) {
    const dim3 grid{a.out_features / kGroupRows, mats};
    if (n == 4096)
        hipLaunchKernelGGL((gemv_mfma_iq2ks<4096, FLOOR>), grid, dim3{Gemv2Shape<4096>::THREADS}, 0, st, a);
    else
        hipLaunchKernelGGL((gemv_mfma_iq2ks<2048, FLOOR>), grid, dim3{Gemv2Shape<2048>::THREADS}, 0, st, a);
    return record_launch(hipGetLastError());
}

// Called by the GEMV entry points for IQ2_KS when out_features is a multiple
// of the workgroup's 32 rows; returns -1 when this path does not apply.
int gemv_mfma_dispatch(bool floor, int member, int64_t n, int64_t out, int64_t num_experts, const void *x,
                       const void *const *streams, const uint32_t *sel, uint32_t pairs_per_row, uint32_t mats,
                       void *y, hipStream_t st) {
    if (member != IQK_MEMBER_IQ2_KS || out % kGroupRows) return -1;
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
