// Device-side helpers shared by the routed-expert kernels (gfx950 / CDNA4).
#ifndef IQK_DEVICE_H
#define IQK_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace iqk {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));

enum Member : int { IQ2_KS = 0, IQ2_K = 1, IQ1_S_R4 = 2 };

constexpr uint16_t kHalfNaN = 0x7e00;

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
    return float(__builtin_bit_cast(half_t, uint16_t(bits)));
}

// Round-to-nearest-even float -> fp16 bits (v_cvt_f16_f32 under the default
// round mode; never the round-toward-zero pack).
__device__ __forceinline__ uint32_t float_to_half_bits(float f) {
    return uint32_t(__builtin_bit_cast(uint16_t, half_t(f)));
}

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// fp32 += a.x*b.x + a.y*b.y over fp16 pairs (v_dot2_f32_f16).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c, false);
}

__device__ __forceinline__ uint4_t load_u4(const void *p) { return *reinterpret_cast<const uint4_t *>(p); }

// Wavefront transposed reduction.  Each lane holds R partial sums (one per
// output row) over lanes that share one row group; after log2(R) exchange
// steps each lane holds R=1 value: the full sum of one row over the lanes
// of its group.  `first` is the highest lane-offset to reduce over, `last`
// the lowest; lanes that differ only in offsets >= `first`*2 are separate
// groups and are never mixed.  The row a lane ends up holding is the bit
// pattern of its lane id at the transposed offsets (see row_of_lane).
template <int R>
struct TransposeReduce {
    template <int OFF>
    __device__ __forceinline__ static void step(float *v, int lane) {
        constexpr int half = R / 2;
        const bool upper = (lane & OFF) != 0;
#pragma unroll
        for (int i = 0; i < half; ++i) {
            const float keep = upper ? v[i + half] : v[i];
            const float send = upper ? v[i] : v[i + half];
            v[i] = keep + __shfl_xor(send, OFF);
        }
    }
};

__device__ __forceinline__ int lane_id() { return int(__lane_id()); }

// Shared memory of the grouped work-list scan.
struct TileScan {
    uint32_t scan[4];  // the scanning wavefronts' totals
    uint32_t group, mtile;
};

// The number of M-tiles of the work list (sum over groups of ceil(size / BM)),
// by the same in-block scan as find_mtile; the same value in every thread.
template <int BM, int THREADS = 256>
__device__ __forceinline__ uint32_t count_mtiles(const uint32_t *offs, uint32_t n_groups, TileScan &ts) {
    static_assert(THREADS >= 256, "the first 256 threads scan");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t total = 0;
    for (uint32_t base = 0; base < n_groups; base += 256) {
        const uint32_t g = base + tid;
        uint32_t cnt = 0;
        if (tid < 256 && g < n_groups) cnt = (offs[g + 1] - offs[g] + BM - 1) / BM;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off, 64);
        if (tid < 256 && lane == 0) ts.scan[wave] = cnt;
        __syncthreads();
        total += ts.scan[0] + ts.scan[1] + ts.scan[2] + ts.scan[3];
        __syncthreads();  // the next round rewrites the totals
    }
    return total;
}

// The (group, M-tile) of work item t for a block of THREADS >= 256 threads
// (the first 256 scan): group g of the
// sorted slot ranges [offs[g], offs[g+1]) contributes ceil(size / BM)
// M-tiles, in group order.  An in-block scan of the group sizes, so a launch
// needs no host-side knowledge of the routing.  Returns false (uniformly)
// when t lies beyond the last M-tile.
template <int BM, int THREADS = 256>
__device__ __forceinline__ bool find_mtile(const uint32_t *offs, uint32_t n_groups, uint32_t t, TileScan &ts,
                                           uint32_t &group, uint32_t &mtile) {
    static_assert(THREADS >= 256, "the first 256 threads scan");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) ts.group = 0xffffffffu;
    uint32_t carry = 0;
    for (uint32_t base = 0; base < n_groups; base += 256) {
        const uint32_t g = base + tid;
        uint32_t cnt = 0;
        if (tid < 256 && g < n_groups) {
            const uint32_t c = offs[g + 1] - offs[g];
            cnt = (c + BM - 1) / BM;
        }
        // inclusive prefix within the wavefront, then the four wavefront
        // totals through LDS
        uint32_t incl = cnt;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t up = __shfl_up(incl, off, 64);
            if (lane >= off) incl += up;
        }
        if (tid < 256 && lane == 63) ts.scan[wave] = incl;
        __syncthreads();  // also orders tid 0's reset of ts.group before any match below
        uint32_t before = carry;
        for (int w = 0; w < wave && w < 4; ++w) before += ts.scan[w];
        incl += before;
        const uint32_t excl = incl - cnt;
        if (tid < 256 && cnt && t >= excl && t < incl) {
            ts.group = g;
            ts.mtile = t - excl;
        }
        carry += ts.scan[0] + ts.scan[1] + ts.scan[2] + ts.scan[3];
        __syncthreads();  // the next round rewrites the totals
    }
    __syncthreads();
    group = ts.group;
    mtile = ts.mtile;
    return group != 0xffffffffu;
}

}  // namespace iqk

#endif  // IQK_DEVICE_H
