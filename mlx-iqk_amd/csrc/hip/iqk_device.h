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

}  // namespace iqk

#endif  // IQK_DEVICE_H
