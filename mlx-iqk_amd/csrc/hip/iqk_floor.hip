// The pure byte-stream floor: the time one dispatch needs to read a given
// number of contiguous bytes from HBM, with nothing else in the way -- no
// expert-id read before the first request, no decode, no scattered rows.  A
// decode dispatch is priced against it beside its own deleted-decode floor
// (which keeps the decode's load set, expert-id read included).
//
// Each wavefront reads 4 KiB: every lane issues its four 16-byte loads (lane
// l, load i at byte 16 (64 i + l) of the wavefront's span, so each load
// instruction covers 1 KiB contiguously) before it folds any of them, and the
// folded words reach the output through a wavefront sum, so no load can be
// dropped.

#include "iqk_device.h"
#include "iqk_host.h"

namespace iqk {

constexpr int kStreamThreads = 256;
constexpr uint64_t kStreamWaveBytes = 4096;

__global__ __launch_bounds__(kStreamThreads) void stream_floor_kernel(const uint4_t *src, uint64_t n16,
                                                                      uint32_t *out) {
    const uint64_t wave = uint64_t(blockIdx.x) * (kStreamThreads / 64) + threadIdx.x / 64;
    const uint64_t base = wave * (kStreamWaveBytes / 16) + (threadIdx.x & 63);
    uint4_t v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint64_t idx = base + 64 * i;
        v[i] = idx < n16 ? src[idx] : uint4_t{0u, 0u, 0u, 0u};
    }
    uint32_t h = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) h += (2u * i + 3u) * (v[i].x + 3u * v[i].y + 5u * v[i].z + 7u * v[i].w);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) h += __shfl_xor(h, off, 64);
    if ((threadIdx.x & 63) == 0 && wave * kStreamWaveBytes < n16 * 16) out[wave] = h;
}

// The same stream with more bytes in flight: each lane issues L (4, 8 or 16)
// 16-byte loads before it folds any, so a wavefront requests L KiB at once,
// and the wavefronts stride over the span (one chunk of L KiB a wavefront per
// pass; with fewer wavefronts than chunks, each takes every `stride`-th).
template <int L>
__global__ __launch_bounds__(kStreamThreads) void stream_floor_wide_kernel(const uint4_t *src, uint64_t n16,
                                                                           uint64_t chunks, uint32_t *out) {
    const uint64_t wave = uint64_t(blockIdx.x) * (kStreamThreads / 64) + threadIdx.x / 64;
    const uint64_t stride = uint64_t(gridDim.x) * (kStreamThreads / 64);
    uint32_t h = 0;
    for (uint64_t c = wave; c < chunks; c += stride) {  // uniform per wavefront
        const uint64_t base = c * (64 * L) + (threadIdx.x & 63);
        uint4_t v[L];
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const uint64_t idx = base + 64 * i;
            v[i] = idx < n16 ? src[idx] : uint4_t{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < L; ++i) h += (2u * i + 3u) * (v[i].x + 3u * v[i].y + 5u * v[i].z + 7u * v[i].w);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) h += __shfl_xor(h, off, 64);
    if ((threadIdx.x & 63) == 0) out[wave] = h;
}

}  // namespace iqk

extern "C" int iqk_stream_floor_wide(const void *src, uint64_t bytes, int loads_per_lane, uint64_t max_waves,
                                     uint32_t *out, void *stream) {
    using namespace iqk;
    if (bytes == 0) return IQK_OK;
    if (!src || !out || bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16) return IQK_ERR_ARGUMENT;
    if (loads_per_lane != 4 && loads_per_lane != 8 && loads_per_lane != 16) return IQK_ERR_ARGUMENT;
    const uint64_t chunk = 1024 * uint64_t(loads_per_lane);  // bytes a wavefront requests at once
    const uint64_t chunks = (bytes + chunk - 1) / chunk;
    const uint64_t waves = max_waves ? (chunks < max_waves ? chunks : max_waves) : chunks;
    const uint64_t blocks = (waves + kStreamThreads / 64 - 1) / (kStreamThreads / 64);
    if (blocks > 0x7fffffffull) return IQK_ERR_ARGUMENT;
    const auto n16 = bytes / 16;
    const auto *s16 = static_cast<const uint4_t *>(src);
    switch (loads_per_lane) {
        case 4:
            hipLaunchKernelGGL(stream_floor_wide_kernel<4>, dim3{uint32_t(blocks)}, dim3{kStreamThreads}, 0,
                               as_stream(stream), s16, n16, chunks, out);
            break;
        case 8:
            hipLaunchKernelGGL(stream_floor_wide_kernel<8>, dim3{uint32_t(blocks)}, dim3{kStreamThreads}, 0,
                               as_stream(stream), s16, n16, chunks, out);
            break;
        default:
            hipLaunchKernelGGL(stream_floor_wide_kernel<16>, dim3{uint32_t(blocks)}, dim3{kStreamThreads}, 0,
                               as_stream(stream), s16, n16, chunks, out);
    }
    return record_launch(hipGetLastError());
}

extern "C" int iqk_stream_floor(const void *src, uint64_t bytes, uint32_t *out, void *stream) {
    using namespace iqk;
    if (bytes == 0) return IQK_OK;
    if (!src || !out || bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16) return IQK_ERR_ARGUMENT;
    const uint64_t waves = (bytes + kStreamWaveBytes - 1) / kStreamWaveBytes;
    const uint64_t blocks = (waves + kStreamThreads / 64 - 1) / (kStreamThreads / 64);
    if (blocks > 0x7fffffffull) return IQK_ERR_ARGUMENT;
    hipLaunchKernelGGL(stream_floor_kernel, dim3{uint32_t(blocks)}, dim3{kStreamThreads}, 0, as_stream(stream),
                       static_cast<const uint4_t *>(src), bytes / 16, out);
    return record_launch(hipGetLastError());
}
