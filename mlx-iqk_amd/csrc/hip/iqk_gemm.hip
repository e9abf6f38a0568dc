// Sorted grouped GEMM for the prefill contraction (gfx950 fp16 MFMA).
//
// Reference: the prefill route's mx.gather_mm over the dequantized experts
// with sorted_indices=True (src/mlx_iqk/nn.py:221-238; mlx 0.31.2, not
// vendored).  y[p] = x[row(p)] @ W[group(p)]^T for every slot p, fp16
// operands, f32 accumulation, one fp16 rounding of each output.
//
// Work list.  Slots are sorted by group; a group of c slots needs ceil(c/BM)
// M-tiles.  Block (t, n) finds the group owning M-tile t with an in-block scan
// of the group sizes, so the launch needs no host-side knowledge of the
// routing (no device->host sync) and no workspace; the grid is sized for the
// worst case ceil(n_slots/BM) + n_groups M-tiles and surplus blocks exit.
//
// Tile.  256 threads, four wavefronts, BM x BN = 64 x 256; each wavefront
// owns a 64 x 64 sub-tile as 4 x 4 v_mfma_f32_16x16x32_f16 tiles.  Any
// out_features works: a lane's B row is its D column, so columns at or beyond
// out_features are neither loaded nor stored, lane by lane.  With both
// operands k-contiguous (x rows and W rows), an MFMA operand fragment is 16
// contiguous bytes per lane, loaded straight from global memory and reused
// four times from registers.

#include "iqk_device.h"
#include "iqk_host.h"

namespace iqk {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

constexpr int kGemmBM = 64;
constexpr int kGemmBN = 256;

struct GemmArgs {
    const uint16_t *x;
    const uint16_t *w;
    const uint32_t *offs;
    const uint32_t *xr;
    const uint32_t *yr;
    uint16_t *y;
    uint32_t K, N, n_groups, n_slots, n_x_rows;
};

__device__ __forceinline__ half8_t load_frag(const uint16_t *p) {
    return __builtin_bit_cast(half8_t, *reinterpret_cast<const uint4_t *>(p));
}

__global__ __launch_bounds__(256) void grouped_gemm_kernel(GemmArgs a) {
    __shared__ TileScan ts;
    const int tid = threadIdx.x;
    uint32_t g, mtile;
    if (!find_mtile<kGemmBM>(a.offs, a.n_groups, blockIdx.x, ts, g, mtile)) return;  // surplus block

    // Offsets and row indices are device data: a slot outside [0, n_slots)
    // is never stored, and a row outside x is never read (zero operand; the
    // slot's output row is NaN).
    const uint32_t gend = min(a.offs[g + 1], a.n_slots);
    const uint32_t m0 = a.offs[g] + mtile * kGemmBM;
    const int wave = tid / 64, lane = tid % 64;
    const int lr = lane % 16, lk = 8 * (lane / 16);
    const uint32_t n0 = blockIdx.y * kGemmBN + wave * 64;

    const uint16_t *ap[4];
    bool av[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t p = m0 + 16 * i + lr;
        const uint32_t xrow = p < gend ? a.xr[p] : a.n_x_rows;
        av[i] = xrow < a.n_x_rows;
        ap[i] = a.x + size_t(av[i] ? xrow : 0u) * a.K + lk;
    }
    const uint16_t *bp[4];
    bool bv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        bv[j] = n0 + 16 * j + lr < a.N;  // this lane's column
        bp[j] = a.w + (size_t(g) * a.N + (bv[j] ? n0 + 16 * j + lr : 0u)) * a.K + lk;
    }

    float4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    const half8_t zero = {};
    half8_t af[4], bf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) af[i] = av[i] ? load_frag(ap[i]) : zero;
#pragma unroll
    for (int j = 0; j < 4; ++j) bf[j] = bv[j] ? load_frag(bp[j]) : zero;
    for (uint32_t k0 = 32; k0 <= a.K; k0 += 32) {
        half8_t an[4], bn[4];
        const bool more = k0 < a.K;
        if (more) {
#pragma unroll
            for (int i = 0; i < 4; ++i) an[i] = av[i] ? load_frag(ap[i] + k0) : zero;
#pragma unroll
            for (int j = 0; j < 4; ++j) bn[j] = bv[j] ? load_frag(bp[j] + k0) : zero;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        if (more) {
#pragma unroll
            for (int i = 0; i < 4; ++i) { af[i] = an[i]; bf[i] = bn[i]; }
        }
    }

    // D layout: lane holds rows 4*(lane/16) + r of column lane%16.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t p = m0 + 16 * i + 4 * (lane / 16) + r;
            if (p >= gend) continue;
            const uint32_t yrow = a.yr ? a.yr[p] : p;
            if (yrow >= a.n_slots) continue;
            const bool real = a.xr[p] < a.n_x_rows;  // else the row is NaN
            uint16_t *yp = a.y + size_t(yrow) * a.N + n0 + lr;  // only columns with bv[j] are stored
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (bv[j]) yp[16 * j] = real ? uint16_t(float_to_half_bits(acc[i][j][r])) : kHalfNaN;
        }
    }
}

}  // namespace iqk

extern "C" int iqk_grouped_gemm(int64_t in_features, int64_t out_features, int64_t n_groups, int64_t n_slots,
                                const void *x, int64_t n_x_rows, const void *w, const uint32_t *group_offsets,
                                const uint32_t *x_rows, const uint32_t *y_rows, void *y, void *stream) {
    using namespace iqk;
    if (in_features <= 0 || in_features % 32 || in_features > (int64_t(1) << 20)) return IQK_ERR_GEOMETRY;
    if (out_features <= 0 || out_features > (int64_t(1) << 20)) return IQK_ERR_GEOMETRY;
    if (n_groups < 0 || n_groups > (int64_t(1) << 20) || n_slots < 0 || n_slots > (int64_t(1) << 30))
        return IQK_ERR_ARGUMENT;
    if (n_x_rows < 0 || n_x_rows > 0xffffffffll) return IQK_ERR_ARGUMENT;
    if (n_groups == 0 || n_slots == 0) return IQK_OK;
    if (!x || !w || !group_offsets || !x_rows || !y) return IQK_ERR_ARGUMENT;
    GemmArgs a;
    a.x = static_cast<const uint16_t *>(x);
    a.w = static_cast<const uint16_t *>(w);
    a.offs = group_offsets;
    a.xr = x_rows;
    a.yr = y_rows;
    a.y = static_cast<uint16_t *>(y);
    a.K = uint32_t(in_features);
    a.N = uint32_t(out_features);
    a.n_groups = uint32_t(n_groups);
    a.n_slots = uint32_t(n_slots);
    a.n_x_rows = uint32_t(n_x_rows);
    const uint64_t mtiles = (uint64_t(n_slots) + kGemmBM - 1) / kGemmBM + uint64_t(n_groups);
    if (mtiles > 0x7fffffffull) return IQK_ERR_ARGUMENT;
    const dim3 grid{uint32_t(mtiles), uint32_t((out_features + kGemmBN - 1) / kGemmBN)}, block{256};
    hipLaunchKernelGGL(grouped_gemm_kernel, grid, block, 0, as_stream(stream), a);
    return record_launch(hipGetLastError());
}
