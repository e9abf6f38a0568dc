// The prefill route's pair grouping on the device: token-expert pairs ->
// expert-sorted slots, in one launch.
//
// Reference: the sorted prefill hands mx.gather_mm pairs sorted by expert
// (mlx_lm's _gather_sort, src/mlx_iqk/nn.py:221-238, sorted_indices=True)
// and gather_mm groups them by rhs index.  Here the grouping is one kernel
// whose outputs are exactly what the prefill kernels take: group offsets in
// slots, and each slot's activation row and output row.
//
// A pair's key is its expert id; an id >= num_experts keys as expert 0 (its
// slots keep an activation row past x, so the prefill kernels answer them with
// NaN rows and read nothing).  Expert e's slots are
//   [#{pairs keyed below e}, #{pairs keyed below e + 1}),
// its pairs in pair order (a stable counting sort).
//
// One workgroup per expert, so a launch spreads over the chip; no workspace.
// Its eight wavefronts each take a contiguous eighth of the pairs and hold
// their ids in registers (re-read from L2 only past 2048 pairs a wavefront):
//   1. each wavefront counts, by ballots, its pairs keyed below e and keyed e;
//   2. the eight totals through LDS give the group offset and each
//      wavefront's first slot (the offset + the e-pairs of the wavefronts
//      before it);
//   3. each wavefront with e-pairs writes them in order, a pair's slot being
//      its wavefront's next slot + its rank among the ballot's lanes.
// Every block reads the whole id list (4 bytes a pair from L2); the time is
// the two ballot passes over one wavefront's share, about P / 512 steps.

#include "iqk_device.h"
#include "iqk_host.h"

namespace iqk {

constexpr int kRouteThreads = 512;
constexpr int kRouteWaves = kRouteThreads / 64;
constexpr int kRouteMaxExperts = 4096;
constexpr int kRoutePer = 32;  // ids a lane holds per round
constexpr uint32_t kRouteRound = 64u * kRoutePer;  // pairs a wavefront holds

struct RouteArgs {
    const uint32_t *ids;
    uint32_t *offs;
    uint32_t *xr;
    uint32_t *yr;
    uint32_t P, E, M, ppx, n_x_rows;
};

__global__ __launch_bounds__(kRouteThreads) void route_kernel(RouteArgs a) {
    __shared__ uint32_t tot[2][kRouteWaves];  // per wavefront: pairs keyed below e, keyed e
    const uint32_t e = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t below = (uint64_t(1) << lane) - 1u;
    // wavefront w takes pairs [lo, hi): contiguous, in wavefront order
    const uint32_t share = (a.P + 64u * kRouteWaves - 1u) / (64u * kRouteWaves) * 64u;
    const uint32_t lo = min(a.P, uint32_t(wave) * share), hi = min(a.P, lo + share);

    // raw ids of pairs base + 64 i + lane; lanes past hi load pair hi - 1 and
    // are masked by `live` (only called with lo <= base < hi)
    uint32_t raw[kRoutePer];
    const auto load = [&](uint32_t base) {
#pragma unroll
        for (int i = 0; i < kRoutePer; ++i) raw[i] = a.ids[min(base + uint32_t(64 * i + lane), hi - 1u)];
    };

    uint32_t lt = 0, eq = 0;
    for (uint32_t base = lo; base < hi; base += kRouteRound) {
        load(base);
#pragma unroll
        for (int i = 0; i < kRoutePer; ++i) {
            const bool live = base + uint32_t(64 * i + lane) < hi;
            const uint32_t key = raw[i] < a.E ? raw[i] : 0u;
            lt += uint32_t(__popcll(__ballot(live && key < e)));
            eq += uint32_t(__popcll(__ballot(live && key == e)));
        }
    }
    if (lane == 0) {
        tot[0][wave] = lt;
        tot[1][wave] = eq;
    }
    __syncthreads();
    uint32_t first = 0, slot = 0;
#pragma unroll
    for (int w = 0; w < kRouteWaves; ++w) {
        first += tot[0][w];
        if (w < wave) slot += tot[1][w];
    }
    slot += first;
    if (threadIdx.x == 0) {
        a.offs[e] = first * a.M;
        if (e == a.E - 1u) a.offs[a.E] = a.P * a.M;
    }
    if (eq == 0) return;  // uniform: no e-pairs in this wavefront's share

    for (uint32_t base = lo; base < hi; base += kRouteRound) {
        if (hi - lo > kRouteRound) load(base);  // one round: the ids are still held
#pragma unroll
        for (int i = 0; i < kRoutePer; ++i) {
            const uint32_t p = base + uint32_t(64 * i + lane);
            const bool valid = raw[i] < a.E;
            const bool mine = p < hi && (valid ? raw[i] : 0u) == e;
            const uint64_t m = __ballot(mine);
            if (m == 0) continue;  // uniform
            if (mine) {
                const uint32_t s = (slot + uint32_t(__popcll(m & below))) * a.M;
                const uint32_t xrow = valid ? (p / a.ppx) * a.M : a.n_x_rows;
                for (uint32_t r = 0; r < a.M; ++r) {
                    a.yr[s + r] = p * a.M + r;
                    a.xr[s + r] = valid ? xrow + r : a.n_x_rows;
                }
            }
            slot += uint32_t(__popcll(m));
        }
    }
}

}  // namespace iqk

extern "C" int iqk_route(const uint32_t *ids, int64_t n_pairs, int64_t num_experts, int64_t rows_per_pair,
                         int64_t pairs_per_x_row, int64_t n_x_rows, uint32_t *group_offsets, uint32_t *x_rows,
                         uint32_t *y_rows, void *stream) {
    using namespace iqk;
    if (num_experts <= 0 || num_experts > kRouteMaxExperts) return IQK_ERR_ARGUMENT;
    if (n_pairs < 0 || rows_per_pair <= 0 || pairs_per_x_row <= 0 || n_x_rows < 0) return IQK_ERR_ARGUMENT;
    // each factor bounded first, so the products below cannot overflow
    constexpr int64_t kLim = int64_t(1) << 31;
    if (n_pairs >= kLim || rows_per_pair >= kLim || pairs_per_x_row >= kLim || n_x_rows >= kLim)
        return IQK_ERR_ARGUMENT;
    if (n_pairs * rows_per_pair >= kLim) return IQK_ERR_ARGUMENT;
    if (!group_offsets || (n_pairs && (!ids || !x_rows || !y_rows))) return IQK_ERR_ARGUMENT;
    // every activation row a valid pair names lies in x
    if (n_pairs && ((n_pairs - 1) / pairs_per_x_row + 1) * rows_per_pair > n_x_rows) return IQK_ERR_ARGUMENT;
    RouteArgs a;
    a.ids = ids;
    a.offs = group_offsets;
    a.xr = x_rows;
    a.yr = y_rows;
    a.P = uint32_t(n_pairs);
    a.E = uint32_t(num_experts);
    a.M = uint32_t(rows_per_pair);
    a.ppx = uint32_t(pairs_per_x_row);
    a.n_x_rows = uint32_t(n_x_rows);
    hipLaunchKernelGGL(route_kernel, dim3{uint32_t(num_experts)}, dim3{kRouteThreads}, 0, as_stream(stream), a);
    return record_launch(hipGetLastError());
}
