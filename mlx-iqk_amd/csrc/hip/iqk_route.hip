// The prefill route's pair grouping on the device: token-expert pairs ->
// expert-sorted slots, in one launch.
//
// Reference: the sorted prefill hands mx.gather_mm pairs sorted by expert
// (mlx_lm's _gather_sort, src/mlx_iqk/nn.py:221-238, sorted_indices=True)
// and gather_mm groups them by rhs index.  Here the grouping is one kernel
// whose outputs are exactly what the prefill kernels take: group offsets in
// slots, and each slot's activation row and output row.
//
// One workgroup of 1024 threads, everything in LDS (no workspace).  A pass
// loads 16 ids a thread at once (16384 pairs: one memory latency), kept in
// registers for both phases, and takes them 1024 at a time (a batch);
// within a wavefront the lanes holding one expert
// id find each other by ballots over the id bits (an id >= num_experts counts
// for expert 0: its slots keep an activation row past x, so the prefill
// kernels answer them with NaN rows and read nothing), and the lowest such
// lane speaks for all of them.
//   1. histogram: one LDS atomic per (wavefront, expert) of a batch;
//   2. an exclusive scan of the counts -> group offsets and per-expert cursors;
//   3. a stable scatter: each wavefront posts its per-expert counts of the
//      batch in a byte table, a pair's slot is its expert's cursor + the
//      counts of the wavefronts before it + its rank among its wavefront's
//      lanes, and the cursors then advance by the batch's counts.  Pairs keep
//      their order within an expert, so the slot lists are the same on every
//      call; three barriers a batch.

#include "iqk_device.h"
#include "iqk_host.h"

namespace iqk {

constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / 64;
constexpr int kRouteMaxExperts = 4096;        // LDS counters; 12 id bits
constexpr int kRouteIdBits = 12;
constexpr int kRoutePer = 16;                  // ids a thread holds
constexpr uint32_t kRouteSpan = kRoutePer * kRouteThreads;  // pairs a pass holds

struct RouteArgs {
    const uint32_t *ids;
    uint32_t *offs;
    uint32_t *xr;
    uint32_t *yr;
    uint32_t P, E, M, ppx, n_x_rows;
};

// The lanes of this wavefront that hold e (among the `live` ones).
__device__ __forceinline__ uint64_t same_lanes(uint32_t e, bool live) {
    uint64_t same = __ballot(live);
#pragma unroll
    for (int b = 0; b < kRouteIdBits; ++b) {
        const uint64_t ones = __ballot((e >> b) & 1u);
        same &= ((e >> b) & 1u) ? ones : ~ones;
    }
    return same;
}

__global__ __launch_bounds__(kRouteThreads) void route_kernel(RouteArgs a) {
    __shared__ uint32_t cur[kRouteMaxExperts];
    __shared__ uint8_t wcnt[kRouteWaves][kRouteMaxExperts];  // a batch's counts per wavefront (<= 64)
    __shared__ uint32_t wtot[kRouteWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t below = (uint64_t(1) << lane) - 1u;

    for (uint32_t e = tid; e < a.E; e += kRouteThreads) {
        cur[e] = 0;
#pragma unroll
        for (int w = 0; w < kRouteWaves; ++w) wcnt[w][e] = 0;
    }
    // ids of pairs span + 1024 i + tid, i < kRoutePer (past P: none)
    uint32_t id[kRoutePer];
    const auto load_span = [&](uint32_t span) {
#pragma unroll
        for (int i = 0; i < kRoutePer; ++i) {
            const uint32_t p = span + uint32_t(kRouteThreads * i + tid);
            id[i] = p < a.P ? a.ids[p] : 0u;
        }
    };
    __syncthreads();
    for (uint32_t span = 0; span < a.P; span += kRouteSpan) {
        load_span(span);
#pragma unroll
        for (int i = 0; i < kRoutePer; ++i) {
            const uint32_t p = span + uint32_t(kRouteThreads * i + tid);
            const bool live = p < a.P;
            const uint32_t e = id[i] < a.E ? id[i] : 0u;
            const uint64_t same = same_lanes(e, live);
            if (live && (same & below) == 0) atomicAdd(&cur[e], uint32_t(__popcll(same)));
        }
    }
    __syncthreads();

    // exclusive scan: thread t owns experts 4t .. 4t+3
    uint32_t c[4], sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t e = 4 * uint32_t(tid) + i;
        c[i] = e < a.E ? cur[e] : 0u;
        sum += c[i];
    }
    uint32_t incl = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t up = __shfl_up(incl, off, 64);
        if (lane >= off) incl += up;
    }
    if (lane == 63) wtot[wave] = incl;
    __syncthreads();
    uint32_t before = incl - sum;
    for (int w = 0; w < wave; ++w) before += wtot[w];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t e = 4 * uint32_t(tid) + i;
        if (e < a.E) {
            cur[e] = before;
            a.offs[e] = before * a.M;
        }
        before += c[i];
    }
    if (tid == 0) a.offs[a.E] = a.P * a.M;
    __syncthreads();

    for (uint32_t span = 0; span < a.P; span += kRouteSpan) {
        if (a.P > kRouteSpan) load_span(span);  // one span: the ids are still held
#pragma unroll
        for (int i = 0; i < kRoutePer; ++i) {
            if (span + uint32_t(kRouteThreads * i) >= a.P) break;  // uniform
            const uint32_t p = span + uint32_t(kRouteThreads * i + tid);
            const bool live = p < a.P;
            const bool valid = id[i] < a.E;
            const uint32_t e = valid ? id[i] : 0u;
            const uint64_t same = same_lanes(e, live);
            const uint32_t rank = __popcll(same & below);
            const bool leader = live && rank == 0;
            if (leader) wcnt[wave][e] = uint8_t(__popcll(same));
            __syncthreads();
            uint32_t slot = 0;
            if (live) {
                slot = cur[e] + rank;
                for (int w = 0; w < wave; ++w) slot += wcnt[w][e];
            }
            __syncthreads();  // every cursor and count read before any changes
            if (leader) {
                atomicAdd(&cur[e], uint32_t(__popcll(same)));
                wcnt[wave][e] = 0;
            }
            if (live) {
                const uint32_t xrow = valid ? (p / a.ppx) * a.M : a.n_x_rows;
                for (uint32_t r = 0; r < a.M; ++r) {
                    a.yr[slot * a.M + r] = p * a.M + r;
                    a.xr[slot * a.M + r] = valid ? xrow + r : a.n_x_rows;
                }
            }
            __syncthreads();  // cursors advanced, counts cleared for the next batch
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
    if (n_pairs * rows_per_pair >= (int64_t(1) << 31) || n_x_rows >= (int64_t(1) << 31)) return IQK_ERR_ARGUMENT;
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
    hipLaunchKernelGGL(route_kernel, dim3{1}, dim3{kRouteThreads}, 0, as_stream(stream), a);
    return record_launch(hipGetLastError());
}
