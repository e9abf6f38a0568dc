// Stacked-expert dequant producer and its floor (gfx950).
//
// Reference: the Metal dequantization (src/mlx_iqk/kernels.py:580-676,
// launched by src/mlx_iqk/nn.py:155-169) and its floor
// (bench/floors.py:179-220).
//
// One thread reconstructs 64 consecutive weights of one row.  Stores go out
// coalesced: each thread stages its 128 bytes (and where they go) in LDS, and
// after one barrier lane l of a wavefront stores the 16-byte chunks 64u + l
// of the wavefront's 8 KiB, so every store instruction writes one contiguous
// KiB (a thread storing its own 128 bytes would give 16 bytes per 128-byte
// line per instruction: about 3.5 TB/s instead of 5.6 TB/s on MI355X).
// Bit-exactness: every weight is the CPU dequantizer's f32
// chain dl = d * float(index), y = dl * float(value), each product exact, then
// one round-to-nearest-even conversion.  Because a sub-block has only four
// distinct values, the four fp16 results are formed once per sub-block and
// each pair of output weights is one v_perm_b32 from that 8-byte table; the
// table entry for a code is exactly the value the per-weight chain would
// produce.
//
// The producer writes the experts the caller selects into compact slots
// (slot_of_expert), so a prefill reconstructs each routed expert once.

#include "iqk_device.h"
#include "iqk_host.h"
#include "iqk_pool.h"

#define IQK_GRID_STORAGE __constant__ static const __attribute__((aligned(16)))
#include "../iq1s_grid.h"

namespace iqk {

struct DequantArgs {
    const void *s0, *s1, *s2, *s3, *s4;
    const int32_t *slot_of_expert;
    uint32_t num_experts;
    uint32_t out_features;
    uint32_t row_start;  // first source row inside each expert
    uint32_t rows;       // rows per expert written: w[slot][0..rows)
    uint32_t n_slots;
    uint16_t *w;
};

// The stream words behind 64 weights of one row (IQ1_S_R4: q.x, q.y are the
// eight index bytes, hb the two qh words).
struct RawChunk {
    uint4_t q;
    uint32_t sc, hb, ab, dvb;
};

template <int MEMBER, int N>
__device__ __forceinline__ RawChunk load_chunk(const DequantArgs &a, uint64_t row, int lc) {
    RawChunk c{};
    if constexpr (MEMBER == IQ2_KS || MEMBER == IQ2_K) {
        c.q = load_u4(static_cast<const uint32_t *>(a.s0) + row * (N / 16) + 4 * lc);
        if constexpr (MEMBER == IQ2_KS) {
            c.sc = static_cast<const uint8_t *>(a.s1)[row * (N / 64) + lc];
            c.hb = static_cast<const uint8_t *>(a.s2)[row * (N / 256) + lc / 4];
            c.ab = static_cast<const uint8_t *>(a.s3)[row * (N / 256) + lc / 4];
            c.dvb = static_cast<const uint16_t *>(a.s4)[row];
        } else {
            c.sc = static_cast<const uint16_t *>(a.s1)[row * (N / 64) + lc];
            c.ab = static_cast<const uint8_t *>(a.s2)[row * (N / 128) + lc / 2];
            c.dvb = static_cast<const uint16_t *>(a.s3)[row * (N / 256) + lc / 4];
        }
    } else {
        const uint2_t q = *reinterpret_cast<const uint2_t *>(static_cast<const uint32_t *>(a.s0) + row * (N / 32) + 2 * lc);
        c.q = uint4_t{q.x, q.y, 0u, 0u};
        c.hb = *reinterpret_cast<const uint32_t *>(static_cast<const uint16_t *>(a.s1) + row * (N / 32) + 2 * lc);
        c.dvb = static_cast<const uint16_t *>(a.s2)[row];
    }
    return c;
}

// The 64 weights of a chunk as 32 fp16 pairs (the floor: a hash of the loaded
// words in every pair).
template <int MEMBER, bool FLOOR>
__device__ __forceinline__ void decode_chunk(const RawChunk &c, int lc, const uint16_t *grid, uint32_t *out) {
    if constexpr (FLOOR) {
        const uint32_t iacc = c.q.x + 3u * c.q.y + 5u * c.q.z + 7u * c.q.w + 59u * c.sc + 61u * c.hb + 71u * c.ab +
                              67u * c.dvb;
        const uint32_t hv = float_to_half_bits(float(iacc & 0xffu));
#pragma unroll
        for (int i = 0; i < 32; ++i) out[i] = hv | (hv << 16);
    } else if constexpr (MEMBER == IQ2_KS || MEMBER == IQ2_K) {
        const float d = half_bits_to_float(c.dvb);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t idx, alpha;
            if constexpr (MEMBER == IQ2_KS) {  // sub-block 2*lc + w/2 (32 weights)
                const int t = w / 2, bsh = 2 * (lc % 4);
                idx = ((c.sc >> (4 * t)) & 15u) | (((c.hb >> (bsh + t)) & 1u) << 4);
                idx -= 16u;
                alpha = (c.ab >> (bsh + t)) & 1u;
            } else {  // sub-block 4*lc + w (16 weights)
                idx = ((c.sc >> (4 * w)) & 15u) - 8u;
                alpha = (c.ab >> (4 * (lc % 2) + w)) & 1u;
            }
            const float dl = d * float(int(idx));
            const float v0 = alpha ? -26.f : -31.f, v1 = alpha ? -8.f : -13.f;
            const float v2 = alpha ? 6.f : 1.f, v3 = alpha ? 22.f : 17.f;
            const Pool p = make_pool(dl, v0, v1, v2, v3);
            expand_word(c.q[w], p, out + 8 * w);
        }
    } else {
        const float d = half_bits_to_float(c.dvb);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const uint32_t qw = c.q[b];
            const uint32_t h = (c.hb >> (16 * b)) & 0xffffu;
            const float dl = d * float(int(2 * ((h >> 12) & 7u) + 1));
            const float sh = (h & 0x8000u) ? -0.125f : 0.125f;
            // grid field f in {0,1,2} decodes to f - 1; field 3 never occurs
            const Pool p = make_pool(dl, -1.f + sh, 0.f + sh, 1.f + sh, 2.f + sh);
            const uint32_t c0 = grid[(qw & 0xffu) | ((h & 7u) << 8)];
            const uint32_t c1 = grid[((qw >> 8) & 0xffu) | (((h >> 3) & 7u) << 8)];
            const uint32_t c2 = grid[((qw >> 16) & 0xffu) | (((h >> 6) & 7u) << 8)];
            const uint32_t c3 = grid[(qw >> 24) | (((h >> 9) & 7u) << 8)];
            expand_word(c0 | (c1 << 16), p, out + 16 * b);
            expand_word(c2 | (c3 << 16), p, out + 16 * b + 8);
        }
    }
}

// LDS slot of one thread: its 128 output bytes, its destination (null when
// the thread has nothing to write) and 8 bytes of padding, so the slots of
// consecutive lanes start 36 banks apart.
constexpr int kStageDwords = 36;

template <int MEMBER, int N, bool FLOOR>
__global__ __launch_bounds__(256) void dequant_kernel(DequantArgs a) {
    constexpr int TPR = N / 64;  // threads per row
    __shared__ __attribute__((aligned(16))) uint16_t grid[MEMBER == IQ1_S_R4 ? IQK_IQ1S_GRID_SIZE : 8];
    __shared__ __attribute__((aligned(16))) uint32_t stage[256 * kStageDwords];
    static_assert(IQK_IQ1S_GRID_SIZE * 2 == 256 * 16, "one 16-byte grid chunk per thread");
    // IQ1_S_R4's grid load goes out before the stream loads: loads return in
    // order, so its LDS store and the block barrier below complete while the
    // stream words are still in flight.
    uint4_t gridv{};
    if constexpr (MEMBER == IQ1_S_R4 && !FLOOR) gridv = reinterpret_cast<const uint4_t *>(iqk_iq1s_grid_codes)[threadIdx.x];
    const uint64_t gid = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t lin = gid / TPR;  // (expert, range row)
    const int lc = int(gid % TPR);
    const uint32_t expert = uint32_t(lin / a.rows);
    const int32_t slot = expert < a.num_experts ? (a.slot_of_expert ? a.slot_of_expert[expert] : int32_t(expert)) : -1;
    const bool valid = slot >= 0 && uint32_t(slot) < a.n_slots;
    uint32_t out[32];
    uint16_t *dst = nullptr;
    RawChunk raw{};
    if (valid) {
        const uint32_t r = uint32_t(lin - uint64_t(expert) * a.rows);
        const uint64_t row = uint64_t(expert) * a.out_features + a.row_start + r;  // stacked source row
        dst = a.w + (uint64_t(slot) * a.rows + r) * N + 64 * lc;
        raw = load_chunk<MEMBER, N>(a, row, lc);
    }
    if constexpr (MEMBER == IQ1_S_R4 && !FLOOR) {
        reinterpret_cast<uint4_t *>(grid)[threadIdx.x] = gridv;
        __syncthreads();
    }
    if (valid) decode_chunk<MEMBER, FLOOR>(raw, lc, grid, out);
    uint32_t *mine = stage + threadIdx.x * kStageDwords;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        reinterpret_cast<uint4_t *>(mine)[i] = uint4_t{out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]};
    *reinterpret_cast<uint64_t *>(mine + 32) = reinterpret_cast<uint64_t>(dst);
    // A wavefront's stage is written and read by its own lanes, and LDS
    // accesses of one wavefront complete in order: a wavefront-scope fence
    // (ordering for the compiler) replaces a block barrier, so no wavefront
    // waits for the others of its block.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // chunk c = 64u + l of this wavefront: part c % 8 of its thread c / 8
    const int l = threadIdx.x & 63;
    const uint32_t *wave_stage = stage + (threadIdx.x & ~63) * kStageDwords;
    // all eight chunks into distinct registers first: a store's data registers
    // are not reused while it is in flight, so the eight stores go out back to back
    uint4_t val[8];
    uint4_t *to[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const uint32_t *src = wave_stage + (8 * u + (l >> 3)) * kStageDwords;
        to[u] = reinterpret_cast<uint4_t *>(*reinterpret_cast<const uint64_t *>(src + 32));
        val[u] = reinterpret_cast<const uint4_t *>(src)[l & 7];
    }
    // Non-temporal: the stack is read back only by a later dispatch, so its
    // lines need not stay in cache (measured 3-6% faster than plain stores).
#pragma unroll
    for (int u = 0; u < 8; ++u)
        if (to[u]) __builtin_nontemporal_store(val[u], &to[u][l & 7]);
}

template <int MEMBER, bool FLOOR>
int launch_dequant(int64_t n, const DequantArgs &a, hipStream_t st) {
    const uint64_t threads = uint64_t(a.num_experts) * a.rows * uint64_t(n / 64);
    const uint64_t blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffffull) return IQK_ERR_GEOMETRY;
    const dim3 grid{uint32_t(blocks)}, block{256};
    if (n == 4096)
        hipLaunchKernelGGL((dequant_kernel<MEMBER, 4096, FLOOR>), grid, block, 0, st, a);
    else
        hipLaunchKernelGGL((dequant_kernel<MEMBER, 2048, FLOOR>), grid, block, 0, st, a);
    return record_launch(hipGetLastError());
}

// Every producer entry point: rows [row_start, row_start + rows) of each
// selected expert into w[slot][0..rows).
template <bool FLOOR>
int dequant_entry(int member, int64_t n, int64_t out, int64_t num_experts, const void *const *streams,
                  int n_streams, int64_t row_start, int64_t rows, const int32_t *slot_of_expert, int64_t n_slots,
                  void *w, void *stream) {
    const int g = iqk_check_dequant_geometry(member, n, out);
    if (g != IQK_OK) return g;
    if (row_start < 0 || rows <= 0 || row_start + rows > out) return IQK_ERR_GEOMETRY;
    if (!w || !streams_ok(streams, n_streams, member)) return IQK_ERR_ARGUMENT;
    if (num_experts <= 0 || num_experts > 0xffffffffll || n_slots < 0 || n_slots > 0xffffffffll)
        return IQK_ERR_ARGUMENT;
    if (!slot_of_expert && n_slots < num_experts) return IQK_ERR_ARGUMENT;
    if (n_slots == 0) return IQK_OK;
    DequantArgs a;
    a.s0 = streams[0]; a.s1 = streams[1]; a.s2 = streams[2];
    a.s3 = n_streams > 3 ? streams[3] : nullptr;
    a.s4 = n_streams > 4 ? streams[4] : nullptr;
    a.slot_of_expert = slot_of_expert;
    a.num_experts = uint32_t(num_experts);
    a.out_features = uint32_t(out);
    a.row_start = uint32_t(row_start);
    a.rows = uint32_t(rows);
    a.n_slots = uint32_t(n_slots);
    a.w = static_cast<uint16_t *>(w);
    hipStream_t st = as_stream(stream);
    switch (member) {
        case IQK_MEMBER_IQ2_KS: return launch_dequant<IQ2_KS, FLOOR>(n, a, st);
        case IQK_MEMBER_IQ2_K: return launch_dequant<IQ2_K, FLOOR>(n, a, st);
        default: return launch_dequant<IQ1_S_R4, FLOOR>(n, a, st);
    }
}

}  // namespace iqk

extern "C" {

int iqk_check_dequant_geometry(int member, int64_t n, int64_t out) {
    if (!iqk::member_ok(member)) return IQK_ERR_MEMBER;
    if (!iqk::width_sized(n)) return IQK_ERR_GEOMETRY;
    if (out <= 0 || out > (int64_t(1) << 24)) return IQK_ERR_GEOMETRY;
    return IQK_OK;
}

int iqk_dequant(int member, int64_t n, int64_t out, int64_t num_experts, const void *const *streams,
                int n_streams, const int32_t *slot_of_expert, int64_t n_slots, void *w, void *stream) {
    return iqk::dequant_entry<false>(member, n, out, num_experts, streams, n_streams, 0, out, slot_of_expert,
                                     n_slots, w, stream);
}

int iqk_dequant_rows(int member, int64_t n, int64_t out, int64_t num_experts, const void *const *streams,
                     int n_streams, int64_t row_start, int64_t rows, const int32_t *slot_of_expert, int64_t n_slots,
                     void *w, void *stream) {
    return iqk::dequant_entry<false>(member, n, out, num_experts, streams, n_streams, row_start, rows,
                                     slot_of_expert, n_slots, w, stream);
}

int iqk_dequant_floor(int member, int64_t n, int64_t out, int64_t num_experts, const void *const *streams,
                      int n_streams, const int32_t *slot_of_expert, int64_t n_slots, void *w, void *stream) {
    return iqk::dequant_entry<true>(member, n, out, num_experts, streams, n_streams, 0, out, slot_of_expert,
                                    n_slots, w, stream);
}

}  // extern "C"
