// Sorted grouped GEMM for the prefill contraction (gfx950 fp16 MFMA).
//
// Reference: the prefill route's mx.gather_mm over the dequantized experts
// with sorted_indices=True (src/mlx_iqk/nn.py:221-238; mlx 0.31.2, not
// vendored).  y[p] = x[row(p)] @ W[group(p)]^T for every slot p, fp16
// operands, f32 accumulation, one fp16 rounding of each output.
//
// The prefill's cost is streaming the fp16 weights (16 MiB per expert
// projection, each read once per 64-slot M-tile), so the kernel is shaped
// for HBM: a block keeps several steps of its weights in flight, and the
// M-tiles of one expert run on one XCD, back to back, so a weight block's
// second and later reads come from that XCD's L2.
//
// Work list.  Slots are sorted by group; a group of c slots needs ceil(c/BM)
// M-tiles.  A first in-block scan of the group sizes counts the M-tiles T
// (no host-side knowledge of the routing: no device->host sync, no
// workspace); XCD x (blocks b with b % 8 == x) takes M-tiles
// [x ceil(T/8), (x+1) ceil(T/8)) in order, each with all its column blocks
// one after another, so the column blocks of a tile share its activations in
// L2 and consecutive tiles of an expert share its weights.  A second scan
// finds the tile's group.  The grid is sized for the worst case
// ceil(n_slots/BM) + n_groups tiles; surplus blocks exit.
//
// Tile.  512 threads, eight wavefronts, BM x BN = 64 x 256; wavefront w owns
// weight rows 32w .. 32w+31 of the block (the columns of
// v_mfma_f32_32x32x16_f16) for both 32-slot row blocks; reduction steps of
// 64.  A tile with at most 32 real slots skips its second row block's MFMAs.
// Any out_features works: a lane's B row is its D column, so columns at or
// beyond out_features read an in-bounds row and are never stored.
//
// Two forms of the step loop:
// * grouped_gemm_lds_kernel (K a multiple of 64, the prefill's case): both
//   operands go from global memory straight into LDS (16-byte
//   global_load_lds_dwordx4), one load instruction moving 8 rows x 128
//   contiguous bytes, so it touches 8 cache lines.  Register loads in the
//   MFMA's layout (each lane its own weight row) touch 32 lines an
//   instruction, and measured ~15% slower on the Zipf prefill (996 against
//   849 us per projection) at the same bytes.  Each wavefront streams its
//   own 32 weight rows into four 32 KiB stages (three steps ahead, no
//   registers held), the activations go into three 8 KiB stages (two ahead),
//   and a lane stores chunk c of its row at c ^ (row / 2 % 8), so the MFMA
//   operand reads (16 rows, one chunk each) cover all 64 banks once.
// * grouped_gemm_kernel (any K a multiple of 32): register staging, the
//   step's activations copied to LDS, the weights loaded in the MFMA's layout
//   three steps ahead in four rotating register sets; the last step may end
//   past K (its upper half is zeroed).

#include <type_traits>

#include "iqk_device.h"
#include "iqk_host.h"

namespace iqk {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kGemmBM = 64;                   // slots per tile
constexpr int kGemmWaves = 8;
constexpr int kGemmThreads = 64 * kGemmWaves;
constexpr int kGemmBN = 32 * kGemmWaves;      // weight rows (output columns) per block
constexpr int kGemmBK = 64;                   // reduction elements per step
constexpr int kGemmU = kGemmBK / 16;          // MFMAs (16-wide k chunks) per step and row block
constexpr int kGemmAStride = 2 * kGemmBK + 16;  // LDS bytes per staged activation row
constexpr int kGemmAChunks = kGemmBK / 8;     // 16-byte activation chunks per row and step
constexpr int kGemmARows = kGemmThreads / kGemmAChunks;  // slot rows one staging pass covers
constexpr int kGemmAPer = kGemmBM / kGemmARows;          // staging passes (16-byte chunks a thread moves a step)
// Register sets per operand of grouped_gemm_kernel: loads run kGemmStages - 1
// steps ahead (on the 2048-token Zipf prefill, gate [2048 x 4096], two sets
// measured 1113 us, four 987 us; eight sets, or four of 128-wide steps, spill
// at 256 VGPRs).
constexpr int kGemmStages = 4;
static_assert(kGemmBM % kGemmARows == 0 && kGemmThreads % kGemmAChunks == 0, "whole staging passes");

struct GemmArgs {
    const uint16_t *x;
    const uint16_t *w;
    const uint32_t *offs;
    const uint32_t *xr;
    const uint32_t *yr;
    uint16_t *y;
    uint32_t K, N, n_groups, n_slots, n_x_rows;
};

// The general form: any K a multiple of 32 (the last step may end past K;
// its upper half is zeroed) and any step count.
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(2)))
void grouped_gemm_kernel(GemmArgs a) {
    __shared__ TileScan ts;
    __shared__ __attribute__((aligned(16))) uint8_t as[2][kGemmBM * kGemmAStride];
    // per slot of the tile: its output row, bit 31 set when its activations
    // are real (else the row is NaN), or kNoStore
    __shared__ uint32_t slot_dst[kGemmBM];
    constexpr uint32_t kNoStore = 0x7fffffffu;  // above any row (n_slots <= 2^30)

    const int tid = threadIdx.x;
    const uint32_t ncb = (a.N + kGemmBN - 1) / kGemmBN;  // column blocks
    const uint32_t tiles = count_mtiles<kGemmBM, kGemmThreads>(a.offs, a.n_groups, ts);
    const uint32_t per_xcd = (tiles + 7) / 8;
    const uint32_t xcd = blockIdx.x & 7u, j = blockIdx.x >> 3;
    if (j / ncb >= per_xcd) return;  // surplus block (uniform)
    const uint32_t tile = xcd * per_xcd + j / ncb, cblock = j % ncb;
    if (tile >= tiles) return;
    uint32_t g, mtile;
    if (!find_mtile<kGemmBM, kGemmThreads>(a.offs, a.n_groups, tile, ts, g, mtile)) return;

    // Offsets and row indices are device data: a slot outside [0, n_slots)
    // is never stored, and a row outside x is never read (zero operand; the
    // slot's output row is NaN).
    const uint32_t gend = min(a.offs[g + 1], a.n_slots);
    const uint32_t m0 = a.offs[g] + mtile * kGemmBM;
    const uint32_t n0 = cblock * kGemmBN;
    const uint32_t ksteps = (a.K + kGemmBK - 1) / kGemmBK;

    // activation staging: thread t moves 16 bytes (chunk t % C) of slot rows
    // t / C + R i a step (C chunks a row, R rows a pass, i < kGemmAPer)
    const int arow = tid / kGemmAChunks, achunk = tid % kGemmAChunks;
    // every load below reads an in-bounds address (a dead row reads row 0,
    // which exists: the entry point refuses an empty x)
    const uint16_t *asrc[kGemmAPer];
#pragma unroll
    for (int i = 0; i < kGemmAPer; ++i) {
        const int row = arow + kGemmARows * i;
        const uint32_t ap = m0 + uint32_t(row);
        const uint32_t xrow = ap < gend ? a.xr[ap] : a.n_x_rows;
        const bool alive = xrow < a.n_x_rows;
        asrc[i] = a.x + size_t(alive ? xrow : 0u) * a.K;
        if (achunk == 0) {  // one thread a slot: the epilogue's destination, read once
            uint32_t dst = kNoStore;
            if (ap < gend) {
                const uint32_t yrow = a.yr ? a.yr[ap] : ap;
                if (yrow < a.n_slots) dst = yrow | (alive ? 0x80000000u : 0u);
            }
            slot_dst[row] = dst;
        }
    }
    // A dead slot's activations feed only its own output row, which is never
    // stored (or stored as NaN), so they need no zeroing; elements past K
    // would feed every row and are zeroed.
    using AStage = uint4_t[kGemmAPer];
    const auto load_a = [&](uint32_t s, AStage &v) {
        s = min(s, ksteps - 1);
#pragma unroll
        for (int i = 0; i < kGemmAPer; ++i) {
            // the element offset in the row, clamped to its last 8 elements
            // (K >= 32, so K - 8 does not wrap): a chunk past K reads inside
            // its own row and is zeroed
            uint32_t k = s * kGemmBK + 8 * achunk;
            const bool live = k < a.K;
            k = min(k, a.K - 8);
            const uint4_t t = load_u4(asrc[i] + k);
            v[i] = live ? t : uint4_t{0u, 0u, 0u, 0u};
        }
    };
    const auto store_a = [&](int buf, const AStage &v) {
#pragma unroll
        for (int i = 0; i < kGemmAPer; ++i)
            *reinterpret_cast<uint4_t *>(as[buf] + (arow + kGemmARows * i) * kGemmAStride + 16 * achunk) = v[i];
    };

    // this lane's weight row: column n0 + 32 wave + l % 32; chunk 2u + h of a
    // step feeds MFMA u (lanes h = l / 32 hold its two k halves)
    const int wave = tid >> 6, l = tid & 63, ln = l & 31, h = l >> 5;
    const uint32_t col = n0 + 32 * wave + ln;
    const bool bv = col < a.N;
    const uint16_t *bsrc = a.w + (size_t(g) * a.N + (bv ? col : 0u)) * a.K + 8 * h;
    // a column past out_features reads column 0 and is never stored (a D
    // column depends on its own B column only), so it needs no zeroing
    const auto load_b = [&](uint32_t s, uint4_t (&b)[kGemmU]) {
        s = min(s, ksteps - 1);
#pragma unroll
        for (int u = 0; u < kGemmU; ++u) {
            uint32_t k = s * kGemmBK + 16 * u;
            const bool live = k + 8 * h < a.K;
            k = min(k, a.K - 8 * h - 8);
            const uint4_t v = load_u4(bsrc + k);
            b[u] = live ? v : uint4_t{0u, 0u, 0u, 0u};
        }
    };

    // ST register sets per operand rotate through the steps: step s computes
    // with B(s), issues the loads of step s + ST - 1 into the set step s - 1
    // freed, and stages A(s + 1) into LDS before its barrier, so every load
    // has ST - 1 steps to land and no set is copied.
    uint4_t bq[kGemmStages][kGemmU];
    AStage aq[kGemmStages];
#pragma unroll
    for (int i = 0; i + 1 < kGemmStages; ++i) {
        load_a(i, aq[i]);
        load_b(i, bq[i]);
    }
    store_a(0, aq[0]);
    __syncthreads();  // the first activations and the slot table are in LDS

    float16_t acc[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[mb][r] = 0.f;

    const auto run_steps = [&](auto slot_blocks) {
        constexpr int MB = decltype(slot_blocks)::value;
        // bc: B(s); bn: the set B(s + ST - 1) loads into; as1: A(s + 1),
        // staged at the end of the step; an: the set A(s + ST - 1) loads into
        const auto step = [&](uint32_t s, const uint4_t (&bc)[kGemmU], uint4_t (&bn)[kGemmU], const AStage &as1,
                              AStage &an) {
            load_a(s + kGemmStages - 1, an);
            load_b(s + kGemmStages - 1, bn);
            const uint8_t *ab = as[s & 1] + ln * kGemmAStride + 16 * h;
#pragma unroll
            for (int u = 0; u < kGemmU; ++u) {
                const half8_t bf = __builtin_bit_cast(half8_t, bc[u]);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    const half8_t af = __builtin_bit_cast(half8_t, *reinterpret_cast<const uint4_t *>(
                                                                       ab + 32 * mb * kGemmAStride + 32 * u));
                    acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc[mb], 0, 0, 0);
                }
            }
            // the buffer every wavefront finished reading before the last
            // barrier (after the last step: a stage nobody reads)
            store_a((s + 1) & 1, as1);
            __syncthreads();
        };
        for (uint32_t s = 0; s < ksteps; s += kGemmStages) {  // the step count and its bounds are uniform
#pragma unroll
            for (int i = 0; i < kGemmStages; ++i) {
                if (s + i < ksteps)
                    step(s + i, bq[i], bq[(i + kGemmStages - 1) % kGemmStages], aq[(i + 1) % kGemmStages],
                         aq[(i + kGemmStages - 1) % kGemmStages]);
            }
        }
    };
    if (gend - m0 <= 32)  // uniform per block
        run_steps(std::integral_constant<int, 1>{});
    else
        run_steps(std::integral_constant<int, 2>{});

    // D layout (32x32): lane l, register r holds row 8(r/4) + 4(l/32) + r%4
    // of column l % 32.
    if (!bv) return;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t dst = slot_dst[32 * mb + 8 * (r >> 2) + 4 * h + (r & 3)];
            if (dst != kNoStore)
                a.y[size_t(dst & 0x7fffffffu) * a.N + col] =
                    (dst >> 31) ? uint16_t(float_to_half_bits(acc[mb][r])) : kHalfNaN;
        }
    }
}


// -- the direct-to-LDS form (K a multiple of 64) -----------------------------------

// One 16-byte load per lane from global memory into LDS: lane l's 16 bytes
// land at LDS byte lds + 16 l (M0 holds the wavefront's LDS base).  Written
// as inline asm rather than the compiler's builtin: with the builtin every
// __syncthreads() waits for all such loads in flight (vmcnt(0)), which would
// drain the pipeline each step; here the waits are explicit (below) and the
// compiler sees no load to wait for.
// M0 is declared clobbered; no other code in these kernels uses M0 (no LDS
// DMA builtin, message or relative register indexing), so nothing live is lost.
// An LDS DMA that reads M0 right after an SALU write of it needs one wait
// state on this generation (the compiler's hazard pass cannot see inside
// inline asm, so the s_nop is written here).  The asm's only register
// operands are the address and the LDS base; every MFMA result register of
// the kernel is a live accumulator, so no operand can be an MFMA destination
// still being written.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void load_to_lds16(uint32_t lds, const void *src) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(src)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

template <typename T>
__device__ __forceinline__ uint32_t lds_offset(T *p) {
    return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t *)(p)));
}

constexpr int kLdsRow = 2 * kGemmBK;              // bytes of one row's step: 128
constexpr int kLdsBStages = 4;                     // weight loads run three steps ahead
constexpr int kLdsAStages = 3;                     // activation loads two steps ahead
constexpr int kLdsBStage = kGemmBN * kLdsRow;      // 32 KiB: 256 weight rows
constexpr int kLdsAStage = kGemmBM * kLdsRow;      // 8 KiB: 64 slot rows
constexpr int kLdsWaveRows = kGemmBN / kGemmWaves; // 32 weight rows a wavefront streams
static_assert(kLdsRow == 128 && kGemmBM == 8 * kGemmWaves && kLdsWaveRows == 8 * kGemmU,
              "a load instruction moves 8 rows of 128 bytes; each wavefront 8 slot rows and its 32 weight rows");

// Step s of a wavefront issues A(s + 2) then B(s + 3) (1 + kGemmU loads), after
// a prologue B(0), A(0), B(1), A(1), B(2).  Loads complete in order, so when
// step s starts, A(s) and B(s) have landed once at most the 2 kGemmU + 1 loads
// issued after A(s) -- B(s+1), A(s+1), B(s+2) -- are outstanding.
static_assert(2 * kGemmU + 1 == 9, "the step's wait count below");

__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(2)))
void grouped_gemm_lds_kernel(GemmArgs a) {
    __shared__ TileScan ts;
    __shared__ __attribute__((aligned(16))) uint8_t bst[kLdsBStages * kLdsBStage];
    __shared__ __attribute__((aligned(16))) uint8_t ast[kLdsAStages * kLdsAStage];
    __shared__ uint32_t slot_dst[kGemmBM];  // as in grouped_gemm_kernel
    constexpr uint32_t kNoStore = 0x7fffffffu;

    const int tid = threadIdx.x;
    const uint32_t ncb = (a.N + kGemmBN - 1) / kGemmBN;
    const uint32_t tiles = count_mtiles<kGemmBM, kGemmThreads>(a.offs, a.n_groups, ts);
    const uint32_t per_xcd = (tiles + 7) / 8;
    const uint32_t xcd = blockIdx.x & 7u, j = blockIdx.x >> 3;
    if (j / ncb >= per_xcd) return;  // surplus block (uniform)
    const uint32_t tile = xcd * per_xcd + j / ncb, cblock = j % ncb;
    if (tile >= tiles) return;
    uint32_t g, mtile;
    if (!find_mtile<kGemmBM, kGemmThreads>(a.offs, a.n_groups, tile, ts, g, mtile)) return;

    const uint32_t gend = min(a.offs[g + 1], a.n_slots);
    const uint32_t m0 = a.offs[g] + mtile * kGemmBM;
    const uint32_t n0 = cblock * kGemmBN;
    const uint32_t ksteps = a.K / kGemmBK;
    const int wave = tid >> 6, l = tid & 63, ln = l & 31, h = l >> 5;

    if (tid < kGemmBM) {  // one thread a slot: the epilogue's destination, read once
        const uint32_t ap = m0 + uint32_t(tid);
        uint32_t dst = kNoStore;
        if (ap < gend) {
            const uint32_t yrow = a.yr ? a.yr[ap] : ap;
            if (yrow < a.n_slots) dst = yrow | (a.xr[ap] < a.n_x_rows ? 0x80000000u : 0u);
        }
        slot_dst[tid] = dst;
    }
    // A load instruction of wavefront w moves 8 rows r = 8 i + l / 8 (i = w for
    // the slots, i = u for load u of its weight rows), 128 bytes each; lane l
    // carries the row's chunk (l % 8) ^ (r / 2 % 8) into LDS position l % 8,
    // so LDS row r holds chunk c at position c ^ (r / 2 % 8).  Dead slots and
    // weight rows past out_features read row 0 (in bounds, never stored).
    const auto chunk = [&](int i) { return 8u * (uint32_t(l & 7) ^ (uint32_t(4 * i + (l >> 4)) & 7u)); };
    const uint16_t *asrc;
    {
        const uint32_t ap = m0 + uint32_t(8 * wave + (l >> 3));
        const uint32_t xrow = ap < gend ? a.xr[ap] : a.n_x_rows;
        asrc = a.x + size_t(xrow < a.n_x_rows ? xrow : 0u) * a.K + chunk(wave);
    }
    const uint16_t *bsrc[kGemmU];
#pragma unroll
    for (int u = 0; u < kGemmU; ++u) {
        const uint32_t r = n0 + uint32_t(kLdsWaveRows * wave + 8 * u + (l >> 3));
        bsrc[u] = a.w + (size_t(g) * a.N + (r < a.N ? r : 0u)) * a.K + chunk(u);
    }
    const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t a_lds = lds_offset(ast) + wv * (8 * kLdsRow);
    const uint32_t b_lds = lds_offset(bst) + wv * (kLdsWaveRows * kLdsRow);
    // A load for a step past the last re-reads the last step's bytes (in
    // bounds) into the stage of step s, which no later step reads: that stage
    // held step s - 3 (activations) or s - 4 (weights), already consumed.
    const auto issue_a = [&](uint32_t s) {
        const uint32_t k = min(s, ksteps - 1);
        load_to_lds16(a_lds + (s % kLdsAStages) * kLdsAStage, asrc + k * kGemmBK);
    };
    const auto issue_b = [&](uint32_t s) {
        const uint32_t k = min(s, ksteps - 1);
#pragma unroll
        for (int u = 0; u < kGemmU; ++u)
            load_to_lds16(b_lds + (s % kLdsBStages) * kLdsBStage + 8 * kLdsRow * u, bsrc[u] + k * kGemmBK);
    };
    issue_b(0);
    issue_a(0);
    issue_b(1);
    issue_a(1);
    issue_b(2);

    float16_t acc[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[mb][r] = 0.f;

    __syncthreads();  // the slot table
    // row ln's chunk positions, as a byte xor (rows 32 mb + ln of the slots
    // have the same); the 16 rows of a half-wavefront's read fill all 64 banks
    const uint32_t swz = 16u * (uint32_t(ln >> 1) & 7u);
    const auto run_steps = [&](auto slot_blocks) {
        constexpr int MB = decltype(slot_blocks)::value;
        for (uint32_t s = 0; s < ksteps; ++s) {  // the step count is uniform
            // this wavefront's A(s) and B(s) have landed and its LDS reads of
            // step s - 1 have returned; after the barrier every wavefront's
            // A(s) has landed, and every wavefront is done with step s - 1,
            // whose stages the loads below refill
            asm volatile("s_waitcnt vmcnt(9) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            issue_a(s + 2);
            issue_b(s + 3);
            const uint8_t *ab = ast + (s % kLdsAStages) * kLdsAStage + ln * kLdsRow;
            const uint8_t *bb = bst + (s % kLdsBStages) * kLdsBStage + (kLdsWaveRows * wave + ln) * kLdsRow;
#pragma unroll
            for (int u = 0; u < kGemmU; ++u) {
                // chunk 2u + h of the row (lanes h = l / 32 hold the MFMA's two k halves)
                const uint32_t co = (32u * u + 16u * h) ^ swz;
                const half8_t bf = __builtin_bit_cast(half8_t, *reinterpret_cast<const uint4_t *>(bb + co));
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    const half8_t af = __builtin_bit_cast(
                        half8_t, *reinterpret_cast<const uint4_t *>(ab + 32 * kLdsRow * mb + co));
                    acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc[mb], 0, 0, 0);
                }
            }
        }
    };
    if (gend - m0 <= 32)  // uniform per block
        run_steps(std::integral_constant<int, 1>{});
    else
        run_steps(std::integral_constant<int, 2>{});
    // no load into LDS may still be in flight when the block's LDS is released
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // D layout (32x32): lane l, register r holds row 8(r/4) + 4(l/32) + r%4
    // of column l % 32.
    const uint32_t col = n0 + uint32_t(kLdsWaveRows * wave + ln);
    if (col >= a.N) return;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t dst = slot_dst[32 * mb + 8 * (r >> 2) + 4 * h + (r & 3)];
            if (dst != kNoStore)
                a.y[size_t(dst & 0x7fffffffu) * a.N + col] =
                    (dst >> 31) ? uint16_t(float_to_half_bits(acc[mb][r])) : kHalfNaN;
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
    if (!x || !w || !group_offsets || !x_rows || !y || n_x_rows == 0) return IQK_ERR_ARGUMENT;
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
    // blocks: 8 XCDs x ceil(worst-case tiles / 8) x column blocks
    const uint64_t mtiles = (uint64_t(n_slots) + kGemmBM - 1) / kGemmBM + uint64_t(n_groups);
    const uint64_t blocks = 8 * ((mtiles + 7) / 8) * uint64_t((out_features + kGemmBN - 1) / kGemmBN);
    if (blocks > 0x7fffffffull) return IQK_ERR_ARGUMENT;
    if (in_features % kGemmBK == 0)
        hipLaunchKernelGGL(grouped_gemm_lds_kernel, dim3{uint32_t(blocks)}, dim3{kGemmThreads}, 0, as_stream(stream), a);
    else
        hipLaunchKernelGGL(grouped_gemm_kernel, dim3{uint32_t(blocks)}, dim3{kGemmThreads}, 0, as_stream(stream), a);
    return record_launch(hipGetLastError());
}
