// Fused dequant-in-MFMA grouped GEMM: the prefill contraction straight from
// the relayout streams (gfx950, fp16 MFMA, f32 accumulation).
//
// Reference: the prefill route dequantizes the whole stack to fp16
// (src/mlx_iqk/nn.py:155-169) and contracts it with mx.gather_mm over the
// sorted pairs (nn.py:221-238).  Here each workgroup decodes the weight rows
// it needs straight into MFMA operands, so a prefill reads the 2-bit streams
// (1122 B per 4096-wide IQ2_KS row) instead of writing and re-reading 8 KiB of
// fp16 per row.  IQ2_K's operands are the producer's fp16 weights bit for bit
// (the same four-entry tables).  IQ2_KS and IQ1_S_R4 scale each weight row by
// one fp16 d, so their operands are the exact products n = idx v (IQ1_S_R4:
// (2s+1)(g + shift)), fp16 without rounding, and d multiplies the row's f32
// sums once in the epilogue: a weight enters as d n instead of fp16(d n), and
// a one-hot activation row still yields fp16(d n), the producer's weight.
//
// Work list: as the grouped GEMM, with group g = expert g: the slots (pair
// rows) are sorted by expert, expert g owns [offs[g], offs[g+1]), and a block
// takes one M-tile of the list (64 slots) and one column block c (weight rows
// [256c, 256c + 256) of the requested row range).  XCD x (blocks b with
// b % 8 == x) takes a contiguous eighth of the M-tiles, each with all its
// column blocks one after another, so the column blocks of a tile share its
// activations in that XCD's L2 and an expert's M-tiles share its streams
// there (dealing M-tile 8i + x to XCD x instead fetched 1.32x the unique
// bytes from HBM, an expert's tiles landing on several XCDs).
//
// Tile: 512 threads, eight wavefronts.  Wavefront w owns weight rows
// 32w .. 32w+31 of the block (the 32 columns of v_mfma_f32_32x32x16_f16) for
// all 64 slots (two 32-row MFMA blocks): two 16-register accumulators, so a
// wavefront needs about 128 VGPRs and four fit per SIMD.
// Reduction steps of 128: lane (n, kg) = (l % 32, l / 32) decodes the 64
// weights of sub-blocks 2kg and 2kg+1 of the step (k = 128s + 64kg .. +64)
// of its row and feeds them to the step's eight MFMAs u as weights
// 8(u % 4) .. +7 of sub-block 2kg + u / 4, in the order (0,4,1,5,2,6,3,7) that
// the byte-split table lookup produces; the staged activations are permuted
// to match.  A lane thus builds its fp16 tables once per sub-block, and the
// MFMA's k index maps to the same weight for A and B.  The step's
// activations (64 slots x 128 fp16) are staged in LDS, double buffered, one
// barrier per step, and read one MFMA operand at a time; the code words of
// the next step are loaded while this one computes.  The block's scale planes
// (all 256 rows, whole reduction axis) are copied to LDS once, rows padded so
// the 32 rows a wavefront reads at once fall in distinct banks.
//
// IQ1_S_R4: the lane's two 32-weight blocks of a step bring their index bytes
// and qh words with the step's loads (no scale planes), and the grid sits in
// LDS as each entry's pool selectors (16 KiB); two grid entries expand like
// one 16-code word, with the block's pool of exact products (2s+1)(g +
// shift), the row's d applied to the sums as for IQ2_KS.

#include <type_traits>

#include "iqk_device.h"
#include "iqk_host.h"
#include "iqk_pool.h"

#define IQK_GRID_STORAGE __constant__ static const __attribute__((aligned(16)))
#include "../iq1s_grid.h"

namespace iqk {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kFusedWaves = 8;                   // wavefronts per block, 32 weight rows each
constexpr int kFusedThreads = 64 * kFusedWaves;
constexpr int kFusedBM = 64;                     // slots per block
constexpr int kFusedBN = 32 * kFusedWaves;       // weight rows per block
constexpr int kFusedKS = 128;                    // reduction elements per step
constexpr int kXStride = 2 * kFusedKS + 16;      // LDS bytes per staged activation row
constexpr int kXChunks = 2 * kFusedKS / 16;      // 16-byte chunks of a staged row per step
constexpr int kXRows = kFusedThreads / kXChunks; // rows one staging pass covers
constexpr int kXPer = kFusedBM / kXRows;         // staging passes a step
static_assert(kFusedBM % kXRows == 0 && kFusedThreads >= 256, "whole staging passes; the work-list scan needs 256 threads");
static_assert(kXRows == 32, "staging pass i is the 32-row MFMA slot block i");

struct FusedArgs {
    const uint16_t *x;
    const void *s0, *s1, *s2, *s3, *s4;
    const uint32_t *offs;  // [n_groups + 1]
    const uint32_t *xr, *yr;
    uint16_t *y;
    uint32_t N;         // output columns: weight rows row_start .. row_start + N of each expert
    uint32_t out_rows;  // rows per expert in the streams
    uint32_t row_start;
    uint32_t n_groups, n_slots, n_x_rows;
};

// A block's scale planes in LDS.  IQ2_KS: scl u8 [K/64], sch u8 [K/256],
// sex u8 [K/256], dv f16 per row.  IQ2_K: scl u16 [K/64], sex u8 [K/128],
// dv f16 [K/256].  Row strides are padded to an odd number of dwords.
// IQ2_K at K = 4096 keeps its dv plane out of LDS (DV_IN_LDS false): with it
// the planes (52 KB for 256 rows) and the activations would fit one block a
// CU; without it (43 KB), two.  Its lanes load their super-block scales
// instead, one 32-bit word (two super-blocks) every four steps.
template <int MEMBER, int K>
struct FusedScales {
    static constexpr bool KS = MEMBER == IQ2_KS;
    static constexpr bool DV_IN_LDS = !(MEMBER == IQ2_K && K == 4096);
    static constexpr int SCL = KS ? K / 64 : K / 32;    // bytes per row
    static constexpr int HB = KS ? K / 256 : 0;
    static constexpr int EX = KS ? K / 256 : K / 128;
    static constexpr int DV = KS ? 2 : K / 128;
    static constexpr int pad(int b) { return b == 0 ? 0 : ((b + 3) / 4 % 2 ? (b + 3) / 4 * 4 : (b + 3) / 4 * 4 + 4); }
    static constexpr int SCL_S = pad(SCL), HB_S = pad(HB), EX_S = pad(EX), DV_S = pad(DV);
    uint8_t scl[kFusedBN * SCL_S];
    uint8_t hb[KS ? kFusedBN * HB_S : 4];
    uint8_t ex[kFusedBN * EX_S];
    uint8_t dv[DV_IN_LDS ? kFusedBN * DV_S : 4];
};

// Copy `rows` (1 .. kFusedBN) rows of a plane (BYTES a row, consecutive in
// global memory) into LDS rows of STRIDE bytes, in 32-bit units where the
// rows are whole dwords (every plane but IQ2_KS's per-row scale), else
// 16-bit units.  Straight-line: every thread issues all its loads, then all
// its stores, so the plane costs one memory latency; units past `rows`
// re-read the last unit and land in LDS rows nobody stores from.
template <int BYTES, int STRIDE>
__device__ __forceinline__ void copy_plane(const uint8_t *src, int rows, uint8_t *dst, int tid) {
    using Unit = std::conditional_t<BYTES % 4 == 0, uint32_t, uint16_t>;
    static_assert(BYTES % sizeof(Unit) == 0 && STRIDE % sizeof(Unit) == 0, "whole units a row");
    constexpr int UNITS_PER_ROW = BYTES / sizeof(Unit);
    constexpr int UNITS = kFusedBN * UNITS_PER_ROW;
    constexpr int PER = (UNITS + kFusedThreads - 1) / kFusedThreads;
    const int last = rows * UNITS_PER_ROW - 1;
    Unit v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) v[i] = reinterpret_cast<const Unit *>(src)[min(tid + kFusedThreads * i, last)];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int u = tid + kFusedThreads * i;
        if (UNITS % kFusedThreads == 0 || u < UNITS) {
            const int r = u / UNITS_PER_ROW, c = u - r * UNITS_PER_ROW;
            *reinterpret_cast<Unit *>(dst + r * STRIDE + sizeof(Unit) * c) = v[i];
        }
    }
}

// IQ2_K's exact pool products n_c = v_c x m (m = nibble - 8 the scale index,
// v the alphabet), as fp16 pairs (word 0: n0 | n1 << 16, word 1: n2 | n3 <<
// 16), by (alphabet << 4 | nibble), each exact in fp16 (|n| <= 248), signed
// zeros included (a negative value times a zero index is -0).
struct Iq2kProducts {
    uint32_t w[2 * 32];
};

constexpr Iq2kProducts make_iq2k_products() {
    Iq2kProducts t{};
    constexpr int v[2][4] = {{-31, -13, 1, 17}, {-26, -8, 6, 22}};
    for (int alpha = 0; alpha < 2; ++alpha)
        for (int nib = 0; nib < 16; ++nib) {
            const int e = 16 * alpha + nib;
            const _Float16 m = _Float16(short(nib - 8));
            for (int c = 0; c < 4; ++c) {
                const _Float16 n = _Float16(short(v[alpha][c])) * m;
                t.w[2 * e + c / 2] |= uint32_t(__builtin_bit_cast(uint16_t, n)) << (16 * (c % 2));
            }
        }
    return t;
}

__constant__ const Iq2kProducts kIq2kProducts = make_iq2k_products();

// IQ1_S_R4's exact pool products n_c = (2s + 1) (g_c + shift), g = -1 .. 2,
// shift = 1/8 (negative when qh bit 15 is set), by qh bits 12-15 (s | sign
// << 3): at most 8 significant bits, so exact in fp16, and d x n rounded
// once is the producer's f32 chain d (2s+1) (g + shift) rounded once.
struct Iq1Products {
    uint32_t w[2 * 16];
};

constexpr Iq1Products make_iq1_products() {
    Iq1Products t{};
    for (int e = 0; e < 16; ++e) {
        const int s = e & 7, sign = e & 8 ? -1 : 1;
        for (int c = 0; c < 4; ++c) {
            const _Float16 n = _Float16(float((2 * s + 1) * (8 * (c - 1) + sign)) / 8.f);
            t.w[2 * e + c / 2] |= uint32_t(__builtin_bit_cast(uint16_t, n)) << (16 * (c % 2));
        }
    }
    return t;
}

// A four-entry fp16 table (n0 | n1 << 16, n2 | n3 << 16) as a v_perm pool:
// the low bytes of n0 .. n3, then their high bytes.
constexpr uint2_t split_pool(uint32_t n01, uint32_t n23) {
    return {(n01 & 0xffu) | ((n01 >> 8) & 0xff00u) | ((n23 & 0xffu) << 16) | ((n23 & 0xff0000u) << 8),
            ((n01 >> 8) & 0xffu) | ((n01 >> 16) & 0xff00u) | (((n23 >> 8) & 0xffu) << 16) | ((n23 >> 24) << 24)};
}

// IQ1_S_R4's products as pools.
struct Iq1Pools {
    uint2_t p[16];
};

constexpr Iq1Pools make_iq1_pools() {
    Iq1Pools t{};
    const Iq1Products q = make_iq1_products();
    for (int e = 0; e < 16; ++e) t.p[e] = split_pool(q.w[2 * e], q.w[2 * e + 1]);
    return t;
}

__constant__ const Iq1Pools kIq1Pools = make_iq1_pools();

// IQ2_KS's exact products n_c = v_c x idx as pools, by (alphabet << 5 |
// idx + 16): |n| <= 496, so each is exact in fp16 (a negative value times a
// zero index is -0, as in the producer's chain).
struct Iq2ksPools {
    uint2_t p[64];
};

constexpr Iq2ksPools make_iq2ks_pools() {
    Iq2ksPools t{};
    constexpr int v[2][4] = {{-31, -13, 1, 17}, {-26, -8, 6, 22}};
    for (int alpha = 0; alpha < 2; ++alpha)
        for (int i5 = 0; i5 < 32; ++i5) {
            const _Float16 m = _Float16(short(i5 - 16));
            uint32_t w[2] = {0u, 0u};
            for (int c = 0; c < 4; ++c) {
                const _Float16 n = _Float16(short(v[alpha][c])) * m;
                w[c / 2] |= uint32_t(__builtin_bit_cast(uint16_t, n)) << (16 * (c % 2));
            }
            t.p[32 * alpha + i5] = split_pool(w[0], w[1]);
        }
    return t;
}

__constant__ const Iq2ksPools kIq2ksPools = make_iq2ks_pools();

// The pool d x n_c from exact fp16 products n_c: one correctly rounded
// packed fp16 multiply a pair.  The producer's f32 chain forms the same exact
// product (at most 11 + 9 significant bits, so no f32 rounding) and rounds
// it to fp16 once, so the entries are equal bit for bit, signed zeros
// included.  The words pass as scalars: __builtin_bit_cast of a vector
// element (n.y of a uint2_t) reads the vector's first element in this
// compiler.
__device__ __forceinline__ Pool scale_products(uint32_t n01, uint32_t n23, _Float16 d) {
    const uint32_t p01 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, n01) * d);
    const uint32_t p23 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, n23) * d);
    return {perm(p23, p01, 0x06040200u), perm(p23, p01, 0x07050301u)};
}

// The v_perm tables of lane (row, kg) at step s, one per 16-weight word of
// its 64 weights: IQ2_KS sub-blocks 4s + 2kg + h (two words each), IQ2_K
// sub-blocks 8s + 4kg + w (one word each).  IQ2_KS's tables are its exact
// products idx v (the row scale d is applied to the sums), one LDS read of
// `ptab` by (alphabet, scale index): against forming d idx v in fp16 a step
// (two tables), the Zipf prefill's gate projection measured 381.1 -> 365.1
// us.  IQ2_K's are d n with n = v x m from `ptab`, its d being per
// super-block: the same fp16 products as the producer's f32 chain.  IQ2_K's
// super-block scale comes from the dv plane, or (no dv plane in LDS) from
// dvw, the lane's dv word of steps 4(s/4) .. +3 (scales of super-blocks
// 2(s/4) and 2(s/4)+1).
template <int MEMBER, int K>
__device__ __forceinline__ void fused_pools(const FusedScales<MEMBER, K> &sc, int row, int s, int kg, uint32_t dvw,
                                            const uint2_t *ptab, Pool *p) {
    using S = FusedScales<MEMBER, K>;
    if constexpr (MEMBER == IQ2_KS) {
        const uint32_t scl = sc.scl[row * S::SCL_S + 2 * s + kg];  // nibbles of sub-blocks 4s+2kg, +1
        const uint32_t hb = sc.hb[row * S::HB_S + (s >> 1)];
        const uint32_t ab = sc.ex[row * S::EX_S + (s >> 1)];
        const int bit = 4 * (s & 1) + 2 * kg;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            // alphabet << 5 | the 5-bit scale index (idx + 16)
            const uint32_t e = ((scl >> (4 * h)) & 15u) | (((hb >> (bit + h)) & 1u) << 4) | (((ab >> (bit + h)) & 1u) << 5);
            const uint2_t q = ptab[e];
            p[2 * h] = {q.x, q.y};
            p[2 * h + 1] = p[2 * h];
        }
    } else {
        const uint32_t scw = *reinterpret_cast<const uint16_t *>(sc.scl + row * S::SCL_S + 2 * (2 * s + kg));
        const uint32_t ab = (sc.ex[row * S::EX_S + s] >> (4 * kg)) & 15u;
        _Float16 dd;
        if constexpr (S::DV_IN_LDS)
            dd = half_of_bits(*reinterpret_cast<const uint16_t *>(sc.dv + row * S::DV_S + 2 * (s >> 1)));
        else
            dd = half_of_bits(dvw >> (16 * ((s >> 1) & 1)));
        // byte w: the table offset 8 (alpha_w << 4 | nibble_w) of word w; a
        // v_perm spreads the scale word's bytes to (b0, b0, b1, b1), shifts
        // put nibble w at bits 3-6 of byte w, and the multiply copies
        // alphabet bit w to bit 8w (no two copies meet, so no carries;
        // pinned, or it becomes a quarter-rate 32-bit multiply)
        const uint32_t scp = perm(scw, scw, 0x01010000u);
        uint32_t a8 = __umul24(ab, 0x204081u);
        asm volatile("" : "+v"(a8));
        const uint32_t kofs = ((scp << 3) & 0x00780078u) | ((scp >> 1) & 0x78007800u) | ((a8 & 0x01010101u) << 7);
        const uint8_t *tab = reinterpret_cast<const uint8_t *>(ptab);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint2_t n = *reinterpret_cast<const uint2_t *>(tab + ((kofs >> (8 * w)) & 0xffu));
            p[w] = scale_products(uint32_t(n.x), uint32_t(n.y), dd);
        }
    }
}

// IQ1_S_R4 at one step: blocks b = 0, 1 of the lane (index bytes q[b], qh
// word b of q.z).  Pools p[2b], p[2b+1] are block b's (the products
// (2s+1) (g + shift) from the LDS table `ptab`; the row scale d is applied
// to the sums: 394.9 -> 377.4 us on the Zipf prefill's gate projection
// against forming d (2s+1) (g + shift) a block), and sels[2b+t] holds the
// pool selectors of the block's 8-weight groups 2t and 2t+1, read whole from
// the block's LDS table of them (grid_selectors): no shifts and masks a step.
// Against 16-bit code words expanded by expand_word_paired (their selectors
// formed a step) the Zipf prefill's gate projection measured 390.4 -> 379.1
// us, bit-identical: 28 fewer VALU a step for four times the LDS bytes of
// the lookups.
__device__ __forceinline__ void fused_iq1(uint4_t q, const uint2_t *grid, const uint2_t *ptab, Pool *p,
                                          uint4_t *sels) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const uint32_t qw = q[b], h = (q.z >> (16 * b)) & 0xffffu;
        // grid field 3 never occurs: four products, by qh bits 12-15
        const uint2_t n = ptab[(h >> 12) & 15u];
        p[2 * b] = {n.x, n.y};
        p[2 * b + 1] = p[2 * b];
        uint2_t c[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) c[t] = grid[((qw >> (8 * t)) & 0xffu) | (((h >> (3 * t)) & 7u) << 8)];
        sels[2 * b] = uint4_t{c[0].x, c[0].y, c[1].x, c[1].y};
        sels[2 * b + 1] = uint4_t{c[2].x, c[2].y, c[3].x, c[3].y};
    }
}

struct FusedGrid {
    uint2_t sel[IQK_IQ1S_GRID_SIZE];  // grid_selectors of every grid entry, 16 KiB
};

// Pool selectors of one grid entry (positions i at bits 2i): (p0, p4, p1,
// p5) and (p2, p6, p3, p7), one position a byte.
__device__ __forceinline__ uint2_t grid_selectors(uint32_t x) {
    return {(x & 0x0303u) | ((x << 14) & 0x03030000u), ((x >> 4) & 0x0303u) | ((x << 10) & 0x03030000u)};
}

// The 16 weights of two grid entries from their selectors (sel.xy entry 0,
// sel.zw entry 1), in expand_word_paired's output order for the 16-code word
// of the two entries (dword 2j: positions j, j+4 of entry 0; dword 2j+1: of
// entry 1), so the MFMAs and the staged activations are the same as for a
// code word.
__device__ __forceinline__ void expand_sel_paired(uint4_t sel, Pool p, uint32_t *out) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t e = sel[i];
        const uint32_t lo = perm(p.lo, p.lo, e), hi = perm(p.hi, p.hi, e);
        out[4 * (i & 1) + (i >> 1)] = perm(hi, lo, 0x05010400u);
        out[4 * (i & 1) + (i >> 1) + 2] = perm(hi, lo, 0x07030602u);
    }
}

template <int MEMBER, int K>
__global__ __launch_bounds__(kFusedThreads) __attribute__((amdgpu_waves_per_eu(4)))
void fused_gemm_kernel(FusedArgs a) {
    constexpr bool IQ1 = MEMBER == IQ1_S_R4;
    using S = FusedScales<IQ1 ? IQ2_KS : MEMBER, K>;
    constexpr int STEPS = K / kFusedKS;
    // Steps a code-word group: IQ1_S_R4 4, the IQ2 members 1.  Two-step
    // groups for the IQ2 members measured within 1% (IQ2_K gate 404.4 ->
    // 402.6 us, IQ2_KS gate 381.9 -> 380.8 us with 32 bytes of spills at 128
    // VGPRs; IQ2_K at 2048 wide has no room for them): with one step a
    // group, a line of their code plane is loaded four times, not 8 or 16.
    constexpr int G = IQ1 ? 4 : 1;
    static_assert(STEPS % G == 0, "whole groups of steps");
    __shared__ TileScan ts;
    __shared__ __attribute__((aligned(16))) uint8_t xs[2][kFusedBM * kXStride];
    // per slot of the tile: its output row, bit 31 set when its activations
    // are real (else its output row is NaN), or kNoStore
    __shared__ uint32_t slot_dst[kFusedBM];
    __shared__ uint2_t ptab[MEMBER == IQ2_K ? 32 : IQ1 ? 16 : 64];  // pool products (IQ2_K) or pools
    constexpr uint32_t kNoStore = 0x7fffffffu;  // above any row (n_slots <= 2^30)
    __shared__ __attribute__((aligned(16))) std::conditional_t<IQ1, FusedGrid, S> sc;

    const int tid = threadIdx.x;
    const uint32_t ncb = (a.N + kFusedBN - 1) / kFusedBN;  // column blocks
    const uint32_t tiles = count_mtiles<kFusedBM, kFusedThreads>(a.offs, a.n_groups, ts);
    const uint32_t per_xcd = (tiles + 7) / 8;
    const uint32_t xcd = blockIdx.x & 7u, j = blockIdx.x >> 3;
    if (j / ncb >= per_xcd) return;  // surplus block (uniform)
    const uint32_t tile = xcd * per_xcd + j / ncb, cblock = j % ncb;
    if (tile >= tiles) return;
    uint32_t g, mtile;
    if (!find_mtile<kFusedBM, kFusedThreads>(a.offs, a.n_groups, tile, ts, g, mtile)) return;
    g = __builtin_amdgcn_readfirstlane(g);  // uniform (read from LDS): the stream bases stay scalar

    // Offsets and row indices are device data: a slot outside [0, n_slots)
    // is never stored, a row outside x is never read (its output row is NaN),
    // and a weight row past out_features is never stored.  Loads of such
    // rows read an in-bounds row instead, so the step has no branches but
    // (IQ1_S_R4) the one that skips staging activation rows past the tile's
    // end.
    const uint32_t gend = min(a.offs[g + 1], a.n_slots);
    const uint32_t m0 = a.offs[g] + mtile * kFusedBM;
    const uint32_t n0 = cblock * kFusedBN;
    const int rows_here = int(min(uint32_t(kFusedBN), a.N - n0));
    const size_t row0 = size_t(g) * a.out_rows + a.row_start + n0;  // first stacked weight row of the block

    if constexpr (MEMBER == IQ2_K) {
        if (tid < 32) ptab[tid] = reinterpret_cast<const uint2_t *>(kIq2kProducts.w)[tid];
    } else if constexpr (IQ1) {
        if (tid < 16) ptab[tid] = kIq1Pools.p[tid];
    } else {
        if (tid < 64) ptab[tid] = kIq2ksPools.p[tid];
    }
    // scale planes of the block's rows (IQ1_S_R4: the grid as pool selectors)
    if constexpr (IQ1) {
        static_assert(IQK_IQ1S_GRID_SIZE == 4 * kFusedThreads, "four grid entries a thread");
        const uint2_t cw = reinterpret_cast<const uint2_t *>(iqk_iq1s_grid_codes)[tid];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            sc.sel[4 * tid + i] = grid_selectors(((i < 2 ? cw.x : cw.y) >> (16 * (i & 1))) & 0xffffu);
    } else {
        copy_plane<S::SCL, S::SCL_S>(static_cast<const uint8_t *>(a.s1) + row0 * S::SCL, rows_here, sc.scl, tid);
    }
    if constexpr (MEMBER == IQ2_KS) {
        copy_plane<S::HB, S::HB_S>(static_cast<const uint8_t *>(a.s2) + row0 * S::HB, rows_here, sc.hb, tid);
        copy_plane<S::EX, S::EX_S>(static_cast<const uint8_t *>(a.s3) + row0 * S::EX, rows_here, sc.ex, tid);
        copy_plane<S::DV, S::DV_S>(static_cast<const uint8_t *>(a.s4) + row0 * S::DV, rows_here, sc.dv, tid);
    } else if constexpr (MEMBER == IQ2_K) {
        copy_plane<S::EX, S::EX_S>(static_cast<const uint8_t *>(a.s2) + row0 * S::EX, rows_here, sc.ex, tid);
        if constexpr (S::DV_IN_LDS)
            copy_plane<S::DV, S::DV_S>(static_cast<const uint8_t *>(a.s3) + row0 * S::DV, rows_here, sc.dv, tid);
    }

    // activation staging: thread t moves 16-byte chunk t % kXChunks of slot
    // rows t / kXChunks + kXRows i a step, so the eight lanes of each LDS
    // store phase write 128 contiguous bytes (a thread's two chunks side by
    // side had every store phase hit each bank twice).  Byte offsets into x
    // are 32-bit (the entry point refuses an x of 4 GiB or more).
    // A row past the tile's last slot feeds only MFMA rows that are never
    // stored, so IQ1_S_R4 neither loads nor stages it per step (its LDS row
    // keeps the zeros written at the tile's start): a partial tile (most
    // tiles of a skewed routing) stages only its slots.  Measured on the 2048-token Zipf prefill:
    // IQ1_S_R4 -4%; the IQ2 members, whose step the branch splits for the
    // scheduler, +1 to +2%, so they stage every row.
    const int xrow_l = tid / kXChunks, xchunk = tid % kXChunks;
    const uint8_t *xbase = reinterpret_cast<const uint8_t *>(a.x);
    uint32_t xoff[kXPer];
    bool xlive[kXPer];
#pragma unroll
    for (int i = 0; i < kXPer; ++i) {
        const int row = xrow_l + kXRows * i;
        const uint32_t xp = m0 + uint32_t(row);
        const uint32_t xrow = xp < gend ? a.xr[xp] : a.n_x_rows;
        const bool xv = xrow < a.n_x_rows;
        // a dead slot reads row 0 (the entry point refuses an empty x); its
        // products feed only its own output row, never stored as a value
        // chunks 8 .. 15 (lane group 1's half of a step) start 64G elements
        // after chunks 0 .. 7 in x, 64 in the staged row (see x_step)
        xoff[i] = (xv ? xrow : 0u) * uint32_t(2 * K) + uint32_t(16 * xchunk) + (xchunk >= 8 ? 128u * (G - 1) : 0u);
        xlive[i] = !IQ1 || xp < gend;
        if (xchunk == 0) {  // one thread a slot: the epilogue's destination, read once
            uint32_t dst = kNoStore;
            if (xp < gend) {
                const uint32_t yrow = a.yr ? a.yr[xp] : xp;
                if (yrow < a.n_slots) dst = yrow | (xv ? 0x80000000u : 0u);
            }
            slot_dst[row] = dst;
        }
    }
    // Staging pass i covers slot block i (rows 32i .. 32i+31): a tile of
    // MB slot blocks loads and stages passes 0 .. MB-1 only.
    // Steps go in groups of G (below): step Gp + j stages the 64 elements
    // from 128Gp + 64j (lane group 0's) and from 128Gp + 64G + 64j (lane
    // group 1's).
    const auto x_step = [&](int s) { return uint32_t(256 * G * (s / G) + 128 * (s % G)); };
    const auto load_x = [&](int s, uint4_t *v, auto passes) {
#pragma unroll
        for (int i = 0; i < decltype(passes)::value; ++i)
            if (xlive[i]) v[i] = load_u4(xbase + xoff[i] + x_step(s));
    };
    // Each 8-element chunk is stored in the order (0,4,1,5,2,6,3,7), the
    // order expand_word_paired gives the weights.  A row past the tile's last
    // slot is staged as zeros, so the MFMAs of those rows multiply zeros: the
    // kernel is bound by the clock its power allows, and zero operands draw
    // less (IQ2_KS gate 400.7 -> 392.5 us, IQ2_K gate 426.7 -> 417.0 us on
    // the 2048-token Zipf prefill; the rows were a dead slot's real data).
    // The IQ2 members stage every row, the dead ones through v_perm
    // selectors of 0x0c bytes (which give zero bytes: no instruction added);
    // IQ1_S_R4 zeroes its dead rows in both buffers once.
    uint32_t xsel_lo[kXPer], xsel_hi[kXPer];
#pragma unroll
    for (int i = 0; i < kXPer; ++i) {
        const bool dead = m0 + uint32_t(xrow_l + kXRows * i) >= gend;
        xsel_lo[i] = dead ? 0x0c0c0c0cu : 0x05040100u;
        xsel_hi[i] = dead ? 0x0c0c0c0cu : 0x07060302u;
        if (IQ1 && dead) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
                *reinterpret_cast<uint4_t *>(xs[b] + (xrow_l + kXRows * i) * kXStride + 16 * xchunk) =
                    uint4_t{0u, 0u, 0u, 0u};
        }
    }
    const auto store_x = [&](int buf, const uint4_t *v, auto passes) {
        uint8_t *dst = xs[buf] + xrow_l * kXStride + 16 * xchunk;
#pragma unroll
        for (int i = 0; i < decltype(passes)::value; ++i)
            if (xlive[i])
                *reinterpret_cast<uint4_t *>(dst + kXRows * kXStride * i) =
                    uint4_t{perm(v[i].z, v[i].x, xsel_lo[i]), perm(v[i].z, v[i].x, xsel_hi[i]),
                            perm(v[i].w, v[i].y, xsel_lo[i]), perm(v[i].w, v[i].y, xsel_hi[i])};
    };

    // this lane's weight row and code words; a row past out_features reads
    // the block's first row.  The block's first row of each plane is a
    // uniform base, the lane's offsets from it are 32-bit (the entry point
    // refuses an expert plane of 4 GiB or more).  The steps go in groups of
    // G, lane group kg taking elements 128Gp + 64G kg .. +64G-1 of group p
    // (64j .. 64j+63 of those in its step j), so a lane loads its code bytes
    // once a group: IQ2 members 16G bytes (four words a step), IQ1_S_R4 (G =
    // 4) 32 bytes of index words and 16 of qh words.  A 128-byte line of a
    // code plane is then loaded 4/G times (IQ2; IQ1_S_R4 two and four times
    // against eight and sixteen with a load a step: 2.13x its unique bytes
    // fetched, 440.5 -> 411.9 us on the Zipf prefill gate).
    const int wave = tid >> 6, l = tid & 63, ln = l & 31, kg = l >> 5;
    const int lrow = 32 * wave + ln;
    const bool wv = lrow < rows_here;
    constexpr uint32_t QROW = IQ1 ? K / 8 : K / 4;  // code-plane bytes a row
    const uint8_t *qbase = static_cast<const uint8_t *>(a.s0) + row0 * QROW;
    const uint8_t *hbase = static_cast<const uint8_t *>(a.s1) + row0 * (K / 16);
    const uint32_t wl = wv ? uint32_t(lrow) : 0u;
    const uint32_t qoff = wl * QROW + uint32_t((IQ1 ? 8 : 16) * G * kg), hoff = wl * uint32_t(K / 16) + uint32_t(16 * kg);
    struct CodeGroup {
        uint4_t w[IQ1 ? 3 : G];  // IQ2: step j's words; IQ1_S_R4: 8 blocks' index words, then their qh halves
    };
    const auto load_group = [&](int p) {
        CodeGroup gr;
        if constexpr (IQ1) {
            gr.w[0] = load_u4(qbase + qoff + uint32_t(64 * p));
            gr.w[1] = load_u4(qbase + qoff + uint32_t(64 * p + 16));
            gr.w[2] = load_u4(hbase + hoff + uint32_t(32 * p));
        } else {
#pragma unroll
            for (int j = 0; j < G; ++j) gr.w[j] = load_u4(qbase + qoff + uint32_t(32 * G * p + 16 * j));
        }
        return gr;
    };
    // step j of a group; IQ1_S_R4: blocks 2j, 2j+1 (index words, qh halves in one word)
    const auto group_step = [](const CodeGroup &gr, int j) {
        if constexpr (IQ1) {
            const uint4_t &w = gr.w[j >> 1];
            return uint4_t{(j & 1) ? w.z : w.x, (j & 1) ? w.w : w.y, gr.w[2][j], 0u};
        } else {
            return gr.w[j];
        }
    };

    uint4_t xa[kXPer];
    constexpr std::integral_constant<int, kXPer> kAllPasses{};
    load_x(0, xa, kAllPasses);
    // IQ2_K without a dv plane in LDS: this lane's dv words, one per four steps
    const uint32_t *dvp = reinterpret_cast<const uint32_t *>(static_cast<const uint8_t *>(a.s3) + row0 * (K / 128) +
                                                             wl * uint32_t(K / 128));
    constexpr bool DV_WORDS = MEMBER == IQ2_K && !S::DV_IN_LDS;
    uint32_t dvw = DV_WORDS ? dvp[0] : 0u, dvn = 0u;
    CodeGroup grp = load_group(0), grpn{};
    store_x(0, xa, kAllPasses);
    __syncthreads();  // scale planes and the first activations are in LDS
    // row scale, applied to the sums: IQ2_KS from LDS (rows past out_features
    // read LDS junk, never stored), IQ1_S_R4 from its stream (an in-bounds
    // row); IQ2_K's are per super-block, in its pools
    _Float16 d = 0.f16;
    if constexpr (MEMBER == IQ2_KS)
        d = half_of_bits(*reinterpret_cast<const uint16_t *>(sc.dv + lrow * S::DV_S));
    else if constexpr (IQ1)
        d = half_of_bits(static_cast<const uint16_t *>(a.s2)[row0 + wl]);

    // A tile of at most 32 real slots (most experts of a skewed routing)
    // runs the second slot block's MFMAs for nothing: skip them (its slots
    // 32 .. 63 are past the tile's end, never stored, so their accumulators
    // do not exist).
    const auto run_steps = [&](auto slot_blocks) {
        constexpr int MB = decltype(slot_blocks)::value;
        float16_t acc[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mb][r] = 0.f;
        for (int s0 = 0; s0 < STEPS; s0 += G) {
#pragma unroll
          for (int j = 0; j < G; ++j) {
            const int s = s0 + j;
            const bool more = s + 1 < STEPS;
            if (more) load_x(s + 1, xa, slot_blocks);
            if (j == 0 && s0 + G < STEPS) grpn = load_group((s0 + G) / G);  // the next group, a group ahead
            if constexpr (DV_WORDS) {
                if ((s & 3) == 0 && s + 4 < STEPS) dvn = dvp[(s >> 2) + 1];  // the next group's word, a group ahead
            }
            Pool p[4];
            uint32_t words[4];
            uint4_t sels[IQ1 ? 4 : 1];
            if constexpr (IQ1) {
                fused_iq1(group_step(grp, j), sc.sel, ptab, p, sels);
            } else {
                // the lane's sub-blocks are those the one-step order gives
                // step G(s/G) + kg's lane group j
                fused_pools<MEMBER, K>(sc, lrow, G * (s / G) + (G > 1 ? kg : 0), G > 1 ? j : kg, dvw, ptab, p);
                const uint4_t q = group_step(grp, j);
#pragma unroll
                for (int w = 0; w < 4; ++w) words[w] = q[w];
            }
            const uint8_t *xb = xs[s & 1] + ln * kXStride + 128 * kg;
            // A operands of MFMA u (slot blocks 0 .. MB-1)
            const auto read_a = [&](int u, half8_t *af) {
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    af[mb] = __builtin_bit_cast(half8_t, *reinterpret_cast<const uint4_t *>(
                                                             xb + 32 * mb * kXStride + 64 * (u >> 2) + 16 * (u & 3)));
            };
            half8_t af[MB], afn[MB];
            read_a(0, af);
            // Word w feeds MFMAs u = 2w, 2w+1 (weights 16(w%2) + 8h .. +7 of
            // sub-block 2kg + w/2, paired order); expanding word w+1 overlaps
            // word w's MFMAs.
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t bw[8];
                if constexpr (IQ1)
                    expand_sel_paired(sels[w], p[w], bw);
                else
                    expand_word_paired(words[w], p[w], bw);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int u = 2 * w + h;
                    if (u < 7) read_a(u + 1, afn);
                    const half8_t bf = __builtin_bit_cast(half8_t, uint4_t{bw[h], bw[2 + h], bw[4 + h], bw[6 + h]});
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb) {
                        acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[mb], bf, acc[mb], 0, 0, 0);
                        af[mb] = afn[mb];
                    }
                }
            }
            if (more) store_x((s + 1) & 1, xa, slot_blocks);  // the buffer every wavefront finished reading before the last barrier
            if (j == G - 1) grp = grpn;
            if constexpr (DV_WORDS) {
                if ((s & 3) == 3) dvw = dvn;
            }
            __syncthreads();
          }
        }

        const float dscale = float(d);
        // D layout (32x32): lane l, register r holds row 8(r/4) + 4(l/32) +
        // r%4 of column l % 32.
        if (!wv) return;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t dst = slot_dst[32 * mb + 8 * (r >> 2) + 4 * kg + (r & 3)];
                if (dst != kNoStore)
                    a.y[size_t(dst & 0x7fffffffu) * a.N + n0 + lrow] =
                        (dst >> 31) ? uint16_t(float_to_half_bits(MEMBER == IQ2_K ? acc[mb][r] : acc[mb][r] * dscale))
                                    : kHalfNaN;
            }
        }
    };
    if (gend - m0 <= 32)  // uniform per block
        run_steps(std::integral_constant<int, 1>{});
    else
        run_steps(std::integral_constant<int, 2>{});
}

template <int MEMBER>
int launch_fused(int64_t k, const FusedArgs &a, uint32_t n_slots, hipStream_t st) {
    const uint64_t mtiles = (uint64_t(n_slots) + kFusedBM - 1) / kFusedBM + uint64_t(a.n_groups);
    const uint64_t blocks = (mtiles + 7) / 8 * 8 * ((a.N + kFusedBN - 1) / kFusedBN);
    if (blocks > 0x7fffffffull) return IQK_ERR_ARGUMENT;
    const dim3 grid{uint32_t(blocks)}, block{kFusedThreads};
    if (k == 4096)
        hipLaunchKernelGGL((fused_gemm_kernel<MEMBER, 4096>), grid, block, 0, st, a);
    else
        hipLaunchKernelGGL((fused_gemm_kernel<MEMBER, 2048>), grid, block, 0, st, a);
    return record_launch(hipGetLastError());
}

}  // namespace iqk

extern "C" int iqk_fused_gemm(int member, int64_t in_features, int64_t out_features, int64_t num_experts,
                              const void *x, int64_t n_x_rows, const void *const *streams, int n_streams,
                              int64_t row_start, int64_t rows, const uint32_t *group_offsets,
                              const uint32_t *x_rows, const uint32_t *y_rows, int64_t n_slots, void *y,
                              void *stream) {
    using namespace iqk;
    if (!member_ok(member)) return IQK_ERR_MEMBER;
    if (!width_sized(in_features)) return IQK_ERR_GEOMETRY;
    if (out_features <= 0 || out_features > (int64_t(1) << 24)) return IQK_ERR_GEOMETRY;
    // 32-bit offsets within an expert's code plane (in/4 bytes a row) and x
    if (out_features * (in_features / 4) >= (int64_t(1) << 32)) return IQK_ERR_GEOMETRY;
    if (row_start < 0 || rows <= 0 || row_start + rows > out_features) return IQK_ERR_GEOMETRY;
    if (num_experts <= 0 || num_experts > (int64_t(1) << 20)) return IQK_ERR_ARGUMENT;
    if (n_slots < 0 || n_slots > (int64_t(1) << 30) || n_x_rows < 0 || n_x_rows > 0xffffffffll)
        return IQK_ERR_ARGUMENT;
    if (n_slots == 0) return IQK_OK;
    if (!x || !y || !group_offsets || !x_rows || !streams_ok(streams, n_streams, member)) return IQK_ERR_ARGUMENT;
    if (n_x_rows == 0 || n_x_rows * in_features * 2 >= (int64_t(1) << 32)) return IQK_ERR_ARGUMENT;
    FusedArgs a;
    a.x = static_cast<const uint16_t *>(x);
    a.s0 = streams[0]; a.s1 = streams[1]; a.s2 = streams[2];
    a.s3 = n_streams > 3 ? streams[3] : nullptr;
    a.s4 = n_streams > 4 ? streams[4] : nullptr;
    a.offs = group_offsets;
    a.xr = x_rows;
    a.yr = y_rows;
    a.y = static_cast<uint16_t *>(y);
    a.N = uint32_t(rows);
    a.out_rows = uint32_t(out_features);
    a.row_start = uint32_t(row_start);
    a.n_groups = uint32_t(num_experts);
    a.n_slots = uint32_t(n_slots);
    a.n_x_rows = uint32_t(n_x_rows);
    hipStream_t st = as_stream(stream);
    switch (member) {
        case IQK_MEMBER_IQ2_KS: return launch_fused<IQ2_KS>(in_features, a, uint32_t(n_slots), st);
        case IQK_MEMBER_IQ2_K: return launch_fused<IQ2_K>(in_features, a, uint32_t(n_slots), st);
        default: return launch_fused<IQ1_S_R4>(in_features, a, uint32_t(n_slots), st);
    }
}
