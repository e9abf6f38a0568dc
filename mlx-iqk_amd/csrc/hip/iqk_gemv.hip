// Decode GEMV over selected experts, and its deleted-decode floor (gfx950).
//
// Reference: the Metal decode GEMV (src/mlx_iqk/kernels.py:286-401, launched
// by src/mlx_iqk/nn.py:240-271) and its floor (bench/floors.py:86-176).
//
// Layout of the work.  One 64-lane wavefront owns 16 consecutive output rows
// of one (token, expert) pair.  Each lane owns a fixed 64-weight chunk of the
// reduction axis, so a 4096-wide row is one 1 KiB coalesced sweep of 64
// 128-bit loads and a 2048-wide row is half a wavefront.  The lane's
// activations are loaded once and reused for all 16 rows.
//
// Decode.  The two alphabets (-31,-13,1,17) and (-26,-8,6,22) are both
// v = 2*w + off with w in (-16,-7,0,8) and off = 1 or 6.  Every w is exact in
// fp16 with a zero low byte, so a single v_perm_b32 whose selector is built
// from the packed 2-bit codes with one and-or turns two codes into an fp16
// pair of w values, which v_dot2_f32_f16 multiplies against a pre-permuted
// activation pair in f32.  Pairs whose codes sit in the low byte lanes of the
// selector instead look up a low byte under a constant high byte, giving
// 9 + w/16; the affine terms (off * sum(x), the 9 * sum(x) bias) are per-lane,
// per-sub-block constants folded in once per sub-block.  Every product is
// exact; the accumulation is f32.  IQ1_S_R4 decodes its grid words (looked up
// from LDS) through the same path with the ternary table (-1, 0, 1).
//
// Reduction.  Each lane accumulates one partial per row; a transposed
// butterfly over the lanes of a row leaves each lane one full row sum.

#include "iqk_device.h"
#include "iqk_host.h"

#define IQK_GRID_STORAGE __constant__ static const
#include "../iq1s_grid.h"

namespace iqk {

struct GemvArgs {
    const uint32_t *x;  // f16 pairs
    const void *s0, *s1, *s2, *s3, *s4;
    const uint32_t *sel;
    const uint32_t *toks;  // NULL: pair m reads x row m / pairs_per_row; else toks[m]
    uint32_t n_x_rows;
    uint32_t pairs_per_row;
    uint32_t num_experts;
    uint32_t out_features;
    uint16_t *y;
};

// v_perm pools: slots 0-3 = low bytes L(c) under a constant high byte,
// slots 4-7 = high bytes of the exact fp16 values (low byte 0).
constexpr uint32_t kIq2PoolHi = 0x4800C7CCu;  // fp16 hi bytes of -16, -7, 0, 8
constexpr uint32_t kIq2PoolLo = 0xC0804800u;  // L = 8*(w+16): 0, 72, 128, 192
constexpr uint32_t kIq1PoolHi = 0x403C00BCu;  // fp16 hi bytes of -1, 0, 1, (2)
constexpr uint32_t kIq1PoolLo = 0xC0804000u;  // L = 64*f: 0, 64, 128, 192

// Selector for the pair of codes in byte lanes 1 and 3: (0x00 | hi(slot 4+c)).
// Selector for the pair in byte lanes 0 and 2: (lo(slot c) | hi(slot 7)).
__device__ __forceinline__ uint32_t sel_hi(uint32_t t) { return (t & 0x03000300u) | 0x040C040Cu; }
__device__ __forceinline__ uint32_t sel_lo(uint32_t t) { return (t & 0x00030003u) | 0x07000700u; }

// 16 codes of one word.  For shift s the byte lanes of qw>>2s hold codes
// s, 4+s, 8+s, 12+s; xa[s] pairs activations (4+s, 12+s), xb[s] (s, 8+s).
template <uint32_t HI, uint32_t LO>
__device__ __forceinline__ void decode_word(uint32_t qw, const uint32_t *xa, const uint32_t *xb,
                                            float &a1, float &a2) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint32_t t = qw >> (2 * s);
        a2 = dot2(perm(HI, LO, sel_hi(t)), xa[s], a2);
        a1 = dot2(perm(HI, LO, sel_lo(t)), xb[s], a1);
    }
}

// The lane's 64 activations as the 32 fp16 pairs decode_word consumes, plus
// per-word sums: xsum[w] = sum of the word's 16 activations, xlo[w] = sum over
// the positions decoded through the low-byte selector (s and 8+s).
struct LaneX {
    uint32_t xa[16], xb[16];
    float xsum[4], xlo[4];
};

__device__ __forceinline__ void load_lane_x(const uint32_t *xrow, LaneX &lx) {
    uint32_t xw[32];
    const uint4_t *p = reinterpret_cast<const uint4_t *>(xrow);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint4_t v = p[i];
        xw[4 * i + 0] = v.x; xw[4 * i + 1] = v.y; xw[4 * i + 2] = v.z; xw[4 * i + 3] = v.w;
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint32_t sel = (s & 1) ? 0x07060302u : 0x05040100u;
            const int a = 16 * w + 4 + s, b = 16 * w + s;
            lx.xa[4 * w + s] = perm(xw[(a + 8) / 2], xw[a / 2], sel);
            lx.xb[4 * w + s] = perm(xw[(b + 8) / 2], xw[b / 2], sel);
        }
        float sum = 0.f, lo = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int k = 16 * w + j;
            const float v = half_bits_to_float((xw[k / 2] >> (16 * (k % 2))) & 0xffffu);
            sum += v;
            if ((j & 7) < 4) lo += v;
        }
        lx.xsum[w] = sum;
        lx.xlo[w] = lo;
    }
}

// Transposed butterfly: RC partials per lane -> one row sum per lane.
template <int RC, int OFF>
__device__ __forceinline__ void treduce(float *v, int lane, int &idx) {
    if constexpr (RC > 1) {
        constexpr int H = RC / 2;
        const bool up = (lane & OFF) != 0;
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const float keep = up ? v[i + H] : v[i];
            const float send = up ? v[i] : v[i + H];
            v[i] = keep + __shfl_xor(send, OFF);
        }
        if (up) idx += H;
        treduce<H, OFF / 2>(v, lane, idx);
    } else {
#pragma unroll
        for (int o = OFF; o >= 1; o >>= 1) v[0] += __shfl_xor(v[0], o);
    }
}

template <int MEMBER, int N, bool FLOOR>
__global__ __launch_bounds__(64) void gemv_kernel(GemvArgs a) {
    constexpr int LPR = N / 64;     // lanes per row
    constexpr int RPS = 64 / LPR;   // rows per wavefront step
    constexpr int R = 16 / RPS;     // rows per lane
    const int lane = threadIdx.x;
    const int lc = lane % LPR, rsub = lane / LPR;
    const uint32_t m = blockIdx.y;
    const uint32_t row0 = blockIdx.x * 16;
    const uint32_t e = a.sel[m];
    const uint32_t tok = a.toks ? a.toks[m] : m / a.pairs_per_row;
    uint16_t *yrow = a.y + size_t(m) * a.out_features + row0;
    if (e >= a.num_experts || tok >= a.n_x_rows) {
        if (lane < 16) yrow[lane] = kHalfNaN;
        return;
    }

    __shared__ uint16_t grid[MEMBER == IQ1_S_R4 ? IQK_IQ1S_GRID_SIZE : 1];
    if constexpr (MEMBER == IQ1_S_R4 && !FLOOR) {
        for (int i = lane; i < IQK_IQ1S_GRID_SIZE; i += 64) grid[i] = iqk_iq1s_grid_codes[i];
        __syncthreads();
    }

    const uint32_t *xrow = a.x + size_t(tok) * (N / 2) + 32 * lc;
    const size_t rowbase = size_t(e) * a.out_features + row0 + rsub;

    // Stream loads for all of this lane's rows, issued before any decode.
    uint4_t q[R];
    uint2_t q1[R];
    uint32_t sc[R], hb[R], ab[R], dvb[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const size_t row = rowbase + size_t(i) * RPS;
        if constexpr (MEMBER == IQ2_KS) {
            q[i] = load_u4(static_cast<const uint32_t *>(a.s0) + row * (N / 16) + 4 * lc);
            sc[i] = static_cast<const uint8_t *>(a.s1)[row * (N / 64) + lc];
            hb[i] = static_cast<const uint8_t *>(a.s2)[row * (N / 256) + lc / 4];
            ab[i] = static_cast<const uint8_t *>(a.s3)[row * (N / 256) + lc / 4];
            dvb[i] = static_cast<const uint16_t *>(a.s4)[row];
        } else if constexpr (MEMBER == IQ2_K) {
            q[i] = load_u4(static_cast<const uint32_t *>(a.s0) + row * (N / 16) + 4 * lc);
            sc[i] = static_cast<const uint16_t *>(a.s1)[row * (N / 64) + lc];
            ab[i] = static_cast<const uint8_t *>(a.s2)[row * (N / 128) + lc / 2];
            dvb[i] = static_cast<const uint16_t *>(a.s3)[row * (N / 256) + lc / 4];
        } else {
            q1[i] = *reinterpret_cast<const uint2_t *>(static_cast<const uint32_t *>(a.s0) + row * (N / 32) + 2 * lc);
            hb[i] = *reinterpret_cast<const uint32_t *>(static_cast<const uint16_t *>(a.s1) + row * (N / 32) + 2 * lc);
            dvb[i] = static_cast<const uint16_t *>(a.s2)[row];
        }
    }

    float acc[R];
    if constexpr (FLOOR) {
        // Deleted decode: every loaded word folds into an odd-prime integer
        // accumulator whose low byte reaches the output.
        uint32_t iacc = 0;
        const uint4_t *xp = reinterpret_cast<const uint4_t *>(xrow);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint4_t v = xp[i];
            iacc += (2 * i + 3) * v.x + (2 * i + 5) * v.y + (2 * i + 7) * v.z + (2 * i + 11) * v.w;
        }
#pragma unroll
        for (int i = 0; i < R; ++i) {
            if constexpr (MEMBER == IQ1_S_R4) {
                iacc += q1[i].x + 3u * q1[i].y + 59u * hb[i] + 67u * dvb[i];
            } else {
                iacc += q[i].x + 3u * q[i].y + 5u * q[i].z + 7u * q[i].w + 59u * sc[i] + 71u * ab[i] + 67u * dvb[i];
                if constexpr (MEMBER == IQ2_KS) iacc += 61u * hb[i];
            }
            acc[i] = float(iacc & 0xffu);
        }
    } else {
        LaneX lx;
        load_lane_x(xrow, lx);
        if constexpr (MEMBER == IQ2_KS) {
            float K0[2], K1[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const float xs = lx.xsum[2 * t] + lx.xsum[2 * t + 1];
                const float xl = lx.xlo[2 * t] + lx.xlo[2 * t + 1];
                K0[t] = fmaf(-288.f, xl, xs);
                K1[t] = fmaf(5.f, xs, K0[t]);
            }
            const int bsh = 2 * (lc % 4);
#pragma unroll
            for (int i = 0; i < R; ++i) {
                float tot = 0.f;
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    float a1 = 0.f, a2 = 0.f;
                    decode_word<kIq2PoolHi, kIq2PoolLo>(q[i][2 * t], lx.xa + 8 * t, lx.xb + 8 * t, a1, a2);
                    decode_word<kIq2PoolHi, kIq2PoolLo>(q[i][2 * t + 1], lx.xa + 8 * t + 4, lx.xb + 8 * t + 4, a1, a2);
                    const uint32_t nib = (sc[i] >> (4 * t)) & 15u;
                    const uint32_t hi = (hb[i] >> (bsh + t)) & 1u;
                    const uint32_t alpha = (ab[i] >> (bsh + t)) & 1u;
                    const float S = fmaf(a1, 32.f, fmaf(a2, 2.f, alpha ? K1[t] : K0[t]));
                    tot = fmaf(float(int(nib | (hi << 4)) - 16), S, tot);
                }
                acc[i] = tot * half_bits_to_float(dvb[i]);
            }
        } else if constexpr (MEMBER == IQ2_K) {
            float K0[4], K1[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                K0[w] = fmaf(-288.f, lx.xlo[w], lx.xsum[w]);
                K1[w] = fmaf(5.f, lx.xsum[w], K0[w]);
            }
            const int bsh = 4 * (lc % 2);
#pragma unroll
            for (int i = 0; i < R; ++i) {
                float tot = 0.f;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    float a1 = 0.f, a2 = 0.f;
                    decode_word<kIq2PoolHi, kIq2PoolLo>(q[i][w], lx.xa + 4 * w, lx.xb + 4 * w, a1, a2);
                    const uint32_t nib = (sc[i] >> (4 * w)) & 15u;
                    const uint32_t alpha = (ab[i] >> (bsh + w)) & 1u;
                    const float S = fmaf(a1, 32.f, fmaf(a2, 2.f, alpha ? K1[w] : K0[w]));
                    tot = fmaf(float(int(nib) - 8), S, tot);
                }
                acc[i] = tot * half_bits_to_float(dvb[i]);
            }
        } else {
            float Kp[2], Km[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const float xs = lx.xsum[2 * b] + lx.xsum[2 * b + 1];
                const float xl = lx.xlo[2 * b] + lx.xlo[2 * b + 1];
                Kp[b] = fmaf(-17.f, xl, 0.125f * xs);
                Km[b] = fmaf(-17.f, xl, -0.125f * xs);
            }
#pragma unroll
            for (int i = 0; i < R; ++i) {
                float tot = 0.f;
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const uint32_t qw = b ? q1[i].y : q1[i].x;
                    const uint32_t h = (hb[i] >> (16 * b)) & 0xffffu;
                    const uint32_t c0 = grid[(qw & 0xffu) | ((h & 7u) << 8)];
                    const uint32_t c1 = grid[((qw >> 8) & 0xffu) | (((h >> 3) & 7u) << 8)];
                    const uint32_t c2 = grid[((qw >> 16) & 0xffu) | (((h >> 6) & 7u) << 8)];
                    const uint32_t c3 = grid[(qw >> 24) | (((h >> 9) & 7u) << 8)];
                    float a1 = 0.f, a2 = 0.f;
                    decode_word<kIq1PoolHi, kIq1PoolLo>(c0 | (c1 << 16), lx.xa + 8 * b, lx.xb + 8 * b, a1, a2);
                    decode_word<kIq1PoolHi, kIq1PoolLo>(c2 | (c3 << 16), lx.xa + 8 * b + 4, lx.xb + 8 * b + 4, a1, a2);
                    const float S = fmaf(a1, 8.f, a2 + ((h & 0x8000u) ? Km[b] : Kp[b]));
                    tot = fmaf(float(2 * ((h >> 12) & 7u) + 1), S, tot);
                }
                acc[i] = tot * half_bits_to_float(dvb[i]);
            }
        }
    }

    int idx = 0;
    treduce<R, LPR / 2>(acc, lane, idx);
    if ((lane & 3) == 0) yrow[idx * RPS + rsub] = uint16_t(float_to_half_bits(acc[0]));
}

template <int MEMBER, bool FLOOR>
int launch_gemv(int64_t n, const GemvArgs &a, uint32_t mats, hipStream_t st) {
    const dim3 grid{a.out_features / 16, mats}, block{64};
    if (n == 4096)
        hipLaunchKernelGGL((gemv_kernel<MEMBER, 4096, FLOOR>), grid, block, 0, st, a);
    else
        hipLaunchKernelGGL((gemv_kernel<MEMBER, 2048, FLOOR>), grid, block, 0, st, a);
    return record_launch(hipGetLastError());
}

// The int8-MFMA path (iqk_gemv_mfma.hip); -1 when it does not apply.
int gemv_mfma_dispatch(int floor, int member, int64_t n, int64_t out, int64_t num_experts, const void *x,
                       int64_t n_x_rows, const void *const *streams, int n_streams, const uint32_t *sel,
                       const uint32_t *toks, bool union_runs, uint32_t pairs_per_row, uint32_t mats, void *y,
                       hipStream_t st);

// All GEMV entry points.  toks NULL: pair m reads x row m / pairs_per_row
// (n_x_rows = mats / pairs_per_row); else x row toks[m] < n_x_rows (a row
// beyond is a NaN output row).
// FLOOR: 0 the decode, 1 its deleted-decode floor, 2 that floor keeping
// IQ1_S_R4's grid lookups (the VALU path, which has no staged grid, serves 2
// as 1).
template <int FLOOR>
int gemv_entry(int member, int64_t n, int64_t out, int64_t num_experts, const void *x, int64_t n_x_rows,
               const void *const *streams, int n_streams, const uint32_t *sel, const uint32_t *toks,
               uint32_t pairs_per_row, uint32_t mats, void *y, void *stream, bool union_runs = false) {
    const int g = iqk_check_gemv_geometry(member, n, out);
    if (g != IQK_OK) return g;
    if (toks && member == IQK_MEMBER_IQ1_S_R4) return IQK_ERR_MEMBER;  // no sorted/union form
    if (!x || !sel || !y || !streams_ok(streams, n_streams, member)) return IQK_ERR_ARGUMENT;
    if (num_experts <= 0 || num_experts > 0xffffffffll || pairs_per_row == 0 || mats % pairs_per_row)
        return IQK_ERR_ARGUMENT;
    if (n_x_rows < 0 || n_x_rows > 0xffffffffll) return IQK_ERR_ARGUMENT;
    if (mats == 0) return IQK_OK;
    // a pair whose row is out of range reads row 0 (and writes NaN): x needs one
    if (n_x_rows == 0) return IQK_ERR_ARGUMENT;
    if (mats > 65535u) return IQK_ERR_ARGUMENT;
    hipStream_t st = as_stream(stream);
    const int r = gemv_mfma_dispatch(FLOOR, member, n, out, num_experts, x, n_x_rows, streams, n_streams, sel,
                                     toks, union_runs, pairs_per_row, mats, y, st);
    if (r >= 0) return r;
    GemvArgs a;
    a.x = static_cast<const uint32_t *>(x);
    a.s0 = streams[0]; a.s1 = streams[1]; a.s2 = streams[2];
    a.s3 = n_streams > 3 ? streams[3] : nullptr;
    a.s4 = n_streams > 4 ? streams[4] : nullptr;
    a.sel = sel;
    a.toks = toks;
    a.n_x_rows = uint32_t(n_x_rows);
    a.pairs_per_row = pairs_per_row;
    a.num_experts = uint32_t(num_experts);
    a.out_features = uint32_t(out);
    a.y = static_cast<uint16_t *>(y);
    switch (member) {
        case IQK_MEMBER_IQ2_KS: return launch_gemv<IQ2_KS, FLOOR != 0>(n, a, mats, st);
        case IQK_MEMBER_IQ2_K: return launch_gemv<IQ2_K, FLOOR != 0>(n, a, mats, st);
        default: return launch_gemv<IQ1_S_R4, FLOOR != 0>(n, a, mats, st);
    }
}

}  // namespace iqk

extern "C" {

int iqk_check_gemv_geometry(int member, int64_t n, int64_t out) {
    if (!iqk::member_ok(member)) return IQK_ERR_MEMBER;
    if (!iqk::width_sized(n)) return IQK_ERR_GEOMETRY;
    if (out <= 0 || out % 16 || out > (int64_t(1) << 24)) return IQK_ERR_GEOMETRY;
    return IQK_OK;
}

int iqk_gemv(int member, int64_t n, int64_t out, int64_t num_experts, const void *x,
             const void *const *streams, int n_streams, const uint32_t *sel, uint32_t pairs_per_row,
             uint32_t mats, void *y, void *stream) {
    const int64_t rows = pairs_per_row ? mats / pairs_per_row : 0;
    return iqk::gemv_entry<0>(member, n, out, num_experts, x, rows, streams, n_streams, sel, nullptr,
                                  pairs_per_row, mats, y, stream);
}

int iqk_gemv_floor(int member, int64_t n, int64_t out, int64_t num_experts, const void *x,
                   const void *const *streams, int n_streams, const uint32_t *sel, uint32_t pairs_per_row,
                   uint32_t mats, void *y, void *stream) {
    const int64_t rows = pairs_per_row ? mats / pairs_per_row : 0;
    return iqk::gemv_entry<1>(member, n, out, num_experts, x, rows, streams, n_streams, sel, nullptr,
                                 pairs_per_row, mats, y, stream);
}

int iqk_gemv_floor_grid(int member, int64_t n, int64_t out, int64_t num_experts, const void *x,
                        const void *const *streams, int n_streams, const uint32_t *sel, uint32_t pairs_per_row,
                        uint32_t mats, void *y, void *stream) {
    const int64_t rows = pairs_per_row ? mats / pairs_per_row : 0;
    return iqk::gemv_entry<2>(member, n, out, num_experts, x, rows, streams, n_streams, sel, nullptr,
                              pairs_per_row, mats, y, stream);
}

int iqk_gemv_sorted(int member, int64_t n, int64_t out, int64_t num_experts, const void *x, int64_t n_x_rows,
                    const void *const *streams, int n_streams, const uint32_t *sorted_ids, const uint32_t *toks,
                    uint32_t mats, void *y, void *stream) {
    if (member == IQK_MEMBER_IQ1_S_R4) return IQK_ERR_MEMBER;  // no sorted form
    if (!toks && mats) return IQK_ERR_ARGUMENT;
    return iqk::gemv_entry<0>(member, n, out, num_experts, x, n_x_rows, streams, n_streams, sorted_ids, toks,
                                   1u, mats, y, stream);
}

// The union form: adjacent pairs with one expert id share a workgroup, which
// loads and expands the expert's rows once for them (see
// gemv_mfma_union_kernel).  Where the int8-MFMA path does not apply (out not
// a multiple of 32) it is the sorted dispatch.
int iqk_gemv_union(int member, int64_t n, int64_t out, int64_t num_experts, const void *x, int64_t n_x_rows,
                   const void *const *streams, int n_streams, const uint32_t *sorted_ids, const uint32_t *toks,
                   uint32_t mats, void *y, void *stream) {
    if (member == IQK_MEMBER_IQ1_S_R4) return IQK_ERR_MEMBER;  // no union form
    if (!toks && mats) return IQK_ERR_ARGUMENT;
    return iqk::gemv_entry<0>(member, n, out, num_experts, x, n_x_rows, streams, n_streams, sorted_ids, toks,
                                   1u, mats, y, stream, true);
}

}  // extern "C"
