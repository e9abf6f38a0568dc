// MI355X (gfx950) routed-expert kernels for the IQ_K relayout: the C ABI.
//
// This library replaces the reference's kernel seam: Metal source built per
// geometry and dispatched through mx.fast.metal_kernel (reference:
// src/mlx_iqk/kernels.py:751-887, called from src/mlx_iqk/nn.py:155-271).
// Every entry point is asynchronous on the caller's HIP stream (`stream` is
// a hipStream_t; NULL is the default stream), takes device pointers only,
// allocates nothing and never synchronises.
//
// Return codes: IQK_OK, or a refusal raised before anything is launched
// (unknown member, unsized geometry, bad argument), or IQK_ERR_LAUNCH with the
// HIP error kept for iqk_hip_last_error().  The reference refuses the same
// geometries in Python before compiling (src/mlx_iqk/kernels.py:100-142);
// here the refusal is also enforced at the ABI, so a caller that skips the
// Python guards still cannot launch an unsized kernel.
//
// Streams: the member's relayout streams in component order, each a
// contiguous stacked tensor [num_experts, out_features, ...]:
//   IQ2_KS   qs u32, scl u8, sch u8, sex u8, dv f16        (5 streams)
//   IQ2_K    qs u32, scl u8, sex u8, dv f16                (4 streams)
//   IQ1_S_R4 qs u32, qh u16, dv f16                        (3 streams)
// The shared tables (the fp16 alphabet, the IQ1_S grid) are compiled into
// the library; the reference passes them as kernel inputs instead
// (src/mlx_iqk/nn.py:56-94).
//
// Expert ids read from device memory are bounds-checked in the kernels: an
// id >= num_experts produces NaN outputs for that pair (or skips that expert
// in the producer), never an out-of-bounds read.
#ifndef IQK_HIP_H
#define IQK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IQK_HIP_ABI_VERSION 5

#define IQK_MEMBER_IQ2_KS 0
#define IQK_MEMBER_IQ2_K 1
#define IQK_MEMBER_IQ1_S_R4 2

#define IQK_OK 0
#define IQK_ERR_MEMBER 1
#define IQK_ERR_GEOMETRY 2
#define IQK_ERR_ARGUMENT 3
#define IQK_ERR_LAUNCH 4

int iqk_hip_abi_version(void);
// The hipError_t of the most recent IQK_ERR_LAUNCH on this thread (0 if none).
int iqk_hip_last_error(void);
// No counterpart in the reference (its kernels compile from source at run
// time): a digest of the sources and flags this library was built from, so a
// loader can refuse a stale build (NUL-terminated hex, static storage).
const char *iqk_hip_source_hash(void);
// Geometry guards, the ABI form of check_gemv_geometry / check_dequant_geometry
// (reference: src/mlx_iqk/kernels.py:100-129): IQK_OK or the refusal code.
int iqk_check_gemv_geometry(int member, int64_t in_features, int64_t out_features);
int iqk_check_dequant_geometry(int member, int64_t in_features, int64_t out_features);

// Decode GEMV over token-expert pairs (replaces gemv_kernel + its dispatch,
// src/mlx_iqk/kernels.py:792-810, src/mlx_iqk/nn.py:240-271):
//   y[m, r] = fp16( sum_k W[sel[m]][r][k] * x[m / pairs_per_row][k] )
// x: f16 [mats / pairs_per_row, in_features]; sel: u32 [mats] (device);
// y: f16 [mats, out_features].  pairs_per_row is the reference's `dims`.
int iqk_gemv(int member, int64_t in_features, int64_t out_features, int64_t num_experts,
             const void *x, const void *const *streams, int n_streams,
             const uint32_t *sel, uint32_t pairs_per_row, uint32_t mats,
             void *y, void *stream);

// The GEMV's deleted-decode floor: identical loads, the decode replaced by an
// integer fold of every loaded word that reaches y (reference:
// bench/floors.py:86-176).  Same arguments; y holds no meaningful values.
int iqk_gemv_floor(int member, int64_t in_features, int64_t out_features, int64_t num_experts,
                   const void *x, const void *const *streams, int n_streams,
                   const uint32_t *sel, uint32_t pairs_per_row, uint32_t mats,
                   void *y, void *stream);

// IQ1_S_R4's floor as the reference prices it (bench/floors.py:14-17): the
// deleted-decode floor with the decode's grid lookups kept -- the grid staged
// in LDS and every entry the blocks index read, folded into the hash.  The
// other members have no lookups: for them this is iqk_gemv_floor.  Same
// arguments as iqk_gemv_floor.
int iqk_gemv_floor_grid(int member, int64_t in_features, int64_t out_features, int64_t num_experts,
                        const void *x, const void *const *streams, int n_streams,
                        const uint32_t *sel, uint32_t pairs_per_row, uint32_t mats,
                        void *y, void *stream);

// The pure byte-stream floor of the pricing (no counterpart in the
// reference's kernel seam; the reference prices against its deleted-decode
// floors only): one dispatch that reads `bytes` contiguous bytes of src (16-byte
// aligned, bytes a multiple of 16) with no expert-id read and no decode, and
// writes a fold of them to out (u32 [ceil(bytes / 4096)], no meaningful values).
int iqk_stream_floor(const void *src, uint64_t bytes, uint32_t *out, void *stream);
// No counterpart either: the byte-stream floor with more bytes in flight --
// each lane issues loads_per_lane (4, 8 or 16) 16-byte loads before folding
// any, and at most max_waves wavefronts (0: one per chunk) stride over the
// span in chunks of loads_per_lane KiB.  `out` holds one u32 per wavefront:
// blocks of four wavefronts covering min(chunks, max_waves or chunks).
int iqk_stream_floor_wide(const void *src, uint64_t bytes, int loads_per_lane, uint64_t max_waves, uint32_t *out,
                          void *stream);

// Decode GEMV over expert-sorted pairs, one workgroup per pair (replaces
// gemv_sorted_kernel + IqkSwitchLinear.gemv_sorted,
// src/mlx_iqk/kernels.py:404-482, 813-832, src/mlx_iqk/nn.py:273-299):
//   y[p, r] = fp16( sum_k W[sorted_ids[p]][r][k] * x[toks[p]][k] )
// x: f16 [n_x_rows, in_features]; sorted_ids, toks: u32 [mats] (device);
// y: f16 [mats, out_features].  Each output element is iqk_gemv's, bit for
// bit, so y is iqk_gemv's rows in the caller's sorted order.  A pair whose
// toks entry is >= n_x_rows, or whose id is >= num_experts, gets a NaN row.
// IQK_MEMBER_IQ2_KS and IQK_MEMBER_IQ2_K only (IQ1_S_R4: IQK_ERR_MEMBER).
int iqk_gemv_sorted(int member, int64_t in_features, int64_t out_features, int64_t num_experts,
                    const void *x, int64_t n_x_rows, const void *const *streams, int n_streams,
                    const uint32_t *sorted_ids, const uint32_t *toks, uint32_t mats,
                    void *y, void *stream);

// The same contraction, each run of equal adjacent ids decoded together
// (replaces gemv_union_kernel + IqkSwitchLinear.gemv_union,
// src/mlx_iqk/kernels.py:484-578, 834-853, src/mlx_iqk/nn.py:301-333).
// Arguments, output and refusals as iqk_gemv_sorted.  A workgroup serves
// three adjacent pairs (pairs 3z .. 3z+2): for each run of equal ids among
// them it loads and expands the expert's rows once and runs each pair's MFMAs
// and folds on them, so every output element is iqk_gemv's, bit for bit.
// (The reference computes a whole run in one threadgroup; here a run is cut
// at multiples of three: more staged pairs a workgroup cost occupancy.)
int iqk_gemv_union(int member, int64_t in_features, int64_t out_features, int64_t num_experts,
                   const void *x, int64_t n_x_rows, const void *const *streams, int n_streams,
                   const uint32_t *sorted_ids, const uint32_t *toks, uint32_t mats,
                   void *y, void *stream);

// Stacked-expert dequant producer (replaces dequant_kernel + dispatch,
// src/mlx_iqk/kernels.py:855-869, src/mlx_iqk/nn.py:155-169):
//   w[slot(e)][r][k] = fp16( d * float(index) * value )   bit-exact,
// for every source expert e < num_experts with 0 <= slot(e) < n_slots;
// slot(e) = slot_of_expert[e] (device i32 [num_experts]) or e when the
// pointer is NULL.  Experts with no slot are skipped.  w: f16 [n_slots,
// out_features, in_features].
int iqk_dequant(int member, int64_t in_features, int64_t out_features, int64_t num_experts,
                const void *const *streams, int n_streams,
                const int32_t *slot_of_expert, int64_t n_slots,
                void *w, void *stream);

// The producer over out-row range [row_start, row_start + rows) (replaces
// dequant_range_kernel + IqkSwitchLinear.dequantized_range,
// src/mlx_iqk/kernels.py:679-758, 872-888, src/mlx_iqk/nn.py:171-201):
//   w[slot(e)][r][k] = the full producer's w[slot(e)][row_start + r][k]
// bit for bit, w: f16 [n_slots, rows, in_features], slots as iqk_dequant.
// IQK_ERR_GEOMETRY unless 0 <= row_start, 0 < rows and
// row_start + rows <= out_features.  iqk_dequant is the case row_start = 0,
// rows = out_features.
int iqk_dequant_rows(int member, int64_t in_features, int64_t out_features, int64_t num_experts,
                     const void *const *streams, int n_streams, int64_t row_start, int64_t rows,
                     const int32_t *slot_of_expert, int64_t n_slots,
                     void *w, void *stream);

// The producer's floor: identical loads and stores, decode deleted
// (reference: bench/floors.py:179-220).
int iqk_dequant_floor(int member, int64_t in_features, int64_t out_features, int64_t num_experts,
                      const void *const *streams, int n_streams,
                      const int32_t *slot_of_expert, int64_t n_slots,
                      void *w, void *stream);

// Sorted grouped GEMM on fp16 MFMA with f32 accumulation, the prefill
// contraction (replaces mx.gather_mm(x, W.swapaxes(-1,-2), rhs_indices,
// sorted_indices=True), src/mlx_iqk/nn.py:221-238).  Work items ("slots")
// are sorted by group; group g owns slots [group_offsets[g],
// group_offsets[g+1]).  For slot p:
//   y[y_rows[p]][n] = fp16( sum_k x[x_rows[p]][k] * w[g][n][k] )
// x: f16 [n_x_rows, in_features]; w: f16 [n_groups, out_features, in_features];
// y: f16 [n_slots, out_features]; group_offsets: u32 [n_groups + 1] (device,
// non-decreasing, last = n_slots); x_rows, y_rows: u32 [n_slots] (device;
// y_rows NULL = identity, else a permutation of [0, n_slots)).  Device-side
// indices out of range are never dereferenced: a slot whose x_rows entry is
// >= n_x_rows gets a NaN output row, a y_rows entry >= n_slots is not
// stored.  in_features % 32 == 0;
// any out_features > 0.
int iqk_grouped_gemm(int64_t in_features, int64_t out_features, int64_t n_groups, int64_t n_slots,
                     const void *x, int64_t n_x_rows, const void *w, const uint32_t *group_offsets,
                     const uint32_t *x_rows, const uint32_t *y_rows, void *y, void *stream);

// Fused prefill contraction straight from the streams: the weights formed
// inside an fp16 MFMA grouped GEMM, never stored (replaces dequant_kernel /
// dequant_range_kernel + mx.gather_mm(x, W.swapaxes(-1,-2), rhs_indices,
// sorted_indices=True), src/mlx_iqk/nn.py:155-238).  Slots are sorted by
// expert; expert e owns slots [group_offsets[e], group_offsets[e+1]):
//   y[y_rows[p]][n] = fp16( sum_k x[x_rows[p]][k] * W[e][row_start + n][k] ),
// 0 <= n < rows, f32 accumulation.  IQ2_K: W is iqk_dequant's fp16 value bit
// for bit.  IQ2_KS, IQ1_S_R4 (one scale d a row): the sum runs over the
// exact products n = W / d and is multiplied by d once, so W enters
// unrounded (a one-hot x row yields iqk_dequant's fp16 weight).  The
// summation order differs from iqk_dequant + iqk_grouped_gemm; it does not
// depend on row_start, so row ranges concatenate to the full call bit for
// bit.  y: f16 [n_slots, rows];
// group_offsets: u32 [num_experts + 1] (device, non-decreasing, last =
// n_slots); x, x_rows, y_rows as iqk_grouped_gemm.  IQK_ERR_GEOMETRY unless
// 0 <= row_start < row_start + rows <= out_features.  All three members.
int iqk_fused_gemm(int member, int64_t in_features, int64_t out_features, int64_t num_experts,
                   const void *x, int64_t n_x_rows, const void *const *streams, int n_streams,
                   int64_t row_start, int64_t rows, const uint32_t *group_offsets,
                   const uint32_t *x_rows, const uint32_t *y_rows, int64_t n_slots,
                   void *y, void *stream);

// The prefill route's grouping of token-expert pairs into expert-sorted
// slots, on the device, in one launch (replaces the pair sort the reference's
// sorting caller performs, mlx_lm's _gather_sort, and the grouping inside
// mx.gather_mm's sorted path, src/mlx_iqk/nn.py:221-238).  Pair p names
// expert ids[p] (u32) and owns rows_per_pair slots; its activation rows are
// (p / pairs_per_x_row) * rows_per_pair + r, its output rows p *
// rows_per_pair + r (r < rows_per_pair).  Outputs, ready for iqk_fused_gemm
// and iqk_grouped_gemm: group_offsets u32 [num_experts + 1] (slots of
// experts < e; the last is n_pairs * rows_per_pair), and per slot x_rows and
// y_rows u32 [n_pairs * rows_per_pair].  Slots are sorted by expert and keep
// the pairs' order within an expert, so the lists are the same on every
// call.  An id >= num_experts counts for expert 0 with x_rows = n_x_rows, so
// the prefill kernels give its rows NaN and read nothing.  num_experts <=
// 4096; n_x_rows must hold every activation row a pair names.
int iqk_route(const uint32_t *ids, int64_t n_pairs, int64_t num_experts, int64_t rows_per_pair,
              int64_t pairs_per_x_row, int64_t n_x_rows, uint32_t *group_offsets, uint32_t *x_rows,
              uint32_t *y_rows, void *stream);

// ik wire rows -> the member's relayout streams, on the GPU (replaces
// format.pack for rows already in device memory, src/mlx_iqk/format.py:478-588,
// 612-678): the bytes pack writes, bit for bit.  wire: u8 [rows, ik row bytes]
// (4-byte aligned); streams: the member's planes in component order, each
// [rows, ...] contiguous (qs 16-byte aligned, the others 4-byte aligned).
// in_features: a multiple of 256 (IQ1_S_R4: of 32); IQ1_S_R4 rows: a multiple
// of 4 (its four-row groups).
int iqk_pack(int member, int64_t in_features, int64_t rows, const void *wire,
             void *const *streams, int n_streams, void *stream);

#ifdef __cplusplus
}
#endif

#endif  // IQK_HIP_H
