// ik wire -> relayout streams on the GPU (gfx950): format.pack for rows
// already in device memory.
//
// Reference: the relayout is src/mlx_iqk/format.py:478-588 (per member) and
// :612-678 (pack), done there on the CPU in numpy.  The bytes written here are
// pack's, bit for bit.
//
// A block takes whole wire rows (IQ1_S_R4: whole four-row groups), copies
// their contiguous wire bytes into LDS with dword loads (a block's rows start
// 4-byte aligned: it takes an even number of rows, and every wire row is an
// even number of bytes), and then one thread per 256-weight block (IQ1_S_R4:
// per 32-weight block of a group) reads its bytes from LDS and writes its
// share of every output plane; consecutive threads write consecutive bytes of
// each plane's row.
//
// 2-bit members: wire qs byte 32h + 16f + j (h, f in {0,1}, j < 16) carries
// in field s (bits 2s, 2s+1) the code of weight 128h + 32s + 16f + j, so
// relayout word W of a block (weights 16W .. 16W+15) gathers field
// s = (W / 2) % 4 of wire bytes 32(W / 8) + 16(W % 2) + 0..15.

#include <algorithm>

#include "iqk_device.h"
#include "iqk_host.h"

namespace iqk {

constexpr int kPackThreads = 256;
constexpr int kPackLdsBytes = 40960;
constexpr int kPackBatch = 8;  // wire dwords a thread loads before it stores them

struct PackArgs {
    const uint8_t *wire;
    void *s0, *s1, *s2, *s3, *s4;
    uint32_t rows;       // wire rows (IQ1_S_R4: a multiple of 4)
    uint32_t row_bytes;  // ik wire bytes per row
    uint32_t nb;         // blocks per row (IQ1_S_R4: 32-weight blocks)
    uint32_t rows_per_block;
};

// `count` bytes of LDS starting at byte `off` (any alignment) as words.
__device__ __forceinline__ void lds_words(const uint8_t *lds, uint32_t off, uint32_t *out, int count_words) {
    const uint32_t *base = reinterpret_cast<const uint32_t *>(lds + (off & ~3u));
    const uint32_t sh = off & 3u;
    uint32_t prev = base[0];
    for (int i = 0; i < count_words; ++i) {
        const uint32_t next = base[i + 1];
        out[i] = __builtin_amdgcn_alignbyte(next, prev, sh);
        prev = next;
    }
}

// Field s of the four bytes of q, packed as four 2-bit codes (byte k's field
// at bits 2k, 2k+1).
__device__ __forceinline__ uint32_t gather_field(uint32_t q, int s) {
    const uint32_t t = (q >> (2 * s)) & 0x03030303u;
    const uint32_t u = t | (t >> 6);
    return (u | (u >> 12)) & 0xffu;
}

// The 16 relayout words of one 256-weight block from its 64 wire qs bytes.
__device__ __forceinline__ void relayout_codes(const uint32_t *q, uint32_t *out) {
#pragma unroll
    for (int w = 0; w < 16; ++w) {
        const uint32_t *src = q + 8 * (w >> 3) + 4 * (w & 1);  // wire bytes 32h + 16f .. +15
        const int s = (w >> 1) & 3;
        out[w] = gather_field(src[0], s) | (gather_field(src[1], s) << 8) | (gather_field(src[2], s) << 16) |
                 (gather_field(src[3], s) << 24);
    }
}

template <int MEMBER>
__global__ __launch_bounds__(kPackThreads) void pack_kernel(PackArgs a) {
    // the block's wire rows (+ 16 bytes, read past by lds_words): sized at
    // launch, so a CU holds as many blocks as their rows allow
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x;
    const uint32_t r0 = blockIdx.x * a.rows_per_block;
    const uint32_t rows_here = min(a.rows_per_block, a.rows - r0);
    const uint64_t first = uint64_t(r0) * a.row_bytes;  // 4-byte aligned (even rows per block, even row bytes)
    const uint32_t bytes = rows_here * a.row_bytes;
    const uint32_t *src = reinterpret_cast<const uint32_t *>(a.wire + first);
    // in batches of kPackBatch loads a thread, all issued before any store,
    // so the copy costs a memory latency a batch, not one per dword
    const uint32_t words = bytes / 4;
    for (uint32_t i0 = 0; i0 < words; i0 += kPackBatch * kPackThreads) {
        uint32_t v[kPackBatch];
#pragma unroll
        for (int j = 0; j < kPackBatch; ++j) {
            const uint32_t i = i0 + uint32_t(j * kPackThreads + tid);
            v[j] = src[min(i, words - 1u)];  // past the end: re-reads the last dword, never stored
        }
#pragma unroll
        for (int j = 0; j < kPackBatch; ++j) {
            const uint32_t i = i0 + uint32_t(j * kPackThreads + tid);
            if (i < words) reinterpret_cast<uint32_t *>(lds)[i] = v[j];
        }
    }
    if ((bytes & 3u) && tid == 0)  // an odd last row leaves one 16-bit unit
        *reinterpret_cast<uint16_t *>(lds + (bytes & ~3u)) = *reinterpret_cast<const uint16_t *>(a.wire + first + (bytes & ~3u));
    __syncthreads();

    if constexpr (MEMBER == IQ2_KS || MEMBER == IQ2_K) {
        const uint32_t items = rows_here * a.nb;
        for (uint32_t it = tid; it < items; it += kPackThreads) {
            const uint32_t rl = it / a.nb, b = it - rl * a.nb;
            const uint64_t row = r0 + rl;
            const uint32_t rbase = rl * a.row_bytes;
            uint32_t q[16], words[16];
            if constexpr (MEMBER == IQ2_KS) {  // [d f16] then blocks [extra u16, scales[4], qs[64]]
                const uint32_t off = rbase + 2 + 70 * b;
                uint32_t hdr[2];
                lds_words(lds, off, hdr, 2);
                lds_words(lds, off + 6, q, 16);
                static_cast<uint8_t *>(a.s3)[row * a.nb + b] = uint8_t(hdr[0]);        // sex: extra low byte
                static_cast<uint8_t *>(a.s2)[row * a.nb + b] = uint8_t(hdr[0] >> 8);   // sch: extra high byte
                static_cast<uint32_t *>(a.s1)[row * a.nb + b] = __builtin_amdgcn_alignbyte(hdr[1], hdr[0], 2);  // scales[4]
                if (b == 0) static_cast<uint16_t *>(a.s4)[row] = *reinterpret_cast<const uint16_t *>(lds + rbase);
            } else {  // blocks [d f16, extra u16, scales[8], qs[64]]
                const uint32_t off = rbase + 76 * b;
                uint32_t hdr[3];
                lds_words(lds, off, hdr, 3);
                lds_words(lds, off + 12, q, 16);
                static_cast<uint16_t *>(a.s3)[row * a.nb + b] = uint16_t(hdr[0]);            // dv
                static_cast<uint16_t *>(a.s2)[row * a.nb + b] = uint16_t(hdr[0] >> 16);      // sex, 2 bytes (LE)
                uint32_t *scl = reinterpret_cast<uint32_t *>(static_cast<uint8_t *>(a.s1) + (row * a.nb + b) * 8);
                scl[0] = hdr[1];
                scl[1] = hdr[2];
            }
            relayout_codes(q, words);
            uint4_t *qs = reinterpret_cast<uint4_t *>(static_cast<uint32_t *>(a.s0) + (row * a.nb + b) * 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) qs[i] = uint4_t{words[4 * i], words[4 * i + 1], words[4 * i + 2], words[4 * i + 3]};
        }
    } else {  // IQ1_S_R4: groups [d f16 x4] then blocks [qs[16] (byte 4t + k: row k), qh u16 x4]
        const uint32_t gbytes = 4 * a.row_bytes;
        const uint32_t items = (rows_here / 4) * a.nb;
        for (uint32_t it = tid; it < items; it += kPackThreads) {
            const uint32_t gl = it / a.nb, b = it - gl * a.nb;
            const uint64_t row = r0 + 4 * gl;  // first row of the group
            const uint32_t gbase = gl * gbytes;
            const uint32_t *blk = reinterpret_cast<const uint32_t *>(lds + gbase + 8 + 24 * b);  // 4-byte aligned
            const uint32_t q0 = blk[0], q1 = blk[1], q2 = blk[2], q3 = blk[3];
            const uint32_t t01 = perm(q1, q0, 0x05010400u), t23 = perm(q3, q2, 0x05010400u);  // bytes 0, 1
            const uint32_t u01 = perm(q1, q0, 0x07030602u), u23 = perm(q3, q2, 0x07030602u);  // bytes 2, 3
            const uint32_t rq[4] = {perm(t23, t01, 0x05040100u), perm(t23, t01, 0x07060302u),
                                    perm(u23, u01, 0x05040100u), perm(u23, u01, 0x07060302u)};
            const uint32_t h01 = blk[4], h23 = blk[5];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                static_cast<uint32_t *>(a.s0)[(row + k) * a.nb + b] = rq[k];
                static_cast<uint16_t *>(a.s1)[(row + k) * a.nb + b] = uint16_t((k < 2 ? h01 : h23) >> (16 * (k & 1)));
            }
            if (b == 0) {
                const uint32_t *dv = reinterpret_cast<const uint32_t *>(lds + gbase);
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    static_cast<uint16_t *>(a.s2)[row + k] = uint16_t(dv[k >> 1] >> (16 * (k & 1)));
            }
        }
    }
}

}  // namespace iqk

extern "C" int iqk_pack(int member, int64_t in_features, int64_t rows, const void *wire, void *const *streams,
                        int n_streams, void *stream) {
    using namespace iqk;
    if (!member_ok(member)) return IQK_ERR_MEMBER;
    const bool iq1 = member == IQK_MEMBER_IQ1_S_R4;
    const int64_t block = iq1 ? 32 : 256;
    if (in_features <= 0 || in_features % block || in_features > (int64_t(1) << 20)) return IQK_ERR_GEOMETRY;
    if (rows < 0 || rows > 0xffffffffll || (iq1 && rows % 4)) return IQK_ERR_GEOMETRY;
    if (rows == 0) return IQK_OK;
    if (!wire || !streams || n_streams != stream_count(member)) return IQK_ERR_ARGUMENT;
    for (int i = 0; i < n_streams; ++i)
        if (!streams[i]) return IQK_ERR_ARGUMENT;
    // the kernel reads the wire as dwords and writes code words 16 bytes at a time
    if (reinterpret_cast<uintptr_t>(wire) % 4 || reinterpret_cast<uintptr_t>(streams[0]) % 16) return IQK_ERR_ARGUMENT;
    for (int i = 1; i < n_streams; ++i)
        if (reinterpret_cast<uintptr_t>(streams[i]) % 4) return IQK_ERR_ARGUMENT;
    const int64_t nb = in_features / block;
    const int64_t row_bytes = member == IQK_MEMBER_IQ2_KS ? 2 + 70 * nb : member == IQK_MEMBER_IQ2_K ? 76 * nb : 2 + 6 * nb;
    if (rows * row_bytes > (int64_t(1) << 40)) return IQK_ERR_ARGUMENT;
    // rows per block: an even number (a multiple of 4 for IQ1_S_R4) whose bytes fit the LDS copy,
    // about 256 work items per block
    const int64_t unit = iq1 ? 4 : 2;
    const int64_t per_unit_items = iq1 ? nb : 2 * nb;
    int64_t units = std::max<int64_t>(1, kPackThreads / per_unit_items);
    units = std::min<int64_t>(units, kPackLdsBytes / (unit * row_bytes));
    if (units < 1) return IQK_ERR_GEOMETRY;  // one row group does not fit the LDS copy
    PackArgs a;
    a.wire = static_cast<const uint8_t *>(wire);
    a.s0 = streams[0]; a.s1 = streams[1]; a.s2 = streams[2];
    a.s3 = n_streams > 3 ? streams[3] : nullptr;
    a.s4 = n_streams > 4 ? streams[4] : nullptr;
    a.rows = uint32_t(rows);
    a.row_bytes = uint32_t(row_bytes);
    a.nb = uint32_t(nb);
    a.rows_per_block = uint32_t(units * unit);
    const dim3 grid{uint32_t((rows + a.rows_per_block - 1) / a.rows_per_block)}, blk{kPackThreads};
    const size_t lds = (size_t(a.rows_per_block) * a.row_bytes + 16 + 15) / 16 * 16;
    hipStream_t st = as_stream(stream);
    switch (member) {
        case IQK_MEMBER_IQ2_KS: hipLaunchKernelGGL(pack_kernel<IQ2_KS>, grid, blk, lds, st, a); break;
        case IQK_MEMBER_IQ2_K: hipLaunchKernelGGL(pack_kernel<IQ2_K>, grid, blk, lds, st, a); break;
        default: hipLaunchKernelGGL(pack_kernel<IQ1_S_R4>, grid, blk, lds, st, a); break;
    }
    return record_launch(hipGetLastError());
}
