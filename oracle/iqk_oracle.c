/*
 * ORACLE — test infrastructure only.  Nothing in the product links, loads or
 * calls this file; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may.  It is the checker, never the thing measured.
 *
 * A plain-C, one-weight-at-a-time restatement of the reference's CPU
 * dequantizers on ik wire bytes, written from the block layouts rather than
 * from the reference's loops:
 *
 *   oracle_dequant_iq2_ks   vendor/ik_llama/iqk_iq2.cpp:532-562 (row layout 79-83)
 *   oracle_dequant_iq2_k    vendor/ik_llama/iqk_iq2.cpp:502-529 (block layout 70-75)
 *   oracle_dequant_iq1_s_r4 vendor/ik_llama/iqk_iq1sr4.cpp:581-602 (block 72-76),
 *                           decode grid vendor/ik_llama/iqk_iq1sr4.cpp:257-265
 *
 * Every reconstruction is the float32 chain y = (d * float(idx)) * float(v)
 * (IQ1_S_R4: y = (d * float(2ls+1)) * (float(g) + shift)), all products exact.
 * fp16 -> float is decoded from the bits here, independently of any compiler
 * half type.
 *
 * Pinning: tests/test_oracle.py checks these functions against the compiled
 * reference codec (oracle/_ref, where it builds), against committed golden
 * vectors made by it, and against closed forms (one-hot blocks whose every
 * weight is a known product).
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

#include "../mlx-iqk_amd/csrc/iq1s_grid.h"

static float oracle_half(uint16_t h) {
    int sign = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(1024 + m), e - 25);
    return sign ? -v : v;
}

static const int oracle_values[8] = {-31, -13, 1, 17, -26, -8, 6, 22};

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* IQ2_KS row: d f16, then per 256 weights {extra u16, scales[4], qs[64]}. */
static void dequant_row_iq2_ks(const uint8_t *row, float *y, int n) {
    float d = oracle_half(rd16(row));
    for (int k = 0; k < n; ++k) {
        const uint8_t *blk = row + 2 + 70 * (k / 256);
        int w = k % 256;
        int sb = w / 32;                       /* 32-weight sub-block */
        uint16_t extra = rd16(blk);
        int lo = (blk[2 + sb / 2] >> (4 * (sb % 2))) & 15;
        int hi = (extra >> (8 + sb)) & 1;
        int alpha = (extra >> sb) & 1;
        int byte = 32 * (w / 128) + (w % 32);
        int code = (blk[6 + byte] >> (2 * (sb % 4))) & 3;
        float dl = d * (float)((lo | (hi << 4)) - 16);
        y[k] = dl * (float)oracle_values[4 * alpha + code];
    }
}

/* IQ2_K block: {d f16, extra u16, scales[8], qs[64]} per 256 weights. */
static void dequant_row_iq2_k(const uint8_t *row, float *y, int n) {
    for (int k = 0; k < n; ++k) {
        const uint8_t *blk = row + 76 * (k / 256);
        int w = k % 256;
        int sb = w / 16;                       /* 16-weight sub-block */
        float d = oracle_half(rd16(blk));
        uint16_t extra = rd16(blk + 2);
        int idx = ((blk[4 + sb / 2] >> (4 * (sb % 2))) & 15) - 8;
        int alpha = (extra >> sb) & 1;
        int byte = 32 * (w / 128) + 16 * ((w / 16) % 2) + (w % 16);
        int code = (blk[12 + byte] >> (2 * ((w / 32) % 4))) & 3;
        float dl = d * (float)idx;
        y[k] = dl * (float)oracle_values[4 * alpha + code];
    }
}

/* IQ1_S_R4 four-row group: 4 x d f16, then per 32 weights
 * {qs[16] (byte 4i+k: row k, sub-group i), qh[4] u16 (row k)}. */
static void dequant_group_iq1_s_r4(const uint8_t *grp, float *y, int n) {
    for (int r = 0; r < 4; ++r) {
        float d = oracle_half(rd16(grp + 2 * r));
        for (int k = 0; k < n; ++k) {
            const uint8_t *blk = grp + 8 + 24 * (k / 32);
            int i = (k % 32) / 8, j = k % 8;
            uint16_t qh = rd16(blk + 16 + 2 * r);
            int index = blk[4 * i + r] | (((qh >> (3 * i)) & 7) << 8);
            int g = (int)((iqk_iq1s_grid_codes[index] >> (2 * j)) & 3) - 1;
            float shift = (qh & 0x8000) ? -0.125f : 0.125f;
            float dl = d * (float)(2 * ((qh >> 12) & 7) + 1);
            y[(int64_t)r * n + k] = dl * ((float)g + shift);
        }
    }
}

int oracle_dequant_iq2_ks(const void *src, float *dst, int64_t rows, int64_t n) {
    if (n <= 0 || n % 256 || rows < 0) return 1;
    size_t rb = 2 + 70 * (size_t)(n / 256);
    for (int64_t r = 0; r < rows; ++r)
        dequant_row_iq2_ks((const uint8_t *)src + r * rb, dst + r * n, (int)n);
    return 0;
}

int oracle_dequant_iq2_k(const void *src, float *dst, int64_t rows, int64_t n) {
    if (n <= 0 || n % 256 || rows < 0) return 1;
    size_t rb = 76 * (size_t)(n / 256);
    for (int64_t r = 0; r < rows; ++r)
        dequant_row_iq2_k((const uint8_t *)src + r * rb, dst + r * n, (int)n);
    return 0;
}

int oracle_dequant_iq1_s_r4(const void *src, float *dst, int64_t rows, int64_t n) {
    if (n <= 0 || n % 32 || rows <= 0 || rows % 4) return 1;
    size_t rb = 2 + 6 * (size_t)(n / 32);
    for (int64_t r = 0; r < rows; r += 4)
        dequant_group_iq1_s_r4((const uint8_t *)src + r * rb, dst + r * n, (int)n);
    return 0;
}
