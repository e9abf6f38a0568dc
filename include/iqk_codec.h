// CPU codec for the routed IQ_K members: ik-wire quantizers and dequantizers.
//
// Same entry points, argument meaning and error convention as the vendored
// ik codec the reference binds through ctypes (reference:
// vendor/ik_llama/iqk_iq2.h:21-45, vendor/ik_llama/iqk_iq1sr4.h:25-46;
// bound at src/mlx_iqk/codec.py:113-181), so the reference's codec shim can
// load this library unchanged:
//
//   * row sizes return 0 for a refused geometry;
//   * quantizers return the bytes written, 0 for a refused geometry;
//   * dequantizers return 0 on success, non-zero for a refused geometry.
//
// Rows are quantized in parallel (rows of the 2-bit members and four-row
// groups of IQ1_S_R4 are independent); the bytes do not depend on the thread
// count.  IQ1_S_R4 row counts must be multiples of 4, widths multiples of 32;
// the 2-bit members need widths that are multiples of 256.
#ifndef IQK_CODEC_H
#define IQK_CODEC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// replaces iqk_iq2.h:25-26 / iqk_iq1sr4.h:27
size_t iqk_row_size_iq2_k(int64_t n_per_row);
size_t iqk_row_size_iq2_ks(int64_t n_per_row);
size_t iqk_row_size_iq1_s_r4(int64_t n_per_row);

// replaces iqk_iq2.h:31-34 / iqk_iq1sr4.h:34-35.  imatrix may be NULL.
size_t iqk_quantize_iq2_k(const float *src, void *dst, int64_t nrows,
                          int64_t n_per_row, const float *imatrix);
size_t iqk_quantize_iq2_ks(const float *src, void *dst, int64_t nrows,
                           int64_t n_per_row, const float *imatrix);
size_t iqk_quantize_iq1_s_r4(const float *src, void *dst, int64_t nrows,
                             int64_t n_per_row, const float *imatrix);

// replaces iqk_iq2.h:38-41 / iqk_iq1sr4.h:40-41
int iqk_dequantize_iq2_k(const void *src, float *dst, int64_t nrows, int64_t n_per_row);
int iqk_dequantize_iq2_ks(const void *src, float *dst, int64_t nrows, int64_t n_per_row);
int iqk_dequantize_iq1_s_r4(const void *src, float *dst, int64_t nrows, int64_t n_per_row);

// replaces iqk_iq2.h:44-45 / iqk_iq1sr4.h:44
size_t iqk_block_size_iq2_k(void);
size_t iqk_block_size_iq2_ks(void);
size_t iqk_block_size_iq1_s_r4(void);

// No counterpart in the reference (its codec is single-threaded): worker
// threads the quantizers may use; 0 restores the default (the
// IQK_CODEC_THREADS environment variable, else the CPU count).
void iqk_codec_set_threads(int threads);
int iqk_codec_threads(void);

#ifdef __cplusplus
}
#endif

#endif  // IQK_CODEC_H
