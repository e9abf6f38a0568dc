// Host-side helpers shared by the ABI entry points.
#ifndef IQK_HOST_H
#define IQK_HOST_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iqk_hip.h"

namespace iqk {

// Remember a launch failure's hipError_t for iqk_hip_last_error().
int record_launch(hipError_t err);

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline int stream_count(int member) {
    return member == IQK_MEMBER_IQ2_KS ? 5 : member == IQK_MEMBER_IQ2_K ? 4 : member == IQK_MEMBER_IQ1_S_R4 ? 3 : -1;
}

inline bool member_ok(int member) { return stream_count(member) > 0; }

// Widths with a sized kernel: the down (2048) and gate/up (4096) widths, the
// only ones the reference sizes (src/mlx_iqk/kernels.py:77-78).
inline bool width_sized(int64_t n) { return n == 2048 || n == 4096; }

inline bool streams_ok(const void *const *streams, int n_streams, int member) {
    if (!streams || n_streams != stream_count(member)) return false;
    for (int i = 0; i < n_streams; ++i)
        if (!streams[i]) return false;
    return true;
}

}  // namespace iqk

#endif  // IQK_HOST_H
