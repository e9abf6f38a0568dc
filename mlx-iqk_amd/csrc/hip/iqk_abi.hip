// ABI bookkeeping shared by every entry point.
#include "iqk_host.h"

#ifndef IQK_SOURCE_HASH
#define IQK_SOURCE_HASH "unknown"
#endif

namespace iqk {

static thread_local int g_last_hip_error = 0;

int record_launch(hipError_t err) {
    if (err == hipSuccess) return IQK_OK;
    g_last_hip_error = int(err);
    return IQK_ERR_LAUNCH;
}

}  // namespace iqk

extern "C" {

int iqk_hip_abi_version(void) { return IQK_HIP_ABI_VERSION; }

int iqk_hip_last_error(void) { return iqk::g_last_hip_error; }

const char *iqk_hip_source_hash(void) { return IQK_SOURCE_HASH; }

}  // extern "C"
