// Host-side helpers shared by the C-ABI translation units that call HIP.
#pragma once

#include <hip/hip_runtime.h>

#include "abi_common.h"

namespace ssl {

// Maps a HIP error (after a launch or API call) to SSL_ERR_HIP with its text.
int check_hip(hipError_t e, const char* what);

// Compute units of the current device (cached per device).
int device_cus();

// The checked build's status word for calls that pass none (null otherwise).
unsigned long long* check_word_ptr();

// Workspace bytes an ssl_slr_forward call cannot do without (the query reports
// more: room for the partial tiles of split prefill calls).
int64_t slr_workspace_min(int64_t M, int64_t NB, int32_t block_p, int64_t r_pad, int64_t m_pad,
                          int64_t n_slots, int32_t dtype);

}  // namespace ssl
