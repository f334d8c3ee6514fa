// Host-side helpers shared by the C-ABI translation units that call HIP.
#pragma once

#include <hip/hip_runtime.h>

#include "abi_common.h"

namespace ssl {

// Maps a HIP error (after a launch or API call) to SSL_ERR_HIP with its text.
int check_hip(hipError_t e, const char* what);

// Compute units of the current device (cached per device).
int device_cus();

}  // namespace ssl
