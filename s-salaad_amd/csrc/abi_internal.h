// Host-side helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ssalaad_amd.h"

namespace ssl {

// Records `msg` as the thread's last error and returns `code`.
int fail(int code, const char* fmt, ...);
// Maps a HIP error (after a launch or API call) to SSL_ERR_HIP with its text.
int check_hip(hipError_t e, const char* what);
void clear_error();

inline int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }
inline bool aligned(const void* p, int64_t a) { return ((uintptr_t)p % (uintptr_t)a) == 0; }
inline int elem_bytes(int dtype) { return dtype == SSL_F32 ? 4 : 2; }

// Token rows per workgroup tile (16 · MT) for a call with M rows.
inline int tile_mt(int64_t M) { return M <= 16 ? 1 : (M <= 32 ? 2 : 4); }

}  // namespace ssl
