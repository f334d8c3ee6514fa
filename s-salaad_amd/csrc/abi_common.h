// Host-side helpers shared by the C-ABI translation units that need no HIP
// runtime (the planners build with a plain C++ compiler too).
#pragma once

#include <stdint.h>

#include "../../include/ssalaad_amd.h"

// 1 in the library's checked build (device bounds checks; slr_common.h)
#ifndef SSL_DEVICE_CHECKS
#define SSL_DEVICE_CHECKS 0
#endif

namespace ssl {

// Records `msg` as the thread's last error and returns `code`.
int fail(int code, const char* fmt, ...);
void clear_error();

inline int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }
inline bool aligned(const void* p, int64_t a) { return ((uintptr_t)p % (uintptr_t)a) == 0; }
inline int elem_bytes(int dtype) { return dtype == SSL_F32 ? 4 : 2; }

// Token rows per workgroup tile (16 · MT) for a call with M rows.
inline int tile_mt(int64_t M) { return M <= 16 ? 1 : (M <= 32 ? 2 : 4); }

// Test hooks set through ssl_debug_set (host-side values read at launch time).
struct DebugKnobs {
  int64_t prefill_group;  // 0: the library's choice; 1: narrow, 2: tall row tiles
  int64_t wait_polls;     // polls before a bounded wait gives up (0: the default)
  int64_t wait_unreachable;  // nonzero: every wait's target is out of reach
  int64_t prefill_split;     // 0: the library's choice; 1: never; 2-4: that many parts
  int64_t chain_frag;        // 0: the library's choice; 1: never; 2: always (32/64-wide)
  int64_t topk_groups;       // 0: the library's choice; 1: one workgroup; 2: many
};
DebugKnobs& debug_knobs();

}  // namespace ssl
