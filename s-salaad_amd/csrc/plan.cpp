// Host-side work planning and error reporting for the C ABI.
//
// A plan turns a BSR structure into workgroup chunks. Block-row `by` owns the
// unit list [its nblk sparse blocks][lr_units low-rank units]; units cost q
// (one q-wide block of p rows) or 32 (32 ranks of p rows of A). Rows costing
// more than `target_cost` are split into k nearly equal consecutive chunks.
// This is the load-balancing step for skewed block structures: a row with ten
// times the mean block count gets ten times as many workgroups.
#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "abi_internal.h"

namespace ssl {

static thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return SSL_OK;
  return fail(SSL_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

void clear_error() { g_last_error.clear(); }

}  // namespace ssl

using namespace ssl;

extern "C" {

int ssl_version(void) { return 1; }

const char* ssl_last_error(void) { return g_last_error.c_str(); }

int ssl_plan_build(const int32_t* crow_host, int64_t NB, const int32_t* rows_host, int64_t n_rows,
                   int32_t block_q, int32_t lr_units, int64_t target_cost, int32_t* table_out,
                   int64_t table_capacity, int64_t* n_chunks, int64_t* n_slots) {
  clear_error();
  if (!crow_host || !n_chunks || !n_slots || NB < 0 || block_q <= 0 || lr_units < 0)
    return fail(SSL_ERR_INVALID, "invalid plan arguments");
  if (crow_host[0] != 0) return fail(SSL_ERR_INVALID, "crow[0] must be 0");
  for (int64_t b = 0; b < NB; ++b)
    if (crow_host[b + 1] < crow_host[b]) return fail(SSL_ERR_INVALID, "crow must be non-decreasing");
  const int64_t nr = rows_host ? n_rows : NB;
  int64_t chunks = 0, slots = 0;
  int64_t prev = -1;
  for (int64_t i = 0; i < nr; ++i) {
    const int64_t by = rows_host ? rows_host[i] : i;
    if (by < 0 || by >= NB) return fail(SSL_ERR_INVALID, "row %lld out of range", (long long)by);
    if (by <= prev) return fail(SSL_ERR_INVALID, "rows must be strictly ascending");
    prev = by;
    const int64_t blk0 = crow_host[by];
    const int64_t nblk = crow_host[by + 1] - blk0;
    const int64_t units = nblk + lr_units;
    if (units == 0) {
      // A listed row without blocks: the in-place kernel would only rewrite the
      // row with its own value, so it gets no chunk.
      continue;
    }
    const int64_t cost = nblk * block_q + (int64_t)lr_units * 32;
    int64_t k = 1;
    if (target_cost > 0) k = (cost + target_cost - 1) / target_cost;
    if (k < 1) k = 1;
    if (k > units) k = units;
    // Chunk boundaries at equal fractions of the row's cost; pc(u) is the cost
    // of the row's first u units.
    auto pc = [&](int64_t u) {
      return u <= nblk ? u * block_q : nblk * block_q + (u - nblk) * 32;
    };
    int64_t ub = 0;
    for (int64_t j = 0; j < k; ++j) {
      int64_t ue;
      if (j == k - 1) {
        ue = units;
      } else {
        const int64_t goal = cost * (j + 1) / k;
        ue = ub + 1;  // every chunk holds at least one unit
        while (ue < units - (k - 1 - j) && pc(ue) < goal) ue++;
      }
      if (table_out) {
        if (chunks >= table_capacity) return fail(SSL_ERR_CAPACITY, "plan table capacity exceeded");
        int32_t* d = table_out + chunks * SSL_PLAN_STRIDE;
        d[0] = (int32_t)by;
        d[1] = (int32_t)ub;
        d[2] = (int32_t)ue;
        d[3] = (int32_t)j;
        d[4] = (int32_t)k;
        d[5] = (int32_t)(k > 1 ? slots : 0);
        d[6] = (int32_t)nblk;
        d[7] = (int32_t)blk0;
      }
      ++chunks;
      ub = ue;
    }
    if (k > 1) slots += k;
  }
  *n_chunks = chunks;
  *n_slots = slots;
  return SSL_OK;
}

}  // extern "C"
