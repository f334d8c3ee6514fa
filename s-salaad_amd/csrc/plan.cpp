// Host-side work planning and error reporting for the C ABI.
//
// A plan turns a BSR structure into workgroup chunks. Block-row `by` owns
// `nblk` sparse blocks (cost q each: one q-wide block of p rows) and `lr_units`
// low-rank units (cost 32 each: 32 ranks of p rows of A). A row costing more
// than `target_cost` is split into k chunks of nearly equal cost. This is the
// load-balancing step for skewed block structures: a row with ten times the
// mean block count gets ten times as many workgroups.
//
// Without low-rank units the k chunks take consecutive, equal shares of the
// row's blocks and are combined by whichever finishes last. With low-rank units
// the row's last chunk is its finaliser: it takes all the low-rank units (they
// need the latent, which is ready only later in the launch) and a smaller
// share of blocks, waits for the other chunks' partial sums and runs the
// epilogue. Finaliser chunks are listed after every other chunk, so a chunk only
// ever waits for chunks that precede it in the table (and in launch order).
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <array>
#include <string>
#include <vector>

#include "abi_common.h"

namespace ssl {

// Part tables of prefill plans (ssl_prefill_parts_build): record size, the
// shortest part worth its exchange of partial tiles, the most parts a group
// takes.
constexpr int64_t kPartRecordInts = 8;
constexpr int64_t kPartMinSteps = 32;
constexpr int64_t kMaxParts = 16;

static thread_local std::string g_last_error;
static DebugKnobs g_knobs{};

DebugKnobs& debug_knobs() { return g_knobs; }

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

// The structure checks every planner makes before it reads an index: crow
// starts at 0 and never decreases, every block's column lies in [0, NBK), and
// the listed rows are strictly ascending block-rows. The kernels index x, the
// block values and the plan with these numbers, so nothing the host has not
// checked reaches the device.
static int check_structure(const int32_t* crow, const int32_t* col, int64_t NB, int64_t NBK,
                           const int32_t* rows, int64_t n_rows) {
  if (crow[0] != 0) return fail(SSL_ERR_INVALID, "crow[0] must be 0");
  for (int64_t b = 0; b < NB; ++b)
    if (crow[b + 1] < crow[b]) return fail(SSL_ERR_INVALID, "crow must be non-decreasing");
  const int64_t nnz = crow[NB];
  if (nnz > 0 && !col) return fail(SSL_ERR_INVALID, "col indices needed for %lld blocks", (long long)nnz);
  if (nnz > 0 && NBK <= 0) return fail(SSL_ERR_INVALID, "NBK must be positive when blocks exist");
  for (int64_t k = 0; k < nnz; ++k)
    if (col[k] < 0 || col[k] >= NBK)
      return fail(SSL_ERR_INVALID, "col[%lld] = %d outside [0, %lld)", (long long)k, col[k],
                  (long long)NBK);
  const int64_t nr = rows ? n_rows : NB;
  int64_t prev = -1;
  for (int64_t i = 0; i < nr; ++i) {
    const int64_t by = rows ? rows[i] : i;
    if (by < 0 || by >= NB) return fail(SSL_ERR_INVALID, "row %lld out of range", (long long)by);
    if (by <= prev) return fail(SSL_ERR_INVALID, "rows must be strictly ascending");
    prev = by;
  }
  return SSL_OK;
}

}  // namespace ssl

using namespace ssl;

extern "C" {

int ssl_version(void) { return 3; }

const char* ssl_last_error(void) { return g_last_error.c_str(); }

int ssl_debug_set(int32_t knob, int64_t value) {
  clear_error();
  DebugKnobs& k = debug_knobs();
  switch (knob) {
    case SSL_DEBUG_PREFILL_TILE:
      if (value < 0 || value > 3) return fail(SSL_ERR_INVALID, "prefill tile override must be 0 to 3");
      k.prefill_group = value;
      return SSL_OK;
    case SSL_DEBUG_WAIT_POLLS:
      if (value < 0 || value > (1LL << 30)) return fail(SSL_ERR_INVALID, "wait polls out of range");
      k.wait_polls = value;
      return SSL_OK;
    case SSL_DEBUG_WAIT_UNREACHABLE:
      k.wait_unreachable = value != 0;
      return SSL_OK;
    case SSL_DEBUG_PREFILL_SPLIT:
      if (value < 0 || value > 4) return fail(SSL_ERR_INVALID, "prefill split override must be 0 to 4");
      k.prefill_split = value;
      return SSL_OK;
    case SSL_DEBUG_CHAIN_FRAG:
      if (value < 0 || value > 2) return fail(SSL_ERR_INVALID, "chain fragment override must be 0 to 2");
      k.chain_frag = value;
      return SSL_OK;
    case SSL_DEBUG_TOPK_GROUPS:
      if (value < 0 || value > 2) return fail(SSL_ERR_INVALID, "select override must be 0 to 2");
      k.topk_groups = value;
      return SSL_OK;
  }
  return fail(SSL_ERR_INVALID, "unknown debug knob %d", knob);
}

int ssl_plan_build(const int32_t* crow_host, const int32_t* col_host, int64_t NB, int64_t NBK,
                   const int32_t* rows_host, int64_t n_rows, int32_t block_q, int32_t lr_units,
                   int64_t target_cost, int32_t* table_out, int64_t table_capacity,
                   int64_t* n_chunks, int64_t* n_slots) {
  clear_error();
  if (!crow_host || !n_chunks || !n_slots || NB < 0 || block_q <= 0 || lr_units < 0 ||
      (rows_host && n_rows < 0) || (table_out && table_capacity < 0))
    return fail(SSL_ERR_INVALID, "invalid plan arguments");
  if (int rc = check_structure(crow_host, col_host, NB, NBK, rows_host, n_rows)) return rc;
  const int64_t nr = rows_host ? n_rows : NB;
  // Two passes: non-finaliser chunks first, then finalisers (pass 1 only when
  // rows have low-rank units).
  int64_t chunks = 0, slots = 0;
  for (int pass = 0; pass < (lr_units > 0 ? 2 : 1); ++pass) {
    int64_t row_slots = 0;
    for (int64_t i = 0; i < nr; ++i) {
      const int64_t by = rows_host ? rows_host[i] : i;
      const int64_t blk0 = crow_host[by];
      const int64_t nblk = crow_host[by + 1] - blk0;
      if (nblk + lr_units == 0) {
        // A listed row without blocks: the in-place kernel would only rewrite the
        // row with its own value, so it gets no chunk.
        continue;
      }
      const int64_t cost = nblk * block_q + (int64_t)lr_units * 32;
      int64_t k = 1;
      if (target_cost > 0) k = (cost + target_cost - 1) / target_cost;
      if (k < 1) k = 1;
      // Block shares. With low-rank units the finaliser (chunk k-1) takes the
      // low-rank cost first; the blocks are split so every chunk costs about
      // cost/k.
      int64_t nsplit = k;  // chunks that share the blocks
      int64_t fin_blocks = 0;
      if (lr_units > 0) {
        const int64_t share = cost / k;  // cost per chunk
        const int64_t lr_cost = (int64_t)lr_units * 32;
        fin_blocks = share > lr_cost ? (share - lr_cost) / block_q : 0;
        if (fin_blocks > nblk) fin_blocks = nblk;
        nsplit = k - 1;
        if (nsplit == 0) fin_blocks = nblk;
      } else if (k > nblk) {
        k = nsplit = nblk;
      }
      const int64_t rest = nblk - fin_blocks;  // blocks for the non-finaliser chunks
      if (lr_units > 0 && nsplit > rest) nsplit = rest;  // no empty non-finaliser chunk
      const int64_t kept = nsplit + (lr_units > 0 ? 1 : 0);
      for (int64_t j = 0; j < kept; ++j) {
        const bool fin = lr_units > 0 && j == kept - 1;
        if ((pass == 1) != fin && lr_units > 0) continue;
        int64_t sb, se, lb = 0, le = 0;
        if (fin) {
          sb = blk0 + rest;
          se = blk0 + nblk;
          le = lr_units;
        } else {
          sb = blk0 + rest * j / nsplit;
          se = blk0 + rest * (j + 1) / nsplit;
        }
        if (table_out) {
          if (chunks >= table_capacity) return fail(SSL_ERR_CAPACITY, "plan table capacity exceeded");
          int32_t* d = table_out + chunks * SSL_PLAN_STRIDE;
          d[0] = (int32_t)by;
          d[1] = (int32_t)sb;
          d[2] = (int32_t)se;
          d[3] = (int32_t)lb;
          d[4] = (int32_t)le;
          d[5] = (int32_t)j;
          d[6] = (int32_t)kept;
          d[7] = (int32_t)(kept > 1 ? row_slots : 0);
        }
        ++chunks;
      }
      if (kept > 1) row_slots += kept;
    }
    slots = row_slots;
  }
  *n_chunks = chunks;
  *n_slots = slots;
  return SSL_OK;
}

// Step record layout (the prefill row kernel's load mapping): 4 waves, each
// issuing IB = group·p / 32 loads of 8 weight rows per step; load i of wave w
// covers features 8·(w + 4i) .. +7, i.e. slot (8·(w + 4i)) / p.
static int32_t prefill_ib(int32_t block_p, int32_t group) {
  return block_p * group == 64 ? 2 : 0;  // the row kernel's tiles are 64 features wide
}

int32_t ssl_prefill_step_ints(int32_t block_p, int32_t group, int32_t step_cols) {
  if (step_cols != 32 && step_cols != 64) return 0;
  if (block_p <= 0 || step_cols % block_p || group < 1 || group > 16) return 0;
  const int32_t ib = prefill_ib(block_p, group);
  if (ib == 0) return 0;
  const int32_t E = step_cols / block_p;
  return (1 + E + 4 * ib * E + 3) / 4 * 4;
}

int ssl_prefill_plan_build(const int32_t* crow_host, const int32_t* col_host, int64_t NB,
                           int64_t NBK, const int32_t* rows_host, int64_t n_rows, int32_t block_p,
                           int32_t group, int32_t step_cols, int32_t* groups_out,
                           int64_t groups_capacity, int32_t* steps_out, int64_t steps_capacity,
                           int64_t* n_groups, int64_t* n_steps) {
  clear_error();
  const int32_t stride = ssl_prefill_step_ints(block_p, group, step_cols);
  if (!crow_host || !n_groups || !n_steps || NB < 0 || stride == 0 ||
      (rows_host && n_rows < 0) || (groups_out && groups_capacity < 0) ||
      (steps_out && steps_capacity < 0))
    return fail(SSL_ERR_INVALID, "invalid prefill plan arguments");
  if (int rc = check_structure(crow_host, col_host, NB, NBK, rows_host, n_rows)) return rc;
  const int64_t nr = rows_host ? n_rows : NB;
  const int E = step_cols / block_p;  // union entries per step
  const int half = step_cols / 2;     // columns per mask half
  const int gstride = 2 + group;
  int64_t ng = 0, ns = 0;
  std::vector<std::array<int32_t, 3>> items;  // (col, slot, block)
  std::vector<int32_t> ent;                   // entries of one group: (1 + group) each
  for (int64_t i0 = 0; i0 < nr; i0 += group) {
    items.clear();
    ent.clear();
    int32_t rows[16];
    for (int g = 0; g < group; ++g) {
      rows[g] = -1;
      if (i0 + g < nr) {
        const int32_t by = rows_host ? rows_host[i0 + g] : (int32_t)(i0 + g);
        rows[g] = by;
        for (int32_t k = crow_host[by]; k < crow_host[by + 1]; ++k)
          items.push_back({col_host[k], g, k});
      }
    }
    // union entries by column; a slot already taken in the current entry (a
    // repeated column within one row) starts a new entry with the same column
    std::sort(items.begin(), items.end());
    int32_t cur_col = -1, taken = 0;
    for (const auto& it : items) {
      if (it[0] != cur_col || (taken >> it[1]) & 1) {
        ent.push_back(it[0]);
        for (int g = 0; g < group; ++g) ent.push_back(-1);
        cur_col = it[0];
        taken = 0;
      }
      taken |= 1 << it[1];
      ent[ent.size() - group + it[1]] = it[2];
    }
    const int64_t n_ent = (int64_t)ent.size() / (1 + group);
    const int64_t steps = (n_ent + E - 1) / E;
    if (steps_out) {
      if (ns + steps > steps_capacity) return fail(SSL_ERR_CAPACITY, "prefill step capacity exceeded");
      for (int64_t st = 0; st < steps; ++st) {
        int32_t* r = steps_out + (ns + st) * stride;
        for (int32_t w = 0; w < stride; ++w) r[w] = -1;
        int32_t mask = 0;
        const int ib = prefill_ib(block_p, group);
        for (int e = 0; e < E; ++e) {
          const int64_t k = st * E + e;
          if (k >= n_ent) continue;
          const int32_t* en = &ent[(size_t)(k * (1 + group))];
          r[1 + e] = en[0] * block_p;  // first x column of the entry
          for (int g = 0; g < group; ++g) {
            if (en[1 + g] < 0) continue;
            // halves of the step this entry covers
            const int h0 = (e * block_p) / half, h1 = (e * block_p + block_p - 1) / half;
            for (int h = h0; h <= h1; ++h) mask |= 1 << (h * group + g);
          }
          // each wave's loads: blk[e][slot(w, i)] at 1 + E + (w·ib + i)·E + e
          for (int w = 0; w < 4; ++w)
            for (int i = 0; i < ib; ++i)
              r[1 + E + (w * ib + i) * E + e] = en[1 + (8 * (w + 4 * i)) / block_p];
        }
        r[0] = mask;
      }
    }
    if (groups_out) {
      if (ng >= groups_capacity) return fail(SSL_ERR_CAPACITY, "prefill group capacity exceeded");
      int32_t* gr = groups_out + ng * gstride;
      gr[0] = (int32_t)ns;
      gr[1] = (int32_t)(ns + steps);
      for (int g = 0; g < group; ++g) gr[2 + g] = rows[g];
    }
    ns += steps;
    ++ng;
  }
  *n_groups = ng;
  *n_steps = ns;
  return SSL_OK;
}

int ssl_prefill_parts_build(const int32_t* groups_host, int64_t n_groups, int32_t group,
                            int32_t* parts_out, int64_t parts_capacity, int64_t* n_parts,
                            int64_t* split_parts) {
  clear_error();
  if (!n_parts || !split_parts || n_groups < 0 || group < 1 || group > 4 ||
      (n_groups > 0 && !groups_host) || (parts_out && parts_capacity < 0))
    return fail(SSL_ERR_INVALID, "invalid part table arguments");
  *n_parts = 0;
  *split_parts = 0;
  const int64_t gstride = 2 + group;
  int64_t total = 0, longest = 0, prev_end = 0;
  for (int64_t g = 0; g < n_groups; ++g) {
    const int64_t b = groups_host[g * gstride], e = groups_host[g * gstride + 1];
    if (b != prev_end || e < b) return fail(SSL_ERR_INVALID, "group %lld: step ranges must tile the plan", (long long)g);
    prev_end = e;
    total += e - b;
    if (e - b > longest) longest = e - b;
  }
  if (n_groups == 0) return SSL_OK;
  // parts of about the mean group's steps (at least kPartMinSteps), only for
  // structures whose longest group is more than twice that
  const int64_t mean = (total + n_groups - 1) / n_groups;
  const int64_t target = mean > kPartMinSteps ? mean : kPartMinSteps;
  if (longest <= 2 * target) return SSL_OK;
  int64_t np = 0, sp = 0;
  for (int64_t g = 0; g < n_groups; ++g) {
    const int64_t b = groups_host[g * gstride], n = groups_host[g * gstride + 1] - b;
    int64_t k = (n + target - 1) / target;
    if (k < 1) k = 1;
    if (k > kMaxParts) k = kMaxParts;
    const int64_t chunk = k > 1 ? (n + k - 1) / k : n;
    if (k > 1) k = (n + chunk - 1) / chunk;
    for (int64_t j = 0; j < k; ++j) {
      if (parts_out) {
        if (np >= parts_capacity) return fail(SSL_ERR_CAPACITY, "part table capacity exceeded");
        int32_t* r = parts_out + np * kPartRecordInts;
        const int64_t b0 = b + j * chunk, b1 = (b0 + chunk < b + n) ? b0 + chunk : b + n;
        r[0] = (int32_t)g;
        r[1] = (int32_t)b0;
        r[2] = (int32_t)(k > 1 ? b1 : b + n);
        r[3] = (int32_t)j;
        r[4] = (int32_t)k;
        r[5] = (int32_t)(k > 1 ? sp : 0);
        r[6] = r[7] = 0;
      }
      ++np;
    }
    if (k > 1) sp += k;
  }
  *n_parts = np;
  *split_parts = sp;
  return SSL_OK;
}

}  // extern "C"
