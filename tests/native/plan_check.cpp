// Host-only exerciser of the C-ABI planners (ssl_plan_build,
// ssl_prefill_plan_build, ssl_debug_set), built with AddressSanitizer and
// UndefinedBehaviorSanitizer by tests/test_sanitize.py. It feeds random
// structures (empty rows, skewed rows, repeated columns, row lists, every
// capacity from zero up) and invalid ones, and checks every returned table
// against the structure it came from. Exit status 0 = every check passed.
#include <stdio.h>
#include <stdlib.h>

#include <random>
#include <vector>

#include "ssalaad_amd.h"

static int g_fail = 0;
#define CHECK(c)                                                      \
  do {                                                                \
    if (!(c)) {                                                       \
      fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #c); \
      ++g_fail;                                                       \
    }                                                                 \
  } while (0)

struct Structure {
  int64_t NB, NBK;
  std::vector<int32_t> crow, col, rows;
};

static Structure random_structure(std::mt19937& rng) {
  Structure s;
  s.NB = rng() % 40;
  s.NBK = 1 + rng() % 30;
  s.crow.push_back(0);
  for (int64_t b = 0; b < s.NB; ++b) {
    int n = (rng() % 4 == 0) ? 0 : rng() % (1 + 2 * s.NBK);  // empty, or up to 2·NBK (repeats)
    for (int i = 0; i < n; ++i) s.col.push_back((int32_t)(rng() % s.NBK));
    s.crow.push_back((int32_t)s.col.size());
  }
  for (int64_t b = 0; b < s.NB; ++b)
    if (rng() % 2) s.rows.push_back((int32_t)b);
  return s;
}

// A row list, never NULL when one is wanted (NULL means "every row").
static const int32_t* row_list(const Structure& s, bool use_rows) {
  static const int32_t none = 0;
  if (!use_rows) return nullptr;
  return s.rows.empty() ? &none : s.rows.data();
}

static void check_plan(const Structure& s, bool use_rows, int32_t q, int32_t lr, int64_t target) {
  const int32_t* rows = row_list(s, use_rows);
  const int64_t nr = use_rows ? (int64_t)s.rows.size() : s.NB;
  int64_t nc = -1, ns = -1;
  int rc = ssl_plan_build(s.crow.data(), s.col.data(), s.NB, s.NBK, rows, nr, q, lr, target,
                          nullptr, 0, &nc, &ns);
  CHECK(rc == SSL_OK);
  if (rc != SSL_OK) return;
  // every capacity below the count is refused without writing past it
  for (int64_t cap = 0; cap < nc; cap += 1 + nc / 7) {
    std::vector<int32_t> small((size_t)(cap * SSL_PLAN_STRIDE) + 1);  // never a null table
    int64_t a, b;
    CHECK(ssl_plan_build(s.crow.data(), s.col.data(), s.NB, s.NBK, rows, nr, q, lr, target,
                         small.data(), cap, &a, &b) == SSL_ERR_CAPACITY);
  }
  std::vector<int32_t> t((size_t)(nc * SSL_PLAN_STRIDE));
  int64_t nc2, ns2;
  CHECK(ssl_plan_build(s.crow.data(), s.col.data(), s.NB, s.NBK, rows, nr, q, lr, target,
                       t.data(), nc, &nc2, &ns2) == SSL_OK);
  CHECK(nc2 == nc && ns2 == ns);
  // every block of every listed row once, every low-rank unit once per row
  std::vector<int> block_seen(s.col.size(), 0), lr_seen((size_t)s.NB, 0);
  std::vector<int> listed((size_t)s.NB, use_rows ? 0 : 1);
  if (use_rows)
    for (int32_t r : s.rows) listed[r] = 1;
  for (int64_t i = 0; i < nc; ++i) {
    const int32_t* d = &t[(size_t)(i * SSL_PLAN_STRIDE)];
    const int32_t row = d[0];
    CHECK(row >= 0 && row < s.NB && listed[row]);
    if (row < 0 || row >= s.NB) continue;
    CHECK(d[1] >= s.crow[row] && d[1] <= d[2] && d[2] <= s.crow[row + 1]);
    for (int32_t k = d[1]; k < d[2] && k >= 0 && k < (int32_t)s.col.size(); ++k) ++block_seen[k];
    CHECK(d[3] >= 0 && d[3] <= d[4] && d[4] <= lr);
    lr_seen[row] += d[4] - d[3];
    CHECK(d[5] >= 0 && d[5] < d[6]);
    CHECK(d[6] == 1 || (d[7] >= 0 && d[7] + d[6] <= ns));
  }
  for (int64_t r = 0; r < s.NB; ++r) {
    if (!listed[r]) continue;
    for (int32_t k = s.crow[r]; k < s.crow[r + 1]; ++k) CHECK(block_seen[k] == 1);
    CHECK(lr_seen[r] == lr);
  }
}

static void check_prefill(const Structure& s, bool use_rows, int32_t p, int32_t group,
                          int32_t sc) {
  const int32_t* rows = row_list(s, use_rows);
  const int64_t nr = use_rows ? (int64_t)s.rows.size() : s.NB;
  int64_t ng = -1, ne = -1;
  int rc = ssl_prefill_plan_build(s.crow.data(), s.col.data(), s.NB, s.NBK, rows, nr, p, group,
                                  sc, nullptr, 0, nullptr, 0, &ng, &ne);
  CHECK(rc == SSL_OK);
  if (rc != SSL_OK) return;
  const int gstride = 2 + group;
  const int stride = ssl_prefill_step_ints(p, group, sc);
  const int E = sc / p, IB = group * p / 32, half = sc / 2;
  CHECK(stride >= 1 + E + 4 * IB * E);
  if (ng > 0) {
    std::vector<int32_t> g((size_t)((ng - 1) * gstride + 1)), e((size_t)(ne * stride + 1));
    int64_t a, b;
    CHECK(ssl_prefill_plan_build(s.crow.data(), s.col.data(), s.NB, s.NBK, rows, nr, p, group,
                                 sc, g.data(), ng - 1, e.data(), ne, &a, &b) == SSL_ERR_CAPACITY);
  }
  std::vector<int32_t> g((size_t)(ng * gstride)), e((size_t)(ne * stride));
  int64_t ng2, ne2;
  CHECK(ssl_prefill_plan_build(s.crow.data(), s.col.data(), s.NB, s.NBK, rows, nr, p, group,
                               sc, g.data(), ng, e.data(), ne, &ng2, &ne2) == SSL_OK);
  CHECK(ng2 == ng && ne2 == ne);
  std::vector<int> seen(s.col.size(), 0);
  for (int64_t i = 0; i < ng; ++i) {
    const int32_t* gr = &g[(size_t)(i * gstride)];
    CHECK(gr[0] >= 0 && gr[0] <= gr[1] && gr[1] <= ne);
    for (int32_t k = gr[0]; k < gr[1] && k >= 0 && k < ne; ++k) {
      const int32_t* rec = &e[(size_t)(k * stride)];
      for (int en = 0; en < E; ++en) {
        const int32_t c = rec[1 + en];
        CHECK(c == -1 || (c >= 0 && c % p == 0 && c / p < s.NBK));
        // the words of wave w, load i hold slot 8·(w + 4i) / p; all copies agree
        for (int w = 0; w < 4; ++w)
          for (int i = 0; i < IB; ++i) {
            const int sl = 8 * (w + 4 * i) / p;
            CHECK(rec[1 + E + (w * IB + i) * E + en] == rec[1 + E + ((sl * p / 8) % 4 * IB + (sl * p / 8) / 4) * E + en]);
          }
        for (int sl = 0; sl < group; ++sl) {
          const int fw = sl * p / 8;  // first 8-feature run of the slot: wave fw % 4, load fw / 4
          const int32_t blk = rec[1 + E + ((fw % 4) * IB + fw / 4) * E + en];
          if (blk < 0) continue;
          CHECK(c >= 0);
          const int h0 = en * p / half, h1 = (en * p + p - 1) / half;
          CHECK(((rec[0] >> (h0 * group + sl)) & 1) && ((rec[0] >> (h1 * group + sl)) & 1));
          const int32_t row = gr[2 + sl];
          CHECK(row >= 0 && blk >= s.crow[row] && blk < s.crow[row + 1] && s.col[blk] * p == c);
          if (blk >= 0 && blk < (int32_t)s.col.size()) ++seen[blk];
        }
      }
    }
  }
  for (int64_t i = 0; i < nr; ++i) {
    const int32_t r = use_rows ? s.rows[i] : (int32_t)i;
    for (int32_t k = s.crow[r]; k < s.crow[r + 1]; ++k) CHECK(seen[k] == 1);
  }
}

int main() {
  std::mt19937 rng(12345);
  for (int it = 0; it < 3000; ++it) {
    Structure s = random_structure(rng);
    const int32_t q = 16 << (rng() % 3);
    const int32_t lr = (rng() % 3 == 0) ? 0 : 1 + rng() % 8;
    const int64_t target = (rng() % 3 == 0) ? 0 : 1 + rng() % 200;
    check_plan(s, false, q, lr, target);
    check_plan(s, true, q, lr, target);
    const int32_t pp = 16 << (rng() % 3);
    const int32_t group = 64 / pp;
    const int32_t sc = (pp <= 32 && rng() % 2) ? 32 : 64;
    check_prefill(s, false, pp, group, sc);
    check_prefill(s, true, pp, group, sc);
    // corrupted copies are refused
    if (!s.col.empty()) {
      Structure bad = s;
      bad.col[rng() % bad.col.size()] = (rng() % 2) ? -1 : (int32_t)s.NBK;
      int64_t a, b;
      CHECK(ssl_plan_build(bad.crow.data(), bad.col.data(), bad.NB, bad.NBK, nullptr, 0, q, lr,
                           target, nullptr, 0, &a, &b) == SSL_ERR_INVALID);
      CHECK(ssl_prefill_plan_build(bad.crow.data(), bad.col.data(), bad.NB, bad.NBK, nullptr, 0,
                                   pp, group, sc, nullptr, 0, nullptr, 0, &a, &b) == SSL_ERR_INVALID);
    }
    if (s.NB > 1 && s.crow[s.NB] > 0) {
      Structure bad = s;
      bad.crow[1 + rng() % (s.NB - 1)] = s.crow[s.NB] + 1;  // no longer non-decreasing
      int64_t a, b;
      CHECK(ssl_plan_build(bad.crow.data(), bad.col.data(), bad.NB, bad.NBK, nullptr, 0, q, lr,
                           target, nullptr, 0, &a, &b) == SSL_ERR_INVALID);
    }
  }
  int64_t a, b;
  CHECK(ssl_plan_build(nullptr, nullptr, 0, 0, nullptr, 0, 16, 0, 0, nullptr, 0, &a, &b) ==
        SSL_ERR_INVALID);
  CHECK(ssl_debug_set(99, 0) == SSL_ERR_INVALID);
  CHECK(ssl_debug_set(SSL_DEBUG_PREFILL_TILE, 4) == SSL_ERR_INVALID);
  CHECK(ssl_debug_set(SSL_DEBUG_PREFILL_TILE, 0) == SSL_OK);
  CHECK(ssl_last_error() != nullptr);
  if (g_fail) {
    fprintf(stderr, "%d checks failed\n", g_fail);
    return 1;
  }
  printf("plan_check: all checks passed\n");
  return 0;
}
