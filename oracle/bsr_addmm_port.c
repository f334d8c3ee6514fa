/*
 * CPU restatement of the reference AVX2 in-place BSR addmm
 * (ssalaad/cpu_sparse/bsr_addmm_avx2.cpp:67-140), in scalar C.
 *
 * TEST INFRASTRUCTURE ONLY: the oracle's C half. It is linked by tests/ and by
 * bench.py's cpu_baseline leg when the reference build under oracle/_ref is
 * absent; the shipped library never uses it.
 *
 * Same iteration and rounding order as the reference: token rows are split into
 * chunks of at least 8 (at::parallel_for grain, :58-59,83), and for every row and
 * active block-row the fp32 accumulator starts from out, then for each block in
 * col order and each k ascending does acc[j] = fma(x[row, col*B + k], v[k][j], acc[j])
 * (:99-128), so results are bit-identical to the AVX2 kernel, whose ROW_TILE
 * register blocking does not change the per-element operation order.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static void row_range(float* out, const float* x, const int32_t* crow, const int32_t* col,
                      const float* values, const int32_t* active_rows, int64_t m_begin,
                      int64_t m_end, int64_t K, int64_t NB, int64_t ACTIVE_NB, int64_t B) {
  float acc[64];
  for (int64_t r = m_begin; r < m_end; ++r) {
    for (int64_t ai = 0; ai < ACTIVE_NB; ++ai) {
      const int64_t by = active_rows[ai];
      float* o = out + r * NB * B + by * B;
      memcpy(acc, o, (size_t)B * sizeof(float));
      for (int32_t ji = crow[by]; ji < crow[by + 1]; ++ji) {
        const float* xr = x + r * K + (int64_t)col[ji] * B;
        const float* v = values + (int64_t)ji * B * B;
        for (int64_t k = 0; k < B; ++k) {
          const float xv = xr[k];
          const float* vr = v + k * B;
          for (int64_t j = 0; j < B; ++j) acc[j] = fmaf(xv, vr[j], acc[j]);
        }
      }
      memcpy(o, acc, (size_t)B * sizeof(float));
    }
  }
}

/* Returns 0, or -1 for a block size the reference does not support. */
int oracle_bsr_addmm_port(float* out, const float* x, const int32_t* crow, const int32_t* col,
                          const float* values, const int32_t* active_rows, int64_t M, int64_t K,
                          int64_t NB, int64_t ACTIVE_NB, int64_t B, int threads) {
  if (!(B == 8 || B == 16 || B == 32 || B == 64)) return -1;
  const int64_t grain = 8;
  const int64_t nchunks = (M + grain - 1) / grain;
#ifdef _OPENMP
  if (threads < 1) threads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
  for (int64_t c = 0; c < nchunks; ++c) {
    const int64_t b = c * grain, e = (b + grain < M) ? b + grain : M;
    row_range(out, x, crow, col, values, active_rows, b, e, K, NB, ACTIVE_NB, B);
  }
  (void)threads;
  return 0;
}
