/* TEST INFRASTRUCTURE ONLY — the parity oracle, never part of the product.
 *
 * float64 GEMM restating the reference CPU path exactly:
 *   src/qutai/backends/cpu.py:152-162 (`cpu.matmul`): for every output
 *   element, `total = 0.0; for k in range(inner): total += a * b` — IEEE
 *   binary64, products rounded, then sums rounded, k strictly increasing;
 *   src/qutai/backends/cpu_lm.py:11-42 (`cpu_lm.gemm`): the same loop with
 *   the transposed index maps `a[k*rows+i]` / `b[j*inner+k]` and the
 *   `accumulate` form `result = value + old`.
 * Built with -O2 -ffp-contract=off and without -ffast-math (oracle/Makefile),
 * so no FMA contraction or reassociation happens; on x86-64 (SSE2 doubles)
 * every result is bit-identical to the CPython loop above.
 *
 * Rows may be restricted to a list (for sampled checks of large products)
 * and are split over POSIX threads; the per-element summation order does
 * not depend on the split.
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  const double* a;
  const double* b;
  double* out;
  int64_t rows, inner, cols;
  int ta, tb, accumulate;
  const int64_t* row_list;  /* NULL = all rows; else out has len(row_list) rows */
  int64_t nrows;
  int64_t begin, end;       /* range of output rows handled by one thread */
  double* bt;               /* B as [cols][inner] (contiguous k per column) */
} Job;

static void* run(void* arg) {
  Job* j = (Job*)arg;
  double* column = NULL;
  if (j->ta) column = (double*)malloc(sizeof(double) * (size_t)(j->inner ? j->inner : 1));
  for (int64_t r = j->begin; r < j->end; r++) {
    int64_t i = j->row_list ? j->row_list[r] : r;
    const double* arow;
    if (j->ta) {
      for (int64_t k = 0; k < j->inner; k++) column[k] = j->a[k * j->rows + i];
      arow = column;
    } else {
      arow = j->a + i * j->inner;
    }
    for (int64_t c = 0; c < j->cols; c++) {
      const double* bcol = j->bt + c * j->inner;
      double total = 0.0;
      for (int64_t k = 0; k < j->inner; k++) {
        double product = arow[k] * bcol[k];
        total = total + product;
      }
      double* o = j->out + r * j->cols + c;
      *o = j->accumulate ? total + *o : total;
    }
  }
  free(column);
  return NULL;
}

/* out[r][c] for r over the selected rows; returns 0 or -1 (allocation). */
int oracle_gemm_f64(const double* a, const double* b, double* out, int64_t rows, int64_t inner, int64_t cols,
                    int ta, int tb, int accumulate, const int64_t* row_list, int64_t nrows, int threads) {
  if (!row_list) nrows = rows;
  double* bt = (double*)malloc(sizeof(double) * (size_t)((cols * inner) > 0 ? cols * inner : 1));
  if (!bt) return -1;
  for (int64_t c = 0; c < cols; c++)
    for (int64_t k = 0; k < inner; k++) bt[c * inner + k] = tb ? b[c * inner + k] : b[k * cols + c];
  if (threads < 1) threads = 1;
  if (threads > 64) threads = 64;
  if (threads > nrows) threads = nrows > 0 ? (int)nrows : 1;
  pthread_t ids[64];
  Job jobs[64];
  for (int t = 0; t < threads; t++) {
    Job j = {a, b, out, rows, inner, cols, ta, tb, accumulate, row_list, nrows,
             nrows * t / threads, nrows * (t + 1) / threads, bt};
    jobs[t] = j;
  }
  for (int t = 1; t < threads; t++) pthread_create(&ids[t], NULL, run, &jobs[t]);
  run(&jobs[0]);
  for (int t = 1; t < threads; t++) pthread_join(ids[t], NULL);
  free(bt);
  return 0;
}

/* bfloat16 encoder of the reference host path (src/qutai/backends/cuda.py:98-101):
 * fp32 bits, round to nearest even; NaN kept quiet by OR-ing 0x40. */
void oracle_bf16_round(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    uint32_t u;
    memcpy(&u, &x[i], 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) y[i] = (uint16_t)((u >> 16) | 0x40u);
    else y[i] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  }
}
