/*
 * CPU oracle helpers for the LFM2.5 decode path -- TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * this file; the product path never does.
 *
 * oracle_gemv: y[m] = sum_k bf16(W[m,k]) * x[k] accumulated in double. Every
 * product of a BF16 weight and an FP32 activation is exact in double and the
 * double sum of K <= 65536 such terms is within ~1e-16 relative of the exact
 * value, so y is the "FP32 accumulation" of the reference's BF16 linear layers
 * (F.linear, experiments/014_int8_lfm25.py:104-109) without any particular
 * summation order; callers round it to FP32 and then to BF16.
 * Eight partial sums per row (k mod 8) are combined in a fixed tree, and rows
 * are split over OpenMP threads, so results do not depend on the thread count.
 */
#include <stdint.h>
#include <string.h>

static inline double bf16_to_double(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, sizeof f);
  return (double)f;
}

void oracle_gemv(const uint16_t* w, const float* x, int64_t m_rows, int64_t k_cols, double* y) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < m_rows; ++m) {
    const uint16_t* row = w + m * k_cols;
    double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t k = 0;
    for (; k + 8 <= k_cols; k += 8)
      for (int j = 0; j < 8; ++j) acc[j] += bf16_to_double(row[k + j]) * (double)x[k + j];
    for (; k < k_cols; ++k) acc[k & 7] += bf16_to_double(row[k]) * (double)x[k];
    y[m] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  }
}

int oracle_version(void) { return 1; }
