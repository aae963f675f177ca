/*
 * attention_ref.c - CPU oracle for the causal attention forward.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker: the product path
 * (custom_flash_attn / libtfgfa.so) never calls it.
 *
 * A plain restatement, in fp64, of the reference's "manual" attention branch
 * (src/py/model_inference.py:68-75):
 *     attn = Q @ K^T                                       (:69)
 *     attn.masked_fill_(triu(ones, diagonal=1), -inf)      (:70-71, mask buffer :55)
 *     w = softmax(attn / sqrt(d), dim=-1)                  (:72)
 *     out = w @ V                                          (:75)
 * with the scale passed explicitly (the reference fixes it to 1/sqrt(64),
 * src/cpp/v1.cu:16) and the causal mask optional.  Each row is done the textbook
 * way - full score row, then max, then exp-sum, then weighted sum of V - with no
 * blocking or online rescaling, so it shares no algorithmic step with the kernel.
 *
 * It also returns the natural-log log-sum-exp of each row,
 *     lse_i = log(sum_{j<=i} exp(scale * q_i . k_j)) = m_i + log(sum_j exp(scale*s_ij - m_i)),
 * the quantity src/py/triton_implementation.py:153-154 accumulates.
 *
 * Inputs are float32 (the bf16-rounded values, upcast); accumulation is fp64.
 * `rows` (nullable) restricts the computation to a subset of query rows so that
 * large shapes can be checked on a sample; outputs are (BH, nrows, D) and (BH, nrows).
 */
#include <math.h>
#include <stdlib.h>

int oracle_attn_fwd(const float* q, const float* k, const float* v, double* o, double* lse,
                    long BH, long N, long D, double scale, int causal, const long* rows,
                    long nrows) {
  if (!q || !k || !v || !o || BH < 0 || N < 0 || D <= 0 || nrows < 0) return 1;
  if (!rows) nrows = N;
  long total = BH * nrows;
#pragma omp parallel
  {
    double* s = (double*)malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
#pragma omp for schedule(dynamic, 4)
    for (long t = 0; t < total; ++t) {
      const long bh = t / nrows;
      const long r = t % nrows;
      const long i = rows ? rows[r] : r;
      const float* qi = q + (bh * N + i) * D;
      const float* kh = k + bh * N * D;
      const float* vh = v + bh * N * D;
      const long jend = causal ? i + 1 : N; /* triu(diagonal=1) masks j > i */
      double m = -INFINITY;
      for (long j = 0; j < jend; ++j) {
        double acc = 0.0;
        for (long d = 0; d < D; ++d) acc += (double)qi[d] * (double)kh[j * D + d];
        s[j] = acc * scale;
        if (s[j] > m) m = s[j];
      }
      double sum = 0.0;
      for (long j = 0; j < jend; ++j) {
        s[j] = exp(s[j] - m);
        sum += s[j];
      }
      double* oi = o + (bh * nrows + r) * D;
      for (long d = 0; d < D; ++d) oi[d] = 0.0;
      for (long j = 0; j < jend; ++j) {
        const double w = s[j] / sum;
        for (long d = 0; d < D; ++d) oi[d] += w * (double)vh[j * D + d];
      }
      if (lse) lse[bh * nrows + r] = m + log(sum);
    }
    free(s);
  }
  return 0;
}
