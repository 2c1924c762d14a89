/*
 * sdpa_oracle.c -- CPU restatement of scaled-dot-product attention forward,
 * in double precision.  TEST INFRASTRUCTURE ONLY: the GPU parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it as the
 * checker.  Nothing on the product path may call it.
 *
 * What it restates (WifiLast/torch-cmp-patch):
 *   - the math every reference attention kernel implements,
 *     O = softmax(scale * Q K^T) V, with the max-subtracted softmax of
 *     src/cuda/fp16_flash_attention_hfma2.cu:162-192 and
 *     src/cuda/fp32_attention.cu:127-180 (here exact, in one pass per row);
 *   - the default scale 1/sqrt(D): src/main.cpp:1700-1703;
 *   - the causal mask of the reference's own ground truth,
 *     tests_hardware/test_attention_causal.py:44-53 (triu(diagonal=1) masked
 *     to -inf, i.e. key j visible to query i iff j <= i, top-left aligned,
 *     which is torch's is_causal convention also for Sq != Sk).
 * A row with no visible key (only possible when Sk == 0) yields zeros, as
 * torch's math SDPA does for an empty key sequence.
 *
 * Layout: contiguous [B, H, S, D] (q, o) and [B, H, Sk, D] / [B, H, Sk, Dv].
 * Pinning (tests/test_oracle.py): agreement with torch's math SDPA on CPU,
 * closed forms (Sk = 1, scale = 0, causal row 0), permutation invariance,
 * pure-Python brute force on tiny inputs, and the committed golden fixtures.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

int sdpa_oracle_f64(const double* q, const double* k, const double* v, double* o,
                    int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D, int64_t Dv,
                    double scale, int causal) {
  if (B < 0 || H < 0 || Sq < 0 || Sk < 0 || D < 0 || Dv < 0) return 1;
  double* s = (double*)malloc((size_t)(Sk > 0 ? Sk : 1) * sizeof(double));
  if (!s) return 2;
  for (int64_t bh = 0; bh < B * H; ++bh) {
    const double* qh = q + bh * Sq * D;
    const double* kh = k + bh * Sk * D;
    const double* vh = v + bh * Sk * Dv;
    double* oh = o + bh * Sq * Dv;
    for (int64_t i = 0; i < Sq; ++i) {
      const int64_t nvis = causal ? (i + 1 < Sk ? i + 1 : Sk) : Sk;
      double* orow = oh + i * Dv;
      if (nvis == 0) {
        for (int64_t e = 0; e < Dv; ++e) orow[e] = 0.0;
        continue;
      }
      double m = -INFINITY;
      for (int64_t j = 0; j < nvis; ++j) {
        double dot = 0.0;
        for (int64_t d = 0; d < D; ++d) dot += qh[i * D + d] * kh[j * D + d];
        s[j] = scale * dot;
        if (s[j] > m) m = s[j];
      }
      double denom = 0.0;
      for (int64_t j = 0; j < nvis; ++j) {
        s[j] = exp(s[j] - m);
        denom += s[j];
      }
      for (int64_t e = 0; e < Dv; ++e) orow[e] = 0.0;
      for (int64_t j = 0; j < nvis; ++j) {
        const double w = s[j] / denom;
        for (int64_t e = 0; e < Dv; ++e) orow[e] += w * vh[j * Dv + e];
      }
    }
  }
  free(s);
  return 0;
}
