/*
 * Test oracle, TEST INFRASTRUCTURE ONLY: an independent plain-C restatement of the reference's
 * fp64 attention (reference flash_lab/reference.py:16-57) used to cross-check oracle/reference.py.
 * Nothing in the flash_lab package links or calls it.
 *
 * Scalar loops, no BLAS: scores s_j = scale * sum_d q_d k_jd in double; a bottom-right causal
 * mask (key j visible to query i iff j <= i + S_k - S_q); the row max, then
 * l = sum_j exp(s_j - max), o = sum_j exp(s_j - max) v_j / l and lse = max + log(l). A row with
 * no visible key gives o = 0 and lse = -inf. Tensors are contiguous [B, S, H, D] doubles; lse is
 * [B, H, S_q]. Query head h reads KV head h / (H / H_kv).
 */
#include <math.h>
#include <stdlib.h>

int oracle_attention_f64(const double* q, const double* k, const double* v, double* o,
                         double* lse, int batch, int seqlen_q, int seqlen_k, int heads,
                         int heads_kv, int head_dim, int causal, double scale) {
  if (batch <= 0 || seqlen_q <= 0 || seqlen_k <= 0 || heads <= 0 || heads_kv <= 0 ||
      head_dim <= 0 || heads % heads_kv != 0)
    return 1;
  const int group = heads / heads_kv;
  const long offset = (long)seqlen_k - seqlen_q;
  double* s = (double*)malloc(sizeof(double) * (size_t)seqlen_k);
  if (!s) return 2;
  for (int b = 0; b < batch; ++b) {
    for (int h = 0; h < heads; ++h) {
      const int hk = h / group;
      for (int i = 0; i < seqlen_q; ++i) {
        const double* qi = q + (((size_t)b * seqlen_q + i) * heads + h) * head_dim;
        double* oi = o + (((size_t)b * seqlen_q + i) * heads + h) * head_dim;
        long last = causal ? (long)i + offset : (long)seqlen_k - 1;
        if (last > seqlen_k - 1) last = seqlen_k - 1;
        double mx = -INFINITY;
        for (long j = 0; j <= last; ++j) {
          const double* kj = k + (((size_t)b * seqlen_k + j) * heads_kv + hk) * head_dim;
          double dot = 0.0;
          for (int d = 0; d < head_dim; ++d) dot += qi[d] * kj[d];
          s[j] = dot * scale;
          if (s[j] > mx) mx = s[j];
        }
        for (int d = 0; d < head_dim; ++d) oi[d] = 0.0;
        double* lse_i = lse + ((size_t)b * heads + h) * seqlen_q + i;
        if (last < 0) {
          *lse_i = -INFINITY;
          continue;
        }
        double l = 0.0;
        for (long j = 0; j <= last; ++j) {
          const double p = exp(s[j] - mx);
          const double* vj = v + (((size_t)b * seqlen_k + j) * heads_kv + hk) * head_dim;
          l += p;
          for (int d = 0; d < head_dim; ++d) oi[d] += p * vj[d];
        }
        for (int d = 0; d < head_dim; ++d) oi[d] /= l;
        *lse_i = mx + log(l);
      }
    }
  }
  free(s);
  return 0;
}
