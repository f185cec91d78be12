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
#include <string.h>

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

/*
 * Decode (reference flash_lab/reference.py:167-205, one query per sequence and head against the
 * first seq_lens[b] keys of its cache) in double, reading the 16-bit or 32-bit inputs directly so
 * that long caches need no float64 copies. q is [B, H, D], k and v contiguous [B, S_max, H_kv, D],
 * o [B, H, D] and lse [B, H] doubles. elem 0: bf16 bit patterns; elem 2: fp32. The softmax runs in
 * two passes over the scores (max, then exp and sums), like oracle_attention_f64; lengths outside
 * [1, S_max] are rejected (code 3). (batch, head) pairs are independent and run in parallel when
 * built with OpenMP.
 */
static double load_elem(const void* base, size_t index, int elem) {
  if (elem == 0) {
    const unsigned int bits = (unsigned int)((const unsigned short*)base)[index] << 16;
    float f;
    memcpy(&f, &bits, sizeof f);
    return (double)f;
  }
  return (double)((const float*)base)[index];
}

int oracle_decode_f64(const void* q, const void* k, const void* v, const int* seq_lens, double* o,
                      double* lse, int batch, int heads, int heads_kv, int max_seqlen, int head_dim,
                      int elem, double scale) {
  if (batch <= 0 || heads <= 0 || heads_kv <= 0 || max_seqlen <= 0 || head_dim <= 0 ||
      heads % heads_kv != 0 || (elem != 0 && elem != 2))
    return 1;
  for (int b = 0; b < batch; ++b)
    if (seq_lens[b] < 1 || seq_lens[b] > max_seqlen) return 3;
  const int group = heads / heads_kv;
  int failed = 0;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < batch; ++b) {
    for (int h = 0; h < heads; ++h) {
      const int hk = h / group;
      const long n = seq_lens[b];
      double* s = (double*)malloc(sizeof(double) * (size_t)n);
      double* qd = (double*)malloc(sizeof(double) * (size_t)head_dim);
      if (!s || !qd) {
        free(s);
        free(qd);
#pragma omp atomic write
        failed = 2;
        continue;
      }
      for (int d = 0; d < head_dim; ++d)
        qd[d] = load_elem(q, ((size_t)b * heads + h) * head_dim + d, elem);
      double mx = -INFINITY;
      for (long j = 0; j < n; ++j) {
        const size_t row = (((size_t)b * max_seqlen + j) * heads_kv + hk) * head_dim;
        double dot = 0.0;
        for (int d = 0; d < head_dim; ++d) dot += qd[d] * load_elem(k, row + d, elem);
        s[j] = dot * scale;
        if (s[j] > mx) mx = s[j];
      }
      double* oi = o + ((size_t)b * heads + h) * head_dim;
      for (int d = 0; d < head_dim; ++d) oi[d] = 0.0;
      double l = 0.0;
      for (long j = 0; j < n; ++j) {
        const double p = exp(s[j] - mx);
        const size_t row = (((size_t)b * max_seqlen + j) * heads_kv + hk) * head_dim;
        l += p;
        for (int d = 0; d < head_dim; ++d) oi[d] += p * load_elem(v, row + d, elem);
      }
      for (int d = 0; d < head_dim; ++d) oi[d] /= l;
      lse[(size_t)b * heads + h] = mx + log(l);
      free(s);
      free(qd);
    }
  }
  return failed;
}

/*
 * Prefill attention for selected query rows (reference flash_lab/reference.py:60-87: each row keeps
 * its position in the full sequence for the bottom-right causal mask) in double, reading bf16
 * (elem 0) or fp32 (elem 2) inputs in place: q [B, S_q, H, D], k and v [B, S_k, H_kv, D]
 * contiguous, rows[n] in [0, S_q); o [B, n, H, D] and lse [B, H, n] doubles. The same two-pass
 * softmax as oracle_attention_f64 (a row without a visible key gives 0 and -inf); (batch, head,
 * row) triples run in parallel when built with OpenMP.
 */
int oracle_attention_rows_f64(const void* q, const void* k, const void* v, const long* rows,
                              double* o, double* lse, int batch, int seqlen_q, int seqlen_k,
                              int heads, int heads_kv, int head_dim, int n_rows, int causal,
                              int elem, double scale) {
  if (batch <= 0 || seqlen_q <= 0 || seqlen_k <= 0 || heads <= 0 || heads_kv <= 0 ||
      head_dim <= 0 || n_rows <= 0 || heads % heads_kv != 0 || (elem != 0 && elem != 2))
    return 1;
  for (int r = 0; r < n_rows; ++r)
    if (rows[r] < 0 || rows[r] >= seqlen_q) return 3;
  const int group = heads / heads_kv;
  const long offset = (long)seqlen_k - seqlen_q;
  int failed = 0;
  /* One (batch, head) per task: its K and V rows are converted to double once, then every
   * selected query row runs over them. */
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < batch; ++b) {
    for (int h = 0; h < heads; ++h) {
      const int hk = h / group;
      double* kd = (double*)malloc(sizeof(double) * (size_t)seqlen_k * head_dim);
      double* vd = (double*)malloc(sizeof(double) * (size_t)seqlen_k * head_dim);
      double* s = (double*)malloc(sizeof(double) * (size_t)seqlen_k);
      double* qd = (double*)malloc(sizeof(double) * (size_t)head_dim);
      if (!kd || !vd || !s || !qd) {
        free(kd);
        free(vd);
        free(s);
        free(qd);
#pragma omp atomic write
        failed = 2;
        continue;
      }
      for (long j = 0; j < seqlen_k; ++j) {
        const size_t row = (((size_t)b * seqlen_k + j) * heads_kv + hk) * head_dim;
        for (int d = 0; d < head_dim; ++d) {
          kd[j * head_dim + d] = load_elem(k, row + d, elem);
          vd[j * head_dim + d] = load_elem(v, row + d, elem);
        }
      }
      for (int r = 0; r < n_rows; ++r) {
        const long i = rows[r];
        for (int d = 0; d < head_dim; ++d)
          qd[d] = load_elem(q, (((size_t)b * seqlen_q + i) * heads + h) * head_dim + d, elem);
        long last = causal ? i + offset : (long)seqlen_k - 1;
        if (last > seqlen_k - 1) last = seqlen_k - 1;
        double mx = -INFINITY;
        for (long j = 0; j <= last; ++j) {
          const double* kj = kd + j * head_dim;
          double dot = 0.0;
          for (int d = 0; d < head_dim; ++d) dot += qd[d] * kj[d];
          s[j] = dot * scale;
          if (s[j] > mx) mx = s[j];
        }
        double* oi = o + (((size_t)b * n_rows + r) * heads + h) * head_dim;
        for (int d = 0; d < head_dim; ++d) oi[d] = 0.0;
        double* lse_i = lse + ((size_t)b * heads + h) * n_rows + r;
        if (last < 0) {
          *lse_i = -INFINITY;
          continue;
        }
        double l = 0.0;
        for (long j = 0; j <= last; ++j) {
          const double p = exp(s[j] - mx);
          const double* vj = vd + j * head_dim;
          l += p;
          for (int d = 0; d < head_dim; ++d) oi[d] += p * vj[d];
        }
        for (int d = 0; d < head_dim; ++d) oi[d] /= l;
        *lse_i = mx + log(l);
      }
      free(kd);
      free(vd);
      free(s);
      free(qd);
    }
  }
  return failed;
}
