/*
 * Float64 CPU restatement of the reference's attention (test infrastructure:
 * see attention_ref.h for the algorithm and its reference citations). One
 * (batch, query head, query row) at a time, the plain textbook loops: a row
 * of scaled logits, its max and log-sum-exp, then the weighted sums.
 */
#include "attention_ref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static size_t idx4(int b, int h, int n, int H, int N, int D) {
  return (((size_t)b * H + h) * N + n) * (size_t)D;
}

/* Scaled logits s[j] = q_i . k_j * scale for the keys row i sees
 * (j <= i under causal masking, flash_fwd.cuh:239); returns how many. */
static int logits(const double* qi, const double* kh, int N, int D, int i, int causal,
                  double scale, double* s) {
  const int nj = causal ? i + 1 : N;
  for (int j = 0; j < nj; ++j) {
    const double* kj = kh + (size_t)j * D;
    double acc = 0.0;
    for (int d = 0; d < D; ++d) acc += qi[d] * kj[d];
    s[j] = acc * scale;
  }
  return nj;
}

/* In place: s[j] -> P[j] = exp(s[j] - lse); returns lse (natural log). */
static double softmax_row(double* s, int nj) {
  double m = -INFINITY;
  for (int j = 0; j < nj; ++j) m = s[j] > m ? s[j] : m;
  double l = 0.0;
  for (int j = 0; j < nj; ++j) l += exp(s[j] - m);
  const double lse = m + log(l);
  for (int j = 0; j < nj; ++j) s[j] = exp(s[j] - lse);
  return lse;
}

void ora_fwd(const double* q, const double* k, const double* v, double* o, double* lse,
             int B, int Hq, int Hkv, int N, int D, int causal) {
  const int G = Hq / Hkv;
  const double scale = 1.0 / sqrt((double)D);
  double* s = (double*)malloc((size_t)N * sizeof(double));
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hq; ++h) {
      const double* kh = k + idx4(b, h / G, 0, Hkv, N, D);
      const double* vh = v + idx4(b, h / G, 0, Hkv, N, D);
      for (int i = 0; i < N; ++i) {
        const double* qi = q + idx4(b, h, i, Hq, N, D);
        double* oi = o + idx4(b, h, i, Hq, N, D);
        const int nj = logits(qi, kh, N, D, i, causal, scale, s);
        const double l = softmax_row(s, nj);
        if (lse) lse[((size_t)b * Hq + h) * N + i] = l;
        memset(oi, 0, (size_t)D * sizeof(double));
        for (int j = 0; j < nj; ++j)
          for (int d = 0; d < D; ++d) oi[d] += s[j] * vh[(size_t)j * D + d];
      }
    }
  free(s);
}

void ora_bwd(const double* q, const double* k, const double* v, const double* dO, double* dq,
             double* dk, double* dv, int B, int Hq, int Hkv, int N, int D, int causal) {
  const int G = Hq / Hkv;
  const double scale = 1.0 / sqrt((double)D);
  const size_t nq = (size_t)B * Hq * N * D, nk = (size_t)B * Hkv * N * D;
  double* o = (double*)malloc(nq * sizeof(double));
  double* s = (double*)malloc((size_t)N * sizeof(double));
  ora_fwd(q, k, v, o, NULL, B, Hq, Hkv, N, D, causal);
  memset(dq, 0, nq * sizeof(double));
  memset(dk, 0, nk * sizeof(double));
  memset(dv, 0, nk * sizeof(double));
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hq; ++h) {
      const size_t kvo = idx4(b, h / G, 0, Hkv, N, D);
      const double *kh = k + kvo, *vh = v + kvo;
      double *dkh = dk + kvo, *dvh = dv + kvo;
      for (int i = 0; i < N; ++i) {
        const size_t qo = idx4(b, h, i, Hq, N, D);
        const double *qi = q + qo, *gi = dO + qo, *oi = o + qo;
        double* dqi = dq + qo;
        const int nj = logits(qi, kh, N, D, i, causal, scale, s);
        softmax_row(s, nj); /* s = P */
        double dvec = 0.0;  /* Dv = rowsum(dO * O) (flash_bwd.cuh:65-78) */
        for (int d = 0; d < D; ++d) dvec += gi[d] * oi[d];
        for (int j = 0; j < nj; ++j) {
          const double* vj = vh + (size_t)j * D;
          const double* kj = kh + (size_t)j * D;
          double dp = 0.0;
          for (int d = 0; d < D; ++d) dp += gi[d] * vj[d];
          const double ds = s[j] * (dp - dvec);
          for (int d = 0; d < D; ++d) {
            dvh[(size_t)j * D + d] += s[j] * gi[d];
            dkh[(size_t)j * D + d] += ds * qi[d] * scale;
            dqi[d] += ds * kj[d] * scale;
          }
        }
      }
    }
  free(s);
  free(o);
}

double ora_loss(const double* q, const double* k, const double* v, const double* dO,
                int B, int Hq, int Hkv, int N, int D, int causal) {
  const size_t nq = (size_t)B * Hq * N * D;
  double* o = (double*)malloc(nq * sizeof(double));
  ora_fwd(q, k, v, o, NULL, B, Hq, Hkv, N, D, causal);
  double acc = 0.0;
  for (size_t x = 0; x < nq; ++x) acc += dO[x] * o[x];
  free(o);
  return acc;
}
