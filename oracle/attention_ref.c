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

/* ---- options (ora_opts): the row's visibility, logits and softmax ---- */

static int clampi(int x, int lo, int hi) { return x < lo ? lo : x > hi ? hi : x; }

static int sees(const ora_opts* op, int causal, int b, int h, int N, int i, int j) {
  if (causal && j > i) return 0;
  if (op->kv_len && j >= clampi(op->kv_len[b], 1, N)) return 0;
  if (op->window > 0 && j <= i - op->window) return 0;
  if (op->seg_start) {
    int s0 = op->seg_start[(size_t)b * N + i], s1 = op->seg_end[(size_t)b * N + i];
    if (s0 > i) s0 = i;
    if (s1 < i + 1) s1 = i + 1;
    if (j < s0 || j >= s1) return 0;
  }
  if (op->mask) {
    const size_t plane = (size_t)b * op->mask_heads + (op->mask_heads == 1 ? 0 : h);
    if (!op->mask[(plane * N + i) * N + j]) return 0;
  }
  return 1;
}

/* p[j] = P of key j for row i (0 where it does not see j); returns lse
 * (+inf for a row that sees no key, whose p is all zero). */
static double row_ex(const double* qi, const double* kh, int b, int h, int Hq, int N, int D,
                     int i, int causal, double scale, const ora_opts* op, double* p) {
  double m = -INFINITY;
  for (int j = 0; j < N; ++j) {
    if (!sees(op, causal, b, h, N, i, j)) {
      p[j] = -INFINITY;
      continue;
    }
    const double* kj = kh + (size_t)j * D;
    double acc = 0.0;
    for (int d = 0; d < D; ++d) acc += qi[d] * kj[d];
    double s = acc * scale;
    if (op->bias) s += op->bias[(((size_t)b * Hq + h) * N + i) * N + j];
    if (op->alibi) s -= op->alibi[h] * fabs((double)(i - j));
    p[j] = s;
    m = s > m ? s : m;
  }
  if (m == -INFINITY) {
    for (int j = 0; j < N; ++j) p[j] = 0.0;
    return INFINITY;
  }
  double l = 0.0;
  for (int j = 0; j < N; ++j) l += p[j] == -INFINITY ? 0.0 : exp(p[j] - m);
  const double lse = m + log(l);
  for (int j = 0; j < N; ++j) p[j] = p[j] == -INFINITY ? 0.0 : exp(p[j] - lse);
  return lse;
}

static double keep_factor(const ora_opts* op, size_t plane, int N, int i, int j) {
  if (!op->keep) return 1.0;
  return op->keep[(plane * N + i) * N + j] ? op->drop_scale : 0.0;
}

void ora_fwd_ex(const double* q, const double* k, const double* v, double* o, double* lse,
                int B, int Hq, int Hkv, int N, int D, int causal, const ora_opts* op) {
  const int G = Hq / Hkv;
  const double scale = op->scale > 0.0 ? op->scale : 1.0 / sqrt((double)D);
  double* p = (double*)malloc((size_t)N * sizeof(double));
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hq; ++h) {
      const double* kh = k + idx4(b, h / G, 0, Hkv, N, D);
      const double* vh = v + idx4(b, h / G, 0, Hkv, N, D);
      const size_t plane = (size_t)b * Hq + h;
      for (int i = 0; i < N; ++i) {
        const double* qi = q + idx4(b, h, i, Hq, N, D);
        double* oi = o + idx4(b, h, i, Hq, N, D);
        const double l = row_ex(qi, kh, b, h, Hq, N, D, i, causal, scale, op, p);
        if (lse) lse[plane * N + i] = l;
        memset(oi, 0, (size_t)D * sizeof(double));
        for (int j = 0; j < N; ++j) {
          const double w = p[j] * keep_factor(op, plane, N, i, j);
          if (w != 0.0)
            for (int d = 0; d < D; ++d) oi[d] += w * vh[(size_t)j * D + d];
        }
      }
    }
  free(p);
}

void ora_bwd_ex(const double* q, const double* k, const double* v, const double* dO,
                double* dq, double* dk, double* dv, int B, int Hq, int Hkv, int N, int D,
                int causal, const ora_opts* op) {
  const int G = Hq / Hkv;
  const double scale = op->scale > 0.0 ? op->scale : 1.0 / sqrt((double)D);
  const size_t nq = (size_t)B * Hq * N * D, nk = (size_t)B * Hkv * N * D;
  double* own = NULL;
  const double* o = op->o;
  if (!o) {
    own = (double*)malloc(nq * sizeof(double));
    ora_fwd_ex(q, k, v, own, NULL, B, Hq, Hkv, N, D, causal, op);
    o = own;
  }
  double* p = (double*)malloc((size_t)N * sizeof(double));
  memset(dq, 0, nq * sizeof(double));
  memset(dk, 0, nk * sizeof(double));
  memset(dv, 0, nk * sizeof(double));
  if (op->dbias) memset(op->dbias, 0, (size_t)B * Hq * N * N * sizeof(double));
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hq; ++h) {
      const size_t kvo = idx4(b, h / G, 0, Hkv, N, D);
      const double *kh = k + kvo, *vh = v + kvo;
      double *dkh = dk + kvo, *dvh = dv + kvo;
      const size_t plane = (size_t)b * Hq + h;
      for (int i = 0; i < N; ++i) {
        const size_t qo = idx4(b, h, i, Hq, N, D);
        const double *qi = q + qo, *gi = dO + qo, *oi = o + qo;
        double* dqi = dq + qo;
        const double l = row_ex(qi, kh, b, h, Hq, N, D, i, causal, scale, op, p);
        if (op->lse) {  /* P from the saved lse, as the kernels do */
          const double ls = op->lse[plane * N + i];
          for (int j = 0; j < N; ++j)
            if (p[j] != 0.0) p[j] = ls == INFINITY ? 0.0 : p[j] * exp(l - ls);
        }
        double dvec = 0.0; /* Dv = rowsum(dO * O) (flash_bwd.cuh:65-78) */
        for (int d = 0; d < D; ++d) dvec += gi[d] * oi[d];
        for (int j = 0; j < N; ++j) {
          if (p[j] == 0.0) continue;
          const double* vj = vh + (size_t)j * D;
          const double* kj = kh + (size_t)j * D;
          const double z = keep_factor(op, plane, N, i, j);
          double dp = 0.0;
          for (int d = 0; d < D; ++d) dp += gi[d] * vj[d];
          const double ds = p[j] * (z * dp - dvec);
          if (op->dbias) op->dbias[(plane * N + i) * N + j] = ds;
          for (int d = 0; d < D; ++d) {
            dvh[(size_t)j * D + d] += p[j] * z * gi[d];
            dkh[(size_t)j * D + d] += ds * qi[d] * scale;
            dqi[d] += ds * kj[d] * scale;
          }
        }
      }
    }
  free(p);
  free(own);
}

/* ---- dropout draw (fa_dropout_bits) ---- */

static unsigned lowbias32(unsigned x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

unsigned ora_dropout_threshold(float p) {
  const double t = nearbyint((double)p * 65536.0);
  return (unsigned)(t < 0.0 ? 0.0 : t > 65535.0 ? 65535.0 : t);
}

void ora_dropout_keep(unsigned long long seed, unsigned threshold, int P, int N,
                      unsigned char* keep) {
  const unsigned lo = (unsigned)(seed & 0xffffffffull), hi = (unsigned)(seed >> 32);
  const unsigned base = lowbias32(lowbias32(lo) ^ hi);
  for (int pl = 0; pl < P; ++pl) {
    const unsigned kp = lowbias32(base ^ (unsigned)pl);
    for (int i = 0; i < N; ++i) {
      const unsigned r = lowbias32(kp ^ (unsigned)i);
      for (int j = 0; j < N; ++j) {
        const unsigned u = lowbias32(r ^ (unsigned)(j / 2));
        const unsigned draw = (j & 1) ? u >> 16 : u & 0xffffu;
        keep[((size_t)pl * N + i) * N + j] = draw >= threshold;
      }
    }
  }
}
