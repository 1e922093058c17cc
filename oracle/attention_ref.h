/*
 * Float64 CPU restatement of the reference's attention forward and backward,
 * in plain C (test infrastructure only: used by tests/ and the torch-free
 * driver under tests/driver/, never by the library).
 *
 * Same algorithm and citations as oracle/attention.py, which it mirrors:
 *   forward   O = softmax(Q K^T * scale) V, scale = 1/sqrt(D), causal mask
 *             col > row (fa_p100.py:65-75, attention.cu:72-102); LSE = natural
 *             log-sum-exp of the scaled logits (flash_fwd.cuh:321-329)
 *   GQA       query head h reads key/value head h / (Hq/Hkv) (fa_p100.py:58-62,
 *             flash_fwd.cuh:90)
 *   backward  Dv = rowsum(dO * O), P = exp(S*scale - LSE), dV = P^T dO,
 *             dP = dO V^T, dS = P (dP - Dv), dQ = dS K * scale,
 *             dK = dS^T Q * scale (bwd.cu:20-69, flash_bwd.cuh:11-16, 65-78,
 *             267-282, 434-463); GQA dK/dV summed over a group's query heads
 *   loss      sum(dO * O), whose exact gradient the backward is (bwd.cu:73-105)
 *
 * All tensors are dense row-major (B, H, N, D) float64; lse is (B, Hq, N).
 */
#ifndef FA_ORACLE_ATTENTION_REF_H_
#define FA_ORACLE_ATTENTION_REF_H_

#ifdef __cplusplus
extern "C" {
#endif

/* o (B,Hq,N,D) and lse (B,Hq,N); lse may be NULL. */
void ora_fwd(const double* q, const double* k, const double* v, double* o, double* lse,
             int B, int Hq, int Hkv, int N, int D, int causal);

/* dq (B,Hq,N,D), dk and dv (B,Hkv,N,D), all overwritten. Recomputes O and
 * LSE in float64. */
void ora_bwd(const double* q, const double* k, const double* v, const double* dO, double* dq,
             double* dk, double* dv, int B, int Hq, int Hkv, int N, int D, int causal);

/* sum(dO * O) with O from ora_fwd. */
double ora_loss(const double* q, const double* k, const double* v, const double* dO,
                int B, int Hq, int Hkv, int N, int D, int causal);

/* The options of fa_options (include/fa_mi355x.h) on dense float64 / byte
 * host arrays, as oracle/attention.py takes them (an extension: the
 * reference has none of them); a zeroed struct means none. Query row i of
 * entry b and query head h sees key j iff every option present allows it:
 * j <= i (causal), j < kv_len[b] (clamped to [1, N]), j > i - window,
 * [seg_start, seg_end) of row i (clamped to reach i itself), and
 * mask[(b * mask_heads + (mask_heads == 1 ? 0 : h)) * N * N + i * N + j] != 0.
 * The scaled logit gets bias[((b * Hq + h) * N + i) * N + j] added and
 * alibi[h] * |i - j| subtracted. A row that sees no key gets o = 0,
 * lse = +inf and no gradient. Dropout: keep (B*Hq, N, N) bytes and
 * drop_scale, o = (P * keep * drop_scale) V with P and lse the softmax's. */
typedef struct ora_opts {
  double scale;               /* 0: 1/sqrt(D) */
  const int* kv_len;          /* B key lengths, or NULL */
  int window;                 /* 0, or W > 0 (causal) */
  const double* alibi;        /* Hq slopes, or NULL */
  const int* seg_start;       /* B*N sequence bounds: both or neither */
  const int* seg_end;
  const unsigned char* mask;  /* (B, mask_heads, N, N), nonzero = attend, or NULL */
  int mask_heads;             /* 1 or Hq */
  const unsigned char* keep;  /* (B*Hq, N, N), nonzero = keep, or NULL */
  double drop_scale;
  const double* bias;         /* (B, Hq, N, N) dense, or NULL */
  double* dbias;              /* ora_bwd_ex: dS of the scaled logits, (B, Hq, N, N), or NULL */
  const double* o;            /* ora_bwd_ex: saved forward o (B, Hq, N, D) and lse (B, Hq, N) */
  const double* lse;          /* for Dv and P (as the kernels use them), or NULL: recomputed */
} ora_opts;

void ora_fwd_ex(const double* q, const double* k, const double* v, double* o, double* lse,
                int B, int Hq, int Hkv, int N, int D, int causal, const ora_opts* op);
void ora_bwd_ex(const double* q, const double* k, const double* v, const double* dO,
                double* dq, double* dk, double* dv, int B, int Hq, int Hkv, int N, int D,
                int causal, const ora_opts* op);

/* Dropout keep bytes (P, N, N) of fa_dropout_bits' draw: row key
 * r = h(h(h(h(lo) ^ hi) ^ plane) ^ row) of the seed's 32-bit halves
 * (h = lowbias32), key j draws the low (j even) or high (j odd) 16 bits of
 * h(r ^ (j / 2)), kept iff the draw >= threshold. ora_dropout_threshold:
 * round(p * 65536) of p as a float32, in [0, 65535]; the scale is
 * 65536 / (65536 - threshold). */
unsigned ora_dropout_threshold(float p);
void ora_dropout_keep(unsigned long long seed, unsigned threshold, int P, int N,
                      unsigned char* keep);

#ifdef __cplusplus
}
#endif

#endif /* FA_ORACLE_ATTENTION_REF_H_ */
