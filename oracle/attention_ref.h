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

#ifdef __cplusplus
}
#endif

#endif /* FA_ORACLE_ATTENTION_REF_H_ */
