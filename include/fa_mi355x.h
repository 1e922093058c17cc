/*
 * fa_mi355x.h -- C ABI of the MI355X (gfx950) FlashAttention-2 library.
 *
 * The reference exposes this path only as a pybind torch extension named
 * `fa_p100_ext` with two functions, `forward` and `backward`
 * (fa_p100_ext.cu:53-83, 103-142, 144-147), which call straight into
 * `flash::launch` (flash_fwd.cuh:342-355) and `flash_bwd::launch`
 * (flash_bwd.cuh:466-484). This header is the layer beneath that binding:
 * plain pointers and sizes, no torch types, no allocation inside, no global
 * state. The torch extension built beside it (`fa_p100_ext`) and any other
 * host (ctypes, a C++ driver) call these entry points.
 *
 * Conventions shared by every entry point
 *   - Tensors are dense row-major (B, H, N, D): element (b,h,n,d) sits at
 *     ((b*H + h)*N + n)*D + d. q, o, dO, dq are (B, Hq, N, D); k, v, dk, dv
 *     are (B, Hkv, N, D); lse and the Dv workspace are (B, Hq, N) float32.
 *   - fp16 buffers hold IEEE binary16 (`_Float16` / `__half` / torch.half).
 *   - Query head h reads key/value head h / (Hq/Hkv), which is
 *     `repeat_interleave` over the head axis (fa_p100.py:58-62).
 *   - The softmax scale is 1/sqrt(D) (fa_p100_ext.cu:71, 117) unless
 *     fa_options.scale gives another (the fa_fwd_ex / fa_bwd_ex pair).
 *   - `stream` is a hipStream_t (NULL = the null stream). Every launch is
 *     asynchronous on it; the call returns after enqueueing.
 *   - Return value: FA_OK (0), an FA_ERR_* validation code (nothing was
 *     launched), or a hipError_t value reported by the HIP runtime.
 *   - Entry points are reentrant and thread-safe: they keep no state, with
 *     one exception, fa_bwd_noalloc, whose built-in device scratch (16 MiB
 *     per GPU, resident while the library is loaded) is shared by its calls
 *     on one GPU, so calls of it that overlap on one GPU race.
 */
#ifndef FA_MI355X_H_
#define FA_MI355X_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Rows and keys per block of a block-sparse layout (fa_options.block_rows). */
#define FA_SPARSE_BLOCK 128

enum {
  FA_OK = 0,
  FA_ERR_HEAD_DIM = 10001,   /* D not a multiple of 8 in [8, 256] (fa_p100_ext.cu:59, 111: {64, 128}) */
  FA_ERR_SEQLEN = 10002,     /* N <= 0 (fa_p100_ext.cu:60, 112) */
  FA_ERR_HEADS = 10003,      /* Hkv <= 0 or Hq % Hkv != 0 (fa_p100_ext.cu:61, 113) */
  FA_ERR_BATCH = 10004,      /* B <= 0 */
  FA_ERR_NULL = 10005,       /* a required pointer is NULL */
  FA_ERR_WORKSPACE = 10006,  /* workspace smaller than fa_bwd_workspace_bytes() */
  FA_ERR_TOO_LARGE = 10007,  /* (N+256)*D (BNHD: (N+256)*H*D) over 2^31-1, or over 2^29 for a
                                head dim that is not 32, 64, 96, 128 or 256; or a launch's work
                                items over 2^32 */
  FA_ERR_LAYOUT = 10008,     /* layout not FA_LAYOUT_BHND or FA_LAYOUT_BNHD */
  FA_ERR_DTYPE = 10009,      /* element format not supported */
  FA_ERR_WINDOW = 10010,     /* sliding window < 0, or > 0 without causal masking */
  FA_ERR_SEGMENTS = 10011,   /* packed sequences with only one of the two bound arrays */
  FA_ERR_SCALE = 10012,      /* softmax scale negative or not finite */
  FA_ERR_SCRATCH = 10013,    /* fa_bwd_noalloc: the shape needs more than its scratch */
  FA_ERR_MASK = 10014,       /* mask_heads not 1 or Hq, or a backward mask without mask_t */
  FA_ERR_DROPOUT = 10015,    /* dropout p not in [0, 1), a scale not positive and finite, or
                                a backward with drop but without drop_t */
  FA_ERR_BIAS = 10016,       /* a negative bias stride, dbias without bias, or a bias with
                                N > 2^22 or a head dim above 128 */
  FA_ERR_KV_ROWS = 10017,    /* kv_rows < 0, or kv_rows != N together with packed sequences,
                                a mask, dropout or a bias */
  FA_ERR_BLOCKS = 10018      /* a block-sparse layout with a mask, a bias or kv_rows != N, a
                                backward without block_cols, block_cols without block_rows,
                                or (fa_pack_blocks) layout planes not 1 or B by 1 or Hq */
};

/* Memory layouts of the 16-bit tensors, for the entry points that take one:
 * dense (B, H, N, D) as everywhere else, or dense (B, N, H, D) (see
 * fa_fwd_bnhd). */
enum { FA_LAYOUT_BHND = 0, FA_LAYOUT_BNHD = 1 };

/* Element formats of the 16-bit tensors, for the entry points that take one. */
enum { FA_DTYPE_FP16 = 0, FA_DTYPE_BF16 = 1 };

/* Human-readable text for any value returned by this library. */
const char* fa_error_string(int err);

/* Library version string, e.g. "fa_mi355x 1.0 gfx950". */
const char* fa_version(void);

/*
 * Forward pass. Replaces fa_forward (fa_p100_ext.cu:53-83) below its torch
 * checks: writes o (fp16, B,Hq,N,D) and lse (fp32, B,Hq,N; natural log of
 * the row sum of exp(scaled logits), flash_fwd.cuh:324-329).
 * `full_precision` is accepted for the reference's API (fa_p100_ext.cu:44-50);
 * fp16 products are exact in the fp32 MFMA accumulator, so both tiers run the
 * same kernel.
 */
int fa_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
           int B, int Hq, int Hkv, int N, int D, int causal,
           int full_precision, void* stream);

/*
 * fa_fwd on tensors stored as dense (B, N, H, D) instead of (B, H, N, D): q and
 * o with Hq heads, k and v with Hkv heads (lse stays (B, Hq, N)). This is the
 * layout of a transformer block's projections, so a caller holding
 * (B, H, N, D) views of them (fa_p100_hf.py:131-142 transposes them) needs no
 * copy in or out. No counterpart in the reference (the caller made the
 * tensors contiguous, fa_p100_ext.cu:67-69, and copied o back,
 * fa_p100_hf.py:142). Same results, bit for bit, as fa_fwd on the same
 * logical tensors.
 */
int fa_fwd_bnhd(const void* q, const void* k, const void* v, void* o, float* lse,
                int B, int Hq, int Hkv, int N, int D, int causal, void* stream);

/*
 * Bytes of device workspace fa_bwd needs: two (B, Hq, N) float32 vectors, the
 * reference's `dvec` (fa_p100_ext.cu:124) and the saved LSE pre-multiplied by
 * log2(e); then B*Hq*floor(ceil(N/128)/2) uint32 counters; then, for each
 * (b, kv head) and each of those floor(ceil(N/128)/2) pairs of 128-row key
 * tiles, two fp32 partial-sum slots of 128*D*2 floats (the backward's causal
 * load balancing splits a short key tile's work between two workgroups).
 * Each part is rounded up to 256 bytes. 0 for an invalid shape.
 */
size_t fa_bwd_workspace_bytes(int B, int Hq, int Hkv, int N, int D);

/*
 * Backward pass. Replaces fa_backward (fa_p100_ext.cu:103-142) below its torch
 * checks. Inputs q, k, v, dO, o (fp16) and lse (fp32) are the forward's
 * inputs/outputs. Writes dq (fp32, B,Hq,N,D), dk and dv (fp16, B,Hkv,N,D);
 * every element of the three outputs is overwritten. `workspace` must hold
 * fa_bwd_workspace_bytes() bytes. Equivalent to fa_bwd_preprocess() followed
 * by fa_bwd_main(). Deterministic: no atomic adds touch the results (an
 * atomic counter only decides which of two workgroups adds their two partial
 * sums, and fp32 addition is commutative), so repeated calls are bit-identical.
 */
int fa_bwd(const void* q, const void* k, const void* v, const void* dO,
           const void* o, const float* lse, float* dq, void* dk, void* dv,
           void* workspace, size_t workspace_bytes,
           int B, int Hq, int Hkv, int N, int D, int causal, void* stream);

/*
 * fa_bwd with dq written as fp16 (B,Hq,N,D) instead of fp32: each element is
 * the fp32 result rounded to nearest even, bit-identical to fa_bwd followed by
 * a cast. No counterpart in the reference: it serves the autograd backward,
 * which hands dq back in q's dtype (fa_p100.py:45), and saves that cast's pass
 * over dq.
 */
int fa_bwd_half_dq(const void* q, const void* k, const void* v, const void* dO,
                   const void* o, const float* lse, void* dq, void* dk, void* dv,
                   void* workspace, size_t workspace_bytes,
                   int B, int Hq, int Hkv, int N, int D, int causal, void* stream);

/*
 * fa_bwd_half_dq on (B, N, H, D)-stored q, k, v, dO, o, dq, dk, dv (see
 * fa_fwd_bnhd). No counterpart in the reference (see fa_fwd_bnhd and
 * fa_bwd_half_dq); bit-identical to fa_bwd_half_dq on the same logical
 * tensors.
 */
int fa_bwd_bnhd(const void* q, const void* k, const void* v, const void* dO,
                const void* o, const float* lse, void* dq, void* dk, void* dv,
                void* workspace, size_t workspace_bytes,
                int B, int Hq, int Hkv, int N, int D, int causal, void* stream);

/*
 * First phase of fa_bwd, the counterpart of bwd_preprocess
 * (flash_bwd.cuh:65-78): fills `workspace` with dvec = rowsum(dO * o) and
 * lse * log2(e), both fp32 (B,Hq,N), and zeroes its counters. Exposed so a
 * host can time or schedule the phases separately. `workspace_bytes` must
 * cover at least the vectors and counters (fa_bwd_workspace_bytes() does).
 */
int fa_bwd_preprocess(const void* dO, const void* o, const float* lse,
                      void* workspace, size_t workspace_bytes,
                      int B, int Hq, int N, int D, void* stream);

/*
 * Second phase of fa_bwd, the counterpart of bwd_kernel
 * (flash_bwd.cuh:95-464, launched at 479-483): dK, dV (key/value-stationary)
 * and dQ (query-stationary, recomputing S and dP instead of the reference's
 * fp32 atomicAdd) in one launch, from the workspace fa_bwd_preprocess filled.
 * Overwrites dq, dk and dv, and uses the workspace's counters and slots
 * (leaving the counters zero). Two calls must not share a workspace at once.
 */
int fa_bwd_main(const void* q, const void* k, const void* v, const void* dO,
                void* workspace, size_t workspace_bytes, float* dq,
                void* dk, void* dv, int B, int Hq, int Hkv, int N, int D,
                int causal, void* stream);

/*
 * Options of the general pair below; a zeroed struct (or a NULL pointer)
 * means fp16, dense (B, H, N, D), no key lengths, no window, no ALiBi, no
 * packed sequences, no mask, no dropout, no bias.
 *   - dtype: FA_DTYPE_FP16 or FA_DTYPE_BF16 for q, k, v, o, dO, dq, dk, dv
 *     (bf16: products on the bf16 MFMA with fp32 accumulation, P and dS
 *     rounded to bf16 as operands, outputs rounded to nearest even);
 *   - layout: FA_LAYOUT_BHND or FA_LAYOUT_BNHD (see fa_fwd_bnhd);
 *   - kv_len: NULL, or a device array of B int32 key lengths: for batch entry
 *     b only keys [0, kv_len[b]) exist (right padding; values are clamped to
 *     [1, N]), every query row (pad rows included) attends to those keys
 *     only, and dk/dv rows past kv_len[b] come out zero;
 *   - window: 0, or W > 0 (causal only): query row i attends to keys
 *     (i - W, i]. With key lengths too, a pad row more than W past its
 *     entry's length sees no key: its o is 0, its lse +inf, its gradients 0;
 *   - alibi_slopes: NULL, or a device array of Hq fp32 slopes: the scaled
 *     score of query row i and key j of query head h gets
 *     -alibi_slopes[h] * |i - j| added (the usual ALiBi bias);
 *   - seg_start, seg_end: both NULL, or two device arrays of B * N int32:
 *     several sequences packed into each batch entry. Token i of entry b
 *     belongs to the sequence of tokens [seg_start[b*N+i], seg_end[b*N+i])
 *     and attends to keys of that sequence only (with the causal mask, keys
 *     seg_start .. i; without it, the whole sequence). The arrays
 *     must describe contiguous sequences that tile [0, N) (so both never
 *     decrease along a row); other contents give undefined attention values
 *     but no access outside the tensors (each bound is clamped to reach at
 *     least the token itself);
 *   - scale: 0 (the reference's fixed 1/sqrt(D), fa_p100_ext.cu:71, 117), or
 *     a positive softmax scale applied to q . k before the masks; dq and dk
 *     carry it as they carry 1/sqrt(D), and lse is in units of the scaled
 *     logits;
 *   - mask, mask_t, mask_heads: an arbitrary boolean attention mask on top of
 *     every other one (mask = NULL: none). W = ceil(N / 32) words per row;
 *     plane p = b * mask_heads + (mask_heads == 1 ? 0 : h) for query head h
 *     (mask_heads is 1, one plane per batch entry shared by all heads, or Hq).
 *     Query i may attend key j iff bit j % 32 of mask[(p * N + i) * W + j / 32]
 *     is set; mask_t holds the same bits transposed, bit i % 32 of
 *     mask_t[(p * N + j) * W + i / 32]. The forward reads mask, the backward
 *     both (mask_t is required there). fa_pack_mask writes both from a dense
 *     boolean mask. A row with no key left gets o = 0, lse = +inf and zero
 *     gradients;
 *   - drop, drop_t, drop_scale: attention dropout (drop = NULL: none). Keep
 *     bits in the layouts of mask and mask_t with one plane per (b, query
 *     head) (plane b * Hq + h; bit set = keep), and the factor drop_scale
 *     (1 / (1 - p)) the kept probabilities are scaled by: o = (P * Z *
 *     drop_scale) v with P the softmax over every key, lse that softmax's
 *     (dropout does not touch it). The forward reads drop, the backward both
 *     (drop_t is required there) with the same bits and scale as the
 *     forward. fa_dropout_bits draws them;
 *   - bias, bias_stride_b, bias_stride_h, dbias: an additive attention bias
 *     (bias = NULL: none), fp32, added to the scaled logits before the masks
 *     and the softmax: element (b, h, i, j) of query head h at
 *     bias[b * bias_stride_b + h * bias_stride_h + i * N + j] (strides in
 *     elements, 0 to share one plane over batch entries or heads; rows are
 *     dense). The backward writes the bias's gradient, dS of the scaled
 *     logits, to dbias when it is not NULL: dense (B, Hq, N, N) fp32, only
 *     where a query row meets a key it may attend (the caller zeroes dbias
 *     first; reduce over shared dimensions afterwards);
 *   - kv_rows: 0, or the number of key/value rows Nk when it differs from
 *     the query rows (the N of the call): k, v, dk, dv are then
 *     (B, Hkv, Nk, D) (or (B, Nk, Hkv, D)), q, o, dO, dq, lse keep N rows.
 *     Causal masking aligns the last query row with the last key row
 *     (bottom-right): query i sees key j iff j <= i + Nk - N, as in KV-cache
 *     decoding (N = 1) and chunked prefill (N < Nk); with N > Nk the first
 *     N - Nk rows see no key (o = 0, lse = +inf, zero gradients). Windows
 *     and ALiBi distances count from that diagonal, key lengths clamp to
 *     [1, Nk]. Not with packed sequences, a mask, dropout or a bias
 *     (FA_ERR_KV_ROWS); the backward workspace is the one for N rows.
 *     The reference requires q_len == kv_len (fa_p100_hf.py:100-105).
 *   - block_rows, block_cols: a block-sparse layout (block_rows = NULL:
 *     none). With nb = ceil(N / FA_SPARSE_BLOCK) blocks of FA_SPARSE_BLOCK
 *     query rows and as many of keys, query row i may attend key j only if
 *     block (i / FA_SPARSE_BLOCK, j / FA_SPARSE_BLOCK) is visible for its
 *     query head, on top of every other mask; the kernels step over the
 *     visible blocks only, so the work scales with their number. A row with
 *     no visible key gets o = 0, lse = +inf and zero gradients. The lists
 *     fa_pack_blocks writes from a boolean layout: block_rows for query
 *     head h of entry b (plane p = b * Hq + h) and query block r, at
 *     block_rows[(p * nb + r) * (nb + 1)], the count of visible key blocks
 *     and then their indices in ascending order; block_cols for kv head g of
 *     entry b (plane p = b * Hkv + g) and key block c, at
 *     block_cols[(p * nb + c) * (G * nb + 1)] (G = Hq / Hkv), the count of
 *     (query head, query block) pairs that see it and then those pairs as
 *     hg * nb + r (query head g * G + hg) in ascending order. Every entry
 *     past a count must still be a valid index. The forward reads
 *     block_rows, the backward both. Not with a mask, a bias or kv_rows != N
 *     (FA_ERR_BLOCKS); with dropout, causal masking, key lengths, windows,
 *     ALiBi, packed sequences and a scale. No counterpart in the reference,
 *     which raises on block-sparse patterns (README.md:72-75).
 */
typedef struct fa_options {
  int dtype;
  int layout;
  const int* kv_len;
  int window;
  const float* alibi_slopes;
  const int* seg_start;
  const int* seg_end;
  float scale;
  const uint32_t* mask;
  const uint32_t* mask_t;
  int mask_heads;
  const uint32_t* drop;
  const uint32_t* drop_t;
  float drop_scale;
  const float* bias;
  long long bias_stride_b;
  long long bias_stride_h;
  float* dbias;
  int kv_rows;
  const int* block_rows;
  const int* block_cols;
} fa_options;

/*
 * The general pair: every entry point above is one of its cases, plus bf16,
 * key padding, sliding windows, ALiBi, packed sequences and masks (`opts`).
 * fa_bwd_ex writes dq in the element format (fp16 or bf16); lse and the
 * workspace as in fa_bwd. No counterpart in the reference, which raises on
 * bf16, masks and windows (README.md:72-75, fa_p100_ext.cu:33,
 * fa_p100_hf.py:64-82) and has no bias or packing input; the HF hook uses key
 * lengths, windows, packed sequences and masks.
 */
int fa_fwd_ex(const void* q, const void* k, const void* v, void* o, float* lse,
              int B, int Hq, int Hkv, int N, int D, int causal, const fa_options* opts,
              void* stream);
int fa_bwd_ex(const void* q, const void* k, const void* v, const void* dO, const void* o,
              const float* lse, void* dq, void* dk, void* dv, void* workspace,
              size_t workspace_bytes, int B, int Hq, int Hkv, int N, int D, int causal,
              const fa_options* opts, void* stream);

/*
 * Bit-packs a dense boolean mask for fa_options.mask / mask_t. No counterpart
 * in the reference, which takes no mask (fa_p100_hf.py:64-70). `dense` is P
 * planes of N x N bytes, row-major (plane p, query row i, key j at
 * (p * N + i) * N + j; nonzero = may attend), as a torch.bool tensor holds
 * them. Writes P * N * ceil(N/32) words to `bits` and, when `bits_t` is not
 * NULL, as many to `bits_t` (layouts as fa_options.mask / mask_t; bits past N
 * in a row's last word are 0). Asynchronous on `stream`.
 */
int fa_pack_mask(const uint8_t* dense, int P, int N, uint32_t* bits, uint32_t* bits_t,
                 void* stream);

/*
 * Dropout keep bits for fa_options.drop / drop_t. No counterpart in the
 * reference, whose hook raises on dropout (fa_p100_hf.py:83-85). For each of
 * the P = B * H planes, row i and key j < N: with h the 32-bit integer hash
 * lowbias32 (C. Wellons: x ^= x >> 16; x *= 0x7feb352d; x ^= x >> 15;
 * x *= 0x846ca68b; x ^= x >> 16), the row key r = h(h(h(h(lo) ^ hi) ^ plane)
 * ^ i) of the seed's low and high words, and u = h(r ^ (j / 2)), key j draws
 * the low (j even) or high (j odd) 16 bits of u and is kept iff that draw is
 * at least t = min(65535, round(p * 65536)). The drop probability is then
 * t / 65536 and fa_dropout_scale(p) = 65536 / (65536 - t) the matching
 * scale. Writes P * N * ceil(N/32) words to bits and, when bits_t is not
 * NULL, as many to bits_t; bits past N are 0. p must lie in [0, 1)
 * (FA_ERR_DROPOUT otherwise; fa_dropout_scale then returns 0).
 */
int fa_dropout_bits(uint64_t seed, float p, int P, int N, uint32_t* bits, uint32_t* bits_t,
                    void* stream);
/*
 * fa_dropout_bits for causal attention with as many key rows as query rows:
 * the same draw with every bit of a key j > i (row i) cleared, in both
 * layouts. Causal masking never reads those bits, so attention results are
 * the same as with fa_dropout_bits' planes; the draw skips the hashes of
 * words wholly past the diagonal (about half of them). No counterpart in the
 * reference. Errors as fa_dropout_bits.
 */
int fa_dropout_bits_causal(uint64_t seed, float p, int P, int N, uint32_t* bits,
                           uint32_t* bits_t, void* stream);
float fa_dropout_scale(float p);

/*
 * The lists of fa_options.block_rows / block_cols from a boolean block
 * layout. No counterpart in the reference (README.md:72-75: no block-sparse
 * patterns). `layout` is layout_b x layout_h planes of nb x nb bytes
 * (nb = ceil(N / FA_SPARSE_BLOCK); plane (b, h), query block r, key block c
 * at ((b * layout_h + h) * nb + r) * nb + c; nonzero = visible), with
 * layout_b 1 or B and layout_h 1 or Hq (1 shares one plane). Writes
 * B * Hq * nb * (nb + 1) int32 to block_rows and, when block_cols is not
 * NULL, B * Hkv * nb * ((Hq / Hkv) * nb + 1) int32 to block_cols. With
 * causal != 0 the blocks above the diagonal (key block > query block) are
 * left out of both lists, as a causal call never needs them (lists packed
 * without it still give the same results, with more work). Asynchronous on
 * `stream`.
 */
int fa_pack_blocks(const uint8_t* layout, int layout_b, int layout_h, int B, int Hq, int Hkv,
                   int N, int causal, int* block_rows, int* block_cols, void* stream);

/*
 * fa_bwd without a workspace argument and without any allocation. No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory at the call (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The backward's two per-row vectors live in
 * a built-in device array of FA_BWD_NOALLOC_SCRATCH_BYTES per GPU (held until
 * the process ends), so the shape must satisfy 2 * align256(B*Hq*N*4) <=
 * FA_BWD_NOALLOC_SCRATCH_BYTES (B*Hq*N <= 2^21 rows), else FA_ERR_SCRATCH and
 * nothing is launched. The causal load balancing that needs workspace slots is
 * off, so dk and dv may differ from fa_bwd's in the last bits (dq is the same);
 * results are deterministic. `stream` must belong to the current device.
 * Every call on a GPU shares that GPU's scratch: calls that overlap in time
 * on one GPU (other streams, other host threads) race and give wrong results;
 * calls ordered on one stream are fine.
 */
#define FA_BWD_NOALLOC_SCRATCH_BYTES (16u << 20)
int fa_bwd_noalloc(const void* q, const void* k, const void* v, const void* dO,
                   const void* o, const float* lse, float* dq, void* dk, void* dv,
                   int B, int Hq, int Hkv, int N, int D, int causal, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* FA_MI355X_H_ */
