// Host-side launch descriptors shared by the kernels and the C ABI layer.
// Arguments are validated by the C ABI (fa_capi.hip) before these are called.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

// Memory layouts of the (B, H, N, D) fp16 tensors: kBHND is dense (B, H, N, D)
// (the reference's layout); kBNHD stores the same logical tensor as dense
// (B, N, H, D), the layout of the projections in a transformer block.
enum Layout : int { kBHND = 0, kBNHD = 1 };
// Element format of the 16-bit tensors (lse and the workspace are fp32).
enum Dtype : int { kFP16 = 0, kBF16 = 1 };

// Element strides of one (B, H, N, D) tensor with `heads` heads.
struct Strides {
  long long b;  // between batches
  long long h;  // between heads
  int n;        // between rows (sequence positions)
};
inline Strides make_strides(int layout, int heads, int N, int D) {
  if (layout == kBNHD) return {(long long)N * heads * D, (long long)D, heads * D};
  return {(long long)heads * N * D, (long long)N * D, D};
}

struct FwdArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int B, Hq, Hkv, N, D;
  bool causal;
  void* stream;
  int layout = kBHND;  // of q, k, v, o (lse is always dense (B, Hq, N))
  int dtype = kFP16;   // of q, k, v, o
  const int* kv_len = nullptr;  // device, B entries: keys [0, kv_len[b]) exist (else N)
  int window = 0;               // causal sliding window W: row i sees keys (i - W, i]; 0 = none
  const float* alibi = nullptr; // device, Hq slopes: score(i, j) += -slope * |i - j|
  // Packed sequences, device (B, N) each: token i of entry b belongs to the
  // sequence of tokens [seg_start[b][i], seg_end[b][i]) and sees keys of that
  // sequence only (with causal masking, those up to itself).
  const int* seg_start = nullptr;
  const int* seg_end = nullptr;
  float scale = 0.f;  // softmax scale of the logits; 0 = 1/sqrt(D)
  // Arbitrary boolean mask, device, bit-packed in rows of W = ceil(N / 32)
  // words: bit j % 32 of word ((b * mask_heads + h') * N + i) * W + j / 32 is
  // set iff query i may attend key j (h' = query head h when mask_heads == Hq,
  // 0 when mask_heads == 1). Applied on top of every other mask.
  const uint32_t* mask = nullptr;
  int mask_heads = 0;
  // Attention dropout: keep bits in the mask's row layout with one plane per
  // (b, query head) (bit set = keep), and the factor kept probabilities are
  // scaled by (1 / (1 - p)). P stays normalised over every key; only P V
  // sees the dropped probabilities.
  const uint32_t* drop = nullptr;
  float drop_scale = 1.f;
  // Additive attention bias, fp32, added to the scaled logits: element
  // (b, h, i, j) at bias[b * bias_sb + h * bias_sh + i * N + j] (strides in
  // elements; 0 broadcasts over that dimension).
  const float* bias = nullptr;
  long long bias_sb = 0, bias_sh = 0;
  // Rows of k and v when they differ from q's N (0: N). Causal masking then
  // aligns the last query row with the last key row: query i sees key j iff
  // j <= i + Nkv - N, and windows and ALiBi distances count from that
  // diagonal. Only without packed sequences, a mask, dropout or a bias.
  int Nkv = 0;
  // Block-sparse layout (kSparseBlock x kSparseBlock blocks, nb = ceil(N /
  // kSparseBlock) per side), device int32: for plane p = b * Hq + h and query
  // block r, entry ((p * nb + r) * (nb + 1)) holds the count c of the key
  // blocks row block r may attend, followed by those blocks' indices in
  // ascending order (then padding, each a valid index). Keys outside them
  // are masked; the kernels step over the listed blocks only.
  const int* block_rows = nullptr;
};

// Rows and keys per block of a block-sparse layout.
constexpr int kSparseBlock = 128;

// Key rows of a launch: Nkv, or N when Nkv is 0.
inline int key_rows(int N, int Nkv) { return Nkv > 0 ? Nkv : N; }

// Backward workspace, in this order (each part 256-byte aligned):
//   dvec = rowsum(dO * O) and lse2 = LSE * log2(e), (B, Hq, N) fp32 each;
//   one counter per pair of key tiles (u, n_tiles-1-u) per (b, head), which
//   the preprocess kernel zeroes (sized by Hq, which bounds Hkv, so that the
//   preprocess needs no Hkv);
//   two fp32 partial dK/dV slots per such pair and (b, kv head).
// Head dims: any multiple of 8 from 8 to 256 (the `D` of the argument
// structs, the row length in memory). The kernels are compiled for the
// widths 32, 64, 96, 128 and 256 and run a head dim on the smallest that
// holds it: the extra columns load as zeros and are never stored.
inline int padded_head_dim(int D) {
  return D <= 32 ? 32 : D <= 64 ? 64 : D <= 96 ? 96 : D <= 128 ? 128 : 256;
}
inline bool valid_head_dim(int D) { return D >= 8 && D <= 256 && D % 8 == 0; }

constexpr int kBwdTile = 128;  // key rows of one backward workgroup
struct BwdWorkspace {
  size_t dvec, lse2, counters, slots, total;
  int n_counters;
};
inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
inline size_t bwd_slot_floats(int D) {  // dK^T, dV^T at the padded width
  return (size_t)kBwdTile * padded_head_dim(D) * 2;
}
inline BwdWorkspace bwd_workspace(int B, int Hq, int Hkv, int N, int D) {
  BwdWorkspace w;
  const size_t vec = align256((size_t)B * Hq * N * sizeof(float));
  const int pairs_per_head = ((N + kBwdTile - 1) / kBwdTile) / 2;
  w.dvec = 0;
  w.lse2 = vec;
  w.counters = 2 * vec;
  w.n_counters = B * Hq * pairs_per_head;
  w.slots = w.counters + align256((size_t)w.n_counters * sizeof(unsigned));
  w.total = w.slots + (size_t)B * Hkv * pairs_per_head * 2 * bwd_slot_floats(D) * sizeof(float);
  return w;
}

struct BwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* dO;
  const void* o;
  const float* lse;
  float* dvec;   // workspace: rowsum(dO * O), (B, Hq, N)
  float* lse2;   // workspace: LSE * log2(e), (B, Hq, N)
  float* dq;     // fp32 dQ (the reference's dtype), or
  void* dq16;    // when non-null, fp16 dQ here instead (dq is then unused)
  void* dk;
  void* dv;
  int B, Hq, Hkv, N, D;
  bool causal;
  void* stream;
  int layout = kBHND;  // of q, k, v, dO, o, dq, dk, dv (lse, workspace dense)
  unsigned* counters = nullptr;  // workspace: per key-tile pair (zeroed by the preprocess)
  int n_counters = 0;
  // Workspace: partial dK/dV of split key tiles. Null turns the causal split
  // off (every key tile's phase 1 stays in its own workgroup), so neither the
  // slots nor the counters are touched.
  float* slots = nullptr;
  int dtype = kFP16;             // of q, k, v, dO, o, dk, dv and dq16
  const int* kv_len = nullptr;   // as FwdArgs::kv_len
  int window = 0;                // as FwdArgs::window
  const float* alibi = nullptr;  // as FwdArgs::alibi
  const int* seg_start = nullptr;  // as FwdArgs::seg_start
  const int* seg_end = nullptr;    // as FwdArgs::seg_end
  float scale = 0.f;               // as FwdArgs::scale
  const uint32_t* mask = nullptr;  // as FwdArgs::mask
  // The same bits transposed: bit i % 32 of word ((b * mask_heads + h') * N +
  // j) * W + i / 32 (set iff query i may attend key j); required with mask.
  const uint32_t* mask_t = nullptr;
  int mask_heads = 0;              // as FwdArgs::mask_heads
  const uint32_t* drop = nullptr;  // as FwdArgs::drop
  const uint32_t* drop_t = nullptr;  // its transpose (as mask_t); required with drop
  float drop_scale = 1.f;          // as FwdArgs::drop_scale
  const float* bias = nullptr;     // as FwdArgs::bias
  long long bias_sb = 0, bias_sh = 0;
  // Gradient of the bias: dS (the gradient of the scaled logits), dense
  // (B, Hq, N, N) fp32; written where a row meets a key, so the caller
  // zeroes it first. Null: not computed.
  float* dbias = nullptr;
  int Nkv = 0;                     // as FwdArgs::Nkv (k, v, dk, dv rows)
  const int* block_rows = nullptr;  // as FwdArgs::block_rows (required with block_cols)
  // The layout by key block: for plane p = b * Hkv + hkv and key block c,
  // entry ((p * nb + c) * (G * nb + 1)) holds the count of (query head,
  // query block) pairs that attend key block c, followed by those pairs as
  // g * nb + r (query head hkv * G + g, G = Hq / Hkv) in ascending order
  // (then padding, each a valid pair).
  const int* block_cols = nullptr;
};

hipError_t launch_fwd(const FwdArgs& a);
hipError_t launch_bwd_preprocess(const BwdArgs& a);
hipError_t launch_bwd_main(const BwdArgs& a);
// Dense boolean mask (P planes of N x N bytes) to the bit layouts of
// FwdArgs::mask (bits) and BwdArgs::mask_t (bits_t, skipped when null).
hipError_t launch_pack_mask(const uint8_t* dense, int P, int N, uint32_t* bits, uint32_t* bits_t,
                            void* stream);
// Dropout keep bits for P planes of N x N (bits and, when not null, bits_t;
// layouts as the mask's): key j of row i in plane p is kept iff its 16-bit
// draw is at least `threshold` (see fa_dropout_bits); causal: and j <= i.
hipError_t launch_dropout_bits(uint64_t seed, uint32_t threshold, int P, int N, bool causal,
                               uint32_t* bits, uint32_t* bits_t, void* stream);
// A dense block-sparse layout (Bl x Hl planes of nb x nb bytes, nonzero =
// visible; Bl in {1, B} and Hl in {1, Hq} broadcast) to the lists of
// FwdArgs::block_rows and BwdArgs::block_cols (skipped when null). causal:
// blocks wholly above the diagonal (key block > query block) are left out.
hipError_t launch_pack_blocks(const uint8_t* layout, int Bl, int Hl, int B, int Hq, int Hkv,
                              int nb, bool causal, int* rows, int* cols, void* stream);

// Work-items (workgroups x threads) of the largest launch each pass makes for
// a shape (either masking). An AMD dispatch packet counts its grid in
// work-items in 32-bit fields, and the kernels number their work items with
// int, so a shape is launchable when these fit in 32 bits (checked by the C
// ABI before any launch).
// Nkv: rows of k and v (as FwdArgs::Nkv; 0 = N).
unsigned long long fwd_launch_items(int B, int Hq, int N, int D);
unsigned long long bwd_launch_items(int B, int Hq, int Hkv, int N, int D, int Nkv = 0);

}  // namespace fa
