// C ABI entry points (declared in include/fa_mi355x.h).
//
// Validation here mirrors the reference binding's checks that do not need
// torch (fa_p100_ext.cu:59-65, 111-113): head dim, positive N, the head
// grouping. Tensor-type checks ("must be a CUDA tensor", "must be fp16") live
// in the torch extension, where tensors exist. Nothing here allocates or keeps
// state: every kernel's LDS is static, so launches need no attributes set.
#include <limits.h>

#include <cmath>
#include <mutex>

#include "../../include/fa_mi355x.h"
#include "fa_launch.h"

namespace {

// Largest span of one head's rows, in elements: N rows of row_elems 16-bit
// values (D, or H*D in the (B, N, H, D) layout). Buffer resources hold 32-bit
// byte ranges, and a staged tile addresses up to 255 rows past a head's last
// row, which must read as zeros, so their byte offsets must not wrap:
// (N + 256) rows stay below 2^32 bytes. A head dim narrower than its tile
// width marks the extra columns with lane offsets from 2^31 up, so there the
// rows (and the scalar offsets added to those lanes) stay below 2^30 bytes.
bool rows_fit(int N, long long row_elems, int D) {
  const long long limit = fa::padded_head_dim(D) == D ? (long long)INT_MAX : (1LL << 29);
  return (long long)(N + 256) * row_elems <= limit;
}

int check_shape(int B, int Hq, int Hkv, int N, int D) {
  if (!fa::valid_head_dim(D)) return FA_ERR_HEAD_DIM;
  if (N <= 0) return FA_ERR_SEQLEN;
  if (Hkv <= 0 || Hq <= 0 || Hq % Hkv != 0) return FA_ERR_HEADS;
  if (B <= 0) return FA_ERR_BATCH;
  // Kernels index rows of one (b, h) slice with 32-bit ints and whole tensors
  // with 64-bit offsets; every launch is a 1-D grid whose work-item count
  // (workgroups x threads) must fit the dispatch packet's 32-bit field.
  if (!rows_fit(N, D, D)) return FA_ERR_TOO_LARGE;
  constexpr unsigned long long kMaxItems = 0xFFFFFFFFull;
  if (fa::fwd_launch_items(B, Hq, N, D) > kMaxItems ||
      fa::bwd_launch_items(B, Hq, Hkv, N, D) > kMaxItems)
    return FA_ERR_TOO_LARGE;
  return FA_OK;
}

// The (B, N, H, D) layout addresses one head's rows through a buffer range
// that spans all H heads: rows of H * D halves.
int check_bnhd(int Hq, int N, int D) {
  return rows_fit(N, (long long)Hq * D, D) ? FA_OK : FA_ERR_TOO_LARGE;
}

int to_code(hipError_t e) { return e == hipSuccess ? FA_OK : (int)e; }

// ---------------------------------------------------------------------------
// Built-in scratch for fa_bwd_noalloc: the backward's two per-row vectors
// (dvec = rowsum(dO * o) and lse * log2(e)) live in this file-scope device
// array instead of a caller-allocated workspace. Every GPU the library runs on
// holds its own copy until the process ends. In host code `scratch` names a
// host-side stand-in, not a device address, so host code never passes it to a
// kernel: the device address comes from hipGetSymbolAddress, taken once per
// device (with that device current) on the entry point's first call there.
constexpr size_t kScratchBytes = (size_t)FA_BWD_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];
float* g_scratch_ptr[kMaxDevices];

// Device address of the current device's scratch, or an error code.
int scratch_of_current_device(float** out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? static_cast<float*>(p) : nullptr;
  });
  if (g_scratch_err[dev] != hipSuccess) return (int)g_scratch_err[dev];
  if (g_scratch_ptr[dev] == nullptr) return (int)hipErrorInvalidSymbol;
  *out = g_scratch_ptr[dev];
  return FA_OK;
}

}  // namespace

extern "C" {

const char* fa_error_string(int err) {
  switch (err) {
    case FA_OK: return "success";
    case FA_ERR_HEAD_DIM: return "head dim must be a multiple of 8 from 8 to 256";
    case FA_ERR_SEQLEN: return "N must be positive";
    case FA_ERR_HEADS: return "query heads (H) must be a multiple of key/value heads (Hkv)";
    case FA_ERR_BATCH: return "B must be positive";
    case FA_ERR_NULL: return "a required pointer is NULL";
    case FA_ERR_WORKSPACE: return "workspace is smaller than fa_bwd_workspace_bytes()";
    case FA_ERR_TOO_LARGE: return "shape exceeds the kernels' index range";
    case FA_ERR_LAYOUT: return "layout must be FA_LAYOUT_BHND or FA_LAYOUT_BNHD";
    case FA_ERR_DTYPE: return "unsupported element format";
    case FA_ERR_WINDOW: return "sliding window must be >= 0 and needs causal masking";
    case FA_ERR_SEGMENTS:
      return "packed sequences need both seg_start and seg_end";
    case FA_ERR_SCALE: return "softmax scale must be 0 (1/sqrt(D)) or positive and finite";
    case FA_ERR_MASK:
      return "mask_heads must be 1 or Hq, and the backward needs mask_t with mask";
    case FA_ERR_DROPOUT:
      return "dropout p must lie in [0, 1) and its scale be positive and finite; the backward "
             "needs drop_t with drop";
    case FA_ERR_BIAS:
      return "bias strides must not be negative, dbias needs a bias, and a bias needs N <= 2^22 "
             "and a head dim up to 128";
    case FA_ERR_KV_ROWS:
      return "kv_rows must be >= 0, and key rows that differ from the query rows do not combine "
             "with packed sequences, a mask, dropout or a bias";
    case FA_ERR_BLOCKS:
      return "a block-sparse layout does not combine with a mask, a bias or key rows that differ "
             "from the query rows, and the backward needs block_cols with block_rows";
    case FA_ERR_SCRATCH:
      return "fa_bwd_noalloc: 2 * B*Hq*N floats exceed the built-in scratch "
             "(FA_BWD_NOALLOC_SCRATCH_BYTES); use fa_bwd with a workspace";
    default: return hipGetErrorString((hipError_t)err);
  }
}

const char* fa_version(void) { return "fa_mi355x 1.0 gfx950"; }

// Options: every field checked; the defaults are fp16, (B, H, N, D), no key
// lengths, no window, no ALiBi, no packed sequences, no mask.
constexpr fa_options kDefaultOpts = {fa::kFP16, fa::kBHND, nullptr, 0,       nullptr,
                                     nullptr,   nullptr,   0.f,     nullptr, nullptr,
                                     0,         nullptr,   nullptr, 0.f,
                                     nullptr,   0,         0,       nullptr};

// `backward`: the pass reads mask_t too.
// Largest sequence length with a bias: the kernels read the bias through
// buffer resources of 32 rows of N fp32 values, whose sizes stay below 2^32.
// (One N x N fp32 plane at this N is 64 TiB, so no real caller meets it.)
static constexpr int kMaxBiasN = 1 << 22;

static int check_opts(const fa_options& op, int causal, int Hq, int N, int D, bool backward) {
  if (op.dtype != fa::kFP16 && op.dtype != fa::kBF16) return FA_ERR_DTYPE;
  if (op.layout != fa::kBHND && op.layout != fa::kBNHD) return FA_ERR_LAYOUT;
  if (op.window < 0 || (op.window > 0 && !causal)) return FA_ERR_WINDOW;
  if ((op.seg_start != nullptr) != (op.seg_end != nullptr)) return FA_ERR_SEGMENTS;
  if (!(op.scale >= 0.f) || !std::isfinite(op.scale)) return FA_ERR_SCALE;
  if (op.mask != nullptr) {
    if (op.mask_heads != 1 && op.mask_heads != Hq) return FA_ERR_MASK;
    if (backward && op.mask_t == nullptr) return FA_ERR_MASK;
  }
  if (op.drop != nullptr) {
    if (!(op.drop_scale > 0.f) || !std::isfinite(op.drop_scale)) return FA_ERR_DROPOUT;
    if (backward && op.drop_t == nullptr) return FA_ERR_DROPOUT;
  }
  if (op.bias_stride_b < 0 || op.bias_stride_h < 0) return FA_ERR_BIAS;
  if (op.dbias != nullptr && op.bias == nullptr) return FA_ERR_BIAS;
  if (op.bias != nullptr && N > kMaxBiasN) return FA_ERR_BIAS;
  // (the width-256 kernels have no registers left for the bias values)
  if (op.bias != nullptr && fa::padded_head_dim(D) > 128) return FA_ERR_BIAS;
  if (op.kv_rows < 0) return FA_ERR_KV_ROWS;
  if (op.kv_rows > 0 && op.kv_rows != N &&
      (op.seg_start != nullptr || op.mask != nullptr || op.drop != nullptr || op.bias != nullptr))
    return FA_ERR_KV_ROWS;
  if (op.block_rows != nullptr) {
    if (op.mask != nullptr || op.bias != nullptr || (op.kv_rows > 0 && op.kv_rows != N))
      return FA_ERR_BLOCKS;
    if (backward && op.block_cols == nullptr) return FA_ERR_BLOCKS;
  } else if (op.block_cols != nullptr) {
    return FA_ERR_BLOCKS;
  }
  return FA_OK;
}

// The k/v side of a shape whose key rows differ from the query rows
// (fa_options.kv_rows): the same row-span and launch-size limits.
static int check_kv_rows(const fa_options& op, int B, int Hq, int Hkv, int N, int D) {
  if (op.kv_rows <= 0 || op.kv_rows == N) return FA_OK;
  const int NK = op.kv_rows;
  if (!rows_fit(NK, op.layout == fa::kBNHD ? (long long)Hkv * D : D, D)) return FA_ERR_TOO_LARGE;
  if (fa::bwd_launch_items(B, Hq, Hkv, N, D, NK) > 0xFFFFFFFFull) return FA_ERR_TOO_LARGE;
  return FA_OK;
}

// Keep threshold of a drop probability: 16-bit draws >= t are kept.
static uint32_t dropout_threshold(float p) {
  const double t = std::nearbyint((double)p * 65536.0);
  return (uint32_t)(t < 0.0 ? 0.0 : t > 65535.0 ? 65535.0 : t);
}

static int fwd(const void* q, const void* k, const void* v, void* o, float* lse, int B, int Hq,
               int Hkv, int N, int D, int causal, const fa_options& op, void* stream) {
  int rc = check_opts(op, causal, Hq, N, D, false);
  if (rc == FA_OK) rc = check_shape(B, Hq, Hkv, N, D);
  if (rc == FA_OK && op.layout == fa::kBNHD) rc = check_bnhd(Hq, N, D);
  if (rc == FA_OK) rc = check_kv_rows(op, B, Hq, Hkv, N, D);
  if (rc != FA_OK) return rc;
  if (!q || !k || !v || !o || !lse) return FA_ERR_NULL;
  fa::FwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.N = N;
  a.D = D;
  a.causal = causal != 0;
  a.stream = stream;
  a.layout = op.layout;
  a.dtype = op.dtype;
  a.kv_len = op.kv_len;
  a.window = op.window;
  a.alibi = op.alibi_slopes;
  a.seg_start = op.seg_start;
  a.seg_end = op.seg_end;
  a.scale = op.scale;
  a.mask = op.mask;
  a.mask_heads = op.mask_heads;
  a.drop = op.drop;
  a.drop_scale = op.drop ? op.drop_scale : 1.f;
  a.bias = op.bias;
  a.bias_sb = op.bias_stride_b;
  a.bias_sh = op.bias_stride_h;
  a.Nkv = op.kv_rows;
  a.block_rows = op.block_rows;
  return to_code(fa::launch_fwd(a));
}

int fa_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int B, int Hq,
           int Hkv, int N, int D, int causal, int full_precision, void* stream) {
  (void)full_precision;  // fp16 products are exact in the fp32 accumulator
  return fwd(q, k, v, o, lse, B, Hq, Hkv, N, D, causal, kDefaultOpts, stream);
}

int fa_fwd_bnhd(const void* q, const void* k, const void* v, void* o, float* lse, int B, int Hq,
                int Hkv, int N, int D, int causal, void* stream) {
  fa_options op = kDefaultOpts;
  op.layout = fa::kBNHD;
  return fwd(q, k, v, o, lse, B, Hq, Hkv, N, D, causal, op, stream);
}

int fa_fwd_ex(const void* q, const void* k, const void* v, void* o, float* lse, int B, int Hq,
              int Hkv, int N, int D, int causal, const fa_options* opts, void* stream) {
  return fwd(q, k, v, o, lse, B, Hq, Hkv, N, D, causal, opts ? *opts : kDefaultOpts, stream);
}

size_t fa_bwd_workspace_bytes(int B, int Hq, int Hkv, int N, int D) {
  if (check_shape(B, Hq, Hkv, N, D) != FA_OK) return 0;
  return fa::bwd_workspace(B, Hq, Hkv, N, D).total;
}

static int bwd_pre(const void* dO, const void* o, const float* lse, void* workspace,
                   size_t workspace_bytes, int B, int Hq, int N, int D, int layout, int dtype,
                   void* stream) {
  int rc = check_shape(B, Hq, Hq, N, D);
  if (rc == FA_OK && layout == fa::kBNHD) rc = check_bnhd(Hq, N, D);
  if (rc != FA_OK) return rc;
  if (!dO || !o || !lse || !workspace) return FA_ERR_NULL;
  // The vectors and counters this writes lie before the slots, whose offset
  // depends on neither Hkv nor D.
  const fa::BwdWorkspace w = fa::bwd_workspace(B, Hq, Hq, N, D);
  if (workspace_bytes < w.slots) return FA_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  fa::BwdArgs a{};
  a.dO = dO;
  a.o = o;
  a.lse = lse;
  a.dvec = reinterpret_cast<float*>(ws + w.dvec);
  a.lse2 = reinterpret_cast<float*>(ws + w.lse2);
  a.counters = reinterpret_cast<unsigned*>(ws + w.counters);
  a.n_counters = w.n_counters;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hq;
  a.N = N;
  a.D = D;
  a.stream = stream;
  a.layout = layout;
  a.dtype = dtype;
  return to_code(fa::launch_bwd_preprocess(a));
}

int fa_bwd_preprocess(const void* dO, const void* o, const float* lse, void* workspace,
                      size_t workspace_bytes, int B, int Hq, int N, int D, void* stream) {
  return bwd_pre(dO, o, lse, workspace, workspace_bytes, B, Hq, N, D, fa::kBHND, fa::kFP16,
                 stream);
}

// Shared by the main-kernel entry points: fp32 dq or 16-bit dq16.
static int bwd_main(const void* q, const void* k, const void* v, const void* dO,
                    void* workspace, size_t workspace_bytes, float* dq, void* dq16,
                    void* dk, void* dv, int B, int Hq, int Hkv, int N, int D, int causal,
                    const fa_options& op, void* stream) {
  int rc = check_opts(op, causal, Hq, N, D, true);
  if (rc == FA_OK) rc = check_shape(B, Hq, Hkv, N, D);
  if (rc == FA_OK && op.layout == fa::kBNHD) rc = check_bnhd(Hq, N, D);
  if (rc == FA_OK) rc = check_kv_rows(op, B, Hq, Hkv, N, D);
  if (rc != FA_OK) return rc;
  if (!q || !k || !v || !dO || !workspace || !(dq || dq16) || !dk || !dv) return FA_ERR_NULL;
  const fa::BwdWorkspace w = fa::bwd_workspace(B, Hq, Hkv, N, D);
  if (workspace_bytes < w.total) return FA_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  fa::BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.dO = dO;
  a.dvec = reinterpret_cast<float*>(ws + w.dvec);
  a.lse2 = reinterpret_cast<float*>(ws + w.lse2);
  a.counters = reinterpret_cast<unsigned*>(ws + w.counters);
  a.n_counters = w.n_counters;
  a.slots = reinterpret_cast<float*>(ws + w.slots);
  a.dq = dq;
  a.dq16 = dq16;
  a.dk = dk;
  a.dv = dv;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.N = N;
  a.D = D;
  a.causal = causal != 0;
  a.stream = stream;
  a.layout = op.layout;
  a.dtype = op.dtype;
  a.kv_len = op.kv_len;
  a.window = op.window;
  a.alibi = op.alibi_slopes;
  a.seg_start = op.seg_start;
  a.seg_end = op.seg_end;
  a.scale = op.scale;
  a.mask = op.mask;
  a.mask_t = op.mask_t;
  a.mask_heads = op.mask_heads;
  a.drop = op.drop;
  a.drop_t = op.drop_t;
  a.drop_scale = op.drop ? op.drop_scale : 1.f;
  a.bias = op.bias;
  a.bias_sb = op.bias_stride_b;
  a.bias_sh = op.bias_stride_h;
  a.dbias = op.dbias;
  a.Nkv = op.kv_rows;
  a.block_rows = op.block_rows;
  a.block_cols = op.block_cols;
  return to_code(fa::launch_bwd_main(a));
}

// Preprocess + main with dq in the element format.
static int bwd_16(const void* q, const void* k, const void* v, const void* dO, const void* o,
                  const float* lse, void* dq, void* dk, void* dv, void* workspace,
                  size_t workspace_bytes, int B, int Hq, int Hkv, int N, int D, int causal,
                  const fa_options& op, void* stream) {
  int rc = check_opts(op, causal, Hq, N, D, true);
  if (rc == FA_OK) rc = check_shape(B, Hq, Hkv, N, D);
  if (rc == FA_OK) rc = check_kv_rows(op, B, Hq, Hkv, N, D);
  if (rc != FA_OK) return rc;
  if (!workspace || !dq) return FA_ERR_NULL;
  if (workspace_bytes < fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)) return FA_ERR_WORKSPACE;
  rc = bwd_pre(dO, o, lse, workspace, workspace_bytes, B, Hq, N, D, op.layout, op.dtype, stream);
  if (rc != FA_OK) return rc;
  return bwd_main(q, k, v, dO, workspace, workspace_bytes, nullptr, dq, dk, dv, B, Hq, Hkv, N, D,
                  causal, op, stream);
}

int fa_bwd_main(const void* q, const void* k, const void* v, const void* dO, void* workspace,
                size_t workspace_bytes, float* dq, void* dk, void* dv, int B, int Hq, int Hkv,
                int N, int D, int causal, void* stream) {
  if (!dq) return FA_ERR_NULL;
  return bwd_main(q, k, v, dO, workspace, workspace_bytes, dq, nullptr, dk, dv, B, Hq, Hkv, N, D,
                  causal, kDefaultOpts, stream);
}

int fa_bwd_half_dq(const void* q, const void* k, const void* v, const void* dO, const void* o,
                   const float* lse, void* dq, void* dk, void* dv, void* workspace,
                   size_t workspace_bytes, int B, int Hq, int Hkv, int N, int D, int causal,
                   void* stream) {
  return bwd_16(q, k, v, dO, o, lse, dq, dk, dv, workspace, workspace_bytes, B, Hq, Hkv, N, D,
                causal, kDefaultOpts, stream);
}

int fa_bwd_bnhd(const void* q, const void* k, const void* v, const void* dO, const void* o,
                const float* lse, void* dq, void* dk, void* dv, void* workspace,
                size_t workspace_bytes, int B, int Hq, int Hkv, int N, int D, int causal,
                void* stream) {
  fa_options op = kDefaultOpts;
  op.layout = fa::kBNHD;
  return bwd_16(q, k, v, dO, o, lse, dq, dk, dv, workspace, workspace_bytes, B, Hq, Hkv, N, D,
                causal, op, stream);
}

int fa_bwd_ex(const void* q, const void* k, const void* v, const void* dO, const void* o,
              const float* lse, void* dq, void* dk, void* dv, void* workspace,
              size_t workspace_bytes, int B, int Hq, int Hkv, int N, int D, int causal,
              const fa_options* opts, void* stream) {
  return bwd_16(q, k, v, dO, o, lse, dq, dk, dv, workspace, workspace_bytes, B, Hq, Hkv, N, D,
                causal, opts ? *opts : kDefaultOpts, stream);
}

int fa_bwd(const void* q, const void* k, const void* v, const void* dO, const void* o,
           const float* lse, float* dq, void* dk, void* dv, void* workspace,
           size_t workspace_bytes, int B, int Hq, int Hkv, int N, int D, int causal,
           void* stream) {
  const int rc = check_shape(B, Hq, Hkv, N, D);
  if (rc != FA_OK) return rc;
  if (!workspace) return FA_ERR_NULL;
  if (workspace_bytes < fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)) return FA_ERR_WORKSPACE;
  int e = fa_bwd_preprocess(dO, o, lse, workspace, workspace_bytes, B, Hq, N, D, stream);
  if (e != FA_OK) return e;
  return fa_bwd_main(q, k, v, dO, workspace, workspace_bytes, dq, dk, dv, B, Hq, Hkv, N, D,
                     causal, stream);
}

int fa_pack_mask(const uint8_t* dense, int P, int N, uint32_t* bits, uint32_t* bits_t,
                 void* stream) {
  if (N <= 0) return FA_ERR_SEQLEN;
  if (P <= 0) return FA_ERR_BATCH;
  if (!dense || !bits) return FA_ERR_NULL;
  return to_code(fa::launch_pack_mask(dense, P, N, bits, bits_t, stream));
}

int fa_dropout_bits(uint64_t seed, float p, int P, int N, uint32_t* bits, uint32_t* bits_t,
                    void* stream) {
  if (!(p >= 0.f && p < 1.f)) return FA_ERR_DROPOUT;
  if (N <= 0) return FA_ERR_SEQLEN;
  if (P <= 0) return FA_ERR_BATCH;
  if (!bits) return FA_ERR_NULL;
  return to_code(
      fa::launch_dropout_bits(seed, dropout_threshold(p), P, N, false, bits, bits_t, stream));
}

int fa_dropout_bits_causal(uint64_t seed, float p, int P, int N, uint32_t* bits,
                           uint32_t* bits_t, void* stream) {
  if (!(p >= 0.f && p < 1.f)) return FA_ERR_DROPOUT;
  if (N <= 0) return FA_ERR_SEQLEN;
  if (P <= 0) return FA_ERR_BATCH;
  if (!bits) return FA_ERR_NULL;
  return to_code(
      fa::launch_dropout_bits(seed, dropout_threshold(p), P, N, true, bits, bits_t, stream));
}

int fa_pack_blocks(const uint8_t* layout, int layout_b, int layout_h, int B, int Hq, int Hkv,
                   int N, int causal, int* block_rows, int* block_cols, void* stream) {
  if (N <= 0) return FA_ERR_SEQLEN;
  if (Hkv <= 0 || Hq <= 0 || Hq % Hkv != 0) return FA_ERR_HEADS;
  if (B <= 0) return FA_ERR_BATCH;
  if ((layout_b != 1 && layout_b != B) || (layout_h != 1 && layout_h != Hq)) return FA_ERR_BLOCKS;
  if (!layout || !block_rows) return FA_ERR_NULL;
  const int nb = (N + fa::kSparseBlock - 1) / fa::kSparseBlock;
  return to_code(fa::launch_pack_blocks(layout, layout_b, layout_h, B, Hq, Hkv, nb, causal != 0,
                                        block_rows, block_cols, stream));
}

float fa_dropout_scale(float p) {
  if (!(p >= 0.f && p < 1.f)) return 0.f;
  return (float)(65536.0 / (65536.0 - (double)dropout_threshold(p)));
}

int fa_bwd_noalloc(const void* q, const void* k, const void* v, const void* dO, const void* o,
                   const float* lse, float* dq, void* dk, void* dv, int B, int Hq, int Hkv, int N,
                   int D, int causal, void* stream) {
  int rc = check_shape(B, Hq, Hkv, N, D);
  if (rc != FA_OK) return rc;
  // Two (B, Hq, N) fp32 vectors, each 256-byte aligned, must fit.
  const size_t vec = fa::align256((size_t)B * Hq * N * sizeof(float));
  if (2 * vec > kScratchBytes) return FA_ERR_SCRATCH;
  if (!q || !k || !v || !dO || !o || !lse || !dq || !dk || !dv) return FA_ERR_NULL;
  float* ws = nullptr;
  rc = scratch_of_current_device(&ws);
  if (rc != FA_OK) return rc;
  fa::BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.dO = dO;
  a.o = o;
  a.lse = lse;
  // Both vectors are written in full by the preprocess before the main kernel
  // reads them, so nothing in the scratch needs clearing between calls. No
  // counters or slots: the main kernel runs without the causal split.
  a.dvec = ws;
  a.lse2 = ws + vec / sizeof(float);
  a.counters = nullptr;
  a.n_counters = 0;
  a.slots = nullptr;
  a.dq = dq;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.N = N;
  a.D = D;
  a.causal = causal != 0;
  a.stream = stream;
  a.dk = dk;
  a.dv = dv;
  rc = to_code(fa::launch_bwd_preprocess(a));
  if (rc != FA_OK) return rc;
  return to_code(fa::launch_bwd_main(a));
}

}  // extern "C"
