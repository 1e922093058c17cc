// Torch binding `fa_p100_ext`: the drop-in for the reference's pybind module
// (fa_p100_ext.cu:144-147), with the same two functions, argument lists,
// checks, error messages, allocations and return dtypes:
//
//   forward(q, k, v, causal, full_precision) -> [o fp16 (B,Hq,N,D), lse fp32 (B,Hq,N)]
//       fa_p100_ext.cu:53-83
//   backward(q, k, v, dO, o, lse, causal)    -> [dq fp32 (B,Hq,N,D), dk fp16, dv fp16]
//       fa_p100_ext.cu:103-142
//
// and, with no counterpart in the reference, entries used by the autograd
// Function: backward_half_dq (dq as fp16), forward_bnhd / backward_bnhd
// (dense (B, N, H, D) tensors) and forward_dt / backward_dt (fp16 or bf16);
// the last four take bf16 as well as fp16; pack_mask bit-packs a boolean
// mask for their `mask` / `mask_t` arguments and dropout_bits draws the keep
// bits for `drop` / `drop_t`; they also take an fp32 attention `bias` (and
// the backward its gradient buffer `dbias`).
//
// Plain C++ (no device code): every launch goes through the C ABI of
// libfa_mi355x.so (include/fa_mi355x.h). Unlike the reference, which uses the
// legacy default stream without a device guard (flash_fwd.cuh:351,
// flash_bwd.cuh:475-483), launches go to torch's current stream on the
// tensors' device.
#include <torch/extension.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <cmath>
#include <vector>

#include "fa_mi355x.h"

namespace {

void check_in(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
  TORCH_CHECK(t.scalar_type() == at::kHalf, name, " must be fp16");
  TORCH_CHECK(t.dim() == 4, name, " must be (B, H, N, D)");
}

// The entry points added here beside the reference's (forward_dt,
// backward_dt, forward_bnhd, backward_bnhd) also take bf16: q, k, v (and dO,
// o) in one 16-bit format, results in that format.
void check_in16(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
  TORCH_CHECK(t.scalar_type() == at::kHalf || t.scalar_type() == at::kBFloat16, name,
              " must be fp16 or bf16");
  TORCH_CHECK(t.dim() == 4, name, " must be (B, H, N, D)");
}

// Optional key lengths (right padding): int32 (B,) on q's device; nullptr
// when absent.
const int* kv_len_ptr(const c10::optional<at::Tensor>& kv_len, const at::Tensor& q, int B) {
  if (!kv_len.has_value()) return nullptr;
  const at::Tensor& t = *kv_len;
  TORCH_CHECK(t.is_cuda() && t.device() == q.device(), "kv_len must be on q's device");
  TORCH_CHECK(t.scalar_type() == at::kInt, "kv_len must be int32");
  TORCH_CHECK(t.dim() == 1 && t.size(0) == B && t.is_contiguous(), "kv_len must be (B,)");
  return t.data_ptr<int>();
}

int dtype_code(const at::Tensor& q) {
  return q.scalar_type() == at::kBFloat16 ? FA_DTYPE_BF16 : FA_DTYPE_FP16;
}

// Optional ALiBi slopes: fp32 (Hq,) on q's device; nullptr when absent.
const float* alibi_ptr(const c10::optional<at::Tensor>& slopes, const at::Tensor& q, int H) {
  if (!slopes.has_value()) return nullptr;
  const at::Tensor& t = *slopes;
  TORCH_CHECK(t.is_cuda() && t.device() == q.device(), "alibi_slopes must be on q's device");
  TORCH_CHECK(t.scalar_type() == at::kFloat, "alibi_slopes must be fp32");
  TORCH_CHECK(t.dim() == 1 && t.size(0) == H && t.is_contiguous(), "alibi_slopes must be (Hq,)");
  return t.data_ptr<float>();
}

// Optional packed-sequence bounds: int32 (B, N) on q's device; nullptr when absent.
const int* seg_ptr(const c10::optional<at::Tensor>& seg, const at::Tensor& q, int B, int N,
                   const char* name) {
  if (!seg.has_value()) return nullptr;
  const at::Tensor& t = *seg;
  TORCH_CHECK(t.is_cuda() && t.device() == q.device(), name, " must be on q's device");
  TORCH_CHECK(t.scalar_type() == at::kInt, name, " must be int32");
  TORCH_CHECK(t.dim() == 2 && t.size(0) == B && t.size(1) == N && t.is_contiguous(), name,
              " must be (B, N)");
  return t.data_ptr<int>();
}

// Optional bit-packed mask (pack_mask's output): int32 (B, 1 or Hq, N,
// ceil(N/32)) on q's device; nullptr when absent. Sets *heads to dim 1.
const uint32_t* mask_ptr(const c10::optional<at::Tensor>& m, const at::Tensor& q, int B, int H,
                         int N, const char* name, int* heads) {
  if (!m.has_value()) return nullptr;
  const at::Tensor& t = *m;
  TORCH_CHECK(t.is_cuda() && t.device() == q.device(), name, " must be on q's device");
  TORCH_CHECK(t.scalar_type() == at::kInt, name, " must be int32 (packed bits)");
  TORCH_CHECK(t.dim() == 4 && t.size(0) == B && (t.size(1) == 1 || t.size(1) == H) &&
                  t.size(2) == N && t.size(3) == (N + 31) / 32 && t.is_contiguous(),
              name, " must be (B, 1 or Hq, N, ceil(N/32))");
  *heads = (int)t.size(1);
  return reinterpret_cast<const uint32_t*>(t.data_ptr<int>());
}

fa_options make_opts(const at::Tensor& q, int layout, const c10::optional<at::Tensor>& kv_len,
                     int64_t window, const c10::optional<at::Tensor>& alibi,
                     const c10::optional<at::Tensor>& seg_start,
                     const c10::optional<at::Tensor>& seg_end, double scale,
                     const c10::optional<at::Tensor>& mask,
                     const c10::optional<at::Tensor>& mask_t,
                     const c10::optional<at::Tensor>& drop,
                     const c10::optional<at::Tensor>& drop_t, double drop_scale,
                     const c10::optional<at::Tensor>& bias,
                     const c10::optional<at::Tensor>& dbias,
                     const c10::optional<at::Tensor>& block_rows,
                     const c10::optional<at::Tensor>& block_cols, int B, int H, int Hkv, int N) {
  fa_options op{};
  op.dtype = dtype_code(q);
  op.layout = layout;
  op.kv_len = kv_len_ptr(kv_len, q, B);
  op.window = (int)window;
  op.alibi_slopes = alibi_ptr(alibi, q, H);
  op.seg_start = seg_ptr(seg_start, q, B, N, "seg_start");
  op.seg_end = seg_ptr(seg_end, q, B, N, "seg_end");
  op.scale = (float)scale;
  int heads = 0, heads_t = 0;
  op.mask = mask_ptr(mask, q, B, H, N, "mask", &heads);
  op.mask_t = mask_ptr(mask_t, q, B, H, N, "mask_t", &heads_t);
  TORCH_CHECK(!op.mask_t || (op.mask && heads_t == heads), "mask_t must come with a mask of its shape");
  op.mask_heads = heads;
  int dheads = 0, dheads_t = 0;
  op.drop = mask_ptr(drop, q, B, H, N, "drop", &dheads);
  op.drop_t = mask_ptr(drop_t, q, B, H, N, "drop_t", &dheads_t);
  TORCH_CHECK(!op.drop || dheads == H, "drop must hold one plane per query head");
  TORCH_CHECK(!op.drop_t || (op.drop && dheads_t == H), "drop_t must come with drop");
  op.drop_scale = (float)drop_scale;
  if (bias.has_value()) {
    // fp32 (B or 1, Hq or 1, N, N) with dense rows; a dimension of size 1 is
    // shared (stride 0).
    const at::Tensor& t = *bias;
    TORCH_CHECK(t.is_cuda() && t.device() == q.device(), "bias must be on q's device");
    TORCH_CHECK(t.scalar_type() == at::kFloat, "bias must be fp32");
    TORCH_CHECK(t.dim() == 4 && (t.size(0) == B || t.size(0) == 1) &&
                    (t.size(1) == H || t.size(1) == 1) && t.size(2) == N && t.size(3) == N &&
                    t.stride(3) == 1 && t.stride(2) == N,
                "bias must be (B or 1, Hq or 1, N, N) with dense rows");
    op.bias = t.data_ptr<float>();
    op.bias_stride_b = t.size(0) == 1 ? 0 : t.stride(0);
    op.bias_stride_h = t.size(1) == 1 ? 0 : t.stride(1);
  }
  if (dbias.has_value()) {
    const at::Tensor& t = *dbias;
    TORCH_CHECK(t.is_cuda() && t.device() == q.device(), "dbias must be on q's device");
    TORCH_CHECK(t.scalar_type() == at::kFloat && t.dim() == 4 && t.size(0) == B &&
                    t.size(1) == H && t.size(2) == N && t.size(3) == N && t.is_contiguous(),
                "dbias must be fp32 (B, Hq, N, N), contiguous");
    op.dbias = t.data_ptr<float>();
  }
  // Block-sparse lists (pack_blocks): int32 on q's device, of the sizes the
  // shape gives.
  const int64_t nb = (N + FA_SPARSE_BLOCK - 1) / FA_SPARSE_BLOCK;
  auto blocks_ptr = [&](const c10::optional<at::Tensor>& t, int64_t numel, const char* name) {
    if (!t.has_value()) return (const int*)nullptr;
    TORCH_CHECK(t->is_cuda() && t->device() == q.device(), name, " must be on q's device");
    TORCH_CHECK(t->scalar_type() == at::kInt && t->is_contiguous() && t->numel() == numel, name,
                " must be pack_blocks' contiguous int32 list for this shape");
    return (const int*)t->data_ptr<int>();
  };
  op.block_rows = blocks_ptr(block_rows, (int64_t)B * H * nb * (nb + 1), "block_rows");
  op.block_cols =
      blocks_ptr(block_cols, (int64_t)B * Hkv * nb * ((H / Hkv) * nb + 1), "block_cols");
  return op;
}

void check_rc(int rc, const char* what) {
  TORCH_CHECK(rc == FA_OK, what, " failed: ", fa_error_string(rc));
}

void* current_stream(const at::Tensor& t) {
  return (void*)c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

}  // namespace

std::vector<at::Tensor> fa_forward(at::Tensor q, at::Tensor k, at::Tensor v, bool causal,
                                   bool full_precision) {
  check_in(q, "q");
  check_in(k, "k");
  check_in(v, "v");
  q = q.contiguous();
  k = k.contiguous();
  v = v.contiguous();
  const int B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3);
  const int Hkv = k.size(1);
  TORCH_CHECK(D >= 8 && D <= 256 && D % 8 == 0, "head dim must be a multiple of 8 from 8 to 256, got ", D);
  TORCH_CHECK(N > 0, "N must be positive");
  TORCH_CHECK(Hkv > 0 && H % Hkv == 0, "query heads (", H,
              ") must be a multiple of key/value heads (", Hkv, ")");
  TORCH_CHECK(k.sizes() == v.sizes(), "k and v must match");
  TORCH_CHECK(k.size(0) == B && k.size(2) == N && k.size(3) == D,
              "k/v must be (B, Hkv, N, D) matching q's B, N, D");
  TORCH_CHECK(k.device() == q.device() && v.device() == q.device(),
              "q, k and v must be on the same device");

  c10::DeviceGuard guard(q.device());
  auto o = at::empty_like(q);
  auto lse = at::empty({B, H, N}, q.options().dtype(at::kFloat));
  check_rc(fa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr<float>(),
                  B, H, Hkv, N, D, causal ? 1 : 0, full_precision ? 1 : 0, current_stream(q)),
           "fa_fwd");
  return {o, lse};
}

// half_dq: dq comes back as fp16 (the fp32 result rounded to nearest even,
// bit-identical to casting the fp32 dq) for the autograd backward, which
// returns dq in q's dtype (fa_p100.py:45); otherwise fp32 as the reference.
static std::vector<at::Tensor> backward_impl(at::Tensor q, at::Tensor k, at::Tensor v,
                                             at::Tensor dO, at::Tensor o, at::Tensor lse,
                                             bool causal, bool half_dq) {
  check_in(q, "q");
  check_in(dO, "dO");
  q = q.contiguous();
  k = k.contiguous();
  v = v.contiguous();
  dO = dO.contiguous();
  o = o.contiguous();
  lse = lse.contiguous();
  const int B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3);
  const int Hkv = k.size(1);
  TORCH_CHECK(D >= 8 && D <= 256 && D % 8 == 0, "head dim must be a multiple of 8 from 8 to 256, got ", D);
  TORCH_CHECK(N > 0, "N must be positive");
  TORCH_CHECK(Hkv > 0 && H % Hkv == 0, "query heads must be a multiple of kv heads");
  // The reference checks only q and dO here (fa_p100_ext.cu:106); the kernels
  // would read out of bounds on anything else, so the rest is checked too.
  TORCH_CHECK(k.scalar_type() == at::kHalf && v.scalar_type() == at::kHalf &&
                  o.scalar_type() == at::kHalf,
              "k, v and o must be fp16");
  TORCH_CHECK(lse.scalar_type() == at::kFloat, "lse must be fp32");
  TORCH_CHECK(k.sizes() == v.sizes() && k.dim() == 4 && k.size(0) == B && k.size(2) == N &&
                  k.size(3) == D,
              "k/v must be (B, Hkv, N, D) matching q's B, N, D");
  TORCH_CHECK(dO.sizes() == q.sizes() && o.sizes() == q.sizes(), "dO and o must match q");
  TORCH_CHECK(lse.dim() == 3 && lse.size(0) == B && lse.size(1) == H && lse.size(2) == N,
              "lse must be (B, H, N)");

  c10::DeviceGuard guard(q.device());
  auto f32 = q.options().dtype(at::kFloat);
  // Same dtypes as the reference: dq fp32, dk/dv fp16 (fa_p100_ext.cu:118-123).
  auto dq = at::empty({B, H, N, D}, half_dq ? q.options() : f32);
  auto dk = at::empty_like(k);
  auto dv = at::empty_like(k);
  const size_t ws_bytes = fa_bwd_workspace_bytes(B, H, Hkv, N, D);
  auto dvec = at::empty({(int64_t)(ws_bytes / sizeof(float))}, f32);  // rowsum(dO * O)
  if (half_dq)
    check_rc(fa_bwd_half_dq(q.data_ptr(), k.data_ptr(), v.data_ptr(), dO.data_ptr(),
                            o.data_ptr(), lse.data_ptr<float>(), dq.data_ptr(), dk.data_ptr(),
                            dv.data_ptr(), dvec.data_ptr(), ws_bytes, B, H, Hkv, N, D,
                            causal ? 1 : 0, current_stream(q)),
             "fa_bwd_half_dq");
  else
    check_rc(fa_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), dO.data_ptr(), o.data_ptr(),
                    lse.data_ptr<float>(), dq.data_ptr<float>(), dk.data_ptr(), dv.data_ptr(),
                    dvec.data_ptr(), ws_bytes, B, H, Hkv, N, D, causal ? 1 : 0,
                    current_stream(q)),
             "fa_bwd");
  return {dq, dk, dv};
}

std::vector<at::Tensor> fa_backward(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor dO,
                                    at::Tensor o, at::Tensor lse, bool causal) {
  return backward_impl(q, k, v, dO, o, lse, causal, false);
}

std::vector<at::Tensor> fa_backward_half_dq(at::Tensor q, at::Tensor k, at::Tensor v,
                                            at::Tensor dO, at::Tensor o, at::Tensor lse,
                                            bool causal) {
  return backward_impl(q, k, v, dO, o, lse, causal, true);
}

// The (B, N, H, D)-layout pair used by the autograd Function when q, k, v
// arrive as (B, H, N, D) views of (B, N, H, D) storage (what the HF hook
// passes, fa_p100_hf.py:131-140): no copy in, o and the gradients come back
// in the same layout (dq as fp16). Arguments here are the (B, N, H, D)
// tensors themselves; the checks and messages are the reference's, on the
// logical (B, H, N, D) shapes.
static void check_bnhd(const at::Tensor& t, const char* name) {
  check_in16(t, name);
  TORCH_CHECK(t.is_contiguous(), name, " must be dense (B, N, H, D)");
}

std::vector<at::Tensor> fa_forward_bnhd(at::Tensor q, at::Tensor k, at::Tensor v, bool causal,
                                        c10::optional<at::Tensor> kv_len, int64_t window,
    c10::optional<at::Tensor> alibi_slopes,
    c10::optional<at::Tensor> seg_start, c10::optional<at::Tensor> seg_end,
    double scale, c10::optional<at::Tensor> mask, c10::optional<at::Tensor> mask_t,
    c10::optional<at::Tensor> drop, c10::optional<at::Tensor> drop_t, double drop_scale,
    c10::optional<at::Tensor> bias, c10::optional<at::Tensor> dbias,
    c10::optional<at::Tensor> block_rows, c10::optional<at::Tensor> block_cols) {
  check_bnhd(q, "q");
  check_bnhd(k, "k");
  check_bnhd(v, "v");
  const int B = q.size(0), N = q.size(1), H = q.size(2), D = q.size(3);
  const int Hkv = k.size(2);
  TORCH_CHECK(D >= 8 && D <= 256 && D % 8 == 0, "head dim must be a multiple of 8 from 8 to 256, got ", D);
  TORCH_CHECK(N > 0, "N must be positive");
  TORCH_CHECK(Hkv > 0 && H % Hkv == 0, "query heads (", H,
              ") must be a multiple of key/value heads (", Hkv, ")");
  TORCH_CHECK(k.sizes() == v.sizes(), "k and v must match");
  TORCH_CHECK(k.size(0) == B && k.size(1) > 0 && k.size(3) == D,
              "k/v must be (B, Hkv, Nk, D) matching q's B and D");
  TORCH_CHECK(k.device() == q.device() && v.device() == q.device(),
              "q, k and v must be on the same device");
  TORCH_CHECK(k.scalar_type() == q.scalar_type() && v.scalar_type() == q.scalar_type(),
              "q, k and v must have one dtype");
  c10::DeviceGuard guard(q.device());
  auto o = at::empty_like(q);
  auto lse = at::empty({B, H, N}, q.options().dtype(at::kFloat));
  fa_options op =
      make_opts(q, FA_LAYOUT_BNHD, kv_len, window, alibi_slopes, seg_start, seg_end, scale,
                mask, mask_t, drop, drop_t, drop_scale, bias, dbias, block_rows, block_cols,
                B, H, Hkv, N);
  // key rows that differ from the query rows: bottom-right-aligned causal
  op.kv_rows = k.size(1) != N ? (int)k.size(1) : 0;
  check_rc(fa_fwd_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                     lse.data_ptr<float>(), B, H, Hkv, N, D, causal ? 1 : 0, &op,
                     current_stream(q)),
           "fa_fwd_ex");
  return {o, lse};
}

std::vector<at::Tensor> fa_backward_bnhd(at::Tensor q, at::Tensor k, at::Tensor v,
                                         at::Tensor dO, at::Tensor o, at::Tensor lse,
                                         bool causal, c10::optional<at::Tensor> kv_len,
                                         int64_t window, c10::optional<at::Tensor> alibi_slopes,
    c10::optional<at::Tensor> seg_start, c10::optional<at::Tensor> seg_end,
    double scale, c10::optional<at::Tensor> mask, c10::optional<at::Tensor> mask_t,
    c10::optional<at::Tensor> drop, c10::optional<at::Tensor> drop_t, double drop_scale,
    c10::optional<at::Tensor> bias, c10::optional<at::Tensor> dbias,
    c10::optional<at::Tensor> block_rows, c10::optional<at::Tensor> block_cols) {
  for (auto& tn : {std::make_pair(&q, "q"), std::make_pair(&k, "k"), std::make_pair(&v, "v"),
                   std::make_pair(&dO, "dO"), std::make_pair(&o, "o")})
    check_bnhd(*tn.first, tn.second);
  lse = lse.contiguous();
  const int B = q.size(0), N = q.size(1), H = q.size(2), D = q.size(3);
  const int Hkv = k.size(2);
  TORCH_CHECK(D >= 8 && D <= 256 && D % 8 == 0, "head dim must be a multiple of 8 from 8 to 256, got ", D);
  TORCH_CHECK(N > 0, "N must be positive");
  TORCH_CHECK(Hkv > 0 && H % Hkv == 0, "query heads must be a multiple of kv heads");
  TORCH_CHECK(k.sizes() == v.sizes() && k.size(0) == B && k.size(1) > 0 && k.size(3) == D,
              "k/v must be (B, Hkv, Nk, D) matching q's B and D");
  TORCH_CHECK(dO.sizes() == q.sizes() && o.sizes() == q.sizes(), "dO and o must match q");
  TORCH_CHECK(lse.scalar_type() == at::kFloat && lse.dim() == 3 && lse.size(0) == B &&
                  lse.size(1) == H && lse.size(2) == N,
              "lse must be (B, H, N)");
  for (const at::Tensor* t : {&k, &v, &dO, &o})
    TORCH_CHECK(t->scalar_type() == q.scalar_type(), "q, k, v, dO and o must have one dtype");
  c10::DeviceGuard guard(q.device());
  auto dq = at::empty_like(q);  // q's dtype, (B, N, Hq, D)
  auto dk = at::empty_like(k);
  auto dv = at::empty_like(k);
  const size_t ws_bytes = fa_bwd_workspace_bytes(B, H, Hkv, N, D);
  auto ws = at::empty({(int64_t)(ws_bytes / sizeof(float))}, q.options().dtype(at::kFloat));
  fa_options op =
      make_opts(q, FA_LAYOUT_BNHD, kv_len, window, alibi_slopes, seg_start, seg_end, scale,
                mask, mask_t, drop, drop_t, drop_scale, bias, dbias, block_rows, block_cols,
                B, H, Hkv, N);
  // key rows that differ from the query rows: bottom-right-aligned causal
  op.kv_rows = k.size(1) != N ? (int)k.size(1) : 0;
  check_rc(fa_bwd_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(), dO.data_ptr(), o.data_ptr(),
                     lse.data_ptr<float>(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                     ws.data_ptr(), ws_bytes, B, H, Hkv, N, D, causal ? 1 : 0, &op,
                     current_stream(q)),
           "fa_bwd_ex");
  return {dq, dk, dv};
}

// Dense (B, H, N, D) tensors in fp16 or bf16 (one format for all), results in
// that format, dq included, and optional key lengths kv_len (int32 (B,), right
// padding: entry b has keys [0, kv_len[b])), sliding window (causal: row i
// sees keys (i - window, i]; 0 = none), ALiBi slopes (fp32 (Hq,): score
// -slope |i - j|), packed-sequence bounds, a softmax scale and a bit-packed
// mask (pack_mask's bits; the backward needs bits_t as mask_t too). For fp16
// without these, the same kernels as forward and backward_half_dq.
std::vector<at::Tensor> fa_forward_dt(at::Tensor q, at::Tensor k, at::Tensor v, bool causal,
                                      c10::optional<at::Tensor> kv_len, int64_t window,
    c10::optional<at::Tensor> alibi_slopes,
    c10::optional<at::Tensor> seg_start, c10::optional<at::Tensor> seg_end,
    double scale, c10::optional<at::Tensor> mask, c10::optional<at::Tensor> mask_t,
    c10::optional<at::Tensor> drop, c10::optional<at::Tensor> drop_t, double drop_scale,
    c10::optional<at::Tensor> bias, c10::optional<at::Tensor> dbias,
    c10::optional<at::Tensor> block_rows, c10::optional<at::Tensor> block_cols) {
  check_in16(q, "q");
  check_in16(k, "k");
  check_in16(v, "v");
  TORCH_CHECK(k.scalar_type() == q.scalar_type() && v.scalar_type() == q.scalar_type(),
              "q, k and v must have one dtype");
  q = q.contiguous();
  k = k.contiguous();
  v = v.contiguous();
  const int B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3);
  const int Hkv = k.size(1);
  TORCH_CHECK(D >= 8 && D <= 256 && D % 8 == 0, "head dim must be a multiple of 8 from 8 to 256, got ", D);
  TORCH_CHECK(N > 0, "N must be positive");
  TORCH_CHECK(Hkv > 0 && H % Hkv == 0, "query heads (", H,
              ") must be a multiple of key/value heads (", Hkv, ")");
  TORCH_CHECK(k.sizes() == v.sizes(), "k and v must match");
  TORCH_CHECK(k.size(0) == B && k.size(2) > 0 && k.size(3) == D,
              "k/v must be (B, Hkv, Nk, D) matching q's B and D");
  TORCH_CHECK(k.device() == q.device() && v.device() == q.device(),
              "q, k and v must be on the same device");
  c10::DeviceGuard guard(q.device());
  auto o = at::empty_like(q);
  auto lse = at::empty({B, H, N}, q.options().dtype(at::kFloat));
  fa_options op =
      make_opts(q, FA_LAYOUT_BHND, kv_len, window, alibi_slopes, seg_start, seg_end, scale,
                mask, mask_t, drop, drop_t, drop_scale, bias, dbias, block_rows, block_cols,
                B, H, Hkv, N);
  // key rows that differ from the query rows: bottom-right-aligned causal
  op.kv_rows = k.size(2) != N ? (int)k.size(2) : 0;
  check_rc(fa_fwd_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                     lse.data_ptr<float>(), B, H, Hkv, N, D, causal ? 1 : 0, &op,
                     current_stream(q)),
           "fa_fwd_ex");
  return {o, lse};
}

std::vector<at::Tensor> fa_backward_dt(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor dO,
                                       at::Tensor o, at::Tensor lse, bool causal,
                                       c10::optional<at::Tensor> kv_len, int64_t window,
    c10::optional<at::Tensor> alibi_slopes,
    c10::optional<at::Tensor> seg_start, c10::optional<at::Tensor> seg_end,
    double scale, c10::optional<at::Tensor> mask, c10::optional<at::Tensor> mask_t,
    c10::optional<at::Tensor> drop, c10::optional<at::Tensor> drop_t, double drop_scale,
    c10::optional<at::Tensor> bias, c10::optional<at::Tensor> dbias,
    c10::optional<at::Tensor> block_rows, c10::optional<at::Tensor> block_cols) {
  check_in16(q, "q");
  check_in16(dO, "dO");
  q = q.contiguous();
  k = k.contiguous();
  v = v.contiguous();
  dO = dO.contiguous();
  o = o.contiguous();
  lse = lse.contiguous();
  const int B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3);
  const int Hkv = k.size(1);
  TORCH_CHECK(D >= 8 && D <= 256 && D % 8 == 0, "head dim must be a multiple of 8 from 8 to 256, got ", D);
  TORCH_CHECK(N > 0, "N must be positive");
  TORCH_CHECK(Hkv > 0 && H % Hkv == 0, "query heads must be a multiple of kv heads");
  for (const at::Tensor* t : {&k, &v, &dO, &o})
    TORCH_CHECK(t->scalar_type() == q.scalar_type(), "q, k, v, dO and o must have one dtype");
  TORCH_CHECK(lse.scalar_type() == at::kFloat, "lse must be fp32");
  TORCH_CHECK(k.sizes() == v.sizes() && k.dim() == 4 && k.size(0) == B && k.size(2) > 0 &&
                  k.size(3) == D,
              "k/v must be (B, Hkv, Nk, D) matching q's B and D");
  TORCH_CHECK(dO.sizes() == q.sizes() && o.sizes() == q.sizes(), "dO and o must match q");
  TORCH_CHECK(lse.dim() == 3 && lse.size(0) == B && lse.size(1) == H && lse.size(2) == N,
              "lse must be (B, H, N)");
  c10::DeviceGuard guard(q.device());
  auto dq = at::empty_like(q);
  auto dk = at::empty_like(k);
  auto dv = at::empty_like(k);
  const size_t ws_bytes = fa_bwd_workspace_bytes(B, H, Hkv, N, D);
  auto ws = at::empty({(int64_t)(ws_bytes / sizeof(float))}, q.options().dtype(at::kFloat));
  fa_options op =
      make_opts(q, FA_LAYOUT_BHND, kv_len, window, alibi_slopes, seg_start, seg_end, scale,
                mask, mask_t, drop, drop_t, drop_scale, bias, dbias, block_rows, block_cols,
                B, H, Hkv, N);
  // key rows that differ from the query rows: bottom-right-aligned causal
  op.kv_rows = k.size(2) != N ? (int)k.size(2) : 0;
  check_rc(fa_bwd_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(), dO.data_ptr(), o.data_ptr(),
                     lse.data_ptr<float>(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                     ws.data_ptr(), ws_bytes, B, H, Hkv, N, D, causal ? 1 : 0, &op,
                     current_stream(q)),
           "fa_bwd_ex");
  return {dq, dk, dv};
}

// Block layout (Bl, Hl, nb, nb) (bool or uint8; Bl in {1, B}, Hl in {1, Hq};
// nonzero = visible) to the lists the kernels step over (see fa_pack_blocks):
// [block_rows (B, Hq, nb, nb + 1) int32, block_cols (B, Hkv, nb, G*nb + 1)].
std::vector<at::Tensor> fa_pack_blocks_t(at::Tensor layout, int64_t B, int64_t Hq, int64_t Hkv,
                                         int64_t N, bool causal) {
  TORCH_CHECK(layout.is_cuda(), "block layout must be a CUDA tensor");
  TORCH_CHECK(layout.scalar_type() == at::kBool || layout.scalar_type() == at::kByte,
              "block layout must be bool or uint8");
  TORCH_CHECK(B > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && N > 0 && N <= INT32_MAX,
              "B, Hq, Hkv and N must be positive, Hq a multiple of Hkv");
  const int64_t nb = (N + FA_SPARSE_BLOCK - 1) / FA_SPARSE_BLOCK;
  TORCH_CHECK(layout.dim() == 4 && (layout.size(0) == 1 || layout.size(0) == B) &&
                  (layout.size(1) == 1 || layout.size(1) == Hq) && layout.size(2) == nb &&
                  layout.size(3) == nb,
              "block layout must be (B or 1, Hq or 1, nb, nb) with nb = ceil(N / ",
              FA_SPARSE_BLOCK, ") = ", nb);
  layout = layout.contiguous();
  c10::DeviceGuard guard(layout.device());
  auto opts = layout.options().dtype(at::kInt);
  auto rows = at::empty({B, Hq, nb, nb + 1}, opts);
  auto cols = at::empty({B, Hkv, nb, (Hq / Hkv) * nb + 1}, opts);
  check_rc(fa_pack_blocks(reinterpret_cast<const uint8_t*>(layout.data_ptr()),
                          (int)layout.size(0), (int)layout.size(1), (int)B, (int)Hq, (int)Hkv,
                          (int)N, causal ? 1 : 0, rows.data_ptr<int>(), cols.data_ptr<int>(),
                          current_stream(layout)),
           "fa_pack_blocks");
  return {rows, cols};
}

// Dense boolean mask (..., N, N) (nonzero = may attend) to the packed words
// the kernels read: bits (..., N, ceil(N/32)) and, with `transposed`, bits_t
// of the same shape holding the transpose (see fa_pack_mask).
std::vector<at::Tensor> fa_pack_mask_t(at::Tensor dense, bool transposed) {
  TORCH_CHECK(dense.is_cuda(), "mask must be a CUDA tensor");
  TORCH_CHECK(dense.scalar_type() == at::kBool || dense.scalar_type() == at::kByte,
              "mask must be bool or uint8");
  TORCH_CHECK(dense.dim() >= 2 && dense.size(-1) == dense.size(-2) && dense.size(-1) > 0,
              "mask must be (..., N, N)");
  dense = dense.contiguous();
  const int64_t N = dense.size(-1);
  TORCH_CHECK(N <= INT32_MAX, "mask too large");
  const int64_t P = dense.numel() / (N * N);
  TORCH_CHECK(P > 0 && P <= INT32_MAX, "mask must hold at least one plane");
  std::vector<int64_t> shape(dense.sizes().begin(), dense.sizes().end());
  shape.back() = (N + 31) / 32;
  c10::DeviceGuard guard(dense.device());
  auto opts = dense.options().dtype(at::kInt);
  auto bits = at::empty(shape, opts);
  at::Tensor bits_t = transposed ? at::empty(shape, opts) : at::Tensor();
  check_rc(fa_pack_mask(reinterpret_cast<const uint8_t*>(dense.data_ptr()), (int)P, (int)N,
                        reinterpret_cast<uint32_t*>(bits.data_ptr<int>()),
                        transposed ? reinterpret_cast<uint32_t*>(bits_t.data_ptr<int>()) : nullptr,
                        current_stream(dense)),
           "fa_pack_mask");
  if (!transposed) return {bits};
  return {bits, bits_t};
}

// Dropout keep bits for `drop` / `drop_t`: int32 (B, H, N, ceil(N/32)) each on
// the given device, drawn from `seed` with drop probability p (see
// fa_dropout_bits). Without `transposed` only `drop` is drawn (the forward
// reads no other) and the second tensor is undefined (None in Python).
// causal: the bits of keys past each row's diagonal are cleared and not drawn
// (fa_dropout_bits_causal), for causal attention over N keys.
std::vector<at::Tensor> fa_dropout_bits_t(int64_t seed, double p, int64_t B, int64_t H, int64_t N,
                                          int64_t device, bool transposed, bool causal) {
  TORCH_CHECK(p >= 0.0 && p < 1.0, "dropout p must lie in [0, 1), got ", p);
  TORCH_CHECK(B > 0 && H > 0 && N > 0 && B * H <= INT32_MAX && N <= INT32_MAX,
              "dropout bits need positive B, H, N");
  const at::Device dev(at::kCUDA, (c10::DeviceIndex)device);
  c10::DeviceGuard guard(dev);
  auto opts = at::TensorOptions().dtype(at::kInt).device(dev);
  const int64_t W = (N + 31) / 32;
  auto bits = at::empty({B, H, N, W}, opts);
  at::Tensor bits_t;
  if (transposed) bits_t = at::empty({B, H, N, W}, opts);
  check_rc((causal ? fa_dropout_bits_causal : fa_dropout_bits)(
               (uint64_t)seed, (float)p, (int)(B * H), (int)N,
               reinterpret_cast<uint32_t*>(bits.data_ptr<int>()),
               transposed ? reinterpret_cast<uint32_t*>(bits_t.data_ptr<int>()) : nullptr,
               current_stream(bits)),
           causal ? "fa_dropout_bits_causal" : "fa_dropout_bits");
  return {bits, bits_t};
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("dropout_bits", &fa_dropout_bits_t,
        "Dropout keep bits (B, H, N, ceil(N/32)) and their transpose for drop / drop_t",
        py::arg("seed"), py::arg("p"), py::arg("B"), py::arg("H"), py::arg("N"),
        py::arg("device"), py::arg("transposed") = true, py::arg("causal") = false);
  m.def("dropout_scale", [](double p) { return (double)fa_dropout_scale((float)p); },
        "Scale of the kept probabilities for dropout_bits(p): 1 / (1 - the drawn rate)",
        py::arg("p"));
  m.def("pack_blocks", &fa_pack_blocks_t,
        "block-sparse layout (B|1, Hq|1, nb, nb) to the kernels' block lists",
        py::arg("layout"), py::arg("B"), py::arg("Hq"), py::arg("Hkv"), py::arg("N"),
        py::arg("causal"));
  m.def("pack_mask", &fa_pack_mask_t,
        "Bit-packs a dense boolean (..., N, N) mask for the mask / mask_t arguments",
        py::arg("mask"), py::arg("transposed") = true);
  m.def("forward", &fa_forward, "FlashAttention forward (gfx950)");
  m.def("backward", &fa_backward, "FlashAttention backward (gfx950)");
  m.def("backward_half_dq", &fa_backward_half_dq,
        "FlashAttention backward (gfx950), dq as fp16 (used by the autograd Function)");
  m.def("forward_bnhd", &fa_forward_bnhd,
        "FlashAttention forward (gfx950) on dense (B, N, H, D) tensors", py::arg("q"),
        py::arg("k"), py::arg("v"), py::arg("causal"), py::arg("kv_len") = py::none(), py::arg("window") = 0,
        py::arg("alibi_slopes") = py::none(), py::arg("seg_start") = py::none(),
        py::arg("seg_end") = py::none(), py::arg("scale") = 0.0,
        py::arg("mask") = py::none(), py::arg("mask_t") = py::none(),
        py::arg("drop") = py::none(), py::arg("drop_t") = py::none(), py::arg("drop_scale") = 1.0,
        py::arg("bias") = py::none(), py::arg("dbias") = py::none(),
        py::arg("block_rows") = py::none(), py::arg("block_cols") = py::none());
  m.def("backward_bnhd", &fa_backward_bnhd,
        "FlashAttention backward (gfx950) on dense (B, N, H, D) tensors, dq in q's dtype",
        py::arg("q"), py::arg("k"), py::arg("v"), py::arg("dO"), py::arg("o"), py::arg("lse"),
        py::arg("causal"), py::arg("kv_len") = py::none(), py::arg("window") = 0,
        py::arg("alibi_slopes") = py::none(), py::arg("seg_start") = py::none(),
        py::arg("seg_end") = py::none(), py::arg("scale") = 0.0,
        py::arg("mask") = py::none(), py::arg("mask_t") = py::none(),
        py::arg("drop") = py::none(), py::arg("drop_t") = py::none(), py::arg("drop_scale") = 1.0,
        py::arg("bias") = py::none(), py::arg("dbias") = py::none(),
        py::arg("block_rows") = py::none(), py::arg("block_cols") = py::none());
  m.def("forward_dt", &fa_forward_dt,
        "FlashAttention forward (gfx950) on fp16 or bf16 (B, H, N, D) tensors", py::arg("q"),
        py::arg("k"), py::arg("v"), py::arg("causal"), py::arg("kv_len") = py::none(), py::arg("window") = 0,
        py::arg("alibi_slopes") = py::none(), py::arg("seg_start") = py::none(),
        py::arg("seg_end") = py::none(), py::arg("scale") = 0.0,
        py::arg("mask") = py::none(), py::arg("mask_t") = py::none(),
        py::arg("drop") = py::none(), py::arg("drop_t") = py::none(), py::arg("drop_scale") = 1.0,
        py::arg("bias") = py::none(), py::arg("dbias") = py::none(),
        py::arg("block_rows") = py::none(), py::arg("block_cols") = py::none());
  m.def("backward_dt", &fa_backward_dt,
        "FlashAttention backward (gfx950) on fp16 or bf16 (B, H, N, D) tensors, dq in q's dtype",
        py::arg("q"), py::arg("k"), py::arg("v"), py::arg("dO"), py::arg("o"), py::arg("lse"),
        py::arg("causal"), py::arg("kv_len") = py::none(), py::arg("window") = 0,
        py::arg("alibi_slopes") = py::none(), py::arg("seg_start") = py::none(),
        py::arg("seg_end") = py::none(), py::arg("scale") = 0.0,
        py::arg("mask") = py::none(), py::arg("mask_t") = py::none(),
        py::arg("drop") = py::none(), py::arg("drop_t") = py::none(), py::arg("drop_scale") = 1.0,
        py::arg("bias") = py::none(), py::arg("dbias") = py::none(),
        py::arg("block_rows") = py::none(), py::arg("block_cols") = py::none());
}
