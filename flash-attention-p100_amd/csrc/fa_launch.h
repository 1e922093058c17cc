// Host-side launch descriptors shared by the kernels and the C ABI layer.
// Arguments are validated by the C ABI (fa_capi.hip) before these are called.
#pragma once
#include <hip/hip_runtime.h>

namespace fa {

// Memory layouts of the (B, H, N, D) fp16 tensors: kBHND is dense (B, H, N, D)
// (the reference's layout); kBNHD stores the same logical tensor as dense
// (B, N, H, D), the layout of the projections in a transformer block.
enum Layout : int { kBHND = 0, kBNHD = 1 };

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
};

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
};

hipError_t launch_fwd(const FwdArgs& a);
hipError_t launch_bwd_preprocess(const BwdArgs& a);
hipError_t launch_bwd_main(const BwdArgs& a);

}  // namespace fa
