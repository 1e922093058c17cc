// Host-side launch descriptors shared by the kernels and the C ABI layer.
// Arguments are validated by the C ABI (fa_capi.hip) before these are called.
#pragma once
#include <hip/hip_runtime.h>

namespace fa {

struct FwdArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int B, Hq, Hkv, N, D;
  bool causal;
  void* stream;
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
};

hipError_t launch_fwd(const FwdArgs& a);
hipError_t launch_bwd_preprocess(const BwdArgs& a);
hipError_t launch_bwd_main(const BwdArgs& a);

}  // namespace fa
