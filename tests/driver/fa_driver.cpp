// Torch-free driver over the C ABI (test infrastructure): the counterpart of
// the reference's standalone drivers, attention.cu (forward against a CPU
// reference, 4 input regimes), bwd.cu (backward against a float64 analytic
// reference, finite-difference check) and its peak sweep, for this library.
//
//   fa_driver check         GPU forward + backward vs the float64 C oracle
//                           (oracle/attention_ref.c): the reference's 4 input
//                           regimes x D x causal (attention.cu:120-160,
//                           test_fa_p100.py:107-139), plus GQA, ragged N and
//                           split-key-tile shapes, and the general pair's
//                           options (key lengths, window, ALiBi, scale,
//                           packed sequences, mask, dropout, bias) against
//                           the oracle's ora_fwd_ex / ora_bwd_ex. Exit
//                           status 1 on any miss.
//   fa_driver fd            central finite differences of the oracle's loss
//                           against its analytic backward (bwd.cu:136-160,
//                           h = 1e-4, bar 1e-4). CPU only.
//   fa_driver bench [quick] fwd / bwd / fwd+bwd TFLOPS over shapes, FLOPs by
//                           the reference's convention (attention.cu:219,
//                           bwd.cu:246), HIP events around back-to-back calls.
//   fa_driver peak          fp16 MFMA throughput probe: independent
//                           v_mfma_f32_32x32x16_f16 chains on every SIMD, the
//                           measured ceiling for the roofline (the reference's
//                           half2 peak sweep measured its SIMT ceiling).
//   fa_driver mix           the same products as one dependent chain per wave
//                           at two waves per SIMD, each followed by the
//                           softmax's kind of VALU work (fp32 FMAs,
//                           v_exp_f32), and the VALU work alone: cycles per
//                           product per SIMD, what the kernels' instruction
//                           mix allows at best.
//   fa_driver lds           LDS read throughput per CU of the kernels' operand
//                           reads (16-byte and transpose reads of padded and
//                           swizzled D = 128 tiles, through fa_device.h's
//                           layout helpers) at two waves per SIMD.
//   fa_driver dqcost        the dQ traffic a backward without the dQ pass
//                           would carry (the reference's design,
//                           flash_bwd.cuh:434-443, accumulates dQ across key
//                           tiles): one 64 x D fp32 partial per (key tile,
//                           query step) of the causal C3 shape, sent as
//                           global fp32 atomics into dQ, or stored to a
//                           workspace for a later reduction; no compute.
//                           Timed beside the library's own backward.
//
// Inputs come from a fixed-seed splitmix64 + Box-Muller generator, rounded to
// fp16; the oracle sees exactly those fp16 values.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "../../flash-attention-p100_amd/csrc/fa_device.h"
#include "../../include/fa_mi355x.h"
#include "../../oracle/attention_ref.h"

namespace {

#define HIP_OK(x)                                                                  \
  do {                                                                             \
    hipError_t e_ = (x);                                                           \
    if (e_ != hipSuccess) {                                                        \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x,               \
                   hipGetErrorString(e_));                                         \
      std::exit(2);                                                                \
    }                                                                              \
  } while (0)
#define FA_OK_(x)                                                                  \
  do {                                                                             \
    int rc_ = (x);                                                                 \
    if (rc_ != 0) {                                                                \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x,               \
                   fa_error_string(rc_));                                          \
      std::exit(2);                                                                \
    }                                                                              \
  } while (0)

// Bars (BASELINE): forward max-abs <= 4e-3, LSE max-abs <= 1e-3, gradients
// relative L2 <= 1e-2; the reference's max|err|/RMS(ref) < 6e-2 on all
// (test_fa_p100.py:24, 35-37).
constexpr double kFwdMaxAbs = 4e-3, kLseMaxAbs = 1e-3, kGradRelL2 = 1e-2, kRefRel = 6e-2;

struct Rng {
  uint64_t s;
  uint64_t next() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  double uniform() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
  double normal() {
    const double u = uniform(), v = uniform();
    return std::sqrt(-2.0 * std::log(u)) * std::cos(6.283185307179586 * v);
  }
};

struct Shape {
  int B, Hq, Hkv, N, D, causal;
  size_t nq() const { return (size_t)B * Hq * N * D; }
  size_t nk() const { return (size_t)B * Hkv * N * D; }
  size_t nl() const { return (size_t)B * Hq * N; }
  double fwd_flops() const { return 4.0 * B * Hq * (double)N * N * D / (causal ? 2.0 : 1.0); }
};

// fp16 values and the same values as float64.
struct Host16 {
  std::vector<_Float16> h;
  std::vector<double> d;
  void fill(size_t n, Rng& r, double scale) {
    h.resize(n);
    d.resize(n);
    for (size_t i = 0; i < n; ++i) {
      h[i] = (_Float16)(r.normal() * scale);
      d[i] = (double)h[i];
    }
  }
};

template <class T>
T* dalloc(size_t n) {
  void* p = nullptr;
  HIP_OK(hipMalloc(&p, n * sizeof(T) + 256));
  return static_cast<T*>(p);
}

double max_abs(const std::vector<double>& a, const std::vector<double>& b) {
  double m = 0;
  for (size_t i = 0; i < a.size(); ++i) m = std::fmax(m, std::fabs(a[i] - b[i]));
  return m;
}
double rel_l2(const std::vector<double>& a, const std::vector<double>& ref) {
  double num = 0, den = 0;
  for (size_t i = 0; i < a.size(); ++i) {
    num += (a[i] - ref[i]) * (a[i] - ref[i]);
    den += ref[i] * ref[i];
  }
  return std::sqrt(num / (den > 0 ? den : 1e-300));
}
double rel_max_rms(const std::vector<double>& a, const std::vector<double>& ref) {
  double ss = 0;
  for (double x : ref) ss += x * x;
  const double rms = std::sqrt(ss / (double)ref.size());
  return max_abs(a, ref) / (rms > 0 ? rms : 1e-300);
}

// One forward + backward on the GPU through the C ABI; outputs as float64.
struct GpuResult {
  std::vector<double> o, lse, dq, dk, dv;
};
GpuResult run_gpu(const Shape& s, const Host16& q, const Host16& k, const Host16& v,
                  const Host16& g) {
  _Float16 *dq_in = dalloc<_Float16>(s.nq()), *dk_in = dalloc<_Float16>(s.nk()),
           *dv_in = dalloc<_Float16>(s.nk()), *dgo = dalloc<_Float16>(s.nq()),
           *dout = dalloc<_Float16>(s.nq()), *ddk = dalloc<_Float16>(s.nk()),
           *ddv = dalloc<_Float16>(s.nk());
  float *dlse = dalloc<float>(s.nl()), *ddq = dalloc<float>(s.nq());
  HIP_OK(hipMemcpy(dq_in, q.h.data(), s.nq() * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dk_in, k.h.data(), s.nk() * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dv_in, v.h.data(), s.nk() * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dgo, g.h.data(), s.nq() * 2, hipMemcpyHostToDevice));
  const size_t ws_bytes = fa_bwd_workspace_bytes(s.B, s.Hq, s.Hkv, s.N, s.D);
  char* ws = dalloc<char>(ws_bytes);
  FA_OK_(fa_fwd(dq_in, dk_in, dv_in, dout, dlse, s.B, s.Hq, s.Hkv, s.N, s.D, s.causal, 0,
                nullptr));
  FA_OK_(fa_bwd(dq_in, dk_in, dv_in, dgo, dout, dlse, ddq, ddk, ddv, ws, ws_bytes, s.B, s.Hq,
                s.Hkv, s.N, s.D, s.causal, nullptr));
  HIP_OK(hipDeviceSynchronize());
  std::vector<_Float16> h16(s.nq());
  std::vector<float> h32(s.nq());
  GpuResult r;
  auto to_d = [](const auto& src, size_t n) {
    std::vector<double> out(n);
    for (size_t i = 0; i < n; ++i) out[i] = (double)src[i];
    return out;
  };
  HIP_OK(hipMemcpy(h16.data(), dout, s.nq() * 2, hipMemcpyDeviceToHost));
  r.o = to_d(h16, s.nq());
  HIP_OK(hipMemcpy(h32.data(), dlse, s.nl() * 4, hipMemcpyDeviceToHost));
  r.lse = to_d(h32, s.nl());
  HIP_OK(hipMemcpy(h32.data(), ddq, s.nq() * 4, hipMemcpyDeviceToHost));
  r.dq = to_d(h32, s.nq());
  HIP_OK(hipMemcpy(h16.data(), ddk, s.nk() * 2, hipMemcpyDeviceToHost));
  r.dk = to_d(h16, s.nk());
  HIP_OK(hipMemcpy(h16.data(), ddv, s.nk() * 2, hipMemcpyDeviceToHost));
  r.dv = to_d(h16, s.nk());
  for (void* p : {(void*)dq_in, (void*)dk_in, (void*)dv_in, (void*)dgo, (void*)dout,
                  (void*)ddk, (void*)ddv, (void*)dlse, (void*)ddq, (void*)ws})
    HIP_OK(hipFree(p));
  return r;
}

bool check_case(const char* name, const Shape& s, double scale_qk, uint64_t seed) {
  Rng r{seed};
  Host16 q, k, v, g;
  q.fill(s.nq(), r, scale_qk);
  k.fill(s.nk(), r, scale_qk);
  v.fill(s.nk(), r, 1.0);
  g.fill(s.nq(), r, 1.0);
  const GpuResult got = run_gpu(s, q, k, v, g);
  std::vector<double> o(s.nq()), lse(s.nl()), dq(s.nq()), dk(s.nk()), dv(s.nk());
  ora_fwd(q.d.data(), k.d.data(), v.d.data(), o.data(), lse.data(), s.B, s.Hq, s.Hkv, s.N, s.D,
          s.causal);
  ora_bwd(q.d.data(), k.d.data(), v.d.data(), g.d.data(), dq.data(), dk.data(), dv.data(), s.B,
          s.Hq, s.Hkv, s.N, s.D, s.causal);
  const double fo = max_abs(got.o, o), fr = rel_max_rms(got.o, o), fl = max_abs(got.lse, lse);
  // A gradient that is exactly zero in float64 (N = 1: softmax over one key
  // is constant, so dQ = dK = 0) has no relative error: it must be ~0.
  auto grad_ok = [](const std::vector<double>& got, const std::vector<double>& ref, double& l2) {
    bool zero = true;
    for (double x : ref) zero &= x == 0.0;
    if (zero) {
      l2 = max_abs(got, ref);
      return l2 <= 1e-6;
    }
    l2 = rel_l2(got, ref);
    return l2 <= kGradRelL2 && rel_max_rms(got, ref) < kRefRel;
  };
  double q2, k2, v2;
  const bool gq = grad_ok(got.dq, dq, q2), gk = grad_ok(got.dk, dk, k2), gv = grad_ok(got.dv, dv, v2);
  const bool ok = fo <= kFwdMaxAbs && fr < kRefRel && fl <= kLseMaxAbs && gq && gk && gv;
  std::printf("%-22s B%d Hq%-2d Hkv%-2d N%-5d D%-3d %s | o %.1e (%.1e) lse %.1e | dQ %.1e dK %.1e"
              " dV %.1e | %s\n",
              name, s.B, s.Hq, s.Hkv, s.N, s.D, s.causal ? "causal" : "dense ", fo, fr, fl, q2,
              k2, v2, ok ? "ok" : "FAIL");
  std::fflush(stdout);
  return ok;
}

// The C ABI's options (fa_fwd_ex / fa_bwd_ex) against the C oracle's
// ora_fwd_ex / ora_bwd_ex on the same options: key lengths, a window, ALiBi,
// a scale, packed sequences, a mask (packed on the GPU by fa_pack_mask from
// the dense bytes the oracle reads), dropout (bits drawn on the GPU by
// fa_dropout_bits, first checked bit for bit in both layouts against the C
// draw ora_dropout_keep) and a bias with its gradient. The backward's
// reference takes the GPU's saved o and lse, as the kernels do.
enum OptBits { kOptKvLen = 1, kOptWindow = 2, kOptAlibi = 4, kOptScale = 8, kOptSegs = 16,
               kOptMask1 = 32, kOptMaskH = 64, kOptDrop = 128, kOptBias = 256 };

template <class T>
T* dcopy(const std::vector<T>& h) {
  T* p = dalloc<T>(h.size());
  HIP_OK(hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
  return p;
}
template <class T>
std::vector<T> hcopy(const T* p, size_t n) {
  std::vector<T> h(n);
  HIP_OK(hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost));
  return h;
}

// Bit j % 32 of words[(p * N + i) * W + j / 32] == keep[(p * N + i) * N + j]
// (and the transposed words with i and j swapped) over P planes.
bool bits_match(const std::vector<uint32_t>& words, const std::vector<uint32_t>& words_t,
                const std::vector<unsigned char>& keep, int P, int N) {
  const int W = (N + 31) / 32;
  for (int pl = 0; pl < P; ++pl)
    for (int i = 0; i < N; ++i)
      for (int j = 0; j < N; ++j) {
        const bool k = keep[((size_t)pl * N + i) * N + j] != 0;
        const bool a = (words[((size_t)pl * N + i) * W + j / 32] >> (j % 32)) & 1u;
        const bool b = (words_t[((size_t)pl * N + j) * W + i / 32] >> (i % 32)) & 1u;
        if (a != k || b != k) return false;
      }
  return true;
}

bool check_options_case(const char* name, const Shape& s, int opts, uint64_t seed) {
  Rng r{seed};
  Host16 q, k, v, g;
  q.fill(s.nq(), r, 1.0);
  k.fill(s.nk(), r, 1.0);
  v.fill(s.nk(), r, 1.0);
  g.fill(s.nq(), r, 1.0);
  const int B = s.B, Hq = s.Hq, N = s.N, W = (N + 31) / 32;
  const size_t plane_nn = (size_t)N * N;
  fa_options fo{};
  ora_opts oo{};
  std::vector<void*> owned;  // device buffers of this case
  std::vector<int> lens, s0, s1;
  std::vector<float> slopes_f, bias_f;
  std::vector<double> slopes_d, bias_d;
  std::vector<unsigned char> mask, keep;
  bool bits_ok = true;
  if (opts & kOptKvLen) {
    for (int b = 0; b < B; ++b) lens.push_back(1 + (int)(r.next() % (uint64_t)N));
    int* d = dcopy(lens);
    owned.push_back(d);
    fo.kv_len = d;
    oo.kv_len = lens.data();
  }
  if (opts & kOptWindow) fo.window = oo.window = 1 + (int)(r.next() % (uint64_t)N);
  if (opts & kOptAlibi) {
    for (int h = 0; h < Hq; ++h) slopes_f.push_back((float)(0.02 + 0.4 * r.uniform()));
    for (float x : slopes_f) slopes_d.push_back(x);
    float* d = dcopy(slopes_f);
    owned.push_back(d);
    fo.alibi_slopes = d;
    oo.alibi = slopes_d.data();
  }
  if (opts & kOptScale) {
    fo.scale = 0.17f;
    oo.scale = (double)fo.scale;
  }
  if (opts & kOptSegs) {  // up to four sequences per entry, random lengths
    s0.resize((size_t)B * N);
    s1.resize((size_t)B * N);
    for (int b = 0; b < B; ++b) {
      int i = 0;
      while (i < N) {
        const int len = 1 + (int)(r.next() % (uint64_t)(N / 4 + 1));
        const int e = std::min(N, i + len);
        for (int t = i; t < e; ++t) {
          s0[(size_t)b * N + t] = i;
          s1[(size_t)b * N + t] = e;
        }
        i = e;
      }
    }
    int *d0 = dcopy(s0), *d1 = dcopy(s1);
    owned.push_back(d0);
    owned.push_back(d1);
    fo.seg_start = d0;
    fo.seg_end = d1;
    oo.seg_start = s0.data();
    oo.seg_end = s1.data();
  }
  if (opts & (kOptMask1 | kOptMaskH)) {
    const int mh = (opts & kOptMaskH) ? Hq : 1;
    mask.resize((size_t)B * mh * plane_nn);
    for (auto& x : mask) x = r.uniform() < 0.8;
    for (int j = 0; j < N; ++j) mask[(size_t)2 * N + j] = 0;  // row 2 of plane 0 sees nothing
    unsigned char* dm = dcopy(mask);
    uint32_t *bits = dalloc<uint32_t>((size_t)B * mh * N * W),
             *bits_t = dalloc<uint32_t>((size_t)B * mh * N * W);
    owned.insert(owned.end(), {dm, bits, bits_t});
    FA_OK_(fa_pack_mask(dm, B * mh, N, bits, bits_t, nullptr));
    fo.mask = bits;
    fo.mask_t = bits_t;
    fo.mask_heads = mh;
    oo.mask = mask.data();
    oo.mask_heads = mh;
  }
  if (opts & kOptDrop) {
    const float p = 0.2f;
    const unsigned long long dseed = r.next();
    const int P = B * Hq;
    uint32_t *bits = dalloc<uint32_t>((size_t)P * N * W), *bits_t = dalloc<uint32_t>((size_t)P * N * W);
    owned.push_back(bits);
    owned.push_back(bits_t);
    FA_OK_(fa_dropout_bits(dseed, p, P, N, bits, bits_t, nullptr));
    keep.resize((size_t)P * plane_nn);
    ora_dropout_keep(dseed, ora_dropout_threshold(p), P, N, keep.data());
    bits_ok = bits_match(hcopy(bits, (size_t)P * N * W), hcopy(bits_t, (size_t)P * N * W), keep,
                         P, N);
    fo.drop = bits;
    fo.drop_t = bits_t;
    fo.drop_scale = fa_dropout_scale(p);
    oo.keep = keep.data();
    oo.drop_scale = 65536.0 / (65536.0 - ora_dropout_threshold(p));
  }
  float* dbias = nullptr;
  if (opts & kOptBias) {
    bias_f.resize((size_t)B * Hq * plane_nn);
    for (auto& x : bias_f) x = (float)r.normal();
    for (float x : bias_f) bias_d.push_back(x);
    float* d = dcopy(bias_f);
    dbias = dalloc<float>(bias_f.size());
    HIP_OK(hipMemset(dbias, 0, bias_f.size() * sizeof(float)));
    owned.push_back(d);
    owned.push_back(dbias);
    fo.bias = d;
    fo.bias_stride_b = (long long)Hq * plane_nn;
    fo.bias_stride_h = (long long)plane_nn;
    fo.dbias = dbias;
    oo.bias = bias_d.data();
  }
  // GPU forward + backward through the general pair.
  _Float16 *dq_in = dcopy(q.h), *dk_in = dcopy(k.h), *dv_in = dcopy(v.h), *dgo = dcopy(g.h);
  _Float16 *dout = dalloc<_Float16>(s.nq()), *ddq = dalloc<_Float16>(s.nq()),
           *ddk = dalloc<_Float16>(s.nk()), *ddv = dalloc<_Float16>(s.nk());
  float* dlse = dalloc<float>(s.nl());
  const size_t ws_bytes = fa_bwd_workspace_bytes(B, Hq, s.Hkv, N, s.D);
  char* ws = dalloc<char>(ws_bytes);
  owned.insert(owned.end(), {dq_in, dk_in, dv_in, dgo, dout, ddq, ddk, ddv, dlse, ws});
  FA_OK_(fa_fwd_ex(dq_in, dk_in, dv_in, dout, dlse, B, Hq, s.Hkv, N, s.D, s.causal, &fo,
                   nullptr));
  FA_OK_(fa_bwd_ex(dq_in, dk_in, dv_in, dgo, dout, dlse, ddq, ddk, ddv, ws, ws_bytes, B, Hq,
                   s.Hkv, N, s.D, s.causal, &fo, nullptr));
  HIP_OK(hipDeviceSynchronize());
  auto to_d = [](const auto& src) {
    std::vector<double> out(src.size());
    for (size_t i = 0; i < src.size(); ++i) out[i] = (double)src[i];
    return out;
  };
  const std::vector<double> go = to_d(hcopy(dout, s.nq())), glse = to_d(hcopy(dlse, s.nl())),
                            gdq = to_d(hcopy(ddq, s.nq())), gdk = to_d(hcopy(ddk, s.nk())),
                            gdv = to_d(hcopy(ddv, s.nk()));
  std::vector<double> gdb;
  if (dbias) gdb = to_d(hcopy(dbias, bias_f.size()));
  for (void* p : owned) HIP_OK(hipFree(p));

  // The oracle: forward, then the backward from the GPU's saved o and lse.
  std::vector<double> o(s.nq()), lse(s.nl()), dq(s.nq()), dk(s.nk()), dv(s.nk()), db;
  ora_fwd_ex(q.d.data(), k.d.data(), v.d.data(), o.data(), lse.data(), B, Hq, s.Hkv, N, s.D,
             s.causal, &oo);
  oo.o = go.data();
  oo.lse = glse.data();
  if (dbias) {
    db.resize(bias_f.size());
    oo.dbias = db.data();
  }
  ora_bwd_ex(q.d.data(), k.d.data(), v.d.data(), g.d.data(), dq.data(), dk.data(), dv.data(), B,
             Hq, s.Hkv, N, s.D, s.causal, &oo);

  const double zs = (opts & kOptDrop) ? oo.drop_scale : 1.0;
  const double fo_abs = max_abs(go, o), fo_rel = rel_max_rms(go, o);
  double fl = 0;
  bool lse_ok = true;
  for (size_t i = 0; i < lse.size(); ++i) {
    if (std::isinf(lse[i])) {
      lse_ok &= std::isinf(glse[i]);
      continue;
    }
    fl = std::fmax(fl, std::fabs(glse[i] - lse[i]));
  }
  auto grad_ok = [](const std::vector<double>& got, const std::vector<double>& ref, double& l2) {
    bool zero = true;
    for (double x : ref) zero &= x == 0.0;
    if (zero) {  // e.g. every row left with one key: dS cancels exactly in float64
      l2 = max_abs(got, ref);
      return l2 <= 1e-4;
    }
    l2 = rel_l2(got, ref);
    return l2 <= kGradRelL2 && rel_max_rms(got, ref) < kRefRel;
  };
  double q2, k2, v2, b2 = 0;
  const bool gq = grad_ok(gdq, dq, q2), gk = grad_ok(gdk, dk, k2), gv = grad_ok(gdv, dv, v2);
  const bool gb = !dbias || grad_ok(gdb, db, b2);
  const bool ok = bits_ok && fo_abs <= kFwdMaxAbs * zs && fo_rel < kRefRel && lse_ok &&
                  fl <= kLseMaxAbs && gq && gk && gv && gb;
  std::printf("%-22s B%d Hq%-2d Hkv%-2d N%-5d D%-3d %s | o %.1e (%.1e) lse %.1e | dQ %.1e dK %.1e"
              " dV %.1e dbias %.1e%s | %s\n",
              name, B, Hq, s.Hkv, N, s.D, s.causal ? "causal" : "dense ", fo_abs, fo_rel, fl, q2,
              k2, v2, b2, bits_ok ? "" : " | dropout bits differ", ok ? "ok" : "FAIL");
  std::fflush(stdout);
  return ok;
}

int cmd_check() {
  bool ok = true;
  struct Regime {
    const char* name;
    double scale;
  } regimes[] = {{"1 N(0,1)", 1.0}, {"2 large x10", 10.0}, {"3 near-uniform", 0.05},
                 {"4 near-one-hot", 3.0}};
  uint64_t seed = 1;
  for (const Regime& g : regimes)
    for (int D : {64, 128})
      for (int causal : {0, 1}) ok &= check_case(g.name, {1, 4, 4, 256, D, causal}, g.scale, seed++);
  ok &= check_case("GQA ragged", {2, 8, 2, 333, 128, 1}, 1.0, seed++);
  ok &= check_case("GQA ragged", {2, 8, 2, 333, 128, 0}, 1.0, seed++);
  ok &= check_case("MQA split tiles", {1, 4, 1, 1000, 64, 1}, 1.0, seed++);
  ok &= check_case("MHA split tiles", {1, 2, 2, 1536, 128, 1}, 1.0, seed++);
  ok &= check_case("N=1", {1, 2, 1, 1, 64, 1}, 1.0, seed++);
  // The options of the general pair (fa_fwd_ex / fa_bwd_ex).
  ok &= check_options_case("kv_len+window+alibi", {2, 4, 2, 300, 64, 1},
                           kOptKvLen | kOptWindow | kOptAlibi, seed++);
  ok &= check_options_case("scale+segments", {2, 4, 2, 257, 128, 0}, kOptScale | kOptSegs, seed++);
  ok &= check_options_case("shared mask", {1, 4, 2, 333, 80, 1}, kOptMask1, seed++);
  ok &= check_options_case("per-head mask+dropout", {2, 4, 4, 200, 64, 0}, kOptMaskH | kOptDrop,
                           seed++);
  ok &= check_options_case("dropout", {1, 8, 2, 512, 128, 1}, kOptDrop, seed++);
  ok &= check_options_case("bias", {2, 4, 2, 300, 128, 1}, kOptBias, seed++);
  ok &= check_options_case("every option", {2, 4, 2, 301, 64, 1},
                           kOptKvLen | kOptWindow | kOptAlibi | kOptScale | kOptSegs | kOptMaskH |
                               kOptDrop | kOptBias,
                           seed++);
  std::printf("check: %s\n", ok ? "all ok" : "FAILED");
  return ok ? 0 : 1;
}

int cmd_fd() {
  // The reference's method (bwd.cu:136-160): central differences of the loss
  // sum(dO * O) in float64 with h = 1e-4 against the analytic gradient.
  const double h = 1e-4, bar = 1e-4;
  bool ok = true;
  const Shape shapes[] = {{1, 2, 1, 17, 64, 1}, {1, 2, 2, 9, 128, 0}, {2, 4, 2, 13, 64, 1}};
  uint64_t seed = 100;
  for (const Shape& s : shapes) {
    Rng r{seed++};
    std::vector<double> q(s.nq()), k(s.nk()), v(s.nk()), g(s.nq());
    for (auto* t : {&q, &k, &v, &g})
      for (double& x : *t) x = r.normal();
    std::vector<double> dq(s.nq()), dk(s.nk()), dv(s.nk());
    ora_bwd(q.data(), k.data(), v.data(), g.data(), dq.data(), dk.data(), dv.data(), s.B, s.Hq,
            s.Hkv, s.N, s.D, s.causal);
    double worst = 0;
    std::vector<double>* ins[] = {&q, &k, &v};
    const std::vector<double>* grads[] = {&dq, &dk, &dv};
    for (int t = 0; t < 3; ++t)
      for (int n = 0; n < 24; ++n) {
        std::vector<double>& x = *ins[t];
        const size_t i = r.next() % x.size();
        const double x0 = x[i];
        x[i] = x0 + h;
        const double lp = ora_loss(q.data(), k.data(), v.data(), g.data(), s.B, s.Hq, s.Hkv, s.N,
                                   s.D, s.causal);
        x[i] = x0 - h;
        const double lm = ora_loss(q.data(), k.data(), v.data(), g.data(), s.B, s.Hq, s.Hkv, s.N,
                                   s.D, s.causal);
        x[i] = x0;
        worst = std::fmax(worst, std::fabs((lp - lm) / (2 * h) - (*grads[t])[i]));
      }
    const bool pass = worst < bar;
    ok &= pass;
    std::printf("fd B%d Hq%d Hkv%d N%d D%d %s: max |fd - analytic| %.2e %s\n", s.B, s.Hq, s.Hkv,
                s.N, s.D, s.causal ? "causal" : "dense", worst, pass ? "ok" : "FAIL");
  }
  return ok ? 0 : 1;
}

int cmd_bench(bool quick) {
  std::vector<std::pair<const char*, Shape>> shapes = {
      {"C3 headline", {1, 8, 8, 4096, 128, 1}}};
  if (!quick) {
    shapes.insert(shapes.end(), {{"C2", {1, 16, 16, 2048, 64, 1}},
                                 {"C4 GQA ragged", {2, 32, 8, 3001, 128, 0}},
                                 {"C5 layer", {1, 16, 8, 8192, 128, 1}},
                                 {"N=1024", {4, 16, 16, 1024, 128, 1}},
                                 {"N=16384", {1, 8, 8, 16384, 128, 1}},
                                 {"N=4096 D=64", {1, 16, 16, 4096, 64, 1}},
                                 {"N=4096 dense", {1, 8, 8, 4096, 128, 0}}});
  }
  std::printf("%-14s %-28s %9s %9s %9s %8s %8s %8s\n", "shape", "(B,Hq,Hkv,N,D,causal)",
              "fwd ms", "bwd ms", "step ms", "fwd TF", "bwd TF", "step TF");
  for (const auto& entry : shapes) {
    const char* name = entry.first;
    const Shape s = entry.second;
    Rng r{7};
    Host16 q, k, v, g;
    q.fill(s.nq(), r, 1.0);
    k.fill(s.nk(), r, 1.0);
    v.fill(s.nk(), r, 1.0);
    g.fill(s.nq(), r, 1.0);
    _Float16 *dq_in = dalloc<_Float16>(s.nq()), *dk_in = dalloc<_Float16>(s.nk()),
             *dv_in = dalloc<_Float16>(s.nk()), *dgo = dalloc<_Float16>(s.nq()),
             *dout = dalloc<_Float16>(s.nq()), *ddk = dalloc<_Float16>(s.nk()),
             *ddv = dalloc<_Float16>(s.nk());
    float *dlse = dalloc<float>(s.nl()), *ddq = dalloc<float>(s.nq());
    HIP_OK(hipMemcpy(dq_in, q.h.data(), s.nq() * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dk_in, k.h.data(), s.nk() * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dv_in, v.h.data(), s.nk() * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dgo, g.h.data(), s.nq() * 2, hipMemcpyHostToDevice));
    const size_t ws_bytes = fa_bwd_workspace_bytes(s.B, s.Hq, s.Hkv, s.N, s.D);
    char* ws = dalloc<char>(ws_bytes);
    auto fwd = [&] {
      FA_OK_(fa_fwd(dq_in, dk_in, dv_in, dout, dlse, s.B, s.Hq, s.Hkv, s.N, s.D, s.causal, 0,
                    nullptr));
    };
    auto bwd = [&] {
      FA_OK_(fa_bwd(dq_in, dk_in, dv_in, dgo, dout, dlse, ddq, ddk, ddv, ws, ws_bytes, s.B, s.Hq,
                    s.Hkv, s.N, s.D, s.causal, nullptr));
    };
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    const int reps = s.fwd_flops() > 2e11 ? 10 : 50;
    auto timed = [&](auto&& fn) {
      for (int i = 0; i < 5; ++i) fn();
      HIP_OK(hipEventRecord(e0, nullptr));
      for (int i = 0; i < reps; ++i) fn();
      HIP_OK(hipEventRecord(e1, nullptr));
      HIP_OK(hipEventSynchronize(e1));
      float ms = 0;
      HIP_OK(hipEventElapsedTime(&ms, e0, e1));
      return (double)ms / reps;
    };
    const double tf = timed(fwd), tb = timed(bwd), ts = timed([&] { fwd(); bwd(); });
    const double ff = s.fwd_flops(), fb = 2.5 * ff;
    char dims[64];
    std::snprintf(dims, sizeof dims, "(%d,%d,%d,%d,%d,%d)", s.B, s.Hq, s.Hkv, s.N, s.D, s.causal);
    std::printf("%-14s %-28s %9.4f %9.4f %9.4f %8.1f %8.1f %8.1f\n", name, dims, tf, tb, ts,
                ff / tf / 1e9, fb / tb / 1e9, (ff + fb) / ts / 1e9);
    std::fflush(stdout);
    HIP_OK(hipEventDestroy(e0));
    HIP_OK(hipEventDestroy(e1));
    for (void* p : {(void*)dq_in, (void*)dk_in, (void*)dv_in, (void*)dgo, (void*)dout,
                    (void*)ddk, (void*)ddv, (void*)dlse, (void*)ddq, (void*)ws})
      HIP_OK(hipFree(p));
  }
  return 0;
}

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));

// Four independent accumulator chains per wave; every iteration issues four
// 32x32x16 fp16 MFMAs (4 x 32768 flops).
__global__ __launch_bounds__(256) void mfma_peak_kernel(float* out, int iters) {
  const int t = threadIdx.x;
  half8_t a, b;
  for (int e = 0; e < 8; ++e) {
    a[e] = (_Float16)(((t + e) & 7) * 0.001f);
    b[e] = (_Float16)(((t * 3 + e) & 7) * 0.001f);
  }
  floatx16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int i = 0; i < iters; ++i) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
  }
  float s = 0;
  for (int e = 0; e < 16; ++e) s += c0[e] + c1[e] + c2[e] + c3[e];
  out[blockIdx.x * blockDim.x + t] = s;
}

int cmd_peak() {
  hipDeviceProp_t prop;
  HIP_OK(hipGetDeviceProperties(&prop, 0));
  const int cus = prop.multiProcessorCount;
  const int blocks = cus * 4;  // 4 blocks x 4 waves = 4 waves per SIMD
  const int iters = 20000;
  float* out = dalloc<float>((size_t)blocks * 256);
  hipEvent_t e0, e1;
  HIP_OK(hipEventCreate(&e0));
  HIP_OK(hipEventCreate(&e1));
  hipLaunchKernelGGL(mfma_peak_kernel, dim3(blocks), dim3(256), 0, nullptr, out, 100);
  HIP_OK(hipGetLastError());
  HIP_OK(hipDeviceSynchronize());
  double best = 0;
  for (int rep = 0; rep < 3; ++rep) {
    HIP_OK(hipEventRecord(e0, nullptr));
    hipLaunchKernelGGL(mfma_peak_kernel, dim3(blocks), dim3(256), 0, nullptr, out, iters);
    HIP_OK(hipGetLastError());
    HIP_OK(hipEventRecord(e1, nullptr));
    HIP_OK(hipEventSynchronize(e1));
    float ms = 0;
    HIP_OK(hipEventElapsedTime(&ms, e0, e1));
    const double flops = (double)blocks * 4 /*waves*/ * iters * 4 * 32768.0;
    best = std::fmax(best, flops / (ms * 1e-3) / 1e12);
  }
  std::printf("peak: %d CUs, v_mfma_f32_32x32x16_f16 sustained %.1f TFLOP/s (published dense "
              "fp16 peak 2500)\n", cus, best);
  HIP_OK(hipFree(out));
  return 0;
}

// Issue mix of one wave: one dependent chain of 32x32x16 fp16 MFMAs (the
// shape of an S^T product: every product accumulates into the last), each
// followed by NF fp32 FMAs and NE v_exp_f32 on 16 independent values (the
// softmax's work per product), in that order by scheduling groups. NM = 0
// leaves the VALU work alone. The wave's shader clock comes from s_memtime
// against the 100 MHz s_memrealtime.
template <int NM, int NF, int NE>
__global__ __launch_bounds__(256) void mix_kernel(float* out, int iters, long long* clk) {
  const int t = threadIdx.x;
  half8_t a, b;
  for (int e = 0; e < 8; ++e) {
    a[e] = (_Float16)(((t + e) & 7) * 0.001f);
    b[e] = (_Float16)(((t * 3 + e) & 7) * 0.001f);
  }
  floatx16_t c = {};
  float x[16];
  for (int r = 0; r < 16; ++r) x[r] = (t + r) * 1e-3f;
  const long long t0 = clock64(), r0 = wall_clock64();
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      if (NM) c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
#pragma unroll
      for (int v = 0; v < NF; ++v) x[(m * NF + v) & 15] = fmaf(x[(m * NF + v) & 15], 0.5f, -0.25f);
#pragma unroll
      for (int v = 0; v < NE; ++v) x[(m * NE + v + 8) & 15] = __builtin_amdgcn_exp2f(x[(m * NE + v + 8) & 15]);
      if (NM) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // the product
      if (NF + NE) __builtin_amdgcn_sched_group_barrier(0x002, NF + NE, 0);  // its VALU work
    }
  }
  const long long t1 = clock64(), r1 = wall_clock64();
  float s = 0;
  for (int e = 0; e < 16; ++e) s += c[e] + x[e];
  out[blockIdx.x * blockDim.x + t] = s;
  if (t == 0 && blockIdx.x == 0) {
    clk[0] = t1 - t0;
    clk[1] = r1 - r0;
  }
}

// Cycles per SIMD for each (product + its VALU work) at two waves per SIMD
// (the kernels' occupancy), and the VALU instructions alone: what the
// softmax's FMAs and exponentials cost beside the products.
int cmd_mix() {
  hipDeviceProp_t prop;
  HIP_OK(hipGetDeviceProperties(&prop, 0));
  const int cus = prop.multiProcessorCount;
  const int blocks = cus * 2;  // blocks of 4 waves: 2 waves per SIMD
  const int iters = 4000;
  float* out = dalloc<float>((size_t)blocks * 256);
  long long* clk = dalloc<long long>(2);
  hipEvent_t e0, e1;
  HIP_OK(hipEventCreate(&e0));
  HIP_OK(hipEventCreate(&e1));
  struct Case {
    const char* name;
    void (*k)(float*, int, long long*);
    int nm, nvalu;
  };
  const Case cases[] = {
      {"MFMA chain alone", mix_kernel<1, 0, 0>, 1, 0},
      {"MFMA + 4 FMA", mix_kernel<1, 4, 0>, 1, 4},
      {"MFMA + 6 FMA", mix_kernel<1, 6, 0>, 1, 6},
      {"MFMA + 2 exp", mix_kernel<1, 0, 2>, 1, 2},
      {"MFMA + 2 FMA + 2 exp", mix_kernel<1, 2, 2>, 1, 4},
      {"MFMA + 4 exp", mix_kernel<1, 0, 4>, 1, 4},
      {"16 FMA alone", mix_kernel<0, 16, 0>, 0, 16},
      {"16 exp alone", mix_kernel<0, 0, 16>, 0, 16},
  };
  for (const Case& cs : cases) {
    hipLaunchKernelGGL(cs.k, dim3(blocks), dim3(256), 0, nullptr, out, 10, clk);
    HIP_OK(hipGetLastError());
    HIP_OK(hipDeviceSynchronize());
    float best = 1e30f;
    long long hc[2] = {0, 0};
    for (int rep = 0; rep < 3; ++rep) {
      HIP_OK(hipEventRecord(e0, nullptr));
      hipLaunchKernelGGL(cs.k, dim3(blocks), dim3(256), 0, nullptr, out, iters, clk);
      HIP_OK(hipGetLastError());
      HIP_OK(hipEventRecord(e1, nullptr));
      HIP_OK(hipEventSynchronize(e1));
      float ms = 0;
      HIP_OK(hipEventElapsedTime(&ms, e0, e1));
      if (ms < best) {
        best = ms;
        HIP_OK(hipMemcpy(hc, clk, sizeof(hc), hipMemcpyDeviceToHost));
      }
    }
    const double ghz = hc[1] > 0 ? (double)hc[0] / (double)hc[1] * 0.1 : 0.0;
    const double kernel_cycles = best * 1e-3 * ghz * 1e9;
    const double groups = 2.0 * iters * 8;  // per SIMD: 2 waves x iters x 8 groups
    if (cs.nm) {
      const double tf = (double)blocks * 4 * iters * 8 * 32768.0 / (best * 1e-3) / 1e12;
      std::printf("mix: %-22s %7.1f TFLOP/s, %5.1f cycles per product per SIMD at %.2f GHz\n",
                  cs.name, tf, kernel_cycles / groups, ghz);
    } else {
      std::printf("mix: %-22s %5.2f cycles per wave64 instruction per SIMD at %.2f GHz\n", cs.name,
                  kernel_cycles / (groups * cs.nvalu), ghz);
    }
  }
  HIP_OK(hipFree(out));
  HIP_OK(hipFree(clk));
  return 0;
}

// LDS operand reads of the kernels' D = 128 tiles, through the kernels' own
// layout helpers (fa_device.h): PAT 0 16-byte reads of a padded tile
// (tile_read16), 1 16-byte reads of swizzled 256-byte rows (Swz::read16),
// 2 transpose reads of a padded tile (tile_tr_operand), 3 transpose reads of
// swizzled rows (Swz::tr_operand). Each iteration reads eight operands of one
// 32-row block (rows 0-31 or 32-63 of a 64-row tile); the empty asm with a
// memory clobber keeps the compiler from hoisting the reads out of the loop.
template <int PAT>
__global__ __launch_bounds__(256) void lds_kernel(float* out, int iters, long long* clk) {
  using T = fa::Tile<128>;
  using S = fa::Swz<128>;
  constexpr int kHalves = 64 * T::kRowHalves;  // 64 padded rows (17 KB) >= 64 swizzled rows
  __shared__ __align__(16) fa::half_t tile[kHalves];
  const int t = threadIdx.x, lane = t & 63;
  for (int i = t; i < kHalves; i += 256) tile[i] = (fa::half_t)(float)(i & 63);
  __syncthreads();
  const int roff = fa::row_lane_off<128>(lane), troff = fa::tr_lane_off<128>(lane);
  typename S::Offsets so0, so1;
  so0.init(lane, 0);
  so1.init(lane, 32);
  float acc = 0.f;
  const long long t0 = clock64(), r0 = wall_clock64();
  for (int i = 0; i < iters; ++i) {
    const int rb = (i & 1) * 32;
    const typename S::Offsets& so = (i & 1) ? so1 : so0;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      fa::half8 v;
      if (PAT == 0) v = fa::tile_read16<128>(tile, rb, m, roff);
      if (PAT == 1) v = S::read16(tile, so, m);
      if (PAT == 2) v = fa::tile_tr_operand<128>(tile, rb + 16 * (m & 1), 32 * (m >> 1), troff);
      if (PAT == 3) v = S::tr_operand(tile, m & 1, so, m >> 1);
      acc += (float)v[0] + (float)v[7];
    }
    asm volatile("" ::: "memory");
  }
  const long long t1 = clock64(), r1 = wall_clock64();
  out[blockIdx.x * blockDim.x + t] = acc;
  if (t == 0 && blockIdx.x == 0) {
    clk[0] = t1 - t0;
    clk[1] = r1 - r0;
  }
}

// LDS read throughput of those patterns per CU at two waves per SIMD (the
// kernels' occupancy): what the operand reads of a step cost.
int cmd_lds() {
  hipDeviceProp_t prop;
  HIP_OK(hipGetDeviceProperties(&prop, 0));
  const int cus = prop.multiProcessorCount;
  const int blocks = cus * 2;
  const int iters = 4000;
  float* out = dalloc<float>((size_t)blocks * 256);
  long long* clk = dalloc<long long>(2);
  hipEvent_t e0, e1;
  HIP_OK(hipEventCreate(&e0));
  HIP_OK(hipEventCreate(&e1));
  struct Case {
    const char* name;
    void (*k)(float*, int, long long*);
  };
  const Case cases[] = {
      {"16-byte reads, padded rows", lds_kernel<0>},
      {"16-byte reads, swizzled rows", lds_kernel<1>},
      {"transpose reads, padded rows", lds_kernel<2>},
      {"transpose reads, swizzled rows", lds_kernel<3>},
  };
  for (const Case& cs : cases) {
    hipLaunchKernelGGL(cs.k, dim3(blocks), dim3(256), 0, nullptr, out, 10, clk);
    HIP_OK(hipGetLastError());
    HIP_OK(hipDeviceSynchronize());
    float best = 1e30f;
    long long hc[2] = {0, 0};
    for (int rep = 0; rep < 3; ++rep) {
      HIP_OK(hipEventRecord(e0, nullptr));
      hipLaunchKernelGGL(cs.k, dim3(blocks), dim3(256), 0, nullptr, out, iters, clk);
      HIP_OK(hipGetLastError());
      HIP_OK(hipEventRecord(e1, nullptr));
      HIP_OK(hipEventSynchronize(e1));
      float ms = 0;
      HIP_OK(hipEventElapsedTime(&ms, e0, e1));
      if (ms < best) {
        best = ms;
        HIP_OK(hipMemcpy(hc, clk, sizeof(hc), hipMemcpyDeviceToHost));
      }
    }
    const double ghz = hc[1] > 0 ? (double)hc[0] / (double)hc[1] * 0.1 : 0.0;
    const double bytes_per_cu = 8.0 * 64 * iters * 8 * 16.0;  // 8 waves x 64 lanes x 16 B per operand
    std::printf("lds: %-32s %6.1f B/clk per CU at %.2f GHz\n", cs.name,
                bytes_per_cu / (best * 1e-3 * ghz * 1e9), ghz);
  }
  HIP_OK(hipFree(out));
  HIP_OK(hipFree(clk));
  return 0;
}

// One item per (head, key tile u, query step i0) of a causal backward with
// 128-key tiles and 64-row query steps, dealt out evenly over the grid (the
// library balances its causal work the same way). mode 0: each item adds its
// 64 x D fp32 partial into dQ rows i0 .. i0+63 with no-return fp32 atomics;
// mode 1: each item stores the partial to its own workspace slot (the first
// half of a store-then-reduce scheme). Consecutive threads touch consecutive
// floats, so every wave's accesses are fully coalesced.
__global__ __launch_bounds__(256) void dq_traffic_kernel(float* dq, float* ws,
                                                         const int2* items, int n_items,
                                                         int per_block, int N, int D,
                                                         int mode) {
  const int first = blockIdx.x * per_block;
  const int last = min(first + per_block, n_items);
  for (int it = first; it < last; ++it) {
    const int2 hi = items[it];  // (head, first query row)
    float* dst = mode == 0 ? dq + ((size_t)hi.x * N + hi.y) * D : ws + (size_t)it * 64 * D;
    for (int e = threadIdx.x; e < 64 * D; e += 256) {
      const float v = (float)((e + it) & 7) * 0.125f;
      if (mode == 0) unsafeAtomicAdd(dst + e, v);
      else dst[e] = v;
    }
  }
}

int cmd_dqcost() {
  const int B = 1, H = 8, N = 4096, D = 128, tiles = N / 128;
  std::vector<int2> items;
  for (int h = 0; h < H; ++h)
    for (int u = 0; u < tiles; ++u)
      for (int i0 = 128 * u; i0 < N; i0 += 64) items.push_back(make_int2(h, i0));
  const int n_items = (int)items.size();
  hipDeviceProp_t prop;
  HIP_OK(hipGetDeviceProperties(&prop, 0));
  const int blocks = prop.multiProcessorCount;
  const int per_block = (n_items + blocks - 1) / blocks;
  int2* d_items = dalloc<int2>(items.size());
  HIP_OK(hipMemcpy(d_items, items.data(), items.size() * sizeof(int2), hipMemcpyHostToDevice));
  float* dq = dalloc<float>((size_t)B * H * N * D);
  float* ws = dalloc<float>((size_t)n_items * 64 * D);
  HIP_OK(hipMemset(dq, 0, (size_t)B * H * N * D * sizeof(float)));
  hipEvent_t e0, e1;
  HIP_OK(hipEventCreate(&e0));
  HIP_OK(hipEventCreate(&e1));
  const double bytes = (double)n_items * 64 * D * sizeof(float);
  const char* names[2] = {"fp32 atomics into dQ", "stores to a workspace"};
  for (int mode = 0; mode < 2; ++mode) {
    std::vector<float> ms_all;
    for (int rep = 0; rep < 12; ++rep) {
      HIP_OK(hipEventRecord(e0, nullptr));
      hipLaunchKernelGGL(dq_traffic_kernel, dim3(blocks), dim3(256), 0, nullptr, dq, ws, d_items,
                         n_items, per_block, N, D, mode);
      HIP_OK(hipGetLastError());
      HIP_OK(hipEventRecord(e1, nullptr));
      HIP_OK(hipEventSynchronize(e1));
      float ms = 0;
      HIP_OK(hipEventElapsedTime(&ms, e0, e1));
      if (rep >= 2) ms_all.push_back(ms);
    }
    std::sort(ms_all.begin(), ms_all.end());
    const double med = ms_all[ms_all.size() / 2];
    std::printf("dqcost: %d partials of 64 x %d fp32 (%.1f MiB), %s: median %.1f us "
                "(%.0f GB/s)\n", n_items, D, bytes / 1048576.0, names[mode], med * 1e3,
                bytes / (med * 1e-3) / 1e9);
  }
  // The library's backward on the same shape, for scale (fa_bwd: preprocess +
  // the one main kernel, whose dQ pass recomputes S and dP instead).
  Shape s{B, H, H, N, D, true};
  _Float16 *q = dalloc<_Float16>(s.nq()), *k = dalloc<_Float16>(s.nk()),
           *v = dalloc<_Float16>(s.nk()), *g = dalloc<_Float16>(s.nq()),
           *o = dalloc<_Float16>(s.nq()), *dk = dalloc<_Float16>(s.nk()),
           *dv = dalloc<_Float16>(s.nk());
  float* lse = dalloc<float>((size_t)B * H * N);
  Rng rng{77};
  std::vector<_Float16> h(s.nq());
  for (_Float16* t : {q, k, v, g}) {  // standard-normal inputs, as bench.py
    for (auto& x : h) x = (_Float16)rng.normal();
    HIP_OK(hipMemcpy(t, h.data(), h.size() * sizeof(_Float16), hipMemcpyHostToDevice));
  }
  FA_OK_(fa_fwd(q, k, v, o, lse, B, H, H, N, D, 1, 0, nullptr));
  const size_t ws_bytes = fa_bwd_workspace_bytes(B, H, H, N, D);
  void* bws = dalloc<char>(ws_bytes);
  std::vector<float> ms_all;
  for (int rep = 0; rep < 12; ++rep) {
    HIP_OK(hipEventRecord(e0, nullptr));
    FA_OK_(fa_bwd(q, k, v, g, o, lse, dq, dk, dv, bws, ws_bytes, B, H, H, N, D, 1, nullptr));
    HIP_OK(hipEventRecord(e1, nullptr));
    HIP_OK(hipEventSynchronize(e1));
    float ms = 0;
    HIP_OK(hipEventElapsedTime(&ms, e0, e1));
    if (rep >= 2) ms_all.push_back(ms);
  }
  std::sort(ms_all.begin(), ms_all.end());
  std::printf("dqcost: fa_bwd (with its dQ pass) on the same shape: median %.1f us\n",
              ms_all[ms_all.size() / 2] * 1e3);
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  const std::string cmd = argc > 1 ? argv[1] : "";
  if (cmd == "check") return cmd_check();
  if (cmd == "fd") return cmd_fd();
  if (cmd == "bench") return cmd_bench(argc > 2 && std::string(argv[2]) == "quick");
  if (cmd == "peak") return cmd_peak();
  if (cmd == "mix") return cmd_mix();
  if (cmd == "lds") return cmd_lds();
  if (cmd == "dqcost") return cmd_dqcost();
  std::fprintf(stderr, "usage: %s check | fd | bench [quick] | peak | mix | lds | dqcost\n", argv[0]);
  return 2;
}
