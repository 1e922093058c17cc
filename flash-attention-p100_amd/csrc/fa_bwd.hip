// FlashAttention-2 backward for gfx950 (MI355X).
//
// Counterpart of the reference's flash_bwd::bwd_preprocess and
// flash_bwd::bwd_kernel (flash_bwd.cuh:65-78, 95-464), redesigned around
// MFMA. Per (query tile i, key tile j), with L = LSE and Dv = rowsum(dO*O):
//   S = Q K^T            P = exp(S*scale - L)
//   dV += P^T dO         dP = dO V^T
//   dS = P (dP - Dv)     dK += dS^T Q * scale     dQ += dS K * scale
// (flash_bwd.cuh:11-16).
//
// Main kernel layout (K/V stationary, FA2 loop order):
//   * a workgroup owns kBC = 128 key rows; each of its 4 waves owns 32 of
//     them and keeps its K and V rows in registers as MFMA B operands and its
//     dK^T / dV^T blocks in fp32 accumulators for the whole kernel;
//   * it walks the query rows in tiles of kBR = 32 (from the diagonal on,
//     for causal, flash_bwd.cuh:158-161), looping over the query heads of its
//     key/value head for GQA/MQA (flash_bwd.cuh:120-131, 163);
//   * S and dP come out of v_mfma_f32_32x32x16_f16 with lane l holding key
//     column l % 32, so P and dS feed dV^T += dO^T P and dK^T += Q^T dS
//     straight from the accumulators (the product's K index order is chosen
//     to match), with Q^T / dO^T staged transposed in LDS;
//   * dS is also written to LDS (fp16) so the four waves can form
//     dQ = dS K over all 128 keys, one 32-column slice of the head dim per
//     wave, added to the fp32 dQ with atomics (flash_bwd.cuh:434-443);
//   * dead lanes (causal col > row, ragged row/col >= N) contribute exactly
//     zero (flash_bwd.cuh:267-282).
// P and dS are rounded to fp16 only as MFMA operands; S, dP, P and dS are
// computed in fp32.
#include "fa_device.h"
#include "fa_launch.h"

namespace fa {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBC = 32 * kWaves;  // key rows per workgroup
constexpr int kBR = 32;           // query rows per inner tile

template <int D>
struct BwdSmem {
  static constexpr int kKtRow = kBC + 8;   // K^T  [D][kKtRow]
  static constexpr int kQRow = D + 8;      // Q, dO row-major [kBR][kQRow]
  static constexpr int kQtRow = kBR + 4;   // Q^T, dO^T [D][kQtRow]
  static constexpr int kSRow = kBC + 8;    // dS   [kBR][kSRow]
  static constexpr int kKt = 0;
  static constexpr int kQs = kKt + D * kKtRow;
  static constexpr int kQt = kQs + kBR * kQRow;
  static constexpr int kOs = kQt + D * kQtRow;
  static constexpr int kOt = kOs + kBR * kQRow;
  static constexpr int kSs = kOt + D * kQtRow;
  static constexpr int kHalves = kSs + kBR * kSRow;
  static constexpr int kBytes = kHalves * 2 + 2 * kBR * 4;  // + lse2, dvec
};

// ---------------------------------------------------------------------------
// Preprocess: dvec[row] = sum_d float(O[row,d]) * float(dO[row,d]) from the
// fp16-rounded O (flash_bwd.cuh:65-78), fused with clearing dq (the
// reference's cudaMemsetAsync, flash_bwd.cuh:476).
template <int D>
__global__ __launch_bounds__(256) void bwd_pre_kernel(const half_t* __restrict__ O,
                                                      const half_t* __restrict__ dO,
                                                      float* __restrict__ dvec,
                                                      float* __restrict__ dq, long rows) {
  constexpr int kLanesPerRow = D / 8;
  constexpr int kRowsPerBlock = 256 / kLanesPerRow;
  const int tid = threadIdx.x;
  const long row = (long)blockIdx.x * kRowsPerBlock + tid / kLanesPerRow;
  const int c8 = (tid % kLanesPerRow) * 8;
  float acc = 0.f;
  if (row < rows) {
    const half8 o = as_half8(*reinterpret_cast<const u32x4*>(O + row * D + c8));
    const half8 g = as_half8(*reinterpret_cast<const u32x4*>(dO + row * D + c8));
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += (float)o[e] * (float)g[e];
    floatx4 z = {0.f, 0.f, 0.f, 0.f};
    *reinterpret_cast<floatx4*>(dq + row * D + c8) = z;
    *reinterpret_cast<floatx4*>(dq + row * D + c8 + 4) = z;
  }
#pragma unroll
  for (int off = kLanesPerRow / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (row < rows && (tid % kLanesPerRow) == 0) dvec[row] = acc;
}

// ---------------------------------------------------------------------------
// Stages one query tile: Q and dO both row-major and transposed, plus the
// tile's LSE (converted to the log2 domain) and dvec.
template <int D>
__device__ __forceinline__ void stage_q_tile(half_t* smem, float* lse2s, float* dvs,
                                             const half_t* Qg, const half_t* dOg,
                                             const float* Lg, const float* Dg, int i0,
                                             int N, int tid, bool bounds) {
  using S = BwdSmem<D>;
  constexpr int kTasks = (kBR / 4) * (D / 8);  // per tensor
#pragma unroll
  for (int t = tid; t < 2 * kTasks; t += kThreads) {
    const int which = t / kTasks;  // 0: Q, 1: dO
    const int idx = t % kTasks;
    const int rg = idx % (kBR / 4), dg = idx / (kBR / 4);
    const half_t* src = which ? dOg : Qg;
    u32x4 rows[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = i0 + rg * 4 + r;
      rows[r] = load16(src + (size_t)i * D + dg * 8, !bounds || i < N);
    }
    half_t* rm = smem + (which ? S::kOs : S::kQs);
    half_t* tr = smem + (which ? S::kOt : S::kQt);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *reinterpret_cast<u32x4*>(rm + (rg * 4 + r) * S::kQRow + dg * 8) = rows[r];
    u32x2 cols[8];
    transpose_4x8(rows, cols);
#pragma unroll
    for (int c = 0; c < 8; ++c)
      *reinterpret_cast<u32x2*>(tr + (dg * 8 + c) * S::kQtRow + rg * 4) = cols[c];
  }
  if (tid < kBR) {
    const int i = i0 + tid;
    lse2s[tid] = (!bounds || i < N) ? Lg[i] * kLog2e : 0.f;
  } else if (tid < 2 * kBR) {
    const int i = i0 + tid - kBR;
    dvs[tid - kBR] = (!bounds || i < N) ? Dg[i] : 0.f;
  }
}

template <int D, bool CAUSAL, bool BOUNDS>
__global__ __launch_bounds__(kThreads) void bwd_kernel(
    const half_t* __restrict__ Q, const half_t* __restrict__ K,
    const half_t* __restrict__ V, const half_t* __restrict__ dO,
    const float* __restrict__ Lse, const float* __restrict__ Dvec,
    float* __restrict__ dQ, half_t* __restrict__ dK, half_t* __restrict__ dV,
    int N, int Hq, int group, float scale, float scale_log2) {
  using S = BwdSmem<D>;
  extern __shared__ __align__(16) half_t smem[];
  float* lse2s = reinterpret_cast<float*>(smem + S::kHalves);
  float* dvs = lse2s + kBR;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5;
  const int l32 = lane & 31;

  const int j0 = blockIdx.x * kBC;
  const int bkv = blockIdx.y;  // over B*Hkv
  const int Hkv = Hq / group;
  const int b = bkv / Hkv, hkv = bkv % Hkv;
  const size_t kv_off = (size_t)bkv * N * D;
  K += kv_off;
  V += kv_off;
  dK += kv_off;
  dV += kv_off;

  // Stationary K^T in LDS for the dQ product.
  {
    constexpr int kTasks = (kBC / 4) * (D / 8);
#pragma unroll
    for (int t = tid; t < kTasks; t += kThreads) {
      const int rg = t % (kBC / 4), dg = t / (kBC / 4);
      u32x4 rows[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = j0 + rg * 4 + r;
        rows[r] = load16(K + (size_t)j * D + dg * 8, !BOUNDS || j < N);
      }
      u32x2 cols[8];
      transpose_4x8(rows, cols);
#pragma unroll
      for (int c = 0; c < 8; ++c)
        *reinterpret_cast<u32x2*>(smem + S::kKt + (dg * 8 + c) * S::kKtRow + rg * 4) = cols[c];
    }
  }

  // This wave's key rows as B operands (K^T for S, V^T for dP).
  const int jw = j0 + wave * 32;
  const int j_col = jw + l32;
  half8 kb[D / 16], vb[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    const bool ok = !BOUNDS || j_col < N;
    kb[kk] = as_half8(load16(K + (size_t)j_col * D + kk * 16 + h * 8, ok));
    vb[kk] = as_half8(load16(V + (size_t)j_col * D + kk * 16 + h * 8, ok));
  }

  floatx16 dvacc[D / 32], dkacc[D / 32];
#pragma unroll
  for (int c = 0; c < D / 32; ++c) {
    dvacc[c] = zero16();
    dkacc[c] = zero16();
  }

  const int i_start = CAUSAL ? j0 : 0;  // j0 is a multiple of kBR
  for (int g = 0; g < group; ++g) {
    const size_t bhq = (size_t)b * Hq + (size_t)hkv * group + g;
    const half_t* Qg = Q + bhq * N * D;
    const half_t* dOg = dO + bhq * N * D;
    const float* Lg = Lse + bhq * N;
    const float* Dg = Dvec + bhq * N;
    float* dQg = dQ + bhq * N * D;

    for (int i0 = i_start; i0 < N; i0 += kBR) {
      stage_q_tile<D>(smem, lse2s, dvs, Qg, dOg, Lg, Dg, i0, N, tid, BOUNDS);
      __syncthreads();

      half_t* dSs = smem + S::kSs;
      const bool active = !CAUSAL || (i0 + kBR - 1 >= jw);
      if (active) {
        floatx16 sacc = zero16(), pacc = zero16();
        const half_t* qrow = smem + S::kQs + l32 * S::kQRow + h * 8;
        const half_t* orow = smem + S::kOs + l32 * S::kQRow + h * 8;
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          sacc = mfma32(*reinterpret_cast<const half8*>(qrow + kk * 16), kb[kk], sacc);
          pacc = mfma32(*reinterpret_cast<const half8*>(orow + kk * 16), vb[kk], pacc);
        }
        // P and dS; row i = i0 + 8*(r/4) + 4h + r%4, column j_col.
        const bool need_mask = (CAUSAL && i0 < jw + 31) || (BOUNDS && (i0 + kBR > N || jw + 32 > N));
        half8 pb[2], sb[2];
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const floatx4 l4 = *reinterpret_cast<const floatx4*>(lse2s + 8 * g4 + 4 * h);
          const floatx4 d4 = *reinterpret_cast<const floatx4*>(dvs + 8 * g4 + 4 * h);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g4 + e;
            float p = fast_exp2(sacc[r] * scale_log2 - l4[e]);
            if (need_mask) {
              const int i = i0 + 8 * g4 + 4 * h + e;
              const bool dead = (CAUSAL && j_col > i) || (BOUNDS && (i >= N || j_col >= N));
              if (dead) p = 0.f;
            }
            const float ds = p * (pacc[r] - d4[e]);
            pb[r >> 3][r & 7] = (half_t)p;
            sb[r >> 3][r & 7] = (half_t)ds;
            dSs[(8 * g4 + 4 * h + e) * S::kSRow + wave * 32 + l32] = (half_t)ds;
          }
        }
        // dV^T += dO^T P and dK^T += Q^T dS. K-step q covers query rows
        // 16q .. 16q+15; slot (h, e) is row 16q + 8*(e/4) + 4h + e%4.
#pragma unroll
        for (int c = 0; c < D / 32; ++c) {
          const half_t* ot = smem + S::kOt + (c * 32 + l32) * S::kQtRow + 4 * h;
          const half_t* qt = smem + S::kQt + (c * 32 + l32) * S::kQtRow + 4 * h;
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const half4 olo = *reinterpret_cast<const half4*>(ot + 16 * q);
            const half4 ohi = *reinterpret_cast<const half4*>(ot + 16 * q + 8);
            const half4 qlo = *reinterpret_cast<const half4*>(qt + 16 * q);
            const half4 qhi = *reinterpret_cast<const half4*>(qt + 16 * q + 8);
            const half8 ao = {olo[0], olo[1], olo[2], olo[3], ohi[0], ohi[1], ohi[2], ohi[3]};
            const half8 aq = {qlo[0], qlo[1], qlo[2], qlo[3], qhi[0], qhi[1], qhi[2], qhi[3]};
            dvacc[c] = mfma32(ao, pb[q], dvacc[c]);
            dkacc[c] = mfma32(aq, sb[q], dkacc[c]);
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          dSs[(8 * (r >> 2) + 4 * h + (r & 3)) * S::kSRow + wave * 32 + l32] = (half_t)0.f;
      }
      __syncthreads();

      // dQ[i, d] += scale * sum_j dS[i, j] K[j, d] over the workgroup's keys.
      {
        constexpr int kDBlocks = D / 32;                 // 32-column slices
        constexpr int kJSplit = kWaves / kDBlocks;       // waves sharing a slice
        constexpr int kJSteps = kBC / 16 / kJSplit;      // 16-key steps per wave
        const int c = wave % kDBlocks;
        const int js = wave / kDBlocks;
        floatx16 qacc = zero16();
        const half_t* srow = dSs + l32 * S::kSRow + h * 8 + js * kJSteps * 16;
        const half_t* krow = smem + S::kKt + (c * 32 + l32) * S::kKtRow + h * 8 + js * kJSteps * 16;
#pragma unroll
        for (int t = 0; t < kJSteps; ++t)
          qacc = mfma32(*reinterpret_cast<const half8*>(srow + t * 16),
                        *reinterpret_cast<const half8*>(krow + t * 16), qacc);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = i0 + 8 * (r >> 2) + 4 * h + (r & 3);
          if (!BOUNDS || i < N)
            unsafeAtomicAdd(dQg + (size_t)i * D + c * 32 + l32, qacc[r] * scale);
        }
      }
    }
  }

  // dK (scaled) and dV leave once, from the accumulators, as fp16.
  if (!BOUNDS || j_col < N) {
    half_t* dkrow = dK + (size_t)j_col * D;
    half_t* dvrow = dV + (size_t)j_col * D;
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        half4 k4, v4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          k4[e] = (half_t)(dkacc[c][4 * g4 + e] * scale);
          v4[e] = (half_t)dvacc[c][4 * g4 + e];
        }
        *reinterpret_cast<half4*>(dkrow + c * 32 + 8 * g4 + 4 * h) = k4;
        *reinterpret_cast<half4*>(dvrow + c * 32 + 8 * g4 + 4 * h) = v4;
      }
    }
  }
}

template <int D>
hipError_t launch_pre_d(const BwdArgs& a) {
  constexpr int kRowsPerBlock = 256 / (D / 8);
  const long rows = (long)a.B * a.Hq * a.N;
  const dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  hipLaunchKernelGGL((bwd_pre_kernel<D>), grid, dim3(256), 0, (hipStream_t)a.stream,
                     (const half_t*)a.o, (const half_t*)a.dO, a.dvec, a.dq, rows);
  return hipGetLastError();
}

template <int D, bool CAUSAL, bool BOUNDS>
hipError_t launch_main_t(const BwdArgs& a) {
  const dim3 grid((a.N + kBC - 1) / kBC, a.B * a.Hkv);
  const size_t smem = BwdSmem<D>::kBytes;
  static const hipError_t attr = allow_lds(bwd_kernel<D, CAUSAL, BOUNDS>, smem);
  if (attr != hipSuccess) return attr;
  const float scale = 1.f / sqrtf((float)D);
  hipLaunchKernelGGL((bwd_kernel<D, CAUSAL, BOUNDS>), grid, dim3(kThreads), smem,
                     (hipStream_t)a.stream, (const half_t*)a.q, (const half_t*)a.k,
                     (const half_t*)a.v, (const half_t*)a.dO, a.lse, a.dvec, a.dq,
                     (half_t*)a.dk, (half_t*)a.dv, a.N, a.Hq, a.Hq / a.Hkv, scale,
                     scale * kLog2e);
  return hipGetLastError();
}

template <int D>
hipError_t launch_main_d(const BwdArgs& a) {
  const bool bounds = (a.N % kBC) != 0;  // kBC is a multiple of kBR
  if (a.causal) return bounds ? launch_main_t<D, true, true>(a) : launch_main_t<D, true, false>(a);
  return bounds ? launch_main_t<D, false, true>(a) : launch_main_t<D, false, false>(a);
}

}  // namespace

hipError_t launch_bwd_preprocess(const BwdArgs& a) {
  return a.D == 64 ? launch_pre_d<64>(a) : launch_pre_d<128>(a);
}

hipError_t launch_bwd_main(const BwdArgs& a) {
  return a.D == 64 ? launch_main_d<64>(a) : launch_main_d<128>(a);
}

}  // namespace fa
