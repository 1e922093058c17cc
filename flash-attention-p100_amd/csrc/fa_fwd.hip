// FlashAttention-2 forward for gfx950 (MI355X).
//
// Counterpart of the reference's flash::fwd_kernel (flash_fwd.cuh:68-340),
// redesigned around MFMA:
//   * a workgroup is 4 waves; each wave owns 32 query rows (BR = 128 rows per
//     workgroup) and walks the key/value sequence in tiles of BC = 64 rows;
//   * S is computed TRANSPOSED, S^T = K Q^T, on v_mfma_f32_32x32x16_f16 with
//     Q^T held in registers as the B operand for the whole kernel. In the
//     accumulator layout lane l then owns query row l % 32, so the online
//     softmax row max / row sum is a per-lane reduction plus one exchange
//     with the other half of the wave;
//   * P^T leaves the accumulator as fp16 and is fed back as the B operand of
//     O^T += V^T P^T without touching LDS (the K index order of the product
//     is chosen to match the accumulator layout); V is staged transposed
//     (V^T, rows = head dim) in LDS, K row-major, both double-buffered;
//   * the scale is applied to the fp32 logit (never to Q in fp16,
//     flash_fwd.cuh:94-101) with log2(e) folded in so exp2 is used;
//   * causal: key tiles past the workgroup's last row are never loaded
//     (flash_fwd.cuh:127-130) and a wave skips tiles entirely above its own
//     rows; ragged N is handled by zero-filled loads plus -inf masking of
//     key columns >= N (flash_fwd.cuh:226-243).
// Outputs: O (fp16) and LSE = m + log(l) in natural-log units of the scaled
// logits (flash_fwd.cuh:321-339).
#include "fa_device.h"
#include "fa_launch.h"

namespace fa {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBR = 32 * kWaves;  // query rows per workgroup
constexpr int kBC = 64;           // key rows per tile
constexpr int kKPad = 8;          // halves of padding per K row in LDS
constexpr int kVPad = 4;          // halves of padding per V^T row in LDS

template <int D>
struct FwdSmem {
  static constexpr int kKRow = D + kKPad;    // K tile  [kBC][kKRow]
  static constexpr int kVRow = kBC + kVPad;  // V^T tile [D][kVRow]
  static constexpr int kKElems = kBC * kKRow;
  static constexpr int kVElems = D * kVRow;
  static constexpr int kStage = kKElems + kVElems;
  static constexpr int kBytes = 2 * kStage * 2;
};

// Global -> register staging of one K/V tile (rows j0 .. j0+kBC-1).
template <int D>
struct KVStage {
  static constexpr int kKChunks = kBC * D / 8;             // 16-byte chunks of K
  static constexpr int kKPerThread = kKChunks / kThreads;  // 2 (D=64) or 4 (D=128)
  static constexpr int kVTasks = (kBC / 4) * (D / 8);      // 4x8 blocks of V
  static constexpr int kVPerThread = (kVTasks + kThreads - 1) / kThreads;  // 1
  u32x4 k[kKPerThread];
  u32x4 v[kVPerThread][4];

  __device__ __forceinline__ void load(const half_t* K, const half_t* V, int j0, int N,
                                       int tid, bool bounds) {
#pragma unroll
    for (int u = 0; u < kKPerThread; ++u) {
      const int c = tid + u * kThreads;
      const int row = c / (D / 8), col = (c % (D / 8)) * 8;
      const int j = j0 + row;
      k[u] = load16(K + (size_t)j * D + col, !bounds || j < N);
    }
#pragma unroll
    for (int u = 0; u < kVPerThread; ++u) {
      const int t = tid + u * kThreads;
      // j-groups vary fastest across lanes so the transposed LDS writes of a
      // wave land in distinct banks.
      const int jg = t % (kBC / 4), dg = t / (kBC / 4);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = j0 + jg * 4 + r;
        v[u][r] = load16(V + (size_t)j * D + dg * 8, t < kVTasks && (!bounds || j < N));
      }
    }
  }

  __device__ __forceinline__ void store(half_t* Ks, half_t* Vt, int tid) const {
    using S = FwdSmem<D>;
#pragma unroll
    for (int u = 0; u < kKPerThread; ++u) {
      const int c = tid + u * kThreads;
      const int row = c / (D / 8), col = (c % (D / 8)) * 8;
      *reinterpret_cast<u32x4*>(Ks + row * S::kKRow + col) = k[u];
    }
#pragma unroll
    for (int u = 0; u < kVPerThread; ++u) {
      const int t = tid + u * kThreads;
      if (t < kVTasks) {
        const int jg = t % (kBC / 4), dg = t / (kBC / 4);
        u32x2 cols[8];
        transpose_4x8(v[u], cols);
#pragma unroll
        for (int c = 0; c < 8; ++c)
          *reinterpret_cast<u32x2*>(Vt + (dg * 8 + c) * S::kVRow + jg * 4) = cols[c];
      }
    }
  }
};

template <int D, bool CAUSAL, bool BOUNDS>
__global__ __launch_bounds__(kThreads) void fwd_kernel(
    const half_t* __restrict__ Q, const half_t* __restrict__ K,
    const half_t* __restrict__ V, half_t* __restrict__ O, float* __restrict__ Lse,
    int N, int Hq, int group, int n_qtiles, float scale_log2) {
  using S = FwdSmem<D>;
  extern __shared__ __align__(16) half_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5;     // which half of the wave
  const int l32 = lane & 31;

  // Longest causal tiles first: they start before the short ones.
  const int qtile = CAUSAL ? (n_qtiles - 1 - (int)blockIdx.x) : (int)blockIdx.x;
  const int q0 = qtile * kBR;
  const int bh = blockIdx.y;                   // over B*Hq
  const int b = bh / Hq, hq = bh % Hq;
  const int hkv = hq / group;                  // repeat_interleave head map
  const int Hkv = Hq / group;
  const size_t q_off = (size_t)bh * N * D;
  const size_t kv_off = ((size_t)b * Hkv + hkv) * N * D;
  Q += q_off;
  O += q_off;
  K += kv_off;
  V += kv_off;
  Lse += (size_t)bh * N;

  // This wave's query rows and its Q^T operands (B of S^T = K Q^T).
  const int i_base = q0 + wave * 32;
  const int i_row = i_base + l32;
  half8 qb[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk)
    qb[kk] = as_half8(load16(Q + (size_t)i_row * D + kk * 16 + h * 8, !BOUNDS || i_row < N));

  floatx16 oacc[D / 32];
#pragma unroll
  for (int c = 0; c < D / 32; ++c) oacc[c] = zero16();
  float m_run = -INFINITY;  // running max, log2 domain
  float l_run = 0.f;        // running sum of exp2(x - m_run)

  const int kv_end = CAUSAL ? min(N, q0 + kBR) : N;
  const int n_tiles = (kv_end + kBC - 1) / kBC;

  KVStage<D> st;
  st.load(K, V, 0, N, tid, BOUNDS);
  st.store(smem, smem + S::kKElems, tid);
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int j0 = t * kBC;
    const bool has_next = t + 1 < n_tiles;
    if (has_next) st.load(K, V, j0 + kBC, N, tid, BOUNDS);

    half_t* Ks = smem + (t & 1) * S::kStage;
    half_t* Vt = Ks + S::kKElems;

    // A wave whose rows all precede this tile sees only masked keys.
    const bool active = !CAUSAL || j0 <= i_base + 31;
    if (active) {
      floatx16 sacc[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        sacc[s] = zero16();
        const half_t* krow = Ks + (s * 32 + l32) * S::kKRow + h * 8;
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          const half8 a = *reinterpret_cast<const half8*>(krow + kk * 16);
          sacc[s] = mfma32(a, qb[kk], sacc[s]);
        }
      }

      // Scale into the log2 domain and mask.
      const bool need_mask = (CAUSAL && j0 + kBC - 1 > i_base) || (BOUNDS && j0 + kBC > N);
      float mloc = -INFINITY;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = sacc[s][r] * scale_log2;
          if (need_mask) {
            const int j = j0 + s * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            if ((CAUSAL && j > i_row) || (BOUNDS && j >= N)) x = -INFINITY;
          }
          sacc[s][r] = x;
          mloc = fmaxf(mloc, x);
        }
      }
      mloc = fmaxf(mloc, xor32(mloc));
      const float m_new = fmaxf(m_run, mloc);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float corr = fast_exp2(m_run - m_use);
      float lloc = 0.f;
      half8 pb[4];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = fast_exp2(sacc[s][r] - m_use);
          lloc += p;
          pb[2 * s + (r >> 3)][r & 7] = (half_t)p;
        }
      }
      lloc += xor32(lloc);
      l_run = l_run * corr + lloc;
      m_run = m_new;
#pragma unroll
      for (int c = 0; c < D / 32; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[c][r] *= corr;

      // O^T += V^T P^T. K-step (s, q) covers keys 32s+16q .. +15; slot (h, e)
      // is key 32s + 16q + 8*(e/4) + 4h + e%4, matching the accumulator.
#pragma unroll
      for (int c = 0; c < D / 32; ++c) {
        const half_t* vrow = Vt + (c * 32 + l32) * S::kVRow + 4 * h;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const half4 lo = *reinterpret_cast<const half4*>(vrow + ks * 16);
          const half4 hi = *reinterpret_cast<const half4*>(vrow + ks * 16 + 8);
          const half8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          oacc[c] = mfma32(a, pb[ks], oacc[c]);
        }
      }
    }

    if (has_next) {
      half_t* Kn = smem + ((t + 1) & 1) * S::kStage;
      st.store(Kn, Kn + S::kKElems, tid);
    }
    __syncthreads();
  }

  // Epilogue: O = acc / l (fp16), LSE = (m + log2 l) * ln 2.
  if (!BOUNDS || i_row < N) {
    const float inv_l = 1.f / l_run;
    half_t* orow = O + (size_t)i_row * D;
#pragma unroll
    for (int c = 0; c < D / 32; ++c) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        half4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = (half_t)(oacc[c][4 * g + e] * inv_l);
        *reinterpret_cast<half4*>(orow + c * 32 + 8 * g + 4 * h) = o4;
      }
    }
    if (h == 0) Lse[i_row] = (m_run + __log2f(l_run)) * kLn2;
  }
}

template <int D, bool CAUSAL, bool BOUNDS>
hipError_t launch_fwd_t(const FwdArgs& a) {
  const int n_qtiles = (a.N + kBR - 1) / kBR;
  dim3 grid(n_qtiles, a.B * a.Hq);
  const size_t smem = FwdSmem<D>::kBytes;
  const float scale_log2 = kLog2e / sqrtf((float)D);
  // One-time, idempotent: lift the dynamic-LDS cap above the 64 KB default.
  static const hipError_t attr = allow_lds(fwd_kernel<D, CAUSAL, BOUNDS>, smem);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((fwd_kernel<D, CAUSAL, BOUNDS>), grid, dim3(kThreads), smem,
                     (hipStream_t)a.stream, (const half_t*)a.q, (const half_t*)a.k,
                     (const half_t*)a.v, (half_t*)a.o, a.lse, a.N, a.Hq, a.Hq / a.Hkv,
                     n_qtiles, scale_log2);
  return hipGetLastError();
}

template <int D>
hipError_t launch_fwd_d(const FwdArgs& a) {
  const bool bounds = (a.N % kBR) != 0;  // kBR is a multiple of kBC
  if (a.causal) return bounds ? launch_fwd_t<D, true, true>(a) : launch_fwd_t<D, true, false>(a);
  return bounds ? launch_fwd_t<D, false, true>(a) : launch_fwd_t<D, false, false>(a);
}

}  // namespace

hipError_t launch_fwd(const FwdArgs& a) {
  return a.D == 64 ? launch_fwd_d<64>(a) : launch_fwd_d<128>(a);
}

}  // namespace fa
