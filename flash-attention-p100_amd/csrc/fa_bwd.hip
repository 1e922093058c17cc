// FlashAttention-2 backward for gfx950 (MI355X).
//
// Counterpart of the reference's flash_bwd::bwd_preprocess and
// flash_bwd::bwd_kernel (flash_bwd.cuh:65-78, 95-464). Per (query tile i,
// key tile j), with L = LSE and Dv = rowsum(dO*O) (flash_bwd.cuh:11-16):
//   S = Q K^T            P = exp(S*scale - L)
//   dV += P^T dO         dP = dO V^T
//   dS = P (dP - Dv)     dK += dS^T Q * scale     dQ += dS K * scale
//
// The reference accumulates dQ with fp32 atomicAdd from its key-stationary
// blocks (flash_bwd.cuh:434-443). Measured on MI355X, fp32 atomics sustain
// ~1.3 TB/s whatever their scope or locality, about 1/5 of plain stores, and
// at the headline shape that stream alone would outlast the whole backward.
// So dQ gets its own query-stationary pass that recomputes S and dP (7
// products per tile pair instead of 5, but no atomics, no dQ clearing, and a
// deterministic result), and both passes run in ONE launch:
//
//   workgroup (t, b*Hkv + hkv), 4 waves (numbered so that each kv head's
//   workgroups share one XCD and its L2):
//     phase 1: dK, dV for key rows [128t, 128t+128) of kv head hkv,
//              over all query heads of its group and all query tiles
//              (from the diagonal on when causal, flash_bwd.cuh:158-161)
//     phase 2: dQ for query rows [128t, 128t+128) of each query head of the
//              group, over all key tiles (up to the diagonal when causal)
//
// Under causal masking phase 1 shrinks with t while phase 2 grows with t, so
// the workgroups' total work is nearly equal without giving up parallelism.
//
// Both phases run on v_mfma_f32_32x32x16_f16 with 32 rows per wave. Phase 1
// keeps the workgroup's K and V rows resident in LDS (B operands) and each
// wave's dK^T/dV^T in accumulators; P and dS come out of the S/dP accumulators and feed
// dV^T += dO^T P and dK^T += Q^T dS directly, with the dO^T/Q^T operands read
// from the row-major LDS tiles by the LDS transpose read. Phase 2 mirrors the
// forward kernel: S^T = K Q^T and dP^T = V dO^T with Q, dO held as B
// operands, then dQ^T += K^T dS^T. Streamed tiles go from global memory
// straight into double-buffered, XOR-swizzled LDS tiles
// (global_load_lds_dwordx4). Dead lanes (causal col > row, ragged rows/cols
// >= N) contribute exactly zero (flash_bwd.cuh:267-282); tiles that contain
// any take a separate masked path. P and dS are rounded to fp16 only as MFMA
// operands.
#include "fa_device.h"
#include "fa_launch.h"

namespace fa {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTile = 32 * kWaves;  // rows a workgroup owns (keys in phase 1, queries in phase 2)
constexpr int kSub = 64;            // rows per streamed tile (queries in 1, keys in 2)

template <int D>
struct BwdLds {
  static constexpr int kTileHalves = kSub * D;
  static constexpr int kStageHalves = 2 * kTileHalves + 2 * kSub * 2;  // 2 tiles + lse2, dvec
  // Phase 1 also keeps the workgroup's K and V rows (kTile each) resident.
  static constexpr int kKVHalves = 2 * kTile * D;
  static constexpr int kBytes = (2 * kStageHalves + kKVHalves) * 2;
};

// ---------------------------------------------------------------------------
// Preprocess: dvec[row] = sum_d float(O[row,d]) * float(dO[row,d]) from the
// fp16-rounded O (flash_bwd.cuh:65-78), and lse2[row] = LSE[row] * log2(e),
// the form in which the main kernel consumes the saved LSE.
template <int D>
__global__ __launch_bounds__(256) void bwd_pre_kernel(const half_t* __restrict__ O,
                                                      const half_t* __restrict__ dO,
                                                      const float* __restrict__ Lse,
                                                      float* __restrict__ dvec,
                                                      float* __restrict__ lse2, long rows) {
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
  }
#pragma unroll
  for (int off = kLanesPerRow / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (row < rows && (tid % kLanesPerRow) == 0) {
    dvec[row] = acc;
    lse2[row] = Lse[row] * kLog2e;
  }
}

// Direct load of 64 consecutive floats (rows r0 .. r0+63, clamped to N-1).
__device__ __forceinline__ void vec_load64(float* lds, const float* g, int r0, int N, int lane) {
  const int r = min(r0 + lane, N - 1);
  __builtin_amdgcn_global_load_lds((const void*)(g + r),
                                   (__attribute__((address_space(3))) void*)lds, 4, 0, 0);
}

// The MFMA parts of every step run on one straight-line path; only the
// softmax-side VALU branches between its masked and unmasked forms. Keeping
// branches away from the MFMAs lets the compiler keep the loop-carried
// accumulators in place instead of copying them between register files on
// every iteration. Operand reads run one k-step ahead of the MFMAs that
// consume them, fenced so the scheduler does not hoist every read of the step
// (which costs more registers than the kernel has).

// ------------------------------- phase 1 -----------------------------------
template <int D, bool CAUSAL, bool BOUNDS>
struct KVWave {
  floatx16 dvacc[D / 32], dkacc[D / 32];

  // P and dS for one 32-row block m of the query tile, from the S and dP
  // accumulators; masked lanes (causal col > row, rows/cols >= N) give 0.
  template <bool MASK>
  __device__ __forceinline__ void pds(const floatx16& sacc, const floatx16& pacc,
                                      const float* lse2s, const float* dvs, int m, int i0,
                                      int j_col, int N, int h, float c, half8 (&pb)[2],
                                      half8 (&sb)[2]) {
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const floatx4 l4 = *reinterpret_cast<const floatx4*>(lse2s + 32 * m + 8 * g4 + 4 * h);
      const floatx4 d4 = *reinterpret_cast<const floatx4*>(dvs + 32 * m + 8 * g4 + 4 * h);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * g4 + e;
        float p = fast_exp2(fmaf(sacc[r], c, -l4[e]));
        if constexpr (MASK) {
          const int i = i0 + 32 * m + 8 * g4 + 4 * h + e;
          if ((CAUSAL && j_col > i) || (BOUNDS && (i >= N || j_col >= N))) p = 0.f;
        }
        pb[r >> 3][r & 7] = (half_t)p;
        sb[r >> 3][r & 7] = (half_t)(p * (pacc[r] - d4[e]));
      }
    }
  }

  // One 64-row query tile staged at (Qs, Os, lse2s, dvs), rows i0 .. i0+63,
  // against this wave's 32 key rows kr0 .. kr0+31 of the resident LDS tiles
  // (Kt, Vt). K and V are re-read from LDS rather than held in registers, so
  // the whole kernel stays within the MFMA's reach of VGPR accumulators.
  __device__ __forceinline__ void step(const half_t* Qs, const half_t* Os, const float* lse2s,
                                       const float* dvs, const half_t* Kt, const half_t* Vt,
                                       int kr0, int i0, int j_col, int N, int lane, float c,
                                       bool mask) {
    const int h = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      floatx16 sacc = zero16(), pacc = zero16();
      half8 aq = tile_read16<D>(Qs, m * 32 + l32, h), ao = tile_read16<D>(Os, m * 32 + l32, h);
      half8 bk = tile_read16<D>(Kt, kr0 + l32, h), bv = tile_read16<D>(Vt, kr0 + l32, h);
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) {
        half8 nq = aq, no = ao, nk = bk, nv = bv;
        if (kk + 1 < D / 16) {
          nq = tile_read16<D>(Qs, m * 32 + l32, 2 * kk + 2 + h);
          no = tile_read16<D>(Os, m * 32 + l32, 2 * kk + 2 + h);
          nk = tile_read16<D>(Kt, kr0 + l32, 2 * kk + 2 + h);
          nv = tile_read16<D>(Vt, kr0 + l32, 2 * kk + 2 + h);
        }
        sacc = mfma32(aq, bk, sacc);
        pacc = mfma32(ao, bv, pacc);
        __builtin_amdgcn_sched_barrier(0);
        aq = nq;
        ao = no;
        bk = nk;
        bv = nv;
      }
      half8 pb[2], sb[2];
      if (mask) pds<true>(sacc, pacc, lse2s, dvs, m, i0, j_col, N, h, c, pb, sb);
      else pds<false>(sacc, pacc, lse2s, dvs, m, i0, j_col, N, h, c, pb, sb);
      // dV^T += dO^T P, dK^T += Q^T dS; k-step q = query rows 32m+16q .. +15.
#pragma unroll
      for (int cb = 0; cb < D / 32; ++cb) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          dvacc[cb] = mfma32(tile_tr_operand<D>(Os, 32 * m + 16 * q, 32 * cb, lane), pb[q], dvacc[cb]);
          dkacc[cb] = mfma32(tile_tr_operand<D>(Qs, 32 * m + 16 * q, 32 * cb, lane), sb[q], dkacc[cb]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  }
};

// ------------------------------- phase 2 -----------------------------------
template <int D, bool CAUSAL, bool BOUNDS>
struct QWave {
  half8 qb[D / 16], ob[D / 16];  // this wave's Q, dO rows as B operands
  floatx16 qacc[D / 32];
  float lse2, dvv;

  template <bool MASK>
  __device__ __forceinline__ void ds(const floatx16& st, const floatx16& pt, int j0, int s,
                                     int i_row, int N, int h, float c, half8 (&sb)[2]) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float p = fast_exp2(fmaf(st[r], c, -lse2));
      if constexpr (MASK) {
        const int j = j0 + 32 * s + 8 * (r >> 2) + 4 * h + (r & 3);
        if ((CAUSAL && j > i_row) || (BOUNDS && j >= N)) p = 0.f;
      }
      sb[r >> 3][r & 7] = (half_t)(p * (pt[r] - dvv));
    }
  }

  // One 64-row key tile staged at (Ks, Vs), keys j0 .. j0+63.
  __device__ __forceinline__ void step(const half_t* Ks, const half_t* Vs, int j0, int i_row,
                                       int N, int lane, float c, bool mask) {
    const int h = lane >> 5, l32 = lane & 31;
    half8 sb[2][2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      floatx16 st = zero16(), pt = zero16();
      half8 ak = tile_read16<D>(Ks, s * 32 + l32, h), av = tile_read16<D>(Vs, s * 32 + l32, h);
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) {
        half8 nk = ak, nv = av;
        if (kk + 1 < D / 16) {
          nk = tile_read16<D>(Ks, s * 32 + l32, 2 * kk + 2 + h);
          nv = tile_read16<D>(Vs, s * 32 + l32, 2 * kk + 2 + h);
        }
        st = mfma32(ak, qb[kk], st);
        pt = mfma32(av, ob[kk], pt);
        __builtin_amdgcn_sched_barrier(0);
        ak = nk;
        av = nv;
      }
      if (mask) ds<true>(st, pt, j0, s, i_row, N, h, c, sb[s]);
      else ds<false>(st, pt, j0, s, i_row, N, h, c, sb[s]);
    }
    // dQ^T += K^T dS^T; k-step (s, q) = keys 32s+16q .. +15.
#pragma unroll
    for (int cb = 0; cb < D / 32; ++cb) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int q = 0; q < 2; ++q)
          qacc[cb] = mfma32(tile_tr_operand<D>(Ks, 32 * s + 16 * q, 32 * cb, lane), sb[s][q], qacc[cb]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
};

// ---------------------------------------------------------------------------
template <int D, bool CAUSAL, bool BOUNDS>
__global__ __launch_bounds__(kThreads) void bwd_kernel(
    const half_t* __restrict__ Q, const half_t* __restrict__ K,
    const half_t* __restrict__ V, const half_t* __restrict__ dO,
    const float* __restrict__ Lse2, const float* __restrict__ Dvec,
    float* __restrict__ dQ, half_t* __restrict__ dK, half_t* __restrict__ dV,
    int N, int Hq, int group, int n_tiles, int BHkv, float scale, float scale_log2) {
  using L = BwdLds<D>;
  extern __shared__ __align__(16) half_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5;
  const int l32 = lane & 31;

  const int wi = xcd_work_index(n_tiles * BHkv);
  if (wi < 0) return;
  const int bkv = wi / n_tiles;             // over B*Hkv
  const int t0 = (wi % n_tiles) * kTile;    // first row this workgroup owns
  const int Hkv = Hq / group;
  const int b = bkv / Hkv, hkv = bkv % Hkv;
  const size_t kv_off = (size_t)bkv * N * D;
  const half_t* Kh = K + kv_off;
  const half_t* Vh = V + kv_off;

  auto stage_ptr = [&](int st) { return smem + st * L::kStageHalves; };

  // =========================== phase 1: dK, dV ===========================
  {
    const int jw = t0 + wave * 32;  // this wave's key rows
    const int j_col = jw + l32;
    const bool col_ok = !BOUNDS || j_col < N;
    KVWave<D, CAUSAL, BOUNDS> w;
    half_t* Kt = smem + 2 * L::kStageHalves;  // stationary K, V rows t0 .. t0+kTile-1
    half_t* Vt = Kt + kTile * D;
    tile_load<D, kTile, kWaves>(Kt, Kh, t0, N, wave, lane);
    tile_load<D, kTile, kWaves>(Vt, Vh, t0, N, wave, lane);
#pragma unroll
    for (int cb = 0; cb < D / 32; ++cb) {
      w.dvacc[cb] = zero16();
      w.dkacc[cb] = zero16();
    }

    const int i_start = CAUSAL ? t0 : 0;  // t0 is a multiple of kSub
    const int n_qt = (N - i_start + kSub - 1) / kSub;
    const int n_it = group * n_qt;  // (query head, query tile) pairs, flattened

    auto fetch = [&](int it, half_t* st) {
      const int g = it / n_qt;
      const int i0 = i_start + (it % n_qt) * kSub;
      const size_t bhq = (size_t)b * Hq + (size_t)hkv * group + g;
      tile_load<D, kSub, kWaves>(st, Q + bhq * N * D, i0, N, wave, lane);
      tile_load<D, kSub, kWaves>(st + L::kTileHalves, dO + bhq * N * D, i0, N, wave, lane);
      float* fv = reinterpret_cast<float*>(st + 2 * L::kTileHalves);
      if (wave == 0) vec_load64(fv, Lse2 + bhq * N, i0, N, lane);
      if (wave == 1) vec_load64(fv + kSub, Dvec + bhq * N, i0, N, lane);
    };

    fetch(0, stage_ptr(0));
    wait_vmem();
    __syncthreads();
    for (int it = 0; it < n_it; ++it) {
      const int i0 = i_start + (it % n_qt) * kSub;
      if (it + 1 < n_it) fetch(it + 1, stage_ptr((it + 1) & 1));
      const half_t* Qs = stage_ptr(it & 1);
      const half_t* Os = Qs + L::kTileHalves;
      const float* lse2s = reinterpret_cast<const float*>(Os + L::kTileHalves);
      const float* dvs = lse2s + kSub;
      // Causal tiles wholly above a wave's keys give exact zeros through the
      // masked path; they occur only on the diagonal, so they are not skipped.
      const bool mask = (CAUSAL && i0 < jw + 31) || (BOUNDS && (i0 + kSub > N || jw + 32 > N));
      w.step(Qs, Os, lse2s, dvs, Kt, Vt, wave * 32, i0, j_col, N, lane, scale_log2, mask);
      wait_vmem();
      __syncthreads();
    }

    if (col_ok) {
      half_t* dkrow = dK + kv_off + (size_t)j_col * D;
      half_t* dvrow = dV + kv_off + (size_t)j_col * D;
#pragma unroll
      for (int cb = 0; cb < D / 32; ++cb) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          half4 k4, v4;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            k4[e] = (half_t)(w.dkacc[cb][4 * g4 + e] * scale);
            v4[e] = (half_t)w.dvacc[cb][4 * g4 + e];
          }
          *reinterpret_cast<half4*>(dkrow + cb * 32 + 8 * g4 + 4 * h) = k4;
          *reinterpret_cast<half4*>(dvrow + cb * 32 + 8 * g4 + 4 * h) = v4;
        }
      }
    }
  }

  // ============================== phase 2: dQ ==============================
  {
    const int iw = t0 + wave * 32;  // this wave's query rows
    const int i_row = iw + l32;
    const bool row_ok = !BOUNDS || i_row < N;
    const int kv_end = CAUSAL ? min(N, t0 + kTile) : N;
    const int n_kt = (kv_end + kSub - 1) / kSub;

    for (int g = 0; g < group; ++g) {
      const size_t bhq = (size_t)b * Hq + (size_t)hkv * group + g;
      const half_t* Qg = Q + bhq * N * D;
      const half_t* dOg = dO + bhq * N * D;
      QWave<D, CAUSAL, BOUNDS> w;
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) {
        w.qb[kk] = as_half8(load16(Qg + (size_t)i_row * D + kk * 16 + h * 8, row_ok));
        w.ob[kk] = as_half8(load16(dOg + (size_t)i_row * D + kk * 16 + h * 8, row_ok));
      }
      w.lse2 = row_ok ? Lse2[bhq * N + i_row] : 0.f;
      w.dvv = row_ok ? Dvec[bhq * N + i_row] : 0.f;
#pragma unroll
      for (int cb = 0; cb < D / 32; ++cb) w.qacc[cb] = zero16();

      tile_load<D, kSub, kWaves>(stage_ptr(0), Kh, 0, N, wave, lane);
      tile_load<D, kSub, kWaves>(stage_ptr(0) + L::kTileHalves, Vh, 0, N, wave, lane);
      wait_vmem();
      __syncthreads();
      for (int t = 0; t < n_kt; ++t) {
        const int j0 = t * kSub;
        if (t + 1 < n_kt) {
          half_t* nb = stage_ptr((t + 1) & 1);
          tile_load<D, kSub, kWaves>(nb, Kh, j0 + kSub, N, wave, lane);
          tile_load<D, kSub, kWaves>(nb + L::kTileHalves, Vh, j0 + kSub, N, wave, lane);
        }
        const half_t* Ks = stage_ptr(t & 1);
        const half_t* Vs = Ks + L::kTileHalves;
        const bool mask = (CAUSAL && j0 + kSub - 1 > iw) || (BOUNDS && j0 + kSub > N);
        w.step(Ks, Vs, j0, i_row, N, lane, scale_log2, mask);
        wait_vmem();
        __syncthreads();
      }

      if (row_ok) {
        float* qrow = dQ + bhq * N * D + (size_t)i_row * D;
#pragma unroll
        for (int cb = 0; cb < D / 32; ++cb) {
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            floatx4 v4;
#pragma unroll
            for (int e = 0; e < 4; ++e) v4[e] = w.qacc[cb][4 * g4 + e] * scale;
            *reinterpret_cast<floatx4*>(qrow + cb * 32 + 8 * g4 + 4 * h) = v4;
          }
        }
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
                     (const half_t*)a.o, (const half_t*)a.dO, a.lse, a.dvec, a.lse2, rows);
  return hipGetLastError();
}

template <int D, bool CAUSAL, bool BOUNDS>
hipError_t launch_main_t(const BwdArgs& a) {
  const int n_tiles = (a.N + kTile - 1) / kTile;
  const dim3 grid(xcd_grid(n_tiles * a.B * a.Hkv));
  const size_t smem = BwdLds<D>::kBytes;
  static const hipError_t attr = allow_lds(bwd_kernel<D, CAUSAL, BOUNDS>, smem);
  if (attr != hipSuccess) return attr;
  const float scale = 1.f / sqrtf((float)D);
  hipLaunchKernelGGL((bwd_kernel<D, CAUSAL, BOUNDS>), grid, dim3(kThreads), smem,
                     (hipStream_t)a.stream, (const half_t*)a.q, (const half_t*)a.k,
                     (const half_t*)a.v, (const half_t*)a.dO, a.lse2, a.dvec, a.dq,
                     (half_t*)a.dk, (half_t*)a.dv, a.N, a.Hq, a.Hq / a.Hkv, n_tiles,
                     a.B * a.Hkv, scale, scale * kLog2e);
  return hipGetLastError();
}

template <int D>
hipError_t launch_main_d(const BwdArgs& a) {
  const bool bounds = (a.N % kTile) != 0;  // kTile is a multiple of kSub
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
