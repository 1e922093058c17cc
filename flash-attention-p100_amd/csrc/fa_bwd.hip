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
//   workgroup (t, b*Hkv + hkv), 8 waves (numbered so that each kv head's
//   workgroups share one XCD and its L2):
//     phase 1: dK, dV for key rows [128t, 128t+128) of kv head hkv, over all
//              query heads of its group and all query tiles (from the
//              diagonal on when causal, flash_bwd.cuh:158-161). Wave w owns
//              key rows 32*(w%4) .. +31 and, of each staged 64-row query
//              tile, the 32-row half w/4; the two halves' dK/dV partials are
//              summed through LDS at the end.
//     phase 2: dQ for query rows [128t, 128t+128) of each query head of the
//              group, over all key tiles (up to the diagonal when causal).
//              Wave w owns query rows 32*(w%4) .. +31 and, of each staged
//              64-key tile, the 32-key half w/4; partials summed through LDS.
//
// Under causal masking phase 1 shrinks with t while phase 2 grows with t, so
// the workgroups' total work is nearly equal without giving up parallelism
// (phase-1 steps cost more than phase-2 steps, so the first key tiles also
// hand part of their phase 1 to the workgroup of tile n_tiles-1-t);
// 8 waves keep two waves on every SIMD at the headline shape, so one wave's
// softmax arithmetic overlaps the other's matrix products.
//
// Both phases run on v_mfma_f32_32x32x16_f16. Phase 1 keeps the workgroup's
// K and V rows resident (each wave's 32 K rows as MFMA operands in registers,
// V in LDS: both in registers would exceed the 256 registers a wave has at
// two waves per SIMD) and each wave's dK^T/dV^T in accumulators;
// P and dS come out of the S/dP accumulators and feed dV^T += dO^T P and
// dK^T += Q^T dS directly, with the dO^T/Q^T operands read from the
// row-major LDS tiles by the LDS transpose read. Phase 2 mirrors the forward
// kernel: S^T = K Q^T and dP^T = V dO^T with Q, dO held as B operands, then
// dQ^T += K^T dS^T. Streamed tiles go from global memory straight into
// double-buffered LDS tiles of whole, chunk-swizzled rows (buffer_load ...
// lds, 1 KB per instruction); the resident K/V use padded, row-permuted rows.
// Steps are straight-line code (masking is index arithmetic, compiled in only
// for causal / ragged instantiations): a branch around the MFMAs makes the
// compiler copy the loop-carried accumulators between register files on
// every iteration. Dead lanes (causal col > row, ragged rows/cols >= N)
// contribute exactly zero (flash_bwd.cuh:267-282). P and dS are rounded to
// fp16 only as MFMA operands.
#include <type_traits>

#include "fa_device.h"
#include "fa_launch.h"

namespace fa {
namespace {

constexpr int kTile = 128;  // rows a workgroup owns (keys in phase 1, queries in phase 2)
static_assert(kTile == kBwdTile, "workspace layout assumes this key tile");
// Waves per workgroup and rows per streamed tile (queries in phase 1, keys in
// phase 2) at tile width D. Four row blocks of 32 rows cover kTile; up to
// width 128 two waves share each row block, one per 32-row half of a 64-row
// streamed tile (two waves per SIMD). At width 256 one wave's dK^T and dV^T
// accumulators alone take 256 registers, so each row block has one wave (512
// registers per lane at one wave per SIMD), the streamed tiles have 32 rows
// and the K operands come straight from global memory into registers (a
// resident K tile would not fit in LDS beside V and the staged tiles).
// W4 (width 64, grids of at least two workgroups per CU): one wave per row
// block and 32-row streamed tiles as at width 256, but K resident in LDS and
// at most 256 registers per wave (the kernel needs ~170), so two workgroups
// (54 KB of LDS each) share a CU on separate barriers and one's softmax runs
// beside the other's products. Same-box A/B, bwd_main at H=16 N=4096 D=64
// causal: -4% (minimum) and -7% (median of five rounds); within 0.6% at
// H=16 N=4096 D=64 dense and at H=16/8 N=8192 D=64 causal; +17% at H=16
// N=2048 D=64 causal, whose 256 workgroups leave one per CU, so the launcher
// takes it only where the grid fills both slots. (At width 128 two such
// workgroups do not fit in LDS.)
template <int D, bool W4 = false>
struct BwdShape {
  static constexpr int kWaves = D > 128 || W4 ? 4 : 8;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kHalves = kWaves / 4;  // waves per row block
  static constexpr int kSub = 32 * kHalves;
  static constexpr bool kKGlobal = D > 128;   // K operands loaded from global memory
};
constexpr int kVecStride = 64;  // floats per staged lse2 / dvec run (>= every kSub)
// Causal split of key tile u (see bwd_kernel): floor((group * (n_tiles-1-2u) *
// kSplitNum - kSplitBias) / 256) of its phase-1 iterations move to workgroup
// n_tiles-1-u. Phase-1 steps cost more than phase-2 steps, so the iterations
// move from the phase-1-heavy low tiles to the phase-2-heavy high ones. Swept
// over 50..110 (same-box A/B) with phase 2's operands read ahead: fastest at
// 76..86 for B=1 H=8 N=4096 D=128, 66..76 for H=16 N=2048 D=64 and 76 for
// H=16 N=8192 D=128; 110 lost everywhere (the best rate had been ~50 before
// phase-2 steps got cheaper). With phase 1's operands read ahead too, 66 beat
// 76 and 86 on all three shapes by 0.4-1.7%. Re-swept (56..96) once phase 2
// (and phase 1 at D <= 64) took the causal test on diagonal steps only: 86
// beat 66 by 1.8% at B=1 H=8 N=4096 D=128, within noise at H=16 N=4096
// D=64, H=16 N=8192 D=128 and H=16 N=2048 D=64.
constexpr int kSplitNum = 86;
constexpr int kSplitBias = 5;
// The same rate for the W4 shape (below): swept 65..130 at H=16 N=4096 D=64
// causal (two boxes): 100 beat 86 by 1.4%, 115 and 130 lost; at H=16/8
// N=8192 D=64 within 0.7%.
constexpr int kSplitNumW4 = 100;
// The FEAT bit that selects W4 (kept clear of the per-score input bits).
constexpr int kBwdW4 = 16;

// LDS: every tile is its own __shared__ object (declared in bwd_kernel), so
// the compiler can tell that a step's reads never touch the tiles that the
// next step's direct loads are filling and does not wait for those loads.
template <int D, bool W4 = false>
struct BwdLds {
  using Sh = BwdShape<D, W4>;
  static constexpr int kTileHalves = Stream<D>::template bytes<Sh::kSub>() / 2;  // staged tile
  static constexpr int kKVTileHalves = Tile<D>::template halves<kTile>();  // resident V
  static constexpr int kKTileHalves = Sh::kKGlobal ? 512 : kKVTileHalves;  // resident K
  // Partial-sum exchange regions between the two waves of a row block (they
  // reuse the tiles once a phase's loop is done): D/32 accumulators x 16
  // floats per lane for one wave.
  static constexpr int kRegionBytes = (D / 32) * 16 * 64 * 4;
  static_assert(Sh::kHalves == 1 ||
                    (kRegionBytes <= kTileHalves * 2 && 2 * kRegionBytes <= kKTileHalves * 2),
                "exchange regions exceed the tiles");
};

// Lanes per row of the preprocess: D/8 rounded up to a power of two (the
// row sum is a butterfly over them; lanes past D/8 add zeros).
constexpr int pre_lanes_per_row(int D) { return D / 8 <= 8 ? 8 : D / 8 <= 16 ? 16 : 32; }

// ---------------------------------------------------------------------------
// Preprocess: dvec[row] = sum_d float(O[row,d]) * float(dO[row,d]) from the
// fp16-rounded O (flash_bwd.cuh:65-78), and lse2[row] = LSE[row] * log2(e),
// the form in which the main kernel consumes the saved LSE.
template <int D, bool BF>
__global__ __launch_bounds__(256) void bwd_pre_kernel(const half_t* __restrict__ O,
                                                      const half_t* __restrict__ dO,
                                                      const float* __restrict__ Lse,
                                                      float* __restrict__ dvec,
                                                      float* __restrict__ lse2, long rows,
                                                      int Hq, int N, Strides st,
                                                      unsigned* __restrict__ counters,
                                                      int n_counters, int dr) {
  constexpr int kLanesPerRow = pre_lanes_per_row(D);
  constexpr int kRowsPerBlock = 256 / kLanesPerRow;
  const int tid = threadIdx.x;
  // The main kernel's split-tile counters start at zero (it leaves them zero,
  // but a fresh workspace holds anything). n_counters < rows <= threads.
  if (const long c = (long)blockIdx.x * 256 + tid; c < n_counters) counters[c] = 0u;
  const long row = (long)blockIdx.x * kRowsPerBlock + tid / kLanesPerRow;
  const int c8 = (tid % kLanesPerRow) * 8;
  float acc = 0.f;
  if (row < rows && c8 < dr) {
    // row = (b * Hq + hq) * N + n over the dense (B, Hq, N) vectors.
    const long bh = row / N, n = row - bh * N;
    const size_t off = (size_t)((bh / Hq) * st.b + (bh % Hq) * st.h + n * st.n) + c8;
    const half8 o = as_half8(*reinterpret_cast<const u32x4*>(O + off));
    const half8 g = as_half8(*reinterpret_cast<const u32x4*>(dO + off));
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += from16<BF>(o[e]) * from16<BF>(g[e]);
  }
#pragma unroll
  for (int off = kLanesPerRow / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (row < rows && (tid % kLanesPerRow) == 0) {
    dvec[row] = acc;
    lse2[row] = Lse[row] * kLog2e;
  }
}

// Direct load of 64 consecutive floats (rows r0 .. r0+63 of a per-row
// vector; rows past its end read as zeros).
__device__ __forceinline__ void vec_load64(float* lds, rsrc_t r, int r0, int lane) {
  lds_direct_buf<4>(lds, r, (uint32_t)lane * 4u, (uint32_t)r0 * 4u);
}

// Exchange of per-wave accumulators: waves of the upper half (w >= 4) store
// accumulators [k0, k0 + n) into a region, waves w-4 add them. Layout
// [k][g4][lane] x 4 floats, bank-conflict-free 16-byte accesses.
template <int n, int N_ACC>
__device__ __forceinline__ void partial_store(float* region, const floatx16 (&acc)[N_ACC], int k0,
                                              int lane) {
#pragma unroll
  for (int k = 0; k < n; ++k)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const floatx16& a = acc[k0 + k];
      const floatx4 v = {a[4 * g4], a[4 * g4 + 1], a[4 * g4 + 2], a[4 * g4 + 3]};
      *reinterpret_cast<floatx4*>(region + ((k * 4 + g4) * 64 + lane) * 4) = v;
    }
}
template <int n, int N_ACC>
__device__ __forceinline__ void partial_add(const float* region, floatx16 (&acc)[N_ACC], int k0,
                                            int lane) {
#pragma unroll
  for (int k = 0; k < n; ++k)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const floatx4 v = *reinterpret_cast<const floatx4*>(region + ((k * 4 + g4) * 64 + lane) * 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[k0 + k][4 * g4 + e] += v[e];
    }
}

// A split key tile's partial dK^T/dV^T pass between two workgroups through a
// workspace slot. They may run on different XCDs, whose L2 caches are not
// coherent with each other, so the slot is written and read with
// device-coherent accesses (cache policy sc1: stores write through to the
// device-coherent level before they count as complete, loads bypass
// non-coherent copies). Slot layout [w4][k][g4][lane] x 4 floats: every
// instruction moves 1 KB of consecutive bytes.
constexpr int kDeviceCoherent = 16;  // sc1 bit of the buffer intrinsics' cache-policy operand
template <int n>
__device__ __forceinline__ void slot_store(rsrc_t r, const floatx16 (&acc)[n], int w4, int lane) {
#pragma unroll
  for (int k = 0; k < n; ++k)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const floatx4 v = {acc[k][4 * g4], acc[k][4 * g4 + 1], acc[k][4 * g4 + 2], acc[k][4 * g4 + 3]};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, lane * 16,
                                             ((w4 * n + k) * 4 + g4) * 1024, kDeviceCoherent);
    }
}
template <int n>
__device__ __forceinline__ void slot_add(rsrc_t r, floatx16 (&acc)[n], int w4, int lane) {
#pragma unroll
  for (int k = 0; k < n; ++k)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const floatx4 v = __builtin_bit_cast(
          floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16,
                                                         ((w4 * n + k) * 4 + g4) * 1024,
                                                         kDeviceCoherent));
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[k][4 * g4 + e] += v[e];
    }
}

// ------------------------------- phase 1 -----------------------------------
// acc[0 .. D/32) = dV^T blocks, acc[D/32 .. 2D/32) = dK^T blocks.
// KREG: K's operands stay in registers (kb); otherwise each step reads them
// from the resident K tile, as V's. The copies with a mask, dropout or a bias
// read K from LDS: with it in registers they spill half of kb at D = 128,
// and each reload's wait (loads complete in issue order) also waits for the
// next stage's loads.
// SPLIT (masked instantiations with a boolean mask or a block layout): the
// per-score tests run in a softmax copy of their own, taken only by steps that
// hide a score. (The block-layout copies split too, so that a layout and the
// equivalent element mask run the same arithmetic on visible blocks.)
template <int D, bool CAUSAL, bool BOUNDS, bool BF, bool KREG = true, bool SPLIT = false>
struct KVWave {
  floatx16 acc[2 * (D / 32)];
  half8 kb[KREG ? D / 16 : 1];  // this wave's 32 key rows of K as B operands (loop-invariant)

  // Query rows i0 + 32m .. +31 (m = this wave's half of the staged tile)
  // against key rows kr0 .. kr0+31 (K from kb, V from the resident tile Vt).
  // mtw: the mask bits of key j_col for this step's 32 query rows i0 + 32m ..
  // (bit = row offset; all set without a mask).
  // bv: the step's bias values, replaced by `bnext()` (the next step's) as
  // soon as they are added, so one set of registers carries the prefetch.
  template <class BiasNext>
  __device__ __forceinline__ void step(const half_t* Qs, const half_t* Os, const float* lse2s,
                                       const float* dvs, const half_t* Vt, const half_t* Kt,
                                       int m, int kr0, int i0, int j_col, int row_lo, int row_end,
                                       float alibi_raw, uint32_t mtw, uint32_t ztw, float zs,
                                       floatx16& bv, const BiasNext& bnext, float bias_raw,
                                       int lane, int roff,
                                       const typename Stream<D>::Offsets& so, float c) {
    using S = Stream<D>;
    const int h = lane >> 5;
    floatx16 sacc = zero16(), pacc = zero16();
    // Operands read one k-step ahead of their products.
    half8 qa = S::read16(Qs, so, 0), oa = S::read16(Os, so, 0);
    half8 va = tile_read16<D>(Vt, kr0, 0, roff);
    half8 ka = KREG ? kb[0] : tile_read16<D>(Kt, kr0, 0, roff);
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      half8 qn = qa, on = oa, vn = va, kn = ka;
      if (kk + 1 < D / 16) {
        qn = S::read16(Qs, so, kk + 1);
        on = S::read16(Os, so, kk + 1);
        vn = tile_read16<D>(Vt, kr0, kk + 1, roff);
        if constexpr (!KREG) kn = tile_read16<D>(Kt, kr0, kk + 1, roff);
      }
      __builtin_amdgcn_sched_barrier(0);
      sacc = mfma16<BF>(qa, KREG ? kb[kk] : ka, sacc);
      pacc = mfma16<BF>(oa, va, pacc);
      qa = qn;
      oa = on;
      va = vn;
      ka = kn;
    }
    // P and dS. A lane holds key column j_col and the 16 query rows
    // i = i0 + 32m + 8*g4 + 4h + e; rows from row_end on are masked: past N,
    // past the key's sliding window, or all of them for a key past the
    // entry's key length (its dK/dV rows are stored, as zeros).
    const int base = i0 + 32 * m + 4 * h;
    const int lo = row_lo - base;    // alive when 8*g4 + e >= lo (causal: row_lo = j_col)
    const int hi = row_end - base;   // alive when 8*g4 + e <  hi
    if (BOUNDS && alibi_raw != 0.f) {  // ALiBi: -slope |i - j| in raw-score units
      const float d0 = (float)(base - j_col);
#pragma unroll
      for (int r = 0; r < 16; ++r)
        sacc[r] = fmaf(-alibi_raw, fabsf(d0 + (float)(8 * (r >> 2) + (r & 3))), sacc[r]);
    }
    if (BOUNDS && bias_raw != 0.f) {  // attention bias of the 16 (row, j_col) in raw units
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] = fmaf(bv[r], bias_raw, sacc[r]);
      bv = bnext();
    }
    half8 pb[2], sb[2];
    // This lane's rows are bits idx + 4h of the mask and dropout words:
    // shifted once, every per-score bit position is a constant.
    const uint32_t mth = mtw >> (4 * h), zth = ztw >> (4 * h);
    // At D <= 64 the causal test runs only where some lane's rows start above
    // its key (lo > 0), in a copy a wave ballot picks (measured 2% faster at
    // D = 64); at D = 128 a second copy spilled registers and ran 4% slower.
    // With a mask (SPLIT) the per-score tests run only where some lane has a
    // hidden row (before its left bound, from its row end on, or a clear mask
    // bit; idx runs over 0..3, 8..11, 16..19, 24..27), in a copy the same kind
    // of ballot picks: most steps of a mask hide nothing (C3 shape with an
    // all-true mask: 19% -> 7% over the plain backward). The other masked
    // instantiations keep one copy: a second one spilled registers at D = 128.
    const bool open = lo <= 0 && hi >= 28 && (mth & 0x0F0F0F0Fu) == 0x0F0F0F0Fu;
    const bool edge = SPLIT    ? __builtin_amdgcn_ballot_w64(!open) != 0
                      : BOUNDS ? true
                               : D > 64 || (CAUSAL && __builtin_amdgcn_ballot_w64(lo > 0) != 0);
    auto softmax = [&](auto edge_tag) {
      constexpr bool EDGE = decltype(edge_tag)::value;
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const floatx4 l4 = *reinterpret_cast<const floatx4*>(lse2s + 32 * m + 8 * g4 + 4 * h);
        const floatx4 d4 = *reinterpret_cast<const floatx4*>(dvs + 32 * m + 8 * g4 + 4 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g4 + e, idx = 8 * g4 + e;
          float p = fast_exp2(fmaf(sacc[r], c, -l4[e]));
          if (EDGE && (CAUSAL || BOUNDS)) p = (idx >= lo) ? p : 0.f;
          if (EDGE && BOUNDS) p = (idx < hi && ((mth >> idx) & 1u)) ? p : 0.f;
          // Dropout (keep bits ztw, scale zs): dV sees the kept P, and the
          // gradient of P is the kept dP scaled.
          const bool keep = (zth >> idx) & 1u;
          pb[r >> 3][r & 7] = to16<BF>(keep ? p : 0.f);
          sb[r >> 3][r & 7] = to16<BF>(p * ((keep ? pacc[r] * zs : 0.f) - d4[e]));
        }
      }
    };
    if (edge) softmax(std::true_type{});
    else softmax(std::false_type{});
    // dV^T += dO^T P, dK^T += Q^T dS; k-step q = query rows 32m+16q .. +15.
#pragma unroll
    for (int cb = 0; cb < D / 32; ++cb)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        acc[cb] = mfma16<BF>(S::tr_operand(Os, q, so, cb), pb[q], acc[cb]);
        acc[D / 32 + cb] = mfma16<BF>(S::tr_operand(Qs, q, so, cb), sb[q], acc[D / 32 + cb]);
      }
  }
};

// ------------------------------- phase 2 -----------------------------------
template <int D, bool CAUSAL, bool BOUNDS, bool BF, bool SPLIT = false>
struct QWave {
  half8 qb[D / 16], ob[D / 16];  // this wave's Q, dO rows as B operands
  floatx16 acc[D / 32];          // dQ^T blocks
  float lse2, dvv;

  // Keys j0 + 32s .. +31 (s = this wave's half of the staged 64-key tile).
  // mw: row i_row's mask bits for keys j0 + 32s .. (all set without a mask).
  // bv: as in KVWave::step.
  template <class Issue, class BiasNext>
  __device__ __forceinline__ void step(const half_t* Ks, const half_t* Vs, int s, int j0,
                                       int i_row, int Nk, int key_lo, float alibi_raw,
                                       uint32_t mw, uint32_t zw, float zs, floatx16& bv,
                                       const BiasNext& bnext, float bias_raw, float* dbrow,
                                       bool db_x4, int lane,
                                       const typename Stream<D>::Offsets& so, float c,
                                       const Issue& issue) {
    using S = Stream<D>;
    const int h = lane >> 5;
    floatx16 st = zero16(), pt = zero16();
    // Operands are read one k-step ahead of their products, so that no
    // product waits for its own LDS read.
    half8 ka = S::read16(Ks, so, 0), va = S::read16(Vs, so, 0);
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      half8 kn = ka, vn = va;
      if (kk + 1 < D / 16) {
        kn = S::read16(Ks, so, kk + 1);
        vn = S::read16(Vs, so, kk + 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      st = mfma16<BF>(ka, qb[kk], st);
      pt = mfma16<BF>(va, ob[kk], pt);
      issue(kk);
      ka = kn;
      va = vn;
    }
    // dS^T. A lane holds query row i_row and the 16 keys
    // j = j0 + 32s + 8*g4 + 4h + e. Rows i_row >= N are never stored.
    const int base = j0 + 32 * s + 4 * h;
    const int lo = i_row - base;   // alive when 8*g4 + e <= lo (causal)
    const int hi = Nk - base;      // alive when 8*g4 + e <  hi (ragged N, key length)
    const int lw = key_lo - base;  // alive when 8*g4 + e >= lw (sliding window)
    if (BOUNDS && alibi_raw != 0.f) {  // ALiBi: -slope |i - j| in raw-score units
      const float d0 = (float)(i_row - base);
#pragma unroll
      for (int r = 0; r < 16; ++r)
        st[r] = fmaf(-alibi_raw, fabsf(d0 - (float)(8 * (r >> 2) + (r & 3))), st[r]);
    }
    if (BOUNDS && bias_raw != 0.f) {  // attention bias of the 16 (i_row, key) in raw units
#pragma unroll
      for (int r = 0; r < 16; ++r) st[r] = fmaf(bv[r], bias_raw, st[r]);
      bv = bnext();
    }
    half8 sb[2];
    floatx4 ds4;  // the current run of four keys' dS (16-byte dbias stores)
    const uint32_t mwh = mw >> (4 * h), zwh = zw >> (4 * h);  // as in KVWave::step
    // The causal test changes nothing unless one of some lane's 16 keys lies
    // past its row (lo < 27, the largest idx): only the diagonal steps take
    // it, in a copy a wave ballot picks (measured 1.6% faster at D = 64 and
    // at N = 8192, neutral at B=1 H=8 N=4096 D=128). With a mask (SPLIT) all
    // per-score tests run in that copy, picked where some lane has a hidden
    // key (as in KVWave::step); the other masked instantiations always test.
    const bool open = (!CAUSAL || lo >= 27) && hi >= 28 && lw <= 0 &&
                      (mwh & 0x0F0F0F0Fu) == 0x0F0F0F0Fu;
    const bool edge = SPLIT    ? __builtin_amdgcn_ballot_w64(!open) != 0
                      : BOUNDS ? true
                               : CAUSAL && __builtin_amdgcn_ballot_w64(lo < 27) != 0;
    auto softmax = [&](auto edge_tag) {
      constexpr bool EDGE = decltype(edge_tag)::value;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int idx = 8 * (r >> 2) + (r & 3);
        float p = fast_exp2(fmaf(st[r], c, -lse2));
        if (CAUSAL && EDGE) p = (idx <= lo) ? p : 0.f;
        if (BOUNDS && EDGE) p = (idx < hi && idx >= lw && ((mwh >> idx) & 1u)) ? p : 0.f;
        // Dropout: the gradient of P is the kept dP scaled by zs.
        const bool keep = (zwh >> idx) & 1u;
        const float ds = p * ((keep ? pt[r] * zs : 0.f) - dvv);
        sb[r >> 3][r & 7] = to16<BF>(ds);
        // The bias's gradient is dS itself; keys from the key length on are not
        // stored, except that a 16-byte run (db_x4: N % 4 == 0 and an aligned
        // plane, so no run crosses N) starting before it stores its masked
        // keys' zeros.
        ds4[r & 3] = ds;
        if (BOUNDS && dbrow) {
          if (db_x4) {
            if ((r & 3) == 3 && idx - 3 < hi)
              *reinterpret_cast<floatx4*>(dbrow + base + idx - 3) = ds4;
          } else if (idx < hi) {
            dbrow[base + idx] = ds;
          }
        }
      }
    };
    if (edge) softmax(std::true_type{});
    else softmax(std::false_type{});
    // dQ^T += K^T dS^T; k-step q = keys 32s+16q .. +15 (operands one ahead).
    half8 kt = S::tr_operand(Ks, 0, so, 0);
#pragma unroll
    for (int u = 0; u < 2 * (D / 32); ++u) {
      const int cb = u >> 1, q = u & 1;
      half8 kt_next = kt;
      if (u + 1 < 2 * (D / 32)) kt_next = S::tr_operand(Ks, (u + 1) & 1, so, (u + 1) >> 1);
      __builtin_amdgcn_sched_barrier(0);
      acc[cb] = mfma16<BF>(kt, sb[q], acc[cb]);
      kt = kt_next;
    }
  }
};

// ---------------------------------------------------------------------------
// FEAT: the optional per-score inputs compiled in (Feat, with BOUNDS).
template <int D, bool CAUSAL, bool BOUNDS, int FEAT, bool BF>
__global__ __launch_bounds__((BwdShape<D, (FEAT & kBwdW4) != 0>::kThreads))
__attribute__((amdgpu_waves_per_eu((FEAT & kBwdW4) != 0 ? 2 : 1))) void bwd_kernel(
    const half_t* __restrict__ Q, const half_t* __restrict__ K,
    const half_t* __restrict__ V, const half_t* __restrict__ dO,
    const float* __restrict__ Lse2, const float* __restrict__ Dvec,
    float* __restrict__ dQ, half_t* __restrict__ dQh, half_t* __restrict__ dK,
    half_t* __restrict__ dV,
    int N, int Hq, int group, int n_tiles, int BHkv, float scale, float scale_log2,
    Strides stq, Strides stk, unsigned* __restrict__ counters, float* __restrict__ slots,
    int split_num, int split_bias, const int* __restrict__ kv_len, int window,
    const float* __restrict__ alibi, const int* __restrict__ seg_start,
    const int* __restrict__ seg_end, const uint32_t* __restrict__ mask,
    const uint32_t* __restrict__ mask_t, int mask_heads, const uint32_t* __restrict__ drop,
    const uint32_t* __restrict__ drop_t, float drop_scale, const float* __restrict__ bias,
    long long bias_sb, long long bias_sh, float bias_raw, float* __restrict__ dbias, int dr,
    int NK, const int* __restrict__ block_rows, const int* __restrict__ block_cols) {
  constexpr bool W4 = (FEAT & kBwdW4) != 0;
  constexpr int FI = FEAT & ~kBwdW4;  // the per-score inputs
  using Sh = BwdShape<D, W4>;
  using L = BwdLds<D, W4>;
  constexpr int kWaves = Sh::kWaves, kHalves = Sh::kHalves;
  constexpr int kSub = Sh::kSub;
  constexpr bool KG = Sh::kKGlobal;
  constexpr int kSlotFloats = kTile * D * 2;  // one workgroup's dK^T and dV^T
  // Two stages of (first tile, second tile, lse2 | dvec), and the resident K, V.
  // The larger alignment makes the compiler place the four staged tiles first,
  // in the low 64 KB of LDS, where the tile base fits the 16-bit immediate of
  // ds_read; each read is then one per-lane offset register plus a constant.
  __shared__ __align__(1024) half_t ta0[L::kTileHalves], tb0[L::kTileHalves];
  __shared__ __align__(1024) half_t ta1[L::kTileHalves], tb1[L::kTileHalves];
  __shared__ __align__(16) float vec0[2 * kVecStride], vec1[2 * kVecStride];
  __shared__ __align__(16) half_t kres[L::kKTileHalves], vres[L::kKVTileHalves];
  __shared__ unsigned xflag;  // a split tile's counter, as one thread read it

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar M0 bases
  __builtin_assume(wave >= 0 && wave < kWaves);
  const int w4 = wave & 3;     // row block (keys in phase 1, queries in phase 2)
  const int half = wave >> 2;  // which 32-row half of each streamed tile (0 with one wave)
  const int h = lane >> 5;
  const int l32 = lane & 31;

  const int wi = xcd_work_index(n_tiles * BHkv);
  if (wi < 0) return;
  const int bkv = wi / n_tiles;  // over B*Hkv
  const int Hkv = Hq / group;
  const int b = bkv / Hkv, hkv = bkv % Hkv;
  // Per-entry key length (key padding), clamped to [1, NK] (NK: key rows, N:
  // query rows). kofs = NK - N: causal masking aligns the last query row with
  // the last key row, so query i sees key j iff j <= i + kofs. Workgroup t
  // runs phase 1 for key tile t when there is one and phase 2 for query
  // tile t when there is one.
  const int Nk = kv_len ? min(max(kv_len[b], 1), NK) : NK;
  const int kofs = NK - N;
  const int n_ktiles = (NK + kTile - 1) / kTile, n_qtiles = (N + kTile - 1) / kTile;
  // Causal sliding window (only in the masked instantiation): row i sees keys
  // (i - Wb, i]; 0 = none.
  const int Wb = BOUNDS ? window : 0;
  // Packed sequences (masked instantiation only): token i's sequence is
  // [sst[i], sen[i]). With a window they bound the rows and keys each
  // token reaches: key j reaches rows [j, upper(j)) and row i keys
  // [lower(i), i]; both bounds never decrease, and are clamped so that every
  // token reaches itself and no index leaves [0, N].
  const int* const sst = BOUNDS && seg_start ? seg_start + (size_t)b * N : nullptr;
  const int* const sen = BOUNDS && seg_end ? seg_end + (size_t)b * N : nullptr;
  const bool narrowed = BOUNDS && (Wb > 0 || sst != nullptr);
  auto upper = [&](int j) {
    j = min(j, NK - 1);
    int hi = Wb > 0 ? min(N, j - kofs + Wb) : N;
    if (sen) hi = min(hi, max(sen[j], j + 1));
    return hi;
  };
  auto lower = [&](int i) {
    i = min(i, N - 1);
    int lo = Wb > 0 ? i + kofs - Wb + 1 : 0;
    if (sst) lo = max(lo, min(sst[i], i));
    return max(lo, 0);
  };
  // Without causal masking, packed sequences also bound each row's keys from
  // above (row i sees keys below row_hi(i)) and each key's rows from below
  // (key j reaches rows from col_lo(j) on); both never decrease.
  const bool packed_nc = BOUNDS && !CAUSAL && sst != nullptr;
  auto row_hi = [&](int i) {
    i = min(i, N - 1);
    return packed_nc ? min(Nk, max(sen[i], i + 1)) : Nk;
  };
  auto col_lo = [&](int j) {
    j = min(j, N - 1);
    return packed_nc ? max(0, min(sst[j], j)) : 0;
  };
  const size_t kv_off = (size_t)(b * stk.b + hkv * stk.h);
  const rsrc_t rk = rows_rsrc(K + kv_off, NK, stk.n, dr), rv = rows_rsrc(V + kv_off, NK, stk.n, dr);
  // Offset of query head hq's row 0 in Q, dO, dQ.
  auto q_off = [&](int hq) { return (size_t)(b * stq.b + hq * stq.h); };
  constexpr bool MASKB = Feat<FI>::kMask, DROPB = Feat<FI>::kDrop, BIAS = Feat<FI>::kBias;
  // Block-sparse layout (SPARSE instantiations): nb blocks of kSparseBlock
  // rows (= kTile) per side, kSpb streamed tiles per block. Phase 1 steps
  // over the (query head, query block) pairs listed for its key block, phase
  // 2 over the key blocks listed for its query block; the masks below work
  // on row and key indices, so each step is masked as its position needs.
  constexpr bool SPARSE = Feat<FI>::kBlock;
  // Masked instantiations whose per-score tests run in a softmax copy of
  // their own (KVWave, QWave): all but the bias copy at the causal shapes and
  // the narrow widths; at D = 128 without causal masking only the mask and
  // block-layout copies (the others spilled registers with a second copy).
  constexpr bool kSplit = BOUNDS && !BIAS && (MASKB || SPARSE || CAUSAL || D <= 96);
  constexpr int kSpb = kSparseBlock / kSub;
  static_assert(kSparseBlock == kTile, "a workgroup's rows are one block of the layout");
  const int nb = (N + kSparseBlock - 1) / kSparseBlock;
  // Arbitrary mask (MASKB instantiations): query head hq's bit plane,
  // rows of W32 words, row-major (phase 2: row = query) or transposed (phase
  // 1: row = key). Word indices are clamped (bits past N are masked anyway).
  const int W32 = (N + 31) >> 5;
  auto plane = [&](const uint32_t* m, int hq) {
    return m + ((size_t)b * mask_heads + (mask_heads == 1 ? 0 : hq)) * N * W32;
  };
  // Dropout keep bits (DROPB instantiations): one plane per (b, query head),
  // in the mask's two layouts; zs scales the kept probabilities.
  auto zplane = [&](const uint32_t* z, int hq) { return z + ((size_t)b * Hq + hq) * N * W32; };
  const float zs = DROPB ? drop_scale : 1.f;
  // Attention bias (BIAS instantiation; bias null: none), raw-score factor
  // bias_raw = 1/scale; its gradient dbias, dense (B, Hq, N, N).
  const bool has_bias = BIAS && bias != nullptr;
  const float braw = has_bias ? bias_raw : 0.f;
  auto bplane = [&](int hq) { return bias + b * bias_sb + hq * bias_sh; };
  const int roff = row_lane_off<D>(lane);  // resident tiles (padded rows)
  typename Stream<D>::Offsets so;          // staged tiles, rows 32*half ..
  so.init(lane, 32 * half);

  StreamPlan<D, kSub, kWaves> plan_q, plan_k;  // staged tiles of Q/dO (phase 1), K/V (2)
  plan_q.init(wave, lane, stq.n, dr);
  plan_k.init(wave, lane, stk.n, dr);
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  // 16 KB-class exchange regions (two waves per row block only): the four
  // staged tiles, then the halves of the resident ones.
  auto region = [&](int i) -> float* {
    half_t* t = i == 0 ? ta0 : i == 1 ? tb0 : i == 2 ? ta1 : i == 3 ? tb1
              : i == 4 ? kres : i == 5 ? kres + L::kKVTileHalves / 2
              : i == 6 ? vres : vres + L::kKVTileHalves / 2;
    return reinterpret_cast<float*>(t);
  };

  // =========================== phase 1: dK, dV ===========================
  // Causal balance: phase 1 of key tile u costs more than phase 2 of query
  // tile u saves, so the workgroups of the first tiles would finish last. Key
  // tile u < n_tiles-1-u hands the last split(u) of its (query head, query
  // tile) iterations to the workgroup of tile n_tiles-1-u, which runs them
  // before its own tile. The two partial dK/dV sums meet in a workspace slot:
  // whichever workgroup finishes second adds the other's partial to its own
  // and stores the result (fp32 a + b == b + a, so the outcome does not depend
  // on which one that is).
  // Query rows of key tile u's phase 1: from its diagonal (causal) to the end,
  // or to the last row whose window or sequence reaches the tile.
  auto q_end = [&](int u) { return narrowed ? upper(u * kTile + kTile - 1) : N; };
  // ... and from its diagonal (causal) or the start of its first key's
  // sequence, rounded down to a streamed tile (u * kTile is a multiple of kSub).
  auto q_start = [&](int u) {
    return CAUSAL ? max(0, u * kTile - kofs) / kSub * kSub : col_lo(u * kTile) / kSub * kSub;
  };
  // (none when no query row reaches the tile: with more key rows than query
  // rows and a window, or more query rows than key rows, q_end < q_start)
  auto n_iters = [&](int u) {
    return group * max(0, (q_end(u) - q_start(u) + kSub - 1) / kSub);
  };
  auto split = [&](int u) {
    // (not at width 256: a second inlined copy of phase 1 spilled registers;
    // not with a block layout, whose key tiles have no common amount of work)
    if constexpr (KG || SPARSE) return 0;
    const int m = n_tiles - 1 - 2 * u;
    // windows leave the tiles' work equal; with kofs != 0 the key and query
    // tiles do not pair up
    if (!CAUSAL || m <= 0 || narrowed || kofs != 0) return 0;
    return max(0, min((group * m * split_num - split_bias) >> 8, n_iters(u) - 1));
  };
  const int tw = wi % n_tiles;
  const int partner = n_tiles - 1 - tw;
  const int x_help = partner < tw ? split(partner) : 0;  // run first, for tile `partner`
  const int x_own = tw < partner ? split(tw) : 0;        // given to workgroup `partner`
  const int pairs = n_tiles / 2;
  // One inlined copy per item: a loop over the two items made the compiler
  // keep fewer LDS operands in flight in the step (8% slower).
  auto run_item = [&](const bool helping) {
    const int tile = helping ? partner : tw;
    const int tp0 = tile * kTile;  // first key row of this item
    const int jw = tp0 + w4 * 32;  // this wave's key rows
    const int j_col = jw + l32;
    // Block-sparse: the pairs attending this key block (count first); step
    // `it` runs streamed tile it % kSpb of the (it / kSpb)-th pair.
    const int* const clist =
        SPARSE ? block_cols + ((size_t)bkv * nb + tile) * (group * nb + 1) : nullptr;
    const int n_it = SPARSE ? clist[0] * kSpb : n_iters(tile);
    const int it_begin = helping ? n_it - x_help : 0;
    const int it_end = helping ? n_it : n_it - x_own;
    const bool shared = helping || x_own > 0;
    KVWave<D, CAUSAL, BOUNDS, BF, FI == 0 || KG, kSplit> w;
    {
      TilePlan<D, kTile, kWaves, false> plan_kv;  // resident K, V rows tp0 .. tp0+kTile-1
      plan_kv.init(wave, lane, stk.n, dr);
#pragma unroll
      for (int u = 0; u < decltype(plan_kv)::TL::kParts; ++u) {
        if constexpr (!KG) plan_kv.part(kres, rk, tp0, wave, u);
        plan_kv.part(vres, rv, tp0, wave, u);
      }
    }
    if constexpr (KG) {  // this lane's K row j_col (keys past NK: zeros, all masked)
      const half_t* krow = K + kv_off + (size_t)min(j_col, NK - 1) * stk.n + h * 8;
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk)
        w.kb[kk] = as_half8(load16(krow + kk * 16, j_col < NK && kk * 16 + h * 8 < dr));
    }
#pragma unroll
    for (int k = 0; k < 2 * (D / 32); ++k) w.acc[k] = zero16();

    const int i_start = q_start(tile);
    const int row_lo = CAUSAL ? j_col - kofs : packed_nc ? col_lo(j_col) : -(1 << 30);
    const int n_qt = max(1, (q_end(tile) - i_start + kSub - 1) / kSub);  // (a divisor)
    // Rows this wave's key column reaches (see KVWave::step).
    const int row_end = j_col < Nk ? (narrowed ? upper(j_col) : N) : 0;
    // Query head (of the group) and first query row of flattened step `it`.
    auto qpos = [&](int it, int& g, int& i0) {
      if constexpr (SPARSE) {
        const int e = it / kSpb;
        const int f = clist[1 + e];
        g = f / nb;
        i0 = (f - g * nb) * kSparseBlock + (it - e * kSpb) * kSub;
      } else {
        g = it / n_qt;
        i0 = i_start + (it % n_qt) * kSub;
      }
    };

    // Q, dO tiles and lse2, dvec of flattened step `it` (clamped to the last
    // one, so that every step issues the same loads) into one stage.
    // Without any step (it_end <= 0) this is step 0, loaded but never run: a
    // valid query head whose rows past N read as zeros. (Clamped only from
    // above, a negative index would name a query head past the last one,
    // whose loads' resources start past the tensors' ends.)
    auto fetch = [&](int it, half_t* tq, half_t* to, float* tv) {
      it = max(0, min(it, it_end - 1));
      int g, i0;
      qpos(it, g, i0);
      const int hq = hkv * group + g;
      const size_t bhq = (size_t)b * Hq + hq;
      const rsrc_t rq = rows_rsrc(Q + q_off(hq), N, stq.n, dr);
      const rsrc_t ro = rows_rsrc(dO + q_off(hq), N, stq.n, dr);
#pragma unroll
      for (int u = 0; u < decltype(plan_q)::kParts; ++u) {
        plan_q.part(tq, rq, i0, wave, u);
        plan_q.part(to, ro, i0, wave, u);
      }
      if (wave == 0) vec_load64(tv, make_rsrc(Lse2 + bhq * N, (uint32_t)N * 4), i0, lane);
      if (wave == 1)
        vec_load64(tv + kVecStride, make_rsrc(Dvec + bhq * N, (uint32_t)N * 4), i0, lane);
    };
    // Bias values of step `it` for this lane's key and its 16 query rows,
    // through a resource over the wave's 32 rows (rows past N read zeros, a
    // key past N the next row: both masked); loaded one step ahead.
    const uint32_t bvoff1 = (uint32_t)(4 * h * N + j_col) * 4u;
    auto bload1 = [&](int it) {
      floatx16 v = zero16();
      if (has_bias) {
        int g, i0;
        qpos(it, g, i0);
        const rsrc_t rb = bias_rows_rsrc(bplane(hkv * group + g), i0 + 32 * half, N);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          v[r] = buf_load_f32(rb, bvoff1, (uint32_t)((8 * (r >> 2) + (r & 3)) * N) * 4u);
      }
      return v;
    };
    floatx16 bv1 = bload1(it_begin);
    // One step over the stage of parity P, while the next step's tiles load
    // into the other stage.
    auto step = [&](int it, auto par) {
      constexpr int P = decltype(par)::value;
      const half_t* Qs = P ? ta1 : ta0;
      const half_t* Os = P ? tb1 : tb0;
      const float* lse2s = P ? vec1 : vec0;
      int g, i0;
      qpos(it, g, i0);
      // Causal tiles wholly above a wave's keys give exact zeros through the
      // mask; they occur only on the diagonal, so they are not skipped.
      const float alibi_raw =
          BOUNDS && alibi ? alibi[hkv * group + g] / scale : 0.f;  // step's query head
      // Key j_col's mask word for the step's query rows (clamped: rows past N
      // are masked by row_end, keys past N have row_end = 0).
      const size_t tword =
          (size_t)min(j_col, N - 1) * W32 + min((i0 + 32 * half) >> 5, W32 - 1);
      const uint32_t mtw =
          MASKB && mask_t ? plane(mask_t, hkv * group + g)[tword] : ~0u;
      const uint32_t ztw =
          DROPB && drop_t ? zplane(drop_t, hkv * group + g)[tword] : ~0u;
      // The next stage's loads go out after the step's mask and dropout words:
      // loads complete in issue order, so words loaded after them would hold
      // the softmax until the whole next stage had landed.
      fetch(it + 1, P ? ta0 : ta1, P ? tb0 : tb1, P ? vec0 : vec1);
      // (j_col - kofs: the ALiBi distance counts from the aligned diagonal)
      w.step(Qs, Os, lse2s, lse2s + kVecStride, vres, kres, half, w4 * 32, i0, j_col - kofs, row_lo,
             row_end,
             alibi_raw, mtw, ztw, zs, bv1, [&] { return bload1(min(it + 1, it_end - 1)); },
             braw, lane, roff, so, scale_log2);
      wait_vmem();
      __syncthreads();
    };

    fetch(it_begin, ta0, tb0, vec0);
    wait_vmem();
    __syncthreads();
    if constexpr (FI == 0 && !KG) {
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) w.kb[kk] = tile_read16<D>(kres, w4 * 32, kk, roff);
    }
    int it = it_begin;
    for (; it + 2 <= it_end; it += 2) {
      step(it, P0{});
      step(it + 1, P1{});
    }
    if (it < it_end) step(it, P0{});

    // Sum the two halves' partials (dV^T in region 2*w4, dK^T in region
    // 2*w4 + 1) into the waves of the lower half.
    if constexpr (kHalves == 2) {
      if (half) {
        partial_store<D / 32>(region(2 * w4), w.acc, 0, lane);
        partial_store<D / 32>(region(2 * w4 + 1), w.acc, D / 32, lane);
      }
      __syncthreads();
      if (!half) {
        partial_add<D / 32>(region(2 * w4), w.acc, 0, lane);
        partial_add<D / 32>(region(2 * w4 + 1), w.acc, D / 32, lane);
      }
    }
    bool finish = true;
    if (shared) {
      const int u = helping ? partner : tw;
      unsigned* cnt = counters + (size_t)bkv * pairs + u;
      float* const pair_slots = slots + (size_t)(bkv * pairs + u) * 2 * kSlotFloats;
      const rsrc_t mine = make_rsrc(pair_slots + (helping ? kSlotFloats : 0), kSlotFloats * 4);
      const rsrc_t other = make_rsrc(pair_slots + (helping ? 0 : kSlotFloats), kSlotFloats * 4);
      // The owner usually finishes second: if the helper is done, it adds the
      // helper's partial without publishing its own.
      //
      // Ordering (HIP/HSA scoped memory model; agent scope, as the two
      // workgroups may sit on different XCDs). Publisher: every thread stores
      // its part of the slot, the workgroup barrier orders those stores before
      // thread 0, and thread 0 bumps the counter with an agent-scope
      // acquire-release RMW. Consumer: thread 0 reads the counter with agent
      // acquire semantics (that RMW, or the owner's early load), and the
      // barrier that shares the value orders every thread's slot loads after
      // it. Happens-before is transitive across these three steps (workgroup
      // scope within each workgroup, agent scope between the two), so each
      // consumer thread sees every publisher thread's partial. One thread
      // carries the agent-scope release and acquire: their cache maintenance
      // (L2 write-back, invalidation) then runs once per exchange, not once
      // per wave (measured: one per wave cost 5% of bwd_main at B=1 H=8
      // N=4096 D=128, 14% at H=16 N=8192). The slot accesses themselves
      // use device-coherent loads and stores (sc1).
      finish = false;
      if (!helping) {
        if (tid == 0) xflag = __hip_atomic_load(cnt, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        finish = xflag == 1u;
        __syncthreads();
      }
      if (!finish) {
        if (!half) {
          slot_store<2 * (D / 32)>(mine, w.acc, w4, lane);
          // Each storing wave waits for its own slot stores to complete
          // before the barrier, so the counter bump below cannot overtake
          // them whatever the compiler does for a workgroup-scope barrier.
          wait_vmem();
        }
        __syncthreads();
        if (tid == 0)
          xflag = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        finish = xflag == 1u;
      }
      if (finish) {
        if (!half) slot_add<2 * (D / 32)>(other, w.acc, w4, lane);
        // Both partials are consumed: the counter goes back to zero for the
        // next call (relaxed: the next call is ordered behind this launch).
        if (tid == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    // dK (scaled) and dV leave as fp16.
    if (finish && !half && (!BOUNDS || j_col < NK)) {
      half_t* dkrow = dK + kv_off + (size_t)j_col * stk.n;
      half_t* dvrow = dV + kv_off + (size_t)j_col * stk.n;
#pragma unroll
      for (int cb = 0; cb < D / 32; ++cb) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          half4 k4, v4;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            k4[e] = to16<BF>(w.acc[D / 32 + cb][4 * g4 + e] * scale);
            v4[e] = to16<BF>(w.acc[cb][4 * g4 + e] * zs);  // dropout: dV of the scaled P
          }
          if (cb * 32 + 8 * g4 + 4 * h < dr) {  // columns past the head dim are padding
            *reinterpret_cast<half4*>(dkrow + cb * 32 + 8 * g4 + 4 * h) = k4;
            *reinterpret_cast<half4*>(dvrow + cb * 32 + 8 * g4 + 4 * h) = v4;
          }
        }
      }
    }
    __syncthreads();  // the exchange regions are the next item's or phase's staging memory
  };
  if (tw < n_ktiles) {
    if (x_help > 0) run_item(true);
    run_item(false);
  }
  const int t0 = tw * kTile;  // query rows of phase 2

  // ============================== phase 2: dQ ==============================
  if (tw < n_qtiles) {
    const int iw = t0 + w4 * 32;  // this wave's query rows
    const int i_row = iw + l32;
    const bool row_ok = !BOUNDS || i_row < N;
    const int kv_end = CAUSAL ? min(Nk, t0 + kTile + kofs) : row_hi(t0 + kTile - 1);
    const int lane_hi = row_hi(i_row);  // this lane's row: keys from lane_hi on are masked
    // (at least one step: rows above the first key, when there are more query
    // rows than key rows, mask every key)
    const int n_kt = max(1, (kv_end + kSub - 1) / kSub);
    // With a window, key tiles left of every row's window are skipped, and
    // each row masks the keys left of its own.
    const int t_lo = narrowed ? lower(t0) / kSub : 0;
    const int key_lo = narrowed ? lower(i_row) : -(1 << 30);

    for (int g = 0; g < group; ++g) {
      const int hq = hkv * group + g;
      const size_t bhq = (size_t)b * Hq + hq;
      // Block-sparse: the key blocks this query block attends (count first);
      // step t runs streamed tile t % kSpb of the (t / kSpb)-th block (an
      // empty list: one step, whose rows have lse = +inf, so P = 0).
      const int* const rlist = SPARSE ? block_rows + (bhq * nb + tw) * (nb + 1) : nullptr;
      const int n_steps = SPARSE ? max(1, rlist[0] * kSpb) : n_kt;
      const int t_first = SPARSE ? 0 : t_lo;
      auto stage = [&](int t) {
        if constexpr (!SPARSE) return t;
        const int e = t / kSpb;
        return rlist[1 + e] * kSpb + (t - e * kSpb);
      };
      const float alibi_raw = BOUNDS && alibi ? alibi[hq] / scale : 0.f;
      const half_t* Qg = Q + q_off(hq);
      const half_t* dOg = dO + q_off(hq);
      // This lane's row of the mask (rows past N are never stored).
      const uint32_t* mrow =
          MASKB && mask ? plane(mask, hq) + (size_t)min(i_row, N - 1) * W32 : nullptr;
      const uint32_t* zrow =
          DROPB && drop ? zplane(drop, hq) + (size_t)min(i_row, N - 1) * W32 : nullptr;
      // This lane's bias values of key step t (four runs of four keys, read
      // as in the forward: a resource over the wave's 32 rows, 16-byte loads
      // when N % 4 == 0 on a 16-byte aligned plane) and its gradient row
      // (rows past N: none).
      const float* bpl = has_bias ? bplane(hq) : nullptr;
      const rsrc_t rb2 = bias_rows_rsrc(bpl, iw, N);
      const bool bias_x4 =
          has_bias && (N & 3) == 0 && (reinterpret_cast<uintptr_t>(bpl) & 15u) == 0;
      const uint32_t bvoff2 = (uint32_t)(l32 * N + 32 * half + 4 * h) * 4u;
      float* dbrow = BIAS && dbias && row_ok ? dbias + (bhq * N + i_row) * N : nullptr;
      const bool db_x4 =
          BIAS && dbias && (N & 3) == 0 && (reinterpret_cast<uintptr_t>(dbias) & 15u) == 0;
      auto bload2 = [&](int t) {
        floatx16 v = zero16();
        if (has_bias) {
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const uint32_t soff = (uint32_t)(t * kSub + 8 * g4) * 4u;
            if (bias_x4) {
              const floatx4 x = buf_load_f32x4(rb2, bvoff2, soff);
#pragma unroll
              for (int e = 0; e < 4; ++e) v[4 * g4 + e] = x[e];
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) v[4 * g4 + e] = buf_load_f32(rb2, bvoff2 + 4u * e, soff);
            }
          }
        }
        return v;
      };
      floatx16 bv2 = bload2(stage(t_first));
      QWave<D, CAUSAL, BOUNDS, BF, kSplit> w;
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) {
        const bool col_ok = row_ok && kk * 16 + h * 8 < dr;
        w.qb[kk] = as_half8(load16(Qg + (size_t)i_row * stq.n + kk * 16 + h * 8, col_ok));
        w.ob[kk] = as_half8(load16(dOg + (size_t)i_row * stq.n + kk * 16 + h * 8, col_ok));
      }
      w.lse2 = row_ok ? Lse2[bhq * N + i_row] : 0.f;
      w.dvv = row_ok ? Dvec[bhq * N + i_row] : 0.f;
#pragma unroll
      for (int cb = 0; cb < D / 32; ++cb) w.acc[cb] = zero16();

      // K, V tiles of key step t (clamped to the last one) into a stage.
      auto fetch = [&](int t, half_t* tk, half_t* tv) {
        const int jn = stage(min(t, n_steps - 1)) * kSub;
#pragma unroll
        for (int u = 0; u < decltype(plan_k)::kParts; ++u) {
          plan_k.part(tk, rk, jn, wave, u);
          plan_k.part(tv, rv, jn, wave, u);
        }
      };
      auto step = [&](int t, auto par) {
        constexpr int P = decltype(par)::value;
        // The next stage's loads go out between this step's products.
        const int jn = stage(min(t + 1, n_steps - 1)) * kSub;
        auto issue = [&](int q) {
          constexpr int kParts = decltype(plan_k)::kParts;
          static_assert(2 * kParts <= D / 16, "every load needs an issue point");
          if (q < 2 * kParts) {
            if (q & 1) plan_k.part(P ? tb0 : tb1, rv, jn, wave, q >> 1);
            else plan_k.part(P ? ta0 : ta1, rk, jn, wave, q >> 1);
          }
        };
        const int ts = stage(t);
        const int word = min(ts * (kSub / 32) + half, W32 - 1);  // keys ts*kSub + 32*half ..
        const uint32_t mw = mrow ? mrow[word] : ~0u;
        const uint32_t zw = zrow ? zrow[word] : ~0u;
        w.step(P ? ta1 : ta0, P ? tb1 : tb0, half, ts * kSub, i_row + kofs, lane_hi, key_lo,
               alibi_raw, mw, zw, zs, bv2,
               [&] { return bload2(stage(min(t + 1, n_steps - 1))); }, braw, dbrow, db_x4,
               lane, so, scale_log2, issue);
        wait_vmem();
        __syncthreads();
      };
      fetch(t_first, ta0, tb0);
      wait_vmem();
      __syncthreads();
      int t = t_first;  // buffer parity counts from t_first
      for (; t + 2 <= n_steps; t += 2) {
        step(t, P0{});
        step(t + 1, P1{});
      }
      if (t < n_steps) step(t, P0{});

      if constexpr (kHalves == 2) {
        if (half) partial_store<D / 32>(region(4 + w4), w.acc, 0, lane);
        __syncthreads();
      }
      if (!half && row_ok) {
        if constexpr (kHalves == 2) partial_add<D / 32>(region(4 + w4), w.acc, 0, lane);
        const size_t row_off = q_off(hq) + (size_t)i_row * stq.n;
        if (dQh) {  // fp16 dQ: the fp32 result rounded to nearest even, as .to(fp16)
#pragma unroll
          for (int cb = 0; cb < D / 32; ++cb)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              half4 v4;
#pragma unroll
              for (int e = 0; e < 4; ++e) v4[e] = to16<BF>(w.acc[cb][4 * g4 + e] * scale);
              if (cb * 32 + 8 * g4 + 4 * h < dr)
                *reinterpret_cast<half4*>(dQh + row_off + cb * 32 + 8 * g4 + 4 * h) = v4;
            }
        } else {
#pragma unroll
          for (int cb = 0; cb < D / 32; ++cb)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              floatx4 v4;
#pragma unroll
              for (int e = 0; e < 4; ++e) v4[e] = w.acc[cb][4 * g4 + e] * scale;
              if (cb * 32 + 8 * g4 + 4 * h < dr)
                *reinterpret_cast<floatx4*>(dQ + row_off + cb * 32 + 8 * g4 + 4 * h) = v4;
            }
        }
      }
      __syncthreads();  // the exchange regions are the next head's staging memory
    }
  }
}

template <int D, bool BF>
hipError_t launch_pre_d(const BwdArgs& a) {
  constexpr int kRowsPerBlock = 256 / pre_lanes_per_row(D);
  const long rows = (long)a.B * a.Hq * a.N;
  const dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  hipLaunchKernelGGL((bwd_pre_kernel<D, BF>), grid, dim3(256), 0, (hipStream_t)a.stream,
                     (const half_t*)a.o, (const half_t*)a.dO, a.lse, a.dvec, a.lse2, rows, a.Hq,
                     a.N, make_strides(a.layout, a.Hq, a.N, a.D), a.counters, a.n_counters, a.D);
  return hipGetLastError();
}

template <int D, bool CAUSAL, bool BOUNDS, int FEAT, bool BF>
hipError_t launch_main_t(const BwdArgs& a) {
  const int NK = key_rows(a.N, a.Nkv);
  const int n_tiles = (max(a.N, NK) + kTile - 1) / kTile;
  const dim3 grid(xcd_grid(n_tiles * a.B * a.Hkv));
  using Sh = BwdShape<D, (FEAT & kBwdW4) != 0>;
  // D is the tile width; a.D the head dim in memory, which sets the default
  // scale and the strides.
  const float scale = a.scale > 0.f ? a.scale : 1.f / sqrtf((float)a.D);
  hipLaunchKernelGGL((bwd_kernel<D, CAUSAL, BOUNDS, FEAT, BF>), grid, dim3(Sh::kThreads), 0,
                     (hipStream_t)a.stream, (const half_t*)a.q, (const half_t*)a.k,
                     (const half_t*)a.v, (const half_t*)a.dO, a.lse2, a.dvec, a.dq,
                     (half_t*)a.dq16, (half_t*)a.dk, (half_t*)a.dv, a.N, a.Hq, a.Hq / a.Hkv, n_tiles,
                     a.B * a.Hkv, scale, scale * kLog2e, make_strides(a.layout, a.Hq, a.N, a.D),
                     make_strides(a.layout, a.Hkv, NK, a.D), a.counters, a.slots,
                     a.slots ? ((FEAT & kBwdW4) ? kSplitNumW4 : kSplitNum) * 64 / Sh::kSub : 0,
                     a.slots ? kSplitBias : 0, a.kv_len, a.window,
                     a.alibi, a.seg_start, a.seg_end, a.mask, a.mask_t, a.mask_heads, a.drop,
                     a.drop_t, a.drop_scale, a.bias, a.bias_sb, a.bias_sh,
                     a.bias ? 1.f / scale : 0.f, a.dbias, a.D, NK, a.block_rows, a.block_cols);
  return hipGetLastError();
}

template <int D, bool BF>
hipError_t launch_main_d(const BwdArgs& a) {
  // Key lengths, windows, packed sequences and ALiBi need the masked
  // instantiation (kTile is a multiple of every kSub); a mask, dropout or a bias
  // one of its copies with those inputs compiled in (Feat).
  const bool bounds = (a.N % kTile) != 0 || a.kv_len != nullptr || a.window > 0 ||
                      a.alibi != nullptr || a.seg_start != nullptr ||
                      key_rows(a.N, a.Nkv) != a.N;
  auto with = [&](auto feat) {
    constexpr int F = decltype(feat)::value;
    return a.causal ? launch_main_t<D, true, true, F, BF>(a)
                    : launch_main_t<D, false, true, F, BF>(a);
  };
  switch (feat_of(a.mask != nullptr, a.drop != nullptr, a.bias != nullptr,
                  a.block_rows != nullptr)) {
    case kFeatBlock: return with(std::integral_constant<int, kFeatBlock>{});
    case kFeatBlock | kFeatDrop:
      return with(std::integral_constant<int, kFeatBlock | kFeatDrop>{});
    case kFeatMask: return with(std::integral_constant<int, kFeatMask>{});
    case kFeatDrop:
      // Keep bits need no bounds: where nothing else does, the unmasked
      // instantiations (not at width 256, where they spill).
      if constexpr (D <= 128) {
        if (!bounds)
          return a.causal ? launch_main_t<D, true, false, kFeatDrop, BF>(a)
                          : launch_main_t<D, false, false, kFeatDrop, BF>(a);
      }
      return with(std::integral_constant<int, kFeatDrop>{});
    case kFeatMask | kFeatDrop: return with(std::integral_constant<int, kFeatMask | kFeatDrop>{});
    case kFeatBias:  // (no bias at width 256: the C ABI refuses it)
      if constexpr (D > 128) return hipErrorInvalidValue;
      else return with(std::integral_constant<int, kFeatBias>{});
    default: break;
  }
  if constexpr (D == 64) {  // W4 where the grid gives every CU two workgroups (BwdShape)
    const long long wgs =
        (long long)((max(a.N, key_rows(a.N, a.Nkv)) + kTile - 1) / kTile) * a.B * a.Hkv;
    if (wgs >= 2LL * kCUs) {
      if (a.causal)
        return bounds ? launch_main_t<D, true, true, kBwdW4, BF>(a)
                      : launch_main_t<D, true, false, kBwdW4, BF>(a);
      return bounds ? launch_main_t<D, false, true, kBwdW4, BF>(a)
                    : launch_main_t<D, false, false, kBwdW4, BF>(a);
    }
  }
  if (a.causal)
    return bounds ? launch_main_t<D, true, true, 0, BF>(a)
                  : launch_main_t<D, true, false, 0, BF>(a);
  return bounds ? launch_main_t<D, false, true, 0, BF>(a)
                : launch_main_t<D, false, false, 0, BF>(a);
}

}  // namespace

unsigned long long bwd_launch_items(int B, int Hq, int Hkv, int N, int D, int Nkv) {
  const unsigned long long rows = (unsigned long long)B * Hq * N;
  const unsigned long long rows_per_block = 256 / pre_lanes_per_row(padded_head_dim(D));
  const unsigned long long pre = (rows + rows_per_block - 1) / rows_per_block * 256;
  const unsigned long long tiles =
      ((unsigned long long)(N > key_rows(N, Nkv) ? N : key_rows(N, Nkv)) + kTile - 1) / kTile;
  const unsigned long long wgs = tiles * (unsigned long long)B * (unsigned long long)Hkv;
  const unsigned long long threads = padded_head_dim(D) > 128 ? 256 : 512;  // BwdShape
  const unsigned long long main = (wgs + kXcds - 1) / kXcds * kXcds * threads;
  return pre > main ? pre : main;
}

hipError_t launch_bwd_preprocess(const BwdArgs& a) {
  const int w = padded_head_dim(a.D);
  if (a.dtype == kBF16)
    return w == 32 ? launch_pre_d<32, true>(a) : w == 64 ? launch_pre_d<64, true>(a)
         : w == 96 ? launch_pre_d<96, true>(a) : w == 128 ? launch_pre_d<128, true>(a)
         : launch_pre_d<256, true>(a);
  return w == 32 ? launch_pre_d<32, false>(a) : w == 64 ? launch_pre_d<64, false>(a)
       : w == 96 ? launch_pre_d<96, false>(a) : w == 128 ? launch_pre_d<128, false>(a)
       : launch_pre_d<256, false>(a);
}

hipError_t launch_bwd_main(const BwdArgs& a) {
  const int w = padded_head_dim(a.D);
  if (a.dtype == kBF16)
    return w == 32 ? launch_main_d<32, true>(a) : w == 64 ? launch_main_d<64, true>(a)
         : w == 96 ? launch_main_d<96, true>(a) : w == 128 ? launch_main_d<128, true>(a)
         : launch_main_d<256, true>(a);
  return w == 32 ? launch_main_d<32, false>(a) : w == 64 ? launch_main_d<64, false>(a)
       : w == 96 ? launch_main_d<96, false>(a) : w == 128 ? launch_main_d<128, false>(a)
       : launch_main_d<256, false>(a);
}

}  // namespace fa
