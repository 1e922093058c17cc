// FlashAttention-2 forward for gfx950 (MI355X).
//
// Counterpart of the reference's flash::fwd_kernel (flash_fwd.cuh:68-340),
// redesigned around MFMA, the CDNA4 LDS and the balance of a causal grid:
//
// Work split. A workgroup is 8 waves and owns a 64-row query tile: waves are
// (row block rb in {0,1}) x (key quarter kq in {0..3}). Each wave owns 32
// query rows and, of every 128 keys staged, the 32 keys of its quarter; the
// four quarters' partial (max, sum, O) are merged through LDS at the end of
// the tile. Under causal masking a workgroup takes query tile x and then
// tile T-1-x, so every workgroup does the same amount of work (the long and
// the short end of the triangle), and the grid of (T/2) x (B*Hq) workgroups
// x 8 waves keeps two waves on every SIMD at the headline shape. Workgroups
// are numbered so that each head's tiles run on one XCD and its K/V stay in
// that XCD's L2.
//
// Per wave and 32-key step, on v_mfma_f32_32x32x16_f16 (fp32 accumulate):
//   * S^T = K Q^T with this wave's Q^T held in registers as the B operand, so
//     in the accumulator lane l owns query row l % 32 and the softmax row
//     max is a per-lane max plus one lane swap with the other half-wave
//     (v_permlane32_swap, no LDS round trip);
//   * the scale is applied to the fp32 logit (never to Q in fp16,
//     flash_fwd.cuh:94-101), folded with log2(e) into one FMA before exp2;
//   * the running max is refreshed lazily: O and the row sum are rescaled
//     only when some row's max grows by more than 2^8, so P stays <= 256 and
//     the rescale (a pass over all O accumulators) is rare;
//   * P^T leaves the accumulator as fp16 and feeds O^T += V^T P^T directly,
//     with V^T read from the row-major V tile by the LDS transpose read;
//   * software pipeline: step j computes the softmax of S_j (made in step
//     j-1) while the products of S_{j+1} run, so each wave has matrix work
//     in flight during its own exponentials. K therefore runs one step ahead
//     of V in the double buffers.
// K and V tiles move from global memory straight into double-buffered,
// padded, row-permuted LDS tiles (buffer_load ... lds), so staging costs
// no registers and no LDS store instructions, and every LDS read address is a
// per-lane base plus an immediate. The next stage's load instructions leave
// a few at a time between the current stage's products: issued all at once,
// they stall every wave until the memory pipeline (64 B/clk per CU) has
// accepted them.
//
// Causal tiles past the diagonal are never loaded (flash_fwd.cuh:127-130);
// diagonal and ragged tiles take a separate masked path (flash_fwd.cuh:
// 226-243). Outputs: O (fp16) and LSE = m + log(l) in natural-log units of
// the scaled logits (flash_fwd.cuh:321-339).
#include <type_traits>

#include "fa_device.h"
#include "fa_launch.h"

namespace fa {
namespace {

constexpr int kBR = 64;    // query rows per tile (2 row blocks of 32)
constexpr float kRescaleLog2 = 8.f;  // lazy-rescale threshold, log2 units

// Waves and staged keys per width. Up to D = 128: 8 waves (two per SIMD) =
// 2 row blocks x 4 key quarters of a 128-key stage. At D = 256 a wave's Q
// operands and O accumulators need ~260 registers and a 128-key K or V tile
// 66 KB of LDS, so 4 waves (one per SIMD, 512 registers each) = 2 row blocks
// x 2 key halves of a 64-key stage.
// W4 (widths 64 and 128, grids of at least two workgroups per CU): the
// 4-wave shape there too, with at most 256 registers per wave so that two
// workgroups share a CU. Their waves then keep no common step barrier, so
// one workgroup's softmax runs beside the other's products: same-box A/B,
// forward -7% at B=2 H=32/8 N=3001 D=128, -4% at H=8 N=4096 D=128 (dense),
// -5% at H=16/8 N=8192 D=128 causal, -9% at H=16 N=4096 D=64 causal, -4% at
// H=16 N=4096 D=64 dense and at H=16/8 N=8192 D=64 causal; +5% at the causal
// B=1 H=8 N=4096 D=128, whose 256 tile pairs leave one 4-wave workgroup per
// CU, so the launcher takes it only where the grid fills both slots. Without
// causal masking the width-64 copies fit 168 registers without spills, so
// three workgroups share a CU: -2.1% at H=16 N=4096 D=64 dense (bit-identical;
// the causal copy then spills 3 registers and ran 2% slower, so it keeps two).
template <int D, bool W4 = false>
struct FwdShape {
  static constexpr int kWaves = D > 128 || W4 ? 4 : 8;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kQuarters = kWaves / 2;  // key slices of 32 per stage
  static constexpr int kKV = 32 * kQuarters;    // keys staged per step
};
// The FEAT bit that selects W4 (kept clear of the per-score input bits).
constexpr int kFwdW4 = 16;

template <int D, bool W4 = false>
struct FwdLds {
  static constexpr int kWaves = FwdShape<D, W4>::kWaves, kKV = FwdShape<D, W4>::kKV;
  static constexpr int kTileHalves = Tile<D>::template halves<kKV>();  // one K or V tile
  static constexpr int kStageHalves = 2 * kTileHalves; // K + V
  // Merge area (reuses the four tiles, kWaves / 4 waves each): per wave,
  // D/32 x 16 floats per lane.
  static_assert((kWaves / 4) * 64 * D * 2 <= kTileHalves * 2, "merge area exceeds a tile");
  static constexpr int kMLFloat2 = kWaves * 64;  // (m, l) per lane
  // Load instructions per wave and tile that every wave issues inside the
  // step; the remaining kInsts % kWaves go out at the start of the step.
  using TL = TileLoad<D, kKV, kWaves>;
  static constexpr int kEvenParts = TL::kInsts / kWaves;
  static constexpr int kIssueSlots = D / 16 + D / 32;
  static_assert(2 * kEvenParts <= kIssueSlots, "more loads than issue points");
};

// Row max over the two half-waves: lanes l and l ^ 32 hold the same query row.
__device__ __forceinline__ float max_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// QLDS: Q's operands are read from a staged LDS tile (qt, rows qrow ..) at
// each product instead of being held in registers (qb); the bias copy does
// this, as its 16 prefetched bias values per lane left no registers for Q.
template <int D, bool CAUSAL, bool BOUNDS, bool BF, bool QLDS = false>
struct FwdWave {
  // Per-wave state for one 32-row query block.
  half8 qb[QLDS ? 1 : D / 16];
  const half_t* qt;
  int qrow;
  floatx16 oacc[D / 32];
  floatx16 sc;  // raw logits S^T of the current step (this wave's 32 keys x 32 rows)
  float m_raw;  // running max of the raw (unscaled) logits; -inf before any key
  float l;      // this lane's partial row sum of p (its 16 of every 32 keys)

  // Q's operand of k-step kk: this wave's rows, columns 16kk .. 16kk+15.
  __device__ __forceinline__ half8 qop(int kk, int roff) const {
    if constexpr (QLDS) return tile_read16<D>(qt, qrow, kk, roff);
    else return qb[kk];
  }

  // S^T = K Q^T for this wave's 32 keys of a staged K tile.
  __device__ __forceinline__ void s_product(const half_t* Ks, int kq, int roff) {
    sc = zero16();
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
      sc = mfma16<BF>(tile_read16<D>(Ks, kq * 32, kk, roff), qop(kk, roff), sc);
  }

  // One software-pipelined step: softmax of sc (the keys j0 .. j0+31 of this
  // step) and O^T += V^T P^T from the V tile Vs, while (NEXT) the next step's
  // S^T is computed from its K tile Kn. `issue(s)` is called at issue points
  // s = 0 .. D/8 - 1 (after each product).
  // MASK: the step may need the causal / ragged mask, applied when `masked`.
  // bv: this step's bias values, replaced by `bnext()` (the next step's) as
  // soon as they are added, so one set of registers carries the prefetch.
  template <bool MASK, bool NEXT, class Issue, class BiasNext>
  __device__ __forceinline__ void step(const half_t* Kn, const half_t* Vs, int kq, int j0,
                                       bool masked, int i_row, int N, int w_lo, float alibi_raw,
                                       uint32_t mw, uint32_t zw, floatx16& bv,
                                       const BiasNext& bnext, float bias_raw, int lane, int roff,
                                       int troff, float c, float thr_raw, const Issue& issue) {
    const int h = lane >> 5;
    // This lane's keys are bits 8g + 4h + e of the step's mask and dropout
    // words: shifted once, every per-score bit position is a constant (with
    // 4h inside it the compiler kept 16 per-lane bit masks in registers).
    const uint32_t mwh = mw >> (4 * h), zwh = zw >> (4 * h);
    floatx16 s = sc;
    floatx16 sn = zero16();
    constexpr int kS = D / 16;  // products of the next S^T
    constexpr int kFront = kS > 2 ? 2 : 1;  // issued before the row max (covers its latency)
    // At width 256 each product's LDS operand is read one product ahead and
    // pinned there (scheduling fence): left to the scheduler, a step's 32
    // operand reads were hoisted to its top and spilled registers. At width
    // 128 the unmasked instantiations pin K's operands the same way: the
    // scheduler had left the step's last four S^T products each waiting for
    // its own read (same-box A/B: forward -2% at B=1 H=8 N=4096 causal, -1%
    // at B=2 H=32/8 N=3001, bit-identical; in the masked instantiations it
    // added spills). At width 64 the same: -2% on the forward at H=16 N=4096
    // causal, -1.6% at H=16/8 N=8192, -1% dense, bit-identical (V's operands
    // pinned too: 1-2% slower). Widths 32 and 96 leave the reads to the
    // scheduler.
    constexpr bool kPin = D > 128;
    constexpr bool kPinK = D > 128 || ((D == 128 || D == 64) && !BOUNDS);
    auto kread = [&](int kk) { return tile_read16<D>(Kn, kq * 32, kk, roff); };
    half8 kcur = kPinK && NEXT ? kread(0) : half8{};
    auto kop = [&](int kk) {
      if constexpr (!kPinK) return kread(kk);
      const half8 a = kcur;
      if (kk + 1 < kS) kcur = kread(kk + 1);
      __builtin_amdgcn_sched_barrier(0);
      return a;
    };
#pragma unroll
    for (int kk = 0; kk < kFront; ++kk)
      if constexpr (NEXT) {
        sn = mfma16<BF>(kop(kk), qop(kk, roff), sn);
        issue(kk);
      }
    // ALiBi (masked instantiation only): -slope |i - j| in raw-score units,
    // from one distance per lane and constant offsets (exact in fp32).
    if (BOUNDS && alibi_raw != 0.f) {
      const float d0 = (float)(i_row - j0 - 4 * h);
#pragma unroll
      for (int r = 0; r < 16; ++r)
        s[r] = fmaf(-alibi_raw, fabsf(d0 - (float)(8 * (r >> 2) + (r & 3))), s[r]);
    }
    // Additive attention bias (the bias instantiation only; bias_raw = 1/scale
    // puts it in raw-score units): bv holds this row's 16 values of the step.
    if (BOUNDS && bias_raw != 0.f) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = fmaf(bv[r], bias_raw, s[r]);
      if constexpr (NEXT) bv = bnext();
    }
    if (MASK && masked) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int bit = 8 * (r >> 2) + (r & 3);
        const int j = j0 + bit + 4 * h;
        // w_lo: the last key left of this row's sliding window (INT_MIN if none);
        // mw: this row's mask bits for keys j0 .. j0+31 (all set without a mask)
        if ((CAUSAL && j > i_row) || (BOUNDS && (j >= N || j <= w_lo || !((mwh >> bit) & 1u))))
          s[r] = -INFINITY;
      }
    }
    float mloc = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mloc = fmaxf(mloc, s[r]);
    mloc = max_halves(mloc);
    // Lazy rescale: only when some row's max grew by more than 2^8.
    if (__builtin_expect(__any(mloc > m_raw + thr_raw), 0)) {
      const float m_new = fmaxf(m_raw, mloc);
      const float corr = (m_raw == -INFINITY) ? 0.f : fast_exp2((m_raw - m_new) * c);
      l *= corr;
#pragma unroll
      for (int cb = 0; cb < D / 32; ++cb)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[cb][r] *= corr;
      m_raw = m_new;
    }
    const float neg = (m_raw == -INFINITY) ? 0.f : -m_raw * c;
    half8 pb[2];
#pragma unroll
    for (int kk = kFront; kk < kS; ++kk) {
      if constexpr (NEXT) {
        sn = mfma16<BF>(kop(kk), qop(kk, roff), sn);
        issue(kk);
      }
      // 16 exponentials spread over the remaining products.
      constexpr int kPer = (16 + kS - kFront - 1) / (kS - kFront);
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        const int r = (kk - kFront) * kPer + e;
        if (r < 16) {
          const float p = fast_exp2(fmaf(s[r], c, neg));
          l += p;
          // Dropout: the row sum keeps every key, P V only the kept ones.
          const int bit = 8 * (r >> 2) + (r & 3);
          pb[r >> 3][r & 7] = to16<BF>(((zwh >> bit) & 1u) ? p : 0.f);
        }
      }
    }
    // O^T += V^T P^T; k-step q covers keys 16q .. 16q+15 of this quarter.
    auto vread = [&](int u) {  // u = q * (D / 32) + cb
      return tile_tr_operand<D>(Vs, kq * 32 + 16 * (u / (D / 32)), 32 * (u % (D / 32)), troff);
    };
    half8 vcur = kPin ? vread(0) : half8{};
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int cb = 0; cb < D / 32; ++cb) {
        const int u = q * (D / 32) + cb;
        half8 va;
        if constexpr (kPin) {
          va = vcur;
          if (u + 1 < D / 16) vcur = vread(u + 1);
          __builtin_amdgcn_sched_barrier(0);
        } else {
          va = vread(u);
        }
        oacc[cb] = mfma16<BF>(va, pb[q], oacc[cb]);
        if constexpr (NEXT) issue(kS + u);
      }
    if constexpr (NEXT) sc = sn;
  }
};

// FEAT: the optional per-score inputs compiled in (Feat, with BOUNDS).
template <int D, bool CAUSAL, bool BOUNDS, int FEAT, bool BF>
__device__ __forceinline__ void fwd_tile(const half_t* __restrict__ Q, const half_t* __restrict__ K,
                                         const half_t* __restrict__ V, half_t* __restrict__ O,
                                         float* __restrict__ Lse, int N, int Nk, int W,
                                         const int* __restrict__ sst, const int* __restrict__ sen,
                                         float alibi_raw, const uint32_t* __restrict__ mbase,
                                         const uint32_t* __restrict__ zbase, float o_scale,
                                         const float* __restrict__ bbase, float bias_raw,
                                         int W32, int sq, int sk, int dr, int kofs,
                                         int qtile, float c, float thr_raw, half_t* kt0,
                                         half_t* vt0,
                                         half_t* kt1, half_t* vt1, float2* ml, half_t* qt,
                                         const int* __restrict__ blist) {
  constexpr bool W4 = (FEAT & kFwdW4) != 0;
  using L = FwdLds<D, W4>;
  constexpr int kWaves = FwdShape<D, W4>::kWaves, kKV = FwdShape<D, W4>::kKV;
  constexpr int kQuarters = FwdShape<D, W4>::kQuarters;
  constexpr bool MASKB = Feat<FEAT>::kMask, DROPB = Feat<FEAT>::kDrop, BIAS = Feat<FEAT>::kBias;
  constexpr bool SPARSE = Feat<FEAT>::kBlock;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar M0 bases
  __builtin_assume(wave >= 0 && wave < kWaves);
  const int h = lane >> 5, l32 = lane & 31;
  const int rb = wave & 1, kq = wave >> 1;
  const int q0 = qtile * kBR;
  const int i_base = q0 + rb * 32;
  const int i_row = i_base + l32;

  FwdWave<D, CAUSAL, BOUNDS, BF, BIAS> w;
  const int roff = row_lane_off<D>(lane), troff = tr_lane_off<D>(lane);
  const bool row_ok = !BOUNDS || i_row < N;
  if constexpr (!BIAS) {
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
      w.qb[kk] = as_half8(load16(Q + (size_t)i_row * sq + kk * 16 + h * 8,
                                 row_ok && kk * 16 + h * 8 < dr));
  } else {
    w.qt = qt;
    w.qrow = rb * 32;
  }
#pragma unroll
  for (int cb = 0; cb < D / 32; ++cb) w.oacc[cb] = zero16();
  w.m_raw = -INFINITY;
  w.l = 0.f;

  // Keys [0, Nk) exist for this batch entry (Nk = the key rows unless key
  // lengths are given); later keys are masked like keys past a ragged N.
  // kofs = key rows - query rows: causal masking aligns the last query row
  // with the last key row, so row i's diagonal key is i + kofs. Without causal
  // masking, packed sequences also end each row's keys at row_hi(i) =
  // min(Nk, sen[i]) (at least i + 1), which does not decrease with i.
  const bool packed_nc = BOUNDS && !CAUSAL && sen != nullptr;
  auto row_hi = [&](int i) {
    i = min(i, N - 1);
    return packed_nc ? min(Nk, max(sen[i], i + 1)) : Nk;
  };
  const int kv_end = CAUSAL ? min(Nk, q0 + kBR + kofs) : row_hi(q0 + kBR - 1);
  // Block-sparse layout (SPARSE instantiations): blist lists the key blocks
  // of this tile's block row (count first). Step v then runs stage(v), stage
  // v % kSpb of the (v / kSpb)-th listed block; the masks below work in
  // stages (key offsets / kKV), so each step is masked as its stage needs. A
  // block row with no visible block runs one step with every key masked.
  constexpr int kSpb = kSparseBlock / kKV;  // stages per block
  const int n_blk = SPARSE ? blist[0] : 0;
  auto stage = [&](int v) {
    if constexpr (!SPARSE) return v;
    const int e = v / kSpb;
    return blist[1 + e] * kSpb + (v - e * kSpb);
  };
  // (at least one step: a tile whose rows all lie above the first key, when
  // there are more query rows than key rows, masks every key)
  const int n_it = SPARSE ? max(1, n_blk * kSpb) : max(1, (kv_end + kKV - 1) / kKV);
  // Leading steps in which this wave's 32x32 block needs no mask. The later
  // ones run masked; blocks wholly past the diagonal or past N give exact
  // zeros there (their few products are not skipped, so every wave issues its
  // share of the loads inside the same code).
  // Causal left bounds: row i sees keys from lower(i) on, the larger of its
  // sliding window's first key i - W + 1 (W = 0: none) and the first token of
  // its packed sequence sst[i] (sst = nullptr: none), clamped to [0, i].
  // lower() does not decrease with i, so this tile's first visible key is
  // lower(q0) and the steps before j_lo are skipped; a wave's steps before
  // n_head (blocks reaching left of its last row's bound) are masked, like the
  // diagonal ones. Only the masked instantiation (BOUNDS) takes left bounds,
  // so the others keep their loop structure.
  const int Wb = BOUNDS ? W : 0;
  const bool narrowed = BOUNDS && (Wb > 0 || sst != nullptr);
  auto lower = [&](int i) {
    i = min(i, N - 1);
    int lo = Wb > 0 ? i + kofs - Wb + 1 : 0;
    if (sst) lo = max(lo, min(sst[i], i));
    return max(lo, 0);
  };
  const int j_first = narrowed ? lower(q0) / kKV : 0;  // first stage any row reaches
  const int j_lo = SPARSE ? 0 : j_first;                 // first step
  const int win_last = narrowed ? lower(i_base + 31) - 1 - kq * 32 : -1;  // last masked block start
  const int n_head = win_last >= 0 ? max(j_first, win_last / kKV + 1) : j_first;
  const int w_lo = narrowed ? lower(i_row) - 1 : INT_MIN;
  int n_full = SPARSE ? INT_MAX : n_it;  // (in stages)
  if (CAUSAL) {
    const int e = i_base + kofs - 31 - kq * 32;  // the wave's blocks stay unmasked up to key e
    n_full = min(n_full, e >= 0 ? e / kKV + 1 : 0);
  }
  // (an empty block row: no key for any row)
  const bool no_keys = SPARSE && n_blk == 0;
  const int k_hi = no_keys ? 0 : row_hi(i_base);  // smallest key bound of this wave's rows
  if (BOUNDS) n_full = min(n_full, k_hi - 32 - kq * 32 >= 0 ? (k_hi - 32 - kq * 32) / kKV + 1 : 0);
  const int lane_hi = no_keys ? 0 : row_hi(i_row);  // this lane's row: keys from lane_hi on are masked
  // Arbitrary mask (MASKB instantiations): this row's bit words; every step
  // then takes the mask. Word w covers keys 32w .. 32w+31, and a wave's 32
  // keys of step j are word (kKV / 32) j + kq (clamped: keys past N are
  // masked anyway).
  // Dropout keep bits (DROPB instantiations; zbase null: keep all) in the
  // same layout, one plane per (b, query head).
  const uint32_t* mrow = MASKB && mbase ? mbase + (size_t)min(i_row, N - 1) * W32 : nullptr;
  const uint32_t* zrow = DROPB && zbase ? zbase + (size_t)min(i_row, N - 1) * W32 : nullptr;
  // With a mask every step runs in the masked loops below, and a step takes
  // the mask only at the bounds above or when some row of the wave's block
  // hides a key (bits past N are zero, so a ragged last word never passes);
  // dropout bits apply in either loop. The bias copy masks every step (one
  // step form: measured 5% faster there).
  if (BIAS) n_full = 0;
  auto mword = [&](int j) { return mrow ? mrow[min(j * (kKV / 32) + kq, W32 - 1)] : ~0u; };
  auto zword = [&](int j) { return zrow ? zrow[min(j * (kKV / 32) + kq, W32 - 1)] : ~0u; };
  // Attention bias (BIAS instantiation; bbase null: none): this row's values
  // for the wave's 16 keys of step j, four runs of four keys, through a
  // resource over the wave's 32 rows (keys past N read the next row or zeros
  // and are masked). Rows of N % 4 == 0 values from a 16-byte aligned plane
  // take one 16-byte load per run; a run never crosses the resource's end.
  const bool has_bias = BIAS && bbase != nullptr;
  const rsrc_t rbias = bias_rows_rsrc(bbase, i_base, N);
  const bool bias_x4 =
      has_bias && (N & 3) == 0 && (reinterpret_cast<uintptr_t>(bbase) & 15u) == 0;
  const uint32_t bvoff = (uint32_t)(l32 * N + kq * 32 + 4 * h) * 4u;
  auto bload = [&](int j) {
    floatx16 v = zero16();
    if (has_bias) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t soff = (uint32_t)(j * kKV + 8 * g) * 4u;
        if (bias_x4) {
          const floatx4 x = buf_load_f32x4(rbias, bvoff, soff);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[4 * g + e] = x[e];
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[4 * g + e] = buf_load_f32(rbias, bvoff + 4u * e, soff);
        }
      }
    }
    return v;
  };

  // Software pipeline over steps j = 0 .. n_it-1. Step j reads K_{j+1} (for
  // the next S^T) from K buffer (j+1)%2 and V_j from V buffer j%2, while it
  // loads K_{j+2} into K buffer j%2 and V_{j+1} into V buffer (j+1)%2 (tile
  // indices clamped to n_it-1, so every step issues the same loads; a
  // redundant copy lands only in a buffer nobody reads in that step).
  using TL = typename L::TL;
  TilePlan<D, kKV, kWaves, false> plan;
  plan.init(wave, lane, sk, dr);
  const rsrc_t rk = rows_rsrc(K, Nk, sk, dr), rv = rows_rsrc(V, Nk, sk, dr);
  const int k0 = stage(j_lo) * kKV, k1 = stage(min(j_lo + 1, n_it - 1)) * kKV;
#pragma unroll
  for (int u = 0; u < TL::kParts; ++u) {
    plan.part(kt0, rk, k0, wave, u);
    plan.part(vt0, rv, k0, wave, u);
    plan.part(kt1, rk, k1, wave, u);
  }
  if constexpr (BIAS) {  // the tile's 64 query rows (rows past N read zeros)
    TilePlan<D, kBR, kWaves, false> plan_q;
    plan_q.init(wave, lane, sq, dr);
    const rsrc_t rq = rows_rsrc(Q, N, sq, dr);
#pragma unroll
    for (int u = 0; u < decltype(plan_q)::kParts; ++u) plan_q.part(qt, rq, q0, wave, u);
  }
  wait_vmem();
  __syncthreads();
  w.s_product(kt0, kq, roff);
  __syncthreads();  // K buffer 0 is refilled by step 0

  // Step j with buffer parity P = j % 2 (a compile-time constant, so the
  // compiler sees that the step's reads never touch the buffers its direct
  // loads fill and does not wait for those loads before them).
  uint32_t mw = mword(stage(j_lo));  // mask bits of the next step to run
  uint32_t zw = zword(stage(j_lo));  // its dropout keep bits
  floatx16 bv = bload(stage(j_lo));  // its bias values
  auto run = [&](int j, auto par_tag, auto mask_tag, auto next_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    constexpr bool NEXT = decltype(next_tag)::value;
    constexpr int P = decltype(par_tag)::value;
    const uint32_t mw_now = mw, zw_now = zw;
    const int js = stage(j), jn = NEXT ? stage(j + 1) : js;  // this and the next step's stage
    if ((MASKB || DROPB) && NEXT) {
      mw = mword(jn);
      zw = zword(jn);
    }
    half_t* lk = P ? kt1 : kt0;  // receives K_{j+2}
    half_t* lv = P ? vt0 : vt1;  // receives V_{j+1}
    const int jk = stage(min(j + 2, n_it - 1)) * kKV;
    const int jv = jn * kKV;
    if (NEXT && L::kEvenParts < TL::kParts && wave < TL::kInsts % kWaves) {
      plan.part(lk, rk, jk, wave, L::kEvenParts);
      plan.part(lv, rv, jv, wave, L::kEvenParts);
    }
    auto issue = [&](int s) {
      if (s < 2 * L::kEvenParts) {
        if (s & 1) plan.part(lv, rv, jv, wave, s >> 1);
        else plan.part(lk, rk, jk, wave, s >> 1);
      }
    };
    const half_t* Kn = P ? kt0 : kt1;  // K_{j+1}
    const half_t* Vs = P ? vt1 : vt0;  // V_j
    // (every lane takes the ballot: without a mask mw_now is all ones)
    const bool hidden = MASKB && __builtin_amdgcn_ballot_w64(mw_now != ~0u) != 0;
    w.template step<MASK, NEXT>(Kn, Vs, kq, js * kKV + kq * 32,
                                js < n_head || js >= n_full || hidden, i_row + kofs,
                                lane_hi, w_lo, alibi_raw, mw_now, zw_now, bv, [&] { return bload(jn); },
                                BIAS ? bias_raw : 0.f, lane,
                                roff, troff, c, thr_raw, issue);
    if (NEXT) {
      wait_vmem();
      __syncthreads();
    }
  };
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using T = std::true_type;
  using F = std::false_type;
  // unmasked steps with a next step (block-sparse: each step's stage decides)
  const int n_plain = MASKB || SPARSE ? 0 : min(n_full, n_it - 1);
  // Buffer parity counts from j_lo. Every wave runs steps j_lo .. n_it-1, one
  // barrier each; only which of them are masked differs between waves.
  int j = j_lo;
  if (narrowed && !SPARSE) {  // masked steps at the rows' left bounds
    for (; j < min(n_head, n_it - 1); ++j) {
      if ((j - j_lo) & 1) run(j, P1{}, T{}, T{});
      else run(j, P0{}, T{}, T{});
    }
    if (((j - j_lo) & 1) && j < n_plain) run(j++, P1{}, T{}, T{});  // even parity for the loop
  }
  for (; j + 2 <= n_plain; j += 2) {
    run(j, P0{}, F{}, T{});
    run(j + 1, P1{}, F{}, T{});
  }
  // With a mask or a block layout every step runs masked: unrolled by buffer
  // parity like the plain loop. (Through the loop below, whose one step copy
  // takes either parity, every step copied the previous step's S^T and all O
  // accumulators between registers: 40 64-bit moves per step.)
  if constexpr (MASKB || SPARSE) {
    if (((j - j_lo) & 1) && j < n_it - 1) {
      run(j, P1{}, T{}, T{});
      ++j;
    }
    for (; j + 2 <= n_it - 1; j += 2) {
      run(j, P0{}, T{}, T{});
      run(j + 1, P1{}, T{}, T{});
    }
  }
  // The remaining steps (the masked ones, usually one or two) take the mask
  // at run time: fewer inlined copies of the step keep the accumulators in
  // one set of registers.
  for (; j < n_it - 1; ++j) {
    if ((j - j_lo) & 1) run(j, P1{}, T{}, T{});
    else run(j, P0{}, T{}, T{});
  }
  // last step: no next S^T, no loads
  if ((j - j_lo) & 1) run(j, P1{}, T{}, F{});
  else run(j, P0{}, T{}, F{});
  __syncthreads();  // every wave is done reading the tiles (they hold the merge area)

  // Merge the key slices of each row block through LDS: each of the four
  // tiles holds the partials of kWaves / 4 waves.
  constexpr int kPerTile = kWaves / 4;
  auto part_of = [&](int src) {
    const int t4 = src / kPerTile;
    half_t* t = t4 == 0 ? kt0 : t4 == 1 ? vt0 : t4 == 2 ? kt1 : vt1;
    return reinterpret_cast<float*>(t) + (src % kPerTile) * (D / 8) * 64 * 4;
  };
#pragma unroll
  for (int cb = 0; cb < D / 32; ++cb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      floatx4 v = {w.oacc[cb][4 * g], w.oacc[cb][4 * g + 1], w.oacc[cb][4 * g + 2],
                   w.oacc[cb][4 * g + 3]};
      *reinterpret_cast<floatx4*>(part_of(wave) + ((cb * 4 + g) * 64 + lane) * 4) = v;
    }
  ml[wave * 64 + lane] = make_float2(w.m_raw, w.l);
  __syncthreads();

  // Wave (rb, kq) finishes d-blocks kq, kq + kQuarters, ... of row block rb
  // (D = 64: kq < 2 only).
#pragma unroll
  for (int ci = 0; ci < (D / 32 + kQuarters - 1) / kQuarters; ++ci) {
    const int cb = kq + ci * kQuarters;
    if (cb >= D / 32) continue;
    float mk[kQuarters], lk[kQuarters];
    float m_star = -INFINITY;
#pragma unroll
    for (int k = 0; k < kQuarters; ++k) {
      const int src = k * 2 + rb;  // wave index of quarter k in this row block
      const float2 a = ml[src * 64 + lane];
      const float2 bb = ml[src * 64 + (lane ^ 32)];
      mk[k] = a.x;
      lk[k] = a.y + bb.y;
      m_star = fmaxf(m_star, mk[k]);
    }
    float wk[kQuarters], l_star = 0.f;
#pragma unroll
    for (int k = 0; k < kQuarters; ++k) {
      wk[k] = (mk[k] == -INFINITY) ? 0.f : fast_exp2((mk[k] - m_star) * c);
      l_star += wk[k] * lk[k];
    }
    // A row that saw no key (key lengths with a window: pad rows past the
    // window) gets O = 0 and LSE = +inf, so its backward P is 0 as well.
    const float inv_l = l_star > 0.f ? o_scale / l_star : 0.f;  // o_scale: dropout's 1/(1-p)
    if (row_ok && cb * 32 < dr) {  // d-blocks past the head dim hold padding
      half_t* orow = O + (size_t)i_row * sq + cb * 32;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < kQuarters; ++k) {
          const int src = k * 2 + rb;
          const floatx4 v =
              *reinterpret_cast<const floatx4*>(part_of(src) + ((cb * 4 + g) * 64 + lane) * 4);
          acc += v * wk[k];
        }
        half4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = to16<BF>(acc[e] * inv_l);
        if (cb * 32 + 8 * g + 4 * h < dr) *reinterpret_cast<half4*>(orow + 8 * g + 4 * h) = o4;
      }
      if (cb == 0 && h == 0)
        Lse[i_row] = l_star > 0.f ? (m_star * c + __log2f(l_star)) * kLn2 : INFINITY;
    }
  }
  __syncthreads();  // the LDS is reused by the next tile
}

template <int D, bool CAUSAL, bool BOUNDS, int FEAT, bool BF>
__global__ __launch_bounds__((FwdShape<D, (FEAT & kFwdW4) != 0>::kThreads))
__attribute__((amdgpu_waves_per_eu((FEAT & kFwdW4) != 0 ? (D == 64 && !CAUSAL ? 3 : 2) : 1)))
void fwd_kernel(
    const half_t* __restrict__ Q, const half_t* __restrict__ K,
    const half_t* __restrict__ V, half_t* __restrict__ O, float* __restrict__ Lse,
    int N, int Hq, int group, int n_qtiles, int gx, int BH, float scale_log2, Strides stq,
    Strides stk, const int* __restrict__ kv_len, int window, const float* __restrict__ alibi,
    const int* __restrict__ seg_start, const int* __restrict__ seg_end,
    const uint32_t* __restrict__ mask, int mask_heads, const uint32_t* __restrict__ drop,
    float drop_scale, const float* __restrict__ bias, long long bias_sb, long long bias_sh,
    float bias_raw, int dr, int NK, const int* __restrict__ block_rows) {
  // K and V tiles of two stages as distinct LDS objects (see fwd_tile), plus
  // (m, l).
  using L = FwdLds<D, (FEAT & kFwdW4) != 0>;
  __shared__ __align__(16) half_t kt0[L::kTileHalves];
  __shared__ __align__(16) half_t vt0[L::kTileHalves];
  __shared__ __align__(16) half_t kt1[L::kTileHalves];
  __shared__ __align__(16) half_t vt1[L::kTileHalves];
  __shared__ float2 ml[L::kMLFloat2];
  // The bias copy's staged Q tile (64 rows; a placeholder elsewhere).
  __shared__ __align__(16) half_t qt[Feat<FEAT>::kBias ? Tile<D>::template halves<kBR>() : 8];
  const int w = xcd_work_index(gx * BH);
  if (w < 0) return;
  const int bh = w / gx;       // over B*Hq
  const int first = w % gx;    // query tile (and, causal, its partner)
  const int b = bh / Hq, hq = bh % Hq;
  const int Hkv = Hq / group;
  const int hkv = hq / group;  // repeat_interleave head map (flash_fwd.cuh:90)
  const size_t q_off = (size_t)(b * stq.b + hq * stq.h);
  const size_t kv_off = (size_t)(b * stk.b + hkv * stk.h);
  const float thr_raw = kRescaleLog2 / scale_log2;
  // Per-entry key length (key padding), clamped to [1, NK] (NK: key rows).
  const int Nk = kv_len ? min(max(kv_len[b], 1), NK) : NK;
  // ALiBi slope of this query head in raw-score units (slope / scale).
  const float alibi_raw = alibi ? alibi[hq] * kLog2e / scale_log2 : 0.f;
  // This (b, head)'s mask plane (a plane shared by all heads when mask_heads == 1).
  const int W32 = (N + 31) >> 5;
  constexpr bool MASKB = Feat<FEAT>::kMask, DROPB = Feat<FEAT>::kDrop, BIAS = Feat<FEAT>::kBias;
  const uint32_t* mbase = MASKB && mask ? mask + ((size_t)b * mask_heads +
                                                   (mask_heads == 1 ? 0 : hq)) * N * W32
                                           : nullptr;
  // ... and its dropout keep bits (one plane per (b, query head)).
  const uint32_t* zbase = DROPB && drop ? drop + (size_t)bh * N * W32 : nullptr;
  // ... and its attention bias plane (element (i, j) at i * N + j).
  const float* bbase = BIAS && bias ? bias + b * bias_sb + hq * bias_sh : nullptr;
  // Causal: tile `first`, then its partner n_qtiles-1-first (one code copy).
  const int second = n_qtiles - 1 - first;
  const int n_tiles = (CAUSAL && second > first) ? 2 : 1;
  // Block-sparse layout: the lists of this head's block rows.
  const int nb = (N + kSparseBlock - 1) / kSparseBlock;
  const int* const brows =
      Feat<FEAT>::kBlock ? block_rows + (size_t)bh * nb * (nb + 1) : nullptr;
  for (int t = 0; t < n_tiles; ++t)
    fwd_tile<D, CAUSAL, BOUNDS, FEAT, BF>(Q + q_off, K + kv_off, V + kv_off, O + q_off,
                                Lse + (size_t)bh * N, N, Nk, window,
                                seg_start ? seg_start + (size_t)b * N : nullptr,
                                seg_end ? seg_end + (size_t)b * N : nullptr, alibi_raw, mbase,
                                zbase, DROPB ? drop_scale : 1.f, bbase, bias_raw, W32, stq.n,
                                stk.n, dr, NK - N,
                                t ? second : first,
                                scale_log2, thr_raw,
                                kt0, vt0, kt1, vt1, ml, qt,
                                brows ? brows + (size_t)((t ? second : first) * kBR /
                                                         kSparseBlock) * (nb + 1)
                                      : nullptr);
}

template <int D, bool CAUSAL, bool BOUNDS, int FEAT, bool BF>
hipError_t launch_fwd_t(const FwdArgs& a) {
  const int n_qtiles = (a.N + kBR - 1) / kBR;
  const int gx = CAUSAL ? (n_qtiles + 1) / 2 : n_qtiles;
  const int BH = a.B * a.Hq;
  dim3 grid(xcd_grid(gx * BH));
  // D is the tile width; a.D the head dim in memory, which sets the default
  // scale and the strides.
  const float scale_log2 = kLog2e * (a.scale > 0.f ? a.scale : 1.f / sqrtf((float)a.D));
  hipLaunchKernelGGL((fwd_kernel<D, CAUSAL, BOUNDS, FEAT, BF>), grid,
                     dim3(FwdShape<D, (FEAT & kFwdW4) != 0>::kThreads), 0,
                     (hipStream_t)a.stream, (const half_t*)a.q, (const half_t*)a.k,
                     (const half_t*)a.v, (half_t*)a.o, a.lse, a.N, a.Hq, a.Hq / a.Hkv,
                     n_qtiles, gx, BH, scale_log2, make_strides(a.layout, a.Hq, a.N, a.D),
                     make_strides(a.layout, a.Hkv, key_rows(a.N, a.Nkv), a.D), a.kv_len,
                     a.window, a.alibi,
                     a.seg_start, a.seg_end, a.mask, a.mask_heads, a.drop, a.drop_scale, a.bias,
                     a.bias_sb, a.bias_sh,
                     a.bias ? 1.f / (a.scale > 0.f ? a.scale : 1.f / sqrtf((float)a.D)) : 0.f, a.D,
                     key_rows(a.N, a.Nkv), a.block_rows);
  return hipGetLastError();
}

template <int D, bool BF>
hipError_t launch_fwd_d(const FwdArgs& a) {
  // Key lengths, windows, packed sequences and ALiBi need the masked
  // instantiation (kKV is a multiple of kBR); a mask, dropout or a bias one
  // of its copies with those inputs compiled in (Feat).
  const bool bounds = (a.N % FwdShape<D>::kKV) != 0 || a.kv_len != nullptr || a.window > 0 ||
                      a.alibi != nullptr || a.seg_start != nullptr ||
                      key_rows(a.N, a.Nkv) != a.N;
  auto with = [&](auto feat) {
    constexpr int F = decltype(feat)::value;
    return a.causal ? launch_fwd_t<D, true, true, F, BF>(a)
                    : launch_fwd_t<D, false, true, F, BF>(a);
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
          return a.causal ? launch_fwd_t<D, true, false, kFeatDrop, BF>(a)
                          : launch_fwd_t<D, false, false, kFeatDrop, BF>(a);
      }
      return with(std::integral_constant<int, kFeatDrop>{});
    case kFeatMask | kFeatDrop: return with(std::integral_constant<int, kFeatMask | kFeatDrop>{});
    case kFeatBias:
      // (the bias copy stages Q in LDS too, which at D = 256 does not fit
      // beside the K/V stages; the C ABI refuses a bias there)
      if constexpr (D > 128) return hipErrorInvalidValue;
      else return with(std::integral_constant<int, kFeatBias>{});
    default: break;
  }
  if constexpr (D == 128 || D == 64) {
    // W4 where the grid gives every CU two workgroups (FwdShape).
    const long long n_qt = (a.N + kBR - 1) / kBR;
    const long long wgs = (a.causal ? (n_qt + 1) / 2 : n_qt) * a.B * a.Hq;
    if (wgs >= 2LL * kCUs) {
      const bool bounds4 = (a.N % FwdShape<D, true>::kKV) != 0 || a.kv_len != nullptr ||
                           a.window > 0 || a.alibi != nullptr || a.seg_start != nullptr ||
                           key_rows(a.N, a.Nkv) != a.N;
      // (not the causal masked copy, which spills 23 registers at this shape)
      if (a.causal && !bounds4) return launch_fwd_t<D, true, false, kFwdW4, BF>(a);
      if (!a.causal)
        return bounds4 ? launch_fwd_t<D, false, true, kFwdW4, BF>(a)
                       : launch_fwd_t<D, false, false, kFwdW4, BF>(a);
    }
  }
  if (a.causal)
    return bounds ? launch_fwd_t<D, true, true, 0, BF>(a)
                  : launch_fwd_t<D, true, false, 0, BF>(a);
  return bounds ? launch_fwd_t<D, false, true, 0, BF>(a)
                : launch_fwd_t<D, false, false, 0, BF>(a);
}

}  // namespace

unsigned long long fwd_launch_items(int B, int Hq, int N, int D) {
  (void)D;
  const unsigned long long tiles = ((unsigned long long)N + kBR - 1) / kBR;  // non-causal grid
  const unsigned long long wgs = tiles * (unsigned long long)B * (unsigned long long)Hq;
  return (wgs + kXcds - 1) / kXcds * kXcds * (padded_head_dim(D) > 128 ? 256 : 512);
}

hipError_t launch_fwd(const FwdArgs& a) {
  const int w = padded_head_dim(a.D);
  if (a.dtype == kBF16)
    return w == 32 ? launch_fwd_d<32, true>(a) : w == 64 ? launch_fwd_d<64, true>(a)
         : w == 96 ? launch_fwd_d<96, true>(a) : w == 128 ? launch_fwd_d<128, true>(a)
                                                         : launch_fwd_d<256, true>(a);
  return w == 32 ? launch_fwd_d<32, false>(a) : w == 64 ? launch_fwd_d<64, false>(a)
       : w == 96 ? launch_fwd_d<96, false>(a) : w == 128 ? launch_fwd_d<128, false>(a)
                                                         : launch_fwd_d<256, false>(a);
}

}  // namespace fa
