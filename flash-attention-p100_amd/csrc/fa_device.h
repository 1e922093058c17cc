// Device-side building blocks shared by the forward and backward kernels.
//
// Everything here targets gfx950 (CDNA4) directly: wave64, the
// v_mfma_f32_32x32x16_f16 matrix instruction, and LDS tiles with padded rows.
//
// MFMA 32x32x16 (fp16 in, fp32 accumulate) register layout, per lane l of 64,
// h = l / 32:
//   A (32x16, M x K): 8 halves, A[l % 32][8h + e],  e = 0..7
//   B (16x32, K x N): 8 halves, B[8h + e][l % 32]
//   C (32x32)       : 16 floats, C[8*(r/4) + 4h + (r%4)][l % 32], r = 0..15
// Because only the products along K are summed, A and B may enumerate the K
// index in any order as long as both use the same order; the kernels use
// this to feed an accumulator straight back in as the next product's operand.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace fa {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ floatx16 mfma32(half8 a, half8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// 16-bit element formats. Tensors hold fp16 (the reference's format) or bf16
// (BF); loads, LDS tiles and stores move either as opaque 16-bit values in
// half_t containers, and only the matrix products and the conversions from
// and to fp32 depend on the format. Conversions round to nearest even.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
template <bool BF>
__device__ __forceinline__ floatx16 mfma16(half8 a, half8 b, floatx16 c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
template <bool BF>
__device__ __forceinline__ half_t to16(float x) {
  if constexpr (BF)
    return __builtin_bit_cast(half_t, (__bf16)x);
  else
    return (half_t)x;
}
template <bool BF>
__device__ __forceinline__ float from16(half_t x) {
  if constexpr (BF)
    return (float)__builtin_bit_cast(__bf16, x);
  else
    return (float)x;
}

__device__ __forceinline__ floatx16 zero16() {
  floatx16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 16-byte global load; returns zeros when `ok` is false.
__device__ __forceinline__ u32x4 load16(const half_t* p, bool ok) {
  u32x4 r = {0u, 0u, 0u, 0u};
  if (ok) r = *reinterpret_cast<const u32x4*>(p);
  return r;
}

__device__ __forceinline__ half8 as_half8(u32x4 v) {
  return __builtin_bit_cast(half8, v);
}

// Swap with the lane 32 positions away (the other half of the wave).
__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4;

// ds_read_b64_tr_b16 (gfx950 LDS transpose read). Within each group of 16
// lanes, lane a + 4t supplies the address of 4 halves at (row t, columns
// 4a .. 4a+3) of a 4 x 16 block; lane n of the group receives column n of
// that block, i.e. the 4 rows of one column.
__device__ __forceinline__ half4 lds_read_tr(const half_t* p) {
  const short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(p));
  return __builtin_bit_cast(half4, v);
}

// ---------------------------------------------------------------------------
// XCD-aware work numbering. MI355X dispatches consecutive workgroups of a
// launch round-robin over its 8 XCDs, each with its own L2. Workgroup L thus
// runs on XCD L % 8; giving that XCD the contiguous work range
// [xcd * per, (xcd + 1) * per) keeps all workgroups of a head (which re-read
// the same K/V or Q/dO tiles) behind one L2. Returns -1 for the few padding
// workgroups when `total` is not a multiple of 8. Only locality depends on the
// dispatch order; correctness does not.
constexpr int kXcds = 8;
constexpr int kCUs = 256;  // 8 XCDs x 32 CUs
__host__ __device__ __forceinline__ int xcd_grid(int total) {
  return ((total + kXcds - 1) / kXcds) * kXcds;
}
__device__ __forceinline__ int xcd_work_index(int total) {
  const int per = (total + kXcds - 1) / kXcds;
  const int L = blockIdx.x;
  const int w = (L % kXcds) * per + L / kXcds;
  return w < total ? w : -1;
}

// ---------------------------------------------------------------------------
// LDS tiles filled by direct global -> LDS loads.
//
// A tile stores rows of D halves padded to S = D/8 + 1 sixteen-byte chunks,
// and keeps logical row R at LDS row perm16(R), which swaps the two low 2-bit
// fields of R (an involution that fixes R's 16-row group). The LDS has 64
// banks of 4 bytes (measured with SQ_LDS_BANK_CONFLICT), i.e. 16 bank groups
// of 16 bytes, and chunk c of LDS row rho sits in group (rho*S + c) mod 16:
//   * the 16-byte MFMA operand reads (16 lanes = 16 consecutive logical rows
//     at one chunk per LDS cycle) hit 16 distinct groups because perm16 (and,
//     for D = 64, the odd factor S = 9) is a bijection mod 16;
//   * the transpose reads (per half-wave: 4 logical rows 4h+t, t = 0..3, at 4
//     consecutive chunks) land on LDS rows 4t+h, spaced by 4, so they also
//     hit 16 distinct groups.
// Every read address is then one per-lane base plus a compile-time offset.
template <int D>
struct Tile {
  static constexpr int kChunks = D / 8;         // data chunks per row
  static constexpr int kStride = kChunks + 1;   // chunks per padded row
  static constexpr int kRowHalves = kStride * 8;
  template <int ROWS>
  static constexpr int insts() { return (ROWS * kStride + 63) / 64; }  // 1 KB wave loads
  template <int ROWS>
  static constexpr int halves() { return insts<ROWS>() * 512; }
};

__host__ __device__ __forceinline__ constexpr int perm16(int r) {
  return (r & ~15) | ((r & 3) << 2) | ((r >> 2) & 3);
}

// Per-lane offset (halves) of the 16-byte operand read of logical row
// rowbase + (lane % 32), rowbase a multiple of 16.
template <int D>
__device__ __forceinline__ int row_lane_off(int lane) {
  return perm16(lane & 31) * Tile<D>::kRowHalves + 8 * (lane >> 5);
}

// Per-lane offset (halves) of the transpose read (see tr_operand()).
template <int D>
__device__ __forceinline__ int tr_lane_off(int lane) {
  const int n = lane & 15, grp = lane >> 4;
  return (4 * (n >> 2) + (grp >> 1)) * Tile<D>::kRowHalves + 16 * (grp & 1) + 4 * (n & 3);
}

// 16-byte MFMA operand: logical row rowbase + lane%32, halves 16*kk + 8*(lane/32) ...+7.
template <int D>
__device__ __forceinline__ half8 tile_read16(const half_t* tile, int rowbase, int kk, int lane_off) {
  return *reinterpret_cast<const half8*>(tile + rowbase * Tile<D>::kRowHalves + 16 * kk + lane_off);
}

// Transpose-read A operand of tr_operand() on a tile: column c0 + lane%32 at
// logical rows rbase + 8*(e/4) + 4*(lane/32) + e%4 (rbase a multiple of 16).
template <int D>
__device__ __forceinline__ half8 tile_tr_operand(const half_t* tile, int rbase, int c0, int tr_off) {
  const half_t* p = tile + rbase * Tile<D>::kRowHalves + c0 + tr_off;
  const half4 lo = lds_read_tr(p);
  const half4 hi = lds_read_tr(p + 2 * Tile<D>::kRowHalves);
  return half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// ---------------------------------------------------------------------------
// Direct global -> LDS loads through a buffer resource (buffer_load ... lds).
// The resource (base, size in bytes) lives in scalar registers; a load is one
// per-lane 32-bit VGPR offset plus a scalar offset, so a kernel can keep the
// per-lane offsets in registers that nothing else ever overwrites, and
// accesses at or past the resource's size return zeros (no clamping needed).
// Keeping address registers untouched matters: the compiler treats an
// LDS-DMA instruction's VGPR operands like store data and waits for the load
// to complete before such a register is reused.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data format
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kRsrcWord3);
}
// A per-lane offset at or above 2^31 marks the columns past a head dim that
// is narrower than the tile: only such head dims use it, and for them the C
// ABI keeps a head's byte range within 2^30, so the offset is past every
// resource and the scalar row offsets added to it cannot carry the sum past
// 2^32. The lane reads zeros.
constexpr uint32_t kOutOfRange = 0x80000000u;

// Optional per-score inputs of a masked (BOUNDS) instantiation: a bit-packed
// mask, dropout keep bits, or an additive bias. Each costs registers in every
// step of the D = 128 copies (the mask or the dropout bits alone ~90 bytes of
// spills per lane, both ~180), so each set the launchers meet has its own
// copy: FEAT = kFeatMask, kFeatDrop, both, or kFeatBias (a bias, with a mask
// and dropout as run-time options). kFeatBlock: a block-sparse layout (steps
// over its visible blocks only), alone or with dropout.
enum : int { kFeatMask = 1, kFeatDrop = 2, kFeatBias = 4, kFeatBlock = 8 };
template <int FEAT>
struct Feat {
  static constexpr bool kMask = (FEAT & (kFeatMask | kFeatBias)) != 0;
  static constexpr bool kDrop = (FEAT & (kFeatDrop | kFeatBias)) != 0;
  static constexpr bool kBias = (FEAT & kFeatBias) != 0;
  static constexpr bool kBlock = (FEAT & kFeatBlock) != 0;
};
// The instantiation serving a set of options (mask, dropout, bias, block
// layout present; the C ABI refuses a block layout with a mask or a bias).
__host__ __device__ constexpr int feat_of(bool mask, bool drop, bool bias, bool block = false) {
  return block ? kFeatBlock | (drop ? kFeatDrop : 0)
       : bias  ? kFeatBias
               : (mask ? kFeatMask : 0) | (drop ? kFeatDrop : 0);
}
// One and four fp32 values at voff + soff of a resource (zeros past its size).
__device__ __forceinline__ float buf_load_f32(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ floatx4 buf_load_f32x4(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
// Attention bias reads from an fp32 plane of N rows of N values: a resource
// over the 32 rows from row0 (fewer at the plane's end, none past it), so
// reads past the plane's last row return zeros, while a key past N in an
// earlier row reads the next row's value, which every caller masks. The C
// ABI keeps N <= 2^22 with a bias, so 32 rows stay below 2^32 bytes.
__device__ __forceinline__ rsrc_t bias_rows_rsrc(const float* plane, int row0, int N) {
  const int rows = max(0, min(32, N - row0));
  return make_rsrc(plane + (size_t)min(row0, N) * N, (uint32_t)rows * (uint32_t)N * 4u);
}
// Each lane loads `size` bytes (4 or 16) from voff + soff into LDS at
// lds + byte_off + size * lane (lds and byte_off wave-uniform). The offset is
// added after the conversion to an LDS address: added to the generic
// pointer, a constant offset makes the compiler fold a generic-to-LDS
// conversion of a constant address, for which it emits an invalid
// instruction.
template <int size>
__device__ __forceinline__ void lds_direct_buf(void* lds, rsrc_t r, uint32_t voff, uint32_t soff,
                                               uint32_t byte_off = 0) {
  static_assert(size == 4 || size == 16, "LDS direct loads of 4 or 16 bytes per lane");
  auto* p = (__attribute__((address_space(3))) char*)lds + byte_off;
  if constexpr (size == 16)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)p, 16,
                                             voff, soff, 0, 0);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)p, 4,
                                             voff, soff, 0, 0);
}

// ---------------------------------------------------------------------------
// Unpadded LDS tiles with an XOR chunk swizzle, for tiles streamed every step.
//
// Row r occupies 2*D contiguous bytes and keeps its 16-byte chunk c at position
// c ^ g(r), where g permutes the low row bits:
//   D = 128 (a row spans all 16 bank groups): g(r) = perm16(r & 15);
//   D = 64 (two rows per 256 bytes): g(r) = ((r >> 1) & 1) << 2 | (r >> 2) & 3.
// The 16-byte operand reads (16 consecutive rows at one chunk) and the
// transpose reads (per half-wave: 4 consecutive rows x 4 consecutive chunks)
// then hit 16 distinct bank groups, and a direct load covers whole rows
// (1024 / (2D) per instruction, every lane fetching one chunk of its row),
// which the memory pipeline serves ~28% faster than the padded-row pattern
// (17 vs 21.75 cycles per instruction per CU). The swizzle is not additive in
// the chunk index, so each lane keeps one byte offset per operand position.
template <int D>
struct Swz {
  static constexpr int kChunks = D / 8;
  static constexpr int kRowBytes = 2 * D;
  static constexpr int kRowsPerInst = 1024 / kRowBytes;
  __host__ __device__ static constexpr int g(int r) {
    return D == 128 ? perm16(r & 15) : ((((r >> 1) & 1) << 2) | ((r >> 2) & 3));
  }
  template <int ROWS>
  static constexpr int bytes() { return ROWS * kRowBytes; }

  // Per-lane byte offsets for a wave that reads rows row0 .. row0+31 of a tile
  // (row0 a multiple of 16): rd[kk] for the 16-byte operand read of row
  // row0 + lane % 32 at halves 16kk + 8(lane / 32); tr[cb][hi] for the
  // transpose read of rows row0 + 4(lane / 32) + 8hi .. +3 at columns
  // 32cb + 16((lane / 16) % 2) + 4(lane % 4) .. +3.
  struct Offsets {
    int rd[D / 16];
    int tr[D / 32][2];
    __device__ __forceinline__ void init(int lane, int row0) {
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk)
        rd[kk] = (row0 + (lane & 31)) * kRowBytes +
                 (((2 * kk) | (lane >> 5)) ^ g(lane & 15)) * 16;
      const int n = lane & 15, grp = lane >> 4, t = n >> 2, a = n & 3;
#pragma unroll
      for (int cb = 0; cb < D / 32; ++cb)
#pragma unroll
        for (int hi = 0; hi < 2; ++hi) {
          const int r = 4 * (grp >> 1) + t + 8 * hi;
          const int x = 2 * (grp & 1) + (a >> 1);
          tr[cb][hi] = (row0 + r) * kRowBytes + ((4 * cb + x) ^ g(r)) * 16 + 8 * (a & 1);
        }
    }
  };

  // 16-byte MFMA operand: row row0 + lane % 32, halves 16kk + 8(lane / 32) .. +7.
  __device__ __forceinline__ static half8 read16(const void* tile, const Offsets& o, int kk) {
    return *reinterpret_cast<const half8*>(reinterpret_cast<const char*>(tile) + o.rd[kk]);
  }
  // Transpose-read A operand (as tile_tr_operand): column 32cb + lane % 32 at
  // rows row0 + 16q + 8(e / 4) + 4(lane / 32) + e % 4. Adding 16 rows keeps
  // the swizzle, so q only moves the address by a constant.
  __device__ __forceinline__ static half8 tr_operand(const void* tile, int q, const Offsets& o,
                                                     int cb) {
    const char* p = reinterpret_cast<const char*>(tile) + 16 * q * kRowBytes;
    const half4 lo = lds_read_tr(reinterpret_cast<const half_t*>(p + o.tr[cb][0]));
    const half4 hi = lds_read_tr(reinterpret_cast<const half_t*>(p + o.tr[cb][1]));
    return half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
};

// Direct-load plan for a swizzled tile of ROWS rows filled by NW waves: every
// wave issues kParts 1 KB instructions; part u covers rows u * kPartRows
// further on, so one VGPR (base) and a scalar offset serve them all.
template <int D, int ROWS, int NW>
struct SwzPlan {
  using S = Swz<D>;
  static constexpr int kInsts = S::template bytes<ROWS>() / 1024;
  static_assert(kInsts % NW == 0, "tile must split evenly over the waves");
  static_assert((S::kRowsPerInst * NW) % 16 == 0, "swizzle must repeat across parts");
  static constexpr int kParts = kInsts / NW;
  static constexpr int kPartRows = S::kRowsPerInst * NW;  // rows per part
  uint32_t base;
  uint32_t row_bytes;  // bytes between consecutive rows in global memory (2*D when dense)

  // dr: the head dim in memory (<= D); chunks past it load as zeros.
  __device__ __forceinline__ void init(int wave, int lane, int row_stride, int dr) {
    row_bytes = 2u * (uint32_t)row_stride;
    const int r = S::kRowsPerInst * wave + lane / S::kChunks;  // row within part 0
    const int c = (lane % S::kChunks) ^ S::g(r);               // global chunk of this lane
    base = (uint32_t)r * row_bytes + (uint32_t)(c * 16) + (c < dr / 8 ? 0u : kOutOfRange);
  }
  // Part u of the load of rows r0 .. r0+ROWS-1 of the buffer `r` (rows of D
  // halves, row_bytes apart) into `tile`; rows past the buffer's end read as
  // zeros.
  __device__ __forceinline__ void part(void* tile, rsrc_t r, int r0, int wave, int u) const {
    lds_direct_buf<16>(tile, r, base, ((uint32_t)r0 + (uint32_t)(u * kPartRows)) * row_bytes,
                       (uint32_t)(u * NW + wave) * 1024u);
  }
};

// The padded-row layout of Tile<D> behind Swz<D>'s interface, for the
// staged tiles of head dims whose rows do not pack into 1 KB load
// instructions (2D does not divide 1024, e.g. D = 96). Logical row R sits at
// LDS row perm16(R) with kStride = D/8 + 1 chunks per row; D/8 even makes
// kStride odd, so both read patterns stay conflict-free (see Tile).
template <int D>
struct Pad {
  using T = Tile<D>;
  static_assert((D / 8) % 2 == 0, "odd row stride needs an even chunk count");
  static constexpr int kRowBytes = T::kRowHalves * 2;
  template <int ROWS>
  static constexpr int bytes() { return T::template halves<ROWS>() * 2; }
  struct Offsets {
    int rd[D / 16];
    int tr[D / 32][2];
    __device__ __forceinline__ void init(int lane, int row0) {
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk)
        rd[kk] = 2 * ((row0 + perm16(lane & 31)) * T::kRowHalves + 16 * kk + 8 * (lane >> 5));
#pragma unroll
      for (int cb = 0; cb < D / 32; ++cb) {
        tr[cb][0] = 2 * (row0 * T::kRowHalves + 32 * cb + tr_lane_off<D>(lane));
        tr[cb][1] = tr[cb][0] + 4 * T::kRowHalves;
      }
    }
  };
  __device__ __forceinline__ static half8 read16(const void* tile, const Offsets& o, int kk) {
    return *reinterpret_cast<const half8*>(reinterpret_cast<const char*>(tile) + o.rd[kk]);
  }
  __device__ __forceinline__ static half8 tr_operand(const void* tile, int q, const Offsets& o,
                                                     int cb) {
    const char* p = reinterpret_cast<const char*>(tile) + 16 * q * kRowBytes;
    const half4 lo = lds_read_tr(reinterpret_cast<const half_t*>(p + o.tr[cb][0]));
    const half4 hi = lds_read_tr(reinterpret_cast<const half_t*>(p + o.tr[cb][1]));
    return half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
};

// Layout and load plan of tiles streamed every step: the swizzled rows for
// the widths whose rows fill the 1 KB load instructions and whose swizzle g
// is defined (64, 128), the padded rows otherwise.
template <int D>
constexpr bool kSwizzled = D == 64 || D == 128;
template <int D>
using Stream = std::conditional_t<kSwizzled<D>, Swz<D>, Pad<D>>;

// Wait until this wave's direct-to-LDS (and other vector memory) loads landed.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Direct loads of logical rows [r0, r0 + ROWS) of a row-major (N, D) fp16
// matrix into a tile by the NW waves of a workgroup: kInsts 1 KB instructions
// (64 lanes x one 16-byte chunk, the padding slot of each row included), wave
// w issuing instructions w, w + NW, ... (kParts at most). With EVEN the tile
// is padded to a whole number of instructions per wave (kHalves), so every
// wave issues exactly kParts and the issue needs no wave-dependent branch.
template <int D, int ROWS, int NW, bool EVEN = false>
struct TileLoad {
  static constexpr int kInsts = Tile<D>::template insts<ROWS>();
  static constexpr int kParts = (kInsts + NW - 1) / NW;  // instructions per wave (at most)
  static constexpr int kHalves = (EVEN ? kParts * NW : kInsts) * 512;
};

template <int D, int ROWS, int NW, bool EVEN>
struct TilePlan {
  using TL = TileLoad<D, ROWS, NW, EVEN>;
  static constexpr int kParts = TL::kParts;
  uint32_t off[TL::kParts];
  uint32_t row_bytes;  // bytes between consecutive rows in global memory (2*D when dense)

  // dr: the head dim in memory (<= D); chunks past it load as zeros.
  __device__ __forceinline__ void init(int wave, int lane, int row_stride, int dr) {
    using T = Tile<D>;
    row_bytes = 2u * (uint32_t)row_stride;
#pragma unroll
    for (int u = 0; u < TL::kParts; ++u) {
      const int p = (u * NW + wave) * 64 + lane;
      const int rho = p / T::kStride;
      const int c = p - rho * T::kStride;
      const int row = rho < ROWS ? perm16(rho) : 0;
      off[u] = (uint32_t)row * row_bytes + (uint32_t)(c < T::kChunks ? c * 16 : 0) +
               (c < T::kChunks && c >= dr / 8 ? kOutOfRange : 0u);
    }
  }
  // Loads part u of the tile whose first row is r0 from the buffer `r` (rows
  // of D halves, row_bytes apart); rows past the buffer's end read as zeros.
  __device__ __forceinline__ void part(half_t* tile, rsrc_t r, int r0, int wave, int u) const {
    const int inst = u * NW + wave;
    if (EVEN || TL::kInsts % NW == 0 || inst < TL::kInsts)
      lds_direct_buf<16>(tile, r, off[u], (uint32_t)r0 * row_bytes, (uint32_t)inst * 1024u);
  }
};

// Load plan of a streamed tile (Stream<D>): SwzPlan, or TilePlan for the
// padded rows, with the same kParts / part() interface.
template <int D, int ROWS, int NW>
using StreamPlan = std::conditional_t<kSwizzled<D>, SwzPlan<D, ROWS, NW>,
                                      TilePlan<D, ROWS, NW, false>>;

// Buffer resource over the n_rows rows of one head: rows of dr halves
// row_stride halves apart. Its size ends right after row n_rows-1, so any row
// index >= n_rows reads as zeros.
__device__ __forceinline__ rsrc_t rows_rsrc(const half_t* base, int n_rows, int row_stride,
                                            int dr) {
  return make_rsrc(base, ((uint32_t)n_rows - 1u) * 2u * (uint32_t)row_stride + 2u * (uint32_t)dr);
}

}  // namespace fa
