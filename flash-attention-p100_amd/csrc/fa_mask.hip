// Bit-packing of a dense boolean attention mask, and generation of dropout
// keep bits, into the two layouts the kernels read: rows of W = ceil(N / 32)
// words per query (the forward and the backward's dQ phase, one word per
// lane and 32-key step) and the transpose, rows of W words per key (the
// backward's dK/dV phase, whose lanes own keys). No counterpart in the
// reference, which takes no mask and raises on dropout (fa_p100_hf.py:64-70, 83-85).
//
// The row packer is HBM-bound byte work: N*N bytes in, N*N/8 bytes out per
// plane (a grid-stride loop over 64-bit word indices keeps its grid small);
// the transposed words are then built from the packed rows (N*N/8 bytes
// each way) by the lane-exchange transpose the dropout generator uses.
// The dropout generator writes N*N/8 bytes per layout and plane and spends
// one hash (two 32-bit multiplies) per two keys (under causal masking only
// on the keys at or left of the diagonal).
#include <hip/hip_runtime.h>

#include "fa_launch.h"

namespace fa {
namespace {

constexpr int kPackThreads = 256;
constexpr long long kPackMaxBlocks = 1 << 16;

// One 32-key word per thread, consecutive threads on consecutive words of a
// row (a wave reads 2 KB of contiguous mask bytes). VEC: rows start 16-byte
// aligned (N % 16 == 0 and an aligned base), so each 16-key half is one load.
template <bool VEC>
__global__ __launch_bounds__(kPackThreads) void pack_rows_kernel(const uint8_t* __restrict__ dense,
                                                                 uint32_t* __restrict__ bits,
                                                                 long long rows, int N, int W) {
  const long long total = rows * W;
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x; g < total; g += stride) {
    const long long r = g / W;
    const int w = (int)(g - r * W);
    const uint8_t* src = dense + r * N + 32 * w;
    const int n = min(32, N - 32 * w);  // keys of this word that exist
    uint32_t word = 0;
    if (VEC) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        if (16 * half < n) {
          const uint4 x = *reinterpret_cast<const uint4*>(src + 16 * half);
          const uint32_t v[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
          for (int e = 0; e < 16; ++e)
            word |= (uint32_t)(((v[e >> 2] >> (8 * (e & 3))) & 0xffu) != 0u) << (16 * half + e);
        }
      }
    } else {
      for (int e = 0; e < n; ++e) word |= (uint32_t)(src[e] != 0) << e;
    }
    bits[g] = word;
  }
}

// Transpose of one 64-row x 32-key block of bit words: lane l holds row
// i0 + l's word w (bits = keys 32w ..); afterwards lane j < 32 holds key
// 32w + j's bits of rows i0 .. i0+31 and lane 32 + j those of rows i0+32 ..
// i0+63, which it stores as that key's transposed word (rows i0/32 and
// i0/32 + 1). Keys past N and words past W are not stored.
//
// Each half-wave transposes its 32 x 32 bit matrix (lane r = row r) in five
// butterfly stages s = 16, 8, 4, 2, 1: lanes r and r ^ s exchange words, and
// the lane with (r & s) == 0 keeps its bits b with (b & s) == 0 and takes the
// partner's such bits shifted up by s, the other lane keeps its bits with
// (b & s) != 0 and takes the partner's shifted down by s, which swaps the
// off-diagonal s x s blocks of every 2s x 2s block (Hacker's Delight 7-3).
// Five exchanges and a few bit operations replace 32 ballots.
__device__ __forceinline__ uint32_t transpose32(uint32_t x, int lane) {
  constexpr uint32_t kKeep[5] = {0x0000FFFFu, 0x00FF00FFu, 0x0F0F0F0Fu, 0x33333333u, 0x55555555u};
#pragma unroll
  for (int t = 0; t < 5; ++t) {
    const int s = 16 >> t;
    const uint32_t y = (uint32_t)__shfl_xor((int)x, s);
    const bool lower = (lane & s) == 0;
    const uint32_t m = lower ? kKeep[t] : ~kKeep[t];  // the bits this lane keeps
    const uint32_t moved = lower ? (y << s) : (y >> s);
    x = (x & m) | (moved & ~m);
  }
  return x;
}

__device__ __forceinline__ void store_transposed(uint32_t word, int lane, int w, int i0, int N,
                                                 int W, uint32_t* __restrict__ plane_t) {
  const uint32_t mine = transpose32(word, lane);
  const int kj = 32 * w + (lane & 31);  // this lane's key
  const int rw = (i0 >> 5) + (lane >> 5);  // its word of query rows
  if (kj < N && rw < W) plane_t[(size_t)kj * W + rw] = mine;
}

// Words per wave of the transpose kernel (a wave per 64 rows alone left half
// the SIMDs idle at B*H = 8, N = 4096).
constexpr int kColWords = 8;

// The transposed words of packed rows: each wave owns 64 rows of one plane
// and kColWords of their words (rows past N read as zero words).
__global__ __launch_bounds__(kPackThreads) void pack_cols_kernel(
    const uint32_t* __restrict__ bits, uint32_t* __restrict__ bits_t, int N, int W,
    int row_blocks, int word_chunks) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int chunk = blockIdx.x % word_chunks;
  const int rest = blockIdx.x / word_chunks;
  const int plane = rest / row_blocks;
  const int i0 = ((rest % row_blocks) * (kPackThreads / 64) + wave) * 64;
  if (i0 >= N) return;  // wave-uniform; no barriers below
  const int i = i0 + lane;
  const uint32_t* row = bits + ((size_t)plane * N + (i < N ? i : 0)) * W;
  uint32_t* plane_t = bits_t + (size_t)plane * N * W;
  const int w_end = min(W, (chunk + 1) * kColWords);
  for (int w = chunk * kColWords; w < w_end; ++w)
    store_transposed(i < N ? row[w] : 0u, lane, w, i0, N, W, plane_t);
}

// Integer hash `lowbias32` (C. Wellons, hash-prospector): xorshift-multiply
// rounds with full avalanche, 2 multiplies per 32-bit output.
__device__ __forceinline__ uint32_t lowbias32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// Dropout keep bits. Draws: row key r = h(h(h(h(seed_lo) ^ seed_hi) ^ plane)
// ^ row); keys 2k and 2k+1 of the row draw the low and high 16 bits of
// h(r ^ k) (h = lowbias32); a key is kept iff its draw >= thr. Rows and keys
// past N get zero bits. causal: keys j > i of row i get zero bits (causal
// attention never reads them), and words whose keys all lie past a wave's
// last row are written as zeros without drawing: about half the hashes of a
// plane.
//
// An item is 256 rows (64 per wave, lane = row) x kDropWords words of one
// plane. Each lane keeps its row's words and stores them as one 16-byte
// run; each wave transposes its 64 x 32 blocks (transpose32) into an LDS
// tile, from which the workgroup stores every key's 8 words of the item's
// rows as one 32-byte run. With one 4-byte store per lane and word (a cache
// line per lane: 512 line writes per 64 x 8 block of either layout against
// 64 and 32 here) the causal draw took 35 us at B*H = 8, N = 4096; 26 us
// with these runs (the full draw took 44 us with the 4-byte stores).
constexpr int kDropWords = 4;
constexpr int kDropRows = kPackThreads;                // rows per item
constexpr int kDropKeys = 32 * kDropWords;             // keys per item
constexpr int kTrStride = kDropRows / 32 + 1;          // LDS words per key (padded)

__device__ __forceinline__ void dropout_item(uint32_t seed_key, uint32_t thr, int N, int W,
                                             int i0, int c, bool causal, bool vec,
                                             uint32_t* __restrict__ bits,
                                             uint32_t* __restrict__ bits_t, uint32_t* tr) {
  const int tid = threadIdx.x, lane = tid & 63, w4 = tid >> 6;
  const int iw = i0 + 64 * w4;  // this wave's first row
  const int i = iw + lane;
  const bool row_ok = i < N;
  const uint32_t key = lowbias32(seed_key ^ (uint32_t)i);
  const int w0 = c * kDropWords;
  const int w_end = min(W, w0 + kDropWords);
  // (words from w_vis on are zero for every row of the wave: past its last
  // row when causal, or rows that all lie past N)
  const int w_vis = iw >= N ? w0 : causal ? min(w_end, (iw + 63) / 32 + 1) : w_end;
  uint32_t words[kDropWords];
#pragma unroll
  for (int wl = 0; wl < kDropWords; ++wl) {
    const int w = w0 + wl;
    uint32_t word = 0u;
    if (w < w_vis) {  // wave-uniform
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const uint32_t u = lowbias32(key ^ (uint32_t)(16 * w + k));
        word |= (uint32_t)((u & 0xffffu) >= thr) << (2 * k);
        word |= (uint32_t)((u >> 16) >= thr) << (2 * k + 1);
      }
      const int nk = N - 32 * w;  // keys of this word that exist (>= 1)
      if (nk < 32) word &= (1u << nk) - 1u;
      if (causal) {  // keys 32w .. i of row i
        const int vis = i - 32 * w + 1;
        word &= vis >= 32 ? ~0u : vis > 0 ? (1u << vis) - 1u : 0u;
      }
      if (!row_ok) word = 0u;
    }
    words[wl] = word;
    if (bits_t) {
      // lane j < 32: key 32w + j's bits of rows iw .. iw+31; lane 32 + j: of
      // rows iw+32 .. iw+63 (row words 2 w4 and 2 w4 + 1 of the item)
      const uint32_t t = w < w_vis ? transpose32(word, lane) : 0u;
      tr[(32 * wl + (lane & 31)) * kTrStride + 2 * w4 + (lane >> 5)] = t;
    }
  }
  if (row_ok) {
    uint32_t* out = bits + (size_t)i * W + w0;
    if (vec && w0 + kDropWords <= W) {
      *reinterpret_cast<uint4*>(out) = make_uint4(words[0], words[1], words[2], words[3]);
    } else {
#pragma unroll
      for (int wl = 0; wl < kDropWords; ++wl)
        if (w0 + wl < W) out[wl] = words[wl];
    }
  }
  if (bits_t) {
    __syncthreads();
    // thread t: key kDropKeys c + t/2, row words i0/32 + 4 (t%2) .. + 3
    const int kl = tid >> 1, half = tid & 1;
    const int kj = 32 * w0 + kl;
    const int rw = i0 / 32 + 4 * half;
    if (kj < N) {
      uint32_t v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = tr[kl * kTrStride + 4 * half + r];
      uint32_t* dst = bits_t + (size_t)kj * W + rw;
      if (vec && rw + 4 <= W) {
        *reinterpret_cast<uint4*>(dst) = make_uint4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (rw + r < W) dst[r] = v[r];
      }
    }
    __syncthreads();  // (the tile is rewritten by the next item)
  }
}

// One workgroup per pair of items: item t of a plane's RB x WC items (row
// block t / WC, word chunk t % WC) with its mirror RB*WC - 1 - t (row block
// RB-1-rb, chunk WC-1-c). Under causal masking an item's hashes fall with
// its chunk and grow with its row block, so the pairs carry about the same
// work. vec: 16-byte stores (W % 4 == 0 and 16-byte aligned planes).
__global__ __launch_bounds__(kPackThreads) void dropout_bits_kernel(
    uint32_t seed_lo, uint32_t seed_hi, uint32_t thr, int N, int W, int RB, int WC, int n_pairs,
    bool causal, bool vec, uint32_t* __restrict__ bits, uint32_t* __restrict__ bits_t) {
  __shared__ uint32_t tr[kDropKeys * kTrStride];
  const int plane = (int)(blockIdx.x / (unsigned)n_pairs), t = (int)(blockIdx.x % (unsigned)n_pairs);
  const uint32_t seed_key =  // (row i's key is then h(seed_key ^ i))
      lowbias32(lowbias32(lowbias32(seed_lo) ^ seed_hi) ^ (uint32_t)plane);
  uint32_t* pb = bits + (size_t)plane * N * W;
  uint32_t* pt = bits_t ? bits_t + (size_t)plane * N * W : nullptr;
  dropout_item(seed_key, thr, N, W, (t / WC) * kDropRows, t % WC, causal, vec, pb, pt, tr);
  const int m = RB * WC - 1 - t;
  if (m != t)  // (workgroup-uniform: both items pass the same barriers)
    dropout_item(seed_key, thr, N, W, (m / WC) * kDropRows, m % WC, causal, vec, pb, pt, tr);
}

// Block-sparse lists (FwdArgs::block_rows, BwdArgs::block_cols) from a dense
// layout of Bl x Hl planes of nb x nb bytes (a plane index broadcasts when
// its count is 1). One thread per list scans its row (query block r of query
// head h) or its column (key block c over the group's query heads) in order,
// so the entries come out ascending; the unused tail repeats the last entry
// (0 for an empty list), so every entry is a valid index. The lists are
// small (nb + 1 ints per block row) next to the attention that reads them.
__device__ __forceinline__ const uint8_t* layout_plane(const uint8_t* layout, int Bl, int Hl,
                                                       int b, int h, int nb) {
  return layout + ((size_t)(Bl == 1 ? 0 : b) * Hl + (Hl == 1 ? 0 : h)) * nb * nb;
}

__global__ __launch_bounds__(kPackThreads) void block_rows_kernel(
    const uint8_t* __restrict__ layout, int Bl, int Hl, int B, int Hq, int nb, bool causal,
    int* __restrict__ rows) {
  const long long t = (long long)blockIdx.x * kPackThreads + threadIdx.x;  // (b, h, r)
  if (t >= (long long)B * Hq * nb) return;
  const int r = (int)(t % nb);
  const long long p = t / nb;
  const int h = (int)(p % Hq), b = (int)(p / Hq);
  const uint8_t* src = layout_plane(layout, Bl, Hl, b, h, nb) + (size_t)r * nb;
  int* out = rows + t * (nb + 1);
  const int end = causal ? r + 1 : nb;  // (causal: key blocks past the query block are hidden)
  int c = 0, last = 0;
  for (int k = 0; k < end; ++k)
    if (src[k]) {
      out[1 + c++] = k;
      last = k;
    }
  for (int k = c; k < nb; ++k) out[1 + k] = last;
  out[0] = c;
}

__global__ __launch_bounds__(kPackThreads) void block_cols_kernel(
    const uint8_t* __restrict__ layout, int Bl, int Hl, int B, int Hq, int Hkv, int nb,
    bool causal, int* __restrict__ cols) {
  const long long t = (long long)blockIdx.x * kPackThreads + threadIdx.x;  // (b, hkv, c)
  if (t >= (long long)B * Hkv * nb) return;
  const int c = (int)(t % nb);
  const long long p = t / nb;
  const int hkv = (int)(p % Hkv), b = (int)(p / Hkv);
  const int G = Hq / Hkv;
  int* out = cols + t * ((long long)G * nb + 1);
  int n = 0, last = 0;
  for (int g = 0; g < G; ++g) {
    const uint8_t* src = layout_plane(layout, Bl, Hl, b, hkv * G + g, nb) + c;
    for (int r = causal ? c : 0; r < nb; ++r)
      if (src[(size_t)r * nb]) {
        last = g * nb + r;
        out[1 + n++] = last;
      }
  }
  for (int k = n; k < G * nb; ++k) out[1 + k] = last;
  out[0] = n;
}

unsigned blocks_for(long long items) {
  const long long b = (items + kPackThreads - 1) / kPackThreads;
  return (unsigned)(b < kPackMaxBlocks ? (b > 0 ? b : 1) : kPackMaxBlocks);
}

}  // namespace

hipError_t launch_pack_mask(const uint8_t* dense, int P, int N, uint32_t* bits, uint32_t* bits_t,
                            void* stream) {
  const int W = (N + 31) / 32;
  const long long rows = (long long)P * N;
  const bool vec = N % 16 == 0 && (reinterpret_cast<uintptr_t>(dense) & 15u) == 0;
  if (vec)
    hipLaunchKernelGGL(pack_rows_kernel<true>, dim3(blocks_for(rows * W)), dim3(kPackThreads), 0,
                       (hipStream_t)stream, dense, bits, rows, N, W);
  else
    hipLaunchKernelGGL(pack_rows_kernel<false>, dim3(blocks_for(rows * W)), dim3(kPackThreads), 0,
                       (hipStream_t)stream, dense, bits, rows, N, W);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || bits_t == nullptr) return e;
  const int row_blocks = (N + kPackThreads - 1) / kPackThreads;
  const int word_chunks = (W + kColWords - 1) / kColWords;
  const long long blocks = (long long)P * row_blocks * word_chunks;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(pack_cols_kernel, dim3((unsigned)blocks), dim3(kPackThreads), 0,
                     (hipStream_t)stream, bits, bits_t, N, W, row_blocks, word_chunks);
  return hipGetLastError();
}

hipError_t launch_pack_blocks(const uint8_t* layout, int Bl, int Hl, int B, int Hq, int Hkv,
                              int nb, bool causal, int* rows, int* cols, void* stream) {
  const long long n_rows = (long long)B * Hq * nb, n_cols = (long long)B * Hkv * nb;
  if ((n_rows + kPackThreads - 1) / kPackThreads > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(block_rows_kernel, dim3((unsigned)((n_rows + kPackThreads - 1) / kPackThreads)),
                     dim3(kPackThreads), 0, (hipStream_t)stream, layout, Bl, Hl, B, Hq, nb, causal,
                     rows);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || cols == nullptr) return e;
  hipLaunchKernelGGL(block_cols_kernel, dim3((unsigned)((n_cols + kPackThreads - 1) / kPackThreads)),
                     dim3(kPackThreads), 0, (hipStream_t)stream, layout, Bl, Hl, B, Hq, Hkv, nb,
                     causal, cols);
  return hipGetLastError();
}

hipError_t launch_dropout_bits(uint64_t seed, uint32_t threshold, int P, int N, bool causal,
                               uint32_t* bits, uint32_t* bits_t, void* stream) {
  const int W = (N + 31) / 32;
  const int RB = (N + kDropRows - 1) / kDropRows;      // row blocks
  const int WC = (W + kDropWords - 1) / kDropWords;    // word chunks
  const long long n_pairs = ((long long)RB * WC + 1) / 2;
  const long long blocks = (long long)P * n_pairs;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  const bool vec = W % 4 == 0 && (reinterpret_cast<uintptr_t>(bits) & 15u) == 0 &&
                   (reinterpret_cast<uintptr_t>(bits_t) & 15u) == 0;
  hipLaunchKernelGGL(dropout_bits_kernel, dim3((unsigned)blocks), dim3(kPackThreads), 0,
                     (hipStream_t)stream, (uint32_t)seed, (uint32_t)(seed >> 32), threshold, N,
                     W, RB, WC, (int)n_pairs, causal, vec, bits, bits_t);
  return hipGetLastError();
}

}  // namespace fa
