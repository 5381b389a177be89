// Fast-posture GEMM on the fp32 matrix cores: v_mfma_f32_16x16x4_f32 on the
// LDS-DMA kernel, v_mfma_f32_32x32x2_f32 on the register-staged one.
//
// Envelope fidelity: the k-sum is blocked and reassociated by the matrix core,
// so results are compared against the exact product within
// |c - exact| <= 1e-5 * sum_k |a_ik * b_kj| (and are deterministic: the same
// inputs give the same bits on every run: no atomics, and a split along k is
// reduced in a fixed order).
//
// Shape: a BM x BN output tile per workgroup, each wave owning a 64x64 block
// (32x64 on the thin tiles). Tiles are 256x128 (eight waves) for products
// with enough tiles, 128x128, or 128x64 / 64x128 when one output extent is at
// most 64 (the attention products with a 64-wide head) or when those tiles
// fill whole rounds, so no half-empty tiles are launched. The LDS-DMA kernel
// stages k 16 deep in three LDS stages written by global_load_lds_dwordx4;
// the register-staged kernel (operands without a unit stride, and the 128x64
// tiles) double-buffers slabs through registers into [k][outer] LDS rows
// padded by 20 floats. A tile wholly inside the operands takes a branch-free
// load path (one uniform test per slab); only edge tiles pay per-element
// bounds checks.
// The forward product and both transposed backward products (A^T G with A
// m-contiguous, G B^T with B k-contiguous; src/function/matmul.rs:76-91) are
// served by the same kernel through the operand-orientation template flags, so
// no transpose is ever materialised.
#include <algorithm>

#include "backend.hpp"
#include "lds_dma.hpp"

namespace topos_hip {
namespace {

using namespace lds_dma;

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
// Four consecutive floats at any 4-byte-aligned address: gfx950 serves
// unaligned global_load_dwordx4, so operands with odd leading dimensions (the
// 50257-wide vocabulary products) keep 16-byte loads.
typedef float float4u __attribute__((ext_vector_type(4), aligned(4)));

constexpr int kTileK = 16;
constexpr int kPad = 20;
constexpr int kGroupM = 8;

// One operand slab (outer extent O, kTileK deep) between its global loads and
// its LDS store as [k][O + kPad]. Element (o, kk) of the operand lives at
// p[o * outer_stride + kk * k_stride]. kInnerK: k is the unit-stride axis
// (lanes step along k), else the outer axis is. kVector: the axis the lanes
// step along has unit stride, so four neighbours are one 16-byte load.
template <int O, int T, bool kInnerK, bool kVector>
struct Slab {
  static constexpr int V = O * kTileK / 4 / T;  // 4-vectors per lane
  float4 v[V];

  // The slab starting at (o0, k0) when it lies wholly inside the operand.
  __device__ inline void load_inside(const float *__restrict__ p, int64_t outer_stride, int64_t k_stride,
                                     int64_t o0, int64_t k0) {
    const int t = threadIdx.x;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const int x = t + T * e;
      const int o = kInnerK ? x / (kTileK / 4) : (x % (O / 4)) * 4;
      const int kk = kInnerK ? (x % (kTileK / 4)) * 4 : x / (O / 4);
      const int64_t go = o0 + o, gk = k0 + kk;
      if (kVector) {
        const float4u u = kInnerK ? *reinterpret_cast<const float4u *>(p + go * outer_stride + gk)
                                  : *reinterpret_cast<const float4u *>(p + gk * k_stride + go);
        v[e] = make_float4(u.x, u.y, u.z, u.w);
      } else if (kInnerK) {
        v[e] = make_float4(p[go * outer_stride + gk * k_stride], p[go * outer_stride + (gk + 1) * k_stride],
                           p[go * outer_stride + (gk + 2) * k_stride], p[go * outer_stride + (gk + 3) * k_stride]);
      } else {
        v[e] = make_float4(p[go * outer_stride + gk * k_stride], p[(go + 1) * outer_stride + gk * k_stride],
                           p[(go + 2) * outer_stride + gk * k_stride], p[(go + 3) * outer_stride + gk * k_stride]);
      }
    }
  }

  // Any slab: elements outside [0, outer_extent) x [.., k_end) read as zero.
  __device__ inline void load_edge(const float *__restrict__ p, int64_t outer_stride, int64_t k_stride,
                                   int64_t outer_extent, int64_t k_end, int64_t o0, int64_t k0) {
    const int t = threadIdx.x;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const int x = t + T * e;
      const int o = kInnerK ? x / (kTileK / 4) : (x % (O / 4)) * 4;
      const int kk = kInnerK ? (x % (kTileK / 4)) * 4 : x / (O / 4);
      const int64_t go = o0 + o, gk = k0 + kk;
      float w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (kInnerK)
          w[q] = (go < outer_extent && gk + q < k_end) ? p[go * outer_stride + (gk + q) * k_stride] : 0.0f;
        else
          w[q] = (gk < k_end && go + q < outer_extent) ? p[(go + q) * outer_stride + gk * k_stride] : 0.0f;
      }
      v[e] = make_float4(w[0], w[1], w[2], w[3]);
    }
  }

  __device__ inline void store(float (*lds)[O + kPad]) const {
    const int t = threadIdx.x;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const int x = t + T * e;
      if (kInnerK) {
        const int o = x / (kTileK / 4), kk = (x % (kTileK / 4)) * 4;
        lds[kk + 0][o] = v[e].x;
        lds[kk + 1][o] = v[e].y;
        lds[kk + 2][o] = v[e].z;
        lds[kk + 3][o] = v[e].w;
      } else {
        const int o = (x % (O / 4)) * 4, kk = x / (O / 4);
        *reinterpret_cast<float4 *>(&lds[kk][o]) = v[e];
      }
    }
  }
};

// The 256x128 tile (eight waves) with 16-byte loads is held to 128
// registers per lane so that two of its workgroups share a CU (four waves
// per SIMD); at the compiler's own choice (129) a CU held one.
// A wave's block of the output tile at (m0, n0) into c, with the bias
// epilogue (bias_mode 0 none, 1 product + bias[col], 2 bias[col] + product).
// kT: block (i, j) holds, for lane l, row 32i + l % 32 and columns
// 32j + 8g + 4(l / 32) + {0..3} in elements 4g..4g+3, stored 16 bytes at a
// time (the caller guarantees c and ldc allow it). Otherwise column
// 32j + l % 32 and rows 32i + 8(r / 4) + 4(l / 32) + r % 4 in element r.
template <int WM, bool kT>
__device__ __forceinline__ void store_block(const floatx16 (&acc)[WM / 32][2], float *__restrict__ c, int64_t ldc,
                                                int64_t m, int64_t n, int64_t m0, int64_t n0, int wm, int wn, int lane,
                                                const float *__restrict__ bias, int64_t bias_cs, int bias_mode) {
  constexpr int WI = WM / 32;
  if (!kT) {
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t col = n0 + wn + 32 * j + (lane % 32);
        if (col >= n) continue;
        const float add = bias_mode != 0 ? bias[col * bias_cs] : 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm + 32 * i + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
          float v = acc[i][j][r];
          if (bias_mode == 1) v = v + add;
          if (bias_mode == 2) v = add + v;
          if (row < m) c[row * ldc + col] = v;
        }
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < WI; ++i) {
    const int64_t row = m0 + wm + 32 * i + (lane % 32);
    if (row >= m) continue;
    float *out = c + row * ldc;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t col = n0 + wn + 32 * j + 8 * g + 4 * (lane / 32);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = acc[i][j][4 * g + e];
          if (bias_mode != 0 && col + e < n) {
            const float add = bias[(col + e) * bias_cs];
            v[e] = bias_mode == 1 ? v[e] + add : add + v[e];
          }
        }
        if (col + 3 < n) {
          *reinterpret_cast<float4 *>(out + col) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (col + e < n) out[col + e] = v[e];
        }
      }
  }
}

template <int BM, int BN, int WM, bool kLeftInnerK, bool kRightInnerK, bool kVector, bool kT>
__global__ __launch_bounds__(BM / WM * BN, BM == 256 && kVector ? 4 : 1) void gemm_mfma_kernel(
    const float *__restrict__ a, int64_t a_rs, int64_t a_cs, const float *__restrict__ b,
    int64_t b_rs, int64_t b_cs, int64_t m, int64_t k, int64_t n, float *__restrict__ c, int64_t ldc,
    int grid_m, int grid_n, int64_t a_bs, int64_t b_bs, int64_t c_bs, int64_t split_len, int64_t split_stride,
    const float *__restrict__ bias, int64_t bias_cs, int bias_mode, int64_t inner, int64_t a_bs2, int64_t b_bs2,
    int64_t c_bs2) {
  constexpr int T = BM / WM * BN;  // one WM x 64 block per wave
  constexpr int WN = BN / 64;
  constexpr int WI = WM / 32;      // 32-row MFMA blocks per wave
  __shared__ float left[2][kTileK][BM + kPad];
  __shared__ float right[2][kTileK][BN + kPad];
  {
    const int64_t outer = (int64_t)blockIdx.y / inner, within = (int64_t)blockIdx.y - outer * inner;
    a += outer * a_bs + within * a_bs2;
    b += outer * b_bs + within * b_bs2;
    c += outer * c_bs + within * c_bs2;
  }
  // Split k: this workgroup sums k in [k_begin, k_end) into its own partial
  // product (the fixed-order reduction adds the partials afterwards).
  const int64_t k_begin = (int64_t)blockIdx.z * split_len;
  const int64_t k_end = min(k, k_begin + split_len);
  c += (int64_t)blockIdx.z * split_stride;

  // Workgroups are dealt to the eight XCDs round-robin; renumber so each XCD
  // receives a contiguous run of tiles, then walk tiles in groups of kGroupM
  // block-rows so neighbouring tiles share operand panels in that XCD's L2.
  const int blocks = grid_m * grid_n;
  int pid = blockIdx.x;
  if (blocks % 8 == 0) pid = (pid % 8) * (blocks / 8) + pid / 8;
  const int in_group = kGroupM * grid_n;
  const int group = pid / in_group;
  const int first_m = group * kGroupM;
  const int group_rows = min(grid_m - first_m, kGroupM);
  const int tile_m = first_m + (pid % in_group) % group_rows;
  const int tile_n = (pid % in_group) / group_rows;
  const int64_t m0 = (int64_t)tile_m * BM;
  const int64_t n0 = (int64_t)tile_n * BN;
  const bool interior = m0 + BM <= m && n0 + BN <= n;

  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  const int wm = (wave / WN) * WM;  // wave's row offset inside the tile
  const int wn = (wave % WN) * 64;  // wave's column offset

  floatx16 acc[WI][2];
#pragma unroll
  for (int i = 0; i < WI; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // Left operand: outer = m (row stride a_rs), inner = k (a_cs).
  // Right operand: outer = n (b_cs), inner = k (b_rs).
  Slab<BM, T, kLeftInnerK, kVector> sa;
  Slab<BN, T, kRightInnerK, kVector> sb;
  // Both operands' loads for one slab. `inside` (the slab lies wholly inside
  // both operands) is uniform and kept the outermost branch: each path is one
  // straight run of loads, all in flight together.
  auto load = [&](int64_t k0) {
    if (interior && k0 + kTileK <= k_end) {
      sa.load_inside(a, a_rs, a_cs, m0, k0);
      sb.load_inside(b, b_cs, b_rs, n0, k0);
    } else {
      sa.load_edge(a, a_rs, a_cs, m, k_end, m0, k0);
      sb.load_edge(b, b_cs, b_rs, n, k_end, n0, k0);
    }
  };
  load(k_begin);
  sa.store(left[0]);
  sb.store(right[0]);
  __syncthreads();

  const int64_t slabs = (k_end - k_begin + kTileK - 1) / kTileK;
  for (int64_t s = 0; s < slabs; ++s) {
    const int cur = (int)(s & 1);
    const bool more = s + 1 < slabs;
    if (more) load(k_begin + (s + 1) * kTileK);
#pragma unroll
    for (int kk = 0; kk < kTileK; kk += 2) {
      const int kr = kk + lane / 32;
      float av[WI];
#pragma unroll
      for (int i = 0; i < WI; ++i) av[i] = left[cur][kr][wm + 32 * i + (lane % 32)];
      const float b0 = right[cur][kr][wn + (lane % 32)];
      const float b1 = right[cur][kr][wn + 32 + (lane % 32)];
#pragma unroll
      for (int i = 0; i < WI; ++i) {  // kT: transposed blocks (store_block)
        acc[i][0] = kT ? __builtin_amdgcn_mfma_f32_32x32x2f32(b0, av[i], acc[i][0], 0, 0, 0)
                       : __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], b0, acc[i][0], 0, 0, 0);
        acc[i][1] = kT ? __builtin_amdgcn_mfma_f32_32x32x2f32(b1, av[i], acc[i][1], 0, 0, 0)
                       : __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], b1, acc[i][1], 0, 0, 0);
      }
    }
    if (more) {
      sa.store(left[cur ^ 1]);
      sb.store(right[cur ^ 1]);
    }
    __syncthreads();
  }

  store_block<WM, kT>(acc, c, ldc, m, n, m0, n0, wm, wn, lane, bias, bias_cs, bias_mode);
}

// ---- the LDS-DMA variant ----
//
// Interior-friendly operands (16-byte aligned rows, k a multiple of 16) are
// staged by global_load_lds_dwordx4: each lane's 16 bytes land in LDS
// without passing through registers, so no LDS store instructions and no
// register staging. Three LDS stages: slab s + 2 is in flight while slab s
// feeds the matrix cores, and each wave waits only for slab s + 1's loads
// (vmcnt) before the one barrier per slab. A wave-wide DMA writes 1 KB at
// consecutive 16-byte positions, so the layouts are chosen through which
// address each lane loads:
//  * k-contiguous operand: 16 rows x 16 k per KB; the k-quad q of local row
//    r sits at position 4r + (q ^ swz(r)) (conflict-free 16-byte fragment
//    reads for 32 or 64 banks). A fragment read gives a lane the four k
//    values of one quad; the 16x16x4 MFMAs then take k = 4g + t from the
//    lanes of group g (the other operand is read in the same k order).
//  * outer-contiguous operand: k-rows of O floats; quad j of row kk sits at
//    quad position j ^ (kk & 4 ? 8 : 0) (rows kk and kk + 4, read by
//    neighbouring lane groups together, land on different banks).
// Rows or columns past the operand's edge load a clamped in-range address;
// they only feed outputs that are not stored.
template <int O>
__device__ __forceinline__ int dma_outer_index(int kk, int o) {
  return kk * O + (((o >> 2) ^ ((kk & 4) ? 8 : 0)) << 2) + (o & 3);
}

// One slab (16 deep) of an operand with outer extent O into `lds`.
template <int O, int W, bool kInnerK>
__device__ __forceinline__ void dma_slab(const float *__restrict__ p, int64_t outer_stride, int64_t k_stride,
                                         int64_t outer_extent, int64_t o0, int64_t k0, float *lds, int wave,
                                         int lane) {
  constexpr int kChunks = O * kTileK / 256;  // 1 KB per wave-wide load
  static_assert(kChunks % W == 0, "whole chunks per wave");
#pragma unroll
  for (int i = 0; i < kChunks / W; ++i) {
    const int c = wave + W * i;
    const float *src;
    if (kInnerK) {
      const int r = lane >> 2;
      const int q = (lane & 3) ^ dma_swizzle(r);
      const int64_t row = min(o0 + 16 * c + r, outer_extent - 1);
      src = p + row * outer_stride + (k0 + 4 * q);
    } else {
      constexpr int kRows = 256 / O;  // k-rows per chunk
      const int kk = c * kRows + lane / (O / 4);
      const int quad = (lane % (O / 4)) ^ ((kk & 4) ? 8 : 0);
      const int64_t col = min(o0 + 4 * quad, outer_extent - 4);
      src = p + (k0 + kk) * k_stride + col;
    }
    TOPOS_COMPILER_FENCE();
    dma_load16(src, lds_byte_address(lds) + 1024 * c);
    TOPOS_COMPILER_FENCE();
  }
}

// The same slab through registers, element by element, with zeros past k_end
// and past the outer extent: the slabs a 16-byte load could not serve (a k
// tail, or a partial quad of an outer-contiguous operand whose extent is not
// a multiple of four). Same LDS layout as dma_slab.
template <int O, int W, bool kInnerK>
__device__ __forceinline__ void guarded_slab(const float *__restrict__ p, int64_t outer_stride, int64_t k_stride,
                                             int64_t outer_extent, int64_t k_end, int64_t o0, int64_t k0, float *lds,
                                             int wave, int lane) {
  constexpr int kChunks = O * kTileK / 256;
#pragma unroll
  for (int i = 0; i < kChunks / W; ++i) {
    const int c = wave + W * i;
    float v[4];
    if (kInnerK) {
      const int r = lane >> 2;
      const int q = (lane & 3) ^ dma_swizzle(r);
      const int64_t row = o0 + 16 * c + r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t kk = k0 + 4 * q + e;
        v[e] = row < outer_extent && kk < k_end ? p[row * outer_stride + kk * k_stride] : 0.0f;
      }
    } else {
      constexpr int kRows = 256 / O;
      const int kk = c * kRows + lane / (O / 4);
      const int quad = (lane % (O / 4)) ^ ((kk & 4) ? 8 : 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t col = o0 + 4 * quad + e;
        v[e] = col < outer_extent && k0 + kk < k_end ? p[(k0 + kk) * k_stride + col * outer_stride] : 0.0f;
      }
    }
    *reinterpret_cast<float4 *>(lds + c * 256 + 4 * lane) = make_float4(v[0], v[1], v[2], v[3]);
  }
}

// One slab's fragment reads and 16x16x4 matrix-core products for a wave's
// WM x 64 block, as (WM / 16) x 4 blocks of 16x16. Lane l reads the four
// consecutive k values 4g..4g+3 (g = l / 16) of its row or column l % 16; MFMA
// t of the slab takes k = 4g + t in its k slot g, so a 16-deep slab is four
// MFMAs of four terms each. (Measured on MI355X against the 32x32x2 form with
// the same tiles: 2-6% faster on the GPT-2 step's shapes.)
template <int BM, int BN, int WM, bool kLeftInnerK, bool kRightInnerK, bool kT>
__device__ __forceinline__ void dma_mfma_slab16(const float *sa, const float *sb, int wm, int wn, int lane,
                                                floatx4 (&acc)[WM / 16][4]) {
  constexpr int WI = WM / 16;
  const int l16 = lane % 16, g = lane / 16;
  float av[WI][4], bv[4][4];
#pragma unroll
  for (int i = 0; i < WI; ++i) {
    const int row = wm + 16 * i + l16;
    if (kLeftInnerK) {
      const float4 v = *reinterpret_cast<const float4 *>(
          sa + 256 * (row >> 4) + 4 * (4 * (row & 15) + (g ^ dma_swizzle(row & 15))));
      av[i][0] = v.x;
      av[i][1] = v.y;
      av[i][2] = v.z;
      av[i][3] = v.w;
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) av[i][t] = sa[dma_outer_index<BM>(4 * g + t, row)];
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = wn + 16 * j + l16;
    if (kRightInnerK) {
      const float4 v = *reinterpret_cast<const float4 *>(
          sb + 256 * (col >> 4) + 4 * (4 * (col & 15) + (g ^ dma_swizzle(col & 15))));
      bv[j][0] = v.x;
      bv[j][1] = v.y;
      bv[j][2] = v.z;
      bv[j][3] = v.w;
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) bv[j][t] = sb[dma_outer_index<BN>(4 * g + t, col)];
    }
  }
  // kT: the products go in as B^T A^T, so a lane holds one output row
  // (16i + l % 16) and four consecutive columns (16j + 4g + {0..3}).
  // Otherwise a lane holds one column (16j + l % 16) and rows 16i + 4g + r.
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = kT ? __builtin_amdgcn_mfma_f32_16x16x4f32(bv[j][t], av[i][t], acc[i][j], 0, 0, 0)
                       : __builtin_amdgcn_mfma_f32_16x16x4f32(av[i][t], bv[j][t], acc[i][j], 0, 0, 0);
}

// A wave's block of 16x16 accumulator blocks (dma_mfma_slab16's layouts) into
// c, with the bias epilogue (bias_mode as store_block's).
template <int WM, bool kT>
__device__ __forceinline__ void store_block16(const floatx4 (&acc)[WM / 16][4], float *__restrict__ c, int64_t ldc,
                                              int64_t m, int64_t n, int64_t m0, int64_t n0, int wm, int wn, int lane,
                                              const float *__restrict__ bias, int64_t bias_cs, int bias_mode) {
  constexpr int WI = WM / 16;
  const int l16 = lane % 16, g = lane / 16;
  if (!kT) {
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t col = n0 + wn + 16 * j + l16;
        if (col >= n) continue;
        const float add = bias_mode != 0 ? bias[col * bias_cs] : 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t row = m0 + wm + 16 * i + 4 * g + r;
          float v = acc[i][j][r];
          if (bias_mode == 1) v = v + add;
          if (bias_mode == 2) v = add + v;
          if (row < m) c[row * ldc + col] = v;
        }
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < WI; ++i) {
    const int64_t row = m0 + wm + 16 * i + l16;
    if (row >= m) continue;
    float *out = c + row * ldc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = n0 + wn + 16 * j + 4 * g;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = acc[i][j][e];
        if (bias_mode != 0 && col + e < n) {
          const float add = bias[(col + e) * bias_cs];
          v[e] = bias_mode == 1 ? v[e] + add : add + v[e];
        }
      }
      if (col + 3 < n) {
        *reinterpret_cast<float4 *>(out + col) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (col + e < n) out[col + e] = v[e];
      }
    }
  }
}

// store_block_staged for 16x16 accumulator blocks of a 64-row wave (kT):
// each half of the wave's 64x64 block (32 rows) is parked in the wave's own
// LDS region, then every store instruction writes four whole 256-byte row
// segments. `stage` holds 32 x 68 floats for this wave.
__device__ __forceinline__ void store_block_staged16(const floatx4 (&acc)[4][4], float *__restrict__ c, int64_t ldc,
                                                     int64_t m0, int64_t n0, int wm, int wn, int lane,
                                                     const float *__restrict__ bias, int64_t bias_cs, int bias_mode,
                                                     float *stage) {
  constexpr int kStride = 68;
  const int l16 = lane % 16, g = lane / 16;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = 16 * j + 4 * g;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = acc[2 * h + ii][j][e];
          if (bias_mode != 0) {
            const float add = bias[(n0 + wn + col + e) * bias_cs];
            v[e] = bias_mode == 1 ? v[e] + add : add + v[e];
          }
        }
        *reinterpret_cast<float4 *>(stage + (16 * ii + l16) * kStride + col) = make_float4(v[0], v[1], v[2], v[3]);
      }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's LDS writes done (lgkmcnt(0))
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int row = 4 * q + lane / 16, col = 4 * (lane % 16);
      const float4 v = *reinterpret_cast<const float4 *>(stage + row * kStride + col);
      *reinterpret_cast<float4 *>(c + (m0 + wm + 32 * h + row) * ldc + n0 + wn + col) = v;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // the reads are done before the next half overwrites
  }
}

template <int BM, int BN, int WM, bool kLeftInnerK, bool kRightInnerK, bool kT>
// (Register budgets: 128 for the 256-row tiles, two workgroups a CU; 168 for
// the others, three a CU.)
__global__ __launch_bounds__(BM / WM * BN, BM == 256 ? 4 : 3) void gemm_dma_kernel(
    const float *__restrict__ a, int64_t a_rs, int64_t a_cs, const float *__restrict__ b, int64_t b_rs,
    int64_t b_cs, int64_t m, int64_t k, int64_t n, float *__restrict__ c, int64_t ldc, int grid_m, int grid_n,
    int64_t a_bs, int64_t b_bs, int64_t c_bs, int64_t split_len, int64_t split_stride,
    const float *__restrict__ bias, int64_t bias_cs, int bias_mode, int64_t inner, int64_t a_bs2, int64_t b_bs2,
    int64_t c_bs2) {
  constexpr int W = BM / WM * BN / 64;  // waves, one WM x 64 block each
  constexpr int WI = WM / 32;           // 32-row MFMA blocks per wave
  constexpr int WN = BN / 64;
  constexpr int SA = BM * kTileK, SB = BN * kTileK;  // floats per stage
  constexpr int kIssue = BM * kTileK / 256 / W + BN * kTileK / 256 / W;  // DMA loads per wave per slab
  __shared__ __attribute__((aligned(1024))) float lds[3 * (SA + SB)];
  {
    const int64_t outer = (int64_t)blockIdx.y / inner, within = (int64_t)blockIdx.y - outer * inner;
    a += outer * a_bs + within * a_bs2;
    b += outer * b_bs + within * b_bs2;
    c += outer * c_bs + within * c_bs2;
  }
  const int64_t k_begin = (int64_t)blockIdx.z * split_len;
  const int64_t k_end = min(k, k_begin + split_len);
  c += (int64_t)blockIdx.z * split_stride;

  const int blocks = grid_m * grid_n;
  int pid = blockIdx.x;
  if (blocks % 8 == 0) pid = (pid % 8) * (blocks / 8) + pid / 8;
  const int in_group = kGroupM * grid_n;
  const int group = pid / in_group;
  const int first_m = group * kGroupM;
  const int group_rows = min(grid_m - first_m, kGroupM);
  const int tile_m = first_m + (pid % in_group) % group_rows;
  const int tile_n = (pid % in_group) / group_rows;
  const int64_t m0 = (int64_t)tile_m * BM;
  const int64_t n0 = (int64_t)tile_n * BN;

  const int lane = threadIdx.x % 64;
  // Wave-uniform (a scalar register): the DMA's LDS addresses, the waves'
  // block origins and the stage offsets stay scalar arithmetic.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const int wm = (wave / WN) * WM;
  const int wn = (wave % WN) * 64;

  floatx4 acc[WM / 16][4];
#pragma unroll
  for (int i = 0; i < WM / 16; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;

  // Slabs a 16-byte load cannot serve go through registers (uniform tests).
  const bool ragged_a = !kLeftInnerK && m % 4 != 0 && m0 + BM > m;
  const bool ragged_b = !kRightInnerK && n % 4 != 0 && n0 + BN > n;
  auto issue = [&](int s, int st) {
    float *stage = lds + st * (SA + SB);
    const int64_t k0 = k_begin + (int64_t)s * kTileK;
    const bool tail = k0 + kTileK > k_end;
    if (tail || ragged_a)
      guarded_slab<BM, W, kLeftInnerK>(a, a_rs, a_cs, m, k_end, m0, k0, stage, wave, lane);
    else
      dma_slab<BM, W, kLeftInnerK>(a, a_rs, a_cs, m, m0, k0, stage, wave, lane);
    if (tail || ragged_b)
      guarded_slab<BN, W, kRightInnerK>(b, b_cs, b_rs, n, k_end, n0, k0, stage + SA, wave, lane);
    else
      dma_slab<BN, W, kRightInnerK>(b, b_cs, b_rs, n, n0, k0, stage + SA, wave, lane);
  };
  const int slabs = (int)((k_end - k_begin + kTileK - 1) / kTileK);
  issue(0, 0);
  if (slabs > 1) {
    issue(1, 1);
    dma_wait<kIssue>();
  } else {
    dma_wait<0>();
  }
  dma_barrier();
  // Three slabs a trip while slab s + 4 is a whole slab (and the tile takes
  // only DMA slabs): the stages are compile-time offsets and a slab has no branch
  // of its own (measured on MI355X: 2-8% on the GPT-2 step's product
  // shapes). The last slabs, and every slab of a ragged edge tile, take the
  // general loop. Slab s lives in stage s % 3.
  int s = 0;
  if (!ragged_a && !ragged_b) {
    auto steady = [&](int st) {
      const int64_t k0 = k_begin + (int64_t)(s + 2) * kTileK;
      float *stage = lds + (st == 0 ? 2 : st - 1) * (SA + SB);
      dma_slab<BM, W, kLeftInnerK>(a, a_rs, a_cs, m, m0, k0, stage, wave, lane);
      dma_slab<BN, W, kRightInnerK>(b, b_cs, b_rs, n, n0, k0, stage + SA, wave, lane);
      const float *sa = lds + st * (SA + SB);
      dma_mfma_slab16<BM, BN, WM, kLeftInnerK, kRightInnerK, kT>(sa, sa + SA, wm, wn, lane, acc);
      dma_wait<kIssue>();
      dma_barrier();
      ++s;
    };
    const int whole = (int)((k_end - k_begin) / kTileK);  // slabs without a k tail
    while (s + 5 <= whole) {
      steady(0);
      steady(1);
      steady(2);
    }
  }
  for (; s < slabs; ++s) {
    if (s + 2 < slabs) issue(s + 2, (s + 2) % 3);
    const float *sa = lds + (s % 3) * (SA + SB);
    const float *sb = sa + SA;
    dma_mfma_slab16<BM, BN, WM, kLeftInnerK, kRightInnerK, kT>(sa, sb, wm, wn, lane, acc);
    if (s + 1 < slabs) {
      if (s + 2 < slabs)
        dma_wait<kIssue>();
      else
        dma_wait<0>();
      dma_barrier();
    }
  }

  // Interior tiles of 64-row waves store through LDS in whole row segments
  // (measured on the attention-scores product, which writes 402 MB for 12.9
  // GFLOP: 198 -> 172 us), where every wave's 32 x 68 stage fits the tile's
  // three slab stages (not the sixteen waves of a 256x256 tile).
  if constexpr (kT && WM == 64 && (BM / WM) * (BN / 64) * 32 * 68 <= 3 * (SA + SB)) {
    if (m0 + BM <= m && n0 + BN <= n) {
      dma_barrier();  // every wave's last fragment reads are done before LDS is reused
      store_block_staged16(acc, c, ldc, m0, n0, wm, wn, lane, bias, bias_cs, bias_mode, lds + wave * 32 * 68);
      return;
    }
  }
  store_block16<WM, kT>(acc, c, ldc, m, n, m0, n0, wm, wn, lane, bias, bias_cs, bias_mode);
}

// The tile shape for an m x n product over k (and `batches`): 128x64 or
// 64x128 when one output extent is at most 64; 256x256 (sixteen waves, LDS-DMA
// operands only, never split) for four rounds or more of such tiles; 256x128 (eight waves, less
// operand traffic per flop than 128x128) when its tiles fill whole rounds of
// two workgroups per CU, or at least one and a half such rounds (measured on
// MI355X: the [8192, 3072] products gain, [8192, 2304] loses); 64x128 when k
// is at most 4096 and those tiles fill whole rounds of three workgroups per
// CU (measured in the GPT-2 step: the [8192, 768] products over k = 768 took
// 95 us against 106 on 128x128 tiles in two ranges, [8192, 2304] over 768
// 262 against 269; [8192, 768] over 3072 ran at 127 TFLOP/s unsplit against
// 121 on 128x128 tiles in two ranges); else 128x128. `per_cu` is how many of
// its workgroups a CU holds at once.
struct TileShape {
  int bm, bn, per_cu;
};
TileShape tile_shape(int64_t m, int64_t n, int64_t k, int64_t batches) {
  if (n <= 64 && m > 64) return {128, 64, 3};
  if (m <= 64 && n > 64) return {64, 128, 3};
  const int64_t wide = ((m + 255) / 256) * ((n + 127) / 128) * batches;
  // (Not when the rows would pad a 256-row tile by more than an eighth: the
  // Llama key gradient, 32 x [128, 2048] over 2048, ran at 66 TFLOP/s on
  // half-empty 256x128 tiles. Nor for k of at most 128, whose tiles are
  // mostly epilogue: the attention scores, on the 64x128 tiles below, took
  // the GPT-2 step from 73.3 to 72.8 ms in a same-box A/B; 128x128 tiles
  // for them measured the same on GPT-2 and 0.3 ms slower on Llama.)
  const bool rows_fill = ((m + 255) / 256 * 256 - m) * 8 <= m;
  // 256x256 tiles (sixteen waves, one workgroup a CU: half the operand
  // traffic per product of 256x128) for products of at least four full
  // rounds of them, unsplit: the GPT-2 vocabulary head, [8192, 50257] over
  // 768, went from 5.06 to 4.78 ms inside the step; [50257, 768] over 8192
  // (591 such tiles) ran 5.5-6.8 ms against 5.1 on 256x128 tiles.
  const bool cols_fill = ((n + 255) / 256 * 256 - n) * 8 <= n;
  if (rows_fill && cols_fill && k > 128 && ((m + 255) / 256) * ((n + 255) / 256) * batches >= 1024)
    return {256, 256, 1};
  if (rows_fill && k > 128 && (wide >= 768 || (wide >= 512 && wide % 512 == 0))) return {256, 128, 2};
  const int64_t thin = ((m + 63) / 64) * ((n + 127) / 128) * batches;
  if (k <= 4096 && thin >= 768 && thin % 768 == 0) return {64, 128, 3};
  return {128, 128, 3};
}

// Rows of one wave's block: 64, or 32 for the thin tiles (128x64, 64x128),
// which then run four waves instead of two. A thin product (an attention
// head's 64-wide operand) has few tiles, so two waves per tile leave most
// SIMDs with a single wave and nothing to hide its waits behind.
constexpr int wave_rows(int bm, int bn) { return bm == 64 || bn == 64 ? 32 : 64; }

template <int BM, int BN, bool kL, bool kR>
void dispatch_vector(bool vector, bool vector_out, dim3 grid, hipStream_t stream, const float *a, int64_t a_rs,
                     int64_t a_cs, const float *b, int64_t b_rs, int64_t b_cs, int64_t m, int64_t k,
                     int64_t n, float *c, int64_t ldc, int gm, int gn, const Batch &batch, int64_t c_bs,
                     int64_t c_bs2, int64_t split_len, int64_t split_stride, const Epilogue &e, int mode) {
  constexpr int WM = wave_rows(BM, BN);
  constexpr int T = BM / WM * BN;
#define TOPOS_MFMA_ARGS                                                                                        \
  a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, gm, gn, batch.a_stride, batch.b_stride, c_bs, split_len,    \
      split_stride, e.bias, e.bias_stride, mode, batch.inner, batch.a_inner, batch.b_inner, c_bs2
  if (vector && vector_out)
    gemm_mfma_kernel<BM, BN, WM, kL, kR, true, true><<<grid, T, 0, stream>>>(TOPOS_MFMA_ARGS);
  else if (vector)
    gemm_mfma_kernel<BM, BN, WM, kL, kR, true, false><<<grid, T, 0, stream>>>(TOPOS_MFMA_ARGS);
  else
    gemm_mfma_kernel<BM, BN, WM, kL, kR, false, false><<<grid, T, 0, stream>>>(TOPOS_MFMA_ARGS);
#undef TOPOS_MFMA_ARGS
}

template <int BM, int BN>
void dispatch_orientation(bool lk, bool rk, bool vector, bool vector_out, dim3 grid, hipStream_t stream, const float *a,
                          int64_t a_rs, int64_t a_cs, const float *b, int64_t b_rs, int64_t b_cs, int64_t m,
                          int64_t k, int64_t n, float *c, int64_t ldc, int gm, int gn, const Batch &batch,
                          int64_t c_bs, int64_t c_bs2, int64_t split_len, int64_t split_stride, const Epilogue &e,
                          int mode) {
  if (lk && rk)
    dispatch_vector<BM, BN, true, true>(vector, vector_out, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, gm, gn, batch, c_bs, c_bs2, split_len, split_stride, e, mode);
  else if (lk)
    dispatch_vector<BM, BN, true, false>(vector, vector_out, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, gm, gn, batch, c_bs, c_bs2, split_len, split_stride, e, mode);
  else if (rk)
    dispatch_vector<BM, BN, false, true>(vector, vector_out, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, gm, gn, batch, c_bs, c_bs2, split_len, split_stride, e, mode);
  else
    dispatch_vector<BM, BN, false, false>(vector, vector_out, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, gm, gn, batch, c_bs, c_bs2, split_len, split_stride, e, mode);
}

template <int BM, int BN>
void dispatch_dma(bool lk, bool rk, bool vector_out, dim3 grid, hipStream_t stream, const float *a, int64_t a_rs,
                  int64_t a_cs,
                  const float *b, int64_t b_rs, int64_t b_cs, int64_t m, int64_t k, int64_t n, float *c, int64_t ldc,
                  int gm, int gn, const Batch &batch, int64_t c_bs, int64_t c_bs2, int64_t split_len,
                  int64_t split_stride, const Epilogue &e, int mode) {
  constexpr int WM = wave_rows(BM, BN);
  constexpr int T = BM / WM * BN;
#define TOPOS_DMA_ARGS                                                                                           \
  a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, gm, gn, batch.a_stride, batch.b_stride, c_bs, split_len, \
      split_stride, e.bias, e.bias_stride, mode, batch.inner, batch.a_inner, batch.b_inner, c_bs2
#define TOPOS_DMA_ORIENT(kT)                                                  \
  if (lk && rk)                                                               \
    gemm_dma_kernel<BM, BN, WM, true, true, kT><<<grid, T, 0, stream>>>(TOPOS_DMA_ARGS);   \
  else if (lk)                                                                \
    gemm_dma_kernel<BM, BN, WM, true, false, kT><<<grid, T, 0, stream>>>(TOPOS_DMA_ARGS);  \
  else if (rk)                                                                \
    gemm_dma_kernel<BM, BN, WM, false, true, kT><<<grid, T, 0, stream>>>(TOPOS_DMA_ARGS);  \
  else                                                                        \
    gemm_dma_kernel<BM, BN, WM, false, false, kT><<<grid, T, 0, stream>>>(TOPOS_DMA_ARGS);
  if (vector_out) {
    TOPOS_DMA_ORIENT(true)
  } else {
    TOPOS_DMA_ORIENT(false)
  }
#undef TOPOS_DMA_ORIENT
#undef TOPOS_DMA_ARGS
}

// A 16-byte load with the nontemporal hint: the partials are read once, and
// the hint leaves the last-level cache to the reduced output, which the next
// launch reads.
__device__ __forceinline__ float4 load_once(const float4 *p) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  const f4v w = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(p));
  return make_float4(w.x, w.y, w.z, w.w);
}

// The fixed-order sum of `splits` partial products (each [count][m][n],
// contiguous) into c: partial 0 seeds, then 1, 2, ... are added in order, so
// the result is the same on every run. Four consecutive elements per lane:
// every split's 16-byte load is issued before the additions. (The caller
// guarantees n % 4 == 0, so a quad never leaves its row, and fewer than 2^32
// quads per partial.) `aligned`: c, ldc and c_bs allow one 16-byte store.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float4 *__restrict__ partials, int splits,
                                                           uint32_t split_quads, uint32_t m, uint32_t row_quads,
                                                           float *__restrict__ c, int64_t ldc, int64_t c_bs,
                                                           const float *__restrict__ bias, int64_t bias_cs,
                                                           int bias_mode, bool aligned) {
  constexpr int kMax = 16;
  for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < split_quads; e += gridDim.x * blockDim.x) {
    float4 v[kMax];
#pragma unroll
    for (int s = 0; s < kMax; ++s)
      if (s < splits) v[s] = load_once(partials + (size_t)s * split_quads + e);
    float4 acc = v[0];
#pragma unroll
    for (int s = 1; s < kMax; ++s)
      if (s < splits) {
        acc.x = acc.x + v[s].x;
        acc.y = acc.y + v[s].y;
        acc.z = acc.z + v[s].z;
        acc.w = acc.w + v[s].w;
      }
    const uint32_t row = e / row_quads, col = (e - row * row_quads) * 4;
    const uint32_t q = row / m, r = row - q * m;
    if (bias_mode != 0) {
      const float b0 = bias[col * bias_cs], b1 = bias[(col + 1) * bias_cs], b2 = bias[(col + 2) * bias_cs],
                  b3 = bias[(col + 3) * bias_cs];
      if (bias_mode == 1) {
        acc.x = acc.x + b0;
        acc.y = acc.y + b1;
        acc.z = acc.z + b2;
        acc.w = acc.w + b3;
      } else {
        acc.x = b0 + acc.x;
        acc.y = b1 + acc.y;
        acc.z = b2 + acc.z;
        acc.w = b3 + acc.w;
      }
    }
    float *out = c + q * c_bs + r * ldc + col;
    if (aligned) {
      *reinterpret_cast<float4 *>(out) = acc;
    } else {
      out[0] = acc.x;
      out[1] = acc.y;
      out[2] = acc.z;
      out[3] = acc.w;
    }
  }
}

// split_reduce_kernel over a contiguous output in quads of the flat
// [count][m][n] array (n need not be a multiple of four; the caller
// guarantees count * m * n is): the same fixed-order sum of the partials,
// then the bias of each element's own column.
__global__ __launch_bounds__(256) void split_reduce_flat_kernel(const float4 *__restrict__ partials, int splits,
                                                                uint32_t split_quads, uint32_t n,
                                                                float *__restrict__ c, const float *__restrict__ bias,
                                                                int64_t bias_cs, int bias_mode, bool aligned) {
  constexpr int kMax = 16;
  for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < split_quads; e += gridDim.x * blockDim.x) {
    float4 v[kMax];
#pragma unroll
    for (int s = 0; s < kMax; ++s)
      if (s < splits) v[s] = load_once(partials + (size_t)s * split_quads + e);
    float4 acc = v[0];
#pragma unroll
    for (int s = 1; s < kMax; ++s)
      if (s < splits) {
        acc.x = acc.x + v[s].x;
        acc.y = acc.y + v[s].y;
        acc.z = acc.z + v[s].z;
        acc.w = acc.w + v[s].w;
      }
    float out[4] = {acc.x, acc.y, acc.z, acc.w};
    if (bias_mode != 0) {
      const uint64_t first = (uint64_t)e * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float b = bias[(int64_t)((first + q) % n) * bias_cs];
        out[q] = bias_mode == 1 ? out[q] + b : b + out[q];
      }
    }
    float *dst = c + (size_t)e * 4;
    if (aligned) {
      *reinterpret_cast<float4 *>(dst) = make_float4(out[0], out[1], out[2], out[3]);
    } else {
      dst[0] = out[0];
      dst[1] = out[1];
      dst[2] = out[2];
      dst[3] = out[3];
    }
  }
}

}  // namespace

void launch_split_reduce(const float *partials, int splits, int64_t m, int64_t n, float *c, int64_t ldc,
                         hipStream_t stream) {
  const int64_t quads = m * n / 4;
  const bool flat = ldc == n && (m * n) % 4 == 0;
  if (splits < 1 || splits > 16 || m < 0 || n < 0 || (!flat && n % 4 != 0) || quads >= (int64_t(1) << 32) ||
      reinterpret_cast<uintptr_t>(partials) % 16 != 0)
    throw Unsupported{"split reduce: partials outside what the reduction takes"};
  if (quads == 0) return;
  int64_t blocks = (quads + 255) / 256;
  if (blocks > 256 * 32) blocks = 256 * 32;
  if (flat) {
    split_reduce_flat_kernel<<<(unsigned)blocks, 256, 0, stream>>>(
        reinterpret_cast<const float4 *>(partials), splits, (uint32_t)quads, (uint32_t)n, c, nullptr, 0, 0,
        reinterpret_cast<uintptr_t>(c) % 16 == 0);
  } else {
    split_reduce_kernel<<<(unsigned)blocks, 256, 0, stream>>>(
        reinterpret_cast<const float4 *>(partials), splits, (uint32_t)quads, (uint32_t)m, (uint32_t)(n / 4), c, ldc,
        0, nullptr, 0, 0, reinterpret_cast<uintptr_t>(c) % 16 == 0 && ldc % 4 == 0);
  }
  check_launch("split_reduce_kernel launch");
}

int mfma_splits(int64_t m, int64_t n, int64_t k, int64_t batches) {
  // A full chip holds per_cu workgroups on each of the 256 CUs; a product
  // with fewer tiles is split along k until it reaches that, each split at
  // least 256 deep (64 below k = 1024), and deep products are split further
  // (up to 2048 workgroups while each split stays 512 deep): measured on
  // MI355X, the partial products' extra traffic costs less than idle CUs.
  const TileShape shape = tile_shape(m, n, k, batches);
  if (shape.bn == 256) return 1;  // four rounds or more of whole tiles
  const int64_t tiles = ((m + shape.bm - 1) / shape.bm) * ((n + shape.bn - 1) / shape.bn) * batches;
  const int64_t full = 256 * shape.per_cu;
  if (tiles >= full) {
    // Enough tiles to fill the chip, but the last round of workgroups may
    // run mostly empty (1179 tiles over 512 slots run as three rounds, the
    // last 30% full). Splitting k multiplies the workgroups and shortens
    // each, so the rounds fill better; it pays when the slab rounds saved
    // outweigh writing and re-reading the partials. Cost model, in rounds of
    // one 16-deep slab on every slot: rounds x slabs, plus the partials'
    // (splits + 1) passes over m x n at 6 TB/s. A split must save 10% and
    // stay 512 deep.
    const double slab_round_s = 2.0 * shape.bm * shape.bn * kTileK * full / (0.7 * 157.3e12);
    const double partial_bytes = 4.0 * (double)batches * (double)m * (double)n;
    auto cost = [&](int64_t s) {
      const int64_t rounds = (tiles * s + full - 1) / full;
      const int64_t slabs = ((k + s - 1) / s + kTileK - 1) / kTileK;
      const double partials = s > 1 ? (double)(s + 1) * partial_bytes / 6e12 / slab_round_s : 0.0;
      return (double)rounds * (double)slabs + partials;
    };
    int64_t best = 1;
    for (int64_t s = 2; s <= 8 && k / s >= 512; ++s)
      if (cost(s) < cost(best)) best = s;
    return cost(best) < 0.9 * cost(1) ? (int)best : 1;
  }
  // Shallow products (k below 1024) split into ranges as short as 64: a
  // 512-cube has 16 tiles, and eight 64-deep ranges ran it at 9.4-11 TFLOP/s
  // against 6.3-7.5 for two 256-deep ones.
  if (k < 128) return 1;
  // Every CU already holds a workgroup: split only as far as two workgroups
  // a CU, into ranges at least 1024 deep, and further only for very deep
  // products (ranges of 8192 or more, up to 2048 workgroups: the vocabulary
  // products). Measured on MI355X: the [1024, 4096] products over k = 1024
  // (256 tiles of 128x128) ran at 98 TFLOP/s unsplit against 86 in three
  // ranges; [4096, 2048] over 2048 (512 tiles) 121 unsplit against 108 in
  // four; [2048, 2048] over 4096 (256 tiles) 118 in three ranges against 113
  // in six, and in the Llama step its 32 launches took 8.71 ms in two ranges
  // against 8.98 in three.
  if (tiles >= 256) {
    int64_t s = 1;
    while ((s + 1) * tiles <= 512 && k / (s + 1) >= 1024) ++s;
    while (s * 2 * tiles <= 2048 && k / (s * 2) >= 8192) s *= 2;
    return (int)std::min<int64_t>(s, 16);
  }
  // Fewer tiles than CUs: the split that minimises the busiest CU's work,
  // ceil(tiles * s / 256) workgroups of k / s each (a CU's matrix cores serve
  // its workgroups in turn), plus the partials' s + 1 passes over the output.
  // Measured on MI355X: [768, 768] over 8192 (36 tiles) ran at 79 TFLOP/s in
  // 16 ranges and 90 in 6 (8: 66); [1024, 1024] over 4096 (64 tiles) at 86
  // in 12 and 98 in 4; [768, 3072] over 8192 (144 tiles) at 117 in 16 and
  // 95 in 4.
  const double slab_s = 2.0 * shape.bm * shape.bn * kTileK / (157.3e12 / 256);
  const double partial_bytes = 4.0 * (double)batches * (double)m * (double)n;
  auto cost = [&](int64_t s) {
    const int64_t per_cu = (tiles * s + 255) / 256;
    const int64_t slabs = ((k + s - 1) / s + kTileK - 1) / kTileK;
    const double partials = s > 1 ? (double)(s + 1) * partial_bytes / 5e12 : 0.0;
    return (double)per_cu * (double)slabs * slab_s + partials;
  };
  int64_t best = 1;
  for (int64_t s = 2; s <= 16 && k / s >= (k < 1024 ? 64 : 256); ++s)
    if (cost(s) < cost(best)) best = s;
  return (int)best;
}

int64_t mfma_split_floats(int64_t m, int64_t n, int64_t k, const Batch &batch, int64_t ldc) {
  // The reduction walks one flat batch axis with 32-bit quad indices, in
  // quads of one row (n % 4 == 0), or in quads of the whole output when it
  // is contiguous (ldc == n, batches back to back) and holds whole quads.
  if (batch.inner != 1 || batch.count < 1) return 0;
  const int64_t split_stride = batch.count * m * n;
  const bool flat = ldc == n && (batch.count == 1 || batch.c_stride == m * n) && split_stride % 4 == 0;
  if (n % 4 != 0 && !flat) return 0;
  const int splits = mfma_splits(m, n, k, batch.count);
  if (splits <= 1 || splits > 16 || split_stride / 4 >= (int64_t(1) << 31)) return 0;
  return splits * split_stride;
}

bool mfma_serves(int64_t a_rs, int64_t a_cs, int64_t b_rs, int64_t b_cs, int64_t m, int64_t k, int64_t n) {
  // Orientation: each operand needs a unit stride along k or along its outer
  // axis; an extent-1 axis leaves its stride unused (any value serves).
  const bool left = a_cs == 1 || m == 1 || a_rs == 1 || k == 1;
  const bool right = b_rs == 1 || n == 1 || b_cs == 1 || k == 1;
  return left && right;
}

bool launch_gemm_mfma(const float *a, int64_t a_rs, int64_t a_cs, const float *b, int64_t b_rs,
                      int64_t b_cs, int64_t m, int64_t k, int64_t n, float *c, int64_t ldc,
                      hipStream_t stream, const Batch &batch, float *workspace, int64_t workspace_floats,
                      const Epilogue &epilogue) {
  if (!mfma_serves(a_rs, a_cs, b_rs, b_cs, m, k, n)) return false;
  const bool left_inner_k = a_cs == 1 || m == 1;
  const bool right_inner_k = b_rs == 1 || n == 1;
  const bool lk = left_inner_k && !(a_rs == 1 && a_cs != 1);
  const bool rk = right_inner_k && !(b_cs == 1 && b_rs != 1);
  // 16-byte loads need a unit stride along the axis the lanes step on (any
  // 4-byte alignment serves).
  const bool vector = (lk ? a_cs == 1 : a_rs == 1) && (rk ? b_rs == 1 : b_cs == 1);
  TileShape shape = tile_shape(m, n, k, batch.count);
  // The 256x256 tiles exist on the LDS-DMA kernel only (unsplit either way).
  if (shape.bn == 256 && !(vector && (lk || m >= 4) && (rk || n >= 4))) shape = {256, 128, 2};
  const int64_t gm = (m + shape.bm - 1) / shape.bm;
  const int64_t gn = (n + shape.bn - 1) / shape.bn;
  if (gm * gn > 0x7fffffff || batch.count > 65535 || batch.count < 1) throw Unsupported{"mfma gemm: grid too large"};
  if (batch.inner < 1) throw Unsupported{"mfma gemm: batch inner extent below one"};
  const int64_t split_stride = batch.count * m * n;
  const int64_t split_floats = mfma_split_floats(m, n, k, batch, ldc);
  int splits = split_floats > 0 ? (int)(split_floats / split_stride) : 1;
  // A workspace too small for the chosen split takes as many ranges as it
  // holds (the no-allocation entry's fixed array), down to none.
  if (splits > 1 && (!workspace || reinterpret_cast<uintptr_t>(workspace) % 16 != 0)) splits = 1;
  if (splits > 1 && workspace_floats < split_floats)
    splits = (int)std::min<int64_t>(splits, workspace_floats / split_stride);
  if (splits < 2) splits = 1;
  int64_t split_len = k;
  if (splits > 1) {
    split_len = ((k + splits - 1) / splits + kTileK - 1) / kTileK * kTileK;
    splits = (int)((k + split_len - 1) / split_len);
  }
  const dim3 grid((unsigned)(gm * gn), (unsigned)batch.count, (unsigned)splits);
  const int bias_mode = epilogue.bias ? (epilogue.bias_first ? 2 : 1) : 0;
  const int gemm_mode = splits > 1 ? 0 : bias_mode;  // with splits, the reduction adds the bias
  // With splits, each partial is written contiguous ([count][m][n]) into the
  // workspace, then reduced into c.
  float *target = splits > 1 ? workspace : c;
  const int64_t target_ld = splits > 1 ? n : ldc;
  // (partials: batch y at y * m * n, as (y / inner) * inner * m * n + (y % inner) * m * n)
  const int64_t target_bs = splits > 1 ? batch.inner * m * n : batch.c_stride;
  const int64_t target_bs2 = splits > 1 ? m * n : batch.c_inner;
  // The LDS-DMA kernel serves the 256x128, 128x128 and 64x128 tiles with
  // 16-byte operand access (the DMA loads need 4-byte alignment only); an
  // outer-contiguous operand needs an outer extent of at least 4 (its clamped
  // edge quads). The 128x64 tile (the attention products with a 64-wide right
  // operand) measured faster on the register-staged kernel with 32x32x2
  // blocks, and the same with 16x16x4 blocks (GPT-2 step, same-box A/B).
  const bool dma = vector && (lk || m >= 4) && (rk || n >= 4);
  // 16-byte output stores: every batch's and split's base and every row
  // start 16-byte aligned.
  const bool vector_out = target_ld % 4 == 0 && reinterpret_cast<uintptr_t>(target) % 16 == 0 &&
                          (batch.count == 1 || (target_bs % 4 == 0 && target_bs2 % 4 == 0)) &&
                          (splits == 1 || split_stride % 4 == 0);
  if (dma && shape.bn == 256)
    dispatch_dma<256, 256>(lk, rk, vector_out, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, target, target_ld, (int)gm, (int)gn, batch, target_bs, target_bs2, split_len, split_stride, epilogue, gemm_mode);
  else if (dma && shape.bm == 256)
    dispatch_dma<256, 128>(lk, rk, vector_out, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, target, target_ld, (int)gm, (int)gn, batch, target_bs, target_bs2, split_len, split_stride, epilogue, gemm_mode);
  else if (dma && shape.bm == 64)
    dispatch_dma<64, 128>(lk, rk, vector_out, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, target, target_ld, (int)gm, (int)gn, batch, target_bs, target_bs2, split_len, split_stride, epilogue, gemm_mode);
  else if (dma && shape.bn == 128)
    dispatch_dma<128, 128>(lk, rk, vector_out, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, target, target_ld, (int)gm, (int)gn, batch, target_bs, target_bs2, split_len, split_stride, epilogue, gemm_mode);
  else if (shape.bm == 256)
    dispatch_orientation<256, 128>(lk, rk, vector, vector_out, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, target, target_ld, (int)gm, (int)gn, batch, target_bs, target_bs2, split_len, split_stride, epilogue, gemm_mode);
  else if (shape.bn == 64)
    dispatch_orientation<128, 64>(lk, rk, vector, vector_out, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, target, target_ld, (int)gm, (int)gn, batch, target_bs, target_bs2, split_len, split_stride, epilogue, gemm_mode);
  else if (shape.bm == 64)
    dispatch_orientation<64, 128>(lk, rk, vector, vector_out, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, target, target_ld, (int)gm, (int)gn, batch, target_bs, target_bs2, split_len, split_stride, epilogue, gemm_mode);
  else
    dispatch_orientation<128, 128>(lk, rk, vector, vector_out, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, target, target_ld, (int)gm, (int)gn, batch, target_bs, target_bs2, split_len, split_stride, epilogue, gemm_mode);
  check_launch("gemm_mfma_kernel launch");
  if (splits > 1) {
    const int64_t quads = split_stride / 4;
    int64_t blocks = (quads + 255) / 256;
    if (blocks > 256 * 32) blocks = 256 * 32;
    if (n % 4 == 0) {
      const bool aligned = reinterpret_cast<uintptr_t>(c) % 16 == 0 && ldc % 4 == 0 && batch.c_stride % 4 == 0;
      split_reduce_kernel<<<(unsigned)blocks, 256, 0, stream>>>(
          reinterpret_cast<const float4 *>(workspace), splits, (uint32_t)quads, (uint32_t)m, (uint32_t)(n / 4), c,
          ldc, batch.c_stride, epilogue.bias, epilogue.bias_stride, bias_mode, aligned);
    } else {
      // A contiguous output whose rows are not whole quads (the 50257-wide
      // products): quads of the flat output.
      const bool aligned = reinterpret_cast<uintptr_t>(c) % 16 == 0;
      split_reduce_flat_kernel<<<(unsigned)blocks, 256, 0, stream>>>(
          reinterpret_cast<const float4 *>(workspace), splits, (uint32_t)quads, (uint32_t)n, c, epilogue.bias,
          epilogue.bias_stride, bias_mode, aligned);
    }
    check_launch("split_reduce_kernel launch");
  }
  return true;
}

}  // namespace topos_hip
