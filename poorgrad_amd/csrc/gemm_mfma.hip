// Fast-posture GEMM on the fp32 matrix cores (v_mfma_f32_32x32x2_f32).
//
// Envelope fidelity: the k-sum is blocked and reassociated by the matrix core,
// so results are compared against the exact product within
// |c - exact| <= 1e-5 * sum_k |a_ik * b_kj| (and are deterministic: the same
// inputs give the same bits on every run: no atomics, and a split along k is
// reduced in a fixed order).
//
// Shape: 128x128 output tile per 256-lane workgroup (four waves in 2x2, each
// wave a 64x64 tile = 2x2 MFMA blocks of 32x32), k staged 16 deep through LDS,
// double-buffered: the next slab's global loads are in flight while the
// current slab feeds the matrix cores. LDS holds both operands k-major
// ([k][m], [k][n]) so an MFMA fragment is one conflict-free 32-lane b32 read.
// The forward product and both transposed backward products (A^T G with A
// m-contiguous, G B^T with B k-contiguous; src/function/matmul.rs:76-91) are
// served by the same kernel through the operand-orientation template flags, so
// no transpose is ever materialised.
#include <algorithm>

#include "backend.hpp"

namespace topos_hip {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kTileM = 128;
constexpr int kTileN = 128;
constexpr int kTileK = 16;
constexpr int kThreads = 256;
constexpr int kPad = 4;
constexpr int kGroupM = 8;

// One operand slab in registers between its global load and its LDS store:
// two 4-vectors per lane (kTile x 128 = 512 vectors over 256 lanes).
struct Slab {
  float4 v[2];
};

// Global -> registers for a 128 (outer) x 16 (k) slab of an operand whose
// element (o, kk) lives at p[o * outer_stride + kk * k_stride].
// kInnerK: k is the unit-stride axis (lanes step along k), else the outer axis
// is. kVector: 16-byte loads are legal (aligned, unit stride, stride % 4 == 0).
template <bool kInnerK, bool kVector>
__device__ inline void load_slab(Slab &slab, const float *__restrict__ p, int64_t outer_stride,
                                 int64_t k_stride, int64_t outer_extent, int64_t k_extent,
                                 int64_t o0, int64_t k0) {
  const int t = threadIdx.x;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    int o, kk;
    if (kInnerK) {  // 128 rows x 4 vectors along k
      o = t / 4 + 64 * e;
      kk = (t % 4) * 4;
    } else {  // 16 k-rows x 32 vectors along the outer axis
      kk = t / 32 + 8 * e;
      o = (t % 32) * 4;
    }
    const int64_t go = o0 + o, gk = k0 + kk;
    float4 value;
    if (kInnerK) {
      if (kVector && go < outer_extent && gk + 3 < k_extent) {
        value = *reinterpret_cast<const float4 *>(p + go * outer_stride + gk);
      } else {
        float w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          w[q] = (go < outer_extent && gk + q < k_extent) ? p[go * outer_stride + (gk + q) * k_stride] : 0.0f;
        value = make_float4(w[0], w[1], w[2], w[3]);
      }
    } else {
      if (kVector && gk < k_extent && go + 3 < outer_extent) {
        value = *reinterpret_cast<const float4 *>(p + gk * k_stride + go);
      } else {
        float w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          w[q] = (gk < k_extent && go + q < outer_extent) ? p[(go + q) * outer_stride + gk * k_stride] : 0.0f;
        value = make_float4(w[0], w[1], w[2], w[3]);
      }
    }
    slab.v[e] = value;
  }
}

// Registers -> LDS [k][outer], matching load_slab's lane mapping.
template <bool kInnerK>
__device__ inline void store_slab(float (*lds)[kTileM + kPad], const Slab &slab) {
  const int t = threadIdx.x;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    if (kInnerK) {
      const int o = t / 4 + 64 * e;
      const int kk = (t % 4) * 4;
      lds[kk + 0][o] = slab.v[e].x;
      lds[kk + 1][o] = slab.v[e].y;
      lds[kk + 2][o] = slab.v[e].z;
      lds[kk + 3][o] = slab.v[e].w;
    } else {
      const int kk = t / 32 + 8 * e;
      const int o = (t % 32) * 4;
      *reinterpret_cast<float4 *>(&lds[kk][o]) = slab.v[e];
    }
  }
}

template <bool kLeftInnerK, bool kRightInnerK, bool kVector>
__global__ __launch_bounds__(kThreads) void gemm_mfma_kernel(
    const float *__restrict__ a, int64_t a_rs, int64_t a_cs, const float *__restrict__ b,
    int64_t b_rs, int64_t b_cs, int64_t m, int64_t k, int64_t n, float *__restrict__ c, int64_t ldc,
    int grid_m, int grid_n, int64_t a_bs, int64_t b_bs, int64_t c_bs, int64_t split_len, int64_t split_stride) {
  __shared__ float left[2][kTileK][kTileM + kPad];
  __shared__ float right[2][kTileK][kTileN + kPad];
  a += (int64_t)blockIdx.y * a_bs;
  b += (int64_t)blockIdx.y * b_bs;
  c += (int64_t)blockIdx.y * c_bs;
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
  const int64_t m0 = (int64_t)tile_m * kTileM;
  const int64_t n0 = (int64_t)tile_n * kTileN;

  const int lane = threadIdx.x % 64;
  const int wave = threadIdx.x / 64;
  const int wm = (wave / 2) * 64;  // wave's row offset inside the tile
  const int wn = (wave % 2) * 64;  // wave's column offset

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // Left operand: outer = m (row stride a_rs), inner = k (a_cs).
  // Right operand: outer = n (b_cs), inner = k (b_rs).
  Slab sa, sb;
  load_slab<kLeftInnerK, kVector>(sa, a, a_rs, a_cs, m, k_end, m0, k_begin);
  load_slab<kRightInnerK, kVector>(sb, b, b_cs, b_rs, n, k_end, n0, k_begin);
  store_slab<kLeftInnerK>(left[0], sa);
  store_slab<kRightInnerK>(right[0], sb);
  __syncthreads();

  const int64_t slabs = (k_end - k_begin + kTileK - 1) / kTileK;
  for (int64_t s = 0; s < slabs; ++s) {
    const int cur = (int)(s & 1);
    const bool more = s + 1 < slabs;
    if (more) {
      load_slab<kLeftInnerK, kVector>(sa, a, a_rs, a_cs, m, k_end, m0, k_begin + (s + 1) * kTileK);
      load_slab<kRightInnerK, kVector>(sb, b, b_cs, b_rs, n, k_end, n0, k_begin + (s + 1) * kTileK);
    }
#pragma unroll
    for (int kk = 0; kk < kTileK; kk += 2) {
      const int kr = kk + lane / 32;
      const float a0 = left[cur][kr][wm + (lane % 32)];
      const float a1 = left[cur][kr][wm + 32 + (lane % 32)];
      const float b0 = right[cur][kr][wn + (lane % 32)];
      const float b1 = right[cur][kr][wn + 32 + (lane % 32)];
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
    }
    if (more) {
      store_slab<kLeftInnerK>(left[cur ^ 1], sa);
      store_slab<kRightInnerK>(right[cur ^ 1], sb);
    }
    __syncthreads();
  }

  // 32x32 accumulator layout: register r of lane l holds
  // row 8 * (r / 4) + 4 * (l / 32) + r % 4, column l % 32.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = n0 + wn + 32 * j + (lane % 32);
      if (col >= n) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm + 32 * i + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
        if (row < m) c[row * ldc + col] = acc[i][j][r];
      }
    }
}

template <bool kL, bool kR>
void dispatch_vector(bool vector, dim3 grid, hipStream_t stream, const float *a, int64_t a_rs,
                     int64_t a_cs, const float *b, int64_t b_rs, int64_t b_cs, int64_t m, int64_t k,
                     int64_t n, float *c, int64_t ldc, int gm, int gn, const Batch &batch, int64_t c_bs,
                     int64_t split_len, int64_t split_stride) {
  if (vector)
    gemm_mfma_kernel<kL, kR, true><<<grid, kThreads, 0, stream>>>(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, gm, gn,
                                                                  batch.a_stride, batch.b_stride, c_bs, split_len,
                                                                  split_stride);
  else
    gemm_mfma_kernel<kL, kR, false><<<grid, kThreads, 0, stream>>>(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, gm, gn,
                                                                   batch.a_stride, batch.b_stride, c_bs, split_len,
                                                                   split_stride);
}

// The fixed-order sum of `splits` partial products (each [count][m][n],
// contiguous) into c: partial 0 seeds, then 1, 2, ... are added in order, so
// the result is the same on every run.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float *__restrict__ partials, int splits,
                                                           int64_t split_stride, int64_t m, int64_t n,
                                                           int64_t count, float *__restrict__ c, int64_t ldc,
                                                           int64_t c_bs) {
  const int64_t total = count * m * n;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    float acc = partials[e];
    for (int s = 1; s < splits; ++s) acc += partials[s * split_stride + e];
    const int64_t q = e / (m * n), r = (e / n) % m, col = e % n;
    c[q * c_bs + r * ldc + col] = acc;
  }
}

}  // namespace

int mfma_splits(int64_t m, int64_t n, int64_t k, int64_t batches) {
  // Enough workgroups to fill the 256 CUs twice, each split at least 256 deep.
  const int64_t tiles = ((m + kTileM - 1) / kTileM) * ((n + kTileN - 1) / kTileN) * batches;
  if (tiles >= 512 || k < 1024) return 1;
  int64_t splits = (512 + tiles - 1) / tiles;
  splits = std::min<int64_t>(splits, k / 256);
  splits = std::min<int64_t>(splits, 16);
  return (int)std::max<int64_t>(splits, 1);
}

bool launch_gemm_mfma(const float *a, int64_t a_rs, int64_t a_cs, const float *b, int64_t b_rs,
                      int64_t b_cs, int64_t m, int64_t k, int64_t n, float *c, int64_t ldc,
                      hipStream_t stream, const Batch &batch, float *workspace, int64_t workspace_floats) {
  // Orientation: each operand needs a unit stride along k or along its outer
  // axis; an extent-1 axis leaves its stride unused (any value serves).
  const bool left_inner_k = a_cs == 1 || m == 1;
  const bool left_outer = a_rs == 1 || k == 1;
  const bool right_inner_k = b_rs == 1 || n == 1;
  const bool right_outer = b_cs == 1 || k == 1;
  if (!(left_inner_k || left_outer) || !(right_inner_k || right_outer)) return false;
  const bool lk = left_inner_k && !(a_rs == 1 && a_cs != 1);
  const bool rk = right_inner_k && !(b_cs == 1 && b_rs != 1);
  // 16-byte loads need the unit-stride axis's partner stride to keep every
  // vector aligned, and aligned base pointers.
  const int64_t left_lead = lk ? a_rs : a_cs;
  const int64_t right_lead = rk ? b_cs : b_rs;
  const bool vector = (reinterpret_cast<uintptr_t>(a) % 16 == 0) &&
                      (reinterpret_cast<uintptr_t>(b) % 16 == 0) && (left_lead % 4 == 0) &&
                      (batch.count == 1 || (batch.a_stride % 4 == 0 && batch.b_stride % 4 == 0)) &&
                      (right_lead % 4 == 0) && (lk ? a_cs == 1 : a_rs == 1) &&
                      (rk ? b_rs == 1 : b_cs == 1);
  const int64_t gm = (m + kTileM - 1) / kTileM;
  const int64_t gn = (n + kTileN - 1) / kTileN;
  if (gm * gn > 0x7fffffff || batch.count > 65535 || batch.count < 1) throw Unsupported{"mfma gemm: grid too large"};
  int splits = mfma_splits(m, n, k, batch.count);
  const int64_t split_stride = batch.count * m * n;
  if (splits > 1 && (!workspace || workspace_floats < splits * split_stride)) splits = 1;
  int64_t split_len = k;
  if (splits > 1) {
    split_len = ((k + splits - 1) / splits + kTileK - 1) / kTileK * kTileK;
    splits = (int)((k + split_len - 1) / split_len);
  }
  const dim3 grid((unsigned)(gm * gn), (unsigned)batch.count, (unsigned)splits);
  // With splits, each partial is written contiguous ([count][m][n]) into the
  // workspace, then reduced into c.
  float *target = splits > 1 ? workspace : c;
  const int64_t target_ld = splits > 1 ? n : ldc;
  const int64_t target_bs = splits > 1 ? m * n : batch.c_stride;
  if (lk && rk)
    dispatch_vector<true, true>(vector, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, target, target_ld, (int)gm, (int)gn, batch, target_bs, split_len, split_stride);
  else if (lk)
    dispatch_vector<true, false>(vector, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, target, target_ld, (int)gm, (int)gn, batch, target_bs, split_len, split_stride);
  else if (rk)
    dispatch_vector<false, true>(vector, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, target, target_ld, (int)gm, (int)gn, batch, target_bs, split_len, split_stride);
  else
    dispatch_vector<false, false>(vector, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, target, target_ld, (int)gm, (int)gn, batch, target_bs, split_len, split_stride);
  check_launch("gemm_mfma_kernel launch");
  if (splits > 1) {
    const int64_t total = split_stride;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 256 * 32) blocks = 256 * 32;
    split_reduce_kernel<<<(unsigned)blocks, 256, 0, stream>>>(workspace, splits, split_stride, m, n, batch.count, c,
                                                              ldc, batch.c_stride);
    check_launch("split_reduce_kernel launch");
  }
  return true;
}

}  // namespace topos_hip
