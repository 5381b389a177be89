// Exact-posture GEMM: bit-identical to the reference slice path,
// src/payload/gemm.rs:140-211.
//
// Every output element is one independent accumulator over ascending k,
// seeded with the first term a[i,0]*b[0,j] (never a zero: 0 + -0 would lose
// the sign of an all negative-zero sum, src/payload/tests/gemm_tests.rs:130-139),
// then acc = RN(acc + RN(a[i,s] * b[s,j])) for s = 1..k-1: a separately rounded
// multiply and add, never a fused multiply-add, never a split of k. That is
// VALU work (two instructions per term) and the kernels are shaped for it:
// 64x64 output tiles per 256-lane workgroup, 4x4 accumulators per lane,
// operands staged k-major through LDS so each lane reads its four rows and
// four columns as two 128-bit LDS loads; small products run one output per
// lane.
#pragma clang fp contract(off)
#include "backend.hpp"

namespace topos_hip {
namespace {

constexpr int kTileK = 32;
constexpr int kThreads = 256;

// How an operand is read: kGeneric element by element at any strides;
// kInnerUnit with k contiguous (a lane loads four consecutive k values at
// once); kOuterUnit with the outer axis contiguous (a lane loads four
// consecutive outer elements at once). 16-byte loads serve any 4-byte
// alignment on gfx950. kWindowRows / kWindowCols: the left operand is a
// convolution's patch matrix (outer = patch rows, k = patch columns) or its
// transpose (outer = patch columns, k = patch rows), each element gathered
// from the source (window_element).
enum { kGeneric = 0, kInnerUnit = 1, kOuterUnit = 2, kWindowRows = 3, kWindowCols = 4 };

// Element (row, col) of the patch matrix: row = (image, out_y, out_x),
// col = (channel, kernel_y, kernel_x), the source element under that window
// position or +0 in the padding (zero_like of an f32 element, as the padded
// copy holds), or +0 when `valid` is false (a slab's overhang). The load is
// unconditional, from the view's first element when the position reads
// nothing, and the value is selected afterwards: loads under branches made
// the compiler wait for each earlier load before the next (the branch's +0
// and the load share a register). The caller launches no window kernel over
// an empty source, so the first element exists.
__device__ __forceinline__ float window_element(const float *__restrict__ src, const WindowShape &w, uint32_t row,
                                                uint32_t col, bool valid) {
  const uint32_t t = w.by_out_width.divide(row), x = row - t * (uint32_t)w.out_width;
  const uint32_t image = w.by_out_height.divide(t), y = t - image * (uint32_t)w.out_height;
  const uint32_t u = w.by_kernel_width.divide(col), kx = col - u * (uint32_t)w.kernel_width;
  const uint32_t channel = w.by_kernel_height.divide(u), ky = u - channel * (uint32_t)w.kernel_height;
  const int32_t hy = (int32_t)(y * (uint32_t)w.stride + ky) - w.padding;
  const int32_t wx = (int32_t)(x * (uint32_t)w.stride + kx) - w.padding;
  const bool inside = valid && (uint32_t)hy < (uint32_t)w.height && (uint32_t)wx < (uint32_t)w.width;
  const int64_t at = inside ? (int64_t)image * w.s_batch + (int64_t)channel * w.s_channel +
                                  (int64_t)hy * w.s_height + (int64_t)wx * w.s_width
                            : 0;
  const float v = src[w.offset + at];
  return inside ? v : 0.0f;
}

// One kTileK x E slab of an operand (outer index o0.., inner k0..) in a
// lane's registers (fetch), then into lds[k][o] (deposit): the next slab's
// loads are in flight while the current slab is multiplied.
template <int E, int kMode>
struct Stage {
  static constexpr int kQuads = E * kTileK / 4;                      // quads a slab
  static constexpr int kQ = (kQuads + kThreads - 1) / kThreads;      // quads a lane
  static constexpr int kS = E * kTileK / kThreads;                   // elements a lane (generic, window)
  float v[(kMode == kInnerUnit || kMode == kOuterUnit) ? 4 * kQ : kS];

  // A patch-matrix slab: consecutive lanes on consecutive patch rows (the
  // source's x positions), whichever of outer and k that is.
  __device__ void fetch_window(const float *__restrict__ p, const WindowShape &w, int64_t outer_extent, int64_t k,
                               int64_t o0, int64_t k0) {
    const int t = threadIdx.x;
#pragma unroll
    for (int e = 0; e < kS; ++e) {
      const int flat = e * kThreads + t;
      const int o = kMode == kWindowRows ? flat % E : flat / kTileK;
      const int kk = kMode == kWindowRows ? flat / E : flat % kTileK;
      const int64_t go = o0 + o, gk = k0 + kk;
      const bool valid = go < outer_extent && gk < k;
      v[e] = kMode == kWindowRows ? window_element(p, w, (uint32_t)go, (uint32_t)gk, valid)
                                  : window_element(p, w, (uint32_t)gk, (uint32_t)go, valid);
    }
  }

  __device__ void fetch(const float *__restrict__ p, int64_t outer_stride, int64_t k_stride, int64_t outer_extent,
                        int64_t k, int64_t o0, int64_t k0) {
    const int t = threadIdx.x;
    if constexpr (kMode == kInnerUnit) {
#pragma unroll
      for (int e = 0; e < kQ; ++e) {
        const int flat = e * kThreads + t;
        const int kq = flat % (kTileK / 4), o = flat / (kTileK / 4);
        const int64_t go = o0 + o, gk = k0 + 4 * kq;
        if (flat < kQuads && go < outer_extent && gk + 3 < k) {
          const float4 w = *reinterpret_cast<const float4 *>(p + go * outer_stride + gk);
          v[4 * e] = w.x;
          v[4 * e + 1] = w.y;
          v[4 * e + 2] = w.z;
          v[4 * e + 3] = w.w;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            v[4 * e + j] = (flat < kQuads && go < outer_extent && gk + j < k) ? p[go * outer_stride + gk + j] : 0.0f;
        }
      }
    } else if constexpr (kMode == kOuterUnit) {
#pragma unroll
      for (int e = 0; e < kQ; ++e) {
        const int flat = e * kThreads + t;
        const int oq = flat % (E / 4), kk = flat / (E / 4);
        const int64_t go = o0 + 4 * oq, gk = k0 + kk;
        if (flat < kQuads && go + 3 < outer_extent && gk < k) {
          const float4 w = *reinterpret_cast<const float4 *>(p + gk * k_stride + go);
          v[4 * e] = w.x;
          v[4 * e + 1] = w.y;
          v[4 * e + 2] = w.z;
          v[4 * e + 3] = w.w;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            v[4 * e + j] = (flat < kQuads && go + j < outer_extent && gk < k) ? p[gk * k_stride + go + j] : 0.0f;
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < kS; ++e) {
        const int flat = e * kThreads + t;
        const int o = flat % E, kk = flat / E;
        const int64_t go = o0 + o, gk = k0 + kk;
        v[e] = (go < outer_extent && gk < k) ? p[go * outer_stride + gk * k_stride] : 0.0f;
      }
    }
  }

  __device__ void deposit(float (*lds)[E + 4]) const {
    const int t = threadIdx.x;
    if constexpr (kMode == kInnerUnit) {
#pragma unroll
      for (int e = 0; e < kQ; ++e) {
        const int flat = e * kThreads + t;
        if (flat >= kQuads) break;
        const int kq = flat % (kTileK / 4), o = flat / (kTileK / 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) lds[4 * kq + j][o] = v[4 * e + j];
      }
    } else if constexpr (kMode == kOuterUnit) {
#pragma unroll
      for (int e = 0; e < kQ; ++e) {
        const int flat = e * kThreads + t;
        if (flat >= kQuads) break;
        const int oq = flat % (E / 4), kk = flat / (E / 4);
        *reinterpret_cast<float4 *>(&lds[kk][4 * oq]) = make_float4(v[4 * e], v[4 * e + 1], v[4 * e + 2], v[4 * e + 3]);
      }
    } else if constexpr (kMode == kWindowCols) {
#pragma unroll
      for (int e = 0; e < kS; ++e) {
        const int flat = e * kThreads + t;
        lds[flat % kTileK][flat / kTileK] = v[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < kS; ++e) {
        const int flat = e * kThreads + t;
        lds[flat / E][flat % E] = v[e];
      }
    }
  }
};

// 64x64 output tiles, 4x4 accumulators a lane: lane (tx, ty) owns rows
// ty*4 + {0..3} and columns tx*4 + {0..3}, so its LDS reads are two float4s
// per k step. The next slab's loads are in flight (Stage) while this slab is
// multiplied from the other LDS buffer. (Measured on MI355X against 128x128
// tiles of 8x8 accumulators: those need about 160 registers a lane, three
// waves a SIMD and no room to prefetch; 4096-cubes went 30-34 -> 43 TFLOP/s.)
template <int EM, int EN, int kLeftMode, int kRightMode>
__global__ __launch_bounds__(kThreads) void gemm_exact_kernel(
    const float *__restrict__ a, int64_t a_rs, int64_t a_cs, const float *__restrict__ b,
    int64_t b_rs, int64_t b_cs, int64_t m, int64_t k, int64_t n, float *__restrict__ c, int64_t ldc,
    int64_t a_bs, int64_t b_bs, int64_t c_bs, const WindowShape w) {
  // RM x RN accumulators a lane, 16 x 16 lanes over the EM x EN tile.
  constexpr int RM = EM / 16, RN = EN / 16;
  static_assert(EM * EN == 16 * 16 * RM * RN && (RM == 4 || RM == 2) && (RN == 4 || RN == 2), "tile shape");
  a += (int64_t)blockIdx.z * a_bs;
  b += (int64_t)blockIdx.z * b_bs;
  c += (int64_t)blockIdx.z * c_bs;
  const int64_t m0 = (int64_t)blockIdx.y * EM;
  const int64_t n0 = (int64_t)blockIdx.x * EN;
  const int tx = threadIdx.x % 16;
  const int ty = threadIdx.x / 16;
  float acc[RM][RN];

  {
    __shared__ __attribute__((aligned(16))) float left2[2][kTileK][EM + 4];
    __shared__ __attribute__((aligned(16))) float right2[2][kTileK][EN + 4];
    Stage<EM, kLeftMode> sa;
    Stage<EN, kRightMode> sb;
    auto fetch_left = [&](int64_t k0) {
      if constexpr (kLeftMode == kWindowRows || kLeftMode == kWindowCols)
        sa.fetch_window(a, w, m, k, m0, k0);
      else
        sa.fetch(a, a_rs, a_cs, m, k, m0, k0);
    };
    fetch_left(0);
    sb.fetch(b, b_cs, b_rs, n, k, n0, 0);
    sa.deposit(left2[0]);
    sb.deposit(right2[0]);
    __syncthreads();
    int cur = 0;
    for (int64_t k0 = 0; k0 < k; k0 += kTileK) {
      const bool more = k0 + kTileK < k;
      if (more) {
        fetch_left(k0 + kTileK);
        sb.fetch(b, b_cs, b_rs, n, k, n0, k0 + kTileK);
      }
      const int steps = (k - k0) < kTileK ? (int)(k - k0) : kTileK;
      for (int s = 0; s < steps; ++s) {
        float av[RM], bv[RN];
        if constexpr (RM == 4) {
          const float4 a4 = *reinterpret_cast<const float4 *>(&left2[cur][s][ty * 4]);
          av[0] = a4.x, av[1] = a4.y, av[2] = a4.z, av[3] = a4.w;
        } else {
          const float2 a2 = *reinterpret_cast<const float2 *>(&left2[cur][s][ty * 2]);
          av[0] = a2.x, av[1] = a2.y;
        }
        if constexpr (RN == 4) {
          const float4 b4 = *reinterpret_cast<const float4 *>(&right2[cur][s][tx * 4]);
          bv[0] = b4.x, bv[1] = b4.y, bv[2] = b4.z, bv[3] = b4.w;
        } else {
          const float2 b2 = *reinterpret_cast<const float2 *>(&right2[cur][s][tx * 2]);
          bv[0] = b2.x, bv[1] = b2.y;
        }
        if (k0 == 0 && s == 0) {
#pragma unroll
          for (int i = 0; i < RM; ++i)
#pragma unroll
            for (int j = 0; j < RN; ++j) acc[i][j] = __fmul_rn(av[i], bv[j]);  // the seed (gemm.rs:151-160)
        } else {
#pragma unroll
          for (int i = 0; i < RM; ++i)
#pragma unroll
            for (int j = 0; j < RN; ++j) acc[i][j] = __fadd_rn(acc[i][j], __fmul_rn(av[i], bv[j]));
        }
      }
      if (more) {
        sa.deposit(left2[cur ^ 1]);
        sb.deposit(right2[cur ^ 1]);
      }
      __syncthreads();
      cur ^= 1;
    }
  }

#pragma unroll
  for (int i = 0; i < RM; ++i) {
    const int64_t row = m0 + ty * RM + i;
    if (row >= m) continue;
#pragma unroll
    for (int j = 0; j < RN; ++j) {
      const int64_t col = n0 + tx * RN + j;
      if (col < n) c[row * ldc + col] = acc[i][j];
    }
  }
}

// Products with too few 64x64 tiles to occupy the chip (the MLP's
// [64, 784] x [784, 128], a 512-cube): one output per lane, 16x16 outputs per
// workgroup, k staged through LDS 64 at a time (the next slab's loads in
// flight during the current one's chain). Each lane runs its element's
// chain, seed then ascending k, exactly as gemm_exact_kernel does.
constexpr int kSmall = 16;
constexpr int kSmallK = 64;

template <bool kLeftUnitInner, bool kRightUnitInner, int kLeftWindow = kGeneric>
__global__ __launch_bounds__(kThreads) void gemm_exact_small_kernel(
    const float *__restrict__ a, int64_t a_rs, int64_t a_cs, const float *__restrict__ b,
    int64_t b_rs, int64_t b_cs, int64_t m, int64_t k, int64_t n, float *__restrict__ c, int64_t ldc,
    int64_t a_bs, int64_t b_bs, int64_t c_bs, const WindowShape w) {
  __shared__ float left[kSmallK][kSmall + 1];
  __shared__ float right[kSmallK][kSmall + 1];
  a += (int64_t)blockIdx.z * a_bs;
  b += (int64_t)blockIdx.z * b_bs;
  c += (int64_t)blockIdx.z * c_bs;
  const int64_t m0 = (int64_t)blockIdx.y * kSmall;
  const int64_t n0 = (int64_t)blockIdx.x * kSmall;
  const int t = threadIdx.x;
  const int ti = t / kSmall, tj = t % kSmall;
  constexpr int kPer = kSmall * kSmallK / kThreads;  // staged values per lane per operand
  float va[kPer], vb[kPer];
  // Lane t's staged elements of slab k0: (row or column, k) pairs, with
  // consecutive lanes on the operand's contiguous axis.
  auto coords = [&](int e, bool unit_inner, int &outer, int &kk) {
    const int flat = e * kThreads + t;
    if (unit_inner) {
      kk = flat % kSmallK;
      outer = flat / kSmallK;
    } else {
      outer = flat % kSmall;
      kk = flat / kSmall;
    }
  };
  auto fetch = [&](int64_t k0) {
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      int o, kk;
      coords(e, kLeftUnitInner, o, kk);
      const int64_t gm = m0 + o, gk = k0 + kk;
      if constexpr (kLeftWindow == kWindowRows)
        va[e] = window_element(a, w, (uint32_t)gm, (uint32_t)gk, gm < m && gk < k);
      else if constexpr (kLeftWindow == kWindowCols)
        va[e] = window_element(a, w, (uint32_t)gk, (uint32_t)gm, gm < m && gk < k);
      else
        va[e] = (gm < m && gk < k) ? a[gm * a_rs + gk * a_cs] : 0.0f;
      coords(e, kRightUnitInner, o, kk);
      const int64_t gn = n0 + o, gkb = k0 + kk;
      vb[e] = (gkb < k && gn < n) ? b[gkb * b_rs + gn * b_cs] : 0.0f;
    }
  };
  float acc = 0.0f;
  fetch(0);
  for (int64_t k0 = 0; k0 < k; k0 += kSmallK) {
    __syncthreads();
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      int o, kk;
      coords(e, kLeftUnitInner, o, kk);
      left[kk][o] = va[e];
      coords(e, kRightUnitInner, o, kk);
      right[kk][o] = vb[e];
    }
    __syncthreads();
    if (k0 + kSmallK < k) fetch(k0 + kSmallK);
    const int steps = (k - k0) < kSmallK ? (int)(k - k0) : kSmallK;
    int s = 0;
    if (k0 == 0) {
      acc = __fmul_rn(left[0][ti], right[0][tj]);  // the seed: the first term itself (gemm.rs:151-160)
      s = 1;
    }
#pragma unroll 8
    for (; s < steps; ++s) acc = __fadd_rn(acc, __fmul_rn(left[s][ti], right[s][tj]));
  }
  const int64_t row = m0 + ti, col = n0 + tj;
  if (row < m && col < n) c[row * ldc + col] = acc;
}

// A convolution's kernel gradient with few outputs (patches^T . b: m patch
// columns by n filters over k patch rows; the MNIST stages' [9, 8] over
// 50176 rows): one output per lane, up to 16x16 outputs a workgroup, each lane's
// chain over ascending patch rows staged 256 deep. The workgroup is eight
// waves: four chain waves (one output a lane) and four producer waves that
// gather the next slab into the other of two LDS buffers while the chain
// waves walk the current one, so the gather's address arithmetic does not
// sit in the chain waves' instruction stream. Producer lane p gathers patch
// row k0 + p for the tile's 16 columns: the row's (image, y, x) is divided
// out once a slab, each column's (channel, ky, kx) once a launch. The chain
// reads 32 terms as sixteen 16-byte LDS reads issued together (rows padded
// by four floats, so the 16 right-hand rows a wave reads fall in distinct
// banks). Batch z (the Fast posture's ranges of whole images) offsets the
// source, b and c.
constexpr int kDeep = 16;
constexpr int kDeepK = 256;

__global__ __launch_bounds__(2 * kThreads) void window_deep_kernel(const float *__restrict__ src,
                                                                   const WindowShape w, const float *__restrict__ b,
                                                                   int64_t b_rs, int64_t b_cs, int64_t m, int64_t k,
                                                                   int64_t n, float *__restrict__ c, int64_t ldc,
                                                                   int64_t a_bs, int64_t b_bs, int64_t c_bs) {
  static_assert(kDeepK == kThreads && kDeep * kDeep == kThreads, "one patch row a lane, one output a lane");
  __shared__ __attribute__((aligned(16))) float left[2][kDeep][kDeepK + 4];
  __shared__ __attribute__((aligned(16))) float right[2][kDeep][kDeepK + 4];
  src += w.offset + (int64_t)blockIdx.z * a_bs;
  b += (int64_t)blockIdx.z * b_bs;
  c += (int64_t)blockIdx.z * c_bs;
  const int64_t m0 = (int64_t)blockIdx.y * kDeep, n0 = (int64_t)blockIdx.x * kDeep;
  const bool producer = threadIdx.x >= kThreads;
  const int t = threadIdx.x & (kThreads - 1), tj = t % kDeep;
  // Chain lanes hold the tile's outputs densely (row-major over its mt x nt
  // outputs), so only the waves that own outputs read the LDS slabs: the
  // chain waves are bound by the LDS bytes they read.
  const int mt = m - m0 < kDeep ? (int)(m - m0) : kDeep, nt = n - n0 < kDeep ? (int)(n - n0) : kDeep;
  const bool owner = t < mt * nt;
  const int out_i = owner ? t / nt : 0, out_j = owner ? t % nt : 0;
  const bool walks = (t & ~63) < mt * nt;  // the wave owns at least one output
  constexpr int32_t kOutside = -(1 << 30);  // a window offset that no in-range sum reaches

  // ---- producers: the gather ----
  // Values of rows past k, of columns past m and of filters past n are never
  // read by a stored output's chain, so their addresses are only clamped in
  // range; the padding's +0 is selected. The tile's columns (patch columns
  // m0 + e, clamped to m - 1): source offset and kernel position.
  int32_t col_ky[kDeep], col_kx[kDeep];
  int64_t col_off[kDeep];
  // Two register sets: a slab's loads are issued two slabs before its
  // deposit (each slab's rows of b come from HBM once; one slab of lead did
  // not cover their latency).
  float va0[kDeep], vb0[kDeep], va1[kDeep], vb1[kDeep];
  const float *b_lane = b;  // b's element (row t / 16, filter n0 + tj, clamped)
  if (producer) {
#pragma unroll
    for (int e = 0; e < kDeep; ++e) {
      const uint32_t o = (uint32_t)(m0 + e < m ? m0 + e : m - 1);
      const uint32_t u = w.by_kernel_width.divide(o), kx = o - u * (uint32_t)w.kernel_width;
      const uint32_t channel = w.by_kernel_height.divide(u), ky = u - channel * (uint32_t)w.kernel_height;
      col_ky[e] = (int32_t)ky;
      col_kx[e] = (int32_t)kx;
      col_off[e] = (int64_t)channel * w.s_channel + (int64_t)ky * w.s_height + (int64_t)kx * w.s_width;
    }
    b_lane = b + (n0 + tj < n ? n0 + tj : n - 1) * b_cs;
  }
  auto fetch = [&](float (&va)[kDeep], float (&vb)[kDeep], int64_t k0) {
    const int64_t r = k0 + t < k ? k0 + t : k - 1;
    const uint32_t q = w.by_out_width.divide((uint32_t)r), x = (uint32_t)r - q * (uint32_t)w.out_width;
    const uint32_t image = w.by_out_height.divide(q), y = q - image * (uint32_t)w.out_height;
    const int32_t y0 = (int32_t)(y * (uint32_t)w.stride) - w.padding;
    const int32_t x0 = (int32_t)(x * (uint32_t)w.stride) - w.padding;
    const int64_t base = (int64_t)image * w.s_batch + (int64_t)y0 * w.s_height + (int64_t)x0 * w.s_width;
    const bool whole = k0 + kDeepK <= k;
    // Unconditional loads (clamped), values selected afterwards: see
    // window_element.
#pragma unroll
    for (int e = 0; e < kDeep; ++e) {
      const int32_t hy = y0 + col_ky[e], wx = x0 + col_kx[e];
      const bool inside = (uint32_t)hy < (uint32_t)w.height && (uint32_t)wx < (uint32_t)w.width;
      const float a_value = src[inside ? base + col_off[e] : 0];
      va[e] = inside ? a_value : 0.0f;
      const int64_t gk = k0 + e * kDeep + t / kDeep;
      vb[e] = b_lane[(whole || gk < k ? gk : k - 1) * b_rs];
    }
  };
  auto deposit = [&](const float (&va)[kDeep], const float (&vb)[kDeep], int buffer) {
#pragma unroll
    for (int e = 0; e < kDeep; ++e) {
      left[buffer][e][t] = va[e];
      right[buffer][tj][e * kDeep + t / kDeep] = vb[e];
    }
  };

  // ---- chain waves: the ordered sum ----
  float acc = 0.0f;
  auto chain = [&](int64_t k0, int buffer) {
    const int steps = (k - k0) < kDeepK ? (int)(k - k0) : kDeepK;
    const float *lrow = left[buffer][out_i], *rrow = right[buffer][out_j];
    int s = 0;
    if (k0 == 0) {
      acc = __fmul_rn(lrow[0], rrow[0]);  // the seed: the first term itself (gemm.rs:151-160)
      for (s = 1; s < 4 && s < steps; ++s) acc = __fadd_rn(acc, __fmul_rn(lrow[s], rrow[s]));
    }
    const int whole = steps & ~3;
    // Blocks of 32 terms: all sixteen 16-byte LDS reads issued before the
    // block's chain, so the LDS latency is met once a block, not once every
    // four terms.
    for (; s + 32 <= whole; s += 32) {
      float4 l[8], r[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        l[q] = *reinterpret_cast<const float4 *>(lrow + s + 4 * q);
        r[q] = *reinterpret_cast<const float4 *>(rrow + s + 4 * q);
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        acc = __fadd_rn(acc, __fmul_rn(l[q].x, r[q].x));
        acc = __fadd_rn(acc, __fmul_rn(l[q].y, r[q].y));
        acc = __fadd_rn(acc, __fmul_rn(l[q].z, r[q].z));
        acc = __fadd_rn(acc, __fmul_rn(l[q].w, r[q].w));
      }
    }
    for (; s < whole; s += 4) {
      const float4 l = *reinterpret_cast<const float4 *>(lrow + s);
      const float4 r = *reinterpret_cast<const float4 *>(rrow + s);
      acc = __fadd_rn(acc, __fmul_rn(l.x, r.x));
      acc = __fadd_rn(acc, __fmul_rn(l.y, r.y));
      acc = __fadd_rn(acc, __fmul_rn(l.z, r.z));
      acc = __fadd_rn(acc, __fmul_rn(l.w, r.w));
    }
    for (; s < steps; ++s) acc = __fadd_rn(acc, __fmul_rn(lrow[s], rrow[s]));
  };

  // Slab s is walked from buffer s % 2 while the producers deposit slab
  // s + 1 (register set (s + 1) % 2, loaded since slab s - 2) into the other
  // buffer and issue slab s + 3's loads into the set just emptied; one
  // barrier a slab. The loop body is written twice, for even and odd s.
  if (producer) {
    fetch(va0, vb0, 0);
    deposit(va0, vb0, 0);
    if (kDeepK < k) fetch(va1, vb1, kDeepK);
    if (2 * kDeepK < k) fetch(va0, vb0, 2 * kDeepK);
  }
  __syncthreads();
  for (int64_t k0 = 0; k0 < k; k0 += 2 * kDeepK) {
    if (producer) {
      if (k0 + kDeepK < k) {
        deposit(va1, vb1, 1);
        if (k0 + 3 * kDeepK < k) fetch(va1, vb1, k0 + 3 * kDeepK);
      }
    } else if (walks) {
      chain(k0, 0);
    }
    __syncthreads();
    if (k0 + kDeepK >= k) break;
    if (producer) {
      if (k0 + 2 * kDeepK < k) {
        deposit(va0, vb0, 0);
        if (k0 + 4 * kDeepK < k) fetch(va0, vb0, k0 + 4 * kDeepK);
      }
    } else if (walks) {
      chain(k0 + kDeepK, 1);
    }
    __syncthreads();
  }
  if (!producer && owner) c[(m0 + out_i) * ldc + n0 + out_j] = acc;
}

}  // namespace

namespace {

template <int EM, int EN, int L>
void launch_exact_right(int right_mode, dim3 grid, hipStream_t stream, const float *a, int64_t a_rs, int64_t a_cs,
                        const float *b, int64_t b_rs, int64_t b_cs, int64_t m, int64_t k, int64_t n, float *c,
                        int64_t ldc, int64_t a_bs, int64_t b_bs, int64_t c_bs, const WindowShape &w) {
  if (right_mode == kInnerUnit)
    gemm_exact_kernel<EM, EN, L, kInnerUnit><<<grid, kThreads, 0, stream>>>(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c,
                                                                            ldc, a_bs, b_bs, c_bs, w);
  else if (right_mode == kOuterUnit)
    gemm_exact_kernel<EM, EN, L, kOuterUnit><<<grid, kThreads, 0, stream>>>(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c,
                                                                            ldc, a_bs, b_bs, c_bs, w);
  else
    gemm_exact_kernel<EM, EN, L, kGeneric><<<grid, kThreads, 0, stream>>>(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c,
                                                                          ldc, a_bs, b_bs, c_bs, w);
}

template <int EM, int EN>
void launch_exact_tile(int left_mode, int right_mode, dim3 grid, hipStream_t stream, const float *a, int64_t a_rs,
                       int64_t a_cs, const float *b, int64_t b_rs, int64_t b_cs, int64_t m, int64_t k, int64_t n,
                       float *c, int64_t ldc, int64_t a_bs, int64_t b_bs, int64_t c_bs, const WindowShape &w) {
  if (left_mode == kInnerUnit)
    launch_exact_right<EM, EN, kInnerUnit>(right_mode, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc,
                                           a_bs, b_bs, c_bs, w);
  else if (left_mode == kOuterUnit)
    launch_exact_right<EM, EN, kOuterUnit>(right_mode, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc,
                                           a_bs, b_bs, c_bs, w);
  else if (left_mode == kWindowRows)
    launch_exact_right<EM, EN, kWindowRows>(right_mode, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc,
                                            a_bs, b_bs, c_bs, w);
  else if (left_mode == kWindowCols)
    launch_exact_right<EM, EN, kWindowCols>(right_mode, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc,
                                            a_bs, b_bs, c_bs, w);
  else
    launch_exact_right<EM, EN, kGeneric>(right_mode, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc,
                                         a_bs, b_bs, c_bs, w);
}

// The exact product with the left operand read as `window_mode` says
// (kGeneric: through a_rs, a_cs; a window mode: gathered through `w`).
void enqueue_exact(int window_mode, const WindowShape &w, const float *a, int64_t a_rs, int64_t a_cs, const float *b,
                   int64_t b_rs, int64_t b_cs, int64_t m, int64_t k, int64_t n, float *c, int64_t ldc,
                   hipStream_t stream, const Batch &batch) {
  if (batch.count > 65535 || batch.count < 1) throw Unsupported{"exact gemm: too many batches for one launch"};
  const int64_t a_bs = batch.a_stride, b_bs = batch.b_stride, c_bs = batch.c_stride;
  const bool window = window_mode != kGeneric;
  const bool left_unit = !window && a_cs == 1;
  const bool right_unit = b_rs == 1 && b_cs != 1;
  // Fewer 64x64 tiles than CUs: one output per lane instead, unless k is
  // deep and 32x32 tiles still give a workgroup per CU (the [768, 768]
  // weight gradient over k = 8192: 14 -> 19.5 TFLOP/s on 32x32 tiles).
  const int64_t small_m = (m + kSmall - 1) / kSmall, small_n = (n + kSmall - 1) / kSmall;
  const int64_t tiles64 = ((m + 63) / 64) * ((n + 63) / 64) * batch.count;
  const int64_t tiles32 = ((m + 31) / 32) * ((n + 31) / 32) * batch.count;
  if (tiles64 < 256 && (k < 2048 || tiles32 < 256) && small_m <= 65535 && small_n <= 0x7fffffff) {
    const dim3 small_grid((unsigned)small_n, (unsigned)small_m, (unsigned)batch.count);
#define TOPOS_SMALL_ARGS a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, a_bs, b_bs, c_bs, w
    // Window modes: consecutive lanes on consecutive patch rows (outer for
    // kWindowRows, k for kWindowCols).
    if (window_mode == kWindowRows && right_unit)
      gemm_exact_small_kernel<false, true, kWindowRows><<<small_grid, kThreads, 0, stream>>>(TOPOS_SMALL_ARGS);
    else if (window_mode == kWindowRows)
      gemm_exact_small_kernel<false, false, kWindowRows><<<small_grid, kThreads, 0, stream>>>(TOPOS_SMALL_ARGS);
    else if (window_mode == kWindowCols && right_unit)
      gemm_exact_small_kernel<true, true, kWindowCols><<<small_grid, kThreads, 0, stream>>>(TOPOS_SMALL_ARGS);
    else if (window_mode == kWindowCols)
      gemm_exact_small_kernel<true, false, kWindowCols><<<small_grid, kThreads, 0, stream>>>(TOPOS_SMALL_ARGS);
    else if (left_unit && right_unit)
      gemm_exact_small_kernel<true, true><<<small_grid, kThreads, 0, stream>>>(TOPOS_SMALL_ARGS);
    else if (left_unit)
      gemm_exact_small_kernel<true, false><<<small_grid, kThreads, 0, stream>>>(TOPOS_SMALL_ARGS);
    else if (right_unit)
      gemm_exact_small_kernel<false, true><<<small_grid, kThreads, 0, stream>>>(TOPOS_SMALL_ARGS);
    else
      gemm_exact_small_kernel<false, false><<<small_grid, kThreads, 0, stream>>>(TOPOS_SMALL_ARGS);
#undef TOPOS_SMALL_ARGS
    check_launch("gemm_exact_small_kernel launch");
    return;
  }
  // The tile: 64x64 (4x4 accumulators a lane, the fewest LDS bytes per
  // term) while that gives at least four workgroups a CU; narrower tiles
  // (4x2, then 2x2 a lane) otherwise, trading LDS reads for occupancy on
  // products with few outputs and long k (the weight gradients, k = 8192).
  // 4x2 a lane already at two workgroups a CU: the [1024, 1024] G.B^T over
  // k = 4096 ran 25.0 TFLOP/s on 2x2 and 29.9 on 4x2 (18.8 on 4x4).
  const int64_t tiles64x32 = ((m + 63) / 64) * ((n + 31) / 32) * batch.count;
  const int shape = tiles64 >= 1024 ? 0 : tiles64x32 >= 512 ? 1 : 2;
  const int em = shape == 2 ? 32 : 64, en = shape == 0 ? 64 : 32;
  const int64_t grid_n = (n + en - 1) / en, grid_m = (m + em - 1) / em;
  if (grid_m > 65535 || grid_n > 0x7fffffff) throw Unsupported{"exact gemm: product too tall for one launch"};
#define TOPOS_EXACT_ARGS a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, a_bs, b_bs, c_bs, w
  const int left_mode = window ? window_mode : left_unit ? kInnerUnit : a_rs == 1 ? kOuterUnit : kGeneric;
  const int right_mode = right_unit ? kInnerUnit : b_cs == 1 ? kOuterUnit : kGeneric;
  const dim3 grid((unsigned)grid_n, (unsigned)grid_m, (unsigned)batch.count);
  if (shape == 0)
    launch_exact_tile<64, 64>(left_mode, right_mode, grid, stream, TOPOS_EXACT_ARGS);
  else if (shape == 1)
    launch_exact_tile<64, 32>(left_mode, right_mode, grid, stream, TOPOS_EXACT_ARGS);
  else
    launch_exact_tile<32, 32>(left_mode, right_mode, grid, stream, TOPOS_EXACT_ARGS);
#undef TOPOS_EXACT_ARGS
  check_launch("gemm_exact_kernel launch");
}

}  // namespace

void launch_gemm_exact(const float *a, int64_t a_rs, int64_t a_cs, const float *b, int64_t b_rs,
                       int64_t b_cs, int64_t m, int64_t k, int64_t n, float *c, int64_t ldc,
                       hipStream_t stream, const Batch &batch) {
  enqueue_exact(kGeneric, WindowShape(), a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, stream, batch);
}

int window_splits(int64_t m, int64_t n, int64_t k, int64_t images) {
  // Enough 16x16 output tiles to fill the chip, or partials the reduction
  // cannot take in quads: one range.
  if (((m + kDeep - 1) / kDeep) * ((n + kDeep - 1) / kDeep) >= 256 || images < 2) return 1;
  if ((m * n) % 4 != 0 && n % 4 != 0) return 1;
  int best = 1;
  for (int s = 2; s <= 16; ++s)
    if (images % s == 0 && k / s >= 512) best = s;
  return best;
}

void launch_window_product(const float *source, const WindowShape &shape, bool transposed, const float *b,
                           int64_t b_rs, int64_t b_cs, int64_t m, int64_t k, int64_t n, float *c, int64_t ldc,
                           hipStream_t stream, float *workspace, int splits) {
  // The patch matrix is [batch * out_height * out_width, channels *
  // kernel_height * kernel_width]; its indices are taken in 32 bits.
  const int64_t rows = transposed ? k : m, columns = transposed ? m : k;
  const int64_t positions = (int64_t)shape.out_height * shape.out_width;
  if (shape.out_height < 1 || shape.out_width < 1 || shape.kernel_height < 1 || shape.kernel_width < 1 ||
      rows % positions != 0 ||
      columns != (int64_t)shape.channels * shape.kernel_height * shape.kernel_width || rows > 0x7fffffff ||
      columns > 0x7fffffff)
    throw Unsupported{"window product: extents outside the patch matrix"};
  if (m == 0 || n == 0) return;
  if (rows == 0 || columns == 0) {
    // An empty source: every output is the empty sum, +0 (the exact kernel
    // with k = 0 reads nothing and writes +0).
    launch_gemm_exact(c, 0, 0, c, 0, 0, m, 0, n, c, ldc, stream);
    return;
  }
  WindowShape w = shape;
  w.by_out_width = Divisor::of((uint32_t)w.out_width);
  w.by_out_height = Divisor::of((uint32_t)w.out_height);
  w.by_kernel_width = Divisor::of((uint32_t)w.kernel_width);
  w.by_kernel_height = Divisor::of((uint32_t)w.kernel_height);
  const int64_t images = rows / positions;
  if (splits > 1 && (!transposed || workspace == nullptr || images % splits != 0 || splits > 16 ||
                     ((m * n) % 4 != 0 && n % 4 != 0)))
    throw Unsupported{"window product: ranges outside what the split form takes"};
  const int64_t tiles = ((m + 63) / 64) * ((n + 63) / 64);
  if (!transposed || (splits <= 1 && tiles >= 256)) {
    enqueue_exact(transposed ? kWindowCols : kWindowRows, w, source, 0, 0, b, b_rs, b_cs, m, k, n, c, ldc, stream,
                  Batch());
    return;
  }
  const int z = splits > 1 ? splits : 1;
  const int64_t range = k / z;  // patch rows of each range: whole images
  const int64_t grid_m = (m + kDeep - 1) / kDeep, grid_n = (n + kDeep - 1) / kDeep;
  if (grid_m > 65535 || grid_n > 0x7fffffff) throw Unsupported{"window product: too many output tiles"};
  const dim3 grid((unsigned)grid_n, (unsigned)grid_m, (unsigned)z);
  float *target = z > 1 ? workspace : c;
  const int64_t target_ld = z > 1 ? n : ldc;
  window_deep_kernel<<<grid, 2 * kThreads, 0, stream>>>(source, w, b, b_rs, b_cs, m, range, n, target, target_ld,
                                                     range / positions * w.s_batch, range * b_rs, m * n);
  check_launch("window_deep_kernel launch");
  if (z > 1) launch_split_reduce(workspace, z, m, n, c, ldc, stream);
}

}  // namespace topos_hip
