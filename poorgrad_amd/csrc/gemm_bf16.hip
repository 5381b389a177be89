// bf16 products, the matmul contract of the bf16 payload
// (src/payload/bf16.rs:235-262): the operands widen to f32 exactly (bf16 is
// the top half of a single), the f32 product is taken, and every output
// element rounds once to bf16 (Bf16::from_f32, :38-46).
//
// Exact posture: the widened operands go through the bit-identical f32
// kernel (gemm::multiply's seed and ascending k), then round: bit-identical.
// Fast posture: gfx950's bf16 matrix cores (v_mfma_f32_32x32x16_bf16),
// which multiply bf16 pairs exactly and accumulate in f32 in their own
// order: the envelope, then the same single rounding.
#pragma clang fp contract(off)
#include "backend.hpp"

namespace topos_hip {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// Bf16::from_f32: round to nearest with ties to even by adding the rounding
// bias to the bits (the carry runs into the exponent, so overflow reaches
// infinity); a NaN keeps its top half with a mantissa bit forced on.
__device__ __forceinline__ uint16_t bf16_of(float x) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, x);
  if (x != x) return (uint16_t)((bits >> 16) | 0x0040u);
  return (uint16_t)((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float f32_of(uint16_t h) { return __builtin_bit_cast(float, (uint32_t)h << 16); }

// Widens an [outer, inner] view (strides outer_stride, inner_stride) into a
// dense f32 [outer][inner] buffer.
__global__ __launch_bounds__(256) void widen_kernel(const uint16_t *__restrict__ in, int64_t outer, int64_t inner,
                                                    int64_t outer_stride, int64_t inner_stride,
                                                    float *__restrict__ out) {
  const int64_t count = outer * inner;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t o = i / inner, j = i - o * inner;
    out[i] = f32_of(in[o * outer_stride + j * inner_stride]);
  }
}

__global__ __launch_bounds__(256) void narrow_kernel(const float *__restrict__ in, int64_t m, int64_t n,
                                                     uint16_t *__restrict__ out, int64_t ldc) {
  const int64_t total = m * n;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / n, c = i - r * n;
    out[r * ldc + c] = bf16_of(in[i]);
  }
}

// The matrix-core kernel: 128x128 output tiles of four waves, each wave a
// 64x64 block of 2x2 MFMA blocks (32x32, k = 16 a product). k is staged 32
// deep through LDS, double-buffered, each operand stored [outer][k] so a
// lane's MFMA operand (eight consecutive k of one row or column) is one
// 16-byte LDS read: lane l takes row (column) l % 32 and k = 8 (l / 32) ..
// 8 (l / 32) + 7 of each 16-deep step, for both operands alike.
// kLeftInnerK / kRightInnerK: the operand's k axis has unit stride (else its
// outer axis has). kVector: 16-byte global loads (every row start 16-byte
// aligned along the unit-stride axis); otherwise element loads.
constexpr int kBK = 32;
constexpr int kRowPad = 8;  // LDS row of 40 bf16 (80 bytes): 16-byte aligned, banks spread

template <bool kInnerK, bool kVector>
struct Bf16Slab;

// k-contiguous operand: 128 rows x 32 k = 512 chunks of eight bf16 (one
// 16-byte load and one 16-byte LDS store each), two a thread; chunk c is
// row c / 4, k octet c % 4.
template <bool kVector>
struct Bf16Slab<true, kVector> {
  uint4 v[2];

  __device__ void fetch(const uint16_t *__restrict__ p, int64_t outer_stride, int64_t k_stride, int64_t outer_extent,
                        int64_t k, int64_t o0, int64_t k0) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int c = threadIdx.x + 256 * e;
      const int64_t go = o0 + c / 4, gk = k0 + 8 * (c % 4);
      if (kVector && go < outer_extent && gk + 7 < k) {
        v[e] = *reinterpret_cast<const uint4 *>(p + go * outer_stride + gk);
      } else {
        uint16_t h[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
          h[q] = (go < outer_extent && gk + q < k) ? p[go * outer_stride + (gk + q) * k_stride] : (uint16_t)0;
        v[e] = make_uint4((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16),
                          (uint32_t)h[4] | ((uint32_t)h[5] << 16), (uint32_t)h[6] | ((uint32_t)h[7] << 16));
      }
    }
  }

  __device__ void deposit(uint16_t (*lds)[kBK + kRowPad]) const {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int c = threadIdx.x + 256 * e;
      *reinterpret_cast<uint4 *>(&lds[c / 4][8 * (c % 4)]) = v[e];
    }
  }
};

// Outer-contiguous operand: a thread takes two neighbouring outer elements
// over eight k rows (eight 4-byte loads, consecutive threads on consecutive
// pairs: coalesced) and writes them as two 16-byte LDS rows; thread t takes
// pair t % 64, k octet t / 64.
template <bool kVector>
struct Bf16Slab<false, kVector> {
  uint32_t w[8];

  __device__ void fetch(const uint16_t *__restrict__ p, int64_t outer_stride, int64_t k_stride, int64_t outer_extent,
                        int64_t k, int64_t o0, int64_t k0) {
    const int t = threadIdx.x;
    const int64_t go = o0 + 2 * (t % 64), gk = k0 + 8 * (t / 64);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t kk = gk + i;
      if (kVector && go + 1 < outer_extent && kk < k) {
        w[i] = *reinterpret_cast<const uint32_t *>(p + kk * k_stride + go);
      } else {
        const uint32_t lo = (go < outer_extent && kk < k) ? p[kk * k_stride + go * outer_stride] : 0u;
        const uint32_t hi = (go + 1 < outer_extent && kk < k) ? p[kk * k_stride + (go + 1) * outer_stride] : 0u;
        w[i] = lo | (hi << 16);
      }
    }
  }

  __device__ void deposit(uint16_t (*lds)[kBK + kRowPad]) const {
    const int t = threadIdx.x;
    const int o = 2 * (t % 64), q = t / 64;
    uint4 lo, hi;
    lo.x = (w[0] & 0xffffu) | (w[1] << 16);
    lo.y = (w[2] & 0xffffu) | (w[3] << 16);
    lo.z = (w[4] & 0xffffu) | (w[5] << 16);
    lo.w = (w[6] & 0xffffu) | (w[7] << 16);
    hi.x = (w[0] >> 16) | (w[1] & 0xffff0000u);
    hi.y = (w[2] >> 16) | (w[3] & 0xffff0000u);
    hi.z = (w[4] >> 16) | (w[5] & 0xffff0000u);
    hi.w = (w[6] >> 16) | (w[7] & 0xffff0000u);
    *reinterpret_cast<uint4 *>(&lds[o][8 * q]) = lo;
    *reinterpret_cast<uint4 *>(&lds[o + 1][8 * q]) = hi;
  }
};

template <bool kLeftInnerK, bool kRightInnerK, bool kVector>
__global__ __launch_bounds__(256) void gemm_bf16_mfma_kernel(const uint16_t *__restrict__ a, int64_t a_rs,
                                                             int64_t a_cs, const uint16_t *__restrict__ b,
                                                             int64_t b_rs, int64_t b_cs, int64_t m, int64_t k,
                                                             int64_t n, uint16_t *__restrict__ c, int64_t ldc,
                                                             int grid_m, int grid_n) {
  __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][128][kBK + kRowPad];
  __shared__ __attribute__((aligned(16))) uint16_t lds_b[2][128][kBK + kRowPad];
  // Groups of eight tile rows walk the columns together (operand panels
  // reused from L2).
  const int pid = blockIdx.x;
  const int in_group = 8 * grid_n;
  const int first_m = (pid / in_group) * 8;
  const int group_rows = min(grid_m - first_m, 8);
  const int64_t m0 = (int64_t)(first_m + (pid % in_group) % group_rows) * 128;
  const int64_t n0 = (int64_t)((pid % in_group) / group_rows) * 128;
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const int wm = (wave / 2) * 64, wn = (wave % 2) * 64;
  const int half = lane / 32, l32 = lane % 32;

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  Bf16Slab<kLeftInnerK, kVector> sa;
  Bf16Slab<kRightInnerK, kVector> sb;
  const int slabs = (int)((k + kBK - 1) / kBK);
  sa.fetch(a, a_rs, a_cs, m, k, m0, 0);
  sb.fetch(b, b_cs, b_rs, n, k, n0, 0);
  sa.deposit(lds_a[0]);
  sb.deposit(lds_b[0]);
  __syncthreads();
  for (int s = 0; s < slabs; ++s) {
    const int buf = s & 1;
    if (s + 1 < slabs) {
      sa.fetch(a, a_rs, a_cs, m, k, m0, (int64_t)(s + 1) * kBK);
      sb.fetch(b, b_cs, b_rs, n, k, n0, (int64_t)(s + 1) * kBK);
    }
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      bf16x8 af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        af[i] = *reinterpret_cast<const bf16x8 *>(&lds_a[buf][wm + 32 * i + l32][16 * ks + 8 * half]);
        bfr[i] = *reinterpret_cast<const bf16x8 *>(&lds_b[buf][wn + 32 * i + l32][16 * ks + 8 * half]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (s + 1 < slabs) {
      sa.deposit(lds_a[buf ^ 1]);
      sb.deposit(lds_b[buf ^ 1]);
    }
    __syncthreads();
  }
  // Accumulator element r of block (i, j): row 8 (r / 4) + 4 (lane / 32) +
  // r % 4 and column lane % 32 of the block.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = n0 + wn + 32 * j + l32;
      if (col >= n) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm + 32 * i + 8 * (r / 4) + 4 * half + (r % 4);
        if (row < m) c[row * ldc + col] = bf16_of(acc[i][j][r]);
      }
    }
}

template <bool kL, bool kR>
void dispatch_bf16(bool vector, dim3 grid, hipStream_t stream, const uint16_t *a, int64_t a_rs, int64_t a_cs,
                   const uint16_t *b, int64_t b_rs, int64_t b_cs, int64_t m, int64_t k, int64_t n, uint16_t *c,
                   int64_t ldc, int gm, int gn) {
  if (vector)
    gemm_bf16_mfma_kernel<kL, kR, true><<<grid, 256, 0, stream>>>(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, gm, gn);
  else
    gemm_bf16_mfma_kernel<kL, kR, false><<<grid, 256, 0, stream>>>(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, gm,
                                                                  gn);
}

unsigned blocks_for(int64_t count) {
  const int64_t blocks = (count + 255) / 256;
  return (unsigned)std::min<int64_t>(std::max<int64_t>(blocks, 1), 256 * 64);
}

}  // namespace

bool bf16_mfma_serves(int64_t a_rs, int64_t a_cs, int64_t b_rs, int64_t b_cs) {
  return (a_cs == 1 || a_rs == 1) && (b_rs == 1 || b_cs == 1);
}

void launch_gemm_bf16_mfma(const uint16_t *a, int64_t a_rs, int64_t a_cs, const uint16_t *b, int64_t b_rs,
                           int64_t b_cs, int64_t m, int64_t k, int64_t n, uint16_t *c, int64_t ldc,
                           hipStream_t stream) {
  const bool lk = a_cs == 1, rk = b_rs == 1;
  // Vector loads: 16 bytes along a k-contiguous operand's rows, 4 bytes along
  // an outer-contiguous operand's k rows; every row start aligned to them.
  const int64_t a_step = lk ? a_rs : a_cs, b_step = rk ? b_cs : b_rs;
  const int a_align = lk ? 8 : 2, b_align = rk ? 8 : 2;  // in elements
  const bool vector = reinterpret_cast<uintptr_t>(a) % (2 * a_align) == 0 &&
                      reinterpret_cast<uintptr_t>(b) % (2 * b_align) == 0 && a_step % a_align == 0 &&
                      b_step % b_align == 0;
  const int64_t gm = (m + 127) / 128, gn = (n + 127) / 128;
  if (gm * gn > 0x7fffffff) throw Unsupported{"bf16 gemm: grid too large"};
  const dim3 grid((unsigned)(gm * gn));
  if (lk && rk)
    dispatch_bf16<true, true>(vector, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, (int)gm, (int)gn);
  else if (lk)
    dispatch_bf16<true, false>(vector, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, (int)gm, (int)gn);
  else if (rk)
    dispatch_bf16<false, true>(vector, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, (int)gm, (int)gn);
  else
    dispatch_bf16<false, false>(vector, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, (int)gm,
                                (int)gn);
  check_launch("gemm_bf16_mfma_kernel launch");
}

void launch_widen_bf16(const uint16_t *in, int64_t outer, int64_t inner, int64_t outer_stride, int64_t inner_stride,
                       float *out, hipStream_t stream) {
  widen_kernel<<<blocks_for(outer * inner), 256, 0, stream>>>(in, outer, inner, outer_stride, inner_stride, out);
  check_launch("widen_kernel launch");
}

void launch_narrow_bf16(const float *in, int64_t m, int64_t n, uint16_t *out, int64_t ldc, hipStream_t stream) {
  narrow_kernel<<<blocks_for(m * n), 256, 0, stream>>>(in, m, n, out, ldc);
  check_launch("narrow_kernel launch");
}

}  // namespace topos_hip
