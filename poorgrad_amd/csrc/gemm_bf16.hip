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

// Outer-contiguous operand: a thread takes four neighbouring outer elements
// over four k rows (four 8-byte loads, consecutive threads on consecutive
// quads: 256 contiguous bytes a k row), transposes them in registers and
// writes four 8-byte LDS pieces, one per outer element; thread t takes outer
// quad t % 32, k quad t / 32.
template <bool kVector>
struct Bf16Slab<false, kVector> {
  uint2 w[4];

  __device__ void fetch(const uint16_t *__restrict__ p, int64_t outer_stride, int64_t k_stride, int64_t outer_extent,
                        int64_t k, int64_t o0, int64_t k0) {
    const int t = threadIdx.x;
    const int64_t go = o0 + 4 * (t % 32), gk = k0 + 4 * (t / 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t kk = gk + i;
      if (kVector && go + 3 < outer_extent && kk < k) {
        w[i] = *reinterpret_cast<const uint2 *>(p + kk * k_stride + go);
      } else {
        uint32_t h[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          h[q] = (go + q < outer_extent && kk < k) ? p[kk * k_stride + (go + q) * outer_stride] : 0u;
        w[i] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
      }
    }
  }

  __device__ void deposit(uint16_t (*lds)[kBK + kRowPad]) const {
    const int t = threadIdx.x;
    const int o = 4 * (t % 32), kq = t / 32;
    // Outer element j of k row i is half (j % 2) of word (j / 2) of w[i].
    const uint2 r0 = make_uint2((w[0].x & 0xffffu) | (w[1].x << 16), (w[2].x & 0xffffu) | (w[3].x << 16));
    const uint2 r1 = make_uint2((w[0].x >> 16) | (w[1].x & 0xffff0000u), (w[2].x >> 16) | (w[3].x & 0xffff0000u));
    const uint2 r2 = make_uint2((w[0].y & 0xffffu) | (w[1].y << 16), (w[2].y & 0xffffu) | (w[3].y << 16));
    const uint2 r3 = make_uint2((w[0].y >> 16) | (w[1].y & 0xffff0000u), (w[2].y >> 16) | (w[3].y & 0xffff0000u));
    *reinterpret_cast<uint2 *>(&lds[o][4 * kq]) = r0;
    *reinterpret_cast<uint2 *>(&lds[o + 1][4 * kq]) = r1;
    *reinterpret_cast<uint2 *>(&lds[o + 2][4 * kq]) = r2;
    *reinterpret_cast<uint2 *>(&lds[o + 3][4 * kq]) = r3;
  }
};

// With `partials` set, range z = blockIdx.z of k ([z * split_len, ..)) is
// multiplied and its f32 sums written unrounded to partials + z * m * n
// (rows n apart); reduce_bf16_kernel adds the ranges and rounds once.
template <bool kLeftInnerK, bool kRightInnerK, bool kVector>
__global__ __launch_bounds__(256) void gemm_bf16_mfma_kernel(const uint16_t *__restrict__ a, int64_t a_rs,
                                                             int64_t a_cs, const uint16_t *__restrict__ b,
                                                             int64_t b_rs, int64_t b_cs, int64_t m, int64_t k,
                                                             int64_t n, uint16_t *__restrict__ c, int64_t ldc,
                                                             int grid_m, int grid_n, float *__restrict__ partials,
                                                             int64_t split_len) {
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
  const int64_t k_begin = partials ? (int64_t)blockIdx.z * split_len : 0;
  const int64_t k_end = partials ? min(k, k_begin + split_len) : k;
  const int slabs = (int)((k_end - k_begin + kBK - 1) / kBK);
  sa.fetch(a, a_rs, a_cs, m, k_end, m0, k_begin);
  sb.fetch(b, b_cs, b_rs, n, k_end, n0, k_begin);
  sa.deposit(lds_a[0]);
  sb.deposit(lds_b[0]);
  __syncthreads();
  for (int s = 0; s < slabs; ++s) {
    const int buf = s & 1;
    if (s + 1 < slabs) {
      sa.fetch(a, a_rs, a_cs, m, k_end, m0, k_begin + (int64_t)(s + 1) * kBK);
      sb.fetch(b, b_cs, b_rs, n, k_end, n0, k_begin + (int64_t)(s + 1) * kBK);
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
        if (row >= m) continue;
        if (partials)
          partials[(int64_t)blockIdx.z * m * n + row * n + col] = acc[i][j][r];
        else
          c[row * ldc + col] = bf16_of(acc[i][j][r]);
      }
    }
}

// The ranges' f32 sums added in range order, then rounded once to bf16.
__global__ __launch_bounds__(256) void reduce_bf16_kernel(const float *__restrict__ partials, int splits, int64_t m,
                                                          int64_t n, uint16_t *__restrict__ c, int64_t ldc) {
  const int64_t total = m * n;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    float acc = partials[i];
    for (int z = 1; z < splits; ++z) acc = acc + partials[(int64_t)z * total + i];
    const int64_t r = i / n, col = i - r * n;
    c[r * ldc + col] = bf16_of(acc);
  }
}

template <bool kL, bool kR>
void dispatch_bf16(bool vector, dim3 grid, hipStream_t stream, const uint16_t *a, int64_t a_rs, int64_t a_cs,
                   const uint16_t *b, int64_t b_rs, int64_t b_cs, int64_t m, int64_t k, int64_t n, uint16_t *c,
                   int64_t ldc, int gm, int gn, float *partials, int64_t split_len) {
  if (vector)
    gemm_bf16_mfma_kernel<kL, kR, true><<<grid, 256, 0, stream>>>(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, gm, gn,
                                                                 partials, split_len);
  else
    gemm_bf16_mfma_kernel<kL, kR, false><<<grid, 256, 0, stream>>>(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, gm,
                                                                  gn, partials, split_len);
}

unsigned blocks_for(int64_t count) {
  const int64_t blocks = (count + 255) / 256;
  return (unsigned)std::min<int64_t>(std::max<int64_t>(blocks, 1), 256 * 64);
}

}  // namespace

bool bf16_mfma_serves(int64_t a_rs, int64_t a_cs, int64_t b_rs, int64_t b_cs) {
  return (a_cs == 1 || a_rs == 1) && (b_rs == 1 || b_cs == 1);
}

int bf16_splits(int64_t m, int64_t n, int64_t k) {
  // Products with fewer 128x128 tiles than four per CU split k into ranges
  // of at least 512 (at most 16 of them) until they have that many
  // workgroups: the [3072, 768] weight gradient over k = 8192 (144 tiles)
  // went from 44 TFLOP/s unsplit to 184 in four ranges and 212 in eight.
  const int64_t tiles = ((m + 127) / 128) * ((n + 127) / 128);
  int64_t s = 1;
  while (s < 16 && tiles * s < 1024 && k / (2 * s) >= 512) s *= 2;
  return (int)s;
}

void launch_gemm_bf16_mfma(const uint16_t *a, int64_t a_rs, int64_t a_cs, const uint16_t *b, int64_t b_rs,
                           int64_t b_cs, int64_t m, int64_t k, int64_t n, uint16_t *c, int64_t ldc,
                           hipStream_t stream, float *partials, int splits) {
  const bool lk = a_cs == 1, rk = b_rs == 1;
  // Vector loads: 16 bytes along a k-contiguous operand's rows, 8 bytes along
  // an outer-contiguous operand's k rows; every row start aligned to them.
  const int64_t a_step = lk ? a_rs : a_cs, b_step = rk ? b_cs : b_rs;
  const int a_align = lk ? 8 : 4, b_align = rk ? 8 : 4;  // in elements
  const bool vector = reinterpret_cast<uintptr_t>(a) % (2 * a_align) == 0 &&
                      reinterpret_cast<uintptr_t>(b) % (2 * b_align) == 0 && a_step % a_align == 0 &&
                      b_step % b_align == 0;
  const int64_t gm = (m + 127) / 128, gn = (n + 127) / 128;
  if (gm * gn > 0x7fffffff) throw Unsupported{"bf16 gemm: grid too large"};
  if (splits < 1 || splits > 16 || (splits > 1 && !partials)) throw Unsupported{"bf16 gemm: split without partials"};
  int64_t split_len = k;
  if (splits > 1) {
    split_len = ((k + splits - 1) / splits + kBK - 1) / kBK * kBK;
    splits = (int)((k + split_len - 1) / split_len);
  }
  float *target = splits > 1 ? partials : nullptr;
  const dim3 grid((unsigned)(gm * gn), 1, (unsigned)splits);
  if (lk && rk)
    dispatch_bf16<true, true>(vector, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, (int)gm, (int)gn,
                              target, split_len);
  else if (lk)
    dispatch_bf16<true, false>(vector, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, (int)gm, (int)gn,
                               target, split_len);
  else if (rk)
    dispatch_bf16<false, true>(vector, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, (int)gm, (int)gn,
                               target, split_len);
  else
    dispatch_bf16<false, false>(vector, grid, stream, a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, (int)gm,
                                (int)gn, target, split_len);
  check_launch("gemm_bf16_mfma_kernel launch");
  if (splits > 1) {
    reduce_bf16_kernel<<<blocks_for(m * n), 256, 0, stream>>>(partials, splits, m, n, c, ldc);
    check_launch("reduce_bf16_kernel launch");
  }
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
