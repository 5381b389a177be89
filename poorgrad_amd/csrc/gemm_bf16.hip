// bf16 products, the matmul contract of the bf16 payload
// (src/payload/bf16.rs:235-262): the operands widen to f32 exactly (bf16 is
// the top half of a single), the f32 product is taken, and every output
// element rounds once to bf16 (Bf16::from_f32, :38-46).
//
// Exact posture: the widened operands go through the bit-identical f32
// kernel (gemm::multiply's seed and ascending k), then round: bit-identical.
// Fast posture: gfx950's bf16 matrix cores (v_mfma_f32_16x16x32_bf16),
// which multiply bf16 pairs exactly and accumulate in f32 in their own
// order: the envelope, then the same single rounding.
#pragma clang fp contract(off)
#include "backend.hpp"
#include "lds_dma.hpp"

#include <type_traits>

namespace topos_hip {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

using namespace lds_dma;

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

// The matrix-core kernel: BM x BN output tiles (256x256 of sixteen waves,
// 256x128 of eight, or 128x128 of four), each wave a 64x64 block of 4x4
// 16x16 accumulator blocks fed by v_mfma_f32_16x16x32_bf16. k is staged 32
// deep in P LDS stages written by global_load_lds_dwordx4 (slab s + P - 1 in
// flight while slab s feeds the matrix cores; one wait and one barrier per
// slab). Both operands are
// k-contiguous here: a 32-deep bf16 row is 64 bytes, the f32 products'
// 16-deep row, so the slab layout is theirs (16 rows a KB, the 16-byte
// octets of k swizzled by row). Lane l reads octet g = l / 16 of row (or
// column) l % 16, eight consecutive k, one 16-byte LDS read, and the MFMA
// takes them for both operands alike, so the k order inside an MFMA is the
// same for A and B. Operands that are not k-contiguous, or whose rows are not
// 4-byte aligned, are first packed into k-contiguous rows (pack kernels
// below). Rows past an operand's edge load a clamped in-range row and feed
// only outputs that are not stored; a slab crossing k_end goes through
// registers with zeros past it.
constexpr int kSlabK = 32;  // bf16 k per slab: 64-byte rows

// One slab of a k-contiguous operand (outer extent O, rows outer_stride
// apart) into `lds`: O / 16 wave-wide DMA loads, spread over the W waves.
template <int O, int W>
__device__ __forceinline__ void bf16_dma_slab(const uint16_t *__restrict__ p, int64_t outer_stride,
                                              int64_t outer_extent, int64_t o0, int64_t k0, float *lds, int wave,
                                              int lane) {
  constexpr int kChunks = O / 16;  // 1 KB per wave-wide load
  static_assert(kChunks % W == 0, "whole chunks per wave");
#pragma unroll
  for (int i = 0; i < kChunks / W; ++i) {
    const int c = wave + W * i;
    const int r = lane >> 2;
    const int q = (lane & 3) ^ dma_swizzle(r);
    const int64_t row = min(o0 + 16 * c + r, outer_extent - 1);
    TOPOS_COMPILER_FENCE();
    dma_load16(p + row * outer_stride + (k0 + 8 * q), lds_byte_address(lds) + 1024 * c);
    TOPOS_COMPILER_FENCE();
  }
}

// The same slab through registers with zeros past k_end (the k tail).
template <int O, int W>
__device__ __forceinline__ void bf16_guarded_slab(const uint16_t *__restrict__ p, int64_t outer_stride,
                                                  int64_t outer_extent, int64_t k_end, int64_t o0, int64_t k0,
                                                  float *lds, int wave, int lane) {
  constexpr int kChunks = O / 16;
#pragma unroll
  for (int i = 0; i < kChunks / W; ++i) {
    const int c = wave + W * i;
    const int r = lane >> 2;
    const int q = (lane & 3) ^ dma_swizzle(r);
    const uint16_t *row = p + min(o0 + 16 * c + r, outer_extent - 1) * outer_stride;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t kk = k0 + 8 * q + 2 * e;
      const uint32_t lo = kk < k_end ? row[kk] : 0u;
      const uint32_t hi = kk + 1 < k_end ? row[kk + 1] : 0u;
      w[e] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4 *>(lds + c * 256 + 4 * lane) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// One slab's fragment reads and matrix-core products for a wave's 64x64
// block. kT: the products go in as B^T A^T, so a lane holds one output row
// (16i + l % 16) and four consecutive columns (16j + 4g + {0..3}); otherwise
// a lane holds one column (16j + l % 16) and rows 16i + 4g + r.
template <bool kT>
__device__ __forceinline__ void bf16_mfma_slab(const float *sa, const float *sb, int wm, int wn, int lane,
                                               floatx4 (&acc)[4][4]) {
  const int l16 = lane % 16, g = lane / 16;
  const int at = 4 * (4 * l16 + (g ^ dma_swizzle(l16)));  // within a 16-row KB
  bf16x8 av[4], bv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) av[i] = *reinterpret_cast<const bf16x8 *>(sa + 256 * ((wm >> 4) + i) + at);
#pragma unroll
  for (int j = 0; j < 4; ++j) bv[j] = *reinterpret_cast<const bf16x8 *>(sb + 256 * ((wn >> 4) + j) + at);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = kT ? __builtin_amdgcn_mfma_f32_16x16x32_bf16(bv[j], av[i], acc[i][j], 0, 0, 0)
                     : __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i], bv[j], acc[i][j], 0, 0, 0);
}

// Waits until the next slab has landed, with `ahead` slabs issued after it
// (uniform, at most A): vmcnt(ahead * kIssue).
template <int kIssue, int A>
__device__ __forceinline__ void wait_for_next(int ahead) {
  if constexpr (A > 0) {
    if (ahead >= A) {
      dma_wait<A * kIssue>();
      return;
    }
    wait_for_next<kIssue, A - 1>(ahead);
  } else {
    dma_wait<0>();
  }
}

// Output element stores: rounded once to bf16 into c (rows ldc apart), or
// the f32 sums of k range z into partials + z * m * n (rows n apart).
// kT: four consecutive columns a lane, one 8-byte (bf16) or 16-byte (f32)
// store when they are inside the output.
template <bool kT, bool kPartials>
__device__ __forceinline__ void bf16_store(const floatx4 (&acc)[4][4], uint16_t *__restrict__ c, int64_t ldc,
                                           float *__restrict__ partials, int64_t m, int64_t n, int64_t m0,
                                           int64_t n0, int wm, int wn, int lane) {
  const int l16 = lane % 16, g = lane / 16;
  if (kT) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = m0 + wm + 16 * i + l16;
      if (row >= m) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t col = n0 + wn + 16 * j + 4 * g;
        if (kPartials) {
          float *out = partials + row * n + col;
          if (col + 3 < n) {
            *reinterpret_cast<float4 *>(out) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (col + e < n) out[e] = acc[i][j][e];
          }
        } else {
          uint16_t *out = c + row * ldc + col;
          if (col + 3 < n) {
            *reinterpret_cast<uint2 *>(out) =
                make_uint2((uint32_t)bf16_of(acc[i][j][0]) | ((uint32_t)bf16_of(acc[i][j][1]) << 16),
                           (uint32_t)bf16_of(acc[i][j][2]) | ((uint32_t)bf16_of(acc[i][j][3]) << 16));
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (col + e < n) out[e] = bf16_of(acc[i][j][e]);
          }
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = n0 + wn + 16 * j + l16;
      if (col >= n) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = m0 + wm + 16 * i + 4 * g + r;
        if (row >= m) continue;
        if (kPartials)
          partials[row * n + col] = acc[i][j][r];
        else
          c[row * ldc + col] = bf16_of(acc[i][j][r]);
      }
    }
}

// Workgroups of one kernel shape that fit a CU's 160 KB of LDS, and the
// waves each SIMD then holds (the register budget: 512 / that many).
constexpr int bf16_lds_bytes(int bm, int bn, int p) { return p * (bm + bn) * kSlabK * 2; }
constexpr int bf16_waves_per_simd(int bm, int bn, int p) {
  return (163840 / bf16_lds_bytes(bm, bn, p)) * (bm / 64) * (bn / 64) / 4;
}

// a: [m][k] rows a_rs apart, b: [n][k] rows b_cs apart (B^T's rows), both
// k-contiguous with 4-byte aligned rows. P stages: slab s + P - 1 is issued
// while slab s feeds the matrix cores. With kPartials, range z = blockIdx.z
// of k ([z * split_len, ..)) writes its f32 sums to partials.
template <int BM, int BN, int P, bool kT, bool kPartials>
__global__ __launch_bounds__(BM * BN / 64, bf16_waves_per_simd(BM, BN, P)) void gemm_bf16_dma_kernel(
    const uint16_t *__restrict__ a, int64_t a_rs, const uint16_t *__restrict__ b, int64_t b_cs, int64_t m,
    int64_t k, int64_t n, uint16_t *__restrict__ c, int64_t ldc, float *__restrict__ partials, int grid_m,
    int grid_n, int64_t split_len) {
  constexpr int WN = BN / 64;
  constexpr int W = BM / 64 * WN;                            // waves, one 64x64 block each
  constexpr int SA = BM * kSlabK / 2, SB = BN * kSlabK / 2;  // 4-byte words per stage
  constexpr int kIssue = (BM / 16 + BN / 16) / W;           // DMA loads per wave per slab
  static_assert((BM / 16) % W == 0 && (BN / 16) % W == 0, "whole chunks per wave");
  static_assert(P >= 2 && (P - 2) * kIssue < 16, "slabs in flight within the vmcnt field");
  __shared__ __attribute__((aligned(1024))) float lds[P * (SA + SB)];

  const int64_t k_begin = kPartials ? (int64_t)blockIdx.z * split_len : 0;
  const int64_t k_end = kPartials ? min(k, k_begin + split_len) : k;
  if (kPartials) partials += (int64_t)blockIdx.z * m * n;

  // Consecutive workgroups go to different XCDs: renumber so each XCD takes
  // a contiguous run of tiles, then groups of eight tile rows walk the
  // columns together (operand panels reused from that XCD's L2).
  const int blocks = grid_m * grid_n;
  int pid = blockIdx.x;
  if (blocks % 8 == 0) pid = (pid % 8) * (blocks / 8) + pid / 8;
  const int in_group = 8 * grid_n;
  const int first_m = (pid / in_group) * 8;
  const int group_rows = min(grid_m - first_m, 8);
  const int64_t m0 = (int64_t)(first_m + (pid % in_group) % group_rows) * BM;
  const int64_t n0 = (int64_t)((pid % in_group) / group_rows) * BN;

  const int lane = threadIdx.x % 64;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const int wm = (wave / WN) * 64, wn = (wave % WN) * 64;

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;

  auto issue = [&](int s) {
    float *stage = lds + (s % P) * (SA + SB);
    const int64_t k0 = k_begin + (int64_t)s * kSlabK;
    if (k0 + kSlabK > k_end) {
      bf16_guarded_slab<BM, W>(a, a_rs, m, k_end, m0, k0, stage, wave, lane);
      bf16_guarded_slab<BN, W>(b, b_cs, n, k_end, n0, k0, stage + SA, wave, lane);
    } else {
      bf16_dma_slab<BM, W>(a, a_rs, m, m0, k0, stage, wave, lane);
      bf16_dma_slab<BN, W>(b, b_cs, n, n0, k0, stage + SA, wave, lane);
    }
  };
  const int slabs = (int)((k_end - k_begin + kSlabK - 1) / kSlabK);
  for (int s = 0; s < P - 1 && s < slabs; ++s) issue(s);
  wait_for_next<kIssue, P - 2>(min(P - 2, slabs - 1));
  dma_barrier();
  // P slabs a trip while every slab issued in it is a whole DMA slab: the
  // stages are compile-time offsets and a slab has no branch of its own.
  // The last slabs take the general loop below.
  int s = 0;
  {
    auto steady = [&](auto stage_index) {
      constexpr int st = decltype(stage_index)::value;  // s % P
      const int64_t k0 = k_begin + (int64_t)(s + P - 1) * kSlabK;
      float *stage = lds + ((st + P - 1) % P) * (SA + SB);
      bf16_dma_slab<BM, W>(a, a_rs, m, m0, k0, stage, wave, lane);
      bf16_dma_slab<BN, W>(b, b_cs, n, n0, k0, stage + SA, wave, lane);
      const float *sa = lds + st * (SA + SB);
      bf16_mfma_slab<kT>(sa, sa + SA, wm, wn, lane, acc);
      dma_wait<(P - 2) * kIssue>();
      dma_barrier();
      ++s;
    };
    const int whole = (int)((k_end - k_begin) / kSlabK);  // slabs without a k tail
    while (s + 2 * P - 1 <= whole) {
      steady(std::integral_constant<int, 0>{});
      steady(std::integral_constant<int, 1>{});
      if constexpr (P > 2) steady(std::integral_constant<int, 2 % P>{});
      if constexpr (P > 3) steady(std::integral_constant<int, 3 % P>{});
      static_assert(P <= 4, "unrolled to four stages");
    }
  }
  for (; s < slabs; ++s) {
    // Stage (s + P - 1) % P held slab s - 1, which every wave finished
    // before the last barrier.
    if (s + P - 1 < slabs) issue(s + P - 1);
    const float *sa = lds + (s % P) * (SA + SB);
    bf16_mfma_slab<kT>(sa, sa + SA, wm, wn, lane, acc);
    if (s + 1 < slabs) {
      wait_for_next<kIssue, P - 2>(min(P - 2, slabs - 2 - s));
      dma_barrier();
    }
  }
  bf16_store<kT, kPartials>(acc, c, ldc, partials, m, n, m0, n0, wm, wn, lane);
}

// Packs an operand view into k-contiguous rows: element (o, kk), at
// p[o * outer_stride + kk * k_stride], goes to q[o * kp + kk]. An
// outer-contiguous view (outer_stride 1) is transposed through 64 x 64 LDS
// tiles: 16-byte loads along the input's rows, 16-byte stores along the
// output's (kVector: those accesses aligned); any other view is gathered
// element by element, consecutive lanes along k.
template <bool kVector>
__global__ __launch_bounds__(256) void pack_transpose_kernel(const uint16_t *__restrict__ p, int64_t outer,
                                                             int64_t kdim, int64_t k_stride,
                                                             uint16_t *__restrict__ q, int64_t kp, int tiles_o) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[64][64 + 8];  // [kk][o], 144-byte rows
  const int t = threadIdx.x;
  const int64_t o0 = (int64_t)(blockIdx.x % tiles_o) * 64, k0 = (int64_t)(blockIdx.x / tiles_o) * 64;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int kk = t / 8 + 32 * e, o = 8 * (t % 8);
    const uint16_t *src = p + (k0 + kk) * k_stride + o0 + o;
    if (kVector && k0 + kk < kdim && o0 + o + 7 < outer) {
      *reinterpret_cast<uint4 *>(&tile[kk][o]) = *reinterpret_cast<const uint4 *>(src);
    } else {
#pragma unroll
      for (int x = 0; x < 8; ++x) tile[kk][o + x] = (k0 + kk < kdim && o0 + o + x < outer) ? src[x] : (uint16_t)0;
    }
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int o = t / 8 + 32 * e, kk = 8 * (t % 8);
    if (o0 + o >= outer) continue;
    uint16_t *dst = q + (o0 + o) * kp + k0 + kk;
    uint32_t w[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) w[x] = (uint32_t)tile[kk + 2 * x][o] | ((uint32_t)tile[kk + 2 * x + 1][o] << 16);
    if (kVector && k0 + kk + 7 < kdim) {
      *reinterpret_cast<uint4 *>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
#pragma unroll
      for (int x = 0; x < 8; ++x)
        if (k0 + kk + x < kdim) dst[x] = tile[kk + x][o];
    }
  }
}

__global__ __launch_bounds__(256) void pack_gather_kernel(const uint16_t *__restrict__ p, int64_t outer,
                                                          int64_t kdim, int64_t outer_stride, int64_t k_stride,
                                                          uint16_t *__restrict__ q, int64_t kp) {
  const int64_t count = outer * kdim;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t o = i / kdim, kk = i - o * kdim;
    q[o * kp + kk] = p[o * outer_stride + kk * k_stride];
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

unsigned blocks_for(int64_t count) {
  const int64_t blocks = (count + 255) / 256;
  return (unsigned)std::min<int64_t>(std::max<int64_t>(blocks, 1), 256 * 64);
}

int64_t whole_words(int64_t halves) { return (halves + 127) / 128 * 64; }  // 4-byte words, 256-byte multiples

// An operand the DMA kernel reads in place: k-contiguous, every row start
// 4-byte aligned (the DMA's 16-byte loads need no more).
bool dma_ready(const uint16_t *p, int64_t outer_stride, int64_t k_stride, int64_t outer) {
  return k_stride == 1 && reinterpret_cast<uintptr_t>(p) % 4 == 0 && (outer_stride % 2 == 0 || outer == 1);
}

struct Bf16Plan {
  bool pack_a = false, pack_b = false;
  int64_t kp = 0;  // packed row length: k rounded up to 8 (16-byte rows)
  int bm = 128, bn = 128;  // tile
  int stages = 3;          // LDS stages (slabs in flight: stages - 1)
  int splits = 1;
  int64_t split_len = 0;
  int64_t a_words = 0, b_words = 0, partial_words = 0;  // workspace pieces
};

Bf16Plan bf16_plan(const uint16_t *a, int64_t a_rs, int64_t a_cs, const uint16_t *b, int64_t b_rs, int64_t b_cs,
                   int64_t m, int64_t k, int64_t n) {
  Bf16Plan plan;
  plan.pack_a = !dma_ready(a, a_rs, a_cs, m);
  plan.pack_b = !dma_ready(b, b_cs, b_rs, n);
  plan.kp = (k + 7) / 8 * 8;
  if (plan.pack_a) plan.a_words = whole_words(m * plan.kp);
  if (plan.pack_b) plan.b_words = whole_words(n * plan.kp);
  // Tile shapes, from a sweep of every shape, stage count and split over the
  // GEMM sweep's products on MI355X: 256x256 tiles (sixteen waves, one
  // workgroup a CU, four stages) when they fill whole rounds without padding
  // either extent by more than an eighth (4096^3: 954-1093 TFLOP/s against
  // 818-928 on 256x128); 256x128 (two a CU, three stages) when those fill a
  // round ([8192, 3072] over 768: 643 against 570 on 256x256, which leaves
  // half a round); else 128x128 (two a CU, four stages: three measured 1-2%
  // slower).
  auto fills = [](int64_t extent, int64_t tile) { return ((extent + tile - 1) / tile * tile - extent) * 8 <= extent; };
  const int64_t big = ((m + 255) / 256) * ((n + 255) / 256);
  if (fills(m, 256) && fills(n, 256) && k >= 1024 && (big % 256 == 0 || big >= 1024)) {
    plan.bm = 256, plan.bn = 256, plan.stages = 4;
  } else if (fills(m, 256) && ((m + 255) / 256) * ((n + 127) / 128) >= 512) {
    plan.bm = 256, plan.bn = 128, plan.stages = 3;
  } else {
    plan.bm = 128, plan.bn = 128, plan.stages = 4;
  }
  // Only products with fewer tiles than CUs split k, into at most four
  // ranges (at most two workgroups a CU), each at least 512 deep (128 below
  // k = 2048). The bf16 matrix cores finish a range quickly, so the partials'
  // extra pass costs more than it does for f32: [8192, 768] over 3072 (384
  // tiles) ran at 575 TFLOP/s unsplit against 453 in two ranges, [1024, 1024]
  // over 4096 (64 tiles) at 262 in four against 233 in eight.
  const int64_t tiles = ((m + plan.bm - 1) / plan.bm) * ((n + plan.bn - 1) / plan.bn);
  const int64_t shortest = k < 2048 ? 128 : 512;
  int64_t s = 1;
  if (tiles < 256)
    while (s < 4 && tiles * (s + 1) <= 512 && k / (s + 1) >= shortest) ++s;
  plan.split_len = k;
  if (s > 1) {
    plan.split_len = ((k + s - 1) / s + kSlabK - 1) / kSlabK * kSlabK;
    s = (k + plan.split_len - 1) / plan.split_len;
  }
  plan.splits = (int)s;
  if (plan.splits > 1) plan.partial_words = plan.splits * m * n;
  return plan;
}

// Packs the [outer, kdim] view (element (o, kk) at p[o * os + kk * ks]) into
// q's k-contiguous rows of kp.
void pack_rows(const uint16_t *p, int64_t outer, int64_t kdim, int64_t os, int64_t ks, uint16_t *q, int64_t kp,
               hipStream_t stream) {
  if (os == 1) {
    const int64_t tiles_o = (outer + 63) / 64, tiles_k = (kdim + 63) / 64;
    if (tiles_o * tiles_k > 0x7fffffff) throw Unsupported{"bf16 gemm: operand too large to pack"};
    const bool vector = reinterpret_cast<uintptr_t>(p) % 16 == 0 && ks % 8 == 0;
    const dim3 grid((unsigned)(tiles_o * tiles_k));
    if (vector)
      pack_transpose_kernel<true><<<grid, 256, 0, stream>>>(p, outer, kdim, ks, q, kp, (int)tiles_o);
    else
      pack_transpose_kernel<false><<<grid, 256, 0, stream>>>(p, outer, kdim, ks, q, kp, (int)tiles_o);
    check_launch("pack_transpose_kernel launch");
  } else {
    pack_gather_kernel<<<blocks_for(outer * kdim), 256, 0, stream>>>(p, outer, kdim, os, ks, q, kp);
    check_launch("pack_gather_kernel launch");
  }
}

template <int BM, int BN, int P>
void dispatch_bf16(bool vector_out, dim3 grid, hipStream_t stream, const uint16_t *a, int64_t a_row,
                   const uint16_t *b, int64_t b_row, int64_t m, int64_t k, int64_t n, uint16_t *c, int64_t ldc,
                   float *partials, int gm, int gn, int64_t split_len) {
  constexpr int T = BM * BN / 64;
#define TOPOS_BF16_LAUNCH(kT, kP) \
  gemm_bf16_dma_kernel<BM, BN, P, kT, kP><<<grid, T, 0, stream>>>(a, a_row, b, b_row, m, k, n, c, ldc, partials, gm, gn, split_len)
  if (partials && vector_out)
    TOPOS_BF16_LAUNCH(true, true);
  else if (partials)
    TOPOS_BF16_LAUNCH(false, true);
  else if (vector_out)
    TOPOS_BF16_LAUNCH(true, false);
  else
    TOPOS_BF16_LAUNCH(false, false);
#undef TOPOS_BF16_LAUNCH
}

// The kernel shapes the planner chooses from: (tile rows, tile columns,
// stages).
#define TOPOS_BF16_SHAPES(X) X(256, 256, 4) X(256, 128, 3) X(128, 128, 4)

void launch_bf16_plan(const Bf16Plan &plan, const uint16_t *a_in, int64_t a_row, const uint16_t *b_in, int64_t b_row,
                      int64_t m, int64_t k, int64_t n, uint16_t *c, int64_t ldc, float *partials, hipStream_t stream) {
  const int64_t gm = (m + plan.bm - 1) / plan.bm, gn = (n + plan.bn - 1) / plan.bn;
  if (gm * gn > 0x7fffffff) throw Unsupported{"bf16 gemm: grid too large"};
  const dim3 grid((unsigned)(gm * gn), 1, (unsigned)plan.splits);
  const bool vector_out = partials ? n % 4 == 0 : ldc % 4 == 0 && reinterpret_cast<uintptr_t>(c) % 8 == 0;
  bool launched = false;
#define TOPOS_BF16_SHAPE(BM, BN, P)                                                                               \
  if (!launched && plan.bm == BM && plan.bn == BN && plan.stages == P) {                                          \
    dispatch_bf16<BM, BN, P>(vector_out, grid, stream, a_in, a_row, b_in, b_row, m, k, n, c, ldc, partials, (int)gm, \
                             (int)gn, plan.split_len);                                                            \
    launched = true;                                                                                              \
  }
  TOPOS_BF16_SHAPES(TOPOS_BF16_SHAPE)
#undef TOPOS_BF16_SHAPE
  if (!launched) throw Unsupported{"bf16 gemm: no kernel for the planned tile"};
  check_launch("gemm_bf16_dma_kernel launch");
  if (partials) {
    reduce_bf16_kernel<<<blocks_for(m * n), 256, 0, stream>>>(partials, plan.splits, m, n, c, ldc);
    check_launch("reduce_bf16_kernel launch");
  }
}

}  // namespace

bool bf16_mfma_serves(int64_t a_rs, int64_t a_cs, int64_t b_rs, int64_t b_cs) {
  return (a_cs == 1 || a_rs == 1) && (b_rs == 1 || b_cs == 1);
}

int64_t bf16_fast_workspace_floats(const uint16_t *a, int64_t a_rs, int64_t a_cs, const uint16_t *b, int64_t b_rs,
                                   int64_t b_cs, int64_t m, int64_t k, int64_t n) {
  const Bf16Plan plan = bf16_plan(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n);
  return plan.a_words + plan.b_words + plan.partial_words;
}

void launch_gemm_bf16_fast(const uint16_t *a, int64_t a_rs, int64_t a_cs, const uint16_t *b, int64_t b_rs,
                           int64_t b_cs, int64_t m, int64_t k, int64_t n, uint16_t *c, int64_t ldc,
                           hipStream_t stream, float *workspace) {
  const Bf16Plan plan = bf16_plan(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n);
  if (plan.a_words + plan.b_words + plan.partial_words > 0 &&
      (!workspace || reinterpret_cast<uintptr_t>(workspace) % 256 != 0))
    throw Unsupported{"bf16 gemm: workspace missing or misaligned"};
  const uint16_t *a_in = a, *b_in = b;
  int64_t a_row = a_rs, b_row = b_cs;
  if (plan.pack_a) {
    uint16_t *q = reinterpret_cast<uint16_t *>(workspace);
    pack_rows(a, m, k, a_rs, a_cs, q, plan.kp, stream);
    a_in = q, a_row = plan.kp;
  }
  if (plan.pack_b) {
    uint16_t *q = reinterpret_cast<uint16_t *>(workspace + plan.a_words);
    pack_rows(b, n, k, b_cs, b_rs, q, plan.kp, stream);
    b_in = q, b_row = plan.kp;
  }
  float *partials = plan.splits > 1 ? workspace + plan.a_words + plan.b_words : nullptr;
  launch_bf16_plan(plan, a_in, a_row, b_in, b_row, m, k, n, c, ldc, partials, stream);
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
