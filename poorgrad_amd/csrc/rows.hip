// Row reductions over the last axis of a contiguous [rows, columns] buffer:
// sum_along / max_along (src/payload/tensor.rs:1073-1124), LogSumExp
// (src/function/log_sum_exp.rs:53-61), LogSoftmax (src/function/log_softmax.rs:51-60),
// softmax = log_softmax.exp (src/graph/composite.rs:43-45) and LayerNorm
// (src/neural/layer_norm.rs:100-132).
//
// Exact posture: each row's fold is one lane's sequential chain, seeded with
// the row's first value and ascending in column order — the interpreter's
// accumulation order, so the bits match. A 256-lane workgroup owns kRows rows;
// all four waves stream coalesced 128-column slabs of those rows, apply the
// pass's elementwise transform (exp(x - peak), (x - mean)^2, ...) — the
// expensive part, spread over every SIMD — and park the values in LDS, where
// wave 0's lane r folds row r in order. Elementwise output passes are plain
// coalesced row-major sweeps using the per-row statistics.
//
// Fast posture: one wave per row, each lane folds a strided share and the
// wave combines by butterfly shuffles (reassociated: envelope fidelity). The
// max fold is order-independent under f32::max (NaN loses; +-0 ties are the
// only order-visible case), so both postures use the same maxima.
#pragma clang fp contract(off)
#include "backend.hpp"
#include "faithful_math.h"

namespace topos_hip {
namespace {

using topos_faithful::exp_f32;
using topos_faithful::ln_f32;
using topos_faithful::max_f32;

constexpr int kThreads = 256;
constexpr int kSlab = 128;  // columns per staged slab

enum Transform { kIdentity, kShiftedExp, kCentredSquare };
enum Fold { kSum, kMax };

// One exact pass over the kRows x columns block: lane r of wave 0 returns the
// ordered fold of T(x[r, c], stat[r]) over c = 0..columns-1.
template <int kRows, Transform kT, Fold kF, bool kVector>
__device__ float exact_fold(const float *__restrict__ x, int64_t rows, int64_t columns, int64_t row0,
                            const float *stat, float (*slab)[kSlab + 1]) {
  constexpr int kQuads = kRows * (kSlab / 4) / kThreads;  // float4s per lane per slab
  const int t = threadIdx.x;
  float acc = 0.0f;
  for (int64_t c0 = 0; c0 < columns; c0 += kSlab) {
    const int width = (columns - c0) < kSlab ? (int)(columns - c0) : kSlab;
    float v[kQuads][4];
#pragma unroll
    for (int e = 0; e < kQuads; ++e) {
      const int q = t + kThreads * e;
      const int r = q / (kSlab / 4);
      const int cq = (q % (kSlab / 4)) * 4;
      const int64_t row = row0 + r;
      if (kVector && row < rows && cq + 3 < width) {
        const float4 w = *reinterpret_cast<const float4 *>(x + row * columns + c0 + cq);
        v[e][0] = w.x; v[e][1] = w.y; v[e][2] = w.z; v[e][3] = w.w;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          v[e][i] = (row < rows && cq + i < width) ? x[row * columns + c0 + cq + i] : 0.0f;
      }
    }
    __syncthreads();  // wave 0 is done folding the previous slab
#pragma unroll
    for (int e = 0; e < kQuads; ++e) {
      const int q = t + kThreads * e;
      const int r = q / (kSlab / 4);
      const int cq = (q % (kSlab / 4)) * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float value = v[e][i];
        if (kT == kShiftedExp) value = exp_f32(value - stat[r]);
        if (kT == kCentredSquare) {
          const float centred = value - stat[r];
          value = centred * centred;
        }
        slab[r][cq + i] = value;
      }
    }
    __syncthreads();
    if (t < kRows) {
      int j = 0;
      if (c0 == 0) {
        acc = slab[t][0];  // the seed: the row's first value
        j = 1;
      }
      for (; j < width; ++j) {
        const float value = slab[t][j];
        acc = (kF == kSum) ? acc + value : max_f32(acc, value);
      }
    }
  }
  return acc;
}

// Coalesced elementwise output pass over the block's rows.
template <int kReduction, int kRows>
__device__ void exact_write(const float *__restrict__ x, int64_t rows, int64_t columns, int64_t row0,
                            const float *first, const float *second, const float *scale,
                            const float *shift, float *__restrict__ out) {
  const int64_t block_rows = (rows - row0) < kRows ? (rows - row0) : kRows;
  const int64_t total = block_rows * columns;
  for (int64_t i = threadIdx.x; i < total; i += kThreads) {
    const int r = (int)(i / columns);
    const int64_t c = i % columns;
    const int64_t at = (row0 + r) * columns + c;
    const float value = x[at];
    float result;
    if (kReduction == TOPOS_HIP_ROWS_LOG_SOFTMAX || kReduction == TOPOS_HIP_ROWS_SOFTMAX) {
      result = (value - first[r]) - second[r];  // shifted - normalizer
      if (kReduction == TOPOS_HIP_ROWS_SOFTMAX) result = exp_f32(result);
    } else {  // layer norm: (x - mean) / deviation * scale + shift
      const float normalized = (value - first[r]) / second[r];
      result = normalized * scale[c] + shift[c];
    }
    out[at] = result;
  }
}

constexpr int kLayerNorm = 100;

template <int kReduction, int kRows, bool kVector>
__global__ __launch_bounds__(kThreads) void rows_exact_kernel(const float *__restrict__ x, int64_t rows,
                                                              int64_t columns, const float *scale,
                                                              const float *shift, float epsilon,
                                                              float *__restrict__ out) {
  __shared__ float slab[kRows][kSlab + 1];
  __shared__ float first[kRows];
  __shared__ float second[kRows];
  const int64_t row0 = (int64_t)blockIdx.x * kRows;
  const int t = threadIdx.x;
  const bool owner = t < kRows && row0 + t < rows;

  if (kReduction == TOPOS_HIP_ROWS_SUM || kReduction == TOPOS_HIP_ROWS_MAX) {
    const float acc = exact_fold<kRows, kIdentity, kReduction == TOPOS_HIP_ROWS_SUM ? kSum : kMax, kVector>(
        x, rows, columns, row0, nullptr, slab);
    if (owner) out[row0 + t] = acc;
    return;
  }
  if (kReduction == kLayerNorm) {
    const float count = (float)columns;  // counted(shape, extent) as f32
    const float total = exact_fold<kRows, kIdentity, kSum, kVector>(x, rows, columns, row0, nullptr, slab);
    if (t < kRows) first[t] = total / count;  // mean
    __syncthreads();
    const float power = exact_fold<kRows, kCentredSquare, kSum, kVector>(x, rows, columns, row0, first, slab);
    if (t < kRows) second[t] = __builtin_sqrtf(power / count + epsilon);  // deviation
    __syncthreads();
    exact_write<kLayerNorm, kRows>(x, rows, columns, row0, first, second, scale, shift, out);
    return;
  }
  // LogSumExp, LogSoftmax, softmax: peak, then the shifted exponential sum.
  const float peak = exact_fold<kRows, kIdentity, kMax, kVector>(x, rows, columns, row0, nullptr, slab);
  if (t < kRows) first[t] = peak;
  __syncthreads();
  const float total = exact_fold<kRows, kShiftedExp, kSum, kVector>(x, rows, columns, row0, first, slab);
  if (kReduction == TOPOS_HIP_ROWS_LOG_SUM_EXP) {
    if (owner) out[row0 + t] = peak + ln_f32(total);
    return;
  }
  if (t < kRows) second[t] = ln_f32(total);  // normalizer
  __syncthreads();
  exact_write<kReduction, kRows>(x, rows, columns, row0, first, second, nullptr, nullptr, out);
}

// ---- fast posture: one wave per row ----

__device__ inline float wave_sum(float value) {
#pragma unroll
  for (int offset = 32; offset >= 1; offset /= 2) value += __shfl_xor(value, offset, 64);
  return value;
}

__device__ inline float wave_max(float value) {
#pragma unroll
  for (int offset = 32; offset >= 1; offset /= 2) value = max_f32(value, __shfl_xor(value, offset, 64));
  return value;
}

template <int kReduction>
__global__ __launch_bounds__(kThreads) void rows_fast_kernel(const float *__restrict__ x, int64_t rows,
                                                             int64_t columns, const float *scale,
                                                             const float *shift, float epsilon,
                                                             float *__restrict__ out) {
  const int lane = threadIdx.x % 64;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + threadIdx.x / 64;
  if (row >= rows) return;
  const float *src = x + row * columns;
  if (kReduction == TOPOS_HIP_ROWS_MAX) {
    float peak = src[0];
    for (int64_t c = lane; c < columns; c += 64) peak = max_f32(peak, src[c]);
    peak = wave_max(peak);
    if (lane == 0) out[row] = peak;
    return;
  }
  if (kReduction == TOPOS_HIP_ROWS_SUM) {
    float total = 0.0f;
    for (int64_t c = lane; c < columns; c += 64) total += src[c];
    total = wave_sum(total);
    if (lane == 0) out[row] = total;
    return;
  }
  if (kReduction == kLayerNorm) {
    float total = 0.0f;
    for (int64_t c = lane; c < columns; c += 64) total += src[c];
    const float mean = wave_sum(total) / (float)columns;
    float power = 0.0f;
    for (int64_t c = lane; c < columns; c += 64) {
      const float centred = src[c] - mean;
      power += centred * centred;
    }
    const float deviation = __builtin_sqrtf(wave_sum(power) / (float)columns + epsilon);
    for (int64_t c = lane; c < columns; c += 64)
      out[row * columns + c] = ((src[c] - mean) / deviation) * scale[c] + shift[c];
    return;
  }
  float peak = src[0];
  for (int64_t c = lane; c < columns; c += 64) peak = max_f32(peak, src[c]);
  peak = wave_max(peak);
  float total = 0.0f;
  for (int64_t c = lane; c < columns; c += 64) total += exp_f32(src[c] - peak);
  total = wave_sum(total);
  if (kReduction == TOPOS_HIP_ROWS_LOG_SUM_EXP) {
    if (lane == 0) out[row] = peak + ln_f32(total);
    return;
  }
  const float normalizer = ln_f32(total);
  for (int64_t c = lane; c < columns; c += 64) {
    float result = (src[c] - peak) - normalizer;
    if (kReduction == TOPOS_HIP_ROWS_SOFTMAX) result = exp_f32(result);
    out[row * columns + c] = result;
  }
}

// Fast posture, rows that fit in registers (at most 256 * kQ columns, a
// multiple of four): one wave per row holds the row's quads (lane l: quads
// l, l + 64, ...), so every pass after the first load runs from registers
// and the row is read once and written once.
template <int kReduction, int kQ>
__global__ __launch_bounds__(kThreads) void rows_fast_resident_kernel(const float *__restrict__ x, int64_t rows,
                                                                      int64_t columns, const float *scale,
                                                                      const float *shift, float epsilon,
                                                                      float *__restrict__ out) {
  // e^x reads its 32-entry table from LDS (a gather from global memory per
  // call would cost a vector-memory instruction each).
  __shared__ uint64_t exp_table[32];
  constexpr bool kExp = kReduction == TOPOS_HIP_ROWS_SOFTMAX || kReduction == TOPOS_HIP_ROWS_LOG_SOFTMAX ||
                        kReduction == TOPOS_HIP_ROWS_LOG_SUM_EXP;
  if (kExp) {
    if (threadIdx.x < 32) exp_table[threadIdx.x] = topos_faithful::kExpTableDevice[threadIdx.x];
    __syncthreads();
  }
  const int lane = threadIdx.x % 64;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + threadIdx.x / 64;
  if (row >= rows) return;
  const int quads = (int)(columns / 4);
  const float4 *src = reinterpret_cast<const float4 *>(x + row * columns);
  float v[kQ][4];
#pragma unroll
  for (int i = 0; i < kQ; ++i) {
    const int q = lane + 64 * i;
    const float4 w = q < quads ? src[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    v[i][0] = w.x;
    v[i][1] = w.y;
    v[i][2] = w.z;
    v[i][3] = w.w;
  }
  auto valid = [&](int i) { return lane + 64 * i < quads; };
  if (kReduction == TOPOS_HIP_ROWS_SUM || kReduction == kLayerNorm) {
    float total = 0.0f;
#pragma unroll
    for (int i = 0; i < kQ; ++i)
      if (valid(i))
#pragma unroll
        for (int j = 0; j < 4; ++j) total += v[i][j];
    total = wave_sum(total);
    if (kReduction == TOPOS_HIP_ROWS_SUM) {
      if (lane == 0) out[row] = total;
      return;
    }
    const float mean = total / (float)columns;
    float power = 0.0f;
#pragma unroll
    for (int i = 0; i < kQ; ++i)
      if (valid(i))
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float centred = v[i][j] - mean;
          power += centred * centred;
        }
    const float deviation = __builtin_sqrtf(wave_sum(power) / (float)columns + epsilon);
    float4 *dst = reinterpret_cast<float4 *>(out + row * columns);
    const float4 *sc = reinterpret_cast<const float4 *>(scale);
    const float4 *sh = reinterpret_cast<const float4 *>(shift);
#pragma unroll
    for (int i = 0; i < kQ; ++i)
      if (valid(i)) {
        const int q = lane + 64 * i;
        const float4 a = sc[q], b = sh[q];
        dst[q] = make_float4(((v[i][0] - mean) / deviation) * a.x + b.x, ((v[i][1] - mean) / deviation) * a.y + b.y,
                             ((v[i][2] - mean) / deviation) * a.z + b.z, ((v[i][3] - mean) / deviation) * a.w + b.w);
      }
    return;
  }
  // The max fold, seeded with the row's first value (NaN loses under max_f32).
  float peak = x[row * columns];
#pragma unroll
  for (int i = 0; i < kQ; ++i)
    if (valid(i))
#pragma unroll
      for (int j = 0; j < 4; ++j) peak = max_f32(peak, v[i][j]);
  peak = wave_max(peak);
  if (kReduction == TOPOS_HIP_ROWS_MAX) {
    if (lane == 0) out[row] = peak;
    return;
  }
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kQ; ++i)
    if (valid(i))
#pragma unroll
      for (int j = 0; j < 4; ++j) total += topos_faithful::exp_f32_table(v[i][j] - peak, exp_table);
  total = wave_sum(total);
  if (kReduction == TOPOS_HIP_ROWS_LOG_SUM_EXP) {
    if (lane == 0) out[row] = peak + ln_f32(total);
    return;
  }
  const float normalizer = ln_f32(total);
  float4 *dst = reinterpret_cast<float4 *>(out + row * columns);
#pragma unroll
  for (int i = 0; i < kQ; ++i)
    if (valid(i)) {
      float r[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        r[j] = (v[i][j] - peak) - normalizer;
        if (kReduction == TOPOS_HIP_ROWS_SOFTMAX) r[j] = topos_faithful::exp_f32_table(r[j], exp_table);
      }
      dst[lane + 64 * i] = make_float4(r[0], r[1], r[2], r[3]);
    }
}

// The exact row maximum with the row in one wave's registers: the ordered
// max_f32 fold (src/payload/tensor.rs:1104-1124) is the first occurrence of
// the largest non-NaN term, or the last term when every term is NaN, which
// any partition recovers: each lane keeps its first largest term and that
// term's column, and the butterfly keeps the largest, earliest (so a -0
// before a +0 of the same row wins, as in the fold).
template <int kQ>
__global__ __launch_bounds__(kThreads) void rows_max_exact_resident_kernel(const float *__restrict__ x, int64_t rows,
                                                                           int64_t columns, float *__restrict__ out) {
  const int lane = threadIdx.x % 64;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + threadIdx.x / 64;
  if (row >= rows) return;
  const int quads = (int)(columns / 4);
  const float4 *src = reinterpret_cast<const float4 *>(x + row * columns);
  float v[kQ][4];
#pragma unroll
  for (int i = 0; i < kQ; ++i) {
    const int q = lane + 64 * i;
    const float4 w = q < quads ? src[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    v[i][0] = w.x;
    v[i][1] = w.y;
    v[i][2] = w.z;
    v[i][3] = w.w;
  }
  float mv = 0.0f;
  int mi = -1;
#pragma unroll
  for (int i = 0; i < kQ; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float value = v[i][j];
      if (lane + 64 * i < quads && value == value && (mi < 0 || value > mv)) {
        mv = value;
        mi = 4 * (lane + 64 * i) + j;
      }
    }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float ov = __shfl_xor(mv, off, 64);
    const int oi = __shfl_xor(mi, off, 64);
    if (oi >= 0 && (mi < 0 || ov > mv || (!(mv > ov) && oi < mi))) {
      mv = ov;
      mi = oi;
    }
  }
  if (lane == 0) out[row] = mi < 0 ? x[row * columns + columns - 1] : mv;
}

template <int kQ>
bool try_max_exact(const float *x, int64_t rows, int64_t columns, float *out, hipStream_t stream) {
  if (columns > 256 * kQ) return false;
  rows_max_exact_resident_kernel<kQ><<<(unsigned)((rows + 3) / 4), kThreads, 0, stream>>>(x, rows, columns, out);
  return true;
}

template <int kReduction, int kQ>
bool try_resident(const float *x, int64_t rows, int64_t columns, const float *scale, const float *shift,
                  float epsilon, float *out, hipStream_t stream) {
  if (columns > 256 * kQ) return false;
  const int64_t blocks = (rows + 3) / 4;
  rows_fast_resident_kernel<kReduction, kQ><<<(unsigned)blocks, kThreads, 0, stream>>>(x, rows, columns, scale, shift,
                                                                                       epsilon, out);
  return true;
}

template <int kReduction>
void launch_one(const float *x, int64_t rows, int64_t columns, int numerics, const float *scale,
                const float *shift, float epsilon, float *out, hipStream_t stream) {
  if (numerics == TOPOS_HIP_FAST) {
    auto aligned = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const bool full = kReduction == TOPOS_HIP_ROWS_SOFTMAX || kReduction == TOPOS_HIP_ROWS_LOG_SOFTMAX ||
                      kReduction == kLayerNorm;
    if (columns % 4 == 0 && aligned(x) && (!full || aligned(out)) &&
        (kReduction != kLayerNorm || (aligned(scale) && aligned(shift)))) {
      if (try_resident<kReduction, 2>(x, rows, columns, scale, shift, epsilon, out, stream) ||
          try_resident<kReduction, 4>(x, rows, columns, scale, shift, epsilon, out, stream) ||
          try_resident<kReduction, 8>(x, rows, columns, scale, shift, epsilon, out, stream) ||
          try_resident<kReduction, 16>(x, rows, columns, scale, shift, epsilon, out, stream)) {
        check_launch("row reduction launch");
        return;
      }
    }
    const int64_t blocks = (rows + 3) / 4;
    rows_fast_kernel<kReduction><<<(unsigned)blocks, kThreads, 0, stream>>>(x, rows, columns, scale, shift, epsilon, out);
  } else {
    constexpr int kRows = 64;
    const int64_t blocks = (rows + kRows - 1) / kRows;
    const bool vector = reinterpret_cast<uintptr_t>(x) % 16 == 0 && columns % 4 == 0;
    if (vector)
      rows_exact_kernel<kReduction, kRows, true><<<(unsigned)blocks, kThreads, 0, stream>>>(x, rows, columns, scale, shift, epsilon, out);
    else
      rows_exact_kernel<kReduction, kRows, false><<<(unsigned)blocks, kThreads, 0, stream>>>(x, rows, columns, scale, shift, epsilon, out);
  }
  check_launch("row reduction launch");
}

}  // namespace

void launch_rows(int reduction, const float *x, int64_t rows, int64_t columns, int numerics,
                 float *out, hipStream_t stream) {
  if (rows <= 0 || columns <= 0) throw InvalidArgument{"row reduction needs a non-empty operand"};
  if (rows > 0x7fffffffLL * 4) throw Unsupported{"row reduction: too many rows for one launch"};
  switch (reduction) {
    case TOPOS_HIP_ROWS_SUM: launch_one<TOPOS_HIP_ROWS_SUM>(x, rows, columns, numerics, nullptr, nullptr, 0.0f, out, stream); break;
    case TOPOS_HIP_ROWS_MAX: launch_one<TOPOS_HIP_ROWS_MAX>(x, rows, columns, numerics, nullptr, nullptr, 0.0f, out, stream); break;
    case TOPOS_HIP_ROWS_LOG_SOFTMAX: launch_one<TOPOS_HIP_ROWS_LOG_SOFTMAX>(x, rows, columns, numerics, nullptr, nullptr, 0.0f, out, stream); break;
    case TOPOS_HIP_ROWS_SOFTMAX: launch_one<TOPOS_HIP_ROWS_SOFTMAX>(x, rows, columns, numerics, nullptr, nullptr, 0.0f, out, stream); break;
    case TOPOS_HIP_ROWS_LOG_SUM_EXP: launch_one<TOPOS_HIP_ROWS_LOG_SUM_EXP>(x, rows, columns, numerics, nullptr, nullptr, 0.0f, out, stream); break;
    default: throw InvalidArgument{"unknown row reduction"};
  }
}

bool launch_rows_max_exact(const float *x, int64_t rows, int64_t columns, float *out, hipStream_t stream) {
  if (rows <= 0 || columns <= 0 || columns % 4 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0 ||
      rows > 0x7fffffffLL * 4)
    return false;
  const bool served = try_max_exact<2>(x, rows, columns, out, stream) || try_max_exact<4>(x, rows, columns, out, stream) ||
                      try_max_exact<8>(x, rows, columns, out, stream) || try_max_exact<16>(x, rows, columns, out, stream);
  if (served) check_launch("row maximum launch");
  return served;
}

void launch_layer_norm(const float *x, int64_t rows, int64_t columns, const float *scale,
                       const float *shift, float epsilon, int numerics, float *out,
                       hipStream_t stream) {
  if (rows <= 0 || columns <= 0) throw InvalidArgument{"layer norm needs a non-empty operand"};
  launch_one<kLayerNorm>(x, rows, columns, numerics, scale, shift, epsilon, out, stream);
}

}  // namespace topos_hip
