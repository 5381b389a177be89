// Indexing, ordered scatter, the last passes of the exact whole-tensor sum,
// and the device-resident optimizer steps.
//
//   gather  (src/payload/tensor.rs:1554-1576): row copy by selection index.
//   scatter (src/payload/tensor.rs:1582-1618): zero-seeded scatter-add that
//           accumulates each target row's sources in source order. The
//           row-sorted source list (CSR) is built when the selection is
//           bound, so one lane owns one output element and adds its sources
//           in ascending order: deterministic, no atomics.
//   one-hot (Storage::Selection read through Tensor::get, tensor.rs:220-240).
//   sum     (tensor.rs:1055-1063): the ordered fold of the nonzero terms the
//           generated passes compacted. Dropping the +-0 terms of a sequential
//           sum changes nothing once a nonzero term has been added (x + +-0 = x,
//           and an exact cancellation gives +0, which +-0 terms keep), and
//           +-0 + x = x; so the fold over the nonzero terms, seeded with the
//           first of them, is the interpreter's sum. With no nonzero term the
//           sum is -0 exactly when every term is -0.
//   SGD / AdamW (src/neural/optimizer.rs:40-51, src/neural/adam.rs:62-171):
//           the optimizer's operation sequence per element.
#pragma clang fp contract(off)
#include "backend.hpp"

namespace topos_hip {
namespace {

__global__ __launch_bounds__(256) void gather_kernel(const float *__restrict__ table, int64_t row_stride,
                                                     int64_t column_stride, const int32_t *__restrict__ indices,
                                                     int64_t rows, int64_t row_size, float *__restrict__ out) {
  const int64_t total = rows * row_size;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / row_size, j = e % row_size;
    out[e] = table[(int64_t)indices[r] * row_stride + j * column_stride];
  }
}

__global__ __launch_bounds__(256) void scatter_kernel(const float *__restrict__ gradient, int64_t row_stride,
                                                      int64_t column_stride, const int32_t *__restrict__ row_start,
                                                      const int32_t *__restrict__ sources, int64_t rows,
                                                      int64_t row_size, float *__restrict__ out) {
  const int64_t total = rows * row_size;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = e / row_size, j = e % row_size;
    float acc = 0.0f;  // the zero-seeded accumulator
    for (int32_t p = row_start[t]; p < row_start[t + 1]; ++p)
      acc = acc + gradient[(int64_t)sources[p] * row_stride + j * column_stride];
    out[e] = acc;
  }
}

__global__ __launch_bounds__(256) void one_hot_kernel(const int32_t *__restrict__ indices, int64_t rows,
                                                      int64_t vocab, float one, float *__restrict__ out) {
  const int64_t total = rows * vocab;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / vocab, c = e % vocab;
    out[e] = indices[r] == (int32_t)c ? one : 0.0f;
  }
}

// Exclusive scan of the per-chunk nonzero counts, one workgroup: each lane
// owns a contiguous run of chunks.
__global__ __launch_bounds__(1024) void scan_kernel(const int32_t *__restrict__ counts, int64_t chunks,
                                                    int64_t *__restrict__ offsets) {
  __shared__ int64_t totals[1024];
  const int t = threadIdx.x;
  const int64_t per = (chunks + 1023) / 1024;
  const int64_t begin = t * per, end = begin + per < chunks ? begin + per : chunks;
  int64_t mine = 0;
#pragma unroll 8
  for (int64_t c = begin; c < end; ++c) mine += counts[c];
  totals[t] = mine;
  __syncthreads();
  if (t == 0) {
    int64_t running = 0;
    for (int i = 0; i < 1024; ++i) {
      const int64_t v = totals[i];
      totals[i] = running;
      running += v;
    }
    offsets[chunks] = running;  // the total number of nonzero terms
  }
  __syncthreads();
  int64_t running = totals[t];
#pragma unroll 8
  for (int64_t c = begin; c < end; ++c) {
    offsets[c] = running;
    running += counts[c];
  }
}

// The ordered fold of the compacted terms (one lane).
__global__ void ordered_sum_kernel(const float *__restrict__ compacted, const int64_t *__restrict__ offsets,
                                   int64_t chunks, const int32_t *__restrict__ positive_zero,
                                   float *__restrict__ out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  const int64_t n = offsets[chunks];
  if (n == 0) {
    int any_positive = 0;
    for (int64_t c = 0; c < chunks; ++c) any_positive |= positive_zero[c];
    out[0] = any_positive ? 0.0f : -0.0f;
    return;
  }
  float acc = compacted[0];
  int64_t i = 1;
  for (; i + 4 <= n; i += 4) {
    const float a = compacted[i], b = compacted[i + 1], c = compacted[i + 2], d = compacted[i + 3];
    acc = acc + a;
    acc = acc + b;
    acc = acc + c;
    acc = acc + d;
  }
  for (; i < n; ++i) acc = acc + compacted[i];
  out[0] = acc;
}

__global__ __launch_bounds__(256) void sgd_kernel(float *__restrict__ parameter, const float *__restrict__ gradient,
                                                  int64_t count, float rate) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
    parameter[i] = parameter[i] - gradient[i] * rate;
}

__global__ __launch_bounds__(256) void adamw_kernel(float *__restrict__ parameter, const float *__restrict__ gradient,
                                                    float *__restrict__ first, float *__restrict__ second,
                                                    int64_t count, float beta1, float beta2, float first_share,
                                                    float second_share, float first_correction,
                                                    float second_correction, float epsilon, float rate,
                                                    float decay, int decayed) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
    const float g = gradient[i];
    const float m = first[i] * beta1 + g * first_share;
    const float squared = g * g;
    const float v = second[i] * beta2 + squared * second_share;
    first[i] = m;
    second[i] = v;
    const float corrected_first = m / first_correction;
    const float corrected_second = v / second_correction;
    const float direction = corrected_first / (__builtin_sqrtf(corrected_second) + epsilon);
    const float current = parameter[i];
    const float stepped = current - direction * rate;
    parameter[i] = decayed ? stepped - (current * decay) * rate : stepped;
  }
}

unsigned blocks_for(int64_t count) {
  int64_t b = (count + 255) / 256;
  if (b < 1) b = 1;
  if (b > 256 * 32) b = 256 * 32;
  return (unsigned)b;
}

}  // namespace

void launch_gather(const float *table, int64_t row_stride, int64_t column_stride, const int32_t *indices,
                   int64_t rows, int64_t row_size, float *out, hipStream_t stream) {
  gather_kernel<<<blocks_for(rows * row_size), 256, 0, stream>>>(table, row_stride, column_stride, indices, rows,
                                                                 row_size, out);
  check_launch("gather_kernel launch");
}

void launch_scatter(const float *gradient, int64_t row_stride, int64_t column_stride, const int32_t *row_start,
                    const int32_t *sources, int64_t rows, int64_t row_size, float *out, hipStream_t stream) {
  scatter_kernel<<<blocks_for(rows * row_size), 256, 0, stream>>>(gradient, row_stride, column_stride, row_start,
                                                                  sources, rows, row_size, out);
  check_launch("scatter_kernel launch");
}

void launch_one_hot(const int32_t *indices, int64_t rows, int64_t vocab, float one, float *out, hipStream_t stream) {
  one_hot_kernel<<<blocks_for(rows * vocab), 256, 0, stream>>>(indices, rows, vocab, one, out);
  check_launch("one_hot_kernel launch");
}

void launch_scan(const int32_t *counts, int64_t chunks, int64_t *offsets, hipStream_t stream) {
  scan_kernel<<<1, 1024, 0, stream>>>(counts, chunks, offsets);
  check_launch("scan_kernel launch");
}

void launch_ordered_fold(const float *compacted, const int64_t *offsets, int64_t chunks, const int32_t *positive_zero,
                         float *out, hipStream_t stream) {
  ordered_sum_kernel<<<1, 64, 0, stream>>>(compacted, offsets, chunks, positive_zero, out);
  check_launch("ordered_sum_kernel launch");
}

void launch_sgd(float *parameter, const float *gradient, int64_t count, float rate, hipStream_t stream) {
  if (count <= 0) return;
  sgd_kernel<<<blocks_for(count), 256, 0, stream>>>(parameter, gradient, count, rate);
  check_launch("sgd_kernel launch");
}

void launch_adamw(float *parameter, const float *gradient, float *first, float *second, int64_t count, float beta1,
                  float beta2, float first_share, float second_share, float first_correction,
                  float second_correction, float epsilon, float rate, float decay, int decayed,
                  hipStream_t stream) {
  if (count <= 0) return;
  adamw_kernel<<<blocks_for(count), 256, 0, stream>>>(parameter, gradient, first, second, count, beta1, beta2,
                                                      first_share, second_share, first_correction,
                                                      second_correction, epsilon, rate, decay, decayed);
  check_launch("adamw_kernel launch");
}

}  // namespace topos_hip
