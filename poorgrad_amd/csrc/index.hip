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
//           generated pass gathered per chunk. Dropping the +-0 terms of a sequential
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

// The ordered fold of a whole-tensor sum's nonzero terms, gathered per chunk:
// chunk c's count[c] terms sit, in element order, at slots[c * chunk_size].
// One workgroup walks the chunks in passes of 256 x 16 (each lane reads the
// counts of 16 consecutive chunks; the next pass's counts are loaded while
// this one is copied). A block prefix lists the pass's nonempty chunks in
// order with each one's place among the pass's terms; their terms are copied
// into an LDS stage in element order (a lane per chunk when every chunk
// holds few terms, else chunk by chunk with all lanes), and lane 0 folds the
// stage whenever it fills. With no nonzero term the sum is -0 exactly when
// every term is -0.
constexpr int kFoldThreads = 256;
constexpr int kFoldPer = 16;
constexpr int kFoldPass = kFoldThreads * kFoldPer;
constexpr int kFoldStage = 8192;

__global__ __launch_bounds__(kFoldThreads) void slot_fold_kernel(const float *__restrict__ slots,
                                                                 const int32_t *__restrict__ counts,
                                                                 const int32_t *__restrict__ positive_zero,
                                                                 int64_t chunks, int64_t chunk_size,
                                                                 float *__restrict__ out) {
  __shared__ __attribute__((aligned(16))) float stage[kFoldStage];
  __shared__ int wave_terms[kFoldThreads / 64], wave_entries[kFoldThreads / 64], wave_most[kFoldThreads / 64];
  __shared__ int entry_chunk[kFoldPass], entry_count[kFoldPass], entry_place[kFoldPass];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  float acc = 0.0f;   // lane 0's running fold
  bool have = false;  // lane 0: a term is folded
  int any_plus = 0;
  int fill = 0;       // staged terms (the same in every lane)
  auto flush = [&]() {
    __syncthreads();
    if (t == 0) {
      int i = 0;
      if (!have && fill > 0) {
        acc = stage[0];
        have = true;
        i = 1;
      }
      for (; i < fill && (i & 3) != 0; ++i) acc = acc + stage[i];
      // Eight 16-byte LDS reads in flight ahead of each 32 additions.
      for (; i + 32 <= fill; i += 32) {
        float4 q[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) q[u] = *reinterpret_cast<const float4 *>(&stage[i + 4 * u]);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          acc = acc + q[u].x;
          acc = acc + q[u].y;
          acc = acc + q[u].z;
          acc = acc + q[u].w;
        }
      }
      for (; i < fill; ++i) acc = acc + stage[i];
    }
    __syncthreads();
    fill = 0;
  };
  int next[kFoldPer];
  auto load = [&](int64_t first) {
    const int64_t mine = first + (int64_t)t * kFoldPer;
    if (mine + kFoldPer <= chunks) {
#pragma unroll
      for (int q = 0; q < kFoldPer; q += 4) {
        const int4 c4 = *reinterpret_cast<const int4 *>(counts + mine + q);
        const int4 p4 = *reinterpret_cast<const int4 *>(positive_zero + mine + q);
        next[q] = c4.x;
        next[q + 1] = c4.y;
        next[q + 2] = c4.z;
        next[q + 3] = c4.w;
        any_plus |= p4.x | p4.y | p4.z | p4.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < kFoldPer; ++q) {
        next[q] = mine + q < chunks ? counts[mine + q] : 0;
        any_plus |= mine + q < chunks ? positive_zero[mine + q] : 0;
      }
    }
  };
  load(0);
  for (int64_t first = 0; first < chunks; first += kFoldPass) {
    int cnt[kFoldPer];
    int terms = 0, entries = 0, most = 0;
#pragma unroll
    for (int q = 0; q < kFoldPer; ++q) {
      cnt[q] = next[q];
      terms += cnt[q];
      entries += cnt[q] > 0 ? 1 : 0;
      most = max(most, cnt[q]);
    }
    if (first + kFoldPass < chunks) load(first + kFoldPass);
    // Block prefixes of this lane's terms and nonempty chunks.
    int terms_in = terms, entries_in = entries;
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(terms_in, off, 64), z = __shfl_up(entries_in, off, 64);
      if (lane >= off) {
        terms_in += y;
        entries_in += z;
      }
      most = max(most, __shfl_xor(most, off, 64));
    }
    if (lane == 63) {
      wave_terms[wave] = terms_in;
      wave_entries[wave] = entries_in;
    }
    if (lane == 0) wave_most[wave] = most;
    __syncthreads();
    int place = terms_in - terms, slot = entries_in - entries, total = 0, listed = 0;
    for (int w = 0; w < kFoldThreads / 64; ++w) {
      if (w < wave) {
        place += wave_terms[w];
        slot += wave_entries[w];
      }
      total += wave_terms[w];
      listed += wave_entries[w];
      most = max(most, wave_most[w]);
    }
#pragma unroll
    for (int q = 0; q < kFoldPer; ++q)
      if (cnt[q] > 0) {
        entry_chunk[slot] = t * kFoldPer + q;
        entry_count[slot] = cnt[q];
        entry_place[slot] = place;
        ++slot;
        place += cnt[q];
      }
    __syncthreads();
    if (total > 0) {
      if (fill + total > kFoldStage) flush();
      if (total <= kFoldStage && most <= 64) {
        // A lane per nonempty chunk (few terms each).
        for (int e = t; e < listed; e += kFoldThreads) {
          const float *src = slots + (first + entry_chunk[e]) * chunk_size;
          const int n = entry_count[e], at = fill + entry_place[e];
          for (int j = 0; j < n; ++j) stage[at + j] = src[j];
        }
        fill += total;  // the next flush's barrier orders these stores before lane 0 reads them
      } else {
        // Chunk by chunk, all lanes on consecutive terms.
        for (int e = 0; e < listed; ++e) {
          const float *src = slots + (first + entry_chunk[e]) * chunk_size;
          const int n = entry_count[e];
          for (int j0 = 0; j0 < n;) {
            if (fill == kFoldStage) flush();
            const int piece = min(n - j0, kFoldStage - fill);
            for (int j = t; j < piece; j += kFoldThreads) stage[fill + j] = src[j0 + j];
            fill += piece;
            j0 += piece;
          }
        }
      }
    }
    __syncthreads();  // the entry lists and wave totals are rewritten next pass
  }
  flush();
  any_plus = __syncthreads_or(any_plus);
  if (t == 0) out[0] = have ? acc : (any_plus ? 0.0f : -0.0f);
}

__global__ __launch_bounds__(256) void sgd_kernel(float *__restrict__ parameter, const float *__restrict__ gradient,
                                                  int64_t count, float rate) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
    parameter[i] = parameter[i] - gradient[i] * rate;
}

// One element of AdamW::step (src/neural/adam.rs:62-171), in the optimizer's
// operation order: the new moments m, v and parameter p from the gradient g,
// the old moments m0, v0 and the current parameter.
__device__ __forceinline__ void adamw_value(float g, float m0, float v0, float current, float beta1, float beta2,
                                            float first_share, float second_share, float first_correction,
                                            float second_correction, float epsilon, float rate, float decay,
                                            int decayed, float &m, float &v, float &p) {
  m = m0 * beta1 + g * first_share;
  const float squared = g * g;
  v = v0 * beta2 + squared * second_share;
  const float corrected_first = m / first_correction;
  const float corrected_second = v / second_correction;
  const float direction = corrected_first / (__builtin_sqrtf(corrected_second) + epsilon);
  const float stepped = current - direction * rate;
  p = decayed ? stepped - (current * decay) * rate : stepped;
}

// The same element through the buffers.
__device__ __forceinline__ void adamw_element(float *__restrict__ parameter, const float *__restrict__ gradient,
                                              float *__restrict__ first, float *__restrict__ second, int64_t i,
                                              float beta1, float beta2, float first_share, float second_share,
                                              float first_correction, float second_correction, float epsilon,
                                              float rate, float decay, int decayed) {
  float m, v, p;
  adamw_value(gradient[i], first[i], second[i], parameter[i], beta1, beta2, first_share, second_share,
              first_correction, second_correction, epsilon, rate, decay, decayed, m, v, p);
  first[i] = m;
  second[i] = v;
  parameter[i] = p;
}

__global__ __launch_bounds__(256) void adamw_kernel(float *__restrict__ parameter, const float *__restrict__ gradient,
                                                    float *__restrict__ first, float *__restrict__ second,
                                                    int64_t count, float beta1, float beta2, float first_share,
                                                    float second_share, float first_correction,
                                                    float second_correction, float epsilon, float rate,
                                                    float decay, int decayed) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
    adamw_element(parameter, gradient, first, second, i, beta1, beta2, first_share, second_share, first_correction,
                  second_correction, epsilon, rate, decay, decayed);
}

// Many parameters in one launch: the table's tensors laid end to end in
// quads (tensor j owns quads [quad_start[j], quad_start[j + 1]), its last quad
// possibly short), each lane finding its tensor by binary search over the quad
// starts. A whole quad whose four buffers are 16-byte aligned moves in 16-byte
// loads and stores (the gradient's with the nontemporal hint: it is read once),
// any other quad element by element; both apply adamw_value per element, so
// the bits are the single-parameter kernel's. The table travels as the
// kernel's argument, so the launch needs no device memory of its own.
__global__ __launch_bounds__(256) void adamw_multi_kernel(AdamTable table, float beta1, float beta2,
                                                          float first_share, float second_share,
                                                          float first_correction, float second_correction,
                                                          float epsilon, float rate, float decay) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  const int64_t total = table.quad_start[table.count];
  for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < total; q += (int64_t)gridDim.x * blockDim.x) {
    int lo = 0, hi = table.count - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) / 2;
      if (table.quad_start[mid] <= q) lo = mid;
      else hi = mid - 1;
    }
    const int64_t first = (q - table.quad_start[lo]) * 4;
    const int64_t n = table.start[lo + 1] - table.start[lo];
    float *parameter = table.parameter[lo];
    const float *gradient = table.gradient[lo];
    float *m1 = table.first[lo];
    float *m2 = table.second[lo];
    const int decayed = table.decayed[lo];
    const bool aligned = ((reinterpret_cast<uintptr_t>(parameter + first) | reinterpret_cast<uintptr_t>(gradient + first) |
                           reinterpret_cast<uintptr_t>(m1 + first) | reinterpret_cast<uintptr_t>(m2 + first)) & 15) == 0;
    if (first + 4 <= n && aligned) {
      const f4v g = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(gradient + first));
      const f4v a = *reinterpret_cast<const f4v *>(m1 + first);
      const f4v b = *reinterpret_cast<const f4v *>(m2 + first);
      const f4v c = *reinterpret_cast<const f4v *>(parameter + first);
      f4v m, v, p;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float me, ve, pe;
        adamw_value(g[e], a[e], b[e], c[e], beta1, beta2, first_share, second_share, first_correction,
                    second_correction, epsilon, rate, decay, decayed, me, ve, pe);
        m[e] = me;
        v[e] = ve;
        p[e] = pe;
      }
      *reinterpret_cast<f4v *>(m1 + first) = m;
      *reinterpret_cast<f4v *>(m2 + first) = v;
      *reinterpret_cast<f4v *>(parameter + first) = p;
    } else {
      for (int64_t i = first; i < first + 4 && i < n; ++i)
        adamw_element(parameter, gradient, m1, m2, i, beta1, beta2, first_share, second_share, first_correction,
                      second_correction, epsilon, rate, decay, decayed);
    }
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

void launch_slot_fold(const float *slots, const int32_t *counts, const int32_t *positive_zero, int64_t chunks,
                      int64_t chunk_size, float *out, hipStream_t stream) {
  slot_fold_kernel<<<1, kFoldThreads, 0, stream>>>(slots, counts, positive_zero, chunks, chunk_size, out);
  check_launch("slot_fold_kernel launch");
}

void launch_sgd(float *parameter, const float *gradient, int64_t count, float rate, hipStream_t stream) {
  if (count <= 0) return;
  sgd_kernel<<<blocks_for(count), 256, 0, stream>>>(parameter, gradient, count, rate);
  check_launch("sgd_kernel launch");
}

void launch_adamw_multi(const AdamTable &table, float beta1, float beta2, float first_share, float second_share,
                        float first_correction, float second_correction, float epsilon, float rate, float decay,
                        hipStream_t stream) {
  if (table.count <= 0 || table.start[table.count] <= 0) return;
  AdamTable quads = table;
  quads.quad_start[0] = 0;
  for (int j = 0; j < table.count; ++j)
    quads.quad_start[j + 1] = quads.quad_start[j] + (table.start[j + 1] - table.start[j] + 3) / 4;
  int64_t blocks = (quads.quad_start[table.count] + 255) / 256;
  if (blocks > 256 * 64) blocks = 256 * 64;
  adamw_multi_kernel<<<(unsigned)blocks, 256, 0, stream>>>(quads, beta1, beta2, first_share, second_share,
                                                           first_correction, second_correction, epsilon, rate, decay);
  check_launch("adamw_multi_kernel launch");
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
