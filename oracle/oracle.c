/* CPU oracle restating the topos interpreter's f32 arithmetic.
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Built with -ffp-contract=off. */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- src/neural/init.rs:50-102 ---- */

/* splitmix64 (init.rs:50-56): advance by the golden-ratio increment, then two
 * xor-shift-multiply rounds and a final xor-shift. */
uint64_t oracle_splitmix64(uint64_t *state) {
  *state += 0x9E3779B97F4A7C15ull;
  uint64_t mixed = *state;
  mixed = (mixed ^ (mixed >> 30)) * 0xBF58476D1CE4E5B9ull;
  mixed = (mixed ^ (mixed >> 27)) * 0x94D049BB133111EBull;
  return mixed ^ (mixed >> 31);
}

/* unit() (init.rs:58-60): the top 53 bits over 2^53, in [0, 1). */
double oracle_unit(uint64_t *state) {
  return (double)(oracle_splitmix64(state) >> 11) / (double)(1ull << 53);
}

/* standard_normal() (init.rs:62-66): Box-Muller cosine branch; the radius
 * draw comes first, then the angle draw. */
double oracle_standard_normal(uint64_t *state) {
  const double radius = sqrt(-2.0 * log(1.0 - oracle_unit(state)));
  const double angle = 6.283185307179586 * oracle_unit(state); /* f64::consts::TAU */
  return radius * cos(angle);
}

/* init::uniform (init.rs:88-91): (unit * 2 - 1) * scale, rounded once. */
void oracle_uniform_f32(uint64_t *state, double scale, size_t count, float *out) {
  for (size_t i = 0; i < count; ++i) out[i] = (float)((oracle_unit(state) * 2.0 - 1.0) * scale);
}

void oracle_uniform_f64(uint64_t *state, double scale, size_t count, double *out) {
  for (size_t i = 0; i < count; ++i) out[i] = (oracle_unit(state) * 2.0 - 1.0) * scale;
}

/* init::normal (init.rs:93-102): standard_normal * deviation, rounded once. */
void oracle_normal_f32(uint64_t *state, double deviation, size_t count, float *out) {
  for (size_t i = 0; i < count; ++i) out[i] = (float)(oracle_standard_normal(state) * deviation);
}

void oracle_normal_f64(uint64_t *state, double deviation, size_t count, double *out) {
  for (size_t i = 0; i < count; ++i) out[i] = oracle_standard_normal(state) * deviation;
}

/* ---- src/payload/gemm.rs:140-211 ---- */

/* Every output element keeps its own accumulator, seeded with its first
 * term and advanced in ascending k, exactly as seed_row/accumulate_row do;
 * the loops only visit the elements in a cache-friendlier order (column
 * blocks whose slab of b stays in cache across rows, four rows per pass over
 * a k step), which changes no element's sequence of roundings. */
void oracle_gemm_rows_f32(const float *a, int64_t a_row_stride, int64_t a_col_stride,
                          const float *b, int64_t b_row_stride, int64_t b_col_stride, int64_t m,
                          int64_t n, int64_t k, int64_t row_begin, int64_t row_end, float *product) {
  (void)m;
  enum { kColumns = 512, kRows = 4 };
  for (int64_t c0 = 0; c0 < n; c0 += kColumns) {
    const int64_t c1 = c0 + kColumns < n ? c0 + kColumns : n;
    for (int64_t r0 = row_begin; r0 < row_end; r0 += kRows) {
      const int64_t rows = r0 + kRows <= row_end ? kRows : row_end - r0;
      /* seed_row (gemm.rs:166-183): the first term, never a zero. */
      for (int64_t r = 0; r < rows; ++r) {
        const float a_first = a[(r0 + r) * a_row_stride];
        float *out = product + (r0 + r) * n;
        for (int64_t column = c0; column < c1; ++column) out[column] = a_first * b[column * b_col_stride];
      }
      /* accumulate_row (gemm.rs:193-211): ascending inner steps. */
      for (int64_t step = 1; step < k; ++step) {
        const float *b_row = b + step * b_row_stride;
        for (int64_t r = 0; r < rows; ++r) {
          const float a_value = a[(r0 + r) * a_row_stride + step * a_col_stride];
          float *out = product + (r0 + r) * n;
          if (b_col_stride == 1) {
            for (int64_t column = c0; column < c1; ++column) {
              const float term = a_value * b_row[column];
              out[column] = out[column] + term;
            }
          } else {
            for (int64_t column = c0; column < c1; ++column) {
              const float term = a_value * b_row[column * b_col_stride];
              out[column] = out[column] + term;
            }
          }
        }
      }
    }
  }
}

void oracle_gemm_f32(const float *a, int64_t a_row_stride, int64_t a_col_stride, const float *b,
                     int64_t b_row_stride, int64_t b_col_stride, int64_t m, int64_t n, int64_t k,
                     float *product) {
  oracle_gemm_rows_f32(a, a_row_stride, a_col_stride, b, b_row_stride, b_col_stride, m, n, k, 0, m,
                       product);
}

/* ---- src/payload/elementary.rs:116-143 ---- */

/* f32::max as compiled for x86-64 (llvm.maxnum): NaN loses, a +-0 tie
 * answers the first operand. Pinned against llvm.maxnum.f32 built by clang on
 * runtime operands (tests/native/maxnum_probe.c, test_oracle_rows_pinned.py). */
static float max_f32(float x, float y) {
  if (x != x) return y;
  if (y != y) return x;
  return y > x ? y : x;
}

float oracle_unary_f32(int op, float x) {
  switch (op) {
    case ORACLE_NEG: return -x;
    case ORACLE_EXP: return expf(x);
    case ORACLE_LN: return logf(x);
    case ORACLE_SQRT: return sqrtf(x);
    case ORACLE_TANH: return tanhf(x);
  }
  abort();
}

float oracle_binary_f32(int op, float x, float y) {
  switch (op) {
    case ORACLE_ADD: return x + y;
    case ORACLE_SUB: return x - y;
    case ORACLE_MUL: return x * y;
    case ORACLE_DIV: return x / y;
    case ORACLE_POWF: return powf(x, y);
    case ORACLE_MAX: return max_f32(x, y);
    case ORACLE_STEP: return x >= y ? 1.0f : 0.0f;
  }
  abort();
}

void oracle_map_f32(int op, const float *x, size_t count, float *y) {
  for (size_t i = 0; i < count; ++i) y[i] = oracle_unary_f32(op, x[i]);
}

void oracle_zip_f32(int op, const float *x, const float *y, size_t count, float *out) {
  for (size_t i = 0; i < count; ++i) out[i] = oracle_binary_f32(op, x[i], y[i]);
}

/* ---- src/payload/tensor.rs:1055-1124 ---- */

/* sum (tensor.rs:1055-1063): left fold seeded by the first element. */
float oracle_sum_f32(const float *x, size_t count) {
  float total = x[0];
  for (size_t i = 1; i < count; ++i) total = total + x[i];
  return total;
}

/* sum_along (tensor.rs:1073-1093): per (outer, inner), ascending over the
 * reduced extent, seeded by step 0. */
void oracle_sum_along_f32(const float *x, int64_t outer, int64_t extent, int64_t inner, float *out) {
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t i = 0; i < inner; ++i) {
      float total = x[(o * extent) * inner + i];
      for (int64_t s = 1; s < extent; ++s) total = total + x[(o * extent + s) * inner + i];
      out[o * inner + i] = total;
    }
}

/* max_along (tensor.rs:1104-1124): the same walk folding f32::max. */
void oracle_max_along_f32(const float *x, int64_t outer, int64_t extent, int64_t inner, float *out) {
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t i = 0; i < inner; ++i) {
      float largest = x[(o * extent) * inner + i];
      for (int64_t s = 1; s < extent; ++s) largest = max_f32(largest, x[(o * extent + s) * inner + i]);
      out[o * inner + i] = largest;
    }
}

/* ---- fused rules ---- */

/* src/function/log_softmax.rs:51-60 over axis 1 of [rows, columns]. */
void oracle_log_softmax_rows_f32(const float *x, int64_t rows, int64_t columns, float *out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *row = x + r * columns;
    float *dst = out + r * columns;
    float peak = row[0];
    for (int64_t c = 1; c < columns; ++c) peak = max_f32(peak, row[c]);
    /* shifted = x - peak; normalizer = ln(sum_along(exp(shifted))) */
    float total = expf(row[0] - peak);
    for (int64_t c = 1; c < columns; ++c) total = total + expf(row[c] - peak);
    const float normalizer = logf(total);
    for (int64_t c = 0; c < columns; ++c) dst[c] = (row[c] - peak) - normalizer;
  }
}

void oracle_softmax_rows_f32(const float *x, int64_t rows, int64_t columns, float *out) {
  oracle_log_softmax_rows_f32(x, rows, columns, out);
  for (int64_t i = 0; i < rows * columns; ++i) out[i] = expf(out[i]);
}

/* src/function/log_sum_exp.rs:53-61 over axis 1. */
void oracle_log_sum_exp_rows_f32(const float *x, int64_t rows, int64_t columns, float *out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *row = x + r * columns;
    float peak = row[0];
    for (int64_t c = 1; c < columns; ++c) peak = max_f32(peak, row[c]);
    float total = expf(row[0] - peak);
    for (int64_t c = 1; c < columns; ++c) total = total + expf(row[c] - peak);
    out[r] = peak + logf(total);
  }
}

/* src/neural/layer_norm.rs:100-132 over axis 1, with mean_along =
 * sum_along / counted (src/graph/composite.rs:54-59). */
void oracle_layer_norm_rows_f32(const float *x, int64_t rows, int64_t columns, const float *scale,
                                const float *shift, float epsilon, float *out) {
  const float count = (float)columns;
  for (int64_t r = 0; r < rows; ++r) {
    const float *row = x + r * columns;
    float *dst = out + r * columns;
    float total = row[0];
    for (int64_t c = 1; c < columns; ++c) total = total + row[c];
    const float mean = total / count;
    float first = row[0] - mean;
    float power = first * first;
    for (int64_t c = 1; c < columns; ++c) {
      const float centred = row[c] - mean;
      power = power + centred * centred;
    }
    const float variance = power / count;
    const float deviation = sqrtf(variance + epsilon);
    for (int64_t c = 0; c < columns; ++c) {
      const float normalized = (row[c] - mean) / deviation;
      dst[c] = normalized * scale[c] + shift[c];
    }
  }
}

/* ---- src/payload/bf16.rs:38-53 ---- */

uint16_t oracle_bf16_from_f32(float x) {
  uint32_t bits;
  memcpy(&bits, &x, sizeof bits);
  if (x != x) return (uint16_t)((bits >> 16) | 0x0040u);
  const uint32_t rounding_bias = 0x7FFFu + ((bits >> 16) & 1u);
  return (uint16_t)((bits + rounding_bias) >> 16);
}

void oracle_bf16_round(const float *x, size_t count, uint16_t *out) {
  for (size_t i = 0; i < count; ++i) out[i] = oracle_bf16_from_f32(x[i]);
}

void oracle_bf16_widen(const uint16_t *x, size_t count, float *out) {
  for (size_t i = 0; i < count; ++i) {
    const uint32_t bits = (uint32_t)x[i] << 16;
    memcpy(&out[i], &bits, sizeof bits);
  }
}
