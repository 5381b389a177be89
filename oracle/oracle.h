/* CPU oracle: a single-threaded C restatement of the topos interpreter's f32
 * arithmetic for the execution path the HIP backend replaces.
 *
 * TEST INFRASTRUCTURE ONLY. The parity tests, the smoke check and the CPU
 * baseline leg of the benchmark call this code as the checker; no product code
 * links or calls it.
 *
 * Every function names the reference file:line it restates. Arithmetic is IEEE
 * single precision with one rounding per operation: the file is compiled with
 * -ffp-contract=off and without fast-math, transcendentals call the host libm
 * exactly as Rust's f32 methods do, and every accumulation is sequential in
 * ascending index, seeded from the first term.
 */
#ifndef TOPOS_ORACLE_H
#define TOPOS_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- seeded synthetic data: src/neural/init.rs:50-102 ---- */
uint64_t oracle_splitmix64(uint64_t *state);
double oracle_unit(uint64_t *state);
double oracle_standard_normal(uint64_t *state);
/* init::uniform(seed, scale) drawing `count` elements; the f64 stream rounded
 * once per element to f32. `state` carries the generator between draws. */
void oracle_uniform_f32(uint64_t *state, double scale, size_t count, float *out);
void oracle_normal_f32(uint64_t *state, double deviation, size_t count, float *out);
void oracle_uniform_f64(uint64_t *state, double scale, size_t count, double *out);
void oracle_normal_f64(uint64_t *state, double deviation, size_t count, double *out);

/* ---- GEMM: src/payload/gemm.rs:140-211 ----
 * product[i, j] = a[i,0]*b[0,j], then += a[i,s]*b[s,j] for s = 1..k-1, with a
 * separately rounded multiply and add. Operands read through (row, column)
 * element strides; the product is contiguous row-major [m, n]. */
void oracle_gemm_f32(const float *a, int64_t a_row_stride, int64_t a_col_stride, const float *b,
                     int64_t b_row_stride, int64_t b_col_stride, int64_t m, int64_t n, int64_t k,
                     float *product);
/* Rows [row_begin, row_end) only: independent output rows, bit-identical to the
 * whole product (used to time a bounded sample). */
void oracle_gemm_rows_f32(const float *a, int64_t a_row_stride, int64_t a_col_stride,
                          const float *b, int64_t b_row_stride, int64_t b_col_stride, int64_t m,
                          int64_t n, int64_t k, int64_t row_begin, int64_t row_end, float *product);

/* ---- scalar semantics: src/payload/elementary.rs:116-143 ---- */
enum oracle_unary { ORACLE_NEG = 0, ORACLE_EXP = 1, ORACLE_LN = 2, ORACLE_SQRT = 3, ORACLE_TANH = 4 };
enum oracle_binary {
  ORACLE_ADD = 0,
  ORACLE_SUB = 1,
  ORACLE_MUL = 2,
  ORACLE_DIV = 3,
  ORACLE_POWF = 4,
  ORACLE_MAX = 5,
  ORACLE_STEP = 6
};
float oracle_unary_f32(int op, float x);
float oracle_binary_f32(int op, float x, float y);
/* Elementwise over contiguous buffers (src/payload/tensor.rs:365-510). */
void oracle_map_f32(int op, const float *x, size_t count, float *y);
void oracle_zip_f32(int op, const float *x, const float *y, size_t count, float *out);

/* ---- reductions: src/payload/tensor.rs:1055-1124 ----
 * The operand is viewed as [outer, extent, inner] in logical order. */
float oracle_sum_f32(const float *x, size_t count);
void oracle_sum_along_f32(const float *x, int64_t outer, int64_t extent, int64_t inner, float *out);
void oracle_max_along_f32(const float *x, int64_t outer, int64_t extent, int64_t inner, float *out);

/* ---- fused rules over the last axis of a contiguous [rows, columns] ----
 * LogSoftmax forward (src/function/log_softmax.rs:51-60): peak = max_along,
 * shifted = x - peak, out = shifted - ln(sum_along(exp(shifted))). */
void oracle_log_softmax_rows_f32(const float *x, int64_t rows, int64_t columns, float *out);
/* softmax = log_softmax(x).exp() (src/graph/composite.rs:43-45). */
void oracle_softmax_rows_f32(const float *x, int64_t rows, int64_t columns, float *out);
/* LogSumExp forward (src/function/log_sum_exp.rs:53-61): peak + ln(sum(exp(x - peak))). */
void oracle_log_sum_exp_rows_f32(const float *x, int64_t rows, int64_t columns, float *out);
/* LayerNorm forward (src/neural/layer_norm.rs:100-132) over rows: mean by
 * sum_along / counted, centred, biased variance, sqrt(var + eps), divide,
 * then * scale[j] + shift[j]. */
void oracle_layer_norm_rows_f32(const float *x, int64_t rows, int64_t columns, const float *scale,
                                const float *shift, float epsilon, float *out);

/* ---- the bf16 payload (src/payload/bf16.rs) ----
 * Bf16::from_f32 (:38-46): round to nearest, ties to even, by adding the
 * rounding bias to the bits; a NaN keeps its top half with bit 0x40 set. */
uint16_t oracle_bf16_from_f32(float x);
void oracle_bf16_round(const float *x, size_t count, uint16_t *out);
/* Bf16::to_f32 (:50-53): the bits shifted into the top half of a single. */
void oracle_bf16_widen(const uint16_t *x, size_t count, float *out);

#ifdef __cplusplus
}
#endif
#endif
