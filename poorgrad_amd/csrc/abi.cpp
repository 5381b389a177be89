// The C ABI of libtopos_hip (include/topos_hip.h): manifest, status, the
// offered task face, the device face and the chain entry points.
#include <cstdio>
#include <cstring>
#include <map>
#include <vector>

#include "backend.hpp"

namespace topos_hip {
topos_hip_chain *create_chain(const topos_hip_chain_desc &d, bool load);
void launch_chain(const topos_hip_chain &chain, const float *const *inputs, float *const *outputs,
                  hipStream_t stream);
}  // namespace topos_hip

using namespace topos_hip;

namespace {

// Task-face thresholds, the cost heuristics of the Fast posture's chain
// (never correctness boundaries, src/backend/numerics.rs:7-14). Each task
// pays two PCIe copies in and one out, as the CUDA rung does
// (src/backend/cuda/kernels/mod.rs:28-34).
constexpr size_t kGemmFlopThreshold = size_t(1) << 24;
constexpr size_t kMapThreshold = size_t(1) << 17;

// Size-classed device buffers for the task face (the CUDA rung's Pool,
// src/backend/cuda/kernels/pool.rs:11-101): power-of-two classes up to
// 256 MiB, at most 1 GiB parked; larger requests are allocated exactly.
class Pool {
 public:
  void *take(size_t bytes) {
    const size_t size = rounded(bytes);
    auto it = parked_.find(size);
    if (it != parked_.end() && !it->second.empty()) {
      void *p = it->second.back();
      it->second.pop_back();
      parked_bytes_ -= size;
      return p;
    }
    Context &context = Context::get();
    context.tick("malloc");
    void *p = nullptr;
    check(context.runtime().malloc(&p, size), "hipMalloc");
    return p;
  }
  void give(void *p, size_t bytes) {
    if (!p) return;
    const size_t size = rounded(bytes);
    if (size <= kLargestClass && parked_bytes_ + size <= kParkedCap) {
      parked_[size].push_back(p);
      parked_bytes_ += size;
      return;
    }
    Context::get().runtime().free(p);
  }

 private:
  static constexpr size_t kLargestClass = size_t(256) << 20;
  static constexpr size_t kParkedCap = size_t(1) << 30;
  static size_t rounded(size_t bytes) {
    if (bytes > kLargestClass) return bytes;
    size_t size = 256;
    while (size < bytes) size <<= 1;
    return size;
  }
  std::map<size_t, std::vector<void *>> parked_;
  size_t parked_bytes_ = 0;
};

Pool &pool() {
  static Pool *p = new Pool();
  return *p;
}

// A device buffer borrowed from the pool for one task.
struct Borrowed {
  void *p = nullptr;
  size_t bytes = 0;
  explicit Borrowed(size_t n) : bytes(n) { p = pool().take(n); }
  ~Borrowed() { pool().give(p, bytes); }
  Borrowed(const Borrowed &) = delete;
  Borrowed &operator=(const Borrowed &) = delete;
};

bool fits_i32(size_t value) { return value <= 0x7fffffffu; }

// The elements a strided rows x columns view spans, 1 + (rows - 1) * row_stride
// + (columns - 1) * column_stride; false when that overflows size_t.
bool span(size_t rows, size_t columns, size_t row_stride, size_t column_stride, size_t *out) {
  size_t along_rows = 0, along_columns = 0, sum = 0;
  if (__builtin_mul_overflow(rows - 1, row_stride, &along_rows)) return false;
  if (__builtin_mul_overflow(columns - 1, column_stride, &along_columns)) return false;
  if (__builtin_add_overflow(along_rows, along_columns, &sum)) return false;
  if (__builtin_add_overflow(sum, size_t(1), out)) return false;
  return true;
}

// Enqueues the product with the posture's kernel: the matrix cores under
// Fast when their loaders cover the strides, else the exact kernel (a
// bit-identical result meets every posture, src/backend/coverage.rs:35-44).
void enqueue_gemm(const float *a, int64_t a_rs, int64_t a_cs, const float *b, int64_t b_rs,
                  int64_t b_cs, int64_t m, int64_t k, int64_t n, int numerics, float *c,
                  int64_t ldc, hipStream_t stream) {
  Context &context = Context::get();
  if (!context.runtime().launches_kernels) {
    context.tick("gemm launch");
    return;
  }
  if (numerics == TOPOS_HIP_FAST && mfma_serves(a_rs, a_cs, b_rs, b_cs, m, k, n)) {
    const int64_t floats = mfma_split_floats(m, n, k, Batch(), ldc);
    if (floats == 0) {
      if (launch_gemm_mfma(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, stream)) return;
    } else {
      bool served = false;
      context.with_workspace(floats, stream, [&](float *workspace) {
        served = launch_gemm_mfma(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, stream, Batch(), workspace, floats);
      });
      if (served) return;
    }
  }
  launch_gemm_exact(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, stream);
}

int ready_for_device_face() {
  const int status = Context::get().status();
  return status;
}

}  // namespace

extern "C" {

int topos_hip_abi_version(void) { return TOPOS_HIP_ABI_VERSION; }

int topos_hip_dispatch(void) { return TOPOS_HIP_DISPATCH_OFFERED; }

int topos_hip_compiled(void) { return 1; }

int topos_hip_coverage(int formula, int *fidelity, unsigned *precisions) {
  // One cell per formula. Gemm serves under the envelope: the member picks the
  // matrix-core kernel under Fast and the bit-identical kernel under Exact
  // from the posture it is handed, and the envelope is the weaker guarantee
  // the cell may promise. Map is bit-identical: every operation matches the
  // host libm on all 2^32 inputs. Three composed formulas are elected onto
  // device programs, each bit-identical under Exact (the composed
  // recording's bits, as src/backend/fused.rs:18-50 declares for the
  // reference's own fused kernels, whose products take the envelope under
  // Fast through the gemm seam): WindowProduct as window products that
  // gather the patch matrix (under Fast a kernel gradient with few outputs
  // runs in ranges of whole images), ReduceWindow as lanes viewed from the
  // source in one launch, BatchNormTraining as one column program.
  // BatchNormInference stays absent, as in the reference.
  switch (formula) {
    case TOPOS_HIP_FORMULA_GEMM:
      if (fidelity) *fidelity = TOPOS_HIP_ENVELOPE;
      if (precisions) *precisions = TOPOS_HIP_PRECISION_F32;
      return 1;
    case TOPOS_HIP_FORMULA_MAP:
    case TOPOS_HIP_FORMULA_WINDOW_PRODUCT:
    case TOPOS_HIP_FORMULA_REDUCE_WINDOW:
    case TOPOS_HIP_FORMULA_BATCH_NORM_TRAINING:
      if (fidelity) *fidelity = TOPOS_HIP_BIT_IDENTICAL;
      if (precisions) *precisions = TOPOS_HIP_PRECISION_F32;
      return 1;
    default:
      return 0;
  }
}

int topos_hip_status(void) { return Context::get().status(); }

const char *topos_hip_status_reason(void) { return Context::get().reason().c_str(); }

const char *topos_hip_status_string(int code) {
  switch (code) {
    case TOPOS_HIP_OK: return "ok";
    case TOPOS_HIP_DECLINED: return "declined: compute on the reference path";
    case TOPOS_HIP_NO_DEVICE: return "no HIP device is visible";
    case TOPOS_HIP_SETUP_FAILED: return "backend setup failed";
    case TOPOS_HIP_POISONED: return "backend disabled after a runtime error";
    case TOPOS_HIP_INVALID_ARGUMENT: return "invalid argument";
    case TOPOS_HIP_RUNTIME_ERROR: return "a HIP call failed; the backend is now poisoned";
    case TOPOS_HIP_UNSUPPORTED: return "not covered by the kernels";
  }
  return "unknown status code";
}

int topos_hip_fake_runtime(int fail_after_calls) {
  return Context::get().install_fake(fail_after_calls) ? TOPOS_HIP_OK : TOPOS_HIP_INVALID_ARGUMENT;
}

int64_t topos_hip_workspace_bytes(void) { return Context::get().workspace_bytes(); }

int topos_hip_gemm_f32(const float *a, size_t a_len, size_t a_row_stride, size_t a_col_stride,
                       const float *b, size_t b_len, size_t b_row_stride, size_t b_col_stride,
                       size_t m, size_t k, size_t n, int numerics, float *product) {
  // GemmTask::new's contract (src/payload/gemm.rs:57-89).
  if (!a || !b || !product || m == 0 || k == 0 || n == 0) return TOPOS_HIP_INVALID_ARGUMENT;
  if (numerics != TOPOS_HIP_EXACT && numerics != TOPOS_HIP_FAST) return TOPOS_HIP_INVALID_ARGUMENT;
  if (!fits_i32(m) || !fits_i32(n) || !fits_i32(k)) return TOPOS_HIP_DECLINED;
  size_t a_span = 0, b_span = 0;
  if (!span(m, k, a_row_stride, a_col_stride, &a_span) || !span(k, n, b_row_stride, b_col_stride, &b_span))
    return TOPOS_HIP_INVALID_ARGUMENT;  // the reference's span arithmetic overflows (gemm.rs:57-89)
  if (a_len < a_span || b_len < b_span) return TOPOS_HIP_INVALID_ARGUMENT;
  // Declines that need no device (src/backend/cuda/kernels/mod.rs:69-89).
  if (m == 1 || n == 1) return TOPOS_HIP_DECLINED;
  const double flops = 2.0 * (double)m * (double)n * (double)k;
  if (flops < (double)kGemmFlopThreshold) return TOPOS_HIP_DECLINED;
  Context &context = Context::get();
  if (context.status() != TOPOS_HIP_OK) return TOPOS_HIP_DECLINED;
  std::lock_guard<std::mutex> guard(context.task_lock());
  return guarded([&] {
    Borrowed da(a_span * sizeof(float)), db(b_span * sizeof(float)), dc(m * n * sizeof(float));
    context.tick("copy a");
    check(context.runtime().copy_to_device(da.p, a, a_span * sizeof(float)), "hipMemcpy(a)");
    context.tick("copy b");
    check(context.runtime().copy_to_device(db.p, b, b_span * sizeof(float)), "hipMemcpy(b)");
    enqueue_gemm(static_cast<const float *>(da.p), (int64_t)a_row_stride, (int64_t)a_col_stride,
                 static_cast<const float *>(db.p), (int64_t)b_row_stride, (int64_t)b_col_stride,
                 (int64_t)m, (int64_t)k, (int64_t)n, numerics, static_cast<float *>(dc.p),
                 (int64_t)n, nullptr);
    context.tick("copy product");
    check(context.runtime().copy_to_host(product, dc.p, m * n * sizeof(float)), "hipMemcpy(product)");
  });
}

int topos_hip_map_f32(int operation, const float *elements, size_t count, int numerics, float *out) {
  if (operation < TOPOS_HIP_MAP_EXP || operation > TOPOS_HIP_MAP_TANH) return TOPOS_HIP_INVALID_ARGUMENT;
  if (numerics != TOPOS_HIP_EXACT && numerics != TOPOS_HIP_FAST) return TOPOS_HIP_INVALID_ARGUMENT;
  if ((!elements || !out) && count) return TOPOS_HIP_INVALID_ARGUMENT;
  if (count < kMapThreshold || count > 0xffffffffu) return TOPOS_HIP_DECLINED;
  Context &context = Context::get();
  if (context.status() != TOPOS_HIP_OK) return TOPOS_HIP_DECLINED;
  std::lock_guard<std::mutex> guard(context.task_lock());
  return guarded([&] {
    Borrowed dx(count * sizeof(float)), dy(count * sizeof(float));
    context.tick("copy elements");
    check(context.runtime().copy_to_device(dx.p, elements, count * sizeof(float)), "hipMemcpy(elements)");
    if (context.runtime().launches_kernels)
      launch_map(operation, static_cast<const float *>(dx.p), (int64_t)count, static_cast<float *>(dy.p), nullptr);
    else
      context.tick("map launch");
    context.tick("copy mapped");
    check(context.runtime().copy_to_host(out, dy.p, count * sizeof(float)), "hipMemcpy(mapped)");
  });
}

int topos_hip_gemm_f32_device(const float *a, int64_t a_row_stride, int64_t a_col_stride,
                              const float *b, int64_t b_row_stride, int64_t b_col_stride,
                              int64_t m, int64_t k, int64_t n, int numerics, float *product,
                              int64_t ldc, void *stream) {
  if (!a || !b || !product || m <= 0 || k <= 0 || n <= 0 || ldc < n) return TOPOS_HIP_INVALID_ARGUMENT;
  if (a_row_stride < 0 || a_col_stride < 0 || b_row_stride < 0 || b_col_stride < 0)
    return TOPOS_HIP_INVALID_ARGUMENT;
  if (numerics != TOPOS_HIP_EXACT && numerics != TOPOS_HIP_FAST) return TOPOS_HIP_INVALID_ARGUMENT;
  const int status = ready_for_device_face();
  if (status != TOPOS_HIP_OK) return status;
  return guarded([&] {
    enqueue_gemm(a, a_row_stride, a_col_stride, b, b_row_stride, b_col_stride, m, k, n, numerics,
                 product, ldc, static_cast<hipStream_t>(stream));
  });
}

int topos_hip_gemm_bf16_device(const uint16_t *a, int64_t a_row_stride, int64_t a_col_stride, const uint16_t *b,
                               int64_t b_row_stride, int64_t b_col_stride, int64_t m, int64_t k, int64_t n,
                               int numerics, uint16_t *product, int64_t ldc, void *stream) {
  if (!a || !b || !product || m <= 0 || k <= 0 || n <= 0 || ldc < n) return TOPOS_HIP_INVALID_ARGUMENT;
  if (a_row_stride < 0 || a_col_stride < 0 || b_row_stride < 0 || b_col_stride < 0)
    return TOPOS_HIP_INVALID_ARGUMENT;
  if (numerics != TOPOS_HIP_EXACT && numerics != TOPOS_HIP_FAST) return TOPOS_HIP_INVALID_ARGUMENT;
  size_t a_span = 0, b_span = 0;
  if (!span((size_t)m, (size_t)k, (size_t)a_row_stride, (size_t)a_col_stride, &a_span) ||
      !span((size_t)k, (size_t)n, (size_t)b_row_stride, (size_t)b_col_stride, &b_span) ||
      a_span > ((size_t)1 << 40) || b_span > ((size_t)1 << 40))
    return TOPOS_HIP_INVALID_ARGUMENT;
  const int status = ready_for_device_face();
  if (status != TOPOS_HIP_OK) return status;
  Context &context = Context::get();
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return guarded([&] {
    if (!context.runtime().launches_kernels) {
      context.tick("bf16 gemm launch");
      return;
    }
    if (numerics == TOPOS_HIP_FAST && bf16_mfma_serves(a_row_stride, a_col_stride, b_row_stride, b_col_stride)) {
      const int64_t floats =
          bf16_fast_workspace_floats(a, a_row_stride, a_col_stride, b, b_row_stride, b_col_stride, m, k, n);
      if (floats > 0)
        context.with_workspace(floats, s, [&](float *w) {
          launch_gemm_bf16_fast(a, a_row_stride, a_col_stride, b, b_row_stride, b_col_stride, m, k, n, product, ldc,
                                s, w);
        });
      else
        launch_gemm_bf16_fast(a, a_row_stride, a_col_stride, b, b_row_stride, b_col_stride, m, k, n, product, ldc, s,
                              nullptr);
      return;
    }
    // The exact contract step by step: widen both operands, the bit-identical
    // f32 product, one rounding per output. Each operand is packed densely
    // (its unit-stride axis kept innermost), so the workspace is bounded by
    // the product's own sizes, whatever the views' spans.
    const int64_t a_floats = (m * k + 63) / 64 * 64, b_floats = (k * n + 63) / 64 * 64;
    context.with_workspace(a_floats + b_floats + m * n, s, [&](float *w) {
      auto widen = [&](const uint16_t *src, int64_t rows, int64_t cols, int64_t rs, int64_t cs, float *dst,
                       int64_t *packed_rs, int64_t *packed_cs) {
        if (rs == 1 && cs != 1) {  // column-contiguous: packed as [cols][rows]
          launch_widen_bf16(src, cols, rows, cs, rs, dst, s);
          *packed_rs = 1, *packed_cs = rows;
        } else {
          launch_widen_bf16(src, rows, cols, rs, cs, dst, s);
          *packed_rs = cols, *packed_cs = 1;
        }
      };
      int64_t ars, acs, brs, bcs;
      widen(a, m, k, a_row_stride, a_col_stride, w, &ars, &acs);
      widen(b, k, n, b_row_stride, b_col_stride, w + a_floats, &brs, &bcs);
      float *wc = w + a_floats + b_floats;
      launch_gemm_exact(w, ars, acs, w + a_floats, brs, bcs, m, k, n, wc, n, s);
      launch_narrow_bf16(wc, m, n, product, ldc, s);
    });
  });
}

int topos_hip_map_f32_device(int operation, const float *x, int64_t count, float *y, void *stream) {
  if (operation < TOPOS_HIP_MAP_EXP || operation > TOPOS_HIP_MAP_TANH || count < 0) return TOPOS_HIP_INVALID_ARGUMENT;
  if (count > 0 && (!x || !y)) return TOPOS_HIP_INVALID_ARGUMENT;
  const int status = ready_for_device_face();
  if (status != TOPOS_HIP_OK) return status;
  return guarded([&] { launch_map(operation, x, count, y, static_cast<hipStream_t>(stream)); });
}

int topos_hip_rows_f32_device(int reduction, const float *x, int64_t rows, int64_t columns,
                              int numerics, float *out, void *stream) {
  if (!x || !out || rows <= 0 || columns <= 0) return TOPOS_HIP_INVALID_ARGUMENT;
  if (numerics != TOPOS_HIP_EXACT && numerics != TOPOS_HIP_FAST) return TOPOS_HIP_INVALID_ARGUMENT;
  const int status = ready_for_device_face();
  if (status != TOPOS_HIP_OK) return status;
  if (reduction < TOPOS_HIP_ROWS_SUM || reduction > TOPOS_HIP_ROWS_LOG_SUM_EXP) return TOPOS_HIP_INVALID_ARGUMENT;
  return guarded([&] {
    // The row maximum is exact in both postures: rows that fit one wave's
    // registers take the one-read kernel.
    if (reduction == TOPOS_HIP_ROWS_MAX &&
        launch_rows_max_exact(x, rows, columns, out, static_cast<hipStream_t>(stream)))
      return;
    if (numerics == TOPOS_HIP_EXACT)
      launch_rows_program(reduction, x, rows, columns, out, static_cast<hipStream_t>(stream));
    else
      launch_rows(reduction, x, rows, columns, numerics, out, static_cast<hipStream_t>(stream));
  });
}

int topos_hip_layer_norm_f32_device(const float *x, int64_t rows, int64_t columns,
                                    const float *scale, const float *shift, float epsilon,
                                    int numerics, float *out, void *stream) {
  if (!x || !scale || !shift || !out || rows <= 0 || columns <= 0) return TOPOS_HIP_INVALID_ARGUMENT;
  if (numerics != TOPOS_HIP_EXACT && numerics != TOPOS_HIP_FAST) return TOPOS_HIP_INVALID_ARGUMENT;
  const int status = ready_for_device_face();
  if (status != TOPOS_HIP_OK) return status;
  return guarded([&] {
    if (numerics == TOPOS_HIP_EXACT)
      launch_layer_norm_program(x, rows, columns, scale, shift, epsilon, out, static_cast<hipStream_t>(stream));
    else
      launch_layer_norm(x, rows, columns, scale, shift, epsilon, numerics, out, static_cast<hipStream_t>(stream));
  });
}

int topos_hip_chain_create(const topos_hip_chain_desc *desc, topos_hip_chain **chain) {
  if (!desc || !chain) return TOPOS_HIP_INVALID_ARGUMENT;
  *chain = nullptr;
  const int status = ready_for_device_face();
  if (status != TOPOS_HIP_OK) return status;
  Context &context = Context::get();
  return guarded([&] { *chain = create_chain(*desc, context.runtime().launches_kernels); });
}

int topos_hip_chain_launch(const topos_hip_chain *chain, const float *const *inputs,
                           float *const *outputs, void *stream) {
  if (!chain || !outputs) return TOPOS_HIP_INVALID_ARGUMENT;
  const int status = ready_for_device_face();
  if (status != TOPOS_HIP_OK) return status;
  return guarded([&] { launch_chain(*chain, inputs, outputs, static_cast<hipStream_t>(stream)); });
}


}  // extern "C"
