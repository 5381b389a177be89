// Internal interfaces of libtopos_hip: the process context (setup, poison,
// the device-runtime table), and the kernel launchers each .hip file provides.
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/topos_hip.h"

namespace topos_hip {

// The device calls the library makes outside kernel launches, as a table so a
// fake runtime can stand in on machines without a GPU (the Api::fake pattern
// of src/backend/cuda/kernels/context.rs:101-162).
struct Runtime {
  hipError_t (*malloc)(void **, size_t);
  hipError_t (*free)(void *);
  hipError_t (*copy_to_device)(void *, const void *, size_t);
  hipError_t (*copy_to_host)(void *, const void *, size_t);
  hipError_t (*synchronize)();
  bool launches_kernels;  // false in the fake runtime
};

// Thrown inside the library when a HIP call fails; the ABI layer catches it,
// poisons, and answers TOPOS_HIP_RUNTIME_ERROR or TOPOS_HIP_DECLINED.
struct RuntimeFailure {
  std::string message;
};

// Thrown when the request breaks its contract; never poisons.
struct InvalidArgument {
  std::string message;
};

// Thrown by device-face launchers for shapes or strides their kernels do not
// cover.
struct Unsupported {
  std::string message;
};

// Throws RuntimeFailure on a HIP error, naming the call.
void check(hipError_t status, const char *what);

class Context {
 public:
  // The process-wide context, set up on first use (OnceLock semantics).
  static Context &get();

  int status();  // TOPOS_HIP_OK / NO_DEVICE / SETUP_FAILED / POISONED
  const std::string &reason() const { return reason_; }
  void poison(const std::string &message);
  bool poisoned() const { return poisoned_.load(); }

  const Runtime &runtime() const { return runtime_; }
  bool install_fake(int fail_after_calls);
  // Counts one device call for the fake runtime's failure countdown; throws
  // RuntimeFailure when the countdown reaches the failing call.
  void tick(const char *what);

  // Runs `enqueue(workspace)` with a grow-only device buffer of at least
  // `floats` floats for one device-face split product on `stream`. The
  // buffer's users are serialised: the lock is held from the buffer's
  // choice to the launch, each use is ordered on the GPU after the previous
  // one (on any stream) by an event, and a regrow waits for the last use
  // before freeing the old buffer.
  template <class Enqueue>
  void with_workspace(int64_t floats, hipStream_t stream, Enqueue enqueue) {
    std::lock_guard<std::mutex> guard(workspace_lock_);
    float *buffer = workspace_for(floats, stream);
    enqueue(buffer);
    if (runtime_.launches_kernels) check(hipEventRecord(workspace_used_, stream), "hipEventRecord(workspace)");
    workspace_in_use_ = runtime_.launches_kernels;
  }

  int64_t workspace_bytes() {
    std::lock_guard<std::mutex> guard(workspace_lock_);
    return workspace_floats_ * (int64_t)sizeof(float);
  }

  int device_count() const { return device_count_; }
  int architecture_major() const { return arch_major_; }
  std::mutex &task_lock() { return task_lock_; }

 private:
  Context() = default;
  void setup();

  std::once_flag once_;
  std::mutex reason_lock_;
  int setup_status_ = TOPOS_HIP_SETUP_FAILED;
  std::string reason_;
  std::atomic<bool> poisoned_{false};
  Runtime runtime_{};
  bool fake_ = false;
  std::atomic<int> fake_countdown_{-1};
  int device_count_ = 0;
  int arch_major_ = 0;
  std::mutex task_lock_;
  float *workspace_for(int64_t floats, hipStream_t stream);
  std::mutex workspace_lock_;
  float *workspace_ = nullptr;
  int64_t workspace_floats_ = 0;
  hipEvent_t workspace_used_ = nullptr;
  bool workspace_in_use_ = false;
};

// Runs `body`, mapping the library's exceptions to status codes; a runtime
// failure poisons the library for good.
template <class Body>
int guarded(Body body) {
  try {
    body();
    return TOPOS_HIP_OK;
  } catch (const InvalidArgument &) {
    return TOPOS_HIP_INVALID_ARGUMENT;
  } catch (const Unsupported &) {
    return TOPOS_HIP_UNSUPPORTED;
  } catch (const RuntimeFailure &e) {
    Context::get().poison(e.message);
    return TOPOS_HIP_RUNTIME_ERROR;
  } catch (const std::bad_alloc &) {
    Context::get().poison("host allocation failed");
    return TOPOS_HIP_RUNTIME_ERROR;
  }
}

// The message of the last InvalidArgument/Unsupported a program call raised
// on this thread (for diagnostics; status codes stay the contract).
std::string &last_refusal();

// Checks the launch status of the kernel just enqueued.
void check_launch(const char *what);

// ---- kernel launchers (device face); throw on failure ----

// A batch of equally shaped products: product `i` reads a + i * a_bs and
// b + i * b_bs and writes c + i * c_bs (the batch odometer of
// src/payload/tensor.rs:950-1006 flattened to one axis).
// Leading (batch) axes of a product. Batch y sits at
// (y / inner) * x_stride + (y % inner) * x_inner for x in a, b, c: one
// strided batch axis (inner = 1), or two merged ones (attention heads viewed
// as one axis of batch x heads).
struct Batch {
  int64_t count = 1;
  int64_t a_stride = 0, b_stride = 0, c_stride = 0;
  int64_t inner = 1;
  int64_t a_inner = 0, b_inner = 0, c_inner = 0;
};

// A per-column vector added to a product as it is written: c = p + bias[j]
// (or bias[j] + p when `bias_first`), the interpreter's separate addition
// (one f32 rounding) fused into the store (linear layers' bias).
struct Epilogue {
  const float *bias = nullptr;
  int64_t bias_stride = 0;
  bool bias_first = false;
};

// gemm_exact.hip: bit-identical to src/payload/gemm.rs:140-211.
void launch_gemm_exact(const float *a, int64_t a_rs, int64_t a_cs, const float *b, int64_t b_rs,
                       int64_t b_cs, int64_t m, int64_t k, int64_t n, float *c, int64_t ldc,
                       hipStream_t stream, const Batch &batch = Batch());

// Division of a 32-bit index below 2^31 by a fixed divisor d >= 1 as a
// multiply and a shift: with l = ceil(log2 d) and magic = ceil(2^(32+l) / d),
// floor(i * magic / 2^(32+l)) = floor(i / d), since the magic's excess over
// 2^(32+l) / d adds less than i / 2^(32+l) < 2^-(l+1) <= 1/(2d) to a quotient
// whose fraction is at most (d - 1) / d. (i * magic < 2^31 * 2^33 fits 64
// bits.)
struct Divisor {
  uint64_t magic = 1ull << 32;
  uint32_t shift = 32;
  static Divisor of(uint32_t d) {
    Divisor v;
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    v.shift = 32 + l;  // l <= 31 for d <= 2^31
    v.magic = ((1ull << v.shift) - 1) / d + 1;
    return v;
  }
  __host__ __device__ uint32_t divide(uint32_t i) const { return (uint32_t)(((uint64_t)i * magic) >> shift); }
};

// The im2col matrix of a convolution, never materialised: row r = (image,
// out_y, out_x), column q = (channel, kernel_y, kernel_x) of the padded,
// strided windows of a rank-4 [batch, channels, height, width] source read
// through any strides; +0 where a window leaves the source (the padding).
// The patch matrix of src/payload/tensor.rs:1475-1544.
struct WindowShape {
  int64_t offset = 0;
  int64_t s_batch = 0, s_channel = 0, s_height = 0, s_width = 0;
  int32_t channels = 0, height = 0, width = 0;
  int32_t kernel_height = 0, kernel_width = 0, out_height = 0, out_width = 0, stride = 1, padding = 0;
  // Set by launch_window_product from the extents above.
  Divisor by_out_width, by_out_height, by_kernel_width, by_kernel_height;
};
// WindowProduct (src/payload/tensorial.rs:112-122, elected by
// src/engine/pattern/window.rs:58-150): patches . b ([m, k] . [k, n], m the
// patch rows) or, transposed, patches^T . b ([m, k] with m the patch columns
// and k the patch rows: the kernel gradient), bit-identical to
// gemm::multiply over the materialised patches. With `splits` > 1 (the
// transposed form only, window_splits' choice, and a workspace of splits * m
// * n floats) the patch rows are cut at image boundaries into that many
// ranges, each range's chain is exact, and the partials are added in range
// order: deterministic, within the Fast envelope, not bit-identical.
void launch_window_product(const float *source, const WindowShape &w, bool transposed, const float *b, int64_t b_rs,
                           int64_t b_cs, int64_t m, int64_t k, int64_t n, float *c, int64_t ldc,
                           hipStream_t stream, float *workspace = nullptr, int splits = 1);
// The ranges a Fast kernel gradient (patches^T . b, m patch columns, n
// filters, k patch rows over `images` images) is cut into: 1 when its
// outputs fill the chip or its chains are short, else the largest divisor of
// `images` up to 16 that leaves each range at least 512 rows.
int window_splits(int64_t m, int64_t n, int64_t k, int64_t images);
// gemm_mfma.hip: c[i][j] = ((p_0 + p_1) + p_2) + ... over `splits`
// contiguous [m][n] partials (c's rows ldc apart), m * n % 4 == 0 or n % 4 ==
// 0, m * n < 2^33.
void launch_split_reduce(const float *partials, int splits, int64_t m, int64_t n, float *c, int64_t ldc,
                         hipStream_t stream);
// gemm_mfma.hip: fp32 MFMA product within the stated envelope. Returns false
// when the stride pattern is outside its loaders (caller falls back).
// With a workspace of at least mfma_splits(m, n, k, count) * count * m * n
// floats, a product with too few output tiles to fill the chip is split
// along k into that many partial products, reduced in a fixed order
// (deterministic; envelope fidelity like the unsplit kernel).
int mfma_splits(int64_t m, int64_t n, int64_t k, int64_t batches);
// The workspace floats launch_gemm_mfma uses for this product (output
// leading dimension ldc): the split partials, splits * count * m * n, or 0
// when the product runs unsplit.
int64_t mfma_split_floats(int64_t m, int64_t n, int64_t k, const Batch &batch, int64_t ldc);
// Whether launch_gemm_mfma takes operands with these strides (else the
// caller's exact fallback runs). Its products are never -0: every
// accumulator starts at +0, and a sum of +0 with any zero is +0.
bool mfma_serves(int64_t a_rs, int64_t a_cs, int64_t b_rs, int64_t b_cs, int64_t m, int64_t k, int64_t n);
bool launch_gemm_mfma(const float *a, int64_t a_rs, int64_t a_cs, const float *b, int64_t b_rs,
                      int64_t b_cs, int64_t m, int64_t k, int64_t n, float *c, int64_t ldc,
                      hipStream_t stream, const Batch &batch = Batch(), float *workspace = nullptr,
                      int64_t workspace_floats = 0, const Epilogue &epilogue = Epilogue());

// backward.cpp: appends Run::backward's reverse scan from the scalar
// `target` to a forward node table, and maps each node of `wrt` to the node
// holding the target's gradient with respect to it (flagged readable).
void append_engine_backward(std::vector<topos_hip_node> &nodes, std::vector<topos_hip_leaf> &leaves, int64_t target,
                            const std::vector<int64_t> &wrt, std::map<int64_t, int64_t> &gradient_of);

// gemm_bf16.hip: bf16 products (operands and product as bf16 bit patterns).
bool bf16_mfma_serves(int64_t a_rs, int64_t a_cs, int64_t b_rs, int64_t b_cs);
// The fast product's workspace, in floats (256-byte aligned): operands the
// matrix-core kernel cannot read in place (not k-contiguous, or rows not
// 4-byte aligned) packed into k-contiguous rows, and, for products with few
// tiles, the f32 sums of each k range (added in range order, then rounded
// once: the envelope, then the same single rounding).
int64_t bf16_fast_workspace_floats(const uint16_t *a, int64_t a_rs, int64_t a_cs, const uint16_t *b, int64_t b_rs,
                                   int64_t b_cs, int64_t m, int64_t k, int64_t n);
void launch_gemm_bf16_fast(const uint16_t *a, int64_t a_rs, int64_t a_cs, const uint16_t *b, int64_t b_rs,
                           int64_t b_cs, int64_t m, int64_t k, int64_t n, uint16_t *c, int64_t ldc,
                           hipStream_t stream, float *workspace);
// Widens an [outer, inner] bf16 view into a dense f32 [outer][inner] buffer.
void launch_widen_bf16(const uint16_t *in, int64_t outer, int64_t inner, int64_t outer_stride, int64_t inner_stride,
                       float *out, hipStream_t stream);
void launch_narrow_bf16(const float *in, int64_t m, int64_t n, uint16_t *out, int64_t ldc, hipStream_t stream);

// window.hip: Fold (src/payload/tensor.rs:1392-1462). The operand is read
// through its layout: output element (outer, position, inner) sums, from +0
// in ascending k, source[outer + window * window_stride + k * element_stride
// + inner] over the windows covering the position. The output is contiguous
// [outer..., extent, inner...].
struct FoldGeometry {
  int outer_rank = 0, inner_rank = 0;
  int64_t outer_shape[TOPOS_HIP_MAX_RANK] = {}, outer_strides[TOPOS_HIP_MAX_RANK] = {};
  int64_t inner_shape[TOPOS_HIP_MAX_RANK] = {}, inner_strides[TOPOS_HIP_MAX_RANK] = {};
  int64_t window_stride = 0, element_stride = 0;
  int64_t count = 1, size = 1, step = 1, dilation = 1, extent = 1;
  int64_t inner_volume = 1, total = 0;
};
void launch_fold(const float *source, const FoldGeometry &geometry, float *out, hipStream_t stream);

// index.hip
void launch_gather(const float *table, int64_t row_stride, int64_t column_stride, const int32_t *indices,
                   int64_t rows, int64_t row_size, float *out, hipStream_t stream);
void launch_scatter(const float *gradient, int64_t row_stride, int64_t column_stride, const int32_t *row_start,
                    const int32_t *sources, int64_t rows, int64_t row_size, float *out, hipStream_t stream);
void launch_one_hot(const int32_t *indices, int64_t rows, int64_t vocab, float one, float *out, hipStream_t stream);
// Folds a whole-tensor sum's gathered nonzero terms in element order (chunk
// c's counts[c] terms at slots + c * chunk_size) into out[0].
void launch_slot_fold(const float *slots, const int32_t *counts, const int32_t *positive_zero, int64_t chunks,
                      int64_t chunk_size, float *out, hipStream_t stream);
void launch_sgd(float *parameter, const float *gradient, int64_t count, float rate, hipStream_t stream);
void launch_adamw(float *parameter, const float *gradient, float *first, float *second, int64_t count, float beta1,
                  float beta2, float first_share, float second_share, float first_correction,
                  float second_correction, float epsilon, float rate, float decay, int decayed,
                  hipStream_t stream);

// Up to kAdamTensors parameters of one AdamW step, passed by value as the
// kernel argument (about 2 KB, within the argument limit).
constexpr int kAdamTensors = 48;
struct AdamTable {
  float *parameter[kAdamTensors];
  const float *gradient[kAdamTensors];
  float *first[kAdamTensors];
  float *second[kAdamTensors];
  int64_t start[kAdamTensors + 1];
  int64_t quad_start[kAdamTensors + 1];  // filled by launch_adamw_multi
  int32_t decayed[kAdamTensors];
  int32_t count;
};
void launch_adamw_multi(const AdamTable &table, float beta1, float beta2, float first_share, float second_share,
                        float first_correction, float second_correction, float epsilon, float rate, float decay,
                        hipStream_t stream);

// map.hip: host-libm-faithful unary maps over contiguous buffers.
void launch_map(int operation, const float *x, int64_t count, float *y, hipStream_t stream);

// rows.hip: row reductions over contiguous [rows, columns].
void launch_rows(int reduction, const float *x, int64_t rows, int64_t columns, int numerics,
                 float *out, hipStream_t stream);
void launch_layer_norm(const float *x, int64_t rows, int64_t columns, const float *scale,
                       const float *shift, float epsilon, int numerics, float *out,
                       hipStream_t stream);

// rows_device.cpp: the exact posture of the two above as generated row
// programs (cached per shape).
// The exact row maximum over rows of at most 4096 columns (a multiple of
// four, 16-byte aligned) held in registers; false when the shape is not
// served (the caller then runs the row program).
bool launch_rows_max_exact(const float *x, int64_t rows, int64_t columns, float *out, hipStream_t stream);
void launch_rows_program(int reduction, const float *x, int64_t rows, int64_t columns, float *out,
                         hipStream_t stream);
void launch_layer_norm_program(const float *x, int64_t rows, int64_t columns, const float *scale,
                               const float *shift, float epsilon, float *out, hipStream_t stream);

}  // namespace topos_hip
