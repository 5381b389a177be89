// Internal interfaces of libtopos_hip: the process context (setup, poison,
// the device-runtime table), and the kernel launchers each .hip file provides.
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/topos_hip.h"

// A compiled chain kernel (topos_hip_chain_create).
struct topos_hip_chain {
  std::string source;
  hipModule_t module = nullptr;
  hipFunction_t function = nullptr;
  int n_inputs = 0;
  int n_outputs = 0;
  int64_t volume = 0;
  bool quads = false;             // innermost extent % 4 == 0: quad path legal
  std::vector<bool> vector_in;    // input may use 16-byte loads (given alignment)
  std::vector<int64_t> in_offset;
};

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
};

// Throws RuntimeFailure on a HIP error, naming the call.
void check(hipError_t status, const char *what);
// Checks the launch status of the kernel just enqueued.
void check_launch(const char *what);

// ---- kernel launchers (device face); throw on failure ----

// gemm_exact.hip: bit-identical to src/payload/gemm.rs:140-211.
void launch_gemm_exact(const float *a, int64_t a_rs, int64_t a_cs, const float *b, int64_t b_rs,
                       int64_t b_cs, int64_t m, int64_t k, int64_t n, float *c, int64_t ldc,
                       hipStream_t stream);
// gemm_mfma.hip: fp32 MFMA product within the stated envelope. Returns false
// when the stride pattern is outside its loaders (caller falls back).
bool launch_gemm_mfma(const float *a, int64_t a_rs, int64_t a_cs, const float *b, int64_t b_rs,
                      int64_t b_cs, int64_t m, int64_t k, int64_t n, float *c, int64_t ldc,
                      hipStream_t stream);

// map.hip: host-libm-faithful unary maps over contiguous buffers.
void launch_map(int operation, const float *x, int64_t count, float *y, hipStream_t stream);

// rows.hip: row reductions over contiguous [rows, columns].
void launch_rows(int reduction, const float *x, int64_t rows, int64_t columns, int numerics,
                 float *out, hipStream_t stream);
void launch_layer_norm(const float *x, int64_t rows, int64_t columns, const float *scale,
                       const float *shift, float epsilon, int numerics, float *out,
                       hipStream_t stream);

}  // namespace topos_hip
