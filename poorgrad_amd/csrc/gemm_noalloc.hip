// The device-face product for callers that cannot allocate (code under HIP
// graph capture, serving loops, harnesses that forbid hipMalloc):
// topos_hip_gemm_f32_device_noalloc. It launches the same kernels as
// topos_hip_gemm_f32_device; the only difference is where the split-k
// partials of a Fast product live. Instead of the library's grow-only
// workspace (a hipMalloc on first use and on growth) they go to `scratch`, a
// fixed device array that the code object carries, so no call allocates.
//
// Each GPU holds its own copy of `scratch` from the moment this code object
// is loaded on it until the process ends. Every call on one GPU shares that
// copy: calls that overlap on one GPU (two streams, two threads) race on it.
// The split-k partials are written in full before the reduction reads them,
// so nothing needs clearing between calls.
#include "backend.hpp"

// 64 MiB: the partials of every split product whose splits x m x n fit in
// 16 Mi floats (for example 16 splits of a 1024 x 1024 product).
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace topos_hip {
namespace {

constexpr int kMaxDevices = 64;
std::mutex scratch_lock;
float *scratch_addresses[kMaxDevices] = {};

// The device address of `scratch` on the current device. In host code the
// array's name is only a host-side stand-in, so its address is looked up once
// per device (with that device current) and kept; every use goes through it.
float *scratch_on_current_device() {
  int device = 0;
  check(hipGetDevice(&device), "hipGetDevice");
  if (device < 0 || device >= kMaxDevices) throw Unsupported{"no-allocation product: device ordinal beyond 63"};
  std::lock_guard<std::mutex> guard(scratch_lock);
  if (!scratch_addresses[device]) {
    void *address = nullptr;
    check(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    scratch_addresses[device] = static_cast<float *>(address);
  }
  return scratch_addresses[device];
}

// Enqueues the product as topos_hip_gemm_f32_device does, with any split-k
// partials in `scratch`. A product whose chosen split needs more than the
// array holds splits into as many ranges as fit (or none), so the array is
// never exceeded; its result then stays within the Fast envelope but is not
// the allocating entry's bit pattern.
void enqueue_gemm_noalloc(const float *a, int64_t a_rs, int64_t a_cs, const float *b, int64_t b_rs, int64_t b_cs,
                          int64_t m, int64_t k, int64_t n, int numerics, float *c, int64_t ldc, hipStream_t stream) {
  Context &context = Context::get();
  if (!context.runtime().launches_kernels) {
    context.tick("gemm launch");
    return;
  }
  if (numerics == TOPOS_HIP_FAST && mfma_serves(a_rs, a_cs, b_rs, b_cs, m, k, n)) {
    // The same split choice as the allocating entry point, so both give the
    // same bits whenever its partials fit the scratch.
    const int64_t floats = std::min<int64_t>(mfma_split_floats(m, n, k, Batch(), ldc),
                                             (int64_t)(kScratchBytes / sizeof(float)));
    float *workspace = floats ? scratch_on_current_device() : nullptr;
    if (launch_gemm_mfma(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, stream, Batch(), workspace, floats)) return;
  }
  launch_gemm_exact(a, a_rs, a_cs, b, b_rs, b_cs, m, k, n, c, ldc, stream);
}

}  // namespace
}  // namespace topos_hip

using namespace topos_hip;

extern "C" int topos_hip_gemm_f32_device_noalloc(const float *a, int64_t a_row_stride, int64_t a_col_stride,
                                                 const float *b, int64_t b_row_stride, int64_t b_col_stride,
                                                 int64_t m, int64_t k, int64_t n, int numerics, float *product,
                                                 int64_t ldc, void *stream) {
  last_refusal().clear();
  if (!a || !b || !product || m <= 0 || k <= 0 || n <= 0 || ldc < n) return TOPOS_HIP_INVALID_ARGUMENT;
  if (a_row_stride < 0 || a_col_stride < 0 || b_row_stride < 0 || b_col_stride < 0)
    return TOPOS_HIP_INVALID_ARGUMENT;
  if (numerics != TOPOS_HIP_EXACT && numerics != TOPOS_HIP_FAST) return TOPOS_HIP_INVALID_ARGUMENT;
  const int status = Context::get().status();
  if (status != TOPOS_HIP_OK) return status;
  return guarded([&] {
    try {
      enqueue_gemm_noalloc(a, a_row_stride, a_col_stride, b, b_row_stride, b_col_stride, m, k, n, numerics,
                           product, ldc, static_cast<hipStream_t>(stream));
    } catch (const InvalidArgument &e) {
      last_refusal() = e.message;
      throw;
    }
  });
}
