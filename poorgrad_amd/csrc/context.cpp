// Process context: lazy one-time setup, sticky poison, and the device-runtime
// table (real HIP or the fake stand-in used by CPU-only tests).
//
// Mirrors the lifecycle of the reference's CUDA rung: a OnceLock'd context
// whose setup error is typed NoDevice/Failed (src/backend/cuda/kernels/context.rs:29-43,
// 217-288) and a OnceLock'd poison message that makes every later offer decline
// (src/backend/cuda/kernels/mod.rs:36-58, 94-121).
#include <cstdlib>
#include <cstring>

#include "backend.hpp"

namespace topos_hip {

namespace {

hipError_t real_malloc(void **p, size_t n) { return hipMalloc(p, n); }
hipError_t real_free(void *p) { return hipFree(p); }
hipError_t real_to_device(void *d, const void *s, size_t n) {
  return hipMemcpy(d, s, n, hipMemcpyHostToDevice);
}
hipError_t real_to_host(void *d, const void *s, size_t n) {
  return hipMemcpy(d, s, n, hipMemcpyDeviceToHost);
}
hipError_t real_sync() { return hipDeviceSynchronize(); }

hipError_t fake_malloc(void **p, size_t n) {
  *p = std::malloc(n ? n : 1);
  return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t fake_free(void *p) {
  std::free(p);
  return hipSuccess;
}
hipError_t fake_copy(void *d, const void *s, size_t n) {
  std::memcpy(d, s, n);
  return hipSuccess;
}
hipError_t fake_sync() { return hipSuccess; }

}  // namespace

Context &Context::get() {
  // Never destroyed: kernels and device memory stay valid until process exit,
  // like the reference's never-dropped OnceLock context.
  static Context *context = new Context();
  return *context;
}

bool Context::install_fake(int fail_after_calls) {
  bool installed = false;
  std::call_once(once_, [&] {
    fake_ = true;
    fake_countdown_.store(fail_after_calls);
    runtime_ = Runtime{fake_malloc, fake_free, fake_copy, fake_copy, fake_sync, false};
    device_count_ = 1;
    setup_status_ = TOPOS_HIP_OK;
    installed = true;
  });
  return installed;
}

void Context::setup() {
  runtime_ = Runtime{real_malloc, real_free, real_to_device, real_to_host, real_sync, true};
  int count = 0;
  const hipError_t status = hipGetDeviceCount(&count);
  if (status == hipErrorNoDevice || (status == hipSuccess && count == 0)) {
    setup_status_ = TOPOS_HIP_NO_DEVICE;
    reason_ = "no HIP device is visible";
    return;
  }
  if (status != hipSuccess) {
    // hipGetDeviceCount reports a missing driver or device in several ways;
    // every one of them means this machine has no usable GPU.
    setup_status_ = TOPOS_HIP_NO_DEVICE;
    reason_ = std::string("hipGetDeviceCount failed: ") + hipGetErrorString(status);
    return;
  }
  device_count_ = count;
  hipDeviceProp_t properties;
  const hipError_t probe = hipGetDeviceProperties(&properties, 0);
  if (probe != hipSuccess) {
    setup_status_ = TOPOS_HIP_SETUP_FAILED;
    reason_ = std::string("hipGetDeviceProperties failed: ") + hipGetErrorString(probe);
    return;
  }
  if (std::strncmp(properties.gcnArchName, "gfx950", 6) != 0) {
    setup_status_ = TOPOS_HIP_SETUP_FAILED;
    reason_ = std::string("device 0 is ") + properties.gcnArchName +
              "; this library carries gfx950 code objects only";
    return;
  }
  arch_major_ = properties.major;
  setup_status_ = TOPOS_HIP_OK;
}

int Context::status() {
  std::call_once(once_, [this] { setup(); });
  if (setup_status_ != TOPOS_HIP_OK) return setup_status_;
  if (poisoned_.load()) return TOPOS_HIP_POISONED;
  return TOPOS_HIP_OK;
}

void Context::poison(const std::string &message) {
  std::lock_guard<std::mutex> guard(reason_lock_);
  if (!poisoned_.exchange(true)) reason_ = message;  // the first reason sticks
}

void Context::tick(const char *what) {
  if (!fake_) return;
  const int left = fake_countdown_.fetch_sub(1);
  if (left == 0) throw RuntimeFailure{std::string("fake runtime failure injected at ") + what};
}

float *Context::workspace_for(int64_t floats, hipStream_t stream) {
  if (runtime_.launches_kernels && !workspace_used_)
    check(hipEventCreateWithFlags(&workspace_used_, hipEventDisableTiming), "hipEventCreate(workspace)");
  if (floats > workspace_floats_) {
    if (workspace_) {
      if (workspace_in_use_) check(hipEventSynchronize(workspace_used_), "hipEventSynchronize(workspace)");
      runtime_.free(workspace_);
      workspace_ = nullptr;
      workspace_floats_ = 0;
      workspace_in_use_ = false;
    }
    void *p = nullptr;
    check(runtime_.malloc(&p, (size_t)floats * sizeof(float)), "hipMalloc(workspace)");
    workspace_ = static_cast<float *>(p);
    workspace_floats_ = floats;
  }
  if (workspace_in_use_) check(hipStreamWaitEvent(stream, workspace_used_, 0), "hipStreamWaitEvent(workspace)");
  return workspace_;
}

void check(hipError_t status, const char *what) {
  if (status != hipSuccess)
    throw RuntimeFailure{std::string(what) + " failed: " + hipGetErrorString(status)};
}

void check_launch(const char *what) { check(hipGetLastError(), what); }

}  // namespace topos_hip
