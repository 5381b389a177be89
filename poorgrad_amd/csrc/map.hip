// Whole-buffer transcendental maps (MapOperation, src/payload/elementary.rs:13-22),
// bit-identical to the host libm under both postures: exp/ln/tanh through the
// restated glibc algorithms of faithful_math.h, sqrt through the correctly
// rounded IEEE square root (f32::sqrt is correctly rounded,
// src/payload/elementary.rs:52-56). Grid-stride, 16-byte loads and stores.
#pragma clang fp contract(off)
#include "backend.hpp"
#include "faithful_math.h"

namespace topos_hip {
namespace {

template <int kOp>
__device__ inline float apply(float x) {
  if (kOp == TOPOS_HIP_MAP_EXP) return topos_faithful::exp_f32(x);
  if (kOp == TOPOS_HIP_MAP_LN) return topos_faithful::ln_f32(x);
  if (kOp == TOPOS_HIP_MAP_SQRT) return __builtin_sqrtf(x);
  return topos_faithful::tanh_f32(x);
}

template <int kOp>
__global__ __launch_bounds__(256) void map_kernel(const float *__restrict__ x, int64_t count,
                                                  float *__restrict__ y, bool vector) {
  const int64_t lanes = (int64_t)gridDim.x * blockDim.x;
  const int64_t first = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (vector) {
    const int64_t quads = count / 4;
    for (int64_t q = first; q < quads; q += lanes) {
      const float4 v = reinterpret_cast<const float4 *>(x)[q];
      reinterpret_cast<float4 *>(y)[q] =
          make_float4(apply<kOp>(v.x), apply<kOp>(v.y), apply<kOp>(v.z), apply<kOp>(v.w));
    }
    for (int64_t i = quads * 4 + first; i < count; i += lanes) y[i] = apply<kOp>(x[i]);
  } else {
    for (int64_t i = first; i < count; i += lanes) y[i] = apply<kOp>(x[i]);
  }
}

}  // namespace

void launch_map(int operation, const float *x, int64_t count, float *y, hipStream_t stream) {
  if (count <= 0) return;
  const bool vector =
      reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0;
  int64_t blocks = (count / 4 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 256 * 16) blocks = 256 * 16;  // 16 workgroups per CU, then grid-stride
  switch (operation) {
    case TOPOS_HIP_MAP_EXP: map_kernel<TOPOS_HIP_MAP_EXP><<<(unsigned)blocks, 256, 0, stream>>>(x, count, y, vector); break;
    case TOPOS_HIP_MAP_LN: map_kernel<TOPOS_HIP_MAP_LN><<<(unsigned)blocks, 256, 0, stream>>>(x, count, y, vector); break;
    case TOPOS_HIP_MAP_SQRT: map_kernel<TOPOS_HIP_MAP_SQRT><<<(unsigned)blocks, 256, 0, stream>>>(x, count, y, vector); break;
    case TOPOS_HIP_MAP_TANH: map_kernel<TOPOS_HIP_MAP_TANH><<<(unsigned)blocks, 256, 0, stream>>>(x, count, y, vector); break;
    default: throw InvalidArgument{"unknown map operation"};
  }
  check_launch("map_kernel launch");
}

}  // namespace topos_hip
