// Fold: the adjoint of the sliding-window view (Unfold), summing each
// position's window elements back onto the folded axis.
//
// Tensor::fold (src/payload/tensor.rs:1392-1462) walks every output position
// and adds, from +0 and in ascending window-element order k, the element k of
// each window w with w * step + k * dilation == position. One lane owns one
// output element and performs exactly that walk, so the result is the
// interpreter's bit for bit and needs no atomics: a position's terms are read
// through the operand's strides (any view: permuted, broadcast, narrowed).
#pragma clang fp contract(off)
#include "backend.hpp"

namespace topos_hip {
namespace {

__global__ __launch_bounds__(256) void fold_kernel(const float *__restrict__ source, FoldGeometry g,
                                                   float *__restrict__ out) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < g.total;
       e += (int64_t)gridDim.x * blockDim.x) {
    int64_t inner = e % g.inner_volume;
    const int64_t rest_index = e / g.inner_volume;
    const int64_t position = rest_index % g.extent;
    int64_t outer = rest_index / g.extent;
    int64_t at = 0;
    for (int d = g.inner_rank - 1; d >= 0; --d) {
      at += (inner % g.inner_shape[d]) * g.inner_strides[d];
      inner /= g.inner_shape[d];
    }
    for (int d = g.outer_rank - 1; d >= 0; --d) {
      at += (outer % g.outer_shape[d]) * g.outer_strides[d];
      outer /= g.outer_shape[d];
    }
    float total = 0.0f;  // zero_like().promote(): +0
    for (int64_t k = 0; k < g.size; ++k) {
      const int64_t reach = k * g.dilation;
      if (reach > position) break;
      const int64_t rest = position - reach;
      if (rest % g.step != 0) continue;
      const int64_t window = rest / g.step;
      if (window >= g.count) continue;
      total = total + source[at + window * g.window_stride + k * g.element_stride];
    }
    out[e] = total;
  }
}

unsigned blocks_for(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return (unsigned)(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

}  // namespace

void launch_fold(const float *source, const FoldGeometry &geometry, float *out, hipStream_t stream) {
  if (geometry.total <= 0) return;
  fold_kernel<<<blocks_for(geometry.total), 256, 0, stream>>>(source, geometry, out);
  check_launch("fold_kernel launch");
}

}  // namespace topos_hip
