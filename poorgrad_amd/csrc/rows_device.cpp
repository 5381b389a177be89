// The device face's exact row reductions and LayerNorm as generated row
// programs (codegen.hpp): the same exact folds and elementwise steps as the
// plan face's row groups, so one kernel family serves both. A program is
// generated and compiled on first use of a (reduction, rows, columns,
// epsilon) and cached for the process.
#include <map>
#include <mutex>
#include <tuple>

#include "codegen.hpp"

namespace topos_hip {
namespace {

constexpr int kLayerNormKind = 100;

std::mutex programs_lock;
std::map<std::tuple<int, int64_t, int64_t, uint32_t>, std::pair<RowProgram, Generated>> &programs() {
  static auto *cache = new std::map<std::tuple<int, int64_t, int64_t, uint32_t>, std::pair<RowProgram, Generated>>();
  return *cache;
}

ExprInput matrix(int64_t columns) {
  ExprInput in;
  in.strides[0] = columns;
  in.strides[1] = 1;
  return in;
}

ExprInput literal(float value) {
  ExprInput in;
  in.kind = ExprInput::kLiteral;
  in.one = value;
  return in;
}

RowNode op(int kind, int chain_op, RowRef a, RowRef b = RowRef{}) {
  RowNode n;
  n.kind = kind;
  n.op = chain_op;
  n.a = a;
  n.b = b;
  return n;
}

RowRef input(int i) { return RowRef{RowRef::kInput, i}; }
RowRef full(int i) { return RowRef{RowRef::kFull, i}; }
RowRef row(int i) { return RowRef{RowRef::kRow, i}; }

// Inputs: 0 = x; layer norm adds 1 = scale, 2 = shift (rows of stride 0),
// 3 = count, 4 = epsilon (literals).
RowProgram program_for(int kind, int64_t rows, int64_t columns, float epsilon) {
  RowProgram p;
  p.rank = 2;
  p.shape[0] = rows;
  p.shape[1] = columns;
  p.inputs.push_back(matrix(columns));
  switch (kind) {
    case TOPOS_HIP_ROWS_SUM:
      p.nodes.push_back(op(RowNode::kSum, 0, input(0)));
      p.row_outputs.push_back(0);
      break;
    case TOPOS_HIP_ROWS_MAX:
      p.nodes.push_back(op(RowNode::kMax, 0, input(0)));
      p.row_outputs.push_back(0);
      break;
    case TOPOS_HIP_ROWS_LOG_SUM_EXP:
      p.nodes.push_back(op(RowNode::kLogSumExp, 0, input(0)));
      p.row_outputs.push_back(0);
      break;
    case TOPOS_HIP_ROWS_LOG_SOFTMAX:
      p.nodes.push_back(op(RowNode::kLogSoftmax, 0, input(0)));
      p.full_outputs.push_back(0);
      break;
    case TOPOS_HIP_ROWS_SOFTMAX:  // log_softmax(1).exp() (src/graph/composite.rs:43-45)
      p.nodes.push_back(op(RowNode::kLogSoftmax, 0, input(0)));
      p.nodes.push_back(op(RowNode::kFullOp, TOPOS_HIP_CHAIN_EXP, full(0)));
      p.full_outputs.push_back(1);
      break;
    case kLayerNormKind: {  // src/neural/layer_norm.rs:100-132
      ExprInput scale, shift;
      scale.strides[1] = 1;  // [columns] broadcast along the rows
      shift.strides[1] = 1;
      p.inputs.push_back(scale);
      p.inputs.push_back(shift);
      p.inputs.push_back(literal((float)columns));  // counted(shape, extent) as f32
      p.inputs.push_back(literal(epsilon));
      p.nodes.push_back(op(RowNode::kSum, 0, input(0)));                                  // 0 total
      p.nodes.push_back(op(RowNode::kRowOp, TOPOS_HIP_CHAIN_DIV, row(0), input(3)));      // 1 mean
      p.nodes.push_back(op(RowNode::kFullOp, TOPOS_HIP_CHAIN_SUB, input(0), row(1)));     // 2 centred
      p.nodes.push_back(op(RowNode::kFullOp, TOPOS_HIP_CHAIN_MUL, full(2), full(2)));     // 3 square
      p.nodes.push_back(op(RowNode::kSum, 0, full(3)));                                   // 4 power
      p.nodes.push_back(op(RowNode::kRowOp, TOPOS_HIP_CHAIN_DIV, row(4), input(3)));      // 5 variance
      p.nodes.push_back(op(RowNode::kRowOp, TOPOS_HIP_CHAIN_ADD, row(5), input(4)));      // 6 + epsilon
      p.nodes.push_back(op(RowNode::kRowOp, TOPOS_HIP_CHAIN_SQRT, row(6)));               // 7 deviation
      p.nodes.push_back(op(RowNode::kFullOp, TOPOS_HIP_CHAIN_DIV, full(2), row(7)));      // 8 normalised
      p.nodes.push_back(op(RowNode::kFullOp, TOPOS_HIP_CHAIN_MUL, full(8), input(1)));    // 9 * scale
      p.nodes.push_back(op(RowNode::kFullOp, TOPOS_HIP_CHAIN_ADD, full(9), input(2)));    // 10 + shift
      p.full_outputs.push_back(10);
      break;
    }
    default:
      throw InvalidArgument{"unknown row reduction"};
  }
  return p;
}

const std::pair<RowProgram, Generated> &cached(int kind, int64_t rows, int64_t columns, float epsilon) {
  const auto key = std::make_tuple(kind, rows, columns, __builtin_bit_cast(uint32_t, epsilon));
  std::lock_guard<std::mutex> guard(programs_lock);
  auto it = programs().find(key);
  if (it != programs().end()) return it->second;
  RowProgram p = program_for(kind, rows, columns, epsilon);
  Generated g = generate_row_program(p);
  compile_kernels({g}, true);
  return programs().emplace(key, std::make_pair(p, g)).first->second;
}

}  // namespace

void launch_rows_program(int reduction, const float *x, int64_t rows, int64_t columns, float *out,
                         hipStream_t stream) {
  const auto &entry = cached(reduction, rows, columns, 0.0f);
  const void *inputs[1] = {x};
  float *outputs[1] = {out};
  const bool full_result = !entry.first.full_outputs.empty();
  launch_row_program(entry.second, entry.first, inputs, full_result ? outputs : nullptr,
                     full_result ? nullptr : outputs, stream);
}

void launch_layer_norm_program(const float *x, int64_t rows, int64_t columns, const float *scale,
                               const float *shift, float epsilon, float *out, hipStream_t stream) {
  const auto &entry = cached(kLayerNormKind, rows, columns, epsilon);
  const void *inputs[5] = {x, scale, shift, nullptr, nullptr};
  float *outputs[1] = {out};
  launch_row_program(entry.second, entry.first, inputs, outputs, nullptr, stream);
}

}  // namespace topos_hip
