// Generated kernels: an elementwise expression over strided views, emitted
// as HIP source and compiled by hipRTC for gfx950 (cached per source text).
//
// One expression model serves three kernel shapes:
//   - a chain: the expression's requested results written contiguous, four
//     consecutive elements per lane (16-byte loads and stores where legal);
//   - a fold: the expression reduced along one axis in ascending order, one
//     lane per output, seeded with the first term (the sequential folds of
//     src/payload/tensor.rs:1055-1124);
//   - the two passes of an exact whole-tensor sum over a large operand (count
//     and compact the nonzero terms), whose final ordered fold runs in
//     index.hip.
// Every operation rounds to f32 exactly as the interpreter's materialised
// intermediate does: no contraction, no fast math, libm-faithful
// transcendentals.
#pragma once
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "backend.hpp"

namespace topos_hip {

constexpr int kMaxRank = TOPOS_HIP_MAX_RANK;
static_assert(kMaxRank == 6, "the shape initialisers below list six axes");

struct ExprInput {
  // kLiteral: the constant `one` everywhere, embedded in the source (its
  // pointer argument is unused).
  enum Kind { kStrided = 0, kSelection = 1, kPadded = 2, kLiteral = 3 };
  int kind = kStrided;
  // kStrided / kPadded: element (c0..) lives at offset + sum c_d * strides[d]
  // (kPadded: with the pad axis coordinate shifted by -pad_start, and +0
  // outside the window).
  int64_t offset = 0;
  int64_t strides[kMaxRank] = {};
  // kSelection: the expression is [rows, vocab]; the element is `one` where
  // indices[c0] == c1, else +0.
  float one = 1.0f;
  // kPadded: the window [pad_start, pad_start + pad_len) along pad_axis.
  int pad_axis = 0;
  int64_t pad_start = 0;
  int64_t pad_len = 0;
};

// Operand references: >= 0 an earlier step, < 0 input (-ref - 1).
struct ExprStep {
  int op = 0;  // TOPOS_HIP_CHAIN_*
  int left = 0;
  int right = 0;
};

struct Expr {
  int rank = 0;
  int64_t shape[kMaxRank] = {1, 1, 1, 1, 1, 1};
  std::vector<ExprInput> inputs;
  std::vector<ExprStep> steps;
  std::vector<int> outputs;  // references; a fold reads outputs[0]
  int64_t volume() const {
    int64_t v = 1;
    for (int d = 0; d < rank; ++d) v *= shape[d];
    return v;
  }
};

enum FoldKind { kFoldSum = 0, kFoldMax = 1 };

bool is_unary(int op);
bool is_binary(int op);

// A generated kernel: its source, then (after compile_kernels) its loaded
// function.
struct Kernel {
  std::string source;
  hipFunction_t function = nullptr;
  bool loaded = false;
};
using Generated = std::shared_ptr<Kernel>;

// Compiles every distinct source not yet in the process cache, in parallel
// (hipRTC, gfx950), and, when `load`, loads the modules. Kernels whose source
// is cached share the cached module.
void compile_kernels(const std::vector<Generated> &kernels, bool load);

// Chain: outputs[o] receives volume() contiguous floats.
Generated generate_chain(const Expr &e);
void launch_generated_chain(const Generated &g, const Expr &e, const void *const *inputs,
                            float *const *outputs, hipStream_t stream);

// A pure copy of one strided input whose innermost axis has a non-unit
// stride while another axis has unit stride, both extents multiples of 64:
// generate_transpose_copy moves it in 64 x 64 tiles through LDS. The output
// receives volume() contiguous floats.
bool transposing_copy(const Expr &e);
Generated generate_transpose_copy(const Expr &e);
void launch_transpose_copy(const Generated &g, const Expr &e, const void *input, float *output, hipStream_t stream);

// Fold along `axis`: the output is the expression's shape without that axis,
// contiguous.
Generated generate_fold(const Expr &e, int axis, FoldKind kind);
void launch_generated_fold(const Generated &g, const Expr &e, int axis, const void *const *inputs,
                           float *out, hipStream_t stream);

// A row program: one launch evaluating a group of row-local nodes of a plan
// over the [rows, columns] view of `shape` (columns = the last axis, rows =
// the leading axes flattened). Full values live per element, row values per
// row; a row value enters full expressions broadcast along the row. Folds
// (sum, max, and the max-then-shifted-exponential-sum pairs of LogSumExp and
// LogSoftmax) are the interpreter's: one lane per row, ascending, seeded with
// the row's first term. The kernel makes one pass over the columns per fold
// level and a last pass writing the requested full values (contiguous
// [rows, columns]) and row values (contiguous [rows]).
struct RowRef {
  enum Kind { kInput = 0, kFull = 1, kRow = 2 };
  int kind = kInput;
  int index = 0;  // an input, or an earlier node
};

struct RowNode {
  // kFullOp / kRowOp: TOPOS_HIP_CHAIN_* `op` on a (and b); kSum / kMax: the
  // ordered fold of full operand a; kLogSumExp: max + ln(sum exp(a - max));
  // kLogSoftmax (a full value): (a - max) - ln(sum exp(a - max)).
  enum Kind { kFullOp = 0, kRowOp = 1, kSum = 2, kMax = 3, kLogSumExp = 4, kLogSoftmax = 5 };
  int kind = kFullOp;
  int op = 0;
  RowRef a, b;
  bool full() const { return kind == kFullOp || kind == kLogSoftmax; }
};

struct RowProgram {
  int rank = 0;
  int64_t shape[kMaxRank] = {1, 1, 1, 1, 1, 1};
  std::vector<ExprInput> inputs;   // layouts over the full shape (row inputs: stride 0 on the last axis)
  std::vector<RowNode> nodes;      // in evaluation order
  std::vector<int> full_outputs;   // full nodes written [rows, columns]
  std::vector<int> row_outputs;    // row nodes written [rows]
  // Rank 2 only: full outputs written [columns, rows] (a column program's
  // [R, C] nodes, row-major), one element a store.
  bool transposed_outputs = false;
  int64_t columns() const { return shape[rank - 1]; }
  int64_t rows() const {
    int64_t r = 1;
    for (int d = 0; d + 1 < rank; ++d) r *= shape[d];
    return r;
  }
};

Generated generate_row_program(const RowProgram &p);
void launch_row_program(const Generated &g, const RowProgram &p, const void *const *inputs,
                        float *const *full_outputs, float *const *row_outputs, hipStream_t stream);

// Whole-tensor exact sum over a large operand, in chunks of kSumChunk flat
// elements (one workgroup each, lanes on consecutive elements): one pass
// writes each chunk's nonzero terms, in element order, to the front of the
// chunk's own slot range [chunk * kSumChunk, ...), with the chunk's count and
// whether it holds a +0 (launch_slot_fold then folds the slots in order).
constexpr int64_t kSumChunk = 4096;
Generated generate_sum_gather(const Expr &e);
void launch_sum_gather(const Generated &g, const Expr &e, const void *const *inputs, float *slots, int32_t *counts,
                       int32_t *positive_zero, hipStream_t stream);

}  // namespace topos_hip
