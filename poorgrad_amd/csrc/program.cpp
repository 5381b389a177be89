// The plan face: a topos forward plan, lowered to a node table, executed on
// one GPU from one pre-sized HBM arena.
//
// Planning restates what Plan::new and Plan::forward decide
// (src/engine/plan.rs:143-283, 514-641) and adds the device's own choices:
//
//   reachability  wanted = the ancestor closure of the readable nodes;
//   values        every node's value is a storage plus a layout
//                 (src/payload/layout.rs:23-335): a view (transpose, permute,
//                 narrow, broadcast, broadcast_along, view-legal reshape) is a
//                 new layout over its operand's storage and launches nothing;
//                 a Constant payload is a layout of zero strides over one
//                 element (host-known constants are folded at plan time with
//                 the same f32 operations); a Selection is an index buffer;
//   fusion        an elementwise node whose only consumer is another
//                 elementwise node, or a sum, is not materialised: the
//                 consumer's generated kernel recomputes it in registers (the
//                 interpreter's per-node rounding is kept, so the bits do not
//                 change); a pad consumed by one elementwise node becomes a
//                 windowed input of that node's kernel;
//   launches      one per materialised elementwise tree (a generated chain),
//                 per reduction (a generated fold, the row kernels, or the
//                 exact gathered whole-tensor sum), per product (the GEMM
//                 kernels, batched over leading axes), per gather/scatter;
//   liveness      a storage lives from the launch that writes it to the last
//                 launch that reads it (readable values to the end of the
//                 run); arena offsets are assigned first-fit over those
//                 intervals.
#include <algorithm>
#include <array>
#include <climits>
#include <cmath>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <sstream>
#include <vector>

#include "codegen.hpp"
#include "faithful_math.h"

namespace topos_hip {

std::string &last_refusal() {
  static thread_local std::string message;
  return message;
}

namespace {

// The largest reduced extent a column program (a transposed row group) takes:
// its strided column reads stay within what a workgroup keeps resident.
constexpr int64_t kColumnProgramRows = 2048;

struct Layout {
  int rank = 0;
  int64_t shape[kMaxRank] = {1, 1, 1, 1, 1, 1};
  int64_t strides[kMaxRank] = {};
  int64_t offset = 0;
  int64_t volume() const {
    int64_t v = 1;
    for (int d = 0; d < rank; ++d) v *= shape[d];
    return v;
  }
};

Layout contiguous(int rank, const int64_t *shape, int64_t offset = 0) {
  Layout l;
  l.rank = rank;
  l.offset = offset;
  int64_t running = 1;
  for (int d = rank - 1; d >= 0; --d) {
    l.shape[d] = shape[d];
    l.strides[d] = running;
    running *= shape[d];
  }
  return l;
}

Layout constant_layout(int rank, const int64_t *shape, int64_t offset) {
  Layout l;
  l.rank = rank;
  l.offset = offset;
  for (int d = 0; d < rank; ++d) l.shape[d] = shape[d];
  return l;
}

// Layout::is_contiguous (layout.rs): extent-1 axes may hold any stride.
bool is_contiguous(const Layout &l) {
  int64_t expected = 1;
  for (int d = l.rank - 1; d >= 0; --d) {
    if (l.shape[d] != 1 && l.strides[d] != expected) return false;
    expected *= l.shape[d];
  }
  return true;
}

// Layout::reshape (layout.rs:...) answers a contiguous layout for any shape
// and a unit-axis view when only extent-1 axes move; otherwise the
// interpreter copies the elements out in logical order. Any layout whose
// groups of merged source axes are themselves contiguous is a view of the
// same elements in the same logical order, so it is taken as a view here
// too (no value changes: a copy and a view read identical elements).
bool reshape_view(const Layout &from, int rank, const int64_t *shape, Layout &out) {
  if (is_contiguous(from)) {
    out = contiguous(rank, shape, from.offset);
    return true;
  }
  // Source and target axes without the extent-1 ones.
  std::vector<int64_t> os, ost, ns;
  std::vector<int> nidx;
  for (int d = 0; d < from.rank; ++d)
    if (from.shape[d] != 1) {
      os.push_back(from.shape[d]);
      ost.push_back(from.strides[d]);
    }
  for (int d = 0; d < rank; ++d)
    if (shape[d] != 1) {
      ns.push_back(shape[d]);
      nidx.push_back(d);
    }
  std::vector<int64_t> nst(ns.size(), 0);
  size_t oi = 0, ni = 0;
  while (oi < os.size() && ni < ns.size()) {
    int64_t op = os[oi], np = ns[ni];
    size_t oj = oi + 1, nj = ni + 1;
    while (op != np) {
      if (np < op) {
        if (nj >= ns.size()) return false;
        np *= ns[nj++];
      } else {
        if (oj >= os.size()) return false;
        op *= os[oj++];
      }
    }
    for (size_t k = oi; k + 1 < oj; ++k)
      if (ost[k] != ost[k + 1] * os[k + 1]) return false;  // merged axes must be contiguous
    nst[nj - 1] = ost[oj - 1];
    for (size_t k = nj - 1; k-- > ni;) nst[k] = nst[k + 1] * ns[k + 1];
    oi = oj;
    ni = nj;
  }
  if (oi != os.size() || ni != ns.size()) return false;
  Layout l;
  l.rank = rank;
  l.offset = from.offset;
  for (int d = 0; d < rank; ++d) {
    l.shape[d] = shape[d];
    l.strides[d] = 0;
  }
  for (size_t k = 0; k < ns.size(); ++k) l.strides[nidx[k]] = nst[k];
  out = l;
  return true;
}

// narrow(axis, start, len) of reshape(`from`, shape) as a view of `from`
// when the reshape as a whole is none: each group of merged source axes must
// be contiguous, except the narrowed target axis, whose range may instead lie
// within one run of its group's innermost source axis (the other axes of the
// group then take fixed indices). This is how a lane of the max-pool window
// lanes ([b, c, oh, ow, kh * kw] of a [b, c, oh, ow, kh, kw] window view,
// src/neural/pooling.rs:10-41) reads the source directly: lane l fixes
// (l / kw, l % kw). The elements are those the copy would hold, in the same
// logical order.
bool narrow_reshape_view(const Layout &from, int rank, const int64_t *shape, int axis, int64_t start, int64_t len,
                         Layout &out) {
  if (axis < 0 || axis >= rank || shape[axis] <= 1 || start < 0 || len < 1 || start + len > shape[axis]) return false;
  std::vector<int64_t> os, ost, ns;
  std::vector<int> nidx;
  for (int d = 0; d < from.rank; ++d)
    if (from.shape[d] != 1) {
      os.push_back(from.shape[d]);
      ost.push_back(from.strides[d]);
    }
  int narrowed = -1;
  for (int d = 0; d < rank; ++d)
    if (shape[d] != 1) {
      if (d == axis) narrowed = (int)ns.size();
      ns.push_back(shape[d]);
      nidx.push_back(d);
    }
  std::vector<int64_t> nst(ns.size(), 0);
  int64_t offset = from.offset;
  size_t oi = 0, ni = 0;
  while (oi < os.size() && ni < ns.size()) {
    int64_t op = os[oi], np = ns[ni];
    size_t oj = oi + 1, nj = ni + 1;
    while (op != np) {
      if (np < op) {
        if (nj >= ns.size()) return false;
        np *= ns[nj++];
      } else {
        if (oj >= os.size()) return false;
        op *= os[oj++];
      }
    }
    if ((int)ni <= narrowed && narrowed < (int)nj) {
      if (nj - ni != 1) return false;  // the narrowed axis must be its group's only target axis
      const int64_t inner = os[oj - 1];
      if (start % inner + len > inner) return false;
      int64_t rest = start / inner;
      for (size_t k = oj - 1; k-- > oi;) {
        offset += (rest % os[k]) * ost[k];
        rest /= os[k];
      }
      offset += (start % inner) * ost[oj - 1];
      nst[ni] = len > 1 ? ost[oj - 1] : 0;
    } else {
      for (size_t k = oi; k + 1 < oj; ++k)
        if (ost[k] != ost[k + 1] * os[k + 1]) return false;
      nst[nj - 1] = ost[oj - 1];
      for (size_t k = nj - 1; k-- > ni;) nst[k] = nst[k + 1] * ns[k + 1];
    }
    oi = oj;
    ni = nj;
  }
  if (oi != os.size() || ni != ns.size()) return false;
  Layout l;
  l.rank = rank;
  l.offset = offset;
  for (int d = 0; d < rank; ++d) {
    l.shape[d] = d == axis ? len : shape[d];
    l.strides[d] = 0;
  }
  for (size_t k = 0; k < ns.size(); ++k) l.strides[nidx[k]] = nst[k];
  out = l;
  return true;
}

enum class StorageKind { kArena, kParameter, kInput, kLeaf, kPool, kSelectionInput, kSelectionLeaf };

struct Storage {
  StorageKind kind = StorageKind::kArena;
  int64_t index = -1;  // slot, leaf index or pool index
  int64_t bytes = 0;   // arena storages
  int64_t offset = -1; // arena byte offset
  int first = INT_MAX;
  int last = -1;
  bool pinned = false;
  bool side = false;  // written on the side stream: placed in the side region
  // selections
  int64_t rows = 0, vocab = 0;
  float one = 1.0f;
};

struct Value {
  // kWindow: a convolution's patch matrix (or its transpose) over the dense
  // source `storage`/`layout`, read only by window products.
  enum Kind { kNone, kDense, kSelection, kInline, kPadInline, kWindow } kind = kNone;
  int storage = -1;
  Layout layout;
  bool constant = false;
  bool host_known = false;
  float host_value = 0.0f;
  // No element is -0 (a matrix-core product, and views of one).
  bool never_minus_zero = false;
  // A rank-3 view whose axis 0 merges two strided axes (batch x heads):
  // index y sits at (y / split_inner) * split_outer_stride + (y % split_inner)
  // * split_inner_stride, and layout.strides[0] is unused. Only products
  // read such a value (their two-level batch strides); anything else copies
  // it first.
  int64_t split_inner = 0;
  int64_t split_outer_stride = 0, split_inner_stride = 0;
  // A reshape that is no view of `layout` as a whole, left unresolved because
  // only narrows read it and each of them is a view (narrow_reshape_view):
  // `layout` is the reshape's operand's, the node's shape the reshape's.
  bool reshape_pending = false;
  WindowShape window;
  bool window_transposed = false;
};

// Device buffers of a bound selection: its indices and their row-sorted
// order (CSR over the vocabulary) for the ordered scatter.
struct SelectionBuffers {
  int32_t *indices = nullptr;
  int32_t *row_start = nullptr;
  int32_t *sources = nullptr;
  int64_t rows = 0, vocab = 0;
};

bool is_elementwise(int op) {
  switch (op) {
    case TOPOS_HIP_OP_ADD: case TOPOS_HIP_OP_SUB: case TOPOS_HIP_OP_MUL: case TOPOS_HIP_OP_DIV:
    case TOPOS_HIP_OP_NEG: case TOPOS_HIP_OP_TANH: case TOPOS_HIP_OP_EXP: case TOPOS_HIP_OP_LN:
    case TOPOS_HIP_OP_SQRT: case TOPOS_HIP_OP_POWF: case TOPOS_HIP_OP_MAXIMUM: case TOPOS_HIP_OP_RELU:
    case TOPOS_HIP_OP_STEP:
      return true;
  }
  return false;
}

int arity(int op) {
  switch (op) {
    case TOPOS_HIP_OP_LEAF: case TOPOS_HIP_OP_PARAMETER: case TOPOS_HIP_OP_INPUT: return 0;
    case TOPOS_HIP_OP_ADD: case TOPOS_HIP_OP_SUB: case TOPOS_HIP_OP_MUL: case TOPOS_HIP_OP_DIV:
    case TOPOS_HIP_OP_MATMUL: case TOPOS_HIP_OP_BROADCAST: case TOPOS_HIP_OP_BROADCAST_ALONG:
    case TOPOS_HIP_OP_GATHER: case TOPOS_HIP_OP_SCATTER: case TOPOS_HIP_OP_POWF: case TOPOS_HIP_OP_MAXIMUM:
    case TOPOS_HIP_OP_STEP:
      return 2;
  }
  return 1;
}

const char *op_name(int op) {
  static const char *names[] = {"Leaf", "Parameter", "Input", "Add", "Sub", "Mul", "Div", "Neg", "Tanh", "Exp",
                                "Ln", "MatMul", "Transpose", "Sum", "SumAlong", "Broadcast", "BroadcastAlong",
                                "Reshape", "Permute", "Narrow", "Pad", "Unfold", "Fold", "Gather", "Scatter",
                                "LogSoftmax", "LogSumExp", "Sqrt", "Powf", "Maximum", "Relu", "Step"};
  return op >= 0 && op <= TOPOS_HIP_OP_STEP ? names[op] : "?";
}

// f32 arithmetic of one elementwise node on host-known constants: the same
// operations the kernels and the interpreter perform.
float fold_scalar(int op, float a, float b) {
  using namespace topos_faithful;
  switch (op) {
    case TOPOS_HIP_OP_ADD: return a + b;
    case TOPOS_HIP_OP_SUB: return a - b;
    case TOPOS_HIP_OP_MUL: return a * b;
    case TOPOS_HIP_OP_DIV: return a / b;
    case TOPOS_HIP_OP_NEG: return -a;
    case TOPOS_HIP_OP_TANH: return tanh_f32(a);
    case TOPOS_HIP_OP_EXP: return exp_f32(a);
    case TOPOS_HIP_OP_LN: return ln_f32(a);
    case TOPOS_HIP_OP_SQRT: return std::sqrt(a);
    case TOPOS_HIP_OP_POWF: return pow_f32(a, b);
    case TOPOS_HIP_OP_MAXIMUM: return max_f32(a, b);
    case TOPOS_HIP_OP_RELU: return max_f32(a, 0.0f);
    case TOPOS_HIP_OP_STEP: return step_f32(a, b);
  }
  throw InvalidArgument{"not an elementwise operation"};
}

// The sequential sum of `count` copies of `value` (tensor.rs:1055-1093 over a
// Constant payload); stops once further terms cannot change the total.
float fold_repeated(float value, int64_t count) {
  float acc = value;
  for (int64_t i = 1; i < count; ++i) {
    const float next = acc + value;
    if (next == acc || next != next) {
      acc = next;
      break;
    }
    acc = next;
  }
  return acc;
}

int chain_op(int op) {
  switch (op) {
    case TOPOS_HIP_OP_ADD: return TOPOS_HIP_CHAIN_ADD;
    case TOPOS_HIP_OP_SUB: return TOPOS_HIP_CHAIN_SUB;
    case TOPOS_HIP_OP_MUL: return TOPOS_HIP_CHAIN_MUL;
    case TOPOS_HIP_OP_DIV: return TOPOS_HIP_CHAIN_DIV;
    case TOPOS_HIP_OP_NEG: return TOPOS_HIP_CHAIN_NEG;
    case TOPOS_HIP_OP_TANH: return TOPOS_HIP_CHAIN_TANH;
    case TOPOS_HIP_OP_EXP: return TOPOS_HIP_CHAIN_EXP;
    case TOPOS_HIP_OP_LN: return TOPOS_HIP_CHAIN_LN;
    case TOPOS_HIP_OP_SQRT: return TOPOS_HIP_CHAIN_SQRT;
    case TOPOS_HIP_OP_MAXIMUM: return TOPOS_HIP_CHAIN_MAX;
    case TOPOS_HIP_OP_STEP: return TOPOS_HIP_CHAIN_STEP;
    case TOPOS_HIP_OP_POWF: return TOPOS_HIP_CHAIN_POWF;
  }
  throw Unsupported{std::string("no device kernel computes ") + op_name(op) + " of a non-constant operand"};
}

}  // namespace

}  // namespace topos_hip

using namespace topos_hip;

struct topos_hip_program {
  // ---- the program ----
  std::vector<topos_hip_node> nodes;
  std::vector<topos_hip_leaf> leaves;
  std::vector<float> leaf_data;
  std::vector<int32_t> leaf_indices;
  int numerics = TOPOS_HIP_EXACT;
  bool device = true;  // false under the fake runtime: plan and compile only
  // The engine-backward route: node -> the node holding the target's
  // gradient with respect to it (topos_hip_program_create_backward).
  std::map<int64_t, int64_t> gradient_of;

  // ---- the plan ----
  std::vector<bool> wanted, readable;
  std::vector<bool> mfma_product;  // a product the matrix-core kernel computes (never -0)
  // A per-column addend a matrix-core product adds as it is written (a
  // linear layer's bias), filled in when the addition is planned.
  struct BiasEpilogue {
    int storage = -1;
    int64_t offset = 0, stride = 0;
    bool first = false;  // bias + product rather than product + bias
  };
  // Where a product writes: its storage, row stride and batch strides (a
  // product read only through a copying reshape of its permuted view writes
  // straight into the reshape's layout instead).
  struct ProductOutput {
    int storage = -1;
    int64_t ldc = 0;
    Batch batch;
  };
  struct ProductLaunch {
    int launch;
    std::shared_ptr<BiasEpilogue> bias;
    std::shared_ptr<ProductOutput> output;
    bool flat = true;
  };
  std::map<int64_t, ProductLaunch> product_launch;
  std::map<int, int64_t> product_of_storage;  // a matrix-core product's output storage -> its node
  std::vector<std::vector<int>> consumers;
  std::vector<Value> values;
  std::vector<Storage> storages;
  std::vector<float> pool;  // host-known constants, in device order
  std::map<int64_t, int> parameter_storage, input_storage, leaf_storage;
  struct Exec {
    topos_hip_program *program;
    hipStream_t stream;
  };
  struct Launch {
    std::string what;
    std::vector<int> reads, writes;
    std::function<void(const Exec &)> run;
    std::string kind;
    double flops = 0, bytes = 0;
    bool side = false;     // runs on the side stream
    int wait_for = -1;     // side launch: the main launch whose completion it awaits
    bool signals = false;  // main launch: records its event for side launches
  };
  std::vector<Launch> launches;
  std::vector<Generated> pending;  // generated kernels, compiled together after planning
  // A generated chain launch: its expression grows while it is the last
  // launch planned (a following chain over the same shape whose inputs are
  // complete by then joins it as one more output); its source is generated
  // once planning ends.
  struct ChainRecord {
    int launch = -1;
    Expr e;
    std::vector<int> storage_of;  // per expression input
    std::vector<int> outs;        // per expression output
    std::string ops;
    Generated g;
  };
  std::vector<std::shared_ptr<ChainRecord>> chains;
  std::shared_ptr<ChainRecord> open_chain;
  std::map<int64_t, int> output_storage;  // readable node -> storage holding it contiguous
  std::map<int64_t, int64_t> output_offset;
  uint64_t arena_bytes = 0;
  int64_t fused_groups = 0;
  std::string description;

  // ---- device state ----
  char *arena = nullptr;
  float *constants = nullptr;  // pool then leaf data
  int64_t leaf_data_offset = 0;
  std::map<int64_t, const float *> parameters, inputs;
  std::map<int64_t, SelectionBuffers> selection_inputs;
  std::map<int64_t, SelectionBuffers> selection_leaves;
  std::vector<void *> allocations;

  // The side stream and the events that order it after the main stream.
  hipStream_t side_stream = nullptr;
  std::map<int, hipEvent_t> signal_events;
  hipEvent_t side_start = nullptr, side_done = nullptr;
  int64_t side_launches = 0;

  // A run captured as a HIP graph (replay): captured on a stream of the
  // program's own (the caller's may be the legacy default stream, which
  // cannot capture), launched on the caller's. Kernel arguments are captured
  // by value, so any bind drops it.
  hipStream_t capture_stream = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;

  // One program, many host threads (a Plan is Send + Sync,
  // src/engine/plan.rs:20): every entry point that enqueues, binds or reads
  // holds `lock`, and each run first waits (on the GPU, not the host) for the
  // previous run's completion, recorded in `run_done` on that run's stream,
  // so runs on different streams never overlap on the one arena. A value a
  // run leaves in the arena is valid until the next run of the program.
  mutable std::mutex lock;
  hipEvent_t run_done = nullptr;
  hipStream_t last_stream = nullptr;
  bool ran = false;

  // Orders a run enqueued on `stream` after the previous run.
  void serialize_before(hipStream_t stream) {
    if (ran && stream != last_stream) check(hipStreamWaitEvent(stream, run_done, 0), "hipStreamWaitEvent(run)");
  }
  void record_after(hipStream_t stream) {
    check(hipEventRecord(run_done, stream), "hipEventRecord(run done)");
    last_stream = stream;
    ran = true;
  }

  ~topos_hip_program() {
    if (!device) return;
    drop_graph();
    if (run_done) hipEventDestroy(run_done);
    if (capture_stream) hipStreamDestroy(capture_stream);
    for (auto &kv : signal_events) hipEventDestroy(kv.second);
    if (side_done) hipEventDestroy(side_done);
    if (side_start) hipEventDestroy(side_start);
    if (side_stream) hipStreamDestroy(side_stream);
    for (void *p : allocations) hipFree(p);
    for (auto &kv : selection_inputs) {
      hipFree(kv.second.indices);
      hipFree(kv.second.row_start);
      hipFree(kv.second.sources);
    }
  }

  // ================= planning =================

  const topos_hip_node &node(int64_t i) const { return nodes[i]; }

  [[noreturn]] void refuse(int64_t i, const std::string &why) const {
    throw InvalidArgument{"node " + std::to_string(i) + " (" + op_name(nodes[i].op) + "): " + why};
  }

  static bool same_shape(const topos_hip_node &a, const topos_hip_node &b) {
    if (a.rank != b.rank) return false;
    for (int d = 0; d < a.rank; ++d)
      if (a.shape[d] != b.shape[d]) return false;
    return true;
  }

  static int64_t volume_of(const topos_hip_node &n) {
    int64_t v = 1;
    for (int d = 0; d < n.rank; ++d) v *= n.shape[d];
    return v;
  }

  // Checks the table: operand references, arities, and each recorded shape
  // against the shape the variant infers (Function::infer_shape,
  // src/function/function.rs:386-431).
  void validate() {
    const int64_t n = (int64_t)nodes.size();
    for (int64_t i = 0; i < n; ++i) {
      const topos_hip_node &x = nodes[i];
      if (x.op < 0 || x.op > TOPOS_HIP_OP_STEP) refuse(i, "unknown operation");
      if (x.rank < 0 || x.rank > kMaxRank) refuse(i, "rank beyond the library's six axes");
      for (int d = 0; d < x.rank; ++d)
        if (x.shape[d] <= 0) refuse(i, "empty axis");
      const int k = arity(x.op);
      for (int j = 0; j < 2; ++j) {
        if (j < k && (x.operands[j] < 0 || x.operands[j] >= i)) refuse(i, "operand must name an earlier node");
        if (j >= k && x.operands[j] != -1) refuse(i, "unused operand slot must be -1");
      }
      const topos_hip_node *a = k > 0 ? &nodes[x.operands[0]] : nullptr;
      const topos_hip_node *b = k > 1 ? &nodes[x.operands[1]] : nullptr;
      auto expect = [&](bool ok, const char *what) {
        if (!ok) refuse(i, what);
      };
      switch (x.op) {
        case TOPOS_HIP_OP_LEAF: {
          expect(x.slot >= 0 && x.slot < (int64_t)leaves.size(), "leaf payload index");
          const topos_hip_leaf &leaf = leaves[x.slot];
          if (leaf.kind == TOPOS_HIP_LEAF_DENSE)
            expect(leaf.offset >= 0 && leaf.count == volume_of(x) &&
                       leaf.offset + leaf.count <= (int64_t)leaf_data.size(),
                   "dense leaf payload span");
          else if (leaf.kind == TOPOS_HIP_LEAF_SELECTION) {
            expect(x.rank == 2 && leaf.count == x.shape[0] && leaf.offset >= 0 &&
                       leaf.offset + leaf.count <= (int64_t)leaf_indices.size(),
                   "selection leaf payload span");
            for (int64_t r = 0; r < leaf.count; ++r)
              expect(leaf_indices[leaf.offset + r] >= 0 && leaf_indices[leaf.offset + r] < x.shape[1],
                     "selection index out of vocabulary");
          } else
            expect(leaf.kind == TOPOS_HIP_LEAF_CONSTANT, "leaf payload kind");
          break;
        }
        case TOPOS_HIP_OP_PARAMETER:
        case TOPOS_HIP_OP_INPUT:
          expect(x.slot >= 0, "slot");
          if (x.flags & TOPOS_HIP_NODE_SELECTION) expect(x.op == TOPOS_HIP_OP_INPUT && x.rank == 2, "selection input shape");
          break;
        case TOPOS_HIP_OP_ADD: case TOPOS_HIP_OP_SUB: case TOPOS_HIP_OP_MUL: case TOPOS_HIP_OP_DIV:
        case TOPOS_HIP_OP_POWF: case TOPOS_HIP_OP_MAXIMUM: case TOPOS_HIP_OP_STEP:
          expect(same_shape(*a, *b) && same_shape(x, *a), "elementwise operands and result share one shape");
          break;
        case TOPOS_HIP_OP_NEG: case TOPOS_HIP_OP_TANH: case TOPOS_HIP_OP_EXP: case TOPOS_HIP_OP_LN:
        case TOPOS_HIP_OP_SQRT: case TOPOS_HIP_OP_RELU: case TOPOS_HIP_OP_LOG_SOFTMAX:
          expect(same_shape(x, *a), "the result keeps the operand's shape");
          if (x.op == TOPOS_HIP_OP_LOG_SOFTMAX) expect(x.params[0] >= 0 && x.params[0] < a->rank, "axis");
          break;
        case TOPOS_HIP_OP_MATMUL: {
          expect(a->rank >= 2 && a->rank == b->rank && x.rank == a->rank, "matmul ranks");
          const int s = a->rank - 2;
          for (int d = 0; d < s; ++d) expect(a->shape[d] == b->shape[d] && x.shape[d] == a->shape[d], "batch axes");
          expect(a->shape[s + 1] == b->shape[s] && x.shape[s] == a->shape[s] && x.shape[s + 1] == b->shape[s + 1],
                 "matmul inner dimensions");
          break;
        }
        case TOPOS_HIP_OP_TRANSPOSE:
          if (a->rank < 2) {
            expect(same_shape(x, *a), "transpose below rank 2 is the identity");
          } else {
            expect(a->rank == 2 && x.rank == 2 && x.shape[0] == a->shape[1] && x.shape[1] == a->shape[0],
                   "transpose supports rank 2");
          }
          break;
        case TOPOS_HIP_OP_SUM:
          expect(x.rank == 0, "sum is a scalar");
          break;
        case TOPOS_HIP_OP_SUM_ALONG: case TOPOS_HIP_OP_LOG_SUM_EXP: {
          const int64_t axis = x.params[0];
          expect(axis >= 0 && axis < a->rank && x.rank == a->rank - 1, "axis");
          for (int d = 0, e = 0; d < a->rank; ++d)
            if (d != axis) expect(x.shape[e++] == a->shape[d], "the result drops the axis");
          break;
        }
        case TOPOS_HIP_OP_BROADCAST:
          expect(volume_of(*a) == 1 && same_shape(x, *b), "broadcast spreads one element over the like shape");
          break;
        case TOPOS_HIP_OP_BROADCAST_ALONG: {
          const int64_t axis = x.params[0];
          expect(same_shape(x, *b) && axis >= 0 && axis < b->rank && a->rank == b->rank - 1, "broadcast_along");
          for (int d = 0, e = 0; d < b->rank; ++d)
            if (d != axis) expect(a->shape[e++] == b->shape[d], "broadcast_along needs the remaining shape");
          break;
        }
        case TOPOS_HIP_OP_RESHAPE:
          expect(volume_of(x) == volume_of(*a), "reshape keeps the volume");
          break;
        case TOPOS_HIP_OP_PERMUTE: {
          expect(x.rank == a->rank, "permute rank");
          bool seen[kMaxRank] = {};
          for (int d = 0; d < x.rank; ++d) {
            const int64_t o = x.params[d];
            expect(o >= 0 && o < a->rank && !seen[o], "permute order");
            seen[o] = true;
            expect(x.shape[d] == a->shape[o], "permuted shape");
          }
          break;
        }
        case TOPOS_HIP_OP_NARROW: {
          const int64_t axis = x.params[0], start = x.params[1], len = x.params[2];
          expect(axis >= 0 && axis < a->rank && x.rank == a->rank && len > 0 && start >= 0 &&
                     start + len <= a->shape[axis],
                 "narrow window");
          for (int d = 0; d < x.rank; ++d) expect(x.shape[d] == (d == axis ? len : a->shape[d]), "narrowed shape");
          break;
        }
        case TOPOS_HIP_OP_PAD: {
          const int64_t axis = x.params[0], start = x.params[1], full = x.params[2];
          expect(axis >= 0 && axis < a->rank && x.rank == a->rank && start >= 0 && start + a->shape[axis] <= full,
                 "pad window");
          for (int d = 0; d < x.rank; ++d) expect(x.shape[d] == (d == axis ? full : a->shape[d]), "padded shape");
          break;
        }
        case TOPOS_HIP_OP_GATHER:
          expect(b->rank == 2 && a->rank >= 1 && b->shape[1] == a->shape[0] && x.rank == a->rank &&
                     x.shape[0] == b->shape[0],
                 "gather shapes");
          for (int d = 1; d < x.rank; ++d) expect(x.shape[d] == a->shape[d], "gathered rows");
          break;
        case TOPOS_HIP_OP_SCATTER:
          expect(b->rank == 2 && a->rank >= 1 && a->shape[0] == b->shape[0] && x.params[0] == b->shape[1] &&
                     x.rank == a->rank && x.shape[0] == x.params[0],
                 "scatter shapes");
          for (int d = 1; d < x.rank; ++d) expect(x.shape[d] == a->shape[d], "scattered rows");
          break;
        case TOPOS_HIP_OP_UNFOLD: {  // Unfold::infer_shape (src/function/unfold.rs:40-70)
          const int64_t axis = x.params[0], size = x.params[1], step = x.params[2], dilation = x.params[3];
          expect(axis >= 0 && axis < a->rank && x.rank == a->rank + 1 && size > 0 && step > 0 && dilation > 0,
                 "unfold parameters");
          int64_t span = 0;
          expect(!__builtin_mul_overflow(dilation, size - 1, &span) && span < a->shape[axis], "unfold window span");
          for (int d = 0; d < x.rank; ++d) {
            const int64_t want = d < axis ? a->shape[d]
                                 : d == axis ? (a->shape[axis] - span - 1) / step + 1
                                 : d == axis + 1 ? size
                                                 : a->shape[d - 1];
            expect(x.shape[d] == want, "unfolded shape");
          }
          break;
        }
        case TOPOS_HIP_OP_FOLD: {  // Fold::infer_shape (src/function/fold.rs:42-82)
          const int64_t axis = x.params[0], size = x.params[1], step = x.params[2], dilation = x.params[3],
                        extent = x.params[4];
          expect(axis >= 0 && axis + 1 < a->rank && x.rank == a->rank - 1 && size > 0 && step > 0 && dilation > 0,
                 "fold parameters");
          int64_t span = 0;
          expect(!__builtin_mul_overflow(dilation, size - 1, &span) && span < extent, "fold window span");
          expect(a->shape[axis] == (extent - span - 1) / step + 1 && a->shape[axis + 1] == size, "fold window pair");
          for (int d = 0; d < x.rank; ++d)
            expect(x.shape[d] == (d < axis ? a->shape[d] : d == axis ? extent : a->shape[d + 1]), "folded shape");
          break;
        }
      }
    }
  }

  // Operand links whose values are read. The `like` operand of Broadcast and
  // BroadcastAlong contributes its shape only (recorded, hence known), so a
  // node reached only that way needs no computation: skipping it changes no
  // readable value.
  static int value_links(int op) {
    return (op == TOPOS_HIP_OP_BROADCAST || op == TOPOS_HIP_OP_BROADCAST_ALONG) ? 1 : arity(op);
  }

  // Plan::new's reachability (src/engine/plan.rs:150-172) over value links.
  void mark_wanted() {
    const int64_t n = (int64_t)nodes.size();
    wanted.assign(n, false);
    readable.assign(n, false);
    for (int64_t i = 0; i < n; ++i)
      if (nodes[i].flags & TOPOS_HIP_NODE_READABLE) wanted[i] = readable[i] = true;
    // A readable duplicate reads its original's value, which must then be
    // materialised like a readable node.
    for (int64_t i = 0; i < n; ++i)
      if (readable[i] && alias_of[i] >= 0) wanted[alias_of[i]] = readable[alias_of[i]] = true;
    for (int64_t i = n - 1; i >= 0; --i) {
      if (!wanted[i] || alias_of[i] >= 0) continue;
      for (int j = 0; j < value_links(nodes[i].op); ++j) wanted[nodes[i].operands[j]] = true;
    }
    consumers.assign(n, {});
    for (int64_t i = 0; i < n; ++i) {
      if (!wanted[i] || alias_of[i] >= 0) continue;
      for (int j = 0; j < value_links(nodes[i].op); ++j) {
        auto &c = consumers[nodes[i].operands[j]];
        if (c.empty() || c.back() != i) c.push_back((int)i);
      }
    }
  }

  // ---- common subexpressions ----

  // alias_of[i] >= 0: node i repeats an earlier node (same operation, same
  // operands after this rewrite, same parameters and shape), so it has the
  // same value bit for bit; later nodes read the earlier one instead.
  std::vector<int64_t> alias_of;

  void deduplicate() {
    const int64_t n = (int64_t)nodes.size();
    alias_of.assign(n, -1);
    std::vector<int64_t> rep(n);
    std::map<std::vector<int64_t>, int64_t> seen;
    for (int64_t i = 0; i < n; ++i) {
      rep[i] = i;
      topos_hip_node &x = nodes[i];
      for (int j = 0; j < arity(x.op); ++j) x.operands[j] = rep[x.operands[j]];
      if (x.op == TOPOS_HIP_OP_LEAF || x.op == TOPOS_HIP_OP_PARAMETER || x.op == TOPOS_HIP_OP_INPUT) continue;
      std::vector<int64_t> key = {x.op, x.rank, x.operands[0], x.operands[1]};
      for (int d = 0; d < kMaxRank; ++d) key.push_back(x.params[d]);
      for (int d = 0; d < x.rank; ++d) key.push_back(x.shape[d]);
      auto it = seen.find(key);
      if (it != seen.end()) {
        rep[i] = it->second;
        alias_of[i] = it->second;
      } else {
        seen.emplace(std::move(key), i);
      }
    }
  }

  // ---- window products ----

  // WindowProduct (src/engine/pattern/window.rs:58-150): the canonical
  // im2col chain reshape(permute(unfold(unfold(pad(pad(x)))))) of conv2d
  // (src/neural/convolution.rs:24-118). Its interiors (pads, unfolds,
  // permute) are read only inside the chain, so nothing is launched for
  // them; the root's value is the patch matrix itself (a kWindow value) and
  // the products that read it, forward (patches . kernel) and, through the
  // transpose the MatMul rule records, the kernel gradient (patches^T . g),
  // gather each element from x. Unlike the reference's election (forward
  // plans only: there the patches' second reader, the kernel gradient, keeps
  // the chain materialised), both products read the patch matrix in place.
  struct WindowRoot {
    int64_t source = -1;
    int32_t kernel_height = 0, kernel_width = 0, stride = 1, padding = 0;
  };
  std::map<int64_t, WindowRoot> window_roots;
  std::vector<bool> window_interior;

  bool sole_reader(int64_t i, int64_t reader) const {
    return wanted[i] && !readable[i] && alias_of[i] < 0 && consumers[i].size() == 1 && consumers[i][0] == reader;
  }

  // Whether every reader of node i (the patch matrix) is a product taking
  // it as the left operand, directly or through one transpose.
  bool window_readers_ok(int64_t i) const {
    if (consumers[i].empty()) return false;
    for (int c : consumers[i]) {
      const topos_hip_node &y = nodes[c];
      if (y.op == TOPOS_HIP_OP_MATMUL) {
        if (y.operands[0] != i || y.operands[1] == i || y.rank != 2) return false;
      } else if (y.op == TOPOS_HIP_OP_TRANSPOSE) {
        if (readable[c] || consumers[c].empty()) return false;
        for (int d : consumers[c]) {
          const topos_hip_node &z = nodes[d];
          if (z.op != TOPOS_HIP_OP_MATMUL || z.operands[0] != c || z.operands[1] == c || z.rank != 2) return false;
        }
      } else {
        return false;
      }
    }
    return true;
  }

  void form_window_products() {
    const int64_t n = (int64_t)nodes.size();
    window_interior.assign(n, false);
    for (int64_t i = 0; i < n; ++i) {
      const topos_hip_node &x = nodes[i];
      if (!wanted[i] || readable[i] || alias_of[i] >= 0 || x.op != TOPOS_HIP_OP_RESHAPE || x.rank != 2) continue;
      const int64_t permuted = x.operands[0];
      const topos_hip_node &p = nodes[permuted];
      static const int64_t order[6] = {0, 2, 4, 1, 3, 5};
      if (p.op != TOPOS_HIP_OP_PERMUTE || p.rank != 6 || !sole_reader(permuted, i) ||
          !std::equal(order, order + 6, p.params))
        continue;
      const int64_t across = p.operands[0];
      const topos_hip_node &uw = nodes[across];
      if (uw.op != TOPOS_HIP_OP_UNFOLD || !sole_reader(across, permuted) || uw.params[0] != 4 || uw.params[3] != 1)
        continue;
      const int64_t down = uw.operands[0];
      const topos_hip_node &uh = nodes[down];
      if (uh.op != TOPOS_HIP_OP_UNFOLD || !sole_reader(down, across) || uh.params[0] != 2 || uh.params[3] != 1 ||
          uh.params[2] != uw.params[2])
        continue;
      std::vector<int64_t> interiors = {permuted, across, down};
      int64_t source = uh.operands[0];
      int64_t padding = 0;
      // Symmetric zero pads fold into the gather (a +0 outside the source).
      if (nodes[source].op == TOPOS_HIP_OP_PAD && sole_reader(source, down) && nodes[source].params[0] == 3) {
        const int64_t below = nodes[source].operands[0];
        const topos_hip_node &pw = nodes[source], &ph = nodes[below];
        if (ph.op == TOPOS_HIP_OP_PAD && sole_reader(below, source) && ph.params[0] == 2) {
          const topos_hip_node &base = nodes[ph.operands[0]];
          if (base.rank == 4 && ph.params[1] == pw.params[1] && ph.params[2] == base.shape[2] + 2 * ph.params[1] &&
              pw.params[2] == base.shape[3] + 2 * pw.params[1]) {
            interiors.push_back(source);
            interiors.push_back(below);
            padding = ph.params[1];
            source = ph.operands[0];
          }
        }
      }
      const topos_hip_node &src = nodes[source];
      if (src.rank != 4 || is_selection_node(source)) continue;
      const int64_t kh = uh.params[1], kw = uw.params[1], step = uh.params[2];
      const int64_t ph = src.shape[2] + 2 * padding, pw = src.shape[3] + 2 * padding;
      if (kh < 1 || kw < 1 || step < 1 || kh > ph || kw > pw) continue;
      const int64_t oh = (ph - kh) / step + 1, ow = (pw - kw) / step + 1;
      if (x.shape[0] != src.shape[0] * oh * ow || x.shape[1] != src.shape[1] * kh * kw) continue;
      if (x.shape[0] > 0x7fffffff || x.shape[1] > 0x7fffffff || ph > 0x7fffffff || pw > 0x7fffffff) continue;
      if (!window_readers_ok(i)) continue;
      WindowRoot root;
      root.source = source;
      root.kernel_height = (int32_t)kh;
      root.kernel_width = (int32_t)kw;
      root.stride = (int32_t)step;
      root.padding = (int32_t)padding;
      window_roots[i] = root;
      for (int64_t j : interiors) window_interior[j] = true;
    }
  }

  // The patch-matrix value of window root i over its planned source.
  Value window_value(int64_t i) {
    const WindowRoot &root = window_roots.at(i);
    const Value &src = dense_operand(root.source);
    if (src.kind != Value::kDense || src.reshape_pending)
      throw RuntimeFailure{"window product over a source without a dense layout"};
    const topos_hip_node &s = nodes[root.source];
    Value v = src;
    v.kind = Value::kWindow;
    v.constant = v.host_known = v.never_minus_zero = false;
    WindowShape &w = v.window;
    w.offset = src.layout.offset;
    w.s_batch = src.layout.strides[0];
    w.s_channel = src.layout.strides[1];
    w.s_height = src.layout.strides[2];
    w.s_width = src.layout.strides[3];
    w.channels = (int32_t)s.shape[1];
    w.height = (int32_t)s.shape[2];
    w.width = (int32_t)s.shape[3];
    w.kernel_height = root.kernel_height;
    w.kernel_width = root.kernel_width;
    w.stride = root.stride;
    w.padding = root.padding;
    w.out_height = (int32_t)((s.shape[2] + 2 * root.padding - root.kernel_height) / root.stride + 1);
    w.out_width = (int32_t)((s.shape[3] + 2 * root.padding - root.kernel_width) / root.stride + 1);
    v.layout = contiguous(nodes[i].rank, nodes[i].shape);
    return v;
  }

  // A product whose left operand is a patch matrix: exact window kernels
  // (bit-identical to the product over the materialised patches). Under Fast
  // a kernel gradient with few outputs cuts its patch rows into ranges of
  // whole images, each an exact chain, added in range order (the envelope).
  void plan_window_matmul(int64_t i) {
    const topos_hip_node &x = nodes[i];
    const int64_t m = x.shape[0], n = x.shape[1], k = nodes[x.operands[0]].shape[1];
    const Value a = values[x.operands[0]];
    const Value b = dense_operand(x.operands[1]);
    if (b.kind != Value::kDense || b.reshape_pending) throw RuntimeFailure{"window product operand without a layout"};
    const int out = arena_storage(m * n * 4);
    const int64_t brs = b.layout.strides[0], bcs = b.layout.strides[1];
    const WindowShape w = a.window;
    const bool transposed = a.window_transposed;
    const int64_t a_offset = 0, b_offset = b.layout.offset;
    const int64_t positions = (int64_t)w.out_height * w.out_width;
    int splits = 1;
    int workspace = -1;
    if (numerics == TOPOS_HIP_FAST && transposed && positions > 0 && k % positions == 0) {
      splits = window_splits(m, n, k, k / positions);
      if (splits > 1) workspace = arena_storage((int64_t)splits * m * n * 4);
    }
    std::ostringstream what;
    what << "gemm window " << (transposed ? "patches^T" : "patches") << " (" << m << "," << n << "," << k << ") kernel "
         << w.kernel_height << "x" << w.kernel_width << " stride " << w.stride << " pad " << w.padding << " b[" << brs
         << "," << bcs << "]";
    if (splits > 1) what << " in " << splits << " ranges";
    std::vector<int> writes = {out};
    if (workspace >= 0) writes.push_back(workspace);
    add_launch(what.str(), {a.storage, b.storage}, writes, [this, a, b, w, transposed, out, m, n, k, brs, bcs,
                                                            a_offset, b_offset, splits, workspace](const Exec &ex) {
      launch_window_product((const float *)base(a.storage) + a_offset, w, transposed,
                            (const float *)base(b.storage) + b_offset, brs, bcs, m, k, n, (float *)base(out), n,
                            ex.stream, workspace >= 0 ? (float *)base(workspace) : nullptr, splits);
    });
    launches.back().flops = 2.0 * (double)m * n * k;
    const double source = (double)(w.channels) * w.height * w.width * (double)(transposed ? k : m) /
                          ((double)w.out_height * w.out_width);
    launches.back().bytes = 4.0 * (source + (double)k * n + (double)m * n);
    values[i] = dense_value(out, contiguous(x.rank, x.shape));
  }

  // ---- row groups ----

  // A row group: nodes over one [rows, columns] iteration space (full nodes
  // share `shape`; row nodes drop its last axis) whose reductions all run
  // along the last axis, evaluated by one generated row program. Members are
  // elementwise nodes of either shape, broadcasts of row nodes along the last
  // axis, and last-axis SumAlong / LogSumExp / LogSoftmax. The group is
  // launched at its last member; no node outside it consumes a member before
  // that point, and every outside operand is planned before it.
  // A transposed group (a column program) runs over a rank-2 [R, C] space
  // whose reductions all run along axis 0, as a row program over [C, R]:
  // full nodes are read and written through transposed layouts, row nodes
  // are [C] (BatchNorm's statistics, src/neural/batch_norm.rs:149-176).
  struct RowGroup {
    std::vector<int64_t> members;  // ascending
    int rank = 0;
    int64_t shape[kMaxRank] = {1, 1, 1, 1, 1, 1};  // the program's space ([C, R] when transposed)
    bool transposed = false;
  };
  std::vector<RowGroup> row_groups;
  std::vector<int> group_of;

  static bool group_full(const topos_hip_node &x, const RowGroup &g) {
    if (x.rank != g.rank) return false;
    if (g.transposed) return x.shape[0] == g.shape[1] && x.shape[1] == g.shape[0];
    for (int d = 0; d < g.rank; ++d)
      if (x.shape[d] != g.shape[d]) return false;
    return true;
  }
  static bool group_row(const topos_hip_node &x, const RowGroup &g) {
    if (x.rank != g.rank - 1) return false;
    if (g.transposed) return x.shape[0] == g.shape[0];
    for (int d = 0; d < x.rank; ++d)
      if (x.shape[d] != g.shape[d]) return false;
    return true;
  }

  bool is_selection_node(int64_t i) const {
    const topos_hip_node &x = nodes[i];
    if (x.op == TOPOS_HIP_OP_INPUT) return (x.flags & TOPOS_HIP_NODE_SELECTION) != 0;
    return x.op == TOPOS_HIP_OP_LEAF && leaves[x.slot].kind == TOPOS_HIP_LEAF_SELECTION;
  }

  bool row_eligible(int64_t i, const RowGroup &g) const {
    const topos_hip_node &x = nodes[i];
    if (!wanted[i] || group_of[i] >= 0 || alias_of[i] >= 0) return false;
    if (x.op == TOPOS_HIP_OP_SUM_ALONG && is_selection_node(x.operands[0])) return false;
    const int last = g.transposed ? 0 : g.rank - 1;  // the reduced axis
    if (g.transposed) {
      // Operands a transposed program cannot read: selections and inline pads.
      for (int j = 0; j < value_links(x.op); ++j) {
        const int64_t o = x.operands[j];
        if (is_selection_node(o) || nodes[o].op == TOPOS_HIP_OP_PAD) return false;
      }
    }
    if (is_elementwise(x.op)) return group_full(x, g) || group_row(x, g);
    switch (x.op) {
      case TOPOS_HIP_OP_BROADCAST_ALONG: return x.params[0] == last && group_full(x, g);
      case TOPOS_HIP_OP_SUM_ALONG:
      case TOPOS_HIP_OP_LOG_SUM_EXP: return x.params[0] == last && group_row(x, g);
      case TOPOS_HIP_OP_LOG_SOFTMAX: return x.params[0] == last && group_full(x, g);
    }
    return false;
  }

  void form_row_groups() {
    const int64_t n = (int64_t)nodes.size();
    group_of.assign(n, -1);
    for (int64_t seed = 0; seed < n; ++seed) {
      if (!wanted[seed] || group_of[seed] >= 0 || alias_of[seed] >= 0) continue;
      const topos_hip_node &x = nodes[seed];
      RowGroup g;
      if (x.op == TOPOS_HIP_OP_SUM_ALONG || x.op == TOPOS_HIP_OP_LOG_SUM_EXP) {
        const topos_hip_node &a = nodes[x.operands[0]];
        if (x.op == TOPOS_HIP_OP_SUM_ALONG && is_selection_node(x.operands[0])) continue;
        if (x.params[0] == a.rank - 1) {
          g.rank = a.rank;
          for (int d = 0; d < a.rank; ++d) g.shape[d] = a.shape[d];
        } else if (x.params[0] == 0 && a.rank == 2 && a.shape[0] <= kColumnProgramRows) {
          g.rank = 2;
          g.transposed = true;
          g.shape[0] = a.shape[1];
          g.shape[1] = a.shape[0];
        } else {
          continue;
        }
      } else if (x.op == TOPOS_HIP_OP_LOG_SOFTMAX) {
        if (x.params[0] == x.rank - 1) {
          g.rank = x.rank;
          for (int d = 0; d < x.rank; ++d) g.shape[d] = x.shape[d];
        } else if (x.params[0] == 0 && x.rank == 2 && x.shape[0] <= kColumnProgramRows) {
          g.rank = 2;
          g.transposed = true;
          g.shape[0] = x.shape[1];
          g.shape[1] = x.shape[0];
        } else {
          continue;
        }
      } else {
        continue;
      }
      const int id = (int)row_groups.size();
      std::vector<int64_t> members;
      auto add = [&](int64_t j) {
        group_of[j] = id;
        members.push_back(j);
      };
      // Eligible operands whose every consumer is a member join the group.
      auto close_over_operands = [&]() {
        for (bool changed = true; changed;) {
          changed = false;
          for (size_t m = 0; m < members.size(); ++m) {
            const topos_hip_node &y = nodes[members[m]];
            for (int j = 0; j < value_links(y.op); ++j) {
              const int64_t o = y.operands[j];
              if (!row_eligible(o, g) || readable[o]) continue;
              bool inside = true;
              for (int c : consumers[o]) inside = inside && group_of[c] == id;
              if (inside) {
                add(o);
                changed = true;
              }
            }
          }
        }
      };
      add(seed);
      close_over_operands();
      // Consumers in plan order, up to the first outside consumer of a member.
      for (int64_t j = seed + 1; j < n; ++j) {
        if (!wanted[j] || alias_of[j] >= 0) continue;
        bool consumes = false;
        for (int k = 0; k < value_links(nodes[j].op); ++k) consumes = consumes || group_of[nodes[j].operands[k]] == id;
        if (!consumes) continue;
        if (!row_eligible(j, g)) break;
        add(j);
      }
      close_over_operands();
      std::sort(members.begin(), members.end());
      if (g.transposed) {
        // A column program reads its columns strided, so it pays only where
        // it saves launches: statistics broadcast back over the rows (two or
        // more reductions and a broadcast along axis 0). A lone column sum
        // stays a column fold.
        int reductions = 0, broadcasts = 0;
        for (int64_t m : members) {
          const int op = nodes[m].op;
          reductions += op == TOPOS_HIP_OP_SUM_ALONG || op == TOPOS_HIP_OP_LOG_SUM_EXP || op == TOPOS_HIP_OP_LOG_SOFTMAX;
          broadcasts += op == TOPOS_HIP_OP_BROADCAST_ALONG;
        }
        if (reductions < 2 || broadcasts < 1) {
          for (int64_t m : members) group_of[m] = -1;
          continue;
        }
      }
      g.members = members;
      row_groups.push_back(g);
    }
  }

  // The input of a row program that reads node o (planned, outside the
  // group) over the group's iteration space: a full node through its layout,
  // a row node through its layout with stride 0 along the last axis.
  int row_input(RowProgram &p, std::vector<int> &storage_of, std::map<int64_t, int> &input_of, int64_t o,
                bool transposed) {
    auto found = input_of.find(o);
    if (found != input_of.end()) return found->second;
    const topos_hip_node &x = nodes[o];
    const Value &v = values[o];
    const bool row = x.rank == p.rank - 1;
    ExprInput in;
    int storage = v.storage;
    if (v.kind == Value::kDense && v.host_known) {
      in.kind = ExprInput::kLiteral;
      in.one = v.host_value;
      storage = -1;
    } else if (v.kind == Value::kDense && transposed) {
      if (v.split_inner > 0 || v.reshape_pending) throw RuntimeFailure{"column program operand without a layout"};
      in.kind = ExprInput::kStrided;
      in.offset = v.layout.offset;
      in.strides[0] = row ? v.layout.strides[0] : v.layout.strides[1];
      in.strides[1] = row ? 0 : v.layout.strides[0];
    } else if (transposed) {
      throw RuntimeFailure{"column program operand without a dense value"};
    } else if (v.kind == Value::kDense) {
      in.kind = ExprInput::kStrided;
      in.offset = v.layout.offset;
      for (int d = 0; d < x.rank; ++d) in.strides[d] = v.layout.strides[d];
      if (row) in.strides[p.rank - 1] = 0;
    } else if (v.kind == Value::kSelection && !row) {
      in.kind = ExprInput::kSelection;
      in.one = storages[v.storage].one;
    } else if (v.kind == Value::kPadInline && !row) {
      const Value &src = values[x.operands[0]];
      if (src.kind != Value::kDense) throw RuntimeFailure{"padded input of a non-dense value"};
      in.kind = ExprInput::kPadded;
      in.offset = src.layout.offset;
      for (int d = 0; d < x.rank; ++d) in.strides[d] = src.layout.strides[d];
      in.pad_axis = (int)x.params[0];
      in.pad_start = x.params[1];
      in.pad_len = nodes[x.operands[0]].shape[x.params[0]];
      storage = src.storage;
    } else {
      throw RuntimeFailure{"row program operand without a readable value"};
    }
    p.inputs.push_back(in);
    storage_of.push_back(storage);
    const int index = (int)p.inputs.size() - 1;
    input_of[o] = index;
    return index;
  }

  void plan_row_group(int id) {
    const RowGroup &g = row_groups[id];
    RowProgram p;
    p.rank = g.rank;
    for (int d = 0; d < g.rank; ++d) p.shape[d] = g.shape[d];
    p.transposed_outputs = g.transposed;
    std::vector<int> storage_of;
    std::map<int64_t, int> input_of;
    std::map<int64_t, RowRef> ref_of;
    auto ref = [&](int64_t o) -> RowRef {
      if (group_of[o] == id) return ref_of.at(o);
      return RowRef{RowRef::kInput, row_input(p, storage_of, input_of, o, g.transposed)};
    };
    int zero_input = -1;
    for (int64_t m : g.members) {
      const topos_hip_node &x = nodes[m];
      if (x.op == TOPOS_HIP_OP_BROADCAST_ALONG) {
        ref_of[m] = ref(x.operands[0]);
        continue;
      }
      RowNode rn;
      const bool full = group_full(x, g);
      if (is_elementwise(x.op)) {
        rn.kind = full ? RowNode::kFullOp : RowNode::kRowOp;
        rn.a = ref(x.operands[0]);
        if (x.op == TOPOS_HIP_OP_RELU) {
          if (zero_input < 0) {
            ExprInput zero;
            zero.kind = ExprInput::kLiteral;
            zero.one = 0.0f;  // zero_like of an f32 element: +0
            p.inputs.push_back(zero);
            storage_of.push_back(-1);
            zero_input = (int)p.inputs.size() - 1;
          }
          rn.op = TOPOS_HIP_CHAIN_MAX;
          rn.b = RowRef{RowRef::kInput, zero_input};
        } else {
          rn.op = chain_op(x.op);
          if (is_binary(rn.op)) rn.b = ref(x.operands[1]);
        }
      } else {
        rn.kind = x.op == TOPOS_HIP_OP_SUM_ALONG    ? RowNode::kSum
                  : x.op == TOPOS_HIP_OP_LOG_SUM_EXP ? RowNode::kLogSumExp
                                                     : RowNode::kLogSoftmax;
        rn.a = ref(x.operands[0]);
      }
      p.nodes.push_back(rn);
      ref_of[m] = RowRef{rn.full() ? RowRef::kFull : RowRef::kRow, (int)p.nodes.size() - 1};
    }
    // Members read outside the group (or readable) are written out; a
    // broadcast member read outside is its row operand, viewed.
    auto outside = [&](int64_t m) {
      if (readable[m]) return true;
      for (int c : consumers[m])
        if (group_of[c] != id) return true;
      return false;
    };
    std::map<int64_t, int> full_out, row_out;  // member -> output position
    std::vector<int64_t> broadcast_views;
    for (int64_t m : g.members) {
      if (!outside(m)) continue;
      int64_t w = m;
      if (nodes[m].op == TOPOS_HIP_OP_BROADCAST_ALONG) {
        broadcast_views.push_back(m);
        w = nodes[m].operands[0];
        if (group_of[w] != id) continue;  // an outside operand: already has a value
      }
      const RowRef r = ref_of.at(w);
      if (r.kind == RowRef::kFull && !full_out.count(w)) {
        full_out[w] = (int)p.full_outputs.size();
        p.full_outputs.push_back(r.index);
      } else if (r.kind == RowRef::kRow && !row_out.count(w)) {
        row_out[w] = (int)p.row_outputs.size();
        p.row_outputs.push_back(r.index);
      }
    }
    const int64_t rows = p.rows(), columns = p.columns();
    std::vector<int> full_storage, row_storage, writes;
    for (size_t o = 0; o < p.full_outputs.size(); ++o) {
      full_storage.push_back(arena_storage(rows * columns * 4));
      writes.push_back(full_storage.back());
    }
    for (size_t o = 0; o < p.row_outputs.size(); ++o) {
      row_storage.push_back(arena_storage(rows * 4));
      writes.push_back(row_storage.back());
    }
    Generated gen = generate_row_program(p);
    pending.push_back(gen);
    ++fused_groups;
    int folds = 0;
    for (const RowNode &rn : p.nodes)
      folds += rn.kind == RowNode::kSum ? 1 : (rn.kind == RowNode::kLogSumExp || rn.kind == RowNode::kLogSoftmax) ? 2 : 0;
    std::ostringstream what;
    what << (g.transposed ? "columns [" : "rows [");
    for (int d = 0; d < p.rank; ++d) what << (d ? "," : "") << p.shape[g.transposed ? p.rank - 1 - d : d];
    what << "] " << p.inputs.size() << " inputs, " << p.nodes.size() << " nodes, " << folds << " folds, "
         << p.full_outputs.size() << "+" << p.row_outputs.size() << " outputs";
    add_launch(what.str(), real(storage_of), writes,
               [this, p, gen, storage_of, full_storage, row_storage](const Exec &ex) {
                 auto in = pointers_for(storage_of);
                 std::vector<float *> fo, ro;
                 for (int s : full_storage) fo.push_back((float *)base(s));
                 for (int s : row_storage) ro.push_back((float *)base(s));
                 launch_row_program(gen, p, in.data(), fo.data(), ro.data(), ex.stream);
               });
    {
      Expr e;
      e.rank = p.rank;
      for (int d = 0; d < p.rank; ++d) e.shape[d] = p.shape[d];
      e.inputs = p.inputs;
      account(e, (double)rows * columns * p.full_outputs.size() + (double)rows * p.row_outputs.size());
    }
    int64_t row_shape[kMaxRank];
    for (int d = 0; d + 1 < p.rank; ++d) row_shape[d] = p.shape[d];
    // A transposed program writes its [R, C] nodes row-major.
    Layout full_layout = contiguous(p.rank, p.shape);
    if (g.transposed) {
      const int64_t node_shape[2] = {p.shape[1], p.shape[0]};
      full_layout = contiguous(2, node_shape);
    }
    for (auto &kv : full_out) values[kv.first] = dense_value(full_storage[kv.second], full_layout);
    for (auto &kv : row_out) values[kv.first] = dense_value(row_storage[kv.second], contiguous(p.rank - 1, row_shape));
    for (int64_t b : broadcast_views) {
      const Value &a = values[nodes[b].operands[0]];
      if (g.transposed) {
        Layout l;
        l.rank = 2;
        l.offset = a.layout.offset;
        l.shape[0] = columns;
        l.shape[1] = rows;
        l.strides[0] = 0;
        l.strides[1] = a.layout.strides[0];
        values[b] = view_of(a, l);
        continue;
      }
      Layout l;
      l.rank = p.rank;
      l.offset = a.layout.offset;
      for (int d = 0; d + 1 < p.rank; ++d) {
        l.shape[d] = p.shape[d];
        l.strides[d] = a.layout.strides[d];
      }
      l.shape[p.rank - 1] = columns;
      l.strides[p.rank - 1] = 0;
      values[b] = view_of(a, l);
    }
  }

  // ---- storages ----

  int new_storage(StorageKind kind, int64_t index = -1, int64_t bytes = 0) {
    Storage s;
    s.kind = kind;
    s.index = index;
    s.bytes = bytes;
    storages.push_back(s);
    return (int)storages.size() - 1;
  }
  int arena_storage(int64_t bytes) { return new_storage(StorageKind::kArena, -1, std::max<int64_t>(bytes, 4)); }

  int pool_constant(float v) {
    pool.push_back(v);
    return new_storage(StorageKind::kPool, (int64_t)pool.size() - 1);
  }

  Value dense_value(int storage, const Layout &layout) {
    Value v;
    v.kind = Value::kDense;
    v.storage = storage;
    v.layout = layout;
    return v;
  }

  Value host_constant(const topos_hip_node &x, float value) {
    Value v = dense_value(pool_constant(value), constant_layout(x.rank, x.shape, 0));
    v.constant = true;
    v.host_known = true;
    v.host_value = value;
    return v;
  }

  // A value that reads as `source` in the layout `layout` (views keep the
  // constant flags: a view of a Constant is a Constant).
  Value view_of(const Value &source, const Layout &layout) {
    Value v = source;
    v.layout = layout;
    return v;
  }

  // ---- launches ----

  int add_launch(const std::string &what, std::vector<int> reads, std::vector<int> writes,
                 std::function<void(const Exec &)> run) {
    Launch l{what, std::move(reads), std::move(writes), std::move(run)};
    l.kind = what.substr(0, what.find(' '));
    launches.push_back(std::move(l));
    return (int)launches.size() - 1;
  }

  // Algorithmic bytes of the last launch: each distinct element of a
  // non-literal input read once (a stride-0 axis adds no elements), each
  // output element written once.
  static double distinct_elements(const Expr &e, const ExprInput &in) {
    if (in.kind == ExprInput::kLiteral) return 0;
    if (in.kind == ExprInput::kSelection) return (double)e.shape[0];  // the indices
    double v = 1;
    for (int d = 0; d < e.rank; ++d)
      if (in.strides[d] != 0) v *= (double)(in.kind == ExprInput::kPadded && d == in.pad_axis ? in.pad_len : e.shape[d]);
    return v;
  }
  void account(const Expr &e, double outputs, double flops = 0) {
    double reads = 0;
    for (const ExprInput &in : e.inputs) reads += distinct_elements(e, in);
    launches.back().bytes = 4.0 * (reads + outputs);
    launches.back().flops = flops;
  }

  // Pointer resolution at run time.
  char *base(int storage_id) const {
    const Storage &s = storages[storage_id];
    switch (s.kind) {
      case StorageKind::kArena: return arena + s.offset;
      case StorageKind::kParameter: {
        auto it = parameters.find(s.index);
        if (it == parameters.end()) throw InvalidArgument{"parameter slot " + std::to_string(s.index) + " is not bound"};
        return (char *)it->second;
      }
      case StorageKind::kInput: {
        auto it = inputs.find(s.index);
        if (it == inputs.end()) throw InvalidArgument{"input slot " + std::to_string(s.index) + " is not bound"};
        return (char *)it->second;
      }
      case StorageKind::kPool: return (char *)(constants + s.index);
      case StorageKind::kLeaf: return (char *)(constants + leaf_data_offset + s.index);
      case StorageKind::kSelectionInput: {
        auto it = selection_inputs.find(s.index);
        if (it == selection_inputs.end())
          throw InvalidArgument{"selection input slot " + std::to_string(s.index) + " is not bound"};
        return (char *)it->second.indices;
      }
      case StorageKind::kSelectionLeaf: return (char *)selection_leaves.at(s.index).indices;
    }
    return nullptr;
  }

  const SelectionBuffers &selection_buffers(int storage_id) const {
    const Storage &s = storages[storage_id];
    if (s.kind == StorageKind::kSelectionInput) {
      auto it = selection_inputs.find(s.index);
      if (it == selection_inputs.end())
        throw InvalidArgument{"selection input slot " + std::to_string(s.index) + " is not bound"};
      return it->second;
    }
    return selection_leaves.at(s.index);
  }

  // ---- expressions ----

  bool is_inline(int64_t i) const { return values[i].kind == Value::kInline; }

  // Appends node `i`'s expression (its inlined subtree) to `e`, returning its
  // reference. `memo` maps nodes to references, `inputs_of` maps leaf nodes to
  // input positions, `storage_of` lists each input's storage.
  int expr_of(int64_t i, Expr &e, std::map<int64_t, int> &memo, std::vector<int> &storage_of,
              int64_t compute_root = -1) {
    auto found = memo.find(i);
    if (found != memo.end()) return found->second;
    const topos_hip_node &x = nodes[i];
    const Value &v = values[i];
    int result;
    if (v.kind == Value::kInline || i == compute_root) {
      // An elementwise node computed in registers.
      const int a = expr_of(x.operands[0], e, memo, storage_of);
      int b = 0;
      int op;
      if (x.op == TOPOS_HIP_OP_RELU) {
        ExprInput zero;
        zero.kind = ExprInput::kLiteral;
        zero.one = 0.0f;  // zero_like of an f32 element: +0
        e.inputs.push_back(zero);
        storage_of.push_back(-1);
        b = -(int)e.inputs.size();
        op = TOPOS_HIP_CHAIN_MAX;
      } else {
        op = chain_op(x.op);
        if (is_binary(op)) b = expr_of(x.operands[1], e, memo, storage_of);
      }
      e.steps.push_back(ExprStep{op, a, b});
      result = (int)e.steps.size() - 1;
    } else {
      if (v.split_inner > 0) throw RuntimeFailure{"a merged-batch view read by a generated expression"};
      ExprInput in;
      int storage = v.storage;
      if (v.kind == Value::kDense && v.host_known) {
        in.kind = ExprInput::kLiteral;
        in.one = v.host_value;
        storage = -1;
      } else if (v.kind == Value::kDense) {
        in.kind = ExprInput::kStrided;
        in.offset = v.layout.offset;
        for (int d = 0; d < e.rank; ++d) in.strides[d] = v.layout.strides[d];
      } else if (v.kind == Value::kSelection) {
        in.kind = ExprInput::kSelection;
        in.one = storages[v.storage].one;
      } else if (v.kind == Value::kPadInline) {
        const Value &src = values[x.operands[0]];
        if (src.kind != Value::kDense) throw RuntimeFailure{"padded input of a non-dense value"};
        // (A window of a host-known constant reads its pool element through
        // zero strides.)
        in.kind = ExprInput::kPadded;
        in.offset = src.layout.offset;
        for (int d = 0; d < e.rank; ++d) in.strides[d] = src.layout.strides[d];
        in.pad_axis = (int)x.params[0];
        in.pad_start = x.params[1];
        in.pad_len = nodes[x.operands[0]].shape[x.params[0]];
        storage = src.storage;
      } else {
        throw RuntimeFailure{"expression leaf without a value"};
      }
      e.inputs.push_back(in);
      storage_of.push_back(storage);
      result = -(int)e.inputs.size();
    }
    memo[i] = result;
    return result;
  }

  Expr expression_for(int64_t root, std::vector<int> &storage_of) {
    Expr e;
    const topos_hip_node &x = nodes[root];
    e.rank = x.rank;
    for (int d = 0; d < x.rank; ++d) e.shape[d] = x.shape[d];
    std::map<int64_t, int> memo;
    e.outputs.push_back(expr_of(root, e, memo, storage_of, root));
    return e;
  }

  std::vector<const void *> pointers_for(const std::vector<int> &storage_of) const {
    std::vector<const void *> p(storage_of.size(), nullptr);
    for (size_t i = 0; i < storage_of.size(); ++i)
      if (storage_of[i] >= 0) p[i] = base(storage_of[i]);
    return p;
  }

  static std::vector<int> real(const std::vector<int> &storage_of) {
    std::vector<int> r;
    for (int s : storage_of)
      if (s >= 0) r.push_back(s);
    return r;
  }

  std::string describe_expr(const Expr &e) const {
    std::ostringstream s;
    s << "[";
    for (int d = 0; d < e.rank; ++d) s << (d ? "," : "") << e.shape[d];
    s << "] " << e.inputs.size() << " inputs, " << e.steps.size() << " steps";
    return s.str();
  }

  // A generated chain computing node `root` (and its inlined subtree) into a
  // fresh contiguous arena buffer.
  Value emit_chain(int64_t root) {
    std::vector<int> storage_of;
    Expr e = expression_for(root, storage_of);
    const int out = arena_storage(e.volume() * 4);
    const topos_hip_node &n = nodes[root];
    if (join_open_chain(e, storage_of, out, op_name(n.op))) return dense_value(out, contiguous(n.rank, n.shape));
    auto record = std::make_shared<ChainRecord>();
    record->e = e;
    record->storage_of = storage_of;
    record->outs = {out};
    record->ops = op_name(n.op);
    ++fused_groups;
    add_launch(std::string("chain ") + record->ops + " " + describe_expr(e), real(storage_of), {out},
               [this, record](const Exec &x) {
                 auto p = pointers_for(record->storage_of);
                 std::vector<float *> q;
                 for (int o : record->outs) q.push_back((float *)base(o));
                 launch_generated_chain(record->g, record->e, p.data(), q.data(), x.stream);
               });
    account(e, (double)e.volume());
    record->launch = (int)launches.size() - 1;
    chains.push_back(record);
    open_chain = record;
    return dense_value(out, contiguous(n.rank, n.shape));
  }

  // Generates every chain's source. A joined chain's output that no other
  // launch reads and no readable value keeps stays in registers (it was
  // written only for the members that joined after it).
  void finish_chains() {
    std::vector<int> readers(storages.size(), 0);
    for (const Launch &l : launches)
      for (int r : l.reads) ++readers[r];
    for (auto &record : chains) {
      Launch &l = launches[record->launch];
      Expr &e = record->e;
      std::vector<int> kept_outputs, kept_storages;
      for (size_t k = 0; k < record->outs.size(); ++k) {
        const int o = record->outs[k];
        if (readers[o] > 0 || storages[o].pinned || k + 1 == record->outs.size()) {
          kept_outputs.push_back(e.outputs[k]);
          kept_storages.push_back(o);
        }
      }
      if (kept_storages.size() != record->outs.size()) {
        e.outputs = kept_outputs;
        record->outs = kept_storages;
        l.writes = kept_storages;
        double reads = 0;
        for (const ExprInput &in : e.inputs) reads += distinct_elements(e, in);
        l.bytes = 4.0 * (reads + (double)e.volume() * (double)e.outputs.size());
        l.what = "chain " + record->ops + " " + describe_expr(e) + ", " + std::to_string(e.outputs.size()) +
                 " outputs";
      }
      record->g = generate_chain(e);
      pending.push_back(record->g);
    }
  }

  static bool same_input(const ExprInput &a, const ExprInput &b, int rank) {
    if (a.kind != b.kind || a.offset != b.offset) return false;
    if (a.kind == ExprInput::kLiteral || a.kind == ExprInput::kSelection)
      return __builtin_bit_cast(uint32_t, a.one) == __builtin_bit_cast(uint32_t, b.one);
    for (int d = 0; d < rank; ++d)
      if (a.strides[d] != b.strides[d]) return false;
    return a.kind != ExprInput::kPadded ||
           (a.pad_axis == b.pad_axis && a.pad_start == b.pad_start && a.pad_len == b.pad_len);
  }

  // Joins chain `e` (writing `out`) to the open chain when that chain is the
  // last launch, iterates the same shape, and every input of `e` is either
  // complete before it or one of its outputs read in its own layout (then
  // the joined expression takes the value from registers). The operations
  // and their order per element are unchanged, so are the bits.
  bool join_open_chain(const Expr &e, const std::vector<int> &storage_of, int out, const std::string &op) {
    auto record = open_chain;
    if (!record || record->launch != (int)launches.size() - 1) return false;
    Expr m = record->e;
    if (m.rank != e.rank || m.outputs.size() >= 8) return false;
    for (int d = 0; d < e.rank; ++d)
      if (m.shape[d] != e.shape[d]) return false;
    const Layout whole = contiguous(e.rank, e.shape);
    std::vector<int> so = record->storage_of;
    std::vector<int> mapped(e.inputs.size());
    for (size_t j = 0; j < e.inputs.size(); ++j) {
      const ExprInput &in = e.inputs[j];
      const int storage = storage_of[j];
      int produced = -1;
      for (size_t k = 0; k < record->outs.size(); ++k)
        if (storage >= 0 && record->outs[k] == storage) produced = (int)k;
      if (produced >= 0) {
        if (in.kind != ExprInput::kStrided || in.offset != 0) return false;
        for (int d = 0; d < e.rank; ++d)
          if (e.shape[d] != 1 && in.strides[d] != whole.strides[d]) return false;
        mapped[j] = m.outputs[produced];
        continue;
      }
      int found = -1;
      for (size_t i = 0; i < m.inputs.size() && found < 0; ++i)
        if (so[i] == storage && same_input(m.inputs[i], in, e.rank)) found = (int)i;
      if (found < 0) {
        m.inputs.push_back(in);
        so.push_back(storage);
        found = (int)m.inputs.size() - 1;
      }
      mapped[j] = -(found + 1);
    }
    if (m.inputs.size() > 24) return false;
    const int shift = (int)m.steps.size();
    auto remap = [&](int r) { return r >= 0 ? r + shift : mapped[-r - 1]; };
    for (const ExprStep &x : e.steps)
      m.steps.push_back(ExprStep{x.op, remap(x.left), is_binary(x.op) ? remap(x.right) : x.right});
    m.outputs.push_back(remap(e.outputs[0]));
    record->e = m;
    record->storage_of = so;
    record->outs.push_back(out);
    record->ops += "+" + op;
    Launch &l = launches[record->launch];
    l.reads = real(so);
    l.writes = record->outs;
    l.what = "chain " + record->ops + " " + describe_expr(m) + ", " + std::to_string(m.outputs.size()) + " outputs";
    double reads = 0;
    for (const ExprInput &in : m.inputs) reads += distinct_elements(m, in);
    l.bytes = 4.0 * (reads + (double)m.volume() * (double)m.outputs.size());
    return true;
  }

  // Copies any dense/constant value into a fresh contiguous buffer.
  Value materialize(int64_t i) {
    const Value &v = values[i];
    const topos_hip_node &n = nodes[i];
    if (v.kind == Value::kSelection) {
      const int out = arena_storage(volume_of(n) * 4);
      const int sel = v.storage;
      const float one = storages[sel].one;
      const int64_t rows = n.shape[0], vocab = n.shape[1];
      add_launch("one-hot " + std::to_string(rows) + "x" + std::to_string(vocab), {sel}, {out},
                 [this, sel, out, rows, vocab, one](const Exec &x) {
                   launch_one_hot((const int32_t *)base(sel), rows, vocab, one, (float *)base(out), x.stream);
                 });
      return dense_value(out, contiguous(n.rank, n.shape));
    }
    if (v.kind != Value::kDense) throw RuntimeFailure{"materialising a value without storage"};
    if (v.reshape_pending) throw RuntimeFailure{"materialising a pending reshape"};
    Expr e;
    e.rank = n.rank;
    for (int d = 0; d < n.rank; ++d) e.shape[d] = n.shape[d];
    ExprInput in;
    std::vector<int> storage_of;
    if (v.split_inner > 0) {
      // The merged axis copied as its two axes (the same element order).
      e.rank = n.rank + 1;
      e.shape[0] = n.shape[0] / v.split_inner;
      e.shape[1] = v.split_inner;
      for (int d = 1; d < n.rank; ++d) e.shape[d + 1] = n.shape[d];
      in.offset = v.layout.offset;
      in.strides[0] = v.split_outer_stride;
      in.strides[1] = v.split_inner_stride;
      for (int d = 1; d < n.rank; ++d) in.strides[d + 1] = v.layout.strides[d];
      storage_of.push_back(v.storage);
    } else if (v.host_known) {
      in.kind = ExprInput::kLiteral;
      in.one = v.host_value;
      storage_of.push_back(-1);
    } else {
      in.offset = v.layout.offset;
      for (int d = 0; d < n.rank; ++d) in.strides[d] = v.layout.strides[d];
      storage_of.push_back(v.storage);
    }
    e.inputs.push_back(in);
    e.outputs.push_back(-1);
    const int out = arena_storage(e.volume() * 4);
    if (transposing_copy(e)) {
      Generated g = generate_transpose_copy(e);
      pending.push_back(g);
      add_launch("copy (tiles) " + describe_expr(e), real(storage_of), {out},
                 [this, e, g, storage_of, out](const Exec &x) {
                   auto p = pointers_for(storage_of);
                   launch_transpose_copy(g, e, p[0], (float *)base(out), x.stream);
                 });
      account(e, (double)e.volume());
      return dense_value(out, contiguous(n.rank, n.shape));
    }
    Generated g = generate_chain(e);
    pending.push_back(g);
    add_launch("copy " + describe_expr(e), real(storage_of), {out}, [this, e, g, storage_of, out](const Exec &x) {
      auto p = pointers_for(storage_of);
      float *q = (float *)base(out);
      launch_generated_chain(g, e, p.data(), &q, x.stream);
    });
    account(e, (double)e.volume());
    return dense_value(out, contiguous(n.rank, n.shape));
  }

  // Reshape i copies a permuted view of a matrix-core product's output that
  // nothing else reads (attention heads merged back into rows): the product
  // writes straight into the reshape's contiguous layout instead, through
  // its row and two-level batch strides, and the reshape is a view of that.
  bool retarget_product(int64_t source, int64_t i, Value &out) {
    const Value &v = values[source];
    if (numerics != TOPOS_HIP_FAST || v.kind != Value::kDense || v.split_inner > 0 || v.layout.offset != 0)
      return false;
    auto found = product_of_storage.find(v.storage);
    if (found == product_of_storage.end()) return false;
    const int64_t product = found->second;
    ProductLaunch &record = product_launch.at(product);
    if (!record.flat || record.bias->storage >= 0) return false;
    // Views, and +0 + v planned as v itself (the zero-seeded gradient
    // accumulation), between the product and the reshape.
    for (int64_t node = product; node != i;) {
      if (readable[node] || consumers[node].size() != 1) return false;
      const int64_t from = node;
      node = consumers[node][0];
      const topos_hip_node &y = nodes[node];
      if (node == i || y.op == TOPOS_HIP_OP_RESHAPE || y.op == TOPOS_HIP_OP_PERMUTE) continue;
      const bool identity = y.op == TOPOS_HIP_OP_ADD &&
                            static_plus_zero(y.operands[0] == from ? y.operands[1] : y.operands[0]) &&
                            values[node].kind == Value::kDense && values[node].storage == v.storage;
      if (!identity) return false;
    }
    const topos_hip_node &p = nodes[product];
    if (p.rank != 3) return false;
    const int64_t count = p.shape[0], m = p.shape[1], n = p.shape[2];
    const Layout &l = v.layout;
    const Layout target = contiguous(l.rank, l.shape);
    int col = -1, row = -1, outer = -1, inner_axis = -1;
    for (int d = 0; d < l.rank; ++d) {
      if (l.shape[d] == 1) continue;
      if (l.strides[d] == 1 && l.shape[d] == n && col < 0) col = d;
      else if (l.strides[d] == n && l.shape[d] == m && row < 0) row = d;
      else if (l.strides[d] == m * n && inner_axis < 0) inner_axis = d;
      else if (outer < 0) outer = d;
      else return false;
    }
    if (col != l.rank - 1 || row < 0 || (n > 1 && col < 0)) return false;
    int64_t inner = 1, c_stride = 0, c_inner = 0;
    if (outer >= 0) {
      // Two batch axes: (y / inner) along `outer`, (y % inner) along `inner_axis`.
      if (inner_axis < 0) return false;
      inner = l.shape[inner_axis];
      if (l.strides[outer] != inner * m * n || l.shape[outer] * inner != count) return false;
      c_stride = target.strides[outer];
      c_inner = target.strides[inner_axis];
    } else if (inner_axis >= 0) {
      if (l.shape[inner_axis] != count) return false;
      c_stride = target.strides[inner_axis];
    } else if (count != 1) {
      return false;
    }
    Batch batch = record.output->batch;
    if (inner > 1) {
      if (batch.inner == 1) {
        batch.a_inner = batch.a_stride;
        batch.a_stride *= inner;
        batch.b_inner = batch.b_stride;
        batch.b_stride *= inner;
        batch.inner = inner;
      } else if (batch.inner != inner) {
        return false;
      }
      batch.c_stride = c_stride;
      batch.c_inner = c_inner;
    } else {
      if (batch.inner != 1) return false;
      batch.c_stride = c_stride;
    }
    const int storage = arena_storage(count * m * n * 4);
    record.output->storage = storage;
    record.output->ldc = target.strides[row];
    record.output->batch = batch;
    for (int &w : launches[record.launch].writes)
      if (w == v.storage) w = storage;
    product_of_storage.erase(found);
    const topos_hip_node &x = nodes[i];
    out = dense_value(storage, contiguous(x.rank, x.shape));
    out.never_minus_zero = true;
    return true;
  }

  // Makes node i's value usable as a strided dense operand.
  // Node i, a reshape of a value laid out as `from`, is read only by
  // narrows, each of which narrow_reshape_view resolves to a view of `from`.
  bool narrows_view_through(int64_t i, const Layout &from) const {
    if (readable[i] || consumers[i].empty()) return false;
    const topos_hip_node &x = nodes[i];
    for (int c : consumers[i]) {
      const topos_hip_node &y = nodes[c];
      Layout l;
      if (y.op != TOPOS_HIP_OP_NARROW ||
          !narrow_reshape_view(from, x.rank, x.shape, (int)y.params[0], y.params[1], y.params[2], l))
        return false;
    }
    return true;
  }

  const Value &dense_operand(int64_t i) {
    if (values[i].kind == Value::kSelection || values[i].split_inner > 0) values[i] = materialize(i);
    return values[i];
  }

  // A constant +0 known from the graph alone (a +0 Constant leaf, or a view
  // of one): the zero_like seed of recorded gradient accumulations.
  bool static_plus_zero(int64_t j) const {
    const topos_hip_node &x = nodes[j];
    if (x.op == TOPOS_HIP_OP_LEAF) {
      const topos_hip_leaf &leaf = leaves[x.slot];
      return leaf.kind == TOPOS_HIP_LEAF_CONSTANT && __builtin_bit_cast(uint32_t, leaf.value) == 0;
    }
    if (x.op == TOPOS_HIP_OP_BROADCAST || x.op == TOPOS_HIP_OP_BROADCAST_ALONG || x.op == TOPOS_HIP_OP_RESHAPE ||
        x.op == TOPOS_HIP_OP_PERMUTE || x.op == TOPOS_HIP_OP_TRANSPOSE)
      return static_plus_zero(x.operands[0]);
    return false;
  }

  // Node i is read only by products, directly or through permutations that
  // keep axis 0 first, or through +0 + i when i has no -0 element (planned
  // as i itself); and nothing reads it from the host.
  bool feeds_products_only(int64_t i, bool never_minus_zero) const {
    if (readable[i]) return false;
    for (int c : consumers[i]) {
      const topos_hip_node &x = nodes[c];
      if (x.op == TOPOS_HIP_OP_MATMUL && x.rank == 3) continue;
      if (x.op == TOPOS_HIP_OP_PERMUTE && x.params[0] == 0 && feeds_products_only(c, never_minus_zero)) continue;
      if (x.op == TOPOS_HIP_OP_ADD && never_minus_zero && group_of[c] < 0) {
        const int64_t other = x.operands[0] == i ? x.operands[1] : x.operands[0];
        if (other != i && static_plus_zero(other) && feeds_products_only(c, never_minus_zero)) continue;
      }
      return false;
    }
    return !consumers[i].empty();
  }

  // ---- the node loop ----

  bool inline_candidate(int64_t i) const {
    if (readable[i] || consumers[i].size() != 1) return false;
    const topos_hip_node &c = nodes[consumers[i][0]];
    return is_elementwise(c.op) || c.op == TOPOS_HIP_OP_SUM_ALONG || c.op == TOPOS_HIP_OP_SUM;
  }

  void plan_node(int64_t i) {
    const topos_hip_node &x = nodes[i];
    Value &out = values[i];
    switch (x.op) {
      case TOPOS_HIP_OP_LEAF: {
        const topos_hip_leaf &leaf = leaves[x.slot];
        if (leaf.kind == TOPOS_HIP_LEAF_CONSTANT) {
          out = host_constant(x, leaf.value);
        } else if (leaf.kind == TOPOS_HIP_LEAF_DENSE) {
          out = dense_value(new_storage(StorageKind::kLeaf, leaf.offset), contiguous(x.rank, x.shape));
        } else {
          const int s = new_storage(StorageKind::kSelectionLeaf, x.slot);
          storages[s].rows = x.shape[0];
          storages[s].vocab = x.shape[1];
          storages[s].one = leaf.value;
          out.kind = Value::kSelection;
          out.storage = s;
        }
        return;
      }
      case TOPOS_HIP_OP_PARAMETER: {
        auto it = parameter_storage.find(x.slot);
        const int s = it != parameter_storage.end() ? it->second
                                                    : (parameter_storage[x.slot] = new_storage(StorageKind::kParameter, x.slot));
        out = dense_value(s, contiguous(x.rank, x.shape));
        return;
      }
      case TOPOS_HIP_OP_INPUT: {
        if (x.flags & TOPOS_HIP_NODE_SELECTION) {
          const int s = new_storage(StorageKind::kSelectionInput, x.slot);
          storages[s].rows = x.shape[0];
          storages[s].vocab = x.shape[1];
          storages[s].one = __builtin_bit_cast(float, (uint32_t)x.params[0]);
          out.kind = Value::kSelection;
          out.storage = s;
          return;
        }
        auto it = input_storage.find(x.slot);
        const int s = it != input_storage.end() ? it->second
                                                : (input_storage[x.slot] = new_storage(StorageKind::kInput, x.slot));
        out = dense_value(s, contiguous(x.rank, x.shape));
        return;
      }
      case TOPOS_HIP_OP_TRANSPOSE: {
        if (values[x.operands[0]].kind == Value::kWindow) {
          out = values[x.operands[0]];
          out.window_transposed = !out.window_transposed;
          out.layout = contiguous(x.rank, x.shape);
          return;
        }
        const Value &a = dense_operand(x.operands[0]);
        Layout l = a.layout;
        if (l.rank == 2) {
          std::swap(l.shape[0], l.shape[1]);
          std::swap(l.strides[0], l.strides[1]);
        }
        out = view_of(a, l);
        return;
      }
      case TOPOS_HIP_OP_PERMUTE: {
        if (values[x.operands[0]].split_inner > 0 && x.params[0] == 0) {
          Value v = values[x.operands[0]];
          Layout l = v.layout;
          for (int d = 1; d < x.rank; ++d) {
            l.shape[d] = v.layout.shape[x.params[d]];
            l.strides[d] = v.layout.strides[x.params[d]];
          }
          v.layout = l;
          out = v;
          return;
        }
        const Value &a = dense_operand(x.operands[0]);
        Layout l = a.layout;
        for (int d = 0; d < x.rank; ++d) {
          l.shape[d] = a.layout.shape[x.params[d]];
          l.strides[d] = a.layout.strides[x.params[d]];
        }
        out = view_of(a, l);
        return;
      }
      case TOPOS_HIP_OP_NARROW: {
        const int axis = (int)x.params[0];
        if (values[x.operands[0]].reshape_pending) {
          const Value &a = values[x.operands[0]];
          const topos_hip_node &r = nodes[x.operands[0]];
          Layout l;
          if (!narrow_reshape_view(a.layout, r.rank, r.shape, axis, x.params[1], x.params[2], l))
            throw RuntimeFailure{"a narrow of a pending reshape is no view"};
          out = view_of(a, l);
          out.reshape_pending = false;
          return;
        }
        const Value &a = dense_operand(x.operands[0]);
        Layout l = a.layout;
        l.shape[axis] = x.params[2];
        l.offset += x.params[1] * l.strides[axis];
        out = view_of(a, l);
        return;
      }
      case TOPOS_HIP_OP_BROADCAST: {
        const Value &a = dense_operand(x.operands[0]);
        out = view_of(a, constant_layout(x.rank, x.shape, a.layout.offset));
        out.constant = true;
        return;
      }
      case TOPOS_HIP_OP_BROADCAST_ALONG: {
        const Value &a = dense_operand(x.operands[0]);
        const int axis = (int)x.params[0];
        Layout l;
        l.rank = x.rank;
        l.offset = a.layout.offset;
        for (int d = 0, e = 0; d < x.rank; ++d) {
          l.shape[d] = x.shape[d];
          l.strides[d] = d == axis ? 0 : a.layout.strides[e++];
        }
        out = view_of(a, l);
        return;
      }
      case TOPOS_HIP_OP_RESHAPE: {
        const Value &a = dense_operand(x.operands[0]);
        if (a.constant) {
          out = view_of(a, constant_layout(x.rank, x.shape, a.layout.offset));
          return;
        }
        Layout l;
        if (reshape_view(a.layout, x.rank, x.shape, l)) {
          out = view_of(a, l);
          return;
        }
        // Merging the two leading axes of a rank-4 view that only products
        // read (attention heads as one batch axis): the products take the two
        // strides themselves, with no copy.
        const Layout &al = a.layout;
        if (numerics == TOPOS_HIP_FAST && al.rank == 4 && x.rank == 3 && x.shape[0] == al.shape[0] * al.shape[1] &&
            x.shape[1] == al.shape[2] && x.shape[2] == al.shape[3] && al.shape[1] > 1 &&
            feeds_products_only(i, a.never_minus_zero)) {
          Value v = a;
          v.layout.rank = 3;
          v.layout.shape[0] = x.shape[0];
          v.layout.strides[0] = 0;
          for (int d = 1; d < 3; ++d) {
            v.layout.shape[d] = al.shape[d + 1];
            v.layout.strides[d] = al.strides[d + 1];
          }
          v.layout.shape[3] = 1;
          v.layout.strides[3] = 0;
          v.split_inner = al.shape[1];
          v.split_outer_stride = al.strides[0];
          v.split_inner_stride = al.strides[1];
          out = v;
          return;
        }
        if (retarget_product(x.operands[0], i, out)) return;
        // Read only by narrows that are each a view of the operand (the lanes
        // of a max-pool window): no copy, the narrows view the operand.
        if (narrows_view_through(i, a.layout)) {
          out = a;
          out.reshape_pending = true;
          return;
        }
        // Not a view (layout.rs reshape answers None): the interpreter copies
        // the elements out in logical order.
        Value copied = materialize(x.operands[0]);
        out = view_of(copied, contiguous(x.rank, x.shape));
        return;
      }
      case TOPOS_HIP_OP_UNFOLD: {
        // Layout::unfold (src/payload/layout.rs:299-331): the axis becomes
        // (count, size) with window starts `step` and window elements
        // `dilation` source steps apart; an extent-1 axis gets stride 0.
        const Value &a = dense_operand(x.operands[0]);
        const int axis = (int)x.params[0];
        const int64_t along = a.layout.strides[axis];
        Layout l;
        l.rank = x.rank;
        l.offset = a.layout.offset;
        for (int d = 0; d < x.rank; ++d) {
          l.shape[d] = x.shape[d];
          if (d < axis) l.strides[d] = a.layout.strides[d];
          if (d > axis + 1) l.strides[d] = a.layout.strides[d - 1];
        }
        if (x.shape[axis] > 1 && __builtin_mul_overflow(x.params[2], along, &l.strides[axis]))
          refuse(i, "unfold stride overflows");
        if (x.shape[axis + 1] > 1 && __builtin_mul_overflow(x.params[3], along, &l.strides[axis + 1]))
          refuse(i, "unfold stride overflows");
        out = view_of(a, l);
        return;
      }
      default:
        break;
    }
    if (is_elementwise(x.op)) {
      plan_elementwise(i);
      return;
    }
    switch (x.op) {
      case TOPOS_HIP_OP_PAD: plan_pad(i); return;
      case TOPOS_HIP_OP_MATMUL: plan_matmul(i); return;
      case TOPOS_HIP_OP_SUM_ALONG: plan_sum_along(i); return;
      case TOPOS_HIP_OP_SUM: plan_sum(i); return;
      case TOPOS_HIP_OP_LOG_SOFTMAX:
      case TOPOS_HIP_OP_LOG_SUM_EXP: plan_rows(i); return;
      case TOPOS_HIP_OP_GATHER: plan_gather(i); return;
      case TOPOS_HIP_OP_SCATTER: plan_scatter(i); return;
      case TOPOS_HIP_OP_FOLD: plan_fold(i); return;
    }
    refuse(i, "no plan for this operation");
  }

  void plan_elementwise(int64_t i) {
    const topos_hip_node &x = nodes[i];
    const int k = arity(x.op);
    bool all_constant = true, all_known = true;
    for (int j = 0; j < k; ++j) {
      const Value &a = values[x.operands[j]];
      if (!(a.kind == Value::kDense && a.constant)) all_constant = false;
      if (!(a.kind == Value::kDense && a.host_known)) all_known = false;
    }
    if (all_known) {
      const float a = values[x.operands[0]].host_value;
      const float b = k > 1 ? values[x.operands[1]].host_value : 0.0f;
      values[i] = host_constant(x, fold_scalar(x.op, a, b));
      return;
    }
    // +0 + v (or v + +0) of a value with no -0 element is v itself: the
    // addition only maps -0 to +0. Matrix-core products are never -0, nor are
    // views of them (the zero-seeded gradient accumulation behind every
    // backward product, and behind the views its gradient flows through).
    if (x.op == TOPOS_HIP_OP_ADD) {
      for (int side = 0; side < 2; ++side) {
        const Value &zero = values[x.operands[side]];
        const Value &v = values[x.operands[1 - side]];
        if (zero.kind == Value::kDense && zero.host_known && __builtin_bit_cast(uint32_t, zero.host_value) == 0 &&
            v.kind == Value::kDense && v.never_minus_zero) {
          values[i] = v;
          return;
        }
      }
    }
    if (x.op == TOPOS_HIP_OP_ADD && fuse_bias(i)) return;
    if (all_constant) {
      // A Constant payload computed at run time: one element, rank 0.
      Expr e;
      e.rank = 0;
      std::vector<int> storage_of;
      std::map<int64_t, int> memo;
      int refs[2] = {0, 0};
      for (int j = 0; j < k; ++j) {
        const Value &a = values[x.operands[j]];
        ExprInput in;
        if (a.host_known) {
          in.kind = ExprInput::kLiteral;
          in.one = a.host_value;
          storage_of.push_back(-1);
        } else {
          in.offset = a.layout.offset;
          storage_of.push_back(a.storage);
        }
        e.inputs.push_back(in);
        refs[j] = -(int)e.inputs.size();
      }
      if (x.op == TOPOS_HIP_OP_RELU) {
        ExprInput zero;
        zero.kind = ExprInput::kLiteral;
        zero.one = 0.0f;
        e.inputs.push_back(zero);
        storage_of.push_back(-1);
        e.steps.push_back(ExprStep{TOPOS_HIP_CHAIN_MAX, refs[0], -(int)e.inputs.size()});
      } else {
        e.steps.push_back(ExprStep{chain_op(x.op), refs[0], refs[1]});
      }
      e.outputs.push_back(0);
      const int out = arena_storage(4);
      Generated g = generate_chain(e);
      pending.push_back(g);
    pending.push_back(g);
      add_launch(std::string("scalar ") + op_name(x.op), real(storage_of), {out},
                 [this, e, g, storage_of, out](const Exec &ex) {
                   auto p = pointers_for(storage_of);
                   float *q = (float *)base(out);
                   launch_generated_chain(g, e, p.data(), &q, ex.stream);
                 });
      values[i] = dense_value(out, constant_layout(x.rank, x.shape, 0));
      values[i].constant = true;
      return;
    }
    if (inline_candidate(i)) {
      values[i].kind = Value::kInline;
      return;
    }
    values[i].kind = Value::kNone;  // the root of its own expression
    values[i] = emit_chain(i);
  }

  // product + bias (or bias + product), the bias repeated along every axis
  // but the last (Linear::express, src/neural/linear.rs:94-105): the
  // matrix-core kernel that writes the product adds the bias in its store,
  // the same one f32 addition. Served when the product is read by this
  // addition only and the bias is complete before the product's launch.
  bool fuse_bias(int64_t i) {
    const topos_hip_node &x = nodes[i];
    for (int side = 0; side < 2; ++side) {
      const int64_t p = x.operands[side], q = x.operands[1 - side];
      auto it = product_launch.find(p);
      if (it == product_launch.end() || !mfma_product[p] || readable[p] || consumers[p].size() != 1 ||
          it->second.bias->storage >= 0)
        continue;
      const Value &b = values[q];
      if (b.kind != Value::kDense || b.storage < 0 || b.layout.rank != x.rank) continue;
      bool repeated = true;
      for (int d = 0; d + 1 < x.rank; ++d) repeated = repeated && b.layout.strides[d] == 0;
      if (!repeated) continue;
      const int l = it->second.launch;
      bool ready = true;
      for (size_t later = l; later < launches.size(); ++later)
        for (int w : launches[later].writes) ready = ready && w != b.storage;
      if (!ready) continue;
      BiasEpilogue &e = *it->second.bias;
      e.storage = b.storage;
      e.offset = b.layout.offset;
      e.stride = b.layout.strides[x.rank - 1];
      e.first = side == 1;
      launches[l].reads.push_back(b.storage);
      launches[l].what += e.first ? " bias+" : " +bias";
      launches[l].bytes += 4.0 * (double)x.shape[x.rank - 1];
      values[i] = values[p];
      values[i].never_minus_zero = false;
      return true;
    }
    return false;
  }

  void plan_pad(int64_t i) {
    const topos_hip_node &x = nodes[i];
    dense_operand(x.operands[0]);
    if (!readable[i] && consumers[i].size() == 1 && is_elementwise(nodes[consumers[i][0]].op)) {
      values[i].kind = Value::kPadInline;
      return;
    }
    // Materialised: a chain whose one input is the padded window.
    values[i].kind = Value::kPadInline;
    std::vector<int> storage_of;
    Expr e;
    e.rank = x.rank;
    for (int d = 0; d < x.rank; ++d) e.shape[d] = x.shape[d];
    std::map<int64_t, int> memo;
    e.outputs.push_back(expr_of(i, e, memo, storage_of));
    const int out = arena_storage(e.volume() * 4);
    Generated g = generate_chain(e);
    pending.push_back(g);
    add_launch("pad " + describe_expr(e), real(storage_of), {out}, [this, e, g, storage_of, out](const Exec &ex) {
      auto p = pointers_for(storage_of);
      float *q = (float *)base(out);
      launch_generated_chain(g, e, p.data(), &q, ex.stream);
    });
    account(e, (double)e.volume());
    values[i] = dense_value(out, contiguous(x.rank, x.shape));
  }

  // Flattens the batch axes of a rank >= 3 operand to one stride when the
  // layout allows it.
  static bool batch_stride(const Layout &l, int batch_axes, int64_t &stride) {
    if (batch_axes == 0) {
      stride = 0;
      return true;
    }
    for (int d = 0; d + 1 < batch_axes; ++d)
      if (l.shape[d + 1] != 1 && l.strides[d] != l.shape[d + 1] * l.strides[d + 1]) return false;
    stride = l.strides[batch_axes - 1];
    return true;
  }

  // A rank-2 product read only through a transpose (the tied embedding's
  // gradient (h^T dlogits)^T): computed as B^T A^T into [n, m], so the
  // transpose is the contiguous layout its reader wants instead of a
  // column-strided one. Every output element is the same chain of the same
  // products in the same ascending k order (a * b = b * a in IEEE
  // arithmetic), so the exact posture keeps its bits.
  // Under Fast the product may also reach the transpose through zero-seeded
  // accumulations (+0 + product), which are planned as the product itself
  // because a matrix-core product is never -0.
  bool read_transposed(int64_t i) const {
    const topos_hip_node &x = nodes[i];
    const Value &a = values[x.operands[0]], &b = values[x.operands[1]];
    if (x.rank != 2 || readable[i] || a.split_inner != 0 || b.split_inner != 0 || a.kind != Value::kDense ||
        b.kind != Value::kDense)
      return false;
    const bool mfma = numerics == TOPOS_HIP_FAST &&
                      mfma_serves(b.layout.strides[1], b.layout.strides[0], a.layout.strides[1], a.layout.strides[0],
                                  x.shape[1], nodes[x.operands[0]].shape[1], x.shape[0]);
    int64_t v = i;
    for (int hop = 0; hop < 4; ++hop) {
      if (consumers[v].size() != 1) return false;
      const int64_t c = consumers[v][0];
      const topos_hip_node &y = nodes[c];
      if (y.op == TOPOS_HIP_OP_TRANSPOSE) return true;
      if (!(mfma && y.op == TOPOS_HIP_OP_ADD && group_of[c] < 0 && alias_of[c] < 0)) return false;
      const int64_t other = y.operands[0] == v ? y.operands[1] : y.operands[0];
      if (other == v || !static_plus_zero(other)) return false;
      v = c;
    }
    return false;
  }

  void plan_transposed_matmul(int64_t i) {
    const topos_hip_node &x = nodes[i];
    const int64_t m = x.shape[0], n = x.shape[1], k = nodes[x.operands[0]].shape[1];
    const Value a = dense_operand(x.operands[0]);
    const Value b = dense_operand(x.operands[1]);
    // D = B^T A^T (n x m): its left operand B^T, its right A^T, as views.
    const int64_t ars = b.layout.strides[1], acs = b.layout.strides[0];
    const int64_t brs = a.layout.strides[1], bcs = a.layout.strides[0];
    const int64_t a_offset = b.layout.offset, b_offset = a.layout.offset;
    const int left = b.storage, right = a.storage;
    const int out = arena_storage(m * n * 4);
    const bool mfma = numerics == TOPOS_HIP_FAST && mfma_serves(ars, acs, brs, bcs, n, k, m);
    int64_t workspace_floats = 0;
    int workspace = -1;
    if (numerics == TOPOS_HIP_FAST) {
      const int splits = mfma_splits(n, m, k, 1);
      if (splits > 1) {
        workspace_floats = (int64_t)splits * m * n;
        workspace = arena_storage(workspace_floats * 4);
      }
    }
    std::ostringstream what;
    what << "gemm " << (numerics == TOPOS_HIP_FAST ? "mfma" : "exact") << " 1x(" << n << "," << m << "," << k
         << ") a[" << ars << "," << acs << "] b[" << brs << "," << bcs << "] transposed";
    std::vector<int> writes = {out};
    if (workspace >= 0) writes.push_back(workspace);
    const int numerics_ = numerics;
    add_launch(what.str(), {left, right}, writes,
               [this, left, right, out, a_offset, b_offset, ars, acs, brs, bcs, m, n, k, numerics_, workspace,
                workspace_floats](const Exec &ex) {
                 const float *pa = (const float *)base(left) + a_offset;
                 const float *pb = (const float *)base(right) + b_offset;
                 float *pc = (float *)base(out);
                 float *pw = workspace >= 0 ? (float *)base(workspace) : nullptr;
                 if (numerics_ == TOPOS_HIP_FAST &&
                     launch_gemm_mfma(pa, ars, acs, pb, brs, bcs, n, k, m, pc, m, ex.stream, Batch(), pw,
                                      workspace_floats))
                   return;
                 launch_gemm_exact(pa, ars, acs, pb, brs, bcs, n, k, m, pc, m, ex.stream);
               });
    launches.back().flops = 2.0 * (double)m * n * k;
    launches.back().bytes = 4.0 * ((double)m * k + (double)k * n + (double)m * n);
    Layout l;
    l.rank = 2;
    l.shape[0] = m;
    l.shape[1] = n;
    l.strides[0] = 1;
    l.strides[1] = m;
    values[i] = dense_value(out, l);
    values[i].never_minus_zero = mfma;
  }

  void plan_matmul(int64_t i) {
    if (values[nodes[i].operands[0]].kind == Value::kWindow) {
      plan_window_matmul(i);
      return;
    }
    if (read_transposed(i)) {
      plan_transposed_matmul(i);
      return;
    }
    const topos_hip_node &x = nodes[i];
    const int r = x.rank, s = r - 2;
    const int64_t m = x.shape[s], n = x.shape[s + 1], k = nodes[x.operands[0]].shape[s + 1];
    // Merged-batch operands: served by the matrix-core kernel's two-level
    // batch strides when both merges agree, else copied.
    const Value &va = values[x.operands[0]], &vb = values[x.operands[1]];
    int64_t inner = va.split_inner > 0 ? va.split_inner : vb.split_inner;
    if (inner > 0) {
      const Layout &la = va.layout, &lb = vb.layout;
      const bool agree = (va.split_inner == 0 || va.split_inner == inner) &&
                         (vb.split_inner == 0 || vb.split_inner == inner);
      if (!(numerics == TOPOS_HIP_FAST && r == 3 && agree &&
            mfma_serves(la.strides[1], la.strides[2], lb.strides[1], lb.strides[2], m, k, n)))
        inner = 0;
    }
    const Value a = inner > 0 ? values[x.operands[0]] : dense_operand(x.operands[0]);
    const Value b = inner > 0 ? values[x.operands[1]] : dense_operand(x.operands[1]);
    int64_t batches = 1;
    for (int d = 0; d < s; ++d) batches *= x.shape[d];
    const int out = arena_storage(batches * m * n * 4);
    Batch batch;
    batch.count = batches;
    batch.c_stride = m * n;
    bool flat;
    if (inner > 0) {
      // Batch y at (y / inner) * stride + (y % inner) * inner stride.
      auto two_level = [inner](const Value &v, int64_t &outer, int64_t &within) {
        if (v.split_inner > 0) {
          outer = v.split_outer_stride;
          within = v.split_inner_stride;
        } else {
          within = v.layout.strides[0];
          outer = within * inner;
        }
      };
      batch.inner = inner;
      two_level(a, batch.a_stride, batch.a_inner);
      two_level(b, batch.b_stride, batch.b_inner);
      batch.c_inner = m * n;
      batch.c_stride = inner * m * n;
      flat = true;
    } else {
      flat = batch_stride(a.layout, s, batch.a_stride) && batch_stride(b.layout, s, batch.b_stride);
    }
    // Per-launch offsets when the batch axes do not flatten: one product per
    // batch index, each at its own operand offsets.
    std::vector<std::array<int64_t, 3>> parts;
    if (flat) {
      parts.push_back({a.layout.offset, b.layout.offset, 0});
    } else {
      for (int64_t q = 0; q < batches; ++q) {
        int64_t rem = q, ao = a.layout.offset, bo = b.layout.offset;
        for (int d = s - 1; d >= 0; --d) {
          const int64_t c = rem % x.shape[d];
          rem /= x.shape[d];
          ao += c * a.layout.strides[d];
          bo += c * b.layout.strides[d];
        }
        parts.push_back({ao, bo, q * m * n});
      }
      batch = Batch();
      batch.c_stride = m * n;
    }
    const int64_t ars = a.layout.strides[s], acs = a.layout.strides[s + 1];
    const int64_t brs = b.layout.strides[s], bcs = b.layout.strides[s + 1];
    const int numerics_ = numerics;
    mfma_product[i] = numerics == TOPOS_HIP_FAST && mfma_serves(ars, acs, brs, bcs, m, k, n);
    // Scratch for the partial products of a split along k (fast posture).
    int64_t workspace_floats = 0;
    int workspace = -1;
    if (numerics == TOPOS_HIP_FAST) {
      const int splits = mfma_splits(m, n, k, batch.count);
      if (splits > 1) {
        workspace_floats = (int64_t)splits * batch.count * m * n;
        workspace = arena_storage(workspace_floats * 4);
      }
    }
    std::ostringstream what;
    what << "gemm " << (numerics == TOPOS_HIP_FAST ? "mfma" : "exact") << " " << batches << "x(" << m << "," << n
         << "," << k << ") a[" << ars << "," << acs << "] b[" << brs << "," << bcs << "]";
    std::vector<int> writes = {out};
    if (workspace >= 0) writes.push_back(workspace);
    auto bias = std::make_shared<BiasEpilogue>();
    auto output = std::make_shared<ProductOutput>();
    output->storage = out;
    output->ldc = n;
    output->batch = batch;
    const int launch =
        add_launch(what.str(), {a.storage, b.storage}, writes,
                   [this, a, b, output, parts, m, n, k, ars, acs, brs, bcs, numerics_, workspace, workspace_floats,
                    bias](const Exec &ex) {
                     const float *pa = (const float *)base(a.storage);
                     const float *pb = (const float *)base(b.storage);
                     float *pc = (float *)base(output->storage);
                     const Batch &batch = output->batch;
                     const int64_t ldc = output->ldc;
                     float *pw = workspace >= 0 ? (float *)base(workspace) : nullptr;
                     Epilogue epilogue;
                     if (bias->storage >= 0) {
                       epilogue.bias = (const float *)base(bias->storage) + bias->offset;
                       epilogue.bias_stride = bias->stride;
                       epilogue.bias_first = bias->first;
                     }
                     for (const auto &part : parts) {
                       const float *qa = pa + part[0], *qb = pb + part[1];
                       float *qc = pc + part[2];
                       if (numerics_ == TOPOS_HIP_FAST &&
                           launch_gemm_mfma(qa, ars, acs, qb, brs, bcs, m, k, n, qc, ldc, ex.stream, batch, pw,
                                            workspace_floats, epilogue))
                         continue;
                       // A fused bias, two-level batches and a retargeted output
                       // are planned only where the matrix-core kernel serves.
                       launch_gemm_exact(qa, ars, acs, qb, brs, bcs, m, k, n, qc, ldc, ex.stream, batch);
                     }
                   });
    if (mfma_product[i]) {
      product_launch[i] = ProductLaunch{launch, bias, output, flat};
      product_of_storage[out] = i;
    }
    launches.back().flops = 2.0 * (double)batches * m * n * k;
    launches.back().bytes = 4.0 * (double)batches * ((double)m * k + (double)k * n + (double)m * n);
    values[i] = dense_value(out, contiguous(x.rank, x.shape));
    values[i].never_minus_zero = mfma_product[i];
  }

  // The expression a reduction folds: the operand's inlined tree, or the
  // operand's value read through its layout.
  Expr reduction_expression(int64_t operand, std::vector<int> &storage_of) {
    const topos_hip_node &a = nodes[operand];
    Expr e;
    e.rank = a.rank;
    for (int d = 0; d < a.rank; ++d) e.shape[d] = a.shape[d];
    std::map<int64_t, int> memo;
    e.outputs.push_back(expr_of(operand, e, memo, storage_of));
    return e;
  }

  // A selection's ordered sums are fixed by `one` and the shape: a row
  // holds +0 everywhere but `one` at its index, so its fold is one + 0
  // (one itself in a single-column row: +0 + one = one for every non-zero,
  // and +0 for a zero `one`); the whole selection's row-major fold is the
  // fold of one such value per row, since zero terms leave a non-zero
  // accumulator unchanged.
  float selection_row_sum(const Value &v, int64_t vocab) const {
    const float one = storages[v.storage].one;
    return vocab > 1 ? fold_scalar(TOPOS_HIP_OP_ADD, 0.0f, one) : one;
  }

  void plan_sum_along(int64_t i) {
    const topos_hip_node &x = nodes[i];
    const int64_t operand = x.operands[0];
    const int axis = (int)x.params[0];
    const Value &a = values[operand];
    if (a.kind == Value::kDense && a.host_known) {
      values[i] = host_constant(x, fold_repeated(a.host_value, nodes[operand].shape[axis]));
      return;
    }
    if (a.kind == Value::kSelection && axis == 1) {
      values[i] = host_constant(x, selection_row_sum(a, nodes[operand].shape[1]));
      return;
    }
    std::vector<int> storage_of;
    Expr e = reduction_expression(operand, storage_of);
    const int out = arena_storage(volume_of(x) * 4);
    Generated g = generate_fold(e, axis, kFoldSum);
    pending.push_back(g);
    ++fused_groups;
    add_launch("fold sum axis " + std::to_string(axis) + " " + describe_expr(e), real(storage_of), {out},
               [this, e, g, storage_of, out, axis](const Exec &ex) {
                 auto p = pointers_for(storage_of);
                 launch_generated_fold(g, e, axis, p.data(), (float *)base(out), ex.stream);
               });
    account(e, (double)volume_of(x));
    values[i] = dense_value(out, contiguous(x.rank, x.shape));
  }

  void plan_sum(int64_t i) {
    const topos_hip_node &x = nodes[i];
    const int64_t operand = x.operands[0];
    const Value &a = values[operand];
    if (a.kind == Value::kDense && a.host_known) {
      values[i] = host_constant(x, fold_repeated(a.host_value, volume_of(nodes[operand])));
      return;
    }
    if (a.kind == Value::kSelection) {
      const topos_hip_node &o = nodes[operand];
      values[i] = host_constant(x, fold_repeated(selection_row_sum(a, o.shape[1]), o.shape[0]));
      return;
    }
    std::vector<int> storage_of;
    Expr e = reduction_expression(operand, storage_of);
    const int64_t volume = e.volume();
    const int64_t chunks = (volume + kSumChunk - 1) / kSumChunk;
    const int out = arena_storage(4);
    const int counts = arena_storage(chunks * 4);
    const int flags = arena_storage(chunks * 4);
    const int slots = arena_storage(chunks * kSumChunk * 4);
    Generated gather = generate_sum_gather(e);
    pending.push_back(gather);
    ++fused_groups;
    std::vector<int> reads = real(storage_of);
    add_launch("sum (ordered, gathered) " + describe_expr(e), reads, {out, counts, flags, slots},
               [this, e, gather, storage_of, out, counts, flags, slots, chunks](const Exec &ex) {
                 auto p = pointers_for(storage_of);
                 launch_sum_gather(gather, e, p.data(), (float *)base(slots), (int32_t *)base(counts),
                                   (int32_t *)base(flags), ex.stream);
                 launch_slot_fold((const float *)base(slots), (const int32_t *)base(counts),
                                  (const int32_t *)base(flags), chunks, kSumChunk, (float *)base(out), ex.stream);
               });
    account(e, 1.0);
    Value v = dense_value(out, constant_layout(0, x.shape, 0));
    v.constant = true;
    values[i] = v;
  }

  // LogSoftmax / LogSumExp along `axis`: the row kernels over a contiguous
  // [rows, extent] operand (permuted into place when the axis is not last).
  void plan_rows(int64_t i) {
    const topos_hip_node &x = nodes[i];
    const int64_t operand = x.operands[0];
    const topos_hip_node &a = nodes[operand];
    const int axis = (int)x.params[0];
    Value v = dense_operand(operand);
    const bool last = axis == a.rank - 1;
    bool direct = v.kind == Value::kDense && !v.constant && last && is_contiguous(v.layout);
    int source = v.storage;
    int64_t source_offset = v.layout.offset;
    int order[kMaxRank];
    for (int d = 0, e = 0; d < a.rank; ++d)
      if (d != axis) order[e++] = d;
    order[a.rank - 1] = axis;
    if (!direct) {
      // Copy the operand with the axis moved last.
      Expr e;
      e.rank = a.rank;
      ExprInput in;
      std::vector<int> storage_of;
      for (int d = 0; d < a.rank; ++d) {
        e.shape[d] = a.shape[order[d]];
        in.strides[d] = v.layout.strides[order[d]];
      }
      if (v.host_known) {
        in.kind = ExprInput::kLiteral;
        in.one = v.host_value;
        storage_of.push_back(-1);
      } else {
        in.offset = v.layout.offset;
        storage_of.push_back(v.storage);
      }
      e.inputs.push_back(in);
      e.outputs.push_back(-1);
      const int copy = arena_storage(e.volume() * 4);
      Generated g = generate_chain(e);
      pending.push_back(g);
    pending.push_back(g);
      add_launch("copy (axis last) " + describe_expr(e), real(storage_of), {copy},
                 [this, e, g, storage_of, copy](const Exec &ex) {
                   auto p = pointers_for(storage_of);
                   float *q = (float *)base(copy);
                   launch_generated_chain(g, e, p.data(), &q, ex.stream);
                 });
      account(e, (double)e.volume());
      source = copy;
      source_offset = 0;
    }
    const int64_t extent = a.shape[axis];
    const int64_t rows = volume_of(a) / extent;
    const bool full = x.op == TOPOS_HIP_OP_LOG_SOFTMAX;
    const int out = arena_storage((full ? volume_of(a) : rows) * 4);
    const int kind = full ? TOPOS_HIP_ROWS_LOG_SOFTMAX : TOPOS_HIP_ROWS_LOG_SUM_EXP;
    // Row reductions are exact in both postures (only products take the
    // matrix-core envelope).
    const int numerics_ = TOPOS_HIP_EXACT;
    add_launch(std::string(full ? "log_softmax " : "log_sum_exp ") + std::to_string(rows) + "x" +
                   std::to_string(extent),
               {source}, {out}, [this, source, source_offset, out, rows, extent, kind, numerics_](const Exec &ex) {
                 launch_rows(kind, (const float *)base(source) + source_offset, rows, extent, numerics_,
                             (float *)base(out), ex.stream);
               });
    launches.back().kind = "rows";
    launches.back().bytes = 4.0 * ((double)rows * extent + (full ? (double)rows * extent : (double)rows));
    if (!full) {
      values[i] = dense_value(out, contiguous(x.rank, x.shape));
      return;
    }
    // The result in the permuted order, viewed back in the node's axes.
    int64_t permuted_shape[kMaxRank];
    for (int d = 0; d < a.rank; ++d) permuted_shape[d] = a.shape[order[d]];
    const Layout p = contiguous(a.rank, permuted_shape);
    Layout l;
    l.rank = a.rank;
    for (int d = 0; d < a.rank; ++d) {
      l.shape[order[d]] = permuted_shape[d];
      l.strides[order[d]] = p.strides[d];
    }
    values[i] = dense_value(out, l);
  }

  // A [rows, row_size] reading of a rank >= 1 layout (row = axis 0).
  static bool as_rows(const Layout &l, int64_t &row_stride, int64_t &column_stride) {
    row_stride = l.strides[0];
    if (l.rank == 1) {
      column_stride = 0;
      return true;
    }
    for (int d = 1; d + 1 < l.rank; ++d)
      if (l.shape[d + 1] != 1 && l.strides[d] != l.shape[d + 1] * l.strides[d + 1]) return false;
    column_stride = l.strides[l.rank - 1];
    return true;
  }

  // Fold (src/payload/tensor.rs:1392-1462): one kernel reading the operand
  // through its layout, writing the folded value contiguous.
  void plan_fold(int64_t i) {
    const topos_hip_node &x = nodes[i];
    const Value a = dense_operand(x.operands[0]);
    const Layout &l = a.layout;
    const int axis = (int)x.params[0];
    FoldGeometry g;
    g.outer_rank = axis;
    for (int d = 0; d < axis; ++d) {
      g.outer_shape[d] = l.shape[d];
      g.outer_strides[d] = l.strides[d];
    }
    g.inner_rank = l.rank - axis - 2;
    for (int d = 0; d < g.inner_rank; ++d) {
      g.inner_shape[d] = l.shape[axis + 2 + d];
      g.inner_strides[d] = l.strides[axis + 2 + d];
      g.inner_volume *= l.shape[axis + 2 + d];
    }
    g.window_stride = l.strides[axis];
    g.element_stride = l.strides[axis + 1];
    g.count = l.shape[axis];
    g.size = x.params[1];
    g.step = x.params[2];
    g.dilation = x.params[3];
    g.extent = x.params[4];
    g.total = volume_of(x);
    const int out = arena_storage(g.total * 4);
    const int source = a.storage;
    const int64_t offset = l.offset;
    std::ostringstream what;
    what << "fold [";
    for (int d = 0; d < l.rank; ++d) what << (d ? "," : "") << l.shape[d];
    what << "] axis " << axis << " onto " << g.extent;
    add_launch(what.str(), {source}, {out}, [this, source, offset, g, out](const Exec &ex) {
      launch_fold((const float *)base(source) + offset, g, (float *)base(out), ex.stream);
    });
    launches.back().bytes = 4.0 * ((double)volume_of(nodes[x.operands[0]]) + (double)g.total);
    values[i] = dense_value(out, contiguous(x.rank, x.shape));
  }

  void plan_gather(int64_t i) {
    const topos_hip_node &x = nodes[i];
    Value t = dense_operand(x.operands[0]);
    const Value &sel = values[x.operands[1]];
    if (sel.kind != Value::kSelection) refuse(i, "gather needs a selection (Tensor::selection) operand");
    int64_t rs, cs;
    if (!as_rows(t.layout, rs, cs)) {
      t = materialize(x.operands[0]);
      as_rows(t.layout, rs, cs);
    }
    const int64_t rows = x.shape[0], row_size = volume_of(x) / rows;
    const int out = arena_storage(volume_of(x) * 4);
    const int table = t.storage, selection = sel.storage;
    const int64_t offset = t.layout.offset;
    add_launch("gather " + std::to_string(rows) + "x" + std::to_string(row_size), {table, selection}, {out},
               [this, table, selection, out, offset, rs, cs, rows, row_size](const Exec &ex) {
                 launch_gather((const float *)base(table) + offset, rs, cs, (const int32_t *)base(selection), rows,
                               row_size, (float *)base(out), ex.stream);
               });
    launches.back().bytes = 4.0 * (2.0 * rows * row_size + rows);
    values[i] = dense_value(out, contiguous(x.rank, x.shape));
  }

  void plan_scatter(int64_t i) {
    const topos_hip_node &x = nodes[i];
    Value g = dense_operand(x.operands[0]);
    const Value &sel = values[x.operands[1]];
    if (sel.kind != Value::kSelection) refuse(i, "scatter needs a selection (Tensor::selection) operand");
    int64_t rs, cs;
    if (!as_rows(g.layout, rs, cs)) {
      g = materialize(x.operands[0]);
      as_rows(g.layout, rs, cs);
    }
    const int64_t rows = x.shape[0], row_size = volume_of(x) / rows;
    const int out = arena_storage(volume_of(x) * 4);
    const int gradient = g.storage, selection = sel.storage;
    const int64_t offset = g.layout.offset;
    add_launch("scatter " + std::to_string(rows) + "x" + std::to_string(row_size), {gradient, selection}, {out},
               [this, gradient, selection, out, offset, rs, cs, rows, row_size](const Exec &ex) {
                 const SelectionBuffers &b = selection_buffers(selection);
                 launch_scatter((const float *)base(gradient) + offset, rs, cs, b.row_start, b.sources, rows,
                                row_size, (float *)base(out), ex.stream);
               });
    launches.back().bytes = 4.0 * ((double)nodes[x.operands[0]].shape[0] * row_size + (double)rows * row_size);
    values[i] = dense_value(out, contiguous(x.rank, x.shape));
  }

  // Every readable node ends in a contiguous buffer the caller can read.
  void finish_readables() {
    for (int64_t i = 0; i < (int64_t)nodes.size(); ++i) {
      if (!readable[i]) continue;
      const Value &v = values[i];
      const topos_hip_node &x = nodes[i];
      const bool in_place = v.kind == Value::kDense && !v.constant && is_contiguous(v.layout) &&
                            (storages[v.storage].kind != StorageKind::kArena ||
                             (v.layout.offset == 0 && storages[v.storage].bytes == volume_of(x) * 4)) &&
                            storages[v.storage].kind != StorageKind::kPool;
      const bool scalar_buffer = v.kind == Value::kDense && v.constant && !v.host_known && volume_of(x) == 1 &&
                                 storages[v.storage].kind == StorageKind::kArena;
      if (in_place || scalar_buffer) {
        output_storage[i] = v.storage;
        output_offset[i] = v.layout.offset;
      } else {
        const Value copied = materialize(i);
        output_storage[i] = copied.storage;
        output_offset[i] = 0;
      }
      storages[output_storage[i]].pinned = true;
    }
  }

  // First-fit offsets over the storages' live intervals.
  void assign_arena() {
    for (size_t l = 0; l < launches.size(); ++l) {
      for (int s : launches[l].writes) storages[s].first = std::min(storages[s].first, (int)l);
      for (int s : launches[l].reads) storages[s].last = std::max(storages[s].last, (int)l);
      for (int s : launches[l].writes) storages[s].last = std::max(storages[s].last, (int)l);
    }
    std::vector<std::vector<int>> born(launches.size()), dies(launches.size());
    for (size_t s = 0; s < storages.size(); ++s) {
      Storage &st = storages[s];
      if (st.kind != StorageKind::kArena || st.first == INT_MAX || st.side) continue;
      born[st.first].push_back((int)s);
      if (!st.pinned) dies[st.last].push_back((int)s);
    }
    std::map<int64_t, int64_t> free_blocks;  // offset -> bytes
    int64_t top = 0;
    auto round = [](int64_t b) { return (b + 255) / 256 * 256; };
    for (size_t l = 0; l < launches.size(); ++l) {
      for (int s : born[l]) {
        const int64_t need = round(storages[s].bytes);
        auto fit = free_blocks.end();
        for (auto it = free_blocks.begin(); it != free_blocks.end(); ++it)
          if (it->second >= need) {
            fit = it;
            break;
          }
        if (fit != free_blocks.end()) {
          storages[s].offset = fit->first;
          const int64_t rest = fit->second - need, at = fit->first + need;
          free_blocks.erase(fit);
          if (rest > 0) free_blocks[at] = rest;
        } else if (!free_blocks.empty() && std::prev(free_blocks.end())->first + std::prev(free_blocks.end())->second == top) {
          // Grow the last free block at the top.
          auto last = std::prev(free_blocks.end());
          storages[s].offset = last->first;
          top = last->first + need;
          free_blocks.erase(last);
        } else {
          storages[s].offset = top;
          top += need;
        }
      }
      for (int s : dies[l]) {
        int64_t at = storages[s].offset, size = round(storages[s].bytes);
        auto next = free_blocks.lower_bound(at);
        if (next != free_blocks.end() && at + size == next->first) {
          size += next->second;
          next = free_blocks.erase(next);
        }
        if (next != free_blocks.begin()) {
          auto prev = std::prev(next);
          if (prev->first + prev->second == at) {
            at = prev->first;
            size += prev->second;
            free_blocks.erase(prev);
          }
        }
        free_blocks[at] = size;
      }
    }
    // The side region: storages the side stream writes never share memory
    // with main-stream storages. A side launch waits only for its inputs, so
    // it may run ahead of main launches that still use memory first-fit would
    // otherwise have handed to its outputs.
    for (Storage &st : storages)
      if (st.kind == StorageKind::kArena && st.side && st.first != INT_MAX) {
        st.offset = top;
        top += round(st.bytes);
      }
    arena_bytes = (uint64_t)std::max<int64_t>(top, 256);
  }

  void describe() {
    std::ostringstream s;
    s << "arena " << arena_bytes << " bytes, " << launches.size() << " launches, " << fused_groups
      << " generated kernels\n";
    for (size_t l = 0; l < launches.size(); ++l)
      s << l << ": " << launches[l].what << (launches[l].side ? " [side]" : "") << "\n";
    description = s.str();
  }

  // Short dead-end branches run on a side stream, overlapping the main
  // chain: a launch whose downstream is at most kSideDepth launches, all of
  // them side launches themselves (a parameter gradient's product or fold
  // and the zero-seeded accumulation behind it), except trailing ones fed
  // only by the main stream. A side launch waits for the
  // event of its latest main-stream producer; the run ends with the main
  // stream waiting for the side stream. Every storage a side launch touches
  // is kept to the end of the run, so no later main launch reuses its memory
  // while the side stream may still use it.
  void assign_streams() {
    const size_t count = launches.size();
    std::vector<int> producer(storages.size(), -1);
    for (size_t l = 0; l < count; ++l)
      for (int s : launches[l].writes) producer[s] = (int)l;
    std::vector<std::vector<int>> readers(count);
    for (size_t l = 0; l < count; ++l)
      for (int s : launches[l].reads)
        if (producer[s] >= 0 && producer[s] != (int)l) readers[producer[s]].push_back((int)l);
    constexpr int kSideDepth = 4;
    std::vector<int> downstream(count, 0);  // an over-count of the launches downstream
    for (size_t q = count; q-- > 0;) {
      bool side = true;
      int below = 0;
      for (int r : readers[q]) {
        side = side && launches[r].side;
        below += 1 + downstream[r];
      }
      downstream[q] = std::min(below, 1 << 20);
      launches[q].side = side && below <= kSideDepth;
    }
    // Side launches that cannot start before the main stream's last launch
    // ends (they read its output, or a launch moved here) and read nothing
    // a side launch writes run on the main stream instead: it is idle by
    // then, while the side stream still works through the branches queued
    // before them (in the GPT-2 step, layer 0's LayerNorm gradient and the
    // embedding scatters behind its weight gradient). A launch that reads a
    // side launch's output stays on the side stream, which orders it.
    int last_main = -1;
    for (size_t l = 0; l < count; ++l)
      if (!launches[l].side) last_main = (int)l;
    if (last_main >= 0) {
      std::vector<bool> at_end(count, false);
      at_end[last_main] = true;
      for (size_t l = (size_t)last_main + 1; l < count; ++l) {
        bool from_main = true, after_end = false;
        for (int s : launches[l].reads) {
          const int p = producer[s];
          if (p < 0 || p == (int)l) continue;
          if (launches[p].side) from_main = false;
          if (at_end[p]) after_end = true;
        }
        if (from_main && after_end) launches[l].side = false, at_end[l] = true;
      }
    }
    for (size_t l = 0; l < count; ++l) {
      Launch &launch = launches[l];
      if (!launch.side) continue;
      ++side_launches;
      for (int s : launch.reads) {
        storages[s].pinned = true;
        const int p = producer[s];
        if (p >= 0 && !launches[p].side) launch.wait_for = std::max(launch.wait_for, p);
      }
      for (int s : launch.writes) storages[s].pinned = storages[s].side = true;
      if (launch.wait_for >= 0) launches[launch.wait_for].signals = true;
    }
  }

  void plan() {
    validate();
    deduplicate();
    mark_wanted();
    form_row_groups();
    form_window_products();
    values.assign(nodes.size(), Value());
    mfma_product.assign(nodes.size(), false);
    for (int64_t i = 0; i < (int64_t)nodes.size(); ++i) {
      if (!wanted[i] || alias_of[i] >= 0 || window_interior[i]) continue;
      if (window_roots.count(i)) {
        values[i] = window_value(i);
        continue;
      }
      const int group = group_of[i];
      if (group >= 0) {
        if (i == row_groups[group].members.back()) plan_row_group(group);
        continue;
      }
      plan_node(i);
    }
    // A duplicate (wanted only when readable) reads its original's value.
    for (int64_t i = 0; i < (int64_t)nodes.size(); ++i)
      if (wanted[i] && alias_of[i] >= 0) values[i] = values[alias_of[i]];
    open_chain.reset();
    finish_readables();
    finish_chains();
    assign_streams();
    assign_arena();
    compile_kernels(pending, device);
    describe();
  }

  // ================= device state =================

  void upload_constants() {
    // The pool, then every dense leaf payload, in one allocation.
    std::vector<float> all(pool);
    leaf_data_offset = (int64_t)all.size();
    all.insert(all.end(), leaf_data.begin(), leaf_data.end());
    if (all.empty()) all.push_back(0.0f);
    void *p = nullptr;
    check(hipMalloc(&p, all.size() * 4), "hipMalloc(constants)");
    allocations.push_back(p);
    constants = (float *)p;
    check(hipMemcpy(constants, all.data(), all.size() * 4, hipMemcpyHostToDevice), "hipMemcpy(constants)");
    for (const Storage &s : storages)
      if (s.kind == StorageKind::kSelectionLeaf && !selection_leaves.count(s.index)) {
        const topos_hip_leaf &leaf = leaves[s.index];
        selection_leaves[s.index] = upload_selection(&leaf_indices[leaf.offset], s.rows, s.vocab, true);
      }
  }

  // Copies a selection's indices and its row-sorted order to the device.
  SelectionBuffers upload_selection(const int32_t *indices, int64_t rows, int64_t vocab, bool track) {
    std::vector<int32_t> row_start(vocab + 1, 0), sources(rows);
    for (int64_t r = 0; r < rows; ++r) ++row_start[indices[r] + 1];
    for (int64_t v = 0; v < vocab; ++v) row_start[v + 1] += row_start[v];
    std::vector<int32_t> cursor(row_start.begin(), row_start.end() - 1);
    for (int64_t r = 0; r < rows; ++r) sources[cursor[indices[r]]++] = (int32_t)r;  // ascending source order
    SelectionBuffers b;
    b.rows = rows;
    b.vocab = vocab;
    void *p = nullptr;
    check(hipMalloc(&p, rows * 4), "hipMalloc(selection)");
    b.indices = (int32_t *)p;
    check(hipMalloc(&p, (vocab + 1) * 4), "hipMalloc(selection rows)");
    b.row_start = (int32_t *)p;
    check(hipMalloc(&p, std::max<int64_t>(rows, 1) * 4), "hipMalloc(selection sources)");
    b.sources = (int32_t *)p;
    if (track) {
      allocations.push_back(b.indices);
      allocations.push_back(b.row_start);
      allocations.push_back(b.sources);
    }
    check(hipMemcpy(b.indices, indices, rows * 4, hipMemcpyHostToDevice), "hipMemcpy(selection)");
    check(hipMemcpy(b.row_start, row_start.data(), (vocab + 1) * 4, hipMemcpyHostToDevice), "hipMemcpy(rows)");
    check(hipMemcpy(b.sources, sources.data(), rows * 4, hipMemcpyHostToDevice), "hipMemcpy(sources)");
    return b;
  }

  void drop_graph() {
    if (graph_exec) hipGraphExecDestroy(graph_exec);
    if (graph) hipGraphDestroy(graph);
    graph_exec = nullptr;
    graph = nullptr;
  }

  // The arena and the side stream's objects: created before the first run
  // (and before any capture, which must not allocate).
  void prepare() {
    if (!device) throw InvalidArgument{"the fake runtime plans programs but does not run them"};
    if (!arena) {
      void *p = nullptr;
      check(hipMalloc(&p, arena_bytes), "hipMalloc(arena)");
      allocations.push_back(p);
      arena = (char *)p;
    }
    if (!run_done) check(hipEventCreateWithFlags(&run_done, hipEventDisableTiming), "hipEventCreate(run done)");
    if (side_launches > 0 && !side_stream) {
      check(hipStreamCreateWithFlags(&side_stream, hipStreamNonBlocking), "hipStreamCreate(side)");
      check(hipEventCreateWithFlags(&side_done, hipEventDisableTiming), "hipEventCreate(side)");
      check(hipEventCreateWithFlags(&side_start, hipEventDisableTiming), "hipEventCreate(side)");
      for (size_t l = 0; l < launches.size(); ++l)
        if (launches[l].signals) {
          hipEvent_t e;
          check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate(signal)");
          signal_events[(int)l] = e;
        }
    }
  }

  // One run as the launch of a captured graph: the first replay (or the
  // first after a bind) captures run() on the program's capture stream.
  void replay(hipStream_t stream) {
    prepare();
    if (!graph_exec) {
      if (!capture_stream)
        check(hipStreamCreateWithFlags(&capture_stream, hipStreamNonBlocking), "hipStreamCreate(capture)");
      check(hipStreamBeginCapture(capture_stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
      try {
        run(capture_stream);
      } catch (...) {
        hipGraph_t partial = nullptr;
        hipStreamEndCapture(capture_stream, &partial);
        if (partial) hipGraphDestroy(partial);
        throw;
      }
      check(hipStreamEndCapture(capture_stream, &graph), "hipStreamEndCapture");
      check(hipGraphInstantiate(&graph_exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    }
    check(hipGraphLaunch(graph_exec, stream), "hipGraphLaunch");
  }

  void run(hipStream_t stream, float *milliseconds = nullptr) {
    prepare();
    // Every binding must be present before anything is enqueued.
    for (const Storage &s : storages) {
      if (s.first == INT_MAX && s.last < 0) continue;
      if (s.kind == StorageKind::kParameter && !parameters.count(s.index))
        throw InvalidArgument{"parameter slot " + std::to_string(s.index) + " is not bound"};
      if (s.kind == StorageKind::kInput && !inputs.count(s.index))
        throw InvalidArgument{"input slot " + std::to_string(s.index) + " is not bound"};
      if (s.kind == StorageKind::kSelectionInput && !selection_inputs.count(s.index))
        throw InvalidArgument{"selection input slot " + std::to_string(s.index) + " is not bound"};
    }
    const Exec ex{this, stream};
    if (!milliseconds) {
      if (side_launches == 0) {
        for (const Launch &l : launches) l.run(ex);
        return;
      }
      // The side stream first waits for everything enqueued on the main
      // stream before this run (the caller's writes to parameters and inputs).
      check(hipEventRecord(side_start, stream), "hipEventRecord(start)");
      check(hipStreamWaitEvent(side_stream, side_start, 0), "hipStreamWaitEvent(start)");
      const Exec side_ex{this, side_stream};
      for (size_t l = 0; l < launches.size(); ++l) {
        const Launch &launch = launches[l];
        if (launch.side) {
          if (launch.wait_for >= 0)
            check(hipStreamWaitEvent(side_stream, signal_events.at(launch.wait_for), 0), "hipStreamWaitEvent");
          launch.run(side_ex);
        } else {
          launch.run(ex);
          if (launch.signals) check(hipEventRecord(signal_events.at((int)l), stream), "hipEventRecord(signal)");
        }
      }
      check(hipEventRecord(side_done, side_stream), "hipEventRecord(side done)");
      check(hipStreamWaitEvent(stream, side_done, 0), "hipStreamWaitEvent(side done)");
      return;
    }
    std::vector<hipEvent_t> events(launches.size() + 1);
    for (hipEvent_t &e : events) check(hipEventCreate(&e), "hipEventCreate");
    check(hipEventRecord(events[0], stream), "hipEventRecord");
    for (size_t l = 0; l < launches.size(); ++l) {
      launches[l].run(ex);
      check(hipEventRecord(events[l + 1], stream), "hipEventRecord");
    }
    check(hipEventSynchronize(events.back()), "hipEventSynchronize");
    for (size_t l = 0; l < launches.size(); ++l)
      check(hipEventElapsedTime(&milliseconds[l], events[l], events[l + 1]), "hipEventElapsedTime");
    for (hipEvent_t &e : events) hipEventDestroy(e);
  }
};

namespace {

// Validates the table's buffers, then plans the program over `p`'s node
// table (shared by the forward and the engine-backward entry points).
int plan_program(std::unique_ptr<topos_hip_program> p, const float *leaf_data, int64_t leaf_data_len,
                 const int32_t *leaf_indices, int64_t leaf_indices_len, int numerics,
                 topos_hip_program **program) {
  p->leaf_data.assign(leaf_data, leaf_data + leaf_data_len);
  p->leaf_indices.assign(leaf_indices, leaf_indices + leaf_indices_len);
  p->numerics = numerics;
  p->device = Context::get().runtime().launches_kernels;
  const int code = guarded([&] {
    try {
      p->plan();
    } catch (const InvalidArgument &e) {
      last_refusal() = e.message;
      throw;
    } catch (const Unsupported &e) {
      last_refusal() = e.message;
      throw;
    }
    if (p->device) p->upload_constants();
  });
  if (code == TOPOS_HIP_OK) *program = p.release();
  return code;
}

bool table_arguments_valid(const topos_hip_node *nodes, int64_t n_nodes, const topos_hip_leaf *leaves,
                           int64_t n_leaves, const float *leaf_data, int64_t leaf_data_len,
                           const int32_t *leaf_indices, int64_t leaf_indices_len, int numerics,
                           topos_hip_program **program) {
  if (!program || n_nodes <= 0 || !nodes || (n_leaves > 0 && !leaves) || (leaf_data_len > 0 && !leaf_data) ||
      (leaf_indices_len > 0 && !leaf_indices) || n_leaves < 0 || leaf_data_len < 0 || leaf_indices_len < 0)
    return false;
  return numerics == TOPOS_HIP_EXACT || numerics == TOPOS_HIP_FAST;
}

}  // namespace

extern "C" {

int topos_hip_program_create(const topos_hip_node *nodes, int64_t n_nodes, const topos_hip_leaf *leaves,
                             int64_t n_leaves, const float *leaf_data, int64_t leaf_data_len,
                             const int32_t *leaf_indices, int64_t leaf_indices_len, int numerics,
                             topos_hip_program **program) {
  if (!table_arguments_valid(nodes, n_nodes, leaves, n_leaves, leaf_data, leaf_data_len, leaf_indices,
                             leaf_indices_len, numerics, program))
    return TOPOS_HIP_INVALID_ARGUMENT;
  *program = nullptr;
  const int status = Context::get().status();
  if (status != TOPOS_HIP_OK) return status;
  last_refusal().clear();
  auto p = std::make_unique<topos_hip_program>();
  p->nodes.assign(nodes, nodes + n_nodes);
  p->leaves.assign(leaves, leaves + n_leaves);
  return plan_program(std::move(p), leaf_data, leaf_data_len, leaf_indices, leaf_indices_len, numerics, program);
}

int topos_hip_program_create_backward(const topos_hip_node *nodes, int64_t n_nodes, const topos_hip_leaf *leaves,
                                      int64_t n_leaves, const float *leaf_data, int64_t leaf_data_len,
                                      const int32_t *leaf_indices, int64_t leaf_indices_len, int numerics,
                                      int64_t target, const int64_t *wrt, int64_t n_wrt,
                                      topos_hip_program **program) {
  if (!table_arguments_valid(nodes, n_nodes, leaves, n_leaves, leaf_data, leaf_data_len, leaf_indices,
                             leaf_indices_len, numerics, program) ||
      n_wrt < 0 || (n_wrt > 0 && !wrt))
    return TOPOS_HIP_INVALID_ARGUMENT;
  *program = nullptr;
  const int status = Context::get().status();
  if (status != TOPOS_HIP_OK) return status;
  last_refusal().clear();
  auto p = std::make_unique<topos_hip_program>();
  p->nodes.assign(nodes, nodes + n_nodes);
  p->leaves.assign(leaves, leaves + n_leaves);
  const int code = guarded([&] {
    try {
      append_engine_backward(p->nodes, p->leaves, target, std::vector<int64_t>(wrt, wrt + n_wrt), p->gradient_of);
    } catch (const InvalidArgument &e) {
      last_refusal() = e.message;
      throw;
    } catch (const Unsupported &e) {
      last_refusal() = e.message;
      throw;
    }
  });
  if (code != TOPOS_HIP_OK) return code;
  return plan_program(std::move(p), leaf_data, leaf_data_len, leaf_indices, leaf_indices_len, numerics, program);
}

int topos_hip_program_gradient(const topos_hip_program *program, int64_t node, int64_t *gradient_node) {
  if (!program || !gradient_node) return TOPOS_HIP_INVALID_ARGUMENT;
  const auto it = program->gradient_of.find(node);
  if (it == program->gradient_of.end()) return TOPOS_HIP_INVALID_ARGUMENT;
  *gradient_node = it->second;
  return TOPOS_HIP_OK;
}

int topos_hip_program_info(const topos_hip_program *program, uint64_t *arena_bytes, int64_t *launches,
                           int64_t *fused_groups) {
  if (!program) return TOPOS_HIP_INVALID_ARGUMENT;
  if (arena_bytes) *arena_bytes = program->arena_bytes;
  if (launches) *launches = (int64_t)program->launches.size();
  if (fused_groups) *fused_groups = program->fused_groups;
  return TOPOS_HIP_OK;
}

int topos_hip_program_bind(topos_hip_program *program, int is_input, int32_t slot, const float *device) {
  if (!program || !device || slot < 0) return TOPOS_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> guard(program->lock);
  auto &bound = (is_input ? program->inputs : program->parameters);
  auto old = bound.find(slot);
  if (old == bound.end() || old->second != device) program->drop_graph();
  bound[slot] = device;
  return TOPOS_HIP_OK;
}

int topos_hip_program_bind_selection(topos_hip_program *program, int32_t slot, const int32_t *indices, int64_t rows,
                                     float one) {
  if (!program || !indices || rows <= 0) return TOPOS_HIP_INVALID_ARGUMENT;
  const Storage *declared = nullptr;
  for (const Storage &s : program->storages)
    if (s.kind == StorageKind::kSelectionInput && s.index == slot) declared = &s;
  if (!declared) return TOPOS_HIP_INVALID_ARGUMENT;
  if (declared->rows != rows || __builtin_bit_cast(uint32_t, declared->one) != __builtin_bit_cast(uint32_t, one))
    return TOPOS_HIP_INVALID_ARGUMENT;
  for (int64_t r = 0; r < rows; ++r)
    if (indices[r] < 0 || indices[r] >= declared->vocab) return TOPOS_HIP_INVALID_ARGUMENT;
  if (!program->device) return TOPOS_HIP_OK;
  const int64_t vocab = declared->vocab;
  std::lock_guard<std::mutex> guard(program->lock);
  program->drop_graph();
  return guarded([&] {
    auto old = program->selection_inputs.find(slot);
    if (old != program->selection_inputs.end()) {
      check(hipDeviceSynchronize(), "hipDeviceSynchronize(rebind selection)");
      hipFree(old->second.indices);
      hipFree(old->second.row_start);
      hipFree(old->second.sources);
      program->selection_inputs.erase(old);
    }
    program->selection_inputs[slot] = program->upload_selection(indices, rows, vocab, false);
  });
}

int topos_hip_program_run(topos_hip_program *program, void *stream) {
  if (!program) return TOPOS_HIP_INVALID_ARGUMENT;
  const int status = Context::get().status();
  if (status != TOPOS_HIP_OK) return status;
  std::lock_guard<std::mutex> guard(program->lock);
  return guarded([&] {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    program->prepare();
    program->serialize_before(s);
    program->run(s);
    program->record_after(s);
  });
}

int topos_hip_program_replay(topos_hip_program *program, void *stream) {
  if (!program) return TOPOS_HIP_INVALID_ARGUMENT;
  const int status = Context::get().status();
  if (status != TOPOS_HIP_OK) return status;
  std::lock_guard<std::mutex> guard(program->lock);
  return guarded([&] {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    program->prepare();
    program->serialize_before(s);
    program->replay(s);
    program->record_after(s);
  });
}

int topos_hip_program_run_profiled(topos_hip_program *program, void *stream, float *milliseconds) {
  if (!program || !milliseconds) return TOPOS_HIP_INVALID_ARGUMENT;
  const int status = Context::get().status();
  if (status != TOPOS_HIP_OK) return status;
  std::lock_guard<std::mutex> guard(program->lock);
  return guarded([&] {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    program->prepare();
    program->serialize_before(s);
    program->run(s, milliseconds);
    program->record_after(s);
  });
}

int topos_hip_program_launch(const topos_hip_program *program, int64_t launch, const char **kind, double *flops,
                             double *bytes) {
  if (!program || launch < 0 || launch >= (int64_t)program->launches.size()) return TOPOS_HIP_INVALID_ARGUMENT;
  const auto &l = program->launches[launch];
  if (kind) *kind = l.kind.c_str();
  if (flops) *flops = l.flops;
  if (bytes) *bytes = l.bytes;
  return TOPOS_HIP_OK;
}

namespace {
int program_output(const topos_hip_program *program, int64_t node, const float **device) {
  if (!program || !device) return TOPOS_HIP_INVALID_ARGUMENT;
  auto it = program->output_storage.find(node);
  if (it == program->output_storage.end()) return TOPOS_HIP_INVALID_ARGUMENT;
  if (!program->device || (program->storages[it->second].kind == StorageKind::kArena && !program->arena))
    return TOPOS_HIP_INVALID_ARGUMENT;
  int code = guarded([&] {
    *device = (const float *)program->base(it->second) + program->output_offset.at(node);
  });
  return code;
}
}  // namespace

int topos_hip_program_output(const topos_hip_program *program, int64_t node, const float **device) {
  if (!program) return TOPOS_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> guard(program->lock);
  return program_output(program, node, device);
}

int topos_hip_program_read(const topos_hip_program *program, int64_t node, float *host, int64_t count) {
  if (!program || !host || node < 0 || node >= (int64_t)program->nodes.size()) return TOPOS_HIP_INVALID_ARGUMENT;
  if (count != topos_hip_program::volume_of(program->nodes[node])) return TOPOS_HIP_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> guard(program->lock);
  const float *device = nullptr;
  const int code = program_output(program, node, &device);
  if (code != TOPOS_HIP_OK) return code;
  return guarded([&] {
    check(hipDeviceSynchronize(), "hipDeviceSynchronize(read)");
    check(hipMemcpy(host, device, count * 4, hipMemcpyDeviceToHost), "hipMemcpy(read)");
  });
}

const char *topos_hip_last_refusal(void) { return last_refusal().c_str(); }

const char *topos_hip_program_describe(const topos_hip_program *program) {
  return program ? program->description.c_str() : "";
}

void topos_hip_program_destroy(topos_hip_program *program) { delete program; }

int topos_hip_sgd_step_f32(float *parameter, const float *gradient, int64_t count, float rate, void *stream) {
  if (count < 0 || (count > 0 && (!parameter || !gradient))) return TOPOS_HIP_INVALID_ARGUMENT;
  const int status = Context::get().status();
  if (status != TOPOS_HIP_OK) return status;
  return guarded([&] { launch_sgd(parameter, gradient, count, rate, static_cast<hipStream_t>(stream)); });
}

int topos_hip_adamw_step_f32(float *parameter, const float *gradient, float *first, float *second, int64_t count,
                             float beta1, float beta2, float first_share, float second_share, float first_correction,
                             float second_correction, float epsilon, float rate, float decay, int decayed,
                             void *stream) {
  if (count < 0 || (count > 0 && (!parameter || !gradient || !first || !second))) return TOPOS_HIP_INVALID_ARGUMENT;
  const int status = Context::get().status();
  if (status != TOPOS_HIP_OK) return status;
  return guarded([&] {
    launch_adamw(parameter, gradient, first, second, count, beta1, beta2, first_share, second_share, first_correction,
                 second_correction, epsilon, rate, decay, decayed, static_cast<hipStream_t>(stream));
  });
}

int topos_hip_adamw_step_multi_f32(const topos_hip_adamw_tensor *tensors, int64_t count, float beta1, float beta2,
                                   float first_share, float second_share, float first_correction,
                                   float second_correction, float epsilon, float rate, float decay, void *stream) {
  if (count < 0 || (count > 0 && !tensors)) return TOPOS_HIP_INVALID_ARGUMENT;
  for (int64_t j = 0; j < count; ++j) {
    const topos_hip_adamw_tensor &x = tensors[j];
    if (x.count < 0 || (x.count > 0 && (!x.parameter || !x.gradient || !x.first || !x.second)))
      return TOPOS_HIP_INVALID_ARGUMENT;
  }
  const int status = Context::get().status();
  if (status != TOPOS_HIP_OK) return status;
  return guarded([&] {
    AdamTable table{};
    auto flush = [&] {
      launch_adamw_multi(table, beta1, beta2, first_share, second_share, first_correction, second_correction,
                         epsilon, rate, decay, static_cast<hipStream_t>(stream));
      table = AdamTable{};
    };
    // Entries of one launch run concurrently, so an entry whose buffers
    // overlap what an earlier entry of the launch writes (a tied parameter
    // listed twice, a gradient aliasing another entry's moment) starts a new
    // launch: the updates then land in table order, as the one-tensor entry
    // applied them.
    auto overlaps = [](const void *p, int64_t n, const void *q, int64_t m) {
      const char *a = static_cast<const char *>(p), *b = static_cast<const char *>(q);
      return a < b + m * (int64_t)sizeof(float) && b < a + n * (int64_t)sizeof(float);
    };
    auto conflicts = [&](const topos_hip_adamw_tensor &x) {
      for (int i = 0; i < table.count; ++i) {
        const int64_t n = table.start[i + 1] - table.start[i];
        const void *written[3] = {table.parameter[i], table.first[i], table.second[i]};
        const void *mine[4] = {x.parameter, x.first, x.second, x.gradient};
        for (const void *w : written)
          for (const void *q : mine)
            if (overlaps(w, n, q, x.count)) return true;
        const void *my_writes[3] = {x.parameter, x.first, x.second};
        for (const void *q : my_writes)
          if (overlaps(table.gradient[i], n, q, x.count)) return true;
      }
      return false;
    };
    for (int64_t j = 0; j < count; ++j) {
      const topos_hip_adamw_tensor &x = tensors[j];
      if (x.count == 0) continue;
      if (table.count > 0 && conflicts(x)) flush();
      const int at = table.count;
      table.parameter[at] = x.parameter;
      table.gradient[at] = x.gradient;
      table.first[at] = x.first;
      table.second[at] = x.second;
      table.decayed[at] = x.decayed != 0;
      table.start[at + 1] = table.start[at] + x.count;
      table.count = at + 1;
      if (table.count == kAdamTensors) flush();
    }
    if (table.count > 0) flush();
  });
}

}  // extern "C"
