// The engine-backward route on the device: Run::backward's reverse scan
// (src/engine/run.rs:229-318) performed by the library over a forward plan's
// node table, appending each derivative rule's operations as nodes of the
// same device program, which then plans and runs forward and backward as one.
//
// The scan follows the reference step for step:
//   * the target must be a scalar (run.rs:242-261);
//   * its gradient is one_like of its value, every other gradient starts as
//     zero_like (a Constant zero) and accumulates `gradient + contribution` in
//     reverse scan order (run.rs:266-313), so the first contribution maps -0
//     to +0 exactly as the interpreter does;
//   * only ancestors run their rules, and only a present (`Some`) cotangent
//     marks its operand an ancestor (run.rs:275-313): a broadcast's reference,
//     a gather's or scatter's selection and both operands of `step` are data
//     edges;
//   * each rule records the operations of its `backward` (src/function/*.rs) in
//     the order the rule evaluates them (the rules are generic over the payload
//     and the recorder alike, src/function/function.rs:480-518, which is why
//     this route and Tape::differentiate's recorded gradients agree bit for
//     bit).
// The forward values the rules read stay live until their last reader: the
// retain-what-backward-reads arena of a Request::backward() plan
// (src/engine/plan.rs:612-621).
#include <map>
#include <optional>
#include <string>
#include <vector>

#include "backend.hpp"

namespace topos_hip {
namespace {

struct Shape {
  int rank = 0;
  int64_t axes[TOPOS_HIP_MAX_RANK] = {};
  int64_t volume() const {
    int64_t v = 1;
    for (int d = 0; d < rank; ++d) v *= axes[d];
    return v;
  }
  bool operator==(const Shape &o) const {
    if (rank != o.rank) return false;
    for (int d = 0; d < rank; ++d)
      if (axes[d] != o.axes[d]) return false;
    return true;
  }
};

using Cotangent = std::optional<int64_t>;

// The node table under construction, with the recording helpers the rules
// use (each mirrors one Tensorial operation of the payload).
class Recorder {
 public:
  Recorder(std::vector<topos_hip_node> &nodes, std::vector<topos_hip_leaf> &leaves)
      : nodes_(nodes), leaves_(leaves) {}

  Shape shape(int64_t node) const {
    Shape s;
    s.rank = nodes_[node].rank;
    for (int d = 0; d < s.rank; ++d) s.axes[d] = nodes_[node].shape[d];
    return s;
  }

  // A Constant payload of `value` over `shape` (counted / zero_like /
  // one_like: Storage::Constant, src/payload/storage.rs:36-51).
  int64_t constant(const Shape &shape, float value) {
    topos_hip_leaf leaf{};
    leaf.kind = TOPOS_HIP_LEAF_CONSTANT;
    leaf.value = value;
    leaves_.push_back(leaf);
    topos_hip_node node = blank(TOPOS_HIP_OP_LEAF, shape);
    node.slot = (int32_t)(leaves_.size() - 1);
    return push(node);
  }
  int64_t zero_like(int64_t x) { return constant(shape(x), 0.0f); }
  int64_t one_like(int64_t x) { return constant(shape(x), 1.0f); }

  int64_t unary(int op, int64_t x) { return record(op, x, -1, shape(x)); }
  int64_t binary(int op, int64_t x, int64_t y) {
    if (!(shape(x) == shape(y))) throw InvalidArgument{"backward: elementwise operands of different shapes"};
    return record(op, x, y, shape(x));
  }
  int64_t add(int64_t x, int64_t y) { return binary(TOPOS_HIP_OP_ADD, x, y); }
  int64_t sub(int64_t x, int64_t y) { return binary(TOPOS_HIP_OP_SUB, x, y); }
  int64_t mul(int64_t x, int64_t y) { return binary(TOPOS_HIP_OP_MUL, x, y); }
  int64_t div(int64_t x, int64_t y) { return binary(TOPOS_HIP_OP_DIV, x, y); }
  int64_t neg(int64_t x) { return unary(TOPOS_HIP_OP_NEG, x); }

  int64_t matmul(int64_t a, int64_t b) {
    Shape sa = shape(a), sb = shape(b), out = sa;
    if (sa.rank < 2 || sa.rank != sb.rank || sa.axes[sa.rank - 1] != sb.axes[sb.rank - 2])
      throw InvalidArgument{"backward: matmul of incompatible shapes"};
    out.axes[out.rank - 1] = sb.axes[sb.rank - 1];
    return record(TOPOS_HIP_OP_MATMUL, a, b, out);
  }
  int64_t transpose(int64_t x) {
    Shape s = shape(x), out = s;
    if (s.rank == 2) std::swap(out.axes[0], out.axes[1]);
    return record(TOPOS_HIP_OP_TRANSPOSE, x, -1, out);
  }
  int64_t permute(int64_t x, const std::vector<int64_t> &order) {
    Shape s = shape(x), out = s;
    topos_hip_node node = blank(TOPOS_HIP_OP_PERMUTE, out);
    for (int d = 0; d < s.rank; ++d) {
      node.shape[d] = s.axes[order[d]];
      node.params[d] = order[d];
    }
    node.operands[0] = (int32_t)x;
    return push(node);
  }
  // The trailing-axes swap of src/function/matmul.rs:89-97.
  int64_t swapped(int64_t x) {
    const int rank = shape(x).rank;
    if (rank <= 2) return transpose(x);
    std::vector<int64_t> order(rank);
    for (int d = 0; d < rank; ++d) order[d] = d;
    std::swap(order[rank - 2], order[rank - 1]);
    return permute(x, order);
  }
  int64_t sum(int64_t x) { return record(TOPOS_HIP_OP_SUM, x, -1, Shape{}); }
  int64_t sum_along(int64_t x, int64_t axis) {
    Shape s = shape(x), out;
    for (int d = 0; d < s.rank; ++d)
      if (d != axis) out.axes[out.rank++] = s.axes[d];
    return record(TOPOS_HIP_OP_SUM_ALONG, x, -1, out, {axis});
  }
  int64_t broadcast_like(int64_t x, int64_t like) {
    if (shape(x).volume() != 1) throw InvalidArgument{"backward: broadcast of more than one element"};
    return record(TOPOS_HIP_OP_BROADCAST, x, like, shape(like));
  }
  int64_t broadcast_along(int64_t x, int64_t axis, int64_t like) {
    return record(TOPOS_HIP_OP_BROADCAST_ALONG, x, like, shape(like), {axis});
  }
  int64_t reshape(int64_t x, const Shape &to) { return record(TOPOS_HIP_OP_RESHAPE, x, -1, to); }
  int64_t narrow(int64_t x, int64_t axis, int64_t start, int64_t length) {
    Shape out = shape(x);
    out.axes[axis] = length;
    return record(TOPOS_HIP_OP_NARROW, x, -1, out, {axis, start, length});
  }
  int64_t pad(int64_t x, int64_t axis, int64_t start, int64_t full) {
    Shape out = shape(x);
    out.axes[axis] = full;
    return record(TOPOS_HIP_OP_PAD, x, -1, out, {axis, start, full});
  }
  int64_t unfold(int64_t x, int64_t axis, int64_t size, int64_t step, int64_t dilation) {
    const Shape s = shape(x);
    Shape out;
    out.rank = s.rank + 1;
    for (int d = 0; d < out.rank; ++d)
      out.axes[d] = d < axis ? s.axes[d]
                    : d == axis ? (s.axes[axis] - dilation * (size - 1) - 1) / step + 1
                    : d == axis + 1 ? size
                                    : s.axes[d - 1];
    if (out.rank > TOPOS_HIP_MAX_RANK) throw InvalidArgument{"backward: unfold beyond the library's axes"};
    return record(TOPOS_HIP_OP_UNFOLD, x, -1, out, {axis, size, step, dilation});
  }
  int64_t fold(int64_t x, int64_t axis, int64_t size, int64_t step, int64_t dilation, int64_t extent) {
    const Shape s = shape(x);
    Shape out;
    out.rank = s.rank - 1;
    for (int d = 0; d < out.rank; ++d) out.axes[d] = d < axis ? s.axes[d] : d == axis ? extent : s.axes[d + 1];
    return record(TOPOS_HIP_OP_FOLD, x, -1, out, {axis, size, step, dilation, extent});
  }
  int64_t gather(int64_t table, int64_t selection) {
    Shape out = shape(table);
    out.axes[0] = shape(selection).axes[0];
    return record(TOPOS_HIP_OP_GATHER, table, selection, out);
  }
  int64_t scatter(int64_t x, int64_t selection, int64_t rows) {
    Shape out = shape(x);
    out.axes[0] = rows;
    return record(TOPOS_HIP_OP_SCATTER, x, selection, out, {rows});
  }
  int64_t step(int64_t x, int64_t threshold) { return binary(TOPOS_HIP_OP_STEP, x, threshold); }
  int64_t powf(int64_t x, int64_t exponent) { return binary(TOPOS_HIP_OP_POWF, x, exponent); }

  size_t size() const { return nodes_.size(); }
  const topos_hip_node &node(int64_t i) const { return nodes_[i]; }

 private:
  static topos_hip_node blank(int op, const Shape &shape) {
    topos_hip_node node{};
    node.op = op;
    node.rank = shape.rank;
    for (int d = 0; d < TOPOS_HIP_MAX_RANK; ++d) node.shape[d] = d < shape.rank ? shape.axes[d] : 0;
    node.operands[0] = node.operands[1] = -1;
    node.slot = -1;
    return node;
  }
  int64_t record(int op, int64_t a, int64_t b, const Shape &shape, std::initializer_list<int64_t> params = {}) {
    topos_hip_node node = blank(op, shape);
    node.operands[0] = (int32_t)a;
    node.operands[1] = (int32_t)b;
    int d = 0;
    for (int64_t p : params) node.params[d++] = p;
    return push(node);
  }
  int64_t push(const topos_hip_node &node) {
    if (nodes_.size() >= (size_t)INT32_MAX) throw InvalidArgument{"backward: node table too large"};
    nodes_.push_back(node);
    return (int64_t)nodes_.size() - 1;
  }

  std::vector<topos_hip_node> &nodes_;
  std::vector<topos_hip_leaf> &leaves_;
};

// One variant's derivative rule (Function::backward,
// src/function/function.rs:480-518): the cotangent of each operand, or none
// for a data edge.
std::vector<Cotangent> rule(Recorder &r, int64_t index, int64_t g) {
  const topos_hip_node node = r.node(index);  // a copy: recording grows the table
  const int64_t a = node.operands[0], b = node.operands[1];
  switch (node.op) {
    case TOPOS_HIP_OP_ADD:  // add.rs:40-42
      return {g, g};
    case TOPOS_HIP_OP_SUB:  // sub.rs:41-43
      return {g, r.neg(g)};
    case TOPOS_HIP_OP_MUL: {  // mul.rs:46-52
      const int64_t first = r.mul(g, b);
      return {first, r.mul(g, a)};
    }
    case TOPOS_HIP_OP_DIV: {  // div.rs:46-52: g / right, -(g * output / right)
      const int64_t first = r.div(g, b);
      const int64_t scaled = r.div(r.mul(g, index), b);
      return {first, r.neg(scaled)};
    }
    case TOPOS_HIP_OP_NEG:  // neg.rs:38-40
      return {r.neg(g)};
    case TOPOS_HIP_OP_TANH: {  // tanh.rs:41-44: one_like - output * output
      const int64_t one = r.one_like(index);
      const int64_t derivative = r.sub(one, r.mul(index, index));
      return {r.mul(g, derivative)};
    }
    case TOPOS_HIP_OP_EXP:  // exp.rs:40-42
      return {r.mul(g, index)};
    case TOPOS_HIP_OP_LN:  // ln.rs:42-45
      return {r.div(g, a)};
    case TOPOS_HIP_OP_SQRT:  // sqrt.rs:43-45: g / (output + output)
      return {r.div(g, r.add(index, index))};
    case TOPOS_HIP_OP_POWF: {  // powf.rs:48-54
      const int64_t lowered = r.sub(b, r.one_like(b));
      const int64_t scaled = r.mul(g, b);
      const int64_t base_cotangent = r.mul(scaled, r.powf(a, lowered));
      const int64_t carried = r.mul(g, index);
      const int64_t exponent_cotangent = r.mul(carried, r.unary(TOPOS_HIP_OP_LN, a));
      return {base_cotangent, exponent_cotangent};
    }
    case TOPOS_HIP_OP_MAXIMUM: {  // maximum.rs:45-51
      const int64_t winners = r.step(a, b);
      const int64_t left = r.mul(g, winners);
      const int64_t right = r.mul(g, r.sub(r.one_like(winners), winners));
      return {left, right};
    }
    case TOPOS_HIP_OP_RELU: {  // relu.rs:47-50: g * operand.step(operand.zero_like())
      const int64_t zero = r.zero_like(a);
      return {r.mul(g, r.step(a, zero))};
    }
    case TOPOS_HIP_OP_STEP:  // step.rs:47-49
      return {std::nullopt, std::nullopt};
    case TOPOS_HIP_OP_MATMUL: {  // matmul.rs:76-82: g . swapped(right), swapped(left) . g
      const int64_t first = r.matmul(g, r.swapped(b));
      return {first, r.matmul(r.swapped(a), g)};
    }
    case TOPOS_HIP_OP_TRANSPOSE:  // transpose.rs:42-44
      return {r.transpose(g)};
    case TOPOS_HIP_OP_SUM:  // sum.rs:38-41
      return {r.broadcast_like(g, a)};
    case TOPOS_HIP_OP_SUM_ALONG:  // sum_along.rs:41-44
      return {r.broadcast_along(g, node.params[0], a)};
    case TOPOS_HIP_OP_BROADCAST:  // broadcast.rs:51-57: g.sum().broadcast_like(operand)
      return {r.broadcast_like(r.sum(g), a), std::nullopt};
    case TOPOS_HIP_OP_BROADCAST_ALONG:  // broadcast_along.rs:52-54
      return {r.sum_along(g, node.params[0]), std::nullopt};
    case TOPOS_HIP_OP_RESHAPE:  // reshape.rs:48-51
      return {r.reshape(g, r.shape(a))};
    case TOPOS_HIP_OP_PERMUTE: {  // permute.rs:68-70: the inverse order
      std::vector<int64_t> inverse(node.rank);
      for (int d = 0; d < node.rank; ++d) inverse[node.params[d]] = d;
      return {r.permute(g, inverse)};
    }
    case TOPOS_HIP_OP_NARROW:  // narrow.rs:70-74
      return {r.pad(g, node.params[0], node.params[1], r.shape(a).axes[node.params[0]])};
    case TOPOS_HIP_OP_PAD:  // pad.rs:68-72
      return {r.narrow(g, node.params[0], node.params[1], r.shape(a).axes[node.params[0]])};
    case TOPOS_HIP_OP_GATHER:  // gather.rs:64-68
      return {r.scatter(g, b, r.shape(a).axes[0]), std::nullopt};
    case TOPOS_HIP_OP_SCATTER:  // scatter.rs:79-82
      return {r.gather(g, b), std::nullopt};
    case TOPOS_HIP_OP_LOG_SOFTMAX: {  // log_softmax.rs:67-72: g - output.exp() * total
      const int64_t axis = node.params[0];
      const int64_t total = r.broadcast_along(r.sum_along(g, axis), axis, g);
      return {r.sub(g, r.mul(r.unary(TOPOS_HIP_OP_EXP, index), total))};
    }
    case TOPOS_HIP_OP_LOG_SUM_EXP: {  // log_sum_exp.rs:65-74
      const int64_t axis = node.params[0];
      const int64_t probabilities = r.unary(TOPOS_HIP_OP_EXP, r.sub(a, r.broadcast_along(index, axis, a)));
      return {r.mul(r.broadcast_along(g, axis, a), probabilities)};
    }
    case TOPOS_HIP_OP_UNFOLD:  // unfold.rs:77-87: the fold onto the operand's extent
      return {r.fold(g, node.params[0], node.params[1], node.params[2], node.params[3],
                     r.shape(a).axes[node.params[0]])};
    case TOPOS_HIP_OP_FOLD:  // fold.rs:91-98: the unfold by the same parameters
      return {r.unfold(g, node.params[0], node.params[1], node.params[2], node.params[3])};
  }
  throw InvalidArgument{"backward: unknown node kind " + std::to_string(node.op)};
}

}  // namespace

void append_engine_backward(std::vector<topos_hip_node> &nodes, std::vector<topos_hip_leaf> &leaves, int64_t target,
                            const std::vector<int64_t> &wrt, std::map<int64_t, int64_t> &gradient_of) {
  const int64_t forward = (int64_t)nodes.size();
  if (target < 0 || target >= forward) throw InvalidArgument{"backward: the target is not a node of the program"};
  for (int64_t w : wrt)
    if (w < 0 || w >= forward) throw InvalidArgument{"backward: a gradient was asked of a node outside the program"};
  if (nodes[target].rank != 0) throw InvalidArgument{"backward requires a scalar target; reduce it with `sum` first"};
  for (int64_t i = 0; i < forward; ++i)
    for (int k = 0; k < 2; ++k)
      if (nodes[i].operands[k] >= i) throw InvalidArgument{"backward: an operand does not precede its consumer"};
  Recorder r(nodes, leaves);
  // gradients[i] < 0: still the zero_like seed (no contribution yet).
  std::vector<int64_t> gradients(target + 1, -1);
  gradients[target] = r.one_like(target);
  std::vector<bool> ancestors(target + 1, false);
  ancestors[target] = true;
  for (int64_t index = target; index >= 0; --index) {
    if (!ancestors[index]) continue;
    const topos_hip_node node = nodes[index];
    const int arity = node.operands[0] < 0 ? 0 : node.operands[1] < 0 ? 1 : 2;
    if (arity == 0) continue;  // Leaf, Parameter, Input: no cotangents
    int64_t g = gradients[index];
    if (g < 0) g = gradients[index] = r.zero_like(index);  // an ancestor reached only through data edges
    const std::vector<Cotangent> cotangents = rule(r, index, g);
    if ((int)cotangents.size() != arity) throw InvalidArgument{"backward: a rule's cotangents do not match its arity"};
    for (int k = 0; k < arity; ++k) {
      if (!cotangents[k]) continue;
      const int64_t link = node.operands[k];
      ancestors[link] = true;
      const int64_t seed = gradients[link] >= 0 ? gradients[link] : r.zero_like(link);
      gradients[link] = r.add(seed, *cotangents[k]);
    }
  }
  for (int64_t w : wrt) {
    if (gradient_of.count(w)) continue;
    // Values after the target, and values the target does not depend on,
    // keep their zero_like gradient.
    const int64_t g = w <= target && gradients[w] >= 0 ? gradients[w] : r.zero_like(w);
    nodes[g].flags |= TOPOS_HIP_NODE_READABLE;
    gradient_of[w] = g;
  }
}

}  // namespace topos_hip
