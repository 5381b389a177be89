// The public chain entry points (topos_hip_chain_*): a chain descriptor of
// the C ABI becomes an expression of the shared code generator (codegen.cpp)
// and is compiled once into a kernel of its own.
//
// The reference has no elementwise fusion: every node of a chain like
// x / (exp(-x) + 1) + b materialises a full tensor through Tensor::zip/map
// (src/payload/tensor.rs:365-510). A generated chain reads each input once
// through its strided view (stride 0 for the broadcast_along / broadcast_like
// operands, src/payload/layout.rs:140-147), keeps every intermediate in
// registers, and writes each requested result once, contiguous.
#include <memory>

#include "codegen.hpp"

struct topos_hip_chain {
  topos_hip::Expr expr;
  topos_hip::Generated generated;
};

namespace topos_hip {

topos_hip_chain *create_chain(const topos_hip_chain_desc &d, bool load) {
  if (d.rank < 0 || d.rank > TOPOS_HIP_MAX_RANK) throw InvalidArgument{"chain rank out of range"};
  if (d.n_inputs < 0 || d.n_steps < 0 || d.n_outputs <= 0) throw InvalidArgument{"chain counts"};
  if ((d.n_inputs && !d.inputs) || (d.n_steps && !d.steps) || !d.outputs)
    throw InvalidArgument{"chain arrays missing"};
  Expr e;
  e.rank = d.rank;
  for (int a = 0; a < d.rank; ++a) e.shape[a] = d.shape[a];
  for (int i = 0; i < d.n_inputs; ++i) {
    const topos_hip_layout &l = d.inputs[i];
    if (l.rank != d.rank) throw InvalidArgument{"chain input rank differs from the chain shape"};
    ExprInput in;
    for (int a = 0; a < d.rank; ++a) {
      if (l.shape[a] != d.shape[a] || l.strides[a] < 0)
        throw InvalidArgument{"chain input layout differs from the chain shape"};
      in.strides[a] = l.strides[a];
    }
    if (l.offset < 0) throw InvalidArgument{"chain input offset"};
    in.offset = l.offset;
    e.inputs.push_back(in);
  }
  for (int s = 0; s < d.n_steps; ++s) e.steps.push_back(ExprStep{d.steps[s].op, d.steps[s].left, d.steps[s].right});
  for (int o = 0; o < d.n_outputs; ++o) e.outputs.push_back(d.outputs[o]);
  auto chain = std::make_unique<topos_hip_chain>();
  chain->expr = e;
  chain->generated = generate_chain(e);
  compile_kernels({chain->generated}, load);
  return chain.release();
}

void launch_chain(const topos_hip_chain &chain, const float *const *inputs, float *const *outputs,
                  hipStream_t stream) {
  if (!chain.expr.inputs.empty() && !inputs) throw InvalidArgument{"chain inputs missing"};
  std::vector<const void *> pointers(chain.expr.inputs.size());
  for (size_t i = 0; i < pointers.size(); ++i) pointers[i] = inputs[i];
  launch_generated_chain(chain.generated, chain.expr, pointers.data(), outputs, stream);
}

}  // namespace topos_hip

extern "C" {

const char *topos_hip_chain_source(const topos_hip_chain *chain) {
  return chain && chain->generated ? chain->generated->source.c_str() : "";
}

void topos_hip_chain_destroy(topos_hip_chain *chain) { delete chain; }

}  // extern "C"
