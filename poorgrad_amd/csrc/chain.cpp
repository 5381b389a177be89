// Generated elementwise/broadcast chain kernels.
//
// The reference has no elementwise fusion: every node of a chain like
// x / (exp(-x) + 1) + b materialises a full tensor through Tensor::zip/map
// (src/payload/tensor.rs:365-510). Here a whole chain becomes one kernel:
// its inputs are read once through their strided views (stride 0 for the
// broadcast_along / broadcast_like operands, src/payload/layout.rs:140-147),
// every intermediate lives in registers, and each requested result is written
// once, contiguous. Each operation rounds to f32 exactly as the materialised
// intermediate would (no contraction, no fast math), so the results are the
// interpreter's bits.
//
// The source is generated per chain with the shape, strides and offsets as
// constants (index arithmetic by constant divisors) and compiled by hipRTC for
// gfx950, cached per process by source text. Each lane handles four
// consecutive output elements: 16-byte loads for unit-stride operands whose
// innermost extent keeps the quad in one row, one load and a splat for
// stride-0 operands, and 16-byte stores.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

#include "backend.hpp"
#include "faithful_math_text.h"  // kFaithfulMathText: faithful_math.h as a string


namespace topos_hip {
namespace {

struct Compiled {
  hipModule_t module;
  hipFunction_t function;
};

std::mutex cache_lock;
std::map<std::string, Compiled> &cache() {
  static auto *compiled = new std::map<std::string, Compiled>();
  return *compiled;
}

const char *unary_expression(int op) {
  switch (op) {
    case TOPOS_HIP_CHAIN_NEG: return "(-%a)";
    case TOPOS_HIP_CHAIN_EXP: return "topos_faithful::exp_f32(%a)";
    case TOPOS_HIP_CHAIN_LN: return "topos_faithful::ln_f32(%a)";
    case TOPOS_HIP_CHAIN_SQRT: return "__builtin_sqrtf(%a)";
    case TOPOS_HIP_CHAIN_TANH: return "topos_faithful::tanh_f32(%a)";
  }
  return nullptr;
}

const char *binary_expression(int op) {
  switch (op) {
    case TOPOS_HIP_CHAIN_ADD: return "(%a + %b)";
    case TOPOS_HIP_CHAIN_SUB: return "(%a - %b)";
    case TOPOS_HIP_CHAIN_MUL: return "(%a * %b)";
    case TOPOS_HIP_CHAIN_DIV: return "(%a / %b)";
    case TOPOS_HIP_CHAIN_MAX: return "topos_faithful::max_f32(%a, %b)";
    case TOPOS_HIP_CHAIN_STEP: return "topos_faithful::step_f32(%a, %b)";
  }
  return nullptr;
}

std::string substitute(const char *pattern, const std::string &a, const std::string &b) {
  std::string out;
  for (const char *p = pattern; *p; ++p) {
    if (p[0] == '%' && p[1] == 'a') {
      out += a;
      ++p;
    } else if (p[0] == '%' && p[1] == 'b') {
      out += b;
      ++p;
    } else {
      out += *p;
    }
  }
  return out;
}

std::string reference(int32_t value, const std::string &lane) {
  if (value < 0) return "in" + std::to_string(-value - 1) + "_" + lane;
  return "s" + std::to_string(value) + "_" + lane;
}

void validate(const topos_hip_chain_desc &d) {
  if (d.rank < 0 || d.rank > TOPOS_HIP_MAX_RANK) throw InvalidArgument{"chain rank out of range"};
  for (int a = 0; a < d.rank; ++a)
    if (d.shape[a] <= 0) throw InvalidArgument{"chain shape must be non-empty"};
  if (d.n_inputs < 0 || d.n_steps < 0 || d.n_outputs <= 0) throw InvalidArgument{"chain counts"};
  if ((d.n_inputs && !d.inputs) || (d.n_steps && !d.steps) || !d.outputs)
    throw InvalidArgument{"chain arrays missing"};
  for (int i = 0; i < d.n_inputs; ++i) {
    const topos_hip_layout &l = d.inputs[i];
    if (l.rank != d.rank) throw InvalidArgument{"chain input rank differs from the chain shape"};
    for (int a = 0; a < d.rank; ++a)
      if (l.shape[a] != d.shape[a] || l.strides[a] < 0)
        throw InvalidArgument{"chain input layout differs from the chain shape"};
    if (l.offset < 0) throw InvalidArgument{"chain input offset"};
  }
  auto check_ref = [&](int32_t v, int32_t step) {
    if (v < 0 ? (-v - 1) >= d.n_inputs : v >= step) throw InvalidArgument{"chain operand reference"};
  };
  for (int s = 0; s < d.n_steps; ++s) {
    const topos_hip_chain_step &st = d.steps[s];
    const bool unary = unary_expression(st.op) != nullptr;
    if (!unary && !binary_expression(st.op)) throw InvalidArgument{"unknown chain operation"};
    check_ref(st.left, s);
    if (!unary) check_ref(st.right, s);
  }
  for (int o = 0; o < d.n_outputs; ++o) check_ref(d.outputs[o], d.n_steps);
}

std::string generate(const topos_hip_chain_desc &d, bool quads, const std::vector<bool> &vector_in) {
  std::ostringstream s;
  s << "#pragma clang fp contract(off)\n" << kFaithfulMathText << "\n";
  s << "extern \"C\" __global__ __launch_bounds__(256) void topos_chain(";
  for (int i = 0; i < d.n_inputs; ++i) s << "const float* __restrict__ p" << i << ", ";
  for (int o = 0; o < d.n_outputs; ++o) s << "float* __restrict__ q" << o << ", ";
  s << "int vector_ok) {\n";
  int64_t volume = 1;
  for (int a = 0; a < d.rank; ++a) volume *= d.shape[a];
  s << "  const long long volume = " << volume << "LL;\n";
  s << "  const long long step = (long long)gridDim.x * 256 * 4;\n";
  s << "  for (long long base = ((long long)blockIdx.x * 256 + threadIdx.x) * 4; base < volume; base += step) {\n";
  const int inner_axis = d.rank - 1;
  // Coordinates of flat index `f` (lane j of the quad), outermost first.
  auto coordinates = [&](const std::string &flat, const std::string &tag) {
    std::string rem = flat;
    for (int a = d.rank - 1; a >= 0; --a) {
      s << "    const long long c" << a << "_" << tag << " = (" << rem << ") % " << d.shape[a] << "LL;\n";
      if (a > 0) {
        s << "    const long long r" << a << "_" << tag << " = (" << rem << ") / " << d.shape[a] << "LL;\n";
        rem = "r" + std::to_string(a) + "_" + tag;
      }
    }
  };
  auto address = [&](const topos_hip_layout &l, const std::string &tag) {
    std::string e = std::to_string(l.offset) + "LL";
    for (int a = 0; a < d.rank; ++a)
      if (l.strides[a] != 0) e += " + c" + std::to_string(a) + "_" + tag + " * " + std::to_string(l.strides[a]) + "LL";
    return e;
  };
  auto body = [&](const std::vector<std::string> &lanes) {
    for (int st = 0; st < d.n_steps; ++st) {
      const topos_hip_chain_step &x = d.steps[st];
      const char *u = unary_expression(x.op);
      for (const std::string &lane : lanes) {
        const std::string a = reference(x.left, lane);
        const std::string expr = u ? substitute(u, a, "") : substitute(binary_expression(x.op), a, reference(x.right, lane));
        s << "    const float s" << st << "_" << lane << " = " << expr << ";\n";
      }
    }
  };
  const std::vector<std::string> lanes = {"0", "1", "2", "3"};
  if (quads && d.rank > 0) {
    s << "    if (base + 3 < volume) {\n";
    coordinates("base", "q");
    for (int i = 0; i < d.n_inputs; ++i) {
      const topos_hip_layout &l = d.inputs[i];
      const long long inner = l.strides[inner_axis];
      s << "    const long long a" << i << " = " << address(l, "q") << ";\n";
      if (inner == 0) {
        s << "    const float in" << i << "_0 = p" << i << "[a" << i << "];\n";
        for (int j = 1; j < 4; ++j) s << "    const float in" << i << "_" << j << " = in" << i << "_0;\n";
      } else if (inner == 1 && vector_in[i]) {
        s << "    float in" << i << "_0, in" << i << "_1, in" << i << "_2, in" << i << "_3;\n";
        s << "    if (vector_ok) { const float4 w = *(const float4*)(p" << i << " + a" << i << ");"
          << " in" << i << "_0 = w.x; in" << i << "_1 = w.y; in" << i << "_2 = w.z; in" << i << "_3 = w.w; }\n";
        s << "    else { in" << i << "_0 = p" << i << "[a" << i << "]; in" << i << "_1 = p" << i << "[a" << i
          << " + 1]; in" << i << "_2 = p" << i << "[a" << i << " + 2]; in" << i << "_3 = p" << i << "[a" << i << " + 3]; }\n";
      } else {
        for (int j = 0; j < 4; ++j)
          s << "    const float in" << i << "_" << j << " = p" << i << "[a" << i << " + " << j * inner << "LL];\n";
      }
    }
    body(lanes);
    for (int o = 0; o < d.n_outputs; ++o) {
      s << "    if (vector_ok) *(float4*)(q" << o << " + base) = make_float4(";
      for (int j = 0; j < 4; ++j) s << (j ? ", " : "") << reference(d.outputs[o], lanes[j]);
      s << ");\n    else {";
      for (int j = 0; j < 4; ++j) s << " q" << o << "[base + " << j << "] = " << reference(d.outputs[o], lanes[j]) << ";";
      s << " }\n";
    }
    s << "    continue;\n    }\n";
  }
  // General path: each of the (up to) four elements on its own.
  s << "    for (int j = 0; j < 4 && base + j < volume; ++j) {\n";
  s << "    const long long f = base + j;\n";
  if (d.rank > 0) coordinates("f", "g");
  for (int i = 0; i < d.n_inputs; ++i)
    s << "    const float in" << i << "_g = p" << i << "[" << address(d.inputs[i], "g") << "];\n";
  body({"g"});
  for (int o = 0; o < d.n_outputs; ++o) s << "    q" << o << "[f] = " << reference(d.outputs[o], "g") << ";\n";
  s << "    }\n  }\n}\n";
  return s.str();
}

// hipRTC: source -> gfx950 code object. Needs no device.
std::vector<char> rtc_compile(const std::string &source) {
  hiprtcProgram program;
  if (hiprtcCreateProgram(&program, source.c_str(), "topos_chain.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
    throw RuntimeFailure{"hiprtcCreateProgram failed"};
  const char *options[] = {"--offload-arch=gfx950", "-O3", "-ffp-contract=off",
                           "-fno-gpu-flush-denormals-to-zero", "-fhip-fp32-correctly-rounded-divide-sqrt",
                           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  const hiprtcResult built = hiprtcCompileProgram(program, (int)(sizeof(options) / sizeof(options[0])), options);
  if (built != HIPRTC_SUCCESS) {
    size_t size = 0;
    hiprtcGetProgramLogSize(program, &size);
    std::string log(size, '\0');
    if (size) hiprtcGetProgramLog(program, &log[0]);
    hiprtcDestroyProgram(&program);
    throw RuntimeFailure{"chain kernel failed to compile: " + log};
  }
  size_t code_size = 0;
  hiprtcGetCodeSize(program, &code_size);
  std::vector<char> code(code_size);
  hiprtcGetCode(program, code.data());
  hiprtcDestroyProgram(&program);
  return code;
}

// Compiles (once per distinct source text) and, when `load`, loads the module.
Compiled compile(const std::string &source, bool load) {
  {
    std::lock_guard<std::mutex> guard(cache_lock);
    auto it = cache().find(source);
    if (it != cache().end() && (it->second.function || !load)) return it->second;
  }
  const std::vector<char> code = rtc_compile(source);
  Compiled compiled{};
  if (load) {
    check(hipModuleLoadData(&compiled.module, code.data()), "hipModuleLoadData(chain)");
    check(hipModuleGetFunction(&compiled.function, compiled.module, "topos_chain"), "hipModuleGetFunction(chain)");
  }
  std::lock_guard<std::mutex> guard(cache_lock);
  auto &slot = cache()[source];
  if (!slot.function) slot = compiled;  // a racing compile of the same text keeps the first module
  return slot;
}

}  // namespace

topos_hip_chain *create_chain(const topos_hip_chain_desc &d, bool load) {
  validate(d);
  auto chain = std::make_unique<topos_hip_chain>();
  chain->n_inputs = d.n_inputs;
  chain->n_outputs = d.n_outputs;
  chain->volume = 1;
  for (int a = 0; a < d.rank; ++a) chain->volume *= d.shape[a];
  chain->quads = d.rank > 0 && d.shape[d.rank - 1] % 4 == 0;
  for (int i = 0; i < d.n_inputs; ++i) {
    const topos_hip_layout &l = d.inputs[i];
    bool vector = l.rank > 0 && l.strides[l.rank - 1] == 1 && l.offset % 4 == 0;
    for (int a = 0; a + 1 < l.rank; ++a)
      if (l.strides[a] % 4 != 0) vector = false;
    chain->vector_in.push_back(vector);
    chain->in_offset.push_back(l.offset);
  }
  chain->source = generate(d, chain->quads, chain->vector_in);
  const Compiled compiled = compile(chain->source, load);
  chain->module = compiled.module;
  chain->function = compiled.function;
  return chain.release();
}

void launch_chain(const topos_hip_chain &chain, const float *const *inputs, float *const *outputs,
                  hipStream_t stream) {
  if (!chain.function) throw RuntimeFailure{"chain kernel was not loaded"};
  int vector_ok = 1;
  for (int i = 0; i < chain.n_inputs; ++i)
    if (chain.vector_in[i] && reinterpret_cast<uintptr_t>(inputs[i]) % 16 != 0) vector_ok = 0;
  for (int o = 0; o < chain.n_outputs; ++o)
    if (reinterpret_cast<uintptr_t>(outputs[o]) % 16 != 0) vector_ok = 0;
  std::vector<void *> arguments;
  std::vector<const void *> pointers(chain.n_inputs + chain.n_outputs);
  for (int i = 0; i < chain.n_inputs; ++i) pointers[i] = inputs[i];
  for (int o = 0; o < chain.n_outputs; ++o) pointers[chain.n_inputs + o] = outputs[o];
  for (auto &p : pointers) arguments.push_back(&p);
  arguments.push_back(&vector_ok);
  int64_t blocks = (chain.volume / 4 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 256 * 8) blocks = 256 * 8;
  check(hipModuleLaunchKernel(chain.function, (unsigned)blocks, 1, 1, 256, 1, 1, 0, stream,
                              arguments.data(), nullptr),
        "hipModuleLaunchKernel(chain)");
}

}  // namespace topos_hip
