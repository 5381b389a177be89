// Generated kernels (codegen.hpp): HIP source per expression, compiled by
// hipRTC for gfx950 and cached per process by source text.
//
// Shapes, strides and offsets are compile-time constants of the generated
// source, so coordinate arithmetic is division by constants and every
// address is a fused integer expression. The same faithful_math.h text the
// prebuilt kernels compile is embedded, so a generated exp is the library's
// exp bit for bit.
#include "codegen.hpp"

#include <hip/hiprtc.h>

#include <algorithm>
#include <atomic>
#include <functional>
#include <map>
#include <mutex>
#include <sstream>
#include <thread>

#include "faithful_math_text.h"  // kFaithfulMathText: faithful_math.h as a string

namespace topos_hip {

namespace {

std::mutex cache_lock;
// Source text -> compiled kernel (loaded or not).
std::map<std::string, Kernel> &cache() {
  static auto *compiled = new std::map<std::string, Kernel>();
  return *compiled;
}

const char *unary_pattern(int op) {
  switch (op) {
    case TOPOS_HIP_CHAIN_NEG: return "(-%a)";
    case TOPOS_HIP_CHAIN_EXP: return "topos_exp(%a)";
    case TOPOS_HIP_CHAIN_LN: return "topos_ln(%a)";
    case TOPOS_HIP_CHAIN_SQRT: return "__builtin_sqrtf(%a)";
    case TOPOS_HIP_CHAIN_TANH: return "topos_faithful::tanh_f32(%a)";
  }
  return nullptr;
}

const char *binary_pattern(int op) {
  switch (op) {
    case TOPOS_HIP_CHAIN_ADD: return "(%a + %b)";
    case TOPOS_HIP_CHAIN_SUB: return "(%a - %b)";
    case TOPOS_HIP_CHAIN_MUL: return "(%a * %b)";
    case TOPOS_HIP_CHAIN_DIV: return "(%a / %b)";
    case TOPOS_HIP_CHAIN_MAX: return "topos_faithful::max_f32(%a, %b)";
    case TOPOS_HIP_CHAIN_STEP: return "topos_faithful::step_f32(%a, %b)";
    case TOPOS_HIP_CHAIN_POWF: return "topos_pow(%a, %b)";
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

std::string ll(int64_t v) { return std::to_string(v) + "LL"; }

std::string float_literal(float v) {
  // Exact: the bit pattern reinterpreted.
  return "__builtin_bit_cast(float, " + std::to_string(__builtin_bit_cast(uint32_t, v)) + "u)";
}

std::string ref(int value, const std::string &lane) {
  if (value < 0) return "in" + std::to_string(-value - 1) + "_" + lane;
  return "s" + std::to_string(value) + "_" + lane;
}

void validate(const Expr &e) {
  if (e.rank < 0 || e.rank > kMaxRank) throw InvalidArgument{"expression rank out of range"};
  for (int d = 0; d < e.rank; ++d)
    if (e.shape[d] <= 0) throw InvalidArgument{"expression shape must be non-empty"};
  if (e.outputs.empty()) throw InvalidArgument{"expression without results"};
  const int n_inputs = (int)e.inputs.size();
  auto check_ref = [&](int v, int step) {
    if (v < 0 ? (-v - 1) >= n_inputs : v >= step) throw InvalidArgument{"expression operand reference"};
  };
  for (size_t s = 0; s < e.steps.size(); ++s) {
    const ExprStep &st = e.steps[s];
    if (!is_unary(st.op) && !is_binary(st.op)) throw InvalidArgument{"unknown expression operation"};
    check_ref(st.left, (int)s);
    if (is_binary(st.op)) check_ref(st.right, (int)s);
  }
  for (int o : e.outputs) check_ref(o, (int)e.steps.size());
  for (const ExprInput &in : e.inputs) {
    if (in.kind == ExprInput::kSelection && e.rank != 2)
      throw InvalidArgument{"a selection input needs a rank-2 expression"};
    if (in.kind == ExprInput::kPadded && (in.pad_axis < 0 || in.pad_axis >= e.rank || in.pad_len <= 0))
      throw InvalidArgument{"padded input window"};
  }
}

// Input i may use 16-byte loads along the innermost axis: unit inner stride
// (gfx950 serves unaligned global_load_dwordx4, so any 4-byte alignment
// does; a padded input's inner window must cover whole quads).
bool vector_input(const Expr &e, const ExprInput &in) {
  if (e.rank == 0 || in.kind == ExprInput::kSelection || in.kind == ExprInput::kLiteral) return false;
  const int inner = e.rank - 1;
  if (in.strides[inner] != 1) return false;
  if (in.kind == ExprInput::kPadded && in.pad_axis == inner && (in.pad_start % 4 != 0 || in.pad_len % 4 != 0))
    return false;
  return true;
}

std::string pointer_type(const ExprInput &in) {
  return in.kind == ExprInput::kSelection ? "const int* __restrict__" : "const float* __restrict__";
}

// Address of input `in` at coordinates `c` (names), the pad axis shifted.
std::string address(const Expr &e, const ExprInput &in, const std::vector<std::string> &c) {
  std::string a = ll(in.offset);
  for (int d = 0; d < e.rank; ++d) {
    if (in.strides[d] == 0) continue;
    std::string coord = c[d];
    if (in.kind == ExprInput::kPadded && d == in.pad_axis) coord = "(" + coord + " - " + ll(in.pad_start) + ")";
    a += " + " + coord + " * " + ll(in.strides[d]);
  }
  return a;
}

std::string window_test(const ExprInput &in, const std::string &coord) {
  return "(" + coord + " >= " + ll(in.pad_start) + " && " + coord + " < " + ll(in.pad_start + in.pad_len) + ")";
}

// Scalar value of input i at coordinates c.
std::string scalar_value(const Expr &e, int i, const std::vector<std::string> &c) {
  const ExprInput &in = e.inputs[i];
  const std::string p = "p" + std::to_string(i);
  if (in.kind == ExprInput::kLiteral) return float_literal(in.one);
  if (in.kind == ExprInput::kSelection)
    return "(" + p + "[" + c[0] + "] == (int)(" + c[1] + ") ? " + float_literal(in.one) + " : 0.0f)";
  const std::string load = p + "[" + address(e, in, c) + "]";
  if (in.kind == ExprInput::kPadded) return "(" + window_test(in, c[in.pad_axis]) + " ? " + load + " : 0.0f)";
  return load;
}

void emit_steps(std::ostringstream &s, const Expr &e, const std::vector<std::string> &lanes) {
  for (size_t k = 0; k < e.steps.size(); ++k) {
    const ExprStep &x = e.steps[k];
    for (const std::string &lane : lanes) {
      const std::string a = ref(x.left, lane);
      const std::string expr = is_unary(x.op) ? substitute(unary_pattern(x.op), a, "")
                                              : substitute(binary_pattern(x.op), a, ref(x.right, lane));
      s << "      const float s" << k << "_" << lane << " = " << expr << ";\n";
    }
  }
}

// Coordinates of flat index `flat` over `shape[0..rank)`, named c<d>_<tag>.
// Below 2^31 elements the divisions run on 32-bit unsigned values (a
// multiply-high and a shift per constant divisor instead of a 64-bit
// sequence); `flat` is then in range for any flat index of the shape.
void emit_coordinates(std::ostringstream &s, int rank, const int64_t *shape, const std::string &flat,
                      const std::string &tag, std::vector<std::string> &names) {
  names.assign(rank, "");
  int64_t volume = 1;
  for (int d = 0; d < rank; ++d) volume *= shape[d];
  const bool narrow = volume < (int64_t(1) << 31);
  std::string rem = flat;
  if (narrow && rank > 1) {
    rem = "u_" + tag;
    s << "      const unsigned " << rem << " = (unsigned)(" << flat << ");\n";
  }
  for (int d = rank - 1; d >= 0; --d) {
    const std::string name = "c" + std::to_string(d) + "_" + tag;
    names[d] = name;
    if (d == 0) {
      s << "      const long long " << name << " = " << rem << ";\n";
    } else if (narrow) {
      s << "      const long long " << name << " = (long long)(" << rem << " % " << shape[d] << "u);\n";
      const std::string next = "r" + std::to_string(d) + "_" + tag;
      s << "      const unsigned " << next << " = " << rem << " / " << shape[d] << "u;\n";
      rem = next;
    } else {
      s << "      const long long " << name << " = (" << rem << ") % " << ll(shape[d]) << ";\n";
      const std::string next = "r" + std::to_string(d) + "_" + tag;
      s << "      const long long " << next << " = (" << rem << ") / " << ll(shape[d]) << ";\n";
      rem = next;
    }
  }
}

std::string preamble() {
  std::string s = "#pragma clang fp contract(off)\n";
  s += kFaithfulMathText;
  // Four consecutive floats at any 4-byte-aligned address (one 16-byte
  // access; gfx950 serves it unaligned).
  s += "\ntypedef float topos_f4 __attribute__((ext_vector_type(4), aligned(4)));\n";
  // A barrier that orders LDS traffic only. __syncthreads() also waits for
  // every outstanding global load (a workgroup-scope fence), which would
  // stall the loads a fold keeps in flight across its barriers. Waiting for
  // lgkmcnt(0) (this lane's LDS reads and writes have completed; vmcnt and
  // expcnt left at their maxima: simm16 0xC07F on gfx9-family targets), then
  // s_barrier, gives every LDS write before the barrier to every LDS read
  // after it. The signal fences keep the compiler from moving memory
  // operations across.
  s += "\n__device__ __forceinline__ void topos_lds_barrier() {\n"
       "  __atomic_signal_fence(__ATOMIC_SEQ_CST);\n"
       "  __builtin_amdgcn_s_waitcnt(0xC07F);\n"
       "  __builtin_amdgcn_s_barrier();\n"
       "  __atomic_signal_fence(__ATOMIC_SEQ_CST);\n"
       "}\n";
  // The exp, ln and log2 tables, copied into LDS by every generated kernel
  // on entry: a per-lane table index then costs an LDS read, not a global
  // load.
  s += "__shared__ uint64_t topos_exp_lds[32];\n"
       "__shared__ topos_faithful::LogRow topos_log_lds[16];\n"
       "__shared__ topos_faithful::LogRow topos_log2_lds[16];\n"
       "__device__ __forceinline__ void topos_tables_init() {\n"
       "  if (threadIdx.x < 32) topos_exp_lds[threadIdx.x] = topos_faithful::kExpTableDevice[threadIdx.x];\n"
       "  if (threadIdx.x < 16) topos_log_lds[threadIdx.x] = topos_faithful::kLogTableDevice[threadIdx.x];\n"
       "  if (threadIdx.x >= 32 && threadIdx.x < 48)\n"
       "    topos_log2_lds[threadIdx.x - 32] = topos_faithful::kLog2TableDevice[threadIdx.x - 32];\n"
       "  __syncthreads();\n"
       "}\n"
       "__device__ __forceinline__ float topos_exp(float x) { return topos_faithful::exp_f32_table(x, topos_exp_lds); }\n"
       // e^x of a lane's four points. When every point of every lane of the
       // wave is at most -104, each e^x rounds to +0 (e^-104 < 2^-150), and
       // the wave skips the evaluation: the masked half of a causal softmax.
       "__device__ __forceinline__ void topos_exp4(float x0, float x1, float x2, float x3, float &y0, float &y1,\n"
       "                                           float &y2, float &y3) {\n"
       "  const bool zero = x0 <= -104.0f && x1 <= -104.0f && x2 <= -104.0f && x3 <= -104.0f;\n"
       "  if (__builtin_amdgcn_ballot_w64(!zero) == 0) {\n"
       "    y0 = 0.0f; y1 = 0.0f; y2 = 0.0f; y3 = 0.0f;\n"
       "  } else {\n"
       "    y0 = topos_exp(x0); y1 = topos_exp(x1); y2 = topos_exp(x2); y3 = topos_exp(x3);\n"
       "  }\n"
       "}\n"
       "__device__ __forceinline__ float topos_ln(float x) { return topos_faithful::ln_f32_table(x, topos_log_lds); }\n"
       "__device__ __forceinline__ float topos_pow(float x, float y) {\n"
       "  return topos_faithful::pow_f32_tables(x, y, topos_log2_lds, topos_exp_lds);\n"
       "}\n";
  return s;
}

std::string signature(const Expr &e, const std::string &tail) {
  std::ostringstream s;
  s << "extern \"C\" __global__ __launch_bounds__(256) void topos_gen(";
  for (size_t i = 0; i < e.inputs.size(); ++i) s << pointer_type(e.inputs[i]) << " p" << i << ", ";
  s << tail << ")";
  return s.str();
}

std::vector<char> rtc_compile(const std::string &source) {
  hiprtcProgram program;
  if (hiprtcCreateProgram(&program, source.c_str(), "topos_gen.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
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
    throw RuntimeFailure{"generated kernel failed to compile: " + log};
  }
  size_t code_size = 0;
  hiprtcGetCodeSize(program, &code_size);
  std::vector<char> code(code_size);
  hiprtcGetCode(program, code.data());
  hiprtcDestroyProgram(&program);
  return code;
}

Generated make(const std::string &source) {
  auto g = std::make_shared<Kernel>();
  g->source = source;
  return g;
}

// An input the launch reads each element of once (no repeated axis), over
// at least 16 MB. Its 16-byte loads carry the nontemporal hint, so they do not
// displace what the last-level cache holds for the next launch (this
// launch's own output among it). Measured on MI355X, a copy over
// [16384, 4096] and a read of its output: 114 against 135 us with plain
// loads. Smaller operands keep plain loads: a program over a few megabytes
// finds them in the caches from launch to launch, which the hint would give
// up (in an A/B on one MI355X the GPT-2 step ran 73.6 ms with this bound
// against 73.7 with the hint on every read-once input).
bool read_once(const Expr &e, const ExprInput &in) {
  if (e.volume() < (int64_t(1) << 22)) return false;
  for (int d = 0; d < e.rank; ++d)
    if (e.shape[d] > 1 && in.strides[d] == 0) return false;
  return true;
}

// Emits in<i>_<lanes[j]> (j < 4): the expression inputs at the four points of
// a quad (coordinates `c`, the innermost coordinate c[inner] the quad's first,
// a multiple of four in an innermost extent that is one). Unit-stride inputs
// take one 16-byte load.
void emit_quad_inputs(std::ostringstream &s, const Expr &e, const std::vector<std::string> &c,
                      const std::string &tag, const std::vector<std::string> &lanes, const std::string &indent,
                      const std::vector<bool> *only = nullptr, bool declare = true, bool streaming = false) {
  // declare = false: assign to registers the caller declared (zeroed).
  const std::string cf = declare ? "const float " : "";
  const int inner = e.rank - 1;
  for (size_t i = 0; i < e.inputs.size(); ++i) {
    if (only && !(*only)[i]) continue;
    const ExprInput &in = e.inputs[i];
    const std::string p = "p" + std::to_string(i);
    auto v = [&](int j) { return ref(-(int)i - 1, lanes[j]); };
    if (in.kind == ExprInput::kLiteral) {
      for (int j = 0; j < 4; ++j) s << indent << cf << v(j) << " = " << float_literal(in.one) << ";\n";
      continue;
    }
    if (in.kind == ExprInput::kSelection) {
      const std::string sel = "sel" + std::to_string(i) + "_" + tag;
      s << indent << "const int " << sel << " = " << p << "[" << c[0] << "];\n";
      for (int j = 0; j < 4; ++j)
        s << indent << cf << v(j) << " = (" << sel << " == (int)(" << c[1] << " + " << j << ")) ? "
          << float_literal(in.one) << " : 0.0f;\n";
      continue;
    }
    const bool padded = in.kind == ExprInput::kPadded;
    const bool inner_window = padded && in.pad_axis == inner;
    // A window test that holds for the whole quad: on an outer axis, or an
    // inner window whose bounds are multiples of four.
    const bool quad_window = padded && (!inner_window || (in.pad_start % 4 == 0 && in.pad_len % 4 == 0));
    const std::string a = "a" + std::to_string(i) + "_" + tag;
    s << indent << "const long long " << a << " = " << address(e, in, c) << ";\n";
    if (!padded || quad_window) {
      const std::string inside = padded ? window_test(in, c[in.pad_axis]) : "true";
      if (declare)
        s << indent << "float " << v(0) << " = 0.0f, " << v(1) << " = 0.0f, " << v(2) << " = 0.0f, " << v(3)
          << " = 0.0f;\n";
      s << indent << "if (" << inside << ") {\n";
      if (in.strides[inner] == 0) {
        s << indent << "  " << v(0) << " = " << p << "[" << a << "]; " << v(1) << " = " << v(0) << "; " << v(2)
          << " = " << v(0) << "; " << v(3) << " = " << v(0) << ";\n";
      } else if (vector_input(e, in)) {
        if (streaming && read_once(e, in))
          s << indent << "  const topos_f4 w = __builtin_nontemporal_load((const topos_f4*)(" << p << " + " << a
            << ")); ";
        else
          s << indent << "  const topos_f4 w = *(const topos_f4*)(" << p << " + " << a << "); ";
        s << v(0) << " = w.x; " << v(1) << " = w.y; " << v(2) << " = w.z; " << v(3) << " = w.w;\n";
      } else {
        for (int j = 0; j < 4; ++j)
          s << indent << "  " << v(j) << " = " << p << "[" << a << " + " << ll(j * in.strides[inner]) << "];\n";
      }
      s << indent << "}\n";
    } else {
      for (int j = 0; j < 4; ++j) {
        const std::string cj = "(" + c[inner] + " + " + std::to_string(j) + ")";
        s << indent << cf << v(j) << " = " << window_test(in, cj) << " ? " << p << "[" << a << " + "
          << ll(j * in.strides[inner]) << "] : 0.0f;\n";
      }
    }
  }
}

void launch(const Generated &g, unsigned blocks, std::vector<void *> &arguments, hipStream_t stream) {
  if (!g || !g->loaded) throw RuntimeFailure{"generated kernel was not loaded"};
  check(hipModuleLaunchKernel(g->function, blocks, 1, 1, 256, 1, 1, 0, stream, arguments.data(), nullptr),
        "hipModuleLaunchKernel(generated)");
}

}  // namespace

void compile_kernels(const std::vector<Generated> &kernels, bool load) {
  // Distinct sources that still need work.
  std::vector<std::string> todo;
  {
    std::lock_guard<std::mutex> guard(cache_lock);
    std::map<std::string, bool> seen;
    for (const Generated &g : kernels) {
      if (!g || seen.count(g->source)) continue;
      seen[g->source] = true;
      auto it = cache().find(g->source);
      if (it == cache().end() || (load && !it->second.loaded)) todo.push_back(g->source);
    }
  }
  // hipRTC in parallel; each thread compiles its share.
  std::vector<std::vector<char>> codes(todo.size());
  std::vector<std::string> failures(todo.size());
  const unsigned hardware = std::max(1u, std::thread::hardware_concurrency());
  const size_t workers = std::min<size_t>(todo.size(), std::min(16u, hardware));
  std::vector<std::thread> threads;
  std::atomic<size_t> next{0};
  for (size_t w = 0; w < workers; ++w)
    threads.emplace_back([&] {
      for (size_t i = next++; i < todo.size(); i = next++) {
        try {
          codes[i] = rtc_compile(todo[i]);
        } catch (const RuntimeFailure &e) {
          failures[i] = e.message;
        }
      }
    });
  for (std::thread &t : threads) t.join();
  for (size_t i = 0; i < todo.size(); ++i)
    if (!failures[i].empty()) throw RuntimeFailure{failures[i]};
  // Load on the calling thread, then publish.
  std::lock_guard<std::mutex> guard(cache_lock);
  for (size_t i = 0; i < todo.size(); ++i) {
    Kernel k;
    k.source = todo[i];
    if (load) {
      hipModule_t module;
      check(hipModuleLoadData(&module, codes[i].data()), "hipModuleLoadData(generated)");
      check(hipModuleGetFunction(&k.function, module, "topos_gen"), "hipModuleGetFunction(generated)");
      k.loaded = true;
    }
    cache()[todo[i]] = k;
  }
  for (const Generated &g : kernels) {
    if (!g) continue;
    const Kernel &k = cache().at(g->source);
    g->function = k.function;
    g->loaded = k.loaded;
  }
}

bool is_unary(int op) { return unary_pattern(op) != nullptr; }
bool is_binary(int op) { return binary_pattern(op) != nullptr; }

// ---- chain ----

namespace {

// Quads per lane per loop iteration of an aligned chain: enough loads in
// flight to cover HBM latency, within a register budget.
int chain_unroll(const Expr &e) {
  int loaded = 0;
  for (const ExprInput &in : e.inputs) loaded += in.kind != ExprInput::kLiteral;
  return loaded <= 3 ? 4 : 2;
}

}  // namespace

Generated generate_chain(const Expr &e) {
  validate(e);
  std::ostringstream s;
  s << preamble();
  std::string tail;
  for (size_t o = 0; o < e.outputs.size(); ++o) tail += (o ? ", " : "") + std::string("float* __restrict__ q") + std::to_string(o);
  s << signature(e, tail) << " {\n  topos_tables_init();\n";
  const int64_t volume = e.volume();
  const std::vector<std::string> lanes = {"0", "1", "2", "3"};
  const int64_t inner_extent = e.rank > 0 ? e.shape[e.rank - 1] : 1;
  if (e.rank > 0 && inner_extent % 4 != 0 && inner_extent >= 8) {
    // An odd innermost extent: quads run along each row from its start
    // (16-byte accesses at any alignment), the row's last partial quad lane
    // by lane.
    // U quads a lane per iteration, every quad's loads issued before any
    // use: a partial quad (a row's last) or one past the end loads its row's
    // first quad instead, which is always whole and in range, and is then
    // evaluated lane by lane.
    const int64_t quads_per_row = (inner_extent + 3) / 4;
    const int64_t total = volume / inner_extent * quads_per_row;
    const int U = chain_unroll(e);
    s << "  for (long long qb = (long long)blockIdx.x * " << 256 * U << "; qb < " << ll(total)
      << "; qb += (long long)gridDim.x * " << 256 * U << ") {\n";
    std::vector<std::string> all_lanes;
    for (int u = 0; u < U; ++u) {
      const std::string tag = "q" + std::to_string(u), U_ = std::to_string(u);
      std::vector<std::string> lanes_u;
      for (int j = 0; j < 4; ++j) lanes_u.push_back(tag + "_" + std::to_string(j));
      all_lanes.insert(all_lanes.end(), lanes_u.begin(), lanes_u.end());
      s << "    const long long qi" << U_ << " = qb + " << 256 * u << " + threadIdx.x;\n";
      s << "    const bool in" << U_ << " = qi" << U_ << " < " << ll(total) << ";\n";
      s << "    const long long row" << U_ << " = in" << U_ << " ? qi" << U_ << " / " << ll(quads_per_row) << " : 0;\n";
      s << "    const long long cq" << U_ << " = in" << U_ << " ? (qi" << U_ << " % " << ll(quads_per_row)
        << ") * 4 : 0;\n";
      s << "    const bool whole" << U_ << " = in" << U_ << " && cq" << U_ << " + 4 <= " << ll(inner_extent) << ";\n";
      s << "    const long long lc" << U_ << " = whole" << U_ << " ? cq" << U_ << " : 0;\n";
      std::vector<std::string> c;
      if (e.rank > 1) emit_coordinates(s, e.rank - 1, e.shape, "row" + U_, tag, c);
      c.push_back("lc" + U_);
      emit_quad_inputs(s, e, c, tag, lanes_u, "    ", nullptr, true, true);
    }
    emit_steps(s, e, all_lanes);
    for (int u = 0; u < U; ++u) {
      const std::string tag = "q" + std::to_string(u), U_ = std::to_string(u);
      s << "    if (whole" << U_ << ") {\n";
      for (size_t o = 0; o < e.outputs.size(); ++o) {
        s << "      *(topos_f4*)(q" << o << " + row" << U_ << " * " << ll(inner_extent) << " + cq" << U_
          << ") = topos_f4{";
        for (int j = 0; j < 4; ++j) s << (j ? ", " : "") << ref(e.outputs[o], tag + "_" + std::to_string(j));
        s << "};\n";
      }
      s << "    }\n";
    }
    for (int u = 0; u < U; ++u) {
      const std::string U_ = std::to_string(u);
      s << "    if (in" << U_ << " && !whole" << U_ << ") {\n";
      s << "      const long long base = row" << U_ << " * " << ll(inner_extent) << " + cq" << U_ << ";\n";
      s << "      for (int j = 0; cq" << U_ << " + j < " << ll(inner_extent) << "; ++j) {\n";
      s << "        const long long f = base + j;\n";
      std::vector<std::string> cg;
      emit_coordinates(s, e.rank, e.shape, "f", "g", cg);
      for (size_t i = 0; i < e.inputs.size(); ++i)
        s << "        const float in" << i << "_g = " << scalar_value(e, (int)i, cg) << ";\n";
      emit_steps(s, e, {"g"});
      for (size_t o = 0; o < e.outputs.size(); ++o) s << "        q" << o << "[f] = " << ref(e.outputs[o], "g") << ";\n";
      s << "      }\n    }\n";
    }
    s << "  }\n}\n";
    return make(s.str());
  }
  const bool quads = e.rank > 0 && e.shape[e.rank - 1] % 4 == 0;
  if (quads) {
    // U quads per lane per iteration, all loads issued before any use; a
    // block whose U * 256 quads lie wholly inside takes the unguarded path.
    const int U = chain_unroll(e);
    const int64_t span = 1024LL * U;
    s << "  for (long long block = (long long)blockIdx.x * " << span << "; block < " << ll(volume)
      << "; block += (long long)gridDim.x * " << span << ") {\n";
    s << "    if (block + " << span << " <= " << ll(volume) << ") {\n";
    std::vector<std::string> all_lanes;
    for (int u = 0; u < U; ++u) {
      const std::string tag = "q" + std::to_string(u);
      std::vector<std::string> lanes_u;
      for (int j = 0; j < 4; ++j) lanes_u.push_back(tag + "_" + std::to_string(j));
      all_lanes.insert(all_lanes.end(), lanes_u.begin(), lanes_u.end());
      s << "      const long long base_" << tag << " = block + (" << 256 * u << " + threadIdx.x) * 4;\n";
      std::vector<std::string> c;
      emit_coordinates(s, e.rank, e.shape, "base_" + tag, tag, c);
      emit_quad_inputs(s, e, c, tag, lanes_u, "      ", nullptr, true, true);
    }
    emit_steps(s, e, all_lanes);
    for (int u = 0; u < U; ++u) {
      const std::string tag = "q" + std::to_string(u);
      for (size_t o = 0; o < e.outputs.size(); ++o) {
        s << "      *(topos_f4*)(q" << o << " + base_" << tag << ") = topos_f4{";
        for (int j = 0; j < 4; ++j) s << (j ? ", " : "") << ref(e.outputs[o], tag + "_" + std::to_string(j));
        s << "};\n";
      }
    }
    s << "    } else {\n";
    s << "      for (int u = 0; u < " << U << "; ++u) {\n";
    s << "        const long long base = block + (u * 256 + threadIdx.x) * 4;\n";
    s << "        if (base >= " << ll(volume) << ") break;\n";
    std::vector<std::string> c;
    emit_coordinates(s, e.rank, e.shape, "base", "q", c);
    emit_quad_inputs(s, e, c, "q", lanes, "        ", nullptr, true, true);
    emit_steps(s, e, lanes);
    for (size_t o = 0; o < e.outputs.size(); ++o) {
      s << "        *(topos_f4*)(q" << o << " + base) = topos_f4{";
      for (int j = 0; j < 4; ++j) s << (j ? ", " : "") << ref(e.outputs[o], lanes[j]);
      s << "};\n";
    }
    s << "      }\n    }\n  }\n}\n";
    return make(s.str());
  }
  s << "  const long long volume = " << ll(volume) << ";\n";
  s << "  const long long stride = (long long)gridDim.x * 1024;\n";
  s << "  for (long long base = ((long long)blockIdx.x * 256 + threadIdx.x) * 4; base < volume; base += stride) {\n";
  s << "    for (int j = 0; j < 4 && base + j < volume; ++j) {\n";
  s << "      const long long f = base + j;\n";
  std::vector<std::string> c;
  if (e.rank > 0) emit_coordinates(s, e.rank, e.shape, "f", "g", c);
  for (size_t i = 0; i < e.inputs.size(); ++i)
    s << "      const float in" << i << "_g = " << scalar_value(e, (int)i, c) << ";\n";
  emit_steps(s, e, {"g"});
  for (size_t o = 0; o < e.outputs.size(); ++o) s << "      q" << o << "[f] = " << ref(e.outputs[o], "g") << ";\n";
  s << "    }\n";
  s << "  }\n}\n";
  return make(s.str());
}

void launch_generated_chain(const Generated &g, const Expr &e, const void *const *inputs, float *const *outputs,
                            hipStream_t stream) {
  std::vector<const void *> pointers;
  for (size_t i = 0; i < e.inputs.size(); ++i) pointers.push_back(inputs[i]);
  for (size_t o = 0; o < e.outputs.size(); ++o) pointers.push_back(outputs[o]);
  std::vector<void *> arguments;
  for (auto &p : pointers) arguments.push_back(&p);
  const bool quads = e.rank > 0 && e.shape[e.rank - 1] % 4 == 0;
  const bool odd_rows = e.rank > 0 && e.shape[e.rank - 1] % 4 != 0 && e.shape[e.rank - 1] >= 8;
  const int64_t per_block = quads || odd_rows ? 1024LL * chain_unroll(e) : 1024;
  int64_t blocks = (e.volume() + per_block - 1) / per_block;
  if (blocks < 1) blocks = 1;
  if (blocks > 256 * 64) blocks = 256 * 64;
  launch(g, (unsigned)blocks, arguments, stream);
}

// ---- transposing copy ----

namespace {

// The axis u < rank - 1 along which the single strided input of a pure copy
// has unit stride while the innermost axis does not, with both extents whole
// 64-element tiles; -1 when the copy does not have that form.
int transpose_axis(const Expr &e) {
  if (e.rank < 2 || e.rank > kMaxRank || e.inputs.size() != 1 || !e.steps.empty() || e.outputs.size() != 1 ||
      e.outputs[0] != -1)
    return -1;
  const ExprInput &in = e.inputs[0];
  const int inner = e.rank - 1;
  if (in.kind != ExprInput::kStrided || in.strides[inner] == 1 || e.shape[inner] % 64 != 0) return -1;
  for (int d = 0; d < inner; ++d)
    if (in.strides[d] == 1 && e.shape[d] % 64 == 0) return d;
  return -1;
}

}  // namespace

bool transposing_copy(const Expr &e) { return transpose_axis(e) >= 0; }

// A copy of a transposed view into a contiguous output (the key gradient of
// attention read through its head permutation): the chain would read the
// input four bytes at a time, 4 KB apart. Each workgroup instead moves one
// 64 x 64 tile of (inner axis, u) through LDS: 16-byte loads along u, where
// the input is contiguous, and 16-byte stores along the output's inner axis.
// Every other axis indexes whole tiles.
Generated generate_transpose_copy(const Expr &e) {
  const int u = transpose_axis(e);
  if (u < 0) throw InvalidArgument{"transposing copy: not a transposed view"};
  const ExprInput &in = e.inputs[0];
  const int inner = e.rank - 1;
  int64_t out_stride[kMaxRank];
  out_stride[inner] = 1;
  for (int d = inner - 1; d >= 0; --d) out_stride[d] = out_stride[d + 1] * e.shape[d + 1];
  // Tile grid: inner tiles fastest, then u tiles, then the other axes.
  std::vector<int> others;
  for (int d = 0; d < inner; ++d)
    if (d != u) others.push_back(d);
  const int64_t ni = e.shape[inner] / 64, nu = e.shape[u] / 64;
  std::ostringstream s;
  s << preamble();
  s << "extern \"C\" __global__ __launch_bounds__(256) void topos_gen(const float* __restrict__ p0, "
       "float* __restrict__ q0) {\n";
  s << "  __shared__ float tile[64][65];\n";
  s << "  long long b = blockIdx.x;\n";
  s << "  const long long ti = b % " << ll(ni) << ";\n  b /= " << ll(ni) << ";\n";
  s << "  const long long tu = b % " << ll(nu) << ";\n  b /= " << ll(nu) << ";\n";
  std::string base_in = ll(in.offset), base_out = "0LL";
  {
    // The other axes' coordinates: b over their extents, the last fastest.
    s << "  long long b0 = b;\n";
    for (int j = (int)others.size() - 1; j >= 0; --j) {
      const int d = others[j];
      const std::string name = "o" + std::to_string(j);
      s << "  const long long " << name << " = b0 % " << ll(e.shape[d]) << ";\n  b0 /= " << ll(e.shape[d]) << ";\n";
      base_in += " + " + name + " * " + ll(in.strides[d]);
      base_out += " + " + name + " * " + ll(out_stride[d]);
    }
  }
  base_in += " + tu * 64LL + ti * " + ll(64 * in.strides[inner]);
  base_out += " + tu * " + ll(64 * out_stride[u]) + " + ti * 64LL";
  s << "  const long long bi = " << base_in << ";\n";
  s << "  const long long bo = " << base_out << ";\n";
  s << "  const int t = threadIdx.x, q = t % 16;\n";
  s << "  #pragma unroll\n";
  s << "  for (int r = 0; r < 4; ++r) {\n";
  s << "    const int j = 16 * r + t / 16;\n";
  s << "    const topos_f4 v = *(const topos_f4*)(p0 + bi + (long long)j * " << ll(in.strides[inner]) << " + 4 * q);\n";
  s << "    tile[j][4 * q] = v.x; tile[j][4 * q + 1] = v.y; tile[j][4 * q + 2] = v.z; tile[j][4 * q + 3] = v.w;\n";
  s << "  }\n";
  s << "  __syncthreads();\n";
  s << "  #pragma unroll\n";
  s << "  for (int r = 0; r < 4; ++r) {\n";
  s << "    const int v_ = 16 * r + t / 16;\n";
  s << "    *(topos_f4*)(q0 + bo + (long long)v_ * " << ll(out_stride[u]) << " + 4 * q) = "
       "topos_f4{tile[4 * q][v_], tile[4 * q + 1][v_], tile[4 * q + 2][v_], tile[4 * q + 3][v_]};\n";
  s << "  }\n";
  s << "}\n";
  return make(s.str());
}

void launch_transpose_copy(const Generated &g, const Expr &e, const void *input, float *output, hipStream_t stream) {
  const int64_t tiles = e.volume() / (64 * 64);
  if (tiles < 1 || tiles > 0x7fffffff) throw Unsupported{"transposing copy: tile count out of range"};
  const void *p = input;
  float *q = output;
  std::vector<void *> arguments = {&p, &q};
  launch(g, (unsigned)tiles, arguments, stream);
}

// ---- fold ----

namespace {

// Outputs per fold workgroup: 64 when that still gives 256 workgroups,
// else 16 (more workgroups, each pulling a narrower band).
int64_t fold_width(int64_t outputs) { return outputs / 64 >= 256 ? 64 : 16; }

}  // namespace

namespace {

// Column form with a quad-divisible innermost extent and 16 outputs per
// workgroup: each lane loads the expression's inputs at quads (four
// consecutive outputs at one step, one 16-byte load per unit-stride input),
// evaluates them, and parks the values transposed in LDS as
// tile[buffer][output][step], so lane j < 16 folds output j from 16-byte LDS
// reads. A tile is kColumnSteps steps. Two register sets hold the raw inputs
// of the next two tiles, their loads in flight while the current tile is
// folded; a set is evaluated only when it is parked (two folds after its
// loads were issued), so no load is waited on before a fold. The two LDS
// buffers alternate, one barrier a tile. Workgroups are renumbered so that
// neighbouring column bands (which share cache lines) run on the same XCD.
// (Measured on MI355X, [8192, 768] folds: 45 us with one input and 93 us
// with three inputs and two steps when the next tile's loads were issued
// just before the fold and evaluated right after them.)
constexpr int kColumnQuads = 8;                                // quads per lane per tile
constexpr int kColumnSteps = kColumnQuads * 256 * 4 / 16;      // 512 steps per tile

Generated generate_column_fold(const Expr &e, int axis, FoldKind kind, const std::vector<int64_t> &rest,
                               const std::vector<int> &rest_axes, int64_t outputs) {
  const int64_t extent = e.shape[axis];
  constexpr int W = 16, H = kColumnSteps;
  std::ostringstream s;
  s << preamble();
  s << signature(e, "float* __restrict__ out") << " {\n  topos_tables_init();\n";
  s << "  __shared__ __attribute__((aligned(16))) float tile[2][" << W << "][" << H + 4 << "];\n";
  s << "  const int t = threadIdx.x;\n";
  s << "  const unsigned blocks = gridDim.x;\n";
  s << "  unsigned b = blockIdx.x;\n";
  s << "  if (blocks % 8 == 0) b = (b % 8) * (blocks / 8) + b / 8;\n";
  s << "  const long long first_output = (long long)b * " << W << ";\n";
  // Quad i of a set: local step (t + 256 i) / 4, local outputs
  // ((t + 256 i) % 4) * 4 + 0..3. A quad outside the operand is clamped to
  // the last step or quad (its values are never folded or written), so
  // every set issues the same loads on every path and the waits before a
  // set is parked count only that set's loads, not the other set's.
  // An input broadcast along the innermost axis loads one value a quad; its
  // three copies are made when the set is parked.
  const int inner = e.rank - 1;
  std::vector<bool> loaded_whole(e.inputs.size());
  for (size_t in = 0; in < e.inputs.size(); ++in)
    loaded_whole[in] = !(e.inputs[in].kind == ExprInput::kStrided && e.inputs[in].strides[inner] == 0);
  auto lanes_of = [](const std::string &prefix, int i) {
    const std::string tag = prefix + std::to_string(i);
    return std::vector<std::string>{tag + "_0", tag + "_1", tag + "_2", tag + "_3"};
  };
  auto declare = [&](const std::string &prefix) {
    for (int i = 0; i < kColumnQuads; ++i) {
      const std::vector<std::string> lanes = lanes_of(prefix, i);
      for (size_t in = 0; in < e.inputs.size(); ++in)
        for (int j = 0; j < (loaded_whole[in] ? 4 : 1); ++j) s << "  float " << ref(-(int)in - 1, lanes[j]) << " = 0.0f;\n";
    }
  };
  auto load = [&](const std::string &k0, const std::string &prefix) {
    for (int i = 0; i < kColumnQuads; ++i) {
      const std::string tag = prefix + std::to_string(i);
      const std::vector<std::string> lanes = lanes_of(prefix, i);
      const std::string lk = "((t + " + std::to_string(256 * i) + ") / 4)";
      const std::string lo = "(((t + " + std::to_string(256 * i) + ") % 4) * 4)";
      s << "    {\n";
      s << "      long long o_" << tag << " = first_output + " << lo << ";\n";
      s << "      if (o_" << tag << " > " << ll(outputs - 4) << ") o_" << tag << " = " << ll(outputs - 4) << ";\n";
      s << "      long long k_" << tag << " = " << k0 << " + " << lk << ";\n";
      s << "      if (k_" << tag << " > " << ll(extent - 1) << ") k_" << tag << " = " << ll(extent - 1) << ";\n";
      std::vector<std::string> rc;
      emit_coordinates(s, (int)rest.size(), rest.data(), "o_" + tag, tag, rc);
      std::vector<std::string> c(e.rank);
      for (size_t q = 0; q < rest_axes.size(); ++q) c[rest_axes[q]] = rc[q];
      c[axis] = "k_" + tag;
      emit_quad_inputs(s, e, c, tag, lanes, "      ", &loaded_whole, false);
      for (size_t in = 0; in < e.inputs.size(); ++in)
        if (!loaded_whole[in])
          s << "      " << ref(-(int)in - 1, lanes[0]) << " = p" << in << "[" << address(e, e.inputs[in], c) << "];\n";
      s << "    }\n";
    }
  };
  // Evaluates a set's quads and parks them in LDS buffer `buffer`.
  auto park = [&](const std::string &prefix, int buffer) {
    for (int i = 0; i < kColumnQuads; ++i) {
      const std::vector<std::string> lanes = lanes_of(prefix, i);
      const std::string lk = "((t + " + std::to_string(256 * i) + ") / 4)";
      const std::string lo = "(((t + " + std::to_string(256 * i) + ") % 4) * 4)";
      s << "    {\n";
      for (size_t in = 0; in < e.inputs.size(); ++in)
        if (!loaded_whole[in])
          for (int j = 1; j < 4; ++j)
            s << "      const float " << ref(-(int)in - 1, lanes[j]) << " = " << ref(-(int)in - 1, lanes[0]) << ";\n";
      emit_steps(s, e, lanes);
      for (int j = 0; j < 4; ++j)
        s << "    tile[" << buffer << "][" << lo << " + " << j << "][" << lk << "] = " << ref(e.outputs[0], lanes[j])
          << ";\n";
      s << "    }\n";
    }
  };
  const std::string combine = kind == kFoldSum ? "acc + x" : "topos_faithful::max_f32(acc, x)";
  // Lane t < W folds its output over the tile at k0 in LDS buffer `buffer`.
  auto fold = [&](int buffer, const std::string &k0) {
    s << "    if (t < " << W << ") {\n";
    s << "      const long long k0f = " << k0 << ";\n";
    s << "      const int steps = " << ll(extent) << " - k0f < " << H << " ? (int)(" << ll(extent) << " - k0f) : " << H
      << ";\n";
    // A whole tile: 64 steps at a time, sixteen 16-byte LDS reads then the
    // 64 dependent additions. (Measured on MI355X: the [8192, 768] chain
    // runs at about 7.6 cycles a step this way, 9.5 with a ring of 8-14
    // reads each issued as an earlier one is consumed; a chain fed from
    // registers runs at 4.6.)
    s << "      if (steps == " << H << ") {\n";
    for (int g = 0; g < H / 64; ++g) {
      s << "        {\n          float r[64];\n";
      s << "          #pragma unroll\n          for (int j = 0; j < 64; j += 4) { const float4 q = *(const float4*)&tile["
        << buffer << "][t][" << 64 * g << " + j]; r[j] = q.x; r[j + 1] = q.y; r[j + 2] = q.z; r[j + 3] = q.w; }\n";
      if (g == 0)
        s << "          if (k0f == 0) { acc = r[0]; } else { const float x = r[0]; acc = " << combine << "; }\n";
      else
        s << "          { const float x = r[0]; acc = " << combine << "; }\n";
      s << "          #pragma unroll\n          for (int q = 1; q < 64; ++q) { const float x = r[q]; acc = " << combine
        << "; }\n        }\n";
    }
    s << "      } else {\n";
    s << "        int j = 0;\n";
    s << "        if (k0f == 0) { acc = tile[" << buffer << "][t][0]; j = 1; }\n";
    s << "        for (; j < steps; ++j) { const float x = tile[" << buffer << "][t][j]; acc = " << combine << "; }\n";
    s << "      }\n";
    s << "    }\n";
  };
  s << "  float acc = 0.0f;\n";
  declare("a");
  declare("b");
  // Tile 0 parked in buffer 0; tiles 1 (set a) and 2 (set b) in flight.
  load("0LL", "a");
  park("a", 0);
  load(std::to_string(H) + "LL", "a");
  load(std::to_string(2 * H) + "LL", "b");
  // Two tiles an iteration: the barrier before each fold also frees the
  // other buffer (its fold ended before the barrier).
  // Both halves park and load on every path (only the second fold is
  // conditional), so the loop carries set a's loads older than set b's.
  s << "  for (long long k0 = 0; k0 < " << ll(extent) << "; k0 += " << 2 * H << ") {\n";
  s << "    topos_lds_barrier();\n";
  park("a", 1);                                   // tile k0 + H
  load("k0 + " + std::to_string(3 * H), "a");
  fold(0, "k0");
  s << "    topos_lds_barrier();\n";
  park("b", 0);                                   // tile k0 + 2H
  load("k0 + " + std::to_string(4 * H), "b");
  s << "    if (k0 + " << H << " < " << ll(extent) << ") {\n";
  fold(1, "k0 + " + std::to_string(H));
  s << "    }\n";
  s << "  }\n";
  s << "  if (t < " << W << " && first_output + t < " << ll(outputs) << ") out[first_output + t] = acc;\n";
  s << "}\n";
  return make(s.str());
}

}  // namespace

Generated generate_fold(const Expr &e, int axis, FoldKind kind) {
  // A workgroup owns W consecutive outputs (W = 16 or 64). Per tile of
  // H = 4096 / W fold steps, all 256 lanes evaluate the expression at 16
  // (output, step) points each and park the values in LDS; lane j < W then
  // folds output j over the tile in ascending step order. The next tile's
  // loads are issued before the fold of the current one, so they are in
  // flight while it runs.
  //   column form (the fold axis is not the innermost): a lane's output is
  //     lane % W and its steps lane / W + (256 / W) i — consecutive lanes read
  //     consecutive outputs, contiguous when the innermost axis is;
  //   row form (the fold axis is the innermost): a lane's step is lane % H
  //     and its outputs lane / H + (256 / H) i — consecutive lanes read along
  //     a row.
  validate(e);
  if (axis < 0 || axis >= e.rank) throw InvalidArgument{"fold axis out of range"};
  std::ostringstream s;
  s << preamble();
  s << signature(e, "float* __restrict__ out") << " {\n  topos_tables_init();\n";
  std::vector<int64_t> rest;
  std::vector<int> rest_axes;
  for (int d = 0; d < e.rank; ++d)
    if (d != axis) {
      rest.push_back(e.shape[d]);
      rest_axes.push_back(d);
    }
  int64_t outputs = 1;
  for (int64_t x : rest) outputs *= x;
  const int64_t extent = e.shape[axis];
  const bool row_form = axis == e.rank - 1;
  const int W = (int)fold_width(outputs), H = 4096 / W;
  if (!row_form && W == 16 && e.shape[e.rank - 1] % 4 == 0)
    return generate_column_fold(e, axis, kind, rest, rest_axes, outputs);
  s << "  __shared__ float tile[" << W << "][" << H + 1 << "];\n";
  s << "  const int t = threadIdx.x;\n";
  s << "  const long long first_output = (long long)blockIdx.x * " << W << ";\n";
  int counter = 0;
  // The value of the expression at (output o, step k), as register `name`.
  auto point = [&](const std::string &o, const std::string &k, const std::string &name) {
    const std::string tag = "p" + std::to_string(counter++);
    s << "    float " << name << " = 0.0f;\n";
    s << "    if (" << o << " < " << ll(outputs) << " && " << k << " < " << ll(extent) << ") {\n";
    std::vector<std::string> rc;
    if (!rest.empty()) emit_coordinates(s, (int)rest.size(), rest.data(), o, tag, rc);
    std::vector<std::string> c(e.rank);
    for (size_t q = 0; q < rest_axes.size(); ++q) c[rest_axes[q]] = rc[q];
    c[axis] = "(" + k + ")";
    for (size_t i = 0; i < e.inputs.size(); ++i)
      s << "      const float in" << i << "_" << tag << " = " << scalar_value(e, (int)i, c) << ";\n";
    emit_steps(s, e, {tag});
    s << "      " << name << " = " << ref(e.outputs[0], tag) << ";\n    }\n";
  };
  // Point i of this lane, at tile start k0: its (output, local output, step, local step).
  auto coords = [&](int i, const std::string &k0, std::string &o, std::string &lo, std::string &k,
                    std::string &lk) {
    if (row_form) {
      lo = "(t / " + std::to_string(H) + " + " + std::to_string((256 / H) * i) + ")";
      lk = "(t % " + std::to_string(H) + ")";
    } else {
      lo = "(t % " + std::to_string(W) + ")";
      lk = "(t / " + std::to_string(W) + " + " + std::to_string((256 / W) * i) + ")";
    }
    o = "(first_output + " + lo + ")";
    k = "(" + k0 + " + " + lk + ")";
  };
  auto load = [&](const std::string &k0, const std::string &prefix) {
    for (int i = 0; i < 16; ++i) {
      std::string o, lo, k, lk;
      coords(i, k0, o, lo, k, lk);
      point(o, k, prefix + std::to_string(i));
    }
  };
  auto store = [&](const std::string &prefix) {
    for (int i = 0; i < 16; ++i) {
      std::string o, lo, k, lk;
      coords(i, "0", o, lo, k, lk);
      s << "    tile[" << lo << "][" << lk << "] = " << prefix << i << ";\n";
    }
  };
  const std::string combine = kind == kFoldSum ? "acc + x" : "topos_faithful::max_f32(acc, x)";
  s << "  float acc = 0.0f;\n";
  s << "  {\n";
  load("0LL", "v");
  s << "    topos_lds_barrier();\n";
  store("v");
  s << "  }\n";
  s << "  for (long long k0 = 0; k0 < " << ll(extent) << "; k0 += " << H << ") {\n";
  s << "    topos_lds_barrier();\n";
  s << "    {\n";
  load("k0 + " + std::to_string(H), "w");  // the next tile, in flight during this fold
  // Lanes j < W fold: on a full tile the LDS reads of each group of 64 issue
  // before its ordered additions.
  s << "    if (t < " << W << ") {\n";
  s << "      const int steps = " << ll(extent) << " - k0 < " << H << " ? (int)(" << ll(extent) << " - k0) : " << H
    << ";\n";
  s << "      if (steps == " << H << ") {\n";
  for (int g = 0; g < H / 64; ++g) {
    s << "        {\n          float r[64];\n";
    s << "          #pragma unroll\n          for (int j = 0; j < 64; ++j) r[j] = tile[t][" << 64 * g << " + j];\n";
    if (g == 0)
      s << "          if (k0 == 0) { acc = r[0]; } else { const float x = r[0]; acc = " << combine << "; }\n";
    else
      s << "          { const float x = r[0]; acc = " << combine << "; }\n";
    s << "          #pragma unroll\n          for (int q = 1; q < 64; ++q) { const float x = r[q]; acc = " << combine
      << "; }\n        }\n";
  }
  s << "      } else {\n";
  s << "        int j = 0;\n";
  s << "        if (k0 == 0) { acc = tile[t][0]; j = 1; }\n";
  s << "        for (; j < steps; ++j) { const float x = tile[t][j]; acc = " << combine << "; }\n";
  s << "      }\n";
  s << "    }\n";
  s << "    topos_lds_barrier();\n";
  store("w");
  s << "    }\n";
  s << "  }\n";
  s << "  if (t < " << W << " && first_output + t < " << ll(outputs) << ") out[first_output + t] = acc;\n";
  s << "}\n";
  return make(s.str());
}

void launch_generated_fold(const Generated &g, const Expr &e, int axis, const void *const *inputs, float *out,
                           hipStream_t stream) {
  int64_t outputs = 1;
  for (int d = 0; d < e.rank; ++d)
    if (d != axis) outputs *= e.shape[d];
  std::vector<const void *> pointers;
  for (size_t i = 0; i < e.inputs.size(); ++i) pointers.push_back(inputs[i]);
  pointers.push_back(out);
  std::vector<void *> arguments;
  for (auto &p : pointers) arguments.push_back(&p);
  const int64_t width = fold_width(outputs);
  const int64_t blocks = (outputs + width - 1) / width;
  if (blocks > 0x7fffffff) throw Unsupported{"fold: too many outputs for one launch"};
  launch(g, (unsigned)blocks, arguments, stream);
}

// ---- exact whole-tensor sum over a large operand ----

namespace {

// Emits the evaluation of the expression at flat element `f` (logical
// row-major order) into `v`, guarded by f < volume.
void emit_flat_value(std::ostringstream &s, const Expr &e, const std::string &f, const std::string &tag) {
  s << "      float v = 0.0f;\n";
  s << "      const bool live = " << f << " < " << ll(e.volume()) << ";\n";
  s << "      if (live) {\n";
  std::vector<std::string> c;
  if (e.rank > 0) emit_coordinates(s, e.rank, e.shape, f, tag, c);
  for (size_t i = 0; i < e.inputs.size(); ++i)
    s << "      const float in" << i << "_" << tag << " = " << scalar_value(e, (int)i, c) << ";\n";
  emit_steps(s, e, {tag});
  s << "      v = " << ref(e.outputs[0], tag) << ";\n      }\n";
}

// A chunk is kSumChunk consecutive elements, kSumChunk / 256 rounds of 256
// consecutive elements, one per lane in order: wave 0 holds the first 64 of
// a round, wave 1 the next 64, ...
constexpr int kRounds = (int)(kSumChunk / 256);

}  // namespace

Generated generate_sum_gather(const Expr &e) {
  // Every round's value is evaluated first (all loads in flight together);
  // one barrier publishes each wave's per-round term count, then every lane
  // writes its term at (rounds before) + (waves before in its round) + (lanes
  // before in its wave): element order within the chunk.
  validate(e);
  std::ostringstream s;
  s << preamble();
  s << signature(e, "float* __restrict__ slots, int* __restrict__ counts, int* __restrict__ positive_zero")
    << " {\n  topos_tables_init();\n";
  s << "  __shared__ int wave_counts[" << kRounds << "][4];\n  __shared__ int wave_plus[4];\n";
  s << "  const long long chunk = blockIdx.x;\n";
  s << "  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;\n";
  s << "  const unsigned long long below = (1ull << lane) - 1ull;\n";
  s << "  float vals[" << kRounds << "];\n  int before[" << kRounds << "];\n  unsigned keep = 0;\n  int plus_zero = 0;\n";
  // Evaluation without branches (a lane past the end reads element 0 and
  // discards it), so every round's loads are in flight together.
  s << "  unsigned lives = 0;\n";
  s << "  #pragma unroll\n  for (int round = 0; round < " << kRounds << "; ++round) {\n";
  s << "    const long long f = chunk * " << ll(kSumChunk) << " + round * 256 + threadIdx.x;\n";
  s << "    const bool live = f < " << ll(e.volume()) << ";\n";
  s << "    const long long fc = live ? f : 0;\n    {\n";
  {
    std::vector<std::string> c;
    if (e.rank > 0) emit_coordinates(s, e.rank, e.shape, "fc", "x", c);
    for (size_t i = 0; i < e.inputs.size(); ++i)
      s << "      const float in" << i << "_x = " << scalar_value(e, (int)i, c) << ";\n";
    emit_steps(s, e, {"x"});
    s << "      vals[round] = " << ref(e.outputs[0], "x") << ";\n";
  }
  s << "      if (live) lives |= 1u << round;\n";
  s << "    }\n  }\n";
  // A term is zero only when it compares equal to zero; NaN counts as a term.
  s << "  #pragma unroll\n  for (int round = 0; round < " << kRounds << "; ++round) {\n";
  s << "    const float v = vals[round];\n";
  s << "    const bool live = (lives >> round) & 1u;\n";
  s << "    const bool term = live && !(v == 0.0f);\n";
  s << "    if (live && v == 0.0f && !__builtin_signbit(v)) plus_zero = 1;\n";
  s << "    if (term) keep |= 1u << round;\n";
  s << "    const unsigned long long mask = __ballot(term);\n";
  s << "    before[round] = __popcll(mask & below);\n";
  s << "    if (lane == 0) wave_counts[round][wave] = __popcll(mask);\n";
  s << "  }\n";
  s << "  for (int off = 32; off >= 1; off >>= 1) plus_zero |= __shfl_xor(plus_zero, off, 64);\n";
  s << "  if (lane == 0) wave_plus[wave] = plus_zero;\n";
  s << "  __syncthreads();\n";
  s << "  float* __restrict__ out = slots + chunk * " << ll(kSumChunk) << ";\n";
  s << "  int at = 0;\n";
  s << "  #pragma unroll\n  for (int round = 0; round < " << kRounds << "; ++round) {\n";
  s << "    int offset = at;\n";
  s << "    for (int w = 0; w < wave; ++w) offset += wave_counts[round][w];\n";
  s << "    if (keep & (1u << round)) out[offset + before[round]] = vals[round];\n";
  s << "    at += wave_counts[round][0] + wave_counts[round][1] + wave_counts[round][2] + wave_counts[round][3];\n";
  s << "  }\n";
  s << "  if (threadIdx.x == 0) {\n";
  s << "    counts[chunk] = at;\n";
  s << "    positive_zero[chunk] = wave_plus[0] | wave_plus[1] | wave_plus[2] | wave_plus[3];\n  }\n}\n";
  return make(s.str());
}

void launch_sum_gather(const Generated &g, const Expr &e, const void *const *inputs, float *slots, int32_t *counts,
                       int32_t *positive_zero, hipStream_t stream) {
  const int64_t chunks = (e.volume() + kSumChunk - 1) / kSumChunk;
  if (chunks > 0x7fffffff) throw Unsupported{"sum: too many chunks for one launch"};
  std::vector<const void *> pointers(inputs, inputs + e.inputs.size());
  pointers.push_back(slots);
  pointers.push_back(counts);
  pointers.push_back(positive_zero);
  std::vector<void *> arguments;
  for (auto &p : pointers) arguments.push_back(&p);
  launch(g, (unsigned)chunks, arguments, stream);
}


// ---- row programs ----

namespace {

struct RowFold {
  int pass;
  bool max;
  int node;          // the node whose operand a is folded
  bool shifted_exp;  // fold exp(a - rowv[max_slot[node]]) instead of a
  int target;        // row slot receiving the fold
};

struct RowLayout {
  std::vector<int> avail, slot, max_slot, total_slot, lns_slot;
  std::vector<RowFold> folds;
  int passes = 0, slots = 0, levels = 0;
};

RowLayout lay_out(const RowProgram &p) {
  const int n = (int)p.nodes.size();
  RowLayout l;
  l.avail.assign(n, 0);
  l.slot.assign(n, -1);
  l.max_slot.assign(n, -1);
  l.total_slot.assign(n, -1);
  l.lns_slot.assign(n, -1);
  auto check_ref = [&](const RowRef &r, int at, bool want_full, bool want_row) {
    if (r.kind == RowRef::kInput) {
      if (r.index < 0 || r.index >= (int)p.inputs.size()) throw InvalidArgument{"row program input reference"};
      return;
    }
    if (r.index < 0 || r.index >= at) throw InvalidArgument{"row program node reference"};
    const bool full = p.nodes[r.index].full();
    if ((full && !want_full) || (!full && !want_row)) throw InvalidArgument{"row program operand kind"};
  };
  auto level = [&](const RowRef &r) { return r.kind == RowRef::kInput ? 0 : l.avail[r.index]; };
  for (int i = 0; i < n; ++i) {
    const RowNode &x = p.nodes[i];
    switch (x.kind) {
      case RowNode::kFullOp:
      case RowNode::kRowOp: {
        const bool full = x.kind == RowNode::kFullOp;
        if (!is_unary(x.op) && !is_binary(x.op)) throw InvalidArgument{"row program operation"};
        check_ref(x.a, i, full, true);
        int lv = level(x.a);
        if (is_binary(x.op)) {
          check_ref(x.b, i, full, true);
          lv = std::max(lv, level(x.b));
        }
        l.avail[i] = lv;
        if (!full) l.slot[i] = l.slots++;
        break;
      }
      case RowNode::kSum:
      case RowNode::kMax: {
        check_ref(x.a, i, true, false);
        l.slot[i] = l.slots++;
        l.folds.push_back(RowFold{level(x.a), x.kind == RowNode::kMax, i, false, l.slot[i]});
        l.avail[i] = level(x.a) + 1;
        break;
      }
      case RowNode::kLogSumExp:
      case RowNode::kLogSoftmax: {
        check_ref(x.a, i, true, false);
        const int lv = level(x.a);
        l.max_slot[i] = l.slots++;
        l.total_slot[i] = l.slots++;
        l.folds.push_back(RowFold{lv, true, i, false, l.max_slot[i]});
        l.folds.push_back(RowFold{lv + 1, false, i, true, l.total_slot[i]});
        if (x.kind == RowNode::kLogSumExp)
          l.slot[i] = l.slots++;
        else
          l.lns_slot[i] = l.slots++;
        l.avail[i] = lv + 2;
        break;
      }
      default:
        throw InvalidArgument{"row program node kind"};
    }
    l.levels = std::max(l.levels, l.avail[i]);
  }
  for (const RowFold &f : l.folds) l.passes = std::max(l.passes, f.pass + 1);
  for (int o : p.full_outputs)
    if (o < 0 || o >= n || !p.nodes[o].full()) throw InvalidArgument{"row program full output"};
  for (int o : p.row_outputs)
    if (o < 0 || o >= n || p.nodes[o].full()) throw InvalidArgument{"row program row output"};
  return l;
}

// How a row program is laid out on the GPU.
//   resident: a workgroup owns G whole rows (columns <= 2048; G * columns
//     <= 4096 where G >= 4 allows it: a 16 KB slab leaves room for six or
//     more workgroups a CU, whose phases overlap, measured faster than 32 KB
//     slabs on the attention rows [98304, 1024]) and keeps
//     every non-literal input of its points in registers, read once; each
//     fold parks its operand row-major in LDS, max folds reduce contiguous
//     segments and combine them in column order, sum folds run one lane per
//     row in column order;
//   streaming: G rows per workgroup, the columns in slabs of S, every fold
//     level re-reading its inputs, one lane per row folding each slab.
struct RowBlocking {
  bool resident = false;
  int rows = 8;      // G
  int slab = 512;    // S (streaming)
  int width = 4;     // V: columns per point
  int points = 0;    // P: points per lane (resident)
};

RowBlocking row_blocking(const RowProgram &p) {
  RowBlocking b;
  const int64_t c = p.columns();
  b.width = c % 4 == 0 ? 4 : 1;
  int varying = 0;
  for (const ExprInput &in : p.inputs) varying += in.kind != ExprInput::kLiteral;
  if (c * 4 <= 8192) {
    int g = 64;
    while (g > 4 && (int64_t)g * c > 4096) g /= 2;  // G >= 4: a max fold's lanes per row stay in one wave
    auto points = [&](int rows) { return (int)((rows * (c / b.width) + 255) / 256); };
    while (g > 4 && (int64_t)points(g) * b.width * varying > 128) g /= 2;
    if ((int64_t)points(g) * b.width * varying <= 128 && points(g) <= 32) {
      b.resident = true;
      b.rows = g;
      b.points = points(g);
      return b;
    }
  }
  // Streaming: up to 64 rows per workgroup while that leaves 1024
  // workgroups (four per CU, so one workgroup's loads cover another's
  // folds); a slab gives each lane 16 points (V = 1) or 8 quads.
  const int64_t rows = p.rows();
  b.rows = 64;
  while (b.rows > 8 && (rows + b.rows - 1) / b.rows < 1024) b.rows /= 2;
  const int per_lane = b.width == 4 ? 8 : 16;
  b.slab = per_lane * 256 * b.width / b.rows;
  return b;
}

// The ordered sum of row[0 .. count) into `acc` (declared here): seeded with
// the first term, ascending. Reads go out in batches of eight 16-byte LDS
// loads ahead of their additions, so the chain of additions, not LDS
// latency, sets the pace.
void emit_lane_sum(std::ostringstream &s, const std::string &row, int64_t count, bool quads, const std::string &indent) {
  if (quads && count % 4 == 0) {
    const int64_t body = count / 32 * 32;
    s << indent << "float acc;\n";
    s << indent << "#pragma unroll 1\n";
    s << indent << "for (int c = 0; c < " << body << "; c += 32) {\n";
    s << indent << "  float4 w[8];\n";
    s << indent << "  #pragma unroll\n";
    s << indent << "  for (int k = 0; k < 8; ++k) w[k] = *(const float4*)&" << row << "[c + 4 * k];\n";
    s << indent << "  if (c == 0) acc = w[0].x; else acc = acc + w[0].x;\n";
    s << indent << "  acc = acc + w[0].y;\n  " << indent << "acc = acc + w[0].z;\n  " << indent << "acc = acc + w[0].w;\n";
    s << indent << "  #pragma unroll\n";
    s << indent << "  for (int k = 1; k < 8; ++k) { acc = acc + w[k].x; acc = acc + w[k].y; acc = acc + w[k].z; acc = acc + w[k].w; }\n";
    s << indent << "}\n";
    for (int64_t c = body; c < count; c += 4) {
      s << indent << "{ const float4 w = *(const float4*)&" << row << "[" << c << "]; ";
      if (c == 0)
        s << "acc = w.x; ";
      else
        s << "acc = acc + w.x; ";
      s << "acc = acc + w.y; acc = acc + w.z; acc = acc + w.w; }\n";
    }
    return;
  }
  s << indent << "float acc = " << row << "[0];\n";
  s << indent << "#pragma unroll 16\n";
  s << indent << "for (int c = 1; c < " << count << "; ++c) acc = acc + " << row << "[c];\n";
}

// Shared pieces of the two row-program layouts.
struct RowEmit {
  const RowProgram &p;
  const RowLayout &l;
  Expr e;  // the inputs over the full shape, for the shared emitters
  int n;
  RowEmit(const RowProgram &program, const RowLayout &layout) : p(program), l(layout) {
    e.rank = p.rank;
    for (int d = 0; d < p.rank; ++d) e.shape[d] = p.shape[d];
    e.inputs = p.inputs;
    e.outputs.push_back(0);
    n = (int)p.nodes.size();
  }
  // The name of a reference's value in full context (lane `lane`, block row `r`).
  std::string full_name(const RowRef &x, const std::string &lane, const std::string &r) const {
    if (x.kind == RowRef::kInput) return ref(-x.index - 1, lane);
    if (p.nodes[x.index].full()) return "f" + std::to_string(x.index) + "_" + lane;
    return "rowv[" + std::to_string(l.slot[x.index]) + "][" + r + "]";
  }
  // Marks the full nodes and inputs that evaluating `x` needs.
  void need(const RowRef &x, std::vector<bool> &nodes_needed, std::vector<bool> &inputs_needed) const {
    if (x.kind == RowRef::kInput) {
      inputs_needed[x.index] = true;
      return;
    }
    const RowNode &y = p.nodes[x.index];
    if (!y.full() || nodes_needed[x.index]) return;
    nodes_needed[x.index] = true;
    need(y.a, nodes_needed, inputs_needed);
    if (y.kind == RowNode::kFullOp && is_binary(y.op)) need(y.b, nodes_needed, inputs_needed);
  }
  // Emits the needed full nodes for each lane (inputs already named).
  void emit_nodes(std::ostringstream &s, const std::vector<bool> &nodes_needed, const std::vector<std::string> &lanes,
                  const std::string &r, const std::string &indent) const {
    for (int k = 0; k < n; ++k) {
      if (!nodes_needed[k]) continue;
      const RowNode &y = p.nodes[k];
      if (lanes.size() == 4 && y.kind == RowNode::kFullOp && y.op == TOPOS_HIP_CHAIN_EXP) {
        std::string args, outs;
        for (int j = 0; j < 4; ++j) {
          s << indent << "float f" << k << "_" << lanes[j] << ";\n";
          args += full_name(y.a, lanes[j], r) + ", ";
          outs += (j ? ", f" : "f") + std::to_string(k) + "_" + lanes[j];
        }
        s << indent << "topos_exp4(" << args << outs << ");\n";
        continue;
      }
      for (const std::string &lane : lanes) {
        std::string value;
        const std::string a = full_name(y.a, lane, r);
        if (y.kind == RowNode::kLogSoftmax) {
          value = "((" + a + " - rowv[" + std::to_string(l.max_slot[k]) + "][" + r + "]) - rowv[" +
                  std::to_string(l.lns_slot[k]) + "][" + r + "])";
        } else if (is_unary(y.op)) {
          value = substitute(unary_pattern(y.op), a, "");
        } else {
          value = substitute(binary_pattern(y.op), a, full_name(y.b, lane, r));
        }
        s << indent << "const float f" << k << "_" << lane << " = " << value << ";\n";
      }
    }
  }
  // The operands of fold f at a point's four lanes, as a make_float4
  // argument list (a shifted exponential's four go through topos_exp4 first).
  std::string fold_operands4(std::ostringstream &s, const RowFold &f, const std::vector<std::string> &lanes,
                             const std::string &r, const std::string &indent, const std::string &tag) const {
    std::string list;
    if (!f.shifted_exp) {
      for (int j = 0; j < 4; ++j) list += (j ? ", " : "") + fold_operand(f, lanes[j], r);
      return list;
    }
    const std::string shift = " - rowv[" + std::to_string(l.max_slot[f.node]) + "][" + r + "]";
    std::string args;
    for (int j = 0; j < 4; ++j) {
      const std::string e = "e" + tag + "_" + std::to_string(j);
      s << indent << "float " << e << ";\n";
      args += full_name(p.nodes[f.node].a, lanes[j], r) + shift + ", ";
      list += (j ? ", " : "") + e;
    }
    s << indent << "topos_exp4(" << args << list << ");\n";
    return list;
  }
  // The operand of fold f at one lane.
  std::string fold_operand(const RowFold &f, const std::string &lane, const std::string &r) const {
    const std::string a = full_name(p.nodes[f.node].a, lane, r);
    if (!f.shifted_exp) return a;
    return "topos_exp(" + a + " - rowv[" + std::to_string(l.max_slot[f.node]) + "][" + r + "])";
  }
  // Row nodes that become available at `level`, computed by lane t < G.
  void emit_row_stage(std::ostringstream &s, int level, int G) const {
    const int inner = p.rank - 1;
    const int64_t R = p.rows();
    auto row_name = [&](const RowRef &x) -> std::string {
      if (x.kind == RowRef::kInput) return "rin" + std::to_string(x.index);
      return "rowv[" + std::to_string(l.slot[x.index]) + "][t]";
    };
    std::ostringstream body;
    std::vector<bool> inputs_needed(p.inputs.size(), false);
    bool any = false;
    for (int k = 0; k < n; ++k) {
      const RowNode &y = p.nodes[k];
      if ((y.full() && y.kind != RowNode::kLogSoftmax) || l.avail[k] != level) continue;
      if (y.kind == RowNode::kRowOp) {
        if (y.a.kind == RowRef::kInput) inputs_needed[y.a.index] = true;
        if (is_binary(y.op) && y.b.kind == RowRef::kInput) inputs_needed[y.b.index] = true;
        const std::string a = row_name(y.a);
        const std::string v = is_unary(y.op) ? substitute(unary_pattern(y.op), a, "")
                                             : substitute(binary_pattern(y.op), a, row_name(y.b));
        body << "    rowv[" << l.slot[k] << "][t] = " << v << ";\n";
        any = true;
      } else if (y.kind == RowNode::kLogSumExp) {
        body << "    rowv[" << l.slot[k] << "][t] = rowv[" << l.max_slot[k] << "][t] + topos_ln(rowv["
             << l.total_slot[k] << "][t]);\n";
        any = true;
      } else if (y.kind == RowNode::kLogSoftmax) {
        body << "    rowv[" << l.lns_slot[k] << "][t] = topos_ln(rowv[" << l.total_slot[k] << "][t]);\n";
        any = true;
      }
    }
    if (!any) return;
    s << "  if (t < " << G << ") {\n";
    bool inputs = false;
    for (bool x : inputs_needed) inputs = inputs || x;
    if (inputs) {
      s << "    const long long g_row = row0 + t;\n";
      std::vector<std::string> c;
      if (p.rank > 1) emit_coordinates(s, p.rank - 1, p.shape, "g_row", "row", c);
      c.push_back("0LL");
      for (size_t i = 0; i < p.inputs.size(); ++i) {
        if (!inputs_needed[i]) continue;
        const ExprInput &in = p.inputs[i];
        if (in.kind == ExprInput::kSelection || (in.kind == ExprInput::kPadded && in.pad_axis == inner) ||
            (in.kind != ExprInput::kLiteral && in.strides[inner] != 0))
          throw InvalidArgument{"row program: a row operand varies along the row"};
        s << "    const float rin" << i << " = (g_row < " << ll(R) << ") ? " << scalar_value(e, (int)i, c)
          << " : 0.0f;\n";
      }
    }
    s << body.str();
    s << "  }\n";
  }
  std::string tail() const {
    std::string t;
    for (size_t o = 0; o < p.full_outputs.size(); ++o) t += "float* __restrict__ fo" + std::to_string(o) + ", ";
    for (size_t o = 0; o < p.row_outputs.size(); ++o) t += "float* __restrict__ ro" + std::to_string(o) + ", ";
    return t + "int unused";
  }
};

Generated generate_row_resident(const RowProgram &p, const RowLayout &l, const RowBlocking &b) {
  const RowEmit m(p, l);
  const int64_t C = p.columns(), R = p.rows();
  const int V = b.width, G = b.rows, P = b.points;
  const int64_t CV = C / V;
  const int n = m.n;
  std::ostringstream s;
  s << preamble();
  s << signature(m.e, m.tail()) << " {\n  topos_tables_init();\n";
  s << "  __shared__ float rowv[" << std::max(l.slots, 1) << "][" << G << "];\n";
  if (!l.folds.empty())
    s << "  __shared__ __attribute__((aligned(16))) float slab[" << G << "][" << C + 4 << "];\n";
  s << "  const int t = threadIdx.x;\n";
  s << "  const long long row0 = (long long)blockIdx.x * " << G << ";\n";
  // Every input read anywhere, loaded once per point into registers.
  std::vector<bool> nodes_all(n, false), inputs_all(p.inputs.size(), false);
  for (const RowFold &f : l.folds) m.need(p.nodes[f.node].a, nodes_all, inputs_all);
  for (int o : p.full_outputs) m.need(RowRef{RowRef::kFull, o}, nodes_all, inputs_all);
  std::vector<bool> loaded(p.inputs.size(), false);
  for (size_t k = 0; k < p.inputs.size(); ++k) loaded[k] = inputs_all[k] && p.inputs[k].kind != ExprInput::kLiteral;
  auto lanes_of = [&](int i) {
    std::vector<std::string> lanes;
    for (int j = 0; j < V; ++j) lanes.push_back("r" + std::to_string(i) + "_" + std::to_string(j));
    return lanes;
  };
  // Point i of lane t. Four rows of quads in multiples of 64: a wave's
  // point covers all four rows over 16 consecutive quads (lanes 16j..16j+15
  // on row j), so a wave's operands share one column range: a per-column
  // condition (a causal mask) then splits few waves. Otherwise points run
  // row-major over the block.
  const bool banded = G == 4 && V == 4 && CV % 64 == 0;
  for (int i = 0; i < P; ++i) {
    const std::string I = std::to_string(i);
    if (banded) {
      s << "  const int r" << I << " = (t % 64) / 16;\n";
      s << "  const long long col" << I << " = (long long)(" << 64 * i << " + (t / 64) * 16 + t % 16) * 4;\n";
      s << "  const bool ok" << I << " = row0 + r" << I << " < " << ll(R) << ";\n";
    } else {
      s << "  const int q" << I << " = t + " << 256 * i << ";\n";
      s << "  const int r" << I << " = q" << I << " / " << CV << ";\n";
      s << "  const long long col" << I << " = (long long)(q" << I << " % " << CV << ") * " << V << ";\n";
      s << "  const bool ok" << I << " = q" << I << " < " << (int64_t)G * CV << " && row0 + r" << I << " < " << ll(R)
        << ";\n";
    }
    const std::vector<std::string> lanes = lanes_of(i);
    for (size_t k = 0; k < p.inputs.size(); ++k) {
      if (!inputs_all[k]) continue;
      for (const std::string &lane : lanes) {
        if (p.inputs[k].kind == ExprInput::kLiteral)
          s << "  const float " << ref(-(int)k - 1, lane) << " = " << float_literal(p.inputs[k].one) << ";\n";
        else
          s << "  float " << ref(-(int)k - 1, lane) << " = 0.0f;\n";
      }
    }
    s << "  if (ok" << I << ") {\n";
    s << "    const long long g_r" << I << " = row0 + r" << I << ";\n";
    std::vector<std::string> c;
    if (p.rank > 1) emit_coordinates(s, p.rank - 1, p.shape, "g_r" + I, "r" + I, c);
    c.push_back("col" + I);
    if (V == 4) {
      emit_quad_inputs(s, m.e, c, "r" + I, lanes, "    ", &loaded, false, true);
    } else {
      for (size_t k = 0; k < p.inputs.size(); ++k)
        if (loaded[k]) s << "    " << ref(-(int)k - 1, lanes[0]) << " = " << scalar_value(m.e, (int)k, c) << ";\n";
    }
    s << "  }\n";
  }
  m.emit_row_stage(s, 0, G);
  s << "  topos_lds_barrier();\n";
  const int per = 256 / G;  // lanes per row in a max fold
  const int64_t seg = (C + per - 1) / per;
  for (int q = 0; q < l.passes; ++q) {
    for (const RowFold &f : l.folds) {
      if (f.pass != q) continue;
      std::vector<bool> nodes_needed(n, false), inputs_needed(p.inputs.size(), false);
      m.need(p.nodes[f.node].a, nodes_needed, inputs_needed);
      // The operand, row-major into the slab.
      for (int i = 0; i < P; ++i) {
        const std::string I = std::to_string(i);
        const std::vector<std::string> lanes = lanes_of(i);
        s << "  if (ok" << I << ") {\n";
        m.emit_nodes(s, nodes_needed, lanes, "r" + I, "    ");
        if (V == 4) {
          const std::string list = m.fold_operands4(s, f, lanes, "r" + I, "    ", I);
          s << "    *(float4*)&slab[r" << I << "][col" << I << "] = make_float4(" << list << ");\n";
        } else {
          s << "    slab[r" << I << "][col" << I << "] = " << m.fold_operand(f, lanes[0], "r" + I) << ";\n";
        }
        s << "  }\n";
      }
      s << "  topos_lds_barrier();\n";
      if (f.max) {
        // The ordered max_f32 fold is the first occurrence of the largest
        // non-NaN term (the last term when every term is NaN). Lane sg of a
        // row's group takes columns sg, sg + per, ... (conflict-free LDS
        // reads), keeping its first largest term and that term's column; the
        // group then keeps the largest, earliest.
        s << "  {\n";
        s << "    const int rr = t / " << per << ", sg = t % " << per << ";\n";
        s << "    float mv = 0.0f;\n    int mi = -1;\n";
        s << "    #pragma unroll 8\n";
        s << "    for (int c = sg; c < " << C << "; c += " << per << ") {\n";
        s << "      const float x = slab[rr][c];\n";
        s << "      if (x == x && (mi < 0 || x > mv)) { mv = x; mi = c; }\n";
        s << "    }\n";
        s << "    #pragma unroll\n";
        s << "    for (int off = 1; off < " << per << "; off <<= 1) {\n";
        s << "      const float ov = __shfl_xor(mv, off, 64);\n";
        s << "      const int oi = __shfl_xor(mi, off, 64);\n";
        s << "      if (oi >= 0 && (mi < 0 || ov > mv || (!(mv > ov) && oi < mi))) { mv = ov; mi = oi; }\n";
        s << "    }\n";
        s << "    if (sg == 0) rowv[" << f.target << "][rr] = mi < 0 ? slab[rr][" << C - 1 << "] : mv;\n";
        s << "  }\n";
      } else {
        s << "  if (t < " << G << ") {\n";
        emit_lane_sum(s, "slab[t]", C, V == 4, "    ");
        s << "    rowv[" << f.target << "][t] = acc;\n";
        s << "  }\n";
      }
      s << "  topos_lds_barrier();\n";
    }
    m.emit_row_stage(s, q + 1, G);
    s << "  topos_lds_barrier();\n";
  }
  for (int level = l.passes + 1; level <= l.levels; ++level) {
    m.emit_row_stage(s, level, G);
    s << "  topos_lds_barrier();\n";
  }
  if (!p.full_outputs.empty()) {
    std::vector<bool> nodes_needed(n, false), inputs_needed(p.inputs.size(), false);
    for (int o : p.full_outputs) m.need(RowRef{RowRef::kFull, o}, nodes_needed, inputs_needed);
    for (int i = 0; i < P; ++i) {
      const std::string I = std::to_string(i);
      const std::vector<std::string> lanes = lanes_of(i);
      s << "  if (ok" << I << ") {\n";
      m.emit_nodes(s, nodes_needed, lanes, "r" + I, "    ");
      if (p.transposed_outputs)
        s << "    const long long at = col" << I << " * " << ll(R) << " + row0 + r" << I << ";\n";
      else
        s << "    const long long at = (row0 + r" << I << ") * " << ll(C) << " + col" << I << ";\n";
      for (size_t o = 0; o < p.full_outputs.size(); ++o) {
        const int k = p.full_outputs[o];
        if (p.transposed_outputs)
          for (int j = 0; j < V; ++j)
            s << "    fo" << o << "[at + " << ll(j * R) << "] = f" << k << "_" << lanes[j] << ";\n";
        else if (V == 4)
          s << "    *(topos_f4*)(fo" << o << " + at) = topos_f4{f" << k << "_" << lanes[0] << ", f" << k << "_" << lanes[1]
            << ", f" << k << "_" << lanes[2] << ", f" << k << "_" << lanes[3] << "};\n";
        else
          s << "    fo" << o << "[at] = f" << k << "_" << lanes[0] << ";\n";
      }
      s << "  }\n";
    }
  }
  if (!p.row_outputs.empty()) {
    s << "  if (t < " << G << " && row0 + t < " << ll(R) << ") {\n";
    for (size_t o = 0; o < p.row_outputs.size(); ++o)
      s << "    ro" << o << "[row0 + t] = rowv[" << l.slot[p.row_outputs[o]] << "][t];\n";
    s << "  }\n";
  }
  s << "}\n";
  return make(s.str());
}

Generated generate_row_streaming(const RowProgram &p, const RowLayout &l, const RowBlocking &b) {
  const RowEmit m(p, l);
  const int64_t C = p.columns(), R = p.rows();
  const int V = b.width, G = b.rows, S = b.slab;
  const int SV = S / V;               // points per row of a slab
  const int PP = G * SV / 256;        // points per lane per slab
  const int per = 256 / G;            // lanes per row in a max fold
  const int n = m.n;
  int folds_per_pass = 1;
  for (int q = 0; q < l.passes; ++q) {
    int k = 0;
    for (const RowFold &f : l.folds) k += f.pass == q;
    folds_per_pass = std::max(folds_per_pass, k);
  }
  std::ostringstream s;
  s << preamble();
  s << signature(m.e, m.tail()) << " {\n  topos_tables_init();\n";
  s << "  __shared__ float rowv[" << std::max(l.slots, 1) << "][" << G << "];\n";
  if (l.passes > 0)
    s << "  __shared__ __attribute__((aligned(16))) float slab[" << folds_per_pass << "][" << G << "][" << S + 4
      << "];\n";
  s << "  const int t = threadIdx.x;\n";
  s << "  const long long row0 = (long long)blockIdx.x * " << G << ";\n";
  s << "  const int rr = t / " << per << ", sg = t % " << per << ";\n";
  auto lanes_of = [&](int i) {
    std::vector<std::string> lanes;
    for (int j = 0; j < V; ++j) lanes.push_back("s" + std::to_string(i) + "_" + std::to_string(j));
    return lanes;
  };
  for (int i = 0; i < PP; ++i) {
    s << "  const int r" << i << " = (t + " << 256 * i << ") / " << SV << ";\n";
    s << "  const int cu" << i << " = ((t + " << 256 * i << ") % " << SV << ") * " << V << ";\n";
  }
  // Declares registers for the loaded inputs of each point (literals as
  // constants), then emits the loads of the slab at column `c0`: one straight
  // run of loads when the slab lies wholly inside the rows and columns.
  auto declare = [&](const std::vector<bool> &loaded, const std::vector<bool> &inputs_needed) {
    for (int i = 0; i < PP; ++i)
      for (const std::string &lane : lanes_of(i))
        for (size_t k = 0; k < p.inputs.size(); ++k) {
          if (!inputs_needed[k]) continue;
          if (p.inputs[k].kind == ExprInput::kLiteral)
            s << "  const float " << ref(-(int)k - 1, lane) << " = " << float_literal(p.inputs[k].one) << ";\n";
          else if (loaded[k])
            s << "  float " << ref(-(int)k - 1, lane) << " = 0.0f;\n";
        }
  };
  auto load = [&](const std::vector<bool> &loaded, const std::string &c0, const std::string &indent) {
    auto one = [&](int i, bool guarded, const std::string &ind) {
      const std::string I = std::to_string(i);
      s << ind << "{\n";
      s << ind << "  const long long g = row0 + r" << I << ";\n";
      s << ind << "  const long long col = " << c0 << " + cu" << I << ";\n";
      if (guarded) s << ind << "  if (g < " << ll(R) << " && col < " << ll(C) << ") {\n";
      std::vector<std::string> c;
      if (p.rank > 1) emit_coordinates(s, p.rank - 1, p.shape, "g", "s" + I, c);
      c.push_back("col");
      const std::vector<std::string> lanes = lanes_of(i);
      if (V == 4) {
        emit_quad_inputs(s, m.e, c, "s" + I, lanes, ind + "    ", &loaded, false, true);
      } else {
        for (size_t k = 0; k < p.inputs.size(); ++k)
          if (loaded[k]) s << ind << "    " << ref(-(int)k - 1, lanes[0]) << " = " << scalar_value(m.e, (int)k, c) << ";\n";
      }
      if (guarded) s << ind << "  }\n";
      s << ind << "}\n";
    };
    s << indent << "if (row0 + " << G << " <= " << ll(R) << " && " << c0 << " + " << S << " <= " << ll(C) << ") {\n";
    for (int i = 0; i < PP; ++i) one(i, false, indent + "  ");
    s << indent << "} else {\n";
    for (int i = 0; i < PP; ++i) one(i, true, indent + "  ");
    s << indent << "}\n";
  };
  auto loaded_of = [&](const std::vector<bool> &inputs_needed) {
    std::vector<bool> loaded(p.inputs.size(), false);
    for (size_t k = 0; k < p.inputs.size(); ++k) loaded[k] = inputs_needed[k] && p.inputs[k].kind != ExprInput::kLiteral;
    return loaded;
  };

  m.emit_row_stage(s, 0, G);
  s << "  topos_lds_barrier();\n";
  for (int q = 0; q < l.passes; ++q) {
    std::vector<const RowFold *> folds;
    for (const RowFold &f : l.folds)
      if (f.pass == q) folds.push_back(&f);
    std::vector<bool> nodes_needed(n, false), inputs_needed(p.inputs.size(), false);
    for (const RowFold *f : folds) m.need(p.nodes[f->node].a, nodes_needed, inputs_needed);
    const std::vector<bool> loaded = loaded_of(inputs_needed);
    s << "  {\n";
    for (size_t j = 0; j < folds.size(); ++j) {
      if (folds[j]->max)
        s << "  float mv" << j << " = 0.0f;\n  int mi" << j << " = -1;\n";
      else
        s << "  float acc" << j << " = 0.0f;\n";
    }
    declare(loaded, inputs_needed);
    load(loaded, "0LL", "  ");
    s << "  for (long long c0 = 0; c0 < " << ll(C) << "; c0 += " << S << ") {\n";
    // This slab's operands into LDS.
    for (int i = 0; i < PP; ++i) {
      const std::string I = std::to_string(i);
      const std::vector<std::string> lanes = lanes_of(i);
      s << "    if (c0 + cu" << I << " < " << ll(C) << ") {\n";
      m.emit_nodes(s, nodes_needed, lanes, "r" + I, "      ");
      for (size_t j = 0; j < folds.size(); ++j) {
        if (V == 4) {
          const std::string list = m.fold_operands4(s, *folds[j], lanes, "r" + I, "      ", I + "_" + std::to_string(j));
          s << "      *(float4*)&slab[" << j << "][r" << I << "][cu" << I << "] = make_float4(" << list << ");\n";
        } else {
          s << "      slab[" << j << "][r" << I << "][cu" << I << "] = " << m.fold_operand(*folds[j], lanes[0], "r" + I)
            << ";\n";
        }
      }
      s << "    }\n";
    }
    // The next slab's loads, in flight during the folds.
    s << "    if (c0 + " << S << " < " << ll(C) << ") {\n";
    load(loaded, "(c0 + " + std::to_string(S) + ")", "      ");
    s << "    }\n";
    s << "    topos_lds_barrier();\n";
    s << "    const int width = " << ll(C) << " - c0 < " << S << " ? (int)(" << ll(C) << " - c0) : " << S << ";\n";
    for (size_t j = 0; j < folds.size(); ++j) {
      const std::string J = std::to_string(j);
      if (folds[j]->max) {
        s << "    {\n";
        s << "      float sv = 0.0f;\n      int si = -1;\n";
        s << "      #pragma unroll 4\n";
        s << "      for (int c = sg; c < width; c += " << per << ") {\n";
        s << "        const float x = slab[" << J << "][rr][c];\n";
        s << "        if (x == x && (si < 0 || x > sv)) { sv = x; si = c; }\n";
        s << "      }\n";
        s << "      #pragma unroll\n";
        s << "      for (int off = 1; off < " << per << "; off <<= 1) {\n";
        s << "        const float ov = __shfl_xor(sv, off, 64);\n";
        s << "        const int oi = __shfl_xor(si, off, 64);\n";
        s << "        if (oi >= 0 && (si < 0 || ov > sv || (!(sv > ov) && oi < si))) { sv = ov; si = oi; }\n";
        s << "      }\n";
        // Earlier slabs hold earlier columns: they win ties.
        s << "      if (si >= 0 && (mi" << J << " < 0 || sv > mv" << J << ")) { mv" << J << " = sv; mi" << J
          << " = (int)c0 + si; }\n";
        s << "    }\n";
      } else {
        // Blocks of 32 terms: eight 16-byte LDS reads go out ahead of the
        // block's ordered additions.
        const std::string A = "acc" + J;
        s << "    if (t < " << G << ") {\n";
        s << "      const float *row = &slab[" << J << "][t][0];\n";
        s << "      const int blocks = width / 32 * 32;\n";
        s << "      #pragma unroll 1\n";
        s << "      for (int c = 0; c < blocks; c += 32) {\n";
        s << "        float4 w[8];\n";
        s << "        #pragma unroll\n";
        s << "        for (int k = 0; k < 8; ++k) w[k] = *(const float4*)&row[c + 4 * k];\n";
        s << "        if (c0 == 0 && c == 0) " << A << " = w[0].x; else " << A << " = " << A << " + w[0].x;\n";
        s << "        " << A << " = " << A << " + w[0].y; " << A << " = " << A << " + w[0].z; " << A << " = " << A
          << " + w[0].w;\n";
        s << "        #pragma unroll\n";
        s << "        for (int k = 1; k < 8; ++k) { " << A << " = " << A << " + w[k].x; " << A << " = " << A
          << " + w[k].y; " << A << " = " << A << " + w[k].z; " << A << " = " << A << " + w[k].w; }\n";
        s << "      }\n";
        s << "      for (int c = blocks; c < width; ++c) {\n";
        s << "        if (c0 == 0 && c == 0) " << A << " = row[0]; else " << A << " = " << A << " + row[c];\n";
        s << "      }\n";
        s << "    }\n";
      }
    }
    s << "    topos_lds_barrier();\n";
    s << "  }\n";
    // Results: the last slab is still in LDS for an all-NaN max (its last term).
    const int64_t last_slab = (C - 1) / S * S;
    for (size_t j = 0; j < folds.size(); ++j) {
      const std::string J = std::to_string(j);
      if (folds[j]->max)
        s << "  if (sg == 0) rowv[" << folds[j]->target << "][rr] = mi" << J << " < 0 ? slab[" << J << "][rr]["
          << C - 1 - last_slab << "] : mv" << J << ";\n";
      else
        s << "  if (t < " << G << ") rowv[" << folds[j]->target << "][t] = acc" << J << ";\n";
    }
    s << "  }\n";
    m.emit_row_stage(s, q + 1, G);
    s << "  topos_lds_barrier();\n";
  }
  for (int level = l.passes + 1; level <= l.levels; ++level) {
    m.emit_row_stage(s, level, G);
    s << "  topos_lds_barrier();\n";
  }
  if (!p.full_outputs.empty()) {
    std::vector<bool> nodes_needed(n, false), inputs_needed(p.inputs.size(), false);
    for (int o : p.full_outputs) m.need(RowRef{RowRef::kFull, o}, nodes_needed, inputs_needed);
    const std::vector<bool> loaded = loaded_of(inputs_needed);
    s << "  for (long long c0 = 0; c0 < " << ll(C) << "; c0 += " << S << ") {\n";
    declare(loaded, inputs_needed);
    load(loaded, "c0", "    ");
    for (int i = 0; i < PP; ++i) {
      const std::string I = std::to_string(i);
      const std::vector<std::string> lanes = lanes_of(i);
      s << "    if (row0 + r" << I << " < " << ll(R) << " && c0 + cu" << I << " < " << ll(C) << ") {\n";
      m.emit_nodes(s, nodes_needed, lanes, "r" + I, "      ");
      if (p.transposed_outputs)
        s << "      const long long at = (c0 + cu" << I << ") * " << ll(R) << " + row0 + r" << I << ";\n";
      else
        s << "      const long long at = (row0 + r" << I << ") * " << ll(C) << " + c0 + cu" << I << ";\n";
      for (size_t o = 0; o < p.full_outputs.size(); ++o) {
        const int k = p.full_outputs[o];
        if (p.transposed_outputs)
          for (int j = 0; j < V; ++j)
            s << "      fo" << o << "[at + " << ll(j * R) << "] = f" << k << "_" << lanes[j] << ";\n";
        else if (V == 4)
          s << "      *(topos_f4*)(fo" << o << " + at) = topos_f4{f" << k << "_" << lanes[0] << ", f" << k << "_"
            << lanes[1] << ", f" << k << "_" << lanes[2] << ", f" << k << "_" << lanes[3] << "};\n";
        else
          s << "      fo" << o << "[at] = f" << k << "_" << lanes[0] << ";\n";
      }
      s << "    }\n";
    }
    s << "  }\n";
  }
  if (!p.row_outputs.empty()) {
    s << "  if (t < " << G << " && row0 + t < " << ll(R) << ") {\n";
    for (size_t o = 0; o < p.row_outputs.size(); ++o)
      s << "    ro" << o << "[row0 + t] = rowv[" << l.slot[p.row_outputs[o]] << "][t];\n";
    s << "  }\n";
  }
  s << "}\n";
  return make(s.str());
}

}  // namespace

Generated generate_row_program(const RowProgram &p) {
  if (p.rank < 1 || p.rank > kMaxRank) throw InvalidArgument{"row program rank"};
  for (int d = 0; d < p.rank; ++d)
    if (p.shape[d] <= 0) throw InvalidArgument{"row program shape"};
  const RowLayout l = lay_out(p);
  const RowBlocking blocking = row_blocking(p);
  if (blocking.resident) return generate_row_resident(p, l, blocking);
  return generate_row_streaming(p, l, blocking);
}

void launch_row_program(const Generated &g, const RowProgram &p, const void *const *inputs,
                        float *const *full_outputs, float *const *row_outputs, hipStream_t stream) {
  const int G = row_blocking(p).rows;
  std::vector<const void *> pointers;
  for (size_t i = 0; i < p.inputs.size(); ++i) pointers.push_back(inputs[i]);
  for (size_t o = 0; o < p.full_outputs.size(); ++o) pointers.push_back(full_outputs[o]);
  for (size_t o = 0; o < p.row_outputs.size(); ++o) pointers.push_back(row_outputs[o]);
  int unused = 0;
  std::vector<void *> arguments;
  for (auto &q : pointers) arguments.push_back(&q);
  arguments.push_back(&unused);
  const int64_t blocks = (p.rows() + G - 1) / G;
  if (blocks > 0x7fffffff) throw Unsupported{"row program: too many rows for one launch"};
  launch(g, (unsigned)blocks, arguments, stream);
}

}  // namespace topos_hip
