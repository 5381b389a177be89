/* libtopos_hip — the MI355X (gfx950) execution backend for topos.
 *
 * A plain C ABI: no C++ or torch types cross it, only pointers, sizes and
 * integer codes. The topos side binds it at run time (dlopen), exactly as its
 * CUDA rung binds libcudart/libcublas (src/backend/cuda/kernels/context.rs:217-288),
 * so a build without the library or a machine without a GPU is a status answer,
 * never a build failure.
 *
 * Three faces:
 *   - the manifest and status (src/backend/manifest.rs:16-37, backend.rs:128-177);
 *   - the offered task face, host buffers in and out, synchronous — the bodies of
 *     `Task::offer` arms for GemmTask<f32> and MapTask<f32>
 *     (src/backend/task.rs:57-115);
 *   - the device face: the same kernels on HBM-resident buffers, enqueued on a
 *     caller stream (what the plan executor and the benchmark drive);
 *   - the plan face: a device program (the lowered `Plan` columns,
 *     src/engine/plan.rs:311-347) executed from one pre-sized HBM arena.
 *
 * Degrade to slow, never to wrong (src/backend/cuda/kernels/mod.rs:94-121):
 * any runtime HIP failure poisons the library; every later offer declines
 * (TOPOS_HIP_DECLINED) and topos computes on its reference path.
 */
#ifndef TOPOS_HIP_H
#define TOPOS_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TOPOS_HIP_ABI_VERSION 2

/* ---- status codes ---- */
enum {
  TOPOS_HIP_OK = 0,
  /* The task was not served (outside the kernels' mapping, below the cost
   * threshold, or the backend is unavailable/poisoned): the caller computes on
   * the reference path. The `None` of `Task::offer`. */
  TOPOS_HIP_DECLINED = 1,
  /* Setup: no HIP device is visible (SetupError::NoDevice; tests skip). */
  TOPOS_HIP_NO_DEVICE = 2,
  /* Setup: any other one-time setup failure (SetupError::Failed; tests fail). */
  TOPOS_HIP_SETUP_FAILED = 3,
  /* Disabled after a runtime error (BackendUnavailable::Poisoned). */
  TOPOS_HIP_POISONED = 4,
  /* The call violates its contract (a GemmTask whose slice does not span its
   * matrix, an unknown operation, a malformed program): the reference panics
   * here. Does not poison. */
  TOPOS_HIP_INVALID_ARGUMENT = 5,
  /* A HIP call failed during this call; the library is now poisoned. */
  TOPOS_HIP_RUNTIME_ERROR = 6,
  /* A device-face request the kernels do not cover (device face only; the task
   * face answers DECLINED instead). */
  TOPOS_HIP_UNSUPPORTED = 7
};

/* ---- the vocabulary mirrored from src/backend ---- */
enum { TOPOS_HIP_EXACT = 0, TOPOS_HIP_FAST = 1 };              /* Numerics (numerics.rs:24-42) */
enum { TOPOS_HIP_BIT_IDENTICAL = 0, TOPOS_HIP_ENVELOPE = 1 };  /* Fidelity (coverage.rs:13-33) */
enum {                                                         /* Formula (formula.rs:24-37) */
  TOPOS_HIP_FORMULA_GEMM = 0,
  TOPOS_HIP_FORMULA_MAP = 1,
  TOPOS_HIP_FORMULA_WINDOW_PRODUCT = 2,
  TOPOS_HIP_FORMULA_REDUCE_WINDOW = 3,
  TOPOS_HIP_FORMULA_BATCH_NORM_TRAINING = 4,
  TOPOS_HIP_FORMULA_BATCH_NORM_INFERENCE = 5
};
enum { TOPOS_HIP_PRECISION_F32 = 1u, TOPOS_HIP_PRECISION_F64 = 2u }; /* Precision bits */
enum {                                                         /* Dispatch (coverage.rs:87-98) */
  TOPOS_HIP_DISPATCH_OFFERED = 0,
  TOPOS_HIP_DISPATCH_ELECTED = 1,
  TOPOS_HIP_DISPATCH_TRANSLATED = 2
};
enum {                                                         /* MapOperation (elementary.rs:13-22) */
  TOPOS_HIP_MAP_EXP = 0,
  TOPOS_HIP_MAP_LN = 1,
  TOPOS_HIP_MAP_SQRT = 2,
  TOPOS_HIP_MAP_TANH = 3
};

/* ---- manifest and status ---- */

/* ABI version of the loaded library; a binding refuses a mismatch. */
int topos_hip_abi_version(void);
/* How the member's kernels are reached (Manifest::DISPATCH, manifest.rs:17-18):
 * TOPOS_HIP_DISPATCH_OFFERED, buffer tasks offered down the chains at run time,
 * as the CUDA rung (src/backend/cuda/mod.rs:20). */
int topos_hip_dispatch(void);
/* Build facts only, no device probe (Manifest::compiled, manifest.rs:30-32). */
int topos_hip_compiled(void);
/* The coverage cell for one formula (Manifest::coverage, manifest.rs:22-28).
 * Returns 1 and fills `fidelity` and `precisions` (TOPOS_HIP_PRECISION_* bits)
 * when a kernel serves the formula, 0 for Coverage::Absent. */
int topos_hip_coverage(int formula, int *fidelity, unsigned *precisions);
/* Forces the lazy one-time setup (Manifest::status, manifest.rs:34-36; the
 * OnceLock of src/backend/cuda/kernels/mod.rs:36-68). Returns TOPOS_HIP_OK,
 * TOPOS_HIP_NO_DEVICE, TOPOS_HIP_SETUP_FAILED or TOPOS_HIP_POISONED. */
int topos_hip_status(void);
/* The reason held for the last non-OK status (setup error or poison message),
 * or "" — valid for the life of the process. */
const char *topos_hip_status_reason(void);
/* Static text for a status code. */
const char *topos_hip_status_string(int code);

/* ---- offered task face (host buffers, synchronous) ---- */

/* One dense f32 product, the GemmTask of src/payload/gemm.rs:40-125:
 * element (i, j) of `a` is a[i * a_row_stride + j * a_col_stride] (m x k),
 * of `b` is b[i * b_row_stride + j * b_col_stride] (k x n); `a_len`/`b_len`
 * are the slice lengths, which must span the matrices (gemm.rs:57-89).
 * On TOPOS_HIP_OK, `product` holds the contiguous row-major [m, n] product:
 * bit-identical to gemm::multiply under TOPOS_HIP_EXACT, within the envelope
 * |c - exact| <= 1e-5 * sum_k |a_ik * b_kj| under TOPOS_HIP_FAST.
 * TOPOS_HIP_DECLINED: compute on the reference path (GEMV shapes, below the
 * cost threshold, extents beyond i32, or the backend unavailable/poisoned).
 * Replaces the `Backend::Cuda => cuda::gemm_f32(self)` arm of
 * src/backend/task.rs:63-75 (the Hip arm beside it). */
int topos_hip_gemm_f32(const float *a, size_t a_len, size_t a_row_stride, size_t a_col_stride,
                       const float *b, size_t b_len, size_t b_row_stride, size_t b_col_stride,
                       size_t m, size_t k, size_t n, int numerics, float *product);

/* One whole-buffer transcendental, the MapTask of src/backend/task.rs:36-54:
 * `out[i] = op(elements[i])` bit-identical to the host libm under either
 * posture. TOPOS_HIP_DECLINED below the size threshold or when unavailable.
 * Replaces the `Backend::Metal => metal::map_f32(..)` arm of task.rs:103-115. */
int topos_hip_map_f32(int operation, const float *elements, size_t count, int numerics, float *out);

/* ---- device face (HBM-resident buffers, asynchronous on `stream`) ----
 * `stream` is a hipStream_t (NULL: the null stream). Pointers are device
 * addresses. Returns TOPOS_HIP_OK once the work is enqueued. */

/* The same product as topos_hip_gemm_f32 with device operands; the product is
 * row-major with leading dimension `ldc` >= n. Operand strides may be any
 * non-negative values (stride 0 broadcasts). */
int topos_hip_gemm_f32_device(const float *a, int64_t a_row_stride, int64_t a_col_stride,
                              const float *b, int64_t b_row_stride, int64_t b_col_stride,
                              int64_t m, int64_t k, int64_t n, int numerics, float *product,
                              int64_t ldc, void *stream);

/* The same product as topos_hip_gemm_f32_device, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference: it calls
 * no hipMalloc/hipFree on any call. The split-k partials of a Fast product go
 * to a fixed device array of 64 MiB (16 Mi floats) that each GPU holds from
 * library load until the process ends, instead of the library's grow-only
 * workspace. The array is never exceeded: a product whose chosen split needs
 * more splits k into as many ranges as fit (or runs unsplit). Results are
 * bit-identical to topos_hip_gemm_f32_device's whenever its partials fit the
 * array (and always under TOPOS_HIP_EXACT, which needs no scratch); otherwise
 * they stay within the same Fast envelope. No size is refused.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (other streams, other threads) race and must be serialised by the
 * caller. */
int topos_hip_gemm_f32_device_noalloc(const float *a, int64_t a_row_stride, int64_t a_col_stride,
                                      const float *b, int64_t b_row_stride, int64_t b_col_stride,
                                      int64_t m, int64_t k, int64_t n, int numerics, float *product,
                                      int64_t ldc, void *stream);

/* A bf16 product, the matmul contract of the bf16 payload (Bf16::gemm,
 * src/payload/bf16.rs:235-262): `a`, `b` and `product` hold bf16 bit patterns
 * (the top half of an f32); the operands widen to f32 exactly, the f32
 * product is taken, and every output rounds once to bf16, to nearest with
 * ties to even (Bf16::from_f32, :38-46). TOPOS_HIP_EXACT: the f32 product is
 * gemm::multiply's (bit-identical). TOPOS_HIP_FAST: bf16 matrix cores with
 * f32 accumulation, within |c - exact| <= 1e-5 * sum_k |a_ik b_kj| before the
 * rounding, when each operand has a unit stride along one axis (else the
 * exact path). Strides are in elements; the product is row-major with
 * leading dimension `ldc`. */
int topos_hip_gemm_bf16_device(const uint16_t *a, int64_t a_row_stride, int64_t a_col_stride, const uint16_t *b,
                               int64_t b_row_stride, int64_t b_col_stride, int64_t m, int64_t k, int64_t n,
                               int numerics, uint16_t *product, int64_t ldc, void *stream);

/* Elementwise unary map over `count` contiguous elements (MapOperation). */
int topos_hip_map_f32_device(int operation, const float *x, int64_t count, float *y, void *stream);

/* Row reductions over the last axis of a contiguous [rows, columns] buffer,
 * the Tensorial reductions and fused rules of src/payload/tensor.rs:1055-1124,
 * src/function/log_softmax.rs:51-60 and src/function/log_sum_exp.rs:53-61.
 * Sum-type reductions are bit-identical (ascending, first-term seeded) under
 * TOPOS_HIP_EXACT and tree-ordered under TOPOS_HIP_FAST; max is bit-identical
 * under both. */
enum {
  TOPOS_HIP_ROWS_SUM = 0,         /* out[rows]          sum_along(1) */
  TOPOS_HIP_ROWS_MAX = 1,         /* out[rows]          max_along(1) */
  TOPOS_HIP_ROWS_LOG_SOFTMAX = 2, /* out[rows, columns] log_softmax(1) */
  TOPOS_HIP_ROWS_SOFTMAX = 3,     /* out[rows, columns] log_softmax(1).exp() */
  TOPOS_HIP_ROWS_LOG_SUM_EXP = 4  /* out[rows]          logsumexp(1) */
};
int topos_hip_rows_f32_device(int reduction, const float *x, int64_t rows, int64_t columns,
                              int numerics, float *out, void *stream);

/* LayerNorm over the last axis (src/neural/layer_norm.rs:100-132): mean and
 * biased variance by sum / count, (x - mean) / sqrt(var + epsilon), then
 * * scale[j] + shift[j]. */
int topos_hip_layer_norm_f32_device(const float *x, int64_t rows, int64_t columns,
                                    const float *scale, const float *shift, float epsilon,
                                    int numerics, float *out, void *stream);

/* ---- generated elementwise/broadcast chains ----
 * A chain is a straight-line program of f32 elementwise operations over
 * `n_inputs` strided views of one logical shape; each output is written
 * contiguous row-major. It is compiled once (hipRTC, gfx950) into a kernel of
 * its own; every operation rounds to f32 exactly as the interpreter's
 * materialized intermediates do (no contraction, no fast math). */
enum {
  TOPOS_HIP_CHAIN_NEG = 0,
  TOPOS_HIP_CHAIN_EXP = 1,
  TOPOS_HIP_CHAIN_LN = 2,
  TOPOS_HIP_CHAIN_SQRT = 3,
  TOPOS_HIP_CHAIN_TANH = 4,
  TOPOS_HIP_CHAIN_ADD = 16,
  TOPOS_HIP_CHAIN_SUB = 17,
  TOPOS_HIP_CHAIN_MUL = 18,
  TOPOS_HIP_CHAIN_DIV = 19,
  TOPOS_HIP_CHAIN_MAX = 20,  /* f32::max */
  TOPOS_HIP_CHAIN_STEP = 21, /* x >= y ? 1 : 0 */
  TOPOS_HIP_CHAIN_POWF = 22  /* f32::powf: the host libm's powf */
};
#define TOPOS_HIP_MAX_RANK 6
/* A strided view of `rank` axes (the Layout of src/payload/layout.rs:23-31):
 * element (i0..) lives at offset + sum i_d * strides[d], in elements. */
typedef struct {
  int32_t rank;
  int64_t shape[TOPOS_HIP_MAX_RANK];
  int64_t strides[TOPOS_HIP_MAX_RANK];
  int64_t offset;
} topos_hip_layout;
/* Operand references: value >= 0 names an earlier instruction's result,
 * value < 0 names input (-value - 1). */
typedef struct {
  int32_t op;
  int32_t left;
  int32_t right; /* ignored by unary operations */
} topos_hip_chain_step;
typedef struct {
  int32_t rank;
  int64_t shape[TOPOS_HIP_MAX_RANK];      /* the logical shape of every view */
  int32_t n_inputs;
  const topos_hip_layout *inputs;         /* [n_inputs], each over `shape` */
  int32_t n_steps;
  const topos_hip_chain_step *steps;      /* [n_steps] */
  int32_t n_outputs;
  const int32_t *outputs;                 /* [n_outputs] step or input references */
} topos_hip_chain_desc;
typedef struct topos_hip_chain topos_hip_chain;
/* Generates and compiles (or fetches from the process cache) the chain's
 * kernel. */
int topos_hip_chain_create(const topos_hip_chain_desc *desc, topos_hip_chain **chain);
/* inputs[i] is the base pointer the i-th layout's offset and strides address;
 * outputs[o] receives volume(shape) contiguous elements. */
int topos_hip_chain_launch(const topos_hip_chain *chain, const float *const *inputs,
                           float *const *outputs, void *stream);
/* The generated HIP source (for inspection and tests); valid while the chain
 * lives. */
const char *topos_hip_chain_source(const topos_hip_chain *chain);
void topos_hip_chain_destroy(topos_hip_chain *chain);

/* ---- the plan face: device programs ----
 *
 * A device program is a topos forward plan lowered to a node table: the
 * plan's columns functions()/operands()/shapes()/readable()
 * (src/engine/plan.rs:311-347) in recording order, one record per node, plus
 * the leaf payloads. The library plays Plan::forward (plan.rs:514-641) on one
 * GPU: it recomputes reachability and liveness from the readable set, keeps
 * every view (transpose, permute, narrow, broadcasts, view-legal reshapes) as
 * a layout over its source's storage, fuses elementwise trees into generated
 * kernels, and places every materialised value at an offset of one
 * pre-sized HBM arena. Under TOPOS_HIP_EXACT every readable value is
 * bit-identical to the interpreter's (src/engine/run.rs:417-526); under
 * TOPOS_HIP_FAST products and row reductions meet the envelope instead.
 *
 * The producer is the plan consumer a `Backend::Hip` member adds beside
 * emit_stablehlo (src/emission/lower.rs:103-177).
 */

/* Node kinds: the Function variants (src/function/function.rs:26-59). */
enum {
  TOPOS_HIP_OP_LEAF = 0,           /* leaf: payload leaf_index */
  TOPOS_HIP_OP_PARAMETER = 1,      /* slot */
  TOPOS_HIP_OP_INPUT = 2,          /* slot */
  TOPOS_HIP_OP_ADD = 3,
  TOPOS_HIP_OP_SUB = 4,
  TOPOS_HIP_OP_MUL = 5,
  TOPOS_HIP_OP_DIV = 6,
  TOPOS_HIP_OP_NEG = 7,
  TOPOS_HIP_OP_TANH = 8,
  TOPOS_HIP_OP_EXP = 9,
  TOPOS_HIP_OP_LN = 10,
  TOPOS_HIP_OP_MATMUL = 11,
  TOPOS_HIP_OP_TRANSPOSE = 12,
  TOPOS_HIP_OP_SUM = 13,
  TOPOS_HIP_OP_SUM_ALONG = 14,     /* axis = params[0] */
  TOPOS_HIP_OP_BROADCAST = 15,     /* [operand, like] */
  TOPOS_HIP_OP_BROADCAST_ALONG = 16, /* [operand, like], axis = params[0] */
  TOPOS_HIP_OP_RESHAPE = 17,       /* to the node's shape */
  TOPOS_HIP_OP_PERMUTE = 18,       /* order = params[0..rank) */
  TOPOS_HIP_OP_NARROW = 19,        /* axis, start, len = params[0..3) */
  TOPOS_HIP_OP_PAD = 20,           /* axis, start, full_extent = params[0..3) */
  TOPOS_HIP_OP_UNFOLD = 21,        /* axis, size, step, dilation = params[0..4): a strided view */
  TOPOS_HIP_OP_FOLD = 22,          /* axis, size, step, dilation, extent = params[0..5) */
  TOPOS_HIP_OP_GATHER = 23,        /* [table, selection] */
  TOPOS_HIP_OP_SCATTER = 24,       /* [gradient, selection], rows = params[0] */
  TOPOS_HIP_OP_LOG_SOFTMAX = 25,   /* axis = params[0] */
  TOPOS_HIP_OP_LOG_SUM_EXP = 26,   /* axis = params[0] */
  TOPOS_HIP_OP_SQRT = 27,
  TOPOS_HIP_OP_POWF = 28,
  TOPOS_HIP_OP_MAXIMUM = 29,
  TOPOS_HIP_OP_RELU = 30,
  TOPOS_HIP_OP_STEP = 31
};

#define TOPOS_HIP_NODE_READABLE 1u /* a root or an observed value (plan.rs:150-158) */
/* An input fed with a Tensor::selection payload (src/payload/tensor.rs:312-342):
 * the node's shape is [rows, vocab] and params[0] holds the bits of its f32
 * `one`; bind it with topos_hip_program_bind_selection. */
#define TOPOS_HIP_NODE_SELECTION 2u

typedef struct {
  int32_t op;        /* TOPOS_HIP_OP_* */
  int32_t rank;      /* 0..TOPOS_HIP_MAX_RANK */
  int64_t shape[TOPOS_HIP_MAX_RANK]; /* the recorded shape (plan.shapes()) */
  int32_t operands[2];               /* earlier node indices; -1 where unused */
  int64_t params[TOPOS_HIP_MAX_RANK]; /* the variant's own parameters, as listed above */
  int32_t slot;      /* parameter/input slot, or the leaf payload's index */
  uint32_t flags;    /* TOPOS_HIP_NODE_* */
} topos_hip_node;

/* Leaf payloads (the Storage variants of src/payload/storage.rs:36-51). */
enum {
  TOPOS_HIP_LEAF_CONSTANT = 0,  /* `value` everywhere (Storage::Constant) */
  TOPOS_HIP_LEAF_DENSE = 1,     /* `count` row-major floats from leaf_data[offset] */
  TOPOS_HIP_LEAF_SELECTION = 2  /* `count` rows; row r selects leaf_indices[offset + r];
                                   `value` is the selection's one, its zero is +0 */
};
typedef struct {
  int32_t kind;
  float value;
  int64_t offset;
  int64_t count;
} topos_hip_leaf;

typedef struct topos_hip_program topos_hip_program;

/* Validates and plans the program (shape inference per node, views, fusion
 * groups, launch order, arena offsets) and compiles its generated kernels.
 * Every Function variant of src/function/function.rs:26-59 is planned
 * (Unfold as a strided view, Fold as one kernel); TOPOS_HIP_UNSUPPORTED names
 * an operation code no device kernel computes, TOPOS_HIP_INVALID_ARGUMENT a
 * malformed table. */
int topos_hip_program_create(const topos_hip_node *nodes, int64_t n_nodes, const topos_hip_leaf *leaves,
                             int64_t n_leaves, const float *leaf_data, int64_t leaf_data_len,
                             const int32_t *leaf_indices, int64_t leaf_indices_len, int numerics,
                             topos_hip_program **program);
/* The engine-backward route (Run::backward, src/engine/run.rs:229-318) for a
 * plan compiled with Request::backward(): the library appends the reverse
 * scan from the scalar node `target` to the forward table itself — one_like
 * seed, zero_like-seeded accumulation in reverse scan order, only ancestors
 * running their derivative rules (the `backward` of each src/function rule), only present
 * cotangents marking ancestors — and plans forward and backward as one
 * program whose arena keeps every forward value a rule reads. `wrt` lists the
 * nodes whose gradients the caller will read (Run::backward answers every
 * value; a device program keeps those asked for). Gradients equal
 * Tape::differentiate's recorded gradients bit for bit under
 * TOPOS_HIP_EXACT. TOPOS_HIP_INVALID_ARGUMENT for a non-scalar target. */
int topos_hip_program_create_backward(const topos_hip_node *nodes, int64_t n_nodes, const topos_hip_leaf *leaves,
                                      int64_t n_leaves, const float *leaf_data, int64_t leaf_data_len,
                                      const int32_t *leaf_indices, int64_t leaf_indices_len, int numerics,
                                      int64_t target, const int64_t *wrt, int64_t n_wrt,
                                      topos_hip_program **program);
/* The node of an engine-backward program holding the target's gradient with
 * respect to node `node` (one of its `wrt`): read it after a run with
 * topos_hip_program_output / topos_hip_program_read (Gradients::of). */
int topos_hip_program_gradient(const topos_hip_program *program, int64_t node, int64_t *gradient_node);
/* Bytes of the program's HBM arena (liveness-packed), and the number of
 * kernel launches one run enqueues. */
int topos_hip_program_info(const topos_hip_program *program, uint64_t *arena_bytes, int64_t *launches,
                           int64_t *fused_groups);
/* Binds a parameter or dense input slot to caller-owned device memory
 * holding the slot's recorded shape, row-major. The binding holds until
 * rebound; parameters stay resident across runs. */
int topos_hip_program_bind(topos_hip_program *program, int is_input, int32_t slot, const float *device);
/* Binds a selection input slot (Tensor::selection, src/payload/tensor.rs:312-342):
 * `rows` host indices, each below the recorded vocabulary, copied to the
 * device together with their row-sorted order (for the ordered scatter). */
int topos_hip_program_bind_selection(topos_hip_program *program, int32_t slot, const int32_t *indices,
                                     int64_t rows, float one);
/* Enqueues one forward run on `stream` (the arena is reserved on first use). */
int topos_hip_program_run(topos_hip_program *program, void *stream);
/* Enqueues one forward run on `stream` as a single HIP graph launch: the
 * first call (and the first after any bind) captures a run on a stream the
 * program owns and instantiates it; later calls replay that graph. Same
 * results as topos_hip_program_run, with one host call instead of one per
 * kernel. (No counterpart in the reference, which has no device runs.) */
int topos_hip_program_replay(topos_hip_program *program, void *stream);
/* One run with a HIP event pair around every launch, waited for;
 * `milliseconds[l]` receives launch l's duration (an array of `launches`
 * floats, topos_hip_program_info). For measurement, not for the hot loop. */
int topos_hip_program_run_profiled(topos_hip_program *program, void *stream, float *milliseconds);
/* Launch l's kind ("gemm", "chain", "fold", "sum", "rows", "gather",
 * "scatter", "copy", "pad", "scalar", "one-hot") and its algorithmic work: flops
 * for products, and bytes (each distinct input element read once, each
 * output written once) for everything. */
int topos_hip_program_launch(const topos_hip_program *program, int64_t launch, const char **kind, double *flops,
                             double *bytes);
/* The device address of a readable node's value after a run: contiguous
 * row-major, volume(shape) floats, valid until the next run. */
int topos_hip_program_output(const topos_hip_program *program, int64_t node, const float **device);
/* Copies a readable node's value to host memory (`count` = its volume) and
 * waits for it: the synchronous read-out of Run::value. */
int topos_hip_program_read(const topos_hip_program *program, int64_t node, float *host, int64_t count);
/* The reason the last program call on this thread was refused
 * (TOPOS_HIP_INVALID_ARGUMENT / TOPOS_HIP_UNSUPPORTED), or "". */
const char *topos_hip_last_refusal(void);
/* Describes the launch plan (one line per launch) for inspection and tests. */
const char *topos_hip_program_describe(const topos_hip_program *program);
void topos_hip_program_destroy(topos_hip_program *program);

/* ---- device-resident optimizer steps (src/neural/optimizer.rs:40-51,
 * src/neural/adam.rs:62-171) over `count` floats, in place ---- */

/* Sgd::step: parameter - gradient * rate. */
int topos_hip_sgd_step_f32(float *parameter, const float *gradient, int64_t count, float rate,
                           void *stream);
/* One AdamW parameter update with the moment buffers `first`/`second`
 * (updated in place; zero-filled before the first step stands for the
 * optimizer's absent moments, whose Constant-zero scaling gives the same
 * bits). `first_correction`/`second_correction` are 1 - beta^t as the
 * optimizer computes them in f32; `decay` applies when `decayed` != 0 (the
 * rank >= 2 policy of AdamW::step). An empty parameter (count 0) may pass
 * null pointers. */
int topos_hip_adamw_step_f32(float *parameter, const float *gradient, float *first, float *second,
                             int64_t count, float beta1, float beta2, float first_share,
                             float second_share, float first_correction, float second_correction,
                             float epsilon, float rate, float decay, int decayed, void *stream);

/* One parameter of a many-parameter AdamW step. */
typedef struct {
  float *parameter;
  const float *gradient;
  float *first;
  float *second;
  int64_t count;
  int32_t decayed; /* the rank >= 2 decay policy of AdamW::step */
} topos_hip_adamw_tensor;
/* AdamW::step over every parameter of a model (src/neural/adam.rs:62-171,
 * the loop over Parameters at :120-171) in as few launches as possible: each
 * element receives exactly the operations of topos_hip_adamw_step_f32 with
 * the shared scalars, so the two entry points give the same bits. Entries may
 * share memory (a tied parameter listed twice): an entry whose buffers
 * overlap what an earlier entry writes starts a new launch, so overlapping
 * updates apply in table order, as successive one-tensor calls would. */
int topos_hip_adamw_step_multi_f32(const topos_hip_adamw_tensor *tensors, int64_t count, float beta1, float beta2,
                                   float first_share, float second_share, float first_correction,
                                   float second_correction, float epsilon, float rate, float decay, void *stream);

/* ---- test surface ---- */

/* Installs a fake device runtime before first use (Api::fake of
 * src/backend/cuda/kernels/context.rs:101-162): setup succeeds without a GPU,
 * device memory is host memory, kernels are not run, and the device call
 * numbered `fail_after_calls` (0-based) fails, which must poison the library.
 * Returns TOPOS_HIP_INVALID_ARGUMENT once the real runtime is initialised. */
int topos_hip_fake_runtime(int fail_after_calls);

/* Bytes of the device face's grow-only split-k workspace held now (0 until a
 * device-face product first needs one). A diagnostic: lets a test show that
 * topos_hip_gemm_f32_device_noalloc never creates it. */
int64_t topos_hip_workspace_bytes(void);

#ifdef __cplusplus
}
#endif
#endif
