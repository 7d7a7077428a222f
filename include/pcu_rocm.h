/*
 * pcu_rocm.h — C ABI of the MI355X (gfx950) strict owned-tensor backend.
 *
 * The entry points are what the reference's ROCm lowering would bind in place of its
 * generated-HIP executor: the Rust side in Crates/backends keeps its Graph, lowers each
 * selected node to one call below (inside pcu_program_begin/end for one terminal
 * synchronization), and lifts a returned pcu_fault into TensorError /
 * PcuExecutionError. Plain pointers, sizes and enums only; no exceptions cross the ABI;
 * every handle is owned by the caller.
 *
 * Reference interfaces replaced (paths relative to the reference's Crates/):
 *   backends/rocm/tensor.rs:2364-2445,2593-2660  RocmTensorAssessor::{prepare_shared_owned_program,
 *                                                execute_owned_program_outputs*}
 *   backends/rocm/tensor.rs:5208-5250            execute_strict_matmul
 *   backends/rocm/tensor/strict_sgd/strict_sgd.rs:256-297   execute_strict_sgd
 *   backends/rocm/tensor/strict_mse/strict_mse.rs:234       execute_strict_mse
 *   backends/rocm/tensor/relu_backward/relu_backward.rs:136-230  ReLU-backward kernel
 *   backends/rocm/tensor/float.rs:130-227        checked Add/Sub/Mul, ReLU, Add->ReLU
 *   backends/rocm/owned_dispatch.rs:1137-1204,1556-1580  submit_validated / wait (fault word)
 *   backends/rocm/rocm.rs:515-530,1271-1300      allocate / DeviceBuffer copies
 *   backends/rocm/device_kernel.rs:351,416       upload_buffer / download_buffer
 *
 * Threading: a context belongs to one host thread at a time (the reference's PcuTensor is
 * neither Send nor Sync: fusion-pcu/global/arguments.rs:620-623).
 */
#ifndef PCU_ROCM_H
#define PCU_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PCU_ROCM_ABI_VERSION 3

typedef struct pcu_ctx pcu_ctx;

/* Return codes. Arithmetic faults are distinct from runtime errors
 * (fusion-pcu/global.rs:195-275 keeps ArithmeticFault apart from backend failures). */
typedef enum pcu_status {
    PCU_OK = 0,
    PCU_ARITHMETIC_FAULT = 1,  /* *fault filled; outputs of the faulting call unpublished */
    PCU_ERR_ARGUMENT = 2,      /* null pointer, bad enum, inconsistent sizes */
    PCU_ERR_SHAPE = 3,         /* shape does not admit the op (TensorError::MatMulShape, ...) */
    PCU_ERR_UNSUPPORTED = 4,   /* admitted by the reference but not by this backend */
    PCU_ERR_DEVICE = 5,        /* HIP runtime error (message in pcu_last_error) */
    PCU_ERR_OUT_OF_MEMORY = 6,
    PCU_ERR_STATE = 7,         /* call not allowed in the context's current mode */
    PCU_ERR_PROTOCOL = 8       /* malformed device fault status (owned_dispatch.rs:76-141); when
                                * the call takes a pcu_fault*, it holds the node and the raw
                                * word as (ordinal << 3) | kind, for the reference's
                                * HipError::InvalidExecutionFaultWord(word) */
} pcu_status;

typedef enum pcu_dtype { PCU_F32 = 0, PCU_F64 = 1 } pcu_dtype;

/* PcuFloatUnderflowPolicy (core/scalar_float_underflow.rs:47-58). */
typedef enum pcu_underflow {
    PCU_UNDERFLOW_IEEE_AFTER_ROUNDING = 0,
    PCU_UNDERFLOW_REJECT_SUBNORMAL = 1,
    PCU_UNDERFLOW_ALLOW_GRADUAL = 2
} pcu_underflow;

/* PcuExecutionFaultKind, numbered as the reference's packed fault word
 * (backends/rocm/owned_dispatch.rs:87-93). */
typedef enum pcu_fault_kind {
    PCU_FAULT_NONE = 0,
    PCU_FAULT_DIVIDE_BY_ZERO = 1,
    PCU_FAULT_SIGNED_DIVISION_OVERFLOW = 2,
    PCU_FAULT_OVERFLOW = 3,
    PCU_FAULT_UNDERFLOW = 4,
    PCU_FAULT_INVALID = 5
} pcu_fault_kind;

/* TensorArithmeticStep (core/dialect/tensor.rs:425-430); NONE marks an elementwise
 * TensorError::ArithmeticFault. */
typedef enum pcu_step {
    PCU_STEP_NONE = 0,
    PCU_STEP_MULTIPLY = 1,
    PCU_STEP_ADD = 2,
    PCU_STEP_SUBTRACT = 3,
    PCU_STEP_DIVIDE = 4
} pcu_step;

typedef enum pcu_binary_op { PCU_OP_ADD = 0, PCU_OP_SUB = 1, PCU_OP_MUL = 2, PCU_OP_DIV = 3 } pcu_binary_op;

/* One decoded first fault: TensorError::{ArithmeticFault, CompoundArithmeticFault}
 * coordinates (core/dialect/tensor.rs:234-252, fault_domain.rs:122-180). `node` is the
 * index of the faulting call within the program (0 outside program mode). */
typedef struct pcu_fault {
    uint32_t node;
    uint32_t kind;            /* pcu_fault_kind */
    uint32_t step;            /* pcu_step */
    uint32_t reserved;
    uint64_t element_index;   /* row-major output cell; 0 for MSE */
    uint64_t reduction_index; /* k for MatMul, element for MSE (n for its divide), else 0 */
    uint64_t ordinal;         /* position in the op's ordered fault domain */
} pcu_fault;

/* ------------------------------------------------------------------ context */

/* Opens `device`: one HIP stream for ordered work, one side stream for the serial MSE
 * sum, a retained stream-ordered memory pool and a pinned staging buffer. */
pcu_status pcu_ctx_open(int device, pcu_ctx **out);
/* Closing releases the device buffers of the prepared graphs built on the context and
 * detaches them: pcu_prepared_execute and pcu_prepared_take_output on them then return
 * PCU_ERR_STATE, and pcu_prepared_destroy only frees the host object. */
void pcu_ctx_close(pcu_ctx *ctx);
/* Last error text of `ctx` (or of the calling thread when ctx is NULL). */
const char *pcu_last_error(const pcu_ctx *ctx);
int pcu_abi_version(void);
/* Raw hipStream_t of the ordered stream, for callers that share device memory with it. */
void *pcu_ctx_stream(pcu_ctx *ctx);
pcu_status pcu_ctx_synchronize(pcu_ctx *ctx);

/* Engine of the strict MatMul. Every engine gives the same bits and the same first fault.
 *  PCU_MATMUL_VALU: each product is a v_mul and each sum a v_add (F32 and F64).
 *  PCU_MATMUL_MFMA_PRODUCTS: for F32 the matrix cores act as a multiplier array only
 *   (K = 1, +0 accumulator input): every element is one product rounded once. Outputs of
 *   fewer 128 x 128 tiles than CUs made of at most 512 whole 64 x 64 tiles, with K a
 *   multiple of 16, use v_mfma_f32_16x16x1_4b_f32 (four blocks, k0 .. k0 + 3); all other
 *   outputs use v_mfma_f32_32x32x1_2b_f32 (two blocks, k and k + 1). The ordered sums stay
 *   separate v_add_f32 in k order, and no sum is formed in the matrix core. F64 uses the
 *   vector unit.
 *  PCU_MATMUL_AUTO (default): outputs of at most 256 x 256 cells (F32) or 512 x 512 (F64)
 *   run as one fused launch on the vector unit (screen, products and sums, and the exact
 *   first-fault search per 16 x 16 block); larger ones as PCU_MATMUL_MFMA_PRODUCTS.
 *   Choosing VALU or MFMA_PRODUCTS always takes the screened tile kernels.
 * No counterpart in the reference, whose strict MatMul is one integer-emulated thread
 * per cell (backends/rocm/tensor/strict_matmul/strict_matmul.rs:187-239). */
typedef enum pcu_matmul_engine {
    PCU_MATMUL_AUTO = 0,
    PCU_MATMUL_VALU = 1,
    PCU_MATMUL_MFMA_PRODUCTS = 2
} pcu_matmul_engine;
pcu_status pcu_ctx_set_matmul_engine(pcu_ctx *ctx, pcu_matmul_engine engine);

/* ------------------------------------------------------------------- memory
 * Device buffers come from the context's stream-ordered pool (released memory is
 * retained for reuse); uploads and downloads go through the pinned staging buffer. */
pcu_status pcu_buf_alloc(pcu_ctx *ctx, size_t bytes, void **device_ptr);
pcu_status pcu_buf_free(pcu_ctx *ctx, void *device_ptr);
pcu_status pcu_upload(pcu_ctx *ctx, void *device_dst, const void *host_src, size_t bytes);
pcu_status pcu_download(pcu_ctx *ctx, void *host_dst, const void *device_src, size_t bytes);

/* ---------------------------------------------------------------------- ops
 * Operand pointers are device pointers. Outside program mode each call waits for its
 * kernels and returns PCU_ARITHMETIC_FAULT with *fault filled when the op faulted
 * (`fault` may be NULL). Inside program mode the call only enqueues; faults are reported
 * by pcu_program_end. On a fault the output's contents are unspecified and must not be
 * published (the reference never publishes a faulting node's output:
 * backends/cpu/prepared_tensor/prepared_tensor.rs:258-310). The elementwise and SGD calls
 * accept an `out` equal to one of their operands (in place); an `out` that overlaps an
 * operand any other way is rejected with PCU_ERR_ARGUMENT. */

/* out[rows x cols] = op(left) * op(right); op(X) = X^T when the flag is set. Stored
 * shapes: left rows x inner (inner x rows if transposed), right inner x cols (cols x
 * inner if transposed). Ordered k, separately rounded multiply then add, from +0.
 * `out` must not share any byte with `left` or `right` (PCU_ERR_ARGUMENT otherwise; the
 * same holds for pcu_native_matmul and, for the one output element, the MSE calls). */
pcu_status pcu_strict_matmul(pcu_ctx *ctx, pcu_dtype dtype, uint64_t rows, uint64_t inner,
                             uint64_t cols, int transpose_left, int transpose_right,
                             const void *left, const void *right, void *out,
                             pcu_underflow policy, pcu_fault *fault);

/* No counterpart in the reference. For callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the same
 * call and results as pcu_strict_matmul, with the exponent screen's scratch in a fixed array
 * of the library on each device instead of the context's pool, so the call allocates
 * nothing (no hipMalloc, hipFree or pool allocation; it is never per-kernel timed). rows and
 * cols are each at most PCU_NOALLOC_MAX_DIM; larger shapes return PCU_ERR_ARGUMENT. The
 * array (1.5 MiB + 256 B per device, held until the process ends) is shared by every call on
 * the device and keeps the last call's contents; the library clears what must start at zero.
 * Calls that overlap on one device (from two contexts or two host threads) race. The array
 * holds no partial-sum block flags, so under RejectSubnormal the call walks every cell the
 * exponent screen marks (same results and first fault, slower on marked inputs). */
#define PCU_NOALLOC_MAX_DIM 65536u
pcu_status pcu_strict_matmul_noalloc(pcu_ctx *ctx, pcu_dtype dtype, uint64_t rows, uint64_t inner,
                                     uint64_t cols, int transpose_left, int transpose_right,
                                     const void *left, const void *right, void *out,
                                     pcu_underflow policy, pcu_fault *fault);

/* out[i] = left[i] (op) right[i], checked. */
pcu_status pcu_checked_binary(pcu_ctx *ctx, pcu_dtype dtype, pcu_binary_op op, uint64_t n,
                              const void *left, const void *right, void *out,
                              pcu_underflow policy, pcu_fault *fault);
/* out[i] = left[i] (op) c, with c given by its bit pattern (a graph Uniform constant). */
pcu_status pcu_checked_binary_uniform(pcu_ctx *ctx, pcu_dtype dtype, pcu_binary_op op,
                                      uint64_t n, const void *left, uint64_t right_bits,
                                      void *out, pcu_underflow policy, pcu_fault *fault);
pcu_status pcu_checked_relu(pcu_ctx *ctx, pcu_dtype dtype, uint64_t n, const void *input,
                            void *out, pcu_underflow policy, pcu_fault *fault);
pcu_status pcu_checked_relu_backward(pcu_ctx *ctx, pcu_dtype dtype, uint64_t n,
                                     const void *input, const void *upstream, void *out,
                                     pcu_underflow policy, pcu_fault *fault);
/* Fused Add->ReLU for an Add whose only consumer is the ReLU. It counts as two program
 * nodes (the Add, then the ReLU), so node-major fault order is unchanged. */
pcu_status pcu_checked_add_relu(pcu_ctx *ctx, pcu_dtype dtype, uint64_t n, const void *left,
                                const void *right, void *out, pcu_underflow policy,
                                pcu_fault *fault);
/* out[i] = w[i] (-) (rate (x) g[i]); the F32 rate widens exactly for F64. */
pcu_status pcu_strict_sgd(pcu_ctx *ctx, pcu_dtype dtype, uint64_t n, const void *weights,
                          const void *gradient, float learning_rate, void *out,
                          pcu_underflow policy, pcu_fault *fault);
/* *out = (ordered sum of (p[i] (-) t[i])^2) (/) n, into one device element. */
pcu_status pcu_strict_mse(pcu_ctx *ctx, pcu_dtype dtype, uint64_t n, const void *prediction,
                          const void *target, void *out_scalar, pcu_underflow policy,
                          pcu_fault *fault);

/* ------------------------------------------------------------ native ops
 * Explicitly permitted native compound arithmetic (PcuCompoundArithmeticPolicy::
 * BackendDefined in Boundary mode, core/numerical/numerical.rs:21-35). The reference
 * routes these to rocBLAS SGEMM/DGEMM, a squared-difference kernel with rocBLAS ASUM, and
 * a native SGD kernel (backends/rocm/tensor.rs:9016-9052, tensor/native_loss/native_loss.rs,
 * tensor/native_sgd/native_sgd.rs). Reduction order, contraction and special-value
 * behaviour are backend-defined; no arithmetic fault is classified (a non-finite result is
 * an ordinary value). Shapes, pointers and device errors are still checked. Each call is a
 * program node like the strict ops. */

/* out = op(left) * op(right) in the declared precision. F32: matrix-core
 * multiply-accumulate tiles; F64: vector-unit fused multiply-add. */
pcu_status pcu_native_matmul(pcu_ctx *ctx, pcu_dtype dtype, uint64_t rows, uint64_t inner,
                             uint64_t cols, int transpose_left, int transpose_right,
                             const void *left, const void *right, void *out);
/* *out = (sum of (p[i] - t[i])^2) * (1 / count): the difference and the square are rounded
 * on their own, the sum is a fixed-shape tree in the declared precision, and the scale is the
 * rounded reciprocal of the element count (backends/rocm/tensor.rs:8701-8730). */
pcu_status pcu_native_mse(pcu_ctx *ctx, pcu_dtype dtype, uint64_t n, const void *prediction,
                          const void *target, void *out_scalar);
/* out[i] = w[i] - rate * g[i]: the product rounded before the subtraction, or one fused
 * multiply-add when `contracted` (PcuPrecisionPolicy::BackendOptimized,
 * backends/rocm/tensor.rs:4941-4945). */
pcu_status pcu_native_sgd(pcu_ctx *ctx, pcu_dtype dtype, uint64_t n, const void *weights,
                          const void *gradient, float learning_rate, int contracted, void *out);

/* ------------------------------------------------------------------ program
 * Between begin and end every op call is only enqueued and numbered as a node (0, 1, ...;
 * pcu_checked_add_relu takes two numbers). pcu_program_end synchronizes once and reports
 * the first fault in node order, the order the reference's per-node waits observe. */
pcu_status pcu_program_begin(pcu_ctx *ctx);
pcu_status pcu_program_end(pcu_ctx *ctx, pcu_fault *first_fault);
/* Node number the next op call will receive inside the current program. */
uint32_t pcu_program_next_node(const pcu_ctx *ctx);
/* The first fault of the most recent program (an op call outside a program is a program of
 * one node), as that call returned it: PCU_ARITHMETIC_FAULT with *fault filled, or PCU_OK
 * when that program completed without a fault or after pcu_fault_reset. Replaces the
 * reference's per-node read and decode of the packed fault word
 * (backends/rocm/owned_dispatch.rs:76-110) for callers that pass no pcu_fault to the ops. */
pcu_status pcu_fault_read(const pcu_ctx *ctx, pcu_fault *fault);
/* Forget the held fault (the reference re-arms each node's word with the u64::MAX sentinel,
 * backends/rocm/owned_dispatch.rs:20-21). */
pcu_status pcu_fault_reset(pcu_ctx *ctx);

/* ------------------------------------------------------- kernel timing hooks
 * HIP events recorded on the ordered stream around enqueued work, so a caller can time
 * exactly the kernels it launched (elapsed milliseconds between two marks). */
pcu_status pcu_mark(pcu_ctx *ctx, int slot);
pcu_status pcu_elapsed_ms(pcu_ctx *ctx, int from_slot, int to_slot, float *ms);

/* Per-kernel device time: while enabled, every launch of the kernels below is bracketed
 * by HIP events on the stream it runs on; pcu_profile_read synchronizes and returns the
 * accumulated milliseconds and launch count since pcu_profile_enable. No counterpart in
 * the reference (its per-node timing is host-side: backends/rocm/tensor.rs:1969-2020). */
typedef enum pcu_kernel_id {
    PCU_KERNEL_STRICT_GEMM = 0,     /* main strict MatMul tile kernel */
    PCU_KERNEL_GEMM_PREFILTER = 1,  /* exponent prefilter (both operands) */
    PCU_KERNEL_GEMM_REPLAY = 2,     /* exact replay of suspect cells */
    PCU_KERNEL_SGD = 3,
    PCU_KERNEL_BINARY = 4,
    PCU_KERNEL_RELU = 5,
    PCU_KERNEL_RELU_BACKWARD = 6,
    PCU_KERNEL_ADD_RELU = 7,
    PCU_KERNEL_MSE = 8,             /* squares + ordered sum + divide */
    PCU_KERNEL_NATIVE_GEMM = 9,     /* native (BackendDefined) MatMul */
    PCU_KERNEL_NATIVE_SGD = 10,
    PCU_KERNEL_NATIVE_MSE = 11,
    PCU_KERNEL_ELEMENTWISE_CHAIN = 12, /* a prepared program's fused elementwise nodes */
    PCU_KERNEL_COUNT = 13
} pcu_kernel_id;
pcu_status pcu_profile_enable(pcu_ctx *ctx, int on);
pcu_status pcu_profile_read(pcu_ctx *ctx, int kernel, double *total_ms, uint64_t *launches);

/* Measurement aid with no counterpart in the reference: copies `bytes` (a nonzero multiple
 * of 4096; both pointers 16-byte aligned; no overlap) from src to dst, reading with the
 * direct global-to-LDS load (global_load_lds_dwordx4) that the matrix-core MatMul tiles
 * stage with and writing with ordinary stores, then synchronizes. Hardware read counters of
 * one launch of known traffic scale those of the MatMul kernels' direct loads.
 * PCU_ERR_ARGUMENT for an invalid size, alignment or overlap. */
pcu_status pcu_calibrate_direct_copy(pcu_ctx *ctx, const void *src, void *dst, uint64_t bytes);

/* -------------------------------------------------------------------- graph
 * Host mirror of the reference's tensor Graph for the strict path: the builder calls
 * (core/dialect/tensor.rs:4028-4329), reverse mode for an MSE root
 * (core/dialect/tensor/gradients/gradients.rs:31-474), the execution plan
 * (tensor.rs:3234-3300) and a prepared executor (backends/rocm/tensor.rs:5827-6015).
 * Values are node indices in append order. Errors: PCU_ERR_ARGUMENT for UnknownValue and
 * invalid rates, PCU_ERR_SHAPE for ShapeMismatch/MatMulShape/ScalarTypeMismatch,
 * PCU_ERR_UNSUPPORTED for unsupported derivatives or Boundary compounds at prepare. */
typedef struct pcu_graph pcu_graph;
typedef struct pcu_prepared pcu_prepared;

/* Op codes of pcu_node_desc.op. */
typedef enum pcu_graph_op {
    PCU_GRAPH_INPUT = 0,
    PCU_GRAPH_UNIFORM = 1,
    PCU_GRAPH_ADD = 2,
    PCU_GRAPH_SUB = 3,
    PCU_GRAPH_MUL = 4,
    PCU_GRAPH_DIV = 5,
    PCU_GRAPH_SGD_UPDATE = 6,
    PCU_GRAPH_MATMUL = 7,
    PCU_GRAPH_RELU = 8,
    PCU_GRAPH_RELU_BACKWARD = 9,
    PCU_GRAPH_MEAN_SQUARED_ERROR = 10,
    PCU_GRAPH_CONSTANT = 11
} pcu_graph_op;

/* PcuNumericalOptions (core/numerical/numerical.rs:21-78): independent compound-arithmetic,
 * precision and reproducibility requirements captured by every appended node. */
typedef enum pcu_compound_arithmetic {
    PCU_COMPOUND_CHECKED = 0,
    PCU_COMPOUND_BACKEND_DEFINED = 1
} pcu_compound_arithmetic;
typedef enum pcu_precision { PCU_PRECISION_PRESERVE = 0, PCU_PRECISION_BACKEND_OPTIMIZED = 1 } pcu_precision;
typedef enum pcu_reproducibility { PCU_REPRO_UNSPECIFIED = 0, PCU_REPRO_PORTABLE_V1 = 1 } pcu_reproducibility;
typedef struct pcu_numerical_options {
    uint32_t compound_arithmetic; /* pcu_compound_arithmetic */
    uint32_t precision;           /* pcu_precision */
    uint32_t reproducibility;     /* pcu_reproducibility */
} pcu_numerical_options;

/* NodeDescriptor (core/dialect/tensor.rs:3575-3586). numerical_mode: -1 none,
 * 0 Boundary, 1 Strict; underflow_policy: -1 none, else pcu_underflow. Operands are
 * UINT32_MAX when absent. */
typedef struct pcu_node_desc {
    uint32_t op;
    uint32_t left, right;
    uint32_t transpose_left, transpose_right;
    uint32_t dtype;
    int32_t numerical_mode;
    int32_t underflow_policy;
    float learning_rate;
    uint32_t rank;
    uint64_t value_bits;
    uint64_t shape[8];
    pcu_numerical_options options;
    uint32_t reserved;
} pcu_node_desc;

pcu_status pcu_graph_create(pcu_graph **out);
void pcu_graph_destroy(pcu_graph *graph);
/* Graph::set_numerical_mode: compound nodes appended afterwards take this mode. */
pcu_status pcu_graph_set_numerical_mode(pcu_graph *graph, int strict);
pcu_status pcu_graph_input(pcu_graph *graph, pcu_dtype dtype, uint32_t rank, const uint64_t *shape,
                           uint32_t *id);
/* A dense logical tensor filled with one value (its bit pattern), never materialized
 * unless a consumer needs it dense. */
pcu_status pcu_graph_uniform(pcu_graph *graph, pcu_dtype dtype, uint32_t rank,
                             const uint64_t *shape, uint64_t value_bits, uint32_t *id);
/* An owned dense tensor constant (OpDescriptor::Constant, core/dialect/tensor.rs:377; built
 * by Graph::constant_value / constant_typed, :3669-3679): `host_data` holds the product of
 * `shape` elements of `dtype`, row-major, and is copied into the graph by this call. A
 * program that uses the node uploads it once at pcu_prepare and keeps it resident for every
 * execution. It is a leaf: it takes no derivative and is not a prepared input. */
pcu_status pcu_graph_constant(pcu_graph *graph, pcu_dtype dtype, uint32_t rank,
                              const uint64_t *shape, const void *host_data, uint32_t *id);
pcu_status pcu_graph_binary(pcu_graph *graph, pcu_binary_op op, uint32_t left, uint32_t right,
                            uint32_t *id);
pcu_status pcu_graph_relu(pcu_graph *graph, uint32_t input, uint32_t *id);
pcu_status pcu_graph_relu_backward(pcu_graph *graph, uint32_t input, uint32_t upstream,
                                   uint32_t *id);
pcu_status pcu_graph_matmul(pcu_graph *graph, uint32_t left, uint32_t right, int transpose_left,
                            int transpose_right, uint32_t *id);
pcu_status pcu_graph_mean_squared_error(pcu_graph *graph, uint32_t prediction, uint32_t target,
                                        uint32_t *id);
pcu_status pcu_graph_sgd_update(pcu_graph *graph, uint32_t weights, uint32_t gradient,
                                float learning_rate, uint32_t *id);
/* Graph::set_numerical_options (defaults for nodes appended afterwards) and
 * Graph::set_value_numerical_options (core/dialect/tensor.rs:3115-3136). */
pcu_status pcu_graph_set_numerical_options(pcu_graph *graph, const pcu_numerical_options *options);
pcu_status pcu_graph_set_value_numerical_options(pcu_graph *graph, uint32_t id,
                                                 const pcu_numerical_options *options);
/* Graph::set_value_float_underflow_policy / set_value_numerical_mode. */
pcu_status pcu_graph_set_underflow_policy(pcu_graph *graph, uint32_t id, pcu_underflow policy);
pcu_status pcu_graph_set_value_numerical_mode(pcu_graph *graph, uint32_t id, int strict);
/* Graph::backward_mse: grads[i] is the derivative value of node i (UINT32_MAX if none)
 * for every node that existed before the call; capacity >= node count. */
pcu_status pcu_graph_backward_mse(pcu_graph *graph, uint32_t loss, uint32_t *grads,
                                  uint32_t capacity);
/* Graph::backward_mse_for_targets (backward_mse_for is the one-target case). */
pcu_status pcu_graph_backward_mse_for_targets(pcu_graph *graph, uint32_t loss, uint32_t n_targets,
                                              const uint32_t *targets, uint32_t *grads);
uint32_t pcu_graph_node_count(const pcu_graph *graph);
pcu_status pcu_graph_describe(const pcu_graph *graph, uint32_t id, pcu_node_desc *out);
/* execution_plan_for_outputs: node ids in execution order (order may be NULL to query the
 * length; *order_len is its capacity on entry and the plan length on return). */
pcu_status pcu_graph_plan(const pcu_graph *graph, uint32_t n_outputs, const uint32_t *outputs,
                          uint32_t *order, uint32_t *order_len);

/* Admission of compound nodes (MatMul, MeanSquaredError, SgdUpdate) at prepare:
 *  Strict                                            -> the strict kernels;
 *  Boundary + BackendDefined, Unspecified reproducibility, IEEE (or no) underflow policy
 *                                                    -> the native kernels above;
 *  anything else                                     -> PCU_ERR_UNSUPPORTED (the reference
 *    rejects checked result-boundary MatMul: backends/rocm/tensor.rs:9053-9058).
 * Prepare once (plan; fusion of a single-use Add->ReLU, and of runs of up to four
 * consecutive elementwise nodes of one shape, each an operand of the next, into one kernel
 * that keeps one fault word per node; device storage with two banks per output), execute
 * many times. Inputs are device pointers in the order of the graph's Input
 * nodes that the plan uses (pcu_prepared_input_id). An execution that faults publishes
 * nothing and returns the first fault with `node` = its graph node id; the previous
 * outputs stay published, so a resident weight fed back as an input is never lost. */
pcu_status pcu_prepare(pcu_ctx *ctx, const pcu_graph *graph, uint32_t n_outputs,
                       const uint32_t *outputs, pcu_prepared **out);
void pcu_prepared_destroy(pcu_prepared *prepared);
uint32_t pcu_prepared_input_count(const pcu_prepared *prepared);
pcu_status pcu_prepared_input_id(const pcu_prepared *prepared, uint32_t index, uint32_t *id);
pcu_status pcu_prepared_execute(pcu_prepared *prepared, uint32_t n_inputs,
                                const void *const *device_inputs, pcu_fault *fault);
/* Device pointer of published output `index` (NULL before the first success). */
const void *pcu_prepared_output(const pcu_prepared *prepared, uint32_t index);
/* Moves published output `index` to the caller, who frees it with pcu_buf_free; the
 * program takes a fresh pool buffer for that slot. This is how a call returns fresh
 * owners (fusion-pcu/global/arguments.rs:636-660) without a device copy. */
pcu_status pcu_prepared_take_output(pcu_prepared *prepared, uint32_t index, void **device_ptr);

#ifdef __cplusplus
}
#endif
#endif /* PCU_ROCM_H */
