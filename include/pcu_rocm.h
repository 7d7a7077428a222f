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

#define PCU_ROCM_ABI_VERSION 1

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
    PCU_ERR_PROTOCOL = 8       /* malformed device fault status (owned_dispatch.rs:127-141) */
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
void pcu_ctx_close(pcu_ctx *ctx);
/* Last error text of `ctx` (or of the calling thread when ctx is NULL). */
const char *pcu_last_error(const pcu_ctx *ctx);
int pcu_abi_version(void);
/* Raw hipStream_t of the ordered stream, for callers that share device memory with it. */
void *pcu_ctx_stream(pcu_ctx *ctx);
pcu_status pcu_ctx_synchronize(pcu_ctx *ctx);

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
 * backends/cpu/prepared_tensor/prepared_tensor.rs:258-310). */

/* out[rows x cols] = op(left) * op(right); op(X) = X^T when the flag is set. Stored
 * shapes: left rows x inner (inner x rows if transposed), right inner x cols (cols x
 * inner if transposed). Ordered k, separately rounded multiply then add, from +0. */
pcu_status pcu_strict_matmul(pcu_ctx *ctx, pcu_dtype dtype, uint64_t rows, uint64_t inner,
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

/* ------------------------------------------------------------------ program
 * Between begin and end every op call is only enqueued and numbered as a node (0, 1, ...;
 * pcu_checked_add_relu takes two numbers). pcu_program_end synchronizes once and reports
 * the first fault in node order, the order the reference's per-node waits observe. */
pcu_status pcu_program_begin(pcu_ctx *ctx);
pcu_status pcu_program_end(pcu_ctx *ctx, pcu_fault *first_fault);
/* Node number the next op call will receive inside the current program. */
uint32_t pcu_program_next_node(const pcu_ctx *ctx);

/* ------------------------------------------------------- kernel timing hooks
 * HIP events recorded on the ordered stream around enqueued work, so a caller can time
 * exactly the kernels it launched (elapsed milliseconds between two marks). */
pcu_status pcu_mark(pcu_ctx *ctx, int slot);
pcu_status pcu_elapsed_ms(pcu_ctx *ctx, int from_slot, int to_slot, float *ms);

#ifdef __cplusplus
}
#endif
#endif /* PCU_ROCM_H */
