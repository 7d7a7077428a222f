/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle for the strict owned-tensor path.
 *
 * This library is a C restatement of the reference CPU semantics (integer-significand
 * checked IEEE-754 arithmetic and the ordered strict compounds). It exists to check the
 * HIP product path. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it, and only as the checker or as the reported CPU baseline. The product
 * library (fusion-pcu_amd/csrc) never links or calls it.
 *
 * Reference files restated (paths relative to the reference's Crates/):
 *   core/scalar_checked_float.rs            f32 decode/jam/round/pack/add/mul/div/relu/neg
 *   core/scalar_checked_float/f64.rs        f64 twin
 *   core/scalar_float_underflow.rs:61-73    policy rejects()
 *   core/dialect/tensor/reference/strict_{matmul,sgd,mse}/ (*.rs)  ordered compounds
 *   backends/cpu/prepared_tensor/execution/execution.rs:192-302 CPU step runners
 */
#ifndef PCU_ORACLE_H
#define PCU_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* PcuExecutionFaultKind, numbered as the reference's packed fault word
 * (backends/rocm/owned_dispatch.rs:87-93). 0 means "no fault". */
enum {
    ORC_OK = 0,
    ORC_DIVIDE_BY_ZERO = 1,
    ORC_SIGNED_DIVISION_OVERFLOW = 2,
    ORC_OVERFLOW = 3,
    ORC_UNDERFLOW = 4,
    ORC_INVALID = 5
};

/* PcuFloatUnderflowPolicy (core/scalar_float_underflow.rs:47-58). */
enum { ORC_POLICY_IEEE = 0, ORC_POLICY_REJECT_SUBNORMAL = 1, ORC_POLICY_ALLOW_GRADUAL = 2 };

/* TensorArithmeticStep (core/dialect/tensor.rs:425-430), shifted by one so that 0 means
 * "elementwise fault without a compound step" (TensorError::ArithmeticFault). */
enum { ORC_STEP_NONE = 0, ORC_STEP_MULTIPLY = 1, ORC_STEP_ADD = 2, ORC_STEP_SUBTRACT = 3, ORC_STEP_DIVIDE = 4 };

/* Binary elementwise operators (BinaryOp in core/dialect/tensor.rs). */
enum { ORC_OP_ADD = 0, ORC_OP_SUB = 1, ORC_OP_MUL = 2, ORC_OP_DIV = 3 };

typedef struct {
    uint64_t element_index;   /* row-major output cell (0 for MSE) */
    uint64_t reduction_index; /* k for MatMul, i for MSE, 0 otherwise */
    int32_t step;             /* ORC_STEP_* */
    int32_t kind;             /* ORC_* fault kind */
} orc_fault;

/* ---- scalar law: returns the fault kind (ORC_OK on success) ---- */
int orc_add_f32(uint32_t a, uint32_t b, int policy, uint32_t *out);
int orc_sub_f32(uint32_t a, uint32_t b, int policy, uint32_t *out);
int orc_mul_f32(uint32_t a, uint32_t b, int policy, uint32_t *out);
int orc_div_f32(uint32_t a, uint32_t b, int policy, uint32_t *out);
int orc_neg_f32(uint32_t a, int policy, uint32_t *out);
int orc_relu_f32(uint32_t a, int policy, uint32_t *out);
int orc_relu_backward_f32(uint32_t input, uint32_t upstream, int policy, uint32_t *out);
int orc_add_f64(uint64_t a, uint64_t b, int policy, uint64_t *out);
int orc_sub_f64(uint64_t a, uint64_t b, int policy, uint64_t *out);
int orc_mul_f64(uint64_t a, uint64_t b, int policy, uint64_t *out);
int orc_div_f64(uint64_t a, uint64_t b, int policy, uint64_t *out);
int orc_neg_f64(uint64_t a, int policy, uint64_t *out);
int orc_relu_f64(uint64_t a, int policy, uint64_t *out);
int orc_relu_backward_f64(uint64_t input, uint64_t upstream, int policy, uint64_t *out);
/* Exact conversions used by the graph constants. */
uint32_t orc_u64_to_f32_rne(uint64_t v);
uint64_t orc_u64_to_f64_rne(uint64_t v);
uint64_t orc_f32_to_f64_bits(uint32_t v);

/* ---- faithful tensor ops (integer law, single thread, stop at first fault) ----
 * dtype: 0 = f32, 1 = f64. Return 0 on success, 1 on fault (fault filled). */
int orc_binary(int dtype, int op, size_t n, const void *a, const void *b, int b_scalar,
               void *out, int policy, orc_fault *fault);
int orc_relu(int dtype, size_t n, const void *x, void *out, int policy, orc_fault *fault);
int orc_relu_backward(int dtype, size_t n, const void *x, const void *up, void *out,
                      int policy, orc_fault *fault);
int orc_sgd(int dtype, size_t n, const void *w, const void *g, uint32_t rate_f32_bits,
            void *out, int policy, orc_fault *fault);
int orc_mse(int dtype, size_t n, const void *p, const void *t, void *out_scalar, int policy,
            orc_fault *fault);
/* C[rows x cols] = op(A)[rows x inner] * op(B)[inner x cols]; row_begin/row_end select
 * the output rows computed (a subset is used to time the faithful CPU baseline). */
int orc_matmul(int dtype, size_t rows, size_t inner, size_t cols, int transpose_left,
               int transpose_right, const void *a, const void *b, void *c, int policy,
               size_t row_begin, size_t row_end, orc_fault *fault);

/* ---- fast oracle: hardware IEEE (no contraction, no FTZ), OpenMP, with the exact
 * integer routine re-run on every screened lane/cell. Same results as the faithful
 * functions (checked by the oracle's own tests). threads <= 0 means "all". ---- */
int orc_fast_matmul(int dtype, size_t rows, size_t inner, size_t cols, int transpose_left,
                    int transpose_right, const void *a, const void *b, void *c, int policy,
                    int threads, orc_fault *fault);
int orc_fast_binary(int dtype, int op, size_t n, const void *a, const void *b, int b_scalar,
                    void *out, int policy, int threads, orc_fault *fault);
int orc_fast_relu(int dtype, size_t n, const void *x, void *out, int policy, int threads,
                  orc_fault *fault);
int orc_fast_sgd(int dtype, size_t n, const void *w, const void *g, uint32_t rate_f32_bits,
                 void *out, int policy, int threads, orc_fault *fault);
int orc_fast_mse(int dtype, size_t n, const void *p, const void *t, void *out_scalar,
                 int policy, int threads, orc_fault *fault);

/* Host FP environment probe: returns nonzero when MXCSR has FTZ or DAZ set. */
int orc_host_flushes_denormals(void);

#ifdef __cplusplus
}
#endif
#endif
