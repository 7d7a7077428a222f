/*
 * TEST INFRASTRUCTURE ONLY — faithful ordered tensor ops over the integer scalar law.
 *
 * Single-threaded, one checked scalar op after another, stopping at the first fault, as
 * the reference CPU prepared-tensor runners do (backends/cpu/prepared_tensor/execution/
 * execution.rs:192-302) and as the core reference compounds specify
 * (core/dialect/tensor/reference/strict_{matmul,sgd,mse}/ (*.rs)). The checker for the HIP
 * path and the faithful CPU baseline; never part of the product.
 */
#include "oracle.h"

#include <string.h>

static void set_fault(orc_fault *f, uint64_t element, uint64_t reduction, int step, int kind)
{
    if (!f)
        return;
    f->element_index = element;
    f->reduction_index = reduction;
    f->step = step;
    f->kind = kind;
}

typedef int (*bin32)(uint32_t, uint32_t, int, uint32_t *);
typedef int (*bin64)(uint64_t, uint64_t, int, uint64_t *);

static bin32 pick32(int op)
{
    switch (op) {
    case ORC_OP_ADD: return orc_add_f32;
    case ORC_OP_SUB: return orc_sub_f32;
    case ORC_OP_MUL: return orc_mul_f32;
    default: return orc_div_f32;
    }
}

static bin64 pick64(int op)
{
    switch (op) {
    case ORC_OP_ADD: return orc_add_f64;
    case ORC_OP_SUB: return orc_sub_f64;
    case ORC_OP_MUL: return orc_mul_f64;
    default: return orc_div_f64;
    }
}

/* execution.rs:192-211 (reference.rs:182-213): elementwise checked binary, a TensorError::
 * ArithmeticFault at the first failing element. b_scalar: b is one broadcast value (the
 * dense Uniform constant materialised by the reference holds that value everywhere). */
int orc_binary(int dtype, int op, size_t n, const void *a, const void *b, int b_scalar,
               void *out, int policy, orc_fault *fault)
{
    if (dtype == 0) {
        const uint32_t *x = a, *y = b;
        uint32_t *o = out;
        bin32 f = pick32(op);
        for (size_t i = 0; i < n; i++) {
            uint32_t r;
            int k = f(x[i], y[b_scalar ? 0 : i], policy, &r);
            if (k) {
                set_fault(fault, i, 0, ORC_STEP_NONE, k);
                return 1;
            }
            o[i] = r;
        }
    } else {
        const uint64_t *x = a, *y = b;
        uint64_t *o = out;
        bin64 f = pick64(op);
        for (size_t i = 0; i < n; i++) {
            uint64_t r;
            int k = f(x[i], y[b_scalar ? 0 : i], policy, &r);
            if (k) {
                set_fault(fault, i, 0, ORC_STEP_NONE, k);
                return 1;
            }
            o[i] = r;
        }
    }
    return 0;
}

/* execution.rs:212-219 */
int orc_relu(int dtype, size_t n, const void *xin, void *out, int policy, orc_fault *fault)
{
    for (size_t i = 0; i < n; i++) {
        int k;
        if (dtype == 0)
            k = orc_relu_f32(((const uint32_t *)xin)[i], policy, &((uint32_t *)out)[i]);
        else
            k = orc_relu_f64(((const uint64_t *)xin)[i], policy, &((uint64_t *)out)[i]);
        if (k) {
            set_fault(fault, i, 0, ORC_STEP_NONE, k);
            return 1;
        }
    }
    return 0;
}

/* execution.rs:220-230 */
int orc_relu_backward(int dtype, size_t n, const void *x, const void *up, void *out,
                      int policy, orc_fault *fault)
{
    for (size_t i = 0; i < n; i++) {
        int k;
        if (dtype == 0)
            k = orc_relu_backward_f32(((const uint32_t *)x)[i], ((const uint32_t *)up)[i],
                                      policy, &((uint32_t *)out)[i]);
        else
            k = orc_relu_backward_f64(((const uint64_t *)x)[i], ((const uint64_t *)up)[i],
                                      policy, &((uint64_t *)out)[i]);
        if (k) {
            set_fault(fault, i, 0, ORC_STEP_NONE, k);
            return 1;
        }
    }
    return 0;
}

/* execution.rs:231-242; strict_sgd.rs:20-46. p = rate (x) g, then w' = w (-) p. The F64
 * rate is the exact widening of the F32 literal (reference.rs:507-514). */
int orc_sgd(int dtype, size_t n, const void *w, const void *g, uint32_t rate_bits, void *out,
            int policy, orc_fault *fault)
{
    if (dtype == 0) {
        const uint32_t *W = w, *G = g;
        uint32_t *o = out;
        for (size_t i = 0; i < n; i++) {
            uint32_t p, r;
            int k = orc_mul_f32(rate_bits, G[i], policy, &p);
            if (k) {
                set_fault(fault, i, 0, ORC_STEP_MULTIPLY, k);
                return 1;
            }
            k = orc_sub_f32(W[i], p, policy, &r);
            if (k) {
                set_fault(fault, i, 0, ORC_STEP_SUBTRACT, k);
                return 1;
            }
            o[i] = r;
        }
    } else {
        const uint64_t *W = w, *G = g;
        uint64_t *o = out;
        uint64_t rate = orc_f32_to_f64_bits(rate_bits);
        for (size_t i = 0; i < n; i++) {
            uint64_t p, r;
            int k = orc_mul_f64(rate, G[i], policy, &p);
            if (k) {
                set_fault(fault, i, 0, ORC_STEP_MULTIPLY, k);
                return 1;
            }
            k = orc_sub_f64(W[i], p, policy, &r);
            if (k) {
                set_fault(fault, i, 0, ORC_STEP_SUBTRACT, k);
                return 1;
            }
            o[i] = r;
        }
    }
    return 0;
}

/* execution.rs:282-302; strict_mse.rs:22-59. Increasing element order: d = p (-) t,
 * s = d (x) d, total = total (+) s from +0; then total (/) count, count rounded to nearest
 * even (constants/constants.rs:18-28). The divide's reduction index is n. */
int orc_mse(int dtype, size_t n, const void *pp, const void *tt, void *out, int policy,
            orc_fault *fault)
{
    if (dtype == 0) {
        const uint32_t *P = pp, *T = tt;
        uint32_t total = 0;
        for (size_t i = 0; i < n; i++) {
            uint32_t d, s;
            int k = orc_sub_f32(P[i], T[i], policy, &d);
            if (k) {
                set_fault(fault, 0, i, ORC_STEP_SUBTRACT, k);
                return 1;
            }
            k = orc_mul_f32(d, d, policy, &s);
            if (k) {
                set_fault(fault, 0, i, ORC_STEP_MULTIPLY, k);
                return 1;
            }
            k = orc_add_f32(total, s, policy, &total);
            if (k) {
                set_fault(fault, 0, i, ORC_STEP_ADD, k);
                return 1;
            }
        }
        int k = orc_div_f32(total, orc_u64_to_f32_rne(n), policy, (uint32_t *)out);
        if (k) {
            set_fault(fault, 0, n, ORC_STEP_DIVIDE, k);
            return 1;
        }
    } else {
        const uint64_t *P = pp, *T = tt;
        uint64_t total = 0;
        for (size_t i = 0; i < n; i++) {
            uint64_t d, s;
            int k = orc_sub_f64(P[i], T[i], policy, &d);
            if (k) {
                set_fault(fault, 0, i, ORC_STEP_SUBTRACT, k);
                return 1;
            }
            k = orc_mul_f64(d, d, policy, &s);
            if (k) {
                set_fault(fault, 0, i, ORC_STEP_MULTIPLY, k);
                return 1;
            }
            k = orc_add_f64(total, s, policy, &total);
            if (k) {
                set_fault(fault, 0, i, ORC_STEP_ADD, k);
                return 1;
            }
        }
        int k = orc_div_f64(total, orc_u64_to_f64_rne(n), policy, (uint64_t *)out);
        if (k) {
            set_fault(fault, 0, n, ORC_STEP_DIVIDE, k);
            return 1;
        }
    }
    return 0;
}

/* Index of op(A)[r, k] and op(B)[k, c] in their row-major stored operands
 * (strict_matmul.rs:46-55; execution.rs:252-262). */
static inline size_t left_index(int tl, size_t rows, size_t inner, size_t r, size_t k)
{
    return tl ? k * rows + r : r * inner + k;
}
static inline size_t right_index(int tr, size_t inner, size_t cols, size_t k, size_t c)
{
    return tr ? c * inner + k : k * cols + c;
}

/* One output cell: +0 accumulator, k ascending, multiply then add, each checked.
 * Returns the fault kind; *fk receives the faulting k and *fstep its step. Exposed to the
 * fast oracle, which re-runs it on screened cells. */
int orc_matmul_cell(int dtype, size_t rows, size_t inner, size_t cols, int tl, int tr,
                    const void *a, const void *b, size_t r, size_t c, int policy, void *out,
                    size_t *fk, int *fstep)
{
    if (dtype == 0) {
        const uint32_t *A = a, *B = b;
        uint32_t acc = 0;
        for (size_t k = 0; k < inner; k++) {
            uint32_t p;
            int kind = orc_mul_f32(A[left_index(tl, rows, inner, r, k)],
                                   B[right_index(tr, inner, cols, k, c)], policy, &p);
            if (kind) {
                *fk = k;
                *fstep = ORC_STEP_MULTIPLY;
                return kind;
            }
            kind = orc_add_f32(acc, p, policy, &acc);
            if (kind) {
                *fk = k;
                *fstep = ORC_STEP_ADD;
                return kind;
            }
        }
        *(uint32_t *)out = acc;
    } else {
        const uint64_t *A = a, *B = b;
        uint64_t acc = 0;
        for (size_t k = 0; k < inner; k++) {
            uint64_t p;
            int kind = orc_mul_f64(A[left_index(tl, rows, inner, r, k)],
                                   B[right_index(tr, inner, cols, k, c)], policy, &p);
            if (kind) {
                *fk = k;
                *fstep = ORC_STEP_MULTIPLY;
                return kind;
            }
            kind = orc_add_f64(acc, p, policy, &acc);
            if (kind) {
                *fk = k;
                *fstep = ORC_STEP_ADD;
                return kind;
            }
        }
        *(uint64_t *)out = acc;
    }
    return ORC_OK;
}

/* strict_matmul.rs:22-73: row-major cells; the first fault is the lowest cell, then the
 * lowest k, then Multiply before Add. */
int orc_matmul(int dtype, size_t rows, size_t inner, size_t cols, int tl, int tr,
               const void *a, const void *b, void *c, int policy, size_t row_begin,
               size_t row_end, orc_fault *fault)
{
    size_t esize = dtype == 0 ? 4 : 8;
    if (row_end > rows)
        row_end = rows;
    for (size_t r = row_begin; r < row_end; r++) {
        for (size_t col = 0; col < cols; col++) {
            size_t fk = 0;
            int fstep = 0;
            char *dst = (char *)c + (r * cols + col) * esize;
            int kind = orc_matmul_cell(dtype, rows, inner, cols, tl, tr, a, b, r, col, policy,
                                       dst, &fk, &fstep);
            if (kind) {
                set_fault(fault, r * cols + col, fk, fstep, kind);
                return 1;
            }
        }
    }
    return 0;
}
