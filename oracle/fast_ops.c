/*
 * TEST INFRASTRUCTURE ONLY — the fast oracle.
 *
 * Same results as strict_ops.c, computed with the host's IEEE binary32/binary64 unit
 * (round-to-nearest-even, gradual underflow, compiled with -ffp-contract=off so every
 * multiply and add rounds on its own) and OpenMP across independent output cells or
 * elements. Hardware IEEE arithmetic gives the reference's value for every non-faulting
 * operation (pinned by tests/test_oracle_scalar.py); it cannot show tiny-inexact underflow,
 * so every lane or cell that a conservative screen cannot clear is re-run through the
 * integer law of strict_ops.c. Equality with the faithful functions is itself tested.
 * It exists so the full-size configurations can be checked in seconds.
 */
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

int orc_matmul_cell(int dtype, size_t rows, size_t inner, size_t cols, int tl, int tr,
                    const void *a, const void *b, size_t r, size_t c, int policy, void *out,
                    size_t *fk, int *fstep);

static int nthreads(int threads)
{
    return threads > 0 ? threads : omp_get_max_threads();
}

/* floor(log2|x|) of a finite nonzero value; a large value for zero or non-finite, which
 * contribute no tiny product (zero products are exact, non-finite ones show as non-finite
 * outputs). */
static int ilog2_f32(uint32_t bits)
{
    uint32_t e = (bits >> 23) & 0xff, f = bits & 0x7fffff;
    if (e == 0xff || (e == 0 && f == 0))
        return 1 << 20;
    if (e == 0)
        return (31 - __builtin_clz(f)) - 149;
    return (int)e - 127;
}
static int ilog2_f64(uint64_t bits)
{
    uint64_t e = (bits >> 52) & 0x7ff, f = bits & ((1ull << 52) - 1);
    if (e == 0x7ff || (e == 0 && f == 0))
        return 1 << 20;
    if (e == 0)
        return (63 - __builtin_clzll(f)) - 1074;
    return (int)e - 1023;
}

/* Smallest exponent-sum of a nonzero product that needs no exact replay:
 *  IEEE policy:   |p| >= 2^-126 (2^-1022) cannot be tiny after rounding, and no sum of
 *                 such products can be tiny-inexact (IEEE sums are exact when tiny);
 *  Reject policy: products >= 2^-103 (2^-970) are multiples of 2^-126 (2^-1022), so every
 *                 partial sum is zero or normal;
 *  Allow policy:  no underflow fault exists. */
static int risk_threshold(int dtype, int policy)
{
    if (policy == ORC_POLICY_ALLOW_GRADUAL)
        return -(1 << 28);
    if (policy == ORC_POLICY_REJECT_SUBNORMAL)
        return dtype == 0 ? -103 : -970;
    return dtype == 0 ? -126 : -1022;
}

static void record_first(orc_fault *best, int *have, uint64_t elem, uint64_t red, int step,
                         int kind)
{
    if (!*have || elem < best->element_index ||
        (elem == best->element_index && red < best->reduction_index)) {
        best->element_index = elem;
        best->reduction_index = red;
        best->step = step;
        best->kind = kind;
        *have = 1;
    }
}

#define JB 64

#define FAST_MATMUL_BODY(T, BITS_T, ILOG2, ISFIN)                                               \
    const BITS_T *Araw = a, *Braw = b;                                                          \
    T *C = c;                                                                                   \
    T *Aop = malloc(sizeof(T) * rows * inner);                                                  \
    T *Bop = malloc(sizeof(T) * inner * cols);                                                  \
    int *ea = malloc(sizeof(int) * rows), *eb = malloc(sizeof(int) * cols);                     \
    if (!Aop || !Bop || !ea || !eb) {                                                           \
        free(Aop); free(Bop); free(ea); free(eb);                                               \
        return -1;                                                                              \
    }                                                                                           \
    _Pragma("omp parallel for num_threads(nt)")                                                 \
    for (size_t r = 0; r < rows; r++) {                                                         \
        int m = 1 << 20;                                                                        \
        for (size_t k = 0; k < inner; k++) {                                                    \
            BITS_T v = Araw[tl ? k * rows + r : r * inner + k];                                 \
            memcpy(&Aop[r * inner + k], &v, sizeof(T));                                         \
            int e = ILOG2(v);                                                                   \
            m = e < m ? e : m;                                                                  \
        }                                                                                       \
        ea[r] = m;                                                                              \
    }                                                                                           \
    _Pragma("omp parallel for num_threads(nt)")                                                 \
    for (size_t k = 0; k < inner; k++)                                                          \
        for (size_t col = 0; col < cols; col++) {                                               \
            BITS_T v = Braw[tr ? col * inner + k : k * cols + col];                             \
            memcpy(&Bop[k * cols + col], &v, sizeof(T));                                        \
        }                                                                                       \
    _Pragma("omp parallel for num_threads(nt)")                                                 \
    for (size_t col = 0; col < cols; col++) {                                                   \
        int m = 1 << 20;                                                                        \
        for (size_t k = 0; k < inner; k++) {                                                    \
            BITS_T v;                                                                           \
            memcpy(&v, &Bop[k * cols + col], sizeof(T));                                        \
            int e = ILOG2(v);                                                                   \
            m = e < m ? e : m;                                                                  \
        }                                                                                       \
        eb[col] = m;                                                                            \
    }                                                                                           \
    size_t nb = (cols + JB - 1) / JB;                                                           \
    _Pragma("omp parallel for schedule(dynamic, 1) num_threads(nt)")                            \
    for (size_t t = 0; t < nb * ((rows + 15) / 16); t++) {                                      \
        size_t jb = (t % nb) * JB, r0 = (t / nb) * 16;                                          \
        size_t jn = cols - jb < JB ? cols - jb : JB;                                            \
        size_t r1 = r0 + 16 < rows ? r0 + 16 : rows;                                            \
        for (size_t r = r0; r < r1; r++) {                                                      \
            T acc[JB];                                                                          \
            for (size_t j = 0; j < JB; j++)                                                     \
                acc[j] = (T)0;                                                                  \
            const T *arow = &Aop[r * inner];                                                    \
            for (size_t k = 0; k < inner; k++) {                                                \
                T av = arow[k];                                                                 \
                const T *brow = &Bop[k * cols + jb];                                            \
                if (jn == JB) {                                                                 \
                    for (size_t j = 0; j < JB; j++) {                                           \
                        T p = av * brow[j];                                                     \
                        acc[j] = acc[j] + p;                                                    \
                    }                                                                           \
                } else {                                                                        \
                    for (size_t j = 0; j < jn; j++) {                                           \
                        T p = av * brow[j];                                                     \
                        acc[j] = acc[j] + p;                                                    \
                    }                                                                           \
                }                                                                               \
            }                                                                                   \
            for (size_t j = 0; j < jn; j++)                                                     \
                C[r * cols + jb + j] = acc[j];                                                  \
        }                                                                                       \
    }                                                                                           \
    int thr = risk_threshold(dtype, policy);                                                    \
    orc_fault best;                                                                             \
    int have = 0;                                                                               \
    _Pragma("omp parallel num_threads(nt)")                                                     \
    {                                                                                           \
        orc_fault mine;                                                                         \
        int mhave = 0;                                                                          \
        _Pragma("omp for schedule(static)")                                                     \
        for (size_t r = 0; r < rows; r++) {                                                     \
            if (mhave)                                                                          \
                continue;                                                                       \
            for (size_t col = 0; col < cols; col++) {                                           \
                T v = C[r * cols + col];                                                        \
                if (ISFIN(v) && (long)ea[r] + (long)eb[col] >= (long)thr)                       \
                    continue;                                                                   \
                size_t fk = 0;                                                                  \
                int fstep = 0;                                                                  \
                T exact;                                                                        \
                int kind = orc_matmul_cell(dtype, rows, inner, cols, tl, tr, a, b, r, col,      \
                                           policy, &exact, &fk, &fstep);                        \
                if (kind) {                                                                     \
                    record_first(&mine, &mhave, r * cols + col, fk, fstep, kind);               \
                    break;                                                                      \
                }                                                                               \
                C[r * cols + col] = exact;                                                      \
            }                                                                                   \
        }                                                                                       \
        _Pragma("omp critical")                                                                 \
        if (mhave)                                                                              \
            record_first(&best, &have, mine.element_index, mine.reduction_index, mine.step,     \
                         mine.kind);                                                            \
    }                                                                                           \
    free(Aop); free(Bop); free(ea); free(eb);                                                   \
    if (have) {                                                                                 \
        if (fault)                                                                              \
            *fault = best;                                                                      \
        return 1;                                                                               \
    }                                                                                           \
    return 0;

static int isfin_f(float v) { return isfinite(v); }
static int isfin_d(double v) { return isfinite(v); }

int orc_fast_matmul(int dtype, size_t rows, size_t inner, size_t cols, int tl, int tr,
                    const void *a, const void *b, void *c, int policy, int threads,
                    orc_fault *fault)
{
    int nt = nthreads(threads);
    if (dtype == 0) {
        FAST_MATMUL_BODY(float, uint32_t, ilog2_f32, isfin_f)
    } else {
        FAST_MATMUL_BODY(double, uint64_t, ilog2_f64, isfin_d)
    }
}

/* ------------------------------------------------------------------ elementwise */

static int screen_f32(int op, float x, float y, float r, int policy)
{
    if (!isfinite(x) || !isfinite(y) || !isfinite(r))
        return 1;
    float ar = fabsf(r);
    if (policy == ORC_POLICY_REJECT_SUBNORMAL && ar != 0.0f && ar < 1.17549435e-38f)
        return 1;
    if (op == ORC_OP_MUL || op == ORC_OP_DIV) {
        if (op == ORC_OP_DIV && y == 0.0f)
            return 1;
        if (policy != ORC_POLICY_ALLOW_GRADUAL && x != 0.0f && ar <= 1.17549435e-38f)
            return 1;
    }
    return 0;
}
static int screen_f64(int op, double x, double y, double r, int policy)
{
    if (!isfinite(x) || !isfinite(y) || !isfinite(r))
        return 1;
    double ar = fabs(r);
    if (policy == ORC_POLICY_REJECT_SUBNORMAL && ar != 0.0 && ar < 2.2250738585072014e-308)
        return 1;
    if (op == ORC_OP_MUL || op == ORC_OP_DIV) {
        if (op == ORC_OP_DIV && y == 0.0)
            return 1;
        if (policy != ORC_POLICY_ALLOW_GRADUAL && x != 0.0 && ar <= 2.2250738585072014e-308)
            return 1;
    }
    return 0;
}

static inline float hw_f32(int op, float x, float y)
{
    switch (op) {
    case ORC_OP_ADD: return x + y;
    case ORC_OP_SUB: return x - y;
    case ORC_OP_MUL: return x * y;
    default: return x / y;
    }
}
static inline double hw_f64(int op, double x, double y)
{
    switch (op) {
    case ORC_OP_ADD: return x + y;
    case ORC_OP_SUB: return x - y;
    case ORC_OP_MUL: return x * y;
    default: return x / y;
    }
}

int orc_fast_binary(int dtype, int op, size_t n, const void *a, const void *b, int b_scalar,
                    void *out, int policy, int threads, orc_fault *fault)
{
    int nt = nthreads(threads);
    size_t first = (size_t)-1;
    if (dtype == 0) {
        const float *x = a, *y = b;
        float *o = out;
#pragma omp parallel for reduction(min : first) num_threads(nt) schedule(static)
        for (size_t i = 0; i < n; i++) {
            float yv = y[b_scalar ? 0 : i];
            float r = hw_f32(op, x[i], yv);
            o[i] = r;
            if (screen_f32(op, x[i], yv, r, policy)) {
                uint32_t xb, yb, rb;
                memcpy(&xb, &x[i], 4);
                memcpy(&yb, &yv, 4);
                int k = orc_binary(0, op, 1, &xb, &yb, 1, &rb, policy, NULL);
                if (k && i < first)
                    first = i;
            }
        }
    } else {
        const double *x = a, *y = b;
        double *o = out;
#pragma omp parallel for reduction(min : first) num_threads(nt) schedule(static)
        for (size_t i = 0; i < n; i++) {
            double yv = y[b_scalar ? 0 : i];
            double r = hw_f64(op, x[i], yv);
            o[i] = r;
            if (screen_f64(op, x[i], yv, r, policy)) {
                uint64_t xb, yb, rb;
                memcpy(&xb, &x[i], 8);
                memcpy(&yb, &yv, 8);
                int k = orc_binary(1, op, 1, &xb, &yb, 1, &rb, policy, NULL);
                if (k && i < first)
                    first = i;
            }
        }
    }
    if (first == (size_t)-1)
        return 0;
    /* Re-run the faithful element to report its kind. */
    size_t es = dtype == 0 ? 4 : 8;
    char tmp[8];
    orc_fault f;
    orc_binary(dtype, op, 1, (const char *)a + first * es,
               b_scalar ? b : (const char *)b + first * es, 1, tmp, policy, &f);
    f.element_index = first;
    if (fault)
        *fault = f;
    return 1;
}

int orc_fast_relu(int dtype, size_t n, const void *x, void *out, int policy, int threads,
                  orc_fault *fault)
{
    int nt = nthreads(threads);
    size_t first = (size_t)-1;
    size_t es = dtype == 0 ? 4 : 8;
#pragma omp parallel for reduction(min : first) num_threads(nt) schedule(static)
    for (size_t i = 0; i < n; i++) {
        int k;
        if (dtype == 0)
            k = orc_relu_f32(((const uint32_t *)x)[i], policy, &((uint32_t *)out)[i]);
        else
            k = orc_relu_f64(((const uint64_t *)x)[i], policy, &((uint64_t *)out)[i]);
        if (k && i < first)
            first = i;
    }
    if (first == (size_t)-1)
        return 0;
    char tmp[8];
    orc_fault f;
    orc_relu(dtype, 1, (const char *)x + first * es, tmp, policy, &f);
    f.element_index = first;
    if (fault)
        *fault = f;
    return 1;
}

int orc_fast_sgd(int dtype, size_t n, const void *w, const void *g, uint32_t rate_bits,
                 void *out, int policy, int threads, orc_fault *fault)
{
    int nt = nthreads(threads);
    size_t first = (size_t)-1;
    size_t es = dtype == 0 ? 4 : 8;
    if (dtype == 0) {
        float rate;
        memcpy(&rate, &rate_bits, 4);
        const float *W = w, *G = g;
        float *o = out;
#pragma omp parallel for reduction(min : first) num_threads(nt) schedule(static)
        for (size_t i = 0; i < n; i++) {
            float p = rate * G[i];
            float r = W[i] - p;
            o[i] = r;
            if (screen_f32(ORC_OP_MUL, rate, G[i], p, policy) ||
                screen_f32(ORC_OP_SUB, W[i], p, r, policy)) {
                uint32_t tmp;
                if (orc_sgd(0, 1, &W[i], &G[i], rate_bits, &tmp, policy, NULL) && i < first)
                    first = i;
            }
        }
    } else {
        double rate;
        uint64_t rb = orc_f32_to_f64_bits(rate_bits);
        memcpy(&rate, &rb, 8);
        const double *W = w, *G = g;
        double *o = out;
#pragma omp parallel for reduction(min : first) num_threads(nt) schedule(static)
        for (size_t i = 0; i < n; i++) {
            double p = rate * G[i];
            double r = W[i] - p;
            o[i] = r;
            if (screen_f64(ORC_OP_MUL, rate, G[i], p, policy) ||
                screen_f64(ORC_OP_SUB, W[i], p, r, policy)) {
                uint64_t tmp;
                if (orc_sgd(1, 1, &W[i], &G[i], rate_bits, &tmp, policy, NULL) && i < first)
                    first = i;
            }
        }
    }
    if (first == (size_t)-1)
        return 0;
    char tmp[8];
    orc_fault f;
    orc_sgd(dtype, 1, (const char *)w + first * es, (const char *)g + first * es, rate_bits,
            tmp, policy, &f);
    f.element_index = first;
    if (fault)
        *fault = f;
    return 1;
}

int orc_fast_mse(int dtype, size_t n, const void *p, const void *t, void *out, int policy,
                 int threads, orc_fault *fault)
{
    int nt = nthreads(threads);
    size_t es = dtype == 0 ? 4 : 8;
    size_t first = n; /* first element whose Subtract or Multiply faults */
    void *sq = malloc(es * (n ? n : 1));
    if (!sq)
        return -1;
    if (dtype == 0) {
        const float *P = p, *T = t;
        float *S = sq;
#pragma omp parallel for reduction(min : first) num_threads(nt) schedule(static)
        for (size_t i = 0; i < n; i++) {
            float d = P[i] - T[i];
            float s = d * d;
            S[i] = s;
            if (screen_f32(ORC_OP_SUB, P[i], T[i], d, policy) ||
                screen_f32(ORC_OP_MUL, d, d, s, policy)) {
                uint32_t pb, tb, db, sb;
                memcpy(&pb, &P[i], 4);
                memcpy(&tb, &T[i], 4);
                int k = orc_sub_f32(pb, tb, policy, &db);
                if (!k)
                    k = orc_mul_f32(db, db, policy, &sb);
                if (k && i < first)
                    first = i;
            }
        }
    } else {
        const double *P = p, *T = t;
        double *S = sq;
#pragma omp parallel for reduction(min : first) num_threads(nt) schedule(static)
        for (size_t i = 0; i < n; i++) {
            double d = P[i] - T[i];
            double s = d * d;
            S[i] = s;
            if (screen_f64(ORC_OP_SUB, P[i], T[i], d, policy) ||
                screen_f64(ORC_OP_MUL, d, d, s, policy)) {
                uint64_t pb, tb, db, sb;
                memcpy(&pb, &P[i], 8);
                memcpy(&tb, &T[i], 8);
                int k = orc_sub_f64(pb, tb, policy, &db);
                if (!k)
                    k = orc_mul_f64(db, db, policy, &sb);
                if (k && i < first)
                    first = i;
            }
        }
    }
    /* The ordered sum runs up to the first Subtract/Multiply fault; an Add fault before it
     * comes first. Add of finite operands faults only by overflow (IEEE/Allow) or by a
     * subnormal sum (Reject). */
    size_t add_fault = (size_t)-1;
    int add_kind = 0;
    if (dtype == 0) {
        float total = 0.0f;
        const float *S = sq;
        for (size_t i = 0; i < first; i++) {
            total = total + S[i];
            float at = fabsf(total);
            if (!isfinite(total)) {
                add_fault = i;
                add_kind = ORC_OVERFLOW;
                break;
            }
            if (policy == ORC_POLICY_REJECT_SUBNORMAL && at != 0.0f && at < 1.17549435e-38f) {
                add_fault = i;
                add_kind = ORC_UNDERFLOW;
                break;
            }
        }
        if (add_fault == (size_t)-1 && first == n) {
            uint32_t tb, ob;
            memcpy(&tb, &total, 4);
            int k = orc_div_f32(tb, orc_u64_to_f32_rne(n), policy, &ob);
            free(sq);
            if (k) {
                if (fault) {
                    fault->element_index = 0;
                    fault->reduction_index = n;
                    fault->step = ORC_STEP_DIVIDE;
                    fault->kind = k;
                }
                return 1;
            }
            memcpy(out, &ob, 4);
            return 0;
        }
    } else {
        double total = 0.0;
        const double *S = sq;
        for (size_t i = 0; i < first; i++) {
            total = total + S[i];
            double at = fabs(total);
            if (!isfinite(total)) {
                add_fault = i;
                add_kind = ORC_OVERFLOW;
                break;
            }
            if (policy == ORC_POLICY_REJECT_SUBNORMAL && at != 0.0 &&
                at < 2.2250738585072014e-308) {
                add_fault = i;
                add_kind = ORC_UNDERFLOW;
                break;
            }
        }
        if (add_fault == (size_t)-1 && first == n) {
            uint64_t tb, ob;
            memcpy(&tb, &total, 8);
            int k = orc_div_f64(tb, orc_u64_to_f64_rne(n), policy, &ob);
            free(sq);
            if (k) {
                if (fault) {
                    fault->element_index = 0;
                    fault->reduction_index = n;
                    fault->step = ORC_STEP_DIVIDE;
                    fault->kind = k;
                }
                return 1;
            }
            memcpy(out, &ob, 8);
            return 0;
        }
    }
    free(sq);
    if (fault) {
        fault->element_index = 0;
        if (add_fault != (size_t)-1) {
            fault->reduction_index = add_fault;
            fault->step = ORC_STEP_ADD;
            fault->kind = add_kind;
        } else {
            /* Replay the faulting element through the integer law for its step and kind. */
            fault->reduction_index = first;
            if (dtype == 0) {
                uint32_t pb = ((const uint32_t *)p)[first], tb = ((const uint32_t *)t)[first], db, sb;
                int k = orc_sub_f32(pb, tb, policy, &db);
                fault->step = ORC_STEP_SUBTRACT;
                if (!k) {
                    k = orc_mul_f32(db, db, policy, &sb);
                    fault->step = ORC_STEP_MULTIPLY;
                }
                fault->kind = k;
            } else {
                uint64_t pb = ((const uint64_t *)p)[first], tb = ((const uint64_t *)t)[first], db, sb;
                int k = orc_sub_f64(pb, tb, policy, &db);
                fault->step = ORC_STEP_SUBTRACT;
                if (!k) {
                    k = orc_mul_f64(db, db, policy, &sb);
                    fault->step = ORC_STEP_MULTIPLY;
                }
                fault->kind = k;
            }
        }
    }
    return 1;
}
