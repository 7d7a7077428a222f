// Bandwidth-bound strict kernels: checked Add/Sub/Mul/Div (tensor or uniform right
// operand), ReLU, ReLU-backward, fused Add->ReLU, strict SGD and strict MSE.
//
// Layout: dense row-major tensors in HBM. Each thread moves 16 bytes per operand per
// iteration (float4 / double2) in a grid-stride loop when the pointers and length allow,
// so one wave touches 1 KiB contiguous per operand per iteration. Faults are screened per
// lane, resolved exactly only on flagged lanes, and reduced with one ballot per wave and
// one atomicMin per faulting wave into the op's 64-bit fault word.
#include "pcu_device.hpp"
#include "pcu_kernels.hpp"

#pragma clang fp contract(off)

namespace pcu {

template <typename T> struct Vec;
template <> struct Vec<float> {
    using type = float4;
    static constexpr int width = 4;
};
template <> struct Vec<double> {
    using type = double2;
    static constexpr int width = 2;
};

template <typename T>
__device__ __forceinline__ void unpack(const typename Vec<T>::type &v, T *out);
template <>
__device__ __forceinline__ void unpack<float>(const float4 &v, float *o)
{
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
}
template <>
__device__ __forceinline__ void unpack<double>(const double2 &v, double *o)
{
    o[0] = v.x; o[1] = v.y;
}
template <typename T>
__device__ __forceinline__ typename Vec<T>::type pack(const T *o);
template <>
__device__ __forceinline__ float4 pack<float>(const float *o) { return make_float4(o[0], o[1], o[2], o[3]); }
template <>
__device__ __forceinline__ double2 pack<double>(const double *o) { return make_double2(o[0], o[1]); }

template <typename T, int OP>
__device__ __forceinline__ T apply(T a, T b)
{
    if (OP == kOpAdd) return a + b;
    if (OP == kOpSub) return a - b;
    if (OP == kOpMul) return a * b;
    return a / b;
}

template <typename T, int OP>
__device__ __forceinline__ bool suspect(T a, T b, T r, int policy)
{
    if (OP == kOpAdd || OP == kOpSub) return add_suspect(a, b, r, policy);
    if (OP == kOpMul) return mul_suspect(a, b, r, policy);
    return div_suspect(a, b, r, policy);
}

template <typename T, int OP>
__device__ __forceinline__ uint32_t classify(T a, T b, T r, int policy)
{
    if (OP == kOpAdd || OP == kOpSub) return classify_add(a, b, r, policy);
    if (OP == kOpMul) return classify_mul(a, b, r, policy);
    return classify_div(a, b, r, policy);
}

// ------------------------------------------------------------ checked binary

template <typename T, int OP, bool UNIFORM, bool VEC>
__global__ __launch_bounds__(256) void k_binary(const T *__restrict__ a, const T *__restrict__ b,
                                                T b_value, T *__restrict__ out, uint64_t n,
                                                int policy, unsigned long long *fault)
{
    constexpr int W = VEC ? Vec<T>::width : 1;
    uint64_t key = kNoFault;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x * W;
    for (uint64_t base = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * W; base < n;
         base += stride) {
        T x[W], y[W], r[W];
        if (VEC) {
            unpack<T>(*reinterpret_cast<const typename Vec<T>::type *>(a + base), x);
            if (UNIFORM) {
#pragma unroll
                for (int j = 0; j < W; j++) y[j] = b_value;
            } else {
                unpack<T>(*reinterpret_cast<const typename Vec<T>::type *>(b + base), y);
            }
        } else {
            x[0] = a[base];
            y[0] = UNIFORM ? b_value : b[base];
        }
        bool any = false;
#pragma unroll
        for (int j = 0; j < W; j++) {
            r[j] = apply<T, OP>(x[j], y[j]);
            any |= suspect<T, OP>(x[j], y[j], r[j], policy);
        }
        if (VEC)
            *reinterpret_cast<typename Vec<T>::type *>(out + base) = pack<T>(r);
        else
            out[base] = r[0];
        if (any && key == kNoFault) {
#pragma unroll
            for (int j = 0; j < W; j++) {
                uint32_t kind = classify<T, OP>(x[j], y[j], r[j], policy);
                if (kind != kOk && key == kNoFault)
                    key = pack_fault(base + j, kind);
            }
        }
    }
    wave_record_fault(key, fault);
}

// -------------------------------------------------------------------- relu

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void k_relu(const T *__restrict__ x, T *__restrict__ out,
                                              uint64_t n, int policy, unsigned long long *fault)
{
    constexpr int W = VEC ? Vec<T>::width : 1;
    uint64_t key = kNoFault;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x * W;
    for (uint64_t base = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * W; base < n;
         base += stride) {
        T v[W], r[W];
        if (VEC)
            unpack<T>(*reinterpret_cast<const typename Vec<T>::type *>(x + base), v);
        else
            v[0] = x[base];
        bool any = false;
#pragma unroll
        for (int j = 0; j < W; j++) {
            r[j] = relu_select(v[j]);
            any |= !finite_bits(v[j]) || (policy == kPolicyRejectSubnormal && subnormal(r[j]));
        }
        if (VEC)
            *reinterpret_cast<typename Vec<T>::type *>(out + base) = pack<T>(r);
        else
            out[base] = r[0];
        if (any && key == kNoFault) {
#pragma unroll
            for (int j = 0; j < W; j++) {
                uint32_t kind = classify_relu(v[j], r[j], policy);
                if (kind != kOk && key == kNoFault)
                    key = pack_fault(base + j, kind);
            }
        }
    }
    wave_record_fault(key, fault);
}

// ---------------------------------------------------------- relu backward

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void k_relu_backward(const T *__restrict__ x,
                                                       const T *__restrict__ up,
                                                       T *__restrict__ out, uint64_t n,
                                                       int policy, unsigned long long *fault)
{
    constexpr int W = VEC ? Vec<T>::width : 1;
    uint64_t key = kNoFault;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x * W;
    for (uint64_t base = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * W; base < n;
         base += stride) {
        T v[W], u[W], r[W];
        if (VEC) {
            unpack<T>(*reinterpret_cast<const typename Vec<T>::type *>(x + base), v);
            unpack<T>(*reinterpret_cast<const typename Vec<T>::type *>(up + base), u);
        } else {
            v[0] = x[base];
            u[0] = up[base];
        }
        bool any = false;
#pragma unroll
        for (int j = 0; j < W; j++) {
            r[j] = strictly_positive(v[j]) ? u[j] : (T)0;
            any |= !finite_bits(v[j]) || !finite_bits(u[j]) ||
                   (policy == kPolicyRejectSubnormal && subnormal(r[j]));
        }
        if (VEC)
            *reinterpret_cast<typename Vec<T>::type *>(out + base) = pack<T>(r);
        else
            out[base] = r[0];
        if (any && key == kNoFault) {
#pragma unroll
            for (int j = 0; j < W; j++) {
                uint32_t kind = classify_relu_backward(v[j], u[j], r[j], policy);
                if (kind != kOk && key == kNoFault)
                    key = pack_fault(base + j, kind);
            }
        }
    }
    wave_record_fault(key, fault);
}

// ------------------------------------------------------------ fused add->relu
// The Add node's faults go to fault_add and the ReLU node's to fault_relu, so the
// node-major first-fault order is the same as running the two nodes one after the other
// (a ReLU of a successful, hence finite, sum can only fault under RejectSubnormal).

template <typename T, bool UNIFORM, bool VEC>
__global__ __launch_bounds__(256) void k_add_relu(const T *__restrict__ a, const T *__restrict__ b,
                                                  T b_value, T *__restrict__ out, uint64_t n,
                                                  int policy, unsigned long long *fault_add,
                                                  unsigned long long *fault_relu)
{
    constexpr int W = VEC ? Vec<T>::width : 1;
    uint64_t key_add = kNoFault, key_relu = kNoFault;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x * W;
    for (uint64_t base = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * W; base < n;
         base += stride) {
        T x[W], y[W], s[W], r[W];
        if (VEC) {
            unpack<T>(*reinterpret_cast<const typename Vec<T>::type *>(a + base), x);
            if (UNIFORM) {
#pragma unroll
                for (int j = 0; j < W; j++) y[j] = b_value;
            } else {
                unpack<T>(*reinterpret_cast<const typename Vec<T>::type *>(b + base), y);
            }
        } else {
            x[0] = a[base];
            y[0] = UNIFORM ? b_value : b[base];
        }
        bool any = false;
#pragma unroll
        for (int j = 0; j < W; j++) {
            s[j] = x[j] + y[j];
            r[j] = relu_select(s[j]);
            any |= add_suspect(x[j], y[j], s[j], policy) ||
                   (policy == kPolicyRejectSubnormal && subnormal(r[j]));
        }
        if (VEC)
            *reinterpret_cast<typename Vec<T>::type *>(out + base) = pack<T>(r);
        else
            out[base] = r[0];
        if (any) {
#pragma unroll
            for (int j = 0; j < W; j++) {
                uint32_t ka = classify_add(x[j], y[j], s[j], policy);
                if (ka != kOk) {
                    if (key_add == kNoFault)
                        key_add = pack_fault(base + j, ka);
                } else {
                    uint32_t kr = classify_relu(s[j], r[j], policy);
                    if (kr != kOk && key_relu == kNoFault)
                        key_relu = pack_fault(base + j, kr);
                }
            }
        }
    }
    wave_record_fault(key_add, fault_add);
    wave_record_fault(key_relu, fault_relu);
}

// -------------------------------------------------------------------- SGD
// core/dialect/tensor/reference/strict_sgd/strict_sgd.rs:20-46: p = rate (x) g, then
// w' = w (-) p; ordinal 2i (Multiply) and 2i+1 (Subtract).

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void k_sgd(const T *__restrict__ w, const T *__restrict__ g,
                                             T rate, T *__restrict__ out, uint64_t n, int policy,
                                             unsigned long long *fault)
{
    constexpr int W = VEC ? Vec<T>::width : 1;
    uint64_t key = kNoFault;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x * W;
    for (uint64_t base = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * W; base < n;
         base += stride) {
        T wv[W], gv[W], p[W], r[W];
        if (VEC) {
            unpack<T>(*reinterpret_cast<const typename Vec<T>::type *>(w + base), wv);
            unpack<T>(*reinterpret_cast<const typename Vec<T>::type *>(g + base), gv);
        } else {
            wv[0] = w[base];
            gv[0] = g[base];
        }
        bool any = false;
#pragma unroll
        for (int j = 0; j < W; j++) {
            p[j] = rate * gv[j];
            r[j] = wv[j] - p[j];
            any |= mul_suspect(rate, gv[j], p[j], policy) | add_suspect(wv[j], p[j], r[j], policy);
        }
        if (VEC)
            *reinterpret_cast<typename Vec<T>::type *>(out + base) = pack<T>(r);
        else
            out[base] = r[0];
        if (any && key == kNoFault) {
#pragma unroll
            for (int j = 0; j < W; j++) {
                if (key != kNoFault)
                    break;
                uint32_t km = classify_mul(rate, gv[j], p[j], policy);
                if (km != kOk) {
                    key = pack_fault(2 * (base + j), km);
                } else {
                    uint32_t ks = classify_add(wv[j], p[j], r[j], policy);
                    if (ks != kOk)
                        key = pack_fault(2 * (base + j) + 1, ks);
                }
            }
        }
    }
    wave_record_fault(key, fault);
}

// -------------------------------------------------------------------- MSE
// core/dialect/tensor/reference/strict_mse/strict_mse.rs:22-59. Stage 1 (parallel):
// d = p (-) t and s = d (x) d per element, ordinals 3i and 3i+1. Stage 2 (one wave): the
// ordered sum total = total (+) s_i from +0 (ordinal 3i+2), then total (/) count
// (ordinal 3n). The sum is a dependent chain by contract; it stops before the first
// element whose Subtract or Multiply faulted.

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void k_mse_squares(const T *__restrict__ p,
                                                     const T *__restrict__ t,
                                                     T *__restrict__ sq, uint64_t n, int policy,
                                                     unsigned long long *fault)
{
    constexpr int W = VEC ? Vec<T>::width : 1;
    uint64_t key = kNoFault;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x * W;
    for (uint64_t base = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * W; base < n;
         base += stride) {
        T pv[W], tv[W], d[W], s[W];
        if (VEC) {
            unpack<T>(*reinterpret_cast<const typename Vec<T>::type *>(p + base), pv);
            unpack<T>(*reinterpret_cast<const typename Vec<T>::type *>(t + base), tv);
        } else {
            pv[0] = p[base];
            tv[0] = t[base];
        }
        bool any = false;
#pragma unroll
        for (int j = 0; j < W; j++) {
            d[j] = pv[j] - tv[j];
            s[j] = d[j] * d[j];
            any |= add_suspect(pv[j], tv[j], d[j], policy) | mul_suspect(d[j], d[j], s[j], policy);
        }
        if (VEC)
            *reinterpret_cast<typename Vec<T>::type *>(sq + base) = pack<T>(s);
        else
            sq[base] = s[0];
        if (any && key == kNoFault) {
#pragma unroll
            for (int j = 0; j < W; j++) {
                if (key != kNoFault)
                    break;
                uint32_t ks = classify_add(pv[j], tv[j], d[j], policy);
                if (ks != kOk) {
                    key = pack_fault(3 * (base + j), ks);
                } else {
                    uint32_t km = classify_mul(d[j], d[j], s[j], policy);
                    if (km != kOk)
                        key = pack_fault(3 * (base + j) + 1, km);
                }
            }
        }
    }
    wave_record_fault(key, fault);
}

// One wave. Every lane runs the same dependent chain; the squares are read through
// uniform addresses (scalar loads), so each element costs one dependent VALU add.
template <typename T>
__global__ __launch_bounds__(64) void k_mse_ordered_sum(const T *__restrict__ sq, uint64_t n,
                                                        T count, int policy, T *__restrict__ out,
                                                        unsigned long long *fault)
{
    // Elements at or after the first Subtract/Multiply fault are never summed.
    uint64_t w = __atomic_load_n(fault, __ATOMIC_RELAXED);
    uint64_t limit = n;
    if (w != kNoFault)
        limit = (w >> 3) / 3;
    T total = (T)0;
    uint64_t i = 0;
    constexpr int CH = 16;
    for (; i + CH <= limit; i += CH) {
        T s[CH];
#pragma unroll
        for (int j = 0; j < CH; j++) s[j] = sq[i + j];
        T before = total;
#pragma unroll
        for (int j = 0; j < CH; j++) total = total + s[j];
        // Squares and partial sums are nonnegative and finite until an Add overflows, or,
        // under RejectSubnormal, a partial sum is subnormal: replay the chunk to find it.
        bool bad = !finite_bits(total) || (policy == kPolicyRejectSubnormal);
        if (bad) {
            T acc = before;
            for (int j = 0; j < CH; j++) {
                T nxt = acc + s[j];
                uint32_t k = classify_add(acc, s[j], nxt, policy);
                if (k != kOk) {
                    if (__lane_id() == 0)
                        atomicMin(fault, (unsigned long long)pack_fault(3 * (i + j) + 2, k));
                    return;
                }
                acc = nxt;
            }
        }
    }
    for (; i < limit; i++) {
        T nxt = total + sq[i];
        uint32_t k = classify_add(total, sq[i], nxt, policy);
        if (k != kOk) {
            if (__lane_id() == 0)
                atomicMin(fault, (unsigned long long)pack_fault(3 * i + 2, k));
            return;
        }
        total = nxt;
    }
    if (limit < n)
        return;
    T r = total / count;
    uint32_t k = classify_div(total, count, r, policy);
    if (__lane_id() == 0) {
        if (k != kOk)
            atomicMin(fault, (unsigned long long)pack_fault(3 * n, k));
        else
            *out = r;
    }
}

// ================================================================ launchers

static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

static inline unsigned grid_for(uint64_t work_items)
{
    uint64_t blocks = (work_items + 255) / 256;
    if (blocks > 16384)
        blocks = 16384;
    return blocks ? (unsigned)blocks : 1u;
}

template <typename T>
static hipError_t binary_t(hipStream_t s, int op, uint64_t n, const void *a, const void *b,
                           const void *b_value, void *out, int policy, unsigned long long *fault)
{
    const T *A = (const T *)a, *B = (const T *)b;
    T bv = b_value ? *(const T *)b_value : (T)0;
    bool uniform = b == nullptr;
    constexpr int Wd = Vec<T>::width;
    bool vec = n % Wd == 0 && aligned16(a) && aligned16(out) && (uniform || aligned16(b));
    unsigned grid = grid_for(vec ? n / Wd : n);
#define PCU_LAUNCH_BINARY(OPC)                                                                      \
    if (uniform) {                                                                                  \
        if (vec) hipLaunchKernelGGL((k_binary<T, OPC, true, true>), dim3(grid), dim3(256), 0, s, A, B, bv, (T *)out, n, policy, fault); \
        else hipLaunchKernelGGL((k_binary<T, OPC, true, false>), dim3(grid), dim3(256), 0, s, A, B, bv, (T *)out, n, policy, fault); \
    } else {                                                                                        \
        if (vec) hipLaunchKernelGGL((k_binary<T, OPC, false, true>), dim3(grid), dim3(256), 0, s, A, B, bv, (T *)out, n, policy, fault); \
        else hipLaunchKernelGGL((k_binary<T, OPC, false, false>), dim3(grid), dim3(256), 0, s, A, B, bv, (T *)out, n, policy, fault); \
    }
    switch (op) {
    case kOpAdd: PCU_LAUNCH_BINARY(kOpAdd) break;
    case kOpSub: PCU_LAUNCH_BINARY(kOpSub) break;
    case kOpMul: PCU_LAUNCH_BINARY(kOpMul) break;
    default: PCU_LAUNCH_BINARY(kOpDiv) break;
    }
#undef PCU_LAUNCH_BINARY
    return hipGetLastError();
}

hipError_t launch_binary(hipStream_t s, int dtype, int op, uint64_t n, const void *a,
                         const void *b, const void *b_value, void *out, int policy,
                         unsigned long long *fault)
{
    if (n == 0)
        return hipSuccess;
    return dtype == 0 ? binary_t<float>(s, op, n, a, b, b_value, out, policy, fault)
                      : binary_t<double>(s, op, n, a, b, b_value, out, policy, fault);
}

template <typename T>
static hipError_t relu_t(hipStream_t s, uint64_t n, const void *x, void *out, int policy,
                         unsigned long long *fault)
{
    constexpr int Wd = Vec<T>::width;
    bool vec = n % Wd == 0 && aligned16(x) && aligned16(out);
    unsigned grid = grid_for(vec ? n / Wd : n);
    if (vec)
        hipLaunchKernelGGL((k_relu<T, true>), dim3(grid), dim3(256), 0, s, (const T *)x, (T *)out, n, policy, fault);
    else
        hipLaunchKernelGGL((k_relu<T, false>), dim3(grid), dim3(256), 0, s, (const T *)x, (T *)out, n, policy, fault);
    return hipGetLastError();
}

hipError_t launch_relu(hipStream_t s, int dtype, uint64_t n, const void *x, void *out,
                       int policy, unsigned long long *fault)
{
    if (n == 0)
        return hipSuccess;
    return dtype == 0 ? relu_t<float>(s, n, x, out, policy, fault)
                      : relu_t<double>(s, n, x, out, policy, fault);
}

template <typename T>
static hipError_t relu_backward_t(hipStream_t s, uint64_t n, const void *x, const void *up,
                                  void *out, int policy, unsigned long long *fault)
{
    constexpr int Wd = Vec<T>::width;
    bool vec = n % Wd == 0 && aligned16(x) && aligned16(up) && aligned16(out);
    unsigned grid = grid_for(vec ? n / Wd : n);
    if (vec)
        hipLaunchKernelGGL((k_relu_backward<T, true>), dim3(grid), dim3(256), 0, s, (const T *)x, (const T *)up, (T *)out, n, policy, fault);
    else
        hipLaunchKernelGGL((k_relu_backward<T, false>), dim3(grid), dim3(256), 0, s, (const T *)x, (const T *)up, (T *)out, n, policy, fault);
    return hipGetLastError();
}

hipError_t launch_relu_backward(hipStream_t s, int dtype, uint64_t n, const void *x,
                                const void *up, void *out, int policy,
                                unsigned long long *fault)
{
    if (n == 0)
        return hipSuccess;
    return dtype == 0 ? relu_backward_t<float>(s, n, x, up, out, policy, fault)
                      : relu_backward_t<double>(s, n, x, up, out, policy, fault);
}

template <typename T>
static hipError_t add_relu_t(hipStream_t s, uint64_t n, const void *a, const void *b,
                             const void *b_value, void *out, int policy,
                             unsigned long long *fault_add, unsigned long long *fault_relu)
{
    const T *A = (const T *)a, *B = (const T *)b;
    T bv = b_value ? *(const T *)b_value : (T)0;
    bool uniform = b == nullptr;
    constexpr int Wd = Vec<T>::width;
    bool vec = n % Wd == 0 && aligned16(a) && aligned16(out) && (uniform || aligned16(b));
    unsigned grid = grid_for(vec ? n / Wd : n);
    if (uniform) {
        if (vec) hipLaunchKernelGGL((k_add_relu<T, true, true>), dim3(grid), dim3(256), 0, s, A, B, bv, (T *)out, n, policy, fault_add, fault_relu);
        else hipLaunchKernelGGL((k_add_relu<T, true, false>), dim3(grid), dim3(256), 0, s, A, B, bv, (T *)out, n, policy, fault_add, fault_relu);
    } else {
        if (vec) hipLaunchKernelGGL((k_add_relu<T, false, true>), dim3(grid), dim3(256), 0, s, A, B, bv, (T *)out, n, policy, fault_add, fault_relu);
        else hipLaunchKernelGGL((k_add_relu<T, false, false>), dim3(grid), dim3(256), 0, s, A, B, bv, (T *)out, n, policy, fault_add, fault_relu);
    }
    return hipGetLastError();
}

hipError_t launch_add_relu(hipStream_t s, int dtype, uint64_t n, const void *a, const void *b,
                           const void *b_value, void *out, int policy,
                           unsigned long long *fault_add, unsigned long long *fault_relu)
{
    if (n == 0)
        return hipSuccess;
    return dtype == 0 ? add_relu_t<float>(s, n, a, b, b_value, out, policy, fault_add, fault_relu)
                      : add_relu_t<double>(s, n, a, b, b_value, out, policy, fault_add, fault_relu);
}

template <typename T>
static hipError_t sgd_t(hipStream_t s, uint64_t n, const void *w, const void *g, T rate,
                        void *out, int policy, unsigned long long *fault)
{
    constexpr int Wd = Vec<T>::width;
    bool vec = n % Wd == 0 && aligned16(w) && aligned16(g) && aligned16(out);
    unsigned grid = grid_for(vec ? n / Wd : n);
    if (vec)
        hipLaunchKernelGGL((k_sgd<T, true>), dim3(grid), dim3(256), 0, s, (const T *)w, (const T *)g, rate, (T *)out, n, policy, fault);
    else
        hipLaunchKernelGGL((k_sgd<T, false>), dim3(grid), dim3(256), 0, s, (const T *)w, (const T *)g, rate, (T *)out, n, policy, fault);
    return hipGetLastError();
}

hipError_t launch_sgd(hipStream_t s, int dtype, uint64_t n, const void *w, const void *g,
                      double rate, void *out, int policy, unsigned long long *fault)
{
    if (n == 0)
        return hipSuccess;
    return dtype == 0 ? sgd_t<float>(s, n, w, g, (float)rate, out, policy, fault)
                      : sgd_t<double>(s, n, w, g, rate, out, policy, fault);
}

template <typename T>
static hipError_t mse_t(hipStream_t s, uint64_t n, const void *p, const void *t, void *squares,
                        T count, void *out, int policy, unsigned long long *fault)
{
    constexpr int Wd = Vec<T>::width;
    bool vec = n % Wd == 0 && aligned16(p) && aligned16(t) && aligned16(squares);
    unsigned grid = grid_for(vec ? n / Wd : n);
    if (vec)
        hipLaunchKernelGGL((k_mse_squares<T, true>), dim3(grid), dim3(256), 0, s, (const T *)p, (const T *)t, (T *)squares, n, policy, fault);
    else
        hipLaunchKernelGGL((k_mse_squares<T, false>), dim3(grid), dim3(256), 0, s, (const T *)p, (const T *)t, (T *)squares, n, policy, fault);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    hipLaunchKernelGGL((k_mse_ordered_sum<T>), dim3(1), dim3(64), 0, s, (const T *)squares, n, count, policy, (T *)out, fault);
    return hipGetLastError();
}

hipError_t launch_mse(hipStream_t s, int dtype, uint64_t n, const void *p, const void *t,
                      void *squares, double count, void *out, int policy,
                      unsigned long long *fault)
{
    if (n == 0)
        return hipErrorInvalidValue;
    return dtype == 0 ? mse_t<float>(s, n, p, t, squares, (float)count, out, policy, fault)
                      : mse_t<double>(s, n, p, t, squares, count, out, policy, fault);
}

} // namespace pcu
