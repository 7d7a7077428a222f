// Bandwidth-bound strict kernels: checked Add/Sub/Mul/Div (tensor or uniform right
// operand), ReLU, ReLU-backward, fused Add->ReLU, strict SGD and strict MSE.
//
// Layout: dense row-major tensors in HBM. One thread moves one 16-byte vector per operand
// (4 floats or 2 doubles) and the grid covers the whole tensor in 256-thread blocks, with
// non-temporal loads and stores: on MI355X this streams at about 83% of the 8 TB/s HBM
// peak, ahead of every grid-stride shape tried (2^28 f32 SGD: 6.55-6.64 TB/s, against
// 6.32-6.52 with 128-thread blocks and 6.43 / 6.34 with 512 / 1024). The last vector may be partial (scalar
// accesses for its in-range elements). Faults are screened per lane, resolved exactly
// only on flagged lanes, and reduced with one ballot per wave and one atomicMin per
// faulting wave into the op's 64-bit fault word.
#include "pcu_device.hpp"
#include "pcu_kernels.hpp"

#include <limits.h>

#pragma clang fp contract(off)

namespace pcu {

constexpr int kEwThreads = 256;

template <typename T> struct Vec;
template <> struct Vec<float> {
    typedef float type __attribute__((ext_vector_type(4)));
    static constexpr int width = 4;
};
template <> struct Vec<double> {
    typedef double type __attribute__((ext_vector_type(2)));
    static constexpr int width = 2;
};

template <typename T, bool VEC> struct Lanes {
    static constexpr int W = VEC ? Vec<T>::width : 1;
};

// Elements [base, base + W) of p that lie below n (the rest read as +0 and must be masked
// by the caller). A whole vector is one non-temporal 16-byte load.
template <typename T, bool VEC>
__device__ __forceinline__ void load_lanes(const T *p, uint64_t base, uint64_t n,
                                           T (&v)[Lanes<T, VEC>::W])
{
    constexpr int W = Lanes<T, VEC>::W;
    if (VEC && base + W <= n) {
        typedef typename Vec<T>::type V;
        const V q = __builtin_nontemporal_load(reinterpret_cast<const V *>(p + base));
#pragma unroll
        for (int j = 0; j < W; j++)
            v[j] = q[j];
    } else {
#pragma unroll
        for (int j = 0; j < W; j++)
            v[j] = base + j < n ? __builtin_nontemporal_load(p + base + j) : (T)0;
    }
}

template <typename T, bool VEC, bool NT = true>
__device__ __forceinline__ void store_lanes(T *p, uint64_t base, uint64_t n,
                                            const T (&v)[Lanes<T, VEC>::W])
{
    constexpr int W = Lanes<T, VEC>::W;
    if (VEC && base + W <= n) {
        typedef typename Vec<T>::type V;
        V q;
#pragma unroll
        for (int j = 0; j < W; j++)
            q[j] = v[j];
        if (NT)
            __builtin_nontemporal_store(q, reinterpret_cast<V *>(p + base));
        else
            *reinterpret_cast<V *>(p + base) = q;
    } else {
#pragma unroll
        for (int j = 0; j < W; j++)
            if (base + j < n) {
                if (NT)
                    __builtin_nontemporal_store(v[j], p + base + j);
                else
                    p[base + j] = v[j];
            }
    }
}

// First element index of this thread's vector and the distance to its next one (the grid
// normally covers the tensor, so the loop body runs once).
#define PCU_EW_LOOP(W)                                                                          \
    const uint64_t pcu_stride = (uint64_t)gridDim.x * kEwThreads * (W);                         \
    for (uint64_t base = ((uint64_t)blockIdx.x * kEwThreads + threadIdx.x) * (W); base < n;     \
         base += pcu_stride)

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
// The checked elementwise and SGD kernels may run in place (out equal to an operand), so
// none of their pointers is __restrict__: a fault is classified from register values after
// the store, and the compiler may not reload an operand from memory the store overwrote.

template <typename T, int OP, bool UNIFORM, bool VEC>
__global__ __launch_bounds__(kEwThreads) void k_binary(const T *a,
                                                       const T *b, T b_value,
                                                       T *out, uint64_t n,
                                                       int policy, unsigned long long *fault, NodeGate gate)
{
    if (wave_gate_closed(gate))
        return;
    constexpr int W = Lanes<T, VEC>::W;
    uint64_t key = kNoFault;
    PCU_EW_LOOP(W)
    {
        T x[W], y[W], r[W];
        load_lanes<T, VEC>(a, base, n, x);
        if (UNIFORM) {
#pragma unroll
            for (int j = 0; j < W; j++)
                y[j] = b_value;
        } else {
            load_lanes<T, VEC>(b, base, n, y);
        }
        bool any = false;
#pragma unroll
        for (int j = 0; j < W; j++) {
            r[j] = apply<T, OP>(x[j], y[j]);
            any |= base + j < n && suspect<T, OP>(x[j], y[j], r[j], policy);
        }
        store_lanes<T, VEC>(out, base, n, r);
        if (any && key == kNoFault) {
#pragma unroll
            for (int j = 0; j < W; j++) {
                if (base + j >= n || key != kNoFault)
                    continue;
                const uint32_t kind = classify<T, OP>(x[j], y[j], r[j], policy);
                if (kind != kOk)
                    key = pack_fault(base + j, kind);
            }
        }
    }
    wave_record_fault(key, fault, gate);
}

// -------------------------------------------------------------------- relu

template <typename T, bool VEC>
__global__ __launch_bounds__(kEwThreads) void k_relu(const T *x, T *out,
                                                     uint64_t n, int policy,
                                                     unsigned long long *fault, NodeGate gate)
{
    if (wave_gate_closed(gate))
        return;
    constexpr int W = Lanes<T, VEC>::W;
    uint64_t key = kNoFault;
    PCU_EW_LOOP(W)
    {
        T v[W], r[W];
        load_lanes<T, VEC>(x, base, n, v);
        bool any = false;
#pragma unroll
        for (int j = 0; j < W; j++) {
            r[j] = relu_select(v[j]);
            any |= base + j < n &&
                   (!finite_bits(v[j]) || (policy == kPolicyRejectSubnormal && subnormal(r[j])));
        }
        store_lanes<T, VEC>(out, base, n, r);
        if (any && key == kNoFault) {
#pragma unroll
            for (int j = 0; j < W; j++) {
                if (base + j >= n || key != kNoFault)
                    continue;
                const uint32_t kind = classify_relu(v[j], r[j], policy);
                if (kind != kOk)
                    key = pack_fault(base + j, kind);
            }
        }
    }
    wave_record_fault(key, fault, gate);
}

// ---------------------------------------------------------- relu backward

template <typename T, bool VEC>
__global__ __launch_bounds__(kEwThreads) void k_relu_backward(const T *x,
                                                              const T *up,
                                                              T *out, uint64_t n,
                                                              int policy,
                                                              unsigned long long *fault, NodeGate gate)
{
    if (wave_gate_closed(gate))
        return;
    constexpr int W = Lanes<T, VEC>::W;
    uint64_t key = kNoFault;
    PCU_EW_LOOP(W)
    {
        T v[W], u[W], r[W];
        load_lanes<T, VEC>(x, base, n, v);
        load_lanes<T, VEC>(up, base, n, u);
        bool any = false;
#pragma unroll
        for (int j = 0; j < W; j++) {
            r[j] = strictly_positive(v[j]) ? u[j] : (T)0;
            any |= base + j < n && (!finite_bits(v[j]) || !finite_bits(u[j]) ||
                                    (policy == kPolicyRejectSubnormal && subnormal(r[j])));
        }
        store_lanes<T, VEC>(out, base, n, r);
        if (any && key == kNoFault) {
#pragma unroll
            for (int j = 0; j < W; j++) {
                if (base + j >= n || key != kNoFault)
                    continue;
                const uint32_t kind = classify_relu_backward(v[j], u[j], r[j], policy);
                if (kind != kOk)
                    key = pack_fault(base + j, kind);
            }
        }
    }
    wave_record_fault(key, fault, gate);
}

// ------------------------------------------------------------ fused add->relu
// The Add node's faults go to fault_add and the ReLU node's to fault_relu, so the
// node-major first-fault order is the same as running the two nodes one after the other
// (a ReLU of a successful, hence finite, sum can only fault under RejectSubnormal).

template <typename T, bool UNIFORM, bool VEC>
__global__ __launch_bounds__(kEwThreads) void k_add_relu(const T *a,
                                                         const T *b, T b_value,
                                                         T *out, uint64_t n,
                                                         int policy,
                                                         unsigned long long *fault_add,
                                                         unsigned long long *fault_relu, NodeGate gate)
{
    if (wave_gate_closed(gate))
        return;
    constexpr int W = Lanes<T, VEC>::W;
    uint64_t key_add = kNoFault, key_relu = kNoFault;
    PCU_EW_LOOP(W)
    {
        T x[W], y[W], sum[W], r[W];
        load_lanes<T, VEC>(a, base, n, x);
        if (UNIFORM) {
#pragma unroll
            for (int j = 0; j < W; j++)
                y[j] = b_value;
        } else {
            load_lanes<T, VEC>(b, base, n, y);
        }
        bool any = false;
#pragma unroll
        for (int j = 0; j < W; j++) {
            sum[j] = x[j] + y[j];
            r[j] = relu_select(sum[j]);
            any |= base + j < n && (add_suspect(x[j], y[j], sum[j], policy) ||
                                    (policy == kPolicyRejectSubnormal && subnormal(r[j])));
        }
        store_lanes<T, VEC>(out, base, n, r);
        if (any) {
#pragma unroll
            for (int j = 0; j < W; j++) {
                if (base + j >= n)
                    continue;
                const uint32_t ka = classify_add(x[j], y[j], sum[j], policy);
                if (ka != kOk) {
                    if (key_add == kNoFault)
                        key_add = pack_fault(base + j, ka);
                } else {
                    const uint32_t kr = classify_relu(sum[j], r[j], policy);
                    if (kr != kOk && key_relu == kNoFault)
                        key_relu = pack_fault(base + j, kr);
                }
            }
        }
    }
    wave_record_fault(key_add, fault_add, gate);
    wave_record_fault(key_relu, fault_relu, NodeGate{gate.word, gate.node + 1});
}

// ---------------------------------------------------------- fused chains
// Consecutive elementwise nodes of a prepared program, each an operand of the next, in one
// pass over the elements: the values between steps stay in registers, and only the values
// another node reads are stored. Each step's faults go to its own node's word and every
// step is classified as its own kernel classifies it, so the node-major first fault is the
// one the nodes give one after another (a step may also record a fault on a value a
// faulting earlier step produced: the earlier node's fault is the one reported).
template <typename T> __device__ __forceinline__ T chain_uniform(uint64_t bits)
{
    if constexpr (sizeof(T) == 4)
        return __builtin_bit_cast(float, (uint32_t)bits);
    else
        return __builtin_bit_cast(double, bits);
}

template <typename T> __device__ __forceinline__ T chain_binary(int op, T a, T b)
{
    switch (op) {
    case kOpAdd: return a + b;
    case kOpSub: return a - b;
    case kOpMul: return a * b;
    default: return a / b;
    }
}

template <typename T> __device__ __forceinline__ bool chain_suspect(int op, T a, T b, T r, int policy)
{
    if (op == kOpAdd || op == kOpSub) return add_suspect(a, b, r, policy);
    if (op == kOpMul) return mul_suspect(a, b, r, policy);
    return div_suspect(a, b, r, policy);
}

template <typename T> __device__ __forceinline__ uint32_t chain_classify(int op, T a, T b, T r, int policy)
{
    if (op == kOpAdd || op == kOpSub) return classify_add(a, b, r, policy);
    if (op == kOpMul) return classify_mul(a, b, r, policy);
    return classify_div(a, b, r, policy);
}

// A chain's step operations known when the kernel is compiled: op of step s in bits
// 4s..4s+3 of SIG, or SIG < 0 (read from the launch). The common chains get kernels of
// their own, with the other operations' code folded away.
constexpr int chain_sig_op(int sig, int s) { return sig < 0 ? -1 : (sig >> (4 * s)) & 15; }
constexpr int chain_sig(int op0, int op1, int op2 = -1, int op3 = -1)
{
    return op0 | op1 << 4 | (op2 < 0 ? 0 : op2 << 8) | (op3 < 0 ? 0 : op3 << 12);
}
constexpr int kSigSubMul = chain_sig(kOpSub, kOpMul);                          // MSE gradient
constexpr int kSigAddRelu = chain_sig(kOpAdd, kStepRelu);                       // bias + ReLU
constexpr int kSigSubMulReluBack = chain_sig(kOpSub, kOpMul, kStepReluBackward); // C1 backward

// The other operand of step S on the lanes [base, base + W) (nothing for a ReLU).
template <typename T, bool VEC, int S, int SIG>
__device__ __forceinline__ void chain_other(const ChainLaunch &c, uint64_t base, uint64_t n,
                                            T (&o)[Lanes<T, VEC>::W])
{
    constexpr int W = Lanes<T, VEC>::W;
    const ChainStep &st = c.step[S];
    constexpr int kop = chain_sig_op(SIG, S);
    const int op = kop >= 0 ? kop : st.op;
    if (S >= c.steps || op == kStepRelu)
        return;
    if (st.other) {
        load_lanes<T, VEC>((const T *)st.other, base, n, o);
    } else {
        const T u = chain_uniform<T>(st.other_bits);
#pragma unroll
        for (int j = 0; j < W; j++)
            o[j] = u;
    }
}

// The first fault of a chain step on the lanes [base, base + W) (kNoFault: none), the rare
// path once a lane is suspect. Out of line, so that the classifiers' code and registers stay
// out of the streaming loop (inlined into each step they spilled scalar registers into
// vector lanes).
template <typename T, int W> struct LaneVals {
    T x[W];
};
template <typename T, int W>
__device__ __forceinline__ uint64_t chain_first_fault_body(int op, int policy, bool right,
                                                           const LaneVals<T, W> &v,
                                                           const LaneVals<T, W> &o,
                                                           const LaneVals<T, W> &r, uint64_t base,
                                                           uint64_t n)
{
#pragma unroll
    for (int j = 0; j < W; j++) {
        if (base + j >= n)
            break;
        uint32_t kind;
        if (op == kStepRelu) {
            kind = classify_relu(v.x[j], r.x[j], policy);
        } else {
            const T a = right ? o.x[j] : v.x[j], b = right ? v.x[j] : o.x[j];
            kind = op == kStepReluBackward ? classify_relu_backward(a, b, r.x[j], policy)
                                           : chain_classify(op, a, b, r.x[j], policy);
        }
        if (kind != kOk)
            return pack_fault(base + j, kind);
    }
    return kNoFault;
}
// The call itself makes the kernel keep its scalar arguments in vector lanes across it, so
// the kernels with their operations fixed at compile time (small once folded) inline it.
template <typename T, int W>
__device__ __noinline__ uint64_t chain_first_fault(int op, int policy, bool right, LaneVals<T, W> v,
                                                   LaneVals<T, W> o, LaneVals<T, W> r,
                                                   uint64_t base, uint64_t n)
{
    return chain_first_fault_body<T, W>(op, policy, right, v, o, r, base, n);
}

// Step S of a chain on the lanes [base, base + W): v holds the value the step takes and is
// replaced by the step's result, o the step's other operand (chain_other); key keeps the
// step's first fault in this thread.
template <typename T, bool VEC, int S, int SIG>
__device__ __forceinline__ void chain_step(const ChainLaunch &c, uint64_t base, uint64_t n,
                                           T (&v)[Lanes<T, VEC>::W], const T (&o)[Lanes<T, VEC>::W],
                                           uint64_t &key)
{
    constexpr int W = Lanes<T, VEC>::W;
    const ChainStep &st = c.step[S];
    constexpr int kop = chain_sig_op(SIG, S);
    const int op = kop >= 0 ? kop : st.op, policy = st.policy;
    const bool right = st.chain_right != 0;
    T r[W];
    bool any = false;
    if (op == kStepRelu) {
#pragma unroll
        for (int j = 0; j < W; j++) {
            r[j] = relu_select(v[j]);
            any |= base + j < n && (!finite_bits(v[j]) || (policy == kPolicyRejectSubnormal && subnormal(r[j])));
        }
    } else if (op == kStepReluBackward) {
#pragma unroll
        for (int j = 0; j < W; j++) {
            const T x = right ? o[j] : v[j], u = right ? v[j] : o[j];
            r[j] = strictly_positive(x) ? u : (T)0;
            any |= base + j < n && (!finite_bits(x) || !finite_bits(u) ||
                                    (policy == kPolicyRejectSubnormal && subnormal(r[j])));
        }
    } else {
#pragma unroll
        for (int j = 0; j < W; j++) {
            const T a = right ? o[j] : v[j], b = right ? v[j] : o[j];
            r[j] = chain_binary(op, a, b);
            any |= base + j < n && chain_suspect(op, a, b, r[j], policy);
        }
    }
    if (st.out)
        store_lanes<T, VEC>((T *)st.out, base, n, r);
    if (any && key == kNoFault) {
        LaneVals<T, W> lv, lo, lr;
#pragma unroll
        for (int j = 0; j < W; j++) {
            lv.x[j] = v[j];
            lo.x[j] = o[j];
            lr.x[j] = r[j];
        }
        if constexpr (kop >= 0)
            key = chain_first_fault_body<T, W>(op, policy, right, lv, lo, lr, base, n);
        else
            key = chain_first_fault<T, W>(op, policy, right, lv, lo, lr, base, n);
    }
#pragma unroll
    for (int j = 0; j < W; j++)
        v[j] = r[j];
}

// NS = c.steps, a template argument: a kernel for all four steps held every step's
// parameters and registers at once and spilled scalar registers into vector lanes (about 750
// lane reads; a two-step chain ran at half the speed of one checked binary op over the
// same bytes).
template <typename T, bool VEC, int NS, int SIG = -1>
__global__ __launch_bounds__(kEwThreads) void k_chain(ChainLaunch c, uint64_t n, NodeGate gate)
{
    static_assert(NS >= 1 && NS <= kChainMaxSteps && kChainMaxSteps == 4,
                  "one chain_step call per step below");
    if (wave_gate_closed(gate))
        return;
    constexpr int W = Lanes<T, VEC>::W;
    uint64_t k0 = kNoFault, k1 = kNoFault, k2 = kNoFault, k3 = kNoFault;
    PCU_EW_LOOP(W)
    {
        // Every operand is loaded before any step stores: no step reads a value stored in
        // this launch (the plan keeps chain members out of other operands), so the loads go
        // out together, one round trip, instead of one after each step's stores.
        T v[W], o0[W], o1[W], o2[W], o3[W];
        load_lanes<T, VEC>((const T *)c.head, base, n, v);
        chain_other<T, VEC, 0, SIG>(c, base, n, o0);
        if constexpr (NS > 1)
            chain_other<T, VEC, 1, SIG>(c, base, n, o1);
        if constexpr (NS > 2)
            chain_other<T, VEC, 2, SIG>(c, base, n, o2);
        if constexpr (NS > 3)
            chain_other<T, VEC, 3, SIG>(c, base, n, o3);
        chain_step<T, VEC, 0, SIG>(c, base, n, v, o0, k0);
        if constexpr (NS > 1)
            chain_step<T, VEC, 1, SIG>(c, base, n, v, o1, k1);
        if constexpr (NS > 2)
            chain_step<T, VEC, 2, SIG>(c, base, n, v, o2, k2);
        if constexpr (NS > 3)
            chain_step<T, VEC, 3, SIG>(c, base, n, v, o3, k3);
    }
    wave_record_fault(k0, c.step[0].fault, gate);
    if constexpr (NS > 1)
        wave_record_fault(k1, c.step[1].fault, NodeGate{gate.word, gate.node + 1});
    if constexpr (NS > 2)
        wave_record_fault(k2, c.step[2].fault, NodeGate{gate.word, gate.node + 2});
    if constexpr (NS > 3)
        wave_record_fault(k3, c.step[3].fault, NodeGate{gate.word, gate.node + 3});
}

// -------------------------------------------------------------------- SGD
// core/dialect/tensor/reference/strict_sgd/strict_sgd.rs:20-46: p = rate (x) g, then
// w' = w (-) p; ordinal 2i (Multiply) and 2i+1 (Subtract).

// Blocks [bid, ...) of nb blocks over one update.
template <typename T, bool VEC>
__device__ __forceinline__ void sgd_range(const T *w, const T *g, T rate, T *out, uint64_t n,
                                          int policy, unsigned long long *fault, NodeGate gate,
                                          uint64_t bid, uint64_t nb)
{
    if (wave_gate_closed(gate))
        return;
    constexpr int W = Lanes<T, VEC>::W;
    uint64_t key = kNoFault;
    const uint64_t stride = nb * kEwThreads * W;
    for (uint64_t base = (bid * kEwThreads + threadIdx.x) * W; base < n; base += stride) {
        T wv[W], gv[W], p[W], r[W];
        load_lanes<T, VEC>(w, base, n, wv);
        load_lanes<T, VEC>(g, base, n, gv);
        bool any = false;
#pragma unroll
        for (int j = 0; j < W; j++) {
            p[j] = rate * gv[j];
            r[j] = wv[j] - p[j];
            any |= base + j < n && (mul_suspect(rate, gv[j], p[j], policy) |
                                    add_suspect(wv[j], p[j], r[j], policy));
        }
        store_lanes<T, VEC>(out, base, n, r);
        if (any && key == kNoFault) {
#pragma unroll
            for (int j = 0; j < W; j++) {
                if (base + j >= n || key != kNoFault)
                    continue;
                const uint32_t km = classify_mul(rate, gv[j], p[j], policy);
                if (km != kOk) {
                    key = pack_fault(2 * (base + j), km);
                } else {
                    const uint32_t ks = classify_add(wv[j], p[j], r[j], policy);
                    if (ks != kOk)
                        key = pack_fault(2 * (base + j) + 1, ks);
                }
            }
        }
    }
    wave_record_fault(key, fault, gate);
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kEwThreads) void k_sgd(const T *w,
                                                    const T *g, T rate,
                                                    T *out, uint64_t n, int policy,
                                                    unsigned long long *fault, NodeGate gate,
                                                    ProgramClose close)
{
    sgd_range<T, VEC>(w, g, rate, out, n, policy, fault, gate, blockIdx.x, gridDim.x);
    program_close_block(close);
}

// Two updates of one program in one launch: blocks [0, blocks0) take update 0, the rest
// update 1; each keeps its own fault word and gate.
template <typename T> struct SgdPairArgs {
    const T *w[2], *g[2];
    T *out[2];
    T rate[2];
    uint64_t n[2];
    unsigned long long *fault[2];
    NodeGate gate[2];
    unsigned blocks0;
};

template <typename T, bool VEC>
__global__ __launch_bounds__(kEwThreads) void k_sgd_pair(SgdPairArgs<T> a, int policy,
                                                         ProgramClose close)
{
    const bool first = blockIdx.x < a.blocks0;
    const int u = first ? 0 : 1;
    const uint64_t bid = first ? blockIdx.x : blockIdx.x - a.blocks0;
    const uint64_t nb = first ? a.blocks0 : gridDim.x - a.blocks0;
    sgd_range<T, VEC>(a.w[u], a.g[u], a.rate[u], a.out[u], a.n[u], policy, a.fault[u], a.gate[u],
                      bid, nb);
    program_close_block(close);
}

// -------------------------------------------------------------------- MSE
// core/dialect/tensor/reference/strict_mse/strict_mse.rs:22-59. Stage 1 (parallel):
// d = p (-) t and s = d (x) d per element, ordinals 3i and 3i+1. Stage 2 (one wave): the
// ordered sum total = total (+) s_i from +0 (ordinal 3i+2), then total (/) count
// (ordinal 3n). The sum is a dependent chain by contract; it stops before the first
// element whose Subtract or Multiply faulted.

template <typename T, bool VEC>
__global__ __launch_bounds__(kEwThreads) void k_mse_squares(const T *__restrict__ p,
                                                            const T *__restrict__ t,
                                                            T *__restrict__ sq, uint64_t n,
                                                            int policy,
                                                            unsigned long long *fault, NodeGate gate)
{
    if (wave_gate_closed(gate))
        return;
    constexpr int W = Lanes<T, VEC>::W;
    uint64_t key = kNoFault;
    PCU_EW_LOOP(W)
    {
        T pv[W], tv[W], d[W], sv[W];
        load_lanes<T, VEC>(p, base, n, pv);
        load_lanes<T, VEC>(t, base, n, tv);
        bool any = false;
#pragma unroll
        for (int j = 0; j < W; j++) {
            d[j] = pv[j] - tv[j];
            sv[j] = d[j] * d[j];
            any |= base + j < n && (add_suspect(pv[j], tv[j], d[j], policy) |
                                    mul_suspect(d[j], d[j], sv[j], policy));
        }
        // Ordinary stores: the ordered sum reads the squares next.
        store_lanes<T, VEC, false>(sq, base, n, sv);
        if (any && key == kNoFault) {
#pragma unroll
            for (int j = 0; j < W; j++) {
                if (base + j >= n || key != kNoFault)
                    continue;
                const uint32_t ks = classify_add(pv[j], tv[j], d[j], policy);
                if (ks != kOk) {
                    key = pack_fault(3 * (base + j), ks);
                } else {
                    const uint32_t km = classify_mul(d[j], d[j], sv[j], policy);
                    if (km != kOk)
                        key = pack_fault(3 * (base + j) + 1, km);
                }
            }
        }
    }
    wave_record_fault(key, fault, gate);
}

// Ordered sum of the squares, exact and parallel. Every square is +0 or positive, so the
// running total never decreases. While the total stays inside one binade [2^E, 2^(E+1))
// (or below the smallest normal), it is m * u for an integer m and the binade's quantum u,
// and one rounded step total (+) s equals (m + r) * u where r is s/u rounded to the nearest
// integer, a tie going to the r that makes m + r even. So inside a binade the chain is a
// prefix sum of integers whose only coupling is the parity of m at each tie: a two-state
// automaton, which composes associatively and scans in parallel. The first element whose
// step would reach the binade's upper end (or any element a screen cannot place) is
// executed as the real rounded hardware add, checked like every other Add, and starts the
// next phase. Results equal the dependent chain of the contract bit for bit.

template <typename T> struct SumBits;
template <> struct SumBits<float> {
    using U = uint32_t;
    using C = uint32_t;                  // step counts: a binade holds 2^24 quanta at most
    static constexpr int kFrac = 23;     // stored fraction bits
    static constexpr int kQmin = -149;   // exponent of the smallest subnormal
    static constexpr uint32_t kExpAll = 0xff;
    static constexpr int kPer = 16;      // elements per thread of a full-chunk scan
    static constexpr C kBig = 1u << 25;  // r of a step that surely leaves the binade
    static constexpr C kCap = 1u << 30;  // saturation of prefix counts (past any crossing)
};
template <> struct SumBits<double> {
    using U = uint64_t;
    using C = uint64_t;
    static constexpr int kFrac = 52;
    static constexpr int kQmin = -1074;
    static constexpr uint32_t kExpAll = 0x7ff;
    static constexpr int kPer = 8;
    static constexpr C kBig = 1ull << 54;
    static constexpr C kCap = 1ull << 62;
};

constexpr int kSumThreads = 512;

enum : uint32_t { kRBelow = 0, kRAbove = 1, kRTie = 2, kRForce = 3 };

template <typename T>
__device__ __forceinline__ typename SumBits<T>::C sat_add(typename SumBits<T>::C a,
                                                          typename SumBits<T>::C b)
{
    const typename SumBits<T>::C c = a + b; // a, b <= kCap: no wrap
    return c < SumBits<T>::kCap ? c : SumBits<T>::kCap;
}

// Step r of one square s (bits) on the quantum 2^ue, before the tie decision.
template <typename T>
__device__ __forceinline__ void sum_elem(typename SumBits<T>::U b, int ue,
                                         typename SumBits<T>::C &n, uint32_t &cls)
{
    using B = SumBits<T>;
    using U = typename B::U;
    using C = typename B::C;
    const uint32_t e = (uint32_t)(b >> B::kFrac) & B::kExpAll;
    const C f = (C)(b & (((U)1 << B::kFrac) - 1));
    if ((b >> (sizeof(U) * 8 - 1)) || e == B::kExpAll) { // negative or non-finite
        n = B::kBig;
        cls = kRForce;
        return;
    }
    const C sig = e ? (f | ((C)1 << B::kFrac)) : f;
    const int q = e ? (int)e + B::kQmin - 1 : B::kQmin;
    cls = kRBelow;
    if (sig == 0) {
        n = 0;
        return;
    }
    const int sh = q - ue;
    if (sh >= 0) {
        // sh > 0 only for normal squares (sig >= 2^kFrac): from sh = 2 on, r >= kBig.
        n = sh >= 2 ? B::kBig : (sig << sh);
        return;
    }
    const int k = -sh;
    if (k > B::kFrac + 1) { // sig < 2^(kFrac+1) <= half a quantum: rounds to 0
        n = 0;
        return;
    }
    n = sig >> k;
    const C rem = sig & (((C)1 << k) - 1), half = (C)1 << (k - 1);
    cls = rem < half ? kRBelow : (rem > half ? kRAbove : kRTie);
}

template <typename C>
__device__ __forceinline__ C sum_step(C n, uint32_t cls, uint32_t parity)
{
    return n + (C)(cls == kRAbove) + (C)(cls == kRTie && ((parity ^ (uint32_t)n) & 1u));
}

// Effect of a run of steps as a function of the parity of m before it: the added count
// and the parity after it, for each starting parity (bit 0: start even, bit 1: start odd).
template <typename C> struct SumScanT {
    C r0, r1;
    uint32_t p;
};
template <typename T> using SumScan = SumScanT<typename SumBits<T>::C>;

template <typename T> __device__ __forceinline__ SumScan<T> scan_identity() { return SumScan<T>{0, 0, 2u}; }

template <typename T>
__device__ __forceinline__ SumScan<T> scan_compose(const SumScan<T> &a, const SumScan<T> &b)
{
    const uint32_t a0 = a.p & 1u, a1 = (a.p >> 1) & 1u;
    const uint32_t b0 = b.p & 1u, b1 = (b.p >> 1) & 1u;
    SumScan<T> c;
    c.r0 = sat_add<T>(a.r0, a0 ? b.r1 : b.r0);
    c.r1 = sat_add<T>(a.r1, a1 ? b.r1 : b.r0);
    c.p = (a0 ? b1 : b0) | ((a1 ? b1 : b0) << 1);
    return c;
}

template <typename T>
__device__ __forceinline__ SumScan<T> scan_elem(typename SumBits<T>::C n, uint32_t cls)
{
    using C = typename SumBits<T>::C;
    const C r0 = sum_step<C>(n, cls, 0), r1 = sum_step<C>(n, cls, 1);
    return SumScan<T>{r0, r1, (uint32_t)(r0 & 1u) | ((uint32_t)((r1 + 1) & 1u) << 1)};
}

// Cross-lane moves of a summary. DPP (a register read across lanes, no LDS): a lane
// whose source lies outside the pattern, or whose row the row mask leaves out, keeps old.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_c(uint32_t old, uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROW_MASK, 0xf, false);
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_c(uint64_t old, uint64_t v)
{
    const uint32_t lo = dpp_c<CTRL, ROW_MASK>((uint32_t)old, (uint32_t)v);
    const uint32_t hi = dpp_c<CTRL, ROW_MASK>((uint32_t)(old >> 32), (uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

template <typename T, int CTRL, int ROW_MASK>
__device__ __forceinline__ SumScan<T> scan_dpp(const SumScan<T> &v)
{
    const SumScan<T> id = scan_identity<T>();
    return SumScan<T>{dpp_c<CTRL, ROW_MASK>(id.r0, v.r0), dpp_c<CTRL, ROW_MASK>(id.r1, v.r1),
                      dpp_c<CTRL, ROW_MASK>(id.p, v.p)};
}

__device__ __forceinline__ uint32_t readlane_c(uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); }
__device__ __forceinline__ uint64_t readlane_c(uint64_t v, int l)
{
    return ((uint64_t)readlane_c((uint32_t)(v >> 32), l) << 32) | readlane_c((uint32_t)v, l);
}

template <typename T>
__device__ __forceinline__ SumScan<T> scan_readlane(const SumScan<T> &v, int l)
{
    return SumScan<T>{readlane_c(v.r0, l), readlane_c(v.r1, l), readlane_c(v.p, l)};
}

template <typename T>
__device__ __forceinline__ SumScan<T> scan_shfl_up(const SumScan<T> &v, int d)
{
    return SumScan<T>{__shfl_up(v.r0, d, 64), __shfl_up(v.r1, d, 64), __shfl_up(v.p, d, 64)};
}

// DPP patterns of the wave scan: row_shr:1,2,4,8 inside each row of 16 lanes, then
// row_bcast:15 (lane 15 of rows 0 and 2 into rows 1 and 3) and row_bcast:31 (lane 31 into
// rows 2 and 3).
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;

// Inclusive ordered composition over the 64 lanes of a wave.
template <typename T>
__device__ __forceinline__ SumScan<T> wave_scan_incl(SumScan<T> v)
{
    v = scan_compose<T>(scan_dpp<T, kDppRowShr1, 0xf>(v), v);
    v = scan_compose<T>(scan_dpp<T, kDppRowShr2, 0xf>(v), v);
    v = scan_compose<T>(scan_dpp<T, kDppRowShr4, 0xf>(v), v);
    v = scan_compose<T>(scan_dpp<T, kDppRowShr8, 0xf>(v), v);
    v = scan_compose<T>(scan_dpp<T, kDppRowBcast15, 0xa>(v), v);
    v = scan_compose<T>(scan_dpp<T, kDppRowBcast31, 0xc>(v), v);
    return v;
}

// Phase of a total given by its bits: quantum exponent, count m and the count at which
// the next binade starts.
template <typename T>
__device__ __forceinline__ void sum_phase(typename SumBits<T>::U bits, int &ue,
                                          typename SumBits<T>::C &m, typename SumBits<T>::C &mmax)
{
    using B = SumBits<T>;
    using C = typename B::C;
    const uint32_t e = (uint32_t)(bits >> B::kFrac) & B::kExpAll;
    if (e == 0) {
        ue = B::kQmin;
        m = (C)bits;
        mmax = (C)1 << B::kFrac;
    } else {
        ue = (int)e + B::kQmin - 1;
        m = ((C)bits & (((C)1 << B::kFrac) - 1)) | ((C)1 << B::kFrac);
        mmax = (C)1 << (B::kFrac + 1);
    }
}

template <typename T>
__device__ __forceinline__ typename SumBits<T>::U sum_bits(int ue, typename SumBits<T>::C m)
{
    using B = SumBits<T>;
    using U = typename B::U;
    if (ue == B::kQmin && m < ((typename B::C)1 << B::kFrac))
        return (U)m;
    return (U)(((U)(ue - B::kQmin) << B::kFrac) + (U)m);
}

template <typename T>
__device__ __forceinline__ T from_bits(typename SumBits<T>::U b);
template <>
__device__ __forceinline__ float from_bits<float>(uint32_t b) { return __uint_as_float(b); }
template <>
__device__ __forceinline__ double from_bits<double>(uint64_t b) { return __longlong_as_double((long long)b); }

// ----------------------------------------------------- ordered sum: pipeline
// The squares are cut into chunks of 512*P elements (P = 16 for binary32, 8 for binary64).
//  A  k_mse_chunk_sums       per-chunk sum in binary64 (an estimate: order does not matter);
//  B  k_mse_chunk_prefix     the exclusive prefix of those sums: about where the running
//                            total stands at each chunk start;
//  C  k_mse_chunk_summaries  per chunk, in parallel, the summary (count added for an even
//                            and an odd start) of the whole chunk inside one binade, for
//                            the one or two binades the estimate allows;
//  D  k_mse_ordered_walk     one workgroup walks the chunks in order, 512 at a time: a scan
//                            of the summaries made for the running binade folds every chunk
//                            before the first one that has no such summary or reaches the
//                            binade's end. That chunk runs exactly: where crossings are
//                            dense, one wave scans 64 squares at a time; elsewhere the
//                            workgroup scans windows sized from the chunk's estimate. In
//                            both, the first step to reach the binade's end runs as a real,
//                            checked Add.
// The estimate only decides how fast the walk goes, never its value.

struct ChunkSummary {
    uint64_t r0, r1;   // count added starting from an even / odd count
    int32_t ue;        // quantum exponent the summary was made for (kNoPhase: none)
    uint32_t pad;
};
constexpr int32_t kNoPhase = INT32_MIN;
constexpr uint32_t kNoStep = 0xffffffffu;

template <typename T> __device__ __forceinline__ uint64_t sum_chunk_len() { return (uint64_t)kSumThreads * SumBits<T>::kPer; }

__device__ __forceinline__ uint64_t sum_limit(const unsigned long long *fault, uint64_t n)
{
    // Elements at or after the first Subtract/Multiply fault are never summed.
    const uint64_t w = __atomic_load_n(fault, __ATOMIC_RELAXED);
    return w == kNoFault ? n : (w >> 3) / 3;
}

// Quantum exponent of the binade a total of about x lies in.
template <typename T>
__device__ __forceinline__ int32_t phase_ue_of(double x)
{
    using B = SumBits<T>;
    const double min_normal = ldexp(1.0, B::kQmin + B::kFrac);
    if (!(x >= min_normal))
        return B::kQmin;
    int e;
    (void)frexp(x, &e); // x = f * 2^e, f in [1/2, 1): floor(log2 x) = e - 1
    return e - 1 - B::kFrac;
}

// Thread t's P elements of the chunk at base (elements at or past limit read as 0).
template <typename T>
__device__ __forceinline__ void load_chunk(const typename SumBits<T>::U *__restrict__ src,
                                           bool vec_ok, uint64_t base, uint64_t limit, int tid,
                                           typename SumBits<T>::U (&dst)[SumBits<T>::kPer])
{
    using U = typename SumBits<T>::U;
    constexpr int P = SumBits<T>::kPer;
    const uint64_t first = base + (uint64_t)tid * P;
    if (vec_ok && base + sum_chunk_len<T>() <= limit) {
        const uint4 *v = reinterpret_cast<const uint4 *>(src + first);
        constexpr int per16 = 16 / sizeof(U);
#pragma unroll
        for (int q = 0; q < P / per16; q++) {
            const uint4 x = v[q];
            const U *xs = reinterpret_cast<const U *>(&x);
#pragma unroll
            for (int j = 0; j < per16; j++)
                dst[q * per16 + j] = xs[j];
        }
    } else {
#pragma unroll
        for (int j = 0; j < P; j++)
            dst[j] = first + j < limit ? src[first + j] : (U)0;
    }
}

// Ordered composition over the workgroup: every thread gets the summary of all threads
// before it (excl) and of the whole workgroup (total).
template <typename T>
__device__ __forceinline__ void block_scan(const SumScan<T> &mine, int lane, int wave,
                                           SumScan<T> *wave_tot, SumScan<T> &excl,
                                           SumScan<T> &total)
{
    constexpr int kWaves = kSumThreads / 64;
    static_assert(kWaves <= 8, "the wave totals are scanned inside one DPP row");
    const SumScan<T> inc = wave_scan_incl<T>(mine);
    SumScan<T> lane_excl = scan_shfl_up<T>(inc, 1);
    if (lane == 0)
        lane_excl = scan_identity<T>();
    if (lane == 63)
        wave_tot[wave] = inc;
    __syncthreads();
    // Every wave scans the per-wave totals on the first lanes of its first row.
    SumScan<T> wt = lane < kWaves ? wave_tot[lane] : scan_identity<T>();
    wt = scan_compose<T>(scan_dpp<T, kDppRowShr1, 0xf>(wt), wt);
    wt = scan_compose<T>(scan_dpp<T, kDppRowShr2, 0xf>(wt), wt);
    wt = scan_compose<T>(scan_dpp<T, kDppRowShr4, 0xf>(wt), wt);
    total = scan_readlane<T>(wt, kWaves - 1);
    SumScan<T> before = scan_readlane<T>(wt, wave > 0 ? wave - 1 : 0);
    if (wave == 0)
        before = scan_identity<T>();
    excl = scan_compose<T>(before, lane_excl);
}

// A chunk staged in LDS for its exact run: element i sits at slot i + i / kPadEvery (one
// spare slot per 128 bytes), so that runs of 2..16 consecutive elements per thread spread
// over distinct banks.
template <typename T> struct ChunkLds {
    using U = typename SumBits<T>::U;
    static constexpr uint32_t kPadEvery = 128 / sizeof(U);
    static constexpr uint32_t kLen = kSumThreads * SumBits<T>::kPer;
    static constexpr uint32_t kSlots = kLen + kLen / kPadEvery;
    __device__ static __forceinline__ uint32_t slot(uint32_t i) { return i + i / kPadEvery; }
};

// Shared state of the ordered walk. The step slots are double-buffered by iteration: one
// is written during an iteration while the other is cleared for the next.
template <typename T> struct WalkShared {
    typename SumBits<T>::U vals[ChunkLds<T>::kSlots];
    SumScan<T> wave_tot[kSumThreads / 64];
    uint64_t m_first[2];             // count standing before the stopping chunk
    uint32_t first[2];               // stopping chunk of a batch (offset), kNoStep: none
    uint32_t at[2];                  // crossing element of a window, or the element after a
                                     // wave walk (offset); kNoStep: no crossing
    typename SumBits<T>::U total[2]; // total after the crossing Add or the wave walk
    int stop[2];                     // an Add faulted
    int first_cand[2];               // candidate summary the stopping chunk matched, or -1
    // Result of a chunk's run-prefix fold (written by the one thread holding the crossing).
    uint64_t run_m;
    int run_status, run_ue;
    uint32_t run_resume;
    uint64_t limit;
};

// Summary of elements [i0, min(i0 + PER, i1)) of the staged chunk on the quantum 2^ue.
template <typename T, int PER>
__device__ __forceinline__ SumScan<T> run_scan(const typename SumBits<T>::U *vals, uint32_t i0,
                                               uint32_t i1, int ue)
{
    SumScan<T> s = scan_identity<T>();
#pragma unroll
    for (int j = 0; j < PER; j++) {
        if (i0 + j < i1) {
            typename SumBits<T>::C nn;
            uint32_t cls;
            sum_elem<T>(vals[ChunkLds<T>::slot(i0 + j)], ue, nn, cls);
            s = scan_compose<T>(s, scan_elem<T>(nn, cls));
        }
    }
    return s;
}

template <typename T>
__device__ __forceinline__ SumScan<T> run_scan_per(const typename SumBits<T>::U *vals,
                                                   uint32_t per, uint32_t i0, uint32_t i1, int ue)
{
    constexpr int P = SumBits<T>::kPer;
    if (per == 1)
        return run_scan<T, 1>(vals, i0, i1, ue);
    if (per == 2)
        return run_scan<T, 2>(vals, i0, i1, ue);
    if (per == 4)
        return run_scan<T, 4>(vals, i0, i1, ue);
    if (P > 8 && per == 8)
        return run_scan<T, 8>(vals, i0, i1, ue);
    return run_scan<T, P>(vals, i0, i1, ue);
}

// Expected number of squares (at the chunk's mean square) until the running total leaves
// its binade: room quanta of 2^ue left.
__device__ __forceinline__ double expected_gap(double room, int ue, double mean)
{
    return mean > 0.0 ? ldexp(room, ue) / mean : INFINITY;
}

// Elements per thread of the next window: a power of two covering about twice the expected
// gap, from one element per thread up to the whole chunk.
template <typename T>
__device__ __forceinline__ uint32_t window_per(double gap)
{
    constexpr uint32_t P = SumBits<T>::kPer;
    const double span = 2.0 * gap / kSumThreads;
    uint32_t per = 1;
    while (per < P && (double)per < span)
        per <<= 1;
    return per;
}

// Below this expected gap (in squares) one wave walks, 64 squares per scan: a crossing
// then costs one wave scan instead of a workgroup scan of a window. A wave walk stops at
// the first binade whose expected gap reaches kWaveGap, or after kWaveMax squares (then a
// window runs next, whatever the estimate says).
constexpr double kWaveGap = 1024.0;
constexpr uint32_t kWaveMax = 4096;

// The wave walk (wave 0 alone; every value it keeps is uniform over the wave): lane l
// holds square off + l, a wave scan gives each lane the count before it, and the first
// lane whose step reaches the binade's end executes that step as the contract's Add.
// Returns false when that Add faulted (recorded).
template <typename T>
__device__ bool wave_walk(const typename SumBits<T>::U *vals, uint64_t base, uint32_t len,
                          double mean, int policy, unsigned long long *fault,
                          const NodeGate &gate, int lane, uint32_t &off, int &ue,
                          typename SumBits<T>::C &m, typename SumBits<T>::C &mmax)
{
    using U = typename SumBits<T>::U;
    using C = typename SumBits<T>::C;
    const uint32_t end = off + kWaveMax < len ? off + kWaveMax : len;
    while (off < end) {
        const uint32_t i = off + (uint32_t)lane;
        const bool in = i < end;
        U b = 0;
        C nn = 0;
        uint32_t cls = kRBelow;
        if (in) {
            b = vals[ChunkLds<T>::slot(i)];
            sum_elem<T>(b, ue, nn, cls);
        }
        const SumScan<T> inc = wave_scan_incl<T>(in ? scan_elem<T>(nn, cls) : scan_identity<T>());
        SumScan<T> ex = scan_shfl_up<T>(inc, 1);
        if (lane == 0)
            ex = scan_identity<T>();
        const uint32_t p0 = (uint32_t)(m & 1u);
        const C mt = sat_add<T>(m, p0 ? ex.r1 : ex.r0);
        const uint32_t pt = p0 ? (ex.p >> 1) & 1u : ex.p & 1u;
        const C r = sum_step<C>(nn, cls, pt);
        // Counts only grow along the lanes: at most one lane starts below the binade's end
        // and reaches it.
        const bool cross = in && mt < mmax && (cls == kRForce || mt + r >= mmax);
        const uint64_t mask = __ballot(cross);
        if (mask == 0) {
            const SumScan<T> tot = scan_readlane<T>(inc, 63);
            m = sat_add<T>(m, p0 ? tot.r1 : tot.r0);
            off = off + 64 < end ? off + 64 : end;
            continue;
        }
        const int c = __builtin_ctzll(mask);
        U res_bits = 0;
        uint32_t kind = kOk;
        if (lane == c) {
            const T acc = from_bits<T>(sum_bits<T>(ue, mt));
            const T s_i = from_bits<T>(b);
            const T res = acc + s_i;
            kind = classify_add(acc, s_i, res, policy);
            res_bits = (U)bits_of(res);
            if (kind != kOk) {
                atomicMin(fault, (unsigned long long)pack_fault(3 * (base + i) + 2, kind));
                gate_record(gate);
            }
        }
        if (readlane_c(kind, c) != kOk)
            return false;
        sum_phase<T>(readlane_c(res_bits, c), ue, m, mmax);
        off += (uint32_t)c + 1;
        if (expected_gap((double)(mmax - m), ue, mean) >= kWaveGap)
            break;
    }
    return true;
}

// Exact fold of elements [start, len) of the chunk at base from the phase (ue, m, mmax): by
// the wave walk where crossings are dense, elsewhere window by window, where the one thread
// whose run holds the window's first step to reach the binade's end executes that step as
// the contract's Add and the next window starts after it in the new binade. Returns false
// when an Add faulted (recorded).
template <typename T>
__device__ bool exact_chunk(const typename SumBits<T>::U *__restrict__ src, uint64_t base,
                            uint32_t len, uint32_t start, double mean, int policy,
                            unsigned long long *fault, int &ue, typename SumBits<T>::C &m,
                            typename SumBits<T>::C &mmax, WalkShared<T> &sh, const NodeGate &gate)
{
    using U = typename SumBits<T>::U;
    using C = typename SumBits<T>::C;
    constexpr uint32_t P = SumBits<T>::kPer;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (uint32_t i = tid; i < len; i += kSumThreads)
        sh.vals[ChunkLds<T>::slot(i)] = src[base + i];
    if (tid == 0)
        sh.at[0] = sh.at[1] = kNoStep;
    __syncthreads();
    uint32_t off = start, per = 0; // per = 0: no window has run yet
    bool wave_ok = true;
    for (int it = 0; off < len; it++) {
        const int slot = it & 1;
        const double gap = expected_gap((double)(mmax - m), ue, mean);
        if (wave_ok && gap < kWaveGap) {
            if (wave == 0) {
                uint32_t o = off;
                int u = ue;
                C mm = m, mx = mmax;
                const bool ok = wave_walk<T>(sh.vals, base, len, mean, policy, fault, gate, lane,
                                             o, u, mm, mx);
                if (lane == 0) {
                    sh.stop[slot] = !ok;
                    sh.total[slot] = sum_bits<T>(u, mm);
                    sh.at[slot] = o;
                }
            }
            __syncthreads();
            const uint32_t next = sh.at[slot];
            const int stop = sh.stop[slot];
            const U tot = sh.total[slot];
            if (tid == 0)
                sh.at[slot ^ 1] = kNoStep;
            if (stop)
                return false;
            sum_phase<T>(tot, ue, m, mmax);
            wave_ok = next - off < kWaveMax;
            off = next;
            per = 0;
            continue;
        }
        // After a window without a crossing the next one is at least twice as long.
        const uint32_t want = window_per<T>(gap);
        per = per && 2 * per > want ? (2 * per < P ? 2 * per : P) : want;
        const uint32_t wend = off + per * kSumThreads < len ? off + per * kSumThreads : len;
        const uint32_t i0 = off + (uint32_t)tid * per;
        const uint32_t i1 = i0 + per < wend ? i0 + per : wend;
        const SumScan<T> mine = run_scan_per<T>(sh.vals, per, i0, i1, ue);
        SumScan<T> before, total;
        block_scan<T>(mine, lane, wave, sh.wave_tot, before, total);
        const uint32_t p0 = (uint32_t)(m & 1u);
        const C mt = sat_add<T>(m, p0 ? before.r1 : before.r0);
        const uint32_t pt = p0 ? (before.p >> 1) & 1u : before.p & 1u;
        // Counts only grow along the window, so exactly one run can start below the
        // binade's end and reach it.
        if (mt < mmax && sat_add<T>(mt, pt ? mine.r1 : mine.r0) >= mmax) {
            C mm = mt;
            uint32_t pp = pt;
            for (uint32_t i = i0; i < i1; i++) {
                const U b = sh.vals[ChunkLds<T>::slot(i)];
                C nn;
                uint32_t cls;
                sum_elem<T>(b, ue, nn, cls);
                const C r = sum_step<C>(nn, cls, pp);
                if (cls == kRForce || mm + r >= mmax) {
                    // The crossing step, executed and checked as the contract's Add.
                    const T acc = from_bits<T>(sum_bits<T>(ue, mm));
                    const T s_i = from_bits<T>(b);
                    const T res = acc + s_i;
                    const uint32_t kind = classify_add(acc, s_i, res, policy);
                    if (kind != kOk) {
                        atomicMin(fault, (unsigned long long)pack_fault(3 * (base + i) + 2, kind));
                        gate_record(gate);
                        sh.stop[slot] = 1;
                    } else {
                        sh.stop[slot] = 0;
                        sh.total[slot] = (U)bits_of(res);
                    }
                    sh.at[slot] = i;
                    break;
                }
                mm += r;
                pp = (pp + (uint32_t)r) & 1u;
            }
        }
        __syncthreads();
        const uint32_t at = sh.at[slot];
        const int stop = sh.stop[slot];
        const U tot = sh.total[slot];
        if (tid == 0)
            sh.at[slot ^ 1] = kNoStep;
        if (at == kNoStep) {
            m = sat_add<T>(m, p0 ? total.r1 : total.r0);
            off = wend;
            continue;
        }
        if (stop)
            return false;
        sum_phase<T>(tot, ue, m, mmax);
        off = at + 1;
        per = 0;
        wave_ok = true;
    }
    return true;
}

// Summaries kept per chunk: the estimate's binade less and plus 1/512 of it (lo, hi) and,
// when the estimate says the chunk crosses a binade, the binade after hi (where the rest
// of the chunk lands after one crossing).
constexpr int kCands = 3;

template <typename T>
__device__ __forceinline__ SumScan<T> scan_of_summary(const ChunkSummary &c)
{
    using C = typename SumBits<T>::C;
    const C r0 = (C)c.r0, r1 = (C)c.r1;
    return SumScan<T>{r0, r1, (uint32_t)(r0 & 1u) | ((uint32_t)((r1 + 1) & 1u) << 1)};
}

// Run-prefix fold of the chunk at base whose summary `cand` (made for the running binade)
// reaches the binade's end. runs_c holds, per candidate, each thread run's exclusive prefix
// (run t = elements [P*t, P*t + P)). The run where the count reaches the end is the one
// whose prefixes straddle it; its thread walks the run with the automaton, executes the
// crossing step as the contract's Add, and walks the rest of the run in the new binade.
// The runs after it fold at once from the prefixes of a candidate made for the new binade:
// from parity q at the chunk start a candidate's prefix adds E(q) before run t and T(q) over
// the whole chunk, so the runs from t on add T(q) - E(q), for the q whose parity after E is
// the parity actually standing there. Returns 1 when the chunk is folded, 0 when the Add
// faulted (recorded), -1 when a second crossing (or a missing candidate) leaves elements
// [*resume, len) to the windowed path, with (ue, m, mmax) standing before element *resume.
template <typename T>
__device__ int run_prefix_chunk(const typename SumBits<T>::U *__restrict__ src,
                                const SumScan<T> *__restrict__ runs_c,
                                const ChunkSummary *__restrict__ summ_c, int cand, uint64_t base,
                                uint32_t len, int policy, unsigned long long *fault, int &ue,
                                typename SumBits<T>::C &m, typename SumBits<T>::C &mmax,
                                uint32_t &resume, WalkShared<T> &sh, const NodeGate &gate)
{
    using U = typename SumBits<T>::U;
    using C = typename SumBits<T>::C;
    constexpr uint32_t P = SumBits<T>::kPer;
    const int tid = threadIdx.x;
    const SumScan<T> *ry = runs_c + (size_t)cand * kSumThreads;
    const SumScan<T> E = ry[tid];
    const SumScan<T> E1 = tid + 1 < kSumThreads ? ry[tid + 1] : scan_of_summary<T>(summ_c[cand]);
    const uint32_t p0 = (uint32_t)(m & 1u);
    const C mt = sat_add<T>(m, p0 ? E.r1 : E.r0), mt1 = sat_add<T>(m, p0 ? E1.r1 : E1.r0);
    // Counts only grow along the chunk: exactly one run starts below the end and reaches it.
    if (mt < mmax && mt1 >= mmax) {
        uint32_t pt = p0 ? (E.p >> 1) & 1u : E.p & 1u;
        C mm = mt, mx = mmax;
        int u = ue, status = 1;
        bool crossed = false;
        const uint32_t i0 = (uint32_t)tid * P, i1 = i0 + P < len ? i0 + P : len;
        uint32_t at = i1;
        for (uint32_t i = i0; i < i1; i++) {
            const U b = src[base + i];
            C nn;
            uint32_t cls;
            sum_elem<T>(b, u, nn, cls);
            const C r = sum_step<C>(nn, cls, pt);
            if (cls == kRForce || mm + r >= mx) {
                if (crossed) { // a second crossing inside the run
                    status = -1;
                    at = i;
                    break;
                }
                const T acc = from_bits<T>(sum_bits<T>(u, mm));
                const T s_i = from_bits<T>(b);
                const T res = acc + s_i;
                const uint32_t kind = classify_add(acc, s_i, res, policy);
                if (kind != kOk) {
                    atomicMin(fault, (unsigned long long)pack_fault(3 * (base + i) + 2, kind));
                    gate_record(gate);
                    status = 0;
                    break;
                }
                sum_phase<T>((U)bits_of(res), u, mm, mx);
                pt = (uint32_t)(mm & 1u);
                crossed = true;
                continue;
            }
            mm += r;
            pt = (pt + (uint32_t)r) & 1u;
        }
        if (status == 1 && i1 < len) {
            // The runs after this one, from the prefixes of a candidate for the new binade.
            status = -1;
            for (int y = 0; y < kCands; y++) {
                if (summ_c[y].ue != u)
                    continue;
                const SumScan<T> Ey = runs_c[(size_t)y * kSumThreads + tid + 1];
                const SumScan<T> Ty = scan_of_summary<T>(summ_c[y]);
                const int q = (Ey.p & 1u) == pt ? 0 : (((Ey.p >> 1) & 1u) == pt ? 1 : -1);
                if (q < 0)
                    break;
                const C tq = q ? Ty.r1 : Ty.r0, eq = q ? Ey.r1 : Ey.r0;
                if (tq < SumBits<T>::kCap && mm + (tq - eq) < mx) {
                    mm += tq - eq;
                    status = 1;
                }
                break;
            }
        }
        sh.run_status = status;
        sh.run_ue = u;
        sh.run_m = (uint64_t)mm;
        sh.run_resume = at;
    }
    __syncthreads();
    const int status = sh.run_status;
    if (status == 0)
        return 0;
    sum_phase<T>(sum_bits<T>(sh.run_ue, (C)sh.run_m), ue, m, mmax);
    resume = sh.run_resume;
    return status;
}

// A: chunk sums in binary64 (order inside a chunk does not matter: only an estimate).
template <typename T>
__global__ __launch_bounds__(256) void k_mse_chunk_sums(const T *__restrict__ sq, uint64_t n,
                                                        const unsigned long long *fault,
                                                        double *__restrict__ chunk_sum, NodeGate gate)
{
    if (block_gate_closed(gate))
        return;
    __shared__ double part[4];
    const uint64_t limit = sum_limit(fault, n);
    const uint64_t base = (uint64_t)blockIdx.x * sum_chunk_len<T>();
    const uint64_t end = base + sum_chunk_len<T>() < limit ? base + sum_chunk_len<T>() : limit;
    double acc = 0.0;
    for (uint64_t i = base + threadIdx.x; i < end; i += 256)
        acc += (double)sq[i];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        acc += __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0)
        part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0)
        chunk_sum[blockIdx.x] = (part[0] + part[1]) + (part[2] + part[3]);
}

// B: exclusive prefix of the chunk sums (one workgroup; each thread a contiguous run).
constexpr int kPrefixThreads = 1024;
__global__ __launch_bounds__(kPrefixThreads) void k_mse_chunk_prefix(const double *__restrict__ chunk_sum,
                                                                     uint64_t chunks,
                                                                     double *__restrict__ pre,
                                                                     NodeGate gate)
{
    if (block_gate_closed(gate))
        return;
    __shared__ double wave_sum[kPrefixThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t per = (chunks + kPrefixThreads - 1) / kPrefixThreads;
    const uint64_t i0 = (uint64_t)tid * per;
    const uint64_t i1 = i0 + per < chunks ? i0 + per : chunks;
    double own = 0.0;
    for (uint64_t i = i0; i < i1; i++)
        own += chunk_sum[i];
    double inc = own;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const double o = __shfl_up(inc, d, 64);
        if (lane >= d)
            inc += o;
    }
    if (lane == 63)
        wave_sum[wave] = inc;
    __syncthreads();
    double run = inc - own;
    for (int w = 0; w < wave; w++)
        run += wave_sum[w];
    for (uint64_t i = i0; i < i1; i++) {
        pre[i] = run;
        run += chunk_sum[i];
    }
}

// C: summary of chunk blockIdx.x for candidate blockIdx.y (0: the binade of the estimate
// less 1/512 of it; 1: plus 1/512, skipped when both agree; 2: the binade after candidate 1,
// only when the estimate says the chunk crosses), with every thread run's exclusive prefix.
template <typename T>
__global__ __launch_bounds__(kSumThreads) void k_mse_chunk_summaries(
    const T *__restrict__ sq, uint64_t n, const unsigned long long *fault,
    const double *__restrict__ chunk_sum, const double *__restrict__ chunk_pre,
    ChunkSummary *__restrict__ summ, SumScan<T> *__restrict__ runs, NodeGate gate)
{
    if (block_gate_closed(gate))
        return;
    using U = typename SumBits<T>::U;
    constexpr int P = SumBits<T>::kPer;
    __shared__ SumScan<T> wave_tot[kSumThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t c = blockIdx.x;
    const uint64_t limit = sum_limit(fault, n);
    const double pre = chunk_pre[c];
    const int32_t lo = phase_ue_of<T>(pre * (1.0 - 1.0 / 512)), hi = phase_ue_of<T>(pre * (1.0 + 1.0 / 512));
    const int32_t end = phase_ue_of<T>((pre + chunk_sum[c]) * (1.0 + 1.0 / 512));
    ChunkSummary *out = summ + kCands * c + blockIdx.y;
    if ((blockIdx.y == 1 && hi == lo) || (blockIdx.y == 2 && end <= lo)) {
        if (tid == 0)
            *out = ChunkSummary{0, 0, kNoPhase, 0};
        return;
    }
    const int ue = blockIdx.y == 0 ? lo : (blockIdx.y == 1 ? hi : hi + 1);
    const U *src = reinterpret_cast<const U *>(sq);
    U cur[P];
    const uint64_t base = c * sum_chunk_len<T>();
    load_chunk<T>(src, ((uintptr_t)sq & 15u) == 0, base, limit, tid, cur);
    const uint64_t first = base + (uint64_t)tid * P;
    SumScan<T> mine = scan_identity<T>();
#pragma unroll
    for (int j = 0; j < P; j++) {
        typename SumBits<T>::C nn;
        uint32_t cls;
        sum_elem<T>(cur[j], ue, nn, cls);
        if (first + j < limit)
            mine = scan_compose<T>(mine, scan_elem<T>(nn, cls));
    }
    SumScan<T> excl, total;
    block_scan<T>(mine, lane, wave, wave_tot, excl, total);
    runs[(kCands * c + blockIdx.y) * kSumThreads + tid] = excl;
    if (tid == 0)
        *out = ChunkSummary{(uint64_t)total.r0, (uint64_t)total.r1, ue, 0};
}

// D: the ordered walk (one workgroup), then total (/) count.
template <typename T>
__global__ __launch_bounds__(kSumThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_mse_ordered_walk(
    const T *__restrict__ sq, uint64_t n, T count, int policy, T *__restrict__ out,
    unsigned long long *fault, const double *__restrict__ chunk_sum,
    const ChunkSummary *__restrict__ summ, const SumScan<T> *__restrict__ runs, NodeGate gate)
{
    if (block_gate_closed(gate))
        return;
    using U = typename SumBits<T>::U;
    using C = typename SumBits<T>::C;
    constexpr C kBig = SumBits<T>::kBig;
    __shared__ WalkShared<T> sh;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) {
        sh.limit = sum_limit(fault, n);
        sh.first[0] = sh.first[1] = kNoStep;
    }
    __syncthreads();
    const uint64_t limit = sh.limit;
    const U *src = reinterpret_cast<const U *>(sq);
    const uint64_t L = sum_chunk_len<T>();
    const uint64_t chunks = (limit + L - 1) / L;

    int ue;
    C m, mmax;
    sum_phase<T>((U)0, ue, m, mmax); // the total starts at +0
    uint64_t c0 = 0;
    for (int it = 0; c0 < chunks; it++) {
        const int slot = it & 1;
        const uint64_t c = c0 + tid;
        SumScan<T> mine = scan_identity<T>();
        int cand = -1;
        if (c < chunks) {
            for (int y = kCands - 1; y >= 0; y--)
                if (summ[kCands * c + y].ue == ue)
                    cand = y;
            // Summary counts saturate at kCap, past any crossing: they fit C. No summary for
            // this binade: stop here.
            mine = cand >= 0 ? scan_of_summary<T>(summ[kCands * c + cand]) : SumScan<T>{kBig, kBig, 2u};
        }
        SumScan<T> before, total;
        block_scan<T>(mine, lane, wave, sh.wave_tot, before, total);
        const uint32_t p0 = (uint32_t)(m & 1u);
        const C mt = sat_add<T>(m, p0 ? before.r1 : before.r0);
        const uint32_t pt = p0 ? (before.p >> 1) & 1u : before.p & 1u;
        if (c < chunks && mt < mmax && sat_add<T>(mt, pt ? mine.r1 : mine.r0) >= mmax) {
            sh.first[slot] = (uint32_t)tid;
            sh.m_first[slot] = (uint64_t)mt;
            sh.first_cand[slot] = cand;
        }
        __syncthreads();
        const uint32_t first = sh.first[slot];
        const C m_first = (C)sh.m_first[slot];
        const int first_cand = sh.first_cand[slot];
        if (tid == 0)
            sh.first[slot ^ 1] = kNoStep;
        if (first == kNoStep) {
            m = sat_add<T>(m, p0 ? total.r1 : total.r0);
            c0 += kSumThreads;
            continue;
        }
        // Chunks before the stopping one fold; it runs exactly from the count before it:
        // from its run prefixes when it has a summary for this binade, and in windows from
        // wherever that leaves off.
        m = m_first;
        const uint64_t cc = c0 + first;
        const uint64_t base = cc * L;
        const uint32_t len = (uint32_t)(base + L <= limit ? L : limit - base);
        uint32_t resume = 0;
        const int folded = first_cand < 0 ? -1
                                          : run_prefix_chunk<T>(src, runs + kCands * cc * kSumThreads,
                                                                summ + kCands * cc, first_cand, base, len,
                                                                policy, fault, ue, m, mmax, resume, sh, gate);
        if (folded == 0)
            return;
        if (folded < 0 && !exact_chunk<T>(src, base, len, resume, chunk_sum[cc] / (double)len, policy,
                                          fault, ue, m, mmax, sh, gate))
            return;
        c0 = cc + 1;
    }
    if (limit < n || tid != 0)
        return;
    const T total = from_bits<T>(sum_bits<T>(ue, m));
    const T r = total / count;
    const uint32_t kind = classify_div(total, count, r, policy);
    if (kind != kOk) {
        atomicMin(fault, (unsigned long long)pack_fault(3 * n, kind));
        gate_record(gate);
    } else {
        *out = r;
    }
}

// Small inputs (n <= kMseSerialMax), one workgroup. Its four waves form every difference and
// square in parallel into LDS (each thread issues all of its loads before it computes, so
// the inputs arrive in one round trip) and find the first faulting Subtract or Multiply; then
// one wave folds the squares before that element into the total in order, a chunk of 60
// (binary64 30) at a time, each lane holding the chunk's squares in registers and the next
// chunk's loads in flight. The
// squares folded are finite, so a sum can only fault by overflowing (the total turns, and
// stays, infinite) or, under RejectSubnormal, by being subnormal: a chunk is folded with
// plain adds (under RejectSubnormal each partial total is kept and checked after), and folded
// again with the exact add classifier only when that trips. The same results and first fault
// as the pipeline above, in one launch and no scratch.
template <typename T, bool REJECT_SUB>
__global__ __launch_bounds__(256) void k_mse_serial(const T *__restrict__ p, const T *__restrict__ t,
                                                    uint64_t n, T count, int policy,
                                                    T *__restrict__ out, unsigned long long *fault,
                                                    NodeGate gate)
{
    if (block_gate_closed(gate))
        return;
    constexpr int P = 16 / sizeof(T);           // squares per 16-byte LDS read
    constexpr int R = (int)(kMseSerialMax / 256); // elements a thread
    __shared__ __align__(16) T sq[kMseSerialMax];
    __shared__ unsigned long long first_sm; // earliest Subtract or Multiply fault word
    const int tid = threadIdx.x;
    if (tid == 0)
        first_sm = kNoFault;
    T pv[R], tv[R];
#pragma unroll
    for (int j = 0; j < R; j++) {
        const uint64_t i = (uint64_t)tid + 256u * (uint64_t)j;
        if (i < n) {
            pv[j] = p[i];
            tv[j] = t[i];
        }
    }
    __syncthreads();
    uint64_t key = kNoFault;
#pragma unroll
    for (int j = 0; j < R; j++) {
        const uint64_t i = (uint64_t)tid + 256u * (uint64_t)j;
        if (i < n) {
            const T d = pv[j] - tv[j];
            const T s = d * d;
            sq[i] = s;
            if (key == kNoFault) {
                const uint32_t ks = classify_add(pv[j], tv[j], d, policy);
                if (ks != kOk) {
                    key = pack_fault(3 * i, ks);
                } else {
                    const uint32_t km = classify_mul(d, d, s, policy);
                    if (km != kOk)
                        key = pack_fault(3 * i + 1, km);
                }
            }
        }
    }
    if (key != kNoFault)
        atomicMin(&first_sm, (unsigned long long)key);
    __syncthreads();
    if (tid >= 64)
        return;
    const unsigned long long fsm = first_sm;
    const uint64_t limit = fsm == kNoFault ? n : ((fsm >> 3) / 3); // elements summed
    auto record = [&](uint64_t w) {
        if (tid == 0) {
            atomicMin(fault, (unsigned long long)w);
            gate_record(gate);
        }
    };
    T total = (T)0;
    // The exact pass over squares i0 .. i0 + here - 1 from `total`: false when an add faults
    // (recorded).
    auto exact = [&](uint64_t i0, int here) {
        T tot = total;
        for (int j = 0; j < here; j++) {
            const T sj = sq[i0 + j];
            const T nxt = tot + sj;
            const uint32_t k_add = classify_add(tot, sj, nxt, policy);
            if (k_add != kOk) {
                record(pack_fault(3 * (i0 + j) + 2, k_add));
                return false;
            }
            tot = nxt;
        }
        return true;
    };
    // A chunk is 15 LDS reads: with the next chunk's 15 reads issued before its adds, the
    // wait for this chunk (in-order LDS counter, at most 15 outstanding) leaves all of them in
    // flight.
    constexpr int CH = 15 * P;
    auto load = [&](T (&v)[CH], uint64_t i0) {
#pragma unroll
        for (int q = 0; q < CH / P; q++)
            *reinterpret_cast<uint4 *>(&v[P * q]) = *reinterpret_cast<const uint4 *>(&sq[i0 + P * q]);
    };
    // Folds a whole chunk held in v; false when an add faults (recorded).
    auto fold = [&](T (&v)[CH], uint64_t i0) __attribute__((always_inline)) {
        T sum = total;
        bool trip = false;
        if constexpr (!REJECT_SUB) {
#pragma unroll
            for (int j = 0; j < CH; j++)
                sum = sum + v[j];
        } else {
#pragma unroll
            for (int j = 0; j < CH; j++) {
                sum = sum + v[j];
                v[j] = sum;
            }
#pragma unroll
            for (int j = 0; j < CH; j++)
                trip |= subnormal(v[j]);
        }
        if ((!finite_bits(sum) || trip) && !exact(i0, CH))
            return false;
        total = sum;
        return true;
    };
    const uint64_t full = limit / CH * CH;
    T va[CH], vb[CH];
    if (full > 0)
        load(va, 0);
    for (uint64_t i0 = 0; i0 < full; i0 += 2 * CH) {
        const bool second = i0 + CH < full;
        if (second)
            load(vb, i0 + CH);
        if (!fold(va, i0))
            return;
        if (!second)
            break;
        if (i0 + 2 * CH < full)
            load(va, i0 + 2 * CH);
        if (!fold(vb, i0 + CH))
            return;
    }
    if (limit > full) {
        const int here = (int)(limit - full);
        T sum = total;
        bool trip = false;
        for (int j = 0; j < here; j++) {
            sum = sum + sq[full + j];
            trip |= REJECT_SUB && subnormal(sum);
        }
        if ((!finite_bits(sum) || trip) && !exact(full, here))
            return;
        total = sum;
    }
    if (fsm != kNoFault) {
        record(fsm);
        return;
    }
    const T r = total / count;
    const uint32_t kind = classify_div(total, count, r, policy);
    if (kind != kOk)
        record(pack_fault(3 * n, kind));
    else if (tid == 0)
        *out = r;
}

// ------------------------------------------------------------- native compounds
// Explicitly permitted native compound arithmetic (Boundary + BackendDefined): no fault is
// classified; special values and subnormals flow through as the hardware produces them.

// SGD (backends/rocm/tensor/native_sgd/native_sgd.rs:100-145): the product rounded before
// the subtraction, or one fused multiply-add when contraction is permitted.
template <typename T, bool VEC, bool CONTRACT>
__global__ __launch_bounds__(kEwThreads) void k_native_sgd(const T *w,
                                                           const T *g, T rate,
                                                           T *out, uint64_t n, NodeGate gate)
{
    if (wave_gate_closed(gate))
        return;
    constexpr int W = Lanes<T, VEC>::W;
    PCU_EW_LOOP(W)
    {
        T wv[W], gv[W], r[W];
        load_lanes<T, VEC>(w, base, n, wv);
        load_lanes<T, VEC>(g, base, n, gv);
#pragma unroll
        for (int j = 0; j < W; j++) {
            if (CONTRACT) {
                r[j] = fma(-rate, gv[j], wv[j]);
            } else {
                const T p = rate * gv[j];
                r[j] = wv[j] - p;
            }
        }
        store_lanes<T, VEC>(out, base, n, r);
    }
}

// MSE (backends/rocm/tensor/native_loss/native_loss.rs, tensor.rs:5020-5070): rounded
// difference and square, a sum in the declared precision, times the rounded reciprocal
// count. The sum is a fixed-shape tree (per thread, wave, block, then over the blocks), so
// it repeats bit for bit from run to run.
template <typename T>
__device__ __forceinline__ T block_tree_sum(T v, T *part)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        v = v + __shfl_xor(v, off, 64);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0)
        part[wave] = v;
    __syncthreads();
    T total = (T)0;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++)
        total = total + part[w];
    return total;
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kEwThreads) void k_native_mse_partial(const T *__restrict__ p,
                                                                   const T *__restrict__ t,
                                                                   T *__restrict__ partial,
                                                                   uint64_t n, NodeGate gate)
{
    if (block_gate_closed(gate))
        return;
    __shared__ T part[kEwThreads / 64];
    constexpr int W = Lanes<T, VEC>::W;
    T acc = (T)0;
    PCU_EW_LOOP(W)
    {
        T pv[W], tv[W];
        load_lanes<T, VEC>(p, base, n, pv);
        load_lanes<T, VEC>(t, base, n, tv);
        T local = (T)0;
#pragma unroll
        for (int j = 0; j < W; j++) {
            const T d = pv[j] - tv[j];
            const T sq = d * d;
            local = local + (base + j < n ? sq : (T)0);
        }
        acc = acc + local;
    }
    const T total = block_tree_sum(acc, part);
    if (threadIdx.x == 0)
        partial[blockIdx.x] = total;
}

template <typename T>
__global__ __launch_bounds__(1024) void k_native_mse_final(const T *__restrict__ partial,
                                                           uint64_t blocks, T scale,
                                                           T *__restrict__ out, NodeGate gate)
{
    if (block_gate_closed(gate))
        return;
    __shared__ T part[16];
    T acc = (T)0;
    for (uint64_t i = threadIdx.x; i < blocks; i += 1024)
        acc = acc + partial[i];
    const T total = block_tree_sum(acc, part);
    if (threadIdx.x == 0)
        *out = total * scale;
}

// ================================================================ launchers

static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

static inline unsigned grid_for(uint64_t work_items)
{
    // One work item per thread; beyond 2^24 blocks the kernels' loops take the rest.
    uint64_t blocks = (work_items + kEwThreads - 1) / kEwThreads;
    if (blocks > (1ull << 24))
        blocks = 1ull << 24;
    return blocks ? (unsigned)blocks : 1u;
}

template <typename T>
static hipError_t binary_t(hipStream_t s, int op, uint64_t n, const void *a, const void *b,
                           const void *b_value, void *out, int policy, unsigned long long *fault, NodeGate gate)
{
    const T *A = (const T *)a, *B = (const T *)b;
    T bv = b_value ? *(const T *)b_value : (T)0;
    bool uniform = b == nullptr;
    constexpr int Wd = Vec<T>::width;
    bool vec = aligned16(a) && aligned16(out) && (uniform || aligned16(b));
    unsigned grid = grid_for(vec ? (n + Wd - 1) / Wd : n);
#define PCU_LAUNCH_BINARY(OPC)                                                                      \
    if (uniform) {                                                                                  \
        if (vec) hipLaunchKernelGGL((k_binary<T, OPC, true, true>), dim3(grid), dim3(kEwThreads), 0, s, A, B, bv, (T *)out, n, policy, fault, gate); \
        else hipLaunchKernelGGL((k_binary<T, OPC, true, false>), dim3(grid), dim3(kEwThreads), 0, s, A, B, bv, (T *)out, n, policy, fault, gate); \
    } else {                                                                                        \
        if (vec) hipLaunchKernelGGL((k_binary<T, OPC, false, true>), dim3(grid), dim3(kEwThreads), 0, s, A, B, bv, (T *)out, n, policy, fault, gate); \
        else hipLaunchKernelGGL((k_binary<T, OPC, false, false>), dim3(grid), dim3(kEwThreads), 0, s, A, B, bv, (T *)out, n, policy, fault, gate); \
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
                         unsigned long long *fault, NodeGate gate)
{
    if (n == 0)
        return hipSuccess;
    return dtype == 0 ? binary_t<float>(s, op, n, a, b, b_value, out, policy, fault, gate)
                      : binary_t<double>(s, op, n, a, b, b_value, out, policy, fault, gate);
}

template <typename T>
static hipError_t relu_t(hipStream_t s, uint64_t n, const void *x, void *out, int policy,
                         unsigned long long *fault, NodeGate gate)
{
    constexpr int Wd = Vec<T>::width;
    bool vec = aligned16(x) && aligned16(out);
    unsigned grid = grid_for(vec ? (n + Wd - 1) / Wd : n);
    if (vec)
        hipLaunchKernelGGL((k_relu<T, true>), dim3(grid), dim3(kEwThreads), 0, s, (const T *)x, (T *)out, n, policy, fault, gate);
    else
        hipLaunchKernelGGL((k_relu<T, false>), dim3(grid), dim3(kEwThreads), 0, s, (const T *)x, (T *)out, n, policy, fault, gate);
    return hipGetLastError();
}

template <typename T>
static hipError_t chain_t(hipStream_t s, uint64_t n, const ChainLaunch &c, NodeGate gate)
{
    constexpr int Wd = Vec<T>::width;
    bool vec = aligned16(c.head);
    for (int i = 0; i < c.steps; i++)
        vec = vec && aligned16(c.step[i].other) && aligned16(c.step[i].out);
    const unsigned grid = grid_for(vec ? (n + Wd - 1) / Wd : n);
    int sig = 0;
    for (int i = 0; i < c.steps && i < kChainMaxSteps; i++)
        sig |= c.step[i].op << (4 * i);
    const int key = c.steps * 2 + (vec ? 1 : 0);
    if (c.steps == 2 && sig == kSigSubMul) {
        if (vec) hipLaunchKernelGGL((k_chain<T, true, 2, kSigSubMul>), dim3(grid), dim3(kEwThreads), 0, s, c, n, gate);
        else hipLaunchKernelGGL((k_chain<T, false, 2, kSigSubMul>), dim3(grid), dim3(kEwThreads), 0, s, c, n, gate);
        return hipGetLastError();
    }
    if (c.steps == 2 && sig == kSigAddRelu) {
        if (vec) hipLaunchKernelGGL((k_chain<T, true, 2, kSigAddRelu>), dim3(grid), dim3(kEwThreads), 0, s, c, n, gate);
        else hipLaunchKernelGGL((k_chain<T, false, 2, kSigAddRelu>), dim3(grid), dim3(kEwThreads), 0, s, c, n, gate);
        return hipGetLastError();
    }
    if (c.steps == 3 && sig == kSigSubMulReluBack) {
        if (vec) hipLaunchKernelGGL((k_chain<T, true, 3, kSigSubMulReluBack>), dim3(grid), dim3(kEwThreads), 0, s, c, n, gate);
        else hipLaunchKernelGGL((k_chain<T, false, 3, kSigSubMulReluBack>), dim3(grid), dim3(kEwThreads), 0, s, c, n, gate);
        return hipGetLastError();
    }
    switch (key) {
    case 3: hipLaunchKernelGGL((k_chain<T, true, 1>), dim3(grid), dim3(kEwThreads), 0, s, c, n, gate); break;
    case 2: hipLaunchKernelGGL((k_chain<T, false, 1>), dim3(grid), dim3(kEwThreads), 0, s, c, n, gate); break;
    case 5: hipLaunchKernelGGL((k_chain<T, true, 2>), dim3(grid), dim3(kEwThreads), 0, s, c, n, gate); break;
    case 4: hipLaunchKernelGGL((k_chain<T, false, 2>), dim3(grid), dim3(kEwThreads), 0, s, c, n, gate); break;
    case 7: hipLaunchKernelGGL((k_chain<T, true, 3>), dim3(grid), dim3(kEwThreads), 0, s, c, n, gate); break;
    case 6: hipLaunchKernelGGL((k_chain<T, false, 3>), dim3(grid), dim3(kEwThreads), 0, s, c, n, gate); break;
    case 9: hipLaunchKernelGGL((k_chain<T, true, 4>), dim3(grid), dim3(kEwThreads), 0, s, c, n, gate); break;
    case 8: hipLaunchKernelGGL((k_chain<T, false, 4>), dim3(grid), dim3(kEwThreads), 0, s, c, n, gate); break;
    default: return hipErrorInvalidValue; // a chain has 1 to 4 steps
    }
    return hipGetLastError();
}

hipError_t launch_chain(hipStream_t s, int dtype, uint64_t n, const ChainLaunch &c, NodeGate gate)
{
    if (n == 0 || c.steps <= 0)
        return hipSuccess;
    return dtype == 0 ? chain_t<float>(s, n, c, gate) : chain_t<double>(s, n, c, gate);
}

hipError_t launch_relu(hipStream_t s, int dtype, uint64_t n, const void *x, void *out,
                       int policy, unsigned long long *fault, NodeGate gate)
{
    if (n == 0)
        return hipSuccess;
    return dtype == 0 ? relu_t<float>(s, n, x, out, policy, fault, gate)
                      : relu_t<double>(s, n, x, out, policy, fault, gate);
}

template <typename T>
static hipError_t relu_backward_t(hipStream_t s, uint64_t n, const void *x, const void *up,
                                  void *out, int policy, unsigned long long *fault, NodeGate gate)
{
    constexpr int Wd = Vec<T>::width;
    bool vec = aligned16(x) && aligned16(up) && aligned16(out);
    unsigned grid = grid_for(vec ? (n + Wd - 1) / Wd : n);
    if (vec)
        hipLaunchKernelGGL((k_relu_backward<T, true>), dim3(grid), dim3(kEwThreads), 0, s, (const T *)x, (const T *)up, (T *)out, n, policy, fault, gate);
    else
        hipLaunchKernelGGL((k_relu_backward<T, false>), dim3(grid), dim3(kEwThreads), 0, s, (const T *)x, (const T *)up, (T *)out, n, policy, fault, gate);
    return hipGetLastError();
}

hipError_t launch_relu_backward(hipStream_t s, int dtype, uint64_t n, const void *x,
                                const void *up, void *out, int policy,
                                unsigned long long *fault, NodeGate gate)
{
    if (n == 0)
        return hipSuccess;
    return dtype == 0 ? relu_backward_t<float>(s, n, x, up, out, policy, fault, gate)
                      : relu_backward_t<double>(s, n, x, up, out, policy, fault, gate);
}

template <typename T>
static hipError_t add_relu_t(hipStream_t s, uint64_t n, const void *a, const void *b,
                             const void *b_value, void *out, int policy,
                             unsigned long long *fault_add, unsigned long long *fault_relu, NodeGate gate)
{
    const T *A = (const T *)a, *B = (const T *)b;
    T bv = b_value ? *(const T *)b_value : (T)0;
    bool uniform = b == nullptr;
    constexpr int Wd = Vec<T>::width;
    bool vec = aligned16(a) && aligned16(out) && (uniform || aligned16(b));
    unsigned grid = grid_for(vec ? (n + Wd - 1) / Wd : n);
    if (uniform) {
        if (vec) hipLaunchKernelGGL((k_add_relu<T, true, true>), dim3(grid), dim3(kEwThreads), 0, s, A, B, bv, (T *)out, n, policy, fault_add, fault_relu, gate);
        else hipLaunchKernelGGL((k_add_relu<T, true, false>), dim3(grid), dim3(kEwThreads), 0, s, A, B, bv, (T *)out, n, policy, fault_add, fault_relu, gate);
    } else {
        if (vec) hipLaunchKernelGGL((k_add_relu<T, false, true>), dim3(grid), dim3(kEwThreads), 0, s, A, B, bv, (T *)out, n, policy, fault_add, fault_relu, gate);
        else hipLaunchKernelGGL((k_add_relu<T, false, false>), dim3(grid), dim3(kEwThreads), 0, s, A, B, bv, (T *)out, n, policy, fault_add, fault_relu, gate);
    }
    return hipGetLastError();
}

hipError_t launch_add_relu(hipStream_t s, int dtype, uint64_t n, const void *a, const void *b,
                           const void *b_value, void *out, int policy,
                           unsigned long long *fault_add, unsigned long long *fault_relu, NodeGate gate)
{
    if (n == 0)
        return hipSuccess;
    return dtype == 0 ? add_relu_t<float>(s, n, a, b, b_value, out, policy, fault_add, fault_relu, gate)
                      : add_relu_t<double>(s, n, a, b, b_value, out, policy, fault_add, fault_relu, gate);
}

// An SGD launch ends its program (ProgramClose) only on a grid of at most kCloseMaxBlocks
// workgroups: every workgroup takes one ticket on a single counter at its end, and the
// tickets queue behind one another (1024 of them made a 2^20-element update 15 -> 24 us).

template <typename T>
static hipError_t sgd_t(hipStream_t s, uint64_t n, const void *w, const void *g, T rate,
                        void *out, int policy, unsigned long long *fault, NodeGate gate,
                        ProgramClose close, bool *closed)
{
    constexpr int Wd = Vec<T>::width;
    bool vec = aligned16(w) && aligned16(g) && aligned16(out);
    unsigned grid = grid_for(vec ? (n + Wd - 1) / Wd : n);
    if (grid > kCloseMaxBlocks)
        close = ProgramClose{};
    if (closed)
        *closed = close.words != nullptr;
    if (vec)
        hipLaunchKernelGGL((k_sgd<T, true>), dim3(grid), dim3(kEwThreads), 0, s, (const T *)w, (const T *)g, rate, (T *)out, n, policy, fault, gate, close);
    else
        hipLaunchKernelGGL((k_sgd<T, false>), dim3(grid), dim3(kEwThreads), 0, s, (const T *)w, (const T *)g, rate, (T *)out, n, policy, fault, gate, close);
    return hipGetLastError();
}

hipError_t launch_sgd(hipStream_t s, int dtype, uint64_t n, const void *w, const void *g,
                      double rate, void *out, int policy, unsigned long long *fault, NodeGate gate,
                      ProgramClose close, bool *closed)
{
    if (closed)
        *closed = false;
    if (n == 0)
        return hipSuccess;
    return dtype == 0 ? sgd_t<float>(s, n, w, g, (float)rate, out, policy, fault, gate, close, closed)
                      : sgd_t<double>(s, n, w, g, rate, out, policy, fault, gate, close, closed);
}

template <typename T>
static hipError_t sgd_pair_t(hipStream_t s, const SgdJob &j0, const SgdJob &j1, int policy,
                             ProgramClose close, bool *closed)
{
    constexpr int Wd = Vec<T>::width;
    const SgdJob *j[2] = {&j0, &j1};
    bool vec = true;
    for (int u = 0; u < 2; u++)
        vec = vec && aligned16(j[u]->w) && aligned16(j[u]->g) && aligned16(j[u]->out);
    SgdPairArgs<T> a;
    unsigned blocks[2];
    for (int u = 0; u < 2; u++) {
        a.w[u] = (const T *)j[u]->w;
        a.g[u] = (const T *)j[u]->g;
        a.out[u] = (T *)j[u]->out;
        a.rate[u] = (T)j[u]->rate;
        a.n[u] = j[u]->n;
        a.fault[u] = j[u]->fault;
        a.gate[u] = j[u]->gate;
        // grid_for caps each at 2^24 blocks, so the sum fits a launch.
        blocks[u] = grid_for(vec ? (j[u]->n + Wd - 1) / Wd : j[u]->n);
    }
    a.blocks0 = blocks[0];
    const dim3 grid(blocks[0] + blocks[1]);
    if (grid.x > kCloseMaxBlocks)
        close = ProgramClose{};
    if (closed)
        *closed = close.words != nullptr;
    if (vec)
        hipLaunchKernelGGL((k_sgd_pair<T, true>), grid, dim3(kEwThreads), 0, s, a, policy, close);
    else
        hipLaunchKernelGGL((k_sgd_pair<T, false>), grid, dim3(kEwThreads), 0, s, a, policy, close);
    return hipGetLastError();
}

hipError_t launch_sgd_pair(hipStream_t s, int dtype, const SgdJob &j0, const SgdJob &j1, int policy,
                           ProgramClose close, bool *closed)
{
    if (closed)
        *closed = false;
    if (j0.n == 0 || j1.n == 0)
        return hipErrorInvalidValue;
    return dtype == 0 ? sgd_pair_t<float>(s, j0, j1, policy, close, closed)
                      : sgd_pair_t<double>(s, j0, j1, policy, close, closed);
}

// Scratch of one MSE call: the squares, then the chunk sums and the chunk summaries.
static inline size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

template <typename T>
static size_t mse_chunks(uint64_t n)
{
    const uint64_t L = (uint64_t)kSumThreads * SumBits<T>::kPer;
    return (size_t)((n + L - 1) / L);
}

size_t mse_scratch_bytes(int dtype, uint64_t n)
{
    const size_t es = dtype == 0 ? 4 : 8;
    const size_t chunks = dtype == 0 ? mse_chunks<float>(n) : mse_chunks<double>(n);
    const size_t run_bytes = dtype == 0 ? sizeof(SumScan<float>) : sizeof(SumScan<double>);
    return round256(n * es) + 2 * round256(chunks * sizeof(double)) +
           round256(kCands * chunks * sizeof(ChunkSummary)) +
           round256(kCands * chunks * kSumThreads * run_bytes);
}

template <typename T> struct MseScratch {
    T *squares;
    double *chunk_sum, *chunk_pre;
    ChunkSummary *summ;
    SumScan<T> *runs;
    size_t chunks;
    MseScratch(void *scratch, uint64_t n)
    {
        char *base = (char *)scratch;
        chunks = mse_chunks<T>(n);
        squares = (T *)base;
        chunk_sum = (double *)(base + round256(n * sizeof(T)));
        chunk_pre = (double *)((char *)chunk_sum + round256(chunks * sizeof(double)));
        summ = (ChunkSummary *)((char *)chunk_pre + round256(chunks * sizeof(double)));
        runs = (SumScan<T> *)((char *)summ + round256(kCands * chunks * sizeof(ChunkSummary)));
    }
};

template <typename T>
static hipError_t mse_prepare_t(hipStream_t s, uint64_t n, const void *p, const void *t,
                                void *scratch, int policy, unsigned long long *fault, NodeGate gate)
{
    constexpr int Wd = Vec<T>::width;
    const MseScratch<T> m(scratch, n);
    const bool vec = aligned16(p) && aligned16(t) && aligned16(m.squares);
    const unsigned grid = grid_for(vec ? (n + Wd - 1) / Wd : n);
    if (vec)
        hipLaunchKernelGGL((k_mse_squares<T, true>), dim3(grid), dim3(kEwThreads), 0, s, (const T *)p, (const T *)t, m.squares, n, policy, fault, gate);
    else
        hipLaunchKernelGGL((k_mse_squares<T, false>), dim3(grid), dim3(kEwThreads), 0, s, (const T *)p, (const T *)t, m.squares, n, policy, fault, gate);
    hipLaunchKernelGGL((k_mse_chunk_sums<T>), dim3((unsigned)m.chunks), dim3(256), 0, s, (const T *)m.squares, n, (const unsigned long long *)fault, m.chunk_sum, gate);
    hipLaunchKernelGGL(k_mse_chunk_prefix, dim3(1), dim3(kPrefixThreads), 0, s, (const double *)m.chunk_sum, (uint64_t)m.chunks, m.chunk_pre, gate);
    hipLaunchKernelGGL((k_mse_chunk_summaries<T>), dim3((unsigned)m.chunks, kCands), dim3(kSumThreads), 0, s, (const T *)m.squares, n, (const unsigned long long *)fault, (const double *)m.chunk_sum, (const double *)m.chunk_pre, m.summ, m.runs, gate);
    return hipGetLastError();
}

template <typename T>
static hipError_t mse_walk_t(hipStream_t s, uint64_t n, void *scratch, T count, void *out,
                             int policy, unsigned long long *fault, NodeGate gate)
{
    const MseScratch<T> m(scratch, n);
    hipLaunchKernelGGL((k_mse_ordered_walk<T>), dim3(1), dim3(kSumThreads), 0, s, (const T *)m.squares, n, count, policy, (T *)out, fault, (const double *)m.chunk_sum, (const ChunkSummary *)m.summ, (const SumScan<T> *)m.runs, gate);
    return hipGetLastError();
}

hipError_t launch_mse_prepare(hipStream_t s, int dtype, uint64_t n, const void *p, const void *t,
                              void *scratch, int policy, unsigned long long *fault, NodeGate gate)
{
    if (n == 0)
        return hipErrorInvalidValue;
    return dtype == 0 ? mse_prepare_t<float>(s, n, p, t, scratch, policy, fault, gate)
                      : mse_prepare_t<double>(s, n, p, t, scratch, policy, fault, gate);
}

hipError_t launch_mse_walk(hipStream_t s, int dtype, uint64_t n, void *scratch, double count,
                           void *out, int policy, unsigned long long *fault, NodeGate gate)
{
    if (n == 0)
        return hipErrorInvalidValue;
    return dtype == 0 ? mse_walk_t<float>(s, n, scratch, (float)count, out, policy, fault, gate)
                      : mse_walk_t<double>(s, n, scratch, count, out, policy, fault, gate);
}

hipError_t launch_mse_serial(hipStream_t s, int dtype, uint64_t n, const void *p, const void *t,
                             double count, void *out, int policy, unsigned long long *fault,
                             NodeGate gate)
{
    if (n == 0 || n > kMseSerialMax)
        return hipErrorInvalidValue;
    const bool rs = policy == kPolicyRejectSubnormal;
    if (dtype == 0 && rs)
        hipLaunchKernelGGL((k_mse_serial<float, true>), dim3(1), dim3(256), 0, s, (const float *)p, (const float *)t, n, (float)count, policy, (float *)out, fault, gate);
    else if (dtype == 0)
        hipLaunchKernelGGL((k_mse_serial<float, false>), dim3(1), dim3(256), 0, s, (const float *)p, (const float *)t, n, (float)count, policy, (float *)out, fault, gate);
    else if (rs)
        hipLaunchKernelGGL((k_mse_serial<double, true>), dim3(1), dim3(256), 0, s, (const double *)p, (const double *)t, n, count, policy, (double *)out, fault, gate);
    else
        hipLaunchKernelGGL((k_mse_serial<double, false>), dim3(1), dim3(256), 0, s, (const double *)p, (const double *)t, n, count, policy, (double *)out, fault, gate);
    return hipGetLastError();
}

// ------------------------------------------------------------ native launchers

template <typename T>
static hipError_t native_sgd_t(hipStream_t s, uint64_t n, const void *w, const void *g, T rate,
                               bool contracted, void *out, NodeGate gate)
{
    constexpr int Wd = Vec<T>::width;
    const bool vec = aligned16(w) && aligned16(g) && aligned16(out);
    const unsigned grid = grid_for(vec ? (n + Wd - 1) / Wd : n);
    const T *W = (const T *)w, *G = (const T *)g;
    T *O = (T *)out;
    if (vec && contracted) hipLaunchKernelGGL((k_native_sgd<T, true, true>), dim3(grid), dim3(kEwThreads), 0, s, W, G, rate, O, n, gate);
    else if (vec) hipLaunchKernelGGL((k_native_sgd<T, true, false>), dim3(grid), dim3(kEwThreads), 0, s, W, G, rate, O, n, gate);
    else if (contracted) hipLaunchKernelGGL((k_native_sgd<T, false, true>), dim3(grid), dim3(kEwThreads), 0, s, W, G, rate, O, n, gate);
    else hipLaunchKernelGGL((k_native_sgd<T, false, false>), dim3(grid), dim3(kEwThreads), 0, s, W, G, rate, O, n, gate);
    return hipGetLastError();
}

hipError_t launch_native_sgd(hipStream_t s, int dtype, uint64_t n, const void *w, const void *g,
                             double rate, bool contracted, void *out, NodeGate gate)
{
    if (n == 0)
        return hipSuccess;
    return dtype == 0 ? native_sgd_t<float>(s, n, w, g, (float)rate, contracted, out, gate)
                      : native_sgd_t<double>(s, n, w, g, rate, contracted, out, gate);
}

static uint64_t native_mse_blocks(int dtype, uint64_t n)
{
    const uint64_t w = dtype == 0 ? 4 : 2;
    return grid_for((n + w - 1) / w);
}

size_t native_mse_scratch_bytes(int dtype, uint64_t n)
{
    return (size_t)native_mse_blocks(dtype, n) * (dtype == 0 ? 4 : 8);
}

template <typename T>
static hipError_t native_mse_t(hipStream_t s, uint64_t n, const void *p, const void *t,
                               void *scratch, T scale, void *out, NodeGate gate)
{
    constexpr int Wd = Vec<T>::width;
    const bool vec = aligned16(p) && aligned16(t);
    const unsigned grid = grid_for(vec ? (n + Wd - 1) / Wd : n);
    if (vec)
        hipLaunchKernelGGL((k_native_mse_partial<T, true>), dim3(grid), dim3(kEwThreads), 0, s, (const T *)p, (const T *)t, (T *)scratch, n, gate);
    else
        hipLaunchKernelGGL((k_native_mse_partial<T, false>), dim3(grid), dim3(kEwThreads), 0, s, (const T *)p, (const T *)t, (T *)scratch, n, gate);
    hipLaunchKernelGGL((k_native_mse_final<T>), dim3(1), dim3(1024), 0, s, (const T *)scratch, (uint64_t)grid, scale, (T *)out, gate);
    return hipGetLastError();
}

hipError_t launch_native_mse(hipStream_t s, int dtype, uint64_t n, const void *p, const void *t,
                             void *scratch, double scale, void *out, NodeGate gate)
{
    if (n == 0)
        return hipErrorInvalidValue;
    return dtype == 0 ? native_mse_t<float>(s, n, p, t, scratch, (float)scale, out, gate)
                      : native_mse_t<double>(s, n, p, t, scratch, scale, out, gate);
}


// ------------------------------------------------------------ program end
// The fault words go to the host without a copy command: one workgroup copies them into
// coherent pinned memory, resets them (and opens the stage gate) for the next program, and
// then stores the program's sequence number, so the host waits on that one word instead of
// the stream.
__global__ __launch_bounds__(256) void k_program_publish(unsigned long long *words, uint64_t n,
                                                         unsigned long long value, unsigned int *gate,
                                                         unsigned long long *host_words,
                                                         unsigned long long *host_seq, uint64_t seq)
{
    for (uint64_t i = threadIdx.x; i < n; i += blockDim.x) {
        const unsigned long long w = words[i];
        __hip_atomic_store(&host_words[i], w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        words[i] = value;
    }
    if (threadIdx.x == 0)
        *gate = 0xffffffffu;
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_store(host_seq, (unsigned long long)seq, __ATOMIC_RELEASE,
                           __HIP_MEMORY_SCOPE_SYSTEM);
}

hipError_t launch_program_publish(hipStream_t s, unsigned long long *words, uint64_t n,
                                  uint64_t value, unsigned int *gate,
                                  unsigned long long *host_words, unsigned long long *host_seq,
                                  uint64_t seq)
{
    hipLaunchKernelGGL(k_program_publish, dim3(1), dim3(256), 0, s, words, n,
                       (unsigned long long)value, gate, host_words, host_seq, seq);
    return hipGetLastError();
}

} // namespace pcu

