// Device-side fault classification for the strict owned-tensor kernels (gfx950).
//
// Every kernel computes values with the hardware's IEEE-754 binary32/binary64 unit
// (round-to-nearest-even, denormals preserved, no contraction: the library is compiled
// with -ffp-contract=off and -fno-gpu-flush-denormals-to-zero). IEEE RNE gives the
// reference's value for every non-faulting operation (the reference's integer law is
// RNE with gradual underflow: core/scalar_checked_float.rs:361-448). What hardware
// results cannot show directly is the fault classification, which the functions below
// recover exactly:
//   invalid   : a non-finite operand (core/scalar_checked_float.rs:321-322)
//   overflow  : finite operands, infinite rounded result (:416-426)
//   underflow : policy applied to (tiny after rounding at unbounded exponent, inexact
//               after bounded packing, result subnormal) (:390-447,
//               core/scalar_float_underflow.rs:61-73)
// The cheap screens (`*_suspect`) are taken on every lane; the exact routines run only on
// lanes the screen flags.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pcu_kernels.hpp"

#pragma clang fp contract(off)

namespace pcu {

enum : uint32_t {
    kOk = 0,
    kDivideByZero = 1,
    kOverflow = 3,
    kUnderflow = 4,
    kInvalid = 5,
};

enum : int { kPolicyIeee = 0, kPolicyRejectSubnormal = 1, kPolicyAllowGradual = 2 };

constexpr uint64_t kNoFault = ~0ull;

// Packed fault word: (ordinal << 3) | kind; atomicMin keeps the earliest ordinal
// (backends/rocm/owned_dispatch.rs:20,76-110 uses the same packing).
__device__ __forceinline__ uint64_t pack_fault(uint64_t ordinal, uint32_t kind)
{
    return (ordinal << 3) | kind;
}

// ------------------------------------------------------------------ bit helpers

__device__ __forceinline__ uint32_t bits_of(float v) { return __float_as_uint(v); }
__device__ __forceinline__ uint64_t bits_of(double v) { return (uint64_t)__double_as_longlong(v); }

__device__ __forceinline__ bool finite_bits(float v)
{
    return (bits_of(v) & 0x7f800000u) != 0x7f800000u;
}
__device__ __forceinline__ bool finite_bits(double v)
{
    return (bits_of(v) & 0x7ff0000000000000ull) != 0x7ff0000000000000ull;
}

__device__ __forceinline__ bool is_zero(float v) { return (bits_of(v) & 0x7fffffffu) == 0; }
__device__ __forceinline__ bool is_zero(double v) { return (bits_of(v) & 0x7fffffffffffffffull) == 0; }

// Nonzero subnormal encoding.
__device__ __forceinline__ bool subnormal(float v)
{
    uint32_t m = bits_of(v) & 0x7fffffffu;
    return m != 0 && m < 0x00800000u;
}
__device__ __forceinline__ bool subnormal(double v)
{
    uint64_t m = bits_of(v) & 0x7fffffffffffffffull;
    return m != 0 && m < 0x0010000000000000ull;
}

// |v| <= smallest normal (bitwise, so no flush mode can interfere).
__device__ __forceinline__ bool at_most_min_normal(float v)
{
    return (bits_of(v) & 0x7fffffffu) <= 0x00800000u;
}
__device__ __forceinline__ bool at_most_min_normal(double v)
{
    return (bits_of(v) & 0x7fffffffffffffffull) <= 0x0010000000000000ull;
}

// ------------------------------------------------------------- add / subtract
// An IEEE sum that is tiny is exact, so Add/Sub never raise tiny-inexact underflow;
// RejectSubnormalResult still rejects a nonzero subnormal sum (including the zero-operand
// passthrough, core/scalar_checked_float.rs:508-532). Exact cancellation gives +0.

template <typename T>
__device__ __forceinline__ uint32_t classify_add(T a, T b, T r, int policy)
{
    if (!finite_bits(a) || !finite_bits(b))
        return kInvalid;
    if (!finite_bits(r))
        return kOverflow;
    if (policy == kPolicyRejectSubnormal && subnormal(r))
        return kUnderflow;
    return kOk;
}

template <typename T>
__device__ __forceinline__ bool add_suspect(T a, T b, T r, int policy)
{
    return !finite_bits(r) || !finite_bits(a) || !finite_bits(b) ||
           (policy == kPolicyRejectSubnormal && subnormal(r));
}

// ------------------------------------------------------------------- multiply

// Exact tininess/inexactness of a binary32 product: the product of two binary32 values
// is exact in binary64 (48 significant bits), so comparisons against it are exact.
// Tiny after rounding to 24 bits with an unbounded exponent <=> |p| < 2^-126 - 2^-151
// (the midpoint below 2^-126 rounds up to 2^-126 under ties-to-even).
__device__ __forceinline__ uint32_t mul_underflow_exact(float a, float b, float r, int policy)
{
    double p = (double)a * (double)b;
    bool tiny = fabs(p) < 0x1.ffffffp-127;
    bool inexact = (double)r != p;
    if (policy == kPolicyIeee)
        return (tiny && inexact) ? kUnderflow : kOk;
    return (subnormal(r) || (tiny && inexact)) ? kUnderflow : kOk;
}

// Binary64: the 106-bit integer product of the significands decides both facts.
// value(x) = sig * 2^q with sig < 2^53; value(a*b) = P * 2^(qa+qb).
__device__ __forceinline__ void decode_f64(double v, uint64_t &sig, int &q)
{
    uint64_t b = bits_of(v);
    uint64_t e = (b >> 52) & 0x7ff;
    uint64_t f = b & 0x000fffffffffffffull;
    if (e == 0) {
        sig = f;
        q = -1074;
    } else {
        sig = f | 0x0010000000000000ull;
        q = (int)e - 1075;
    }
}

__device__ __forceinline__ int bit_length_u128(uint64_t hi, uint64_t lo)
{
    return hi ? 128 - __clzll(hi) : (lo ? 64 - __clzll(lo) : 0);
}

// Low `n` bits of (hi:lo) are nonzero.
__device__ __forceinline__ bool low_bits_nonzero(uint64_t hi, uint64_t lo, int n)
{
    if (n <= 0)
        return false;
    if (n >= 128)
        return (hi | lo) != 0;
    if (n >= 64)
        return lo != 0 || (hi & ((n == 64) ? 0ull : ((1ull << (n - 64)) - 1))) != 0;
    return (lo & ((1ull << n) - 1)) != 0;
}

// Bit `n` of (hi:lo).
__device__ __forceinline__ uint64_t bit_at(uint64_t hi, uint64_t lo, int n)
{
    if (n < 0 || n >= 128)
        return 0;
    return n >= 64 ? (hi >> (n - 64)) & 1 : (lo >> n) & 1;
}

// Classify an exact value P * 2^q (P = hi:lo > 0) rounded to `prec` bits whose smallest
// normal exponent is `emin` (value >= 2^emin is normal) and whose subnormal quantum is
// 2^qmin. tiny: unbounded rounding < 2^emin; inexact: bounded rounding discards bits.
__device__ __forceinline__ void classify_exact(uint64_t hi, uint64_t lo, int q, int prec, int emin,
                                               int qmin, bool &tiny, bool &inexact)
{
    int len = bit_length_u128(hi, lo);
    int top = len - 1;                 // value in [2^(top+q), 2^(top+q+1))
    int e = top + q;                   // unbounded exponent before rounding
    int drop = top - (prec - 1);       // bits of P below the kept precision
    bool carry = false;
    if (drop > 0) {
        // Round to nearest even at bit `drop`; carry out when all kept bits are ones.
        uint64_t half = bit_at(hi, lo, drop - 1);
        bool sticky = low_bits_nonzero(hi, lo, drop - 1);
        bool lsb = bit_at(hi, lo, drop) != 0;
        bool up = half && (sticky || lsb);
        if (up) {
            // Kept bits all ones <=> P >> drop == 2^prec - 1.
            bool all_ones = true;
            for (int i = drop; i < drop + prec; i++)
                if (!bit_at(hi, lo, i)) {
                    all_ones = false;
                    break;
                }
            carry = all_ones;
        }
    }
    tiny = (e + (carry ? 1 : 0)) < emin;
    // Bounded: the lowest kept weight is max(2^(e - prec + 1), 2^qmin).
    int lowest = e - (prec - 1);
    if (lowest < qmin)
        lowest = qmin;
    inexact = low_bits_nonzero(hi, lo, lowest - q);
}

__device__ __forceinline__ uint32_t mul_underflow_exact(double a, double b, double r, int policy)
{
    uint64_t sa, sb;
    int qa, qb;
    decode_f64(a, sa, qa);
    decode_f64(b, sb, qb);
    uint64_t lo = sa * sb;
    uint64_t hi = __umul64hi(sa, sb);
    bool tiny, inexact;
    classify_exact(hi, lo, qa + qb, 53, -1022, -1074, tiny, inexact);
    if (policy == kPolicyIeee)
        return (tiny && inexact) ? kUnderflow : kOk;
    return (subnormal(r) || (tiny && inexact)) ? kUnderflow : kOk;
}

template <typename T>
__device__ __forceinline__ uint32_t classify_mul(T a, T b, T r, int policy)
{
    if (!finite_bits(a) || !finite_bits(b))
        return kInvalid;
    if (!finite_bits(r))
        return kOverflow;
    if (policy == kPolicyAllowGradual || !at_most_min_normal(r))
        return kOk;
    if (is_zero(a) || is_zero(b))
        return kOk; // exact signed zero (core/scalar_checked_float.rs:553-555)
    return mul_underflow_exact(a, b, r, policy);
}

template <typename T>
__device__ __forceinline__ bool mul_suspect(T a, T b, T r, int policy)
{
    return !finite_bits(r) || !finite_bits(a) || !finite_bits(b) ||
           (policy != kPolicyAllowGradual && at_most_min_normal(r) && !is_zero(a) && !is_zero(b));
}

// --------------------------------------------------------------------- divide
// Binary32: a = q*b exactly <=> (double)r*(double)b == (double)a (48-bit product, exact);
// tiny <=> |a| < (2^-126 - 2^-151)*|b|, a 49-bit exact product in binary64.
__device__ __forceinline__ uint32_t div_underflow_exact(float a, float b, float r, int policy)
{
    double ab = fabs((double)a), bb = fabs((double)b);
    bool tiny = ab < 0x1.ffffffp-127 * bb;
    bool inexact = (double)r * (double)b != (double)a;
    if (policy == kPolicyIeee)
        return (tiny && inexact) ? kUnderflow : kOk;
    return (subnormal(r) || (tiny && inexact)) ? kUnderflow : kOk;
}

// Binary64 long division of the normalised significands: 56 quotient bits plus a sticky
// remainder give the exact rounding facts (the reference divides with the same extent,
// core/scalar_checked_float/f64.rs:372-431).
__device__ __forceinline__ uint32_t div_underflow_exact(double a, double b, double r, int policy)
{
    uint64_t sa, sb;
    int qa, qb;
    decode_f64(a, sa, qa);
    decode_f64(b, sb, qb);
    int la = 63 - __clzll(sa), lb = 63 - __clzll(sb);
    sa <<= (52 - la);
    qa -= (52 - la);
    sb <<= (52 - lb);
    qb -= (52 - lb);
    int q = qa - qb; // quotient = (sa/sb) * 2^q, sa/sb in (1/2, 2)
    uint64_t num = sa;
    if (num < sb) {
        num <<= 1;
        q -= 1;
    }
    // num/sb in [1, 2): produce 56 quotient bits (value Q * 2^(q-55)).
    uint64_t quot = 0, rem = num;
    for (int i = 0; i < 56; i++) {
        quot <<= 1;
        if (rem >= sb) {
            rem -= sb;
            quot |= 1;
        }
        rem <<= 1;
    }
    // Sticky: make the remainder visible as an extra low bit below the 56 quotient bits.
    uint64_t lo = (quot << 1) | (rem != 0 ? 1ull : 0ull);
    uint64_t hi = quot >> 63;
    bool tiny, inexact;
    classify_exact(hi, lo, q - 56, 53, -1022, -1074, tiny, inexact);
    if (policy == kPolicyIeee)
        return (tiny && inexact) ? kUnderflow : kOk;
    return (subnormal(r) || (tiny && inexact)) ? kUnderflow : kOk;
}

template <typename T>
__device__ __forceinline__ uint32_t classify_div(T a, T b, T r, int policy)
{
    if (!finite_bits(a) || !finite_bits(b))
        return kInvalid;
    if (is_zero(b))
        return kDivideByZero;
    if (is_zero(a))
        return kOk;
    if (!finite_bits(r))
        return kOverflow;
    if (policy == kPolicyAllowGradual || !at_most_min_normal(r))
        return kOk;
    return div_underflow_exact(a, b, r, policy);
}

template <typename T>
__device__ __forceinline__ bool div_suspect(T a, T b, T r, int policy)
{
    return !finite_bits(r) || !finite_bits(a) || !finite_bits(b) || is_zero(b) ||
           (policy != kPolicyAllowGradual && at_most_min_normal(r) && !is_zero(a));
}

// ------------------------------------------------------------- relu selection
// core/scalar_checked_float.rs:273-309: non-finite -> invalid; negative or zero -> +0;
// policy applied to the (exact) selected value.
template <typename T>
__device__ __forceinline__ T relu_select(T x);
template <>
__device__ __forceinline__ float relu_select(float x)
{
    uint32_t b = bits_of(x);
    return ((b & 0x80000000u) || (b & 0x7fffffffu) == 0) ? 0.0f : x;
}
template <>
__device__ __forceinline__ double relu_select(double x)
{
    uint64_t b = bits_of(x);
    return ((b >> 63) || (b & 0x7fffffffffffffffull) == 0) ? 0.0 : x;
}

template <typename T>
__device__ __forceinline__ uint32_t classify_relu(T x, T r, int policy)
{
    if (!finite_bits(x))
        return kInvalid;
    if (policy == kPolicyRejectSubnormal && subnormal(r))
        return kUnderflow;
    return kOk;
}

// core/scalar_checked_float.rs:634-652: strictly positive input selects upstream.
template <typename T>
__device__ __forceinline__ bool strictly_positive(T x)
{
    return !(bits_of(x) >> (sizeof(T) * 8 - 1)) && !is_zero(x);
}

template <typename T>
__device__ __forceinline__ uint32_t classify_relu_backward(T x, T up, T r, int policy)
{
    if (!finite_bits(x) || !finite_bits(up))
        return kInvalid;
    if (policy == kPolicyRejectSubnormal && subnormal(r))
        return kUnderflow;
    return kOk;
}

// ---------------------------------------------------------- wave reductions
// Minimum of a 64-bit key over the wavefront (gfx950 waves are 64 lanes wide).
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        uint64_t o = __shfl_xor(v, off, 64);
        v = o < v ? o : v;
    }
    return v;
}

// ------------------------------------------------------------- stage gate
// The program's stage gate holds the lowest program node that has recorded an arithmetic
// fault (0xffffffff while none). A node's kernels skip their work once an earlier node has
// faulted: that node's fault is the one reported, so later work only costs time
// (backends/rocm/owned_dispatch/guarded/guarded.rs gates each stage on the previous stage's
// record). The gate only decreases, so a kernel that starts after it closed for its node
// skips, and any partial result of a kernel that was running when it closed is read only
// by later kernels of the same node, which skip too.
__device__ __forceinline__ void gate_record(const NodeGate &g)
{
    if (g.word)
        atomicMin(g.word, g.node);
}

// Block-uniform test (one read by thread 0, shared through LDS), so a block never splits
// around a barrier or a wave-level reduction. Call it first thing in a kernel.
__device__ __forceinline__ bool block_gate_closed(const NodeGate &g)
{
    __shared__ int closed;
    if (threadIdx.x == 0)
        closed = g.word != nullptr && __atomic_load_n(g.word, __ATOMIC_RELAXED) < g.node;
    __syncthreads();
    return closed != 0;
}

// The same test made by each wave on its own, for kernels with no barrier after it: no LDS
// and no barrier (2% faster for the one-vector-per-thread streaming kernels). Waves of one
// block may then disagree, which only matters where the block synchronizes.
__device__ __forceinline__ bool wave_gate_closed(const NodeGate &g)
{
    if (g.word == nullptr)
        return false;
    return __builtin_amdgcn_readfirstlane(__atomic_load_n(g.word, __ATOMIC_RELAXED)) < g.node;
}

// A MatMul screen's exponent word: (generation << 32) | (kExpBias - e). Under atomicMax a
// word of a later generation replaces any older one and, within one, the smallest e wins.
constexpr int kExpBias = 1 << 21;

__device__ __forceinline__ unsigned long long exp_word(uint32_t gen, int e)
{
    return ((unsigned long long)gen << 32) | (uint32_t)(kExpBias - e);
}
__device__ __forceinline__ int exp_of(unsigned long long w) { return kExpBias - (int)(uint32_t)w; }

// The tile kernels' partial-sum check, one v_cmp_class per sum (class bits 4 and 7:
// negative and positive subnormal) into a lane mask. Masks rotate through four slots: a check
// first ORs into `flag` the mask its slot got four checks earlier (long since written), then
// compares v into the slot, so no scalar OR waits on the compare just before it (a single
// vcc chain ran the checked loop 2.6x slower). The asm keeps every compare beside its sum (v
// is in-out, so the next sum of the cell waits for it): the compiler's own form batched the
// compares and spilled. The slots are named (an indexed array of them was not kept in
// scalar registers). s_or_b64 writes scc, which the asm declares (a loop branch on scc may
// follow it). `cls` holds kClassSubnormal; flush() ORs the slots at the end.
constexpr int kClassSubnormal = (1 << 4) | (1 << 7);
struct SubLanes {
    uint64_t flag = 0, s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    __device__ __forceinline__ uint64_t flush() const { return flag | s0 | s1 | s2 | s3; }
};
__device__ __forceinline__ void check_subnormal(uint64_t &flag, uint64_t &slot, float &v, int cls)
{
    asm volatile("s_or_b64 %0, %0, %1\n\tv_cmp_class_f32_e64 %1, %2, %3"
                 : "+s"(flag), "+s"(slot), "+v"(v)
                 : "v"(cls)
                 : "scc");
}
__device__ __forceinline__ void check_subnormal(uint64_t &flag, uint64_t &slot, double &v, int cls)
{
    asm volatile("s_or_b64 %0, %0, %1\n\tv_cmp_class_f64_e64 %1, %2, %3"
                 : "+s"(flag), "+s"(slot), "+v"(v)
                 : "v"(cls)
                 : "scc");
}
// Checks of four consecutive sums, one slot each.
template <typename T>
__device__ __forceinline__ void check_subnormal4(SubLanes &s, T &a, T &b, T &c, T &d, int cls)
{
    check_subnormal(s.flag, s.s0, a, cls);
    check_subnormal(s.flag, s.s1, b, cls);
    check_subnormal(s.flag, s.s2, c, cls);
    check_subnormal(s.flag, s.s3, d, cls);
}

// Whether the smallest exponent over the tile's rows [m0, m0 + BM) of op(A) plus the
// smallest over its columns [n0, n0 + BN) of op(B) lies below thr (zero and non-finite
// operands count 2^20). Block-wide, with one barrier: every thread of a block of at least
// 128 threads calls it and gets the same answer.
template <int BM, int BN>
__device__ __forceinline__ bool tile_exp_sum_below(const unsigned long long *row_exp,
                                                   const unsigned long long *col_exp, int m0,
                                                   int n0, int M, int N, int thr)
{
    __shared__ int tile_min[2];
    const int tid = threadIdx.x;
    if (tid < 128) {
        const bool rows = tid < 64;
        const int l = tid & 63, base = rows ? m0 : n0, lim = rows ? M : N, ext = rows ? BM : BN;
        const unsigned long long *w = rows ? row_exp : col_exp;
        int e = 1 << 20;
        for (int i = l; i < ext; i += 64)
            if (base + i < lim) {
                const int x = exp_of(w[base + i]);
                e = x < e ? x : e;
            }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const int o = __shfl_xor(e, off, 64);
            e = o < e ? o : e;
        }
        if (l == 0)
            tile_min[tid >> 6] = e;
    }
    __syncthreads();
    // Uniform by construction; readfirstlane tells the compiler, so values that merge after a
    // branch on it may stay in scalar registers.
    return __builtin_amdgcn_readfirstlane(tile_min[0] + tile_min[1]) < thr;
}

// The 16-bit exponent of zero and non-finite entries in the superslab tables (two of them
// still sum far above any threshold).
constexpr short kScanExpNone = 16000;

// A program's end by one wave (see ProgramClose): the words to the pinned mirror, reset,
// the gate opened, then the sequence number, after a system-scope fence.
__device__ __forceinline__ void program_close_wave(const ProgramClose &c)
{
    const int lane = threadIdx.x & 63;
    for (uint64_t i = lane; i < c.n; i += 64) {
        const unsigned long long w =
            __hip_atomic_load(&c.words[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&c.host_words[i], w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        c.words[i] = c.value;
    }
    if (lane == 0)
        *c.gate = 0xffffffffu;
    __threadfence_system();
    if (lane == 0)
        __hip_atomic_store(c.host_seq, (unsigned long long)c.seq, __ATOMIC_RELEASE,
                           __HIP_MEMORY_SCOPE_SYSTEM);
}

// Every workgroup of the launch calls it once, last thing, with all its threads: the last
// workgroup to arrive ends the program. The words the end reads are written only by
// device-scope atomics (fault records, the gate), performed where every XCD sees them. Each
// wave waits until its own memory operations have completed (the barrier alone waits only
// for LDS and scalar operations, so a fault record could still be in flight when the
// workgroup takes its ticket), and then no workgroup needs a device-scope release (on this
// part one writes back and invalidates the XCD's L2: a fence in each of the replay's 4096
// waves cost a faulting 1024^3 call about 70 us); only the last one acquires before it
// reads them.
__device__ __forceinline__ void program_close_block(const ProgramClose &c)
{
    if (c.words == nullptr)
        return;
    __shared__ int last;
    __builtin_amdgcn_s_waitcnt(0); // vmcnt(0) expcnt(0) lgkmcnt(0): the fault records are done
    __syncthreads();
    if (threadIdx.x == 0)
        last = atomicAdd(c.ticket, 1u) + 1u == gridDim.x * gridDim.y * gridDim.z;
    __syncthreads();
    if (last && threadIdx.x < 64) {
        __atomic_thread_fence(__ATOMIC_ACQUIRE);
        if (threadIdx.x == 0)
            *c.ticket = 0u; // every workgroup has taken its ticket
        program_close_wave(c);
    }
}

constexpr int kExpNone = 1 << 20; // zero or non-finite entry: contributes no tiny product

// floor(log2 |v|) of a finite nonzero v (subnormals included), kExpNone for zero and
// non-finite values. Branch-free: the exponent screen applies it to every element of both
// operands.
__device__ __forceinline__ int ilog2_abs(float v)
{
    const uint32_t b = bits_of(v) & 0x7fffffffu, e = b >> 23;
    const int sub = (31 - __clz(b | 1u)) - 149; // e == 0: b is the fraction
    const int r = e ? (int)e - 127 : sub;
    return (e == 0xff || b == 0) ? kExpNone : r;
}
__device__ __forceinline__ int ilog2_abs(double v)
{
    const uint64_t b = bits_of(v) & 0x7fffffffffffffffull, e = b >> 52;
    const int sub = (63 - __clzll(b | 1ull)) - 1074;
    const int r = e ? (int)e - 1023 : sub;
    return (e == 0x7ff || b == 0) ? kExpNone : r;
}
// A superslab table entry from a folded exponent, and back.
__device__ __forceinline__ short scan_exp(int e) { return (short)(e == kExpNone ? kScanExpNone : e); }
__device__ __forceinline__ int unscan_exp(short t) { return t == kScanExpNone ? kExpNone : (int)t; }

// Gating of the partial-sum check in a checking tile, by superslab (64 k). Products of at
// least 2^thr (thr = -103, binary64 -970), and zero, are multiples of the smallest normal
// 2^-126 (2^-1022), and so is every rounded sum of such multiples: a partial sum can only be
// a nonzero subnormal in a superslab that holds a product below 2^thr ("fine" by the screen's
// tables: the tile's smallest op(A) row exponent plus smallest op(B) column exponent over
// the superslab is below thr), or in a later one that a sum which is not such a multiple
// enters (such sums are below 2^-103, 2^-970 in magnitude). So superslab s is checked when it
// is fine, or when s - 1 was checked and one of the wave's partial sums is nonzero and below
// 2^-102 (2^-969) at its start; every other superslab begins and ends on multiples.
// Without tables every slab is checked.
constexpr int kSumMaxSuperSlabs = 1024; // K of at most 65536 when there are tables

// fine[s] for the tile's superslabs from the tables: block-wide, ends with a barrier.
template <int BM, int BN>
__device__ __forceinline__ void tile_fine_superslabs(const SumCheck &sck, int m0, int n0, int M,
                                                     int N, int K, unsigned char *fine)
{
    const int nss = (K + 63) / 64;
    const int lane = threadIdx.x & 63, waves = blockDim.x >> 6;
    for (int s = (int)(threadIdx.x >> 6); s < nss; s += waves) {
        int ea = kScanExpNone, eb = kScanExpNone;
        for (int i = lane; i < BM; i += 64)
            if (m0 + i < M) {
                const int v = sck.a_xmajor ? sck.tbl_a[(size_t)(m0 + i) * nss + s]
                                           : sck.tbl_a[(size_t)s * M + m0 + i];
                ea = v < ea ? v : ea;
            }
        for (int i = lane; i < BN; i += 64)
            if (n0 + i < N) {
                const int v = sck.b_xmajor ? sck.tbl_b[(size_t)(n0 + i) * nss + s]
                                           : sck.tbl_b[(size_t)s * N + n0 + i];
                eb = v < eb ? v : eb;
            }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const int oa = __shfl_xor(ea, off, 64), ob = __shfl_xor(eb, off, 64);
            ea = oa < ea ? oa : ea;
            eb = ob < eb ? ob : eb;
        }
        if (lane == 0)
            fine[s] = ea + eb < sck.thr;
    }
    __syncthreads();
}

// A partial sum that may not be a multiple of the smallest normal: nonzero and below 2^-102
// (binary64 2^-969).
__device__ __forceinline__ bool sum_off_grid(float v)
{
    return (bits_of(v) & 0x7fffffffu) - 1u < 0x0C7FFFFFu;
}
__device__ __forceinline__ bool sum_off_grid(double v)
{
    return (bits_of(v) & 0x7fffffffffffffffull) - 1ull < (54ull << 52) - 1ull;
}

// The wave's gate over slabs of BK k; slabs are presented in order from 0.
template <int BK> struct SumGate {
    static_assert(64 % BK == 0, "a slab lies in one superslab");
    static constexpr int kPer = 64 / BK;
    const unsigned char *fine; // LDS; null: check every slab
    bool chk;
    // Whether slab kt is checked. off_grid() reports whether one of the wave's partial sums
    // is off the grid of multiples (uniform over the wave); it is called only at the start of
    // a superslab that follows a checked one and is not fine itself.
    template <class F> __device__ __forceinline__ bool at(int kt, F &&off_grid)
    {
        if (fine == nullptr)
            return true;
        if (kt % kPer == 0) {
            bool c = __builtin_amdgcn_readfirstlane(fine[kt / kPer]) != 0;
            if (!c && chk)
                c = off_grid();
            chk = c;
        }
        return chk;
    }
};

// The partial-sum block word of output cell (row, col).
__device__ __forceinline__ void flag_sum_block(const SumCheck &sck, int row, int col)
{
    sck.flag[(size_t)(row >> 5) * sck.blocks_n + (uint32_t)(col >> 5)] = sck.gen;
}

// Record the wave's earliest packed fault with one atomic. `key` is kNoFault on lanes
// without a fault; the ballot keeps the fault-free path to one instruction. A fault word
// (as opposed to a scratch word such as the MatMul's first suspect cell) also closes the
// stage gate for later nodes.
__device__ __forceinline__ void wave_record_fault(uint64_t key, unsigned long long *word,
                                                  const NodeGate &gate = NodeGate{nullptr, 0})
{
    if (__ballot(key != kNoFault) == 0)
        return;
    uint64_t m = wave_min_u64(key);
    if (__lane_id() == 0) {
        atomicMin(word, (unsigned long long)m);
        gate_record(gate);
    }
}

// Record the workgroup's earliest key with one atomic: every thread of a workgroup of NW
// waves calls it (it holds a barrier). A MatMul tile with a NaN operand marks whole rows or
// columns suspect, and one atomic a wave on the one word then queues every wave of the grid
// behind the others (binary32 MFMA tiles, 16 waves a workgroup at 1024^3: 134 us a call
// against 91). The binary64 VALU tiles keep one atomic a wave: the barrier measured 13-15%
// slower there at every size, clean or not.
template <int NW> __device__ __forceinline__ void block_record_min(uint64_t key, unsigned long long *word)
{
    __shared__ unsigned long long wave_key[NW];
    const uint64_t wk = __ballot(key != kNoFault) ? wave_min_u64(key) : kNoFault;
    if (__lane_id() == 0)
        wave_key[threadIdx.x / 64] = wk;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long m = wave_key[0];
#pragma unroll
        for (int w = 1; w < NW; w++)
            m = wave_key[w] < m ? wave_key[w] : m;
        if (m != kNoFault)
            atomicMin(word, m);
    }
}

} // namespace pcu
