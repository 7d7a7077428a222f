// Strict F32/F64 MatMul for gfx950.
//
// Contract (core/dialect/tensor/reference/strict_matmul/strict_matmul.rs:22-73): each
// output cell starts from +0 and walks k in increasing order, rounding the product and
// then the sum on their own (no FMA, no MFMA, no reassociation). The first fault is the
// lowest (row-major cell, k, Multiply before Add).
//
// Three launches:
//  1. prefilter   per-row minimum exponent of op(A) and per-column minimum exponent of
//                 op(B) over finite nonzero entries (bandwidth-bound, ~2 reads of A and B).
//  2. main        LDS-staged 128x128 output tile per 256-thread workgroup, 8x8 register
//                 block per thread, k in order with separate v_mul/v_add. The epilogue
//                 marks a cell suspect when its result is non-finite (the only trace an
//                 invalid operand or an overflow leaves) or when the two exponents allow a
//                 product small enough to be tiny (the only way an underflow can arise),
//                 and keeps the first suspect cell with one atomicMin per wave.
//  3. replay      exact ordered re-execution of suspect cells in row-major order from the
//                 first suspect, with per-op classification; stops once the earliest fault
//                 found lies before the cells still to visit. Returns at once when no cell
//                 is suspect, which is the fault-free path.
#include "pcu_device.hpp"
#include "pcu_gemm_stage.hpp"
#include "pcu_kernels.hpp"

#include <limits.h>

#pragma clang fp contract(off)

namespace pcu {

constexpr int kExpNone = 1 << 20; // zero or non-finite entry: contributes no tiny product

// Branch-free: the prefilter applies it to every element of both operands.
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

__device__ __forceinline__ int wave_min_i32(int v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        int o = __shfl_xor(v, off, 64);
        v = o < v ? o : v;
    }
    return v;
}

// Minimum exponents for the underflow screen, one entry per row of op(A) and per column of
// op(B). Depending on the transposes, each is the minimum over a row or over a column of a
// stored matrix. An entry is a 64-bit word (generation << 32) | (kExpBias - e): the column
// jobs fold their 64-row groups with atomicMax, under which a word of the current MatMul
// (larger generation) replaces any older one and, within it, the largest kExpBias - e is the
// smallest e. So no entry needs opening before the screen, and both jobs of a MatMul run in
// one launch. Readers take e = kExpBias - (low 32 bits).

// One exponent job: per-row minima of a stored R x C matrix (rows) or per-column (cols).
template <typename T> struct ExpJob {
    const T *X;
    uint64_t R, C;
    bool rows;
    bool vec; // C a multiple of 16 bytes and X 16-byte aligned
    unsigned long long *out;
};

// Rows job, block `bid`: one wave per row, four rows per 256-thread block; four 16-byte loads
// per lane in flight.
template <typename T, bool VEC>
__device__ __forceinline__ void exp_rows_block(const ExpJob<T> &j, uint64_t bid, uint32_t gen)
{
    const uint64_t r = bid * 4 + threadIdx.x / 64;
    if (r >= j.R)
        return; // whole wave exits together
    const int lane = threadIdx.x % 64;
    const uint64_t C = j.C;
    int m = kExpNone;
    const T *row = j.X + r * C;
    if (VEC) {
        constexpr int P = 16 / sizeof(T);
        constexpr uint64_t S = 64 * P; // elements one pass of the wave covers
        constexpr int U = 4;
        uint64_t c = (uint64_t)lane * P;
        for (; c + (U - 1) * S < C; c += U * S) {
            uint4 q[U];
#pragma unroll
            for (int u = 0; u < U; u++)
                q[u] = *reinterpret_cast<const uint4 *>(row + c + u * S);
#pragma unroll
            for (int u = 0; u < U; u++) {
                const T *v = reinterpret_cast<const T *>(&q[u]);
#pragma unroll
                for (int k = 0; k < P; k++) {
                    const int e = ilog2_abs(v[k]);
                    m = e < m ? e : m;
                }
            }
        }
        for (; c < C; c += S) {
            const uint4 q = *reinterpret_cast<const uint4 *>(row + c);
            const T *v = reinterpret_cast<const T *>(&q);
#pragma unroll
            for (int k = 0; k < P; k++) {
                const int e = ilog2_abs(v[k]);
                m = e < m ? e : m;
            }
        }
    } else {
        for (uint64_t c = lane; c < C; c += 64) {
            const int e = ilog2_abs(row[c]);
            m = e < m ? e : m;
        }
    }
    m = wave_min_i32(m);
    if (lane == 0)
        j.out[r] = exp_word(gen, m);
}

// Columns job, block `bid` = (column block cb, 64-row group rg): 64 column-runs (16 bytes
// each) by 4 row groups of 16 rows; the row groups meet in LDS and the block folds its
// minimum into out with one atomicMax per column. Fewer rows per block measured slower: the
// atomics on one column then contend.
template <typename T, bool VEC>
__device__ __forceinline__ void exp_cols_block(const ExpJob<T> &j, uint64_t bid, uint32_t gen,
                                               int (*part)[64 * 16 / sizeof(T)])
{
    constexpr int P = VEC ? 16 / sizeof(T) : 1;
    const uint64_t R = j.R, C = j.C, ncb = (C + 64 * P - 1) / (64 * P);
    const uint64_t cb = bid % ncb, rg = bid / ncb;
    const int cx = threadIdx.x % 64, ry = threadIdx.x / 64;
    const uint64_t c0 = (cb * 64 + cx) * P;
    const uint64_t r0 = rg * 64;
    const uint64_t r1 = r0 + 64 < R ? r0 + 64 : R;
    const T *X = j.X;
    int m[P];
#pragma unroll
    for (int k = 0; k < P; k++)
        m[k] = kExpNone;
    if (c0 < C) {
        uint64_t r = r0 + ry;
        if (VEC) {
            // Four rows per step: four 16-byte loads per thread in flight.
            for (; r + 12 < r1; r += 16) {
                uint4 q[4];
#pragma unroll
                for (int u = 0; u < 4; u++)
                    q[u] = *reinterpret_cast<const uint4 *>(X + (r + 4 * u) * C + c0);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const T *v = reinterpret_cast<const T *>(&q[u]);
#pragma unroll
                    for (int k = 0; k < P; k++) {
                        const int e = ilog2_abs(v[k]);
                        m[k] = e < m[k] ? e : m[k];
                    }
                }
            }
        }
        for (; r < r1; r += 4) {
            const T *p = X + r * C + c0;
            if (VEC) {
                const uint4 q = *reinterpret_cast<const uint4 *>(p);
                const T *v = reinterpret_cast<const T *>(&q);
#pragma unroll
                for (int k = 0; k < P; k++) {
                    const int e = ilog2_abs(v[k]);
                    m[k] = e < m[k] ? e : m[k];
                }
            } else {
                const int e = ilog2_abs(p[0]);
                m[0] = e < m[0] ? e : m[0];
            }
        }
    }
#pragma unroll
    for (int k = 0; k < P; k++)
        part[ry][cx * P + k] = m[k];
    __syncthreads();
    if (ry == 0 && c0 < C) {
#pragma unroll
        for (int k = 0; k < P; k++) {
            int v = part[0][cx * P + k];
            for (int g = 1; g < 4; g++)
                v = part[g][cx * P + k] < v ? part[g][cx * P + k] : v;
            atomicMax(&j.out[c0 + k], exp_word(gen, v));
        }
    }
}

template <typename T> __host__ __device__ inline uint64_t exp_blocks(const ExpJob<T> &j)
{
    if (j.rows)
        return (j.R + 3) / 4;
    const uint64_t P = j.vec ? 16 / sizeof(T) : 1;
    return ((j.C + 64 * P - 1) / (64 * P)) * ((j.R + 63) / 64);
}

// Both jobs of a MatMul in one launch: blocks [0, na) run job a, the rest job b. A block's
// branches are uniform, so the columns job's barrier is reached by all of its threads. The
// launch also clears the MatMul's first-suspect word.
template <typename T>
__global__ __launch_bounds__(256) void k_exp_screen(ExpJob<T> a, ExpJob<T> b, uint64_t na,
                                                    uint32_t gen, unsigned long long *suspect,
                                                    NodeGate gate)
{
    __shared__ int part[4][64 * 16 / sizeof(T)];
    if (block_gate_closed(gate))
        return;
    if (blockIdx.x == 0 && threadIdx.x == 0)
        *suspect = kNoFault;
    const bool first = blockIdx.x < na;
    const ExpJob<T> &j = first ? a : b;
    const uint64_t bid = first ? blockIdx.x : blockIdx.x - na;
    if (j.rows) {
        if (j.vec)
            exp_rows_block<T, true>(j, bid, gen);
        else
            exp_rows_block<T, false>(j, bid, gen);
    } else {
        if (j.vec)
            exp_cols_block<T, true>(j, bid, gen, part);
        else
            exp_cols_block<T, false>(j, bid, gen, part);
    }
}

__global__ void k_fill_i32(int *p, uint64_t n, int v)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

__global__ void k_fill_u32(unsigned int *p, uint64_t n, unsigned int v)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

__global__ void k_fill_u64(unsigned long long *p, uint64_t n, unsigned long long v)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// ------------------------------------------------------------------- main tile

constexpr int BM = 128, BN = 128; // output tile of every MatMul kernel here

// Tile shape of the vector-unit kernel: 128 x 128 outputs per 256-thread workgroup (8 x 8
// per thread); binary64 stages twice as deep a k-slab, halving its barriers.
template <typename T> struct ValuCfg {
    static constexpr int BM = 128, BN = 128, BK = sizeof(T) == 4 ? 8 : 16;
    static constexpr int kThreads = 256;
    static constexpr int LDA = BM + 4, LDB = BN + 4; // row pitch of the k-major LDS stages
    static constexpr int EA = BM * BK / kThreads, EB = BN * BK / kThreads;
    // Binary64 splits a thread's 8 elements of a B k-row into 16-byte runs 32 apart when A
    // is untransposed (1.3-2% faster at 4096^3 and 2048x4096x2048) and keeps one contiguous
    // run under a transposed A (splitting measured 2.5% slower there).
    template <bool TA> static constexpr bool kSplitRunsB = sizeof(T) == 8 && !TA;
};

// NATIVE (explicitly permitted native compound arithmetic): one fused multiply-add per
// (cell, k) and no fault screen.
// WHOLE: every slab of every tile is whole (see the MFMA kernel).
template <typename T, bool TA, bool TB, bool VA, bool VB, bool NATIVE = false, bool WHOLE = false>
__global__ __launch_bounds__(256, 2) void k_strict_gemm(
    const T *__restrict__ A, const T *__restrict__ B, T *__restrict__ C, int M, int N, int K,
    const unsigned long long *__restrict__ row_exp, const unsigned long long *__restrict__ col_exp,
    int thr, int check_risk, int vec_c, unsigned long long *suspect, NodeGate gate)
{
    if (block_gate_closed(gate))
        return;
    using Cfg = ValuCfg<T>;
    constexpr int BK = Cfg::BK;
    // Reading each k row's operands one row ahead measured 2-8% faster with a transposed
    // operand or a partial tile, and 3-9% slower for whole untransposed binary64 tiles.
    constexpr bool kAhead = TA || TB || !WHOLE;
    __shared__ __align__(16) T As[2][BK][Cfg::LDA];
    __shared__ __align__(16) T Bs[2][BK][Cfg::LDB];

    const int tid = threadIdx.x;
    const int tx = tid % 16, ty = tid / 16;
    // The lane's 8 columns come in RUN adjacent columns per run: binary32 lanes own 2 runs
    // of 4 (64 columns apart), binary64 lanes 4 runs of 2 (32 apart), so that each 16-byte
    // LDS read of B covers 256 contiguous bytes over the 16 lanes of a row (no bank
    // conflicts) and each 16-byte store is coalesced the same way.
    constexpr int RUN = 16 / sizeof(T), RUNS = 8 / RUN, RUN_STRIDE = BN / RUNS;
    auto col_of = [&](int j) { return (j / RUN) * RUN_STRIDE + tx * RUN + (j % RUN); };

    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tile_m, tile_n;
    tile_of(blockIdx.x, tiles_m, tiles_n, tile_m, tile_n);
    const int m0 = tile_m * BM, n0 = tile_n * BN;

    T acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 8; j++)
            acc[i][j] = (T)0;

    SlabStager<T, Cfg, TA, TB, VA, VB> stage;

    const int ktiles = (K + BK - 1) / BK;
    if (WHOLE)
        stage.begin_whole(A, B, M, N, K, m0, n0, tid);
    if (ktiles > 0) {
        if (WHOLE)
            stage.fetch_whole();
        else
            stage.fetch(A, B, M, N, K, m0, n0, 0, tid);
        stage.stash(As[0], Bs[0], tid);
    }
    __syncthreads();
    for (int kt = 0; kt < ktiles; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < ktiles) {
            if (WHOLE)
                stage.fetch_whole();
            else
                stage.fetch(A, B, M, N, K, m0, n0, (kt + 1) * BK, tid);
        }
        if constexpr (kAhead) {
            // The slab is unrolled; row k + 1's operands are read from LDS into the other
            // register set before row k is computed, and sched_barrier keeps the reads
            // there. Binary64 forms products 4 at a time to stay within two waves' registers.
            constexpr int PB = sizeof(T) == 8 ? 4 : 8;
            T a[2][8], b[2][8];
            auto rd = [&](int k) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    a[k & 1][i] = As[cur][k][ty * 4 + i];
                    a[k & 1][4 + i] = As[cur][k][64 + ty * 4 + i];
                }
#pragma unroll
                for (int j = 0; j < 8; j++)
                    b[k & 1][j] = Bs[cur][k][col_of(j)];
            };
            rd(0);
#pragma unroll
            for (int k = 0; k < BK; k++) {
                if (k + 1 < BK)
                    rd(k + 1);
                __builtin_amdgcn_sched_barrier(0);
                const T(&x)[8] = a[k & 1];
                const T(&y)[8] = b[k & 1];
                // Per row, the products first and then their sums: no add waits on the
                // multiply just before it.
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if (NATIVE) {
#pragma unroll
                        for (int j = 0; j < 8; j++)
                            acc[i][j] = fma(x[i], y[j], acc[i][j]);
                    } else {
#pragma unroll
                        for (int h = 0; h < 8; h += PB) {
                            T p[PB];
#pragma unroll
                            for (int j = 0; j < PB; j++)
                                p[j] = x[i] * y[h + j];
#pragma unroll
                            for (int j = 0; j < PB; j++)
                                acc[i][h + j] = acc[i][h + j] + p[j];
                        }
                    }
                    // Emits nothing; ties the row's eight sums to this point of the stream.
                    asm volatile("" : "+v"(acc[i][0]), "+v"(acc[i][1]), "+v"(acc[i][2]),
                                 "+v"(acc[i][3]), "+v"(acc[i][4]), "+v"(acc[i][5]),
                                 "+v"(acc[i][6]), "+v"(acc[i][7]));
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
#pragma unroll(sizeof(T) == 4 ? BK : 2)
            for (int k = 0; k < BK; k++) {
                T a[8], b[8];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    a[i] = As[cur][k][ty * 4 + i];
                    a[4 + i] = As[cur][k][64 + ty * 4 + i];
                }
#pragma unroll
                for (int j = 0; j < 8; j++)
                    b[j] = Bs[cur][k][col_of(j)];
                // Per row, the eight rounded products first and then the eight rounded sums:
                // no add waits on the multiply just before it (F64 measured 4% faster than
                // alternating multiply/add through one temporary).
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if (NATIVE) {
#pragma unroll
                        for (int j = 0; j < 8; j++)
                            acc[i][j] = fma(a[i], b[j], acc[i][j]);
                    } else {
                        T p[8];
#pragma unroll
                        for (int j = 0; j < 8; j++)
                            p[j] = a[i] * b[j];
#pragma unroll
                        for (int j = 0; j < 8; j++)
                            acc[i][j] = acc[i][j] + p[j];
                    }
                }
            }
        }
        if (kt + 1 < ktiles)
            stage.stash(As[cur ^ 1], Bs[cur ^ 1], tid);
        __syncthreads();
    }

    // Epilogue: publish the tile and find the first suspect cell of this lane.
    uint64_t key = kNoFault;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int r = m0 + (i < 4 ? ty * 4 + i : 64 + ty * 4 + (i - 4));
        if (r >= M)
            continue;
        int rexp = check_risk ? exp_of(row_exp[r]) : 0;
#pragma unroll
        for (int h = 0; h < RUNS; h++) {
            int c0 = n0 + col_of(h * RUN);
            T *dst = C + (size_t)r * N + c0;
            if (vec_c && c0 + RUN <= N) {
                if (sizeof(T) == 4)
                    *reinterpret_cast<float4 *>(dst) =
                        make_float4(acc[i][h * 4], acc[i][h * 4 + 1], acc[i][h * 4 + 2], acc[i][h * 4 + 3]);
                else
                    *reinterpret_cast<double2 *>(dst) = make_double2(acc[i][h * 2], acc[i][h * 2 + 1]);
            } else {
#pragma unroll
                for (int j = 0; j < RUN; j++)
                    if (c0 + j < N)
                        dst[j] = acc[i][h * RUN + j];
            }
#pragma unroll
            for (int j = 0; j < RUN; j++) {
                int c = c0 + j;
                if (NATIVE || c >= N)
                    continue;
                bool bad = !finite_bits(acc[i][h * RUN + j]);
                if (check_risk)
                    bad |= rexp + exp_of(col_exp[c]) < thr;
                if (bad) {
                    uint64_t cell = (uint64_t)r * N + c;
                    key = cell < key ? cell : key;
                }
            }
        }
    }
    if (!NATIVE)
        wave_record_fault(key, suspect);
}

// --------------------------------------------------------------- exact replay

template <typename T>
__global__ __launch_bounds__(256) void k_strict_gemm_replay(
    const T *__restrict__ A, const T *__restrict__ B, const T *__restrict__ C, uint64_t M,
    uint64_t N, uint64_t K, int ta, int tb, const unsigned long long *__restrict__ row_exp,
    const unsigned long long *__restrict__ col_exp, int thr, int check_risk, int policy,
    const unsigned long long *suspect, unsigned long long *fault, NodeGate gate)
{
    if (block_gate_closed(gate))
        return; // an earlier node faulted: that fault is the one reported
    const uint64_t first = *suspect;
    if (first == kNoFault)
        return;
    const uint64_t cells = M * N;
    const uint64_t threads = (uint64_t)gridDim.x * blockDim.x;
    const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (uint64_t base = first; base < cells; base += threads) {
        uint64_t best = __atomic_load_n(fault, __ATOMIC_RELAXED);
        if (best != kNoFault && K > 0 && ((best >> 3) / 2) / K < base)
            break;
        uint64_t cell = base + tid;
        if (cell >= cells)
            break;
        uint64_t r = cell / N, c = cell % N;
        bool bad = !finite_bits(C[cell]);
        if (check_risk)
            bad |= exp_of(row_exp[r]) + exp_of(col_exp[c]) < thr;
        if (!bad)
            continue;
        T total = (T)0;
        for (uint64_t k = 0; k < K; k++) {
            T a = ta ? A[k * M + r] : A[r * K + k];
            T b = tb ? B[c * K + k] : B[k * N + c];
            T p = a * b;
            uint32_t kind = classify_mul(a, b, p, policy);
            if (kind != kOk) {
                atomicMin(fault, (unsigned long long)pack_fault((cell * K + k) * 2, kind));
                gate_record(gate);
                break;
            }
            T nxt = total + p;
            kind = classify_add(total, p, nxt, policy);
            if (kind != kOk) {
                atomicMin(fault, (unsigned long long)pack_fault((cell * K + k) * 2 + 1, kind));
                gate_record(gate);
                break;
            }
            total = nxt;
        }
    }
}

// ================================================================= launchers

size_t matmul_scratch_bytes(uint64_t rows, uint64_t cols)
{
    size_t r = ((rows * sizeof(unsigned long long)) + 255) & ~(size_t)255;
    size_t c = ((cols * sizeof(unsigned long long)) + 255) & ~(size_t)255;
    return r + c + 256;
}

MatmulScratch matmul_scratch_carve(void *base, uint64_t rows, uint64_t cols)
{
    char *p = (char *)base;
    size_t r = ((rows * sizeof(unsigned long long)) + 255) & ~(size_t)255;
    size_t c = ((cols * sizeof(unsigned long long)) + 255) & ~(size_t)255;
    MatmulScratch s;
    s.row_exp = (unsigned long long *)p;
    s.col_exp = (unsigned long long *)(p + r);
    s.suspect = (unsigned long long *)(p + r + c);
    return s;
}

hipError_t launch_fill_u64(hipStream_t s, unsigned long long *p, uint64_t n, uint64_t value)
{
    if (n == 0)
        return hipSuccess;
    unsigned grid = (unsigned)((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024);
    hipLaunchKernelGGL(k_fill_u64, dim3(grid), dim3(256), 0, s, p, n, (unsigned long long)value);
    return hipGetLastError();
}

__global__ void k_program_open(unsigned long long *words, uint64_t n, unsigned long long value,
                               unsigned int *gate)
{
    const uint64_t i0 = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (uint64_t i = i0; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        words[i] = value;
    if (i0 == 0)
        *gate = 0xffffffffu;
}

hipError_t launch_program_open(hipStream_t s, unsigned long long *words, uint64_t n, uint64_t value,
                               unsigned int *gate)
{
    unsigned grid = (unsigned)((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024);
    grid = grid ? grid : 1;
    hipLaunchKernelGGL(k_program_open, dim3(grid), dim3(256), 0, s, words, n, (unsigned long long)value, gate);
    return hipGetLastError();
}

hipError_t launch_fill_u32(hipStream_t s, unsigned int *p, uint64_t n, uint32_t value)
{
    if (n == 0)
        return hipSuccess;
    unsigned grid = (unsigned)((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024);
    hipLaunchKernelGGL(k_fill_u32, dim3(grid), dim3(256), 0, s, p, n, (unsigned int)value);
    return hipGetLastError();
}

static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// The exponent screen of op(A) rows and op(B) columns, both jobs in one launch.
template <typename T>
static void prefilter(hipStream_t s, ExpJob<T> ja, ExpJob<T> jb, uint32_t gen,
                      unsigned long long *suspect, NodeGate gate)
{
    for (ExpJob<T> *j : {&ja, &jb})
        j->vec = j->C % (16 / sizeof(T)) == 0 && aligned16(j->X);
    const uint64_t na = exp_blocks(ja), nb = exp_blocks(jb);
    hipLaunchKernelGGL(k_exp_screen<T>, dim3((unsigned)(na + nb)), dim3(256), 0, s, ja, jb, na, gen, suspect, gate);
}

template <typename T, bool TA, bool TB>
static void gemm_dispatch(hipStream_t s, dim3 grid, const T *A, const T *B, T *C, int M, int N,
                          int K, const unsigned long long *re, const unsigned long long *ce,
                          int thr, int risk, unsigned long long *suspect, NodeGate gate)
{
    bool va = (TA ? (M % 4 == 0) : (K % 4 == 0)) && aligned16(A);
    bool vb = (TB ? (K % 4 == 0) : (N % 4 == 0)) && aligned16(B);
    int vc = (N % 4 == 0) && aligned16(C);
    using Cfg = ValuCfg<T>;
    if (va && vb && M % Cfg::BM == 0 && N % Cfg::BN == 0 && K % Cfg::BK == 0)
        hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, true, true, false, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, gate);
    else if (va && vb)
        hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, true, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, gate);
    else if (va)
        hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, true, false>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, gate);
    else if (vb)
        hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, false, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, gate);
    else
        hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, false, false>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, gate);
}

template <typename T>
static hipError_t strict_matmul_t(hipStream_t s, uint64_t M, uint64_t K, uint64_t N, bool ta,
                                  bool tb, const T *A, const T *B, T *C, int policy,
                                  MatmulScratch sc, unsigned long long *fault, NodeGate gate,
                                  hipEvent_t *ev, int engine)
{
    if (M == 0 || N == 0)
        return hipSuccess;
    // Smallest exponent sum of a product that needs no replay (see pcu_device.hpp):
    // IEEE: a product >= 2^-126 (2^-1022) is never tiny; RejectSubnormal: products
    // >= 2^-103 (2^-970) are multiples of the smallest normal, so no partial sum is
    // subnormal; AllowGradual: underflow is never a fault.
    const bool f32 = sizeof(T) == 4;
    int risk = policy != kPolicyAllowGradual;
    int thr = policy == kPolicyRejectSubnormal ? (f32 ? -103 : -970) : (f32 ? -126 : -1022);
    if (ev)
        (void)hipEventRecord(ev[0], s);
    if (risk && K > 0) {
        // op(A) row r is stored row r (A is M x K) or stored column r (A is K x M); op(B)
        // column c is stored column c (B is K x N) or stored row c (B is N x K).
        const ExpJob<T> ja{A, ta ? K : M, ta ? M : K, !ta, false, sc.row_exp};
        const ExpJob<T> jb{B, tb ? N : K, tb ? K : N, tb, false, sc.col_exp};
        prefilter<T>(s, ja, jb, sc.gen, sc.suspect, gate);
    } else {
        risk = 0; // AllowGradual, or an empty reduction: no underflow screen
        hipLaunchKernelGGL(k_fill_u64, dim3(1), dim3(64), 0, s, sc.suspect, (uint64_t)1, (unsigned long long)kNoFault);
    }
    dim3 grid((unsigned)(((M + BM - 1) / BM) * ((N + BN - 1) / BN)));
    const int m = (int)M, n = (int)N, k = (int)K;
    if (ev)
        (void)hipEventRecord(ev[1], s);
    if (f32 && engine != kEngineValu) {
        (void)launch_gemm_mfma_f32(s, m, n, k, ta, tb, (const float *)A, (const float *)B,
                                   (float *)C, sc.row_exp, sc.col_exp, thr, risk, sc.suspect, gate);
    } else if (!ta && !tb) gemm_dispatch<T, false, false>(s, grid, A, B, C, m, n, k, sc.row_exp, sc.col_exp, thr, risk, sc.suspect, gate);
    else if (!ta && tb) gemm_dispatch<T, false, true>(s, grid, A, B, C, m, n, k, sc.row_exp, sc.col_exp, thr, risk, sc.suspect, gate);
    else if (ta && !tb) gemm_dispatch<T, true, false>(s, grid, A, B, C, m, n, k, sc.row_exp, sc.col_exp, thr, risk, sc.suspect, gate);
    else gemm_dispatch<T, true, true>(s, grid, A, B, C, m, n, k, sc.row_exp, sc.col_exp, thr, risk, sc.suspect, gate);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    if (ev)
        (void)hipEventRecord(ev[2], s);
    hipLaunchKernelGGL(k_strict_gemm_replay<T>, dim3(1024), dim3(256), 0, s, A, B, (const T *)C, M, N, K,
                       (int)ta, (int)tb, sc.row_exp, sc.col_exp, thr, risk, policy,
                       (const unsigned long long *)sc.suspect, fault, gate);
    if (ev)
        (void)hipEventRecord(ev[3], s);
    return hipGetLastError();
}

template <bool TA, bool TB>
static void native_f64_dispatch(hipStream_t s, dim3 grid, const double *A, const double *B,
                                double *C, int M, int N, int K, NodeGate gate)
{
    const bool va = (TA ? (M % 4 == 0) : (K % 4 == 0)) && aligned16(A);
    const bool vb = (TB ? (K % 4 == 0) : (N % 4 == 0)) && aligned16(B);
    const int vc = (N % 4 == 0) && aligned16(C);
    using Cfg = ValuCfg<double>;
    if (va && vb && M % Cfg::BM == 0 && N % Cfg::BN == 0 && K % Cfg::BK == 0)
        hipLaunchKernelGGL((k_strict_gemm<double, TA, TB, true, true, true, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, nullptr, nullptr, 0, 0, vc, nullptr, gate);
    else if (va && vb)
        hipLaunchKernelGGL((k_strict_gemm<double, TA, TB, true, true, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, nullptr, nullptr, 0, 0, vc, nullptr, gate);
    else if (va)
        hipLaunchKernelGGL((k_strict_gemm<double, TA, TB, true, false, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, nullptr, nullptr, 0, 0, vc, nullptr, gate);
    else if (vb)
        hipLaunchKernelGGL((k_strict_gemm<double, TA, TB, false, true, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, nullptr, nullptr, 0, 0, vc, nullptr, gate);
    else
        hipLaunchKernelGGL((k_strict_gemm<double, TA, TB, false, false, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, nullptr, nullptr, 0, 0, vc, nullptr, gate);
}

hipError_t launch_native_matmul(hipStream_t s, int dtype, uint64_t rows, uint64_t inner,
                                uint64_t cols, bool ta, bool tb, const void *a, const void *b,
                                void *c, NodeGate gate)
{
    if (rows > (uint64_t)INT_MAX || cols > (uint64_t)INT_MAX || inner > (uint64_t)INT_MAX)
        return hipErrorInvalidValue;
    if (rows == 0 || cols == 0)
        return hipSuccess;
    const int M = (int)rows, N = (int)cols, K = (int)inner;
    if (dtype == 0)
        return launch_native_gemm_f32(s, M, N, K, ta, tb, (const float *)a, (const float *)b, (float *)c, gate);
    const dim3 grid((unsigned)(((rows + BM - 1) / BM) * ((cols + BN - 1) / BN)));
    const double *A = (const double *)a, *B = (const double *)b;
    double *C = (double *)c;
    if (!ta && !tb) native_f64_dispatch<false, false>(s, grid, A, B, C, M, N, K, gate);
    else if (!ta && tb) native_f64_dispatch<false, true>(s, grid, A, B, C, M, N, K, gate);
    else if (ta && !tb) native_f64_dispatch<true, false>(s, grid, A, B, C, M, N, K, gate);
    else native_f64_dispatch<true, true>(s, grid, A, B, C, M, N, K, gate);
    return hipGetLastError();
}

hipError_t launch_strict_matmul(hipStream_t s, int dtype, uint64_t rows, uint64_t inner,
                                uint64_t cols, bool transpose_left, bool transpose_right,
                                const void *a, const void *b, void *c, int policy,
                                MatmulScratch scratch, unsigned long long *fault, NodeGate gate,
                                hipEvent_t *ev, int engine)
{
    if (rows > (uint64_t)INT_MAX || cols > (uint64_t)INT_MAX || inner > (uint64_t)INT_MAX)
        return hipErrorInvalidValue;
    if (dtype == 0)
        return strict_matmul_t<float>(s, rows, inner, cols, transpose_left, transpose_right,
                                      (const float *)a, (const float *)b, (float *)c, policy,
                                      scratch, fault, gate, ev, engine);
    return strict_matmul_t<double>(s, rows, inner, cols, transpose_left, transpose_right,
                                   (const double *)a, (const double *)b, (double *)c, policy,
                                   scratch, fault, gate, ev, kEngineValu);
}

} // namespace pcu
