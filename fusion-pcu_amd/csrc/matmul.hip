// Strict F32/F64 MatMul for gfx950.
//
// Contract (core/dialect/tensor/reference/strict_matmul/strict_matmul.rs:22-73): each
// output cell starts from +0 and walks k in increasing order, rounding the product and
// then the sum on their own (no FMA, no MFMA, no reassociation). The first fault is the
// lowest (row-major cell, k, Multiply before Add).
//
// Four launches:
//  1. prefilter   per-row minimum exponent of op(A) and per-column minimum exponent of
//                 op(B) over finite nonzero entries (bandwidth-bound, ~2 reads of A and B).
//  2. main        LDS-staged 128x128 output tile per 256-thread workgroup, 8x8 register
//                 block per thread, k in order with separate v_mul/v_add. The epilogue
//                 marks a cell suspect when its result is non-finite (the only trace an
//                 invalid operand or an overflow leaves) or when the two exponents allow a
//                 product small enough to be tiny (the only way an underflow can arise),
//                 and keeps the first suspect cell with one atomicMin per wave.
//  3. tiny scan   (IEEE policy, only when a cell is marked) a tiled pass over the tiles
//                 the screen marks, finding the cells that can have a tiny product from the
//                 smallest exponent sum over k (16-bit exponents, packed); see
//                 k_gemm_tiny_scan.
//  4. replay      exact ordered re-execution in row-major order from the first suspect:
//                 non-finite cells walked serially, per-op classified; cells the scan
//                 flagged have their K products classified in parallel by a wave. Both stop
//                 once the earliest fault found lies before the cells still to visit. The
//                 fault-free path returns at once.
// Small outputs (engine auto) take one fused launch instead, k_strict_gemm_fused: each
// 16 x 16 block screens its own rows and columns, computes its cells and searches its
// suspect cells exactly.
#include "pcu_device.hpp"
#include "pcu_gemm_stage.hpp"
#include "pcu_kernels.hpp"

#include <limits.h>

#pragma clang fp contract(off)

namespace pcu {


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
    // Optional superslab table: the smallest exponent (kScanExpNone for zero and non-finite
    // entries) of each entry's run of kSuperSlab k. A rows job (k along its rows) writes it
    // entry-major, tbl[row * ceil(C / kSuperSlab) + s]; a columns job (k down its columns)
    // superslab-major, tbl[s * C + column]. Null: no table.
    short *tbl;
    // A fold job: the entries' minima come from this table (laid out as `tbl` above, written
    // by the kernel that produced X) instead of from X, which is not read.
    const short *src = nullptr;
};

// Superslab of the tables above: 64 k, four slabs of the tiny scan, and the 64-row group of a
// columns-job block.
constexpr uint64_t kSuperSlab = 64;

// Rows job, block `bid`: one wave per row, four rows per 256-thread block; four 16-byte loads
// per lane in flight (sixteen measured 3-6% slower over whole screens).
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

// Rows job that also writes the row's superslab table: the same minima, from loops whose trip
// counts are uniform across the wave so the lanes of a superslab can fold their minima.
template <typename T, bool VEC>
__device__ __forceinline__ void exp_rows_block_tbl(const ExpJob<T> &j, uint64_t bid, uint32_t gen)
{
    const uint64_t r = bid * 4 + threadIdx.x / 64;
    if (r >= j.R)
        return; // whole wave exits together
    const int lane = threadIdx.x % 64;
    const uint64_t C = j.C, nss = (C + kSuperSlab - 1) / kSuperSlab;
    const T *row = j.X + r * C;
    short *trow = j.tbl + r * nss;
    int m = kExpNone;
    if (VEC) {
        constexpr int P = 16 / sizeof(T), L = (int)kSuperSlab / P; // lanes a superslab
        constexpr uint64_t S = 64 * P;
        constexpr int U = 4;
        for (uint64_t base = 0; base < C; base += U * S) {
            uint4 q[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const uint64_t c = base + u * S + (uint64_t)lane * P;
                q[u] = c < C ? *reinterpret_cast<const uint4 *>(row + c) : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const uint64_t c = base + u * S + (uint64_t)lane * P;
                const T *v = reinterpret_cast<const T *>(&q[u]);
                int e = kExpNone; // zeros past the end count as zero entries
#pragma unroll
                for (int k = 0; k < P; k++) {
                    const int x = ilog2_abs(v[k]);
                    e = x < e ? x : e;
                }
                m = e < m ? e : m;
#pragma unroll
                for (int off = 1; off < L; off <<= 1) {
                    const int o = __shfl_xor(e, off, 64);
                    e = o < e ? o : e;
                }
                if (lane % L == 0 && c < C)
                    trow[c / kSuperSlab] = (short)(e == kExpNone ? kScanExpNone : e);
            }
        }
    } else {
        for (uint64_t base = 0; base < C; base += 64) { // one superslab a trip
            const uint64_t c = base + lane;
            int e = c < C ? ilog2_abs(row[c]) : kExpNone;
            m = e < m ? e : m;
            e = wave_min_i32(e);
            if (lane == 0)
                trow[base / kSuperSlab] = (short)(e == kExpNone ? kScanExpNone : e);
        }
    }
    m = wave_min_i32(m);
    if (lane == 0)
        j.out[r] = exp_word(gen, m);
}

// Columns job, block `bid` = (column block cb, 64-row group rg): 64 column-runs (16 bytes
// each) by 4 row groups of 16 rows; the row groups meet in LDS and the block folds its
// minimum into out with one atomicMax per column. Fewer rows per block measured slower: the
// atomics on one column then contend. More measured slower too (128 or 256 rows: 4096^3 NN
// 28.1 -> 29.6 / 28.7 us, K = 1024 12.5 -> 14.0 / 18.7 us, binary64 48.0 -> 51.1 / 49.8 us),
// except when both jobs are column jobs (op(A) transposed: 34.7 -> 30.3 us).
constexpr uint64_t kColRows = 64; // rows of a columns-job block
static_assert(kColRows == kSuperSlab, "a columns-job block's rows are one superslab of k");

template <typename T, bool VEC>
__device__ __forceinline__ void exp_cols_block(const ExpJob<T> &j, uint64_t bid, uint32_t gen,
                                               int (*part)[64 * 16 / sizeof(T)])
{
    constexpr int P = VEC ? 16 / sizeof(T) : 1;
    const uint64_t R = j.R, C = j.C, ncb = (C + 64 * P - 1) / (64 * P);
    const uint64_t cb = bid % ncb, rg = bid / ncb;
    const int cx = threadIdx.x % 64, ry = threadIdx.x / 64;
    const uint64_t c0 = (cb * 64 + cx) * P;
    const uint64_t r0 = rg * kColRows;
    const uint64_t r1 = r0 + kColRows < R ? r0 + kColRows : R;
    const T *X = j.X;
    int m[P];
#pragma unroll
    for (int k = 0; k < P; k++)
        m[k] = kExpNone;
    if (c0 < C) {
        uint64_t r = r0 + ry;
        if (VEC) {
            // All sixteen of the thread's rows at once: sixteen 16-byte loads in flight (four
            // at a time measured 4-9% slower where both jobs are column jobs).
            for (; r + 60 < r1; r += 64) {
                uint4 q[16];
#pragma unroll
                for (int u = 0; u < 16; u++)
                    q[u] = *reinterpret_cast<const uint4 *>(X + (r + 4 * u) * C + c0);
#pragma unroll
                for (int u = 0; u < 16; u++) {
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
            // The block's rows are superslab rg of k.
            if (j.tbl && c0 + k < C)
                j.tbl[rg * C + c0 + k] = (short)(v == kExpNone ? kScanExpNone : v);
        }
    }
}

// Fold jobs. Rows: one wave per entry folds its row of the table (64 superslabs of a
// 4096-long k in one load a lane). Columns: 64 entries a block, the four waves taking every
// fourth superslab and meeting in LDS. Each word is written once, by a plain store.
template <typename T>
__device__ __forceinline__ void fold_rows_block(const ExpJob<T> &j, uint64_t bid, uint32_t gen)
{
    const uint64_t r = bid * 4 + threadIdx.x / 64;
    if (r >= j.R)
        return; // whole wave exits together
    const int lane = threadIdx.x % 64;
    const uint64_t nss = (j.C + kSuperSlab - 1) / kSuperSlab;
    const short *t = j.src + r * nss;
    int m = kExpNone;
    for (uint64_t k = lane; k < nss; k += 64) {
        const int e = unscan_exp(t[k]);
        m = e < m ? e : m;
    }
    m = wave_min_i32(m);
    if (lane == 0)
        j.out[r] = exp_word(gen, m);
}

template <typename T>
__device__ __forceinline__ void fold_cols_block(const ExpJob<T> &j, uint64_t bid, uint32_t gen,
                                                int (*part)[64 * 16 / sizeof(T)])
{
    const int cx = threadIdx.x % 64, q = threadIdx.x / 64;
    const uint64_t c = bid * 64 + cx, C = j.C;
    const uint64_t nss = (j.R + kSuperSlab - 1) / kSuperSlab;
    int m = kExpNone;
    if (c < C) {
        uint64_t k = q;
        for (; k + 60 < nss; k += 64) {
            short t[16];
#pragma unroll
            for (int u = 0; u < 16; u++)
                t[u] = j.src[(k + 4 * u) * C + c];
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const int e = unscan_exp(t[u]);
                m = e < m ? e : m;
            }
        }
        for (; k < nss; k += 4) {
            const int e = unscan_exp(j.src[k * C + c]);
            m = e < m ? e : m;
        }
    }
    part[q][cx] = m;
    __syncthreads();
    if (q == 0 && c < C) {
        for (int g = 1; g < 4; g++)
            m = part[g][cx] < m ? part[g][cx] : m;
        j.out[c] = exp_word(gen, m);
    }
}

template <typename T> __host__ __device__ inline uint64_t exp_blocks(const ExpJob<T> &j)
{
    if (j.src)
        return j.rows ? (j.R + 3) / 4 : (j.C + 63) / 64;
    if (j.rows)
        return (j.R + 3) / 4;
    const uint64_t P = j.vec ? 16 / sizeof(T) : 1;
    return ((j.C + 64 * P - 1) / (64 * P)) * ((j.R + kColRows - 1) / kColRows);
}

// Both jobs of a MatMul in one launch: blocks [0, na) run job a, the rest job b. A block's
// branches are uniform, so the columns job's barrier is reached by all of its threads. The
// launch also clears the MatMul's first-suspect word.
// Block 0 of a program's first kernel opens the program (see ProgramOpen).
__device__ __forceinline__ void program_open_block(const ProgramOpen &o)
{
    if (!o.words)
        return;
    for (uint64_t i = threadIdx.x; i < o.n; i += blockDim.x)
        o.words[i] = o.value;
    if (threadIdx.x == 0) {
        o.gate[0] = 0xffffffffu;
        o.gate[1] = 0u; // the ticket of an in-kernel program end (ProgramClose)
    }
}

template <typename T>
__global__ __launch_bounds__(256) void k_exp_screen(ExpJob<T> a, ExpJob<T> b, uint64_t na,
                                                    uint32_t gen, unsigned long long *suspect,
                                                    NodeGate gate, ProgramOpen open)
{
    __shared__ int part[4][64 * 16 / sizeof(T)];
    if (block_gate_closed(gate))
        return;
    if (blockIdx.x == 0) {
        program_open_block(open);
        if (threadIdx.x == 0) {
            suspect[0] = kNoFault; // first suspect cell
            suspect[1] = kNoFault; // first row with a cell the tiny scan flags
        }
    }
    const bool first = blockIdx.x < na;
    const ExpJob<T> &j = first ? a : b;
    const uint64_t bid = first ? blockIdx.x : blockIdx.x - na;
    if (j.src) {
        if (j.rows)
            fold_rows_block<T>(j, bid, gen);
        else
            fold_cols_block<T>(j, bid, gen, part);
    } else if (j.rows) {
        if (j.tbl) {
            if (j.vec)
                exp_rows_block_tbl<T, true>(j, bid, gen);
            else
                exp_rows_block_tbl<T, false>(j, bid, gen);
        } else if (j.vec) {
            exp_rows_block<T, true>(j, bid, gen);
        } else {
            exp_rows_block<T, false>(j, bid, gen);
        }
    } else {
        if (j.vec)
            exp_cols_block<T, true>(j, bid, gen, part);
        else
            exp_cols_block<T, false>(j, bid, gen, part);
    }
}

// The screen's place when there is nothing to screen: the suspect words, and the program.
__global__ void k_matmul_open(unsigned long long *suspect, ProgramOpen open)
{
    program_open_block(open);
    if (threadIdx.x == 0) {
        suspect[0] = kNoFault;
        suspect[1] = kNoFault;
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
constexpr unsigned kGfx950Cus = 256; // compute units of a gfx950 device (MI350X, MI355X)

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

// Direct global -> LDS load of 16 bytes a lane: lane l's run lands at lds + 16 l bytes (lds is
// the wave's base, uniform across the wave).
// Issued from inline assembly, so the compiler does not model it: as a builtin it counts as
// a second kind of LDS event, after which every LDS read waits for all reads before it
// (lgkmcnt(0)) instead of only the ones it needs. The caller waits for it (wait_lds_loads)
// before the barrier that publishes the stage.
__device__ __forceinline__ void load_lds16(const void *g, void *lds)
{
    const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)lds;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(base), "v"(g)
                 : "memory", "m0");
}
__device__ __forceinline__ void wait_lds_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// NATIVE (explicitly permitted native compound arithmetic): one fused multiply-add per
// (cell, k) and no fault screen.
// WHOLE: every slab of every tile is whole (see the MFMA kernel).
// CHECK: the RejectSubnormal form with the partial-sum check (sck), its own instantiation.
template <typename T, bool TA, bool TB, bool VA, bool VB, bool NATIVE = false, bool WHOLE = false,
          bool CHECK = false>
__global__ __launch_bounds__(256, 2) void k_strict_gemm(
    const T *__restrict__ A, const T *__restrict__ B, T *__restrict__ C, int M, int N, int K,
    const unsigned long long *__restrict__ row_exp, const unsigned long long *__restrict__ col_exp,
    int thr, int check_risk, int vec_c, unsigned long long *suspect, SumCheck sck, NodeGate gate)
{
    if (block_gate_closed(gate))
        return;
    using Cfg = ValuCfg<T>;
    constexpr int BK = Cfg::BK;
    // Reading each k row's operands one row ahead measured 2-8% faster with a transposed
    // operand or a partial tile, and 3-9% slower for whole untransposed binary64 tiles.
    constexpr bool kAhead = TA || TB || !WHOLE;
    // Binary64 whole tiles with op(B) untransposed move op(B), and op(A) when transposed, from
    // global memory straight into LDS (global_load_lds_dwordx4: each wave instruction fills
    // one 1 KiB k row of a stage, so the stages keep their padded k-major layout). Their two
    // stages are separate LDS objects indexed at compile time, so the compiler can tell a
    // direct load into one stage from the reads of the other.
    constexpr bool kDirect = sizeof(T) == 8 && WHOLE && !TB;
    __shared__ __align__(16) T As[2][BK][Cfg::LDA];
    __shared__ __align__(16) T Bs[2][BK][Cfg::LDB];
    __shared__ __align__(16) T A0[BK][Cfg::LDA], A1[BK][Cfg::LDA];
    __shared__ __align__(16) T B0[BK][Cfg::LDB], B1[BK][Cfg::LDB];

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
    // RejectSubnormal with the partial-sum check (sck.flag set) launches both forms over the
    // whole grid: a tile that may meet a product below 2^sck.thr is computed by the CHECK form,
    // which checks every partial sum it forms, and every other tile by the plain form.
    if (!NATIVE && sck.flag != nullptr &&
        tile_exp_sum_below<BM, BN>(row_exp, col_exp, m0, n0, M, N, sck.thr) != CHECK)
        return;
    SubLanes subl; // lanes that met a nonzero subnormal partial sum
    const int cls = kClassSubnormal;
    auto run_form = [&](auto &&run) { run(std::integral_constant<bool, CHECK && !NATIVE>{}); };
    // The checking form checks the superslabs that need it (SumGate).
    __shared__ unsigned char fine_ss[kSumMaxSuperSlabs];
    SumGate<BK> sgate{nullptr, false};
    bool chk = true; // the current slab's sums are checked (checking form)
    if constexpr (CHECK && !NATIVE) {
        if (sck.tbl_a != nullptr) {
            tile_fine_superslabs<BM, BN>(sck, m0, n0, M, N, K, fine_ss);
            sgate.fine = fine_ss;
        }
    }

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
    // One slab's products and sums from the stage (Ac, Bc).
    auto compute = [&](const T (*Ac)[Cfg::LDA], const T (*Bc)[Cfg::LDB], auto ck) __attribute__((always_inline)) {
        constexpr bool CK = decltype(ck)::value;
        if constexpr (kAhead) {
            // The slab is unrolled; row k + 1's operands are read from LDS into the other
            // register set before row k is computed, and sched_barrier keeps the reads
            // there. Binary64 forms products 4 at a time to stay within two waves' registers.
            constexpr int PB = sizeof(T) == 8 ? 4 : 8;
            T a[2][8], b[2][8];
            auto rd = [&](int k) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    a[k & 1][i] = Ac[k][ty * 4 + i];
                    a[k & 1][4 + i] = Ac[k][64 + ty * 4 + i];
                }
#pragma unroll
                for (int j = 0; j < 8; j++)
                    b[k & 1][j] = Bc[k][col_of(j)];
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
                            if constexpr (CK) {
                                if (chk) {
#pragma unroll
                                    for (int j = 0; j < PB; j += 4)
                                        check_subnormal4(subl, acc[i][h + j], acc[i][h + j + 1],
                                                         acc[i][h + j + 2], acc[i][h + j + 3], cls);
                                }
                            }
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
            // Binary64 unrolls four k rows (220 VGPRs): two measured up to 6% slower by box
            // and shape, a whole slab spills.
#pragma unroll(sizeof(T) == 4 ? BK : 4)
            for (int k = 0; k < BK; k++) {
                T a[8], b[8];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    a[i] = Ac[k][ty * 4 + i];
                    a[4 + i] = Ac[k][64 + ty * 4 + i];
                }
#pragma unroll
                for (int j = 0; j < 8; j++)
                    b[j] = Bc[k][col_of(j)];
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
                        if constexpr (CK) {
                            if (chk) {
#pragma unroll
                                for (int j = 0; j < 8; j += 4)
                                    check_subnormal4(subl, acc[i][j], acc[i][j + 1],
                                                     acc[i][j + 2], acc[i][j + 3], cls);
                            }
                        }
                    }
                }
            }
        }
    };
    auto off_grid = [&]() {
        bool o = false;
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int j = 0; j < 8; j++)
                o |= sum_off_grid(acc[i][j]);
        return __builtin_amdgcn_ballot_w64(o) != 0;
    };
    // Slab kt; the checking form checks its sums when the gate opens it.
    auto gcompute = [&](const T (*Ac)[Cfg::LDA], const T (*Bc)[Cfg::LDB], int kt, auto ck)
                        __attribute__((always_inline)) {
        if constexpr (decltype(ck)::value)
            chk = sgate.at(kt, off_grid);
        compute(Ac, Bc, ck);
    };
    if constexpr (!kDirect) {
        if (ktiles > 0) {
            if (WHOLE)
                stage.fetch_whole();
            else
                stage.fetch(A, B, M, N, K, m0, n0, 0, tid);
            stage.stash(As[0], Bs[0], tid);
        }
        __syncthreads();
        auto run = [&](auto ck) {
            for (int kt = 0; kt < ktiles; kt++) {
                const int cur = kt & 1;
                if (kt + 1 < ktiles) {
                    if (WHOLE)
                        stage.fetch_whole();
                    else
                        stage.fetch(A, B, M, N, K, m0, n0, (kt + 1) * BK, tid);
                }
                gcompute(As[cur], Bs[cur], kt, ck);
                if (kt + 1 < ktiles)
                    stage.stash(As[cur ^ 1], Bs[cur ^ 1], tid);
                __syncthreads();
            }
        };
        run_form(run);
    } else {
        // Wave w moves k rows w, w + 4, w + 8 and w + 12 of each directly loaded operand; lane
        // l's 16 bytes are the row's columns 2 l and 2 l + 1.
        const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
        const T *gb = B + (size_t)wv * N + n0 + 2 * lane;
        const T *ga = TA ? A + (size_t)wv * M + m0 + 2 * lane : A;
        auto load = [&](T (*Ad)[Cfg::LDA], T (*Bd)[Cfg::LDB]) {
#pragma unroll
            for (int r = 0; r < 4; r++)
                load_lds16(gb + (size_t)4 * r * N, &Bd[wv + 4 * r][0]);
            gb += (size_t)BK * N;
            if constexpr (TA) {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    load_lds16(ga + (size_t)4 * r * M, &Ad[wv + 4 * r][0]);
                ga += (size_t)BK * M;
            } else {
                stage.fetch_whole_a();
            }
        };
        auto stash = [&](T (*Ad)[Cfg::LDA]) {
            if constexpr (!TA)
                stage.stash_a(Ad, tid);
        };
        if (ktiles > 0) {
            load(A0, B0);
            stash(A0);
        }
        wait_lds_loads();
        __syncthreads();
        // Two slabs per trip: stage 0 holds even slabs, stage 1 odd ones.
        auto slab = [&](auto cur_c, int kt, auto ck) __attribute__((always_inline)) {
            constexpr int cur = decltype(cur_c)::value;
            T (*Ac)[Cfg::LDA] = cur ? A1 : A0;
            T (*Bc)[Cfg::LDB] = cur ? B1 : B0;
            T (*An)[Cfg::LDA] = cur ? A0 : A1;
            T (*Bn)[Cfg::LDB] = cur ? B0 : B1;
            if (kt + 1 < ktiles)
                load(An, Bn);
            gcompute(Ac, Bc, kt, ck);
            if (kt + 1 < ktiles)
                stash(An);
            wait_lds_loads();
            __syncthreads();
        };
        auto run = [&](auto ck) {
            for (int kt = 0; kt < ktiles; kt += 2) {
                slab(std::integral_constant<int, 0>{}, kt, ck);
                if (kt + 1 < ktiles)
                    slab(std::integral_constant<int, 1>{}, kt + 1, ck);
            }
        };
        run_form(run);
    }

    // Epilogue: publish the tile and find the first suspect cell of this lane.
    const bool sub = CHECK && ((subl.flush() >> (threadIdx.x & 63)) & 1);
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
                bool bad = !finite_bits(acc[i][h * RUN + j]) || sub;
                if (check_risk)
                    bad |= rexp + exp_of(col_exp[c]) < thr;
                if (sub)
                    flag_sum_block(sck, r, c);
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

// ------------------------------------------------------- binary64, narrow tile
// Strict binary64 on a 128 x 64 output tile per 256-thread workgroup, 8 x 4 per thread:
// 131-135 VGPRs, so three workgroups (three waves per SIMD) share a CU, against two for the
// 8 x 8 block. It serves outputs with fewer than 256 tiles of 128 x 128, less than one
// workgroup per CU: twice the tiles then fill the machine (1000^3: 216 us against 298). On
// full grids the 8 x 8 block is faster (4096^3: 4.34 against 4.55 ms; the narrow block reads
// half again as many operands from LDS per product).
struct NarrowF64Cfg {
    static constexpr int BM = 128, BN = 64, BK = 16;
    static constexpr int kThreads = 256;
    static constexpr int LDA = BM + 4, LDB = BN + 4;
    static constexpr int EA = BM * BK / kThreads, EB = BN * BK / kThreads; // 8 and 4
    // A thread's 4 elements of a B k-row as two 16-byte runs 32 apart (adjacent lanes then
    // store adjacent runs) when A is untransposed.
    template <bool TA> static constexpr bool kSplitRunsB = !TA;
};

template <bool TA, bool TB, bool VA, bool VB, bool WHOLE = false>
__global__ __launch_bounds__(256, 3) void k_strict_gemm_f64n(
    const double *__restrict__ A, const double *__restrict__ B, double *__restrict__ C, int M,
    int N, int K, const unsigned long long *__restrict__ row_exp,
    const unsigned long long *__restrict__ col_exp, int thr, int check_risk, int vec_c,
    unsigned long long *suspect, NodeGate gate)
{
    if (block_gate_closed(gate))
        return;
    using Cfg = NarrowF64Cfg;
    constexpr int BK = Cfg::BK, TBM = Cfg::BM, TBN = Cfg::BN;
    __shared__ __align__(16) double As[2][BK][Cfg::LDA];
    __shared__ __align__(16) double Bs[2][BK][Cfg::LDB];

    const int tid = threadIdx.x;
    const int tx = tid % 16, ty = tid / 16;
    // The lane's 4 columns: 2 runs of 2 adjacent doubles, 32 apart, so each 16-byte LDS read
    // of B covers 256 contiguous bytes over the 16 lanes of a row (no bank conflicts).
    auto col_of = [&](int j) { return (j / 2) * 32 + tx * 2 + (j % 2); };

    const int tiles_m = (M + TBM - 1) / TBM, tiles_n = (N + TBN - 1) / TBN;
    int tile_m, tile_n;
    tile_of(blockIdx.x, tiles_m, tiles_n, tile_m, tile_n);
    const int m0 = tile_m * TBM, n0 = tile_n * TBN;

    double acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            acc[i][j] = 0.0;

    SlabStager<double, Cfg, TA, TB, VA, VB> stage;
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
#pragma unroll 2
        for (int k = 0; k < BK; k++) {
            double a[8], b[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                a[i] = As[cur][k][ty * 4 + i];
                a[4 + i] = As[cur][k][64 + ty * 4 + i];
            }
#pragma unroll
            for (int j = 0; j < 4; j++)
                b[j] = Bs[cur][k][col_of(j)];
            // Per row, the four rounded products first and then their rounded sums.
#pragma unroll
            for (int i = 0; i < 8; i++) {
                double p[4];
#pragma unroll
                for (int j = 0; j < 4; j++)
                    p[j] = a[i] * b[j];
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = acc[i][j] + p[j];
            }
        }
        if (kt + 1 < ktiles)
            stage.stash(As[cur ^ 1], Bs[cur ^ 1], tid);
        __syncthreads();
    }

    uint64_t key = kNoFault;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = m0 + (i < 4 ? ty * 4 + i : 64 + ty * 4 + (i - 4));
        if (r >= M)
            continue;
        const int rexp = check_risk ? exp_of(row_exp[r]) : 0;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int c0 = n0 + col_of(2 * h);
            double *dst = C + (size_t)r * N + c0;
            if (vec_c && c0 + 2 <= N) {
                *reinterpret_cast<double2 *>(dst) = make_double2(acc[i][2 * h], acc[i][2 * h + 1]);
            } else {
#pragma unroll
                for (int j = 0; j < 2; j++)
                    if (c0 + j < N)
                        dst[j] = acc[i][2 * h + j];
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int c = c0 + j;
                if (c >= N)
                    continue;
                bool bad = !finite_bits(acc[i][2 * h + j]);
                if (check_risk)
                    bad |= rexp + exp_of(col_exp[c]) < thr;
                if (bad) {
                    const uint64_t cell = (uint64_t)r * N + c;
                    key = cell < key ? cell : key;
                }
            }
        }
    }
    wave_record_fault(key, suspect);
}

// ------------------------------------------------------------------ tiny scan
// IEEE policy. A cell whose result is finite met no invalid operand and no overflow (both
// leave Inf or NaN for good), and a sum is never tiny-inexact, so its first fault can only
// be a Multiply whose product is tiny and inexact. This tiled pass narrows the screen's marks
// to the cells that can have one, for the replay to classify exactly. A tiny product a * b
// (|a b| < 2^emin before rounding, emin the smallest normal exponent) has
// floor(log2|a|) + floor(log2|b|) < emin, since |a b| >= 2^(ea + eb). So per cell the pass
// takes the smallest exponent sum over k, a (min, +) product of 16-bit exponents, two cells
// per packed add and packed min (one instruction per (cell, k)), and flags the cell when
// that sum is below emin: every cell with a tiny product, and a few whose smallest products
// lie in [2^emin, 2^(emin + 1)). Zero and non-finite operands carry exponent 16000, so
// their sums never flag (a non-finite operand makes its whole row or column non-finite,
// which the serial replay walks). For each output row it keeps the first flagged column,
// and the first flagged row overall. It runs only when the screen marked a cell, skips
// every tile whose row and column exponents rule out a tiny product, and within a tile
// every k slab whose smallest A exponent and smallest B exponent (over the tile's rows and
// columns) do.
typedef short s16x2 __attribute__((ext_vector_type(2)));

template <typename T> __device__ __forceinline__ short scan_exp(T x)
{
    const int e = ilog2_abs(x);
    return (short)(e == kExpNone ? kScanExpNone : e);
}

// Tile of the scan: 128 x 128 cells per 256-thread workgroup, thread (tx, ty) owning rows
// 8 ty .. 8 ty + 7 and columns 8 tx .. 8 tx + 7, so each k row of a stage gives it its eight
// A exponents and eight B exponents as one 16-byte LDS read each. Slabs of 16 k.
template <typename T> struct ScanCfg {
    static constexpr int BM = 128, BN = 128, BK = 16, kThreads = 256;
    static constexpr int LDA = BM, LDB = BN; // (the exponent stages below have their own)
    static constexpr int EA = BM * BK / kThreads, EB = BN * BK / kThreads;
    template <bool TA> static constexpr bool kSplitRunsB = false;
};

// Superslab tables (when the screen filled them): op(A) rows and op(B) columns, entry-major
// (x_major: tbl[x * nss + s]) or superslab-major (tbl[s * extent + x]).
struct ScanTables {
    const short *a = nullptr, *b = nullptr;
    int a_xmajor = 0, b_xmajor = 0;
};
constexpr int kScanMaxSuperSlabs = 1024;

template <typename T, bool TA, bool TB, bool VA, bool VB>
__global__ __launch_bounds__(256, 2) void k_gemm_tiny_scan(
    const T *__restrict__ A, const T *__restrict__ B, int M, int N, int K,
    const unsigned long long *__restrict__ row_exp, const unsigned long long *__restrict__ col_exp,
    int thr, const unsigned long long *suspect, unsigned long long *row_flag,
    unsigned long long *flag_first, uint32_t gen, ScanTables tb, NodeGate gate,
    ProgramClose close)
{
    // No cell marked: nothing to scan (the same word for every thread). Most launches end
    // here, before the gate's block-wide read and its barrier. Then the replay after this
    // kernel finds no suspect cell either and writes no fault word, so a MatMul that ends
    // its program ends it here: one wave publishes at once, and the host need not wait for
    // the replay launch (which then returns without publishing).
    if (__atomic_load_n(suspect, __ATOMIC_RELAXED) == kNoFault) {
        if (close.words != nullptr && blockIdx.x == 0 && threadIdx.x < 64)
            program_close_wave(close);
        return;
    }
    if (block_gate_closed(gate))
        return;
    using Cfg = ScanCfg<T>;
    constexpr int BK = Cfg::BK, EA = Cfg::EA, EB = Cfg::EB;
    // k-major exponent stages; rows padded by 8 exponents (16 bytes) so the scattered
    // exponent stores of a transposing stash spread over the banks.
    constexpr int LA = BM + 8, LB = BN + 8;
    __shared__ __align__(16) short Ae[2][BK][LA];
    __shared__ __align__(16) short Be[2][BK][LB];
    __shared__ int slab_min[2][2][4]; // stage, operand, wave
    __shared__ int ss_min[2][kScanMaxSuperSlabs]; // operand, superslab: the tile's minima

    const int tid = threadIdx.x;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    // The grid holds at most two workgroups a CU (all that fit at once); each takes tiles in
    // turn, so an empty launch dispatches no more workgroups than that.
    for (uint32_t t = blockIdx.x; t < (uint32_t)(tiles_m * tiles_n); t += gridDim.x) {
    int tile_m, tile_n;
    tile_of(t, tiles_m, tiles_n, tile_m, tile_n);
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    // The tile holds a marked cell only if its smallest row exponent plus smallest column
    // exponent is below the threshold.
    const bool marked = tile_exp_sum_below<BM, BN>(row_exp, col_exp, m0, n0, M, N, thr);
    if (marked) {

    const int tx = tid % 16, ty = tid / 16;
    s16x2 mn[8][4]; // row i, columns 2 jp and 2 jp + 1
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int jp = 0; jp < 4; jp++)
            mn[i][jp] = (s16x2){kScanExpNone, kScanExpNone};

    // Global -> registers with the MatMul kernels' staging (elements outside the matrices
    // stage as +0, exponent 16000); registers -> LDS as exponents.
    SlabStager<T, Cfg, TA, TB, VA, VB> stage;
    // Also folds the slab's smallest A and B exponents, one word per wave.
    auto stash = [&](int buf) {
        short ea[EA], eb[EB];
        int amin = kScanExpNone, bmin = kScanExpNone;
#pragma unroll
        for (int i = 0; i < EA; i++) {
            ea[i] = scan_exp(stage.ra[i]);
            amin = ea[i] < amin ? ea[i] : amin;
        }
#pragma unroll
        for (int i = 0; i < EB; i++) {
            eb[i] = scan_exp(stage.rb[i]);
            bmin = eb[i] < bmin ? eb[i] : bmin;
        }
        if (!TA) { // thread: row m, k run of EA
            const int m = tid / (BK / EA), k = (tid % (BK / EA)) * EA;
#pragma unroll
            for (int i = 0; i < EA; i++)
                Ae[buf][k + i][m] = ea[i];
        } else {   // thread: k row, m run of EA
            const int k = tid / (BM / EA), m = (tid % (BM / EA)) * EA;
#pragma unroll
            for (int i = 0; i < EA; i++)
                Ae[buf][k][m + i] = ea[i];
        }
        if (!TB) { // thread: k row, n run of EB
            const int k = tid / (BN / EB), n = (tid % (BN / EB)) * EB;
#pragma unroll
            for (int i = 0; i < EB; i++)
                Be[buf][k][n + i] = eb[i];
        } else {   // thread: column n, k run of EB
            const int n = tid / (BK / EB), k = (tid % (BK / EB)) * EB;
#pragma unroll
            for (int i = 0; i < EB; i++)
                Be[buf][k + i][n] = eb[i];
        }
        amin = wave_min_i32(amin);
        bmin = wave_min_i32(bmin);
        if ((tid & 63) == 0) {
            slab_min[buf][0][tid >> 6] = amin;
            slab_min[buf][1][tid >> 6] = bmin;
        }
    };
    const int ktiles = (K + BK - 1) / BK;
    // One slab's (min, +) from stage `cur`, when its smallest A and B exponents allow a sum
    // below the threshold.
    auto scan_slab = [&](int cur) __attribute__((always_inline)) {
        int amin = slab_min[cur][0][0], bmin = slab_min[cur][1][0];
#pragma unroll
        for (int w = 1; w < 4; w++) {
            amin = slab_min[cur][0][w] < amin ? slab_min[cur][0][w] : amin;
            bmin = slab_min[cur][1][w] < bmin ? slab_min[cur][1][w] : bmin;
        }
        // Every sum of this slab is at least amin + bmin (the same value on every thread).
        if (amin + bmin < thr) {
#pragma unroll 4
            for (int k = 0; k < BK; k++) {
                const uint4 av = *reinterpret_cast<const uint4 *>(&Ae[cur][k][8 * ty]);
                const uint4 bv = *reinterpret_cast<const uint4 *>(&Be[cur][k][8 * tx]);
                const short *a = reinterpret_cast<const short *>(&av);
                const s16x2 *b = reinterpret_cast<const s16x2 *>(&bv);
                // The k row's 32 packed sums first, then the 32 packed minima: no minimum
                // waits on the sum just before it.
                s16x2 t[8][4];
#pragma unroll
                for (int i = 0; i < 8; i++)
#pragma unroll
                    for (int jp = 0; jp < 4; jp++)
                        t[i][jp] = (s16x2){a[i], a[i]} + b[jp];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < 8; i++)
#pragma unroll
                    for (int jp = 0; jp < 4; jp++)
                        mn[i][jp] = __builtin_elementwise_min(mn[i][jp], t[i][jp]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    if (tb.a) {
        // The tile's smallest exponent per superslab of op(A) rows and op(B) columns, from the
        // tables; only superslabs whose two minima sum below the threshold are read.
        constexpr int SS = (int)(kSuperSlab / BK);
        const int nss = (K + (int)kSuperSlab - 1) / (int)kSuperSlab;
        for (int i = tid; i < nss; i += 256) {
            ss_min[0][i] = kScanExpNone;
            ss_min[1][i] = kScanExpNone;
        }
        __syncthreads();
        const int x = tid & 127, half = tid >> 7, lane = tid & 63;
        const bool ain = m0 + x < M, bin = n0 + x < N;
        for (int ss = half; ss < nss; ss += 2) {
            int ea = kScanExpNone, eb = kScanExpNone;
            if (ain)
                ea = tb.a_xmajor ? tb.a[(size_t)(m0 + x) * nss + ss] : tb.a[(size_t)ss * M + m0 + x];
            if (bin)
                eb = tb.b_xmajor ? tb.b[(size_t)(n0 + x) * nss + ss] : tb.b[(size_t)ss * N + n0 + x];
            ea = wave_min_i32(ea);
            eb = wave_min_i32(eb);
            if (lane == 0) {
                atomicMin(&ss_min[0][ss], ea);
                atomicMin(&ss_min[1][ss], eb);
            }
        }
        __syncthreads();
        for (int kt = 0; kt < ktiles; kt++) {
            const int ss = kt / SS;
            if (ss_min[0][ss] + ss_min[1][ss] >= thr) {
                kt = SS * ss + SS - 1; // no product of the superslab sums below the threshold
                continue;
            }
            stage.fetch(A, B, M, N, K, m0, n0, kt * BK, tid);
            stash(0);
            __syncthreads();
            scan_slab(0);
            __syncthreads();
        }
    } else {
        if (ktiles > 0) {
            stage.fetch(A, B, M, N, K, m0, n0, 0, tid);
            stash(0);
        }
        __syncthreads();
        for (int kt = 0; kt < ktiles; kt++) {
            const int cur = kt & 1;
            if (kt + 1 < ktiles)
                stage.fetch(A, B, M, N, K, m0, n0, (kt + 1) * BK, tid);
            scan_slab(cur);
            if (kt + 1 < ktiles)
                stash(cur ^ 1);
            __syncthreads();
        }
    }
    // Past the edges the operands stage as +0 (exponent 16000): those cells never flag.
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = m0 + 8 * ty + i;
        uint32_t first = 0xffffffffu;
#pragma unroll
        for (int j = 7; j >= 0; j--) {
            const int c = n0 + 8 * tx + j;
            const int e = (j & 1) ? mn[i][j >> 1].y : mn[i][j >> 1].x;
            if (c < N && e < thr)
                first = (uint32_t)c;
        }
        if (r < M && first != 0xffffffffu) {
            atomicMax(&row_flag[r], ((unsigned long long)gen << 32) | (0xffffffffu - first));
            atomicMin(flag_first, (unsigned long long)r);
        }
    }
    } // marked
    __syncthreads(); // the next tile reuses the tile-minimum words and the stages
    }
}

// --------------------------------------------------------------- exact replay

// Lane l's value of v, on every lane (l uniform across the wave).
__device__ __forceinline__ float lane_value(float v, int l)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double lane_value(double v, int l)
{
    const uint64_t x = bits_of(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// First fault of one output cell, found by a whole wave (every lane returns the same). One
// pass over k in chunks of 64, the next chunk's operands loaded while the current one is
// classified: the lanes form the chunk's products and classify them, which gives the
// chunk's first faulting Multiply. When `walk_adds` is set (a non-finite result, where a sum
// can overflow, or RejectSubnormal, where a subnormal sum faults), every lane then folds the
// chunk's products before that Multiply in k order, as the contract orders the sums. Those
// products are finite, so a sum there can only fault by overflowing (the running sum turns,
// and stays, infinite) or, under RejectSubnormal, by being subnormal: the chunk is folded
// with plain adds and that check, and only a chunk that trips it is folded again with the
// exact add classifier to name the step. A Multiply at k comes before the Add at k. Returns
// kNoFault or the packed fault word.
template <typename T>
__device__ __forceinline__ uint64_t cell_first_fault(const T *__restrict__ A, const T *__restrict__ B,
                                                     uint64_t M, uint64_t N, uint64_t K, int ta,
                                                     int tb, uint64_t cell, int policy,
                                                     bool walk_adds)
{
    const int lane = threadIdx.x & 63;
    const uint64_t r = cell / N, c = cell % N;
    auto load = [&](uint64_t k0, T &a, T &b) {
        const uint64_t k = k0 + lane;
        a = (T)0;
        b = (T)0;
        if (k < K) {
            a = ta ? A[k * M + r] : A[r * K + k];
            b = tb ? B[c * K + k] : B[k * N + c];
        }
    };
    const bool reject_sub = policy == kPolicyRejectSubnormal;
    T total = (T)0;
    T a, b;
    load(0, a, b);
    for (uint64_t k0 = 0; k0 < K; k0 += 64) {
        T na = (T)0, nb = (T)0;
        if (k0 + 64 < K)
            load(k0 + 64, na, nb);
        const T p = a * b;
        uint32_t kind = kOk;
        if (k0 + lane < K)
            kind = classify_mul(a, b, p, policy);
        const uint64_t mask = __ballot(kind != kOk);
        const int l_m = mask ? __ffsll((long long)mask) - 1 : 64;
        if (walk_adds) {
            const int in_k = K - k0 < 64 ? (int)(K - k0) : 64;
            const int here = l_m < in_k ? l_m : in_k; // products summed before any fault
            T t = total;
            bool sub = false;
            if (here == 64) {
#pragma unroll
                for (int j = 0; j < 64; j++) {
                    t = t + lane_value(p, j);
                    sub |= reject_sub && subnormal(t);
                }
            } else {
                for (int j = 0; j < here; j++) {
                    t = t + lane_value(p, j);
                    sub |= reject_sub && subnormal(t);
                }
            }
            if (!finite_bits(t) || sub) {
                for (int j = 0; j < here; j++) {
                    const T pj = lane_value(p, j);
                    const T nxt = total + pj;
                    const uint32_t k_add = classify_add(total, pj, nxt, policy);
                    if (k_add != kOk)
                        return pack_fault((cell * K + k0 + j) * 2 + 1, k_add);
                    total = nxt;
                }
            }
            total = t;
        }
        if (mask)
            return pack_fault((cell * K + k0 + l_m) * 2, __shfl(kind, l_m, 64));
        a = na;
        b = nb;
    }
    return kNoFault;
}

// Lane 0's value, on every lane of the wave.
__device__ __forceinline__ uint64_t wave_uniform_u64(uint64_t v)
{
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// Two passes over the suspect cells, one wave per cell, each recording the earliest fault
// it finds with atomicMin and stopping once that lies before the cells it has left. Every
// loop is bounded, and each wave's branches are uniform, so each ballot sees its 64 lanes.
//  1. Blocks of 64 cells in row-major order from the first suspect cell: the lanes screen
//     the block's cells at once, and the wave takes its candidates in order with the
//     products and the ordered sums. Candidates: a non-finite result; under RejectSubnormal
//     (where a subnormal partial sum faults too) a cell whose row and column exponents sum
//     below `thr` and whose 32 x 32 block the tile kernel flagged (`sum_flag`: a partial
//     sum in the block came out subnormal), or, when the tile kernel did not check its
//     sums (`serial_screen`), every such cell.
//  2. Tiny (after k_gemm_tiny_scan): rows in order from the first flagged row, each from its
//     first flagged column, skipping cells whose exponents rule out a product below
//     2^tiny_thr. For a finite cell whose partial sums are not subnormal the first fault is
//     the lowest k whose product is tiny (under IEEE: and inexact), so only the products are
//     classified; a cell with a subnormal partial sum is also a pass-1 candidate, whose walk
//     finds the earlier of the two.
template <typename T>
__global__ __launch_bounds__(1024) void k_strict_gemm_replay(
    const T *__restrict__ A, const T *__restrict__ B, const T *__restrict__ C, uint64_t M,
    uint64_t N, uint64_t K, int ta, int tb, const unsigned long long *__restrict__ row_exp,
    const unsigned long long *__restrict__ col_exp, int thr, int tiny_thr, int serial_screen,
    int tiny, int policy, const unsigned long long *suspect, const unsigned long long *row_flag,
    const unsigned long long *flag_first, const unsigned int *sum_flag, uint32_t flag_cols,
    uint32_t gen, unsigned long long *fault, NodeGate gate, ProgramClose close)
{
    // No suspect cell: nothing to replay, whatever the gate says. Most launches end here,
    // before the gate's block-wide read and its barrier; no wave writes a fault word then,
    // so one wave may end the program at once.
    const uint64_t first = *suspect;
    if (first == kNoFault || K == 0) {
        // After a tiny scan (`tiny`), that scan ended the program on the same condition.
        if (close.words != nullptr && !tiny && blockIdx.x == 0 && threadIdx.x < 64)
            program_close_wave(close);
        return;
    }
    // The replay proper; its waves return on their own, then the workgroup takes its ticket.
    [&]() {
    if (block_gate_closed(gate))
        return; // an earlier node faulted: that fault is the one reported
    const uint64_t cells = M * N;
    // The cell of a packed MatMul fault: ordinal = 2 (cell K + k) + step.
    auto cell_of = [&](uint64_t w) { return ((w >> 3) / 2) / K; };
    // One value for the whole wave, so its lanes take every branch together.
    auto best_cell = [&]() {
        const uint64_t w = wave_uniform_u64(__atomic_load_n(fault, __ATOMIC_RELAXED));
        return w == kNoFault ? kNoFault : cell_of(w);
    };
    auto record = [&](uint64_t w) {
        if ((threadIdx.x & 63) == 0) {
            atomicMin(fault, (unsigned long long)w);
            gate_record(gate);
        }
    };
    const int lane = threadIdx.x & 63;
    const uint64_t waves = (uint64_t)gridDim.x * (blockDim.x / 64);
    const uint64_t wave = (uint64_t)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    // The first suspect cell holds a fault when its result is not finite (an invalid operand,
    // or an overflow, leaves Inf or NaN for good), and no earlier cell can hold one (none is
    // marked or non-finite): that cell's first fault is the MatMul's, and one wave finds it.
    if (!finite_bits(C[first])) {
        if (wave == 0) {
            const uint64_t w = cell_first_fault(A, B, M, N, K, ta, tb, first, policy, true);
            if (w != kNoFault)
                record(w);
        }
        return;
    }
    for (uint64_t c0 = (first / 64 + wave) * 64; c0 < cells; c0 += waves * 64) {
        if (best_cell() < c0)
            break; // this wave's blocks only grow
        const uint64_t cell = c0 + lane;
        bool cand = false;
        if (cell < cells) {
            cand = !finite_bits(C[cell]);
            if (serial_screen || sum_flag) {
                const uint64_t r = cell / N, c = cell % N;
                bool marked = exp_of(row_exp[r]) + exp_of(col_exp[c]) < thr;
                if (sum_flag)
                    marked = marked && sum_flag[(r >> 5) * flag_cols + (c >> 5)] == gen;
                cand |= marked;
            }
        }
        uint64_t mask = __ballot(cand);
        while (mask) {
            const int l = __ffsll((long long)mask) - 1;
            mask &= mask - 1;
            const uint64_t x = c0 + l;
            if (best_cell() < x)
                break;
            const uint64_t w = cell_first_fault(A, B, M, N, K, ta, tb, x, policy, true);
            if (w != kNoFault) {
                record(w);
                break; // the block's later cells come after this fault
            }
        }
    }
    if (!tiny)
        return;
    const uint64_t row0 = __atomic_load_n(flag_first, __ATOMIC_RELAXED);
    if (row0 == kNoFault)
        return;
    for (uint64_t r = row0 + wave; r < M; r += waves) {
        const unsigned long long w = wave_uniform_u64(row_flag[r]);
        if ((uint32_t)(w >> 32) != gen)
            continue; // no cell of this row was flagged by this MatMul's scan
        const int rexp = exp_of(row_exp[r]);
        bool done = false;
        for (uint64_t c = 0xffffffffu - (uint32_t)w; c < N && !done; c++) {
            const uint64_t cell = r * N + c;
            if (best_cell() < cell)
                return; // rows only grow: this wave has nothing earlier left
            // Every product of the cell is at least 2^(rexp + colexp): none is tiny.
            if (rexp + exp_of(col_exp[c]) >= tiny_thr)
                continue;
            if (!finite_bits(C[cell]))
                continue; // the first pass took it
            const uint64_t f = cell_first_fault(A, B, M, N, K, ta, tb, cell, policy, false);
            if (f != kNoFault) {
                record(f);
                done = true; // later cells of the row come after this fault
            }
        }
    }
    }();
    program_close_block(close);
}

// ------------------------------------------------------------ small outputs
// Outputs of at most fused_cells<T>() cells: one launch does the whole strict MatMul, spread
// over many CUs. Each 256-thread workgroup owns a 16 x 16 block of cells and walks k in chunks of
// kFusedBK, staging its op(A) rows and op(B) columns in LDS (k contiguous) and folding their
// smallest exponents as it stages them: a block sees all of k for its rows and columns, so
// it screens its own cells. Each thread computes one cell in k order with separately rounded
// products and sums. A cell is suspect when its result is not finite or its row and column
// exponents allow a tiny product (as in the screened path); a block with suspects walks them
// in cell order with the exact per-cell search, a wave per cell, stops once its earliest
// fault lies before the cells left, and folds that fault into the node's word with
// atomicMin, so the word ends with the MatMul's first fault.
constexpr int kFusedBK = 128;
// Measured against the screened path (whole calls): binary32 1.2-1.6x faster up to 256 x 256
// outputs, even at 512 x 2048 x 512, 2.4x slower at 1024^3; binary64 2.3-2.9x faster up to
// 512 x 512, 1.4x slower at 1024^3.
template <typename T> constexpr uint64_t fused_cells() { return sizeof(T) == 4 ? 256 * 256 : 512 * 512; }

template <typename T, bool TA, bool TB>
__global__ __launch_bounds__(256) void k_strict_gemm_fused(
    const T *__restrict__ A, const T *__restrict__ B, T *__restrict__ C, int M, int N, int K,
    int thr, int risk, int policy, unsigned long long *fault, NodeGate gate, ProgramClose close)
{
    if (block_gate_closed(gate)) {
        program_close_block(close);
        return;
    }
    constexpr int P = 16 / (int)sizeof(T), BKP = kFusedBK + P; // row pitch: one 16-byte pad
    __shared__ __align__(16) T As[16][BKP];
    __shared__ __align__(16) T Bs[16][BKP];
    __shared__ int rexp[16], cexp[16];
    __shared__ unsigned long long best; // this block's earliest fault
    __shared__ int n_cand, wave_cnt[4];
    __shared__ short cand[256];
    const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
    const int tiles_n = (N + 15) / 16;
    const int m0 = (int)(blockIdx.x / tiles_n) * 16, n0 = (int)(blockIdx.x % tiles_n) * 16;
    if (tid < 16) {
        rexp[tid] = kExpNone;
        cexp[tid] = kExpNone;
    }
    if (tid == 0)
        best = kNoFault;
    // Thread t stages one row of op(A) and one column of op(B), every 16th k of the chunk,
    // in an order that keeps each global access coalesced.
    const int ra = TA ? tx : ty, ka = TA ? ty : tx; // op(A) row, first k
    const int cb = TB ? ty : tx, kb = TB ? tx : ty; // op(B) column, first k
    T acc = (T)0;
    for (int k0 = 0; k0 < K; k0 += kFusedBK) {
        const int kc = K - k0 < kFusedBK ? K - k0 : kFusedBK;
        __syncthreads(); // the previous chunk is consumed
        // All of the thread's loads of the chunk are issued before any is used, so the chunk
        // arrives in one round trip.
        constexpr int L = kFusedBK / 16;
        T va[L], vb[L];
        const int row = m0 + ra, col = n0 + cb;
#pragma unroll
        for (int j = 0; j < L; j++) {
            const int k = ka + 16 * j;
            va[j] = (T)0;
            if (k < kc && row < M)
                va[j] = TA ? A[(size_t)(k0 + k) * M + row] : A[(size_t)row * K + k0 + k];
        }
#pragma unroll
        for (int j = 0; j < L; j++) {
            const int k = kb + 16 * j;
            vb[j] = (T)0;
            if (k < kc && col < N)
                vb[j] = TB ? B[(size_t)col * K + k0 + k] : B[(size_t)(k0 + k) * N + col];
        }
        int ea = kExpNone, eb = kExpNone;
#pragma unroll
        for (int j = 0; j < L; j++) {
            const int k = ka + 16 * j;
            if (k < kc) {
                As[ra][k] = va[j];
                const int e = ilog2_abs(va[j]);
                ea = e < ea ? e : ea;
            }
        }
#pragma unroll
        for (int j = 0; j < L; j++) {
            const int k = kb + 16 * j;
            if (k < kc) {
                Bs[cb][k] = vb[j];
                const int e = ilog2_abs(vb[j]);
                eb = e < eb ? e : eb;
            }
        }
        if (ea < kExpNone)
            atomicMin(&rexp[ra], ea);
        if (eb < kExpNone)
            atomicMin(&cexp[cb], eb);
        __syncthreads();
        int k = 0;
        for (; k + P <= kc; k += P) {
            const uint4 av = *reinterpret_cast<const uint4 *>(&As[ty][k]);
            const uint4 bv = *reinterpret_cast<const uint4 *>(&Bs[tx][k]);
            const T *a = reinterpret_cast<const T *>(&av);
            const T *b = reinterpret_cast<const T *>(&bv);
#pragma unroll
            for (int j = 0; j < P; j++) {
                const T p = a[j] * b[j];
                acc = acc + p;
            }
        }
        for (; k < kc; k++) {
            const T p = As[ty][k] * Bs[tx][k];
            acc = acc + p;
        }
    }
    __syncthreads(); // every exponent folded
    const int row = m0 + ty, col = n0 + tx;
    bool sus = false;
    if (row < M && col < N) {
        C[(size_t)row * N + col] = acc;
        sus = !finite_bits(acc) || (risk && rexp[ty] + cexp[tx] < thr);
    }
    // The block's suspect cells in cell order (tile index ty * 16 + tx grows with it).
    const int lane = tid & 63, wave = tid >> 6;
    const uint64_t mask = __ballot(sus);
    if (lane == 0)
        wave_cnt[wave] = __popcll(mask);
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; w++)
        before += wave_cnt[w];
    if (sus)
        cand[before + __popcll(mask & ((1ull << lane) - 1))] = (short)tid;
    if (tid == 0)
        n_cand = wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
    __syncthreads();
    const int nc = n_cand;
    if (nc == 0) {
        program_close_block(close);
        return;
    }
    for (int j = wave; j < nc; j += 4) {
        const int i = cand[j];
        const uint64_t cell = (uint64_t)(m0 + (i >> 4)) * N + n0 + (i & 15);
        const uint64_t bw = wave_uniform_u64(__atomic_load_n(&best, __ATOMIC_RELAXED));
        if (bw != kNoFault && ((bw >> 3) / 2) / (uint64_t)K < cell)
            break; // cells only grow along the list
        const uint64_t w = cell_first_fault(A, B, (uint64_t)M, (uint64_t)N, (uint64_t)K, (int)TA,
                                            (int)TB, cell, policy, true);
        if (w != kNoFault && lane == 0)
            atomicMin(&best, (unsigned long long)w);
    }
    __syncthreads();
    if (tid == 0 && best != kNoFault) {
        atomicMin(fault, best);
        gate_record(gate);
    }
    program_close_block(close);
}

// ================================================================= launchers

static size_t sum_flag_bytes(uint64_t rows, uint64_t cols)
{
    return (((rows + 31) / 32) * ((cols + 31) / 32) * sizeof(unsigned int) + 255) & ~(size_t)255;
}

// The superslab tables, when they take at most 32 MiB and K spans at most 1024 superslabs
// (the tiny scan's per-tile list); 0 otherwise. They live in a buffer of their own: in the
// MatMul scratch, a later call of another shape could find their bits where it keeps
// generation-tagged words folded with atomicMax, and such bits may outrank its generation.
size_t slab_table_bytes(uint64_t rows, uint64_t inner, uint64_t cols)
{
    const uint64_t nss = (inner + kSuperSlab - 1) / kSuperSlab;
    const uint64_t bytes = (rows + cols) * nss * sizeof(short);
    if (nss == 0 || nss > 1024 || bytes > (32ull << 20))
        return 0;
    return ((size_t)bytes + 255) & ~(size_t)255;
}

size_t matmul_scratch_bytes(uint64_t rows, uint64_t cols, bool sum_flags)
{
    size_t r = ((rows * sizeof(unsigned long long)) + 255) & ~(size_t)255;
    size_t c = ((cols * sizeof(unsigned long long)) + 255) & ~(size_t)255;
    return r + c + r + 256 + (sum_flags ? sum_flag_bytes(rows, cols) : 0);
}

// The two words reset to kNoFault (first suspect cell, first flagged row) sit in a fixed
// 256-byte head, and the generation-tagged words folded with atomicMax (row and column
// exponents, row flags) after it. Calls of different shapes reuse one buffer, so a word of
// one call can lie where another call keeps a different word; kNoFault (all ones) would
// outrank every later word under atomicMax, so it must never lie in the tagged part.
MatmulScratch matmul_scratch_carve(void *base, uint64_t rows, uint64_t cols, bool sum_flags,
                                   void *tables, uint64_t inner)
{
    char *p = (char *)base;
    size_t r = ((rows * sizeof(unsigned long long)) + 255) & ~(size_t)255;
    size_t c = ((cols * sizeof(unsigned long long)) + 255) & ~(size_t)255;
    MatmulScratch s;
    s.suspect = (unsigned long long *)p;
    s.flag_first = s.suspect + 1;
    s.row_exp = (unsigned long long *)(p + 256);
    s.col_exp = (unsigned long long *)(p + 256 + r);
    s.row_flag = (unsigned long long *)(p + 256 + r + c);
    if (sum_flags) {
        // Tagged with the generation like the exponent words: a word of an earlier call never
        // equals this call's generation, and a pair of them read as one 64-bit word there
        // carries an earlier generation.
        s.sum_flag = (unsigned int *)(p + 256 + r + c + r);
        s.flag_cols = (uint32_t)((cols + 31) / 32);
    }
    if (tables) {
        // Rewritten whole by every screen that fills them.
        const uint64_t nss = (inner + kSuperSlab - 1) / kSuperSlab;
        s.tbl_a = (short *)tables;
        s.tbl_b = s.tbl_a + rows * nss;
    }
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
    if (i0 == 0) {
        gate[0] = 0xffffffffu;
        gate[1] = 0u; // the ticket of an in-kernel program end (ProgramClose)
    }
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

// A stored R x C matrix copied into C x R (R and C multiples of 4, both pointers 16-byte
// aligned): 64 x 64 tiles through LDS, runs of four elements (one or two 16-byte loads and
// stores), rows of the tile padded by one element. Used for a transposed op(B) that the
// tile kernel then loads as an untransposed one: the copy holds the same values, so every
// product, sum and fault of the MatMul is unchanged.
template <typename T> struct alignas(16) Run4 {
    T v[4];
};

template <typename T>
__global__ __launch_bounds__(256) void k_transpose(const T *__restrict__ X, T *__restrict__ Y,
                                                   int R, int C, NodeGate gate)
{
    if (block_gate_closed(gate))
        return;
    __shared__ T t[64][65];
    const int tiles_c = (C + 63) / 64;
    const int r0 = (int)(blockIdx.x / tiles_c) * 64, c0 = (int)(blockIdx.x % tiles_c) * 64;
    const int q = threadIdx.x & 15, row = threadIdx.x >> 4; // 16 runs of 4 floats x 16 rows
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const int i = row + 16 * p, r = r0 + i, c = c0 + 4 * q;
        if (r < R && c < C) {
            const Run4<T> v = *reinterpret_cast<const Run4<T> *>(X + (size_t)r * C + c);
#pragma unroll
            for (int e = 0; e < 4; e++)
                t[i][4 * q + e] = v.v[e];
        }
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const int j = row + 16 * p, c = c0 + j, r = r0 + 4 * q;
        if (c < C && r < R) {
            Run4<T> v;
#pragma unroll
            for (int e = 0; e < 4; e++)
                v.v[e] = t[4 * q + e][j];
            *reinterpret_cast<Run4<T> *>(Y + (size_t)c * R + r) = v;
        }
    }
}

// Largest op(B) copied out (2^28 elements); larger ones are read in place.
constexpr uint64_t kBtMaxElems = 1ull << 28;

bool matmul_bt_wanted(int dtype, uint64_t rows, uint64_t inner, uint64_t cols, bool tl,
                      bool tr, int engine)
{
    if (!tr || (dtype == 0 && engine == kEngineValu) || inner == 0 || inner % 16 != 0)
        return false;
    // Binary64: NT 4096^3 4507 against 4692 us, 2048^3 610 against 674; TT measured no
    // faster (4563 against 4523), its op(A) read-ahead path already hides the staging.
    if (dtype != 0 && tl)
        return false;
    if (engine == kEngineAuto && rows * cols <= fused_cells<float>())
        return false; // the fused small-output launch reads B in place
    // Whole 128 x 128 tiles filling at least one workgroup a CU: the copy measured 2-2.5%
    // faster there (NT 4096^3 1973 against 2021 us, 4096 x 1024 x 4096 510 against 521, TT
    // 4096^3 -2%), and 4.5-7% slower on the 64 x 64 tiles of smaller grids (1024^3 NT 57.1
    // against 54.6 us).
    return rows % 128 == 0 && cols % 128 == 0 && (rows / 128) * (cols / 128) >= 256 &&
           inner * cols <= kBtMaxElems;
}

// The exponent screen of op(A) rows and op(B) columns, both jobs in one launch.
template <typename T>
static void prefilter(hipStream_t s, ExpJob<T> ja, ExpJob<T> jb, uint32_t gen,
                      unsigned long long *suspect, NodeGate gate, ProgramOpen open)
{
    for (ExpJob<T> *j : {&ja, &jb})
        j->vec = j->C % (16 / sizeof(T)) == 0 && aligned16(j->X);
    const uint64_t na = exp_blocks(ja), nb = exp_blocks(jb);
    hipLaunchKernelGGL(k_exp_screen<T>, dim3((unsigned)(na + nb)), dim3(256), 0, s, ja, jb, na, gen, suspect, gate, open);
}

template <typename T, bool TA, bool TB>
static void gemm_dispatch(hipStream_t s, dim3 grid, const T *A, const T *B, T *C, int M, int N,
                          int K, const unsigned long long *re, const unsigned long long *ce,
                          int thr, int risk, unsigned long long *suspect, SumCheck sck,
                          NodeGate gate)
{
    bool va = (TA ? (M % 4 == 0) : (K % 4 == 0)) && aligned16(A);
    bool vb = (TB ? (K % 4 == 0) : (N % 4 == 0)) && aligned16(B);
    int vc = (N % 4 == 0) && aligned16(C);
    using Cfg = ValuCfg<T>;
    if (va && vb && M % Cfg::BM == 0 && N % Cfg::BN == 0 && K % Cfg::BK == 0)
        { hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, true, true, false, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, sck, gate); if (sck.flag) hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, true, true, false, true, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, sck, gate); }
    else if (va && vb)
        { hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, true, true, false, false>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, sck, gate); if (sck.flag) hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, true, true, false, false, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, sck, gate); }
    else if (va)
        { hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, true, false, false, false>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, sck, gate); if (sck.flag) hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, true, false, false, false, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, sck, gate); }
    else if (vb)
        { hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, false, true, false, false>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, sck, gate); if (sck.flag) hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, false, true, false, false, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, sck, gate); }
    else
        { hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, false, false, false, false>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, sck, gate); if (sck.flag) hipLaunchKernelGGL((k_strict_gemm<T, TA, TB, false, false, false, false, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, sck, gate); }
}

template <typename T, bool TA, bool TB>
static void tiny_scan_dispatch(hipStream_t s, dim3 grid, const T *A, const T *B, int M, int N,
                               int K, const MatmulScratch &sc, int thr, ScanTables tb, NodeGate gate,
                               ProgramClose close)
{
    const bool va = (TA ? (M % 4 == 0) : (K % 4 == 0)) && aligned16(A);
    const bool vb = (TB ? (K % 4 == 0) : (N % 4 == 0)) && aligned16(B);
    if (va && vb)
        hipLaunchKernelGGL((k_gemm_tiny_scan<T, TA, TB, true, true>), grid, dim3(256), 0, s, A, B, M, N, K, sc.row_exp, sc.col_exp, thr, sc.suspect, sc.row_flag, sc.flag_first, sc.gen, tb, gate, close);
    else if (va)
        hipLaunchKernelGGL((k_gemm_tiny_scan<T, TA, TB, true, false>), grid, dim3(256), 0, s, A, B, M, N, K, sc.row_exp, sc.col_exp, thr, sc.suspect, sc.row_flag, sc.flag_first, sc.gen, tb, gate, close);
    else if (vb)
        hipLaunchKernelGGL((k_gemm_tiny_scan<T, TA, TB, false, true>), grid, dim3(256), 0, s, A, B, M, N, K, sc.row_exp, sc.col_exp, thr, sc.suspect, sc.row_flag, sc.flag_first, sc.gen, tb, gate, close);
    else
        hipLaunchKernelGGL((k_gemm_tiny_scan<T, TA, TB, false, false>), grid, dim3(256), 0, s, A, B, M, N, K, sc.row_exp, sc.col_exp, thr, sc.suspect, sc.row_flag, sc.flag_first, sc.gen, tb, gate, close);
}

template <bool TA, bool TB>
static void f64n_dispatch(hipStream_t s, const double *A, const double *B, double *C, int M,
                          int N, int K, const unsigned long long *re, const unsigned long long *ce,
                          int thr, int risk, unsigned long long *suspect, NodeGate gate)
{
    using Cfg = NarrowF64Cfg;
    const dim3 grid((unsigned)(((M + Cfg::BM - 1) / Cfg::BM) * ((N + Cfg::BN - 1) / Cfg::BN)));
    const bool va = (TA ? (M % 4 == 0) : (K % 4 == 0)) && aligned16(A);
    const bool vb = (TB ? (K % 4 == 0) : (N % 4 == 0)) && aligned16(B);
    const int vc = (N % 2 == 0) && aligned16(C);
    if (va && vb && M % Cfg::BM == 0 && N % Cfg::BN == 0 && K % Cfg::BK == 0)
        hipLaunchKernelGGL((k_strict_gemm_f64n<TA, TB, true, true, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, gate);
    else if (va && vb)
        hipLaunchKernelGGL((k_strict_gemm_f64n<TA, TB, true, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, gate);
    else if (va)
        hipLaunchKernelGGL((k_strict_gemm_f64n<TA, TB, true, false>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, gate);
    else if (vb)
        hipLaunchKernelGGL((k_strict_gemm_f64n<TA, TB, false, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, gate);
    else
        hipLaunchKernelGGL((k_strict_gemm_f64n<TA, TB, false, false>), grid, dim3(256), 0, s, A, B, C, M, N, K, re, ce, thr, risk, vc, suspect, gate);
}

template <typename T>
static hipError_t strict_matmul_t(hipStream_t s, uint64_t M, uint64_t K, uint64_t N, bool ta,
                                  bool tb, const T *A, const T *B, T *C, int policy,
                                  MatmulScratch sc, unsigned long long *fault, NodeGate gate,
                                  hipEvent_t *ev, int engine, ProgramOpen open,
                                  const GemmEpilogue *epi, bool *epi_done, Prescreen pre,
                                  ProgramClose close, bool *closed)
{
    if (M == 0 || N == 0)
        return hipSuccess;
    // Smallest exponent sums that need no replay: a product >= 2^-126 (2^-1022) is never
    // tiny (tiny_thr); products >= 2^-103 (2^-970) are multiples of the smallest normal, and
    // rounded sums of such multiples stay multiples, so no partial sum of a cell that meets
    // no smaller product is a nonzero subnormal (sub_thr, RejectSubnormal). AllowGradual:
    // underflow is never a fault.
    const bool f32 = sizeof(T) == 4;
    const int tiny_thr = f32 ? -126 : -1022, sub_thr = f32 ? -103 : -970;
    const bool reject = policy == kPolicyRejectSubnormal;
    int risk = policy != kPolicyAllowGradual;
    // Under RejectSubnormal the tile kernels check the partial sums of every tile that may
    // meet a product below 2^sub_thr (all but the narrow binary64 tile, when the scratch has
    // the block words); a cell is then suspect only for a non-finite result, a possibly tiny
    // product or a subnormal partial sum in its lane. Without the check every cell the
    // exponents put below sub_thr is suspect and walked in full.
    const uint64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    const bool sum_check = reject && K > 0 && sc.sum_flag != nullptr && (f32 || tiles >= 256);
    int thr = reject && !sum_check ? sub_thr : tiny_thr;
    SumCheck sck = sum_check ? SumCheck{sc.sum_flag, sc.gen, sc.flag_cols, sub_thr} : SumCheck{};
    if (ev)
        (void)hipEventRecord(ev[0], s);
    if (engine == kEngineAuto && K > 0 && M * N <= fused_cells<T>()) {
        // A program's first node opens the program before any block can record a fault.
        if (open.words)
            hipLaunchKernelGGL(k_matmul_open, dim3(1), dim3(256), 0, s, sc.suspect, open);
        if (ev)
            (void)hipEventRecord(ev[1], s);
        const dim3 grid((unsigned)(((M + 15) / 16) * ((N + 15) / 16)));
        if (grid.x > kCloseMaxBlocks)
            close = ProgramClose{}; // the publication launch ends the program
        if (closed)
            *closed = close.words != nullptr;
        const int m = (int)M, n = (int)N, k = (int)K;
        // The fused kernel walks every cell its exponents mark (no partial-sum check).
        const int fthr = reject ? sub_thr : tiny_thr;
        if (!ta && !tb) hipLaunchKernelGGL((k_strict_gemm_fused<T, false, false>), grid, dim3(256), 0, s, A, B, C, m, n, k, fthr, risk, policy, fault, gate, close);
        else if (!ta && tb) hipLaunchKernelGGL((k_strict_gemm_fused<T, false, true>), grid, dim3(256), 0, s, A, B, C, m, n, k, fthr, risk, policy, fault, gate, close);
        else if (ta && !tb) hipLaunchKernelGGL((k_strict_gemm_fused<T, true, false>), grid, dim3(256), 0, s, A, B, C, m, n, k, fthr, risk, policy, fault, gate, close);
        else hipLaunchKernelGGL((k_strict_gemm_fused<T, true, true>), grid, dim3(256), 0, s, A, B, C, m, n, k, fthr, risk, policy, fault, gate, close);
        if (ev) {
            (void)hipEventRecord(ev[2], s);
            (void)hipEventRecord(ev[3], s);
        }
        return hipGetLastError();
    }
    // The superslab tables let the tiny scan read only the runs of k where a product below
    // 2^tiny_thr is possible; the screen fills them wherever the scan may run (IEEE, and
    // RejectSubnormal with the partial-sum check). On a clean input they cost the screen
    // about 1.5 us at 4096^3; on a fully marked one they cut the scan from 0.84 to 0.17 ms.
    const bool tables = sc.tbl_a != nullptr && (policy == kPolicyIeee || sum_check);
    ScanTables tbls;
    if (tables) {
        // A prescreened operand's table is the one its producer wrote, in the same layout.
        tbls.a = pre.a ? pre.a : sc.tbl_a;
        tbls.b = pre.b ? pre.b : sc.tbl_b;
        tbls.a_xmajor = !ta; // a rows job over A (M x K), else a columns job over A (K x M)
        tbls.b_xmajor = tb;  // a rows job over B (N x K), else a columns job over B (K x N)
    }
    if (tables && sum_check) {
        // The checking tiles check only the superslabs that need it (the tables describe
        // op(B) as stored, also when the tile kernel reads its K x N copy).
        sck.tbl_a = tbls.a;
        sck.tbl_b = tbls.b;
        sck.a_xmajor = tbls.a_xmajor;
        sck.b_xmajor = tbls.b_xmajor;
    }
    if (risk && K > 0) {
        // op(A) row r is stored row r (A is M x K) or stored column r (A is K x M); op(B)
        // column c is stored column c (B is K x N) or stored row c (B is N x K).
        // A prescreened operand is not read: its words are folded from its producer's table.
        const ExpJob<T> ja{A, ta ? K : M, ta ? M : K, !ta, false, sc.row_exp,
                           tables && !pre.a ? sc.tbl_a : nullptr, pre.a};
        const ExpJob<T> jb{B, tb ? N : K, tb ? K : N, tb, false, sc.col_exp,
                           tables && !pre.b ? sc.tbl_b : nullptr, pre.b};
        prefilter<T>(s, ja, jb, sc.gen, sc.suspect, gate, open);
    } else {
        risk = 0; // AllowGradual, or an empty reduction: no underflow screen
        hipLaunchKernelGGL(k_matmul_open, dim3(1), dim3(256), 0, s, sc.suspect, open);
    }
    dim3 grid((unsigned)(((M + BM - 1) / BM) * ((N + BN - 1) / BN)));
    const int m = (int)M, n = (int)N, k = (int)K;
    if (ev)
        (void)hipEventRecord(ev[1], s);
    if (f32 && engine != kEngineValu) {
        // A transposed op(B) (stored N x K) goes to the tile kernel as its K x N copy, which
        // it loads straight into LDS; the screen, tiny scan and replay read B in place.
        const float *Bt = (const float *)B;
        bool tbt = tb;
        if (tb && sc.bt && aligned16(B)) {
            const unsigned tiles = (unsigned)(((N + 63) / 64) * ((K + 63) / 64));
            hipLaunchKernelGGL(k_transpose<float>, dim3(tiles), dim3(256), 0, s, (const float *)B,
                               (float *)sc.bt, n, k, gate);
            Bt = (const float *)sc.bt;
            tbt = false;
        }
        (void)launch_gemm_mfma_f32(s, m, n, k, ta, tbt, (const float *)A, Bt, (float *)C,
                                   sc.row_exp, sc.col_exp, thr, risk, sc.suspect, sck, gate, epi, epi_done);
    } else if (!f32 && (uint64_t)grid.x < 256) {
        const double *dA = (const double *)A, *dB = (const double *)B;
        double *dC = (double *)C;
        if (!ta && !tb) f64n_dispatch<false, false>(s, dA, dB, dC, m, n, k, sc.row_exp, sc.col_exp, thr, risk, sc.suspect, gate);
        else if (!ta && tb) f64n_dispatch<false, true>(s, dA, dB, dC, m, n, k, sc.row_exp, sc.col_exp, thr, risk, sc.suspect, gate);
        else if (ta && !tb) f64n_dispatch<true, false>(s, dA, dB, dC, m, n, k, sc.row_exp, sc.col_exp, thr, risk, sc.suspect, gate);
        else f64n_dispatch<true, true>(s, dA, dB, dC, m, n, k, sc.row_exp, sc.col_exp, thr, risk, sc.suspect, gate);
    } else {
        // A transposed binary64 op(B) on a full grid goes to the tile kernel as its K x N
        // copy, as for the matrix-core engine above.
        const T *Bk = B;
        bool tbk = tb;
        if (!f32 && tb && sc.bt && aligned16(B)) {
            const unsigned tiles = (unsigned)(((N + 63) / 64) * ((K + 63) / 64));
            hipLaunchKernelGGL(k_transpose<T>, dim3(tiles), dim3(256), 0, s, B, (T *)sc.bt, n, k, gate);
            Bk = (const T *)sc.bt;
            tbk = false;
        }
        if (!ta && !tbk) gemm_dispatch<T, false, false>(s, grid, A, Bk, C, m, n, k, sc.row_exp, sc.col_exp, thr, risk, sc.suspect, sck, gate);
        else if (!ta && tbk) gemm_dispatch<T, false, true>(s, grid, A, Bk, C, m, n, k, sc.row_exp, sc.col_exp, thr, risk, sc.suspect, sck, gate);
        else if (ta && !tbk) gemm_dispatch<T, true, false>(s, grid, A, Bk, C, m, n, k, sc.row_exp, sc.col_exp, thr, risk, sc.suspect, sck, gate);
        else gemm_dispatch<T, true, true>(s, grid, A, Bk, C, m, n, k, sc.row_exp, sc.col_exp, thr, risk, sc.suspect, sck, gate);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    if (ev)
        (void)hipEventRecord(ev[2], s);
    // A finite cell whose partial sums are not subnormal can first fault only in a tiny
    // product: the tiled scan narrows the screen's marks to the cells that may have one, for
    // the wave-parallel pass (IEEE, and RejectSubnormal when the tile kernel checked the
    // sums). Otherwise the serial pass walks every marked cell.
    const bool tiny = risk && (policy == kPolicyIeee || sum_check);
    if (tiny) {
        const dim3 sgrid(grid.x < 2u * kGfx950Cus ? grid.x : 2u * kGfx950Cus);
        if (!ta && !tb) tiny_scan_dispatch<T, false, false>(s, sgrid, A, B, m, n, k, sc, tiny_thr, tbls, gate, close);
        else if (!ta && tb) tiny_scan_dispatch<T, false, true>(s, sgrid, A, B, m, n, k, sc, tiny_thr, tbls, gate, close);
        else if (ta && !tb) tiny_scan_dispatch<T, true, false>(s, sgrid, A, B, m, n, k, sc, tiny_thr, tbls, gate, close);
        else tiny_scan_dispatch<T, true, true>(s, sgrid, A, B, m, n, k, sc, tiny_thr, tbls, gate, close);
    }
    const int serial_screen = risk && !tiny;
    // 4096 waves in 256 workgroups: an empty launch (no suspect cell) dispatches a quarter of
    // the workgroups that 256-thread blocks would take.
    if (closed)
        *closed = close.words != nullptr;
    hipLaunchKernelGGL(k_strict_gemm_replay<T>, dim3(256), dim3(1024), 0, s, A, B, (const T *)C, M, N, K,
                       (int)ta, (int)tb, sc.row_exp, sc.col_exp, reject ? sub_thr : tiny_thr, tiny_thr,
                       serial_screen, (int)tiny, policy, (const unsigned long long *)sc.suspect,
                       (const unsigned long long *)sc.row_flag, (const unsigned long long *)sc.flag_first,
                       (const unsigned int *)sck.flag, sc.flag_cols, sc.gen, fault, gate, close);
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
        hipLaunchKernelGGL((k_strict_gemm<double, TA, TB, true, true, true, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, nullptr, nullptr, 0, 0, vc, nullptr, SumCheck{}, gate);
    else if (va && vb)
        hipLaunchKernelGGL((k_strict_gemm<double, TA, TB, true, true, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, nullptr, nullptr, 0, 0, vc, nullptr, SumCheck{}, gate);
    else if (va)
        hipLaunchKernelGGL((k_strict_gemm<double, TA, TB, true, false, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, nullptr, nullptr, 0, 0, vc, nullptr, SumCheck{}, gate);
    else if (vb)
        hipLaunchKernelGGL((k_strict_gemm<double, TA, TB, false, true, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, nullptr, nullptr, 0, 0, vc, nullptr, SumCheck{}, gate);
    else
        hipLaunchKernelGGL((k_strict_gemm<double, TA, TB, false, false, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, nullptr, nullptr, 0, 0, vc, nullptr, SumCheck{}, gate);
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
                                hipEvent_t *ev, int engine, ProgramOpen open,
                                const GemmEpilogue *epi, Prescreen pre, bool *epi_fused,
                                ProgramClose close, bool *closed)
{
    if (closed)
        *closed = false;
    if (rows > (uint64_t)INT_MAX || cols > (uint64_t)INT_MAX || inner > (uint64_t)INT_MAX)
        return hipErrorInvalidValue;
    if (epi && epi->op != 0 && epi->op != kStepRelu && epi->op != kStepReluBackward)
        return hipErrorInvalidValue;
    // The program ends in the MatMul's last kernel only when nothing follows it.
    if (close.words && ((epi && epi->op != 0) || rows == 0 || cols == 0 || !scratch.suspect))
        return hipErrorInvalidValue;
    bool done = false;
    if (epi_fused)
        *epi_fused = false;
    const hipError_t e =
        dtype == 0 ? strict_matmul_t<float>(s, rows, inner, cols, transpose_left, transpose_right,
                                            (const float *)a, (const float *)b, (float *)c, policy,
                                            scratch, fault, gate, ev, engine, open, epi, &done, pre,
                                            close, closed)
                   : strict_matmul_t<double>(s, rows, inner, cols, transpose_left, transpose_right,
                                             (const double *)a, (const double *)b, (double *)c,
                                             policy, scratch, fault, gate, ev, engine, open, epi,
                                             &done, pre, close, closed);
    if (e != hipSuccess || !epi || epi->op == 0)
        return e;
    if (done) {
        if (epi_fused)
            *epi_fused = true;
        return e;
    }
    // The tile kernel that ran has no such epilogue: the node's own kernel follows.
    const uint64_t n = rows * cols;
    if (epi->op == kStepRelu)
        return launch_relu(s, dtype, n, c, epi->out, epi->policy, epi->fault, epi->gate);
    return launch_relu_backward(s, dtype, n, epi->x, c, epi->out, epi->policy, epi->fault, epi->gate);
}

} // namespace pcu
