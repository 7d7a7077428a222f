// Strict F32 MatMul main kernel with the products formed by the matrix cores.
//
// Contract (core/dialect/tensor/reference/strict_matmul/strict_matmul.rs:22-73): every
// output cell starts from +0 and walks k upward; each product is rounded on its own and
// each sum is rounded on its own. The VALU kernel (matmul.hip) spends two vector
// instructions per (cell, k). Here v_mfma_f32_32x32x1_2b_f32 is used as a multiplier
// array only: its K is 1 and its accumulator input is +0, so every output element is the
// single product a*b rounded once to nearest-even, and no sum is formed inside the matrix
// core. The vector unit then folds the products into the accumulators in k order with
// separate v_add_f32. Two facts make this bit-exact:
//  * for a nonzero exact product, RNE(a*b + 0) = RNE(a*b); gfx950 keeps subnormal
//    inputs and results under the library's denormal mode (checked against v_mul_f32 on
//    the device over random, tie-constructed, near-MIN_NORMAL, subnormal and overflowing
//    operands: identical except the sign of an exact zero product);
//  * an exact zero product comes out as +0 where v_mul_f32 gives -0, and that never
//    changes an accumulator: it starts at +0, can never become -0 (a sum is -0 only when
//    both terms are), and x + (+0) = x + (-0) for every x != -0.
// The two blocks of one MFMA carry k and k+1 for the same 32x32 output tile, so one
// instruction yields 2048 products and a lane adds its 16 cells' k-product, then their
// (k+1)-product. Small grids of whole 64x64 tiles use v_mfma_f32_16x16x1_4b_f32 the same
// way (k_strict_gemm_mfma16): its four blocks carry k..k+3 for one 16x16 output tile.
//
// Fault screening (non-finite result, exponent prefilter) and the exact replay of suspect
// cells are shared with the VALU kernel; these kernels record a workgroup's first suspect
// cell with one atomic.
#include "pcu_device.hpp"
#include "pcu_gemm_stage.hpp"
#include "pcu_kernels.hpp"

#pragma clang fp contract(off)

namespace pcu {

typedef float v32f __attribute__((ext_vector_type(32)));

// Workgroup shape: WM x WN waves, each owning SM x SN output subtiles of 32 x 32; k-slabs
// of BK are staged through k-major LDS tiles (two or three stages).
template <int WM_, int WN_, int SM_, int SN_, int BK_, int WAVES_PER_SIMD_> struct MfmaCfg {
    static constexpr int WM = WM_, WN = WN_, SM = SM_, SN = SN_, BK = BK_;
    static constexpr int kWavesPerSimd = WAVES_PER_SIMD_; // occupancy the registers allow
    static constexpr int BM = WM * SM * 32, BN = WN * SN * 32;
    static constexpr int kThreads = 64 * WM * WN;
    static constexpr int LDA = BM + 4, LDB = BN + 4; // row pitch of the k-major LDS tiles
    static constexpr int EA = BM * BK / kThreads;    // A elements one thread stages per slab
    static constexpr int EB = BN * BK / kThreads;
    static_assert(EA % 4 == 0 && EB % 4 == 0, "staging moves whole float4s");
    // A thread staging several float4s of a B k-row takes them BN / (EB / 4) apart (measured
    // 1.5-2.5% faster for the native kernel's 16 elements than one contiguous run).
    template <bool TA> static constexpr bool kSplitRunsB = EB > 4;
};

// Direct global -> LDS load of 16 bytes a lane from base + off bytes: lane l's run lands at
// lds + 16 l bytes. base and lds are uniform across the wave; base stays in scalar registers
// (the scalar unit advances it), which the compiler's form of this load does not do. Issued
// from inline assembly, so the compiler does not track it: the caller waits for it
// (wait_lds_loads) before the barrier that publishes the stage.
__device__ __forceinline__ void load_lds16(const float *base, uint32_t off, float *lds)
{
    const uint32_t m0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)lds;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(m0), "v"(off), "s"(base)
                 : "memory", "m0");
}
__device__ __forceinline__ void wait_lds_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Wait until at most N of this wave's vector memory loads are outstanding: loads complete in
// the order they were issued, so every load before the last N has landed.
template <int N> __device__ __forceinline__ void wait_loads_but()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// WHOLE: every slab of every tile is whole (M, N, K multiples of the tile and slab, 16-byte
// loads allowed), so staging runs on advancing pointers with no bound checks.
// CHECK: the RejectSubnormal form with the partial-sum check (sck), its own instantiation so
// that the plain form keeps its registers and schedule.
// EPI: the whole-tile epilogue (three stages, two subtiles a wave) also evaluates `epi`, a
// ReLU (EPI = kStepRelu) or ReLU backward (kStepReluBackward) of each product cell, with the
// elementwise kernels' classification, recording into that node's own word.
template <class Cfg, bool TA, bool TB, bool VA, bool VB, bool WHOLE = false, bool CHECK = false,
          int EPI = 0>
__global__ __launch_bounds__(Cfg::kThreads, Cfg::kWavesPerSimd) void k_strict_gemm_mfma(
    const float *__restrict__ A, const float *__restrict__ B, float *__restrict__ C, int M,
    int N, int K, const unsigned long long *__restrict__ row_exp,
    const unsigned long long *__restrict__ col_exp, int thr, int check_risk,
    unsigned long long *suspect, SumCheck sck, NodeGate gate, GemmEpilogue epi)
{
    if (block_gate_closed(gate))
        return;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, SM = Cfg::SM, SN = Cfg::SN;
    constexpr int S = SM * SN;
    // Whole tiles run three LDS stages (see the slab loop); tiles with bound checks keep two,
    // since their staging needs more registers and three spill there.
    constexpr int kStages = WHOLE ? 3 : 2;
    // Whole tiles load op(A), and op(B) when untransposed, from global memory straight into
    // LDS (global_load_lds_dwordx4: no staging registers, no LDS stores); those stages are
    // unpadded (see the layouts at the direct loads below). A transposed op(B) goes through
    // registers, which turn its k-contiguous runs into k-major rows.
    constexpr bool kDirectA = WHOLE, kDirectB = WHOLE && !TB;
    constexpr int LDA = kDirectA ? BM : Cfg::LDA, LDB = kDirectB ? BN : Cfg::LDB;
    // Two stages are indexed at run time, three at compile time.
    __shared__ __align__(16) float As[2][BK][LDA];
    __shared__ __align__(16) float Bs[2][BK][LDB];
    __shared__ __align__(16) float As3[3][BK][LDA];
    __shared__ __align__(16) float Bs3[3][BK][LDB];
    auto sa = [&](auto st_c) -> float(*)[LDA] { return As3[decltype(st_c)::value]; };
    auto sb = [&](auto st_c) -> float(*)[LDB] { return Bs3[decltype(st_c)::value]; };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave / Cfg::WN) * SM * 32, wn = (wave % Cfg::WN) * SN * 32;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    // RejectSubnormal with the partial-sum check (sck.flag set) launches both forms over the
    // whole grid: a tile that may meet a product below 2^sck.thr is computed by the CHECK form,
    // which checks every partial sum it forms, and every other tile by the plain form. (One
    // kernel holding both loops spilled registers.)
    if (sck.flag != nullptr &&
        tile_exp_sum_below<BM, BN>(row_exp, col_exp, m0, n0, M, N, sck.thr) != CHECK)
        return;
    SubLanes subl; // lanes that met a nonzero subnormal partial sum
    const int cls = kClassSubnormal;
    auto run_form = [&](auto &&run) { run(std::integral_constant<bool, CHECK>{}); };
    // The checking form checks the superslabs that need it (SumGate).
    __shared__ unsigned char fine_ss[kSumMaxSuperSlabs];
    SumGate<BK> sgate{nullptr, false};
    bool chk = true; // the current slab's sums are checked (checking form)
    if constexpr (CHECK) {
        if (sck.tbl_a != nullptr) {
            tile_fine_superslabs<BM, BN>(sck, m0, n0, M, N, K, fine_ss);
            sgate.fine = fine_ss;
        }
    }

    float acc[S][16];
#pragma unroll
    for (int t = 0; t < S; t++)
#pragma unroll
        for (int r = 0; r < 16; r++)
            acc[t][r] = 0.0f;

    SlabStager<float, Cfg, TA, TB, VA, VB> stage;
    auto off_grid = [&]() {
        bool o = false;
#pragma unroll
        for (int t = 0; t < S; t++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                o |= sum_off_grid(acc[t][r]);
        return __builtin_amdgcn_ballot_w64(o) != 0;
    };
    // Slab kt; the checking form checks its sums when the gate opens it.
    auto gated = [&](auto &&slab_fn, int kt, auto ck) __attribute__((always_inline)) {
        if constexpr (decltype(ck)::value)
            chk = sgate.at(kt, off_grid);
        slab_fn(ck);
    };

    v32f zero;
#pragma unroll
    for (int r = 0; r < 32; r++)
        zero[r] = 0.0f;
    // Wave priority. With three stages, a wave raises its priority while it folds (1.8-1.9%
    // faster at 4096^3): a wave in the middle of its adds keeps issuing them, paired with
    // another wave's, rather than giving way to a wave ready to issue its MFMA. With two
    // stages, raising it around each MFMA issue measured about 0.8% faster at 4096^3 when
    // op(A) and op(B) are staged alike (both transposed or neither) and about 0.4% slower
    // otherwise, so it is used only there.
    constexpr bool kFoldPrio = WHOLE;
    constexpr bool kIssuePrio = !WHOLE && TA == TB;
    auto mma = [&](float a, float b) {
        if (kIssuePrio)
            __builtin_amdgcn_s_setprio(1);
        const v32f r = __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, zero, 0, 0, 0);
        if (kIssuePrio)
            __builtin_amdgcn_s_setprio(0);
        return r;
    };
    // Fold one MFMA's products into a subtile: each cell adds its k product (register r),
    // then its k+1 product (register 16 + r). The sixteen k sums go first, so no add waits
    // on the add just before it (measured 2-3% faster with a transposed operand).
    // The checking form tests each of the 32 sums for a nonzero subnormal as it is formed.
    auto fold = [&](float (&c)[16], const v32f &p, auto ck) {
        constexpr bool CK = decltype(ck)::value;
        if (kFoldPrio)
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int r = 0; r < 16; r++)
            c[r] = c[r] + p[r];
        if constexpr (CK) {
            if (chk) {
#pragma unroll
                for (int r = 0; r < 16; r += 4)
                    check_subnormal4(subl, c[r], c[r + 1], c[r + 2], c[r + 3], cls);
            }
        }
#pragma unroll
        for (int r = 0; r < 16; r++)
            c[r] = c[r] + p[16 + r];
        if constexpr (CK) {
            if (chk) {
#pragma unroll
                for (int r = 0; r < 16; r += 4)
                    check_subnormal4(subl, c[r], c[r + 1], c[r + 2], c[r + 3], cls);
            }
        }
        // Emits nothing; ties the sixteen sums to this point of the instruction stream.
        asm volatile("" : "+v"(c[0]), "+v"(c[1]), "+v"(c[2]), "+v"(c[3]), "+v"(c[4]), "+v"(c[5]),
                     "+v"(c[6]), "+v"(c[7]), "+v"(c[8]), "+v"(c[9]), "+v"(c[10]), "+v"(c[11]),
                     "+v"(c[12]), "+v"(c[13]), "+v"(c[14]), "+v"(c[15]));
        if (kFoldPrio)
            __builtin_amdgcn_s_setprio(0);
    };

    const int ktiles = (K + BK - 1) / BK;
    if (WHOLE)
        stage.begin_whole(A, B, M, N, K, m0, n0, tid);
    const int half = lane >> 5, col = lane & 31;
    if constexpr (kStages == 3) {
        // Three LDS stages: while slab kt is computed from stage kt % 3, slab kt + 1 is already
        // published (stashed during kt - 1, before that iteration's barrier) and slab kt + 2 is
        // staged into the stage slab kt - 1 used. So each wave reads slab kt + 1's first operands
        // and issues its first MFMA before the barrier that ends slab kt: the MFMA runs while
        // the wave waits there, and no slab starts from an empty pipeline.
        //
        // With two subtiles a wave (SN = 2), lane col of subtile j owns tile column
        // wn + 2 col + j, so its two B operands of a k row sit side by side and one 8-byte LDS
        // read, at an immediate offset from the lane's base, fetches both. With one (SN = 1) it
        // owns column wn + col.
        static_assert(SM == 1 && (SN == 1 || SN == 2), "the pipeline below is written for one or two subtiles a wave");
        //
        // Direct loads: each wave moves 1 KiB of op(A) and 1 KiB of op(B) per slab, lane l's 16
        // bytes landing at the wave's LDS base + 16 l. Stage layouts (floats):
        //  * op(B), and op(A) when transposed: k-major rows of R = BN (BM) floats; wave w fills
        //    256 / R consecutive rows from row 256 w / R, and odd rows are rotated by 32
        //    (element x at (x - 32) mod R), so the two half-waves of an operand read (rows 2j
        //    and 2j + 1) fall on different banks;
        //  * op(A) untransposed: k quads, element (k, m) at 4 BM (k / 4) + 4 m + k % 4, so each
        //    lane's 16 bytes (four consecutive k of one row) land whole; BM / 64 waves fill a
        //    quad, 64 rows each.
        constexpr int W = Cfg::kThreads / 64;
        static_assert(BM == 16 * W && BN == 16 * W, "each wave moves 1 KiB of each operand a slab");
        const int wv = __builtin_amdgcn_readfirstlane(wave);
        // Rows layout of R floats: the run (16 bytes) lane l moves, and its offset in floats
        // from the wave's first row; `stride` is the stored row pitch.
        auto row_run = [&](int R, uint64_t stride) {
            const int rr = lane / (R / 4), p = lane % (R / 4);
            const int c = (rr & 1) ? (p + 8) % (R / 4) : p;
            return (uint32_t)(((uint64_t)rr * stride + 4 * c) * 4);
        };
        // Element x of k row 2j + half, from the lane's base: 2 R j + off.
        auto row_off = [&](int R, int x) { return half ? R + ((x - 32) & (R - 1)) : x; };
        const float *ga = nullptr, *gb = nullptr; // wave-uniform bases
        uint32_t lo_a = 0, lo_b = 0;              // the lane's byte offsets from them
        size_t da = 0, db = 0;
        int la = 0, lb = 0, a_off = 0, b_off = 0;
        if constexpr (kDirectA) {
            if (!TA) {
                constexpr int WQ = BM / 64; // waves a quad
                ga = A + (size_t)(m0 + 64 * (wv % WQ)) * K + 4 * (wv / WQ);
                lo_a = (uint32_t)lane * (uint32_t)K * 4u;
                da = BK;
                la = 4 * BM * (wv / WQ) + 256 * (wv % WQ);
                a_off = 4 * (wm + col) + half;
            } else {
                ga = A + (size_t)(256 / BM * wv) * M + m0;
                lo_a = row_run(BM, (uint64_t)M);
                da = (size_t)BK * M;
                la = 256 * wv;
                a_off = row_off(BM, wm + col);
            }
        }
        if constexpr (kDirectB) {
            gb = B + (size_t)(256 / BN * wv) * N + n0;
            lo_b = row_run(BN, (uint64_t)N);
            db = (size_t)BK * N;
            lb = 256 * wv;
            b_off = row_off(BN, SN == 2 ? wn + 2 * col : wn + col);
        }
        // Stage the next slab into stage ST: direct loads, or global -> registers (the stash
        // to LDS follows at the end of the slab).
        auto load_slab = [&](auto st_c) {
            if constexpr (kDirectA) {
                load_lds16(ga, lo_a, &sa(st_c)[0][0] + la);
                ga += da;
            }
            if constexpr (kDirectB) {
                load_lds16(gb, lo_b, &sb(st_c)[0][0] + lb);
                gb += db;
            } else {
                stage.fetch_whole_b();
            }
        };
        auto stash_slab = [&](auto st_c) {
            if constexpr (!kDirectB)
                stage.stash_b(sb(st_c), tid);
        };
        if (ktiles > 0) {
            load_slab(std::integral_constant<int, 0>{});
            stash_slab(std::integral_constant<int, 0>{});
        }
        if (ktiles > 1) {
            load_slab(std::integral_constant<int, 1>{});
            stash_slab(std::integral_constant<int, 1>{});
        }
        wait_lds_loads();
        __syncthreads();
        // Software pipeline over the slab, unrolled: each MFMA is issued, then the products of
        // the one before it are folded. sched_barrier pins that order (left to the scheduler,
        // the same sequence measured about 8% slower). Each k-pair's operands are read from
        // LDS ahead into register slots used in turn: one pair ahead into two slots with two
        // subtiles (their MFMAs alternate within a pair), two pairs ahead into three slots
        // with one (each pair's MFMA is issued before the previous pair is folded). Lanes
        // 0-31 carry k = 2j, lanes 32-63 carry k = 2j + 1 (the MFMA's two blocks).
        constexpr int NP = BK / 2;
        constexpr int kSlots = SN == 2 ? 2 : 3, D = kSlots - 1;
        static_assert((3 * NP) % kSlots == 0, "a trip of three slabs ends on slot 0");
        // Register slot of pair j of the trip's slab c (j may run into the next slab).
        auto slot = [](int c, int j) { return (c * NP + j) % kSlots; };
        float oa[kSlots], ob[kSlots][SN];
        auto rd = [&](auto st_c, int g, int j) {
            if constexpr (kDirectA)
                oa[g] = (&sa(st_c)[0][0])[a_off + (TA ? 2 * BM * j : 4 * BM * (j >> 1) + 2 * (j & 1))];
            else
                oa[g] = sa(st_c)[2 * j + half][wm + col];
            if constexpr (SN == 2) {
                float2 v;
                if constexpr (kDirectB)
                    v = *reinterpret_cast<const float2 *>(&sb(st_c)[0][0] + b_off + 2 * BN * j);
                else
                    v = *reinterpret_cast<const float2 *>(&sb(st_c)[2 * j + half][wn + 2 * col]);
                ob[g][0] = v.x;
                ob[g][SN - 1] = v.y;
            } else if constexpr (kDirectB) {
                ob[g][0] = (&sb(st_c)[0][0])[b_off + 2 * BN * j];
            } else {
                ob[g][0] = sb(st_c)[2 * j + half][wn + col];
            }
        };
        v32f p;
        if (ktiles > 0) {
#pragma unroll
            for (int j = 0; j < D; j++)
                rd(std::integral_constant<int, 0>{}, slot(0, j), j);
            p = mma(oa[0], ob[0][0]);
        }
        // One slab computed from stage CUR; the loop below runs three slabs per trip, so every
        // stage index, and with it every LDS address, is fixed at compile time.
        auto slab = [&](auto cur_c, int kt, auto ck) __attribute__((always_inline)) {
            constexpr int cur = decltype(cur_c)::value, nn = (cur + 2) % 3;
            const std::integral_constant<int, (cur + 1) % 3> nxt_c;
            const std::integral_constant<int, nn> nn_c;
            const bool has_next = kt + 1 < ktiles;
            if (kt + 2 < ktiles)
                load_slab(nn_c);
#pragma unroll
            for (int j = 0; j < NP; j++) {
                if (j + D < NP)
                    rd(cur_c, slot(cur, j + D), j + D);
                else if (has_next)
                    rd(nxt_c, slot(cur, j + D), j + D - NP);
                const int g = slot(cur, j), g1 = slot(cur, j + 1);
                if constexpr (SN == 2) {
                    const v32f q = mma(oa[g], ob[g][SN - 1]);
                    __builtin_amdgcn_sched_barrier(0);
                    fold(acc[0], p, ck);
                    __builtin_amdgcn_sched_barrier(0);
                    if (j + 1 < NP || has_next)
                        p = mma(oa[g1], ob[g1][0]);
                    __builtin_amdgcn_sched_barrier(0);
                    fold(acc[SN - 1], q, ck);
                    __builtin_amdgcn_sched_barrier(0);
                } else {
                    v32f q;
                    const bool more = j + 1 < NP || has_next;
                    if (more)
                        q = mma(oa[g1], ob[g1][0]);
                    __builtin_amdgcn_sched_barrier(0);
                    fold(acc[0], p, ck);
                    __builtin_amdgcn_sched_barrier(0);
                    if (more)
                        p = q;
                }
            }
            if (kt + 2 < ktiles)
                stash_slab(nn_c);
            wait_lds_loads();
            __syncthreads();
        };
        auto run = [&](auto ck) {
            for (int kt = 0; kt < ktiles; kt += 3) {
                gated([&](auto c) { slab(std::integral_constant<int, 0>{}, kt, c); }, kt, ck);
                if (kt + 1 < ktiles)
                    gated([&](auto c) { slab(std::integral_constant<int, 1>{}, kt + 1, c); }, kt + 1, ck);
                if (kt + 2 < ktiles)
                    gated([&](auto c) { slab(std::integral_constant<int, 2>{}, kt + 2, c); }, kt + 2, ck);
            }
        };
        run_form(run);
    } else {
        if (ktiles > 0) {
            if (WHOLE)
                stage.fetch_whole();
            else
                stage.fetch(A, B, M, N, K, m0, n0, 0, tid);
            stage.stash(As[0], Bs[0], tid);
        }
        __syncthreads();
        auto slab2 = [&](int kt, auto ck) __attribute__((always_inline)) {
            const int cur = kt & 1;
            if (kt + 1 < ktiles) {
                if (WHOLE)
                    stage.fetch_whole();
                else
                    stage.fetch(A, B, M, N, K, m0, n0, (kt + 1) * BK, tid);
            }
            // Software pipeline over the whole slab, unrolled: each MFMA is issued, then the
            // products of the one before it are folded. sched_barrier pins that order (left to
            // the scheduler, the same sequence measured about 8% slower), and each k-pair's
            // operands are read from LDS one pair ahead. Lanes 0-31 carry k = 2j, lanes 32-63
            // carry k = 2j + 1 (the MFMA's two blocks).
            constexpr int NP = BK / 2;
            float oa[NP][SM], ob[NP][SN];
            auto rd = [&](int j) {
#pragma unroll
                for (int i = 0; i < SM; i++)
                    oa[j][i] = As[cur][2 * j + half][wm + 32 * i + col];
#pragma unroll
                for (int jj = 0; jj < SN; jj++)
                    ob[j][jj] = Bs[cur][2 * j + half][wn + 32 * jj + col];
            };
            static_assert(SM == 1 && (SN == 1 || SN == 2), "the pipeline below is written for one or two subtiles a wave");
            if constexpr (SN == 2) {
                rd(0);
                v32f p = mma(oa[0][0], ob[0][0]);
#pragma unroll
                for (int j = 0; j < NP; j++) {
                    if (j + 1 < NP)
                        rd(j + 1);
                    const v32f q = mma(oa[j][0], ob[j][SN - 1]);
                    __builtin_amdgcn_sched_barrier(0);
                    fold(acc[0], p, ck);
                    __builtin_amdgcn_sched_barrier(0);
                    if (j + 1 < NP)
                        p = mma(oa[j + 1][0], ob[j + 1][0]);
                    __builtin_amdgcn_sched_barrier(0);
                    fold(acc[SN - 1], q, ck);
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
                // One subtile: each pair's MFMA is issued before the previous pair is folded,
                // operands read two pairs ahead.
                rd(0);
                rd(1);
                v32f p = mma(oa[0][0], ob[0][0]);
#pragma unroll
                for (int j = 0; j < NP; j++) {
                    if (j + 2 < NP)
                        rd(j + 2);
                    v32f q;
                    if (j + 1 < NP)
                        q = mma(oa[j + 1][0], ob[j + 1][0]);
                    __builtin_amdgcn_sched_barrier(0);
                    fold(acc[0], p, ck);
                    __builtin_amdgcn_sched_barrier(0);
                    if (j + 1 < NP)
                        p = q;
                }
            }
            if (kt + 1 < ktiles)
                stage.stash(As[cur ^ 1], Bs[cur ^ 1], tid);
            __syncthreads();
        };
        auto run = [&](auto ck) {
            for (int kt = 0; kt < ktiles; kt++)
                gated([&](auto c) { slab2(kt, c); }, kt, ck);
        };
        run_form(run);
    }

    // Epilogue: for subtile (i, j) the lane owns rows m0+wm+32i+8(r/4)+4*half+(r%4) of column
    // n0+wn+2col+j (three stages, two subtiles: both columns in one 8-byte store, every cell
    // inside M x N) or n0+wn+32j+col.
    const bool sub = CHECK && ((subl.flush() >> lane) & 1);
    uint64_t key = kNoFault;
    if constexpr (kStages == 3 && SN == 1) {
        const int c = n0 + wn + col;
        const int cexp = check_risk ? exp_of(col_exp[c]) : 0;
        if (sub) // the lane's cells: rows m0 + wm .. m0 + wm + 31 of column c
            flag_sum_block(sck, m0 + wm, c);
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = m0 + wm + 8 * (r >> 2) + 4 * half + (r & 3);
            const float v = acc[0][r];
            C[(size_t)row * N + c] = v;
            bool bad = !finite_bits(v) || sub;
            if (check_risk)
                bad |= exp_of(row_exp[row]) + cexp < thr;
            const uint64_t cell = (uint64_t)row * N + c;
            if (bad)
                key = cell < key ? cell : key;
        }
        block_record_min<Cfg::kThreads / 64>(key, suspect);
        return;
    } else if constexpr (kStages == 3) {
        const int c = n0 + wn + 2 * col;
        const int cexp0 = check_risk ? exp_of(col_exp[c]) : 0;
        const int cexp1 = check_risk ? exp_of(col_exp[c + 1]) : 0;
        if (sub) // rows m0 + wm .. m0 + wm + 31 of columns c and c + 1 (c even): one block
            flag_sum_block(sck, m0 + wm, c);
        uint64_t ekey = kNoFault; // the epilogue node's first fault in this lane
        // The node's exponents for its superslab tables: per row of the lane (over its two
        // columns) and per column (over its 16 rows).
        const bool tbl = EPI != 0 && (epi.tbl_rows != nullptr || epi.tbl_cols != nullptr);
        int erow[EPI != 0 ? 16 : 1];
        int ecol0 = kExpNone, ecol1 = kExpNone;
        // The ReLU backward's input at the lane's 32 cells, all loaded before the first
        // store (a load after each store would wait out its latency 16 times).
        float2 xin[EPI == kStepReluBackward ? 16 : 1];
        if constexpr (EPI == kStepReluBackward) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm + 8 * (r >> 2) + 4 * half + (r & 3);
                xin[r] = *reinterpret_cast<const float2 *>(
                    &static_cast<const float *>(epi.x)[(size_t)row * N + c]);
            }
        }
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = m0 + wm + 8 * (r >> 2) + 4 * half + (r & 3);
            const float v0 = acc[0][r], v1 = acc[1][r];
            *reinterpret_cast<float2 *>(&C[(size_t)row * N + c]) = make_float2(v0, v1);
            bool bad0 = !finite_bits(v0) || sub, bad1 = !finite_bits(v1) || sub;
            if (check_risk) {
                const int rexp = exp_of(row_exp[row]);
                bad0 |= rexp + cexp0 < thr;
                bad1 |= rexp + cexp1 < thr;
            }
            const uint64_t cell = (uint64_t)row * N + c;
            if (bad0)
                key = cell < key ? cell : key;
            else if (bad1)
                key = cell + 1 < key ? cell + 1 : key;
            if constexpr (EPI != 0) {
                float r0, r1;
                uint32_t k0, k1;
                if constexpr (EPI == kStepRelu) {
                    r0 = relu_select(v0);
                    r1 = relu_select(v1);
                    k0 = classify_relu(v0, r0, epi.policy);
                    k1 = classify_relu(v1, r1, epi.policy);
                } else {
                    const float2 x = xin[r];
                    r0 = strictly_positive(x.x) ? v0 : 0.0f;
                    r1 = strictly_positive(x.y) ? v1 : 0.0f;
                    k0 = classify_relu_backward(x.x, v0, r0, epi.policy);
                    k1 = classify_relu_backward(x.y, v1, r1, epi.policy);
                }
                *reinterpret_cast<float2 *>(&static_cast<float *>(epi.out)[(size_t)row * N + c]) =
                    make_float2(r0, r1);
                if (tbl) {
                    const int e0 = ilog2_abs(r0), e1 = ilog2_abs(r1);
                    erow[r] = e0 < e1 ? e0 : e1;
                    ecol0 = e0 < ecol0 ? e0 : ecol0;
                    ecol1 = e1 < ecol1 ? e1 : ecol1;
                }
                const uint64_t e = k0 != kOk ? pack_fault(cell, k0)
                                 : k1 != kOk ? pack_fault(cell + 1, k1) : kNoFault;
                ekey = e < ekey ? e : ekey;
            }
        }
        if constexpr (EPI != 0) {
            if (epi.tbl_rows != nullptr) {
                // Row minima over the wave's 64 columns (one superslab): each exchange among
                // the 32 lanes of a half hands over half of the rows still held, so after
                // five the lane holds row r = col / 2 (16 exchanges rather than 80).
#pragma unroll
                for (int w = 8; w >= 1; w >>= 1) {
                    const int bit = 2 * w; // partner lane: col ^ bit
                    const bool upper = (col & bit) != 0;
#pragma unroll
                    for (int i = 0; i < w; i++) {
                        const int give = upper ? erow[i] : erow[i + w];
                        const int keep = upper ? erow[i + w] : erow[i];
                        const int got = __shfl_xor(give, bit, 64);
                        erow[i] = got < keep ? got : keep;
                    }
                }
                {
                    const int got = __shfl_xor(erow[0], 1, 64);
                    const int e = got < erow[0] ? got : erow[0];
                    const int r = col >> 1;
                    if ((col & 1) == 0) {
                        const int row = m0 + wm + 8 * (r >> 2) + 4 * half + (r & 3);
                        epi.tbl_rows[(size_t)row * (N / 64) + (n0 + wn) / 64] = scan_exp(e);
                    }
                }
            }
            if (epi.tbl_cols != nullptr) {
                // Column minima over the wave's 32 rows; the two waves of a 64-row superslab
                // (wm and wm + 32, the same columns) meet in LDS.
                __shared__ int csub[2][Cfg::BN];
                int o = __shfl_xor(ecol0, 32, 64);
                ecol0 = o < ecol0 ? o : ecol0;
                o = __shfl_xor(ecol1, 32, 64);
                ecol1 = o < ecol1 ? o : ecol1;
                const int ss = wm / 64;
                const bool lead = (wm / 32) % 2 == 0;
                if (lead && half == 0) {
                    csub[ss][wn + 2 * col] = ecol0;
                    csub[ss][wn + 2 * col + 1] = ecol1;
                }
                __syncthreads();
                if (!lead && half == 0) {
                    const int p0 = csub[ss][wn + 2 * col], p1 = csub[ss][wn + 2 * col + 1];
                    const int f0 = p0 < ecol0 ? p0 : ecol0, f1 = p1 < ecol1 ? p1 : ecol1;
                    short *t = epi.tbl_cols + (size_t)(m0 / 64 + ss) * N + c;
                    t[0] = scan_exp(f0);
                    t[1] = scan_exp(f1);
                }
            }
            wave_record_fault(ekey, epi.fault, epi.gate);
        }
        block_record_min<Cfg::kThreads / 64>(key, suspect);
        return;
    }
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int i = t / SN, j = t % SN;
        const int c = n0 + wn + 32 * j + col;
        const bool cin = c < N;
        const int cexp = (check_risk && cin) ? exp_of(col_exp[c]) : 0;
        if (sub && cin && m0 + wm + 32 * i < M) // subtile t: one 32 x 32 block
            flag_sum_block(sck, m0 + wm + 32 * i, c);
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * half + (r & 3);
            if (!cin || row >= M)
                continue;
            const float v = acc[t][r];
            C[(size_t)row * N + c] = v;
            bool bad = !finite_bits(v) || sub;
            if (check_risk)
                bad |= exp_of(row_exp[row]) + cexp < thr;
            if (bad) {
                const uint64_t cell = (uint64_t)row * N + c;
                key = cell < key ? cell : key;
            }
        }
    }
    block_record_min<Cfg::kThreads / 64>(key, suspect);
}

// ------------------------------------------------------- 16 x 16 waves, whole tiles
// Outputs too small to give every SIMD several 32 x 32 waves (fewer 128 x 128 tiles than
// CUs): 64 x 64 tiles of sixteen 16 x 16 waves, four times the waves of 32 x 32 subtiles.
// v_mfma_f32_16x16x1_4b_f32 multiplies, in block b, A lane 16 b + i by B lane 16 b + j, and
// lane L's register 4 b + q holds block b's (i = 4 (L / 16) + q, j = L % 16). The four blocks
// carry k0 .. k0 + 3, so each lane folds, for each of its four cells q, registers q, 4 + q,
// 8 + q and 12 + q in k order: 16 adds per 1024 products, the same ceiling as the 32 x 32
// engine. Both operands load straight into LDS in every layout:
//  * k-contiguous (op(A) untransposed, op(B) transposed): k quads, element (k, x) at
//    256 (k / 4) + 4 x + k % 4; one wave instruction fills a quad (64 rows of 16 bytes), and
//    a lane's operand read (x = w + L % 16, k = 4 q + L / 16) covers 64 consecutive words;
//  * x-contiguous (op(A) transposed, op(B) untransposed): k rows of 64 floats, row k rotated
//    by 16 (k % 4), element (k, x) at 64 k + (x + 16 (k % 4)) % 64; one instruction fills four
//    rows, each lane fetching the global run that lands rotated, and the read (four rows, 16
//    columns each) meets 64 distinct banks.
typedef float v16f __attribute__((ext_vector_type(16)));

template <bool TA, bool TB, bool CHECK = false>
__global__ __launch_bounds__(1024, 2) void k_strict_gemm_mfma16(
    const float *__restrict__ A, const float *__restrict__ B, float *__restrict__ C, int M,
    int N, int K, const unsigned long long *__restrict__ row_exp,
    const unsigned long long *__restrict__ col_exp, int thr, int check_risk,
    unsigned long long *suspect, SumCheck sck, NodeGate gate)
{
    if (block_gate_closed(gate))
        return;
    constexpr int T = 64, BK = 16, SZ = T * BK; // tile side, slab, floats a stage
    __shared__ __align__(16) float As0[SZ], As1[SZ], As2[SZ];
    __shared__ __align__(16) float Bs0[SZ], Bs1[SZ], Bs2[SZ];
    auto sa = [&](auto st_c) -> float * {
        constexpr int st = decltype(st_c)::value;
        return st == 0 ? As0 : (st == 1 ? As1 : As2);
    };
    auto sb = [&](auto st_c) -> float * {
        constexpr int st = decltype(st_c)::value;
        return st == 0 ? Bs0 : (st == 1 ? Bs1 : Bs2);
    };
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = 16 * (wv >> 2), wn = 16 * (wv & 3);
    int tm, tn;
    tile_of(blockIdx.x, M / T, N / T, tm, tn);
    const int m0 = tm * T, n0 = tn * T;
    // RejectSubnormal with the partial-sum check: each form takes its own tiles, as in
    // k_strict_gemm_mfma.
    if (sck.flag != nullptr &&
        tile_exp_sum_below<T, T>(row_exp, col_exp, m0, n0, M, N, sck.thr) != CHECK)
        return;
    SubLanes subl;
    const int cls = kClassSubnormal;
    __shared__ unsigned char fine_ss[kSumMaxSuperSlabs];
    SumGate<BK> sgate{nullptr, false};
    bool chk = true; // the current slab's sums are checked (checking form)
    if constexpr (CHECK) {
        if (sck.tbl_a != nullptr) {
            tile_fine_superslabs<T, T>(sck, m0, n0, M, N, K, fine_ss);
            sgate.fine = fine_ss;
        }
    }

    // Loads: waves 0-3 move op(A), waves 4-7 op(B), one 1 KiB instruction each a slab
    // (quad g or rows 4 g .. 4 g + 3 of the slab, g = wave % 4).
    const bool loads = wv < 8, load_a = wv < 4;
    const int g = wv & 3;
    const bool kcontig = load_a ? !TA : TB;        // this wave's operand is k-contiguous
    const float *X = load_a ? A : B;
    const int ld = load_a ? (TA ? M : K) : (TB ? K : N);
    const int x0 = load_a ? m0 : n0;
    const float *gx = nullptr; // wave-uniform base, advancing BK along k a slab
    uint32_t lo = 0;          // the lane's byte offset from it
    size_t dk = 0;
    if (loads) {
        if (kcontig) {
            gx = X + (size_t)x0 * ld + 4 * g;
            lo = (uint32_t)lane * (uint32_t)ld * 4u;
            dk = BK;
        } else {
            const int r = lane >> 4, c = lane & 15;
            gx = X + (size_t)(4 * g) * ld + x0;
            lo = (uint32_t)((r * ld + 4 * ((c - 4 * r) & 15)) * 4);
            dk = (size_t)BK * ld;
        }
    }
    // In both layouts instruction g fills floats 256 g .. 256 g + 255 of the stage.
    auto load_slab = [&](auto st_c) {
        if (loads) {
            load_lds16(gx, lo, (load_a ? sa(st_c) : sb(st_c)) + 256 * g);
            gx += dk;
        }
    };
    // The lane's operand offsets in a stage (quad q adds 256 q in both layouts).
    const int i = lane & 15, b = lane >> 4;
    const int oa = !TA ? 4 * (wm + i) + b : 64 * b + ((wm + i + 16 * b) & 63);
    const int ob = TB ? 4 * (wn + i) + b : 64 * b + ((wn + i + 16 * b) & 63);

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    v16f zero;
#pragma unroll
    for (int r = 0; r < 16; r++)
        zero[r] = 0.0f;
    // Fold one MFMA's products: each cell q adds its k0, k0 + 1, k0 + 2, k0 + 3 products in
    // turn; the four cells' chains interleave.
    auto fold = [&](const v16f &p, auto ck) {
        constexpr bool CK = decltype(ck)::value;
#pragma unroll
        for (int blk = 0; blk < 4; blk++) {
#pragma unroll
            for (int q = 0; q < 4; q++)
                acc[q] = acc[q] + p[4 * blk + q];
            if constexpr (CK) {
                if (chk)
                    check_subnormal4(subl, acc[0], acc[1], acc[2], acc[3], cls);
            }
        }
        asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]));
    };
    const int ktiles = K / BK;
    if (ktiles > 0) {
        load_slab(std::integral_constant<int, 0>{});
        if (ktiles > 1)
            load_slab(std::integral_constant<int, 1>{});
    }
    wait_lds_loads();
    __syncthreads();
    auto slab = [&](auto cur_c, int kt, auto ck) __attribute__((always_inline)) {
        constexpr int cur = decltype(cur_c)::value;
        if (kt + 2 < ktiles)
            load_slab(std::integral_constant<int, (cur + 2) % 3>{});
        const float *as = sa(cur_c), *bs = sb(cur_c);
        float a[4], bb[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            a[q] = as[oa + 256 * q];
            bb[q] = bs[ob + 256 * q];
        }
        v16f p = __builtin_amdgcn_mfma_f32_16x16x1f32(a[0], bb[0], zero, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            v16f nx;
            if (q + 1 < 4)
                nx = __builtin_amdgcn_mfma_f32_16x16x1f32(a[q + 1], bb[q + 1], zero, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            fold(p, ck);
            __builtin_amdgcn_sched_barrier(0);
            if (q + 1 < 4)
                p = nx;
        }
        // The next slab must be in LDS before the barrier publishes it; a loading wave's
        // one load for slab kt + 2, issued this slab, may stay in flight.
        if (loads && kt + 2 < ktiles)
            wait_loads_but<1>();
        else
            wait_lds_loads();
        __syncthreads();
    };
    auto off_grid = [&]() {
        bool o = false;
#pragma unroll
        for (int q = 0; q < 4; q++)
            o |= sum_off_grid(acc[q]);
        return __builtin_amdgcn_ballot_w64(o) != 0;
    };
    auto gated = [&](auto cur_c, int kt, auto ck) __attribute__((always_inline)) {
        if constexpr (decltype(ck)::value)
            chk = sgate.at(kt, off_grid);
        slab(cur_c, kt, ck);
    };
    auto run = [&](auto ck) {
        for (int kt = 0; kt < ktiles; kt += 3) {
            gated(std::integral_constant<int, 0>{}, kt, ck);
            if (kt + 1 < ktiles)
                gated(std::integral_constant<int, 1>{}, kt + 1, ck);
            if (kt + 2 < ktiles)
                gated(std::integral_constant<int, 2>{}, kt + 2, ck);
        }
    };
    run(std::integral_constant<bool, CHECK>{});
    // Epilogue: cells (m0 + wm + 4 (lane / 16) + q, n0 + wn + lane % 16).
    const bool sub = CHECK && ((subl.flush() >> lane) & 1);
    uint64_t key = kNoFault;
    const int c = n0 + wn + i;
    const int cexp = check_risk ? exp_of(col_exp[c]) : 0;
    if (sub) // rows m0 + wm .. m0 + wm + 15 of column c: one 32 x 32 block
        flag_sum_block(sck, m0 + wm, c);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int row = m0 + wm + 4 * b + q;
        const float v = acc[q];
        C[(size_t)row * N + c] = v;
        bool bad = !finite_bits(v) || sub;
        if (check_risk)
            bad |= exp_of(row_exp[row]) + cexp < thr;
        const uint64_t cell = (uint64_t)row * N + c;
        if (bad)
            key = cell < key ? cell : key;
    }
    block_record_min<16>(key, suspect);
}

static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Measurement aid: a copy of known traffic whose reads are global_load_lds_dwordx4, the load
// the whole matrix-core tiles stage with, so that the HBM read counter can be scaled for
// that load (it is scaled for ordinary loads by a copy kernel of ordinary loads). Each
// workgroup moves 4 KiB chunks: wave w loads bytes 1024 w .. 1024 w + 1023 of the chunk
// into its own LDS kilobyte, waits for it, and each lane stores its 16 bytes with an ordinary
// 16-byte store.
__global__ __launch_bounds__(256) void k_direct_copy(const float *src, float *dst, uint64_t chunks)
{
    __shared__ __align__(16) float buf[1024];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
    for (uint64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
        const float *g = src + c * 1024 + (uint64_t)wave * 256;
        load_lds16(g, (uint32_t)lane * 16u, buf + wave * 256);
        wait_lds_loads();
        const float4 v = *reinterpret_cast<const float4 *>(buf + wave * 256 + lane * 4);
        // The store consumes the LDS read, so the read has completed before the wave's next
        // direct load (an asm statement with a memory clobber) overwrites the kilobyte.
        *reinterpret_cast<float4 *>(dst + c * 1024 + (uint64_t)wave * 256 + lane * 4) = v;
    }
}

hipError_t launch_direct_copy(hipStream_t s, const void *src, void *dst, uint64_t bytes)
{
    if (bytes == 0 || bytes % 4096 != 0 || !aligned16(src) || !aligned16(dst))
        return hipErrorInvalidValue;
    const uint64_t chunks = bytes / 4096;
    const unsigned grid = (unsigned)(chunks < 8192 ? chunks : 8192);
    hipLaunchKernelGGL(k_direct_copy, dim3(grid), dim3(256), 0, s, (const float *)src, (float *)dst, chunks);
    return hipGetLastError();
}

template <class Cfg, bool TA, bool TB>
static void mfma_dispatch(hipStream_t s, const float *A, const float *B, float *C, int M, int N,
                          int K, const unsigned long long *re, const unsigned long long *ce,
                          int thr, int risk, unsigned long long *suspect, SumCheck sck,
                          NodeGate gate, const GemmEpilogue *epi, bool *epi_done)
{
    const dim3 grid((unsigned)(((M + Cfg::BM - 1) / Cfg::BM) * ((N + Cfg::BN - 1) / Cfg::BN)));
    const dim3 block(Cfg::kThreads);
    const bool va = (TA ? (M % 4 == 0) : (K % 4 == 0)) && aligned16(A);
    const bool vb = (TB ? (K % 4 == 0) : (N % 4 == 0)) && aligned16(B);
    // Whole tiles store C two floats at a time and load op(A), and op(B) when untransposed,
    // directly: a lane's byte offset from its wave's base must fit 32 bits (at most 63 rows of
    // op(A) untransposed, else at most one row and 128 floats).
    const uint64_t span_a = TA ? (uint64_t)M + 128 : 64 * (uint64_t)K, span_b = (uint64_t)N + 128;
    const bool offsets32 = 4 * span_a <= UINT32_MAX && (TB || 4 * span_b <= UINT32_MAX);
    const bool whole = va && vb && M % Cfg::BM == 0 && N % Cfg::BN == 0 && K % Cfg::BK == 0 &&
                       ((uintptr_t)C & 7u) == 0 && offsets32;
    if constexpr (Cfg::SN == 2) {
        // The whole-tile epilogue evaluates an elementwise node with the product.
        if (whole && epi && (epi->op == kStepRelu || epi->op == kStepReluBackward)) {
            if (epi->op == kStepRelu) {
                hipLaunchKernelGGL((k_strict_gemm_mfma<Cfg, TA, TB, true, true, true, false, kStepRelu>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, *epi);
                if (sck.flag)
                    hipLaunchKernelGGL((k_strict_gemm_mfma<Cfg, TA, TB, true, true, true, true, kStepRelu>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, *epi);
            } else {
                hipLaunchKernelGGL((k_strict_gemm_mfma<Cfg, TA, TB, true, true, true, false, kStepReluBackward>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, *epi);
                if (sck.flag)
                    hipLaunchKernelGGL((k_strict_gemm_mfma<Cfg, TA, TB, true, true, true, true, kStepReluBackward>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, *epi);
            }
            if (epi_done)
                *epi_done = true;
            return;
        }
    }
    if (whole)
        { hipLaunchKernelGGL((k_strict_gemm_mfma<Cfg, TA, TB, true, true, true>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, GemmEpilogue{}); if (sck.flag) hipLaunchKernelGGL((k_strict_gemm_mfma<Cfg, TA, TB, true, true, true, true>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, GemmEpilogue{}); }
    else if (va && vb)
        { hipLaunchKernelGGL((k_strict_gemm_mfma<Cfg, TA, TB, true, true, false>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, GemmEpilogue{}); if (sck.flag) hipLaunchKernelGGL((k_strict_gemm_mfma<Cfg, TA, TB, true, true, false, true>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, GemmEpilogue{}); }
    else if (va)
        { hipLaunchKernelGGL((k_strict_gemm_mfma<Cfg, TA, TB, true, false, false>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, GemmEpilogue{}); if (sck.flag) hipLaunchKernelGGL((k_strict_gemm_mfma<Cfg, TA, TB, true, false, false, true>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, GemmEpilogue{}); }
    else if (vb)
        { hipLaunchKernelGGL((k_strict_gemm_mfma<Cfg, TA, TB, false, true, false>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, GemmEpilogue{}); if (sck.flag) hipLaunchKernelGGL((k_strict_gemm_mfma<Cfg, TA, TB, false, true, false, true>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, GemmEpilogue{}); }
    else
        { hipLaunchKernelGGL((k_strict_gemm_mfma<Cfg, TA, TB, false, false, false>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, GemmEpilogue{}); if (sck.flag) hipLaunchKernelGGL((k_strict_gemm_mfma<Cfg, TA, TB, false, false, false, true>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, GemmEpilogue{}); }
}

template <class Cfg>
static void mfma_launch(hipStream_t s, int M, int N, int K, bool ta, bool tb, const float *A,
                        const float *B, float *C, const unsigned long long *re,
                        const unsigned long long *ce, int thr,
                        int risk, unsigned long long *suspect, SumCheck sck, NodeGate gate,
                        const GemmEpilogue *epi = nullptr, bool *epi_done = nullptr)
{
    if (!ta && !tb) mfma_dispatch<Cfg, false, false>(s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, epi, epi_done);
    else if (!ta && tb) mfma_dispatch<Cfg, false, true>(s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, epi, epi_done);
    else if (ta && !tb) mfma_dispatch<Cfg, true, false>(s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, epi, epi_done);
    else mfma_dispatch<Cfg, true, true>(s, A, B, C, M, N, K, re, ce, thr, risk, suspect, sck, gate, epi, epi_done);
}

// 8 waves of 32 x 64 over a 128 x 128 tile, 123-126 VGPRs (4 waves per SIMD). On MI355X at
// 4096^3 this measured ahead of 4 waves of 64 x 64 (2 waves per SIMD), 16 waves of
// 32 x 32, a 256 x 128 tile, 4-wave tiles of 128 x 64 and 64 x 64, and BK = 32 (which
// spills with the pinned slab).
using GemmCfg = MfmaCfg<4, 2, 1, 2, 16, 4>;
// Outputs of fewer 128 x 128 tiles than CUs: 64 x 64 tiles of four 32 x 32 waves spread the
// same work over four times the workgroups (one wave a SIMD on more CUs rather than two on
// fewer).
using SmallCfg = MfmaCfg<2, 2, 1, 1, 16, 4>;

hipError_t launch_gemm_mfma_f32(hipStream_t s, int M, int N, int K, bool ta, bool tb,
                                const float *A, const float *B, float *C,
                                const unsigned long long *row_exp,
                                const unsigned long long *col_exp, int thr, int risk,
                                unsigned long long *suspect, SumCheck sck, NodeGate gate,
                                const GemmEpilogue *epi, bool *epi_done)
{
    const uint64_t big_tiles = (uint64_t)((M + GemmCfg::BM - 1) / GemmCfg::BM) * ((N + GemmCfg::BN - 1) / GemmCfg::BN);
    // 16 x 16 waves: whole 64 x 64 tiles, 16-byte loads, lane offsets within 32 bits, and
    // at most one round of their workgroups (two 16-wave workgroups a CU): measured 25-30%
    // faster than the 4-wave 64 x 64 tile at 1024^3, 512 x 4096 x 512 and 768 x 2048 x 768,
    // 3% slower at 1920 x 1024 x 1920 (900 tiles).
    const auto fits32 = [](uint64_t bytes) { return bytes <= UINT32_MAX; };
    const uint64_t lda = ta ? (uint64_t)M : (uint64_t)K, ldb = tb ? (uint64_t)K : (uint64_t)N;
    const bool w16 = M % 64 == 0 && N % 64 == 0 && K % 16 == 0 && aligned16(A) && aligned16(B) &&
                     (uint64_t)(M / 64) * (N / 64) <= 512 &&
                     fits32(ta ? (3 * lda + 64) * 4 : 64 * lda * 4) &&
                     fits32(tb ? 64 * ldb * 4 : (3 * ldb + 64) * 4);
    if (big_tiles < 256 && w16) {
        const dim3 grid((unsigned)((M / 64) * (N / 64)));
        if (!ta && !tb) { hipLaunchKernelGGL((k_strict_gemm_mfma16<false, false>), grid, dim3(1024), 0, s, A, B, C, M, N, K, row_exp, col_exp, thr, risk, suspect, sck, gate); if (sck.flag) hipLaunchKernelGGL((k_strict_gemm_mfma16<false, false, true>), grid, dim3(1024), 0, s, A, B, C, M, N, K, row_exp, col_exp, thr, risk, suspect, sck, gate); }
        else if (!ta && tb) { hipLaunchKernelGGL((k_strict_gemm_mfma16<false, true>), grid, dim3(1024), 0, s, A, B, C, M, N, K, row_exp, col_exp, thr, risk, suspect, sck, gate); if (sck.flag) hipLaunchKernelGGL((k_strict_gemm_mfma16<false, true, true>), grid, dim3(1024), 0, s, A, B, C, M, N, K, row_exp, col_exp, thr, risk, suspect, sck, gate); }
        else if (ta && !tb) { hipLaunchKernelGGL((k_strict_gemm_mfma16<true, false>), grid, dim3(1024), 0, s, A, B, C, M, N, K, row_exp, col_exp, thr, risk, suspect, sck, gate); if (sck.flag) hipLaunchKernelGGL((k_strict_gemm_mfma16<true, false, true>), grid, dim3(1024), 0, s, A, B, C, M, N, K, row_exp, col_exp, thr, risk, suspect, sck, gate); }
        else { hipLaunchKernelGGL((k_strict_gemm_mfma16<true, true>), grid, dim3(1024), 0, s, A, B, C, M, N, K, row_exp, col_exp, thr, risk, suspect, sck, gate); if (sck.flag) hipLaunchKernelGGL((k_strict_gemm_mfma16<true, true, true>), grid, dim3(1024), 0, s, A, B, C, M, N, K, row_exp, col_exp, thr, risk, suspect, sck, gate); }
        return hipGetLastError();
    }
    if (big_tiles < 256)
        mfma_launch<SmallCfg>(s, M, N, K, ta, tb, A, B, C, row_exp, col_exp, thr, risk, suspect, sck, gate);
    else
        mfma_launch<GemmCfg>(s, M, N, K, ta, tb, A, B, C, row_exp, col_exp, thr, risk, suspect, sck, gate, epi, epi_done);
    return hipGetLastError();
}


// ------------------------------------------------------------ native F32 MatMul
// Explicitly permitted native compound arithmetic (Boundary + BackendDefined): the matrix
// cores accumulate, v_mfma_f32_32x32x2_f32 folding k and k+1 of a 32x32 subtile per
// instruction in their own order and rounding. No fault is classified.
template <class Cfg, bool TA, bool TB, bool VA, bool VB, bool WHOLE = false>
__global__ __launch_bounds__(Cfg::kThreads, Cfg::kWavesPerSimd) void k_native_gemm_mfma(
    const float *__restrict__ A, const float *__restrict__ B, float *__restrict__ C, int M,
    int N, int K, NodeGate gate)
{
    if (block_gate_closed(gate))
        return;
    typedef float v16f __attribute__((ext_vector_type(16)));
    constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, SM = Cfg::SM, SN = Cfg::SN;
    constexpr int S = SM * SN;
    // Whole tiles load op(A), and op(B) when untransposed, straight into LDS, in the strict
    // kernel's layouts (k-major rows with odd rows rotated by 32 floats; op(A) untransposed
    // in k quads), unpadded; a transposed op(B) goes through registers.
    constexpr bool kDirectA = WHOLE, kDirectB = WHOLE && !TB;
    constexpr int LDA = kDirectA ? BM : Cfg::LDA, LDB = kDirectB ? BN : Cfg::LDB;
    __shared__ __align__(16) float As[2][BK][LDA];
    __shared__ __align__(16) float Bs[2][BK][LDB];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave / Cfg::WN) * SM * 32, wn = (wave % Cfg::WN) * SN * 32;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    v16f acc[S];
#pragma unroll
    for (int t = 0; t < S; t++)
#pragma unroll
        for (int r = 0; r < 16; r++)
            acc[t][r] = 0.0f;

    SlabStager<float, Cfg, TA, TB, VA, VB> stage;
    const int ktiles = (K + BK - 1) / BK;
    if (WHOLE)
        stage.begin_whole(A, B, M, N, K, m0, n0, tid);
    const int half = lane >> 5, col = lane & 31;
    if constexpr (WHOLE) {
        // Wave w moves IPW 1 KiB runs of each directly loaded operand a slab: runs
        // q = IPW w .. IPW w + IPW - 1, run q landing at 256 q floats of the stage. In rows of
        // 128 floats run q is rows 2q (lanes 0-31) and 2q + 1 (lanes 32-63); in k quads it
        // is quad q / 2, rows 64 (q % 2) + lane.
        constexpr int W = Cfg::kThreads / 64, IPW = BM * BK / 256 / W;
        static_assert(BM == 128 && BN == 128 && IPW * W * 256 == BM * BK && IPW % 2 == 0,
                      "the runs below are laid out for 128 x 128 tiles");
        const int wv = __builtin_amdgcn_readfirstlane(wave);
        const int rot = half ? (col + 8) & 31 : col;
        const float *ga = nullptr, *gb = nullptr;
        uint32_t lo_a = 0, lo_b = 0;
        size_t da = 0, db = 0, ra = 0, rb = 0; // slab advance, and run r's base offset / r
        if constexpr (!TA) {
            // run q = IPW w + r: quad IPW w / 2 + r / 2, rows 64 (r % 2) + lane
            ga = A + (size_t)m0 * K + 4 * (IPW / 2 * wv);
            lo_a = (uint32_t)lane * (uint32_t)K * 4u;
            da = BK;
        } else {
            ga = A + (size_t)(2 * IPW * wv) * M + m0;
            lo_a = ((uint32_t)half * (uint32_t)M + 4u * rot) * 4u;
            da = (size_t)BK * M;
            ra = (size_t)2 * M;
        }
        if constexpr (kDirectB) {
            gb = B + (size_t)(2 * IPW * wv) * N + n0;
            lo_b = ((uint32_t)half * (uint32_t)N + 4u * rot) * 4u;
            db = (size_t)BK * N;
            rb = (size_t)2 * N;
        }
        auto run_a = [&](int r) {
            return TA ? ga + r * ra : ga + (size_t)(64 * (r & 1)) * K + 4 * (r >> 1);
        };
        auto load_slab = [&](auto st_c) {
            constexpr int st = decltype(st_c)::value;
#pragma unroll
            for (int r = 0; r < IPW; r++)
                load_lds16(run_a(r), lo_a, &As[st][0][0] + 256 * (IPW * wv + r));
            ga += da;
            if constexpr (kDirectB) {
#pragma unroll
                for (int r = 0; r < IPW; r++)
                    load_lds16(gb + r * rb, lo_b, &Bs[st][0][0] + 256 * (IPW * wv + r));
                gb += db;
            } else {
                stage.fetch_whole_b();
            }
        };
        auto stash_slab = [&](auto st_c) {
            if constexpr (!kDirectB)
                stage.stash_b(Bs[decltype(st_c)::value], tid);
        };
        // Operand offsets of k pair kk (k = kk + half) from the stage base.
        auto a_at = [&](int kk, int i) {
            const int m = wm + 32 * i + col;
            return TA ? 128 * kk + (half ? 128 + ((m - 32) & 127) : m)
                      : 512 * (kk >> 2) + (kk & 3) + 4 * m + half;
        };
        auto b_at = [&](int kk, int j) {
            const int n = wn + 32 * j + col;
            return kDirectB ? 128 * kk + (half ? 128 + ((n - 32) & 127) : n) : (kk + half) * LDB + n;
        };
        if (ktiles > 0) {
            load_slab(std::integral_constant<int, 0>{});
            stash_slab(std::integral_constant<int, 0>{});
        }
        wait_lds_loads();
        __syncthreads();
        // Two slabs a trip, so each stage index is fixed at compile time.
        auto slab = [&](auto cur_c, int kt) __attribute__((always_inline)) {
            constexpr int cur = decltype(cur_c)::value;
            const std::integral_constant<int, cur ^ 1> nxt_c;
            if (kt + 1 < ktiles)
                load_slab(nxt_c);
            const float *as = &As[cur][0][0], *bs = &Bs[cur][0][0];
#pragma unroll
            for (int kk = 0; kk < BK; kk += 2) {
                float a[SM], b[SN];
#pragma unroll
                for (int i = 0; i < SM; i++)
                    a[i] = as[a_at(kk, i)];
#pragma unroll
                for (int j = 0; j < SN; j++)
                    b[j] = bs[b_at(kk, j)];
#pragma unroll
                for (int t = 0; t < S; t++)
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t / SN], b[t % SN], acc[t], 0, 0, 0);
            }
            if (kt + 1 < ktiles)
                stash_slab(nxt_c);
            wait_lds_loads();
            __syncthreads();
        };
        for (int kt = 0; kt < ktiles; kt += 2) {
            slab(std::integral_constant<int, 0>{}, kt);
            if (kt + 1 < ktiles)
                slab(std::integral_constant<int, 1>{}, kt + 1);
        }
    } else {
        if (ktiles > 0) {
            stage.fetch(A, B, M, N, K, m0, n0, 0, tid);
            stage.stash(As[0], Bs[0], tid);
        }
        __syncthreads();
        for (int kt = 0; kt < ktiles; kt++) {
            const int cur = kt & 1;
            if (kt + 1 < ktiles)
                stage.fetch(A, B, M, N, K, m0, n0, (kt + 1) * BK, tid);
#pragma unroll
            for (int kk = 0; kk < BK; kk += 2) {
                float a[SM], b[SN];
#pragma unroll
                for (int i = 0; i < SM; i++)
                    a[i] = As[cur][kk + half][wm + 32 * i + col];
#pragma unroll
                for (int j = 0; j < SN; j++)
                    b[j] = Bs[cur][kk + half][wn + 32 * j + col];
#pragma unroll
                for (int t = 0; t < S; t++)
                    acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t / SN], b[t % SN], acc[t], 0, 0, 0);
            }
            if (kt + 1 < ktiles)
                stage.stash(As[cur ^ 1], Bs[cur ^ 1], tid);
            __syncthreads();
        }
    }
#pragma unroll
    for (int t = 0; t < S; t++) {
        const int c = n0 + wn + 32 * (t % SN) + col;
        if (c >= N)
            continue;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = m0 + wm + 32 * (t / SN) + 8 * (r >> 2) + 4 * half + (r & 3);
            if (row < M)
                C[(size_t)row * N + c] = acc[t][r];
        }
    }
}

template <class Cfg, bool TA, bool TB>
static void native_dispatch(hipStream_t s, const float *A, const float *B, float *C, int M, int N,
                            int K, NodeGate gate)
{
    const dim3 grid((unsigned)(((M + Cfg::BM - 1) / Cfg::BM) * ((N + Cfg::BN - 1) / Cfg::BN)));
    const dim3 block(Cfg::kThreads);
    const bool va = (TA ? (M % 4 == 0) : (K % 4 == 0)) && aligned16(A);
    const bool vb = (TB ? (K % 4 == 0) : (N % 4 == 0)) && aligned16(B);
    // Whole tiles load directly: a lane's byte offset from its run's base must fit 32 bits.
    const uint64_t span_a = TA ? (uint64_t)M + 128 : 64 * (uint64_t)K, span_b = (uint64_t)N + 128;
    const bool offsets32 = 4 * span_a <= UINT32_MAX && (TB || 4 * span_b <= UINT32_MAX);
    const bool whole = va && vb && M % Cfg::BM == 0 && N % Cfg::BN == 0 && K % Cfg::BK == 0 && offsets32;
    if (whole)
        hipLaunchKernelGGL((k_native_gemm_mfma<Cfg, TA, TB, true, true, true>), grid, block, 0, s, A, B, C, M, N, K, gate);
    else if (va && vb)
        hipLaunchKernelGGL((k_native_gemm_mfma<Cfg, TA, TB, true, true>), grid, block, 0, s, A, B, C, M, N, K, gate);
    else if (va)
        hipLaunchKernelGGL((k_native_gemm_mfma<Cfg, TA, TB, true, false>), grid, block, 0, s, A, B, C, M, N, K, gate);
    else if (vb)
        hipLaunchKernelGGL((k_native_gemm_mfma<Cfg, TA, TB, false, true>), grid, block, 0, s, A, B, C, M, N, K, gate);
    else
        hipLaunchKernelGGL((k_native_gemm_mfma<Cfg, TA, TB, false, false>), grid, block, 0, s, A, B, C, M, N, K, gate);
}

// 4 waves of 64 x 64 over a 128 x 128 tile: four independent accumulators per wave keep
// the matrix core busy between dependent MFMAs.
using NativeCfg = MfmaCfg<2, 2, 2, 2, 32, 2>;

hipError_t launch_native_gemm_f32(hipStream_t s, int M, int N, int K, bool ta, bool tb,
                                  const float *A, const float *B, float *C, NodeGate gate)
{
    if (!ta && !tb) native_dispatch<NativeCfg, false, false>(s, A, B, C, M, N, K, gate);
    else if (!ta && tb) native_dispatch<NativeCfg, false, true>(s, A, B, C, M, N, K, gate);
    else if (ta && !tb) native_dispatch<NativeCfg, true, false>(s, A, B, C, M, N, K, gate);
    else native_dispatch<NativeCfg, true, true>(s, A, B, C, M, N, K, gate);
    return hipGetLastError();
}

} // namespace pcu
