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
// (k+1)-product.
//
// Fault screening (non-finite result, exponent prefilter) and the exact replay of suspect
// cells are shared with the VALU kernel.
#include "pcu_device.hpp"
#include "pcu_kernels.hpp"

#pragma clang fp contract(off)

namespace pcu {

typedef float v32f __attribute__((ext_vector_type(32)));

namespace mf {
constexpr int BM = 128, BN = 128, BK = 16;
constexpr int LDA = BM + 4, LDB = BN + 4; // row pitch of the k-major LDS tiles
constexpr int kThreads = 256;              // 4 waves, each a 64x64 quarter of the tile
}

// 8 consecutive elements of a row-major operand at p; `valid` of them in bounds (the rest
// read as +0: a zero product leaves every accumulator unchanged).
template <bool VEC>
__device__ __forceinline__ void load8(const float *__restrict__ p, int valid, float (&v)[8])
{
    if (VEC && valid >= 8) {
        float4 q0 = *reinterpret_cast<const float4 *>(p);
        float4 q1 = *reinterpret_cast<const float4 *>(p + 4);
        v[0] = q0.x; v[1] = q0.y; v[2] = q0.z; v[3] = q0.w;
        v[4] = q1.x; v[5] = q1.y; v[6] = q1.z; v[7] = q1.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++)
            v[i] = i < valid ? p[i] : 0.0f;
    }
}

__device__ __forceinline__ int clamp_valid(int rem) { return rem < 0 ? 0 : (rem > 8 ? 8 : rem); }

// Output tile of workgroup `bid`: blocks are dealt round-robin to the 8 XCDs, so each XCD
// is given one contiguous run of the tile order (its L2 then holds that run's panels),
// and inside the order 8 tile-rows share each B panel.
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int &tm, int &tn)
{
    const int T = tiles_m * tiles_n;
    const int xcd = bid % 8, slot = bid / 8;
    const int L = xcd * (T / 8) + (xcd < T % 8 ? xcd : T % 8) + slot;
    const int group = 8;
    const int per_group = group * tiles_n;
    const int gid = L / per_group;
    const int first_m = gid * group;
    const int gsize = tiles_m - first_m < group ? tiles_m - first_m : group;
    tm = first_m + (L % per_group) % gsize;
    tn = (L % per_group) / gsize;
}

template <bool TA, bool TB, bool VA, bool VB>
__global__ __launch_bounds__(mf::kThreads, 2) void k_strict_gemm_mfma(
    const float *__restrict__ A, const float *__restrict__ B, float *__restrict__ C, int M,
    int N, int K, const int *__restrict__ row_exp, const int *__restrict__ col_exp, int thr,
    int check_risk, unsigned long long *suspect)
{
    using namespace mf;
    __shared__ __align__(16) float As[2][BK][LDA];
    __shared__ __align__(16) float Bs[2][BK][LDB];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    float acc[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                acc[i][j][r] = 0.0f;

    float ra[8], rb[8];
    // Global -> registers for the k-slab starting at k0 (8 elements of each operand).
    auto fetch = [&](int k0) {
        if (!TA) { // A is M x K: row m0 + tid/2, k0 + (tid&1)*8 .. +7
            const int m = m0 + (tid >> 1), k = k0 + (tid & 1) * 8;
            load8<VA>(A + (size_t)m * K + k, m < M ? clamp_valid(K - k) : 0, ra);
        } else {   // A is K x M: row k0 + tid/16, m0 + (tid%16)*8 .. +7
            const int k = k0 + (tid >> 4), m = m0 + (tid & 15) * 8;
            load8<VA>(A + (size_t)k * M + m, k < K ? clamp_valid(M - m) : 0, ra);
        }
        if (!TB) { // B is K x N: row k0 + tid/16, n0 + (tid%16)*8 .. +7
            const int k = k0 + (tid >> 4), n = n0 + (tid & 15) * 8;
            load8<VB>(B + (size_t)k * N + n, k < K ? clamp_valid(N - n) : 0, rb);
        } else {   // B is N x K: row n0 + tid/2, k0 + (tid&1)*8 .. +7
            const int n = n0 + (tid >> 1), k = k0 + (tid & 1) * 8;
            load8<VB>(B + (size_t)n * K + k, n < N ? clamp_valid(K - k) : 0, rb);
        }
    };
    // Registers -> k-major LDS stage `buf`.
    auto stash = [&](int buf) {
        if (!TA) {
            const int m = tid >> 1, k = (tid & 1) * 8;
#pragma unroll
            for (int i = 0; i < 8; i++)
                As[buf][k + i][m] = ra[i];
        } else {
            const int k = tid >> 4, m = (tid & 15) * 8;
            *reinterpret_cast<float4 *>(&As[buf][k][m]) = make_float4(ra[0], ra[1], ra[2], ra[3]);
            *reinterpret_cast<float4 *>(&As[buf][k][m + 4]) = make_float4(ra[4], ra[5], ra[6], ra[7]);
        }
        if (!TB) {
            const int k = tid >> 4, n = (tid & 15) * 8;
            *reinterpret_cast<float4 *>(&Bs[buf][k][n]) = make_float4(rb[0], rb[1], rb[2], rb[3]);
            *reinterpret_cast<float4 *>(&Bs[buf][k][n + 4]) = make_float4(rb[4], rb[5], rb[6], rb[7]);
        } else {
            const int n = tid >> 1, k = (tid & 1) * 8;
#pragma unroll
            for (int i = 0; i < 8; i++)
                Bs[buf][k + i][n] = rb[i];
        }
    };

    v32f zero;
#pragma unroll
    for (int r = 0; r < 32; r++)
        zero[r] = 0.0f;

    const int ktiles = (K + BK - 1) / BK;
    if (ktiles > 0) {
        fetch(0);
        stash(0);
    }
    __syncthreads();
    const int half = lane >> 5, col = lane & 31;
    auto mma = [&](float a, float b) {
        return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, zero, 0, 0, 0);
    };
    // Fold one MFMA's products into a subtile: each cell adds its k product, then its
    // k+1 product (registers r and 16 + r of the same cell).
    auto fold = [&](float (&c)[16], const v32f &p) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            c[r] = c[r] + p[r];
            c[r] = c[r] + p[16 + r];
        }
    };
    for (int kt = 0; kt < ktiles; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < ktiles)
            fetch((kt + 1) * BK);
        // Software pipeline: one MFMA is always in flight while the vector unit folds the
        // previous one (the group barriers ask the scheduler for exactly that alternation).
        // Lanes 0-31 carry k = kk, lanes 32-63 carry k = kk + 1 (the MFMA's two blocks).
        float a0 = As[cur][half][wm + col], a1 = As[cur][half][wm + 32 + col];
        float b0 = Bs[cur][half][wn + col], b1 = Bs[cur][half][wn + 32 + col];
        v32f p = mma(a0, b0);
#pragma unroll 1
        for (int kk = 0; kk < BK - 2; kk += 2) {
            const float na0 = As[cur][kk + 2 + half][wm + col];
            const float na1 = As[cur][kk + 2 + half][wm + 32 + col];
            const float nb0 = Bs[cur][kk + 2 + half][wn + col];
            const float nb1 = Bs[cur][kk + 2 + half][wn + 32 + col];
            v32f q = mma(a0, b1);
            fold(acc[0][0], p);
            p = mma(a1, b0);
            fold(acc[0][1], q);
            q = mma(a1, b1);
            fold(acc[1][0], p);
            p = mma(na0, nb0);
            fold(acc[1][1], q);
#pragma unroll
            for (int g = 0; g < 4; g++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 32, 0); // 32 VALU (a fold)
            }
            a0 = na0; a1 = na1; b0 = nb0; b1 = nb1;
        }
        {   // last k-pair of the stage: nothing further to issue
            v32f q = mma(a0, b1);
            fold(acc[0][0], p);
            p = mma(a1, b0);
            fold(acc[0][1], q);
            q = mma(a1, b1);
            fold(acc[1][0], p);
            fold(acc[1][1], q);
        }
        if (kt + 1 < ktiles)
            stash(cur ^ 1);
        __syncthreads();
    }

    // Epilogue: lane owns column n0+wn+32j+col of rows m0+wm+32i+8(r/4)+4*half+(r%4).
    uint64_t key = kNoFault;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int c = n0 + wn + 32 * j + col;
        const bool cin = c < N;
        const int cexp = (check_risk && cin) ? col_exp[c] : 0;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * half + (r & 3);
                if (!cin || row >= M)
                    continue;
                const float v = acc[i][j][r];
                C[(size_t)row * N + c] = v;
                bool bad = !finite_bits(v);
                if (check_risk)
                    bad |= row_exp[row] + cexp < thr;
                if (bad) {
                    const uint64_t cell = (uint64_t)row * N + c;
                    key = cell < key ? cell : key;
                }
            }
    }
    wave_record_fault(key, suspect);
}

static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

template <bool TA, bool TB>
static void mfma_dispatch(hipStream_t s, dim3 grid, const float *A, const float *B, float *C,
                          int M, int N, int K, const int *re, const int *ce, int thr, int risk,
                          unsigned long long *suspect)
{
    const bool va = (TA ? (M % 4 == 0) : (K % 4 == 0)) && aligned16(A);
    const bool vb = (TB ? (K % 4 == 0) : (N % 4 == 0)) && aligned16(B);
    const dim3 block(mf::kThreads);
    if (va && vb)
        hipLaunchKernelGGL((k_strict_gemm_mfma<TA, TB, true, true>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect);
    else if (va)
        hipLaunchKernelGGL((k_strict_gemm_mfma<TA, TB, true, false>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect);
    else if (vb)
        hipLaunchKernelGGL((k_strict_gemm_mfma<TA, TB, false, true>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect);
    else
        hipLaunchKernelGGL((k_strict_gemm_mfma<TA, TB, false, false>), grid, block, 0, s, A, B, C, M, N, K, re, ce, thr, risk, suspect);
}

hipError_t launch_gemm_mfma_f32(hipStream_t s, int M, int N, int K, bool ta, bool tb,
                                const float *A, const float *B, float *C, const int *row_exp,
                                const int *col_exp, int thr, int risk,
                                unsigned long long *suspect)
{
    const dim3 grid((unsigned)(((M + mf::BM - 1) / mf::BM) * ((N + mf::BN - 1) / mf::BN)));
    if (!ta && !tb) mfma_dispatch<false, false>(s, grid, A, B, C, M, N, K, row_exp, col_exp, thr, risk, suspect);
    else if (!ta && tb) mfma_dispatch<false, true>(s, grid, A, B, C, M, N, K, row_exp, col_exp, thr, risk, suspect);
    else if (ta && !tb) mfma_dispatch<true, false>(s, grid, A, B, C, M, N, K, row_exp, col_exp, thr, risk, suspect);
    else mfma_dispatch<true, true>(s, grid, A, B, C, M, N, K, row_exp, col_exp, thr, risk, suspect);
    return hipGetLastError();
}

} // namespace pcu
