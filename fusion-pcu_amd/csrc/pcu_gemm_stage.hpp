// Global -> LDS staging shared by the strict and native MatMul tile kernels (gfx950).
//
// A workgroup computes a BM x BN output tile and walks k in slabs of BK. Each slab of op(A)
// (BM x BK) and op(B) (BK x BN) goes global -> registers -> a k-major LDS stage, so both
// operands are read from LDS along a row of the stage. Each thread moves EA elements of A and
// EB of B per slab as 16-byte runs; elements outside the matrices stage as +0 (a zero product
// leaves every accumulator unchanged).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pcu {

// E consecutive elements of a row-major operand at p; `valid` of them in bounds.
template <typename T, int E, bool VEC>
__device__ __forceinline__ void load_run(const T *__restrict__ p, int valid, T (&v)[E])
{
    constexpr int P = 16 / (int)sizeof(T); // elements per 16-byte load
    if (VEC && valid >= E) {
#pragma unroll
        for (int q = 0; q < E / P; q++) {
            const uint4 x = reinterpret_cast<const uint4 *>(p)[q];
            const T *xs = reinterpret_cast<const T *>(&x);
#pragma unroll
            for (int j = 0; j < P; j++)
                v[P * q + j] = xs[j];
        }
    } else {
#pragma unroll
        for (int i = 0; i < E; i++)
            v[i] = i < valid ? p[i] : (T)0;
    }
}

__device__ __forceinline__ int clamp_valid(int rem, int e) { return rem < 0 ? 0 : (rem > e ? e : rem); }

// E elements of a row-major operand as 16-byte runs RS elements apart, the first at p;
// `rem` elements lie between p and the end of the row.
template <typename T, int E, int RS, bool VEC>
__device__ __forceinline__ void load_runs(const T *__restrict__ p, int rem, T (&v)[E])
{
    constexpr int P = 16 / (int)sizeof(T);
#pragma unroll
    for (int q = 0; q < E / P; q++) {
        const int valid = clamp_valid(rem - q * RS, P);
        if (VEC && valid == P) {
            const uint4 x = *reinterpret_cast<const uint4 *>(p + q * RS);
            const T *xs = reinterpret_cast<const T *>(&x);
#pragma unroll
            for (int j = 0; j < P; j++)
                v[P * q + j] = xs[j];
        } else {
#pragma unroll
            for (int j = 0; j < P; j++)
                v[P * q + j] = j < valid ? p[q * RS + j] : (T)0;
        }
    }
}

// E elements to LDS at p as 16-byte stores (p 16-byte aligned).
template <typename T, int E>
__device__ __forceinline__ void store_run(T *p, const T (&v)[E])
{
    constexpr int P = 16 / (int)sizeof(T);
#pragma unroll
    for (int q = 0; q < E / P; q++) {
        uint4 x;
        T *xs = reinterpret_cast<T *>(&x);
#pragma unroll
        for (int j = 0; j < P; j++)
            xs[j] = v[P * q + j];
        reinterpret_cast<uint4 *>(p)[q] = x;
    }
}

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

// Cfg provides BM, BN, BK, kThreads, EA, EB, LDA, LDB and kSplitRunsB<TA>.
template <typename T, class Cfg, bool TA, bool TB, bool VA, bool VB> struct SlabStager {
    static constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, EA = Cfg::EA, EB = Cfg::EB;
    static_assert(EA % (16 / sizeof(T)) == 0 && EB % (16 / sizeof(T)) == 0,
                  "staging moves whole 16-byte runs");
    // Untransposed B under Cfg::kSplitRunsB<TA>: a thread's EB elements of a k-row are NRB
    // 16-byte runs RSB apart, so adjacent lanes store adjacent runs to LDS (contiguous runs
    // of EB elements put the stores of lanes EB elements apart on the same banks).
    static constexpr bool kRunsB = Cfg::template kSplitRunsB<TA> && !TB;
    static constexpr int RUN = 16 / (int)sizeof(T), NRB = kRunsB ? EB / RUN : 1;
    static constexpr int TPRB = BN / EB, RSB = BN / NRB, WB = kRunsB ? RUN : EB;
    T ra[EA], rb[EB];
    // Whole slabs (the tile inside M and N, K a multiple of BK, 16-byte loads allowed): the
    // thread's run pointers advance one slab per fetch, with no bound checks.
    const T *pa = nullptr, *pb = nullptr;
    size_t sa = 0, sb = 0;
    __device__ __forceinline__ void begin_whole(const T *__restrict__ A, const T *__restrict__ B,
                                                int M, int N, int K, int m0, int n0, int tid)
    {
        if (!TA) {
            pa = A + (size_t)(m0 + tid / (BK / EA)) * K + (tid % (BK / EA)) * EA;
            sa = BK;
        } else {
            pa = A + (size_t)(tid / (BM / EA)) * M + m0 + (tid % (BM / EA)) * EA;
            sa = (size_t)BK * M;
        }
        if (!TB) {
            pb = B + (size_t)(tid / TPRB) * N + n0 + (tid % TPRB) * WB;
            sb = (size_t)BK * N;
        } else {
            pb = B + (size_t)(n0 + tid / (BK / EB)) * K + (tid % (BK / EB)) * EB;
            sb = BK;
        }
    }
    __device__ __forceinline__ void fetch_whole()
    {
        load_run<T, EA, true>(pa, EA, ra);
        if constexpr (kRunsB)
            load_runs<T, EB, RSB, true>(pb, BN, rb);
        else
            load_run<T, EB, true>(pb, EB, rb);
        pa += sa;
        pb += sb;
    }

    // op(A) alone, for kernels that move op(B) straight to LDS.
    __device__ __forceinline__ void fetch_whole_a()
    {
        load_run<T, EA, true>(pa, EA, ra);
        pa += sa;
    }
    __device__ __forceinline__ void stash_a(T (*As)[Cfg::LDA], int tid) const
    {
        if (!TA) {
            const int m = tid / (BK / EA), k = (tid % (BK / EA)) * EA;
#pragma unroll
            for (int i = 0; i < EA; i++)
                As[k + i][m] = ra[i];
        } else {
            const int k = tid / (BM / EA), m = (tid % (BM / EA)) * EA;
            store_run<T, EA>(&As[k][m], ra);
        }
    }

    // op(B) alone, for kernels that move op(A) straight to LDS.
    __device__ __forceinline__ void fetch_whole_b()
    {
        if constexpr (kRunsB)
            load_runs<T, EB, RSB, true>(pb, BN, rb);
        else
            load_run<T, EB, true>(pb, EB, rb);
        pb += sb;
    }
    __device__ __forceinline__ void stash_b(T (*Bs)[Cfg::LDB], int tid) const
    {
        static_assert(!kRunsB, "op(B) alone is stashed as one run a thread");
        if (!TB) {
            const int k = tid / TPRB, n = (tid % TPRB) * WB;
            store_run<T, EB>(&Bs[k][n], rb);
        } else {
            const int n = tid / (BK / EB), k = (tid % (BK / EB)) * EB;
#pragma unroll
            for (int i = 0; i < EB; i++)
                Bs[k + i][n] = rb[i];
        }
    }

    __device__ __forceinline__ void fetch(const T *__restrict__ A, const T *__restrict__ B, int M,
                                          int N, int K, int m0, int n0, int k0, int tid)
    {
        if (!TA) { // A is M x K: BK/EA threads per row
            const int m = m0 + tid / (BK / EA), k = k0 + (tid % (BK / EA)) * EA;
            load_run<T, EA, VA>(A + (size_t)m * K + k, m < M ? clamp_valid(K - k, EA) : 0, ra);
        } else {   // A is K x M: BM/EA threads per k-row
            const int k = k0 + tid / (BM / EA), m = m0 + (tid % (BM / EA)) * EA;
            load_run<T, EA, VA>(A + (size_t)k * M + m, k < K ? clamp_valid(M - m, EA) : 0, ra);
        }
        if (!TB) { // B is K x N: BN/EB threads per k-row
            const int k = k0 + tid / TPRB, n = n0 + (tid % TPRB) * WB;
            if constexpr (kRunsB)
                load_runs<T, EB, RSB, VB>(B + (size_t)k * N + n, k < K ? N - n : 0, rb);
            else
                load_run<T, EB, VB>(B + (size_t)k * N + n, k < K ? clamp_valid(N - n, EB) : 0, rb);
        } else {   // B is N x K: BK/EB threads per row
            const int n = n0 + tid / (BK / EB), k = k0 + (tid % (BK / EB)) * EB;
            load_run<T, EB, VB>(B + (size_t)n * K + k, n < N ? clamp_valid(K - k, EB) : 0, rb);
        }
    }

    __device__ __forceinline__ void stash(T (*As)[Cfg::LDA], T (*Bs)[Cfg::LDB], int tid) const
    {
        if (!TA) {
            const int m = tid / (BK / EA), k = (tid % (BK / EA)) * EA;
#pragma unroll
            for (int i = 0; i < EA; i++)
                As[k + i][m] = ra[i];
        } else {
            const int k = tid / (BM / EA), m = (tid % (BM / EA)) * EA;
            store_run<T, EA>(&As[k][m], ra);
        }
        if (!TB) {
            const int k = tid / TPRB, n = (tid % TPRB) * WB;
            if constexpr (kRunsB) {
#pragma unroll
                for (int q = 0; q < NRB; q++) {
                    uint4 x;
                    T *xs = reinterpret_cast<T *>(&x);
#pragma unroll
                    for (int j = 0; j < RUN; j++)
                        xs[j] = rb[RUN * q + j];
                    *reinterpret_cast<uint4 *>(&Bs[k][n + q * RSB]) = x;
                }
            } else {
                store_run<T, EB>(&Bs[k][n], rb);
            }
        } else {
            const int n = tid / (BK / EB), k = (tid % (BK / EB)) * EB;
#pragma unroll
            for (int i = 0; i < EB; i++)
                Bs[k + i][n] = rb[i];
        }
    }
};

} // namespace pcu
