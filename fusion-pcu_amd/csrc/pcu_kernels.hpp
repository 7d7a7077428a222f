// Host-side launch interface of the gfx950 kernels (implemented in *.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pcu {

// Stage gate of a launch: the program's gate word (the lowest program node that recorded a
// fault, 0xffffffff while none) and this launch's node number. A node's kernels skip their
// work when an earlier node has faulted. NodeGate{nullptr, 0} is ungated.
struct NodeGate {
    unsigned int *word;
    unsigned int node;
};

enum : int { kOpAdd = 0, kOpSub = 1, kOpMul = 2, kOpDiv = 3 };

// The end of a program done by the launch of its last op (a MatMul that is the program's
// only node, or a final SGD update) instead of a publication launch of its own: the n fault
// words go to the coherent pinned
// mirror host_words and are reset to `value`, the stage gate is opened, and then the
// sequence number `seq` is stored to host_seq (the host waits on it). `ticket` (zero between
// launches) counts the workgroups or waves that have finished when the last of them must do
// it. words == nullptr: no.
// A launch that ends the program takes one ticket per workgroup on a single counter; it
// does so only with at most this many workgroups (else the tickets queue too long).
constexpr unsigned kCloseMaxBlocks = 64;
struct ProgramClose {
    unsigned long long *words = nullptr;
    uint64_t n = 0;
    unsigned long long value = 0;
    unsigned int *gate = nullptr;
    unsigned long long *host_words = nullptr;
    unsigned long long *host_seq = nullptr;
    uint64_t seq = 0;
    unsigned int *ticket = nullptr;
};

// Elementwise family. `b == nullptr` selects the uniform right operand `*b_value`
// (host memory, dtype-sized). Each launcher enqueues on `s` and never synchronizes.
hipError_t launch_binary(hipStream_t s, int dtype, int op, uint64_t n, const void *a,
                         const void *b, const void *b_value, void *out, int policy,
                         unsigned long long *fault, NodeGate gate);
hipError_t launch_relu(hipStream_t s, int dtype, uint64_t n, const void *x, void *out,
                       int policy, unsigned long long *fault, NodeGate gate);
hipError_t launch_relu_backward(hipStream_t s, int dtype, uint64_t n, const void *x,
                                const void *up, void *out, int policy,
                                unsigned long long *fault, NodeGate gate);
hipError_t launch_add_relu(hipStream_t s, int dtype, uint64_t n, const void *a, const void *b,
                           const void *b_value, void *out, int policy,
                           unsigned long long *fault_add, unsigned long long *fault_relu, NodeGate gate);
hipError_t launch_sgd(hipStream_t s, int dtype, uint64_t n, const void *w, const void *g,
                      double rate, void *out, int policy, unsigned long long *fault, NodeGate gate,
                      ProgramClose close = {}, bool *closed = nullptr);
// Two strict SGD updates of one dtype and policy in one launch, each with its own fault word
// and gate (both counts nonzero).
struct SgdJob {
    const void *w, *g;
    void *out;
    uint64_t n;
    double rate;
    unsigned long long *fault;
    NodeGate gate;
};
// Measurement aid: copy `bytes` (a multiple of 4 KiB, 16-byte-aligned pointers) reading
// with global_load_lds_dwordx4 and writing with ordinary stores.
hipError_t launch_direct_copy(hipStream_t s, const void *src, void *dst, uint64_t bytes);
// `close` (when set, and the grid is small enough for one ticket per workgroup): the launch
// also ends the program; *closed tells whether it does.
hipError_t launch_sgd_pair(hipStream_t s, int dtype, const SgdJob &j0, const SgdJob &j1, int policy,
                           ProgramClose close = {}, bool *closed = nullptr);

// A chain of elementwise nodes (checked binary, ReLU, ReLU backward) evaluated in one pass:
// each step takes the value of the step before it (the first takes `head`) and, for a binary
// op or ReLU backward, one more operand. Every step has its own policy and fault word, and
// step s is program node gate.node + s.
enum : int { kStepRelu = 4, kStepReluBackward = 5 };
constexpr int kChainMaxSteps = 4;
struct ChainStep {
    int op;              // kOpAdd..kOpDiv, kStepRelu or kStepReluBackward
    int chain_right;     // the chain's value is the right operand (ReLU backward: the upstream)
    int policy;
    const void *other;   // the other operand, or nullptr for the uniform `other_bits`
    uint64_t other_bits; // the uniform operand's bits (dtype-sized)
    void *out;           // the step's value is stored here, or nullptr (read by the next step only)
    unsigned long long *fault;
};
// An elementwise node that a MatMul evaluates with its product: a ReLU of the product or a
// ReLU backward taking the product as its upstream (input `x`). It keeps its own value,
// policy, fault word and gate; the MatMul still stores its own value.
struct GemmEpilogue {
    int op = 0; // 0: none; kStepRelu or kStepReluBackward
    int policy = 0;
    const void *x = nullptr; // ReLU backward's input, shaped like the product
    void *out = nullptr;
    unsigned long long *fault = nullptr;
    NodeGate gate{nullptr, 0};
    // Superslab tables of the node's value for the MatMuls that read it, or null: the
    // smallest exponent (kScanExpNone for zero and non-finite) of each run of 64 along a
    // row, tbl_rows[row * (N / 64) + column / 64], and down a column,
    // tbl_cols[(row / 64) * N + column]. Written only where the epilogue runs (whole tiles).
    short *tbl_rows = nullptr, *tbl_cols = nullptr;
};

struct ChainLaunch {
    int steps = 0;
    const void *head = nullptr;
    ChainStep step[kChainMaxSteps] = {};
};
hipError_t launch_chain(hipStream_t s, int dtype, uint64_t n, const ChainLaunch &c, NodeGate gate);
// Strict MSE in two launches on one scratch of mse_scratch_bytes(dtype, n) bytes: the
// parallel part (squares, chunk estimates and summaries), then the one-workgroup ordered
// walk and the division, which may run on another stream once the first is done. `count`
// is the element count rounded to the dtype.
size_t mse_scratch_bytes(int dtype, uint64_t n);
hipError_t launch_mse_prepare(hipStream_t s, int dtype, uint64_t n, const void *p, const void *t,
                              void *scratch, int policy, unsigned long long *fault, NodeGate gate);
hipError_t launch_mse_walk(hipStream_t s, int dtype, uint64_t n, void *scratch, double count,
                           void *out, int policy, unsigned long long *fault, NodeGate gate);
// Strict MSE of at most kMseSerialMax elements in one launch of one workgroup, no scratch.
constexpr uint64_t kMseSerialMax = 4096;
hipError_t launch_mse_serial(hipStream_t s, int dtype, uint64_t n, const void *p, const void *t,
                             double count, void *out, int policy, unsigned long long *fault,
                             NodeGate gate);

// Strict MatMul scratch. Exponent words (generation << 32 | bias - minimum exponent) of
// op(A) rows and op(B) columns; per output row, the first column whose cell has a product
// that may be tiny (generation << 32 | 0xffffffff - column, folded with atomicMax); the
// first suspect cell; the first row holding such a cell; and the screen's generation: a
// context increases it per MatMul and clears the words when it wraps or the scratch is new.
struct MatmulScratch {
    unsigned long long *row_exp;    // rows entries
    unsigned long long *col_exp;    // cols entries
    unsigned long long *row_flag;   // rows entries
    unsigned long long *suspect;    // first suspect cell (kNoFault when none)
    unsigned long long *flag_first; // first row with a flagged cell (kNoFault when none)
    uint32_t gen = 1;
    // K x N elements for a transposed op(B) copied out for the tile kernel, or null (the
    // tile kernel then reads B in place). See matmul_bt_wanted.
    void *bt = nullptr;
    // One word per 32 x 32 block of output cells (flag_cols a block row), set to `gen` by a
    // tile kernel when a partial sum of a cell in the block came out a nonzero subnormal
    // (RejectSubnormal); null when the scratch carries none (the no-allocation call).
    unsigned int *sum_flag = nullptr;
    uint32_t flag_cols = 0;
    // Superslab tables of op(A) rows and op(B) columns (the smallest exponent of each run of
    // 64 k, int16), which let the tiny scan skip runs without reading the operands; null when
    // the scratch carries none. The exponent screen fills them when asked.
    short *tbl_a = nullptr, *tbl_b = nullptr;
};

// RejectSubnormal's partial-sum check in a tile kernel. A workgroup whose smallest row
// exponent plus smallest column exponent lies below `thr` (so a product below 2^thr, one
// that is not a multiple of the smallest normal, may occur) checks every partial sum it
// forms for a nonzero subnormal; a lane that meets one marks its cells suspect and sets its
// blocks' words to `gen`. flag == nullptr: no check.
struct SumCheck {
    unsigned int *flag = nullptr;
    uint32_t gen = 0;
    uint32_t blocks_n = 0; // words a block row
    int thr = 0;
    // The screen's superslab tables (see MatmulScratch) or null. With them a checking tile
    // checks only the slabs of superslabs that may hold a product below 2^thr, and the slabs
    // after them while a partial sum might still be subnormal later; without, every slab.
    const short *tbl_a = nullptr, *tbl_b = nullptr;
    int a_xmajor = 0, b_xmajor = 0;
};
// Whether a strict MatMul (F32 on the matrix-core engine, or F64) runs its tile kernel on a
// copy of a transposed op(B) stored K x N (grids of whole 128 x 128 tiles, K a multiple of
// 16): the tile kernels load an untransposed op(B) straight into LDS but stage a transposed
// one through registers.
bool matmul_bt_wanted(int dtype, uint64_t rows, uint64_t inner, uint64_t cols, bool tl,
                      bool tr, int engine);
// `sum_flags`: the scratch also carries the partial-sum block words. The superslab tables
// take a buffer of their own of slab_table_bytes() bytes (0: too large, none), or none.
size_t matmul_scratch_bytes(uint64_t rows, uint64_t cols, bool sum_flags);
size_t slab_table_bytes(uint64_t rows, uint64_t inner, uint64_t cols);
MatmulScratch matmul_scratch_carve(void *base, uint64_t rows, uint64_t cols, bool sum_flags,
                                   void *tables, uint64_t inner);

// Main-kernel engine of the strict F32 MatMul: products from the vector unit (v_mul_f32),
// or from the matrix cores used as a K=1 multiplier array with a +0 accumulator (bit-equal
// products; the ordered sums stay on the vector unit). F64 always uses the vector unit.
enum : int { kEngineAuto = 0, kEngineValu = 1, kEngineMfmaProducts = 2 };

// `epi`: evaluated in the epilogue when the chosen tile kernel supports it (*epi_done set).
hipError_t launch_gemm_mfma_f32(hipStream_t s, int M, int N, int K, bool ta, bool tb,
                                const float *A, const float *B, float *C,
                                const unsigned long long *row_exp,
                                const unsigned long long *col_exp, int thr, int risk,
                                unsigned long long *suspect, SumCheck sck, NodeGate gate,
                                const GemmEpilogue *epi = nullptr, bool *epi_done = nullptr);

// C[rows x cols] = op(A) * op(B), k ascending, each multiply and add rounded on its own.
// Every kernel of the op skips its work once `gate` shows that an earlier program node
// faulted (that earlier fault is reported).
// `ev` (optional, 4 events) is recorded before the prefilter, before and after the main
// kernel, and after the replay.
// The opening of a program (its fault words set to `value`, its stage gate opened) can be
// done by the first kernel of the program's first node instead of a launch of its own: a
// first node is never gated, so that kernel may open the gate while it runs. `open` asks the
// MatMul's first kernel to do it (rows and cols must then be nonzero); words == nullptr: no.
struct ProgramOpen {
    unsigned long long *words = nullptr;
    uint64_t n = 0;
    unsigned long long value = 0;
    unsigned int *gate = nullptr;
};
// Operands whose exponent screen its producer already wrote, as superslab tables in the
// screen's own layouts: op(A)'s rows (a: x-major [M][K/64] when A is untransposed,
// superslab-major [K/64][M] when transposed) and op(B)'s columns (b: superslab-major
// [K/64][N] when B is untransposed, x-major [N][K/64] when transposed). The screen then folds
// their words from these tables instead of reading the operand.
struct Prescreen {
    const short *a = nullptr, *b = nullptr;
};
// With `epi`, the MatMul also evaluates that elementwise node: in the tile kernel's
// epilogue where the kernel supports it (whole 128 x 128 matrix-core tiles: *epi_fused set,
// and the epilogue's tables written), else as its own kernel right after the tile kernel.
hipError_t launch_strict_matmul(hipStream_t s, int dtype, uint64_t rows, uint64_t inner,
                                uint64_t cols, bool transpose_left, bool transpose_right,
                                const void *a, const void *b, void *c, int policy,
                                MatmulScratch scratch, unsigned long long *fault, NodeGate gate,
                                hipEvent_t *ev = nullptr, int engine = kEngineAuto,
                                ProgramOpen open = {}, const GemmEpilogue *epi = nullptr,
                                Prescreen pre = {}, bool *epi_fused = nullptr,
                                ProgramClose close = {}, bool *closed = nullptr);

// Native compound arithmetic (Boundary + BackendDefined): no fault word.
hipError_t launch_native_gemm_f32(hipStream_t s, int M, int N, int K, bool ta, bool tb,
                                  const float *A, const float *B, float *C, NodeGate gate);
hipError_t launch_native_matmul(hipStream_t s, int dtype, uint64_t rows, uint64_t inner,
                                uint64_t cols, bool ta, bool tb, const void *a, const void *b,
                                void *c, NodeGate gate);
hipError_t launch_native_sgd(hipStream_t s, int dtype, uint64_t n, const void *w, const void *g,
                             double rate, bool contracted, void *out, NodeGate gate);
// `scratch` holds native_mse_scratch_bytes(dtype, n) bytes; `scale` is the rounded
// reciprocal of the element count in the dtype.
size_t native_mse_scratch_bytes(int dtype, uint64_t n);
hipError_t launch_native_mse(hipStream_t s, int dtype, uint64_t n, const void *p, const void *t,
                             void *scratch, double scale, void *out, NodeGate gate);

// Small device utilities (fill kernels rather than memsets, so a captured graph replays
// them as kernels).
hipError_t launch_fill_u64(hipStream_t s, unsigned long long *p, uint64_t n, uint64_t value);
hipError_t launch_fill_u32(hipStream_t s, unsigned int *p, uint64_t n, uint32_t value);
// Program start: words[0, n) = value and *gate = 0xffffffff (open), in one launch.
// Program end: host_words[0, n) = words[0, n), then words[0, n) = value and *gate =
// 0xffffffff (the next program starts open), then *host_seq = seq, stored at system scope
// after the copies, so a host that reads seq there may read the words. host_words and
// host_seq are coherent pinned host memory. One launch of one workgroup.
hipError_t launch_program_publish(hipStream_t s, unsigned long long *words, uint64_t n,
                                  uint64_t value, unsigned int *gate,
                                  unsigned long long *host_words, unsigned long long *host_seq,
                                  uint64_t seq);
hipError_t launch_program_open(hipStream_t s, unsigned long long *words, uint64_t n, uint64_t value,
                               unsigned int *gate);

} // namespace pcu
