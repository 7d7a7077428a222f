// Host runtime state behind the C ABI.
#pragma once

#include "../../include/pcu_rocm.h"
#include "pcu_kernels.hpp"

#include <hip/hip_runtime.h>

#include <string>
#include <unordered_map>
#include <vector>

namespace pcu {

extern thread_local std::string g_thread_error;

// Ordered fault domain of one node (core/dialect/tensor/fault_domain/fault_domain.rs:30-34).
// Native: an explicitly permitted native compound, which records no arithmetic fault.
enum class Prim { Elementwise, MatMul, Sgd, Mse, Native };

struct NodeInfo {
    Prim prim;
    uint64_t extent; // elements, or output cells for MatMul
    uint64_t inner;  // MatMul reduction length
};

double count_as(int dtype, uint64_t n);

struct Prepared;
// A prepared graph gives its device buffers back and forgets its context (defined with the
// graph executor).
void prepared_detach(Prepared *p);

struct Ctx {
    static constexpr unsigned kMaxNodes = 4096;
    static constexpr size_t kStagingBytes = 64u << 20;

    int device = -1;
    std::string arch;
    hipStream_t stream = nullptr; // ordered work
    hipStream_t side = nullptr;   // serial MSE sums overlapped with ordered work
    hipEvent_t side_done = nullptr, main_ready = nullptr;
    bool side_pending = false;
    hipMemPool_t pool = nullptr;
    void *staging = nullptr;
    hipEvent_t staging_ev[2] = {nullptr, nullptr};
    hipEvent_t marks[16] = {};
    unsigned long long *fault_words = nullptr; // device, kMaxNodes words
    // Coherent pinned mirror of the fault words, then the sequence word the program-end
    // kernel stores after copying them (see read_words).
    unsigned long long *host_words = nullptr;
    unsigned long long *host_seq = nullptr;
    uint64_t pub_seq = 0;
    // The open program's end is done by its only node's last kernel (a MatMul: see
    // ProgramClose) under this sequence number; 0: read_words launches the publication.
    uint64_t closed_seq = 0;
    bool in_program = false;
    bool implicit_program = false;
    bool words_pending = false; // the open program's words and gate await their reset
    bool words_clean = false;   // the last program's end reset them for the next one
    pcu_fault held_fault{};      // first fault of the most recent program
    pcu_fault protocol_fault{};  // node and raw word of the last malformed fault status
    bool has_held_fault = false; // the open program's fault words and gate await their reset
    std::vector<NodeInfo> nodes;
    std::string error;

    // Per-kernel device timing (pcu_profile_*): event pairs resolved on read.
    struct Timing {
        int kernel;
        hipEvent_t a, b;
    };
    bool profiling = false;
    int matmul_engine = 0; // pcu_matmul_engine
    std::vector<Timing> timings;
    std::vector<hipEvent_t> event_pool;
    double prof_ms[PCU_KERNEL_COUNT] = {};
    uint64_t prof_n[PCU_KERNEL_COUNT] = {};
    hipEvent_t take_event();
    // Records the opening event of a timed region on `s` (nullptr when not profiling).
    hipEvent_t timer_start(hipStream_t s);
    void timer_stop(int kernel, hipEvent_t start, hipStream_t s);
    pcu_status resolve_timings();

    Ctx() = default;
    Ctx(const Ctx &) = delete;
    Ctx &operator=(const Ctx &) = delete;
    ~Ctx();

    pcu_status open(int device);
    void fail(const char *fmt, ...) __attribute__((format(printf, 2, 3)));
    pcu_status hip(hipError_t e, const char *what);

    // ordered_only: the buffer is used only by work later enqueued on the ordered stream
    // (a prepared program's bank), so the allocation is not waited for.
    pcu_status alloc(size_t bytes, void **out, bool ordered_only = false);
    pcu_status release(void *p);
    pcu_status copy(void *dst, const void *src, size_t bytes, bool upload);
    pcu_status join_side();
    // Device scratch kept for the context's lifetime and grown on demand, so an op does not
    // allocate and free per call (a stream-ordered free left a gap of about 6 us before the
    // next kernel). The MatMul screen's buffer is used on the ordered stream only; the MSE
    // buffer is also read by the walk on the side stream, so taking it joins that stream.
    struct Scratch {
        void *p = nullptr;
        size_t cap = 0;
    };
    Scratch matmul_scratch, mse_scratch, bt_scratch, table_scratch;
    uint32_t screen_gen = 0; // generation of the latest MatMul exponent screen
    // Buffers released by the caller are kept for reuse by an allocation of the same size
    // (a training step frees its previous weights and takes as many new ones of the same
    // sizes), instead of a pool free and allocation each (about 7 us of host time per free).
    // Reuse is stream-ordered like the pool's own.
    static constexpr size_t kReuseSlots = 16, kReuseMaxBytes = 1ull << 30;
    struct Released {
        void *p;
        size_t bytes;
    };
    std::vector<Released> reuse;
    size_t reuse_bytes = 0;
    std::unordered_map<void *, size_t> alloc_bytes; // live caller allocations
    // Prepared graphs built on this context: closing the context detaches them (their
    // buffers are released while the context's streams still exist).
    std::vector<Prepared *> prepared;
    pcu_status scratch(Scratch &buf, size_t bytes, bool side_reader, void **out);
    // A buffer that only speeds a call up: nullptr (and no error) when it cannot be had.
    void *optional_scratch(Scratch &buf, size_t bytes);

    pcu_status open_words();
    pcu_status begin_program(bool implicit);
    pcu_status read_words(size_t *used);
    pcu_status decode_node(size_t i, pcu_fault *f);
    pcu_status end_program(pcu_fault *first);
    // Every faulted node in node order (empty when none).
    pcu_status end_program_all(std::vector<pcu_fault> *faults);
    pcu_status add_node(NodeInfo info, unsigned long long **word);
    // The program's stage gate sits after the fault words; a node's gate carries its number.
    unsigned int *gate_word() const { return reinterpret_cast<unsigned int *>(fault_words + kMaxNodes); }
    // Beside the gate: the ticket counter of an in-kernel program end (ProgramClose), zeroed
    // by every program opening and by the workgroup that ends a program.
    unsigned int *ticket_word() const { return gate_word() + 1; }
    // A ProgramClose for the program's end by the launch of its last op (nodes.size() words,
    // under sequence number pub_seq + 1); the op commits it with closed_seq = ++pub_seq once
    // launched.
    ProgramClose program_close() const
    {
        ProgramClose c;
        c.words = fault_words;
        c.n = nodes.size();
        c.value = ~0ull; // no fault
        c.gate = gate_word();
        c.host_words = host_words;
        c.host_seq = host_seq;
        c.seq = pub_seq + 1;
        c.ticket = ticket_word();
        return c;
    }
    // The program's next op is its last: an SGD update (or pair) then ends the program in
    // its own kernel when its grid is small (see op_sgd).
    bool close_next = false;
    void close_with_next_op() { close_next = in_program; }
    pcu_status take_close(ProgramClose *c);
    NodeGate gate_for(const unsigned long long *word) const
    {
        return NodeGate{gate_word(), (unsigned int)(word - fault_words)};
    }
    pcu_status start_op();
    pcu_status finish_op(pcu_status launched, pcu_fault *fault);

    // noalloc: the screen's scratch is the library's fixed per-device array
    // (pcu_strict_matmul_noalloc), so the call allocates nothing.
    // epi: an elementwise node that takes the product as its operand (a ReLU of it, or a
    // ReLU backward with it as upstream), evaluated with the MatMul (op, policy, x and out
    // from `epi`). It is the program node epi_after nodes after the MatMul's: its fault word
    // and gate are filled in here, and the caller adds it there with add_fused_node.
    // pre: operands whose screen their producer wrote (see Prescreen); *epi_fused tells
    // whether the epilogue ran in the tile kernel (and wrote the tables `epi` asked for).
    pcu_status op_matmul(int dtype, uint64_t rows, uint64_t inner, uint64_t cols, int tl, int tr,
                         const void *a, const void *b, void *c, int policy, bool noalloc = false,
                         GemmEpilogue *epi = nullptr, uint32_t epi_after = 0, Prescreen pre = {},
                         bool *epi_fused = nullptr);
    // Adds the program node of an elementwise node already evaluated with its MatMul;
    // `expect` is the fault word op_matmul gave it.
    pcu_status add_fused_node(uint64_t n, const unsigned long long *expect);
    pcu_status op_binary(int dtype, int op, uint64_t n, const void *a, const void *b,
                         const void *b_value, void *out, int policy);
    pcu_status op_relu(int dtype, uint64_t n, const void *x, void *out, int policy);
    pcu_status op_relu_backward(int dtype, uint64_t n, const void *x, const void *up, void *out,
                                int policy);
    pcu_status op_add_relu(int dtype, uint64_t n, const void *a, const void *b,
                           const void *b_value, void *out, int policy);
    // Consecutive elementwise nodes as one launch: one program node per step, in order
    // (each step's fault word is filled in here).
    pcu_status op_chain(int dtype, uint64_t n, ChainLaunch chain);
    pcu_status op_sgd(int dtype, uint64_t n, const void *w, const void *g, float rate, void *out,
                      int policy);
    // Two updates of one dtype and policy, each its own node, in one launch.
    pcu_status op_sgd_pair(int dtype, const uint64_t n[2], const void *const w[2],
                           const void *const g[2], const float rate[2], void *const out[2],
                           int policy);
    pcu_status op_mse(int dtype, uint64_t n, const void *p, const void *t, void *out, int policy,
                      bool on_side);
    pcu_status op_native_matmul(int dtype, uint64_t rows, uint64_t inner, uint64_t cols, int tl,
                                int tr, const void *a, const void *b, void *c);
    pcu_status op_native_mse(int dtype, uint64_t n, const void *p, const void *t, void *out);
    pcu_status op_native_sgd(int dtype, uint64_t n, const void *w, const void *g, float rate,
                             bool contracted, void *out);
};

} // namespace pcu
