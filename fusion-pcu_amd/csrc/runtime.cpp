// Context, memory, staging, fault records and the op-level C ABI (include/pcu_rocm.h).
//
// Execution model: one ordered HIP stream per context. Every op enqueues its kernels and
// records into its own 64-bit fault word (node-indexed array in device memory, filled
// with the no-fault sentinel by a program's first kernel unless the previous program ended
// clean). A program ends with one kernel that copies the used fault words and a sequence
// number into coherent pinned host memory, and the host spins on that sequence word; the
// first word holding a fault in node order is decoded into TensorError coordinates. This
// replaces the
// reference's per-node sentinel upload, launch, event wait and 8-byte readback
// (backends/rocm/owned_dispatch.rs:1137-1204, 1556-1580).
#include "pcu_runtime.hpp"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <unordered_set>

// ------------------------------------------- scratch of the no-allocation strict MatMul
// pcu_strict_matmul_noalloc keeps the MatMul screen's words (one exponent word per row of
// op(A) and per column of op(B), one flag word per output row, then the first-suspect and
// first-flagged-row words) in this array instead of the context's pool, so that call
// allocates nothing. Its size is matmul_scratch_bytes(rows, cols, false) at the largest admitted
// shape: three runs of 8 * 65536 bytes and 256 bytes, i.e. 1.5 MiB + 256 B, which each device
// keeps until the process ends. In host code
// `scratch` is a host-side stand-in: only the address hipGetSymbolAddress returns for the
// current device (kept per device in g_noalloc) may reach a kernel, a fill or a copy.
static constexpr size_t kNoAllocScratchWords = 3 * (size_t)PCU_NOALLOC_MAX_DIM + 32;
static __device__ __align__(256) unsigned long long scratch[kNoAllocScratchWords];

namespace {
constexpr int kNoAllocDevices = 64;
struct NoAllocDevice {
    void *ptr = nullptr;  // this device's address of `scratch`
    bool cleared = false; // its words were zeroed by a fill kernel
    uint32_t gen = 0;     // generation of the latest screen written to it
};
std::mutex g_noalloc_mu;
NoAllocDevice g_noalloc[kNoAllocDevices];
} // namespace

// Set-up, once per device, with `device` current: the device's address of `scratch`.
static hipError_t noalloc_setup(int device)
{
    if (device < 0 || device >= kNoAllocDevices)
        return hipSuccess; // pcu_strict_matmul_noalloc refuses such a device
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    NoAllocDevice &d = g_noalloc[device];
    if (d.ptr)
        return hipSuccess;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess)
        return e;
    d.ptr = p;
    return hipSuccess;
}

namespace pcu {

thread_local std::string g_thread_error;

static const uint64_t kNoFaultWord = ~0ull;

void Ctx::fail(const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    error = buf;
}

pcu_status Ctx::hip(hipError_t e, const char *what)
{
    if (e == hipSuccess)
        return PCU_OK;
    fail("%s: %s", what, hipGetErrorString(e));
    (void)hipGetLastError();
    return e == hipErrorOutOfMemory ? PCU_ERR_OUT_OF_MEMORY : PCU_ERR_DEVICE;
}

pcu_status Ctx::open(int dev)
{
    device = dev;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= dev || dev < 0) {
        fail("no HIP device %d (found %d)", dev, count);
        return PCU_ERR_DEVICE;
    }
    pcu_status st;
    if ((st = hip(hipSetDevice(dev), "hipSetDevice")))
        return st;
    hipDeviceProp_t prop;
    if ((st = hip(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties")))
        return st;
    arch = prop.gcnArchName;
    if (arch.rfind("gfx950", 0) != 0) {
        fail("device %d is %s; this library is built for gfx950 (MI355X) only", dev, arch.c_str());
        return PCU_ERR_UNSUPPORTED;
    }
    if ((st = hip(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate")))
        return st;
    if ((st = hip(hipStreamCreateWithFlags(&side, hipStreamNonBlocking), "hipStreamCreate")))
        return st;
    if ((st = hip(hipEventCreateWithFlags(&side_done, hipEventDisableTiming), "hipEventCreate")))
        return st;
    if ((st = hip(hipEventCreateWithFlags(&main_ready, hipEventDisableTiming), "hipEventCreate")))
        return st;
    for (auto &e : marks)
        if ((st = hip(hipEventCreate(&e), "hipEventCreate")))
            return st;
    // Retain freed pool memory: resident weights and per-call scratch are reused without
    // returning to the OS between calls.
    if ((st = hip(hipDeviceGetDefaultMemPool(&pool, dev), "hipDeviceGetDefaultMemPool")))
        return st;
    uint64_t threshold = ~0ull;
    if ((st = hip(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &threshold),
                  "hipMemPoolSetAttribute")))
        return st;
    if ((st = hip(hipHostMalloc(&staging, kStagingBytes, hipHostMallocDefault), "hipHostMalloc")))
        return st;
    for (auto &e : staging_ev)
        if ((st = hip(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate")))
            return st;
    // The fault words of a program's nodes, then its stage gate (one 32-bit word).
    if ((st = hip(hipMalloc(&fault_words, sizeof(unsigned long long) * (kMaxNodes + 1)), "hipMalloc")))
        return st;
    // Coherent: the program-end kernel stores into it directly (see read_words).
    if ((st = hip(hipHostMalloc((void **)&host_words, sizeof(unsigned long long) * (kMaxNodes + 1),
                                hipHostMallocCoherent), "hipHostMalloc")))
        return st;
    host_seq = host_words + kMaxNodes;
    *host_seq = 0;
    nodes.reserve(kMaxNodes); // adding a node never reallocates
    return hip(noalloc_setup(dev), "hipGetSymbolAddress(scratch)");
}

Ctx::~Ctx()
{
    if (device < 0)
        return;
    (void)hipSetDevice(device);
    while (!prepared.empty())
        prepared_detach(prepared.back()); // removes itself from the list
    if (stream)
        (void)hipStreamSynchronize(stream);
    if (side)
        (void)hipStreamSynchronize(side);
    for (Scratch *b : {&matmul_scratch, &mse_scratch, &bt_scratch, &table_scratch})
        if (b->p)
            (void)hipFreeAsync(b->p, stream);
    for (const Released &r : reuse)
        (void)hipFreeAsync(r.p, stream);
    if (stream)
        (void)hipStreamSynchronize(stream);
    if (fault_words)
        (void)hipFree(fault_words);
    if (host_words)
        (void)hipHostFree(host_words);
    if (staging)
        (void)hipHostFree(staging);
    for (auto &e : staging_ev)
        if (e)
            (void)hipEventDestroy(e);
    for (auto &e : marks)
        if (e)
            (void)hipEventDestroy(e);
    for (auto &t : timings) {
        (void)hipEventDestroy(t.a);
        (void)hipEventDestroy(t.b);
    }
    for (auto &e : event_pool)
        (void)hipEventDestroy(e);
    if (side_done)
        (void)hipEventDestroy(side_done);
    if (main_ready)
        (void)hipEventDestroy(main_ready);
    if (stream)
        (void)hipStreamDestroy(stream);
    if (side)
        (void)hipStreamDestroy(side);
}

pcu_status Ctx::alloc(size_t bytes, void **out, bool ordered_only)
{
    if (!out) {
        fail("null output pointer");
        return PCU_ERR_ARGUMENT;
    }
    *out = nullptr;
    if (bytes == 0)
        bytes = 1;
    pcu_status st = PCU_OK;
    auto hit = std::find_if(reuse.begin(), reuse.end(), [&](const Released &r) { return r.bytes == bytes; });
    if (hit != reuse.end()) {
        *out = hit->p;
        reuse_bytes -= hit->bytes;
        reuse.erase(hit);
    } else if ((st = hip(hipMallocFromPoolAsync(out, bytes, pool, stream), "hipMallocFromPoolAsync"))) {
        return st;
    }
    alloc_bytes[*out] = bytes;
    if (in_program || ordered_only)
        return PCU_OK; // used in stream order (inside a program, until its end)
    // Usable from any stream once the allocation is ordered.
    return hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
}

pcu_status Ctx::release(void *p)
{
    if (!p)
        return PCU_OK;
    // Work still queued on the side stream may read the buffer.
    pcu_status st = join_side();
    if (st)
        return st;
    auto it = alloc_bytes.find(p);
    if (it != alloc_bytes.end()) {
        const size_t bytes = it->second;
        alloc_bytes.erase(it);
        if (reuse.size() < kReuseSlots && reuse_bytes + bytes <= kReuseMaxBytes) {
            reuse.push_back({p, bytes}); // reused in stream order after its queued users
            reuse_bytes += bytes;
            return PCU_OK;
        }
    }
    return hip(hipFreeAsync(p, stream), "hipFreeAsync");
}

pcu_status Ctx::join_side()
{
    if (!side_pending)
        return PCU_OK;
    pcu_status st = hip(hipEventRecord(side_done, side), "hipEventRecord");
    if (st)
        return st;
    st = hip(hipStreamWaitEvent(stream, side_done, 0), "hipStreamWaitEvent");
    side_pending = false;
    return st;
}

pcu_status Ctx::copy(void *dst, const void *src, size_t bytes, bool upload)
{
    if (bytes == 0)
        return PCU_OK;
    if (!dst || !src) {
        fail("null copy pointer");
        return PCU_ERR_ARGUMENT;
    }
    pcu_status st = join_side();
    if (st)
        return st;
    // Double-buffered pinned staging: the host copy into (or out of) one half overlaps the
    // DMA of the other half.
    const size_t half = kStagingBytes / 2;
    char *stage[2] = {(char *)staging, (char *)staging + half};
    size_t off = 0;
    int slot = 0;
    bool used[2] = {false, false};
    if (upload) {
        while (off < bytes) {
            size_t n = std::min(half, bytes - off);
            if (used[slot] && (st = hip(hipEventSynchronize(staging_ev[slot]), "hipEventSynchronize")))
                return st;
            memcpy(stage[slot], (const char *)src + off, n);
            if ((st = hip(hipMemcpyAsync((char *)dst + off, stage[slot], n, hipMemcpyHostToDevice, stream),
                          "hipMemcpyAsync")))
                return st;
            if ((st = hip(hipEventRecord(staging_ev[slot], stream), "hipEventRecord")))
                return st;
            used[slot] = true;
            off += n;
            slot ^= 1;
        }
        return hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    }
    // Download: keep one chunk in flight while the previous one is copied out.
    size_t pending_off = 0, pending_n = 0;
    int pending_slot = -1;
    while (off < bytes || pending_slot >= 0) {
        if (off < bytes) {
            size_t n = std::min(half, bytes - off);
            if ((st = hip(hipMemcpyAsync(stage[slot], (const char *)src + off, n, hipMemcpyDeviceToHost, stream),
                          "hipMemcpyAsync")))
                return st;
            if ((st = hip(hipEventRecord(staging_ev[slot], stream), "hipEventRecord")))
                return st;
            if (pending_slot >= 0) {
                if ((st = hip(hipEventSynchronize(staging_ev[pending_slot]), "hipEventSynchronize")))
                    return st;
                memcpy((char *)dst + pending_off, stage[pending_slot], pending_n);
            }
            pending_off = off;
            pending_n = n;
            pending_slot = slot;
            off += n;
            slot ^= 1;
        } else {
            if ((st = hip(hipEventSynchronize(staging_ev[pending_slot]), "hipEventSynchronize")))
                return st;
            memcpy((char *)dst + pending_off, stage[pending_slot], pending_n);
            pending_slot = -1;
        }
    }
    return PCU_OK;
}

// ---------------------------------------------------------------- programs

pcu_status Ctx::begin_program(bool implicit)
{
    if (in_program) {
        fail("a program is already open on this context");
        return PCU_ERR_STATE;
    }
    pcu_status st = hip(hipSetDevice(device), "hipSetDevice");
    if (st)
        return st;
    in_program = true;
    implicit_program = implicit;
    closed_seq = 0;
    close_next = false;
    nodes.clear();
    // The previous program's end left the words reset and the gate open, unless it failed.
    words_pending = !words_clean;
    words_clean = false;
    return PCU_OK;
}

// The fault words and the stage gate are reset by one kernel (not memsets, so the sequence
// stays capturable), launched right before the program's first kernel: the host work of
// the first op (scratch, events) then runs before it rather than between it and the op.
pcu_status Ctx::open_words()
{
    if (!words_pending)
        return PCU_OK;
    words_pending = false;
    return hip(launch_program_open(stream, fault_words, kMaxNodes, kNoFaultWord, gate_word()),
               "open fault words and stage gate");
}

pcu_status Ctx::add_fused_node(uint64_t n, const unsigned long long *expect)
{
    unsigned long long *word;
    pcu_status st = add_node(NodeInfo{Prim::Elementwise, n, 0}, &word);
    if (st)
        return st;
    if (word != expect) {
        fail("internal: an elementwise node evaluated with its MatMul lost its program position");
        return PCU_ERR_STATE;
    }
    return PCU_OK;
}

pcu_status Ctx::add_node(NodeInfo info, unsigned long long **word)
{
    if (!in_program) {
        fail("no program open");
        return PCU_ERR_STATE;
    }
    if (nodes.size() >= kMaxNodes) {
        fail("program exceeds %u nodes", kMaxNodes);
        return PCU_ERR_STATE;
    }
    *word = fault_words + nodes.size();
    nodes.push_back(info);
    return PCU_OK;
}

// Decode a packed word under the op's ordered fault domain
// (core/dialect/tensor/fault_domain/fault_domain.rs:122-180) and reject statuses no
// admitted op can produce (the reference treats them as protocol errors:
// backends/rocm/owned_dispatch.rs:127-141).
static bool decode_word(const NodeInfo &n, uint64_t word, pcu_fault *f)
{
    uint64_t ordinal = word >> 3;
    uint32_t kind = (uint32_t)(word & 7);
    if (kind != PCU_FAULT_DIVIDE_BY_ZERO && kind != PCU_FAULT_OVERFLOW &&
        kind != PCU_FAULT_UNDERFLOW && kind != PCU_FAULT_INVALID)
        return false;
    f->kind = kind;
    f->ordinal = ordinal;
    f->element_index = 0;
    f->reduction_index = 0;
    f->step = PCU_STEP_NONE;
    switch (n.prim) {
    case Prim::Elementwise:
        if (ordinal >= n.extent)
            return false;
        f->element_index = ordinal;
        return true;
    case Prim::MatMul: {
        if (n.inner == 0 || ordinal >= n.extent * n.inner * 2)
            return false;
        uint64_t pair = ordinal / 2;
        f->element_index = pair / n.inner;
        f->reduction_index = pair % n.inner;
        f->step = (ordinal & 1) ? PCU_STEP_ADD : PCU_STEP_MULTIPLY;
        // The first Add of a cell adds a checked product to +0: it cannot fault.
        if ((ordinal & 1) && f->reduction_index == 0)
            return false;
        return kind != PCU_FAULT_DIVIDE_BY_ZERO;
    }
    case Prim::Sgd:
        if (ordinal >= n.extent * 2)
            return false;
        f->element_index = ordinal / 2;
        f->step = (ordinal & 1) ? PCU_STEP_SUBTRACT : PCU_STEP_MULTIPLY;
        return kind != PCU_FAULT_DIVIDE_BY_ZERO;
    case Prim::Mse:
        if (ordinal > n.extent * 3)
            return false;
        if (ordinal == n.extent * 3) {
            f->reduction_index = n.extent;
            f->step = PCU_STEP_DIVIDE;
            return kind == PCU_FAULT_UNDERFLOW;
        }
        f->reduction_index = ordinal / 3;
        f->step = ordinal % 3 == 0 ? PCU_STEP_SUBTRACT
                                   : (ordinal % 3 == 1 ? PCU_STEP_MULTIPLY : PCU_STEP_ADD);
        return kind != PCU_FAULT_DIVIDE_BY_ZERO;
    case Prim::Native:
        return false; // native kernels never write their word
    }
    return false;
}

// Ends the open program: one copy of its fault words to host_words and one
// synchronization. *used is the program's node count.
pcu_status Ctx::read_words(size_t *used)
{
    *used = 0;
    if (!in_program) {
        fail("no program open");
        return PCU_ERR_STATE;
    }
    in_program = false;
    pcu_status st = join_side();
    if (st)
        return st;
    *used = nodes.size();
    if (!*used)
        return hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    uint64_t seq = closed_seq;
    closed_seq = 0;
    if (seq == 0) {
        // Nodes that launched nothing (empty shapes) still have their words read.
        if ((st = open_words()))
            return st;
        // One kernel copies the words into the coherent mirror, resets them and the gate for
        // the next program (which then needs no opening launch), and stores this program's
        // sequence number last; the host spins on that word. Against a D2H copy and a stream
        // synchronization this saves the copy command and the runtime's wake-up. A program
        // whose only node is a MatMul or a strict SGD update, or whose last launch is a
        // strict SGD update on a small grid, had one of its own kernels do the same
        // (closed_seq): a MatMul's tiny scan when no cell is suspect, else its replay.
        seq = ++pub_seq;
        if ((st = hip(launch_program_publish(stream, fault_words, *used, kNoFaultWord,
                                             gate_word(), host_words, host_seq, seq),
                      "program publish")))
            return st;
    }
    for (unsigned spin = 1;; spin++) {
        if (__atomic_load_n(host_seq, __ATOMIC_ACQUIRE) == seq)
            break;
        if ((spin & 1023) == 0) {
            // Now and then ask the runtime: an error ends the wait, and a stream that is done
            // must have stored the word.
            const hipError_t e = hipStreamQuery(stream);
            if (e == hipErrorNotReady)
                continue;
            if (e != hipSuccess)
                return hip(e, "hipStreamQuery");
            if (__atomic_load_n(host_seq, __ATOMIC_ACQUIRE) != seq) {
                fail("program end: the stream finished without storing its fault words");
                return PCU_ERR_DEVICE;
            }
            break;
        }
        __builtin_ia32_pause();
    }
    words_clean = true;
    return PCU_OK;
}

// Node i's word, read by read_words and holding a fault, as a decoded record.
pcu_status Ctx::decode_node(size_t i, pcu_fault *f)
{
    memset(f, 0, sizeof *f);
    const uint64_t w = host_words[i];
    if (!decode_word(nodes[i], w, f)) {
        fail("malformed fault word 0x%016llx at node %zu", (unsigned long long)w, i);
        // The raw word travels back as (ordinal << 3) | kind for the caller's
        // InvalidExecutionFaultWord(word) (backends/rocm/owned_dispatch.rs:95).
        memset(&protocol_fault, 0, sizeof protocol_fault);
        protocol_fault.node = (uint32_t)i;
        protocol_fault.kind = (uint32_t)(w & 7);
        protocol_fault.ordinal = w >> 3;
        return PCU_ERR_PROTOCOL;
    }
    f->node = (uint32_t)i;
    return PCU_OK;
}

pcu_status Ctx::end_program_all(std::vector<pcu_fault> *faults)
{
    faults->clear();
    size_t used = 0;
    pcu_status st = read_words(&used);
    if (st)
        return st;
    for (size_t i = 0; i < used; i++) {
        if (host_words[i] == kNoFaultWord)
            continue;
        pcu_fault f;
        if ((st = decode_node(i, &f)))
            return st;
        faults->push_back(f);
    }
    has_held_fault = !faults->empty();
    if (has_held_fault)
        held_fault = faults->front();
    return PCU_OK;
}

// The first fault in node order; every word is still validated. Allocates nothing.
pcu_status Ctx::end_program(pcu_fault *first)
{
    size_t used = 0;
    pcu_status st = read_words(&used);
    if (st)
        return st;
    bool found = false;
    pcu_fault earliest{};
    for (size_t i = 0; i < used; i++) {
        if (host_words[i] == kNoFaultWord)
            continue;
        pcu_fault f;
        if ((st = decode_node(i, &f))) {
            if (first)
                *first = protocol_fault;
            return st;
        }
        if (!found) {
            earliest = f;
            found = true;
        }
    }
    has_held_fault = found;
    if (!found)
        return PCU_OK;
    held_fault = earliest;
    if (first)
        *first = earliest;
    return PCU_ARITHMETIC_FAULT;
}

pcu_status Ctx::finish_op(pcu_status launched, pcu_fault *fault)
{
    if (!implicit_program)
        return launched;
    if (launched) {
        in_program = false;
        (void)hipStreamSynchronize(stream);
        return launched;
    }
    implicit_program = false;
    return end_program(fault);
}

pcu_status Ctx::start_op()
{
    if (in_program)
        return hip(hipSetDevice(device), "hipSetDevice");
    return begin_program(true);
}

// Scratch comes from the stream-ordered pool and is released on the same stream right
// after the op's kernels, so later ops reuse it without a host round trip.
pcu_status Ctx::scratch(Scratch &buf, size_t bytes, bool side_reader, void **out)
{
    pcu_status st;
    if (side_reader && (st = join_side())) // an earlier walk may still read the buffer
        return st;
    if (bytes > buf.cap) {
        // Ordered after every earlier use on this stream.
        if (buf.p && (st = hip(hipFreeAsync(buf.p, stream), "hipFreeAsync")))
            return st;
        buf.p = nullptr;
        buf.cap = 0;
        if ((st = hip(hipMallocFromPoolAsync(&buf.p, bytes, pool, stream), "hipMallocFromPoolAsync")))
            return st;
        buf.cap = bytes;
    }
    *out = buf.p;
    return PCU_OK;
}

void *Ctx::optional_scratch(Scratch &buf, size_t bytes)
{
    if (bytes <= buf.cap)
        return buf.p;
    if (buf.p && hipFreeAsync(buf.p, stream) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr; // keep the old buffer: it is still owned here
    }
    buf.p = nullptr;
    buf.cap = 0;
    if (hipMallocFromPoolAsync(&buf.p, bytes, pool, stream) != hipSuccess) {
        // Clear the runtime's last error, which the next launch check would otherwise read.
        (void)hipGetLastError();
        buf.p = nullptr;
        return nullptr;
    }
    buf.cap = bytes;
    return buf.p;
}

// ------------------------------------------------------------------ timing

hipEvent_t Ctx::take_event()
{
    if (!event_pool.empty()) {
        hipEvent_t e = event_pool.back();
        event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess)
        return nullptr;
    return e;
}

hipEvent_t Ctx::timer_start(hipStream_t s)
{
    if (!profiling)
        return nullptr;
    hipEvent_t e = take_event();
    if (e)
        (void)hipEventRecord(e, s);
    return e;
}

void Ctx::timer_stop(int kernel, hipEvent_t start, hipStream_t s)
{
    if (!start)
        return;
    hipEvent_t e = take_event();
    if (!e)
        return;
    (void)hipEventRecord(e, s);
    timings.push_back({kernel, start, e});
}

pcu_status Ctx::resolve_timings()
{
    pcu_status st = join_side();
    if (st)
        return st;
    if ((st = hip(hipStreamSynchronize(stream), "hipStreamSynchronize")))
        return st;
    // Adjacent regions may share an event (the MatMul's prefilter/main/replay marks), so
    // every event goes back to the pool once, or two later timers would share it.
    std::unordered_set<hipEvent_t> returned;
    for (const Timing &t : timings) {
        float ms = 0.0f;
        if ((st = hip(hipEventElapsedTime(&ms, t.a, t.b), "hipEventElapsedTime")))
            return st;
        prof_ms[t.kernel] += ms;
        prof_n[t.kernel] += 1;
        for (hipEvent_t e : {t.a, t.b})
            if (returned.insert(e).second)
                event_pool.push_back(e);
    }
    timings.clear();
    return PCU_OK;
}

// ---------------------------------------------------------------------- ops

static bool valid_dtype(int d) { return d == PCU_F32 || d == PCU_F64; }
static bool valid_policy(int p) { return p >= 0 && p <= 2; }
static size_t dsize(int d) { return d == PCU_F32 ? 4 : 8; }

// [p, p + pb) and [q, q + qb) share a byte.
static bool ranges_overlap(const void *p, uint64_t pb, const void *q, uint64_t qb)
{
    const uintptr_t a = (uintptr_t)p, b = (uintptr_t)q;
    return p && q && pb && qb && a < b + qb && b < a + pb;
}

// Elementwise kernels read element i of each operand and then write element i of out, so
// an out that is exactly an operand (an in-place update) is safe; any other overlap lets a
// lane overwrite an element another lane has yet to read.
static bool partial_overlap(const void *out, const void *in, uint64_t bytes)
{
    return out != in && ranges_overlap(out, bytes, in, bytes);
}

// A MatMul reads every operand element many times, from many workgroups, while others
// write the output (and the replay re-reads the operands after the output is written), so
// the output may share no byte with either operand. The reference cannot meet this case:
// its outputs are always fresh owners.
static bool matmul_out_overlaps(int dtype, uint64_t rows, uint64_t inner, uint64_t cols,
                                const void *a, const void *b, const void *c)
{
    const uint64_t ds = dsize(dtype);
    return ranges_overlap(c, rows * cols * ds, a, rows * inner * ds) ||
           ranges_overlap(c, rows * cols * ds, b, inner * cols * ds);
}

pcu_status Ctx::op_matmul(int dtype, uint64_t rows, uint64_t inner, uint64_t cols, int tl,
                          int tr, const void *a, const void *b, void *c, int policy, bool noalloc,
                          GemmEpilogue *epi, uint32_t epi_after, Prescreen pre, bool *epi_fused)
{
    if (epi_fused)
        *epi_fused = false;
    if (!valid_dtype(dtype) || !valid_policy(policy) || !c || ((rows * inner) && !a) ||
        ((inner * cols) && !b)) {
        fail("strict_matmul: invalid argument");
        return PCU_ERR_ARGUMENT;
    }
    if (matmul_out_overlaps(dtype, rows, inner, cols, a, b, c)) {
        fail("strict_matmul: the output overlaps an operand");
        return PCU_ERR_ARGUMENT;
    }
    if (noalloc) {
        if (rows > PCU_NOALLOC_MAX_DIM || cols > PCU_NOALLOC_MAX_DIM) {
            fail("strict_matmul_noalloc: rows and cols are each limited to %u by its fixed "
                 "scratch (got %llu x %llu)", (unsigned)PCU_NOALLOC_MAX_DIM,
                 (unsigned long long)rows, (unsigned long long)cols);
            return PCU_ERR_ARGUMENT;
        }
        if (device >= kNoAllocDevices || !g_noalloc[device].ptr) {
            fail("strict_matmul_noalloc: no scratch address for device %d", device);
            return PCU_ERR_STATE;
        }
    }
    const uint64_t cells = rows * cols, ds = dsize(dtype);
    if (epi) {
        // The tile kernel stores the product and the node's value side by side while other
        // tiles still read A and B, and the checks after it read the product back: the
        // value may overlap none of them (x, read cell by cell, only exactly).
        const bool relu = epi->op == kStepRelu, back = epi->op == kStepReluBackward;
        if (noalloc || (!relu && !back) || !valid_policy(epi->policy) ||
            (cells && (!epi->out || (back && !epi->x)))) {
            fail("strict_matmul: invalid elementwise epilogue");
            return PCU_ERR_ARGUMENT;
        }
        const uint64_t ob = cells * ds;
        if (cells && (ranges_overlap(epi->out, ob, c, ob) ||
                      ranges_overlap(epi->out, ob, a, rows * inner * ds) ||
                      ranges_overlap(epi->out, ob, b, inner * cols * ds) ||
                      (back && (partial_overlap(epi->out, epi->x, ob) ||
                                ranges_overlap(epi->x, ob, c, ob))))) {
            fail("strict_matmul: the epilogue's value overlaps an operand");
            return PCU_ERR_ARGUMENT;
        }
    }
    unsigned long long *word;
    NodeInfo info{Prim::MatMul, cells, inner};
    pcu_status st = add_node(info, &word);
    if (st)
        return st;
    const bool first_node = nodes.size() == 1;
    if (epi) {
        // The elementwise node's word: the program node it will be added as, epi_after
        // nodes after this one.
        const size_t at = nodes.size() + (size_t)epi_after;
        if (at >= kMaxNodes) {
            fail("program exceeds %u nodes", kMaxNodes);
            return PCU_ERR_STATE;
        }
        epi->fault = fault_words + at;
        epi->gate = gate_for(epi->fault);
    }
    if (rows == 0 || cols == 0)
        return PCU_OK;
    // The screen's exponent words carry a generation that only grows, so a later screen
    // outranks every word left by earlier ones; new scratch, or a wrapped counter, is
    // cleared first (by a fill kernel).
    void *sc = nullptr;
    size_t clear_words = 0; // words to zero before this screen (0: none)
    uint32_t gen = 0;
    if (noalloc) {
        // The device's fixed array, shared by every context on the device.
        std::lock_guard<std::mutex> lock(g_noalloc_mu);
        NoAllocDevice &d = g_noalloc[device];
        sc = d.ptr;
        if (!d.cleared || d.gen == UINT32_MAX) {
            clear_words = kNoAllocScratchWords;
            d.cleared = true;
            d.gen = 0;
        }
        gen = ++d.gen;
    } else {
        const Scratch old = matmul_scratch;
        if ((st = scratch(matmul_scratch, matmul_scratch_bytes(rows, cols, true), false, &sc)))
            return st;
        if (matmul_scratch.p != old.p || matmul_scratch.cap != old.cap || screen_gen == UINT32_MAX) {
            clear_words = matmul_scratch.cap / 8;
            screen_gen = 0;
        }
        gen = ++screen_gen;
    }
    // The fixed array has no partial-sum block words and no superslab tables: under
    // RejectSubnormal the no-allocation call walks every cell its exponents mark. The tables
    // only speed the tiny scan up (IEEE and RejectSubnormal), so a table buffer that cannot
    // be had is left out.
    void *tables = nullptr;
    if (!noalloc && policy != PCU_UNDERFLOW_ALLOW_GRADUAL) {
        const size_t tb = slab_table_bytes(rows, inner, cols);
        if (tb)
            tables = optional_scratch(table_scratch, tb);
    }
    MatmulScratch s = matmul_scratch_carve(sc, rows, cols, !noalloc, tables, inner);
    s.gen = gen;
    // The copy of a transposed op(B) for the tile kernel; the no-allocation call reads B in
    // place.
    // The copy is only a speed-up: when it cannot be allocated the tile kernel reads B in
    // place, as for every other layout.
    if (!noalloc && matmul_bt_wanted(dtype, rows, inner, cols, tl != 0, tr != 0, matmul_engine))
        s.bt = optional_scratch(bt_scratch, (size_t)(inner * cols * dsize(dtype)));

    // Per-kernel timing takes events from a pool that may grow, so the no-allocation call
    // is never timed.
    const bool timed = profiling && !noalloc;
    hipEvent_t ev[4] = {nullptr, nullptr, nullptr, nullptr};
    if (timed)
        for (auto &x : ev)
            x = take_event();
    // As the program's first node, the MatMul's first kernel opens the program (one launch
    // fewer; a first node is never gated, so nothing waits on the gate it opens).
    ProgramOpen open;
    if (words_pending && first_node) {
        words_pending = false;
        open = {fault_words, kMaxNodes, kNoFaultWord, gate_word()};
    } else if ((st = open_words())) {
        return st;
    }
    if (clear_words &&
        (st = hip(launch_fill_u64(stream, (unsigned long long *)sc, clear_words, 0),
                  "clear MatMul screen words")))
        return st;
    // A one-call program (this MatMul its only node) ends in the MatMul's last kernel: one
    // launch fewer. The no-allocation call keeps the publication launch (its scratch is the
    // device's shared array).
    ProgramClose close;
    if (implicit_program && first_node && !noalloc && !epi)
        close = program_close();
    bool closed = false;
    hipError_t e = launch_strict_matmul(stream, dtype, rows, inner, cols, tl != 0, tr != 0, a,
                                        b, c, policy, s, word, gate_for(word),
                                        timed ? ev : nullptr, matmul_engine, open, epi,
                                        noalloc ? Prescreen{} : pre, epi_fused, close, &closed);
    if ((st = hip(e, "strict_matmul launch")))
        return st;
    if (closed)
        closed_seq = ++pub_seq;
    if (timed) {
        timings.push_back({PCU_KERNEL_GEMM_PREFILTER, ev[0], ev[1]});
        timings.push_back({PCU_KERNEL_STRICT_GEMM, ev[1], ev[2]});
        timings.push_back({PCU_KERNEL_GEMM_REPLAY, ev[2], ev[3]});
    }
    return PCU_OK;
}

pcu_status Ctx::op_binary(int dtype, int op, uint64_t n, const void *a, const void *b,
                          const void *b_value, void *out, int policy)
{
    if (!valid_dtype(dtype) || !valid_policy(policy) || op < 0 || op > 3 ||
        (n && (!a || !out || (!b && !b_value)))) {
        fail("checked_binary: invalid argument");
        return PCU_ERR_ARGUMENT;
    }
    if (partial_overlap(out, a, n * dsize(dtype)) || partial_overlap(out, b, n * dsize(dtype))) {
        fail("checked_binary: the output partly overlaps an operand");
        return PCU_ERR_ARGUMENT;
    }
    unsigned long long *word;
    pcu_status st = add_node(NodeInfo{Prim::Elementwise, n, 0}, &word);
    if (st)
        return st;
    if ((st = open_words()))
        return st;
    hipEvent_t t = timer_start(stream);
    st = hip(launch_binary(stream, dtype, op, n, a, b, b_value, out, policy, word, gate_for(word)), "checked_binary launch");
    timer_stop(PCU_KERNEL_BINARY, t, stream);
    return st;
}

pcu_status Ctx::op_relu(int dtype, uint64_t n, const void *x, void *out, int policy)
{
    if (!valid_dtype(dtype) || !valid_policy(policy) || (n && (!x || !out))) {
        fail("checked_relu: invalid argument");
        return PCU_ERR_ARGUMENT;
    }
    if (partial_overlap(out, x, n * dsize(dtype))) {
        fail("checked_relu: the output partly overlaps the input");
        return PCU_ERR_ARGUMENT;
    }
    unsigned long long *word;
    pcu_status st = add_node(NodeInfo{Prim::Elementwise, n, 0}, &word);
    if (st)
        return st;
    if ((st = open_words()))
        return st;
    hipEvent_t t = timer_start(stream);
    st = hip(launch_relu(stream, dtype, n, x, out, policy, word, gate_for(word)), "checked_relu launch");
    timer_stop(PCU_KERNEL_RELU, t, stream);
    return st;
}

pcu_status Ctx::op_chain(int dtype, uint64_t n, ChainLaunch c)
{
    if (!valid_dtype(dtype) || c.steps < 1 || c.steps > kChainMaxSteps || (n && !c.head)) {
        fail("elementwise chain: invalid argument");
        return PCU_ERR_ARGUMENT;
    }
    const uint64_t bytes = n * dsize(dtype);
    for (int i = 0; i < c.steps; i++) {
        const ChainStep &st = c.step[i];
        if (!valid_policy(st.policy) || st.op < kOpAdd || st.op > kStepReluBackward ||
            (i == c.steps - 1 && n && !st.out)) {
            fail("elementwise chain: invalid step %d", i);
            return PCU_ERR_ARGUMENT;
        }
        // A stored value may alias an operand exactly (each element is read before it is
        // written, by the same thread) but not in part.
        for (int j = 0; j < c.steps; j++)
            if (partial_overlap(st.out, c.step[j].other, bytes)) {
                fail("elementwise chain: a step's output partly overlaps an operand");
                return PCU_ERR_ARGUMENT;
            }
        if (partial_overlap(st.out, c.head, bytes)) {
            fail("elementwise chain: a step's output partly overlaps an operand");
            return PCU_ERR_ARGUMENT;
        }
        // The kernel loads every operand before any step stores, so no later step may
        // take an earlier step's stored value as its other operand.
        for (int j = i + 1; j < c.steps; j++)
            if (st.out && n && ranges_overlap(st.out, bytes, c.step[j].other, bytes)) {
                fail("elementwise chain: step %d reads the value step %d stores", j, i);
                return PCU_ERR_ARGUMENT;
            }
    }
    unsigned long long *first = nullptr;
    for (int i = 0; i < c.steps; i++) {
        unsigned long long *word;
        pcu_status st = add_node(NodeInfo{Prim::Elementwise, n, 0}, &word);
        if (st)
            return st;
        c.step[i].fault = word;
        if (!first)
            first = word;
    }
    pcu_status st = open_words();
    if (st)
        return st;
    hipEvent_t t = timer_start(stream);
    st = hip(launch_chain(stream, dtype, n, c, gate_for(first)), "elementwise chain launch");
    timer_stop(PCU_KERNEL_ELEMENTWISE_CHAIN, t, stream);
    return st;
}

pcu_status Ctx::op_relu_backward(int dtype, uint64_t n, const void *x, const void *up, void *out,
                                 int policy)
{
    if (!valid_dtype(dtype) || !valid_policy(policy) || (n && (!x || !up || !out))) {
        fail("checked_relu_backward: invalid argument");
        return PCU_ERR_ARGUMENT;
    }
    if (partial_overlap(out, x, n * dsize(dtype)) || partial_overlap(out, up, n * dsize(dtype))) {
        fail("checked_relu_backward: the output partly overlaps an operand");
        return PCU_ERR_ARGUMENT;
    }
    unsigned long long *word;
    pcu_status st = add_node(NodeInfo{Prim::Elementwise, n, 0}, &word);
    if (st)
        return st;
    if ((st = open_words()))
        return st;
    hipEvent_t t = timer_start(stream);
    st = hip(launch_relu_backward(stream, dtype, n, x, up, out, policy, word, gate_for(word)),
             "checked_relu_backward launch");
    timer_stop(PCU_KERNEL_RELU_BACKWARD, t, stream);
    return st;
}

pcu_status Ctx::op_add_relu(int dtype, uint64_t n, const void *a, const void *b,
                            const void *b_value, void *out, int policy)
{
    if (!valid_dtype(dtype) || !valid_policy(policy) || (n && (!a || !out || (!b && !b_value)))) {
        fail("checked_add_relu: invalid argument");
        return PCU_ERR_ARGUMENT;
    }
    if (partial_overlap(out, a, n * dsize(dtype)) || partial_overlap(out, b, n * dsize(dtype))) {
        fail("checked_add_relu: the output partly overlaps an operand");
        return PCU_ERR_ARGUMENT;
    }
    unsigned long long *w_add, *w_relu;
    pcu_status st = add_node(NodeInfo{Prim::Elementwise, n, 0}, &w_add);
    if (st)
        return st;
    if ((st = add_node(NodeInfo{Prim::Elementwise, n, 0}, &w_relu)))
        return st;
    if ((st = open_words()))
        return st;
    hipEvent_t t = timer_start(stream);
    st = hip(launch_add_relu(stream, dtype, n, a, b, b_value, out, policy, w_add, w_relu, gate_for(w_add)),
             "checked_add_relu launch");
    timer_stop(PCU_KERNEL_ADD_RELU, t, stream);
    return st;
}

// The F64 rate is the exact widening of the F32 literal (reference.rs:507-514); a float
// converts to double exactly.
static bool sgd_args_ok(Ctx *c, int dtype, uint64_t n, const void *w, const void *g, float rate,
                        void *out, int policy)
{
    if (!valid_dtype(dtype) || !valid_policy(policy) || (n && (!w || !g || !out))) {
        c->fail("strict_sgd: invalid argument");
        return false;
    }
    if (partial_overlap(out, w, n * dsize(dtype)) || partial_overlap(out, g, n * dsize(dtype))) {
        c->fail("strict_sgd: the output partly overlaps an operand");
        return false;
    }
    uint32_t rb;
    memcpy(&rb, &rate, 4);
    if ((rb & 0x7f800000u) == 0x7f800000u) {
        c->fail("strict_sgd: learning rate must be finite (TensorError::InvalidLearningRate)");
        return false;
    }
    return true;
}

pcu_status Ctx::op_sgd_pair(int dtype, const uint64_t n[2], const void *const w[2],
                            const void *const g[2], const float rate[2], void *const out[2],
                            int policy)
{
    if (n[0] == 0 || n[1] == 0) {
        // An empty update launches nothing: the two go alone (and the program ends with its
        // publication launch).
        close_next = false;
        pcu_status st = op_sgd(dtype, n[0], w[0], g[0], rate[0], out[0], policy);
        return st ? st : op_sgd(dtype, n[1], w[1], g[1], rate[1], out[1], policy);
    }
    for (int u = 0; u < 2; u++)
        if (!sgd_args_ok(this, dtype, n[u], w[u], g[u], rate[u], out[u], policy))
            return PCU_ERR_ARGUMENT;
    unsigned long long *word[2];
    pcu_status st;
    for (int u = 0; u < 2; u++)
        if ((st = add_node(NodeInfo{Prim::Sgd, n[u], 0}, &word[u])))
            return st;
    if ((st = open_words()))
        return st;
    SgdJob j[2];
    for (int u = 0; u < 2; u++)
        j[u] = SgdJob{w[u], g[u], out[u], n[u], (double)rate[u], word[u], gate_for(word[u])};
    ProgramClose close;
    if ((st = take_close(&close)))
        return st;
    bool closed = false;
    hipEvent_t t = timer_start(stream);
    st = hip(launch_sgd_pair(stream, dtype, j[0], j[1], policy, close, &closed), "strict_sgd launch");
    timer_stop(PCU_KERNEL_SGD, t, stream);
    if (!st && closed)
        closed_seq = ++pub_seq;
    return st;
}

// The close for the program's last op (close_with_next_op): every word its end reads must
// be final when that op's kernel runs, so work still on the side stream is joined first.
pcu_status Ctx::take_close(ProgramClose *c)
{
    *c = ProgramClose{};
    if (!close_next)
        return PCU_OK;
    close_next = false;
    pcu_status st = join_side();
    if (st)
        return st;
    *c = program_close();
    return PCU_OK;
}

pcu_status Ctx::op_sgd(int dtype, uint64_t n, const void *w, const void *g, float rate,
                       void *out, int policy)
{
    if (!sgd_args_ok(this, dtype, n, w, g, rate, out, policy))
        return PCU_ERR_ARGUMENT;
    unsigned long long *word;
    pcu_status st = add_node(NodeInfo{Prim::Sgd, n, 0}, &word);
    if (st)
        return st;
    if ((st = open_words()))
        return st;
    if (implicit_program && nodes.size() == 1)
        close_next = true; // a single pcu_strict_sgd call: its kernel ends the program
    ProgramClose close;
    if ((st = take_close(&close)))
        return st;
    bool closed = false;
    hipEvent_t t = timer_start(stream);
    st = hip(launch_sgd(stream, dtype, n, w, g, (double)rate, out, policy, word, gate_for(word),
                        close, &closed),
             "strict_sgd launch");
    timer_stop(PCU_KERNEL_SGD, t, stream);
    if (!st && closed)
        closed_seq = ++pub_seq;
    return st;
}

// Element count rounded to nearest even (core/dialect/tensor/constants/constants.rs:18-28).
double count_as(int dtype, uint64_t n)
{
    if (dtype == PCU_F64)
        return (double)n; // u64 -> binary64 conversion rounds to nearest even
    // u64 -> binary32 rounded to nearest even with integer operations.
    if (n == 0)
        return 0.0;
    int top = 63 - __builtin_clzll(n);
    uint64_t sig;
    int exp = top;
    if (top <= 23) {
        sig = n;
    } else {
        int shift = top - 23;
        uint64_t q = n >> shift, rem = n & ((1ull << shift) - 1), half = 1ull << (shift - 1);
        sig = q + ((rem > half || (rem == half && (q & 1))) ? 1 : 0);
        if (sig == (1ull << 24)) {
            sig >>= 1;
            exp += 1;
        }
        return ldexp((double)sig, exp - 23);
    }
    return (double)sig;
}

pcu_status Ctx::op_mse(int dtype, uint64_t n, const void *p, const void *t, void *out,
                       int policy, bool on_side)
{
    if (!valid_dtype(dtype) || !valid_policy(policy) || !p || !t || !out) {
        fail("strict_mse: invalid argument");
        return PCU_ERR_ARGUMENT;
    }
    if (ranges_overlap(out, dsize(dtype), p, n * dsize(dtype)) ||
        ranges_overlap(out, dsize(dtype), t, n * dsize(dtype))) {
        fail("strict_mse: the output overlaps an operand");
        return PCU_ERR_ARGUMENT;
    }
    if (n == 0) {
        fail("strict_mse: empty input (TensorError::ShapeMismatch)");
        return PCU_ERR_SHAPE;
    }
    unsigned long long *word;
    pcu_status st = add_node(NodeInfo{Prim::Mse, n, 0}, &word);
    if (st)
        return st;
    if (n <= kMseSerialMax) {
        // One wave folds a small input in order; it overlaps the following work on the side
        // stream as the walk does.
        if ((st = open_words()))
            return st;
        hipStream_t s = stream;
        if (on_side) {
            if ((st = hip(hipEventRecord(main_ready, stream), "hipEventRecord")))
                return st;
            if ((st = hip(hipStreamWaitEvent(side, main_ready, 0), "hipStreamWaitEvent")))
                return st;
            s = side;
            side_pending = true;
        }
        hipEvent_t t1 = timer_start(s);
        if ((st = hip(launch_mse_serial(s, dtype, n, p, t, count_as(dtype, n), out, policy, word,
                                        gate_for(word)), "strict_mse launch")))
            return st;
        timer_stop(PCU_KERNEL_MSE, t1, s);
        return PCU_OK;
    }
    void *sq = nullptr;
    if ((st = scratch(mse_scratch, mse_scratch_bytes(dtype, n), true, &sq)))
        return st;
    if ((st = open_words()))
        return st;
    hipEvent_t t0 = timer_start(stream);
    if ((st = hip(launch_mse_prepare(stream, dtype, n, p, t, sq, policy, word, gate_for(word)),
                  "strict_mse launch")))
        return st;
    timer_stop(PCU_KERNEL_MSE, t0, stream);
    hipStream_t s = stream;
    if (on_side) {
        // The one-workgroup ordered walk overlaps the following ordered work on the side
        // stream, which starts once everything enqueued so far is done.
        if ((st = hip(hipEventRecord(main_ready, stream), "hipEventRecord")))
            return st;
        if ((st = hip(hipStreamWaitEvent(side, main_ready, 0), "hipStreamWaitEvent")))
            return st;
        s = side;
        side_pending = true;
    }
    hipEvent_t t1 = timer_start(s);
    if ((st = hip(launch_mse_walk(s, dtype, n, sq, count_as(dtype, n), out, policy, word, gate_for(word)),
                  "strict_mse launch")))
        return st;
    timer_stop(PCU_KERNEL_MSE, t1, s);
    return PCU_OK;
}

// ------------------------------------------------------------ native compounds
// Boundary + BackendDefined (core/numerical/numerical.rs:21-35): no arithmetic fault is
// classified; argument, shape and device errors still are.

pcu_status Ctx::op_native_matmul(int dtype, uint64_t rows, uint64_t inner, uint64_t cols, int tl,
                                 int tr, const void *a, const void *b, void *c)
{
    if (!valid_dtype(dtype) || !c || ((rows * inner) && !a) || ((inner * cols) && !b)) {
        fail("native_matmul: invalid argument");
        return PCU_ERR_ARGUMENT;
    }
    if (matmul_out_overlaps(dtype, rows, inner, cols, a, b, c)) {
        fail("native_matmul: the output overlaps an operand");
        return PCU_ERR_ARGUMENT;
    }
    unsigned long long *word;
    pcu_status st = add_node(NodeInfo{Prim::Native, rows * cols, inner}, &word);
    if (st)
        return st;
    if (rows == 0 || cols == 0)
        return PCU_OK;
    if ((st = open_words()))
        return st;
    hipEvent_t t = timer_start(stream);
    st = hip(launch_native_matmul(stream, dtype, rows, inner, cols, tl != 0, tr != 0, a, b, c, gate_for(word)),
             "native_matmul launch");
    timer_stop(PCU_KERNEL_NATIVE_GEMM, t, stream);
    return st;
}

pcu_status Ctx::op_native_sgd(int dtype, uint64_t n, const void *w, const void *g, float rate,
                              bool contracted, void *out)
{
    if (!valid_dtype(dtype) || (n && (!w || !g || !out))) {
        fail("native_sgd: invalid argument");
        return PCU_ERR_ARGUMENT;
    }
    if (partial_overlap(out, w, n * dsize(dtype)) || partial_overlap(out, g, n * dsize(dtype))) {
        fail("native_sgd: the output partly overlaps an operand");
        return PCU_ERR_ARGUMENT;
    }
    uint32_t rb;
    memcpy(&rb, &rate, 4);
    if ((rb & 0x7f800000u) == 0x7f800000u) {
        // native_sgd.rs:64-70 admits finite learning rates only.
        fail("native_sgd: learning rate must be finite");
        return PCU_ERR_ARGUMENT;
    }
    unsigned long long *word;
    pcu_status st = add_node(NodeInfo{Prim::Native, n, 0}, &word);
    if (st)
        return st;
    if ((st = open_words()))
        return st;
    hipEvent_t t = timer_start(stream);
    st = hip(launch_native_sgd(stream, dtype, n, w, g, (double)rate, contracted, out, gate_for(word)), "native_sgd launch");
    timer_stop(PCU_KERNEL_NATIVE_SGD, t, stream);
    return st;
}

pcu_status Ctx::op_native_mse(int dtype, uint64_t n, const void *p, const void *t, void *out)
{
    if (!valid_dtype(dtype) || !p || !t || !out) {
        fail("native_mse: invalid argument");
        return PCU_ERR_ARGUMENT;
    }
    if (ranges_overlap(out, dsize(dtype), p, n * dsize(dtype)) ||
        ranges_overlap(out, dsize(dtype), t, n * dsize(dtype))) {
        fail("native_mse: the output overlaps an operand");
        return PCU_ERR_ARGUMENT;
    }
    if (n == 0) {
        fail("native_mse: empty input (TensorError::ShapeMismatch)");
        return PCU_ERR_SHAPE;
    }
    unsigned long long *word;
    pcu_status st = add_node(NodeInfo{Prim::Native, n, 0}, &word);
    if (st)
        return st;
    // Scale: the rounded reciprocal of the rounded count (tensor.rs:8701-8730); host IEEE
    // division rounds to nearest even in each precision.
    double scale;
    if (dtype == PCU_F32) {
        const float count = (float)count_as(dtype, n); // exact: count_as already rounded it
        const volatile float one = 1.0f;
        scale = (double)(one / count);
    } else {
        scale = 1.0 / count_as(dtype, n);
    }
    void *sc = nullptr;
    if ((st = scratch(mse_scratch, native_mse_scratch_bytes(dtype, n), true, &sc)))
        return st;
    if ((st = open_words()))
        return st;
    hipEvent_t t0 = timer_start(stream);
    st = hip(launch_native_mse(stream, dtype, n, p, t, sc, scale, out, gate_for(word)), "native_mse launch");
    timer_stop(PCU_KERNEL_NATIVE_MSE, t0, stream);
    return st;
}

} // namespace pcu

// ======================================================================= C ABI

using pcu::Ctx;

static pcu_status bad_ctx()
{
    pcu::g_thread_error = "null context";
    return PCU_ERR_ARGUMENT;
}

extern "C" {

int pcu_abi_version(void) { return PCU_ROCM_ABI_VERSION; }

pcu_status pcu_ctx_open(int device, pcu_ctx **out)
{
    if (!out) {
        pcu::g_thread_error = "null output pointer";
        return PCU_ERR_ARGUMENT;
    }
    *out = nullptr;
    Ctx *c = new (std::nothrow) Ctx();
    if (!c) {
        pcu::g_thread_error = "out of host memory";
        return PCU_ERR_OUT_OF_MEMORY;
    }
    pcu_status st = c->open(device);
    if (st) {
        pcu::g_thread_error = c->error;
        delete c;
        return st;
    }
    *out = reinterpret_cast<pcu_ctx *>(c);
    return PCU_OK;
}

void pcu_ctx_close(pcu_ctx *ctx) { delete reinterpret_cast<Ctx *>(ctx); }

const char *pcu_last_error(const pcu_ctx *ctx)
{
    if (!ctx)
        return pcu::g_thread_error.c_str();
    return reinterpret_cast<const Ctx *>(ctx)->error.c_str();
}

void *pcu_ctx_stream(pcu_ctx *ctx) { return ctx ? (void *)reinterpret_cast<Ctx *>(ctx)->stream : nullptr; }

pcu_status pcu_ctx_synchronize(pcu_ctx *ctx)
{
    if (!ctx)
        return bad_ctx();
    Ctx *c = reinterpret_cast<Ctx *>(ctx);
    pcu_status st = c->join_side();
    if (st)
        return st;
    return c->hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

pcu_status pcu_buf_alloc(pcu_ctx *ctx, size_t bytes, void **device_ptr)
{
    if (!ctx)
        return bad_ctx();
    return reinterpret_cast<Ctx *>(ctx)->alloc(bytes, device_ptr);
}

pcu_status pcu_buf_free(pcu_ctx *ctx, void *device_ptr)
{
    if (!ctx)
        return bad_ctx();
    return reinterpret_cast<Ctx *>(ctx)->release(device_ptr);
}

pcu_status pcu_upload(pcu_ctx *ctx, void *device_dst, const void *host_src, size_t bytes)
{
    if (!ctx)
        return bad_ctx();
    Ctx *c = reinterpret_cast<Ctx *>(ctx);
    if (c->in_program) {
        c->fail("pcu_upload inside a program");
        return PCU_ERR_STATE;
    }
    return c->copy(device_dst, host_src, bytes, true);
}

pcu_status pcu_download(pcu_ctx *ctx, void *host_dst, const void *device_src, size_t bytes)
{
    if (!ctx)
        return bad_ctx();
    Ctx *c = reinterpret_cast<Ctx *>(ctx);
    if (c->in_program) {
        c->fail("pcu_download inside a program");
        return PCU_ERR_STATE;
    }
    return c->copy(host_dst, device_src, bytes, false);
}

#define PCU_OP_PROLOGUE                       \
    if (!ctx)                                 \
        return bad_ctx();                     \
    Ctx *c = reinterpret_cast<Ctx *>(ctx);    \
    pcu_status st = c->start_op();            \
    if (st)                                   \
        return st;

pcu_status pcu_strict_matmul(pcu_ctx *ctx, pcu_dtype dtype, uint64_t rows, uint64_t inner,
                             uint64_t cols, int transpose_left, int transpose_right,
                             const void *left, const void *right, void *out,
                             pcu_underflow policy, pcu_fault *fault)
{
    PCU_OP_PROLOGUE
    st = c->op_matmul(dtype, rows, inner, cols, transpose_left, transpose_right, left, right, out, policy);
    return c->finish_op(st, fault);
}

pcu_status pcu_strict_matmul_noalloc(pcu_ctx *ctx, pcu_dtype dtype, uint64_t rows, uint64_t inner,
                                     uint64_t cols, int transpose_left, int transpose_right,
                                     const void *left, const void *right, void *out,
                                     pcu_underflow policy, pcu_fault *fault)
{
    PCU_OP_PROLOGUE
    st = c->op_matmul(dtype, rows, inner, cols, transpose_left, transpose_right, left, right, out,
                      policy, true);
    return c->finish_op(st, fault);
}

pcu_status pcu_native_matmul(pcu_ctx *ctx, pcu_dtype dtype, uint64_t rows, uint64_t inner,
                             uint64_t cols, int transpose_left, int transpose_right,
                             const void *left, const void *right, void *out)
{
    PCU_OP_PROLOGUE
    st = c->op_native_matmul(dtype, rows, inner, cols, transpose_left, transpose_right, left, right, out);
    return c->finish_op(st, nullptr);
}

pcu_status pcu_native_mse(pcu_ctx *ctx, pcu_dtype dtype, uint64_t n, const void *prediction,
                          const void *target, void *out_scalar)
{
    PCU_OP_PROLOGUE
    st = c->op_native_mse(dtype, n, prediction, target, out_scalar);
    return c->finish_op(st, nullptr);
}

pcu_status pcu_native_sgd(pcu_ctx *ctx, pcu_dtype dtype, uint64_t n, const void *weights,
                          const void *gradient, float learning_rate, int contracted, void *out)
{
    PCU_OP_PROLOGUE
    st = c->op_native_sgd(dtype, n, weights, gradient, learning_rate, contracted != 0, out);
    return c->finish_op(st, nullptr);
}

pcu_status pcu_checked_binary(pcu_ctx *ctx, pcu_dtype dtype, pcu_binary_op op, uint64_t n,
                              const void *left, const void *right, void *out,
                              pcu_underflow policy, pcu_fault *fault)
{
    PCU_OP_PROLOGUE
    if (n && !right) {
        c->fail("checked_binary: null right operand");
        return c->finish_op(PCU_ERR_ARGUMENT, fault);
    }
    st = c->op_binary(dtype, op, n, left, right, nullptr, out, policy);
    return c->finish_op(st, fault);
}

pcu_status pcu_checked_binary_uniform(pcu_ctx *ctx, pcu_dtype dtype, pcu_binary_op op,
                                      uint64_t n, const void *left, uint64_t right_bits,
                                      void *out, pcu_underflow policy, pcu_fault *fault)
{
    PCU_OP_PROLOGUE
    uint32_t b32 = (uint32_t)right_bits;
    const void *value = dtype == PCU_F32 ? (const void *)&b32 : (const void *)&right_bits;
    st = c->op_binary(dtype, op, n, left, nullptr, value, out, policy);
    return c->finish_op(st, fault);
}

pcu_status pcu_checked_relu(pcu_ctx *ctx, pcu_dtype dtype, uint64_t n, const void *input,
                            void *out, pcu_underflow policy, pcu_fault *fault)
{
    PCU_OP_PROLOGUE
    st = c->op_relu(dtype, n, input, out, policy);
    return c->finish_op(st, fault);
}

pcu_status pcu_checked_relu_backward(pcu_ctx *ctx, pcu_dtype dtype, uint64_t n,
                                     const void *input, const void *upstream, void *out,
                                     pcu_underflow policy, pcu_fault *fault)
{
    PCU_OP_PROLOGUE
    st = c->op_relu_backward(dtype, n, input, upstream, out, policy);
    return c->finish_op(st, fault);
}

pcu_status pcu_checked_add_relu(pcu_ctx *ctx, pcu_dtype dtype, uint64_t n, const void *left,
                                const void *right, void *out, pcu_underflow policy,
                                pcu_fault *fault)
{
    PCU_OP_PROLOGUE
    if (n && !right) {
        c->fail("checked_add_relu: null right operand");
        return c->finish_op(PCU_ERR_ARGUMENT, fault);
    }
    st = c->op_add_relu(dtype, n, left, right, nullptr, out, policy);
    return c->finish_op(st, fault);
}

pcu_status pcu_strict_sgd(pcu_ctx *ctx, pcu_dtype dtype, uint64_t n, const void *weights,
                          const void *gradient, float learning_rate, void *out,
                          pcu_underflow policy, pcu_fault *fault)
{
    PCU_OP_PROLOGUE
    st = c->op_sgd(dtype, n, weights, gradient, learning_rate, out, policy);
    return c->finish_op(st, fault);
}

pcu_status pcu_strict_mse(pcu_ctx *ctx, pcu_dtype dtype, uint64_t n, const void *prediction,
                          const void *target, void *out_scalar, pcu_underflow policy,
                          pcu_fault *fault)
{
    PCU_OP_PROLOGUE
    st = c->op_mse(dtype, n, prediction, target, out_scalar, policy, false);
    return c->finish_op(st, fault);
}

pcu_status pcu_program_begin(pcu_ctx *ctx)
{
    if (!ctx)
        return bad_ctx();
    return reinterpret_cast<Ctx *>(ctx)->begin_program(false);
}

pcu_status pcu_program_end(pcu_ctx *ctx, pcu_fault *first_fault)
{
    if (!ctx)
        return bad_ctx();
    return reinterpret_cast<Ctx *>(ctx)->end_program(first_fault);
}

uint32_t pcu_program_next_node(const pcu_ctx *ctx)
{
    return ctx ? (uint32_t)reinterpret_cast<const Ctx *>(ctx)->nodes.size() : 0;
}

pcu_status pcu_fault_read(const pcu_ctx *ctx, pcu_fault *fault)
{
    if (!ctx || !fault)
        return PCU_ERR_ARGUMENT;
    const Ctx *c = reinterpret_cast<const Ctx *>(ctx);
    if (!c->has_held_fault)
        return PCU_OK;
    *fault = c->held_fault;
    return PCU_ARITHMETIC_FAULT;
}

pcu_status pcu_fault_reset(pcu_ctx *ctx)
{
    if (!ctx)
        return bad_ctx();
    reinterpret_cast<Ctx *>(ctx)->has_held_fault = false;
    return PCU_OK;
}

pcu_status pcu_ctx_set_matmul_engine(pcu_ctx *ctx, pcu_matmul_engine engine)
{
    if (!ctx)
        return bad_ctx();
    if (engine < PCU_MATMUL_AUTO || engine > PCU_MATMUL_MFMA_PRODUCTS)
        return PCU_ERR_ARGUMENT;
    Ctx *c = reinterpret_cast<Ctx *>(ctx);
    if (engine == PCU_MATMUL_MFMA_PRODUCTS)
        engine = PCU_MATMUL_AUTO; // F64 has no K=1 matrix form: AUTO is the same choice
    c->matmul_engine = (int)engine;
    return PCU_OK;
}

pcu_status pcu_profile_enable(pcu_ctx *ctx, int on)
{
    if (!ctx)
        return bad_ctx();
    Ctx *c = reinterpret_cast<Ctx *>(ctx);
    pcu_status st = c->resolve_timings();
    if (st)
        return st;
    for (int i = 0; i < PCU_KERNEL_COUNT; i++) {
        c->prof_ms[i] = 0.0;
        c->prof_n[i] = 0;
    }
    c->profiling = on != 0;
    return PCU_OK;
}

pcu_status pcu_profile_read(pcu_ctx *ctx, int kernel, double *total_ms, uint64_t *launches)
{
    if (!ctx)
        return bad_ctx();
    Ctx *c = reinterpret_cast<Ctx *>(ctx);
    if (kernel < 0 || kernel >= PCU_KERNEL_COUNT || !total_ms || !launches) {
        c->fail("profile read: invalid argument");
        return PCU_ERR_ARGUMENT;
    }
    if (c->in_program) {
        c->fail("profile read inside a program");
        return PCU_ERR_STATE;
    }
    pcu_status st = c->resolve_timings();
    if (st)
        return st;
    *total_ms = c->prof_ms[kernel];
    *launches = c->prof_n[kernel];
    return PCU_OK;
}

pcu_status pcu_calibrate_direct_copy(pcu_ctx *ctx, const void *src, void *dst, uint64_t bytes)
{
    if (!ctx)
        return bad_ctx();
    Ctx *c = reinterpret_cast<Ctx *>(ctx);
    if (c->in_program) {
        c->fail("calibration copy inside a program");
        return PCU_ERR_STATE;
    }
    if (!src || !dst || bytes == 0 || bytes % 4096 != 0 || ((uintptr_t)src & 15u) ||
        ((uintptr_t)dst & 15u) || pcu::ranges_overlap(dst, bytes, src, bytes)) {
        c->fail("calibration copy: invalid argument");
        return PCU_ERR_ARGUMENT;
    }
    pcu_status st = c->hip(pcu::launch_direct_copy(c->stream, src, dst, bytes), "calibration copy launch");
    if (st)
        return st;
    return c->hip(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

pcu_status pcu_mark(pcu_ctx *ctx, int slot)
{
    if (!ctx)
        return bad_ctx();
    Ctx *c = reinterpret_cast<Ctx *>(ctx);
    if (slot < 0 || slot >= (int)(sizeof(c->marks) / sizeof(c->marks[0]))) {
        c->fail("mark slot out of range");
        return PCU_ERR_ARGUMENT;
    }
    return c->hip(hipEventRecord(c->marks[slot], c->stream), "hipEventRecord");
}

pcu_status pcu_elapsed_ms(pcu_ctx *ctx, int from_slot, int to_slot, float *ms)
{
    if (!ctx)
        return bad_ctx();
    Ctx *c = reinterpret_cast<Ctx *>(ctx);
    int n = (int)(sizeof(c->marks) / sizeof(c->marks[0]));
    if (from_slot < 0 || to_slot < 0 || from_slot >= n || to_slot >= n || !ms) {
        c->fail("mark slot out of range");
        return PCU_ERR_ARGUMENT;
    }
    pcu_status st = c->hip(hipEventSynchronize(c->marks[to_slot]), "hipEventSynchronize");
    if (st)
        return st;
    return c->hip(hipEventElapsedTime(ms, c->marks[from_slot], c->marks[to_slot]), "hipEventElapsedTime");
}

} // extern "C"
