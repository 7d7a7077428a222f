// Host-side tensor graph: the reference's Graph builder, reverse-mode derivative of an MSE
// root, execution plan, and a prepared executor over the strict kernels.
#pragma once

#include "pcu_runtime.hpp"

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace pcu {

enum class Op : uint32_t {
    Input = 0,
    Uniform = 1,
    Add = 2,
    Sub = 3,
    Mul = 4,
    Div = 5,
    SgdUpdate = 6,
    MatMul = 7,
    Relu = 8,
    ReluBackward = 9,
    MeanSquaredError = 10,
    Constant = 11,
};

enum class Mode : int32_t { None = -1, Boundary = 0, Strict = 1 };

// How many launches after a strict MatMul the plan looks for the ReLU (backward) that its
// tile kernel can evaluate (reverse mode places the weight gradient's MatMul between the
// input gradient's MatMul and its ReLU backward).
constexpr int kEpiWindow = 4;

// PcuNumericalOptions (core/numerical/numerical.rs:71-78): every node captures the graph's
// options when it is appended.
struct NumOptions {
    uint32_t compound = 0;        // 0 Checked, 1 BackendDefined
    uint32_t precision = 0;       // 0 Preserve, 1 BackendOptimized
    uint32_t reproducibility = 0; // 0 Unspecified, 1 PortableV1
};

// How the prepared executor runs a compound node.
enum class Route : int { Scalar, Strict, Native };

struct Node {
    Op op = Op::Input;
    uint32_t a = UINT32_MAX, b = UINT32_MAX; // operands
    bool tl = false, tr = false;             // MatMul transposes
    float lr = 0.0f;                         // SgdUpdate rate
    uint64_t value_bits = 0;                 // Uniform value (dtype-sized bit pattern)
    // Constant payload: the dense row-major elements, owned by the graph (shared by the
    // copies a prepared program keeps).
    std::shared_ptr<const std::vector<unsigned char>> data;
    std::vector<uint64_t> shape;
    int dtype = 0;                           // 0 f32, 1 f64
    Mode mode = Mode::None;                  // numerical mode (MatMul/MSE/SGD/ReluBackward)
    int policy = -1;                         // float underflow policy; -1 when none
    NumOptions options;                      // numerical options captured at append
};

struct Graph {
    std::vector<Node> nodes;
    Mode mode = Mode::Boundary; // default numerical mode for new compound nodes
    NumOptions options;         // default numerical options for new nodes
    std::string error;

    uint32_t push(Node n);
    pcu_status check_id(uint32_t id) const;
    uint64_t elements(uint32_t id) const;

    pcu_status input(int dtype, const std::vector<uint64_t> &shape, uint32_t *id);
    pcu_status uniform(int dtype, const std::vector<uint64_t> &shape, uint64_t bits, uint32_t *id);
    pcu_status constant(int dtype, const std::vector<uint64_t> &shape, const void *host_data,
                        uint32_t *id);
    pcu_status binary(Op op, uint32_t a, uint32_t b, uint32_t *id);
    pcu_status relu(uint32_t x, uint32_t *id);
    pcu_status relu_backward(uint32_t x, uint32_t up, uint32_t *id);
    pcu_status matmul(uint32_t a, uint32_t b, bool tl, bool tr, uint32_t *id);
    pcu_status mse(uint32_t p, uint32_t t, uint32_t *id);
    pcu_status sgd(uint32_t w, uint32_t g, float lr, uint32_t *id);

    // gradients.rs: build_backward_mse with optional targets. `grads` gets one entry per
    // node that existed before the call (UINT32_MAX when the node has no derivative).
    pcu_status backward(uint32_t loss, const std::vector<uint32_t> *targets,
                        std::vector<uint32_t> *grads);
    pcu_status plan(const std::vector<uint32_t> &outputs, std::vector<uint32_t> *order) const;
};

struct Prepared {
    Ctx *ctx = nullptr;
    Graph graph;                    // frozen copy
    std::vector<uint32_t> order;    // plan
    std::vector<uint32_t> outputs;  // requested outputs (graph ids)
    std::vector<uint32_t> inputs;   // Input nodes in graph order
    std::vector<void *> buf[2];     // per-node device buffers, two banks for outputs
    std::vector<int> is_output;     // per node
    std::vector<int> fused_into;    // Add fused into the ReLU at this id (or -1)
    std::vector<int> mse_side;      // MSE runs on the side stream
    // Fused elementwise chains: chain_next links a chain's nodes in order (UINT32_MAX at its
    // end); chain_len is the step count at its head, 0 elsewhere; chain_member marks the
    // nodes after the head (launched with it); chain_store marks the nodes whose value is
    // stored (the last step, outputs and values other nodes read).
    std::vector<uint32_t> chain_next;
    std::vector<int> chain_len;
    std::vector<char> chain_member, chain_store;
    // Consecutive strict SGD updates of one dtype and policy, the second not reading the
    // first, run as one launch: sgd_partner[first] = second, sgd_second[second] = 1.
    std::vector<uint32_t> sgd_partner;
    std::vector<char> sgd_second;
    // A strict MatMul followed within a few launches by a ReLU of its product, or by a
    // ReLU backward taking the product as upstream, evaluates that node with its own launch:
    // gemm_epi[matmul] = node (UINT32_MAX: none), epi_member[node] = 1. The node keeps its
    // place in the program (its fault word and gate), so fault order is unchanged.
    // prog_pos: each launching node's first program node index.
    std::vector<uint32_t> gemm_epi;
    std::vector<char> epi_member;
    std::vector<uint32_t> prog_pos;
    // The superslab tables (see Prescreen) that such an epilogue writes for the strict F32
    // MatMuls reading its node's value, per node: along its rows and down its columns (null:
    // not wanted). Those MatMuls then fold their screen words from the tables instead of
    // reading the value again.
    std::vector<void *> pre_rows, pre_cols;
    std::vector<Route> route;       // per node: scalar IR, strict or native compound
    std::vector<void *> dense_uniform;
    std::vector<void *> constant_buf; // resident copy of each planned Constant, uploaded at build
    int bank = 0;                   // bank written by the next execution
    bool published = false;
    std::vector<void *> published_ptr;
    std::string error;

    ~Prepared();
    pcu_status build(Ctx *c, const Graph &g, const std::vector<uint32_t> &outs);
    pcu_status execute(const std::vector<const void *> &device_inputs, pcu_fault *fault);
    void *value_ptr(uint32_t id, const std::vector<const void *> &in, int bank) const;
    // The launch of the chain that starts at `head`.
    ChainLaunch chain_launch(uint32_t head, const std::vector<const void *> &in, int bank_w) const;
};

} // namespace pcu
