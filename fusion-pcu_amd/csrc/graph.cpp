// Tensor graph builder, reverse-mode MSE derivative, execution plan, and the prepared
// executor that lowers each planned node onto the strict kernels with one terminal
// synchronization per execution.
//
// Builder and derivative rules follow the reference's core graph (paths relative to the
// reference's Crates/): Graph::push core/dialect/tensor.rs:3588-3620, builders :4028-4329,
// execution_plan_for_outputs :3234-3300, reverse mode core/dialect/tensor/gradients/
// gradients.rs:31-474. The executor replaces RocmOwnedPreparedTensorGraph
// (backends/rocm/tensor.rs:5827-6015).
#include "pcu_graph.hpp"

#include <algorithm>
#include <cstring>
#include <new>

namespace pcu {

static bool is_float(int dtype) { return dtype == 0 || dtype == 1; }

// --------------------------------------------------------------------- builder

uint32_t Graph::push(Node n)
{
    // Only compound primitives carry a numerical mode; floating elementwise arithmetic and
    // every compound get the default underflow policy (tensor.rs:3593-3611).
    bool compound = n.op == Op::MatMul || n.op == Op::MeanSquaredError || n.op == Op::SgdUpdate ||
                    n.op == Op::ReluBackward;
    n.mode = compound ? mode : Mode::None;
    bool elementwise = n.op == Op::Add || n.op == Op::Sub || n.op == Op::Mul || n.op == Op::Div ||
                       n.op == Op::Relu;
    n.policy = (is_float(n.dtype) && (elementwise || compound)) ? 0 : -1;
    n.options = options; // tensor.rs:3612-3618: every node captures the graph's options
    nodes.push_back(std::move(n));
    return (uint32_t)(nodes.size() - 1);
}

pcu_status Graph::check_id(uint32_t id) const
{
    return id < nodes.size() ? PCU_OK : PCU_ERR_ARGUMENT;
}

uint64_t Graph::elements(uint32_t id) const
{
    uint64_t n = 1;
    for (uint64_t d : nodes[id].shape)
        n *= d;
    return n;
}

static bool shape_overflows(const std::vector<uint64_t> &shape)
{
    unsigned __int128 n = 1;
    for (uint64_t d : shape) {
        n *= d;
        if (n > (unsigned __int128)UINT64_MAX)
            return true;
    }
    return false;
}

pcu_status Graph::input(int dtype, const std::vector<uint64_t> &shape, uint32_t *id)
{
    if (!is_float(dtype) || !id) {
        error = "input: unsupported scalar type";
        return PCU_ERR_UNSUPPORTED;
    }
    if (shape_overflows(shape)) {
        error = "input: ShapeOverflow";
        return PCU_ERR_SHAPE;
    }
    Node n;
    n.op = Op::Input;
    n.shape = shape;
    n.dtype = dtype;
    *id = push(n);
    return PCU_OK;
}

pcu_status Graph::uniform(int dtype, const std::vector<uint64_t> &shape, uint64_t bits, uint32_t *id)
{
    if (!is_float(dtype) || !id) {
        error = "uniform: unsupported scalar type";
        return PCU_ERR_UNSUPPORTED;
    }
    if (shape_overflows(shape)) {
        error = "uniform: ShapeOverflow";
        return PCU_ERR_SHAPE;
    }
    Node n;
    n.op = Op::Uniform;
    n.shape = shape;
    n.dtype = dtype;
    n.value_bits = dtype == 0 ? (bits & 0xffffffffull) : bits;
    *id = push(n);
    return PCU_OK;
}

// Graph::constant_value / constant_typed (core/dialect/tensor.rs:3669-3679): an owned dense tensor constant,
// a leaf of the graph like Input. Its elements are copied into the graph here and uploaded
// once when a program that uses it is prepared.
pcu_status Graph::constant(int dtype, const std::vector<uint64_t> &shape, const void *host_data,
                           uint32_t *id)
{
    if (!is_float(dtype) || !id) {
        error = "constant: unsupported scalar type";
        return PCU_ERR_UNSUPPORTED;
    }
    if (shape_overflows(shape)) {
        error = "constant: ShapeOverflow";
        return PCU_ERR_SHAPE;
    }
    unsigned __int128 bytes = dtype == 0 ? 4 : 8;
    for (uint64_t d : shape)
        bytes *= d;
    if (bytes > (unsigned __int128)(SIZE_MAX / 2)) {
        error = "constant: ShapeOverflow";
        return PCU_ERR_SHAPE;
    }
    if (bytes && !host_data) {
        error = "constant: null data";
        return PCU_ERR_ARGUMENT;
    }
    auto data = std::make_shared<std::vector<unsigned char>>((size_t)bytes);
    if (bytes)
        memcpy(data->data(), host_data, (size_t)bytes);
    Node n;
    n.op = Op::Constant;
    n.shape = shape;
    n.dtype = dtype;
    n.data = std::move(data);
    *id = push(n);
    return PCU_OK;
}

// same_shape_binary (tensor.rs:4067-4110): equal shapes and scalar types.
pcu_status Graph::binary(Op op, uint32_t a, uint32_t b, uint32_t *id)
{
    if (check_id(a) || check_id(b) || !id) {
        error = "binary: UnknownValue";
        return PCU_ERR_ARGUMENT;
    }
    if (nodes[a].shape != nodes[b].shape) {
        error = "binary: ShapeMismatch";
        return PCU_ERR_SHAPE;
    }
    if (nodes[a].dtype != nodes[b].dtype) {
        error = "binary: ScalarTypeMismatch";
        return PCU_ERR_SHAPE;
    }
    Node n;
    n.op = op;
    n.a = a;
    n.b = b;
    n.shape = nodes[a].shape;
    n.dtype = nodes[a].dtype;
    *id = push(n);
    return PCU_OK;
}

pcu_status Graph::relu(uint32_t x, uint32_t *id)
{
    if (check_id(x) || !id) {
        error = "relu: UnknownValue";
        return PCU_ERR_ARGUMENT;
    }
    Node n;
    n.op = Op::Relu;
    n.a = x;
    n.shape = nodes[x].shape;
    n.dtype = nodes[x].dtype;
    *id = push(n);
    return PCU_OK;
}

pcu_status Graph::relu_backward(uint32_t x, uint32_t up, uint32_t *id)
{
    if (check_id(x) || check_id(up) || !id) {
        error = "relu_backward: UnknownValue";
        return PCU_ERR_ARGUMENT;
    }
    if (nodes[x].shape != nodes[up].shape) {
        error = "relu_backward: ShapeMismatch";
        return PCU_ERR_SHAPE;
    }
    if (nodes[x].dtype != nodes[up].dtype) {
        error = "relu_backward: ScalarTypeMismatch";
        return PCU_ERR_SHAPE;
    }
    Node n;
    n.op = Op::ReluBackward;
    n.a = x;
    n.b = up;
    n.shape = nodes[x].shape;
    n.dtype = nodes[x].dtype;
    *id = push(n);
    return PCU_OK;
}

// matmul_transposed (tensor.rs:4176-4233)
pcu_status Graph::matmul(uint32_t a, uint32_t b, bool tl, bool tr, uint32_t *id)
{
    if (check_id(a) || check_id(b) || !id) {
        error = "matmul: UnknownValue";
        return PCU_ERR_ARGUMENT;
    }
    const auto &sa = nodes[a].shape, &sb = nodes[b].shape;
    if (sa.size() != 2 || sb.size() != 2) {
        error = "matmul: MatMulShape (rank)";
        return PCU_ERR_SHAPE;
    }
    uint64_t rows = tl ? sa[1] : sa[0], inner = tl ? sa[0] : sa[1];
    uint64_t inner_b = tr ? sb[1] : sb[0], cols = tr ? sb[0] : sb[1];
    if (inner != inner_b) {
        error = "matmul: MatMulShape";
        return PCU_ERR_SHAPE;
    }
    if (shape_overflows({rows, cols})) {
        error = "matmul: ShapeOverflow";
        return PCU_ERR_SHAPE;
    }
    if (nodes[a].dtype != nodes[b].dtype) {
        error = "matmul: ScalarTypeMismatch";
        return PCU_ERR_SHAPE;
    }
    Node n;
    n.op = Op::MatMul;
    n.a = a;
    n.b = b;
    n.tl = tl;
    n.tr = tr;
    n.shape = {rows, cols};
    n.dtype = nodes[a].dtype;
    *id = push(n);
    return PCU_OK;
}

// mean_squared_error (tensor.rs:4299-4329): equal nonempty shapes, scalar result.
pcu_status Graph::mse(uint32_t p, uint32_t t, uint32_t *id)
{
    if (check_id(p) || check_id(t) || !id) {
        error = "mean_squared_error: UnknownValue";
        return PCU_ERR_ARGUMENT;
    }
    if (nodes[p].shape != nodes[t].shape || elements(p) == 0) {
        error = "mean_squared_error: ShapeMismatch";
        return PCU_ERR_SHAPE;
    }
    if (nodes[p].dtype != nodes[t].dtype) {
        error = "mean_squared_error: ScalarTypeMismatch";
        return PCU_ERR_SHAPE;
    }
    Node n;
    n.op = Op::MeanSquaredError;
    n.a = p;
    n.b = t;
    n.shape = {};
    n.dtype = nodes[p].dtype;
    *id = push(n);
    return PCU_OK;
}

// sgd_update (tensor.rs:4028-4066): equal shapes/types and a finite F32 rate.
pcu_status Graph::sgd(uint32_t w, uint32_t g, float lr, uint32_t *id)
{
    if (check_id(w) || check_id(g) || !id) {
        error = "sgd_update: UnknownValue";
        return PCU_ERR_ARGUMENT;
    }
    if (nodes[w].shape != nodes[g].shape) {
        error = "sgd_update: ShapeMismatch";
        return PCU_ERR_SHAPE;
    }
    if (nodes[w].dtype != nodes[g].dtype) {
        error = "sgd_update: ScalarTypeMismatch";
        return PCU_ERR_SHAPE;
    }
    uint32_t bits;
    memcpy(&bits, &lr, 4);
    if ((bits & 0x7f800000u) == 0x7f800000u) {
        error = "sgd_update: InvalidLearningRate";
        return PCU_ERR_ARGUMENT;
    }
    Node n;
    n.op = Op::SgdUpdate;
    n.a = w;
    n.b = g;
    n.lr = lr;
    n.shape = nodes[w].shape;
    n.dtype = nodes[w].dtype;
    *id = push(n);
    return PCU_OK;
}

// ------------------------------------------------------------------ gradients

static void operands_of(const Node &n, uint32_t out[2], int *count)
{
    *count = 0;
    if (n.a != UINT32_MAX)
        out[(*count)++] = n.a;
    if (n.b != UINT32_MAX)
        out[(*count)++] = n.b;
}

// Bit pattern of a binary64 constant in `dtype` (exact for every constant the rules use:
// -1, the widened -rate, and 2/n).
static uint64_t const_bits(int dtype, double v)
{
    if (dtype == 0) {
        float f = (float)v;
        uint32_t b;
        memcpy(&b, &f, 4);
        return b;
    }
    uint64_t b;
    memcpy(&b, &v, 8);
    return b;
}

struct Backward {
    Graph &g;
    std::vector<uint32_t> grads; // per original node
    const std::vector<char> &needed;

    pcu_status accumulate(uint32_t target, uint32_t addition)
    {
        // gradients.rs:240-251
        if (grads[target] == UINT32_MAX) {
            grads[target] = addition;
            return PCU_OK;
        }
        uint32_t sum;
        pcu_status st = g.binary(Op::Add, grads[target], addition, &sum);
        if (st)
            return st;
        grads[target] = sum;
        return PCU_OK;
    }

    // gradients.rs:253-272
    pcu_status filled_like(uint32_t like, double scalar, uint32_t *id)
    {
        const Node &n = g.nodes[like];
        return g.uniform(n.dtype, n.shape, const_bits(n.dtype, scalar), id);
    }

    // gradients.rs:139-201
    pcu_status mse_rule(uint32_t p, uint32_t t)
    {
        if (!needed[p] && !needed[t])
            return PCU_OK;
        const Node &pn = g.nodes[p];
        std::vector<uint64_t> shape = pn.shape;
        uint64_t count = g.elements(p);
        int dtype = pn.dtype;
        double scale_value;
        if (dtype == 0) {
            float c = (float)count_as(0, count);
            scale_value = (double)(2.0f / c); // checked 2 (/) count_f32: exact or RNE
        } else {
            scale_value = 2.0 / count_as(1, count);
        }
        uint32_t scale, pd = UINT32_MAX, td = UINT32_MAX, pgrad = UINT32_MAX, tgrad = UINT32_MAX;
        pcu_status st = g.uniform(dtype, shape, const_bits(dtype, scale_value), &scale);
        if (st)
            return st;
        if (needed[p] && (st = g.binary(Op::Sub, p, t, &pd)))
            return st;
        if (needed[t] && (st = g.binary(Op::Sub, t, p, &td)))
            return st;
        if (pd != UINT32_MAX && (st = g.binary(Op::Mul, pd, scale, &pgrad)))
            return st;
        if (td != UINT32_MAX && (st = g.binary(Op::Mul, td, scale, &tgrad)))
            return st;
        if (pgrad != UINT32_MAX && (st = accumulate(p, pgrad)))
            return st;
        if (tgrad != UINT32_MAX && (st = accumulate(t, tgrad)))
            return st;
        return PCU_OK;
    }

    // gradients.rs:203-239
    pcu_status matmul_rule(uint32_t left, uint32_t right, uint32_t grad, bool tl, bool tr)
    {
        uint32_t lg = UINT32_MAX, rg = UINT32_MAX;
        pcu_status st;
        if (needed[left]) {
            st = tl ? g.matmul(right, grad, tr, true, &lg) : g.matmul(grad, right, false, !tr, &lg);
            if (st)
                return st;
        }
        if (needed[right]) {
            st = tr ? g.matmul(grad, left, true, tl, &rg) : g.matmul(left, grad, !tl, false, &rg);
            if (st)
                return st;
        }
        if (lg != UINT32_MAX && (st = accumulate(left, lg)))
            return st;
        if (rg != UINT32_MAX && (st = accumulate(right, rg)))
            return st;
        return PCU_OK;
    }

    // gradients.rs:31-137
    pcu_status node_rule(const Node &n, uint32_t grad)
    {
        pcu_status st;
        switch (n.op) {
        case Op::Input:
        case Op::Constant:
        case Op::Uniform:
            return PCU_OK;
        case Op::Add:
            if (needed[n.a] && (st = accumulate(n.a, grad)))
                return st;
            if (needed[n.b] && (st = accumulate(n.b, grad)))
                return st;
            return PCU_OK;
        case Op::Sub:
            if (needed[n.a] && (st = accumulate(n.a, grad)))
                return st;
            if (needed[n.b]) {
                uint32_t neg, rg;
                if ((st = filled_like(n.b, -1.0, &neg)) || (st = g.binary(Op::Mul, grad, neg, &rg)) ||
                    (st = accumulate(n.b, rg)))
                    return st;
            }
            return PCU_OK;
        case Op::Mul: {
            uint32_t lg = UINT32_MAX, rg = UINT32_MAX;
            if (needed[n.a] && (st = g.binary(Op::Mul, grad, n.b, &lg)))
                return st;
            if (needed[n.b] && (st = g.binary(Op::Mul, grad, n.a, &rg)))
                return st;
            if (lg != UINT32_MAX && (st = accumulate(n.a, lg)))
                return st;
            if (rg != UINT32_MAX && (st = accumulate(n.b, rg)))
                return st;
            return PCU_OK;
        }
        case Op::SgdUpdate: {
            uint32_t ig = UINT32_MAX;
            if (needed[n.b]) {
                // -rate, widened exactly (the F32 literal's sign flipped, then widened).
                uint32_t scaled;
                if ((st = filled_like(n.b, -(double)n.lr, &scaled)) ||
                    (st = g.binary(Op::Mul, grad, scaled, &ig)))
                    return st;
            }
            if (needed[n.a] && (st = accumulate(n.a, grad)))
                return st;
            if (ig != UINT32_MAX && (st = accumulate(n.b, ig)))
                return st;
            return PCU_OK;
        }
        case Op::MatMul:
            return matmul_rule(n.a, n.b, grad, n.tl, n.tr);
        case Op::MeanSquaredError:
            return mse_rule(n.a, n.b);
        case Op::Relu:
            if (needed[n.a]) {
                uint32_t ig;
                if ((st = g.relu_backward(n.a, grad, &ig)) || (st = accumulate(n.a, ig)))
                    return st;
            }
            return PCU_OK;
        default:
            g.error = "gradient: unsupported operation";
            return PCU_ERR_UNSUPPORTED;
        }
    }
};

// with_source_scope (gradients.rs:448-474): derived nodes take the source node's numerical
// mode (Boundary when it has none), its numerical options and, where they carry a policy,
// its underflow policy.
template <typename F>
static pcu_status with_source_scope(Graph &g, uint32_t source, F &&append)
{
    Mode mode = g.nodes[source].mode == Mode::None ? Mode::Boundary : g.nodes[source].mode;
    int policy = g.nodes[source].policy;
    Mode previous = g.mode;
    NumOptions previous_options = g.options;
    g.mode = mode;
    g.options = g.nodes[source].options;
    size_t first_new = g.nodes.size();
    pcu_status st = append();
    if (policy >= 0)
        for (size_t i = first_new; i < g.nodes.size(); i++)
            if (g.nodes[i].policy >= 0)
                g.nodes[i].policy = policy;
    g.mode = previous;
    g.options = previous_options;
    return st;
}

// build_backward_mse (gradients.rs:281-444) with preflight derivative_dependencies.
pcu_status Graph::backward(uint32_t loss, const std::vector<uint32_t> *targets,
                           std::vector<uint32_t> *out)
{
    if (check_id(loss)) {
        error = "backward: UnknownValue";
        return PCU_ERR_ARGUMENT;
    }
    if (nodes[loss].op != Op::MeanSquaredError) {
        error = "backward: GradientRootNotMse";
        return PCU_ERR_ARGUMENT;
    }
    size_t original = nodes.size();
    std::vector<char> visited(original, 0);
    std::vector<uint32_t> pending{loss};
    while (!pending.empty()) {
        uint32_t i = pending.back();
        pending.pop_back();
        if (visited[i])
            continue;
        visited[i] = 1;
        const Node &n = nodes[i];
        if ((i != loss && n.op == Op::MeanSquaredError) || n.op == Op::Div || n.op == Op::ReluBackward) {
            error = "backward: UnsupportedGradient";
            return PCU_ERR_UNSUPPORTED;
        }
        uint32_t ops[2];
        int c;
        operands_of(n, ops, &c);
        for (int k = 0; k < c; k++)
            pending.push_back(ops[k]);
    }
    std::vector<char> needed(original, 1);
    if (targets) {
        if (targets->empty()) {
            error = "backward: EmptyOutputs";
            return PCU_ERR_ARGUMENT;
        }
        std::fill(needed.begin(), needed.end(), 0);
        for (uint32_t t : *targets) {
            if (check_id(t) || t >= original || !visited[t]) {
                error = "backward: UnsupportedGradient (target not in the loss closure)";
                return PCU_ERR_UNSUPPORTED;
            }
            needed[t] = 1;
        }
        for (uint32_t i = 0; i <= loss; i++) {
            uint32_t ops[2];
            int c;
            operands_of(nodes[i], ops, &c);
            for (int k = 0; k < c; k++)
                if (needed[ops[k]])
                    needed[i] = 1;
        }
    }
    Backward bw{*this, std::vector<uint32_t>(original, UINT32_MAX), needed};
    bool loss_requested = !targets || std::find(targets->begin(), targets->end(), loss) != targets->end();
    pcu_status st;
    if (!loss_requested) {
        uint32_t p = nodes[loss].a, t = nodes[loss].b;
        st = with_source_scope(*this, loss, [&] { return bw.mse_rule(p, t); });
    } else {
        st = with_source_scope(*this, loss, [&] {
            uint32_t one;
            pcu_status s2 = uniform(nodes[loss].dtype, {}, const_bits(nodes[loss].dtype, 1.0), &one);
            if (!s2)
                bw.grads[loss] = one;
            return s2;
        });
    }
    if (st)
        return st;
    for (int64_t i = loss; i >= 0; i--) {
        uint32_t grad = bw.grads[i];
        if (grad == UINT32_MAX)
            continue;
        Node src = nodes[i]; // copy: the vector grows while rules append
        if (src.op == Op::Input || src.op == Op::Constant || src.op == Op::Uniform)
            continue;
        if (src.op == Op::MeanSquaredError && loss_requested && (uint32_t)i == loss) {
            st = with_source_scope(*this, (uint32_t)i, [&] { return bw.mse_rule(src.a, src.b); });
        } else if (src.op == Op::MeanSquaredError) {
            continue; // the root's rule already ran (its derivative ignores the cotangent)
        } else {
            st = with_source_scope(*this, (uint32_t)i, [&] { return bw.node_rule(src, grad); });
        }
        if (st)
            return st;
    }
    *out = bw.grads;
    return PCU_OK;
}

// execution_plan_for_outputs (tensor.rs:3234-3300): requested outputs' closures plus every
// checked node's closure, in graph order.
pcu_status Graph::plan(const std::vector<uint32_t> &outputs, std::vector<uint32_t> *order) const
{
    if (outputs.empty())
        return PCU_ERR_ARGUMENT;
    std::vector<char> selected(nodes.size(), 0);
    auto close = [&](uint32_t start) {
        std::vector<uint32_t> stack{start};
        while (!stack.empty()) {
            uint32_t i = stack.back();
            stack.pop_back();
            if (selected[i])
                continue;
            selected[i] = 1;
            uint32_t ops[2];
            int c;
            operands_of(nodes[i], ops, &c);
            for (int k = 0; k < c; k++)
                stack.push_back(ops[k]);
        }
    };
    for (size_t k = 0; k < outputs.size(); k++) {
        if (check_id(outputs[k]))
            return PCU_ERR_ARGUMENT;
        for (size_t j = 0; j < k; j++)
            if (outputs[j] == outputs[k])
                return PCU_ERR_ARGUMENT; // DuplicateOutput
        close(outputs[k]);
    }
    for (uint32_t i = 0; i < nodes.size(); i++)
        if (nodes[i].policy >= 0 || nodes[i].mode != Mode::None)
            close(i);
    order->clear();
    for (uint32_t i = 0; i < nodes.size(); i++)
        if (selected[i])
            order->push_back(i);
    return PCU_OK;
}

// ------------------------------------------------------------------- executor

static size_t dsize(int dtype) { return dtype == 0 ? 4 : 8; }

void prepared_detach(Prepared *p)
{
    Ctx *ctx = p->ctx;
    if (!ctx)
        return;
    (void)ctx->join_side();
    (void)hipStreamSynchronize(ctx->stream);
    for (int b = 0; b < 2; b++)
        for (void *&q : p->buf[b])
            if (q) {
                (void)ctx->release(q);
                q = nullptr;
            }
    for (auto *list : {&p->dense_uniform, &p->constant_buf, &p->pre_rows, &p->pre_cols})
        for (void *&q : *list)
            if (q) {
                (void)ctx->release(q);
                q = nullptr;
            }
    auto &list = ctx->prepared;
    list.erase(std::remove(list.begin(), list.end(), p), list.end());
    p->ctx = nullptr;
    p->published = false;
}

Prepared::~Prepared() { prepared_detach(this); }

pcu_status Prepared::build(Ctx *c, const Graph &g, const std::vector<uint32_t> &outs)
{
    ctx = c;
    c->prepared.push_back(this);
    graph = g;
    outputs = outs;
    pcu_status st = graph.plan(outputs, &order);
    if (st) {
        error = "prepare: invalid output selection";
        return st;
    }
    size_t n = graph.nodes.size();
    for (int b = 0; b < 2; b++)
        buf[b].assign(n, nullptr);
    is_output.assign(n, 0);
    fused_into.assign(n, -1);
    mse_side.assign(n, 0);
    dense_uniform.assign(n, nullptr);
    constant_buf.assign(n, nullptr);
    pre_rows.assign(n, nullptr);
    pre_cols.assign(n, nullptr);
    for (uint32_t o : outputs)
        is_output[o] = 1;
    std::vector<uint32_t> uses(n, 0);
    std::vector<char> in_plan(n, 0);
    for (uint32_t i : order)
        in_plan[i] = 1;
    for (uint32_t i : order) {
        const Node &nd = graph.nodes[i];
        if (nd.a != UINT32_MAX)
            uses[nd.a]++;
        if (nd.b != UINT32_MAX)
            uses[nd.b]++;
    }
    route.assign(n, Route::Scalar);
    for (uint32_t i : order) {
        const Node &nd = graph.nodes[i];
        // Admission of compound primitives (backends/rocm/tensor.rs:9016-9058,
        // tensor/native_loss/native_loss.rs:66-120, tensor/native_sgd/native_sgd.rs:46-100):
        // Strict runs the checked ordered kernels; Boundary runs only under explicitly
        // permitted native compound arithmetic with unspecified reproducibility and the IEEE
        // (or no) underflow policy; a checked result-boundary compound is not implemented.
        if (nd.op == Op::MatMul || nd.op == Op::MeanSquaredError || nd.op == Op::SgdUpdate) {
            if (nd.mode == Mode::Strict) {
                route[i] = Route::Strict;
            } else if (nd.options.compound != 1) {
                error = "prepare: checked result-boundary compound arithmetic is not implemented; "
                        "select strict checking or explicitly permit native compound arithmetic";
                return PCU_ERR_UNSUPPORTED;
            } else if (nd.options.reproducibility != 0) {
                error = "prepare: native compound arithmetic has no portable reproducibility profile";
                return PCU_ERR_UNSUPPORTED;
            } else if (nd.policy > 0) {
                error = "prepare: native compound arithmetic admits only the IEEE underflow policy";
                return PCU_ERR_UNSUPPORTED;
            } else {
                route[i] = Route::Native;
            }
        }
        if (nd.op == Op::Input)
            inputs.push_back(i);
    }
    // Fuse an Add whose only consumer is a ReLU (and which is not an output) into it.
    for (uint32_t i : order) {
        const Node &nd = graph.nodes[i];
        if (nd.op == Op::Relu) {
            uint32_t a = nd.a;
            const Node &an = graph.nodes[a];
            if (an.op == Op::Add && uses[a] == 1 && !is_output[a] && an.policy == nd.policy &&
                graph.nodes[an.a].op != Op::Uniform)
                fused_into[a] = (int)i;
        }
    }
    // Chains: consecutive launching elementwise nodes (checked binary, ReLU, ReLU backward)
    // of one dtype and shape, each an operand of the next, run as one kernel with one fault
    // word per node (launch order and fault order unchanged; the values between them stay
    // in registers). A later step may not read an earlier step's stored value as its other
    // operand, so every value a step reads was written before the launch.
    chain_next.assign(n, UINT32_MAX);
    chain_len.assign(n, 0);
    chain_member.assign(n, 0);
    chain_store.assign(n, 1);
    {
        auto launches = [&](uint32_t i) {
            const Op op = graph.nodes[i].op;
            return op != Op::Input && op != Op::Constant && op != Op::Uniform && fused_into[i] < 0;
        };
        auto chainable = [&](uint32_t i) {
            const Node &nd = graph.nodes[i];
            const bool elementwise = nd.op == Op::Add || nd.op == Op::Sub || nd.op == Op::Mul ||
                                     nd.op == Op::Div || nd.op == Op::Relu || nd.op == Op::ReluBackward;
            // A ReLU that has absorbed its Add already runs as one kernel.
            return elementwise && !(nd.op == Op::Relu && fused_into[nd.a] == (int)i);
        };
        auto binary = [&](uint32_t i) {
            const Op op = graph.nodes[i].op;
            return op == Op::Add || op == Op::Sub || op == Op::Mul || op == Op::Div;
        };
        std::vector<uint32_t> run;
        for (uint32_t i : order)
            if (launches(i))
                run.push_back(i);
        for (size_t k = 0; k < run.size();) {
            const uint32_t h = run[k];
            const Node &hn = graph.nodes[h];
            // The head's chain operand must be dense: a binary node takes its dense side.
            bool ok = chainable(h) && !(binary(h) && graph.nodes[hn.a].op == Op::Uniform &&
                                        graph.nodes[hn.b].op == Op::Uniform);
            std::vector<uint32_t> members{h};
            while (ok && k + members.size() < run.size() && (int)members.size() < kChainMaxSteps) {
                const uint32_t x = members.back(), y = run[k + members.size()];
                const Node &yn = graph.nodes[y];
                if (!chainable(y) || yn.dtype != hn.dtype || graph.nodes[y].shape != hn.shape)
                    break;
                if (yn.op == Op::Relu) {
                    if (yn.a != x)
                        break;
                } else {
                    if ((yn.a == x) == (yn.b == x))
                        break; // x is not an operand, or is both
                    const uint32_t other = yn.a == x ? yn.b : yn.a;
                    if (std::find(members.begin(), members.end(), other) != members.end())
                        break;
                }
                members.push_back(y);
            }
            if (members.size() > 1) {
                chain_len[h] = (int)members.size();
                for (size_t j = 0; j < members.size(); j++) {
                    const uint32_t m = members[j];
                    if (j + 1 < members.size())
                        chain_next[m] = members[j + 1];
                    if (j > 0)
                        chain_member[m] = 1;
                    chain_store[m] = j + 1 == members.size() || is_output[m] || uses[m] > 1;
                }
            }
            k += members.size();
        }
    }
    sgd_partner.assign(n, UINT32_MAX);
    sgd_second.assign(n, 0);
    {
        std::vector<uint32_t> run;
        for (uint32_t i : order) {
            const Op op = graph.nodes[i].op;
            if (op != Op::Input && op != Op::Constant && op != Op::Uniform && fused_into[i] < 0 &&
                !chain_member[i])
                run.push_back(i);
        }
        auto strict_sgd = [&](uint32_t i) {
            return graph.nodes[i].op == Op::SgdUpdate && route[i] == Route::Strict;
        };
        for (size_t k = 0; k + 1 < run.size(); k++) {
            const uint32_t x = run[k], y = run[k + 1];
            const Node &xn = graph.nodes[x], &yn = graph.nodes[y];
            if (strict_sgd(x) && strict_sgd(y) && !sgd_second[x] && xn.dtype == yn.dtype &&
                xn.policy == yn.policy && yn.a != x && yn.b != x && graph.elements(x) > 0 &&
                graph.elements(y) > 0) {
                sgd_partner[x] = y;
                sgd_second[y] = 1;
            }
        }
    }
    gemm_epi.assign(n, UINT32_MAX);
    epi_member.assign(n, 0);
    prog_pos.assign(n, UINT32_MAX);
    {
        // Launch order, and each launch's program nodes (a chain: one per step; an Add
        // fused into its ReLU and a paired SGD: two), as the execution loop adds them.
        std::vector<uint32_t> run;
        std::vector<int> pos(n, -1);
        uint32_t next = 0;
        for (uint32_t i : order) {
            const Node &nd = graph.nodes[i];
            if (nd.op == Op::Input || nd.op == Op::Constant || nd.op == Op::Uniform ||
                fused_into[i] >= 0 || chain_member[i] || sgd_second[i])
                continue;
            pos[i] = (int)run.size();
            run.push_back(i);
            prog_pos[i] = next;
            if (chain_len[i] > 1)
                next += (uint32_t)chain_len[i];
            else if ((nd.op == Op::Relu && fused_into[nd.a] == (int)i) ||
                     sgd_partner[i] != UINT32_MAX)
                next += 2;
            else
                next += 1;
        }
        // The node's operands other than the product must be ready when the MatMul runs:
        // not produced by a launch between the two.
        auto ready = [&](uint32_t v, size_t at) { return pos[v] < 0 || (size_t)pos[v] < at; };
        for (size_t k = 0; k < run.size(); k++) {
            const uint32_t m = run[k];
            const Node &mn = graph.nodes[m];
            if (mn.op != Op::MatMul || route[m] != Route::Strict)
                continue;
            for (size_t j = k + 1; j < run.size() && j <= k + kEpiWindow; j++) {
                const uint32_t r = run[j];
                const Node &rn = graph.nodes[r];
                if (epi_member[r] || chain_len[r] > 1 || rn.dtype != mn.dtype || rn.shape != mn.shape)
                    continue;
                const bool relu = rn.op == Op::Relu && rn.a == m;
                const bool back = rn.op == Op::ReluBackward && rn.b == m && rn.a != m && ready(rn.a, k);
                if (relu || back) {
                    gemm_epi[m] = r;
                    epi_member[r] = 1;
                    break;
                }
            }
        }
    }
    // Tables an epilogue writes for the strict F32 MatMuls that read its node's value: op(A)
    // rows are the value's rows when A is untransposed, its columns when transposed; op(B)
    // columns are its columns when B is untransposed, its rows when transposed. Only for
    // values of whole 128 x 128 tiles (where the epilogue can run).
    std::vector<char> want_rows(n, 0), want_cols(n, 0);
    for (uint32_t q : order) {
        const Node &qn = graph.nodes[q];
        if (qn.op != Op::MatMul || route[q] != Route::Strict || qn.dtype != 0)
            continue;
        for (int side = 0; side < 2; side++) {
            const uint32_t r = side == 0 ? qn.a : qn.b;
            if (!epi_member[r] || graph.nodes[r].dtype != 0 || graph.nodes[r].shape.size() != 2)
                continue;
            const bool transposed = side == 0 ? qn.tl : qn.tr;
            if (side == 0 ? !transposed : transposed)
                want_rows[r] = 1;
            else
                want_cols[r] = 1;
        }
    }
    // The ordered MSE sum runs on the side stream when nothing in the plan consumes its
    // value (the training-loss case): it then overlaps the backward pass. A small one (one
    // kernel of one workgroup) stays on the main stream: the fork and join cost the host
    // more than the overlap saves.
    for (uint32_t i : order)
        if (graph.nodes[i].op == Op::MeanSquaredError && uses[i] == 0 && route[i] == Route::Strict &&
            graph.elements(graph.nodes[i].a) > kMseSerialMax)
            mse_side[i] = 1;
    // Device storage: one buffer per computed node; outputs get two banks so a faulting
    // execution never overwrites the published results. A Constant is uploaded once here
    // and stays resident for every execution (the reference allocates and uploads its
    // constants with the plan's scratch: backends/rocm/tensor.rs:2955-2980).
    for (uint32_t i : order) {
        const Node &nd = graph.nodes[i];
        if (nd.op == Op::Constant) {
            const size_t bytes = nd.data ? nd.data->size() : 0;
            if ((st = ctx->alloc(bytes, &constant_buf[i])))
                return st;
            if (bytes && (st = ctx->copy(constant_buf[i], nd.data->data(), bytes, true)))
                return st;
            continue;
        }
        if (nd.op == Op::Input || nd.op == Op::Uniform || fused_into[i] >= 0 || !chain_store[i])
            continue;
        size_t bytes = graph.elements(i) * dsize(nd.dtype);
        for (int b = 0; b < (is_output[i] ? 2 : 1); b++)
            if ((st = ctx->alloc(bytes, &buf[b][i])))
                return st;
    }
    for (uint32_t r : order) {
        if (!want_rows[r] && !want_cols[r])
            continue;
        const auto &sh = graph.nodes[r].shape;
        const uint64_t m = sh[0], w = sh[1];
        if (m == 0 || w == 0 || m % 128 != 0 || w % 128 != 0)
            continue; // never whole tiles: its MatMul launches the elementwise kernel
        if (want_rows[r] && (st = ctx->alloc(m * (w / 64) * sizeof(short), &pre_rows[r])))
            return st;
        if (want_cols[r] && (st = ctx->alloc((m / 64) * w * sizeof(short), &pre_cols[r])))
            return st;
    }
    published_ptr.assign(outputs.size(), nullptr);
    return PCU_OK;
}

void *Prepared::value_ptr(uint32_t id, const std::vector<const void *> &in, int bank) const
{
    const Node &nd = graph.nodes[id];
    if (nd.op == Op::Input) {
        for (size_t k = 0; k < inputs.size(); k++)
            if (inputs[k] == id)
                return const_cast<void *>(in[k]);
        return nullptr;
    }
    if (nd.op == Op::Uniform)
        return dense_uniform[id];
    if (nd.op == Op::Constant)
        return constant_buf[id];
    return buf[is_output[id] ? bank : 0][id];
}

ChainLaunch Prepared::chain_launch(uint32_t head, const std::vector<const void *> &in, int bank_w) const
{
    ChainLaunch c;
    // A Uniform operand that was not materialized goes in as its bits.
    auto dense = [&](uint32_t id) {
        return graph.nodes[id].op != Op::Uniform || dense_uniform[id] != nullptr;
    };
    auto set_other = [&](ChainStep &st, uint32_t id, int dtype) {
        if (dense(id)) {
            st.other = value_ptr(id, in, bank_w);
        } else {
            const uint64_t bits = graph.nodes[id].value_bits;
            st.other_bits = dtype == 0 ? (uint32_t)bits : bits;
        }
    };
    uint32_t prev = UINT32_MAX;
    for (uint32_t m = head; m != UINT32_MAX; m = chain_next[m]) {
        const Node &nd = graph.nodes[m];
        ChainStep &st = c.step[c.steps++];
        st.policy = nd.policy < 0 ? 0 : nd.policy;
        st.out = chain_store[m] ? value_ptr(m, in, bank_w) : nullptr;
        st.op = nd.op == Op::Add ? kOpAdd : nd.op == Op::Sub ? kOpSub : nd.op == Op::Mul ? kOpMul
              : nd.op == Op::Div ? kOpDiv : nd.op == Op::Relu ? kStepRelu : kStepReluBackward;
        if (nd.op == Op::Relu) {
            if (prev == UINT32_MAX)
                c.head = value_ptr(nd.a, in, bank_w);
        } else if (prev == UINT32_MAX) {
            // The head reads its dense left operand, or its right one when the left is an
            // unmaterialized Uniform.
            const bool left = dense(nd.a);
            c.head = value_ptr(left ? nd.a : nd.b, in, bank_w);
            st.chain_right = left ? 0 : 1;
            set_other(st, left ? nd.b : nd.a, nd.dtype);
        } else {
            st.chain_right = nd.b == prev ? 1 : 0;
            set_other(st, nd.b == prev ? nd.a : nd.b, nd.dtype);
        }
        prev = m;
    }
    return c;
}

pcu_status Prepared::execute(const std::vector<const void *> &in, pcu_fault *fault)
{
    if (in.size() != inputs.size()) {
        error = "execute: wrong number of inputs (MissingInput/ExtraInput)";
        return PCU_ERR_ARGUMENT;
    }
    pcu_status st;
    // Uniform operands that a kernel cannot take as a broadcast scalar are materialized once.
    for (uint32_t i : order) {
        const Node &nd = graph.nodes[i];
        auto needs_dense = [&](uint32_t operand, bool right_scalar_ok) {
            return graph.nodes[operand].op == Op::Uniform && !right_scalar_ok;
        };
        uint32_t ops[2] = {nd.a, nd.b};
        for (int k = 0; k < 2; k++) {
            uint32_t o = ops[k];
            if (o == UINT32_MAX || graph.nodes[o].op != Op::Uniform || dense_uniform[o])
                continue;
            bool elementwise = nd.op == Op::Add || nd.op == Op::Sub || nd.op == Op::Mul || nd.op == Op::Div;
            bool commutes = nd.op == Op::Add || nd.op == Op::Mul;
            bool scalar_ok = elementwise && (k == 1 || (commutes && graph.nodes[nd.b].op != Op::Uniform));
            if (!needs_dense(o, scalar_ok))
                continue;
            const Node &u = graph.nodes[o];
            size_t bytes = graph.elements(o) * dsize(u.dtype);
            if ((st = ctx->alloc(bytes, &dense_uniform[o])))
                return st;
            // Fill: upload the value pattern once (cold path).
            std::vector<unsigned char> host(bytes);
            for (size_t e = 0; e < graph.elements(o); e++)
                memcpy(host.data() + e * dsize(u.dtype), &u.value_bits, dsize(u.dtype));
            if ((st = ctx->copy(dense_uniform[o], host.data(), bytes, true)))
                return st;
        }
    }
    const int bank_w = bank;
    if ((st = ctx->begin_program(false)))
        return st;
    std::vector<uint32_t> prog_to_graph;
    std::vector<unsigned long long *> epi_word(graph.nodes.size(), nullptr);
    std::vector<char> tables_written(graph.nodes.size(), 0); // this execution, by an epilogue
    // The program's last launching node: a strict SGD update (or pair) there ends the program
    // in its own kernel instead of a publication launch.
    uint32_t last_launch = UINT32_MAX;
    for (uint32_t i : order) {
        const Node &nd = graph.nodes[i];
        if (nd.op == Op::Input || nd.op == Op::Constant || nd.op == Op::Uniform ||
            fused_into[i] >= 0 || chain_member[i] || sgd_second[i])
            continue;
        last_launch = i;
    }
    auto ptr = [&](uint32_t id) { return value_ptr(id, in, bank_w); };
    // The tables this execution's epilogues wrote for a strict F32 MatMul's operands.
    auto prescreen = [&](uint32_t q) {
        const Node &qn = graph.nodes[q];
        Prescreen p;
        if (qn.dtype != 0)
            return p;
        if (tables_written[qn.a])
            p.a = (const short *)(qn.tl ? pre_cols[qn.a] : pre_rows[qn.a]);
        if (tables_written[qn.b])
            p.b = (const short *)(qn.tr ? pre_rows[qn.b] : pre_cols[qn.b]);
        return p;
    };
    for (uint32_t i : order) {
        const Node &nd = graph.nodes[i];
        if (nd.op == Op::Input || nd.op == Op::Constant || nd.op == Op::Uniform || fused_into[i] >= 0 ||
            chain_member[i] || sgd_second[i])
            continue;
        if (epi_member[i]) {
            // Evaluated with its MatMul; its program node takes its own place here.
            if ((st = ctx->add_fused_node(graph.elements(i), epi_word[i]))) {
                pcu_fault ignore;
                (void)ctx->end_program(&ignore);
                error = ctx->error;
                return st;
            }
            prog_to_graph.push_back(i);
            continue;
        }
        uint64_t n = graph.elements(i);
        int policy = nd.policy < 0 ? 0 : nd.policy;
        if (chain_len[i] > 1) {
            st = ctx->op_chain(nd.dtype, n, chain_launch(i, in, bank_w));
            for (uint32_t m = i; m != UINT32_MAX; m = chain_next[m])
                prog_to_graph.push_back(m);
            if (st) {
                pcu_fault ignore;
                (void)ctx->end_program(&ignore);
                error = ctx->error;
                return st;
            }
            continue;
        }
        switch (nd.op) {
        case Op::Add:
        case Op::Sub:
        case Op::Mul:
        case Op::Div: {
            int op = nd.op == Op::Add ? kOpAdd : nd.op == Op::Sub ? kOpSub : nd.op == Op::Mul ? kOpMul : kOpDiv;
            uint32_t l = nd.a, r = nd.b;
            bool lu = graph.nodes[l].op == Op::Uniform && !dense_uniform[l];
            bool ru = graph.nodes[r].op == Op::Uniform && !dense_uniform[r];
            if (lu && !ru)
                std::swap(l, r); // Add/Mul commute bitwise in IEEE arithmetic
            bool uniform = graph.nodes[r].op == Op::Uniform && !dense_uniform[r];
            const void *bval = uniform ? (const void *)&graph.nodes[r].value_bits : nullptr;
            uint32_t b32 = (uint32_t)graph.nodes[r].value_bits;
            if (uniform && nd.dtype == 0)
                bval = &b32;
            st = ctx->op_binary(nd.dtype, op, n, ptr(l), uniform ? nullptr : ptr(r), bval, ptr(i), policy);
            prog_to_graph.push_back(i);
            break;
        }
        case Op::Relu: {
            int a = (int)nd.a;
            if (fused_into[a] == (int)i) {
                const Node &an = graph.nodes[a];
                uint32_t l = an.a, r = an.b;
                bool ru = graph.nodes[r].op == Op::Uniform && !dense_uniform[r];
                uint32_t b32 = (uint32_t)graph.nodes[r].value_bits;
                const void *bval = ru ? (nd.dtype == 0 ? (const void *)&b32 : (const void *)&graph.nodes[r].value_bits) : nullptr;
                st = ctx->op_add_relu(nd.dtype, n, ptr(l), ru ? nullptr : ptr(r), bval, ptr(i), policy);
                prog_to_graph.push_back((uint32_t)a);
                prog_to_graph.push_back(i);
            } else {
                st = ctx->op_relu(nd.dtype, n, ptr(nd.a), ptr(i), policy);
                prog_to_graph.push_back(i);
            }
            break;
        }
        case Op::ReluBackward:
            st = ctx->op_relu_backward(nd.dtype, n, ptr(nd.a), ptr(nd.b), ptr(i), policy);
            prog_to_graph.push_back(i);
            break;
        case Op::MatMul: {
            const auto &sa = graph.nodes[nd.a].shape;
            uint64_t inner = nd.tl ? sa[0] : sa[1];
            if (route[i] == Route::Native)
                st = ctx->op_native_matmul(nd.dtype, nd.shape[0], inner, nd.shape[1], nd.tl, nd.tr,
                                           ptr(nd.a), ptr(nd.b), ptr(i));
            else if (gemm_epi[i] != UINT32_MAX) {
                const uint32_t r = gemm_epi[i];
                const Node &rn = graph.nodes[r];
                GemmEpilogue epi;
                epi.op = rn.op == Op::Relu ? kStepRelu : kStepReluBackward;
                epi.policy = rn.policy < 0 ? 0 : rn.policy;
                epi.x = rn.op == Op::Relu ? nullptr : ptr(rn.a);
                epi.out = ptr(r);
                epi.tbl_rows = (short *)pre_rows[r];
                epi.tbl_cols = (short *)pre_cols[r];
                bool fused = false;
                st = ctx->op_matmul(nd.dtype, nd.shape[0], inner, nd.shape[1], nd.tl, nd.tr,
                                    ptr(nd.a), ptr(nd.b), ptr(i), policy, false, &epi,
                                    prog_pos[r] - prog_pos[i] - 1, prescreen(i), &fused);
                epi_word[r] = epi.fault;
                tables_written[r] = fused && (epi.tbl_rows || epi.tbl_cols);
            } else
                st = ctx->op_matmul(nd.dtype, nd.shape[0], inner, nd.shape[1], nd.tl, nd.tr,
                                    ptr(nd.a), ptr(nd.b), ptr(i), policy, false, nullptr, 0,
                                    prescreen(i));
            prog_to_graph.push_back(i);
            break;
        }
        case Op::MeanSquaredError:
            if (route[i] == Route::Native)
                st = ctx->op_native_mse(nd.dtype, graph.elements(nd.a), ptr(nd.a), ptr(nd.b), ptr(i));
            else
                st = ctx->op_mse(nd.dtype, graph.elements(nd.a), ptr(nd.a), ptr(nd.b), ptr(i),
                                 policy, mse_side[i] != 0);
            prog_to_graph.push_back(i);
            break;
        case Op::SgdUpdate:
            if (i == last_launch && route[i] == Route::Strict && !epi_member[i])
                ctx->close_with_next_op();
            if (route[i] == Route::Native) {
                st = ctx->op_native_sgd(nd.dtype, n, ptr(nd.a), ptr(nd.b), nd.lr,
                                        nd.options.precision == 1, ptr(i));
            } else if (sgd_partner[i] != UINT32_MAX) {
                const uint32_t j = sgd_partner[i];
                const Node &jn = graph.nodes[j];
                const uint64_t cnt[2] = {n, graph.elements(j)};
                const void *const w[2] = {ptr(nd.a), ptr(jn.a)};
                const void *const g[2] = {ptr(nd.b), ptr(jn.b)};
                const float lr[2] = {nd.lr, jn.lr};
                void *const out[2] = {ptr(i), ptr(j)};
                st = ctx->op_sgd_pair(nd.dtype, cnt, w, g, lr, out, policy);
                prog_to_graph.push_back(i);
                prog_to_graph.push_back(j);
                break;
            } else {
                st = ctx->op_sgd(nd.dtype, n, ptr(nd.a), ptr(nd.b), nd.lr, ptr(i), policy);
            }
            prog_to_graph.push_back(i);
            break;
        default:
            break;
        }
        if (st) {
            pcu_fault ignore;
            (void)ctx->end_program(&ignore);
            error = ctx->error;
            return st;
        }
    }
    // One terminal synchronization; every node's fault word is read and the earliest graph
    // node wins (a node that the reference would never reach may also have faulted here).
    std::vector<pcu_fault> faults;
    st = ctx->end_program_all(&faults);
    if (st == PCU_ERR_PROTOCOL && fault) {
        *fault = ctx->protocol_fault;
        fault->node = prog_to_graph[ctx->protocol_fault.node];
    }
    if (st) {
        error = ctx->error;
        return st;
    }
    const pcu_fault *first = nullptr;
    for (const pcu_fault &f : faults)
        if (!first || prog_to_graph[f.node] < prog_to_graph[first->node])
            first = &f;
    if (first) {
        if (fault) {
            *fault = *first;
            fault->node = prog_to_graph[first->node];
        }
        return PCU_ARITHMETIC_FAULT; // nothing published; the previous bank stays current
    }
    for (size_t k = 0; k < outputs.size(); k++)
        published_ptr[k] = value_ptr(outputs[k], in, bank_w);
    published = true;
    bank ^= 1;
    return PCU_OK;
}

} // namespace pcu

// ======================================================================= C ABI

using pcu::Graph;
using pcu::Op;
using pcu::Prepared;

static pcu_status graph_fail(Graph *g, pcu_status st)
{
    if (st && g)
        pcu::g_thread_error = g->error;
    return st;
}

extern "C" {

pcu_status pcu_graph_create(pcu_graph **out)
{
    if (!out)
        return PCU_ERR_ARGUMENT;
    Graph *g = new (std::nothrow) Graph();
    if (!g)
        return PCU_ERR_OUT_OF_MEMORY;
    *out = reinterpret_cast<pcu_graph *>(g);
    return PCU_OK;
}

void pcu_graph_destroy(pcu_graph *g) { delete reinterpret_cast<Graph *>(g); }

pcu_status pcu_graph_set_numerical_mode(pcu_graph *gh, int strict)
{
    if (!gh)
        return PCU_ERR_ARGUMENT;
    reinterpret_cast<Graph *>(gh)->mode = strict ? pcu::Mode::Strict : pcu::Mode::Boundary;
    return PCU_OK;
}

pcu_status pcu_graph_input(pcu_graph *gh, pcu_dtype dtype, uint32_t rank, const uint64_t *shape,
                           uint32_t *id)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g || (rank && !shape))
        return PCU_ERR_ARGUMENT;
    return graph_fail(g, g->input(dtype, std::vector<uint64_t>(shape, shape + rank), id));
}

pcu_status pcu_graph_uniform(pcu_graph *gh, pcu_dtype dtype, uint32_t rank, const uint64_t *shape,
                             uint64_t value_bits, uint32_t *id)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g || (rank && !shape))
        return PCU_ERR_ARGUMENT;
    return graph_fail(g, g->uniform(dtype, std::vector<uint64_t>(shape, shape + rank), value_bits, id));
}

pcu_status pcu_graph_constant(pcu_graph *gh, pcu_dtype dtype, uint32_t rank, const uint64_t *shape,
                              const void *host_data, uint32_t *id)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g || (rank && !shape))
        return PCU_ERR_ARGUMENT;
    return graph_fail(g, g->constant(dtype, std::vector<uint64_t>(shape, shape + rank), host_data, id));
}

pcu_status pcu_graph_binary(pcu_graph *gh, pcu_binary_op op, uint32_t a, uint32_t b, uint32_t *id)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g || op < 0 || op > 3)
        return PCU_ERR_ARGUMENT;
    Op o = op == PCU_OP_ADD ? Op::Add : op == PCU_OP_SUB ? Op::Sub : op == PCU_OP_MUL ? Op::Mul : Op::Div;
    return graph_fail(g, g->binary(o, a, b, id));
}

pcu_status pcu_graph_relu(pcu_graph *gh, uint32_t x, uint32_t *id)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g)
        return PCU_ERR_ARGUMENT;
    return graph_fail(g, g->relu(x, id));
}

pcu_status pcu_graph_relu_backward(pcu_graph *gh, uint32_t input, uint32_t upstream, uint32_t *id)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g)
        return PCU_ERR_ARGUMENT;
    return graph_fail(g, g->relu_backward(input, upstream, id));
}

pcu_status pcu_graph_matmul(pcu_graph *gh, uint32_t a, uint32_t b, int transpose_left,
                            int transpose_right, uint32_t *id)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g)
        return PCU_ERR_ARGUMENT;
    return graph_fail(g, g->matmul(a, b, transpose_left != 0, transpose_right != 0, id));
}

pcu_status pcu_graph_mean_squared_error(pcu_graph *gh, uint32_t prediction, uint32_t target, uint32_t *id)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g)
        return PCU_ERR_ARGUMENT;
    return graph_fail(g, g->mse(prediction, target, id));
}

pcu_status pcu_graph_sgd_update(pcu_graph *gh, uint32_t weights, uint32_t gradient,
                                float learning_rate, uint32_t *id)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g)
        return PCU_ERR_ARGUMENT;
    return graph_fail(g, g->sgd(weights, gradient, learning_rate, id));
}

pcu_status pcu_graph_set_underflow_policy(pcu_graph *gh, uint32_t id, pcu_underflow policy)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g || g->check_id(id) || policy < 0 || policy > 2)
        return PCU_ERR_ARGUMENT;
    g->nodes[id].policy = policy;
    return PCU_OK;
}

pcu_status pcu_graph_set_value_numerical_mode(pcu_graph *gh, uint32_t id, int strict)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g || g->check_id(id))
        return PCU_ERR_ARGUMENT;
    if (g->nodes[id].mode == pcu::Mode::None) {
        // tensor.rs:3154-3166: scalar nodes carry no mode (UnsupportedNumericalMode).
        g->error = "set_value_numerical_mode: UnsupportedNumericalMode (not a compound node)";
        return graph_fail(g, PCU_ERR_UNSUPPORTED);
    }
    g->nodes[id].mode = strict ? pcu::Mode::Strict : pcu::Mode::Boundary;
    return PCU_OK;
}

static bool valid_options(const pcu_numerical_options *o)
{
    return o && o->compound_arithmetic <= 1 && o->precision <= 1 && o->reproducibility <= 1;
}

static pcu::NumOptions to_options(const pcu_numerical_options *o)
{
    pcu::NumOptions r;
    r.compound = o->compound_arithmetic;
    r.precision = o->precision;
    r.reproducibility = o->reproducibility;
    return r;
}

pcu_status pcu_graph_set_numerical_options(pcu_graph *gh, const pcu_numerical_options *options)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g || !valid_options(options))
        return PCU_ERR_ARGUMENT;
    g->options = to_options(options);
    return PCU_OK;
}

pcu_status pcu_graph_set_value_numerical_options(pcu_graph *gh, uint32_t id,
                                                 const pcu_numerical_options *options)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g || g->check_id(id) || !valid_options(options))
        return PCU_ERR_ARGUMENT;
    g->nodes[id].options = to_options(options);
    return PCU_OK;
}

pcu_status pcu_graph_backward_mse(pcu_graph *gh, uint32_t loss, uint32_t *grads, uint32_t capacity)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g || !grads)
        return PCU_ERR_ARGUMENT;
    if (capacity < g->nodes.size())
        return PCU_ERR_ARGUMENT;
    std::vector<uint32_t> out;
    pcu_status st = g->backward(loss, nullptr, &out);
    if (st)
        return graph_fail(g, st);
    for (size_t i = 0; i < out.size(); i++)
        grads[i] = out[i];
    return PCU_OK;
}

pcu_status pcu_graph_backward_mse_for_targets(pcu_graph *gh, uint32_t loss, uint32_t n_targets,
                                              const uint32_t *targets, uint32_t *grads)
{
    Graph *g = reinterpret_cast<Graph *>(gh);
    if (!g || (n_targets && (!targets || !grads)))
        return PCU_ERR_ARGUMENT;
    std::vector<uint32_t> t(targets, targets + n_targets), out;
    pcu_status st = g->backward(loss, &t, &out);
    if (st)
        return graph_fail(g, st);
    for (uint32_t k = 0; k < n_targets; k++) {
        if (out[targets[k]] == UINT32_MAX) {
            g->error = "backward: UnsupportedGradient";
            return graph_fail(g, PCU_ERR_UNSUPPORTED);
        }
        grads[k] = out[targets[k]];
    }
    return PCU_OK;
}

uint32_t pcu_graph_node_count(const pcu_graph *gh)
{
    return gh ? (uint32_t)reinterpret_cast<const Graph *>(gh)->nodes.size() : 0;
}

pcu_status pcu_graph_describe(const pcu_graph *gh, uint32_t id, pcu_node_desc *out)
{
    const Graph *g = reinterpret_cast<const Graph *>(gh);
    if (!g || !out || g->check_id(id))
        return PCU_ERR_ARGUMENT;
    const pcu::Node &n = g->nodes[id];
    memset(out, 0, sizeof *out);
    out->op = (uint32_t)n.op;
    out->left = n.a;
    out->right = n.b;
    out->transpose_left = n.tl;
    out->transpose_right = n.tr;
    out->dtype = (uint32_t)n.dtype;
    out->numerical_mode = (int32_t)n.mode;
    out->underflow_policy = n.policy;
    out->learning_rate = n.lr;
    out->value_bits = n.value_bits;
    out->rank = (uint32_t)n.shape.size();
    for (size_t k = 0; k < n.shape.size() && k < 8; k++)
        out->shape[k] = n.shape[k];
    out->options.compound_arithmetic = n.options.compound;
    out->options.precision = n.options.precision;
    out->options.reproducibility = n.options.reproducibility;
    return PCU_OK;
}

pcu_status pcu_graph_plan(const pcu_graph *gh, uint32_t n_outputs, const uint32_t *outputs,
                          uint32_t *order, uint32_t *order_len)
{
    const Graph *g = reinterpret_cast<const Graph *>(gh);
    if (!g || !order_len || (n_outputs && !outputs))
        return PCU_ERR_ARGUMENT;
    std::vector<uint32_t> o;
    pcu_status st = g->plan(std::vector<uint32_t>(outputs, outputs + n_outputs), &o);
    if (st)
        return st;
    if (order) {
        if (*order_len < o.size())
            return PCU_ERR_ARGUMENT;
        std::copy(o.begin(), o.end(), order);
    }
    *order_len = (uint32_t)o.size();
    return PCU_OK;
}

pcu_status pcu_prepare(pcu_ctx *ctx, const pcu_graph *gh, uint32_t n_outputs, const uint32_t *outputs,
                       pcu_prepared **out)
{
    if (!ctx || !gh || !out || (n_outputs && !outputs))
        return PCU_ERR_ARGUMENT;
    *out = nullptr;
    Prepared *p = new (std::nothrow) Prepared();
    if (!p)
        return PCU_ERR_OUT_OF_MEMORY;
    pcu::Ctx *c = reinterpret_cast<pcu::Ctx *>(ctx);
    pcu_status st = p->build(c, *reinterpret_cast<const Graph *>(gh),
                             std::vector<uint32_t>(outputs, outputs + n_outputs));
    if (st) {
        c->error = p->error.empty() ? c->error : p->error;
        delete p;
        return st;
    }
    *out = reinterpret_cast<pcu_prepared *>(p);
    return PCU_OK;
}

void pcu_prepared_destroy(pcu_prepared *p) { delete reinterpret_cast<Prepared *>(p); }

uint32_t pcu_prepared_input_count(const pcu_prepared *ph)
{
    return ph ? (uint32_t)reinterpret_cast<const Prepared *>(ph)->inputs.size() : 0;
}

pcu_status pcu_prepared_input_id(const pcu_prepared *ph, uint32_t index, uint32_t *id)
{
    const Prepared *p = reinterpret_cast<const Prepared *>(ph);
    if (!p || !id || index >= p->inputs.size())
        return PCU_ERR_ARGUMENT;
    *id = p->inputs[index];
    return PCU_OK;
}

pcu_status pcu_prepared_execute(pcu_prepared *ph, uint32_t n_inputs, const void *const *device_inputs,
                                pcu_fault *fault)
{
    Prepared *p = reinterpret_cast<Prepared *>(ph);
    if (!p || (n_inputs && !device_inputs))
        return PCU_ERR_ARGUMENT;
    if (!p->ctx) {
        pcu::g_thread_error = "prepared_execute: its context was closed";
        return PCU_ERR_STATE;
    }
    std::vector<const void *> in(device_inputs, device_inputs + n_inputs);
    pcu_status st = p->execute(in, fault);
    if (st && st != PCU_ARITHMETIC_FAULT)
        p->ctx->error = p->error.empty() ? p->ctx->error : p->error;
    return st;
}

const void *pcu_prepared_output(const pcu_prepared *ph, uint32_t index)
{
    const Prepared *p = reinterpret_cast<const Prepared *>(ph);
    if (!p || !p->published || index >= p->published_ptr.size())
        return nullptr;
    return p->published_ptr[index];
}

pcu_status pcu_prepared_take_output(pcu_prepared *ph, uint32_t index, void **device_ptr)
{
    Prepared *p = reinterpret_cast<Prepared *>(ph);
    if (!p || !device_ptr || index >= p->outputs.size())
        return PCU_ERR_ARGUMENT;
    *device_ptr = nullptr;
    if (!p->ctx) {
        pcu::g_thread_error = "take_output: its context was closed";
        return PCU_ERR_STATE;
    }
    if (!p->published || !p->published_ptr[index]) {
        p->ctx->fail("take_output: output %u is not published", index);
        return PCU_ERR_STATE;
    }
    uint32_t id = p->outputs[index];
    const pcu::Node &nd = p->graph.nodes[id];
    if (nd.op == Op::Input || nd.op == Op::Constant || nd.op == Op::Uniform || p->fused_into[id] >= 0) {
        p->ctx->fail("take_output: output %u is not computed by the program", index);
        return PCU_ERR_UNSUPPORTED;
    }
    int published_bank = p->bank ^ 1; // execute() flips after publishing
    void *fresh = nullptr;
    size_t bytes = p->graph.elements(id) * (nd.dtype == 0 ? 4 : 8);
    // The replacement bank is written only by later executions, in stream order.
    pcu_status st = p->ctx->alloc(bytes, &fresh, true);
    if (st)
        return st;
    *device_ptr = p->buf[published_bank][id];
    p->buf[published_bank][id] = fresh;
    p->published_ptr[index] = nullptr;
    return PCU_OK;
}

} // extern "C"
