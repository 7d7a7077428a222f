"""Host-only checks of the C++ graph layer (no GPU needed): builder metadata, reverse-mode
node order and the execution plan match the oracle's restatement of the reference, and the
reference's own graph known answers hold."""
import numpy as np
import pytest

from oracle import graph as og


@pytest.fixture(scope="module")
def G(pcu_pkg):
    from fusion_pcu_amd import graph
    return graph


def _seq_product(g):
    out = []
    for i in range(g.node_count()):
        d = g.describe(i)
        ops = tuple(x for x in (d["left"], d["right"]) if x is not None)
        o = d["numerical_options"]
        out.append((d["op"], ops, d["shape"], d["numerical_mode"], d["underflow_policy"],
                    d["transpose_left"] if d["op"] == "MatMul" else None,
                    d["transpose_right"] if d["op"] == "MatMul" else None,
                    d["value_bits"] if d["op"] == "Uniform" else None,
                    (o["compound_arithmetic"], o["precision"], o["reproducibility"])))
    return out


def _seq_oracle(g):
    out = []
    for n in g.nodes:
        bits = None
        if n.op == "Uniform":
            v = np.asarray(n.params["value"])
            bits = int(v.view(np.uint32 if v.dtype == np.float32 else np.uint64))
        out.append((n.op, n.operands, n.shape, n.mode,
                    n.policy, n.params.get("tl") if n.op == "MatMul" else None,
                    n.params.get("tr") if n.op == "MatMul" else None, bits, n.options))
    return out


def _build_pair(G, build):
    p = G.Graph()
    o = og.Graph()
    build(p, o)
    return p, o


def test_c1_training_graph_matches_oracle(G):
    def build(p, o):
        ids = {}
        for g, key in ((p, "p"), (o, "o")):
            g.set_numerical_mode(True) if key == "p" else setattr(g, "mode", "Strict")
            x = g.input((64, 128), np.float32)
            w = g.input((128, 64), np.float32)
            b = g.input((64, 64), np.float32)
            y = g.input((64, 64), np.float32)
            pred = g.relu(g.add(g.matmul(x, w), b))
            loss = g.mean_squared_error(pred, y)
            gw, gb = g.backward_mse_for_targets(loss, [w, b])
            ids[key] = (g.sgd_update(w, gw, 0.01), g.sgd_update(b, gb, 0.01), loss)
        build.ids = ids
    p, o = _build_pair(G, build)
    assert _seq_product(p) == _seq_oracle(o)
    outs = list(build.ids["p"])
    assert p.plan(outs) == o.plan(list(build.ids["o"]))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_mlp_graph_matches_oracle(G, dtype):
    og_graph, ids = og.mlp_graph((16, 32, 32, 8), 4, dtype, 1e-3)
    p = G.Graph()
    p.set_numerical_mode(True)
    x = p.input((4, 16), dtype)
    w1 = p.input((16, 32), dtype)
    w2 = p.input((32, 32), dtype)
    w3 = p.input((32, 8), dtype)
    y = p.input((4, 8), dtype)
    h1 = p.relu(p.matmul(x, w1))
    h2 = p.relu(p.matmul(h1, w2))
    pred = p.matmul(h2, w3)
    loss = p.mean_squared_error(pred, y)
    g1, g2, g3 = p.backward_mse_for_targets(loss, [w1, w2, w3])
    outs = [p.sgd_update(w1, g1, 1e-3), p.sgd_update(w2, g2, 1e-3), p.sgd_update(w3, g3, 1e-3), loss]
    assert _seq_product(p) == _seq_oracle(og_graph)
    assert p.plan(outs) == og_graph.plan(ids["outputs"])


def test_all_target_backward_with_transposes_sub_mul_and_sgd_rules(G):
    """Exercise every derivative rule (Add, Sub, Mul, ReLU, transposed MatMul, SGD, MSE with
    both operands needed) on both implementations."""
    def build(g, strict):
        if strict == "p":
            g.set_numerical_mode(True)
        else:
            g.mode = "Strict"
        a = g.input((3, 2), np.float64)
        b = g.input((4, 3), np.float64)
        c = g.input((2, 4), np.float64)
        m = g.matmul(a, b, True, True)          # (2,4)
        s = g.sub(m, c)
        t = g.mul(s, c)
        u = g.add(t, g.relu(s))
        v = g.sgd_update(u, c, 0.25)
        loss = g.mean_squared_error(v, c)
        return g.backward_mse(loss)
    p = G.Graph()
    o = og.Graph()
    gp = build(p, "p")
    go = build(o, "o")
    assert gp == go
    assert _seq_product(p) == _seq_oracle(o)


def test_reference_gradient_order_known_answer(G):
    """gradients/tests.rs:254-290: a requested prediction derivative appends exactly
    Uniform(2/n), Sub, Mul and no root seed."""
    for dtype in (np.float32, np.float64):
        g = G.Graph()
        g.set_numerical_mode(True)
        p = g.input((2,), dtype)
        t = g.input((2,), dtype)
        loss = g.mean_squared_error(p, t)
        before = g.node_count()
        d = g.backward_mse_for(loss, p)
        ops = [g.describe(i)["op"] for i in range(before, g.node_count())]
        assert ops == ["Uniform", "Sub", "Mul"]
        scale = g.describe(before)
        assert scale["shape"] == (2,)
        one = np.array(1.0, dtype=dtype).view(np.uint32 if dtype == np.float32 else np.uint64)
        assert scale["value_bits"] == int(one)
        assert d == g.node_count() - 1


def test_graph_errors(G, pcu_pkg):
    g = G.Graph()
    a = g.input((2, 3), np.float32)
    b = g.input((2, 3), np.float32)
    with pytest.raises(pcu_pkg.PcuExecutionError):
        g.matmul(a, b)                      # MatMulShape
    c = g.input((3,), np.float32)
    with pytest.raises(pcu_pkg.PcuExecutionError):
        g.add(a, c)                         # ShapeMismatch
    with pytest.raises(pcu_pkg.PcuExecutionError):
        g.backward_mse(g.add(a, b))         # GradientRootNotMse
    with pytest.raises(pcu_pkg.PcuExecutionError):
        g.sgd_update(a, b, float("nan"))    # InvalidLearningRate
    d = g.div(a, b)
    loss = g.mean_squared_error(d, b)
    with pytest.raises(pcu_pkg.PcuExecutionError):
        g.backward_mse(loss)                # UnsupportedGradient (Div)


def test_plan_retains_unused_checked_nodes(G):
    """Checked nodes run even when no output needs them (tensor.rs:3264-3278)."""
    g = G.Graph()
    g.set_numerical_mode(True)
    x = g.input((1, 1), np.float32)
    discarded = g.matmul(x, x)
    assert discarded in g.plan([x])


def test_numerical_options_capture_and_derivative_inheritance(G):
    """PcuNumericalOptions are captured by every node when it is appended
    (core/dialect/tensor.rs:3612-3618), Graph::set_value_numerical_options changes one node
    (:3129-3136), and reverse mode appends derivative nodes under the source node's mode and
    options (gradients.rs:448-474)."""
    def build(p, o):
        for g, key in ((p, "p"), (o, "o")):
            x = g.input((8, 4), np.float32)
            w = g.input((4, 3), np.float32)
            y = g.input((8, 3), np.float32)
            if key == "p":
                g.set_numerical_options(native_compound=True)
            else:
                g.options = ("BackendDefined", "Preserve", "Unspecified")
            pred = g.relu(g.matmul(x, w))
            loss = g.mean_squared_error(pred, y)
            if key == "p":
                g.set_numerical_options(backend_precision=True, deterministic=True)
            else:
                g.options = ("Checked", "BackendOptimized", "PortableV1")
            (gw,) = g.backward_mse_for_targets(loss, [w])
            g.sgd_update(w, gw, 0.5)
    p, o = _build_pair(G, build)
    assert _seq_product(p) == _seq_oracle(o)
    d = [p.describe(i) for i in range(p.node_count())]
    assert d[0]["numerical_options"]["compound_arithmetic"] == "Checked"       # before the change
    assert d[3]["numerical_mode"] == "Boundary" and d[3]["numerical_options"]["compound_arithmetic"] == "BackendDefined"
    assert d[-1]["numerical_options"] == {"compound_arithmetic": "Checked", "precision": "BackendOptimized",
                                          "reproducibility": "PortableV1"}
    p.set_value_numerical_options(3, native_compound=False, backend_precision=True)
    assert p.describe(3)["numerical_options"]["precision"] == "BackendOptimized"
    assert p.describe(3)["numerical_options"]["compound_arithmetic"] == "Checked"


def test_set_value_numerical_mode_rejects_scalar_nodes(G, pcu_pkg):
    """Graph::set_value_numerical_mode returns UnsupportedNumericalMode for a node that
    carries no numerical mode (core/dialect/tensor.rs:3154-3166)."""
    g = G.Graph()
    x = g.input((4,), np.float32)
    r = g.relu(x)
    with pytest.raises(pcu_pkg.PcuExecutionError):
        g.set_value_numerical_mode(r, True)
    y = g.input((4,), np.float32)
    m = g.mean_squared_error(r, y)
    g.set_value_numerical_mode(m, True)
    assert g.describe(m)["numerical_mode"] == "Strict"


def _constant_pair(G, dtype, targets_include_constant):
    """relu(X @ W + C) with C a Constant (OpDescriptor::Constant) -> MSE vs Y -> gradients
    -> SGD on W, built on the C++ graph and on the oracle's restatement."""
    rng = np.random.default_rng(7)
    c = rng.uniform(-1, 1, (8, 4)).astype(dtype)
    ids = {}
    p, o = G.Graph(), og.Graph()
    for g, key in ((p, "p"), (o, "o")):
        g.set_numerical_mode(True) if key == "p" else setattr(g, "mode", "Strict")
        x = g.input((8, 16), dtype)
        w = g.input((16, 4), dtype)
        k = g.constant(c)
        y = g.input((8, 4), dtype)
        loss = g.mean_squared_error(g.relu(g.add(g.matmul(x, w), k)), y)
        targets = [w, k] if targets_include_constant else [w]
        grads = g.backward_mse_for_targets(loss, targets)
        ids[key] = {"x": x, "w": w, "k": k, "y": y, "loss": loss, "grads": grads,
                    "upd": g.sgd_update(w, grads[0], 0.01)}
    return p, o, ids, c


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("with_constant_target", [False, True])
def test_constant_node_graph_matches_oracle(G, dtype, with_constant_target):
    p, o, ids, _ = _constant_pair(G, dtype, with_constant_target)
    assert _seq_product(p) == _seq_oracle(o)
    k = ids["p"]["k"]
    d = p.describe(k)
    assert d["op"] == "Constant" and d["shape"] == (8, 4) and d["dtype"] == np.dtype(dtype)
    assert d["numerical_mode"] is None and d["underflow_policy"] is None
    assert d["left"] is None and d["right"] is None
    outs = [ids["p"]["upd"], ids["p"]["loss"]]
    assert p.plan(outs) == o.plan([ids["o"]["upd"], ids["o"]["loss"]])
    assert k in p.plan(outs)
    # A constant is a leaf: the reverse pass appends nothing that reads a derivative of it.
    for i in range(p.node_count()):
        dd = p.describe(i)
        assert not (dd["op"] not in ("Add", "MatMul", "Relu", "MeanSquaredError") and k in
                    (dd["left"], dd["right"]) and i > ids["p"]["loss"])
    if with_constant_target:
        # The constant's gradient is the cotangent its Add consumer passes on, as for an Input.
        assert ids["p"]["grads"][1] is not None


def test_constant_builder_errors(G, pcu_pkg):
    import ctypes
    from fusion_pcu_amd import _abi
    lib = pcu_pkg.lib()
    g = G.Graph()
    shape = (ctypes.c_uint64 * 2)(2, 3)
    out = ctypes.c_uint32()
    # Non-empty constant without data.
    assert lib.pcu_graph_constant(g.handle, _abi.PCU_F32, 2, shape, None, ctypes.byref(out)) == \
        _abi.PCU_ERR_ARGUMENT
    # Unsupported scalar type code.
    data = np.zeros(6, np.float32)
    assert lib.pcu_graph_constant(g.handle, 7, 2, shape, data.ctypes.data_as(ctypes.c_void_p),
                                  ctypes.byref(out)) == _abi.PCU_ERR_UNSUPPORTED
    # A shape whose element count overflows.
    big = (ctypes.c_uint64 * 2)(1 << 40, 1 << 40)
    assert lib.pcu_graph_constant(g.handle, _abi.PCU_F32, 2, big, data.ctypes.data_as(ctypes.c_void_p),
                                  ctypes.byref(out)) == _abi.PCU_ERR_SHAPE
    # An empty constant needs no data; a scalar (rank 0) holds one element.
    zero = (ctypes.c_uint64 * 1)(0)
    assert lib.pcu_graph_constant(g.handle, _abi.PCU_F64, 1, zero, None, ctypes.byref(out)) == _abi.PCU_OK
    k = g.constant(np.float32(2.5))
    assert g.describe(k)["shape"] == () and g.describe(k)["op"] == "Constant"
    # Shape rules of its consumers apply as for any other value.
    a = g.input((2, 3), np.float32)
    with pytest.raises(pcu_pkg.PcuExecutionError):
        g.add(a, k)


def test_constant_data_is_copied_at_append(G):
    """The graph owns its copy: changing the caller's array afterwards changes nothing
    (checked through the oracle's restatement, which also copies)."""
    arr = np.arange(6, dtype=np.float32).reshape(2, 3)
    o = og.Graph()
    k = o.constant(arr)
    arr[:] = -1
    assert o.nodes[k].params["value"].tolist() == [[0, 1, 2], [3, 4, 5]]
