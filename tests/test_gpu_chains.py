"""GPU parity of fused elementwise chains in prepared programs. Consecutive checked Add,
Subtract, Multiply, Divide, ReLU and ReLU-backward nodes of one shape, each an operand of
the next, run as one kernel that keeps one fault word per node. Random chains (uniform
operands on either side, per-node underflow policies, intermediates that are outputs or
operands of later nodes, planted special values) are checked against the oracle's graph
evaluation: the first faulting node with its coordinates, or every output's bits."""
import numpy as np
import pytest

from oracle import graph as og

pytestmark = pytest.mark.gpu

_OPS = ["Add", "Sub", "Mul", "Div", "Relu", "ReluBackward"]


@pytest.fixture(scope="module")
def G(pcu_pkg):
    from fusion_pcu_amd import graph
    graph.configure(0)
    return graph


def _bits(a):
    a = np.asarray(a)
    return a.view(np.uint32 if a.dtype == np.float32 else np.uint64)


def _random_program(G, rng, dtype, shape):
    """(device graph, oracle graph, {input ids: array}, [(device id, oracle id)] outputs).
    Both graphs are built call for call, so their node ids agree."""
    info = np.finfo(dtype)
    specials = np.array([np.nan, np.inf, -np.inf, info.max * dtype(0.75), info.tiny * dtype(0.5),
                         info.smallest_subnormal, info.tiny * dtype(3), dtype(0), -dtype(0)], dtype=dtype)
    uniforms = [0.5, -1.25, 3.0, 2.0 ** -70, -(2.0 ** 60), 0.0]
    g, r = G.Graph(), og.Graph()
    g.set_numerical_mode(True)
    r.mode = "Strict"
    inputs, pool = {}, []
    for _ in range(3):
        a = rng.uniform(-2, 2, shape).astype(dtype)
        if rng.random() < 0.4:
            for _ in range(int(rng.integers(1, 4))):
                a.reshape(-1)[int(rng.integers(a.size))] = rng.choice(specials)
        ids = (g.input(shape, dtype), r.input(shape, dtype))
        inputs[ids] = a
        pool.append(ids)
    values, cur = [], None
    for _ in range(int(rng.integers(2, 8))):
        op = _OPS[int(rng.integers(len(_OPS)))]
        x = pool[int(rng.integers(len(pool)))] if cur is None or rng.random() < 0.1 else cur
        pick = rng.random()
        if pick < 0.25:
            v = float(rng.choice(uniforms))
            other = (g.uniform(shape, dtype, v), r.uniform(shape, dtype, v))
        elif pick < 0.85 or not values:
            other = pool[int(rng.integers(len(pool)))]
        else:
            other = values[int(rng.integers(len(values)))]  # an earlier value
        if op == "Relu":
            node = (g.relu(x[0]), r.relu(x[1]))
        else:
            a, b = (x, other) if rng.random() < 0.5 else (other, x)
            if op == "ReluBackward":
                node = (g.relu_backward(a[0], b[0]), r.relu_backward(a[1], b[1]))
            else:
                code = {"Add": 0, "Sub": 1, "Mul": 2, "Div": 3}[op]
                node = (g.binary(code, a[0], b[0]), r.binary(op, a[1], b[1]))
        policy = int(rng.integers(0, 3))
        g.set_underflow_policy(node[0], policy)
        r.nodes[node[1]].policy = policy
        values.append(node)
        cur = node
    outs = [cur] + [v for v in values[:-1] if rng.random() < 0.3]
    return g, r, inputs, outs


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_elementwise_chain_fusion_fuzz(G, pcu_pkg, dtype):
    rng = np.random.default_rng(71 if dtype == np.float32 else 72)
    ctx = pcu_pkg.Context(0)
    ctx.profile(True)
    faults = clean = 0
    for case in range(40):
        shape = (int(rng.integers(1, 90)), int(rng.integers(1, 70)))
        g, r, inputs, outs = _random_program(G, rng, dtype, shape)
        vals, rfault = r.evaluate({ids[1]: a for ids, a in inputs.items()}, [o[1] for o in outs])
        prep = g.prepare(ctx, [o[0] for o in outs])
        dev = {ids[0]: ctx.upload(a) for ids, a in inputs.items()}
        try:
            prep.execute([dev[i].ptr for i in prep.input_ids])
            gfault = None
        except pcu_pkg.PcuExecutionError as e:
            f = e.tensor_fault
            assert f is not None, str(e)
            gfault = (f.node, f.element_index, f.reduction_index, int(f.step), int(f.kind))
        want = None if rfault is None else (rfault.node, rfault.fault.element_index,
                                            rfault.fault.reduction_index, int(rfault.fault.step),
                                            int(rfault.fault.kind))
        assert gfault == want, (case, shape)
        if want is not None:
            faults += 1
            continue
        clean += 1
        for k, (gid, rid) in enumerate(outs):
            d = prep.output_desc[k]
            got = pcu_pkg.DeviceArray(ctx, prep.output_ptr(k), d["shape"], d["dtype"]).numpy()
            np.testing.assert_array_equal(_bits(got).reshape(-1), _bits(vals[rid]).reshape(-1),
                                          err_msg=str((case, shape, k)))
    _, chains = ctx.kernel_time("elementwise_chain")
    ctx.profile(False)
    ctx.close()
    assert faults >= 5 and clean >= 5, (faults, clean)
    assert chains >= 20, chains
