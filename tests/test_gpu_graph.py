"""GPU parity of the prepared-graph path (the reference facade's capture + call) against
the oracle's graph restatement: the C1 training loop with resident weights, the
reference's own end-to-end known answers, transactional faults and small MLPs."""
import numpy as np
import pytest

import oracle
from oracle import graph as og

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def G(pcu_pkg):
    from fusion_pcu_amd import graph
    graph.configure(0)
    return graph


def _bits(a):
    a = np.asarray(a)
    return a.view(np.uint32 if a.dtype == np.float32 else np.uint64)


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_c1_ten_steps_resident_weights(G, dtype):
    """C1: X 64x128, W 128x64, b 64x64, Y 64x64 uniform[-1,1] (seeds 1..4), lr 0.01, 10
    strict steps with W and b resident between calls; every step bit-exact."""
    from fusion_pcu_amd import synthetic as syn
    x = syn.uniform(1, (64, 128), dtype)
    w = syn.uniform(2, (128, 64), dtype)
    b = syn.uniform(3, (64, 64), dtype)
    y = syn.uniform(4, (64, 64), dtype)
    step = G.c1_training_step(0.01)
    w_dev, b_dev = w, b
    w_ref, b_ref = w, b
    for it in range(10):
        w_dev, b_dev, loss = step(x, w_dev, b_dev, y)   # device owners fed back
        ref = oracle.graph_c1_step(x, w_ref, b_ref, y, 0.01)
        assert ref["fault"] is None
        w_ref, b_ref = ref["weights"], ref["bias"]
        assert _bits(loss.numpy()).item() == _bits(ref["loss"]).item(), it
        np.testing.assert_array_equal(_bits(w_dev.numpy()), _bits(w_ref), err_msg=f"step {it}")
        np.testing.assert_array_equal(_bits(b_dev.numpy()), _bits(b_ref), err_msg=f"step {it}")
    assert isinstance(w_dev, G.PcuTensor)


def test_readme_known_answer(G):
    """README.md:95-180: update (SGD 0.5) -> linear (strict matmul + bias) -> activate
    (ReLU) gives [[0, 4], [3, 0]]."""

    @G.function(strict=True)
    def update(weights, gradients):
        return G.sgd_update(weights, gradients, 0.5)

    @G.function(strict=True)
    def linear(inp, weights, bias):
        return G.matmul(inp, weights) + bias

    @G.function()
    def activate(inp):
        return G.relu(inp)

    inp = np.array([[1.0, 2.0, 3.0], [-1.0, 0.0, 2.0]], np.float32)
    weights = np.array([[1.0, -2.0], [0.0, 1.0], [2.0, 1.0]], np.float32)
    grads = np.array([[2.0, -2.0], [0.0, 2.0], [2.0, 0.0]], np.float32)
    bias = np.array([[-8.0, 2.0], [1.0, -5.0]], np.float32)
    trained = update(weights, grads)
    result = activate(linear(inp, trained, bias))
    matrix = np.zeros((2, 2), np.float32)
    result.read_into(matrix)
    assert matrix.tolist() == [[0.0, 4.0], [3.0, 0.0]]


def test_checked_training_example_known_answer(G):
    """fusion-pcu/examples/checked-training/checked-training.rs:11-79: loss 0.5 and
    weights [2, -1] -> [1.5, -1.0] after one step with rate 0.5."""

    @G.function(strict=True)
    def loss_fn(inp, weights, target):
        return G.mean_squared_error(G.relu(G.matmul(inp, weights)), target)

    @G.function(strict=True)
    def training_step(inp, weights, target):
        pre = G.matmul(inp, weights)
        pred = G.relu(pre)
        loss = G.mean_squared_error(pred, target)
        grad = G.gradient(loss, weights)
        return G.sgd_update(weights, grad, 0.5)

    inp = np.array([[1.0, 0.0], [0.0, 1.0]], np.float32)
    target = np.array([[1.0], [0.0]], np.float32)
    weights = G.PcuTensor.from_numpy(np.array([[2.0], [-1.0]], np.float32))
    before = loss_fn(inp, weights, target).numpy()
    updated = training_step(inp, weights, target).numpy()
    assert _bits(before).item() == _bits(np.float32(0.5)).item()
    assert _bits(updated).reshape(-1).tolist() == _bits(np.array([1.5, -1.0], np.float32)).tolist()


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_cpu_prepared_training_and_transactional_fault(G, pcu_pkg, dtype):
    """backends/cpu/tests/prepared_tensor/prepared_tensor.rs:25-108: all-target backward,
    outputs (loss, weight gradient, updated weights); a NaN input faults and leaves the
    published outputs untouched; the next call succeeds."""
    g = G.Graph()
    g.set_numerical_mode(True)
    inp = g.input((2, 2), dtype)
    wts = g.input((2, 2), dtype)
    tgt = g.input((2, 2), dtype)
    pred = g.relu(g.matmul(inp, wts))
    loss = g.mean_squared_error(pred, tgt)
    grads = g.backward_mse(loss)
    wg = grads[wts]
    upd = g.sgd_update(wts, wg, 0.125)
    outs = [loss, wg, upd]
    ctx = G.default_context()
    prep = g.prepare(ctx, outs)
    x = np.array([1.0, -2.0, 3.0, 4.0], dtype).reshape(2, 2)
    w = np.array([0.5, -0.25, 1.0, 0.75], dtype).reshape(2, 2)
    y = np.array([0.0, 1.0, 2.0, -1.0], dtype).reshape(2, 2)
    ref_g = og.Graph()
    ref_g.mode = "Strict"
    ri, rw, rt = ref_g.input((2, 2), dtype), ref_g.input((2, 2), dtype), ref_g.input((2, 2), dtype)
    rl = ref_g.mean_squared_error(ref_g.relu(ref_g.matmul(ri, rw)), rt)
    rgrads = ref_g.backward_mse(rl)
    rupd = ref_g.sgd_update(rw, rgrads[rw], 0.125)
    vals, fault = ref_g.evaluate({ri: x, rw: w, rt: y}, [rl, rgrads[rw], rupd])
    assert fault is None
    dx, dw, dy = ctx.upload(x), ctx.upload(w), ctx.upload(y)
    by_id = {inp: dx.ptr, wts: dw.ptr, tgt: dy.ptr}
    prep.execute([by_id[i] for i in prep.input_ids])
    got = [pcu_pkg.DeviceArray(ctx, prep.output_ptr(k), d["shape"], d["dtype"]).numpy()
           for k, d in enumerate(prep.output_desc)]
    for have, want in zip(got, [vals[rl], vals[rgrads[rw]], vals[rupd]]):
        np.testing.assert_array_equal(_bits(have), _bits(want))
    published = [prep.output_ptr(k) for k in range(3)]
    bad = x.copy()
    bad[0, 0] = np.nan
    dbad = ctx.upload(bad)
    by_id[inp] = dbad.ptr
    with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
        prep.execute([by_id[i] for i in prep.input_ids])
    _, rfault = ref_g.evaluate({ri: bad, rw: w, rt: y}, [rl, rgrads[rw], rupd])
    tf = exc.value.tensor_fault
    assert (tf.element_index, tf.reduction_index, int(tf.step), int(tf.kind)) == \
        (rfault.fault.element_index, rfault.fault.reduction_index, rfault.fault.step, rfault.fault.kind)
    assert [prep.output_ptr(k) for k in range(3)] == published
    again = [pcu_pkg.DeviceArray(ctx, prep.output_ptr(k), d["shape"], d["dtype"]).numpy()
             for k, d in enumerate(prep.output_desc)]
    for have, want in zip(again, got):
        np.testing.assert_array_equal(_bits(have), _bits(want))
    by_id[inp] = dx.ptr
    prep.execute([by_id[i] for i in prep.input_ids])


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_small_mlp_steps_parity(G, dtype):
    """The C5 graph at reduced width (batch 128, 96 -> 256 -> 256 -> 64), three steps."""
    from fusion_pcu_amd import synthetic as syn
    dims, batch, lr = (96, 256, 256, 64), 128, 1e-3
    x = syn.uniform(51, (batch, dims[0]), dtype)
    y = syn.uniform(52, (batch, dims[3]), dtype)
    ws = [syn.xavier_uniform(53 + i, dims[i], dims[i + 1], dtype) for i in range(3)]
    step = G.mlp_training_step(lr)
    ref_graph, ids = og.mlp_graph(dims, batch, dtype, lr)
    dev = list(ws)
    ref = list(ws)
    for it in range(3):
        w1, w2, w3, loss = step(x, *dev, y)
        dev = [w1, w2, w3]
        vals, fault = ref_graph.evaluate({ids["x"]: x, ids["w1"]: ref[0], ids["w2"]: ref[1],
                                          ids["w3"]: ref[2], ids["y"]: y}, ids["outputs"])
        assert fault is None
        ref = [vals[o] for o in ids["outputs"][:3]]
        assert _bits(loss.numpy()).item() == _bits(vals[ids["outputs"][3]]).item()
        for have, want in zip(dev, ref):
            np.testing.assert_array_equal(_bits(have.numpy()), _bits(want), err_msg=f"step {it}")


def test_first_faulting_node_matches_oracle(G, pcu_pkg):
    """A graph whose later nodes would also fault reports the earliest node, like the
    reference's ordered per-node execution."""
    from fusion_pcu_amd import synthetic as syn
    x = syn.uniform(61, (32, 48), np.float32)
    w = syn.uniform(62, (48, 16), np.float32)
    b = syn.uniform(63, (32, 16), np.float32)
    y = syn.uniform(64, (32, 16), np.float32)
    w[7, 3] = np.float32(3.0e38)
    w[9, 3] = np.float32(3.0e38)
    x[:, 7] = 1.0
    x[:, 9] = 1.0
    step = G.c1_training_step(0.01)
    with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
        step(x, w, b, y)
    ref = oracle.graph_c1_step(x, w, b, y, 0.01)
    assert ref["fault"] is not None
    tf = exc.value.tensor_fault
    rf = ref["fault"]
    assert (tf.node, tf.element_index, tf.reduction_index, int(tf.step), int(tf.kind)) == \
        (rf.node, rf.fault.element_index, rf.fault.reduction_index, rf.fault.step, rf.fault.kind)


def test_prepared_graph_outliving_its_context(G, pcu_pkg):
    """Closing a context releases the device buffers of the prepared graphs built on it and
    detaches them: a later execution is refused (PcuExecutionError) and destroying the
    prepared graph afterwards touches nothing of the closed context."""
    import gc
    ctx = pcu_pkg.Context(0)
    g = G.Graph()
    g.set_numerical_mode(True)
    x = g.input((8, 4), np.float32)
    w = g.input((4, 8), np.float32)
    out = g.relu(g.matmul(x, w))
    prep = g.prepare(ctx, [out])
    dx = ctx.upload(np.ones((8, 4), np.float32))
    dw = ctx.upload(np.full((4, 8), 0.5, np.float32))
    prep.execute([dx.ptr, dw.ptr])
    got = prep.take_output(0).numpy()
    assert np.array_equal(got, np.full((8, 8), 2.0, np.float32))
    ptrs = [dx.ptr, dw.ptr]
    dx.free()
    dw.free()
    ctx.close()
    with pytest.raises(pcu_pkg.PcuExecutionError):
        prep.execute(ptrs)  # refused before any pointer is used
    del prep
    gc.collect()


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_c1_graph_random_shapes_and_faults_fuzz(G, pcu_pkg, dtype):
    """Seeded fuzz of the prepared C1 training graph (forward, MSE, reverse mode, SGD) over
    12 random shapes, with a special value planted in some inputs: the step's outputs, or
    its first faulting node and coordinates, match the oracle's graph restatement."""
    rng = np.random.default_rng(17 if dtype == np.float32 else 18)
    info = np.finfo(dtype)
    specials = np.array([np.nan, np.inf, info.max, info.tiny * dtype(0.5),
                         info.smallest_subnormal], dtype=dtype)
    step = G.c1_training_step(0.01)
    for case in range(12):
        m, k, n = (int(v) for v in rng.integers(1, 96, size=3))
        x, w, b, y = (rng.uniform(-1, 1, s).astype(dtype) for s in ((m, k), (k, n), (m, n), (m, n)))
        for arr in (x, w, b, y):
            if rng.random() < 0.25:
                arr.reshape(-1)[int(rng.integers(arr.size))] = rng.choice(specials)
        ref = oracle.graph_c1_step(x, w, b, y, 0.01)
        if ref["fault"] is None:
            w2, b2, loss = step(x, w, b, y)
            assert _bits(loss.numpy()).item() == _bits(ref["loss"]).item(), case
            np.testing.assert_array_equal(_bits(w2.numpy()), _bits(ref["weights"]), err_msg=str(case))
            np.testing.assert_array_equal(_bits(b2.numpy()), _bits(ref["bias"]), err_msg=str(case))
        else:
            with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
                step(x, w, b, y)
            tf, rf = exc.value.tensor_fault, ref["fault"]
            assert (tf.node, tf.element_index, tf.reduction_index, int(tf.step), int(tf.kind)) == \
                (rf.node, rf.fault.element_index, rf.fault.reduction_index, rf.fault.step,
                 rf.fault.kind), (case, m, k, n)


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_constant_node_graph_parity(G, pcu_pkg, dtype):
    """OpDescriptor::Constant (core/dialect/tensor.rs:377): relu(X @ W + C) with C a graph
    constant, MSE vs Y, gradients for W and C, SGD on W. C is uploaded once at prepare and
    is not a prepared input; three executions with W fed back are bit-exact against the
    oracle's graph. A NaN in a second graph's constant faults at the Add, at the oracle's
    element."""
    from fusion_pcu_amd import synthetic as syn
    x = syn.uniform(61, (32, 48), dtype)
    w0 = syn.uniform(62, (48, 24), dtype)
    c = syn.uniform(63, (32, 24), dtype)
    y = syn.uniform(64, (32, 24), dtype)

    def build(g, cval):
        xi, wi = g.input(x.shape, dtype), g.input(w0.shape, dtype)
        k = g.constant(cval)
        yi = g.input(y.shape, dtype)
        loss = g.mean_squared_error(g.relu(g.add(g.matmul(xi, wi), k)), yi)
        gw, gk = g.backward_mse_for_targets(loss, [wi, k])
        return xi, wi, yi, [g.sgd_update(wi, gw, 0.01), gk, loss]

    ctx = G.default_context()
    g = G.Graph()
    g.set_numerical_mode(True)
    xi, wi, yi, outs = build(g, c)
    prep = g.prepare(ctx, outs)
    assert sorted(prep.input_ids) == sorted([xi, wi, yi])
    r = og.Graph()
    r.mode = "Strict"
    rxi, rwi, ryi, routs = build(r, c)
    dx, dy = ctx.upload(x), ctx.upload(y)
    w_dev, w_ref = ctx.upload(w0), w0
    for it in range(3):
        by_id = {xi: dx.ptr, wi: w_dev.ptr, yi: dy.ptr}
        prep.execute([by_id[i] for i in prep.input_ids])
        vals, fault = r.evaluate({rxi: x, rwi: w_ref, ryi: y}, routs)
        assert fault is None
        got = [prep.take_output(k).numpy() for k in range(3)]
        for have, want in zip(got, [vals[o] for o in routs]):
            np.testing.assert_array_equal(_bits(have), _bits(want), err_msg=f"step {it}")
        w_ref = vals[routs[0]]
        w_dev = ctx.upload(got[0])

    bad = c.copy()
    bad[5, 7] = np.nan
    g2 = G.Graph()
    g2.set_numerical_mode(True)
    xi2, wi2, yi2, outs2 = build(g2, bad)
    prep2 = g2.prepare(ctx, outs2)
    r2 = og.Graph()
    r2.mode = "Strict"
    rx2, rw2, ry2, routs2 = build(r2, bad)
    _, rfault = r2.evaluate({rx2: x, rw2: w0, ry2: y}, routs2)
    by_id = {xi2: dx.ptr, wi2: ctx.upload(w0).ptr, yi2: dy.ptr}
    with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
        prep2.execute([by_id[i] for i in prep2.input_ids])
    tf = exc.value.tensor_fault
    assert rfault is not None and tf.node == rfault.node
    assert (tf.element_index, tf.reduction_index, int(tf.step), int(tf.kind)) == \
        (rfault.fault.element_index, rfault.fault.reduction_index, rfault.fault.step,
         rfault.fault.kind) == (5 * 24 + 7, 0, 0, 5)


def test_constant_through_the_facade(G):
    """pcu::constant inside a strict function: the constant is a graph node of the
    captured program (not an extra call argument), and repeated calls reuse it."""
    rng = np.random.default_rng(3)
    bias = rng.uniform(-1, 1, (16, 8)).astype(np.float32)

    @G.function(strict=True)
    def affine(inp, weights):
        return G.relu(G.matmul(inp, weights) + G.constant(bias))

    x = rng.uniform(-1, 1, (16, 32)).astype(np.float32)
    w = rng.uniform(-1, 1, (32, 8)).astype(np.float32)
    for _ in range(2):
        got = affine(x, w).numpy()
    entry = next(iter(affine.cache.values()))
    assert len(entry.prepared.input_ids) == 2
    assert any(entry.prepared.graph.describe(i)["op"] == "Constant"
               for i in range(entry.prepared.graph.node_count()))
    mm, f1 = oracle.matmul(x, w)
    s, f2 = oracle.binary(oracle.OP_ADD, mm.reshape(-1), bias.reshape(-1))
    want, f3 = oracle.relu(s)
    assert f1 is None and f2 is None and f3 is None
    np.testing.assert_array_equal(_bits(got).reshape(-1), _bits(want))


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_paired_sgd_updates_fault_order(G, pcu_pkg, dtype):
    """Two consecutive strict SGD updates of a prepared graph run as one launch, each with
    its own fault word: with a fault planted in the first update, the second, both or
    neither (odd and 16-byte-multiple sizes), the outputs, or the first faulting node and its
    coordinates, match the oracle's ordered graph."""
    big = dtype(3.0e38) if dtype == np.float32 else dtype(1.7e308)
    ctx = G.default_context()
    rng = np.random.default_rng(23)
    for n1, n2 in ((37, 1000), (4096, 8192), (5, 3)):
        g = G.Graph()
        g.set_numerical_mode(True)
        w1, g1 = g.input((n1,), dtype), g.input((n1,), dtype)
        w2, g2 = g.input((n2,), dtype), g.input((n2,), dtype)
        outs = [g.sgd_update(w1, g1, 4.0), g.sgd_update(w2, g2, 0.5)]
        prep = g.prepare(ctx, outs)
        ref = og.Graph()
        ref.mode = "Strict"
        r1, rg1 = ref.input((n1,), dtype), ref.input((n1,), dtype)
        r2, rg2 = ref.input((n2,), dtype), ref.input((n2,), dtype)
        routs = [ref.sgd_update(r1, rg1, 4.0), ref.sgd_update(r2, rg2, 0.5)]
        for plant in ("none", "first", "second", "both"):
            a1, b1 = rng.uniform(-1, 1, n1).astype(dtype), rng.uniform(-1, 1, n1).astype(dtype)
            a2, b2 = rng.uniform(-1, 1, n2).astype(dtype), rng.uniform(-1, 1, n2).astype(dtype)
            if plant in ("first", "both"):
                b1[n1 // 2] = big  # 4 x big overflows in the first update's Multiply
            if plant in ("second", "both"):
                a2[n2 - 1] = -big
                b2[n2 - 1] = big  # -big - 0.5 big overflows in the second update's Subtract
            vals, rf = ref.evaluate({r1: a1, rg1: b1, r2: a2, rg2: b2}, routs)
            assert (rf is None) == (plant == "none"), (plant, rf)
            dev = {w1: ctx.upload(a1), g1: ctx.upload(b1), w2: ctx.upload(a2), g2: ctx.upload(b2)}
            try:
                if rf is None:
                    prep.execute([dev[i].ptr for i in prep.input_ids])
                    for k, want in enumerate(routs):
                        d = prep.output_desc[k]
                        have = pcu_pkg.DeviceArray(ctx, prep.output_ptr(k), d["shape"], d["dtype"]).numpy()
                        np.testing.assert_array_equal(_bits(have), _bits(vals[want]))
                else:
                    with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
                        prep.execute([dev[i].ptr for i in prep.input_ids])
                    tf = exc.value.tensor_fault
                    assert (tf.node, tf.element_index, tf.reduction_index, int(tf.step), int(tf.kind)) == \
                        (rf.node, rf.fault.element_index, rf.fault.reduction_index, rf.fault.step,
                         rf.fault.kind), (n1, n2, plant)
            finally:
                for d in dev.values():
                    d.free()


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_mse_then_chain_fault_order(G, pcu_pkg, dtype):
    """A serial MSE followed by an elementwise chain that the MSE does not feed (each node
    with its own fault word): with a fault planted in the chain, in the MSE, in both or in
    neither, at odd and whole sizes up to the serial limit, the outputs, or the first
    faulting node and its coordinates, match the oracle's ordered graph."""
    big = dtype(3.0e38) if dtype == np.float32 else dtype(1.7e308)
    ctx = G.default_context()
    rng = np.random.default_rng(31)
    for n in (37, 1000, 4096):
        g = G.Graph()
        g.set_numerical_mode(True)
        p, y = g.input((n,), dtype), g.input((n,), dtype)
        q, r = g.input((n,), dtype), g.input((n,), dtype)
        loss = g.mean_squared_error(p, y)
        d = g.mul(g.sub(q, r), g.uniform((n,), dtype, 3.0))
        out = g.relu(d)
        outs = [loss, out]
        prep = g.prepare(ctx, outs)
        ref = og.Graph()
        ref.mode = "Strict"
        rp, ry, rq, rr = (ref.input((n,), dtype) for _ in range(4))
        rloss = ref.mean_squared_error(rp, ry)
        rout = ref.relu(ref.mul(ref.sub(rq, rr), ref.uniform((n,), dtype, 3.0)))
        for plant in ("none", "chain", "mse", "both"):
            a = [rng.uniform(-1, 1, n).astype(dtype) for _ in range(4)]
            if plant in ("chain", "both"):
                a[2][n // 3], a[3][n // 3] = big, -big  # q - r overflows in the Subtract
            if plant in ("mse", "both"):
                a[0][n - 1] = np.nan  # the MSE's Subtract is invalid at its last element
            vals, rf = ref.evaluate({rp: a[0], ry: a[1], rq: a[2], rr: a[3]}, [rloss, rout])
            assert (rf is None) == (plant == "none"), (plant, rf)
            dev = {p: ctx.upload(a[0]), y: ctx.upload(a[1]), q: ctx.upload(a[2]), r: ctx.upload(a[3])}
            try:
                if rf is None:
                    prep.execute([dev[i].ptr for i in prep.input_ids])
                    for k, want in enumerate((rloss, rout)):
                        desc = prep.output_desc[k]
                        have = pcu_pkg.DeviceArray(ctx, prep.output_ptr(k), desc["shape"], desc["dtype"]).numpy()
                        np.testing.assert_array_equal(_bits(have), _bits(vals[want]))
                else:
                    with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
                        prep.execute([dev[i].ptr for i in prep.input_ids])
                    tf = exc.value.tensor_fault
                    assert (tf.node, tf.element_index, tf.reduction_index, int(tf.step), int(tf.kind)) == \
                        (rf.node, rf.fault.element_index, rf.fault.reduction_index, rf.fault.step,
                         rf.fault.kind), (n, plant)
            finally:
                for x in dev.values():
                    x.free()


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_mse_then_final_sgd_fault_order(G, pcu_pkg, dtype):
    """An MSE (serial and ordered-walk sizes) followed by a strict SGD update, the last
    launch of the program: that update publishes the program's fault words when its grid is
    small and leaves them to the host when it is large. With a fault planted in the MSE's
    sum, in the update, in both or in neither, the outputs, or the first faulting node and
    its coordinates, match the oracle's ordered graph, so a fault written by an earlier
    launch is not lost by the launch that ends the program."""
    big = dtype(3.0e38) if dtype == np.float32 else dtype(1.7e308)
    half = dtype(1.5e19) if dtype == np.float32 else dtype(1.0e154)  # squares sum past the top
    ctx = G.default_context()
    rng = np.random.default_rng(47)
    for n, nw in ((1000, 1000), (20000, 1000), (20000, 1 << 20)):
        g = G.Graph()
        g.set_numerical_mode(True)
        p, t = g.input((n,), dtype), g.input((n,), dtype)
        w, gr = g.input((nw,), dtype), g.input((nw,), dtype)
        outs = [g.mean_squared_error(p, t), g.sgd_update(w, gr, 0.5)]
        prep = g.prepare(ctx, outs)
        ref = og.Graph()
        ref.mode = "Strict"
        rp, rt = ref.input((n,), dtype), ref.input((n,), dtype)
        rw, rg = ref.input((nw,), dtype), ref.input((nw,), dtype)
        routs = [ref.mean_squared_error(rp, rt), ref.sgd_update(rw, rg, 0.5)]
        for plant in ("none", "mse", "sgd", "both"):
            a = [rng.uniform(-1, 1, n).astype(dtype), rng.uniform(-1, 1, n).astype(dtype),
                 rng.uniform(-1, 1, nw).astype(dtype), rng.uniform(-1, 1, nw).astype(dtype)]
            if plant in ("mse", "both"):
                a[0][n // 2:n // 2 + 4] = half  # the ordered sum of squares overflows in an Add
            if plant in ("sgd", "both"):
                a[2][nw - 1], a[3][nw - 1] = -big, big  # -big - 0.5 big overflows
            vals, rf = ref.evaluate({rp: a[0], rt: a[1], rw: a[2], rg: a[3]}, routs)
            assert (rf is None) == (plant == "none"), (plant, rf)
            dev = {p: ctx.upload(a[0]), t: ctx.upload(a[1]), w: ctx.upload(a[2]), gr: ctx.upload(a[3])}
            try:
                if rf is None:
                    prep.execute([dev[i].ptr for i in prep.input_ids])
                    for k, want in enumerate(routs):
                        d = prep.output_desc[k]
                        have = pcu_pkg.DeviceArray(ctx, prep.output_ptr(k), d["shape"], d["dtype"]).numpy()
                        np.testing.assert_array_equal(_bits(have), _bits(vals[want]))
                else:
                    with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
                        prep.execute([dev[i].ptr for i in prep.input_ids])
                    tf = exc.value.tensor_fault
                    assert (tf.node, tf.element_index, tf.reduction_index, int(tf.step), int(tf.kind)) == \
                        (rf.node, rf.fault.element_index, rf.fault.reduction_index, rf.fault.step,
                         rf.fault.kind), (n, nw, plant)
            finally:
                for x in dev.values():
                    x.free()


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_matmul_relu_epilogue_fault_order(G, pcu_pkg, dtype):
    """A strict MatMul followed by a ReLU of its product, and one followed by a ReLU
    backward taking its product as upstream, each a node of its own with its own fault word:
    F32 at whole 128 x 128 tiles on the large tile kernel evaluates the elementwise node in
    that kernel's epilogue, other shapes and F64 launch it after the MatMul. With faults
    planted in a MatMul operand (invalid, overflow), in the ReLU backward's input, in both, a
    subnormal product under a RejectSubnormal ReLU, or none, the outputs, or the first
    faulting node and its coordinates, match the oracle's ordered graph."""
    big = dtype(3.0e38) if dtype == np.float32 else dtype(1.7e308)
    tiny = dtype(2.0 ** -70) if dtype == np.float32 else dtype(2.0 ** -530)
    ctx = G.default_context()
    rng = np.random.default_rng(37)
    for m, k, n in ((2048, 64, 2048), (2048, 128, 2176), (2048, 64, 2050), (256, 64, 256)):
        g = G.Graph()
        g.set_numerical_mode(True)
        a, b = g.input((m, k), dtype), g.input((k, n), dtype)
        b2, x = g.input((k, n), dtype), g.input((m, n), dtype)
        p = g.matmul(a, b)
        h = g.relu(p)
        hb = g.relu_backward(x, g.matmul(a, b2))
        g.set_underflow_policy(h, 1)
        outs = [h, hb, p]
        prep = g.prepare(ctx, outs)
        ref = og.Graph()
        ref.mode = "Strict"
        ra, rb = ref.input((m, k), dtype), ref.input((k, n), dtype)
        rb2, rx = ref.input((k, n), dtype), ref.input((m, n), dtype)
        rp = ref.matmul(ra, rb)
        rh = ref.relu(rp)
        rhb = ref.relu_backward(rx, ref.matmul(ra, rb2))
        ref.nodes[rh].policy = 1
        routs = [rh, rhb, rp]
        for plant in ("none", "matmul", "overflow", "relu_x", "both", "subnormal"):
            va = rng.uniform(-1, 1, (m, k)).astype(dtype)
            vb = rng.uniform(-1, 1, (k, n)).astype(dtype)
            vb2 = rng.uniform(-1, 1, (k, n)).astype(dtype)
            vx = rng.uniform(-1, 1, (m, n)).astype(dtype)
            if plant in ("matmul", "both"):
                va[m // 3, k // 2] = np.nan  # the first MatMul is invalid from row m / 3 on
            if plant == "overflow":
                vb2[k - 1, n - 1] = big
                va[m - 1, k - 1] = big  # the second MatMul overflows at its last cell
            if plant in ("relu_x", "both"):
                vx[m // 2, n - 3] = np.inf  # the ReLU backward is invalid there
            if plant == "subnormal":
                va[m // 4, :] = 0
                va[m // 4, 0] = tiny
                vb[0, n // 5] = tiny  # an exact subnormal product: a RejectSubnormal ReLU faults
            vals, rf = ref.evaluate({ra: va, rb: vb, rb2: vb2, rx: vx}, routs)
            assert (rf is None) == (plant == "none"), (plant, rf)
            dev = {a: ctx.upload(va), b: ctx.upload(vb), b2: ctx.upload(vb2), x: ctx.upload(vx)}
            try:
                if rf is None:
                    prep.execute([dev[i].ptr for i in prep.input_ids])
                    for j, want in enumerate(routs):
                        d = prep.output_desc[j]
                        have = pcu_pkg.DeviceArray(ctx, prep.output_ptr(j), d["shape"], d["dtype"]).numpy()
                        np.testing.assert_array_equal(_bits(have), _bits(vals[want]), err_msg=f"{m}x{k}x{n}")
                else:
                    with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
                        prep.execute([dev[i].ptr for i in prep.input_ids])
                    tf = exc.value.tensor_fault
                    assert (tf.node, tf.element_index, tf.reduction_index, int(tf.step), int(tf.kind)) == \
                        (rf.node, rf.fault.element_index, rf.fault.reduction_index, rf.fault.step,
                         rf.fault.kind), (m, k, n, plant)
            finally:
                for v in dev.values():
                    v.free()


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_relu_backward_epilogue_after_another_matmul(G, pcu_pkg, dtype):
    """The reverse-mode order: a MatMul, an independent MatMul, then the ReLU backward of the
    first product. The ReLU backward is evaluated with the first MatMul but keeps its place
    after the second, so with both later nodes faulting the second MatMul is reported; when
    the ReLU backward's input is the second MatMul's product it runs on its own. The ReLU
    backward's fault: an exact subnormal product (no MatMul fault) under its RejectSubnormal
    policy where its input is positive. Outputs or the first faulting node and its
    coordinates match the oracle's ordered graph."""
    big = dtype(3.0e38) if dtype == np.float32 else dtype(1.7e308)
    tiny = dtype(2.0 ** -70) if dtype == np.float32 else dtype(2.0 ** -530)
    ctx = G.default_context()
    rng = np.random.default_rng(41)
    m, k, n = 2048, 64, 2048
    for x_from_second in (False, True):
        g = G.Graph()
        g.set_numerical_mode(True)
        a, b = g.input((m, k), dtype), g.input((k, n), dtype)
        a2, b2 = g.input((m, k), dtype), g.input((k, n), dtype)
        x = g.input((m, n), dtype)
        p = g.matmul(a, b)
        q = g.matmul(a2, b2)
        hb = g.relu_backward(q if x_from_second else x, p)
        g.set_underflow_policy(hb, 1)
        outs = [hb, q]
        prep = g.prepare(ctx, outs)
        ref = og.Graph()
        ref.mode = "Strict"
        ra, rb = ref.input((m, k), dtype), ref.input((k, n), dtype)
        ra2, rb2 = ref.input((m, k), dtype), ref.input((k, n), dtype)
        rx = ref.input((m, n), dtype)
        rp = ref.matmul(ra, rb)
        rq = ref.matmul(ra2, rb2)
        rhb = ref.relu_backward(rq if x_from_second else rx, rp)
        ref.nodes[rhb].policy = 1
        routs = [rhb, rq]
        for plant in ("none", "first", "second", "relu", "second_and_relu", "all"):
            va, vb = rng.uniform(-1, 1, (m, k)).astype(dtype), rng.uniform(-1, 1, (k, n)).astype(dtype)
            va2, vb2 = rng.uniform(-1, 1, (m, k)).astype(dtype), rng.uniform(-1, 1, (k, n)).astype(dtype)
            vx = rng.uniform(-1, 1, (m, n)).astype(dtype)
            if plant in ("first", "all"):
                va[m - 2, 1] = np.nan  # invalid in the first MatMul
            if plant in ("second", "second_and_relu", "all"):
                va2[m // 2, k - 1], vb2[k - 1, 7] = big, big  # overflow in the second MatMul
            if plant in ("relu", "second_and_relu", "all"):
                i, j = m // 4, n // 5
                va[i, :] = 0
                va[i, 0] = tiny
                vb[0, j] = tiny  # first product: exactly tiny * tiny, subnormal
                vx[i, j] = 0.5
                va2[i, :] = 0
                va2[i, 0] = 1
                vb2[0, j] = 1  # second product: 1 at (i, j)
            vals, rf = ref.evaluate({ra: va, rb: vb, ra2: va2, rb2: vb2, rx: vx}, routs)
            assert (rf is None) == (plant == "none"), (plant, rf)
            dev = {a: ctx.upload(va), b: ctx.upload(vb), a2: ctx.upload(va2), b2: ctx.upload(vb2),
                   x: ctx.upload(vx)}
            try:
                if rf is None:
                    prep.execute([dev[i].ptr for i in prep.input_ids if i in dev])
                    for j, want in enumerate(routs):
                        d = prep.output_desc[j]
                        have = pcu_pkg.DeviceArray(ctx, prep.output_ptr(j), d["shape"], d["dtype"]).numpy()
                        np.testing.assert_array_equal(_bits(have), _bits(vals[want]))
                else:
                    with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
                        prep.execute([dev[i].ptr for i in prep.input_ids if i in dev])
                    tf = exc.value.tensor_fault
                    assert (tf.node, tf.element_index, tf.reduction_index, int(tf.step), int(tf.kind)) == \
                        (rf.node, rf.fault.element_index, rf.fault.reduction_index, rf.fault.step,
                         rf.fault.kind), (x_from_second, plant)
            finally:
                for v in dev.values():
                    v.free()


@pytest.mark.parametrize("policy", [0, 1], ids=["ieee", "reject"])
@pytest.mark.parametrize("case", ["a_rows", "a_cols", "b_cols", "b_rows", "back_a_rows"])
def test_matmul_reads_its_operand_screen_from_the_producing_epilogue(G, pcu_pkg, case, policy):
    """A strict F32 MatMul whose operand is the value of a ReLU (or ReLU backward) that an
    earlier MatMul evaluated in its epilogue takes that operand's exponent screen from the
    superslab tables the epilogue wrote: op(A) rows or columns (A untransposed or
    transposed), op(B) columns or rows. A tiny product planted in the consumer is flagged
    only by the producer's tables (the consumer no longer reads the operand for its screen),
    so its underflow fault, with its cell and k, must match the oracle; so must a clean run's
    bits and an invalid operand elsewhere. Under RejectSubnormal (every node) the tables
    also gate the consumer's partial-sum check."""
    dt = np.float32
    ctx = G.default_context()
    rng = np.random.default_rng(43)
    m, k1, n, w = 2048, 64, 2048, 128
    back = case.startswith("back")
    g = G.Graph()
    g.set_numerical_mode(True)
    x, w1 = g.input((m, k1), dt), g.input((k1, n), dt)
    xr = g.input((m, n), dt)
    prod = g.matmul(x, w1)
    h = g.relu_backward(xr, prod) if back else g.relu(prod)
    if case in ("a_rows", "back_a_rows"):
        wq = g.input((n, w), dt)
        q = g.matmul(h, wq)
    elif case == "a_cols":
        wq = g.input((m, w), dt)
        q = g.matmul(h, wq, True, False)
    elif case == "b_cols":
        wq = g.input((w, m), dt)
        q = g.matmul(wq, h)
    else:
        wq = g.input((w, n), dt)
        q = g.matmul(wq, h, False, True)
    for node in (prod, h, q):
        g.set_underflow_policy(node, policy)
    prep = g.prepare(ctx, [q, h])
    ref = og.Graph()
    ref.mode = "Strict"
    rx, rw1, rxr = ref.input((m, k1), dt), ref.input((k1, n), dt), ref.input((m, n), dt)
    rprod = ref.matmul(rx, rw1)
    rh = ref.relu_backward(rxr, rprod) if back else ref.relu(rprod)
    wshape = {"a_rows": (n, w), "back_a_rows": (n, w), "a_cols": (m, w), "b_cols": (w, m), "b_rows": (w, n)}[case]
    rwq = ref.input(wshape, dt)
    tl, tr = case == "a_cols", case == "b_rows"
    rq = ref.matmul(rh, rwq, tl, tr) if case.startswith(("a", "back")) else ref.matmul(rwq, rh, tl, tr)
    for node in (rprod, rh, rq):
        ref.nodes[node].policy = policy
    tiny = dt(2.0 ** -50)
    for plant in ("none", "tiny", "sum", "invalid"):
        vx = rng.uniform(-1, 1, (m, k1)).astype(dt)
        vw1 = rng.uniform(-1, 1, (k1, n)).astype(dt)
        vxr = rng.uniform(0.25, 1, (m, n)).astype(dt)  # the ReLU backward passes its upstream
        vw = rng.uniform(-1, 1, wshape).astype(dt)
        if plant in ("tiny", "sum"):
            # "tiny": a product with a value near 2^-100 is tiny and inexact. "sum": normal
            # products near 2^-120 of both signs, whose running sums can come out subnormal
            # (a fault under RejectSubnormal only, found by the partial-sum check the tables
            # gate; exact under IEEE).
            small = dt(1.2345 * 2.0 ** -30)
            if plant == "sum":
                small = (rng.choice([-1.0, 1.0], size=wshape[0] if case.startswith(("a", "back")) else wshape[1])
                         * rng.uniform(0.5, 1.0, wshape[0] if case.startswith(("a", "back")) else wshape[1])
                         * 2.0 ** -20).astype(dt)
            if case in ("a_rows", "back_a_rows", "b_rows"):
                i = m // 3  # value row i near 2^-100
                vx[i, :] = 0
                vx[i, 0] = tiny
                vw1[0, :] = (rng.uniform(0.5, 1, n) * tiny).astype(dt)
            else:
                j = n // 3  # value column j near 2^-100
                vw1[:, j] = 0
                vw1[0, j] = tiny
                vx[:, 0] = (rng.uniform(0.5, 1, m) * tiny).astype(dt)
            if case.startswith(("a", "back")):
                vw[:, w // 2] = small
            else:
                vw[w // 2, :] = small
        if plant == "invalid":
            vw[wshape[0] - 1, 3] = np.nan
        vals, rf = ref.evaluate({rx: vx, rw1: vw1, rxr: vxr, rwq: vw}, [rq, rh])
        if plant != "sum":
            assert (rf is None) == (plant == "none"), (plant, rf)
        if plant == "tiny" or (plant == "sum" and rf is not None):
            assert rf.node == rq and int(rf.fault.kind) == 4, rf  # the consumer's underflow
        dev = {x: ctx.upload(vx), w1: ctx.upload(vw1), xr: ctx.upload(vxr), wq: ctx.upload(vw)}
        try:
            if rf is None:
                prep.execute([dev[i].ptr for i in prep.input_ids])
                for j2, want in enumerate((rq, rh)):
                    d = prep.output_desc[j2]
                    have = pcu_pkg.DeviceArray(ctx, prep.output_ptr(j2), d["shape"], d["dtype"]).numpy()
                    np.testing.assert_array_equal(_bits(have), _bits(vals[want]))
            else:
                with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
                    prep.execute([dev[i].ptr for i in prep.input_ids])
                tf = exc.value.tensor_fault
                assert (tf.node, tf.element_index, tf.reduction_index, int(tf.step), int(tf.kind)) == \
                    (rf.node, rf.fault.element_index, rf.fault.reduction_index, rf.fault.step,
                     rf.fault.kind), (case, plant)
        finally:
            for v in dev.values():
                v.free()
