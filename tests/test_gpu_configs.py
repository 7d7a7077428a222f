"""BASELINE configurations at full size on the GPU, bit-exact against the fast oracle
(whose equality with the faithful integer law is itself tested on the CPU)."""
import sys

import numpy as np
import pytest

import oracle
from oracle import graph as og

pytestmark = [pytest.mark.gpu, pytest.mark.slow]


def say(msg):
    print(f"[configs] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def ctx(pcu_pkg):
    c = pcu_pkg.Context(0)
    yield c
    c.close()


def _bits(a):
    a = np.asarray(a)
    return a.view(np.uint32 if a.dtype == np.float32 else np.uint64)


def _gpu_fault(pcu_pkg, fn):
    try:
        return fn(), None
    except pcu_pkg.PcuExecutionError as e:
        f = e.tensor_fault
        return None, (f.element_index, f.reduction_index, int(f.step), int(f.kind))


def _of(f):
    return None if f is None else (f.element_index, f.reduction_index, f.step, f.kind)


def test_c2_f32_1024_cubed_and_fault_variants(ctx, pcu_pkg):
    """C2: strict F32 1024^3; variant A sets 0.1% of A to 3.0e38 (Add overflow where two
    same-signed huge products meet in a row); variant B sets 0.1% of B to NaN (Multiply
    invalid; the first faulting index must match the CPU backend)."""
    from fusion_pcu_amd import synthetic as syn
    n = 1024
    a = syn.uniform(21, (n, n), np.float32)
    b = syn.uniform(22, (n, n), np.float32)
    cnt = int(np.ceil(0.001 * n * n))  # 1,049
    da, db = ctx.upload(a), ctx.upload(b)
    got = ctx.strict_matmul(da, db).numpy()
    ref, rf = oracle.matmul(a, b)
    assert rf is None
    np.testing.assert_array_equal(_bits(got), _bits(ref))
    say("C2 clean ok")
    aa = a.copy()
    aa.reshape(-1)[syn.sample_indices(23, n * n, cnt)] = np.float32(3.0e38)
    _, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_matmul(ctx.upload(aa), db).numpy())
    _, rf = oracle.matmul(aa, b)
    assert rf is not None and gf == _of(rf), (gf, rf)
    say(f"C2 variant A fault {gf}")
    bb = b.copy()
    bb.reshape(-1)[syn.sample_indices(24, n * n, cnt)] = np.float32(np.nan)
    _, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_matmul(da, ctx.upload(bb)).numpy())
    _, rf = oracle.matmul(a, bb)
    assert rf is not None and gf == _of(rf), (gf, rf)
    # The first fault is cell (0, c*) with c* the lowest column holding a NaN, at its first
    # NaN row, Multiply/Invalid.
    cols = np.where(np.isnan(bb).any(axis=0))[0]
    cstar = cols.min()
    kstar = np.where(np.isnan(bb[:, cstar]))[0].min()
    assert gf == (int(cstar), int(kstar), 1, 5)
    say(f"C2 variant B fault {gf}")


def test_c3_f64_4096_matmul_bias_relu(ctx, pcu_pkg):
    """C3: strict F64 4096^3 (A, B normal(0,1)), then checked bias add (normal(0,1)) and
    ReLU, bit-exact; run through the prepared graph (the Add->ReLU pair fuses)."""
    from fusion_pcu_amd import graph as G
    from fusion_pcu_amd import synthetic as syn
    n = 4096
    say("C3 generating inputs")
    a = syn.normal(31, (n, n), 1.0, np.float64)
    b = syn.normal(32, (n, n), 1.0, np.float64)
    bias = syn.normal(33, (n, n), 1.0, np.float64)
    g = G.Graph()
    g.set_numerical_mode(True)
    ia, ib, ic = g.input((n, n), np.float64), g.input((n, n), np.float64), g.input((n, n), np.float64)
    out = g.relu(g.add(g.matmul(ia, ib), ic))
    prep = g.prepare(ctx, [out])
    dev = {ia: ctx.upload(a), ib: ctx.upload(b), ic: ctx.upload(bias)}
    prep.execute([dev[i].ptr for i in prep.input_ids])
    got = pcu_pkg.DeviceArray(ctx, prep.output_ptr(0), (n, n), np.float64).numpy()
    say("C3 GPU done; oracle")
    mm, f1 = oracle.matmul(a, b)
    assert f1 is None
    s, f2 = oracle.binary(oracle.OP_ADD, mm, bias)
    assert f2 is None
    ref, f3 = oracle.relu(s)
    assert f3 is None
    np.testing.assert_array_equal(_bits(got), _bits(ref))
    say("C3 bit-exact")


def test_c4_sgd_add_relu_2p28(ctx, pcu_pkg):
    """C4: strict F32 SGD over 2^28 elements (w normal(0,1), g normal(0,1e-3), lr 0.01,
    a 1% slice of w near 1e-38, i.e. subnormal), then checked add and ReLU over the same
    size; plus the variant whose slice also has |g| ~ 1e-37, which must fault with a
    Multiply underflow at the slice's first index."""
    from fusion_pcu_amd import synthetic as syn
    n = 1 << 28
    say("C4 generating inputs")
    w = syn.normal(41, (n,), 1.0, np.float32)
    g = syn.normal(42, (n,), 1e-3, np.float32)
    lo = n // 2
    sl = slice(lo, lo + n // 100)
    w[sl] = np.float32(1e-38)
    dw, dg = ctx.upload(w), ctx.upload(g)
    got = ctx.strict_sgd(dw, dg, 0.01).numpy()
    ref, rf = oracle.sgd(w, g, 0.01)
    assert rf is None
    assert np.array_equal(_bits(got), _bits(ref))
    del got
    say("C4 SGD bit-exact")
    dr = ctx.upload(ref)
    got = ctx.checked_add_relu(dr, dg).numpy()
    s, f1 = oracle.binary(oracle.OP_ADD, ref, g)
    r2, f2 = oracle.relu(s)
    assert f1 is None and f2 is None
    assert np.array_equal(_bits(got), _bits(r2))
    del got, s, r2
    say("C4 add+relu bit-exact")
    g2 = g.copy()
    g2[sl] = np.float32(1.3e-37)
    _, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_sgd(dw, ctx.upload(g2), 0.01).numpy())
    _, rf = oracle.sgd(w, g2, 0.01)
    assert gf == _of(rf) == (lo, 0, 1, 4), (gf, rf)
    say(f"C4 underflow variant fault {gf}")


def test_c5_mlp_full_size_hundred_steps(pcu_pkg):
    """C5: strict F32 MLP 1024 -> 4096 -> 4096 -> 1024, batch 4096, lr 1e-3, Xavier
    weights; all 100 training steps with resident weights. Every step's loss bits and a
    SHA-256 of every updated weight tensor match the oracle's run, committed as
    tests/golden/c5_100_steps.json by tests/golden/make_c5_fixture.py (the oracle needs
    about 1.2 TFLOP of ordered CPU arithmetic per step, too slow to repeat here)."""
    import hashlib
    import json
    import os
    from fusion_pcu_amd import graph as G
    from fusion_pcu_amd import synthetic as syn
    fixture = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "c5_100_steps.json")))
    seeds = fixture["seeds"]
    G.configure(0)
    dims, batch, lr = (1024, 4096, 4096, 1024), 4096, 1e-3
    say("C5 generating inputs")
    x = syn.uniform(seeds["x"], (batch, dims[0]), np.float32)
    y = syn.uniform(seeds["y"], (batch, dims[3]), np.float32)
    ws = [syn.xavier_uniform(seeds["w"][i], dims[i], dims[i + 1], np.float32) for i in range(3)]
    step = G.mlp_training_step(lr)
    dev = list(ws)
    host = [np.empty(w.shape, np.float32) for w in ws]
    for it, want in enumerate(fixture["steps"]):
        w1, w2, w3, loss = step(x, *dev, y)
        dev = [w1, w2, w3]
        got_loss = "0x%08x" % int(_bits(loss.numpy()))
        assert got_loss == want["loss"], f"step {it}: loss {got_loss} != {want['loss']}"
        for i, (w, h) in enumerate(zip(dev, host)):
            w.read_into(h)
            d = hashlib.sha256(np.ascontiguousarray(h, dtype="<f4").tobytes()).hexdigest()
            assert d == want["w_sha256"][i], f"step {it}: W{i + 1} differs from the oracle"
        if it % 10 == 9:
            say(f"C5 step {it} bit-exact, loss {float(loss.numpy())}")
    assert len(fixture["steps"]) == 100
