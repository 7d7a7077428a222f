"""Pins the oracle's ordered tensor ops (oracle/strict_ops.c, oracle/fast_ops.c).

Anchors: the reference's tensor known-answer tests (tests/golden/tensor_kat.json), exact
integer arithmetic for index/transposition/order questions (small integer-valued inputs
make every rounded step exact, so the result must equal numpy's integer product), brute
force of the first-fault order on tiny inputs, and equality between the faithful
single-thread routines and the fast OpenMP oracle on random and adversarial inputs.
"""
import json
import os
import zlib

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KIND = {"Ok": 0, "DivideByZero": 1, "ArithmeticOverflow": 3, "ArithmeticUnderflow": 4,
        "InvalidFloatingOperand": 5}
STEP = {"None": 0, "Multiply": 1, "Add": 2, "Subtract": 3, "Divide": 4}
POLICY = {"IeeeAfterRounding": 0, "RejectSubnormalResult": 1, "AllowGradualUnderflow": 2}


def _arr(spec, dtype):
    itype = np.uint32 if dtype == np.float32 else np.uint64
    bits = np.array([int(b, 16) for b in spec["bits"]], dtype=itype)
    return bits.view(dtype).reshape(spec["shape"]) if spec["shape"] else bits.view(dtype).reshape(())


def _run_case(case, fast):
    dtype = np.float32 if case["dtype"] == "f32" else np.float64
    policy = POLICY[case["policy"]]
    ins = [_arr(s, dtype) for s in case["inputs"]]
    if case["op"] == "matmul":
        return oracle.matmul(ins[0], ins[1], case["params"]["tl"], case["params"]["tr"],
                             policy=policy, fast=fast)
    if case["op"] == "sgd":
        rate = np.array([int(case["params"]["rate"], 16)], dtype=np.uint32).view(np.float32)[0]
        return oracle.sgd(ins[0].reshape(-1), ins[1].reshape(-1), rate, policy=policy, fast=fast)
    if case["op"] == "mse":
        return oracle.mse(ins[0].reshape(-1), ins[1].reshape(-1), policy=policy, fast=fast)
    raise AssertionError(case["op"])


TENSOR_CASES = json.load(open(os.path.join(GOLDEN, "tensor_kat.json")))["cases"]


@pytest.mark.parametrize("fast", [False, True], ids=["faithful", "fast"])
@pytest.mark.parametrize("case", TENSOR_CASES, ids=lambda c: f"{c['op']}-{c['dtype']}-{c['source']}")
def test_reference_tensor_known_answers(case, fast):
    out, fault = _run_case(case, fast)
    if case["fault"] is not None:
        e, r, step, kind = case["fault"]
        assert fault is not None, case
        assert (fault.element_index, fault.reduction_index, fault.step, fault.kind) == \
            (e, r, STEP[step], KIND[kind]), (fault, case)
    else:
        assert fault is None, (fault, case)
        itype = np.uint32 if case["dtype"] == "f32" else np.uint64
        got = [int(v) for v in np.asarray(out).reshape(-1).view(itype)]
        assert got == [int(v, 16) for v in case["output"]], case


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("tl,tr", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_matmul_integer_inputs_equal_exact_product(dtype, tl, tr):
    rng = np.random.default_rng(11 + tl * 2 + tr)
    m, k, n = 37, 53, 29
    a = rng.integers(-8, 9, size=(k, m) if tl else (m, k))
    b = rng.integers(-8, 9, size=(n, k) if tr else (k, n))
    exact = (a.T if tl else a) @ (b.T if tr else b)
    for fast in (False, True):
        out, fault = oracle.matmul(a.astype(dtype), b.astype(dtype), bool(tl), bool(tr),
                                   fast=fast)
        assert fault is None
        np.testing.assert_array_equal(out, exact.astype(dtype))


def test_mse_and_sgd_integer_closed_forms():
    p = np.arange(1, 65, dtype=np.float32)
    t = np.zeros_like(p)
    out, fault = oracle.mse(p, t)
    assert fault is None and out == np.float32(sum(i * i for i in range(1, 65)) / 64)
    w = np.arange(-10, 10, dtype=np.float64)
    g = np.arange(20, dtype=np.float64)
    out, fault = oracle.sgd(w, g, 0.25)
    assert fault is None
    np.testing.assert_array_equal(out, w - 0.25 * g)


def _adversarial(rng, shape, dtype, fill):
    x = rng.uniform(-1, 1, size=shape).astype(dtype)
    flat = x.reshape(-1)
    n = flat.size
    idx = rng.choice(n, size=max(1, n // 50), replace=False)
    big = np.finfo(dtype).max / 2
    tiny = np.finfo(dtype).tiny
    choices = {
        "huge": [big, -big],
        "nan": [np.nan, np.inf, -np.inf],
        "tiny": [tiny, -tiny * 0.75, tiny * 2 ** -10, 2 * tiny],
        "zero": [0.0, -0.0],
    }[fill]
    flat[idx] = rng.choice(np.array(choices, dtype=dtype), size=idx.size)
    return x


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("fill", ["huge", "nan", "tiny", "zero"])
@pytest.mark.parametrize("policy", [0, 1, 2])
def test_fast_matmul_equals_faithful(dtype, fill, policy):
    rng = np.random.default_rng(zlib.crc32(f"{np.dtype(dtype)}-{fill}-{policy}".encode()))
    for tl, tr in ((0, 0), (1, 0), (0, 1)):
        m, k, n = 19, 23, 17
        a = _adversarial(rng, (k, m) if tl else (m, k), dtype, fill)
        b = _adversarial(rng, (n, k) if tr else (k, n), dtype, fill if fill != "nan" else "zero")
        if fill == "tiny":
            a *= dtype(2.0 ** -60)  # bring products into the tiny range
        o1, f1 = oracle.matmul(a, b, bool(tl), bool(tr), policy=policy, fast=False)
        o2, f2 = oracle.matmul(a, b, bool(tl), bool(tr), policy=policy, fast=True)
        assert f1 == f2
        if f1 is None:
            np.testing.assert_array_equal(o1.view(np.uint8), o2.view(np.uint8))


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("fill", ["huge", "nan", "tiny", "zero"])
@pytest.mark.parametrize("policy", [0, 1, 2])
def test_fast_elementwise_sgd_mse_equal_faithful(dtype, fill, policy):
    rng = np.random.default_rng(zlib.crc32(f"ew-{np.dtype(dtype)}-{fill}-{policy}".encode()))
    n = 4000
    a = _adversarial(rng, (n,), dtype, fill)
    b = _adversarial(rng, (n,), dtype, "zero" if fill == "nan" else fill)
    if fill == "tiny":
        b *= dtype(2.0 ** -30)
    for op in range(4):
        for scalar in (False, True):
            bb = b[:1] if scalar else b
            r1 = oracle.binary(op, a, bb, policy=policy, fast=False)
            r2 = oracle.binary(op, a, bb, policy=policy, fast=True)
            assert r1[1] == r2[1], (op, scalar, r1[1], r2[1])
            if r1[1] is None:
                np.testing.assert_array_equal(r1[0].view(np.uint8), r2[0].view(np.uint8))
    for rate in (0.01, 2.0 ** -100, 3.0):
        r1 = oracle.sgd(a, b, rate, policy=policy, fast=False)
        r2 = oracle.sgd(a, b, rate, policy=policy, fast=True)
        assert r1[1] == r2[1]
        if r1[1] is None:
            np.testing.assert_array_equal(r1[0].view(np.uint8), r2[0].view(np.uint8))
    r1 = oracle.mse(a, b, policy=policy, fast=False)
    r2 = oracle.mse(a, b, policy=policy, fast=True)
    assert r1[1] == r2[1]
    if r1[1] is None:
        assert r1[0].tobytes() == r2[0].tobytes()
    r1 = oracle.relu(a, policy=policy, fast=False)
    r2 = oracle.relu(a, policy=policy, fast=True)
    assert r1[1] == r2[1]


def test_first_fault_order_brute_force():
    """Every position of one NaN in A / B must be reported at (cell, k, Multiply) with the
    lowest such coordinate, and an overflow pair at its Add."""
    rng = np.random.default_rng(3)
    m, k, n = 4, 5, 3
    for _ in range(40):
        a = rng.uniform(-1, 1, size=(m, k)).astype(np.float32)
        b = rng.uniform(-1, 1, size=(k, n)).astype(np.float32)
        r0, k0 = rng.integers(m), rng.integers(k)
        a[r0, k0] = np.nan
        _, f = oracle.matmul(a, b, fast=False)
        assert (f.element_index, f.reduction_index, f.step, f.kind) == (r0 * n, k0, 1, 5)
        a[r0, k0] = 0.5
        big = np.float32(3.0e38)
        a[r0, :] = 0.25
        a[r0, k0] = big
        k1 = (k0 + 1) % k
        a[r0, k1] = big
        b[:, :] = 1.0
        _, f = oracle.matmul(a, b, fast=False)
        assert (f.element_index, f.reduction_index, f.step, f.kind) == \
            (r0 * n, max(k0, k1), 2, 3)


def test_c5_fixture_first_step_matches_the_oracle():
    """tests/golden/c5_100_steps.json starts where the committed oracle does: step 0's loss
    and weight digests are recomputed here (about 15 s on 8 host cores)."""
    import hashlib
    import importlib.util
    import json
    import os
    from oracle import graph as og
    here = os.path.dirname(os.path.abspath(__file__))
    fixture = json.load(open(os.path.join(here, "golden", "c5_100_steps.json")))
    path = os.path.join(os.path.dirname(here), "fusion-pcu_amd", "synthetic.py")
    spec = importlib.util.spec_from_file_location("pcu_synthetic_c5", path)
    syn = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(syn)
    dims, batch = (1024, 4096, 4096, 1024), 4096
    s = fixture["seeds"]
    x = syn.uniform(s["x"], (batch, dims[0]), np.float32)
    y = syn.uniform(s["y"], (batch, dims[3]), np.float32)
    ws = [syn.xavier_uniform(s["w"][i], dims[i], dims[i + 1], np.float32) for i in range(3)]
    g, ids = og.mlp_graph(dims, batch, np.float32, 1e-3)
    vals, fault = g.evaluate({ids["x"]: x, ids["w1"]: ws[0], ids["w2"]: ws[1], ids["w3"]: ws[2],
                              ids["y"]: y}, ids["outputs"])
    assert fault is None
    first = fixture["steps"][0]
    loss = vals[ids["outputs"][3]]
    assert "0x%08x" % int(np.asarray(loss, np.float32).view(np.uint32)) == first["loss"]
    for i in range(3):
        w = vals[ids["outputs"][i]]
        assert hashlib.sha256(np.ascontiguousarray(w, dtype="<f4").tobytes()).hexdigest() == \
            first["w_sha256"][i]
