"""GPU parity of every op-level entry point against the CPU oracle (bit-exact values and
first-fault coordinates), through the C ABI. Sizes are chosen so the oracle finishes in
seconds; the full BASELINE sizes live in test_gpu_configs.py."""
import json
import os

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
POLICY = {"IeeeAfterRounding": 0, "RejectSubnormalResult": 1, "AllowGradualUnderflow": 2}
OP_NAMES = ["add", "sub", "mul", "div"]


@pytest.fixture(scope="module")
def ctx(pcu_pkg):
    c = pcu_pkg.Context(0)
    yield c
    c.close()


def _gpu_fault(pcu_pkg, fn):
    """Run fn; return (result, oracle-style fault tuple or None)."""
    try:
        return fn(), None
    except pcu_pkg.PcuExecutionError as e:
        assert e.tensor_fault is not None, e
        f = e.tensor_fault
        return None, (f.element_index, f.reduction_index, int(f.step), int(f.kind))


def _ofault(f):
    return None if f is None else (f.element_index, f.reduction_index, f.step, f.kind)


def _bits(a):
    a = np.asarray(a)
    return a.view(np.uint32 if a.dtype == np.float32 else np.uint64)


def _patterns(rng, n, dtype, low):
    if dtype == np.float32:
        b = rng.integers(0, 2 ** 32, size=n, dtype=np.uint64).astype(np.uint32)
        if low:
            e = rng.integers(0, 90, size=n).astype(np.uint32)
            b = (b & np.uint32(0x807FFFFF)) | (e << np.uint32(23))
        return b.view(np.float32)
    b = rng.integers(0, 2 ** 63, size=n, dtype=np.uint64) * np.uint64(2)
    if low:
        e = rng.integers(0, 560, size=n).astype(np.uint64)
        b = (b & np.uint64(0x800FFFFFFFFFFFFF)) | (e << np.uint64(52))
    return b.view(np.float64)


# ---------------------------------------------------------------- scalar law


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_scalar_law_single_element_parity(ctx, pcu_pkg, dtype):
    """Each op on one element at a time: value and fault kind equal the integer law,
    including tiny-after-rounding underflow near the subnormal range."""
    rng = np.random.default_rng(1234 + (dtype == np.float64))
    a = np.concatenate([_patterns(rng, 150, dtype, False), _patterns(rng, 250, dtype, True)])
    b = np.concatenate([_patterns(rng, 150, dtype, False), _patterns(rng, 250, dtype, True)])
    a[:4] = [np.inf, -0.0, np.nan, np.finfo(dtype).tiny]
    b[:4] = [1.0, 0.0, 0.0, 0.5]
    da, db = ctx.upload(a), ctx.upload(b)
    out = ctx.empty((1,), dtype)
    mism = []
    es = np.dtype(dtype).itemsize
    for i in range(len(a)):
        va = pcu_pkg.DeviceArray(ctx, da.ptr + i * es, (1,), dtype)
        vb = pcu_pkg.DeviceArray(ctx, db.ptr + i * es, (1,), dtype)
        for op in range(4):
            for policy in (0, 1, 2):
                got, gf = _gpu_fault(pcu_pkg, lambda: ctx.checked_binary(op, va, vb, policy, out=out).numpy())
                ref, rf = oracle.binary(op, a[i:i + 1], b[i:i + 1], policy=policy, fast=False)
                if _ofault(rf) != gf or (rf is None and _bits(got)[0] != _bits(ref)[0]):
                    mism.append((OP_NAMES[op], policy, hex(int(_bits(a)[i])), hex(int(_bits(b)[i])), gf, _ofault(rf)))
    assert not mism, mism[:10]


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("n", [1, 3, 4097, 1 << 20])
def test_binary_arrays_parity(ctx, pcu_pkg, dtype, n):
    rng = np.random.default_rng(n)
    a = rng.uniform(-4, 4, n).astype(dtype)
    b = rng.uniform(-4, 4, n).astype(dtype)
    b[b == 0] = 1
    da, db = ctx.upload(a), ctx.upload(b)
    for op in range(4):
        for uniform in (False, True):
            rhs = b[0] if uniform else db
            got = ctx.checked_binary(op, da, rhs).numpy()
            ref, rf = oracle.binary(op, a, b[:1] if uniform else b)
            assert rf is None
            np.testing.assert_array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_binary_first_fault_parity(ctx, pcu_pkg, dtype):
    rng = np.random.default_rng(99)
    n = 100_003
    for trial in range(6):
        a = rng.uniform(-1, 1, n).astype(dtype)
        b = rng.uniform(-1, 1, n).astype(dtype)
        k = rng.integers(1, 6)
        idx = rng.choice(n, size=k, replace=False)
        kinds = [np.nan, np.inf, np.finfo(dtype).max, np.finfo(dtype).tiny * 0.5,
                 np.finfo(dtype).tiny]
        a[idx] = rng.choice(np.array(kinds, dtype=dtype), size=k)
        b[idx] = rng.choice(np.array([2.0, 0.0, -np.finfo(dtype).max, 0.25], dtype=dtype), size=k)
        da, db = ctx.upload(a), ctx.upload(b)
        for op in range(4):
            for policy in (0, 1, 2):
                _, gf = _gpu_fault(pcu_pkg, lambda: ctx.checked_binary(op, da, db, policy))
                _, rf = oracle.binary(op, a, b, policy=policy)
                assert gf == _ofault(rf), (trial, OP_NAMES[op], policy, gf, rf)


# --------------------------------------------------------------------- relu


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_relu_family_parity(ctx, pcu_pkg, dtype):
    rng = np.random.default_rng(5)
    n = 65_537
    x = np.concatenate([_patterns(rng, n // 2, dtype, True), rng.uniform(-2, 2, n - n // 2).astype(dtype)])
    x = x[np.isfinite(x)]
    up = rng.uniform(-2, 2, x.size).astype(dtype)
    dx, dup = ctx.upload(x), ctx.upload(up)
    for policy in (0, 1, 2):
        got, gf = _gpu_fault(pcu_pkg, lambda: ctx.checked_relu(dx, policy).numpy())
        ref, rf = oracle.relu(x, policy=policy)
        assert gf == _ofault(rf)
        if rf is None:
            np.testing.assert_array_equal(_bits(got), _bits(ref))
        got, gf = _gpu_fault(pcu_pkg, lambda: ctx.checked_relu_backward(dx, dup, policy).numpy())
        ref, rf = oracle.relu_backward(x, up, policy=policy)
        assert gf == _ofault(rf)
        if rf is None:
            np.testing.assert_array_equal(_bits(got), _bits(ref))
    x2 = x.copy()
    x2[777] = np.nan
    _, gf = _gpu_fault(pcu_pkg, lambda: ctx.checked_relu(ctx.upload(x2)))
    assert gf == (777, 0, 0, 5)
    up2 = up.copy()
    up2[333] = -np.inf
    _, gf = _gpu_fault(pcu_pkg, lambda: ctx.checked_relu_backward(dx, ctx.upload(up2)))
    assert gf == (333, 0, 0, 5)


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_fused_add_relu_reports_add_then_relu(ctx, pcu_pkg, dtype):
    rng = np.random.default_rng(8)
    n = 10_000
    a = rng.uniform(-1, 1, n).astype(dtype)
    b = rng.uniform(-1, 1, n).astype(dtype)
    da, db = ctx.upload(a), ctx.upload(b)
    got = ctx.checked_add_relu(da, db).numpy()
    s, _ = oracle.binary(oracle.OP_ADD, a, b)
    ref, _ = oracle.relu(s)
    np.testing.assert_array_equal(_bits(got), _bits(ref))
    # An Add overflow at 900 is node 0 even though a later element would fault too.
    a[900] = np.finfo(dtype).max
    b[900] = np.finfo(dtype).max
    a[5000] = np.nan
    da, db = ctx.upload(a), ctx.upload(b)
    with ctx.program():
        pass
    try:
        with ctx.program():
            ctx.checked_add_relu(da, db)
        raise AssertionError("expected a fault")
    except pcu_pkg.PcuExecutionError as e:
        f = e.tensor_fault
        assert (f.node, f.element_index, int(f.kind)) == (0, 900, 3)


# ---------------------------------------------------------------------- SGD


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("n", [1, 5, 1 << 16, (1 << 20) + 3])
def test_sgd_parity(ctx, pcu_pkg, dtype, n):
    rng = np.random.default_rng(n + 17)
    w = rng.normal(0, 1, n).astype(dtype)
    g = rng.normal(0, 1e-3, n).astype(dtype)
    dw, dg = ctx.upload(w), ctx.upload(g)
    for rate in (0.01, 0.1, 1.0e-3):
        got = ctx.strict_sgd(dw, dg, rate).numpy()
        ref, rf = oracle.sgd(w, g, rate)
        assert rf is None
        np.testing.assert_array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_sgd_faults_parity(ctx, pcu_pkg, dtype):
    rng = np.random.default_rng(31)
    n = 50_000
    for trial in range(8):
        w = rng.normal(0, 1, n).astype(dtype)
        g = rng.normal(0, 1e-3, n).astype(dtype)
        sl = slice(1000 + trial * 3000, 1000 + trial * 3000 + 500)
        w[sl] = np.finfo(dtype).tiny * 0.9  # near-subnormal weights (the C4 slice)
        if trial % 2:
            g[sl] = np.finfo(dtype).tiny * 7  # 0.01 * g is tiny and inexact
        if trial == 2:
            g[40_000] = np.inf
        if trial == 4:
            w[20] = np.nan
        if trial == 6:
            w[7] = np.finfo(dtype).max
            g[7] = -np.finfo(dtype).max
        dw, dg = ctx.upload(w), ctx.upload(g)
        for policy in (0, 1, 2):
            rate = 1.0 if trial == 6 else 0.01
            got, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_sgd(dw, dg, rate, policy).numpy())
            ref, rf = oracle.sgd(w, g, rate, policy=policy)
            assert gf == _ofault(rf), (trial, policy, gf, rf)
            if rf is None:
                np.testing.assert_array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("n", [1000, 65_536, 65_537, 300_000])
def test_sgd_call_end_on_small_and_large_grids(ctx, pcu_pkg, dtype, n):
    """A single strict SGD call ends its one-node program in its own kernel when its grid
    has at most 64 workgroups (the last workgroup to take a ticket publishes the fault
    word), and with a publication launch otherwise; the sizes reach both (1000 elements:
    one workgroup; 65 536: 64 workgroups for binary32, the most that end in-kernel, and 128
    for binary64; 65 537: 65 and 129; 300 000: several hundred). Clean, one fault in the
    middle, and faults in the first and the last workgroups, called back to back, each
    against the oracle."""
    rng = np.random.default_rng(n + 5)
    big = np.finfo(dtype).max
    for plant in ("none", "middle", "ends", "none"):
        w = rng.normal(0, 1, n).astype(dtype)
        g = rng.normal(0, 1e-3, n).astype(dtype)
        if plant == "middle":
            w[n // 2] = np.nan
        if plant == "ends":
            w[n - 1], g[n - 1] = -big, big  # w - g overflows in the last workgroup
            g[3] = np.inf                    # and an earlier Invalid in the first
        dw, dg = ctx.upload(w), ctx.upload(g)
        got, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_sgd(dw, dg, 1.0).numpy())
        ref, rf = oracle.sgd(w, g, 1.0)
        assert gf == _ofault(rf), (n, plant, gf, rf)
        assert (rf is None) == (plant == "none"), (n, plant, rf)
        if rf is None:
            np.testing.assert_array_equal(_bits(got), _bits(ref))
        dw.free()
        dg.free()


# ---------------------------------------------------------------------- MSE


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("n", [1, 2, 17, 4096, 100_000, 1 << 20])
def test_mse_parity(ctx, pcu_pkg, dtype, n):
    rng = np.random.default_rng(n)
    p = rng.uniform(-1, 1, n).astype(dtype)
    t = rng.uniform(-1, 1, n).astype(dtype)
    got = ctx.strict_mse(ctx.upload(p), ctx.upload(t)).numpy()
    ref, rf = oracle.mse(p, t)
    assert rf is None
    assert _bits(got).item() == _bits(ref).item()


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("n", [1000, 30_000], ids=["one-workgroup", "pipeline"])
def test_mse_faults_parity(ctx, pcu_pkg, dtype, n):
    """Invalid, Multiply overflow, Add overflow, tiny squares and a lone tiny square under
    every policy, at a size the one-workgroup kernel takes (at most 4096 elements) and at one
    the parallel pipeline takes."""
    rng = np.random.default_rng(77)
    big = np.finfo(dtype).max
    cases = []
    p = rng.uniform(-1, 1, n).astype(dtype); t = rng.uniform(-1, 1, n).astype(dtype)
    p[123] = np.nan; cases.append((p.copy(), t.copy()))
    p[123] = 0.5; p[50] = big; p[51] = big; cases.append((p.copy(), t.copy()))      # Multiply overflow
    p[50] = 0.5; p[51] = 0.5
    p[10:20] = np.sqrt(big) * 0.9; cases.append((p.copy(), t.copy()))             # Add overflow
    p[10:20] = 0.5
    p[:] = np.finfo(dtype).tiny * 3; t[:] = 0; cases.append((p.copy(), t.copy()))  # tiny squares
    p[:] = 0; t[:] = 0; p[0] = np.finfo(dtype).tiny * 2 ** 20; cases.append((p.copy(), t.copy()))
    for i, (pp, tt) in enumerate(cases):
        for policy in (0, 1, 2):
            got, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_mse(ctx.upload(pp), ctx.upload(tt), policy).numpy())
            ref, rf = oracle.mse(pp, tt, policy=policy)
            assert gf == _ofault(rf), (i, policy, gf, rf)
            if rf is None:
                assert _bits(got).item() == _bits(ref).item()


def _tie_heavy(rng, n, dtype, lo, hi):
    """Differences d = m * 2^k with small odd m, so the squares are 9-, 25-, 49-multiples
    of even powers of two: many steps of the ordered sum land exactly on rounding ties or
    next to them, and the total crosses many binades."""
    m = rng.choice(np.array([1, 3, 5, 7], dtype=np.float64), n)
    k = rng.integers(lo, hi, n).astype(np.float64)
    return (m * np.exp2(k) * rng.choice([-1.0, 1.0], n)).astype(dtype)


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_mse_ordered_sum_rounding_stress(ctx, pcu_pkg, dtype):
    """The ordered sum of squares at sizes around the kernel's chunking (4096 and 8192
    elements), with rounding ties, subnormal totals, huge steps after a tiny total and
    overflow at chosen positions: bit-exact against the oracle's dependent chain."""
    rng = np.random.default_rng(2024)
    info = np.finfo(dtype)
    sub_k = (-74, -62) if dtype == np.float32 else (-537, -505)
    sizes = [1, 63, 4095, 4096, 4097, 8191, 8192, 8193, 3 * 8192 + 5, 70_001]
    for n in sizes:
        cases = [
            _tie_heavy(rng, n, dtype, -20, 4),
            _tie_heavy(rng, n, dtype, -14, -10),
            _tie_heavy(rng, n, dtype, *sub_k),
            np.concatenate([_tie_heavy(rng, n // 2, dtype, -30, -20),
                            _tie_heavy(rng, n - n // 2, dtype, 5, 9)]),
            rng.uniform(-1, 1, n).astype(dtype),
        ]
        if n > 2:
            big = np.full(n, np.sqrt(info.max) * dtype(0.75), dtype)
            big[: n // 3] = dtype(0.5)
            cases.append(big)  # Add overflow once two huge squares meet
        for i, p in enumerate(cases):
            t = np.zeros(n, dtype)
            got, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_mse(ctx.upload(p), ctx.upload(t)).numpy())
            ref, rf = oracle.mse(p, t)
            assert gf == _ofault(rf), (n, i, gf, rf)
            if rf is None:
                assert _bits(got).item() == _bits(ref).item(), (n, i, got, ref)


def test_mse_ordered_sum_estimate_misses(ctx, pcu_pkg):
    """The ordered sum steps over whole chunks using summaries made for the binade that a
    binary64 estimate of the running total predicts. Here the binary32 total sits at
    5792^2 = 2^25 - 7168 and every further square (0.99^2 < half an ulp) is absorbed,
    while the exact sum keeps growing past 2^25 (1 + 1/512): from about the ninth chunk on,
    no summary matches the true binade and every chunk takes the exact path. The result
    must still be the dependent chain's, bit for bit."""
    n = 150_000
    p = np.full(n, 0.99, np.float32)
    p[0] = np.float32(5792.0)
    t = np.zeros(n, np.float32)
    got = ctx.strict_mse(ctx.upload(p), ctx.upload(t)).numpy()
    ref, rf = oracle.mse(p, t)
    assert rf is None
    assert _bits(got).item() == _bits(ref).item()
    assert ref * np.float32(n) == np.float32(5792.0 ** 2)  # the total never moved


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_mse_ordered_sum_uneven_chunks(ctx, pcu_pkg, dtype):
    """Chunks whose squares are far from their mean: the walk folds a chunk exactly in
    windows sized from the chunk's mean square, so windows that are too short (no crossing:
    fold and widen) and too long (several crossings) both occur. Also zero prefixes, a
    steady exponential climb with a crossing every few thousand squares, sparse spikes, and
    binade crossings in the last chunk of a 512-chunk batch and past it. Bit-exact against
    the oracle's dependent chain."""
    rng = np.random.default_rng(99)
    L = 8192 if dtype == np.float32 else 4096   # elements per chunk of the ordered sum
    n = 6 * L + 77
    half = np.where((np.arange(n) % L) < L // 2, dtype(1e-3), dtype(1.0))
    zeros_then = np.concatenate([np.zeros(L + L // 2, dtype), rng.uniform(-1, 1, n - L - L // 2).astype(dtype)])
    climb = np.exp2(np.arange(n) / 4000.0).astype(dtype)
    spikes = np.full(n, 1e-4, dtype)
    spikes[::997] = dtype(300.0)
    tail_heavy = rng.uniform(-1e-3, 1e-3, n).astype(dtype)
    tail_heavy[n - L // 3:] = rng.uniform(100, 200, L // 3).astype(dtype)
    cases = [half, zeros_then, climb, spikes, tail_heavy]
    # Every total a whole count: the k-th binade starts at square 2^k, in chunks 2^(k-13)-1
    # (binary32) or 2^(k-12)-1 (binary64), among them the last of the first 512-chunk batch.
    ones_n = 1024 * L + 5
    cases.append(np.ones(ones_n, dtype))
    for i, p in enumerate(cases):
        t = np.zeros(p.size, dtype)
        got, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_mse(ctx.upload(p), ctx.upload(t)).numpy())
        ref, rf = oracle.mse(p, t)
        assert gf == _ofault(rf), (i, gf, rf)
        if rf is None:
            assert _bits(got).item() == _bits(ref).item(), (i, got, ref)


# ------------------------------------------------------------------- MatMul


ENGINES = ["auto", "valu", "mfma_products"]


@pytest.fixture(params=ENGINES)
def engine(request, ctx):
    """Runs a MatMul test once per engine; every engine must give the oracle's bits and
    first fault. "auto" runs outputs of at most 256 x 256 cells (F32) or 512 x 512 (F64) as
    one fused launch; "valu" and "mfma_products" always take the screened tile kernels
    (F64 uses the vector unit under both)."""
    ctx.set_matmul_engine(request.param)
    yield request.param
    ctx.set_matmul_engine("auto")


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("shape", [(1, 1, 1), (2, 3, 2), (65, 3, 17), (128, 128, 128),
                                   (129, 67, 255), (300, 257, 130), (512, 1024, 256),
                                   (33, 1, 257), (1, 513, 1), (255, 17, 129),
                                   # whole-slab kernels: one slab, and whole in two of three
                                   (128, 16, 128), (256, 32, 384), (256, 48, 130), (130, 64, 256),
                                   # whole, with 3, 4 and 6 slabs (every trip count of the
                                   # three-stage slab loop)
                                   (128, 48, 128), (256, 64, 128), (128, 96, 256),
                                   # whole 64 x 64 tiles of 16 x 16 waves: 1, 5 and 17 slabs
                                   (64, 16, 64), (192, 80, 320), (448, 272, 512)])
def test_matmul_parity_all_transposes(ctx, pcu_pkg, dtype, shape, engine):
    m, k, n = shape
    rng = np.random.default_rng(m * 7 + k * 3 + n)
    for tl in (False, True):
        for tr in (False, True):
            a = rng.uniform(-1, 1, (k, m) if tl else (m, k)).astype(dtype)
            b = rng.uniform(-1, 1, (n, k) if tr else (k, n)).astype(dtype)
            got = ctx.strict_matmul(ctx.upload(a), ctx.upload(b), tl, tr).numpy()
            ref, rf = oracle.matmul(a, b, tl, tr)
            assert rf is None
            np.testing.assert_array_equal(_bits(got), _bits(ref), err_msg=f"{shape} {tl} {tr}")


def _run_tensor_case(ctx, pcu_pkg, case):
    dtype = np.float32 if case["dtype"] == "f32" else np.float64
    itype = np.uint32 if dtype == np.float32 else np.uint64
    ins = []
    for s in case["inputs"]:
        arr = np.array([int(x, 16) for x in s["bits"]], dtype=itype).view(dtype)
        ins.append(arr.reshape(s["shape"]) if s["shape"] else arr.reshape(1))
    policy = POLICY[case["policy"]]
    if case["op"] == "matmul":
        fn = lambda: ctx.strict_matmul(ctx.upload(ins[0]), ctx.upload(ins[1]), case["params"]["tl"],
                                       case["params"]["tr"], policy).numpy()
    elif case["op"] == "sgd":
        rate = np.array([int(case["params"]["rate"], 16)], dtype=np.uint32).view(np.float32)[0]
        fn = lambda: ctx.strict_sgd(ctx.upload(ins[0].reshape(-1)), ctx.upload(ins[1].reshape(-1)),
                                    rate, policy).numpy()
    else:
        fn = lambda: ctx.strict_mse(ctx.upload(ins[0].reshape(-1)), ctx.upload(ins[1].reshape(-1)),
                                    policy).numpy()
    return fn, itype


STEP = {"Multiply": 1, "Add": 2, "Subtract": 3, "Divide": 4}
KIND = {"ArithmeticOverflow": 3, "ArithmeticUnderflow": 4, "InvalidFloatingOperand": 5}


@pytest.mark.parametrize("case", json.load(open(os.path.join(GOLDEN, "tensor_kat.json")))["cases"],
                         ids=lambda c: f"{c['op']}-{c['dtype']}-{c['source']}")
def test_reference_tensor_known_answers_on_gpu(ctx, pcu_pkg, case, engine):
    fn, itype = _run_tensor_case(ctx, pcu_pkg, case)
    got, gf = _gpu_fault(pcu_pkg, fn)
    if case["fault"] is not None:
        e, r, step, kind = case["fault"]
        assert gf == (e, r, STEP[step], KIND[kind]), (gf, case)
    else:
        assert gf is None, (gf, case)
        assert [int(v) for v in np.asarray(got).reshape(-1).view(itype)] == [int(v, 16) for v in case["output"]]


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_matmul_fault_variants_parity(ctx, pcu_pkg, dtype, engine):
    """The C2 fault variants at 256^3: 0.1% of A set to 3.0e38 (Add overflow) and 0.1% of
    B set to NaN (Multiply invalid at the lowest cell), plus tiny operands (underflow)."""
    rng = np.random.default_rng(2024)
    m = k = n = 256
    a = rng.uniform(-1, 1, (m, k)).astype(dtype)
    b = rng.uniform(-1, 1, (k, n)).astype(dtype)
    huge = dtype(3.0e38) if dtype == np.float32 else dtype(1.7e308)
    cnt = int(np.ceil(0.001 * m * k))
    for variant in range(4):
        aa, bb = a.copy(), b.copy()
        if variant == 0:
            aa.reshape(-1)[rng.choice(m * k, cnt * 8, replace=False)] = huge
        elif variant == 1:
            bb.reshape(-1)[rng.choice(k * n, cnt, replace=False)] = np.nan
        elif variant == 2:
            aa[100:110, :] *= dtype(np.finfo(dtype).tiny)  # tiny-inexact products in rows 100..109
        else:
            bb[:, 7] = np.finfo(dtype).tiny * 0.5  # exact tiny products? rounding decides
        for policy in (0, 1, 2):
            got, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_matmul(ctx.upload(aa), ctx.upload(bb), False, False, policy).numpy())
            ref, rf = oracle.matmul(aa, bb, policy=policy)
            assert gf == _ofault(rf), (variant, policy, gf, rf)
            if rf is None:
                np.testing.assert_array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_matmul_random_fault_placement_fuzz(ctx, pcu_pkg, dtype, engine):
    """Seeded fuzz of the first-fault search: 24 random shapes, layouts and underflow
    policies, each with up to three operands of A and of B replaced by NaN, an infinity, a
    huge value (overflowing products and sums), a value whose products are tiny and mostly
    inexact, or a subnormal. The GPU must report the oracle's first (cell, k, step, kind)
    or, when the oracle has none, its bits."""
    rng = np.random.default_rng(7 if dtype == np.float32 else 8)
    info = np.finfo(dtype)
    specials = np.array([np.nan, np.inf, -np.inf, info.max, -info.max,
                         info.tiny * dtype(2.0 ** 20), -info.tiny * dtype(3.0),
                         info.smallest_subnormal * dtype(3.0)], dtype=dtype)
    for case in range(24):
        m, k, n = (int(v) for v in rng.integers(1, 200, size=3))
        tl, tr = bool(rng.integers(2)), bool(rng.integers(2))
        policy = int(rng.integers(3))
        a = rng.uniform(-1, 1, (k, m) if tl else (m, k)).astype(dtype)
        b = rng.uniform(-1, 1, (n, k) if tr else (k, n)).astype(dtype)
        for x in (a, b):
            cnt = min(int(rng.integers(0, 4)), x.size)
            if cnt:
                x.reshape(-1)[rng.choice(x.size, cnt, replace=False)] = rng.choice(specials, size=cnt)
        got, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_matmul(ctx.upload(a), ctx.upload(b), tl, tr, policy).numpy())
        ref, rf = oracle.matmul(a, b, tl, tr, policy=policy)
        assert gf == _ofault(rf), (case, m, k, n, tl, tr, policy, gf, rf)
        if rf is None:
            np.testing.assert_array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("grid", ["small", "full"])
@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_matmul_whole_tile_fuzz(ctx, pcu_pkg, dtype, engine, grid):
    """The same first-fault fuzz over whole tiles only (M and N multiples of 128, K of 16),
    where the main kernels load operands straight into LDS in per-layout arrangements and run
    three slabs a trip. "small" outputs have fewer 128 x 128 tiles than the GPU has CUs (F32
    runs 64 x 64 tiles, F64 its narrow tile); "full" ones have at least as many (the 128 x
    128 kernels). 12 seeded cases over every layout and policy, a third clean (bits
    compared) and the rest with up to five special operands, so faults land in different
    slabs and stages; the GPU must give the oracle's first fault or, without one, its bits."""
    rng = np.random.default_rng((31 if dtype == np.float32 else 32) + (grid == "full") * 10)
    info = np.finfo(dtype)
    specials = np.array([np.nan, np.inf, -np.inf, info.max, -info.max,
                         info.tiny * dtype(2.0 ** 20), -info.tiny * dtype(3.0),
                         info.smallest_subnormal * dtype(3.0)], dtype=dtype)
    full_shapes = [(2048, 2048), (4096, 1024), (1024, 4096), (2048, 2560)]
    for case in range(12):
        if grid == "small":
            m, n = (128 * int(v) for v in rng.integers(1, 4, size=2))
            k = 16 * int(rng.integers(1, 25))
        else:
            m, n = full_shapes[int(rng.integers(len(full_shapes)))]
            k = 16 * int(rng.integers(1, 9))
        tl, tr = case % 2 == 1, (case // 2) % 2 == 1
        policy = int(rng.integers(3))
        a = rng.uniform(-1, 1, (k, m) if tl else (m, k)).astype(dtype)
        b = rng.uniform(-1, 1, (n, k) if tr else (k, n)).astype(dtype)
        for x in (a, b):
            cnt = int(rng.integers(0, 6)) if case % 3 else 0
            if cnt:
                x.reshape(-1)[rng.choice(x.size, cnt, replace=False)] = rng.choice(specials, size=cnt)
        got, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_matmul(ctx.upload(a), ctx.upload(b), tl, tr, policy).numpy())
        ref, rf = oracle.matmul(a, b, tl, tr, policy=policy)
        assert gf == _ofault(rf), (case, m, k, n, tl, tr, policy, gf, rf)
        if rf is None:
            np.testing.assert_array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("shape", [(128, 0, 128), (2048, 0, 2048), (65, 0, 17), (0, 5, 7), (6, 5, 0)],
                         ids=["small-grid", "full-grid", "ragged", "no-rows", "no-cols"])
def test_matmul_empty_reduction_and_empty_output(ctx, pcu_pkg, dtype, shape, engine):
    """An empty reduction (K = 0) leaves every cell at the +0 it starts from
    (strict_matmul.rs:22-73), on whole tiles of either grid and on ragged ones, in every
    layout and policy; an empty output launches nothing and is no fault."""
    m, k, n = shape
    for tl in (False, True):
        for tr in (False, True):
            a = np.zeros((k, m) if tl else (m, k), dtype)
            b = np.zeros((n, k) if tr else (k, n), dtype)
            for policy in (0, 1, 2):
                got = ctx.strict_matmul(ctx.upload(a), ctx.upload(b), tl, tr, policy).numpy()
                ref, rf = oracle.matmul(a, b, tl, tr, policy=policy)
                assert rf is None and got.shape == (m, n)
                np.testing.assert_array_equal(_bits(got), _bits(ref))
                assert not _bits(got).any()


@pytest.mark.parametrize("policy", [0, 1, 2])
def test_matmul_signed_zero_and_subnormal_products(ctx, pcu_pkg, policy, engine):
    """Operands whose products are exact zeros of either sign, subnormal, or straddle the
    smallest normal, with subnormal inputs on both sides: under every underflow policy the
    F32 MatMul must give the oracle's bits and first fault (the matrix-core engine returns
    +0 for a -0 product, which must never show in a result)."""
    rng = np.random.default_rng(99 + policy)
    m, k, n = 96, 70, 80
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    a[rng.random((m, k)) < 0.3] = np.float32(-0.0)
    b[rng.random((k, n)) < 0.3] = np.float32(0.0)
    a[::3] *= np.float32(2.0 ** -70)
    b[:, ::5] *= np.float32(2.0 ** -60)
    sub = np.array([1, 3, 0x7fffff, 0x400000, 0x12345], np.uint32).view(np.float32)
    a[5, :5] = sub
    b[:5, 7] = sub * np.float32(2.0 ** 100)
    a[-1] = np.float32(-0.0)
    for tl, tr in ((False, False), (True, True)):
        aa = np.ascontiguousarray(a.T) if tl else a
        bb = np.ascontiguousarray(b.T) if tr else b
        got, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_matmul(ctx.upload(aa), ctx.upload(bb), tl, tr, policy).numpy())
        ref, rf = oracle.matmul(aa, bb, tl, tr, policy=policy)
        assert gf == _ofault(rf), (policy, tl, tr, gf, rf)
        if rf is None:
            np.testing.assert_array_equal(_bits(got), _bits(ref))


# ------------------------------------------------------------------ program


def test_program_reports_first_node_and_recovers(ctx, pcu_pkg):
    rng = np.random.default_rng(3)
    a = rng.uniform(-1, 1, (64, 32)).astype(np.float32)
    b = rng.uniform(-1, 1, (32, 48)).astype(np.float32)
    da, db = ctx.upload(a), ctx.upload(b)
    bad = b.copy()
    bad[5, 9] = np.nan
    dbad = ctx.upload(bad)
    dnan = ctx.upload(np.array([np.nan], np.float32))
    # node 0 fine, node 1 faults at (cell 9, k 5), node 2 faults too: node 1 is reported.
    try:
        with ctx.program():
            ctx.strict_matmul(da, db)
            ctx.strict_matmul(da, dbad)
            ctx.checked_relu(dnan)
        raise AssertionError("expected fault")
    except pcu_pkg.PcuExecutionError as e:
        f = e.tensor_fault
        assert (f.node, f.element_index, f.reduction_index, int(f.step), int(f.kind)) == (1, 9, 5, 1, 5)
    # A fault never poisons the next call (backends/rocm/tensor/strict_matmul/hardware.rs:244-313).
    got = ctx.strict_matmul(da, db).numpy()
    ref, _ = oracle.matmul(a, b)
    np.testing.assert_array_equal(_bits(got), _bits(ref))
    with ctx.program():
        x = ctx.strict_matmul(da, db)
        y = ctx.checked_relu(x)
    ref2, _ = oracle.relu(ref)
    np.testing.assert_array_equal(_bits(y.numpy()), _bits(ref2))


def _chain_inputs(rng, dtype, m, k, n):
    """Fresh inputs of the fuzzed chain; some get one special value planted."""
    info = np.finfo(dtype)
    specials = np.array([np.nan, np.inf, -np.inf, info.max, info.tiny * dtype(0.75),
                         info.smallest_subnormal], dtype=dtype)
    shapes = {"x": (m, k), "w": (k, n), "bias": (m, n), "up": (m, n), "g": (k, n), "t": (m, n)}
    out = {}
    for name, shape in shapes.items():
        v = rng.uniform(-1, 1, shape).astype(dtype)
        if rng.random() < 0.3:
            v.reshape(-1)[int(rng.integers(v.size))] = rng.choice(specials)
        out[name] = v
    return out


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_program_random_chains_fuzz(ctx, pcu_pkg, dtype):
    """Seeded fuzz of program mode over 16 chains: y = x.w (node 0), z = y + bias (1),
    r = relu(z) (2), relu_backward(z, up) (3), sgd(w, g) (4), mse(r, t) (5), with random
    shapes and a special value planted in some fresh inputs. The program reports the first
    faulting node in node order with the oracle's coordinates (later nodes are gated); when
    no node faults, every node's bits match the oracle's."""
    rng = np.random.default_rng(41 if dtype == np.float32 else 42)
    rate = 0.01
    for case in range(16):
        m, k, n = (int(v) for v in rng.integers(1, 160, size=3))
        v = _chain_inputs(rng, dtype, m, k, n)
        # Oracle, node by node, stopping at the first fault.
        expect, outs = None, []
        for node, run in enumerate([
                lambda: oracle.matmul(v["x"], v["w"]),
                lambda: oracle.binary(0, outs[0], v["bias"]),
                lambda: oracle.relu(outs[1]),
                lambda: oracle.relu_backward(outs[1], v["up"]),
                lambda: oracle.sgd(v["w"], v["g"], rate),
                lambda: oracle.mse(outs[2], v["t"])]):
            res, fault = run()
            if fault is not None:
                expect = (node,) + _ofault(fault)
                break
            outs.append(res)
        d = {name: ctx.upload(arr) for name, arr in v.items()}
        got = []
        try:
            with ctx.program():
                gy = ctx.strict_matmul(d["x"], d["w"])
                gz = ctx.checked_binary(0, gy, d["bias"])
                gr = ctx.checked_relu(gz)
                gb = ctx.checked_relu_backward(gz, d["up"])
                gw = ctx.strict_sgd(d["w"], d["g"], rate)
                gl = ctx.strict_mse(gr, d["t"])
                got = [gy, gz, gr, gb, gw, gl]
            gf = None
        except pcu_pkg.PcuExecutionError as e:
            f = e.tensor_fault
            gf = (f.node, f.element_index, f.reduction_index, int(f.step), int(f.kind))
        assert gf == expect, (case, m, k, n, gf, expect)
        if expect is None:
            for node, (g, r) in enumerate(zip(got, outs)):
                np.testing.assert_array_equal(_bits(np.asarray(g.numpy()).reshape(-1)),
                                              _bits(np.asarray(r).reshape(-1)), err_msg=str((case, node)))


def test_held_fault_read_and_reset(ctx, pcu_pkg):
    """pcu_fault_read returns the first fault of the most recent call, as that call
    reported it; a clean call clears it, and so does pcu_fault_reset."""
    a = np.ones((3, 4), np.float32)
    b = np.ones((4, 2), np.float32)
    da, db = ctx.upload(a), ctx.upload(b)
    ctx.strict_matmul(da, db)
    assert ctx.last_fault() is None
    a[1, 2] = np.nan
    dbad = ctx.upload(a)
    with pytest.raises(pcu_pkg.PcuExecutionError) as e:
        ctx.strict_matmul(dbad, db)
    held = ctx.last_fault()
    assert held == e.value.tensor_fault
    assert (held.element_index, held.reduction_index) == (2, 2)  # row 1, col 0, k = 2
    ctx.reset_fault()
    assert ctx.last_fault() is None
    with pytest.raises(pcu_pkg.PcuExecutionError):
        ctx.strict_matmul(dbad, db)
    assert ctx.last_fault() is not None
    ctx.strict_matmul(da, db)
    assert ctx.last_fault() is None


@pytest.mark.parametrize("engine_name", ["valu", "mfma_products"])
def test_program_stage_gate_skips_nodes_after_a_fault(ctx, pcu_pkg, engine_name):
    """Stage gating (backends/rocm/owned_dispatch/guarded/guarded.rs): once a node has
    faulted, the kernels of later nodes skip their work; earlier nodes always run, and the
    reported fault is the earliest one."""
    ctx.set_matmul_engine(engine_name)
    try:
        rng = np.random.default_rng(4)
        a = rng.uniform(-1, 1, (256, 128)).astype(np.float32)
        b = rng.uniform(-1, 1, (128, 192)).astype(np.float32)
        da, db = ctx.upload(a), ctx.upload(b)
        sentinel = np.full((256, 192), 7.0, np.float32)
        out = ctx.upload(sentinel)
        dnan = ctx.upload(np.array([1.0, np.nan, 2.0], np.float32))
        relu_out = ctx.empty((3,), np.float32)
        # node 0 faults, node 1 (a MatMul) is skipped
        with pytest.raises(pcu_pkg.PcuExecutionError) as e:
            with ctx.program():
                ctx.checked_relu(dnan, out=relu_out)
                ctx.strict_matmul(da, db, out=out)
        f = e.value.tensor_fault
        assert (f.node, f.element_index, int(f.kind)) == (0, 1, 5)
        assert np.array_equal(out.numpy().view(np.uint32), sentinel.view(np.uint32))
        # an earlier node always runs: node 0 (the MatMul) completes, node 1 faults
        with pytest.raises(pcu_pkg.PcuExecutionError) as e:
            with ctx.program():
                ctx.strict_matmul(da, db, out=out)
                ctx.checked_relu(dnan, out=relu_out)
        assert e.value.tensor_fault.node == 1
        ref, _ = oracle.matmul(a, b)
        np.testing.assert_array_equal(_bits(out.numpy()), _bits(ref))
        # the next program starts with an open gate
        out2 = ctx.upload(sentinel)
        with ctx.program():
            ctx.strict_matmul(da, db, out=out2)
        np.testing.assert_array_equal(_bits(out2.numpy()), _bits(ref))
    finally:
        ctx.set_matmul_engine("auto")


@pytest.mark.parametrize("policy", list(POLICY), ids=list(POLICY))
def test_program_opened_by_its_first_matmul(ctx, pcu_pkg, policy):
    """A MatMul that is a program's first node opens the program from its own first kernel
    (the screen, or its stand-in when there is nothing to screen): after a program whose
    node 0 faulted, the next program's fault words and stage gate must read as fresh, so
    its node 1 still runs and is the node reported."""
    pol = POLICY[policy]
    rng = np.random.default_rng(21)
    a = rng.uniform(-1, 1, (128, 64)).astype(np.float32)
    b = rng.uniform(-1, 1, (64, 96)).astype(np.float32)
    da, db = ctx.upload(a), ctx.upload(b)
    dnan = ctx.upload(np.array([1.0, np.nan], np.float32))
    ref, _ = oracle.matmul(a, b, policy=pol)
    for _ in range(2):
        with pytest.raises(pcu_pkg.PcuExecutionError) as e:
            with ctx.program():
                ctx.checked_relu(dnan)
        assert e.value.tensor_fault.node == 0
        with pytest.raises(pcu_pkg.PcuExecutionError) as e:
            with ctx.program():
                out = ctx.strict_matmul(da, db, False, False, pol)
                ctx.checked_relu(dnan)
        f = e.value.tensor_fault
        assert (f.node, f.element_index, int(f.kind)) == (1, 1, 5)
        np.testing.assert_array_equal(_bits(out.numpy()), _bits(ref))
        got = ctx.strict_matmul(da, db, False, False, pol).numpy()
        np.testing.assert_array_equal(_bits(got), _bits(ref))
        assert ctx.last_fault() is None


# ------------------------------------------------------------ output aliasing


def test_output_overlapping_an_operand_is_rejected(ctx, pcu_pkg):
    """A MatMul output may share no byte with an operand; an elementwise or SGD output may
    be exactly an operand (in place) but may not overlap one any other way. Rejections are
    PCU_ERR_ARGUMENT from the C ABI, before any kernel runs; the in-place forms are
    bit-exact."""
    import ctypes
    from fusion_pcu_amd import _abi
    lib = pcu_pkg.lib()
    rng = np.random.default_rng(17)
    a = rng.uniform(-1, 1, (64, 64)).astype(np.float32)
    big = ctx.upload(np.concatenate([a.reshape(-1), a.reshape(-1)]))
    base = big.ptr
    f = _abi.Fault()
    st = lib.pcu_strict_matmul(ctx.handle, 0, 64, 64, 64, 0, 0, base, base + 64 * 64 * 4,
                               base + 4 * 64, 0, ctypes.byref(f))
    assert st == _abi.PCU_ERR_ARGUMENT, st
    assert "overlap" in ctx.error_text()
    # Every range below lies inside `big` (2 * 64 * 64 floats); each call must be refused.
    st = lib.pcu_native_matmul(ctx.handle, 0, 64, 64, 64, 0, 0, base, base + 64 * 64 * 4,
                               base + 64 * 64 * 4 - 4)
    assert st == _abi.PCU_ERR_ARGUMENT
    st = lib.pcu_checked_relu(ctx.handle, 0, 64 * 64, base, base + 16, 0, ctypes.byref(f))
    assert st == _abi.PCU_ERR_ARGUMENT
    st = lib.pcu_strict_sgd(ctx.handle, 0, 64 * 64, base, base + 64 * 64 * 4, ctypes.c_float(0.01),
                            base + 64 * 64 * 4 - 64, 0, ctypes.byref(f))
    assert st == _abi.PCU_ERR_ARGUMENT
    st = lib.pcu_strict_mse(ctx.handle, 0, 64 * 64, base, base + 64 * 64 * 4, base + 8, 0,
                            ctypes.byref(f))
    assert st == _abi.PCU_ERR_ARGUMENT
    # In place: SGD into its own weights, ReLU into its own input.
    g = rng.uniform(-1e-3, 1e-3, 64 * 64).astype(np.float32)
    dw, dg = ctx.upload(a.reshape(-1)), ctx.upload(g)
    ctx.strict_sgd(dw, dg, 0.01, out=dw)
    want, wf = oracle.sgd(a.reshape(-1), g, 0.01)
    assert wf is None
    np.testing.assert_array_equal(_bits(dw.numpy()), _bits(want))
    ctx.checked_relu(dw, out=dw)
    want2, wf2 = oracle.relu(want)
    assert wf2 is None
    np.testing.assert_array_equal(_bits(dw.numpy()), _bits(want2))


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_in_place_calls_report_the_oracles_first_fault(ctx, pcu_pkg, dtype):
    """Every in-place form (out equal to an operand) with planted faults of several kinds.
    The kernels store a whole vector before they classify its flagged lanes, so the store
    overwrites the operand a fault is classified from: the reported first fault must still
    be the oracle's on the original operands."""
    rng = np.random.default_rng(23)
    n = 70_001
    big, tiny = np.finfo(dtype).max, np.finfo(dtype).tiny

    def fresh():
        return rng.uniform(-1, 1, n).astype(dtype)

    def spots():
        return sorted(int(x) for x in rng.choice(n, 3, replace=False))

    # checked Add / Multiply into either operand: a tiny-inexact product, an overflow, a NaN
    for op, into in ((0, "a"), (0, "b"), (2, "a"), (2, "b")):
        a, b = fresh(), fresh()
        i, j, k = spots()
        a[i], b[i] = tiny, dtype(1.0 / 3.0)
        a[j], b[j] = big, big if op == 0 else dtype(2.0)
        b[k] = np.nan
        _, rf = oracle.binary(op, a, b)
        assert rf is not None
        da, db = ctx.upload(a), ctx.upload(b)
        out = da if into == "a" else db
        _, gf = _gpu_fault(pcu_pkg, lambda: ctx.checked_binary(op, da, db, out=out))
        assert gf == _ofault(rf), (op, into, gf, rf)
        da.free()
        db.free()
    # ReLU backward into its input or its upstream gradient: a NaN input, an infinite upstream
    for into in ("x", "up"):
        x, up = fresh(), fresh()
        i, j, _ = spots()
        x[j] = np.nan
        up[i] = -np.inf
        _, rf = oracle.relu_backward(x, up)
        assert rf is not None
        dx, du = ctx.upload(x), ctx.upload(up)
        out = dx if into == "x" else du
        _, gf = _gpu_fault(pcu_pkg, lambda: ctx.checked_relu_backward(dx, du, out=out))
        assert gf == _ofault(rf), (into, gf, rf)
        dx.free()
        du.free()
    # SGD into its weights: an invalid Multiply (NaN gradient) and an overflowing Subtract
    w, g = fresh(), fresh() * dtype(1e-3)
    i, j, _ = spots()
    w[i], g[i] = -big, big
    g[j] = np.nan
    _, rf = oracle.sgd(w, g, 0.01)
    assert rf is not None
    dw, dg = ctx.upload(w), ctx.upload(g)
    _, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_sgd(dw, dg, 0.01, out=dw))
    assert gf == _ofault(rf), (gf, rf)
    dw.free()
    dg.free()
    # fused Add -> ReLU into its left operand: the Add's overflow comes first
    a, b = fresh(), fresh()
    i, j, _ = spots()
    a[i], b[i] = big, big
    a[j] = np.inf
    _, rf = oracle.binary(0, a, b)
    assert rf is not None
    da, db = ctx.upload(a), ctx.upload(b)
    _, gf = _gpu_fault(pcu_pkg, lambda: ctx.checked_add_relu(da, db, out=da))
    assert gf == _ofault(rf), (gf, rf)
    da.free()
    db.free()


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_matmul_first_fault_late_in_a_long_reduction(ctx, pcu_pkg, dtype, engine):
    """The replay's walk of one cell over K = 1000 (sixteen chunks of 64, the last one
    partial), every layout and policy, against the oracle: (a) cell (2, 3) overflows in the
    Add at k 700, its first non-finite cell; (b) the same with a NaN at k 650 of column 3,
    so cell (0, 3)'s Multiply at k 650 is first; (c) the overflow moved into the partial
    last chunk (k 990); (d) the k 700 overflow with a NaN and an infinity in later rows, whose
    cells are all non-finite; (e) row 1 zero but for two normal products at k 400 and 500
    whose sum is subnormal: finite cells the screen marks, where RejectSubnormal faults in
    the Add at k 500 of cell (1, 0) and the other policies have no fault."""
    m, k, n = 5, 1000, 7
    f32 = dtype == np.float32
    rng = np.random.default_rng(77 if f32 else 78)
    huge = dtype(3.0e38) if f32 else dtype(1.7e308)

    def base(k1, k2):
        a = rng.uniform(-1, 1, (m, k)).astype(dtype)
        b = rng.uniform(-1, 1, (k, n)).astype(dtype)
        a[2, k1] = a[2, k2] = huge
        b[k1, :] = b[k2, :] = dtype(0.25)  # the other columns of row 2 stay finite
        b[k1, 3] = b[k2, 3] = dtype(1.0)
        return a, b

    cases = [("add-overflow-k700", *base(100, 700))]
    a, b = base(100, 700)
    b[650, 3] = np.nan
    cases.append(("mul-invalid-k650", a, b))
    cases.append(("add-overflow-k990", *base(30, 990)))
    a, b = base(100, 700)
    a[3, 900], a[4, 10] = np.nan, np.inf
    cases.append(("overflow-before-later-nan", a, b))
    a = rng.uniform(-1, 1, (m, k)).astype(dtype)
    b = rng.uniform(-1, 1, (k, n)).astype(dtype)
    e = -125 if f32 else -1021
    a[1, :] = 0
    a[1, 400], a[1, 500] = dtype(2.0 ** e), dtype(-1.25 * 2.0 ** e)
    b[400, :] = b[500, :] = dtype(1.0)
    cases.append(("subnormal-sum-k500", a, b))
    want = {"add-overflow-k700": (2 * n + 3, 700), "mul-invalid-k650": (3, 650),
            "add-overflow-k990": (2 * n + 3, 990), "overflow-before-later-nan": (2 * n + 3, 700)}
    for name, a, b in cases:
        for tl in (False, True):
            for tr in (False, True):
                aa = np.ascontiguousarray(a.T) if tl else a
                bb = np.ascontiguousarray(b.T) if tr else b
                for policy in (0, 1, 2):
                    got, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_matmul(ctx.upload(aa), ctx.upload(bb), tl, tr, policy).numpy())
                    ref, rf = oracle.matmul(aa, bb, tl, tr, policy=policy)
                    assert gf == _ofault(rf), (name, tl, tr, policy, gf, rf)
                    if rf is None:
                        np.testing.assert_array_equal(_bits(got), _bits(ref), err_msg=f"{name} {tl} {tr} {policy}")
                    if name in want:
                        assert _ofault(rf)[:2] == want[name], (name, policy, rf)
                    elif policy == 1:
                        assert _ofault(rf)[:2] == (n, 500), rf
                    else:
                        assert rf is None, (name, policy, rf)


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_matmul_replay_paths_for_marked_cells(ctx, pcu_pkg, dtype, engine):
    """The replay's two passes under the IEEE policy, every layout, against the oracle:
    (a) every cell marked by the exponent screen, no tiny product, no fault (the tiled tiny
    scan clears everything); (b) every row flagged by exact subnormal products (no fault)
    before a tiny-inexact product at cell (17, 33), k 9, so the wave pass walks flagged but
    clean cells first; (c) a NaN in row 40 and an inexact tiny product in row 50: the serial
    pass's Invalid wins; (d) the same with the tiny product moved to row 10: the wave pass's
    Underflow wins."""
    f32 = dtype == np.float32
    m, k, n = 300, 200, 260
    rng = np.random.default_rng(123 if f32 else 124)
    p2 = lambda e: dtype(2.0 ** e)
    clean_e = -120 if f32 else -1016
    exact_a, exact_b = (-100, -40) if f32 else (-1000, -60)
    inexact_a, inexact_b = (-100, -30) if f32 else (-1000, -40)

    def base():
        a = rng.uniform(-1, 1, (m, k)).astype(dtype)
        b = rng.uniform(-1, 1, (k, n)).astype(dtype)
        return a, b

    cases = []
    a, b = base()
    a[:, 5] = p2(clean_e) * np.where(rng.random(m) < 0.5, -1, 1).astype(dtype)
    b[5, :] = (rng.uniform(0.5, 1.0, n) * np.where(rng.random(n) < 0.5, -1, 1)).astype(dtype)
    cases.append(("clean", a, b))
    a, b = base()
    a[:, 5], b[5, :] = p2(exact_a), p2(exact_b)
    a[17, 9], b[9, 33] = dtype(1.5) * p2(inexact_a), dtype(1.3) * p2(inexact_b)
    cases.append(("exact-then-inexact", a, b))
    for row, name in ((50, "serial-wins"), (10, "tiny-wins")):
        a, b = base()
        a[40, 3] = np.nan
        a[row, 9], b[9, 33] = dtype(1.5) * p2(inexact_a), dtype(1.3) * p2(inexact_b)
        cases.append((name, a, b))
    for name, a, b in cases:
        for tl in (False, True):
            for tr in (False, True):
                aa = np.ascontiguousarray(a.T) if tl else a
                bb = np.ascontiguousarray(b.T) if tr else b
                got, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_matmul(ctx.upload(aa), ctx.upload(bb), tl, tr, 0).numpy())
                ref, rf = oracle.matmul(aa, bb, tl, tr, policy=0)
                assert gf == _ofault(rf), (name, tl, tr, gf, rf)
                if rf is None:
                    np.testing.assert_array_equal(_bits(got), _bits(ref), err_msg=f"{name} {tl} {tr}")
        if name == "clean":
            assert rf is None
        elif name == "exact-then-inexact":
            assert _ofault(rf)[:2] == (17 * n + 33, 9)


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("shape", [(128, 32, 128), (128, 32, 144), (512, 64, 512), (640, 64, 640)],
                         ids=["fused64", "fused72", "mid", "large"])
def test_matmul_call_end_paths(ctx, pcu_pkg, dtype, shape):
    """A single strict MatMul call ends its one-node program in one of its own kernels: the
    one-launch small-output kernel when its grid has at most 64 workgroups (128 x 128: 64),
    else a publication launch (128 x 144: 72); on the screened path the tiny scan when no
    cell is suspect and the replay otherwise (512 x 512 binary32; binary64 takes the
    one-launch kernel up to 512 x 512, so 640 x 640 reaches its screened path). Clean, a NaN
    operand, a tiny-inexact product and clean again, back to back, against the oracle."""
    m, k, n = shape
    rng = np.random.default_rng(m * 7 + n + k)
    tiny_a, tiny_b = (-100, -30) if dtype == np.float32 else (-1000, -40)
    for plant in ("none", "nan", "tiny", "none"):
        a = rng.uniform(-1, 1, (m, k)).astype(dtype)
        b = rng.uniform(-1, 1, (k, n)).astype(dtype)
        if plant == "nan":
            a[m - 3, 5] = np.nan
        if plant == "tiny":
            a[3, 7], b[7, n - 2] = dtype(1.5 * 2.0 ** tiny_a), dtype(1.3 * 2.0 ** tiny_b)
        got, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_matmul(ctx.upload(a), ctx.upload(b), False, False, 0).numpy())
        ref, rf = oracle.matmul(a, b, False, False, policy=0)
        assert gf == _ofault(rf), (shape, plant, gf, rf)
        assert (rf is None) == (plant == "none"), (shape, plant, rf)
        if rf is None:
            np.testing.assert_array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("tl,tr", [(False, False), (True, False), (False, True), (True, True)],
                         ids=["nn", "tn", "nt", "tt"])
def test_matmul_full_grid_replay_paths(ctx, pcu_pkg, tl, tr):
    """The replay's passes under IEEE on F32 full grids of whole 128 x 128 tiles (the
    large matrix-core tile kernels, with op(B) transposed read from its K x N copy), every
    layout, two shapes (2048 x 192 x 2048 and 32768 x 192 x 128), each call after a clean
    call of another shape, against the oracle: (a) every cell marked by the exponent
    screen, no tiny product, no fault; (b) exact subnormal products in every cell of the
    first 128 rows before a tiny-inexact product at (17, 33), k 9; (c) a NaN in row 40 and
    a tiny product in row 50: Invalid; (d) the tiny product in row 10 before that NaN:
    Underflow; (e) a tiny product at k 1 of the NaN row's first cell, before the NaN at
    k 3; (f) a tiny product in the last row and the last superslab of k."""
    rng = np.random.default_rng(77)
    p2 = lambda e: np.float32(2.0 ** e)
    other = (ctx.upload(rng.uniform(-1, 1, (2048, 64)).astype(np.float32)),
             ctx.upload(rng.uniform(-1, 1, (64, 4096)).astype(np.float32)))
    for m, k, n in ((2048, 192, 2048), (32768, 192, 128)):
        def base():
            return (rng.uniform(-1, 1, (m, k)).astype(np.float32),
                    rng.uniform(-1, 1, (k, n)).astype(np.float32))
        cases = []
        a, b = base()
        a[:, 5] = p2(-120) * np.where(rng.random(m) < 0.5, -1, 1).astype(np.float32)
        b[5, :] = (rng.uniform(0.5, 1.0, n) * np.where(rng.random(n) < 0.5, -1, 1)).astype(np.float32)
        cases.append(("clean-marked", a, b))
        a, b = base()
        a[:128, 5], b[5, :] = p2(-100), p2(-40)
        a[17, 9], b[9, 33] = np.float32(1.5) * p2(-100), np.float32(1.3) * p2(-30)
        cases.append(("exact-then-inexact", a, b))
        for row, name in ((50, "nan-first"), (10, "tiny-first")):
            a, b = base()
            a[40, 3] = np.nan
            a[row, 9], b[9, 33] = np.float32(1.5) * p2(-100), np.float32(1.3) * p2(-30)
            cases.append((name, a, b))
        a, b = base()
        a[40, 3] = np.nan
        a[40, 1], b[1, 0] = np.float32(1.5) * p2(-100), np.float32(1.3) * p2(-30)
        cases.append(("tiny-in-the-nan-cell", a, b))
        a, b = base()
        a[m - 1, k - 2], b[k - 2, n - 3] = np.float32(1.5) * p2(-100), np.float32(1.3) * p2(-30)
        cases.append(("last-superslab", a, b))
        for name, a, b in cases:
            aa = np.ascontiguousarray(a.T) if tl else a
            bb = np.ascontiguousarray(b.T) if tr else b
            ctx.strict_matmul(other[0], other[1], policy=0).free()
            got, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_matmul(ctx.upload(aa), ctx.upload(bb), tl, tr, 0).numpy())
            ref, rf = oracle.matmul(aa, bb, tl, tr, policy=0)
            assert gf == _ofault(rf), (m, k, n, name, gf, rf)
            if rf is None:
                np.testing.assert_array_equal(_bits(got), _bits(ref), err_msg=f"{name} {m}x{k}x{n}")
            expect = {"clean-marked": None, "exact-then-inexact": (17 * n + 33, 9),
                      "nan-first": (40 * n, 3), "tiny-first": (10 * n + 33, 9),
                      "tiny-in-the-nan-cell": (40 * n, 1),
                      "last-superslab": ((m - 1) * n + n - 3, k - 2)}[name]
            assert (None if rf is None else _ofault(rf)[:2]) == expect, (name, rf)


@pytest.mark.parametrize("policy", [0, 1], ids=["ieee", "reject_subnormal"])
def test_matmul_screen_after_calls_of_other_shapes(ctx, pcu_pkg, policy, engine):
    """Regression: MatMul calls of different shapes share one scratch buffer. A word that one
    call leaves at its "none" value (all ones) must never sit where a later call folds
    generation-tagged words with atomicMax (a column's minimum exponent, a row's first
    flagged column): nothing outranks it there, and that column or row was never screened.
    Each column c of a small output gets its own pair of calls: a clean call of another
    shape, then one whose only fault is a tiny inexact product in row 0, column c, at k 3."""
    rng = np.random.default_rng(41)
    rows, inner, cols = 8, 16, 80
    clean = {}
    for shape in ((8, 8), (8, 40), (8, 72), (16, 8), (24, 40), (40, 8)):
        a = rng.uniform(-1, 1, (shape[0], 12)).astype(np.float32)
        b = rng.uniform(-1, 1, (12, shape[1])).astype(np.float32)
        clean[shape] = (ctx.upload(a), ctx.upload(b))
    a = rng.uniform(-1, 1, (rows, inner)).astype(np.float32)
    a[0, 3] = np.float32(1.5 * 2.0 ** -100)
    da = ctx.upload(a)
    for c in range(cols):
        b = rng.uniform(-1, 1, (inner, cols)).astype(np.float32)
        b[3, :] = np.float32(1.0)
        b[3, c] = np.float32(1.3 * 2.0 ** -30)
        db = ctx.upload(b)
        for shape, (ca, cb) in clean.items():
            ctx.strict_matmul(ca, cb, policy=policy).free()
            _, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_matmul(da, db, policy=policy).numpy())
            assert gf == (c, 3, 1, 4), (shape, c, gf)
        db.free()
    _, rf = oracle.matmul(a, b, policy=policy)
    assert _ofault(rf) == (cols - 1, 3, 1, 4)


@pytest.mark.parametrize("shape", [(2048, 64, 2048), (2080, 33, 2050)], ids=["whole", "ragged"])
def test_matmul_f64_full_grid_tile(ctx, pcu_pkg, shape):
    """Binary64 outputs of at least 256 tiles of 128 x 128 take the 8 x 8-per-thread tile
    (smaller ones the 8 x 4 tile that the other tests reach): every layout, clean and with
    planted NaN, overflow and tiny-inexact operands, against the oracle."""
    m, k, n = shape
    rng = np.random.default_rng(m + k + n)
    for tl in (False, True):
        for tr in (False, True):
            a = rng.uniform(-1, 1, (k, m) if tl else (m, k))
            b = rng.uniform(-1, 1, (n, k) if tr else (k, n))
            for plant in (None, "nan", "huge", "tiny"):
                aa, bb = a.copy(), b.copy()
                if plant == "nan":
                    aa.reshape(-1)[rng.integers(aa.size)] = np.nan
                elif plant == "huge":
                    aa.reshape(-1)[rng.choice(aa.size, 64, replace=False)] = 1.5e308
                elif plant == "tiny":
                    bb.reshape(-1)[rng.choice(bb.size, 8, replace=False)] = 1.3 * 2.0 ** -1040
                got, gf = _gpu_fault(pcu_pkg, lambda: ctx.strict_matmul(ctx.upload(aa), ctx.upload(bb), tl, tr, 0).numpy())
                ref, rf = oracle.matmul(aa, bb, tl, tr, policy=0)
                assert gf == _ofault(rf), (shape, tl, tr, plant, gf, rf)
                if rf is None:
                    np.testing.assert_array_equal(_bits(got), _bits(ref), err_msg=f"{shape} {tl} {tr}")


def test_calibration_direct_copy(ctx, pcu_pkg):
    """The measurement copy (direct global-to-LDS reads) moves every byte, and refuses sizes
    that are not whole 4 KiB chunks."""
    rng = np.random.default_rng(8)
    for n in (1024, 1024 * 37, 1 << 22):
        x = rng.standard_normal(n).astype(np.float32)
        dx = ctx.upload(x)
        dy = ctx.empty((n,), np.float32)
        ctx.calibrate_direct_copy(dx, dy)
        assert np.array_equal(dy.numpy().view(np.uint32), x.view(np.uint32))
        dx.free()
        dy.free()
    dx, dy = ctx.upload(np.zeros(1000, np.float32)), ctx.empty((1000,), np.float32)
    with pytest.raises(pcu_pkg.PcuExecutionError):
        ctx.calibrate_direct_copy(dx, dy)
    dx.free()
    dy.free()
