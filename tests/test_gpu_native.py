"""Explicitly permitted native compound arithmetic (Boundary mode + BackendDefined) on the
GPU: MatMul, MSE and SGD through the C ABI and through the prepared graph.

The reference leaves the reduction order, contraction and special-value behaviour of these
compounds to the backend (core/numerical/numerical.rs:21-35) and raises no arithmetic fault
for them. Where a result is fixed, these tests check it bit for bit:
- the preserved SGD (a rounded product, then a rounded subtraction);
- the contracted SGD (one fused multiply-add, checked against the C library's fma).
Where it is backend-defined, they check a rigorous error bound with the tolerance written
out: a K-term dot product in precision u is within gamma_K = K u / (1 - K u) of the exact
one, relative to sum |a||b|, whatever the order and contraction.
"""
import ctypes
import ctypes.util

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

U = {np.float32: 2.0 ** -24, np.float64: 2.0 ** -53}


@pytest.fixture(scope="module")
def ctx(pcu_pkg):
    c = pcu_pkg.Context(0)
    yield c
    c.close()


def _bits(a):
    a = np.asarray(a)
    return a.view(np.uint32 if a.dtype == np.float32 else np.uint64)


def _gamma(k, u):
    return k * u / (1.0 - k * u)


def _op(x, t):
    return x.T if t else x


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("shape", [(1, 1, 1), (65, 3, 17), (128, 256, 128), (300, 257, 130),
                                   (200, 100, 260), (512, 1024, 384),
                                   # whole tiles with one and with three slabs of 32
                                   (128, 32, 256), (256, 96, 384)])
def test_native_matmul_within_the_dot_product_bound(ctx, dtype, shape):
    m, k, n = shape
    rng = np.random.default_rng(m + 3 * k + 7 * n)
    u = U[dtype]
    for tl in (False, True):
        for tr in (False, True):
            a = rng.uniform(-1, 1, (k, m) if tl else (m, k)).astype(dtype)
            b = rng.uniform(-1, 1, (n, k) if tr else (k, n)).astype(dtype)
            got = ctx.native_matmul(ctx.upload(a), ctx.upload(b), tl, tr).numpy().astype(np.float64)
            A, B = _op(a, tl).astype(np.float64), _op(b, tr).astype(np.float64)
            exact = A @ B
            scale = np.abs(A) @ np.abs(B)
            # f32: the float64 product is exact to far below the f32 bound. f64: the
            # float64 reference carries its own gamma_K error, hence the factor 2.
            tol = _gamma(k, u) * scale * (1.0 if dtype == np.float32 else 2.0)
            assert np.all(np.abs(got - exact) <= tol), (shape, tl, tr)


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_native_matmul_specials_propagate_without_a_fault(ctx, dtype):
    rng = np.random.default_rng(5)
    a = rng.uniform(-1, 1, (64, 32)).astype(dtype)
    b = rng.uniform(-1, 1, (32, 48)).astype(dtype)
    a[3, 7] = np.nan
    b[5, 9] = np.inf
    got = ctx.native_matmul(ctx.upload(a), ctx.upload(b)).numpy()  # no PcuExecutionError
    assert np.all(np.isnan(got[3]))
    others = np.delete(np.arange(64), 3)
    assert np.all(~np.isfinite(got[others, 9]))
    clean = np.delete(np.delete(got, 3, axis=0), 9, axis=1)
    assert np.all(np.isfinite(clean))


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_native_sgd_preserved_equals_the_rounded_product_then_subtraction(ctx, dtype):
    """Fault-free inputs: the preserved native update has the strict update's values; with
    special values it simply propagates them."""
    rng = np.random.default_rng(7)
    n = (1 << 20) + 3
    w = rng.normal(0, 1, n).astype(dtype)
    g = rng.normal(0, 1e-3, n).astype(dtype)
    got = ctx.native_sgd(ctx.upload(w), ctx.upload(g), 0.01).numpy()
    ref, rf = oracle.sgd(w, g, 0.01)
    assert rf is None
    np.testing.assert_array_equal(_bits(got), _bits(ref))
    w[10], g[11] = np.inf, np.nan
    got = ctx.native_sgd(ctx.upload(w), ctx.upload(g), 0.01).numpy()
    assert np.isposinf(got[10]) and np.isnan(got[11])


def _libm_fma(dtype):
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    fn = libm.fmaf if dtype == np.float32 else libm.fma
    ct = ctypes.c_float if dtype == np.float32 else ctypes.c_double
    fn.restype = ct
    fn.argtypes = [ct, ct, ct]
    return fn


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_native_sgd_contracted_equals_one_fused_multiply_add(ctx, dtype):
    """PcuPrecisionPolicy::BackendOptimized: w' = fma(-rate, g, w) rounded once
    (backends/rocm/tensor/native_sgd/native_sgd.rs:120-145). The C library's fma is
    correctly rounded."""
    rng = np.random.default_rng(8)
    n = 4099
    w = rng.normal(0, 1, n).astype(dtype)
    g = rng.normal(0, 1, n).astype(dtype)
    rate = np.float32(0.0137)
    got = ctx.native_sgd(ctx.upload(w), ctx.upload(g), float(rate), contracted=True).numpy()
    fma = _libm_fma(dtype)
    r = dtype(rate)  # the F32 rate widens exactly for F64
    ref = np.array([fma(-float(r), float(gi), float(wi)) for wi, gi in zip(w, g)], dtype=dtype)
    np.testing.assert_array_equal(_bits(got), _bits(ref))
    # Contraction is observable: the fused result differs from the preserved one somewhere.
    pre = ctx.native_sgd(ctx.upload(w), ctx.upload(g), float(rate)).numpy()
    assert np.any(_bits(pre) != _bits(got))


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("n", [1, 5, 4097, 1 << 20, (1 << 22) + 11])
def test_native_mse_within_the_sum_bound_and_repeatable(ctx, dtype, n):
    """Squares rounded on their own, a tree sum in the declared precision, times the
    rounded reciprocal count: within (gamma_n + 2u) of the exact mean of the rounded
    squares, and the same bits on every call."""
    rng = np.random.default_rng(n)
    p = rng.uniform(-1, 1, n).astype(dtype)
    t = rng.uniform(-1, 1, n).astype(dtype)
    dp, dt = ctx.upload(p), ctx.upload(t)
    got = ctx.native_mse(dp, dt).numpy()
    again = ctx.native_mse(dp, dt).numpy()
    assert _bits(got).item() == _bits(again).item()
    d = (p - t).astype(dtype)
    sq = (d * d).astype(dtype).astype(np.float64)
    exact = np.sum(sq, dtype=np.longdouble) / n
    u = U[dtype]
    assert abs(float(got) - float(exact)) <= (_gamma(n, u) + 2 * u) * float(exact) + 1e-300


def test_native_graph_admission(ctx, pcu_pkg):
    """Prepare admits a Boundary compound only with native compound arithmetic, unspecified
    reproducibility and the IEEE underflow policy (backends/rocm/tensor.rs:9016-9058)."""
    from fusion_pcu_amd import graph as G

    def build(**opts):
        g = G.Graph()
        if opts:
            g.set_numerical_options(**opts)
        a, b = g.input((8, 4), np.float32), g.input((4, 2), np.float32)
        return g, g.matmul(a, b)

    g, out = build()
    with pytest.raises(pcu_pkg.PcuExecutionError) as e:
        g.prepare(ctx, [out])
    assert e.value.status == 4  # PCU_ERR_UNSUPPORTED: checked result-boundary MatMul
    g, out = build(native_compound=True, deterministic=True)
    with pytest.raises(pcu_pkg.PcuExecutionError):
        g.prepare(ctx, [out])
    g, out = build(native_compound=True)
    g.set_underflow_policy(out, 1)
    with pytest.raises(pcu_pkg.PcuExecutionError):
        g.prepare(ctx, [out])
    g, out = build(native_compound=True)
    prep = g.prepare(ctx, [out])
    assert prep is not None


def _mlp_reference(x, ws, y, lr):
    """The C5 training step in float64: forward, MSE, reverse mode, SGD."""
    x, y = x.astype(np.float64), y.astype(np.float64)
    w1, w2, w3 = (w.astype(np.float64) for w in ws)
    z1 = x @ w1
    h1 = np.maximum(z1, 0)
    z2 = h1 @ w2
    h2 = np.maximum(z2, 0)
    pred = h2 @ w3
    n = pred.size
    loss = np.mean((pred - y) ** 2)
    g3 = 2.0 / n * (pred - y)
    dw3 = h2.T @ g3
    g2 = (g3 @ w3.T) * (z2 > 0)
    dw2 = h1.T @ g2
    g1 = (g2 @ w2.T) * (z1 > 0)
    dw1 = x.T @ g1
    return [w1 - lr * dw1, w2 - lr * dw2, w3 - lr * dw3], loss


def test_native_mlp_training_step_tracks_float64(pcu_pkg):
    """The C5 graph captured with flag(native_compound) at reduced width: native MatMuls,
    MSE and SGD with checked elementwise nodes, within a relative tolerance of the float64
    step (the backend-defined sums differ from it by about K * 2^-24)."""
    from fusion_pcu_amd import graph as G
    from fusion_pcu_amd import synthetic as syn
    G.configure(0)
    dims, batch, lr = (96, 256, 256, 64), 128, 1e-3
    x = syn.uniform(61, (batch, dims[0]), np.float32)
    y = syn.uniform(62, (batch, dims[3]), np.float32)
    ws = [syn.xavier_uniform(63 + i, dims[i], dims[i + 1], np.float32) for i in range(3)]
    step = G.mlp_training_step(lr, native=True)
    w1, w2, w3, loss = step(x, *ws, y)
    ref_ws, ref_loss = _mlp_reference(x, ws, y, lr)
    assert abs(float(loss.numpy()) - ref_loss) <= 1e-5 * ref_loss
    for have, want in zip((w1, w2, w3), ref_ws):
        np.testing.assert_allclose(have.numpy(), want, rtol=0, atol=1e-5)


def test_native_graph_faults_come_from_checked_nodes(pcu_pkg):
    """A native MatMul raises nothing for a NaN operand; the checked ReLU that consumes its
    output does (InvalidFloatingOperand at the first non-finite element)."""
    from fusion_pcu_amd import graph as G
    G.configure(0)

    @G.function(native_compound=True)
    def fwd(x, w):
        return G.relu(G.matmul(x, w))

    x = np.ones((4, 3), np.float32)
    w = np.ones((3, 5), np.float32)
    x[2, 1] = np.nan
    with pytest.raises(pcu_pkg.PcuExecutionError) as e:
        fwd(x, w)
    f = e.value.tensor_fault
    assert int(f.kind) == 5 and f.element_index == 2 * 5
