"""The matrix-core product engine of the strict F32 MatMul, pinned on the device.

The default F32 engine forms every product with v_mfma_f32_32x32x1_2b_f32 (K = 1, +0
accumulator) and folds it into the ordered sum with a separate v_add_f32. Its parity rests
on a hardware property: each MFMA element is the product rounded once to nearest-even,
with subnormal inputs and results kept, equal to v_mul_f32 except that an exact zero
product comes out +0 (which no accumulator starting from +0 can show). These tests
publish about 16.8 M products straight from the engine (K = 1: C = +0 + a*b, and K = 2:
C = (+0 + a0*b0) + a1*b1) over 4096 x 4096 outputs and compare every bit with the CPU
oracle and with the vector engine, under all three underflow policies.

Operand pools (4 segments of 1024 per side, so the outer product meets every pair):
  ties       (1 + j 2^-12) 2^e: products 1 + (i+j) 2^-12 + ij 2^-24, an exact
             round-to-nearest tie whenever ij is odd and no carry moves the binade
  wide       random significands, exponents over most of the range (no overflow)
  near       exponents around -63 on both sides: products straddle 2^-126 and fill
             the subnormal range, many of them inexact
  subnormal  subnormal A entries (and signed zeros) against B entries up to 2^61
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

N = 4096
SEG = N // 4


@pytest.fixture(scope="module")
def ctx(pcu_pkg):
    c = pcu_pkg.Context(0)
    yield c
    c.set_matmul_engine("auto")
    c.close()


def _bits(a):
    return np.asarray(a).view(np.uint32)


def _f32(sign, exp, frac):
    """Normal binary32 values from unbiased exponents and 23-bit fractions."""
    b = (sign.astype(np.uint32) << np.uint32(31)) | ((exp + 127).astype(np.uint32) << np.uint32(23)) \
        | frac.astype(np.uint32)
    return b.view(np.float32)


def _pool(rng, side):
    sign = lambda n: rng.integers(0, 2, n)
    frac = lambda n: rng.integers(0, 1 << 23, n)
    j = rng.integers(1, 4096, SEG)
    ties = _f32(sign(SEG), rng.integers(-40, 41, SEG), j << 11)  # 1 + j 2^-12
    if side == "a":
        wide = _f32(sign(SEG), rng.integers(-100, 61, SEG), frac(SEG))
        near = _f32(sign(SEG), rng.integers(-70, -55, SEG), frac(SEG))
        sub = (rng.integers(1, 1 << 23, SEG).astype(np.uint32)
               | (sign(SEG).astype(np.uint32) << np.uint32(31))).view(np.float32)
        sub[rng.random(SEG) < 0.1] = np.float32(0.0)
        sub[rng.random(SEG) < 0.05] = np.float32(-0.0)
        last = sub
    else:
        wide = _f32(sign(SEG), rng.integers(-70, 61, SEG), frac(SEG))
        near = _f32(sign(SEG), rng.integers(-70, -55, SEG), frac(SEG))
        big = _f32(sign(SEG), rng.integers(40, 61, SEG), frac(SEG))
        big[rng.random(SEG) < 0.1] = np.float32(-0.0)
        last = big
    return np.concatenate([ties, wide, near, last])


def _operands(seed, k):
    rng = np.random.default_rng(seed)
    a = np.stack([rng.permutation(_pool(rng, "a")) if c else _pool(rng, "a") for c in range(k)], 1)
    b = np.stack([rng.permutation(_pool(rng, "b")) if r else _pool(rng, "b") for r in range(k)], 0)
    return np.ascontiguousarray(a), np.ascontiguousarray(b)


def _run(ctx, pcu_pkg, a, b, policy, engine):
    ctx.set_matmul_engine(engine)
    da, db = ctx.upload(a), ctx.upload(b)
    try:
        out = ctx.strict_matmul(da, db, False, False, policy)
        got = out.numpy()
        out.free()
        return got, None
    except pcu_pkg.PcuExecutionError as e:
        f = e.tensor_fault
        return None, (f.element_index, f.reduction_index, int(f.step), int(f.kind))
    finally:
        da.free()
        db.free()


def _of(f):
    return None if f is None else (f.element_index, f.reduction_index, f.step, f.kind)


@pytest.mark.parametrize("k", [1, 2])
@pytest.mark.parametrize("policy", [2, 0, 1], ids=["allow_gradual", "ieee", "reject_subnormal"])
def test_mfma_products_bit_exact_over_constructed_operands(ctx, pcu_pkg, k, policy):
    a, b = _operands(1000 + k, k)
    ref, rf = oracle.matmul(a, b, policy=policy)
    results = {}
    for engine in ("mfma_products", "valu"):
        got, gf = _run(ctx, pcu_pkg, a, b, policy, engine)
        assert gf == _of(rf), (engine, gf, rf)
        if rf is None:
            np.testing.assert_array_equal(_bits(got), _bits(ref), err_msg=engine)
        results[engine] = got
    if policy == 2:
        # The sweep really reaches the cases it is meant for (AllowGradual publishes all).
        p = np.abs(ref.astype(np.float64))
        tiny = np.finfo(np.float32).tiny
        assert np.count_nonzero((p > 0) & (p < tiny)) > 200_000           # subnormal results
        assert np.count_nonzero((p >= tiny) & (p < 4 * tiny)) > 20_000    # just above 2^-126
        assert np.count_nonzero(ref == 0) > 100_000                       # exact or rounded zeros
        assert np.array_equal(_bits(results["mfma_products"]), _bits(results["valu"]))
    if k == 1 and policy == 2:
        # Round-to-nearest ties are among the products (ties segment times ties segment):
        # the exact binary64 product lies halfway between two binary32 neighbours.
        ex = (a[:SEG, 0].astype(np.float64)[:, None] * b[0, :SEG].astype(np.float64)[None, :])
        lo = ex.astype(np.float32)
        up = np.nextafter(lo, np.float32(np.inf) * np.sign(lo))
        mid = (lo.astype(np.float64) + up.astype(np.float64)) / 2
        assert np.count_nonzero(mid == ex) > 50_000


@pytest.mark.parametrize("k", [1, 2])
def test_mfma_products_fault_coordinates(ctx, pcu_pkg, k):
    """Overflowing and non-finite operands in the same sweep: both engines report the
    oracle's first (cell, k, step, kind) under every policy."""
    a, b = _operands(2000 + k, k)
    rng = np.random.default_rng(31 + k)
    cases = [
        ("overflow", lambda a, b: (a.__setitem__((1500, k - 1), np.float32(3.0e38)),
                                   b.__setitem__((k - 1, 2000), np.float32(2.0e10)))),
        ("nan", lambda a, b: b.__setitem__((0, int(rng.integers(N))), np.float32(np.nan))),
        ("inf", lambda a, b: a.__setitem__((int(rng.integers(N)), 0), np.float32(-np.inf))),
    ]
    for name, plant in cases:
        aa, bb = a.copy(), b.copy()
        plant(aa, bb)
        for policy in (0, 1, 2):
            ref, rf = oracle.matmul(aa, bb, policy=policy)
            assert rf is not None
            for engine in ("mfma_products", "valu"):
                _, gf = _run(ctx, pcu_pkg, aa, bb, policy, engine)
                assert gf == _of(rf), (name, policy, engine, gf, rf)


# ------------------------------------------------- the four-block 16 x 16 product form
# Outputs of fewer 128 x 128 tiles than CUs made of at most 512 whole 64 x 64 tiles, with K a
# multiple of 16 (C2's 1024^3 among them), go to k_strict_gemm_mfma16, which forms its
# products with v_mfma_f32_16x16x1_4b_f32: four blocks of 16 x 16 products, one k each
# (k0 .. k0 + 3), published straight from the matrix core. 1024 x K x 1024 with K = 16 or
# 32 is such a shape (64 tiles of 128 x 128, 256 of 64 x 64).
M16 = 1024
LAYOUTS = [(False, False), (False, True), (True, False), (True, True)]
LAYOUT_IDS = ["nn", "nt", "tn", "tt"]


def _stored(a, b, ta, tb):
    """The stored operands of a layout: op(A) = a, op(B) = b."""
    return (np.ascontiguousarray(a.T) if ta else a), (np.ascontiguousarray(b.T) if tb else b)


def _run_layout(ctx, pcu_pkg, a, b, policy, engine, ta, tb):
    ctx.set_matmul_engine(engine)
    sa, sb = _stored(a, b, ta, tb)
    da, db = ctx.upload(sa), ctx.upload(sb)
    try:
        out = ctx.strict_matmul(da, db, ta, tb, policy)
        got = out.numpy()
        out.free()
        return got, None
    except pcu_pkg.PcuExecutionError as e:
        f = e.tensor_fault
        return None, (f.element_index, f.reduction_index, int(f.step), int(f.kind))
    finally:
        da.free()
        db.free()


@pytest.fixture(scope="module")
def pools():
    rng = np.random.default_rng(4242)
    return _pool(rng, "a"), _pool(rng, "b")


def _single_products(pools, i, j, k, seed):
    """op(A) (M16 x k) whose row r holds one nonzero, A-pool segment i's value r, at k = r % k;
    op(B) (k x M16) whose every row is a permutation of B-pool segment j. Cell (r, c) is
    then ((+0 + 0 b) + ...) + a_r B[r % k, c] + ...: the one product rounded once (zero
    products leave a +0 or nonzero sum unchanged), so every A value of segment i meets every
    B value of segment j, and every block of every MFMA (k0 .. k0 + 3 for each k0) publishes
    products. The 16 (i, j) segment pairs meet all 4096 x 4096 pool pairs."""
    pa, pb = pools
    rng = np.random.default_rng(seed)
    a = np.zeros((M16, k), np.float32)
    a[np.arange(M16), np.arange(M16) % k] = rng.permutation(pa[i * SEG:(i + 1) * SEG])
    b = np.stack([rng.permutation(pb[j * SEG:(j + 1) * SEG]) for _ in range(k)])
    return a, b


@pytest.mark.parametrize("k", [16, 32])
def test_mfma16_single_products_bit_exact(ctx, pcu_pkg, pools, k):
    """Every pool pair once, as a published single product, in all four layouts and both
    engines under AllowGradual; the first fault under IEEE and RejectSubnormal."""
    tiny = np.finfo(np.float32).tiny
    n_sub = n_ties = 0
    for i in range(4):
        for j in range(4):
            a, b = _single_products(pools, i, j, k, 100 * k + 4 * i + j)
            for policy in (2, 0, 1):
                ref, rf = oracle.matmul(a, b, policy=policy)
                layouts = LAYOUTS if policy == 2 else LAYOUTS[:1]
                for ta, tb in layouts:
                    for engine in ("mfma_products", "valu"):
                        got, gf = _run_layout(ctx, pcu_pkg, a, b, policy, engine, ta, tb)
                        assert gf == _of(rf), (i, j, policy, ta, tb, engine, gf, rf)
                        if rf is None:
                            np.testing.assert_array_equal(
                                _bits(got), _bits(ref), err_msg=f"{i}{j} {ta}{tb} {engine}")
                if policy == 2:
                    p = np.abs(ref.astype(np.float64))
                    n_sub += np.count_nonzero((p > 0) & (p < tiny))
                    if i == 0 and j == 0:
                        # ties x ties: exact binary64 products halfway between two floats
                        nz = a[np.arange(M16), np.arange(M16) % k].astype(np.float64)
                        ex = nz[:, None] * b[np.arange(M16) % k].astype(np.float64)
                        lo = ex.astype(np.float32)
                        up = np.nextafter(lo, np.float32(np.inf) * np.sign(lo))
                        mid = (lo.astype(np.float64) + up.astype(np.float64)) / 2
                        n_ties += np.count_nonzero(mid == ex)
    # The sweep reaches the cases it is meant for.
    assert n_sub > 200_000
    assert n_ties > 50_000


def _dense(pools, k, seed):
    """Dense op(A) (M16 x k) and op(B) (k x M16) from the pools: column c of A and row r of
    B are permutations of a pool's first M16 entries of a random segment mix."""
    pa, pb = pools
    rng = np.random.default_rng(seed)
    a = np.stack([rng.permutation(pa)[:M16] for _ in range(k)], 1)
    b = np.stack([rng.permutation(pb)[:M16] for _ in range(k)], 0)
    return np.ascontiguousarray(a), np.ascontiguousarray(b)


@pytest.mark.parametrize("k", [16, 48, 80])
def test_mfma16_dense_sums_bit_exact(ctx, pcu_pkg, pools, k):
    """Dense reductions over one, three and five slabs (the three-stage rotation and its
    tail): every output bit and first fault against the oracle, all layouts and policies."""
    a, b = _dense(pools, k, 7000 + k)
    for policy in (2, 0, 1):
        ref, rf = oracle.matmul(a, b, policy=policy)
        for ta, tb in LAYOUTS:
            for engine in ("mfma_products", "valu"):
                got, gf = _run_layout(ctx, pcu_pkg, a, b, policy, engine, ta, tb)
                assert gf == _of(rf), (policy, ta, tb, engine, gf, rf)
                if rf is None:
                    np.testing.assert_array_equal(_bits(got), _bits(ref), err_msg=f"{ta}{tb} {engine}")


@pytest.mark.parametrize("layout", LAYOUTS, ids=LAYOUT_IDS)
def test_mfma16_fault_coordinates(ctx, pcu_pkg, pools, layout):
    """Overflowing and non-finite operands planted in the dense K = 16 sweep: both engines
    report the oracle's first (cell, k, step, kind) under every policy."""
    ta, tb = layout
    a, b = _dense(pools, 16, 8016)
    rng = np.random.default_rng(77)
    cases = [
        ("overflow", lambda a, b: (a.__setitem__((700, 9), np.float32(3.0e38)),
                                   b.__setitem__((9, 300), np.float32(2.0e10)))),
        ("nan", lambda a, b: b.__setitem__((int(rng.integers(16)), int(rng.integers(M16))),
                                           np.float32(np.nan))),
        ("inf", lambda a, b: a.__setitem__((int(rng.integers(M16)), int(rng.integers(16))),
                                           np.float32(-np.inf))),
    ]
    for name, plant in cases:
        aa, bb = a.copy(), b.copy()
        plant(aa, bb)
        for policy in (0, 1, 2):
            _, rf = oracle.matmul(aa, bb, policy=policy)
            assert rf is not None
            for engine in ("mfma_products", "valu"):
                _, gf = _run_layout(ctx, pcu_pkg, aa, bb, policy, engine, ta, tb)
                assert gf == _of(rf), (name, policy, engine, gf, rf)
