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
