"""RejectSubnormal on the screened tile kernels, against the oracle.

Under RejectSubnormalResult (core/scalar_float_underflow.rs:61-73) a nonzero subnormal
partial sum faults as well as a tiny product. A product of at least 2^-103 (2^-970 for
binary64) is a multiple of the smallest normal, and rounded sums of such multiples stay
multiples, so only a cell that meets a smaller product can have a subnormal partial sum. The
tile kernels check every partial sum of a tile whose row and column exponents allow such a
product, mark the cells of each lane that met a subnormal sum, and flag their 32 x 32
blocks; the replay walks only those cells (and the tiny scan's candidates for products).

Each case plants, in zeroed rows of op(A), a pair of products that cancel to a subnormal
partial sum at a chosen k (and, in some, tiny products elsewhere), on shapes that reach each
tile kernel: the 128 x 128 matrix-core tile (whole, three stages), the 16 x 16-wave tile,
the 64 x 64 tile with bound checks, the vector-unit binary32 tile and the binary64 tile.
Every output bit and first fault is compared with the oracle under all three policies.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx(pcu_pkg):
    c = pcu_pkg.Context(0)
    yield c
    c.set_matmul_engine("auto")
    c.close()


def _bits(a):
    a = np.asarray(a)
    return a.view(np.uint32 if a.dtype == np.float32 else np.uint64)


def _run(ctx, pcu_pkg, a, b, tl, tr, policy):
    da, db = ctx.upload(a), ctx.upload(b)
    try:
        out = ctx.strict_matmul(da, db, tl, tr, policy)
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


def _plant_cancellation(a, b, r, c, k1, k2, dtype):
    """Row r of op(A) zero but for k1 and k2; cell (r, c)'s products there are
    2^e (1 + ulp) and -2^e, so its partial sum at k2 is 2^e ulp: subnormal. The row's other
    cells get 2^e (1 + ulp) b1 - 2^e b2 for their own column entries, normal in general."""
    f32 = dtype == np.float32
    e, ulp = (-104, 2.0 ** -23) if f32 else (-971, 2.0 ** -52)
    a[r, :] = 0
    a[r, k1] = dtype(2.0 ** e * (1 + ulp))
    a[r, k2] = dtype(-(2.0 ** e))
    b[k1, c] = b[k2, c] = dtype(1.0)


SHAPES = [  # (M, K, N, dtype, engine): the tile kernel each reaches
    (2048, 64, 2048, np.float32, "mfma_products"),   # 128 x 128 whole tiles, three stages
    (1024, 48, 1024, np.float32, "mfma_products"),   # 16 x 16 waves, whole 64 x 64 tiles
    (1000, 40, 700, np.float32, "mfma_products"),    # 64 x 64 tiles with bound checks
    (512, 64, 640, np.float32, "valu"),              # vector-unit binary32
    (2048, 32, 2048, np.float64, "valu"),            # binary64 8 x 8 block, full grid
]
IDS = ["mfma128", "mfma16", "mfma64-ragged", "valu-f32", "valu-f64"]


@pytest.mark.parametrize("shape", SHAPES, ids=IDS)
def test_reject_subnormal_partial_sums(ctx, pcu_pkg, shape):
    m, k, n, dtype, engine = shape
    ctx.set_matmul_engine(engine)
    rng = np.random.default_rng(m + k + n)
    f32 = dtype == np.float32
    cases = []
    # (1) one subnormal partial sum, first slab to last slab
    for k1, k2 in ((0, 3), (5, k // 2), (1, k - 1)):
        a = rng.uniform(-1, 1, (m, k)).astype(dtype)
        b = rng.uniform(-1, 1, (k, n)).astype(dtype)
        r, c = int(rng.integers(m)), int(rng.integers(n))
        _plant_cancellation(a, b, r, c, k1, k2, dtype)
        cases.append((f"sum-at-k{k2}", a, b))
    # (2) two planted cells: the later row's pair cancels in an earlier k; plus a tiny
    #     product (subnormal under every policy's screen) in a third row after both
    a = rng.uniform(-1, 1, (m, k)).astype(dtype)
    b = rng.uniform(-1, 1, (k, n)).astype(dtype)
    r1, r2 = sorted(int(x) for x in rng.choice(m - 1, 2, replace=False))
    _plant_cancellation(a, b, r1, n - 1, 2, k - 2, dtype)
    _plant_cancellation(a, b, r2, 0, 1, 4, dtype)
    a[m - 1, 7] = dtype(2.0 ** (-140 if f32 else -1060))
    cases.append(("two-cells-and-tiny", a, b))
    # (3) a tiny product in a cell before the subnormal sum's cell
    a = rng.uniform(-1, 1, (m, k)).astype(dtype)
    b = rng.uniform(-1, 1, (k, n)).astype(dtype)
    _plant_cancellation(a, b, m // 2, n // 2, 3, 9, dtype)
    a[m // 4, k - 1] = dtype(3 * 2.0 ** (-140 if f32 else -1060))  # a subnormal operand
    cases.append(("tiny-before-sum", a, b))
    # (4) every cell marked (one tiny column of op(A)), no fault under RejectSubnormal
    a = rng.uniform(-1, 1, (m, k)).astype(dtype)
    b = rng.uniform(-1, 1, (k, n)).astype(dtype)
    sign = np.where(rng.random(m) < 0.5, -1.0, 1.0)
    a[:, 0] = (2.0 ** (-120 if f32 else -1000) * sign).astype(dtype)
    b[0, :] = (rng.uniform(0.5, 1.0, n) * np.where(rng.random(n) < 0.5, -1.0, 1.0)).astype(dtype)
    cases.append(("all-marked-clean", a, b))
    try:
        for name, a, b in cases:
            for tl, tr in ((False, False), (True, False), (False, True)):
                aa = np.ascontiguousarray(a.T) if tl else a
                bb = np.ascontiguousarray(b.T) if tr else b
                for policy in (1, 0, 2):
                    ref, rf = oracle.matmul(aa, bb, tl, tr, policy=policy)
                    if name.startswith("sum-at") and policy == 1:
                        assert rf is not None and rf.step == 2, (name, rf)  # an Add faults
                    if name == "all-marked-clean" and policy == 1:
                        assert rf is None
                    got, gf = _run(ctx, pcu_pkg, aa, bb, tl, tr, policy)
                    assert gf == _of(rf), (name, tl, tr, policy, gf, rf)
                    if rf is None:
                        np.testing.assert_array_equal(_bits(got), _bits(ref),
                                                      err_msg=f"{name} {tl}{tr} {policy}")
    finally:
        ctx.set_matmul_engine("auto")


def test_reject_subnormal_after_calls_of_other_shapes(pcu_pkg):
    """A fresh context runs RejectSubnormal MatMuls of smaller shapes (each filling its
    superslab tables and partial-sum block words), then the planted 2048 x 32 x 2048 case,
    whose scratch reuses those bytes for its generation-tagged words: the first fault must
    still be the oracle's. (With the tables kept in the MatMul scratch, their bits outranked
    the new generation under atomicMax and the planted fault went unseen.)"""
    with pcu_pkg.Context(0) as c:
        rng = np.random.default_rng(99)
        for (m, k, n) in ((2048, 64, 2048), (1024, 48, 1024), (1000, 40, 700), (512, 64, 640)):
            a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
            b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
            a[:, 0] = np.float32(2.0 ** -120)  # every tile marked: tables and block words written
            for policy in (1, 0):
                ref, rf = oracle.matmul(a, b, policy=policy)
                got, gf = _run(c, pcu_pkg, a, b, False, False, policy)
                assert gf == _of(rf), ((m, k, n), policy, gf, rf)
        for dtype in (np.float32, np.float64):
            for engine in ("valu", "mfma_products"):
                c.set_matmul_engine(engine)
                a = rng.uniform(-1, 1, (2048, 32)).astype(dtype)
                b = rng.uniform(-1, 1, (32, 2048)).astype(dtype)
                _plant_cancellation(a, b, 1500, 77, 0, 3, dtype)
                _, rf = oracle.matmul(a, b, policy=1)
                assert rf is not None and rf.step == 2
                _, gf = _run(c, pcu_pkg, a, b, False, False, 1)
                assert gf == _of(rf), (dtype, engine, gf, rf)


DEEP = [  # (M, K, N, dtype, engine): the same tile kernels over four superslabs of 64 k
    (2048, 256, 2048, np.float32, "mfma_products"),
    (1024, 256, 1024, np.float32, "mfma_products"),
    (1000, 200, 700, np.float32, "mfma_products"),
    (512, 256, 640, np.float32, "valu"),
    (2048, 256, 2048, np.float64, "valu"),
]


def _plant_carried(a, b, r, c, kc, dtype, fault):
    """Row r of op(A) zero but for k = 3 and k = kc (superslab 2): cell (r, c) first adds
    the largest value below 2^-103 (binary64 2^-970), a product below that bound and so not
    a multiple of the smallest normal; superslab 1 adds nothing; at kc it adds -2^-103
    (2^-970), a product at the bound, which leaves the subnormal -2^-127 (-2^-1023) when
    `fault`, or -2^-102 (-2^-969), which leaves a normal sum. op(B)'s superslab 2 is kept in
    +-[1, 2), so no product there is below the bound: the check reaches kc only because the
    partial sum entering superslabs 1 and 2 is off the grid of multiples."""
    f32 = dtype == np.float32
    bound, eps = (2.0 ** -103, 2.0 ** -24) if f32 else (2.0 ** -970, 2.0 ** -53)
    rng = np.random.default_rng(r + c + kc)
    k = b.shape[0]
    hi = min(192, k)
    b[128:hi, :] = (rng.uniform(1.0, 2.0, (hi - 128, b.shape[1]))
                    * np.where(rng.random((hi - 128, b.shape[1])) < 0.5, -1.0, 1.0)).astype(dtype)
    a[r, :] = 0
    a[r, 3] = dtype(bound * (1 - eps))
    a[r, kc] = dtype(-bound if fault else -2 * bound)
    b[3, c] = b[kc, c] = dtype(1.0)


@pytest.mark.parametrize("shape", DEEP, ids=IDS)
def test_reject_subnormal_across_superslabs(ctx, pcu_pkg, shape):
    """The checking tiles check a superslab when a product in it may fall below 2^-103, or
    when a partial sum entering it is off the grid of multiples of the smallest normal: a
    subnormal sum formed from an off-grid sum carried across superslabs with no small
    product, a cancellation in the last superslabs, and a carried sum that stays normal."""
    m, k, n, dtype, engine = shape
    ctx.set_matmul_engine(engine)
    rng = np.random.default_rng(7 * m + k + n)
    cases = []
    for name, fault in (("carried-subnormal", True), ("carried-normal", False)):
        a = rng.uniform(-1, 1, (m, k)).astype(dtype)
        b = rng.uniform(-1, 1, (k, n)).astype(dtype)
        _plant_carried(a, b, int(rng.integers(m)), int(rng.integers(n)), 150, dtype, fault)
        cases.append((name, a, b))
    a = rng.uniform(-1, 1, (m, k)).astype(dtype)
    b = rng.uniform(-1, 1, (k, n)).astype(dtype)
    _plant_cancellation(a, b, int(rng.integers(m)), int(rng.integers(n)), k - 50, k - 3, dtype)
    cases.append(("late-cancellation", a, b))
    try:
        for name, a, b in cases:
            for tl, tr in ((False, False), (True, False), (False, True)):
                aa = np.ascontiguousarray(a.T) if tl else a
                bb = np.ascontiguousarray(b.T) if tr else b
                for policy in (1, 0):
                    ref, rf = oracle.matmul(aa, bb, tl, tr, policy=policy)
                    if policy == 1 and name != "carried-normal":
                        assert rf is not None and rf.step == 2 and rf.kind == 4, (name, rf)
                    if name == "carried-subnormal" and policy == 1:
                        assert rf.reduction_index == 150, rf
                    got, gf = _run(ctx, pcu_pkg, aa, bb, tl, tr, policy)
                    assert gf == _of(rf), (name, tl, tr, policy, gf, rf)
                    if rf is None:
                        np.testing.assert_array_equal(_bits(got), _bits(ref),
                                                      err_msg=f"{name} {tl}{tr} {policy}")
    finally:
        ctx.set_matmul_engine("auto")


@pytest.mark.parametrize("shape", DEEP, ids=IDS)
def test_tiny_products_through_superslab_tables(ctx, pcu_pkg, shape):
    """The tiny scan reads only the 64-k superslabs whose table minima allow a tiny product
    (under IEEE and RejectSubnormal): an inexact tiny product planted in the first, a middle
    or the last superslab, some behind an exact tiny product of the same cell in an earlier
    superslab, under every transpose pair, against the oracle."""
    m, k, n, dtype, engine = shape
    ctx.set_matmul_engine(engine)
    f32 = dtype == np.float32
    half, ulp = (2.0 ** -70, 2.0 ** -23) if f32 else (2.0 ** -530, 2.0 ** -52)
    rng = np.random.default_rng(11 * m + k + n)
    cases = []
    for k_exact, k_inexact in ((None, 5), (3, k // 2 + 7), (70, k - 2)):
        a = rng.uniform(-1, 1, (m, k)).astype(dtype)
        b = rng.uniform(-1, 1, (k, n)).astype(dtype)
        r, c = int(rng.integers(m)), int(rng.integers(n))
        if k_exact is not None:
            a[r, k_exact] = dtype(half)  # half * half is an exact subnormal: no fault
            b[k_exact, c] = dtype(half)
        a[r, k_inexact] = dtype(half * (1 + ulp))  # half^2 (1 + ulp): tiny and inexact
        b[k_inexact, c] = dtype(half)
        cases.append((f"inexact-at-k{k_inexact}", a, b))
    try:
        for name, a, b in cases:
            for tl, tr in ((False, False), (True, False), (False, True)):
                aa = np.ascontiguousarray(a.T) if tl else a
                bb = np.ascontiguousarray(b.T) if tr else b
                for policy in (0, 1):
                    ref, rf = oracle.matmul(aa, bb, tl, tr, policy=policy)
                    if policy == 0:
                        assert rf is not None and rf.kind == 4, (name, rf)
                    got, gf = _run(ctx, pcu_pkg, aa, bb, tl, tr, policy)
                    assert gf == _of(rf), (name, tl, tr, policy, gf, rf)
    finally:
        ctx.set_matmul_engine("auto")


FUZZ_FAMILIES = [  # (M, N, K choices, dtype, engine): each reaches one tile kernel
    (2048, 2048, (64, 144, 256), np.float32, "mfma_products"),  # whole 128 x 128, three stages
    (2100, 2000, (48, 200), np.float32, "mfma_products"),       # 128 x 128 with bound checks
    (1024, 1024, (112, 256), np.float32, "mfma_products"),      # 16 x 16 waves, 64 x 64 tiles
    (1000, 700, (40, 177), np.float32, "mfma_products"),        # 64 x 64 with bound checks
    (640, 520, (96, 250), np.float32, "valu"),                  # vector-unit binary32
    (2048, 2048, (80, 192), np.float64, "valu"),                # binary64 full grid
]
FUZZ_IDS = ["mfma128", "mfma128-ragged", "mfma16", "mfma64-ragged", "valu-f32", "valu-f64"]


@pytest.mark.parametrize("family", FUZZ_FAMILIES, ids=FUZZ_IDS)
def test_reject_subnormal_gating_fuzz(ctx, pcu_pkg, family):
    """Seeded fuzz of the superslab-gated partial-sum check: per case one to three planted
    cancellations at random k (either side of a superslab boundary), sometimes an off-grid
    sum carried into a later superslab, and random tiny operands, under RejectSubnormal
    (and IEEE for every other case), in random transpose pairs; bits and first fault
    against the oracle."""
    m, n, ks, dtype, engine = family
    ctx.set_matmul_engine(engine)
    f32 = dtype == np.float32
    rng = np.random.default_rng(1000 + m + n + len(ks))
    try:
        for case in range(8):
            k = int(ks[case % len(ks)])
            a = rng.uniform(-1, 1, (m, k)).astype(dtype)
            b = rng.uniform(-1, 1, (k, n)).astype(dtype)
            if k >= 192 and rng.random() < 0.5:
                _plant_carried(a, b, int(rng.integers(m)), int(rng.integers(n)), 150, dtype,
                               bool(rng.random() < 0.5))
            for _ in range(int(rng.integers(1, 4))):
                k1 = int(rng.integers(0, k - 1))
                k2 = int(rng.integers(k1 + 1, k))
                _plant_cancellation(a, b, int(rng.integers(m)), int(rng.integers(n)), k1, k2, dtype)
            for _ in range(int(rng.integers(0, 3))):
                e = int(rng.integers(-150, -100)) if f32 else int(rng.integers(-1070, -960))
                a[int(rng.integers(m)), int(rng.integers(k))] = dtype(2.0 ** e * rng.uniform(1, 2))
            tl, tr = bool(rng.random() < 0.4), bool(rng.random() < 0.4)
            aa = np.ascontiguousarray(a.T) if tl else a
            bb = np.ascontiguousarray(b.T) if tr else b
            for policy in ((1, 0) if case % 2 else (1,)):
                ref, rf = oracle.matmul(aa, bb, tl, tr, policy=policy)
                got, gf = _run(ctx, pcu_pkg, aa, bb, tl, tr, policy)
                assert gf == _of(rf), (case, k, tl, tr, policy, gf, rf)
                if rf is None:
                    np.testing.assert_array_equal(_bits(got), _bits(ref),
                                                  err_msg=f"case {case} k {k} {tl}{tr} {policy}")
    finally:
        ctx.set_matmul_engine("auto")
