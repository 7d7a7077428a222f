"""pcu_strict_matmul_noalloc (the strict MatMul whose screen scratch is the library's fixed
per-device array) against pcu_strict_matmul, both through the C ABI: the same bits and the
same first fault on consecutive calls, the second with a smaller input, and a refusal
beyond PCU_NOALLOC_MAX_DIM."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx(pcu_pkg):
    c = pcu_pkg.Context(0)
    yield c
    c.close()


def _bits(a):
    a = np.asarray(a)
    return a.view(np.uint32 if a.dtype == np.float32 else np.uint64)


def _call(ctx, entry, a, b, tl, tr, policy, rows, inner, cols):
    """One call of `entry` on fresh device copies; returns (status, output bits, fault)."""
    from fusion_pcu_amd import _abi
    from fusion_pcu_amd import dtype_code
    da, db = ctx.upload(a), ctx.upload(b)
    out = ctx.empty((rows, cols), a.dtype)
    f = _abi.Fault()
    st = entry(ctx.handle, dtype_code(a.dtype), rows, inner, cols, int(tl), int(tr), da.ptr, db.ptr,
               out.ptr, policy, ctypes.byref(f))
    got = out.numpy() if st == _abi.PCU_OK else None
    fault = (f.element_index, f.reduction_index, f.step, f.kind) if st == _abi.PCU_ARITHMETIC_FAULT else None
    for x in (da, db, out):
        x.free()
    return st, got, fault


CASES = [  # (rows, inner, cols, transposes, dtype, policy, planted special or None)
    (1000, 300, 700, (False, False), np.float32, 0, None),
    (129, 67, 255, (True, False), np.float32, 1, None),
    (300, 257, 130, (False, True), np.float64, 0, None),
    (65, 3, 17, (True, True), np.float64, 2, None),
    (512, 128, 384, (False, False), np.float32, 0, ("a", 7777, np.nan)),
    (200, 90, 100, (False, False), np.float32, 0, ("b", 4321, 1e-30)),
    (96, 40, 33, (True, False), np.float64, 0, ("a", 99, np.inf)),
    # Full F32 grids with op(B) transposed: the allocating entry point copies op(B) out as
    # K x N for its tile kernel, the no-allocation one reads B in place.
    (2048, 48, 2048, (False, True), np.float32, 0, ("b", 50000, np.inf)),
    (2048, 64, 2048, (True, True), np.float32, 1, None),
]


@pytest.mark.parametrize("engine", ["auto", "valu"])
def test_noalloc_matches_the_allocating_entry_point(ctx, pcu_pkg, engine):
    lib = pcu_pkg.lib()
    ctx.set_matmul_engine(engine)
    rng = np.random.default_rng(5)
    try:
        # Consecutive calls with shapes that shrink and grow, so each call's screen words sit
        # over words the previous call left in the shared array.
        for rows, inner, cols, (tl, tr), dtype, policy, special in CASES:
            a = rng.uniform(-1, 1, (inner, rows) if tl else (rows, inner)).astype(dtype)
            b = rng.uniform(-1, 1, (cols, inner) if tr else (inner, cols)).astype(dtype)
            if special is not None:
                which, idx, val = special
                (a if which == "a" else b).reshape(-1)[idx] = val
            ref = _call(ctx, lib.pcu_strict_matmul, a, b, tl, tr, policy, rows, inner, cols)
            got = _call(ctx, lib.pcu_strict_matmul_noalloc, a, b, tl, tr, policy, rows, inner, cols)
            assert got[0] == ref[0], (rows, inner, cols, got[0], ref[0])
            assert got[2] == ref[2], (rows, inner, cols, got[2], ref[2])
            if ref[1] is not None:
                np.testing.assert_array_equal(_bits(got[1]), _bits(ref[1]))
    finally:
        ctx.set_matmul_engine("auto")


def test_noalloc_two_calls_second_smaller(ctx, pcu_pkg):
    """Two calls in a row, the second with a smaller input: the smaller call must not see
    the larger call's screen words."""
    lib = pcu_pkg.lib()
    rng = np.random.default_rng(6)
    big_a = rng.uniform(-1, 1, (2048, 512)).astype(np.float32)
    big_b = rng.uniform(-1, 1, (512, 1536)).astype(np.float32)
    big_a[:, 3] = np.float32(2.0 ** -110)  # every row suspect; some products tiny and inexact
    small_a = rng.uniform(-1, 1, (100, 64)).astype(np.float32)
    small_b = rng.uniform(-1, 1, (64, 90)).astype(np.float32)
    for a, b in ((big_a, big_b), (small_a, small_b)):
        rows, inner, cols = a.shape[0], a.shape[1], b.shape[1]
        ref = _call(ctx, lib.pcu_strict_matmul, a, b, False, False, 0, rows, inner, cols)
        got = _call(ctx, lib.pcu_strict_matmul_noalloc, a, b, False, False, 0, rows, inner, cols)
        assert got[0] == ref[0] and got[2] == ref[2], (got[0], got[2], ref[0], ref[2])
        if ref[1] is not None:
            np.testing.assert_array_equal(_bits(got[1]), _bits(ref[1]))


def test_noalloc_refuses_shapes_beyond_its_scratch(ctx, pcu_pkg):
    from fusion_pcu_amd import _abi
    lib = pcu_pkg.lib()
    rows = 65537
    a = ctx.empty((rows, 1), np.float32)
    b = ctx.empty((1, 1), np.float32)
    out = ctx.empty((rows, 1), np.float32)
    f = _abi.Fault()
    st = lib.pcu_strict_matmul_noalloc(ctx.handle, 0, rows, 1, 1, 0, 0, a.ptr, b.ptr, out.ptr, 0,
                                       ctypes.byref(f))
    assert st == _abi.PCU_ERR_ARGUMENT
    assert "65536" in ctx.error_text()
    st = lib.pcu_strict_matmul_noalloc(ctx.handle, 0, 1, 1, rows, 0, 0, b.ptr, a.ptr, out.ptr, 0,
                                       ctypes.byref(f))
    assert st == _abi.PCU_ERR_ARGUMENT
    for x in (a, b, out):
        x.free()


def test_noalloc_allocates_nothing(pcu_pkg):
    """A fresh context whose only MatMuls are no-allocation calls, a full F32 grid with op(B)
    transposed among them (where the allocating entry point keeps a K x N copy of op(B)):
    the device memory pool's used bytes, current and high-water, do not move across the
    calls, so neither the screen scratch nor the copy of op(B) is allocated."""
    from fusion_pcu_amd import _abi
    from fusion_pcu_amd import dtype_code
    lib = pcu_pkg.lib()
    hip = ctypes.CDLL("libamdhip64.so")
    used_current, used_high = 7, 8  # hipMemPoolAttrUsedMemCurrent, hipMemPoolAttrUsedMemHigh
    pool = ctypes.c_void_p()
    assert hip.hipDeviceGetDefaultMemPool(ctypes.byref(pool), 0) == 0

    def pool_bytes(attr):
        v = ctypes.c_uint64()
        assert hip.hipMemPoolGetAttribute(pool, attr, ctypes.byref(v)) == 0
        return v.value

    rng = np.random.default_rng(8)
    shapes = [(2048, 48, 2048, (False, True), np.float32, 0),
              (1000, 300, 700, (False, False), np.float32, 1),
              (300, 257, 130, (False, True), np.float64, 0),
              (1024, 64, 1024, (True, False), np.float32, 0)]
    with pcu_pkg.Context(0) as c:
        calls, bufs = [], []
        for rows, inner, cols, (tl, tr), dtype, policy in shapes:
            a = rng.uniform(-1, 1, (inner, rows) if tl else (rows, inner)).astype(dtype)
            b = rng.uniform(-1, 1, (cols, inner) if tr else (inner, cols)).astype(dtype)
            da, db, out = c.upload(a), c.upload(b), c.empty((rows, cols), dtype)
            bufs += [da, db, out]
            calls.append((dtype_code(dtype), rows, inner, cols, int(tl), int(tr), da.ptr, db.ptr,
                          out.ptr, policy))
        c.synchronize()
        assert hip.hipDeviceSynchronize() == 0
        used0 = pool_bytes(used_current)
        zero = ctypes.c_uint64(0)
        high_reset = hip.hipMemPoolSetAttribute(pool, used_high, ctypes.byref(zero)) == 0
        f = _abi.Fault()
        for _ in range(2):
            for args in calls:
                st = lib.pcu_strict_matmul_noalloc(c.handle, *args, ctypes.byref(f))
                assert st == _abi.PCU_OK, (args[1:4], st, c.error_text())
        c.synchronize()
        assert hip.hipDeviceSynchronize() == 0
        assert pool_bytes(used_current) == used0
        if high_reset:  # reset to the current usage (or to 0): no allocation rose above it
            assert pool_bytes(used_high) <= used0
        for x in bufs:
            x.free()
