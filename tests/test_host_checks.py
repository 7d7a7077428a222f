"""Host-side argument checks of the op-level Python face (no GPU needed): every call
rejects a second operand or an out= buffer whose shape or scalar type differs from what the
op writes, with PcuExecutionError(PCU_ERR_SHAPE), before any pointer reaches the C ABI
(the reference returns TensorError::ShapeMismatch for these: core/dialect/tensor.rs
:4067-4110)."""
import numpy as np
import pytest


class _NoCalls:
    """Stands in for the loaded library: any C ABI call fails the test."""

    def __getattr__(self, name):
        raise AssertionError(f"{name} reached the C ABI")


@pytest.fixture()
def ctx(pcu_pkg):
    c = object.__new__(pcu_pkg.Context)
    c._lib = _NoCalls()
    c.handle = None
    c.device = 0
    return c


def _arr(pcu_pkg, ctx, shape, dtype=np.float32):
    return pcu_pkg.DeviceArray(ctx, 0x10000, shape, dtype)


CASES = [
    # (call, operands built from (shape, dtype) pairs, keyword out)
    ("strict_sgd", [((64,), np.float32), ((32,), np.float32)], None),
    ("strict_sgd", [((64,), np.float32), ((64,), np.float64)], None),
    ("strict_sgd", [((64,), np.float32), ((64,), np.float32)], ((63,), np.float32)),
    ("strict_mse", [((8, 8), np.float32), ((8, 7), np.float32)], None),
    ("strict_mse", [((8, 8), np.float32), ((8, 8), np.float32)], ((1,), np.float64)),
    ("checked_relu", [((5, 5), np.float64)], ((5, 5), np.float32)),
    ("checked_relu_backward", [((5, 5), np.float32), ((25,), np.float32)], None),
    ("checked_relu_backward", [((5, 5), np.float32), ((5, 5), np.float32)], ((5, 4), np.float32)),
    ("checked_add_relu", [((4, 4), np.float32), ((4, 2), np.float32)], None),
    ("checked_add_relu", [((4, 4), np.float32), ((4, 4), np.float32)], ((4, 4), np.float64)),
    ("strict_matmul", [((4, 3), np.float32), ((3, 5), np.float32)], ((4, 4), np.float32)),
    ("strict_matmul", [((4, 3), np.float64), ((3, 5), np.float64)], ((4, 5), np.float32)),
    ("native_matmul", [((4, 3), np.float32), ((3, 5), np.float32)], ((5, 4), np.float32)),
    ("native_mse", [((16,), np.float32), ((15,), np.float32)], None),
    ("native_sgd", [((16,), np.float32), ((16,), np.float32)], ((8,), np.float32)),
]


@pytest.mark.parametrize("name,operands,out", CASES,
                         ids=[f"{c[0]}-{i}" for i, c in enumerate(CASES)])
def test_mismatched_operand_or_out_is_rejected_before_the_abi(pcu_pkg, ctx, name, operands, out):
    args = [_arr(pcu_pkg, ctx, s, d) for s, d in operands]
    if name in ("strict_sgd", "native_sgd"):
        args.append(0.01)
    kw = {} if out is None else {"out": _arr(pcu_pkg, ctx, *out)}
    with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
        getattr(ctx, name)(*args, **kw)
    assert exc.value.status == 3  # PCU_ERR_SHAPE


@pytest.mark.parametrize("op", [0, 1, 2, 3])
def test_binary_rejects_mismatches(pcu_pkg, ctx, op):
    a = _arr(pcu_pkg, ctx, (6, 6))
    for b in (_arr(pcu_pkg, ctx, (36,)), _arr(pcu_pkg, ctx, (6, 6), np.float64)):
        with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
            ctx.checked_binary(op, a, b)
        assert exc.value.status == 3
    with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
        ctx.checked_binary(op, a, _arr(pcu_pkg, ctx, (6, 6)), out=_arr(pcu_pkg, ctx, (6, 5)))
    assert exc.value.status == 3
    with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
        ctx.checked_binary(op, a, 2.0, out=_arr(pcu_pkg, ctx, (6, 6), np.float64))
    assert exc.value.status == 3


def test_matmul_shape_rules(pcu_pkg, ctx):
    a = _arr(pcu_pkg, ctx, (4, 3))
    with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
        ctx.strict_matmul(a, _arr(pcu_pkg, ctx, (4, 5)))
    assert exc.value.status == 3
    with pytest.raises(pcu_pkg.PcuExecutionError) as exc:
        ctx.strict_matmul(a, _arr(pcu_pkg, ctx, (3, 5), np.float64))
    assert exc.value.status == 3
