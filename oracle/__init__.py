"""TEST INFRASTRUCTURE ONLY — Python face of the CPU oracle.

Loads ``oracle/liboracle.so`` (a C restatement of the reference's integer-significand
checked arithmetic and ordered strict compounds; see ``oracle/oracle.h``) and the graph
restatement in ``oracle/graph.py``. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the checker or
as the reported CPU baseline. The product path never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

OK, DIVIDE_BY_ZERO, SIGNED_DIVISION_OVERFLOW, OVERFLOW, UNDERFLOW, INVALID = range(6)
KIND_NAMES = {
    0: "Ok",
    1: "DivideByZero",
    2: "SignedDivisionOverflow",
    3: "ArithmeticOverflow",
    4: "ArithmeticUnderflow",
    5: "InvalidFloatingOperand",
}
POLICY_IEEE, POLICY_REJECT_SUBNORMAL, POLICY_ALLOW_GRADUAL = 0, 1, 2
STEP_NONE, STEP_MULTIPLY, STEP_ADD, STEP_SUBTRACT, STEP_DIVIDE = range(5)
OP_ADD, OP_SUB, OP_MUL, OP_DIV = range(4)


class _CFault(ctypes.Structure):
    _fields_ = [
        ("element_index", ctypes.c_uint64),
        ("reduction_index", ctypes.c_uint64),
        ("step", ctypes.c_int32),
        ("kind", ctypes.c_int32),
    ]


@dataclass(frozen=True)
class Fault:
    """First fault of one op: TensorError::{ArithmeticFault, CompoundArithmeticFault}
    coordinates (core/dialect/tensor.rs:234-252)."""

    element_index: int
    reduction_index: int
    step: int
    kind: int


def build() -> None:
    """Compile liboracle.so with the committed Makefile (this container only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L) -> None:
    u32, u64, i32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int
    sz, vp = ctypes.c_size_t, ctypes.c_void_p
    fp = ctypes.POINTER(_CFault)
    for name in ("add", "sub", "mul", "div"):
        f = getattr(L, f"orc_{name}_f32")
        f.argtypes = [u32, u32, i32, ctypes.POINTER(u32)]
        f.restype = i32
        f = getattr(L, f"orc_{name}_f64")
        f.argtypes = [u64, u64, i32, ctypes.POINTER(u64)]
        f.restype = i32
    for name in ("neg", "relu"):
        f = getattr(L, f"orc_{name}_f32")
        f.argtypes = [u32, i32, ctypes.POINTER(u32)]
        f.restype = i32
        f = getattr(L, f"orc_{name}_f64")
        f.argtypes = [u64, i32, ctypes.POINTER(u64)]
        f.restype = i32
    L.orc_relu_backward_f32.argtypes = [u32, u32, i32, ctypes.POINTER(u32)]
    L.orc_relu_backward_f32.restype = i32
    L.orc_relu_backward_f64.argtypes = [u64, u64, i32, ctypes.POINTER(u64)]
    L.orc_relu_backward_f64.restype = i32
    L.orc_u64_to_f32_rne.argtypes = [u64]
    L.orc_u64_to_f32_rne.restype = u32
    L.orc_u64_to_f64_rne.argtypes = [u64]
    L.orc_u64_to_f64_rne.restype = u64
    L.orc_f32_to_f64_bits.argtypes = [u32]
    L.orc_f32_to_f64_bits.restype = u64
    L.orc_binary.argtypes = [i32, i32, sz, vp, vp, i32, vp, i32, fp]
    L.orc_relu.argtypes = [i32, sz, vp, vp, i32, fp]
    L.orc_relu_backward.argtypes = [i32, sz, vp, vp, vp, i32, fp]
    L.orc_sgd.argtypes = [i32, sz, vp, vp, u32, vp, i32, fp]
    L.orc_mse.argtypes = [i32, sz, vp, vp, vp, i32, fp]
    L.orc_matmul.argtypes = [i32, sz, sz, sz, i32, i32, vp, vp, vp, i32, sz, sz, fp]
    L.orc_fast_matmul.argtypes = [i32, sz, sz, sz, i32, i32, vp, vp, vp, i32, i32, fp]
    L.orc_fast_binary.argtypes = [i32, i32, sz, vp, vp, i32, vp, i32, i32, fp]
    L.orc_fast_relu.argtypes = [i32, sz, vp, vp, i32, i32, fp]
    L.orc_fast_sgd.argtypes = [i32, sz, vp, vp, u32, vp, i32, i32, fp]
    L.orc_fast_mse.argtypes = [i32, sz, vp, vp, vp, i32, i32, fp]
    for f in (L.orc_binary, L.orc_relu, L.orc_relu_backward, L.orc_sgd, L.orc_mse,
              L.orc_matmul, L.orc_fast_matmul, L.orc_fast_binary, L.orc_fast_relu,
              L.orc_fast_sgd, L.orc_fast_mse):
        f.restype = i32
    L.orc_host_flushes_denormals.argtypes = []
    L.orc_host_flushes_denormals.restype = i32


# ----------------------------------------------------------------- scalar law


def _dt(dtype) -> int:
    return 0 if np.dtype(dtype) == np.float32 else 1


def scalar(op: str, dtype, *operands_bits: int, policy: int = POLICY_IEEE):
    """One checked scalar op on raw bit patterns: returns (kind, result_bits)."""
    d = _dt(dtype)
    suffix = "f32" if d == 0 else "f64"
    ctype = ctypes.c_uint32 if d == 0 else ctypes.c_uint64
    out = ctype(0)
    fn = getattr(lib(), f"orc_{op}_{suffix}")
    kind = fn(*operands_bits, policy, ctypes.byref(out))
    return kind, out.value


def u64_to_f32_bits(v: int) -> int:
    return lib().orc_u64_to_f32_rne(v)


def u64_to_f64_bits(v: int) -> int:
    return lib().orc_u64_to_f64_rne(v)


def f32_to_f64_bits(v: int) -> int:
    return lib().orc_f32_to_f64_bits(v)


# ------------------------------------------------------------------ tensor ops


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _fault(rc: int, cf: _CFault) -> Optional[Fault]:
    if rc < 0:
        raise MemoryError("oracle allocation failed")
    if rc == 0:
        return None
    return Fault(int(cf.element_index), int(cf.reduction_index), int(cf.step), int(cf.kind))


def _threads(threads: Optional[int]) -> int:
    return 0 if threads is None else int(threads)


def binary(op: int, a: np.ndarray, b, policy=POLICY_IEEE, fast=True, threads=None):
    """Checked elementwise Add/Sub/Mul/Div; ``b`` may be a 0-d/1-element broadcast scalar."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(np.asarray(b, dtype=a.dtype))
    b_scalar = int(b.size == 1 and a.size != 1)
    out = np.empty_like(a)
    cf = _CFault()
    if fast:
        rc = lib().orc_fast_binary(_dt(a.dtype), op, a.size, _ptr(a), _ptr(b), b_scalar,
                                   _ptr(out), policy, _threads(threads), ctypes.byref(cf))
    else:
        rc = lib().orc_binary(_dt(a.dtype), op, a.size, _ptr(a), _ptr(b), b_scalar, _ptr(out),
                              policy, ctypes.byref(cf))
    return out, _fault(rc, cf)


def relu(x: np.ndarray, policy=POLICY_IEEE, fast=True, threads=None):
    x = np.ascontiguousarray(x)
    out = np.empty_like(x)
    cf = _CFault()
    if fast:
        rc = lib().orc_fast_relu(_dt(x.dtype), x.size, _ptr(x), _ptr(out), policy,
                                 _threads(threads), ctypes.byref(cf))
    else:
        rc = lib().orc_relu(_dt(x.dtype), x.size, _ptr(x), _ptr(out), policy, ctypes.byref(cf))
    return out, _fault(rc, cf)


def relu_backward(x: np.ndarray, up: np.ndarray, policy=POLICY_IEEE):
    x = np.ascontiguousarray(x)
    up = np.ascontiguousarray(up)
    out = np.empty_like(x)
    cf = _CFault()
    rc = lib().orc_relu_backward(_dt(x.dtype), x.size, _ptr(x), _ptr(up), _ptr(out), policy,
                                 ctypes.byref(cf))
    return out, _fault(rc, cf)


def sgd(w: np.ndarray, g: np.ndarray, rate: float, policy=POLICY_IEEE, fast=True,
        threads=None):
    """Strict SGD with an F32 rate (widened exactly for F64)."""
    w = np.ascontiguousarray(w)
    g = np.ascontiguousarray(g)
    out = np.empty_like(w)
    rate_bits = int(np.array(rate, dtype=np.float32).view(np.uint32))
    cf = _CFault()
    if fast:
        rc = lib().orc_fast_sgd(_dt(w.dtype), w.size, _ptr(w), _ptr(g), rate_bits, _ptr(out),
                                policy, _threads(threads), ctypes.byref(cf))
    else:
        rc = lib().orc_sgd(_dt(w.dtype), w.size, _ptr(w), _ptr(g), rate_bits, _ptr(out),
                           policy, ctypes.byref(cf))
    return out, _fault(rc, cf)


def mse(p: np.ndarray, t: np.ndarray, policy=POLICY_IEEE, fast=True, threads=None):
    p = np.ascontiguousarray(p)
    t = np.ascontiguousarray(t)
    out = np.zeros((), dtype=p.dtype)
    cf = _CFault()
    if fast:
        rc = lib().orc_fast_mse(_dt(p.dtype), p.size, _ptr(p), _ptr(t), _ptr(out), policy,
                                _threads(threads), ctypes.byref(cf))
    else:
        rc = lib().orc_mse(_dt(p.dtype), p.size, _ptr(p), _ptr(t), _ptr(out), policy,
                           ctypes.byref(cf))
    return out, _fault(rc, cf)


def matmul_shape(a_shape, b_shape, tl: bool, tr: bool):
    rows, inner = (a_shape[1], a_shape[0]) if tl else (a_shape[0], a_shape[1])
    inner_b, cols = (b_shape[1], b_shape[0]) if tr else (b_shape[0], b_shape[1])
    if inner != inner_b:
        raise ValueError(f"matmul shape mismatch {a_shape} x {b_shape} ({tl}, {tr})")
    return rows, inner, cols


def matmul(a: np.ndarray, b: np.ndarray, tl=False, tr=False, policy=POLICY_IEEE, fast=True,
           threads=None, rows_subset=None):
    """Strict ordered MatMul of op(a) @ op(b). ``rows_subset=(r0, r1)`` computes only those
    output rows with the faithful routine (used to time the faithful CPU baseline)."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    rows, inner, cols = matmul_shape(a.shape, b.shape, tl, tr)
    out = np.zeros((rows, cols), dtype=a.dtype)
    cf = _CFault()
    d = _dt(a.dtype)
    if fast and rows_subset is None:
        rc = lib().orc_fast_matmul(d, rows, inner, cols, int(tl), int(tr), _ptr(a), _ptr(b),
                                   _ptr(out), policy, _threads(threads), ctypes.byref(cf))
    else:
        r0, r1 = rows_subset if rows_subset is not None else (0, rows)
        rc = lib().orc_matmul(d, rows, inner, cols, int(tl), int(tr), _ptr(a), _ptr(b),
                              _ptr(out), policy, r0, r1, ctypes.byref(cf))
    return out, _fault(rc, cf)


def host_flushes_denormals() -> bool:
    return bool(lib().orc_host_flushes_denormals())


from .graph import graph_c1_step  # noqa: E402  (graph.py imports the ops above)
