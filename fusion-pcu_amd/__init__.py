"""fusion_pcu_amd — MI355X-native (gfx950) strict owned-tensor backend for Fusion PCU.

The product is ``libpcu_rocm.so`` (hand-written HIP kernels + C ABI, include/pcu_rocm.h).
This package is the host-side mirror of the reference facade for the strict path: the
error/fault vocabulary (``PcuExecutionError``, ``PcuExecutionFault``), device-resident
tensors, the op-level calls, programs with one terminal synchronization, and the graph
capture API (``pcu.matmul``, ``pcu.relu``, ``pcu.mean_squared_error``, ``pcu.gradient(s)``,
``pcu.sgd_update``) in ``fusion_pcu_amd.graph``. Every arithmetic call runs on the GPU
through the C ABI; there is no CPU fallback.
"""
from __future__ import annotations

import contextlib
import ctypes
import enum
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import numpy as np

from . import _abi

__all__ = [
    "PcuExecutionFaultKind", "TensorArithmeticStep", "PcuFloatUnderflowPolicy",
    "PcuExecutionFault", "CompoundFault", "PcuExecutionError", "Context", "DeviceArray",
    "lib", "library_path",
]


def lib():
    return _abi.load()


def library_path() -> str:
    return _abi.LIB_PATH


class PcuExecutionFaultKind(enum.IntEnum):
    """core/core.rs:25-41 (numbered as the packed fault word)."""
    DivideByZero = 1
    SignedDivisionOverflow = 2
    ArithmeticOverflow = 3
    ArithmeticUnderflow = 4
    InvalidFloatingOperand = 5


class TensorArithmeticStep(enum.IntEnum):
    """core/dialect/tensor.rs:425-430; NONE marks an elementwise ArithmeticFault."""
    NONE = 0
    Multiply = 1
    Add = 2
    Subtract = 3
    Divide = 4


class PcuFloatUnderflowPolicy(enum.IntEnum):
    """core/scalar_float_underflow.rs:47-58."""
    IeeeAfterRounding = 0
    RejectSubnormalResult = 1
    AllowGradualUnderflow = 2


@dataclass(frozen=True)
class PcuExecutionFault:
    """core/core.rs:50-66: kind + the row-major output element as invocation id."""
    kind: PcuExecutionFaultKind
    invocation_id: int
    recovered: bool = False


@dataclass(frozen=True)
class CompoundFault:
    """TensorError::{ArithmeticFault, CompoundArithmeticFault} (core/dialect/tensor.rs:
    234-252): the faulting node, output element, reduction index and step."""
    node: int
    element_index: int
    reduction_index: int
    step: TensorArithmeticStep
    kind: PcuExecutionFaultKind

    @property
    def compound(self) -> bool:
        return self.step != TensorArithmeticStep.NONE


class PcuExecutionError(Exception):
    """fusion-pcu/global.rs:195-275. ``status`` is the C ABI status; an arithmetic fault
    carries ``tensor_fault`` (the structured TensorError coordinates)."""

    def __init__(self, status: int, message: str, tensor_fault: Optional[CompoundFault] = None):
        self.status = status
        self.message = message
        self.tensor_fault = tensor_fault
        super().__init__(f"{_abi.STATUS_NAMES.get(status, status)}: {message}")

    def arithmetic_fault(self) -> Optional[PcuExecutionFault]:
        """fusion-pcu/global.rs:392-449: the element index as invocation id."""
        if self.tensor_fault is None:
            return None
        return PcuExecutionFault(self.tensor_fault.kind, self.tensor_fault.element_index, False)


_NP_DTYPE = {np.dtype(np.float32): _abi.PCU_F32, np.dtype(np.float64): _abi.PCU_F64}


def dtype_code(dtype) -> int:
    try:
        return _NP_DTYPE[np.dtype(dtype)]
    except KeyError:
        raise PcuExecutionError(_abi.PCU_ERR_UNSUPPORTED, f"unsupported scalar type {dtype}")


def _require(what: str, x: "DeviceArray", shape, dtype) -> None:
    """TensorError::ShapeMismatch / ScalarTypeMismatch before any pointer reaches the C ABI:
    the kernels take one element count and raw pointers, so a smaller or narrower buffer
    would be read or written past its end."""
    if x.shape != tuple(shape) or x.dtype != np.dtype(dtype):
        raise PcuExecutionError(
            _abi.PCU_ERR_SHAPE,
            f"ShapeMismatch: {what} is {x.shape} {x.dtype}, expected {tuple(shape)} {np.dtype(dtype)}")


def _fault_from(f: _abi.Fault) -> CompoundFault:
    return CompoundFault(int(f.node), int(f.element_index), int(f.reduction_index),
                         TensorArithmeticStep(int(f.step)), PcuExecutionFaultKind(int(f.kind)))


class DeviceArray:
    """A dense row-major device allocation owned by a Context (the resident backing of a
    PcuTensor; fusion-pcu/global/arguments.rs:636-690)."""

    def __init__(self, ctx: "Context", ptr: int, shape: Tuple[int, ...], dtype):
        self.ctx = ctx
        self.ptr = ptr
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)

    @classmethod
    def _of(cls, ctx: "Context", ptr: int, shape: Tuple[int, ...], dtype: np.dtype) -> "DeviceArray":
        """Wrap a pointer whose shape (a tuple of ints) and dtype (a numpy dtype) are already
        normalized: the per-call path of prepared programs."""
        a = cls.__new__(cls)
        a.ctx = ctx
        a.ptr = ptr
        a.shape = shape
        a.dtype = dtype
        return a

    @property
    def size(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    @property
    def nbytes(self) -> int:
        return self.size * self.dtype.itemsize

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        self.ctx.download_into(out, self)
        return out

    def free(self) -> None:
        if self.ptr:
            self.ctx.free(self)

    def __repr__(self) -> str:
        return f"DeviceArray(shape={self.shape}, dtype={self.dtype}, ptr=0x{self.ptr:x})"


class Context:
    """One pcu_ctx: a device, its ordered stream, memory pool and fault records."""

    def __init__(self, device: int = 0):
        self._lib = lib()
        handle = ctypes.c_void_p()
        st = self._lib.pcu_ctx_open(device, ctypes.byref(handle))
        if st != _abi.PCU_OK:
            raise PcuExecutionError(st, self._lib.pcu_last_error(None).decode())
        self.handle = handle
        self.device = device
        self._program_nodes = None

    # ---------------------------------------------------------------- basics
    def close(self) -> None:
        if self.handle:
            self._lib.pcu_ctx_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def error_text(self) -> str:
        return self._lib.pcu_last_error(self.handle).decode()

    def check(self, st: int, fault: Optional[_abi.Fault] = None) -> None:
        if st == _abi.PCU_OK:
            return
        if st == _abi.PCU_ARITHMETIC_FAULT and fault is not None:
            tf = _fault_from(fault)
            raise PcuExecutionError(st, f"arithmetic fault {tf}", tf)
        raise PcuExecutionError(st, self.error_text())

    def synchronize(self) -> None:
        self.check(self._lib.pcu_ctx_synchronize(self.handle))

    MATMUL_ENGINES = {"auto": 0, "valu": 1, "mfma_products": 2}

    def last_fault(self) -> Optional[CompoundFault]:
        """First fault of the most recent program or op call (pcu_fault_read), or None."""
        f = _abi.Fault()
        st = self._lib.pcu_fault_read(self.handle, ctypes.byref(f))
        if st == _abi.PCU_OK:
            return None
        if st != _abi.PCU_ARITHMETIC_FAULT:
            self.check(st)
        return _fault_from(f)

    def reset_fault(self) -> None:
        """Forget the held fault (pcu_fault_reset)."""
        self.check(self._lib.pcu_fault_reset(self.handle))

    def set_matmul_engine(self, engine: str) -> None:
        """Engine of the strict MatMul ("auto", "valu", "mfma_products"); every engine gives
        the same bits and first fault. "auto" runs small outputs (at most 256 x 256 cells for
        F32, 512 x 512 for F64) as one fused launch and larger F32 ones with matrix-core
        products; "valu" and "mfma_products" always take the screened tile kernels."""
        self.check(self._lib.pcu_ctx_set_matmul_engine(self.handle, self.MATMUL_ENGINES[engine]))

    @property
    def stream(self) -> int:
        return self._lib.pcu_ctx_stream(self.handle)

    # ---------------------------------------------------------------- memory
    def empty(self, shape: Sequence[int], dtype) -> DeviceArray:
        shape = tuple(int(s) for s in shape)
        n = int(np.prod(shape, dtype=np.int64)) if shape else 1
        p = ctypes.c_void_p()
        self.check(self._lib.pcu_buf_alloc(self.handle, n * np.dtype(dtype).itemsize, ctypes.byref(p)))
        return DeviceArray(self, p.value, shape, dtype)

    def upload(self, host: np.ndarray) -> DeviceArray:
        host = np.ascontiguousarray(host)
        dev = self.empty(host.shape, host.dtype)
        self.upload_into(dev, host)
        return dev

    def upload_into(self, dev: DeviceArray, host: np.ndarray) -> None:
        host = np.ascontiguousarray(host, dtype=dev.dtype)
        if host.nbytes != dev.nbytes:
            raise PcuExecutionError(_abi.PCU_ERR_ARGUMENT, "upload size mismatch")
        self.check(self._lib.pcu_upload(self.handle, dev.ptr, host.ctypes.data, host.nbytes))

    def download_into(self, host: np.ndarray, dev: DeviceArray) -> None:
        if not host.flags.c_contiguous or host.nbytes != dev.nbytes:
            raise PcuExecutionError(_abi.PCU_ERR_ARGUMENT, "download size mismatch")
        self.check(self._lib.pcu_download(self.handle, host.ctypes.data, dev.ptr, dev.nbytes))

    def free(self, dev: DeviceArray) -> None:
        self.check(self._lib.pcu_buf_free(self.handle, dev.ptr))
        dev.ptr = 0

    # --------------------------------------------------------------- program
    @contextlib.contextmanager
    def program(self):
        """Enqueue several ops and synchronize once; raises PcuExecutionError carrying
        the first fault in node order."""
        self.check(self._lib.pcu_program_begin(self.handle))
        ok = False
        try:
            yield self
            ok = True
        finally:
            f = _abi.Fault()
            st = self._lib.pcu_program_end(self.handle, ctypes.byref(f))
            if ok:
                self.check(st, f)

    def next_node(self) -> int:
        return int(self._lib.pcu_program_next_node(self.handle))

    def mark(self, slot: int) -> None:
        self.check(self._lib.pcu_mark(self.handle, slot))

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = ctypes.c_float()
        self.check(self._lib.pcu_elapsed_ms(self.handle, a, b, ctypes.byref(ms)))
        return float(ms.value)

    def profile(self, on: bool = True) -> None:
        """Start (and reset) or stop per-kernel HIP-event timing."""
        self.check(self._lib.pcu_profile_enable(self.handle, int(on)))

    def kernel_time(self, kernel: str) -> Tuple[float, int]:
        """(total milliseconds, launches) of one kernel since profile(True)."""
        ms = ctypes.c_double()
        n = ctypes.c_uint64()
        self.check(self._lib.pcu_profile_read(self.handle, _abi.KERNEL_IDS[kernel],
                                              ctypes.byref(ms), ctypes.byref(n)))
        return float(ms.value), int(n.value)

    def calibrate_direct_copy(self, src: "DeviceArray", dst: "DeviceArray") -> None:
        """Measurement aid: copy src into dst (same byte size, a multiple of 4 KiB) reading
        with the direct global-to-LDS load of the matrix-core MatMul tiles (see
        pcu_calibrate_direct_copy); synchronizes."""
        if src.nbytes != dst.nbytes:
            raise PcuExecutionError(_abi.PCU_ERR_SHAPE, "calibration copy: sizes differ")
        self.check(self._lib.pcu_calibrate_direct_copy(self.handle, src.ptr, dst.ptr, src.nbytes))

    # ------------------------------------------------------------------- ops
    def _call(self, fn, *args) -> None:
        f = _abi.Fault()
        st = fn(self.handle, *args, ctypes.byref(f))
        self.check(st, f)

    def strict_matmul(self, a: DeviceArray, b: DeviceArray, transpose_left=False,
                      transpose_right=False, policy=0, out: Optional[DeviceArray] = None):
        if len(a.shape) != 2 or len(b.shape) != 2 or a.dtype != b.dtype:
            raise PcuExecutionError(_abi.PCU_ERR_SHAPE, f"MatMulShape {a.shape} x {b.shape}")
        rows, inner = (a.shape[1], a.shape[0]) if transpose_left else a.shape
        inner_b, cols = (b.shape[1], b.shape[0]) if transpose_right else b.shape
        if inner != inner_b:
            raise PcuExecutionError(_abi.PCU_ERR_SHAPE, f"MatMulShape {a.shape} x {b.shape}")
        if out is None:
            out = self.empty((rows, cols), a.dtype)
        _require("out", out, (rows, cols), a.dtype)
        self._call(self._lib.pcu_strict_matmul, dtype_code(a.dtype), rows, inner, cols,
                   int(transpose_left), int(transpose_right), a.ptr, b.ptr, out.ptr, int(policy))
        return out

    def checked_binary(self, op: int, a: DeviceArray, b, policy=0, out=None):
        if isinstance(b, DeviceArray):
            _require("right", b, a.shape, a.dtype)
        if out is None:
            out = self.empty(a.shape, a.dtype)
        _require("out", out, a.shape, a.dtype)
        if isinstance(b, DeviceArray):
            self._call(self._lib.pcu_checked_binary, dtype_code(a.dtype), op, a.size, a.ptr,
                       b.ptr, out.ptr, int(policy))
        else:
            bits = int(np.array(b, dtype=a.dtype).view(np.uint32 if a.dtype == np.float32 else np.uint64))
            self._call(self._lib.pcu_checked_binary_uniform, dtype_code(a.dtype), op, a.size,
                       a.ptr, bits, out.ptr, int(policy))
        return out

    def checked_relu(self, x: DeviceArray, policy=0, out=None):
        if out is None:
            out = self.empty(x.shape, x.dtype)
        _require("out", out, x.shape, x.dtype)
        self._call(self._lib.pcu_checked_relu, dtype_code(x.dtype), x.size, x.ptr, out.ptr, int(policy))
        return out

    def checked_relu_backward(self, x: DeviceArray, up: DeviceArray, policy=0, out=None):
        _require("upstream", up, x.shape, x.dtype)
        if out is None:
            out = self.empty(x.shape, x.dtype)
        _require("out", out, x.shape, x.dtype)
        self._call(self._lib.pcu_checked_relu_backward, dtype_code(x.dtype), x.size, x.ptr,
                   up.ptr, out.ptr, int(policy))
        return out

    def checked_add_relu(self, a: DeviceArray, b: DeviceArray, policy=0, out=None):
        _require("right", b, a.shape, a.dtype)
        if out is None:
            out = self.empty(a.shape, a.dtype)
        _require("out", out, a.shape, a.dtype)
        self._call(self._lib.pcu_checked_add_relu, dtype_code(a.dtype), a.size, a.ptr, b.ptr,
                   out.ptr, int(policy))
        return out

    def strict_sgd(self, w: DeviceArray, g: DeviceArray, learning_rate: float, policy=0, out=None):
        _require("gradient", g, w.shape, w.dtype)
        if out is None:
            out = self.empty(w.shape, w.dtype)
        _require("out", out, w.shape, w.dtype)
        self._call(self._lib.pcu_strict_sgd, dtype_code(w.dtype), w.size, w.ptr, g.ptr,
                   float(np.float32(learning_rate)), out.ptr, int(policy))
        return out

    def strict_mse(self, p: DeviceArray, t: DeviceArray, policy=0, out=None):
        _require("target", t, p.shape, p.dtype)
        if out is None:
            out = self.empty((), p.dtype)
        _require("out", out, (), p.dtype)
        self._call(self._lib.pcu_strict_mse, dtype_code(p.dtype), p.size, p.ptr, t.ptr,
                   out.ptr, int(policy))
        return out

    # ------------------------------------------------ native compound arithmetic
    # Explicitly permitted native compounds (Boundary + BackendDefined): backend-defined
    # order, contraction and special values; no arithmetic fault is raised.
    def native_matmul(self, a: DeviceArray, b: DeviceArray, transpose_left=False,
                      transpose_right=False, out: Optional[DeviceArray] = None):
        if len(a.shape) != 2 or len(b.shape) != 2 or a.dtype != b.dtype:
            raise PcuExecutionError(_abi.PCU_ERR_SHAPE, f"MatMulShape {a.shape} x {b.shape}")
        rows, inner = (a.shape[1], a.shape[0]) if transpose_left else a.shape
        inner_b, cols = (b.shape[1], b.shape[0]) if transpose_right else b.shape
        if inner != inner_b:
            raise PcuExecutionError(_abi.PCU_ERR_SHAPE, f"MatMulShape {a.shape} x {b.shape}")
        if out is None:
            out = self.empty((rows, cols), a.dtype)
        _require("out", out, (rows, cols), a.dtype)
        self.check(self._lib.pcu_native_matmul(self.handle, dtype_code(a.dtype), rows, inner, cols,
                                               int(transpose_left), int(transpose_right), a.ptr,
                                               b.ptr, out.ptr))
        return out

    def native_mse(self, p: DeviceArray, t: DeviceArray, out=None):
        _require("target", t, p.shape, p.dtype)
        if out is None:
            out = self.empty((), p.dtype)
        _require("out", out, (), p.dtype)
        self.check(self._lib.pcu_native_mse(self.handle, dtype_code(p.dtype), p.size, p.ptr, t.ptr,
                                            out.ptr))
        return out

    def native_sgd(self, w: DeviceArray, g: DeviceArray, learning_rate: float, contracted=False,
                   out=None):
        _require("gradient", g, w.shape, w.dtype)
        if out is None:
            out = self.empty(w.shape, w.dtype)
        _require("out", out, w.shape, w.dtype)
        self.check(self._lib.pcu_native_sgd(self.handle, dtype_code(w.dtype), w.size, w.ptr, g.ptr,
                                            float(np.float32(learning_rate)), int(contracted),
                                            out.ptr))
        return out
