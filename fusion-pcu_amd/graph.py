"""Host mirror of the reference facade's owned-tensor capture API for the strict path.

Reference surface mirrored (paths relative to the reference's Crates/):
  #[pcu(flag(strict))] functions            macros/fusion-pcu-macros.rs:1394-1396, :120-152
  pcu::{matmul, relu, relu_backward, add, sub, mul, mean_squared_error, gradient(s),
       sgd_update, identity, constant}    macros/fusion-pcu-macros/owned.rs:1616-1760
  PcuTensor (device-resident owner)        fusion-pcu/global/arguments.rs:636-690
  PcuTensor::read_into                     fusion-pcu/global/tensor.rs:1401-1450
  cold capture + warm prepared call        fusion-pcu/global/tensor.rs:1455-1489, 1761-2340

A decorated function is traced once per argument signature into a ``Graph`` (the C ABI's
pcu_graph_*), prepared on the GPU (pcu_prepare), and every later call runs that prepared
program with one terminal synchronization. Arguments are numpy arrays (host "RAM
borrows", staged to the device for the call) or ``PcuTensor`` owners (already resident);
results are fresh ``PcuTensor`` owners. Faults raise ``PcuExecutionError``.
"""
from __future__ import annotations

import ctypes
import functools
import threading
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import (CompoundFault, Context, DeviceArray, PcuExecutionError, PcuExecutionFaultKind,
               PcuFloatUnderflowPolicy, TensorArithmeticStep, _abi, dtype_code, lib)

UINT32_MAX = 0xFFFFFFFF

# ------------------------------------------------------------------ the graph


class Graph:
    """pcu_graph: append-only tensor IR (core/dialect/tensor.rs Graph)."""

    def __init__(self):
        self._lib = lib()
        h = ctypes.c_void_p()
        self._check(self._lib.pcu_graph_create(ctypes.byref(h)))
        self.handle = h

    def __del__(self):
        try:
            if self.handle:
                self._lib.pcu_graph_destroy(self.handle)
                self.handle = None
        except Exception:
            pass

    def _check(self, st: int) -> None:
        if st != _abi.PCU_OK:
            raise PcuExecutionError(st, self._lib.pcu_last_error(None).decode())

    def _id(self, fn, *args) -> int:
        out = ctypes.c_uint32()
        self._check(fn(self.handle, *args, ctypes.byref(out)))
        return int(out.value)

    @staticmethod
    def _shape(shape: Sequence[int]):
        arr = (ctypes.c_uint64 * max(1, len(shape)))(*[int(s) for s in shape])
        return len(shape), arr

    def set_numerical_mode(self, strict: bool) -> None:
        self._check(self._lib.pcu_graph_set_numerical_mode(self.handle, int(strict)))

    @staticmethod
    def _options(native_compound: bool, backend_precision: bool, deterministic: bool):
        o = _abi.NumericalOptions()
        o.compound_arithmetic = int(bool(native_compound))
        o.precision = int(bool(backend_precision))
        o.reproducibility = int(bool(deterministic))
        return o

    def set_numerical_options(self, native_compound: bool = False, backend_precision: bool = False,
                              deterministic: bool = False) -> None:
        """Graph::set_numerical_options: PcuNumericalOptions for nodes appended afterwards
        (BackendDefined / BackendOptimized / PortableV1 when the flag is set)."""
        o = self._options(native_compound, backend_precision, deterministic)
        self._check(self._lib.pcu_graph_set_numerical_options(self.handle, ctypes.byref(o)))

    def set_value_numerical_options(self, node: int, native_compound: bool = False,
                                    backend_precision: bool = False,
                                    deterministic: bool = False) -> None:
        o = self._options(native_compound, backend_precision, deterministic)
        self._check(self._lib.pcu_graph_set_value_numerical_options(self.handle, node, ctypes.byref(o)))

    def input(self, shape, dtype) -> int:
        r, s = self._shape(shape)
        return self._id(self._lib.pcu_graph_input, dtype_code(dtype), r, s)

    def uniform(self, shape, dtype, value) -> int:
        r, s = self._shape(shape)
        dt = np.dtype(dtype)
        bits = int(np.array(value, dtype=dt).view(np.uint32 if dt == np.float32 else np.uint64))
        return self._id(self._lib.pcu_graph_uniform, dtype_code(dt), r, s, bits)

    def constant(self, array) -> int:
        """Graph::constant_value (core/dialect/tensor.rs:3669-3679): the array's elements
        are copied into the graph; a prepared program uploads them once."""
        src = np.asarray(array)
        arr = np.ascontiguousarray(src).reshape(src.shape)  # keeps rank 0
        r, s = self._shape(arr.shape)
        return self._id(self._lib.pcu_graph_constant, dtype_code(arr.dtype), r, s,
                        arr.ctypes.data_as(ctypes.c_void_p))

    def binary(self, op: int, a: int, b: int) -> int:
        return self._id(self._lib.pcu_graph_binary, op, a, b)

    def add(self, a, b): return self.binary(_abi.OP_ADD, a, b)
    def sub(self, a, b): return self.binary(_abi.OP_SUB, a, b)
    def mul(self, a, b): return self.binary(_abi.OP_MUL, a, b)
    def div(self, a, b): return self.binary(_abi.OP_DIV, a, b)

    def relu(self, x: int) -> int:
        return self._id(self._lib.pcu_graph_relu, x)

    def relu_backward(self, x: int, up: int) -> int:
        return self._id(self._lib.pcu_graph_relu_backward, x, up)

    def matmul(self, a: int, b: int, transpose_left=False, transpose_right=False) -> int:
        return self._id(self._lib.pcu_graph_matmul, a, b, int(transpose_left), int(transpose_right))

    def mean_squared_error(self, p: int, t: int) -> int:
        return self._id(self._lib.pcu_graph_mean_squared_error, p, t)

    def sgd_update(self, w: int, g: int, learning_rate: float) -> int:
        return self._id(self._lib.pcu_graph_sgd_update, w, g, float(np.float32(learning_rate)))

    def set_underflow_policy(self, node: int, policy: int) -> None:
        self._check(self._lib.pcu_graph_set_underflow_policy(self.handle, node, int(policy)))

    def set_value_numerical_mode(self, node: int, strict: bool) -> None:
        self._check(self._lib.pcu_graph_set_value_numerical_mode(self.handle, node, int(strict)))

    def node_count(self) -> int:
        return int(self._lib.pcu_graph_node_count(self.handle))

    def describe(self, node: int) -> dict:
        d = _abi.NodeDesc()
        self._check(self._lib.pcu_graph_describe(self.handle, node, ctypes.byref(d)))
        return {
            "op": _abi.GRAPH_OPS[d.op],
            "left": None if d.left == UINT32_MAX else int(d.left),
            "right": None if d.right == UINT32_MAX else int(d.right),
            "transpose_left": bool(d.transpose_left),
            "transpose_right": bool(d.transpose_right),
            "dtype": np.dtype(np.float32 if d.dtype == 0 else np.float64),
            "numerical_mode": {-1: None, 0: "Boundary", 1: "Strict"}[d.numerical_mode],
            "underflow_policy": None if d.underflow_policy < 0 else int(d.underflow_policy),
            "learning_rate": float(d.learning_rate),
            "value_bits": int(d.value_bits),
            "shape": tuple(int(d.shape[k]) for k in range(d.rank)),
            "numerical_options": {
                "compound_arithmetic": ("Checked", "BackendDefined")[d.options.compound_arithmetic],
                "precision": ("Preserve", "BackendOptimized")[d.options.precision],
                "reproducibility": ("Unspecified", "PortableV1")[d.options.reproducibility],
            },
        }

    def backward_mse(self, loss: int) -> List[Optional[int]]:
        n = self.node_count()
        buf = (ctypes.c_uint32 * n)()
        self._check(self._lib.pcu_graph_backward_mse(self.handle, loss, buf, n))
        return [None if v == UINT32_MAX else int(v) for v in buf]

    def backward_mse_for_targets(self, loss: int, targets: Sequence[int]) -> List[int]:
        t = (ctypes.c_uint32 * len(targets))(*targets)
        out = (ctypes.c_uint32 * len(targets))()
        self._check(self._lib.pcu_graph_backward_mse_for_targets(self.handle, loss, len(targets), t, out))
        return [int(v) for v in out]

    def backward_mse_for(self, loss: int, target: int) -> int:
        return self.backward_mse_for_targets(loss, [target])[0]

    def plan(self, outputs: Sequence[int]) -> List[int]:
        outs = (ctypes.c_uint32 * len(outputs))(*outputs)
        n = ctypes.c_uint32(0)
        self._check(self._lib.pcu_graph_plan(self.handle, len(outputs), outs, None, ctypes.byref(n)))
        order = (ctypes.c_uint32 * max(1, n.value))()
        self._check(self._lib.pcu_graph_plan(self.handle, len(outputs), outs, order, ctypes.byref(n)))
        return [int(order[i]) for i in range(n.value)]

    def prepare(self, ctx: Context, outputs: Sequence[int]) -> "Prepared":
        return Prepared(ctx, self, outputs)


class Prepared:
    """pcu_prepared: a planned, device-allocated program run many times."""

    def __init__(self, ctx: Context, graph: Graph, outputs: Sequence[int]):
        self.ctx = ctx
        self.graph = graph
        self.outputs = list(outputs)
        self._lib = lib()
        h = ctypes.c_void_p()
        outs = (ctypes.c_uint32 * len(self.outputs))(*self.outputs)
        st = self._lib.pcu_prepare(ctx.handle, graph.handle, len(self.outputs), outs, ctypes.byref(h))
        if st != _abi.PCU_OK:
            raise PcuExecutionError(st, ctx.error_text())
        self.handle = h
        self.input_ids = []
        for i in range(self._lib.pcu_prepared_input_count(h)):
            v = ctypes.c_uint32()
            ctx.check(self._lib.pcu_prepared_input_id(h, i, ctypes.byref(v)))
            self.input_ids.append(int(v.value))
        self.output_desc = [graph.describe(o) for o in self.outputs]
        # Reused per call: the pointer array, the fault record and the outputs' shapes.
        self._ptr_arrays = {}
        self._fault = _abi.Fault()
        self._fault_ref = ctypes.byref(self._fault)
        self._out_meta = [(tuple(int(x) for x in d["shape"]), np.dtype(d["dtype"]))
                          for d in self.output_desc]
        self._take = ctypes.c_void_p()
        self._take_ref = ctypes.byref(self._take)

    def __del__(self):
        try:
            if self.handle:
                self._lib.pcu_prepared_destroy(self.handle)
                self.handle = None
        except Exception:
            pass

    def execute(self, device_ptrs: Sequence[int]) -> None:
        """Run once; on a fault raise PcuExecutionError (nothing is published)."""
        n = len(device_ptrs)
        arr = self._ptr_arrays.get(n)
        if arr is None:
            arr = self._ptr_arrays[n] = (ctypes.c_void_p * max(1, n))()
        for i, p in enumerate(device_ptrs):
            arr[i] = p
        f = self._fault
        st = self._lib.pcu_prepared_execute(self.handle, n, arr, self._fault_ref)
        if st == _abi.PCU_ARITHMETIC_FAULT:
            tf = CompoundFault(int(f.node), int(f.element_index), int(f.reduction_index),
                               TensorArithmeticStep(int(f.step)), PcuExecutionFaultKind(int(f.kind)))
            raise PcuExecutionError(st, f"arithmetic fault {tf}", tf)
        self.ctx.check(st)

    def output_ptr(self, index: int) -> int:
        return self._lib.pcu_prepared_output(self.handle, index) or 0

    def take_output(self, index: int) -> "PcuTensor":
        self.ctx.check(self._lib.pcu_prepared_take_output(self.handle, index, self._take_ref))
        shape, dtype = self._out_meta[index]
        return PcuTensor(DeviceArray._of(self.ctx, self._take.value, shape, dtype), owned=True)


# ------------------------------------------------------------ owners and values


class PcuTensor:
    """A device-resident tensor owner. Passing it to a pcu function reuses its device
    storage (no staging); ``read_into`` is the explicit device-to-host boundary."""

    def __init__(self, array: DeviceArray, owned: bool = True):
        self.array = array
        self.owned = owned

    @property
    def shape(self) -> Tuple[int, ...]:
        return self.array.shape

    @property
    def dtype(self):
        return self.array.dtype

    def read_into(self, out: np.ndarray) -> None:
        if out.shape != self.shape or out.dtype != self.dtype:
            raise PcuExecutionError(_abi.PCU_ERR_SHAPE, f"read_into: expected {self.shape} {self.dtype}")
        self.array.ctx.download_into(out, self.array)

    def numpy(self) -> np.ndarray:
        return self.array.numpy()

    @classmethod
    def from_numpy(cls, host: np.ndarray, ctx: Optional[Context] = None) -> "PcuTensor":
        return cls(( ctx or default_context()).upload(host), owned=True)

    def release(self) -> None:
        if self.owned and self.array.ptr:
            self.array.free()

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def __repr__(self) -> str:
        return f"PcuTensor(shape={self.shape}, dtype={self.dtype})"


_state = threading.local()
_default_ctx: Optional[Context] = None
_default_device = 0


def configure(device: int = 0) -> None:
    """global::configure (fusion-pcu/global.rs:706): the device later calls run on."""
    global _default_device, _default_ctx
    _default_device = device
    if _default_ctx is not None and _default_ctx.device != device:
        _default_ctx = None


def default_context() -> Context:
    global _default_ctx
    if _default_ctx is None:
        _default_ctx = Context(_default_device)
    return _default_ctx


class CaptureValue:
    """PcuTensorGraphValue (fusion-pcu/global/tensor.rs): a value inside a capture."""

    def __init__(self, cap: "_Capture", node: int, shape, dtype):
        self.cap = cap
        self.node = node
        self.shape = tuple(shape)
        self.dtype = np.dtype(dtype)

    def __add__(self, other):
        return add(self, other)

    def __sub__(self, other):
        return sub(self, other)

    def __mul__(self, other):
        return mul(self, other)


class _Capture:
    def __init__(self, strict: bool, policy: int, options: Optional[dict] = None):
        self.graph = Graph()
        self.graph.set_numerical_mode(strict)
        if options:
            self.graph.set_numerical_options(**options)
        self.policy = policy
        self.gradient_sets: Dict[int, Dict[int, int]] = {}

    def value(self, node: int) -> CaptureValue:
        d = self.graph.describe(node)
        if self.policy != PcuFloatUnderflowPolicy.IeeeAfterRounding and d["underflow_policy"] is not None:
            self.graph.set_underflow_policy(node, self.policy)
        return CaptureValue(self, node, d["shape"], d["dtype"])


def _cap() -> _Capture:
    cap = getattr(_state, "capture", None)
    if cap is None:
        raise PcuExecutionError(_abi.PCU_ERR_STATE, "pcu operations run inside a @pcu.function")
    return cap


def _v(x) -> CaptureValue:
    if isinstance(x, CaptureValue):
        if x.cap is not _cap():
            raise PcuExecutionError(_abi.PCU_ERR_ARGUMENT, "value from another capture")
        return x
    raise PcuExecutionError(_abi.PCU_ERR_ARGUMENT, f"expected a captured value, got {type(x)}")


# ----------------------------------------------------------------- pcu:: ops


def matmul(a, b, transpose_left: bool = False, transpose_right: bool = False) -> CaptureValue:
    a, b = _v(a), _v(b)
    return _cap().value(_cap().graph.matmul(a.node, b.node, transpose_left, transpose_right))


def add(a, b) -> CaptureValue:
    a, b = _v(a), _v(b)
    return _cap().value(_cap().graph.add(a.node, b.node))


def sub(a, b) -> CaptureValue:
    a, b = _v(a), _v(b)
    return _cap().value(_cap().graph.sub(a.node, b.node))


def mul(a, b) -> CaptureValue:
    a, b = _v(a), _v(b)
    return _cap().value(_cap().graph.mul(a.node, b.node))


def relu(x) -> CaptureValue:
    x = _v(x)
    return _cap().value(_cap().graph.relu(x.node))


def relu_backward(x, upstream) -> CaptureValue:
    x, upstream = _v(x), _v(upstream)
    return _cap().value(_cap().graph.relu_backward(x.node, upstream.node))


def mean_squared_error(prediction, target) -> CaptureValue:
    p, t = _v(prediction), _v(target)
    return _cap().value(_cap().graph.mean_squared_error(p.node, t.node))


def sgd_update(weights, gradient, learning_rate: float) -> CaptureValue:
    w, g = _v(weights), _v(gradient)
    return _cap().value(_cap().graph.sgd_update(w.node, g.node, learning_rate))


def gradients(loss, targets: Sequence) -> Tuple[CaptureValue, ...]:
    """pcu::gradients (fusion-pcu/global/tensor/gradient/gradient.rs:27-118): one shared
    reverse pass for the requested targets."""
    cap = _cap()
    loss = _v(loss)
    targets = [_v(t) for t in targets]
    cached = cap.gradient_sets.setdefault(loss.node, {})
    if not all(t.node in cached for t in targets):
        ids = cap.graph.backward_mse_for_targets(loss.node, [t.node for t in targets])
        for t, g in zip(targets, ids):
            cached[t.node] = g
    return tuple(CaptureValue(cap, cached[t.node], t.shape, t.dtype) for t in targets)


def gradient(loss, target) -> CaptureValue:
    """pcu::gradient (gradient.rs:124-190)."""
    return gradients(loss, [target])[0]


def identity(x) -> CaptureValue:
    return _v(x)


def constant(array) -> CaptureValue:
    """pcu::constant: a Constant graph node (OpDescriptor::Constant), uploaded once when the
    function is prepared and kept resident for every call."""
    cap = _cap()
    arr = np.asarray(array)
    node = cap.graph.constant(arr)
    return CaptureValue(cap, node, arr.shape, arr.dtype)


# ------------------------------------------------------------------ functions


class _Entry:
    def __init__(self, ctx: Context, prepared: Prepared, arg_nodes: List[int], single: bool):
        self.ctx = ctx
        self.prepared = prepared
        self.arg_nodes = arg_nodes
        self.single = single

    def call(self, args):
        staged = []
        by_node = {}
        try:
            for node, a in zip(self.arg_nodes, args):
                if isinstance(a, PcuTensor):
                    if a.array.ctx is not self.ctx:
                        raise PcuExecutionError(_abi.PCU_ERR_ARGUMENT, "tensor from another context")
                    by_node[node] = a.array.ptr
                else:
                    d = self.ctx.upload(np.ascontiguousarray(a))
                    staged.append(d)
                    by_node[node] = d.ptr
            prep = self.prepared
            prep.execute([by_node[n] for n in prep.input_ids])
            take = prep.take_output
            outs = tuple([take(i) for i in range(len(prep.outputs))])
        finally:
            for d in staged:
                d.free()
        return outs[0] if self.single else outs


def function(strict: bool = False, underflow: int = PcuFloatUnderflowPolicy.IeeeAfterRounding,
             native_compound: bool = False, backend_precision: bool = False,
             deterministic: bool = False):
    """The #[pcu] attribute: ``strict`` is flag(strict); ``underflow`` selects
    flag(ieee_underflow | reject_subnormal_result | allow_gradual_underflow); the numerical
    option flags are flag(native_compound | checked_compound), flag(backend_precision |
    preserve_precision) and flag(deterministic | non_deterministic)
    (macros/fusion-pcu-macros/numerical/numerical.rs:22-31)."""
    options = {"native_compound": native_compound, "backend_precision": backend_precision,
               "deterministic": deterministic}

    def deco(fn):
        cache: Dict[tuple, _Entry] = {}

        @functools.wraps(fn)
        def wrapper(*args):
            # The cache key: the context and each argument's shape and dtype (dtype objects,
            # not their names: formatting a dtype costs microseconds a call).
            ctx = None
            key = []
            for a in args:
                if isinstance(a, PcuTensor):
                    if ctx is None:
                        ctx = a.array.ctx
                    key.append((a.array.shape, a.array.dtype))
                else:
                    arr = a if isinstance(a, np.ndarray) else np.asarray(a)
                    key.append((arr.shape, arr.dtype))
            if ctx is None:
                ctx = default_context()
            key = (id(ctx), tuple(key))
            entry = cache.get(key)
            if entry is None:
                entry = _capture(fn, args, strict, int(underflow), ctx, options)
                cache[key] = entry
            return entry.call(args)

        wrapper.cache = cache
        return wrapper

    return deco


def _capture(fn, args, strict: bool, policy: int, ctx: Context,
             options: Optional[dict] = None) -> _Entry:
    if getattr(_state, "capture", None) is not None:
        raise PcuExecutionError(_abi.PCU_ERR_STATE, "RecursiveTensorSource")
    cap = _Capture(strict, policy, options)
    _state.capture = cap
    try:
        vals = []
        for a in args:
            shape = a.shape if isinstance(a, PcuTensor) else np.shape(a)
            dtype = a.dtype if isinstance(a, PcuTensor) else np.asarray(a).dtype
            node = cap.graph.input(shape, dtype)
            vals.append(CaptureValue(cap, node, shape, dtype))
        result = fn(*vals)
    finally:
        _state.capture = None
    single = not isinstance(result, tuple)
    results = (result,) if single else result
    outs = [_v_in(cap, r).node for r in results]
    prepared = cap.graph.prepare(ctx, outs)
    return _Entry(ctx, prepared, [v.node for v in vals], single)


def _v_in(cap, x) -> CaptureValue:
    if not isinstance(x, CaptureValue) or x.cap is not cap:
        raise PcuExecutionError(_abi.PCU_ERR_ARGUMENT, "a pcu function must return captured values")
    return x


# ------------------------------------------------------------- configurations


def c1_training_step(learning_rate: float = 0.01):
    """Config C1: relu(X@W + b) -> MSE vs Y -> gradients for (W, b) -> strict SGD on both.
    Returns (W', b', loss)."""

    @function(strict=True)
    def step(x, w, b, y):
        prediction = relu(add(matmul(x, w), b))
        loss = mean_squared_error(prediction, y)
        gw, gb = gradients(loss, (w, b))
        return sgd_update(w, gw, learning_rate), sgd_update(b, gb, learning_rate), loss

    return step


def mlp_training_step(learning_rate: float = 1e-3, native: bool = False):
    """Config C5: X@W1 -> relu -> @W2 -> relu -> @W3 -> MSE vs Y -> gradients for
    (W1, W2, W3) -> SGD (benches/tensor_mlp_train/source/source.rs:46-75).
    Returns (W1', W2', W3', loss). ``native`` captures the step in Boundary mode with
    flag(native_compound): the MatMuls, MSE and SGD updates then run as native compounds,
    while the elementwise nodes stay checked."""

    @function(strict=not native, native_compound=native)
    def step(x, w1, w2, w3, y):
        h1 = relu(matmul(x, w1))
        h2 = relu(matmul(h1, w2))
        prediction = matmul(h2, w3)
        loss = mean_squared_error(prediction, y)
        g1, g2, g3 = gradients(loss, (w1, w2, w3))
        return (sgd_update(w1, g1, learning_rate), sgd_update(w2, g2, learning_rate),
                sgd_update(w3, g3, learning_rate), loss)

    return step
