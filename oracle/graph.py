"""TEST INFRASTRUCTURE ONLY — restatement of the reference's tensor graph semantics.

Follows (paths relative to the reference's Crates/):
  Graph::push, builders        core/dialect/tensor.rs:3588-3620, 4028-4329
  reverse mode                 core/dialect/tensor/gradients/gradients.rs:31-474
  execution plan               core/dialect/tensor.rs:3234-3300
  evaluator (first fault)      core/dialect/tensor.rs:4467-4620,
                               backends/cpu/prepared_tensor/prepared_tensor.rs:258-310
Node values are evaluated with the oracle's C ops (fast OpenMP variants, which the
oracle's own tests prove equal to the faithful integer law). Pinned by the reference's
gradient-order test (gradients/tests.rs:254-290: Uniform, Sub, Mul appended; derivative
[1, 2]), the CPU training test (backends/cpu/tests/prepared_tensor/prepared_tensor.rs:25-108)
and the README/example known answers (W -> [1.5, -1.0], loss 0.5).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import numpy as np

from . import (OP_ADD, OP_DIV, OP_MUL, OP_SUB, STEP_NONE, Fault, binary, matmul, mse, relu,
               relu_backward, sgd, u64_to_f32_bits, u64_to_f64_bits)

ELEMENTWISE = {"Add", "Sub", "Mul", "Div", "Relu"}
COMPOUND = {"MatMul", "MeanSquaredError", "SgdUpdate", "ReluBackward"}


@dataclass
class Node:
    op: str
    operands: tuple
    shape: tuple
    dtype: np.dtype
    mode: Optional[str] = None       # "Strict" / "Boundary" for compound ops
    policy: Optional[int] = None     # underflow policy when checked
    params: dict = field(default_factory=dict)
    # PcuNumericalOptions captured at append (core/dialect/tensor.rs:3612-3618):
    # (compound_arithmetic, precision, reproducibility)
    options: tuple = ("Checked", "Preserve", "Unspecified")


@dataclass
class NodeFault:
    node: int
    fault: Fault


class Graph:
    def __init__(self):
        self.nodes: List[Node] = []
        self.mode = "Boundary"
        self.options = ("Checked", "Preserve", "Unspecified")

    # -------------------------------------------------------------- builder
    def push(self, op, operands, shape, dtype, **params) -> int:
        mode = self.mode if op in COMPOUND else None
        policy = 0 if (op in ELEMENTWISE or mode is not None) else None
        self.nodes.append(Node(op, tuple(operands), tuple(shape), np.dtype(dtype), mode, policy, params,
                               self.options))
        return len(self.nodes) - 1

    def input(self, shape, dtype) -> int:
        return self.push("Input", (), shape, dtype)

    def uniform(self, shape, dtype, value) -> int:
        return self.push("Uniform", (), shape, dtype, value=np.array(value, dtype=dtype))

    def constant(self, array) -> int:
        """Graph::constant_value (core/dialect/tensor.rs:3669-3679): a dense leaf."""
        arr = np.array(array, copy=True)
        return self.push("Constant", (), arr.shape, arr.dtype, value=arr)

    def _same(self, a, b):
        if self.nodes[a].shape != self.nodes[b].shape or self.nodes[a].dtype != self.nodes[b].dtype:
            raise ValueError("ShapeMismatch")

    def binary(self, op, a, b) -> int:
        self._same(a, b)
        return self.push(op, (a, b), self.nodes[a].shape, self.nodes[a].dtype)

    def add(self, a, b): return self.binary("Add", a, b)
    def sub(self, a, b): return self.binary("Sub", a, b)
    def mul(self, a, b): return self.binary("Mul", a, b)

    def relu(self, x) -> int:
        return self.push("Relu", (x,), self.nodes[x].shape, self.nodes[x].dtype)

    def relu_backward(self, x, up) -> int:
        self._same(x, up)
        return self.push("ReluBackward", (x, up), self.nodes[x].shape, self.nodes[x].dtype)

    def matmul(self, a, b, tl=False, tr=False) -> int:
        sa, sb = self.nodes[a].shape, self.nodes[b].shape
        rows, inner = (sa[1], sa[0]) if tl else (sa[0], sa[1])
        inner_b, cols = (sb[1], sb[0]) if tr else (sb[0], sb[1])
        if inner != inner_b:
            raise ValueError("MatMulShape")
        return self.push("MatMul", (a, b), (rows, cols), self.nodes[a].dtype, tl=tl, tr=tr)

    def mean_squared_error(self, p, t) -> int:
        self._same(p, t)
        return self.push("MeanSquaredError", (p, t), (), self.nodes[p].dtype)

    def sgd_update(self, w, g, lr) -> int:
        self._same(w, g)
        return self.push("SgdUpdate", (w, g), self.nodes[w].shape, self.nodes[w].dtype,
                         lr=np.float32(lr))

    def elements(self, i) -> int:
        return int(np.prod(self.nodes[i].shape, dtype=np.int64)) if self.nodes[i].shape else 1

    # ------------------------------------------------------------- gradients
    def _scoped(self, source, fn):
        """with_source_scope (gradients.rs:448-474): the source's mode (Boundary when it has
        none), its numerical options and, where derived nodes carry one, its underflow
        policy."""
        src = self.nodes[source]
        prev, prev_options = self.mode, self.options
        self.mode = src.mode or "Boundary"
        self.options = src.options
        first = len(self.nodes)
        try:
            return fn()
        finally:
            if src.policy is not None:
                for n in self.nodes[first:]:
                    if n.policy is not None:
                        n.policy = src.policy
            self.mode, self.options = prev, prev_options

    def _scale_value(self, p):
        count = self.elements(p)
        if self.nodes[p].dtype == np.float32:
            c = np.array([u64_to_f32_bits(count)], dtype=np.uint32).view(np.float32)[0]
            return np.float32(np.float32(2.0) / c)
        c = np.array([u64_to_f64_bits(count)], dtype=np.uint64).view(np.float64)[0]
        return np.float64(2.0) / c

    def _mse_rule(self, grads, p, t, needed):
        """append_mse_gradients (gradients.rs:139-201)."""
        if not needed[p] and not needed[t]:
            return
        scale = self.uniform(self.nodes[p].shape, self.nodes[p].dtype, self._scale_value(p))
        pd = self.sub(p, t) if needed[p] else None
        td = self.sub(t, p) if needed[t] else None
        pg = self.mul(pd, scale) if pd is not None else None
        tg = self.mul(td, scale) if td is not None else None
        if pg is not None:
            self._acc(grads, p, pg)
        if tg is not None:
            self._acc(grads, t, tg)

    def _acc(self, grads, target, addition):
        """accumulate_gradient (gradients.rs:240-251)."""
        grads[target] = addition if grads[target] is None else self.add(grads[target], addition)

    def _rule(self, grads, i, g, needed):
        """append_node_gradients (gradients.rs:31-137) and append_matmul_gradients (:203-239)."""
        n = self.nodes[i]
        if n.op in ("Input", "Constant", "Uniform"):
            return
        if n.op == "Add":
            a, b = n.operands
            if needed[a]:
                self._acc(grads, a, g)
            if needed[b]:
                self._acc(grads, b, g)
        elif n.op == "Sub":
            a, b = n.operands
            if needed[a]:
                self._acc(grads, a, g)
            if needed[b]:
                neg = self.uniform(self.nodes[b].shape, self.nodes[b].dtype, -1.0)
                self._acc(grads, b, self.mul(g, neg))
        elif n.op == "Mul":
            a, b = n.operands
            lg = self.mul(g, b) if needed[a] else None
            rg = self.mul(g, a) if needed[b] else None
            if lg is not None:
                self._acc(grads, a, lg)
            if rg is not None:
                self._acc(grads, b, rg)
        elif n.op == "SgdUpdate":
            w, ug = n.operands
            ig = None
            if needed[ug]:
                rate = -np.float64(n.params["lr"])
                scaled = self.uniform(self.nodes[ug].shape, self.nodes[ug].dtype, rate)
                ig = self.mul(g, scaled)
            if needed[w]:
                self._acc(grads, w, g)
            if ig is not None:
                self._acc(grads, ug, ig)
        elif n.op == "MatMul":
            a, b = n.operands
            tl, tr = n.params["tl"], n.params["tr"]
            lg = rg = None
            if needed[a]:
                lg = self.matmul(b, g, tr, True) if tl else self.matmul(g, b, False, not tr)
            if needed[b]:
                rg = self.matmul(g, a, True, tl) if tr else self.matmul(a, g, not tl, False)
            if lg is not None:
                self._acc(grads, a, lg)
            if rg is not None:
                self._acc(grads, b, rg)
        elif n.op == "MeanSquaredError":
            self._mse_rule(grads, n.operands[0], n.operands[1], needed)
        elif n.op == "Relu":
            (x,) = n.operands
            if needed[x]:
                self._acc(grads, x, self.relu_backward(x, g))
        else:
            raise ValueError("UnsupportedGradient")

    def backward_mse(self, loss: int, targets: Optional[Sequence[int]] = None):
        """build_backward_mse (gradients.rs:281-444)."""
        if self.nodes[loss].op != "MeanSquaredError":
            raise ValueError("GradientRootNotMse")
        original = len(self.nodes)
        visited = [False] * original
        stack = [loss]
        while stack:
            i = stack.pop()
            if visited[i]:
                continue
            visited[i] = True
            if (i != loss and self.nodes[i].op == "MeanSquaredError") or \
                    self.nodes[i].op in ("Div", "ReluBackward"):
                raise ValueError("UnsupportedGradient")
            stack.extend(self.nodes[i].operands)
        if targets is not None:
            needed = [False] * original
            for t in targets:
                if not visited[t]:
                    raise ValueError("UnsupportedGradient")
                needed[t] = True
            for i in range(loss + 1):
                needed[i] = needed[i] or any(needed[o] for o in self.nodes[i].operands)
        else:
            needed = [True] * original
        grads: List[Optional[int]] = [None] * original
        if targets is not None and loss not in targets:
            p, t = self.nodes[loss].operands
            self._scoped(loss, lambda: self._mse_rule(grads, p, t, needed))
        else:
            one = self._scoped(loss, lambda: self.uniform((), self.nodes[loss].dtype, 1.0))
            grads[loss] = one
        for i in range(loss, -1, -1):
            if grads[i] is None:
                continue
            g = grads[i]
            self._scoped(i, lambda: self._rule(grads, i, g, needed))
        return grads

    def backward_mse_for_targets(self, loss, targets):
        grads = self.backward_mse(loss, list(targets))
        return [grads[t] for t in targets]

    # ----------------------------------------------------------------- plan
    def plan(self, outputs: Sequence[int]) -> List[int]:
        selected = [False] * len(self.nodes)

        def close(i):
            stack = [i]
            while stack:
                j = stack.pop()
                if selected[j]:
                    continue
                selected[j] = True
                stack.extend(self.nodes[j].operands)

        for o in outputs:
            close(o)
        for i, n in enumerate(self.nodes):
            if n.policy is not None or n.mode is not None:
                close(i)
        return [i for i, s in enumerate(selected) if s]

    # ------------------------------------------------------------- evaluate
    def evaluate(self, inputs: Dict[int, np.ndarray], outputs: Sequence[int], fast: bool = True):
        """Run the plan in order; stop at the first fault. Returns (values, NodeFault|None)."""
        vals: Dict[int, np.ndarray] = {}
        for i in self.plan(outputs):
            n = self.nodes[i]
            pol = 0 if n.policy is None else n.policy
            ops = [vals.get(o) for o in n.operands]
            if n.op == "Input":
                v, f = np.ascontiguousarray(inputs[i], dtype=n.dtype).reshape(n.shape), None
            elif n.op == "Constant":
                v, f = n.params["value"].reshape(n.shape), None
            elif n.op == "Uniform":
                v, f = np.full(n.shape, n.params["value"], dtype=n.dtype), None
            elif n.op in ("Add", "Sub", "Mul", "Div"):
                code = {"Add": OP_ADD, "Sub": OP_SUB, "Mul": OP_MUL, "Div": OP_DIV}[n.op]
                v, f = binary(code, ops[0].reshape(-1), ops[1].reshape(-1), policy=pol, fast=fast)
            elif n.op == "Relu":
                v, f = relu(ops[0].reshape(-1), policy=pol, fast=fast)
            elif n.op == "ReluBackward":
                v, f = relu_backward(ops[0].reshape(-1), ops[1].reshape(-1), policy=pol)
            elif n.op == "MatMul":
                if n.mode != "Strict":
                    raise ValueError("UnsupportedNumericalMode")
                v, f = matmul(ops[0], ops[1], n.params["tl"], n.params["tr"], policy=pol, fast=fast)
            elif n.op == "MeanSquaredError":
                if n.mode != "Strict":
                    raise ValueError("UnsupportedNumericalMode")
                v, f = mse(ops[0].reshape(-1), ops[1].reshape(-1), policy=pol, fast=fast)
            elif n.op == "SgdUpdate":
                if n.mode != "Strict":
                    raise ValueError("UnsupportedNumericalMode")
                v, f = sgd(ops[0].reshape(-1), ops[1].reshape(-1), float(n.params["lr"]),
                           policy=pol, fast=fast)
            else:
                raise ValueError(n.op)
            if f is not None:
                return vals, NodeFault(i, f)
            vals[i] = np.asarray(v).reshape(n.shape)
        return vals, None


# ------------------------------------------------------------- configurations


def c1_graph(shapes, dtype=np.float32, lr=0.01):
    """relu(X@W + b) -> MSE vs Y -> gradients (W, b) -> SGD both. Returns (graph, ids)."""
    g = Graph()
    g.mode = "Strict"
    x = g.input(shapes["x"], dtype)
    w = g.input(shapes["w"], dtype)
    b = g.input(shapes["b"], dtype)
    y = g.input(shapes["y"], dtype)
    pred = g.relu(g.add(g.matmul(x, w), b))
    loss = g.mean_squared_error(pred, y)
    gw, gb = g.backward_mse_for_targets(loss, [w, b])
    w2 = g.sgd_update(w, gw, lr)
    b2 = g.sgd_update(b, gb, lr)
    return g, {"x": x, "w": w, "b": b, "y": y, "loss": loss, "w_out": w2, "b_out": b2}


def graph_c1_step(x, w, b, y, lr=0.01, fast=True):
    g, ids = c1_graph({"x": x.shape, "w": w.shape, "b": b.shape, "y": y.shape}, x.dtype, lr)
    vals, fault = g.evaluate({ids["x"]: x, ids["w"]: w, ids["b"]: b, ids["y"]: y},
                             [ids["w_out"], ids["b_out"], ids["loss"]], fast=fast)
    if fault is not None:
        return {"fault": fault}
    return {"fault": None, "weights": vals[ids["w_out"]], "bias": vals[ids["b_out"]],
            "loss": vals[ids["loss"]]}


def mlp_graph(dims, batch, dtype=np.float32, lr=1e-3):
    """C5: X@W1 -> relu -> @W2 -> relu -> @W3 -> MSE -> gradients (W1,W2,W3) -> SGD."""
    g = Graph()
    g.mode = "Strict"
    d0, d1, d2, d3 = dims
    x = g.input((batch, d0), dtype)
    w1 = g.input((d0, d1), dtype)
    w2 = g.input((d1, d2), dtype)
    w3 = g.input((d2, d3), dtype)
    y = g.input((batch, d3), dtype)
    h1 = g.relu(g.matmul(x, w1))
    h2 = g.relu(g.matmul(h1, w2))
    pred = g.matmul(h2, w3)
    loss = g.mean_squared_error(pred, y)
    g1, g2, g3 = g.backward_mse_for_targets(loss, [w1, w2, w3])
    outs = [g.sgd_update(w1, g1, lr), g.sgd_update(w2, g2, lr), g.sgd_update(w3, g3, lr), loss]
    return g, {"x": x, "w1": w1, "w2": w2, "w3": w3, "y": y, "outputs": outs}
