"""Pins the oracle's scalar law (oracle/checked_float.c).

Three independent anchors, so that a plausible restatement mistake fails one of them:
  1. the reference's own known-answer tests, transcribed in tests/golden/scalar_kat.json;
  2. the host's IEEE-754 unit (numpy, round-to-nearest-even, gradual underflow) for every
     non-faulting value, the reference's own randomized check
     (core/scalar_checked_float/tests.rs:305-353, f64_tests.rs:298-344);
  3. exact rational arithmetic (fractions.Fraction) for the fault classification:
     overflow, and IEEE 754-2019 7.5(a) tininess-after-rounding with inexactness.
"""
import json
import os
from fractions import Fraction

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KIND = {"Ok": 0, "DivideByZero": 1, "ArithmeticOverflow": 3, "ArithmeticUnderflow": 4,
        "InvalidFloatingOperand": 5}
POLICY = {"IeeeAfterRounding": 0, "RejectSubnormalResult": 1, "AllowGradualUnderflow": 2}


def _load(name):
    with open(os.path.join(GOLDEN, name)) as fh:
        return json.load(fh)


@pytest.mark.parametrize("case", _load("scalar_kat.json")["cases"],
                         ids=lambda c: f"{c['dtype']}-{c['op']}-{c['source']}")
def test_reference_scalar_known_answers(case):
    dtype = np.float32 if case["dtype"] == "f32" else np.float64
    operands = [int(x, 16) for x in case["operands"]]
    kind, bits = oracle.scalar(case["op"], dtype, *operands, policy=POLICY[case["policy"]])
    assert kind == KIND[case["kind"]], case
    if case["result"] is not None:
        assert bits == int(case["result"], 16), (hex(bits), case)


def test_reference_conversion_known_answers():
    conv = _load("scalar_kat.json")["conversions"]
    for n, bits in conv["u64_to_f32"]:
        assert oracle.u64_to_f32_bits(n) == int(bits, 16), n
    for n, bits in conv["u64_to_f64"]:
        assert oracle.u64_to_f64_bits(n) == int(bits, 16), n
    for src, dst in conv["f32_to_f64"]:
        assert oracle.f32_to_f64_bits(int(src, 16)) == int(dst, 16), src


def test_host_fp_environment_keeps_denormals():
    assert not oracle.host_flushes_denormals()


# ---------------------------------------------------------------- closed forms

F32_TINY_LIMIT = Fraction(2) ** -126 - Fraction(2) ** -151   # below: tiny after rounding
F64_TINY_LIMIT = Fraction(2) ** -1022 - Fraction(2) ** -1076


def _patterns(rng, n, dtype, low_exponents):
    """Random finite bit patterns; ``low_exponents`` concentrates them near the subnormal
    boundary so products and quotients land in the tiny range."""
    if dtype == np.float32:
        bits = rng.integers(0, 2 ** 32, size=n, dtype=np.uint64).astype(np.uint32)
        if low_exponents:
            exp = rng.integers(0, 90, size=n).astype(np.uint32)
            bits = (bits & np.uint32(0x807FFFFF)) | (exp << np.uint32(23))
        finite = (bits & np.uint32(0x7F800000)) != np.uint32(0x7F800000)
        return bits[finite]
    bits = rng.integers(0, 2 ** 63, size=n, dtype=np.uint64) * np.uint64(2) + \
        rng.integers(0, 2, size=n, dtype=np.uint64)
    if low_exponents:
        exp = rng.integers(0, 560, size=n).astype(np.uint64)
        bits = (bits & np.uint64(0x800FFFFFFFFFFFFF)) | (exp << np.uint64(52))
    finite = (bits & np.uint64(0x7FF0000000000000)) != np.uint64(0x7FF0000000000000)
    return bits[finite]


def _expected_kind(op, x, y, r, dtype, policy):
    """Fault kind from exact rationals: x, y finite; r the host IEEE result."""
    limit = F32_TINY_LIMIT if dtype == np.float32 else F64_TINY_LIMIT
    min_normal = float(np.finfo(dtype).tiny)
    if op == "div" and y == 0:
        return 1
    if not np.isfinite(r):
        return 3
    if op in ("add", "sub"):
        subnormal = r != 0 and abs(float(r)) < min_normal
        return 4 if policy == 1 and subnormal else 0
    if x == 0 or (op == "mul" and y == 0):
        return 0
    exact = Fraction(float(x)) * Fraction(float(y)) if op == "mul" else \
        Fraction(float(x)) / Fraction(float(y))
    tiny = abs(exact) < limit
    inexact = Fraction(float(r)) != exact
    subnormal = r != 0 and abs(float(r)) < min_normal
    if policy == 0:
        return 4 if tiny and inexact else 0
    if policy == 1:
        return 4 if subnormal or (tiny and inexact) else 0
    return 0


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("low", [False, True], ids=["wide", "near-subnormal"])
def test_scalar_law_matches_ieee_and_exact_classification(dtype, low):
    rng = np.random.default_rng(0x5EED + int(low) + (dtype == np.float64) * 7)
    a = _patterns(rng, 3000, dtype, low)
    b = _patterns(rng, 3000, dtype, low)
    m = min(len(a), len(b))
    a, b = a[:m], b[:m]
    fa = a.view(dtype)
    fb = b.view(dtype)
    with np.errstate(all="ignore"):
        host = {"add": fa + fb, "sub": fa - fb, "mul": fa * fb, "div": fa / fb}
    mismatches = []
    for op, res in host.items():
        rbits = res.view(a.dtype)
        for i in range(m):
            for policy in (0, 1, 2):
                kind, out = oracle.scalar(op, dtype, int(a[i]), int(b[i]), policy=policy)
                exp_kind = _expected_kind(op, fa[i], fb[i], res[i], dtype, policy)
                if kind != exp_kind or (kind == 0 and out != int(rbits[i])):
                    mismatches.append((op, policy, hex(int(a[i])), hex(int(b[i])), kind,
                                       exp_kind, hex(out), hex(int(rbits[i]))))
                    break
    assert not mismatches, mismatches[:10]


@pytest.mark.parametrize("dtype", [np.float32, np.float64], ids=["f32", "f64"])
def test_relu_neg_relu_backward_closed_forms(dtype):
    rng = np.random.default_rng(7)
    x = _patterns(rng, 2000, dtype, True)
    u = _patterns(rng, 2000, dtype, False)
    m = min(len(x), len(u))
    sign = np.uint64(1 << 63) if dtype == np.float64 else np.uint32(1 << 31)
    for i in range(m):
        xv, uv = int(x[i]), int(u[i])
        fx = x[i:i + 1].view(dtype)[0]
        k, r = oracle.scalar("relu", dtype, xv, policy=2)
        assert k == 0 and r == (xv if fx > 0 else 0)
        k, r = oracle.scalar("neg", dtype, xv, policy=2)
        assert k == 0 and r == xv ^ int(sign)
        k, r = oracle.scalar("relu_backward", dtype, xv, uv, policy=2)
        assert k == 0 and r == (uv if fx > 0 else 0)
