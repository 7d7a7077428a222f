"""Writes tests/golden/scalar_kat.json and tests/golden/tensor_kat.json.

Every case below is transcribed by hand from the reference's own known-answer tests
(file:line cited per group, relative to the reference's Crates/); no reference code is
imported or run. Values are stored as hex bit patterns so the fixtures are exact.
Run: python tests/golden/make_scalar_kat.py
"""
import json
import math
import os
import struct

HERE = os.path.dirname(os.path.abspath(__file__))

OK, DIV0, OVF, UNF, INV = "Ok", "DivideByZero", "ArithmeticOverflow", "ArithmeticUnderflow", "InvalidFloatingOperand"
IEEE, REJECT, ALLOW = "IeeeAfterRounding", "RejectSubnormalResult", "AllowGradualUnderflow"


def f32(x: float) -> str:
    return "0x%08x" % struct.unpack("<I", struct.pack("<f", x))[0]


def f64(x: float) -> str:
    return "0x%016x" % struct.unpack("<Q", struct.pack("<d", x))[0]


def h32(b: int) -> str:
    return "0x%08x" % b


def h64(b: int) -> str:
    return "0x%016x" % b


F32_MAX = 0x7F7FFFFF
F32_MIN_NORMAL = 0x00800000
F64_MAX = 0x7FEFFFFFFFFFFFFF
F64_MIN_NORMAL = 0x0010000000000000

cases = []


def case(src, dtype, op, operands, policy, kind, result=None):
    cases.append({"source": src, "dtype": dtype, "op": op, "operands": operands,
                  "policy": policy, "kind": kind, "result": result})


# core/scalar_checked_float/tests.rs:9-24 rejects_non_finite_inputs_by_bits
for bits in (0x7F800000, 0xFF800000, 0x7F800001, 0xFFC12345):
    for op in ("add", "sub", "mul"):
        case("scalar_checked_float/tests.rs:9-24", "f32", op, [h32(bits), f32(1.0)], IEEE, INV)

# tests.rs:27-66 relu patterns
for bits in (0x00000000, 0x80000000, 0x00000001, 0x007FFFFF, 0x00800000, 0x3F800000,
             0x7F7FFFFF, 0x80000001, 0xBF800000, 0xFF7FFFFF):
    expected = 0 if (bits & 0x80000000) or (bits & 0x7FFFFFFF) == 0 else bits
    case("scalar_checked_float/tests.rs:27-51", "f32", "relu", [h32(bits)], IEEE, OK, h32(expected))
for bits in (0x7F800000, 0xFF800000, 0x7F800001, 0xFFC12345):
    case("scalar_checked_float/tests.rs:52-57", "f32", "relu", [h32(bits)], IEEE, INV)
case("scalar_checked_float/tests.rs:58-62", "f32", "relu", [h32(1)], REJECT, UNF)
case("scalar_checked_float/tests.rs:63-66", "f32", "relu", [h32(1)], ALLOW, OK, h32(1))

# tests.rs:69-87 finite results and overflow
case("scalar_checked_float/tests.rs:71", "f32", "add", [f32(1.5), f32(2.25)], IEEE, OK, f32(3.75))
case("scalar_checked_float/tests.rs:72", "f32", "sub", [f32(1.5), f32(2.25)], IEEE, OK, f32(-0.75))
case("scalar_checked_float/tests.rs:73", "f32", "mul", [f32(1.5), f32(2.25)], IEEE, OK, f32(3.375))
case("scalar_checked_float/tests.rs:74", "f32", "div", [f32(7.5), f32(2.5)], IEEE, OK, f32(3.0))
case("scalar_checked_float/tests.rs:77-80", "f32", "mul", [h32(F32_MAX), f32(2.0)], IEEE, OVF)
case("scalar_checked_float/tests.rs:81-84", "f32", "add", [h32(F32_MAX), h32(F32_MAX)], IEEE, OVF)

# tests.rs:89-146 division of subnormals (AllowGradualUnderflow unless stated)
case("scalar_checked_float/tests.rs:92-99", "f32", "div", [h32(1), h32(F32_MIN_NORMAL)], ALLOW, OK, f32(2.0 ** -23))
case("scalar_checked_float/tests.rs:100-106", "f32", "div", [h32(F32_MIN_NORMAL - 1), h32(F32_MIN_NORMAL)], ALLOW, OK, f32(1.0 - 2.0 ** -23))
case("scalar_checked_float/tests.rs:107-117", "f32", "div", [h32(F32_MIN_NORMAL), h32(1)], ALLOW, OK, f32(2.0 ** 23))
case("scalar_checked_float/tests.rs:118-127", "f32", "div", [h32(1), h32(F32_MIN_NORMAL + 1)], ALLOW, OK,
     h32(int(f32(2.0 ** -23), 16) - 2))
case("scalar_checked_float/tests.rs:128-133", "f32", "div", [h32(3), f32(2.0)], ALLOW, OK, h32(2))
case("scalar_checked_float/tests.rs:134-139", "f32", "div", [h32(5), f32(2.0)], ALLOW, OK, h32(2))
case("scalar_checked_float/tests.rs:140-143", "f32", "div", [h32(1), f32(2.0)], ALLOW, OK, f32(0.0))
case("scalar_checked_float/tests.rs:144-147", "f32", "div", [h32(1), f32(2.0)], IEEE, UNF)

# tests.rs:149-174 division error order and signed zero
for num in (0x00000000, 0x80000000):
    for den in (0x00000000, 0x80000000):
        case("scalar_checked_float/tests.rs:150-157", "f32", "div", [h32(num), h32(den)], IEEE, DIV0)
case("scalar_checked_float/tests.rs:158-161", "f32", "div", [h32(0x7F800000), f32(0.0)], IEEE, INV)
case("scalar_checked_float/tests.rs:162-165", "f32", "div", [f32(0.0), h32(0x7FC00000)], IEEE, INV)
case("scalar_checked_float/tests.rs:166-169", "f32", "div", [h32(0x80000000), f32(2.0)], IEEE, OK, h32(0x80000000))
case("scalar_checked_float/tests.rs:170-173", "f32", "div", [h32(F32_MAX), h32(1)], IEEE, OVF)

# tests.rs:205-225 underflow policies distinguish exact subnormals
case("scalar_checked_float/tests.rs:207-208", "f32", "mul", [h32(1), f32(1.0)], IEEE, OK, h32(1))
case("scalar_checked_float/tests.rs:209-212", "f32", "mul", [h32(1), f32(0.5)], IEEE, UNF)
case("scalar_checked_float/tests.rs:213-217", "f32", "mul", [h32(1), f32(0.5)], ALLOW, OK, f32(0.0))
case("scalar_checked_float/tests.rs:218-222", "f32", "mul", [h32(1), f32(1.0)], REJECT, UNF)

# tests.rs:227-242 tininess uses unbounded-exponent rounding
case("scalar_checked_float/tests.rs:229-233", "f32", "mul", [h32(F32_MIN_NORMAL), h32(0x3F7FFFFF)], IEEE, UNF)
case("scalar_checked_float/tests.rs:234-240", "f32", "mul", [h32(F32_MIN_NORMAL), h32(0x3F7FFFFF)], ALLOW, OK, h32(F32_MIN_NORMAL))

# tests.rs:244-287 signed zero preserved for exact zero results
NZ, PZ = 0x80000000, 0x00000000
case("scalar_checked_float/tests.rs:247-253", "f32", "add", [h32(NZ), h32(PZ)], IEEE, OK, h32(0))
case("scalar_checked_float/tests.rs:254-260", "f32", "add", [h32(NZ), h32(NZ)], IEEE, OK, h32(NZ))
case("scalar_checked_float/tests.rs:261-267", "f32", "add", [h32(PZ), h32(NZ)], IEEE, OK, h32(0))
case("scalar_checked_float/tests.rs:268-274", "f32", "sub", [h32(NZ), h32(PZ)], IEEE, OK, h32(NZ))
case("scalar_checked_float/tests.rs:275-281", "f32", "sub", [h32(PZ), h32(NZ)], IEEE, OK, h32(0))
case("scalar_checked_float/tests.rs:282-285", "f32", "mul", [h32(NZ), f32(2.0)], IEEE, OK, h32(NZ))

# tests.rs:289-303 zero identity obeys RejectSubnormalResult
case("scalar_checked_float/tests.rs:292-297", "f32", "add", [f32(0.0), h32(1)], REJECT, UNF)
case("scalar_checked_float/tests.rs:298-302", "f32", "add", [h32(1), f32(0.0)], REJECT, UNF)

# ---------------------------------------------------------------- binary64
# f64_tests.rs:3-47 relu patterns
for bits in (0x0, 0x8000000000000000, 0x1, 0x000FFFFFFFFFFFFF, 0x0010000000000000,
             0x3FF0000000000000, 0x7FEFFFFFFFFFFFFF, 0x8000000000000001, 0xBFF0000000000000,
             0xFFEFFFFFFFFFFFFF):
    expected = 0 if (bits >> 63) or (bits & ~(1 << 63)) == 0 else bits
    case("scalar_checked_float/f64_tests.rs:5-25", "f64", "relu", [h64(bits)], IEEE, OK, h64(expected))
for bits in (0x7FF0000000000000, 0xFFF0000000000000, 0x7FF0000000000001, 0xFFF8123456789ABC):
    case("scalar_checked_float/f64_tests.rs:26-36", "f64", "relu", [h64(bits)], IEEE, INV)
case("scalar_checked_float/f64_tests.rs:37-41", "f64", "relu", [h64(1)], REJECT, UNF)
case("scalar_checked_float/f64_tests.rs:42-46", "f64", "relu", [h64(1)], ALLOW, OK, h64(1))

# f64_tests.rs:59-83 add/sub ties-to-even and zero signs
case("scalar_checked_float/f64_tests.rs:61-62", "f64", "add", [f64(1.0), f64(2.0 ** -53)], IEEE, OK, f64(1.0))
case("scalar_checked_float/f64_tests.rs:63-67", "f64", "add", [f64(1.0), f64(3 * 2.0 ** -53)], IEEE, OK, f64(1.0 + 2 * 2.0 ** -52))
case("scalar_checked_float/f64_tests.rs:69", "f64", "add", [f64(1.0), f64(-1.0)], IEEE, OK, f64(0.0))
case("scalar_checked_float/f64_tests.rs:70-73", "f64", "add", [h64(1 << 63), h64(1 << 63)], IEEE, OK, h64(1 << 63))
case("scalar_checked_float/f64_tests.rs:74-77", "f64", "sub", [h64(1 << 63), f64(0.0)], IEEE, OK, h64(1 << 63))
case("scalar_checked_float/f64_tests.rs:78-81", "f64", "add", [f64(0.0), h64(1 << 63)], IEEE, OK, f64(0.0))

# f64_tests.rs:85-92 multiply signed zero and exact cancellation
case("scalar_checked_float/f64_tests.rs:86-89", "f64", "mul", [h64(1 << 63), f64(3.0)], IEEE, OK, h64(1 << 63))
case("scalar_checked_float/f64_tests.rs:90", "f64", "mul", [f64(-3.0), f64(0.0)], IEEE, OK, h64(1 << 63))
case("scalar_checked_float/f64_tests.rs:91", "f64", "sub", [f64(1.25), f64(1.25)], IEEE, OK, f64(0.0))

# f64_tests.rs:95-141 underflow policies
half_min = F64_MIN_NORMAL >> 1  # exact subnormal min_normal * 0.5
case("scalar_checked_float/f64_tests.rs:99", "f64", "mul", [h64(F64_MIN_NORMAL), f64(0.5)], IEEE, OK, h64(half_min))
case("scalar_checked_float/f64_tests.rs:100-103", "f64", "mul", [h64(F64_MIN_NORMAL), f64(0.5)], ALLOW, OK, h64(half_min))
case("scalar_checked_float/f64_tests.rs:104-108", "f64", "mul", [h64(F64_MIN_NORMAL), f64(0.5)], REJECT, UNF)
case("scalar_checked_float/f64_tests.rs:110-113", "f64", "mul", [h64(1), f64(0.5)], IEEE, UNF)
case("scalar_checked_float/f64_tests.rs:114-118", "f64", "mul", [h64((1 << 63) | 1), f64(0.5)], ALLOW, OK, h64(1 << 63))
pred_one = 0x3FEFFFFFFFFFFFFF
case("scalar_checked_float/f64_tests.rs:123-126", "f64", "mul", [h64(F64_MIN_NORMAL), h64(pred_one)], IEEE, UNF)
case("scalar_checked_float/f64_tests.rs:127-133", "f64", "mul", [h64(F64_MIN_NORMAL), h64(pred_one)], REJECT, UNF)
case("scalar_checked_float/f64_tests.rs:134-140", "f64", "mul", [h64(F64_MIN_NORMAL), h64(pred_one)], ALLOW, OK, h64(F64_MIN_NORMAL))

# f64_tests.rs:144-176 non-finite operands and overflow
for bits in (0x7FF0000000000000, 0xFFF0000000000000, 0x7FF8000000000000):
    for op in ("add", "sub", "mul"):
        case("scalar_checked_float/f64_tests.rs:145-157", "f64", op, [f64(1.0), h64(bits)], IEEE, INV)
    case("scalar_checked_float/f64_tests.rs:158-161", "f64", "mul", [h64(bits), f64(0.0)], IEEE, INV)
case("scalar_checked_float/f64_tests.rs:164-167", "f64", "add", [h64(F64_MAX), h64(F64_MAX)], IEEE, OVF)
case("scalar_checked_float/f64_tests.rs:168-171", "f64", "mul", [h64(F64_MAX), f64(2.0)], IEEE, OVF)
case("scalar_checked_float/f64_tests.rs:172-175", "f64", "sub", [h64(F64_MAX), h64(F64_MAX | (1 << 63))], IEEE, OVF)

# f64_tests.rs:179-236 division of subnormals
case("scalar_checked_float/f64_tests.rs:182-188", "f64", "div", [h64(1), h64(F64_MIN_NORMAL)], ALLOW, OK, f64(2.0 ** -52))
case("scalar_checked_float/f64_tests.rs:189-195", "f64", "div", [h64(F64_MIN_NORMAL - 1), h64(F64_MIN_NORMAL)], ALLOW, OK, f64(1.0 - 2.0 ** -52))
case("scalar_checked_float/f64_tests.rs:196-202", "f64", "div", [h64(F64_MIN_NORMAL), h64(1)], ALLOW, OK, f64(2.0 ** 52))
case("scalar_checked_float/f64_tests.rs:203-212", "f64", "div", [h64(1), h64(F64_MIN_NORMAL + 1)], ALLOW, OK,
     h64(int(f64(2.0 ** -52), 16) - 2))
case("scalar_checked_float/f64_tests.rs:213-219", "f64", "div", [h64(3), f64(2.0)], ALLOW, OK, h64(2))
case("scalar_checked_float/f64_tests.rs:220-226", "f64", "div", [h64(5), f64(2.0)], ALLOW, OK, h64(2))
case("scalar_checked_float/f64_tests.rs:227-231", "f64", "div", [h64(1), f64(2.0)], ALLOW, OK, f64(0.0))
case("scalar_checked_float/f64_tests.rs:232-235", "f64", "div", [h64(1), f64(2.0)], IEEE, UNF)

# ---------------------------------------------------------------- relu_backward
# relu_backward contract (scalar_checked_float.rs:634-652; f64.rs twin): both operands
# finite, strictly positive input selects upstream, otherwise +0.
case("scalar_checked_float.rs:640-651", "f32", "relu_backward", [f32(2.0), f32(-3.0)], IEEE, OK, f32(-3.0))
case("scalar_checked_float.rs:640-651", "f32", "relu_backward", [h32(0x80000000), f32(5.0)], IEEE, OK, f32(0.0))
case("scalar_checked_float.rs:640-651", "f32", "relu_backward", [f32(0.0), f32(5.0)], IEEE, OK, f32(0.0))
case("scalar_checked_float.rs:640-651", "f32", "relu_backward", [f32(-1.0), h32(0x7FC00000)], IEEE, INV)
case("scalar_checked_float.rs:640-651", "f32", "relu_backward", [h32(1), f32(7.0)], IEEE, OK, f32(7.0))
case("scalar_checked_float.rs:640-651", "f32", "relu_backward", [f32(1.0), h32(1)], REJECT, UNF)

# constants/constants.rs:18-28 + scalar_widen.rs:9-37 conversions
conversions = {
    "u64_to_f32": [[n, f32(float(n))] for n in (0, 1, 2, 3, 4096, 4194304, (1 << 24) + 1, (1 << 24) + 3, 2 ** 64 - 1)],
    "u64_to_f64": [[n, f64(float(n))] for n in (0, 1, 4096, 4194304, (1 << 53) + 1, (1 << 53) + 3, 2 ** 64 - 1)],
    "f32_to_f64": [[f32(x), f64(struct.unpack("<f", struct.pack("<f", x))[0])]
                   for x in (0.1, -2.5, 1.0, 2.0 ** -149, 2.0 ** -130)],
}

with open(os.path.join(HERE, "scalar_kat.json"), "w") as fh:
    json.dump({"cases": cases, "conversions": conversions}, fh, indent=1)

# ------------------------------------------------------------------ tensor KATs
# Strict compound known answers (reference/strict_{matmul,sgd,mse}/tests.rs,
# backends/cpu/tests/prepared_tensor/prepared_tensor.rs). Matrices are row-major;
# "fault" is [element_index, reduction_index, step, kind] or null.
tensor = []


def t(src, kind_of_op, dtype, inputs, params, policy, output=None, fault=None):
    tensor.append({"source": src, "op": kind_of_op, "dtype": dtype, "inputs": inputs,
                   "params": params, "policy": policy, "output": output, "fault": fault})


MAX32 = struct.unpack("<f", struct.pack("<I", F32_MAX))[0]
MAX64 = struct.unpack("<d", struct.pack("<Q", F64_MAX))[0]
NAN = "nan"

# strict_matmul/tests.rs:33-59 (1x2 . 2x1)
t("reference/strict_matmul/tests.rs:33-48", "matmul", "f32",
  [{"shape": [1, 2], "bits": [h32(1), f32(1.0)]}, {"shape": [2, 1], "bits": [f32(0.5), f32(1.0)]}],
  {"tl": False, "tr": False}, IEEE, fault=[0, 0, "Multiply", UNF])
t("reference/strict_matmul/tests.rs:49-58", "matmul", "f32",
  [{"shape": [1, 2], "bits": [h32(1), f32(1.0)]}, {"shape": [2, 1], "bits": [f32(0.5), f32(1.0)]}],
  {"tl": False, "tr": False}, ALLOW, output=[f32(1.0)])
# :62-89 exact subnormal and exact zero
t("reference/strict_matmul/tests.rs:64-67", "matmul", "f32",
  [{"shape": [1, 1], "bits": [h32(1)]}, {"shape": [1, 1], "bits": [f32(1.0)]}],
  {"tl": False, "tr": False}, IEEE, output=[h32(1)])
t("reference/strict_matmul/tests.rs:68-80", "matmul", "f32",
  [{"shape": [1, 1], "bits": [h32(1)]}, {"shape": [1, 1], "bits": [f32(1.0)]}],
  {"tl": False, "tr": False}, REJECT, fault=[0, 0, "Multiply", UNF])
t("reference/strict_matmul/tests.rs:81-88", "matmul", "f32",
  [{"shape": [1, 2], "bits": [f32(1.0), f32(-1.0)]}, {"shape": [2, 1], "bits": [f32(1.0), f32(1.0)]}],
  {"tl": False, "tr": False}, REJECT, output=[f32(0.0)])
# :92-121 ordered overflow before cancellation
for right in ([1.0, 1.0, -1.0], [1.0, 1.0, 0.0]):
    t("reference/strict_matmul/tests.rs:93-107", "matmul", "f32",
      [{"shape": [1, 3], "bits": [h32(F32_MAX)] * 3}, {"shape": [3, 1], "bits": [f32(v) for v in right]}],
      {"tl": False, "tr": False}, ALLOW, fault=[0, 1, "Add", OVF])
t("reference/strict_matmul/tests.rs:108-120", "matmul", "f32",
  [{"shape": [1, 1], "bits": [h32(F32_MAX)]}, {"shape": [1, 1], "bits": [f32(2.0)]}],
  {"tl": False, "tr": False}, IEEE, fault=[0, 0, "Multiply", OVF])
# :124-136 first fault row-major cell, then k, then multiply/add
t("reference/strict_matmul/tests.rs:124-136", "matmul", "f32",
  [{"shape": [2, 2], "bits": [f32(1.0), h32(F32_MAX), h32(F32_MAX), f32(1.0)]},
   {"shape": [2, 2], "bits": [f32(1.0), f32(2.0), f32(2.0), f32(2.0)]}],
  {"tl": False, "tr": False}, IEEE, fault=[0, 1, "Multiply", OVF])
# :139-181 binary64 transposes
t("reference/strict_matmul/tests.rs:140-153", "matmul", "f64",
  [{"shape": [2, 1], "bits": [h64(1), f64(1.0)]}, {"shape": [1, 2], "bits": [f64(0.5), f64(1.0)]}],
  {"tl": True, "tr": True}, IEEE, fault=[0, 0, "Multiply", UNF])
t("reference/strict_matmul/tests.rs:154-168", "matmul", "f64",
  [{"shape": [2, 1], "bits": [h64(1), f64(1.0)]}, {"shape": [1, 2], "bits": [f64(0.5), f64(1.0)]}],
  {"tl": True, "tr": True}, ALLOW, output=[f64(1.0)])
t("reference/strict_matmul/tests.rs:169-180", "matmul", "f64",
  [{"shape": [1, 1], "bits": [h64(F64_MIN_NORMAL)]}, {"shape": [1, 1], "bits": [f64(0.5)]}],
  {"tl": False, "tr": False}, IEEE, output=[h64(F64_MIN_NORMAL >> 1)])
# :227-253 no FMA; non-finite operands
t("reference/strict_matmul/tests.rs:229-237", "matmul", "f32",
  [{"shape": [1, 2], "bits": [f32(-1.0), h32(0x3F800001)]}, {"shape": [2, 1], "bits": [f32(1.0), h32(0x3F7FFFFF)]}],
  {"tl": False, "tr": False}, IEEE, output=[f32(0.0)])
for inv in (0x7FC00000, 0x7F800000, 0xFF800000):
    t("reference/strict_matmul/tests.rs:238-252", "matmul", "f32",
      [{"shape": [1, 1], "bits": [h32(inv)]}, {"shape": [1, 1], "bits": [f32(0.0)]}],
      {"tl": False, "tr": False}, ALLOW, fault=[0, 0, "Multiply", INV])
# :255-290 binary64 overflow before cancellation; MSE of equal values
t("reference/strict_matmul/tests.rs:257-270", "matmul", "f64",
  [{"shape": [1, 3], "bits": [h64(F64_MAX)] * 3}, {"shape": [3, 1], "bits": [f64(1.0), f64(1.0), f64(-1.0)]}],
  {"tl": False, "tr": False}, IEEE, fault=[0, 1, "Add", OVF])
t("reference/strict_matmul/tests.rs:271-289", "mse", "f32",
  [{"shape": [1], "bits": [f32(1.0)]}, {"shape": [1], "bits": [f32(1.0)]}], {}, IEEE, output=[f32(0.0)])

# CPU prepared: backends/cpu/tests/prepared_tensor/prepared_tensor.rs:188-212, :214-235
t("cpu/tests/prepared_tensor/prepared_tensor.rs:188-212", "matmul", "f32",
  [{"shape": [1, 2], "bits": [h32(F32_MAX), h32(0x7FC00000)]},
   {"shape": [2, 2], "bits": [f32(2.0), f32(1.0), f32(0.0), h32(0x7FC00000)]}],
  {"tl": False, "tr": False}, IEEE, fault=[0, 0, "Multiply", OVF])
t("cpu/tests/prepared_tensor/prepared_tensor.rs:214-235", "matmul", "f64",
  [{"shape": [1, 2], "bits": [h64(F64_MAX), h64(F64_MAX)]}, {"shape": [2, 1], "bits": [f64(1.0), f64(1.0)]}],
  {"tl": False, "tr": False}, IEEE, fault=[0, 1, "Add", OVF])
t("cpu/tests/prepared_tensor/prepared_tensor.rs:237-253", "mse", "f64",
  [{"shape": [1], "bits": [h64(F64_MAX)]}, {"shape": [1], "bits": [h64(F64_MAX | (1 << 63))]}], {}, IEEE,
  fault=[0, 0, "Subtract", OVF])

# strict_sgd/tests.rs
t("reference/strict_sgd/tests.rs:20-31", "sgd", "f32",
  [{"shape": [1], "bits": [f32(1.0)]}, {"shape": [1], "bits": [h32(1)]}], {"rate": f32(0.5)}, IEEE,
  fault=[0, 0, "Multiply", UNF])
t("reference/strict_sgd/tests.rs:32-39", "sgd", "f32",
  [{"shape": [1], "bits": [f32(1.0)]}, {"shape": [1], "bits": [h32(1)]}], {"rate": f32(0.5)}, ALLOW,
  output=[f32(1.0)])
t("reference/strict_sgd/tests.rs:43-53", "sgd", "f32",
  [{"shape": [1], "bits": [f32(0.0)]}, {"shape": [1], "bits": [h32(1)]}], {"rate": f32(1.0)}, IEEE,
  output=[h32(0x80000001)])
t("reference/strict_sgd/tests.rs:54-64", "sgd", "f32",
  [{"shape": [1], "bits": [f32(0.0)]}, {"shape": [1], "bits": [h32(1)]}], {"rate": f32(1.0)}, REJECT,
  fault=[0, 0, "Multiply", UNF])
t("reference/strict_sgd/tests.rs:69-77", "sgd", "f32",
  [{"shape": [2], "bits": [h32(F32_MAX), f32(0.0)]}, {"shape": [2], "bits": [h32(F32_MAX | 0x80000000), h32(F32_MAX)]}],
  {"rate": f32(2.0)}, IEEE, fault=[0, 0, "Multiply", OVF])
t("reference/strict_sgd/tests.rs:78-88", "sgd", "f32",
  [{"shape": [2], "bits": [h32(F32_MAX), h32(0x7FC00000)]}, {"shape": [2], "bits": [h32(F32_MAX | 0x80000000), h32(F32_MAX)]}],
  {"rate": f32(1.0)}, IEEE, fault=[0, 0, "Subtract", OVF])
for w, g, step in ((0x7FC00000, 0x3F800000, "Subtract"), (0x3F800000, 0x7F800000, "Multiply"),
                   (0x7FC00000, 0x7FC00000, "Multiply")):
    t("reference/strict_sgd/tests.rs:92-105", "sgd", "f32",
      [{"shape": [1], "bits": [h32(w)]}, {"shape": [1], "bits": [h32(g)]}], {"rate": f32(0.0)}, IEEE,
      fault=[0, 0, step, INV])
t("reference/strict_sgd/tests.rs:109-118", "sgd", "f32",
  [{"shape": [1], "bits": [f32(1.0)]}, {"shape": [1], "bits": [h32(0x3F7FFFFF)]}], {"rate": h32(0x3F800001)}, IEEE,
  output=[f32(0.0)])
t("reference/strict_sgd/tests.rs:119-129", "sgd", "f32",
  [{"shape": [1], "bits": [h32(0x80000000)]}, {"shape": [1], "bits": [f32(0.0)]}], {"rate": f32(1.0)}, IEEE,
  output=[h32(0x80000000)])
t("reference/strict_sgd/tests.rs:133-145", "sgd", "f64",
  [{"shape": [2], "bits": [f64(3.0), h64(1 << 63)]}, {"shape": [2], "bits": [f64(1.0), f64(0.0)]}],
  {"rate": f32(0.1)}, IEEE,
  output=[f64(3.0 - struct.unpack("<f", struct.pack("<f", 0.1))[0]), h64(1 << 63)])
t("reference/strict_sgd/tests.rs:146-157", "sgd", "f64",
  [{"shape": [2], "bits": [f64(3.0), h64(1 << 63)]}, {"shape": [2], "bits": [h64(1), f64(1.0)]}],
  {"rate": f32(0.5)}, IEEE, fault=[0, 0, "Multiply", UNF])
t("reference/strict_sgd/tests.rs:193-203", "sgd", "f64",
  [{"shape": [], "bits": [f64(2.0)]}, {"shape": [], "bits": [f64(2.0)]}], {"rate": f32(0.5)}, IEEE,
  output=[f64(1.0)])

# strict_mse/tests.rs:29-84
for p, tt, idx, step, kind in (
        ([h32(F32_MAX)], [h32(F32_MAX | 0x80000000)], 0, "Subtract", OVF),
        ([h32(F32_MAX)], [f32(0.0)], 0, "Multiply", OVF),
        ([f32(1.0), h32(0x7FC00000)], [f32(0.0), f32(0.0)], 1, "Subtract", INV),
        ([h32(1)], [f32(0.0)], 0, "Multiply", UNF)):
    t("reference/strict_mse/tests.rs:30-66", "mse", "f32",
      [{"shape": [len(p)], "bits": p}, {"shape": [len(tt)], "bits": tt}], {}, IEEE,
      fault=[0, idx, step, kind])
t("reference/strict_mse/tests.rs:67-75", "mse", "f32",
  [{"shape": [2], "bits": [f32(3.0), f32(5.0)]}, {"shape": [2], "bits": [f32(1.0), f32(1.0)]}], {}, IEEE,
  output=[f32(10.0)])
t("reference/strict_mse/tests.rs:86-101", "mse", "f64",
  [{"shape": [2], "bits": [f64(3.0), f64(5.0)]}, {"shape": [2], "bits": [f64(1.0), f64(1.0)]}], {}, IEEE,
  output=[f64(10.0)])
t("reference/strict_mse/tests.rs:102-114", "mse", "f32",
  [{"shape": [1], "bits": [h32(1)]}, {"shape": [1], "bits": [f32(0.0)]}], {}, ALLOW, output=[f32(0.0)])

# cpu/tests/prepared_tensor/prepared_tensor.rs:110-158 transposes (values only; the
# reference asserts equality with its evaluator, so these pin shapes and strides)
l6 = [1.0, -2.0, 4.0, 8.0, 2.0, -0.5]
r12 = [0.25, 2.0, -1.0, 0.5, 4.0, 2.0, 1.0, -1.0, 0.5, 0.25, 0.125, 8.0]
for tl in (False, True):
    for tr in (False, True):
        ls = [3, 2] if tl else [2, 3]
        rs = [4, 3] if tr else [3, 4]
        L = [[l6[i * ls[1] + j] for j in range(ls[1])] for i in range(ls[0])]
        R = [[r12[i * rs[1] + j] for j in range(rs[1])] for i in range(rs[0])]
        opL = [list(col) for col in zip(*L)] if tl else L
        opR = [list(col) for col in zip(*R)] if tr else R
        out = []
        for i in range(2):
            for j in range(4):
                acc = 0.0
                for k in range(3):
                    acc = acc + opL[i][k] * opR[k][j]  # small dyadic values: every step exact
                out.append(acc)
        for dt, conv in (("f32", f32), ("f64", f64)):
            t("cpu/tests/prepared_tensor/prepared_tensor.rs:110-158", "matmul", dt,
              [{"shape": ls, "bits": [conv(v) for v in l6]}, {"shape": rs, "bits": [conv(v) for v in r12]}],
              {"tl": tl, "tr": tr}, IEEE, output=[conv(v) for v in out])

with open(os.path.join(HERE, "tensor_kat.json"), "w") as fh:
    json.dump({"cases": tensor}, fh, indent=1)

print(f"wrote {len(cases)} scalar and {len(tensor)} tensor cases")
