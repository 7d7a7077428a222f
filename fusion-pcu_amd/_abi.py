"""ctypes binding of include/pcu_rocm.h (the library's C ABI).

This is the same binding a Rust maintainer would write with bindgen/extern "C" in
Crates/backends; here it lets the Python mirror and the tests drive the library. The
library must be built in-tree (``fusion-pcu_amd/libpcu_rocm.so``); there is no fallback.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpcu_rocm.so")

PCU_OK = 0
PCU_ARITHMETIC_FAULT = 1
PCU_ERR_ARGUMENT = 2
PCU_ERR_SHAPE = 3
PCU_ERR_UNSUPPORTED = 4
PCU_ERR_DEVICE = 5
PCU_ERR_OUT_OF_MEMORY = 6
PCU_ERR_STATE = 7
PCU_ERR_PROTOCOL = 8

STATUS_NAMES = {
    0: "PCU_OK", 1: "PCU_ARITHMETIC_FAULT", 2: "PCU_ERR_ARGUMENT", 3: "PCU_ERR_SHAPE",
    4: "PCU_ERR_UNSUPPORTED", 5: "PCU_ERR_DEVICE", 6: "PCU_ERR_OUT_OF_MEMORY",
    7: "PCU_ERR_STATE", 8: "PCU_ERR_PROTOCOL",
}

PCU_F32, PCU_F64 = 0, 1
UNDERFLOW_IEEE, UNDERFLOW_REJECT_SUBNORMAL, UNDERFLOW_ALLOW_GRADUAL = 0, 1, 2
OP_ADD, OP_SUB, OP_MUL, OP_DIV = 0, 1, 2, 3


class Fault(ctypes.Structure):
    _fields_ = [
        ("node", ctypes.c_uint32),
        ("kind", ctypes.c_uint32),
        ("step", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("element_index", ctypes.c_uint64),
        ("reduction_index", ctypes.c_uint64),
        ("ordinal", ctypes.c_uint64),
    ]


# Every function the header declares, with its ctypes signature. Tests check that the
# library exports each of these names.
_u32, _u64, _i32, _f32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int, ctypes.c_float
_sz, _vp, _cp = ctypes.c_size_t, ctypes.c_void_p, ctypes.c_char_p
_FP = ctypes.POINTER(Fault)
_VPP = ctypes.POINTER(ctypes.c_void_p)

SIGNATURES = {
    "pcu_abi_version": (_i32, []),
    "pcu_ctx_open": (_i32, [_i32, _VPP]),
    "pcu_ctx_close": (None, [_vp]),
    "pcu_last_error": (_cp, [_vp]),
    "pcu_ctx_stream": (_vp, [_vp]),
    "pcu_ctx_synchronize": (_i32, [_vp]),
    "pcu_ctx_set_matmul_engine": (_i32, [_vp, _i32]),
    "pcu_buf_alloc": (_i32, [_vp, _sz, _VPP]),
    "pcu_buf_free": (_i32, [_vp, _vp]),
    "pcu_upload": (_i32, [_vp, _vp, _vp, _sz]),
    "pcu_download": (_i32, [_vp, _vp, _vp, _sz]),
    "pcu_strict_matmul": (_i32, [_vp, _i32, _u64, _u64, _u64, _i32, _i32, _vp, _vp, _vp, _i32, _FP]),
    "pcu_strict_matmul_noalloc": (_i32, [_vp, _i32, _u64, _u64, _u64, _i32, _i32, _vp, _vp, _vp, _i32, _FP]),
    "pcu_checked_binary": (_i32, [_vp, _i32, _i32, _u64, _vp, _vp, _vp, _i32, _FP]),
    "pcu_checked_binary_uniform": (_i32, [_vp, _i32, _i32, _u64, _vp, _u64, _vp, _i32, _FP]),
    "pcu_checked_relu": (_i32, [_vp, _i32, _u64, _vp, _vp, _i32, _FP]),
    "pcu_checked_relu_backward": (_i32, [_vp, _i32, _u64, _vp, _vp, _vp, _i32, _FP]),
    "pcu_checked_add_relu": (_i32, [_vp, _i32, _u64, _vp, _vp, _vp, _i32, _FP]),
    "pcu_strict_sgd": (_i32, [_vp, _i32, _u64, _vp, _vp, _f32, _vp, _i32, _FP]),
    "pcu_strict_mse": (_i32, [_vp, _i32, _u64, _vp, _vp, _vp, _i32, _FP]),
    "pcu_native_matmul": (_i32, [_vp, _i32, _u64, _u64, _u64, _i32, _i32, _vp, _vp, _vp]),
    "pcu_native_mse": (_i32, [_vp, _i32, _u64, _vp, _vp, _vp]),
    "pcu_native_sgd": (_i32, [_vp, _i32, _u64, _vp, _vp, _f32, _i32, _vp]),
    "pcu_program_begin": (_i32, [_vp]),
    "pcu_program_end": (_i32, [_vp, _FP]),
    "pcu_program_next_node": (_u32, [_vp]),
    "pcu_fault_read": (_i32, [_vp, _FP]),
    "pcu_fault_reset": (_i32, [_vp]),
    "pcu_mark": (_i32, [_vp, _i32]),
    "pcu_elapsed_ms": (_i32, [_vp, _i32, _i32, ctypes.POINTER(ctypes.c_float)]),
    "pcu_profile_enable": (_i32, [_vp, _i32]),
    "pcu_profile_read": (_i32, [_vp, _i32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_uint64)]),
    "pcu_calibrate_direct_copy": (_i32, [_vp, _vp, _vp, ctypes.c_uint64]),
}


class NumericalOptions(ctypes.Structure):
    """pcu_numerical_options (PcuNumericalOptions, core/numerical/numerical.rs:71-78)."""
    _fields_ = [
        ("compound_arithmetic", ctypes.c_uint32),  # 0 Checked, 1 BackendDefined
        ("precision", ctypes.c_uint32),            # 0 Preserve, 1 BackendOptimized
        ("reproducibility", ctypes.c_uint32),      # 0 Unspecified, 1 PortableV1
    ]


class NodeDesc(ctypes.Structure):
    _fields_ = [
        ("op", ctypes.c_uint32),
        ("left", ctypes.c_uint32),
        ("right", ctypes.c_uint32),
        ("transpose_left", ctypes.c_uint32),
        ("transpose_right", ctypes.c_uint32),
        ("dtype", ctypes.c_uint32),
        ("numerical_mode", ctypes.c_int32),
        ("underflow_policy", ctypes.c_int32),
        ("learning_rate", ctypes.c_float),
        ("rank", ctypes.c_uint32),
        ("value_bits", ctypes.c_uint64),
        ("shape", ctypes.c_uint64 * 8),
        ("options", NumericalOptions),
        ("reserved", ctypes.c_uint32),
    ]


_U32P = ctypes.POINTER(ctypes.c_uint32)
_U64P = ctypes.POINTER(ctypes.c_uint64)
SIGNATURES.update({
    "pcu_graph_create": (_i32, [_VPP]),
    "pcu_graph_destroy": (None, [_vp]),
    "pcu_graph_set_numerical_mode": (_i32, [_vp, _i32]),
    "pcu_graph_input": (_i32, [_vp, _i32, _u32, _U64P, _U32P]),
    "pcu_graph_uniform": (_i32, [_vp, _i32, _u32, _U64P, _u64, _U32P]),
    "pcu_graph_constant": (_i32, [_vp, _i32, _u32, _U64P, _vp, _U32P]),
    "pcu_graph_binary": (_i32, [_vp, _i32, _u32, _u32, _U32P]),
    "pcu_graph_relu": (_i32, [_vp, _u32, _U32P]),
    "pcu_graph_relu_backward": (_i32, [_vp, _u32, _u32, _U32P]),
    "pcu_graph_matmul": (_i32, [_vp, _u32, _u32, _i32, _i32, _U32P]),
    "pcu_graph_mean_squared_error": (_i32, [_vp, _u32, _u32, _U32P]),
    "pcu_graph_sgd_update": (_i32, [_vp, _u32, _u32, _f32, _U32P]),
    "pcu_graph_set_underflow_policy": (_i32, [_vp, _u32, _i32]),
    "pcu_graph_set_value_numerical_mode": (_i32, [_vp, _u32, _i32]),
    "pcu_graph_set_numerical_options": (_i32, [_vp, ctypes.POINTER(NumericalOptions)]),
    "pcu_graph_set_value_numerical_options": (_i32, [_vp, _u32, ctypes.POINTER(NumericalOptions)]),
    "pcu_graph_backward_mse": (_i32, [_vp, _u32, _U32P, _u32]),
    "pcu_graph_backward_mse_for_targets": (_i32, [_vp, _u32, _u32, _U32P, _U32P]),
    "pcu_graph_node_count": (_u32, [_vp]),
    "pcu_graph_describe": (_i32, [_vp, _u32, ctypes.POINTER(NodeDesc)]),
    "pcu_graph_plan": (_i32, [_vp, _u32, _U32P, _U32P, _U32P]),
    "pcu_prepare": (_i32, [_vp, _vp, _u32, _U32P, _VPP]),
    "pcu_prepared_destroy": (None, [_vp]),
    "pcu_prepared_input_count": (_u32, [_vp]),
    "pcu_prepared_input_id": (_i32, [_vp, _u32, _U32P]),
    "pcu_prepared_execute": (_i32, [_vp, _u32, ctypes.POINTER(ctypes.c_void_p), _FP]),
    "pcu_prepared_output": (_vp, [_vp, _u32]),
    "pcu_prepared_take_output": (_i32, [_vp, _u32, _VPP]),
})

GRAPH_OPS = ["Input", "Uniform", "Add", "Sub", "Mul", "Div", "SgdUpdate", "MatMul", "Relu",
             "ReluBackward", "MeanSquaredError", "Constant"]

KERNEL_IDS = {
    "strict_gemm": 0, "gemm_prefilter": 1, "gemm_replay": 2, "sgd": 3, "binary": 4,
    "relu": 5, "relu_backward": 6, "add_relu": 7, "mse": 8,
    "native_gemm": 9, "native_sgd": 10, "native_mse": 11, "elementwise_chain": 12,
}

_lib = None


def load():
    """Load the in-tree library; fail loudly when it is absent (never fall back)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python __graft_entry__.py` or "
            "`python fusion-pcu_amd/build.py` (there is no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib
