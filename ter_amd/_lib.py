"""ctypes bindings of libter_hip.so (the C-ABI declared in include/ter_hip.h).

The library is always the in-tree build, ter_amd/libter_hip.so (built by
ter_amd/build.py).  Loading fails loudly when it is missing: there is no
Python or CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libter_hip.so")

# status codes (include/ter_hip.h)
OK = 0
ERR_NULL = -1
ERR_NOTFOUND = -2
ERR_ALLOC = -3
ERR_NARGS = -4
ERR_SHAPE = -5
ERR_PAYLOAD = -6
ERR_HIP = -7
ERR_ALIGN = -8
ERR_FULL = -9
ERR_CONFLICT = -10
ERR_FILE = -11
ERR_FEWARGS = -12

K_MAX = 32768
N_MAX = 1 << 24
M_MAX = 256
STATIC_Q_MAX = 4 << 20

X_I8 = 0
X_F32 = 1
X_F32_RMS = 2
X_F16_RMS = 3
X_RELU2_RMS = 4
X_I16 = 5
X_F16 = 6
X_SILU_MUL = 7
X_SMUL = 8
PLAN_STRIPS, PLAN_STRIDED, PLAN_SHARED = 1, 2, 4  # ter_hip_plan_mode flags
SLOT_MATMUL = b"tk_matmul_t16"
LAYOUT_T16 = 16
ARGMAX_STATE_BYTES = 16512
ROPE_NORM = 0
ROPE_NEOX = 1
BIN_TERT = 0x54455254
BIN_LLRT = 0x4C4C5254
BIN_F16, BIN_F32, BIN_TRITS = 0, 1, 2


class WPK(C.Structure):
    """ter_hip_wpk_t -- the packed weight handle (replaces the reference's
    WPK{data, scale, bytes}, cuda/ter_cuda_forward_packed.cu:400)."""
    _fields_ = [
        ("data", C.c_void_p),
        ("bytes", C.c_size_t),
        ("fix", C.c_void_p),
        ("K", C.c_int32),
        ("N", C.c_int32),
        ("scale", C.c_float),
        ("layout", C.c_int32),
        ("mag", C.c_int32),
    ]


class Act(C.Structure):
    """ter_hip_act_t -- activation operand."""
    _fields_ = [
        ("data", C.c_void_p),
        ("kind", C.c_int32),
        ("scale", C.c_float),
        ("scale_dev", C.c_void_p),
        ("q_out", C.c_void_p),
        ("scale_out", C.c_void_p),
        ("gamma", C.c_void_p),
        ("eps", C.c_float),
        ("up", C.c_void_p),
    ]


class Out(C.Structure):
    """ter_hip_out_t -- output forms of one GEMV / GEMM."""
    _fields_ = [
        ("y", C.c_void_p),
        ("acc", C.c_void_p),
        ("y16", C.c_void_p),
        ("resid", C.c_void_p),
        ("resid16", C.c_void_p),
        ("silu", C.c_void_p),
    ]


class GemvItem(C.Structure):
    _fields_ = [
        ("w", C.POINTER(WPK)),
        ("x", Act),
        ("y", C.c_void_p),
        ("acc", C.c_void_p),
        ("y16", C.c_void_p),
        ("resid", C.c_void_p),
        ("resid16", C.c_void_p),
        ("silu", C.c_void_p),
    ]


class GemmItem(C.Structure):
    _fields_ = [
        ("w", C.POINTER(WPK)),
        ("x", C.c_void_p),
        ("x_scale_dev", C.c_void_p),
        ("M", C.c_int32),
        ("y", C.c_void_p),
        ("acc", C.c_void_p),
        ("y16", C.c_void_p),
        ("resid", C.c_void_p),
        ("resid16", C.c_void_p),
        ("silu", C.c_void_p),
    ]


class BinHeader(C.Structure):
    """ter_hip_bin_header_t -- the 64-byte header of a packed model file."""
    _fields_ = [(n, C.c_uint32) for n in ("magic", "version", "H", "F", "Nl", "V", "Nh", "Nkv", "Hd", "Smax")] + [
        ("rope_theta", C.c_float), ("eps", C.c_float)]


class BinTensor(C.Structure):
    """ter_hip_bin_tensor_t -- one entry of a model file's tensor directory."""
    _fields_ = [
        ("name", C.c_char * 24),
        ("layer", C.c_int32),
        ("kind", C.c_int32),
        ("offset", C.c_int64),
        ("bytes", C.c_int64),
        ("n", C.c_int64),
        ("K", C.c_int32),
        ("N", C.c_int32),
        ("scale", C.c_float),
    ]


class OpCounts(C.Structure):
    _fields_ = [
        ("total_ops", C.c_uint64),
        ("tvmac", C.c_uint64),
        ("tvadd", C.c_uint64),
        ("tvsub", C.c_uint64),
        ("tvmul", C.c_uint64),
    ]


NATIVE_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(C.c_int64), C.c_size_t)

# (name, restype, argtypes) for every exported symbol of include/ter_hip.h
_P = C.c_void_p
SIGNATURES = [
    ("ter_hip_version", C.c_char_p, []),
    ("ter_hip_last_error", C.c_char_p, []),
    ("ter_hip_wpk_bytes", C.c_size_t, [C.c_int32, C.c_int32]),
    ("ter_hip_wpk_init", C.c_int, [C.POINTER(WPK), _P, C.c_size_t, C.c_int32, C.c_int32, C.c_float]),
    ("ter_hip_pack_v11", C.c_int, [C.POINTER(WPK), _P, _P]),
    ("ter_hip_unpack_v11", C.c_int, [C.POINTER(WPK), _P, _P]),
    ("ter_hip_pack_payload", C.c_int, [C.POINTER(WPK), _P, C.c_float, C.POINTER(C.c_int32), _P]),
    ("ter_hip_gemv", C.c_int, [C.POINTER(WPK), C.POINTER(Act), _P, _P, _P]),
    ("ter_hip_gemv_out", C.c_int, [C.POINTER(WPK), C.POINTER(Act), C.POINTER(Out), _P]),
    ("ter_hip_mm_packed_dispatch", C.c_int, [_P, _P, C.POINTER(WPK), _P, C.c_int32, C.c_int32, _P]),
    ("ter_hip_mm_packed_dispatch_f16", C.c_int, [_P, _P, C.POINTER(WPK), _P, C.c_int32, C.c_int32, _P]),
    ("ter_hip_mm_row", C.c_int, [_P, C.c_int32, C.c_int32, C.c_float, C.POINTER(WPK), C.c_int32, _P, _P, _P, _P]),
    ("ter_hip_mm_row_blocked", C.c_int, [_P, C.c_int32, C.c_int32, C.c_float, C.POINTER(WPK), C.c_int32, _P,
                                         C.c_int64, _P, _P, _P, _P]),
    ("ter_hip_plan_create", C.c_int, [C.POINTER(C.c_void_p), C.POINTER(GemvItem), C.c_int32, C.c_int32]),
    ("ter_hip_plan_launch", C.c_int, [_P, _P]),
    ("ter_hip_plan_stats", C.c_int, [_P, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.POINTER(C.c_int32)]),
    ("ter_hip_plan_mode", C.c_int, [_P, C.POINTER(C.c_int32)]),
    ("ter_hip_plan_destroy", None, [_P]),
    ("ter_hip_gemm", C.c_int, [C.POINTER(WPK), C.POINTER(Act), C.c_int32, _P, _P, _P]),
    ("ter_hip_gemm_out", C.c_int, [C.POINTER(WPK), C.POINTER(Act), C.c_int32, C.POINTER(Out), _P]),
    ("ter_hip_gemm_out_static", C.c_int, [C.POINTER(WPK), C.POINTER(Act), C.c_int32, C.POINTER(Out), _P]),
    ("ter_hip_gemm_plan_create", C.c_int, [C.POINTER(C.c_void_p), C.POINTER(GemmItem), C.c_int32, C.c_int32]),
    ("ter_hip_quant_int8", C.c_int, [_P, C.c_int32, C.c_int32, _P, _P, _P]),
    ("ter_hip_pack_i2s", C.c_int, [C.POINTER(WPK), _P, _P]),
    ("ter_hip_rmsnorm_quant", C.c_int, [_P, C.c_int32, _P, C.c_float, C.c_int32, C.c_int32, _P, _P, _P]),
    ("ter_hip_relu2_rmsnorm_quant", C.c_int, [_P, _P, _P, C.c_float, C.c_int32, C.c_int32, _P, _P, _P]),
    ("ter_hip_rmsnorm_f16", C.c_int, [_P, _P, C.c_float, C.c_int32, C.c_int32, _P, _P]),
    ("ter_hip_lm_head_f16", C.c_int, [_P, _P, _P, C.c_int32, C.c_int32, _P]),
    ("ter_hip_argmax_f16", C.c_int, [_P, C.c_int32, _P, _P, _P]),
    ("ter_hip_argmax_f16_step", C.c_int, [_P, C.c_int32, _P, _P, _P, _P]),
    ("ter_hip_lm_head_argmax", C.c_int, [_P, _P, C.c_float, _P, C.c_int32, C.c_int32, _P, _P, _P, _P, _P, _P]),
    ("ter_hip_embed_f16", C.c_int, [_P, C.c_int32, C.c_int32, _P, _P, _P]),
    ("ter_hip_lm_head_argmax_h16", C.c_int, [_P, _P, C.c_float, _P, C.c_int32, C.c_int32, _P, _P, _P, _P, _P, _P]),
    ("ter_hip_embed_h16", C.c_int, [_P, C.c_int32, C.c_int32, _P, _P, _P]),
    ("ter_hip_attn_create", C.c_int, [C.POINTER(C.c_void_p), C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_float,
                                      C.c_int32]),
    ("ter_hip_attn_decode", C.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P]),
    ("ter_hip_rope", C.c_int, [_P, _P, C.c_int32, _P, _P]),
    ("ter_hip_attn_destroy", None, [_P]),
    ("ter_hip_bin_open", C.c_int, [C.c_char_p, C.POINTER(C.c_void_p), C.POINTER(BinHeader)]),
    ("ter_hip_bin_count", C.c_int32, [_P]),
    ("ter_hip_bin_tensor", C.c_int, [_P, C.c_int32, C.POINTER(BinTensor)]),
    ("ter_hip_bin_find", C.c_int32, [_P, C.c_char_p, C.c_int32]),
    ("ter_hip_bin_read_host", C.c_int, [_P, C.c_int32, _P, C.c_int32]),
    ("ter_hip_bin_upload_f16", C.c_int, [_P, C.c_int32, _P, _P]),
    ("ter_hip_bin_upload_wpk", C.c_int, [_P, C.c_int32, C.POINTER(WPK), _P, _P]),
    ("ter_hip_bin_close", None, [_P]),
    ("ter_hip_create", _P, [C.c_int32]),
    ("ter_hip_destroy", None, [_P]),
    ("ter_hip_install_native", C.c_int, [_P, C.c_char_p, NATIVE_FN]),
    ("ter_hip_call", C.c_int, [_P, C.c_char_p, C.POINTER(C.c_int64), C.c_size_t]),
    ("ter_hip_op_counts", None, [_P, C.POINTER(OpCounts)]),
    ("ter_hip_reset_counters", None, [_P]),
    ("ter_hip_synth_v11", C.c_int, [_P, C.c_int32, C.c_int32, C.c_uint64, C.c_uint32, C.c_uint32, _P]),
    ("ter_hip_synth_i8", C.c_int, [_P, C.c_int64, C.c_uint64, C.c_int32, C.c_int32, _P]),
    ("ter_hip_noop", C.c_int, [_P]),
    ("ter_hip_read_probe", C.c_int, [_P, C.c_size_t, C.c_int32, _P, _P]),
]

_lib = None


class TerHipError(RuntimeError):
    def __init__(self, code: int, where: str):
        msg = lib().ter_hip_last_error().decode(errors="replace")
        super().__init__(f"{where} failed with status {code}: {msg}")
        self.code = code


def lib():
    """Load libter_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m ter_amd.build` "
                "(there is no fallback path)")
        # PyTorch ships its own HIP runtime (torch/lib/libamdhip64.so, soname
        # libamdhip64.so.7).  Loaded first, it satisfies this library's
        # libamdhip64.so.7 dependency, so both share one runtime; loaded after
        # this library, torch would bring in a second runtime beside the
        # /opt/rocm one, and this library's launches would find no device.
        # Without torch installed the library loads alone against the system
        # runtime (the C-ABI needs nothing from torch).
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(code: int, where: str) -> None:
    if code != OK:
        raise TerHipError(code, where)
