"""ter_amd -- MI355X (gfx950) packed-trit matmul fabric for ter.

The hot path (packed-trit GEMV / batched GEMM) is hand-written HIP in
ter_amd/csrc, exported through the C-ABI of include/ter_hip.h and bound here
with ctypes.  See ter_amd.fabric for the host interface.
"""
from . import _lib  # noqa: F401
from .fabric import (  # noqa: F401
    ArgmaxState,
    Attention,
    GemmPlan,
    Handle,
    PackedTrits,
    Plan,
    argmax_f16,
    embed_f16,
    embed_h16,
    gemv,
    group_contiguous,
    lm_head_argmax,
    lm_head_f16,
    mm_batched,
    mm_packed_dispatch,
    mm_packed_dispatch_f16,
    mm_row,
    mm_row_blocked,
    noop,
    quant_int8,
    read_probe,
    relu2_rmsnorm_quant,
    rmsnorm_f16,
    rmsnorm_quant,
    synth_i8,
    synth_v11,
)

__all__ = [
    "ArgmaxState",
    "Attention",
    "GemmPlan",
    "Handle",
    "PackedTrits",
    "Plan",
    "argmax_f16",
    "embed_f16",
    "embed_h16",
    "gemv",
    "lm_head_argmax",
    "lm_head_f16",
    "mm_batched",
    "mm_packed_dispatch",
    "mm_packed_dispatch_f16",
    "mm_row",
    "mm_row_blocked",
    "noop",
    "quant_int8",
    "read_probe",
    "relu2_rmsnorm_quant",
    "rmsnorm_f16",
    "rmsnorm_quant",
    "synth_i8",
    "synth_v11",
]
