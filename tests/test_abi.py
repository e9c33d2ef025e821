"""CPU checks of the C-ABI boundary (no device needed).

* libter_hip.so loads and exports every function include/ter_hip.h declares;
* argument validation returns the ter_k4-style codes before any device work
  (null -> -1, unknown kernel -> -2, > 7 args -> -4: src/k4/ter_k4.cpp:52-55);
* the KernelTable native slot (install / find / call, 32 slots, names < 32
  chars: include/ter/kernels.hpp:21-38) dispatches to an installed function.
"""
import ctypes as C
import os
import re

import pytest

from ter_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ter_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b(ter_hip_\w+)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if not n.endswith("_fn")))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) == 56, names
    lib = L.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    bound = {n for n, _, _ in L.SIGNATURES}
    assert set(names) == bound, (set(names) ^ bound)


def test_version_and_sizes():
    lib = L.lib()
    assert b"gfx950" in lib.ter_hip_version()
    # T16: ceil(N/16) strips x ceil(K/256) tiles of 1 KiB + N 8-byte fix-up slots
    assert lib.ter_hip_wpk_bytes(2048, 2048) == 128 * 8 * 1024 + 2048 * 8
    assert lib.ter_hip_wpk_bytes(2560, 640) == 40 * 10 * 1024 + 640 * 8
    assert lib.ter_hip_wpk_bytes(6912, 2560) == 160 * 27 * 1024 + 2560 * 8
    assert lib.ter_hip_wpk_bytes(1, 1) == 1024 + 8
    assert lib.ter_hip_wpk_bytes(0, 4) == 0


def test_wpk_init_validation():
    lib = L.lib()
    w = L.WPK()
    fake = 1 << 20  # never dereferenced: validation happens before device work
    need = lib.ter_hip_wpk_bytes(64, 16)
    assert lib.ter_hip_wpk_init(None, fake, need, 64, 16, 1.0) == L.ERR_NULL
    assert lib.ter_hip_wpk_init(C.byref(w), None, need, 64, 16, 1.0) == L.ERR_NULL
    assert lib.ter_hip_wpk_init(C.byref(w), fake + 4, need, 64, 16, 1.0) == L.ERR_ALIGN
    assert lib.ter_hip_wpk_init(C.byref(w), fake, need - 1, 64, 16, 1.0) == L.ERR_SHAPE
    assert lib.ter_hip_wpk_init(C.byref(w), fake, need, L.K_MAX + 1, 16, 1.0) == L.ERR_SHAPE
    assert lib.ter_hip_wpk_init(C.byref(w), fake, need, 64, 0, 1.0) == L.ERR_SHAPE
    assert lib.ter_hip_wpk_init(C.byref(w), fake, need, 64, 16, 0.5) == L.OK
    assert w.K == 64 and w.N == 16 and w.layout == L.LAYOUT_T16 and w.scale == 0.5
    assert w.fix == fake + 1024  # 1 strip x 1 unit tile, then the fix-up slots


def test_gemv_validation_without_device():
    lib = L.lib()
    w = L.WPK()
    fake = 1 << 20
    assert lib.ter_hip_wpk_init(C.byref(w), fake, lib.ter_hip_wpk_bytes(64, 16), 64, 16, 1.0) == L.OK
    x = L.Act()
    assert lib.ter_hip_gemv(C.byref(w), None, fake, None, None) == L.ERR_NULL
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_NULL  # x.data null
    x.data = fake
    x.kind = 99
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_PAYLOAD
    # silu(gate) * up needs up; fp16 kinds 2-byte aligned; both are GEMV-only
    x.kind = L.X_SILU_MUL
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_NULL
    x.up = fake + 1
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_ALIGN
    x.up = None
    x.kind, x.data = L.X_F16, fake + 1
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_ALIGN
    x.data = fake
    assert lib.ter_hip_gemm(C.byref(w), C.byref(x), 4, fake, None, None) == L.ERR_PAYLOAD
    assert lib.ter_hip_gemm(C.byref(w), C.byref(x), 1, fake, None, None) == L.ERR_PAYLOAD
    # silu(gate) * up from an fp32 silu vector: up required, fp32 alignment, GEMV-only
    x.kind, x.data, x.up = L.X_SMUL, fake, None
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_NULL
    x.up, x.data = fake, fake + 2
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_ALIGN
    x.data = fake
    assert lib.ter_hip_gemm(C.byref(w), C.byref(x), 4, fake, None, None) == L.ERR_PAYLOAD
    x.kind, x.up = L.X_F16, None
    # fp16 residual outputs: 2-byte aligned, GEMVs only
    o = L.Out()
    o.resid16 = fake + 1
    assert lib.ter_hip_gemv_out(C.byref(w), C.byref(x), C.byref(o), None) == L.ERR_ALIGN
    o.resid16 = fake
    xi = L.Act()
    xi.data, xi.kind, xi.scale_dev = fake, L.X_I8, fake
    assert lib.ter_hip_gemm_out(C.byref(w), C.byref(xi), 4, C.byref(o), None) == L.ERR_PAYLOAD
    # the silu output: 4-byte aligned, GEMVs only
    o2 = L.Out()
    o2.silu = fake + 2
    assert lib.ter_hip_gemv_out(C.byref(w), C.byref(x), C.byref(o2), None) == L.ERR_ALIGN
    o2.silu = fake
    assert lib.ter_hip_gemm_out(C.byref(w), C.byref(xi), 4, C.byref(o2), None) == L.ERR_PAYLOAD
    x.kind = L.X_I8
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), None, None, None) == L.ERR_NULL  # no output
    x.kind = L.X_F32
    x.data = fake + 2
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_ALIGN
    # mm_packed_dispatch shape mismatch
    assert lib.ter_hip_mm_packed_dispatch(fake, fake, C.byref(w), fake, 64, 32, None) == L.ERR_SHAPE
    # batched: M out of range, int8 X without per-row scales
    x.data, x.kind = fake, L.X_I8
    assert lib.ter_hip_gemm(C.byref(w), C.byref(x), 0, fake, None, None) == L.ERR_SHAPE
    assert lib.ter_hip_gemm(C.byref(w), C.byref(x), L.M_MAX + 1, fake, None, None) == L.ERR_SHAPE
    assert lib.ter_hip_gemm(C.byref(w), C.byref(x), 8, fake, None, None) == L.ERR_NULL
    # i2_s repack: null codes, K or N not a multiple of 4, N*K not whole 128-blocks
    assert lib.ter_hip_pack_i2s(C.byref(w), None, None) == L.ERR_NULL
    w2 = L.WPK()
    assert lib.ter_hip_wpk_init(C.byref(w2), fake, lib.ter_hip_wpk_bytes(36, 4), 36, 4, 1.0) == L.OK
    assert lib.ter_hip_pack_i2s(C.byref(w2), fake, None) == L.ERR_SHAPE
    assert lib.ter_hip_wpk_init(C.byref(w2), fake, lib.ter_hip_wpk_bytes(64, 6), 64, 6, 1.0) == L.OK
    assert lib.ter_hip_pack_i2s(C.byref(w2), fake, None) == L.ERR_SHAPE
    # RMSNorm kinds: gamma required and aligned, eps >= 0, fp16 X 2-byte aligned
    x.kind, x.data, x.scale_dev = L.X_F32_RMS, fake, None
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_NULL
    x.gamma = fake + 1
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_ALIGN
    x.gamma, x.eps = fake, -1.0
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_SHAPE
    x.kind, x.eps, x.data = L.X_F16_RMS, 1e-5, fake + 1
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_ALIGN
    assert lib.ter_hip_rmsnorm_quant(fake, L.X_I8, fake, 1e-5, 1, 64, fake, fake, None) == L.ERR_PAYLOAD
    assert lib.ter_hip_rmsnorm_quant(fake, L.X_F32_RMS, None, 1e-5, 1, 64, fake, fake, None) == L.ERR_NULL
    assert lib.ter_hip_rmsnorm_quant(fake, L.X_F32_RMS, fake, 1e-5, 0, 64, fake, fake, None) == L.ERR_SHAPE
    assert lib.ter_hip_rmsnorm_quant(fake, L.X_F32_RMS, fake, float("nan"), 1, 64, fake, fake, None) == L.ERR_SHAPE
    # relu^2 kind: up required and 2-byte aligned, gate 2-byte aligned
    x.kind, x.data, x.gamma, x.up = L.X_RELU2_RMS, fake, fake, None
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_NULL
    x.up = fake + 1
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_ALIGN
    x.up, x.data = fake, fake + 1
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_ALIGN
    x.up, x.gamma = None, None
    q = lib.ter_hip_relu2_rmsnorm_quant
    assert q(None, fake, fake, 1e-5, 1, 64, fake, fake, None) == L.ERR_NULL
    assert q(fake, fake, fake, 1e-5, 1, L.K_MAX + 1, fake, fake, None) == L.ERR_SHAPE
    assert q(fake, fake + 1, fake, 1e-5, 1, 64, fake, fake, None) == L.ERR_ALIGN
    assert q(fake, fake, fake, -1.0, 1, 64, fake, fake, None) == L.ERR_SHAPE
    assert lib.ter_hip_rmsnorm_quant(fake, L.X_RELU2_RMS, fake, 1e-5, 1, 64, fake, fake, None) == L.ERR_PAYLOAD
    # output forms: at least one, each aligned to its element
    x.data, x.kind, x.scale_dev = fake, L.X_I8, fake
    o = L.Out()
    assert lib.ter_hip_gemv_out(C.byref(w), C.byref(x), C.byref(o), None) == L.ERR_NULL
    assert lib.ter_hip_gemv_out(C.byref(w), C.byref(x), None, None) == L.ERR_NULL
    o.y16 = fake + 1
    assert lib.ter_hip_gemv_out(C.byref(w), C.byref(x), C.byref(o), None) == L.ERR_ALIGN
    o.y16, o.resid = None, fake + 2
    assert lib.ter_hip_gemv_out(C.byref(w), C.byref(x), C.byref(o), None) == L.ERR_ALIGN
    # a residual output that overlaps the activation the launch reads
    x.kind, x.data, x.gamma = L.X_F32_RMS, fake, fake << 2
    o.resid = fake + 64
    assert lib.ter_hip_gemv_out(C.byref(w), C.byref(x), C.byref(o), None) == L.ERR_CONFLICT
    x.kind, x.gamma = L.X_I8, None
    assert lib.ter_hip_gemm_out(C.byref(w), C.byref(x), 8, C.byref(o), None) == L.ERR_CONFLICT
    o.resid = None
    assert lib.ter_hip_gemm_out(C.byref(w), C.byref(x), 8, C.byref(L.Out()), None) == L.ERR_NULL
    assert lib.ter_hip_mm_packed_dispatch_f16(fake, fake, C.byref(w), fake, 64, 32, None) == L.ERR_SHAPE
    assert lib.ter_hip_mm_packed_dispatch_f16(fake, fake, C.byref(w), None, 64, 16, None) == L.ERR_NULL
    x.gamma, x.data, x.kind = None, fake, L.X_I8
    x.scale_dev = None
    # unknown layout tag
    w.layout = 3
    x.scale_dev = fake
    assert lib.ter_hip_gemv(C.byref(w), C.byref(x), fake, None, None) == L.ERR_PAYLOAD


def test_lm_head_validation_without_device():
    lib = L.lib()
    fake = 1 << 20
    # standalone RMSNorm -> fp16
    assert lib.ter_hip_rmsnorm_f16(None, fake, 1e-5, 1, 64, fake, None) == L.ERR_NULL
    assert lib.ter_hip_rmsnorm_f16(fake, fake, 1e-5, 0, 64, fake, None) == L.ERR_SHAPE
    assert lib.ter_hip_rmsnorm_f16(fake + 2, fake, 1e-5, 1, 64, fake, None) == L.ERR_ALIGN
    assert lib.ter_hip_rmsnorm_f16(fake, fake, -1.0, 1, 64, fake, None) == L.ERR_SHAPE
    # lm_head GEMV: shapes, 4-byte alignment for even H
    assert lib.ter_hip_lm_head_f16(fake, None, fake, 64, 10, None) == L.ERR_NULL
    assert lib.ter_hip_lm_head_f16(fake, fake, fake, 0, 10, None) == L.ERR_SHAPE
    assert lib.ter_hip_lm_head_f16(fake, fake, fake, 64, L.N_MAX + 1, None) == L.ERR_SHAPE
    assert lib.ter_hip_lm_head_f16(fake, fake + 2, fake, 64, 10, None) == L.ERR_ALIGN
    assert lib.ter_hip_lm_head_f16(fake + 2, fake, fake, 64, 10, None) == L.ERR_ALIGN
    # argmax: state and output required
    assert lib.ter_hip_argmax_f16(fake, 10, fake, None, None) == L.ERR_NULL
    assert lib.ter_hip_argmax_f16(fake, 0, fake, fake, None) == L.ERR_SHAPE
    assert lib.ter_hip_argmax_f16(fake, 10, fake, fake + 4, None) == L.ERR_ALIGN
    # fused tail: even H only, token_out and state required, alignment
    args = [fake, fake, 1e-5, fake, 64, 10, None, None, fake, fake, None, None]
    bad = list(args); bad[8] = None
    assert lib.ter_hip_lm_head_argmax(*bad) == L.ERR_NULL
    bad = list(args); bad[4] = 63
    assert lib.ter_hip_lm_head_argmax(*bad) == L.ERR_SHAPE
    bad = list(args); bad[0] = fake + 4
    assert lib.ter_hip_lm_head_argmax(*bad) == L.ERR_ALIGN
    bad = list(args); bad[2] = float("nan")
    assert lib.ter_hip_lm_head_argmax(*bad) == L.ERR_SHAPE


def test_attention_validation_without_device():
    lib = L.lib()
    h = C.c_void_p()
    create = lib.ter_hip_attn_create
    assert create(None, 20, 5, 128, 2048, 5e5, L.ROPE_NEOX) == L.ERR_NULL
    assert create(C.byref(h), 20, 6, 128, 2048, 5e5, L.ROPE_NEOX) == L.ERR_SHAPE   # heads not a multiple
    assert create(C.byref(h), 20, 5, 96, 2048, 5e5, L.ROPE_NEOX) == L.ERR_SHAPE    # head_dim
    assert create(C.byref(h), 20, 5, 128, 4097, 5e5, L.ROPE_NEOX) == L.ERR_SHAPE   # > 64 chunks of 64
    assert create(C.byref(h), 20, 5, 128, 2048, 5e5, 7) == L.ERR_PAYLOAD
    assert create(C.byref(h), 20, 5, 128, 2048, 0.0, L.ROPE_NEOX) == L.ERR_SHAPE
    fake = 1 << 20
    assert lib.ter_hip_attn_decode(None, fake, fake, fake, fake, fake, fake, fake, None) == L.ERR_NULL
    assert lib.ter_hip_rope(None, fake, 1, fake, None) == L.ERR_NULL


def test_mm_row_rejects_activations_beyond_int16():
    # The 9-trit host activations (+-9841, src/tx/forward.cpp:400) run on the
    # int16 GEMV; values that do not fit int16 (10+-trit payloads beyond
    # 32767) are refused instead of computed on the CPU.  The staging buffer
    # must be 16-byte aligned.
    import numpy as np
    lib = L.lib()
    w = L.WPK()
    fake = 1 << 20
    K, N = 64, 16
    assert lib.ter_hip_wpk_init(C.byref(w), fake, lib.ter_hip_wpk_bytes(K, N), K, N, 1.0) == L.OK
    X = np.zeros((2, K), dtype=np.int32)
    out = np.zeros(N, dtype=np.float32)
    for bad in (32768, -32769, 88573):
        X[1, 5] = bad
        rc = lib.ter_hip_mm_row(X.ctypes.data, 1, K, 1.0, C.byref(w), N, out.ctypes.data, fake, fake, None)
        assert rc == L.ERR_PAYLOAD
        assert b"int16" in lib.ter_hip_last_error()
    X[1, 5] = 9841
    rc = lib.ter_hip_mm_row(X.ctypes.data, 1, K, 1.0, C.byref(w), N, out.ctypes.data, fake + 8, fake, None)
    assert rc == L.ERR_ALIGN


def test_int16_activations_are_single_gemv_only():
    lib = L.lib()
    w = L.WPK()
    fake = 1 << 20
    assert lib.ter_hip_wpk_init(C.byref(w), fake, lib.ter_hip_wpk_bytes(64, 16), 64, 16, 1.0) == L.OK
    a = L.Act()
    a.data = fake
    a.kind = L.X_I16
    a.scale_dev = fake
    assert lib.ter_hip_gemm(C.byref(w), C.byref(a), 4, fake, None, None) == L.ERR_PAYLOAD
    # one int16 row through the GEMM entry points is refused the same way
    # (not sent to the fp32 / RMS quantizers, which would ask for q_out)
    assert lib.ter_hip_gemm(C.byref(w), C.byref(a), 1, fake, None, None) == L.ERR_PAYLOAD
    o = L.Out()
    o.y = fake
    assert lib.ter_hip_gemm_out(C.byref(w), C.byref(a), 1, C.byref(o), None) == L.ERR_PAYLOAD
    assert lib.ter_hip_gemm_out_static(C.byref(w), C.byref(a), 1, C.byref(o), None) == L.ERR_PAYLOAD
    items = (L.GemvItem * 1)()
    items[0].w = C.pointer(w)
    items[0].x = a
    items[0].y = fake
    h = C.c_void_p()
    assert lib.ter_hip_plan_create(C.byref(h), items, 1, 0) == L.ERR_PAYLOAD
    a.data = fake + 1
    assert lib.ter_hip_gemv(C.byref(w), C.byref(a), fake, None, None) == L.ERR_ALIGN
    w.mag = 0
    a.data = fake
    assert lib.ter_hip_gemv(C.byref(w), C.byref(a), fake, None, None) == L.ERR_PAYLOAD


def test_pack_payload_rejects_non_ternary_and_blocked():
    import numpy as np
    lib = L.lib()
    w = L.WPK()
    fake = 1 << 20
    K, N = 8, 4
    assert lib.ter_hip_wpk_init(C.byref(w), fake, lib.ter_hip_wpk_bytes(K, N), K, N, 1.0) == L.OK
    p = np.zeros((K, N), dtype=np.int32)
    p[0, 0], p[1, 1], p[2, 2] = 9841, -9841, 3  # two magnitudes -> not ternary
    m = C.c_int32()
    assert lib.ter_hip_pack_payload(C.byref(w), p.ctypes.data, 1.0, C.byref(m), None) == L.ERR_PAYLOAD


def test_plan_validation():
    lib = L.lib()
    h = C.c_void_p()
    items = (L.GemvItem * 1)()
    assert lib.ter_hip_plan_create(None, items, 1, 0) == L.ERR_NULL
    assert lib.ter_hip_plan_create(C.byref(h), items, 0, 0) == L.ERR_SHAPE
    assert lib.ter_hip_plan_create(C.byref(h), items, 1, 0) == L.ERR_NULL  # null weight
    w = L.WPK()
    fake = 1 << 20
    assert lib.ter_hip_wpk_init(C.byref(w), fake, lib.ter_hip_wpk_bytes(64, 16), 64, 16, 1.0) == L.OK
    items2 = (L.GemvItem * 2)()
    for it in items2:
        it.w = C.pointer(w)
        it.x.data = fake
        it.x.kind = L.X_I8
        it.y = fake
    assert lib.ter_hip_plan_create(C.byref(h), items2, 2, 0) == L.ERR_CONFLICT  # same weight twice
    # two weights whose residual outputs overlap (a plain read-modify-write each)
    w2 = L.WPK()
    assert lib.ter_hip_wpk_init(C.byref(w2), fake << 1, lib.ter_hip_wpk_bytes(64, 16), 64, 16, 1.0) == L.OK
    items2[1].w = C.pointer(w2)
    items2[0].y, items2[1].y = None, None
    items2[0].resid, items2[1].resid = fake << 3, (fake << 3) + 4 * 15
    assert lib.ter_hip_plan_create(C.byref(h), items2, 2, 0) == L.ERR_CONFLICT
    items2[1].resid = fake + 8  # item 0 reads X at fake: item 1 must not add into it
    assert lib.ter_hip_plan_create(C.byref(h), items2, 2, 0) == L.ERR_CONFLICT


def test_gemm_plan_validation():
    lib = L.lib()
    h = C.c_void_p()
    items = (L.GemmItem * 1)()
    assert lib.ter_hip_gemm_plan_create(None, items, 1, 0) == L.ERR_NULL
    assert lib.ter_hip_gemm_plan_create(C.byref(h), items, 0, 0) == L.ERR_SHAPE
    assert lib.ter_hip_gemm_plan_create(C.byref(h), items, 1, 0) == L.ERR_NULL  # null weight
    w = L.WPK()
    fake = 1 << 20
    assert lib.ter_hip_wpk_init(C.byref(w), fake, lib.ter_hip_wpk_bytes(64, 16), 64, 16, 1.0) == L.OK
    items[0].w = C.pointer(w)
    assert lib.ter_hip_gemm_plan_create(C.byref(h), items, 1, 0) == L.ERR_NULL  # null X
    items[0].x = fake
    items[0].x_scale_dev = fake
    items[0].y = fake
    for bad_m in (0, L.M_MAX + 1):
        items[0].M = bad_m
        assert lib.ter_hip_gemm_plan_create(C.byref(h), items, 1, 0) == L.ERR_SHAPE
    items[0].M = 8
    items[0].y = None
    assert lib.ter_hip_gemm_plan_create(C.byref(h), items, 1, 0) == L.ERR_NULL  # no output
    items[0].y16 = fake + 1
    assert lib.ter_hip_gemm_plan_create(C.byref(h), items, 1, 0) == L.ERR_ALIGN


def test_kernel_table_slots_and_codes():
    lib = L.lib()
    h = lib.ter_hip_create(-1)  # device -1: calls do not select a device (no GPU here)
    assert h
    try:
        args = (C.c_int64 * 8)(*range(8))
        assert lib.ter_hip_call(None, L.SLOT_MATMUL, args, 1) == L.ERR_NULL
        assert lib.ter_hip_call(h, None, args, 1) == L.ERR_NULL
        assert lib.ter_hip_call(h, b"no_such_kernel", args, 1) == L.ERR_NOTFOUND
        assert lib.ter_hip_call(h, L.SLOT_MATMUL, args, 8) == L.ERR_NARGS
        # the reference's own matmul name is the Sim's 3-argument kernel
        # (r1 = X, r2 = W, r3 = Y: src/kernels/tk_matmul_b_9t.tasm): the
        # native table does not claim it, so a router falls through to the Sim
        sim_args = (C.c_int64 * 3)(100, 200, 300)
        assert lib.ter_hip_call(h, b"tk_matmul_b_9t", sim_args, 3) == L.ERR_NOTFOUND
        # the native matmul slot validates its own arguments
        zero = (C.c_int64 * 6)(0, 0, 0, 0, 0, 1)
        assert lib.ter_hip_call(h, L.SLOT_MATMUL, zero, 6) == L.ERR_NULL     # null W
        assert lib.ter_hip_call(h, L.SLOT_MATMUL, zero, 5) == L.ERR_FEWARGS  # too few
        seen = []

        def native(hh, a, n):
            seen.append([a[i] for i in range(n)])
            return 42

        cb = L.NATIVE_FN(native)
        assert lib.ter_hip_install_native(h, b"tk_custom", cb) == L.OK
        assert lib.ter_hip_call(h, b"tk_custom", args, 7) == 42
        assert seen == [list(range(7))]
        # 32 slots: 2 used (the matmul slot, tk_custom) -> 30 more fit, then full
        for i in range(30):
            assert lib.ter_hip_install_native(h, b"slot%02d" % i, cb) == L.OK
        assert lib.ter_hip_install_native(h, b"one_too_many", cb) == L.ERR_FULL
        # re-installing an existing name replaces it (no new slot needed)
        assert lib.ter_hip_install_native(h, b"slot00", cb) == L.OK
        c = L.OpCounts()
        lib.ter_hip_op_counts(h, C.byref(c))
        assert c.tvmac == 0 and c.total_ops == 0  # failed calls count nothing
        lib.ter_hip_reset_counters(h)
    finally:
        lib.ter_hip_destroy(h)


def test_kernel_table_name_truncation():
    # names keep at most 31 chars (KernelTable::kNameMax = 32, src/sim/call_kernel.cpp:41-42)
    lib = L.lib()
    h = lib.ter_hip_create(-1)
    try:
        cb = L.NATIVE_FN(lambda hh, a, n: 7)
        long_name = b"k" * 40
        assert lib.ter_hip_install_native(h, long_name, cb) == L.OK
        args = (C.c_int64 * 1)(0)
        assert lib.ter_hip_call(h, b"k" * 31, args, 0) == 7
        assert lib.ter_hip_call(h, b"k" * 30, args, 0) == L.ERR_NOTFOUND
    finally:
        lib.ter_hip_destroy(h)


def test_c99_caller_routes_reference_calls_to_the_sim(tmp_path):
    """A strict C99 translation unit compiles against include/ter_hip.h,
    links libter_hip.so and implements the ter_k4_call routing: the
    reference's 3-argument tk_matmul_b_9t call reaches the Sim (stub)."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not installed")
    L.lib()  # the library is built
    exe = str(tmp_path / "k4_router")
    libdir = os.path.dirname(L.LIB_PATH)
    cmd = [gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "c", "k4_router.c"), "-L", libdir, "-lter_hip", f"-Wl,-rpath,{libdir}",
           "-o", exe]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout
    r = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout
