"""NumPy/ctypes front-end of the CPU oracle (test infrastructure only).

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module.  It loads ``oracle/liboracle.so`` (the C
restatement in ``ter_oracle.c``) and, when built, ``oracle/_ref/libter_ref.so``
(the reference's own ``mm_row`` and quantizers compiled from its sources).

Each wrapper names the reference file:line the underlying C function follows;
the C file's header lists which test pins which function.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(HERE, "liboracle.so")
_REF = os.path.join(HERE, "_ref", "libter_ref.so")

_P = C.c_void_p
_lib = None
_ref = None


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def lib():
    """The C oracle; raises if oracle/liboracle.so has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            raise RuntimeError(f"oracle not built: {_LIB} (run make -C oracle)")
        L = C.CDLL(_LIB)
        L.orc_code_to_trit.argtypes = [C.c_uint]
        L.orc_code_to_trit.restype = C.c_int
        L.orc_trit_to_code.argtypes = [C.c_int]
        L.orc_trit_to_code.restype = C.c_uint
        L.orc_v11_pack.argtypes = [_P, C.c_int, C.c_int, _P]
        L.orc_v11_pack.restype = C.c_int
        L.orc_v11_unpack.argtypes = [_P, C.c_int, C.c_int, _P]
        L.orc_v11_unpack.restype = C.c_int
        L.orc_mm_row.argtypes = [_P, C.c_int, C.c_float, _P, C.c_float, C.c_int, C.c_int, _P, _P]
        L.orc_mm_row.restype = None
        L.orc_mm_row_blocked.argtypes = [_P, C.c_int, C.c_float, _P, _P, C.c_int, C.c_int, C.c_int, _P]
        L.orc_mm_row_blocked.restype = None
        L.orc_gemv_v11.argtypes = [_P, C.c_float, _P, C.c_float, C.c_int, C.c_int, _P, _P]
        L.orc_gemv_v11.restype = None
        L.orc_gemm_v11.argtypes = [_P, _P, C.c_int, _P, C.c_float, C.c_int, C.c_int, _P, _P]
        L.orc_gemm_v11.restype = None
        L.orc_quant_int8.argtypes = [_P, C.c_int, _P, _P]
        L.orc_quant_int8.restype = None
        L.orc_quant_int8_rows.argtypes = [_P, C.c_int, C.c_int, _P, _P]
        L.orc_quant_int8_rows.restype = None
        L.orc_half_to_float.argtypes = [C.c_uint16]
        L.orc_half_to_float.restype = C.c_float
        L.orc_rmsnorm_quant.argtypes = [_P, _P, _P, C.c_int, C.c_float, _P, _P, _P]
        L.orc_rmsnorm_quant.restype = None
        L.orc_float_to_half.argtypes = [C.c_float]
        L.orc_float_to_half.restype = C.c_uint16
        L.orc_float_to_half_n.argtypes = [_P, _P, C.c_size_t]
        L.orc_float_to_half_n.restype = None
        L.orc_relu2_rmsnorm_quant.argtypes = [_P, _P, _P, C.c_int, C.c_float, _P, _P, _P]
        L.orc_relu2_rmsnorm_quant.restype = None
        L.orc_residual_add_f16.argtypes = [_P, _P, C.c_int]
        L.orc_residual_add_f16.restype = None
        L.orc_residual_add_h16.argtypes = [_P, _P, C.c_int]
        L.orc_residual_add_h16.restype = None
        L.orc_silu_mul.argtypes = [C.c_uint16, C.c_uint16]
        L.orc_silu_mul.restype = C.c_float
        L.orc_silu_mul_quant.argtypes = [_P, _P, C.c_int, _P, _P, _P]
        L.orc_silu_mul_quant.restype = None
        L.orc_silu_f16.argtypes = [_P, C.c_int, _P]
        L.orc_silu_f16.restype = None
        L.orc_smul_quant.argtypes = [_P, _P, C.c_int, _P, _P, _P]
        L.orc_smul_quant.restype = None
        L.orc_rmsnorm_f16.argtypes = [_P, _P, C.c_int, C.c_float, _P, _P]
        L.orc_rmsnorm_f16.restype = None
        L.orc_lm_head_f16.argtypes = [_P, _P, C.c_int, C.c_int, _P, _P]
        L.orc_lm_head_f16.restype = None
        L.orc_argmax_f16.argtypes = [_P, C.c_int]
        L.orc_argmax_f16.restype = C.c_int
        L.orc_expf.argtypes = [C.c_float]
        L.orc_expf.restype = C.c_float
        L.orc_expf_n.argtypes = [_P, _P, C.c_size_t]
        L.orc_expf_n.restype = None
        L.orc_rope_table.argtypes = [C.c_float, C.c_int, C.c_int, _P]
        L.orc_rope_table.restype = None
        L.orc_rope_f16.argtypes = [_P, C.c_int, C.c_int, _P, C.c_int]
        L.orc_rope_f16.restype = None
        for f in (L.orc_attention_ref, L.orc_attention_splitk):
            f.argtypes = [_P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, _P, _P]
            f.restype = None
        L.orc_quantize_bitnet.argtypes = [_P, C.c_size_t, _P]
        L.orc_quantize_bitnet.restype = C.c_float
        L.orc_quantize_nt.argtypes = [_P, C.c_size_t, C.c_int, _P]
        L.orc_quantize_nt.restype = C.c_float
        L.orc_dequant_i2s.argtypes = [_P, C.c_size_t, _P]
        L.orc_dequant_i2s.restype = None
        L.orc_i2s_to_v11.argtypes = [_P, C.c_int, C.c_int, _P]
        L.orc_i2s_to_v11.restype = C.c_int
        L.orc_gemv_i8w.argtypes = [_P, C.c_float, _P, C.c_float, C.c_int, C.c_int, _P, _P]
        L.orc_gemv_i8w.restype = None
        L.orc_gemm_i8w.argtypes = [_P, _P, C.c_int, _P, C.c_float, C.c_int, C.c_int, _P, _P]
        L.orc_gemm_i8w.restype = None
        L.orc_v11_to_i8.argtypes = [_P, C.c_int, C.c_int, _P]
        L.orc_v11_to_i8.restype = C.c_int
        L.orc_rand_trits.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_uint64, C.c_uint64, _P]
        L.orc_rand_trits.restype = None
        L.orc_mm_row_tvmac.argtypes = [C.c_int, C.c_int]
        L.orc_mm_row_tvmac.restype = C.c_uint64
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(_REF)


def ref():
    """The reference's own code (oracle/_ref); raises if it was not built."""
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"reference build absent: {_REF}")
        R = C.CDLL(_REF)
        R.ter_ref_ctx_new.argtypes = [_P, C.c_int, C.c_int, C.c_float, _P, C.c_int, C.c_float, _P, C.c_int]
        R.ter_ref_ctx_new.restype = _P
        R.ter_ref_ctx_run.argtypes = [_P, C.c_int, _P]
        R.ter_ref_ctx_run.restype = C.c_int
        R.ter_ref_ctx_tvmac.argtypes = [_P]
        R.ter_ref_ctx_tvmac.restype = C.c_uint64
        R.ter_ref_ctx_free.argtypes = [_P]
        R.ter_ref_ctx_free.restype = None
        R.ter_ref_quantize.argtypes = [_P, C.c_int, C.c_int, _P]
        R.ter_ref_quantize.restype = C.c_float
        R.ter_ref_quantize_bitnet.argtypes = [_P, C.c_int, _P]
        R.ter_ref_quantize_bitnet.restype = C.c_float
        _ref = R
    return _ref


# --------------------------------------------------------------------------
# Layout helpers (include/ter/pack.hpp:8-21; tools/convert_llama_to_packed.py:128-140)
# --------------------------------------------------------------------------
def v11_pack(w_kn: np.ndarray) -> np.ndarray:
    """Trits [K][N] (int8 in {-1,0,1}) -> v11 bytes [(N/4)*K]."""
    w = np.ascontiguousarray(w_kn, dtype=np.int8)
    K, N = w.shape
    out = np.zeros((N // 4) * K, dtype=np.uint8)
    rc = lib().orc_v11_pack(_ptr(w), K, N, _ptr(out))
    if rc != 0:
        raise ValueError(f"orc_v11_pack rc={rc}")
    return out


def v11_unpack(v11: np.ndarray, K: int, N: int) -> np.ndarray:
    """v11 bytes -> int32 trits [K][N] (the TritTensor payload orientation)."""
    b = np.ascontiguousarray(v11, dtype=np.uint8)
    out = np.empty((K, N), dtype=np.int32)
    rc = lib().orc_v11_unpack(_ptr(b), K, N, _ptr(out))
    if rc != 0:
        raise ValueError(f"orc_v11_unpack rc={rc}")
    return out


# --------------------------------------------------------------------------
# mm_row and packed GEMV (src/tx/forward.cpp:331-346; cuda/ter_cuda_forward_packed.cu:346-397)
# --------------------------------------------------------------------------
def mm_row(X: np.ndarray, row: int, xs: float, W: np.ndarray, ws: float) -> Tuple[np.ndarray, np.ndarray]:
    """Restated mm_row int path.  X int32 [rows][K], W int32 [K][N].
    Returns (int64 acc[N], fp32 out[N])."""
    X = np.ascontiguousarray(X, dtype=np.int32)
    W = np.ascontiguousarray(W, dtype=np.int32)
    K, N = W.shape
    acc = np.empty(N, dtype=np.int64)
    out = np.empty(N, dtype=np.float32)
    lib().orc_mm_row(_ptr(X), int(row), float(xs), _ptr(W), float(ws), K, N, _ptr(acc), _ptr(out))
    return acc, out


def mm_row_blocked(X, row, xs, W, block_scales, block_size):
    X = np.ascontiguousarray(X, dtype=np.int32)
    W = np.ascontiguousarray(W, dtype=np.int32)
    bsc = np.ascontiguousarray(block_scales, dtype=np.float32)
    K, N = W.shape
    out = np.empty(N, dtype=np.float32)
    lib().orc_mm_row_blocked(_ptr(X), int(row), float(xs), _ptr(W), _ptr(bsc), int(block_size), K, N, _ptr(out))
    return out


def gemv_v11(x: np.ndarray, xs: float, v11: np.ndarray, ws: float, K: int, N: int):
    """int8 x[K] times v11-packed W -> (int32 acc[N], fp32 out[N])."""
    x = np.ascontiguousarray(x, dtype=np.int8)
    b = np.ascontiguousarray(v11, dtype=np.uint8)
    acc = np.empty(N, dtype=np.int32)
    out = np.empty(N, dtype=np.float32)
    lib().orc_gemv_v11(_ptr(x), float(xs), _ptr(b), float(ws), K, N, _ptr(acc), _ptr(out))
    return acc, out


def gemv_i8w(x: np.ndarray, xs: float, W: np.ndarray, ws: float):
    """mm_row's int path at int8 width: int8 x[K] times int8 W [K][N] ->
    (int32 acc[N], fp32 out[N] = float(acc) * (xs * ws))."""
    x = np.ascontiguousarray(x, dtype=np.int8)
    W = np.ascontiguousarray(W, dtype=np.int8)
    K, N = W.shape
    assert x.size == K
    acc = np.empty(N, dtype=np.int32)
    out = np.empty(N, dtype=np.float32)
    lib().orc_gemv_i8w(_ptr(x), float(xs), _ptr(W), float(ws), K, N, _ptr(acc), _ptr(out))
    return acc, out


def gemm_i8w(X: np.ndarray, xs: np.ndarray, W: np.ndarray, ws: float):
    """gemv_i8w per row of int8 X [M][K] with per-row scales xs[M]."""
    X = np.ascontiguousarray(X, dtype=np.int8)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.int8)
    M, K = X.shape
    N = W.shape[1]
    acc = np.empty((M, N), dtype=np.int32)
    out = np.empty((M, N), dtype=np.float32)
    lib().orc_gemm_i8w(_ptr(X), _ptr(xs), M, _ptr(W), float(ws), K, N, _ptr(acc), _ptr(out))
    return acc, out


def v11_to_i8(v11: np.ndarray, K: int, N: int) -> np.ndarray:
    """v11 bytes -> int8 trits [K][N] (v11_unpack at int8 width)."""
    b = np.ascontiguousarray(v11, dtype=np.uint8)
    out = np.empty((K, N), dtype=np.int8)
    assert lib().orc_v11_to_i8(_ptr(b), K, N, _ptr(out)) == 0
    return out


def synth_thresholds(p_zero: float):
    """(t0, t1) of rand_trits / ter_hip_synth_v11 for P(0) = p_zero."""
    t0 = int(round(p_zero * 2 ** 32))
    t1 = t0 + int(round((1.0 - p_zero) / 2.0 * 2 ** 32))
    return t0, min(t1, 2 ** 32 - 1)


def rand_trits_c(seed: int, K: int, N: int, p_zero: float = 1.0 / 3.0) -> np.ndarray:
    """rand_trits in C (same stream and mapping), for full-size inputs."""
    t0, t1 = synth_thresholds(p_zero)
    out = np.empty((K, N), dtype=np.int8)
    lib().orc_rand_trits(seed & _M64, K, N, t0, t1, _ptr(out))
    return out


def gemm_v11(X: np.ndarray, xs: np.ndarray, v11: np.ndarray, ws: float, K: int, N: int):
    """int8 X[M][K] (per-row scales xs[M]) times v11 W -> (int32 acc[M][N], fp32 out[M][N])."""
    X = np.ascontiguousarray(X, dtype=np.int8)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    b = np.ascontiguousarray(v11, dtype=np.uint8)
    M = X.shape[0]
    acc = np.empty((M, N), dtype=np.int32)
    out = np.empty((M, N), dtype=np.float32)
    lib().orc_gemm_v11(_ptr(X), _ptr(xs), M, _ptr(b), float(ws), K, N, _ptr(acc), _ptr(out))
    return acc, out


# --------------------------------------------------------------------------
# Quantizers
# --------------------------------------------------------------------------
def quant_int8(x: np.ndarray) -> Tuple[np.ndarray, np.float32]:
    """quant_int8_k (cuda/ter_cuda_forward_packed.cu:40-62): fp32 -> (int8, act_scale)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.shape, dtype=np.int8)
    s = np.zeros(1, dtype=np.float32)
    lib().orc_quant_int8(_ptr(x), x.size, _ptr(q), _ptr(s))
    return q, s[0]


def quant_int8_rows(x: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    q = np.empty((M, K), dtype=np.int8)
    s = np.empty(M, dtype=np.float32)
    lib().orc_quant_int8_rows(_ptr(x), M, K, _ptr(q), _ptr(s))
    return q, s


def rmsnorm_quant(x: np.ndarray, gamma: np.ndarray, eps: float = 1e-5):
    """rmsnorm_quant_{f32,fp16}_in_k (cuda/ter_cuda_forward_bitnet.cu:64-146):
    x fp32 or fp16 [H], gamma fp16 [H] -> (int8 [H], act_scale, rms_inv)."""
    gamma = np.ascontiguousarray(gamma, dtype=np.float16)
    if x.dtype == np.float16:
        x16, x32 = np.ascontiguousarray(x), None
    else:
        x16, x32 = None, np.ascontiguousarray(x, dtype=np.float32)
    H = (x16 if x16 is not None else x32).size
    q = np.empty(H, dtype=np.int8)
    s = np.zeros(1, dtype=np.float32)
    r = np.zeros(1, dtype=np.float32)
    lib().orc_rmsnorm_quant(_ptr(x32) if x32 is not None else None, _ptr(x16) if x16 is not None else None,
                            _ptr(gamma), H, C.c_float(eps), _ptr(q), _ptr(s), _ptr(r))
    return q, s[0], r[0]


def float_to_half_bits(x: np.ndarray) -> np.ndarray:
    """binary32 -> binary16 bit patterns, round to nearest even."""
    f = np.ascontiguousarray(x, dtype=np.float32).ravel()
    h = np.empty(f.size, dtype=np.uint16)
    lib().orc_float_to_half_n(_ptr(f), _ptr(h), f.size)
    return h


def relu2_rmsnorm_quant(gate: np.ndarray, up: np.ndarray, gamma: np.ndarray, eps: float = 1e-5):
    """relu2_mul_rmsnorm_quant_k (cuda/ter_cuda_forward_bitnet.cu:258-309):
    fp16 gate, up, gamma [F] -> (int8 [F], act_scale, rms_inv)."""
    g = np.ascontiguousarray(gate, dtype=np.float16)
    u = np.ascontiguousarray(up, dtype=np.float16)
    gm = np.ascontiguousarray(gamma, dtype=np.float16)
    F = g.size
    q = np.empty(F, dtype=np.int8)
    s = np.zeros(1, dtype=np.float32)
    r = np.zeros(1, dtype=np.float32)
    lib().orc_relu2_rmsnorm_quant(_ptr(g), _ptr(u), _ptr(gm), F, C.c_float(eps), _ptr(q), _ptr(s), _ptr(r))
    return q, s[0], r[0]


def residual_add_f16(hidden: np.ndarray, y: np.ndarray) -> np.ndarray:
    """add_k_f32 after an fp16 GEMV output: hidden + float(half(y))."""
    h = np.array(hidden, dtype=np.float32, copy=True)
    yy = np.ascontiguousarray(y, dtype=np.float32)
    lib().orc_residual_add_f16(_ptr(h), _ptr(yy), h.size)
    return h


def residual_add_h16(hidden: np.ndarray, y: np.ndarray) -> np.ndarray:
    """add_k (cuda/ter_cuda_forward_packed.cu:113-116) after an fp16 GEMV
    output: fp16 hidden + half(y), rounded to fp16."""
    h = np.array(hidden, dtype=np.float16, copy=True)
    yy = np.ascontiguousarray(y, dtype=np.float32)
    lib().orc_residual_add_h16(_ptr(h), _ptr(yy), h.size)
    return h


def silu_mul_quant(gate: np.ndarray, up: np.ndarray):
    """silu_mul_quant_k (cuda/ter_cuda_forward_packed.cu:312-344): fp16 gate,
    up [F] -> (int8 [F], act_scale, fp32 silu(gate) * up [F])."""
    g = np.ascontiguousarray(gate, dtype=np.float16)
    u = np.ascontiguousarray(up, dtype=np.float16)
    F = g.size
    q = np.empty(F, dtype=np.int8)
    s = np.zeros(1, dtype=np.float32)
    v = np.empty(F, dtype=np.float32)
    lib().orc_silu_mul_quant(_ptr(g), _ptr(u), F, _ptr(q), _ptr(s), _ptr(v))
    return q, s[0], v


def silu_f16(gate: np.ndarray) -> np.ndarray:
    """The first step of silu_mul_quant_k (cuda/ter_cuda_forward_packed.cu:322-324)
    alone: fp16 gate [F] -> fp32 g / (1 + expf(-g))."""
    g = np.ascontiguousarray(gate, dtype=np.float16)
    out = np.empty(g.size, dtype=np.float32)
    lib().orc_silu_f16(_ptr(g), g.size, _ptr(out))
    return out


def smul_quant(s: np.ndarray, up: np.ndarray):
    """The rest of silu_mul_quant_k (:325-343): fp32 silu(gate) [F] times fp16
    up [F] -> (int8 [F], act_scale, fp32 products [F])."""
    ss = np.ascontiguousarray(s, dtype=np.float32)
    u = np.ascontiguousarray(up, dtype=np.float16)
    F = ss.size
    q = np.empty(F, dtype=np.int8)
    sc = np.zeros(1, dtype=np.float32)
    v = np.empty(F, dtype=np.float32)
    lib().orc_smul_quant(_ptr(ss), _ptr(u), F, _ptr(q), _ptr(sc), _ptr(v))
    return q, sc[0], v


def rmsnorm_f16(x: np.ndarray, gamma: np.ndarray, eps: float = 1e-5):
    """rmsnorm_f32_in_k (cuda/ter_cuda_forward_bitnet.cu:37-47): fp32 x [H],
    fp16 gamma [H] -> (fp16 y [H], rms_inv)."""
    xx = np.ascontiguousarray(x, dtype=np.float32)
    gm = np.ascontiguousarray(gamma, dtype=np.float16)
    y = np.empty(xx.size, dtype=np.uint16)
    r = np.zeros(1, dtype=np.float32)
    lib().orc_rmsnorm_f16(_ptr(xx), _ptr(gm), xx.size, C.c_float(eps), _ptr(y), _ptr(r))
    return y.view(np.float16), r[0]


def lm_head_f16(x: np.ndarray, emb: np.ndarray):
    """mm_fp16_lm_head_k (cuda/ter_cuda_forward_bitnet.cu:388-429): fp16 x [H],
    fp16 token_embd [V][H] -> (fp16 logits [V], fp32 pre-rounding values [V])."""
    xx = np.ascontiguousarray(x, dtype=np.float16)
    E = np.ascontiguousarray(emb, dtype=np.float16)
    V, H = E.shape
    lg = np.empty(V, dtype=np.uint16)
    acc = np.empty(V, dtype=np.float32)
    lib().orc_lm_head_f16(_ptr(xx), _ptr(E), H, V, _ptr(lg), _ptr(acc))
    return lg.view(np.float16), acc


def argmax_f16(logits: np.ndarray) -> int:
    """argmax_local_k + argmax_final_k (cuda/ter_cuda_forward_bitnet.cu:454-495)."""
    lg = np.ascontiguousarray(logits, dtype=np.float16)
    return int(lib().orc_argmax_f16(_ptr(lg), lg.size))


def expf(x: np.ndarray) -> np.ndarray:
    """The attention softmax's binary32 exp (orc_expf)."""
    xx = np.ascontiguousarray(x, dtype=np.float32).ravel()
    y = np.empty_like(xx)
    lib().orc_expf_n(_ptr(xx), _ptr(y), xx.size)
    return y.reshape(np.shape(x))


def rope_table(theta: float, hd: int, n_pos: int) -> np.ndarray:
    """NEOX RoPE (cos, sin) table [n_pos][hd/2][2] (rope_k's steps)."""
    cs = np.empty((n_pos, hd // 2, 2), dtype=np.float32)
    lib().orc_rope_table(C.c_float(theta), hd, n_pos, _ptr(cs))
    return cs


def rope_f16(v: np.ndarray, cs_pos: np.ndarray, neox: bool = True) -> np.ndarray:
    """rope_k on fp16 head vectors v [n_heads][hd] with table row cs_pos [hd/2][2]."""
    out = np.array(v, dtype=np.float16, copy=True, order="C")
    nh, hd = out.shape
    cp = np.ascontiguousarray(cs_pos, dtype=np.float32)
    lib().orc_rope_f16(_ptr(out), nh, hd, _ptr(cp), 1 if neox else 0)
    return out


def _attention(fn, q, K, V):
    qq = np.ascontiguousarray(q, dtype=np.float16)
    KK = np.ascontiguousarray(K, dtype=np.float16)
    VV = np.ascontiguousarray(V, dtype=np.float16)
    nh, hd = qq.shape
    seq, nkv, _ = KK.shape
    o16 = np.empty((nh, hd), dtype=np.uint16)
    o32 = np.empty((nh, hd), dtype=np.float32)
    fn(_ptr(qq), _ptr(KK), _ptr(VV), nh, nkv, hd, seq, _ptr(o16), _ptr(o32))
    return o16.view(np.float16), o32


def attention_ref(q, K, V):
    """attention_k (cuda/ter_cuda_forward_bitnet.cu:336-374): q fp16 [nh][hd],
    K, V fp16 [seq][nkv][hd] -> (fp16 out [nh][hd], fp32 pre-rounding)."""
    return _attention(lib().orc_attention_ref, q, K, V)


def attention_splitk(q, K, V):
    """The GPU kernel's chunked order (64-position chunks)."""
    return _attention(lib().orc_attention_splitk, q, K, V)


def quantize_bitnet(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size, dtype=np.int8)
    s = lib().orc_quantize_bitnet(_ptr(x), x.size, _ptr(out))
    return out, np.float32(s)


def quantize_nt(x: np.ndarray, n_trits: int = 9):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size, dtype=np.int32)
    s = lib().orc_quantize_nt(_ptr(x), x.size, int(n_trits), _ptr(out))
    return out, np.float32(s)


def dequant_i2s(buf: np.ndarray, n: int) -> np.ndarray:
    b = np.ascontiguousarray(buf, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    lib().orc_dequant_i2s(_ptr(b), n, _ptr(out))
    return out


def i2s_to_v11(raw: np.ndarray, K: int, N: int) -> np.ndarray:
    b = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty((N // 4) * K, dtype=np.uint8)
    rc = lib().orc_i2s_to_v11(_ptr(b), K, N, _ptr(out))
    if rc != 0:
        raise ValueError(f"orc_i2s_to_v11 rc={rc}")
    return out


def mm_row_tvmac(K: int, N: int) -> int:
    return int(lib().orc_mm_row_tvmac(K, N))


# --------------------------------------------------------------------------
# The reference itself (oracle/_ref), for pinning the restatement and as the
# CPU baseline.
# --------------------------------------------------------------------------
class RefMmRow:
    """Holds reference TritTensors for X [rows][K] and W [K][N]; run() calls
    the reference mm_row (src/tx/forward.cpp:299-352) only."""

    def __init__(self, X: np.ndarray, xs: float, W: np.ndarray, ws: float,
                 block_scales: Optional[np.ndarray] = None, block_size: int = 0):
        X = np.ascontiguousarray(X, dtype=np.int32)
        W = np.ascontiguousarray(W, dtype=np.int32)
        if X.ndim == 1:
            X = X.reshape(1, -1)
        self.rows, self.K = X.shape
        K2, self.N = W.shape
        assert K2 == self.K
        bs = None
        if block_size > 0:
            bs = np.ascontiguousarray(block_scales, dtype=np.float32)
        self._h = ref().ter_ref_ctx_new(_ptr(X), self.rows, self.K, float(xs), _ptr(W), self.N,
                                        float(ws), _ptr(bs) if bs is not None else None, int(block_size))
        if not self._h:
            raise MemoryError("ter_ref_ctx_new failed")
        self.out = np.empty(self.N, dtype=np.float32)

    def run(self, row: int = 0) -> np.ndarray:
        rc = ref().ter_ref_ctx_run(self._h, int(row), _ptr(self.out))
        if rc != 0:
            raise RuntimeError(f"ter_ref_ctx_run rc={rc}")
        return self.out

    def tvmac(self) -> int:
        return int(ref().ter_ref_ctx_tvmac(self._h))

    def close(self):
        if self._h:
            ref().ter_ref_ctx_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def ref_quantize(x: np.ndarray, n_trits: int = 9):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size, dtype=np.int32)
    s = ref().ter_ref_quantize(_ptr(x), x.size, int(n_trits), _ptr(out))
    return out, np.float32(s)


def ref_quantize_bitnet(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size, dtype=np.int8)
    s = ref().ter_ref_quantize_bitnet(_ptr(x), x.size, _ptr(out))
    return out, np.float32(s)


# --------------------------------------------------------------------------
# Portable seeded generators for test inputs (splitmix64; explicit integer ->
# range mappings, so fixtures never depend on a C++ standard library's
# distribution implementation).
# --------------------------------------------------------------------------
_M64 = (1 << 64) - 1


def splitmix64(seed: int, n: int) -> np.ndarray:
    """n outputs of splitmix64 starting from state `seed` (vectorised)."""
    idx = np.arange(1, n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & _M64) + idx * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def rand_trits(seed: int, K: int, N: int, p_zero: float = 1.0 / 3.0) -> np.ndarray:
    """Trits [K][N] in {-1,0,1}: P(0)=p_zero, P(+1)=P(-1)=(1-p_zero)/2."""
    u = (splitmix64(seed, K * N) >> np.uint64(32)).astype(np.uint64)  # 32-bit uniform
    t0 = np.uint64(int(round(p_zero * 2 ** 32)))
    t1 = t0 + np.uint64(int(round((1.0 - p_zero) / 2.0 * 2 ** 32)))
    w = np.where(u < t0, 0, np.where(u < t1, 1, -1)).astype(np.int8)
    return w.reshape(K, N)


def rand_int8(seed: int, n: int, lo: int = -127, hi: int = 127) -> np.ndarray:
    u = (splitmix64(seed, n) >> np.uint64(32)).astype(np.uint64)
    span = np.uint64(hi - lo + 1)
    return ((u * span) >> np.uint64(32)).astype(np.int64).__add__(lo).astype(np.int8)


def rand_normal_f32(seed: int, n: int) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.standard_normal(n, dtype=np.float32)


def gemv_v11_cols(x: np.ndarray, xs: float, v11: np.ndarray, ws: float, K: int, N: int,
                  byte_cols: np.ndarray):
    """orc_gemv_v11 restricted to the v11 byte-columns `byte_cols` (each covers
    output columns 4*jb .. 4*jb+3).  Returns (cols, acc, out) for those columns;
    used to check full-size GEMVs on a sample of columns."""
    jbs = np.asarray(sorted(set(int(j) for j in byte_cols)), dtype=np.int64)
    v = np.ascontiguousarray(v11, dtype=np.uint8).reshape(N // 4, K)[jbs].reshape(-1)
    acc, out = gemv_v11(x, xs, v, ws, K, 4 * len(jbs))
    cols = (4 * jbs[:, None] + np.arange(4)[None, :]).reshape(-1)
    return cols, acc, out
