"""Host-side interface of the gfx950 packed-trit fabric.

Mirrors the reference's operator surface for this path, over the C-ABI of
include/ter_hip.h (ctypes).  PyTorch is used only for device memory and
streams.

Reference names kept:
  PackedTrits           <- WPK{data, scale, bytes}       cuda/ter_cuda_forward_packed.cu:400
  mm_packed_dispatch    <- mm_packed_dispatch(...)       cuda/ter_cuda_forward_packed.cu:493-500
  mm_row                <- mm_row(sim, kt, id, Xt, row, Wt, K, N, out)   src/tx/forward.cpp:299-352
  mm_batched            <- mm_bitnet_addonly_batched_k<M>(...)          cuda/ter_cuda_addonly_batched.cu:31-124
  quant_int8            <- quant_int8_k(x, y, scale_out, N)             cuda/ter_cuda_forward_packed.cu:40-62
  Handle                <- ter_k4_create/call/op_counts/...             include/ter_k4/ter_k4.h:29-55
"""
from __future__ import annotations

import ctypes as C
from typing import List, Optional, Sequence

import numpy as np

from . import _lib as L


def _torch():
    import torch  # imported lazily: the C-ABI checks below need no device
    return torch


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(stream=None) -> Optional[int]:
    if stream is not None:
        return stream
    torch = _torch()
    return torch.cuda.current_stream().cuda_stream


def _require_cuda(t, name: str, dtype=None, numel: Optional[int] = None):
    torch = _torch()
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a CUDA (HIP) tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if numel is not None and t.numel() < numel:
        raise ValueError(f"{name} holds {t.numel()} elements, needs {numel}")


class PackedTrits:
    """A K x N ternary weight resident on the device in the T16 tile layout.

    Built from reference v11 bytes (the packed wire format of
    tools/convert_llama_to_packed.py:128-140) or from a TritTensor payload
    (int32 [K][N], include/ter/numfmt.hpp:17-36)."""

    def __init__(self, K: int, N: int, scale: float, device=None):
        torch = _torch()
        self.K, self.N = int(K), int(N)
        nbytes = L.lib().ter_hip_wpk_bytes(self.K, self.N)
        if nbytes == 0:
            raise ValueError(f"bad shape K={K} N={N}")
        self.buf = torch.empty(nbytes, dtype=torch.uint8, device=device or "cuda")
        self.wpk = L.WPK()
        L.check(L.lib().ter_hip_wpk_init(C.byref(self.wpk), self.buf.data_ptr(), nbytes, self.K, self.N,
                                         float(scale)), "ter_hip_wpk_init")

    @property
    def scale(self) -> float:
        return self.wpk.scale

    @property
    def magnitude(self) -> int:
        """m of a {-m, 0, +m} payload (1 for plain trits): y = float(m * acc) * scale."""
        return self.wpk.mag

    @property
    def nbytes_packed(self) -> int:
        """Algorithmic packed bytes K*N/4 (the reference GB/s convention)."""
        return self.K * self.N // 4

    @classmethod
    def from_v11(cls, v11, K: int, N: int, scale: float, stream=None) -> "PackedTrits":
        torch = _torch()
        if isinstance(v11, np.ndarray):
            v11 = torch.from_numpy(np.ascontiguousarray(v11, dtype=np.uint8)).cuda()
        _require_cuda(v11, "v11", torch.uint8, (N // 4) * K)
        w = cls(K, N, scale, device=v11.device)
        L.check(L.lib().ter_hip_pack_v11(C.byref(w.wpk), v11.data_ptr(), _stream(stream)), "ter_hip_pack_v11")
        return w

    @classmethod
    def from_i2s(cls, i2s, K: int, N: int, scale: float, stream=None) -> "PackedTrits":
        """Device repack of a GGUF i2_s tensor's codes (N*K/4 bytes; the
        per-tensor fp32 scale that follows them in the file is `scale`)."""
        torch = _torch()
        if isinstance(i2s, np.ndarray):
            i2s = torch.from_numpy(np.ascontiguousarray(i2s, dtype=np.uint8)).cuda()
        _require_cuda(i2s, "i2s", torch.uint8, N * K // 4)
        w = cls(K, N, scale, device=i2s.device)
        L.check(L.lib().ter_hip_pack_i2s(C.byref(w.wpk), i2s.data_ptr(), _stream(stream)), "ter_hip_pack_i2s")
        return w

    @classmethod
    def from_payload(cls, payload: np.ndarray, scale: float, stream=None) -> "PackedTrits":
        p = np.ascontiguousarray(payload, dtype=np.int32)
        K, N = p.shape
        w = cls(K, N, scale)
        m = C.c_int32(0)
        L.check(L.lib().ter_hip_pack_payload(C.byref(w.wpk), p.ctypes.data, float(scale), C.byref(m),
                                             _stream(stream)), "ter_hip_pack_payload")
        return w

    def to_v11(self, stream=None):
        torch = _torch()
        out = torch.empty((self.N // 4) * self.K, dtype=torch.uint8, device=self.buf.device)
        L.check(L.lib().ter_hip_unpack_v11(C.byref(self.wpk), out.data_ptr(), _stream(stream)),
                "ter_hip_unpack_v11")
        return out


def group_contiguous(ws: Sequence[PackedTrits]) -> List[PackedTrits]:
    """The weights `ws` copied into one device allocation, their tile streams
    back to back in the given order and their fix-up slots after all of them;
    returns views into it (same shapes, scales and magnitudes).  A strip-mode
    plan whose items read one activation vector (so one K) and whose weights
    are such a group, in the same order, starts its activation and weight
    loads from the launch's arguments instead of waiting for its descriptors
    (the decode steps group each layer's Q/K/V and gate/up this way); a
    stream-K plan over such a group reads one contiguous weight stream."""
    torch = _torch()
    if not ws:
        raise ValueError("group_contiguous needs at least one weight")
    lib = L.lib()
    stream_b = [int(lib.ter_hip_wpk_bytes(w.K, w.N)) - 8 * w.N for w in ws]
    total = sum(stream_b) + sum(8 * w.N for w in ws)
    buf = torch.empty(total, dtype=torch.uint8, device=ws[0].buf.device)
    out = []
    off, foff = 0, sum(stream_b)
    for w, sb in zip(ws, stream_b):
        buf[off:off + sb].copy_(w.buf[:sb])
        buf[foff:foff + 8 * w.N].zero_()  # fix-up slots, zero at rest
        v = PackedTrits.__new__(PackedTrits)
        v.K, v.N, v.buf = w.K, w.N, buf
        v.wpk = L.WPK()
        v.wpk.data = buf.data_ptr() + off
        v.wpk.bytes = lib.ter_hip_wpk_bytes(w.K, w.N)
        v.wpk.fix = buf.data_ptr() + foff
        v.wpk.K, v.wpk.N, v.wpk.scale = w.K, w.N, w.scale
        v.wpk.layout, v.wpk.mag = w.wpk.layout, w.wpk.mag
        out.append(v)
        off += sb
        foff += 8 * w.N
    return out


def _act(x, x_scale=None, x_scale_dev=None, q_out=None, scale_out=None, gamma=None, eps=1e-5, up=None) -> L.Act:
    torch = _torch()
    a = L.Act()
    a.data = x.data_ptr()
    if up is not None and gamma is None:
        # silu(gate) * up, then absmax quantization (silu_mul_quant_k); with an
        # fp32 x, x is silu(gate) already (a gate GEMV's silu output)
        if x.dtype not in (torch.float16, torch.float32) or up.dtype != torch.float16 or not up.is_cuda \
                or up.shape != x.shape:
            raise TypeError("silu activations: gate (fp16) or silu(gate) (fp32) and fp16 up of one shape")
        a.kind = L.X_SILU_MUL if x.dtype == torch.float16 else L.X_SMUL
        a.up = up.data_ptr()
        a.q_out = _ptr(q_out)
        a.scale_out = _ptr(scale_out)
    elif gamma is not None:
        # fused RMSNorm (fp16 gamma) + absmax quantization in the prologue
        if gamma.dtype != torch.float16 or not gamma.is_cuda:
            raise TypeError("gamma must be a CUDA float16 tensor")
        if up is not None:
            if x.dtype != torch.float16 or up.dtype != torch.float16 or not up.is_cuda or up.shape != x.shape:
                raise TypeError("relu^2 activations: gate and up must be CUDA float16 tensors of one shape")
            a.kind = L.X_RELU2_RMS
            a.up = up.data_ptr()
        elif x.dtype == torch.float32:
            a.kind = L.X_F32_RMS
        elif x.dtype == torch.float16:
            a.kind = L.X_F16_RMS
        else:
            raise TypeError(f"RMSNorm activations must be float32 or float16, got {x.dtype}")
        a.gamma = gamma.data_ptr()
        a.eps = float(eps)
        a.q_out = _ptr(q_out)
        a.scale_out = _ptr(scale_out)
    elif x.dtype in (torch.int8, torch.int16):
        a.kind = L.X_I8 if x.dtype == torch.int8 else L.X_I16
        a.scale = float(x_scale) if x_scale is not None else 1.0
        a.scale_dev = _ptr(x_scale_dev)
    elif x.dtype in (torch.float32, torch.float16):
        # absmax quantization in the prologue (quant_int8_k)
        a.kind = L.X_F32 if x.dtype == torch.float32 else L.X_F16
        a.q_out = _ptr(q_out)
        a.scale_out = _ptr(scale_out)
    else:
        raise TypeError(f"activations must be int8, int16, float32 or float16, got {x.dtype}")
    return a


def _out(y, acc, y16, resid, resid16=None, silu=None) -> L.Out:
    o = L.Out()
    o.y, o.acc, o.y16, o.resid, o.resid16 = _ptr(y), _ptr(acc), _ptr(y16), _ptr(resid), _ptr(resid16)
    o.silu = _ptr(silu)
    return o


def gemv(W: PackedTrits, x, y=None, acc=None, x_scale: Optional[float] = None, x_scale_dev=None,
         q_out=None, scale_out=None, gamma=None, eps: float = 1e-5, up=None, y16=None, resid=None, resid16=None,
         silu=None, stream=None):
    """M = 1 GEMV.  x: int8 or int16 [K] (with x_scale or x_scale_dev), or fp32 /
    fp16 [K] (absmax-quantized in the kernel prologue, quant_int8_k); with gamma
    (fp16 [K]), x fp32 or fp16 is RMS-normalized first (rmsnorm_quant_*_in_k
    steps), and with up as well, x is the fp16 gate and the prologue is
    relu2_mul_rmsnorm_quant_k; with up but no gamma, silu_mul_quant_k (x the
    fp16 gate), or its second half (x the fp32 silu(gate) a gate GEMV's silu
    output wrote).  Outputs: y fp32, acc int32, y16 fp16 = half(y), resid fp32
    += half(y), resid16 fp16 = half(resid16 + half(y)), silu fp32 =
    silu(half(y)); y is allocated when none is given.  Returns (y, acc)."""
    torch = _torch()
    _require_cuda(x, "x", None, W.K)
    if y is None and acc is None and y16 is None and resid is None and resid16 is None and silu is None:
        y = torch.empty(W.N, dtype=torch.float32, device=x.device)
    a = _act(x, x_scale, x_scale_dev, q_out, scale_out, gamma, eps, up)
    if y16 is None and resid is None and resid16 is None and silu is None:
        L.check(L.lib().ter_hip_gemv(C.byref(W.wpk), C.byref(a), _ptr(y), _ptr(acc), _stream(stream)),
                "ter_hip_gemv")
    else:
        o = _out(y, acc, y16, resid, resid16, silu)
        L.check(L.lib().ter_hip_gemv_out(C.byref(W.wpk), C.byref(a), C.byref(o), _stream(stream)),
                "ter_hip_gemv_out")
    return y, acc


def mm_packed_dispatch(X, scale_x_dev, W: PackedTrits, out, K: int, N: int, stream=None):
    """The reference launcher signature (cuda/ter_cuda_forward_packed.cu:493-500),
    fp32 out instead of fp16."""
    torch = _torch()
    _require_cuda(X, "X", torch.int8, K)
    _require_cuda(scale_x_dev, "scale_x_dev", torch.float32, 1)
    _require_cuda(out, "out", torch.float32, N)
    L.check(L.lib().ter_hip_mm_packed_dispatch(X.data_ptr(), scale_x_dev.data_ptr(), C.byref(W.wpk),
                                               out.data_ptr(), int(K), int(N), _stream(stream)),
            "ter_hip_mm_packed_dispatch")
    return out


def mm_packed_dispatch_f16(X, scale_x_dev, W: PackedTrits, out, K: int, N: int, stream=None):
    """The reference launcher with its own output type: fp16 out[N] =
    __float2half((float)acc * scale) (cuda/ter_cuda_forward_packed.cu:493-500)."""
    torch = _torch()
    _require_cuda(X, "X", torch.int8, K)
    _require_cuda(scale_x_dev, "scale_x_dev", torch.float32, 1)
    _require_cuda(out, "out", torch.float16, N)
    L.check(L.lib().ter_hip_mm_packed_dispatch_f16(X.data_ptr(), scale_x_dev.data_ptr(), C.byref(W.wpk),
                                                   out.data_ptr(), int(K), int(N), _stream(stream)),
            "ter_hip_mm_packed_dispatch_f16")
    return out


def mm_row(Xt_payload: np.ndarray, row: int, x_scale: float, W: PackedTrits, K: int, N: int) -> np.ndarray:
    """The mm_row contract (src/tx/forward.cpp:299-352): host TritTensor
    payload X (int32 [rows][K]) -> host fp32 out[N], bit for bit the
    reference's.  Rows that fit int8 run the int8 GEMV, rows that fit int16
    (the host forward's 9-trit activations) the int16 GEMV."""
    torch = _torch()
    X = np.ascontiguousarray(Xt_payload, dtype=np.int32)
    out = np.empty(N, dtype=np.float32)
    xs = torch.empty(2 * K, dtype=torch.int8, device=W.buf.device)
    ys = torch.empty(N, dtype=torch.float32, device=W.buf.device)
    L.check(L.lib().ter_hip_mm_row(X.ctypes.data, int(row), int(K), float(x_scale), C.byref(W.wpk), int(N),
                                   out.ctypes.data, xs.data_ptr(), ys.data_ptr(), _stream(None)),
            "ter_hip_mm_row")
    return out


def mm_row_blocked(Xt_payload: np.ndarray, row: int, x_scale: float, W: PackedTrits, K: int, N: int,
                   block_scales, block_size: int) -> np.ndarray:
    """The per-block branch of mm_row (src/tx/forward.cpp:308-330): W's
    TritTensor carries block_scales (fp32 [ceil(K*N / block_size)], here a
    CUDA tensor or a host array); host fp32 out[N], bit for bit the
    reference's double accumulation."""
    torch = _torch()
    X = np.ascontiguousarray(Xt_payload, dtype=np.int32)
    if isinstance(block_scales, np.ndarray):
        block_scales = torch.from_numpy(np.ascontiguousarray(block_scales, dtype=np.float32)).to(W.buf.device)
    _require_cuda(block_scales, "block_scales", torch.float32, -(-K * N // int(block_size)))
    out = np.empty(N, dtype=np.float32)
    xs = torch.empty(2 * K, dtype=torch.int8, device=W.buf.device)
    ys = torch.empty(N, dtype=torch.float32, device=W.buf.device)
    L.check(L.lib().ter_hip_mm_row_blocked(X.ctypes.data, int(row), int(K), float(x_scale), C.byref(W.wpk), int(N),
                                           block_scales.data_ptr(), int(block_size), out.ctypes.data, xs.data_ptr(),
                                           ys.data_ptr(), _stream(None)), "ter_hip_mm_row_blocked")
    return out


def quant_int8(x, q=None, scale_out=None, stream=None):
    """Per-row absmax int8 quantization of fp32 x [M][K] (quant_int8_k steps)."""
    torch = _torch()
    x2 = x.reshape(-1, x.shape[-1])
    M, K = x2.shape
    if q is None:
        q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    if scale_out is None:
        scale_out = torch.empty(M, dtype=torch.float32, device=x.device)
    L.check(L.lib().ter_hip_quant_int8(x2.data_ptr(), M, K, q.data_ptr(), scale_out.data_ptr(), _stream(stream)),
            "ter_hip_quant_int8")
    return q, scale_out


def rmsnorm_quant(x, gamma, eps: float = 1e-5, q=None, scale_out=None, stream=None):
    """Per-row fused RMSNorm + int8 quantization (rmsnorm_quant_{f32,fp16}_in_k,
    cuda/ter_cuda_forward_bitnet.cu:64-146) of x fp32 or fp16 [M][K] with fp16
    gamma [K].  Returns (q int8 [M][K], scale_out fp32 [M])."""
    torch = _torch()
    x2 = x.reshape(-1, x.shape[-1])
    M, K = x2.shape
    kind = {torch.float32: L.X_F32_RMS, torch.float16: L.X_F16_RMS}.get(x.dtype)
    if kind is None:
        raise TypeError(f"x must be float32 or float16, got {x.dtype}")
    if gamma.dtype != torch.float16 or gamma.numel() != K:
        raise TypeError("gamma must be float16 [K]")
    if q is None:
        q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    if scale_out is None:
        scale_out = torch.empty(M, dtype=torch.float32, device=x.device)
    L.check(L.lib().ter_hip_rmsnorm_quant(x2.data_ptr(), kind, gamma.data_ptr(), C.c_float(eps), M, K, q.data_ptr(),
                                          scale_out.data_ptr(), _stream(stream)), "ter_hip_rmsnorm_quant")
    return q, scale_out


def relu2_rmsnorm_quant(gate, up, gamma, eps: float = 1e-5, q=None, scale_out=None, stream=None):
    """Per-row fused relu^2(gate) * up + RMSNorm + int8 quantization
    (relu2_mul_rmsnorm_quant_k, cuda/ter_cuda_forward_bitnet.cu:258-309) of fp16
    gate, up [M][F] with fp16 gamma [F].  Returns (q int8 [M][F], scale_out fp32 [M])."""
    torch = _torch()
    g2, u2 = gate.reshape(-1, gate.shape[-1]), up.reshape(-1, up.shape[-1])
    M, F = g2.shape
    if gate.dtype != torch.float16 or up.dtype != torch.float16 or u2.shape != g2.shape:
        raise TypeError("gate and up must be float16 tensors of one shape")
    if gamma.dtype != torch.float16 or gamma.numel() != F:
        raise TypeError("gamma must be float16 [F]")
    if q is None:
        q = torch.empty((M, F), dtype=torch.int8, device=gate.device)
    if scale_out is None:
        scale_out = torch.empty(M, dtype=torch.float32, device=gate.device)
    L.check(L.lib().ter_hip_relu2_rmsnorm_quant(g2.data_ptr(), u2.data_ptr(), gamma.data_ptr(), C.c_float(eps), M, F,
                                                q.data_ptr(), scale_out.data_ptr(), _stream(stream)),
            "ter_hip_relu2_rmsnorm_quant")
    return q, scale_out


def mm_batched(W: PackedTrits, X, y=None, acc=None, x_scale_dev=None, q_out=None, scale_out=None, gamma=None,
               eps: float = 1e-5, up=None, y16=None, resid=None, stream=None):
    """M > 1 GEMM on MFMA.  X: int8 [M][K] with per-row device scales
    x_scale_dev [M], or fp32 [M][K] (rows quantized into q_out/scale_out,
    allocated here when absent); with gamma (fp16 [K]) the fp32 or fp16 rows
    are RMS-normalized first, with up as well X is the fp16 gate of the
    relu^2 prologue.  Outputs as gemv, [M][N] each.  Returns (y, acc)."""
    torch = _torch()
    _require_cuda(X, "X")
    M = X.shape[0]
    if y is None and acc is None and y16 is None and resid is None:
        y = torch.empty((M, W.N), dtype=torch.float32, device=X.device)
    if X.dtype in (torch.float32, torch.float16):
        if q_out is None:
            q_out = torch.empty((M, W.K), dtype=torch.int8, device=X.device)
        if scale_out is None:
            scale_out = torch.empty(M, dtype=torch.float32, device=X.device)
    a = _act(X, None, x_scale_dev, q_out, scale_out, gamma, eps, up)
    if y16 is None and resid is None:
        L.check(L.lib().ter_hip_gemm(C.byref(W.wpk), C.byref(a), int(M), _ptr(y), _ptr(acc), _stream(stream)),
                "ter_hip_gemm")
    else:
        o = _out(y, acc, y16, resid)
        L.check(L.lib().ter_hip_gemm_out(C.byref(W.wpk), C.byref(a), int(M), C.byref(o), _stream(stream)),
                "ter_hip_gemm_out")
    return y, acc


def rmsnorm_f16(x, gamma, eps: float = 1e-5, y=None, stream=None):
    """Per-row RMSNorm with fp16 output (rmsnorm_f32_in_k,
    cuda/ter_cuda_forward_bitnet.cu:37-47): fp32 x [M][H], fp16 gamma [H]."""
    torch = _torch()
    x2 = x.reshape(-1, x.shape[-1])
    M, H = x2.shape
    if x.dtype != torch.float32 or gamma.dtype != torch.float16 or gamma.numel() != H:
        raise TypeError("x must be float32 [M][H] and gamma float16 [H]")
    if y is None:
        y = torch.empty((M, H), dtype=torch.float16, device=x.device)
    L.check(L.lib().ter_hip_rmsnorm_f16(x2.data_ptr(), gamma.data_ptr(), C.c_float(eps), M, H, y.data_ptr(),
                                        _stream(stream)), "ter_hip_rmsnorm_f16")
    return y


def lm_head_f16(x_norm, token_embd, logits=None, stream=None):
    """fp16 lm_head GEMV (mm_fp16_lm_head_k, cuda/ter_cuda_forward_bitnet.cu:388-429):
    x_norm fp16 [H], token_embd fp16 [V][H] -> logits fp16 [V]."""
    torch = _torch()
    V, H = token_embd.shape
    if x_norm.dtype != torch.float16 or token_embd.dtype != torch.float16 or x_norm.numel() != H:
        raise TypeError("x_norm must be float16 [H] and token_embd float16 [V][H]")
    if logits is None:
        logits = torch.empty(V, dtype=torch.float16, device=x_norm.device)
    L.check(L.lib().ter_hip_lm_head_f16(x_norm.data_ptr(), token_embd.data_ptr(), logits.data_ptr(), H, V,
                                        _stream(stream)), "ter_hip_lm_head_f16")
    return logits


class ArgmaxState:
    """The device state of the one-launch argmax (TER_HIP_ARGMAX_STATE_BYTES,
    zero at rest; every call leaves it zero)."""

    def __init__(self, device="cuda"):
        torch = _torch()
        self.t = torch.zeros(L.ARGMAX_STATE_BYTES // 8, dtype=torch.int64, device=device)

    def ptr(self) -> int:
        return self.t.data_ptr()


def argmax_f16(logits, out_idx=None, state: Optional[ArgmaxState] = None, pos_advance=None, stream=None):
    """argmax of fp16 logits with the reference's index (ties included):
    argmax_local_k + argmax_final_k (cuda/ter_cuda_forward_bitnet.cu:454-495);
    with pos_advance (device int32 [1]) also inc_pos_k
    (cuda/ter_cuda_forward_packed.cu:559)."""
    torch = _torch()
    if logits.dtype != torch.float16:
        raise TypeError("logits must be float16")
    if out_idx is None:
        out_idx = torch.empty(1, dtype=torch.int32, device=logits.device)
    if state is None:
        state = ArgmaxState(logits.device)
    if pos_advance is None:
        L.check(L.lib().ter_hip_argmax_f16(logits.data_ptr(), logits.numel(), out_idx.data_ptr(), state.ptr(),
                                           _stream(stream)), "ter_hip_argmax_f16")
    else:
        if pos_advance.dtype != torch.int32:
            raise TypeError("pos_advance must be int32")
        L.check(L.lib().ter_hip_argmax_f16_step(logits.data_ptr(), logits.numel(), out_idx.data_ptr(), state.ptr(),
                                                pos_advance.data_ptr(), _stream(stream)), "ter_hip_argmax_f16_step")
    return out_idx


def embed_f16(token_embd, token_dev, hidden=None, stream=None):
    """token_embed_lookup_k: hidden fp32 [H] = token_embd[*token_dev] (fp16 [V][H])."""
    torch = _torch()
    V, H = token_embd.shape
    if hidden is None:
        hidden = torch.empty(H, dtype=torch.float32, device=token_embd.device)
    L.check(L.lib().ter_hip_embed_f16(token_embd.data_ptr(), V, H, token_dev.data_ptr(), hidden.data_ptr(),
                                      _stream(stream)), "ter_hip_embed_f16")
    return hidden


def embed_h16(token_embd, token_dev, hidden16=None, stream=None):
    """token_embed_lookup_k of the Llama forward: hidden16 fp16 [H] = token_embd[*token_dev]."""
    torch = _torch()
    V, H = token_embd.shape
    if hidden16 is None:
        hidden16 = torch.empty(H, dtype=torch.float16, device=token_embd.device)
    L.check(L.lib().ter_hip_embed_h16(token_embd.data_ptr(), V, H, token_dev.data_ptr(), hidden16.data_ptr(),
                                      _stream(stream)), "ter_hip_embed_h16")
    return hidden16


def lm_head_argmax(hidden, gamma, token_embd, eps: float = 1e-5, token_out=None, state: Optional[ArgmaxState] = None,
                   x_norm_out=None, logits_out=None, pos_advance=None, stream=None):
    """The decode step's tail in one launch (cuda/ter_cuda_forward_bitnet.cu:890-911,
    cuda/ter_cuda_forward_packed.cu:550-557): RMSNorm of hidden [H] (fp32, or
    the Llama forward's fp16 stream) -> fp16 lm_head over token_embd [V][H] ->
    argmax.  Returns token_out (int32 [1])."""
    torch = _torch()
    V, H = token_embd.shape
    if hidden.dtype not in (torch.float32, torch.float16) or hidden.numel() != H:
        raise TypeError("hidden must be float32 or float16 [H]")
    if gamma.dtype != torch.float16 or token_embd.dtype != torch.float16:
        raise TypeError("gamma and token_embd must be float16")
    if token_out is None:
        token_out = torch.empty(1, dtype=torch.int32, device=hidden.device)
    if state is None:
        state = ArgmaxState(hidden.device)
    fn = "ter_hip_lm_head_argmax" if hidden.dtype == torch.float32 else "ter_hip_lm_head_argmax_h16"
    L.check(getattr(L.lib(), fn)(hidden.data_ptr(), gamma.data_ptr(), C.c_float(eps), token_embd.data_ptr(),
                                 H, V, _ptr(x_norm_out), _ptr(logits_out), token_out.data_ptr(),
                                 state.ptr(), _ptr(pos_advance), _stream(stream)), fn)
    return token_out


class Attention:
    """Decode-attention context (ter_hip_attn_*): RoPE + KV-cache write +
    attention in one launch per layer (rope_k, kv_copy_k, attention_k,
    cuda/ter_cuda_forward_bitnet.cu:185-214, 336-374)."""

    def __init__(self, n_heads: int, n_kv_heads: int, head_dim: int, s_max: int, theta: float,
                 neox: bool = True):
        h = C.c_void_p()
        L.check(L.lib().ter_hip_attn_create(C.byref(h), n_heads, n_kv_heads, head_dim, s_max, C.c_float(theta),
                                            L.ROPE_NEOX if neox else L.ROPE_NORM), "ter_hip_attn_create")
        self._h = h
        self.n_heads, self.n_kv_heads, self.head_dim, self.s_max = n_heads, n_kv_heads, head_dim, s_max

    def decode(self, q, k, v, k_cache, v_cache, pos_dev, out=None, stream=None):
        """q fp16 [nh][hd], k, v fp16 [nkv][hd] (before RoPE); caches fp16
        [s_max][nkv][hd]; pos_dev int32 [1].  Returns out fp16 [nh][hd]."""
        torch = _torch()
        for t, nm in ((q, "q"), (k, "k"), (v, "v"), (k_cache, "k_cache"), (v_cache, "v_cache")):
            if t.dtype != torch.float16 or not t.is_cuda:
                raise TypeError(f"{nm} must be a CUDA float16 tensor")
        if q.numel() != self.n_heads * self.head_dim or k.numel() != self.n_kv_heads * self.head_dim \
                or v.numel() != k.numel():
            raise ValueError("q, k or v has the wrong size")
        if k_cache.numel() < self.s_max * self.n_kv_heads * self.head_dim or v_cache.numel() < k_cache.numel():
            raise ValueError("caches must hold s_max positions")
        if out is None:
            out = torch.empty((self.n_heads, self.head_dim), dtype=torch.float16, device=q.device)
        L.check(L.lib().ter_hip_attn_decode(self._h, q.data_ptr(), k.data_ptr(), v.data_ptr(), k_cache.data_ptr(),
                                            v_cache.data_ptr(), pos_dev.data_ptr(), out.data_ptr(), _stream(stream)),
                "ter_hip_attn_decode")
        return out

    def rope(self, x, pos_dev, stream=None):
        """RoPE in place on fp16 head vectors x [n][hd]."""
        n = x.numel() // self.head_dim
        L.check(L.lib().ter_hip_rope(self._h, x.data_ptr(), n, pos_dev.data_ptr(), _stream(stream)), "ter_hip_rope")
        return x

    def close(self):
        if getattr(self, "_h", None):
            L.lib().ter_hip_attn_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _held(it: dict) -> list:
    """What a plan built from item `it` must keep alive: the device table
    holds raw pointers into the weight buffer (as it was when the plan was
    built) and into every tensor of the item, so none of them may be freed
    while the plan can still be launched."""
    return [it["w"], it["w"].buf] + [v for k, v in it.items() if k != "w" and hasattr(v, "data_ptr")]


class Plan:
    """Many independent GEMVs in one launch (one work list).  `items` is a
    sequence of dicts: {w: PackedTrits, x: tensor, y?, acc?, y16?, resid?,
    resid16?, silu?, x_scale?, x_scale_dev?, q_out?, scale_out?, gamma?, eps?, up?}."""

    def __init__(self, items: Sequence[dict], wg_per_cu: int = 0):
        n = len(items)
        arr = (L.GemvItem * n)()
        self._keep: List = []
        for i, it in enumerate(items):
            W = it["w"]
            arr[i].w = C.pointer(W.wpk)
            arr[i].x = _act(it["x"], it.get("x_scale"), it.get("x_scale_dev"), it.get("q_out"), it.get("scale_out"),
                            it.get("gamma"), it.get("eps", 1e-5), it.get("up"))
            arr[i].y = _ptr(it.get("y"))
            arr[i].acc = _ptr(it.get("acc"))
            arr[i].y16 = _ptr(it.get("y16"))
            arr[i].resid = _ptr(it.get("resid"))
            arr[i].resid16 = _ptr(it.get("resid16"))
            arr[i].silu = _ptr(it.get("silu"))
            self._keep.extend(_held(it))
        h = C.c_void_p()
        L.check(L.lib().ter_hip_plan_create(C.byref(h), arr, n, int(wg_per_cu)), "ter_hip_plan_create")
        self._h = h
        b, m, g = C.c_uint64(), C.c_uint64(), C.c_int32()
        L.check(L.lib().ter_hip_plan_stats(self._h, C.byref(b), C.byref(m), C.byref(g)), "ter_hip_plan_stats")
        self.bytes, self.macs, self.n_wg = b.value, m.value, g.value
        md = C.c_int32()
        L.check(L.lib().ter_hip_plan_mode(self._h, C.byref(md)), "ter_hip_plan_mode")
        self.mode = md.value  # TER_HIP_PLAN_* flags

    def launch(self, stream=None):
        L.check(L.lib().ter_hip_plan_launch(self._h, _stream(stream)), "ter_hip_plan_launch")

    def close(self):
        if getattr(self, "_h", None):
            L.lib().ter_hip_plan_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GemmPlan:
    """Many independent M > 1 GEMMs in one launch.  `items` is a sequence of
    dicts {w: PackedTrits, x: int8 [M][K] tensor, x_scale_dev: fp32 [M]
    tensor, y?: fp32 [M][N], acc?: int32 [M][N], y16?: fp16 [M][N],
    resid?: fp32 [M][N]}."""

    def __init__(self, items: Sequence[dict], wg_per_cu: int = 0):
        n = len(items)
        arr = (L.GemmItem * n)()
        self._keep: List = []
        torch = _torch()
        for i, it in enumerate(items):
            W, x = it["w"], it["x"]
            _require_cuda(x, "x", torch.int8)
            if x.dim() != 2 or x.shape[1] != W.K:
                raise ValueError(f"item {i}: x must be [M][{W.K}]")
            arr[i].w = C.pointer(W.wpk)
            arr[i].x = x.data_ptr()
            arr[i].x_scale_dev = _ptr(it.get("x_scale_dev"))
            arr[i].M = int(x.shape[0])
            arr[i].y = _ptr(it.get("y"))
            arr[i].acc = _ptr(it.get("acc"))
            arr[i].y16 = _ptr(it.get("y16"))
            arr[i].resid = _ptr(it.get("resid"))
            self._keep.extend(_held(it))
        h = C.c_void_p()
        L.check(L.lib().ter_hip_gemm_plan_create(C.byref(h), arr, n, int(wg_per_cu)), "ter_hip_gemm_plan_create")
        self._h = h
        b, m, g = C.c_uint64(), C.c_uint64(), C.c_int32()
        L.check(L.lib().ter_hip_plan_stats(self._h, C.byref(b), C.byref(m), C.byref(g)), "ter_hip_plan_stats")
        self.bytes, self.macs, self.n_wg = b.value, m.value, g.value

    def launch(self, stream=None):
        L.check(L.lib().ter_hip_plan_launch(self._h, _stream(stream)), "ter_hip_plan_launch")

    def close(self):
        if getattr(self, "_h", None):
            L.lib().ter_hip_plan_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Handle:
    """K4-style handle with the KernelTable native slot (ter_k4_create /
    ter_k4_call / ter_k4_op_counts, include/ter_k4/ter_k4.h:29-55)."""

    def __init__(self, device: int = 0):
        self._h = L.lib().ter_hip_create(int(device))
        if not self._h:
            raise MemoryError("ter_hip_create failed")
        self._fns = []

    def install_native(self, name: str, fn) -> int:
        cb = L.NATIVE_FN(fn)
        self._fns.append(cb)
        return L.lib().ter_hip_install_native(self._h, name.encode(), cb)

    def call(self, name: str, args: Sequence[int]) -> int:
        a = (C.c_int64 * max(1, len(args)))(*[int(v) for v in args])
        return L.lib().ter_hip_call(self._h, name.encode() if name is not None else None, a, len(args))

    def matmul(self, W: PackedTrits, x, y=None, acc=None, x_scale=None, x_scale_dev=None, M: int = 1,
               q_out=None, scale_out=None, stream=None) -> int:
        """Call the native packed-GEMV slot (TER_HIP_SLOT_MATMUL)."""
        a = _act(x, x_scale, x_scale_dev, q_out, scale_out)
        self._last_act = a
        args = [C.addressof(W.wpk), C.addressof(a), _ptr(y) or 0, _ptr(acc) or 0, _stream(stream) or 0, int(M)]
        return self.call(L.SLOT_MATMUL.decode(), args)

    def op_counts(self) -> dict:
        c = L.OpCounts()
        L.lib().ter_hip_op_counts(self._h, C.byref(c))
        return {f: getattr(c, f) for f, _ in L.OpCounts._fields_}

    def reset_counters(self):
        L.lib().ter_hip_reset_counters(self._h)

    def close(self):
        if getattr(self, "_h", None):
            L.lib().ter_hip_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def synth_v11(K: int, N: int, seed: int, p_zero: float = 1.0 / 3.0, device="cuda", stream=None):
    """Synthetic reference-v11 weight bytes generated on the device (counter-
    based splitmix64; element k*N+n draws trit 0 with P=p_zero, else +1/-1
    with equal probability)."""
    torch = _torch()
    t0 = int(round(p_zero * 2 ** 32))
    t1 = t0 + int(round((1.0 - p_zero) / 2.0 * 2 ** 32))
    out = torch.empty((N // 4) * K, dtype=torch.uint8, device=device)
    L.check(L.lib().ter_hip_synth_v11(out.data_ptr(), int(K), int(N), int(seed) & (2 ** 64 - 1), t0,
                                      min(t1, 2 ** 32 - 1), _stream(stream)), "ter_hip_synth_v11")
    return out


def noop(stream=None):
    """One empty kernel launch (the launch floor)."""
    L.check(L.lib().ter_hip_noop(_stream(stream)), "ter_hip_noop")


def read_probe(buf, nbytes: int, n_wg: int, sink, stream=None):
    """Pure streaming read of nbytes of `buf` with the GEMV's partition over
    n_wg workgroups (a measurement ceiling; sink: int32 [4 * n_wg])."""
    L.check(L.lib().ter_hip_read_probe(buf.data_ptr(), int(nbytes), int(n_wg), sink.data_ptr(), _stream(stream)),
            "ter_hip_read_probe")


def synth_i8(n: int, seed: int, lo: int = -127, hi: int = 127, device="cuda", stream=None):
    torch = _torch()
    out = torch.empty(n, dtype=torch.int8, device=device)
    L.check(L.lib().ter_hip_synth_i8(out.data_ptr(), int(n), int(seed) & (2 ** 64 - 1), int(lo), int(hi),
                                     _stream(stream)), "ter_hip_synth_i8")
    return out
