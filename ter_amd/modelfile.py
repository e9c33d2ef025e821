"""Packed model files (.bin) through the library's reader (modelfile.hip).

The formats are the flat blobs of the reference's converters:
'TERT' (tools/convert_bitnet_to_packed.py, BitNet b1.58: norms, sub-norms,
relu^2 FFN) and 'LLRT' (tools/convert_llama_to_packed.py, Llama ternarized
per tensor), read by the two load_model_from_bin
(cuda/ter_cuda_forward_bitnet.cu:698-784, cuda/ter_cuda_forward_packed.cu:589-659).
As there, fp16 token_embd is uploaded as stored, fp32 norms become fp16
(round to nearest even), and each projection's v11 bytes and fp32 scale
become a packed weight (here repacked to T16 on the device).
"""
from __future__ import annotations

import ctypes as C
import dataclasses
from typing import List

import numpy as np

from . import _lib as L
from . import bitnet
from .fabric import PackedTrits, _stream

PROJ = bitnet.PROJ


class BinFile:
    """An open model file: header fields, the tensor directory, readers."""

    def __init__(self, path: str):
        h = C.c_void_p()
        hdr = L.BinHeader()
        L.check(L.lib().ter_hip_bin_open(str(path).encode(), C.byref(h), C.byref(hdr)), f"ter_hip_bin_open({path})")
        self._h = h
        self.header = hdr
        self.tensors: List[L.BinTensor] = []
        for i in range(L.lib().ter_hip_bin_count(h)):
            t = L.BinTensor()
            L.check(L.lib().ter_hip_bin_tensor(h, i, C.byref(t)), "ter_hip_bin_tensor")
            self.tensors.append(t)

    @property
    def format(self) -> str:
        return "TERT" if self.header.magic == L.BIN_TERT else "LLRT"

    def find(self, name: str, layer: int = -1) -> int:
        i = L.lib().ter_hip_bin_find(self._h, name.encode(), int(layer))
        if i < 0:
            L.check(i, f"ter_hip_bin_find({name}, {layer})")
        return i

    def read_host(self, i: int, as_f16: bool = False) -> np.ndarray:
        """Tensor i on the host: fp16, fp32 (or fp16 with as_f16) or the v11 bytes."""
        t = self.tensors[i]
        if t.kind == L.BIN_TRITS:
            out = np.empty(t.bytes, np.uint8)
        elif t.kind == L.BIN_F16 or as_f16:
            out = np.empty(t.n, np.float16)
        else:
            out = np.empty(t.n, np.float32)
        L.check(L.lib().ter_hip_bin_read_host(self._h, i, out.ctypes.data, int(as_f16)), "ter_hip_bin_read_host")
        return out

    def upload_f16(self, i: int, stream=None):
        """Tensor i (fp16, or an fp32 norm rounded to fp16) as a device tensor."""
        import torch
        t = self.tensors[i]
        out = torch.empty(t.n, dtype=torch.float16, device="cuda")
        L.check(L.lib().ter_hip_bin_upload_f16(self._h, i, out.data_ptr(), _stream(stream)), "ter_hip_bin_upload_f16")
        return out

    def upload_wpk(self, i: int, stage=None, stream=None) -> PackedTrits:
        """Projection i as a packed weight; `stage` is an optional uint8 device
        buffer of at least K*N/4 bytes for the v11 bytes."""
        import torch
        t = self.tensors[i]
        if stage is None or stage.numel() < t.bytes:
            stage = torch.empty(int(t.bytes), dtype=torch.uint8, device="cuda")
        w = PackedTrits(t.K, t.N, t.scale)
        L.check(L.lib().ter_hip_bin_upload_wpk(self._h, i, C.byref(w.wpk), stage.data_ptr(), _stream(stream)),
                "ter_hip_bin_upload_wpk")
        return w

    def close(self):
        if getattr(self, "_h", None):
            L.lib().ter_hip_bin_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _stage_for(f: BinFile):
    import torch
    n = max(int(t.bytes) for t in f.tensors if t.kind == L.BIN_TRITS)
    return torch.empty(n, dtype=torch.uint8, device="cuda")


def load_bitnet(path: str) -> bitnet.Model:
    """A 'TERT' file as a bitnet.Model (the decoder's input)."""
    with BinFile(path) as f:
        if f.format != "TERT":
            raise ValueError(f"{path}: a {f.format} file, not a BitNet ('TERT') file")
        h = f.header
        if h.H != h.Nh * h.Hd or h.Nh % h.Nkv:
            raise ValueError(f"{path}: H={h.H} is not Nh*Hd={h.Nh}*{h.Hd}, or Nh % Nkv != 0")
        shape = bitnet.Shape(H=h.H, F=h.F, Nl=h.Nl, Nh=h.Nh, Nkv=h.Nkv, Hd=h.Hd, V=h.V, eps=float(h.eps),
                             rope_theta=float(h.rope_theta))
        stage = _stage_for(f)
        layers = []
        for l in range(h.Nl):
            W = {nm: f.upload_wpk(f.find(nm, l), stage) for nm in PROJ}
            layers.append(bitnet.Layer(W, f.upload_f16(f.find("attn_norm", l)), f.upload_f16(f.find("attn_sub_norm", l)),
                                       f.upload_f16(f.find("ffn_norm", l)), f.upload_f16(f.find("ffn_sub_norm", l))))
        emb = f.upload_f16(f.find("token_embd")).view(h.V, h.H)
        return bitnet.Model(shape, layers, emb, f.upload_f16(f.find("output_norm")))


@dataclasses.dataclass
class LlamaLayer:
    W: dict             # name -> PackedTrits
    attn_norm: object   # fp16 [H]
    ffn_norm: object    # fp16 [H]


@dataclasses.dataclass
class LlamaModel:
    """An 'LLRT' file's tensors (the Llama forward's Model, without its host loop)."""
    header: dict
    layers: List[LlamaLayer]
    token_embd: object  # fp16 [V][H] (tied lm_head)
    output_norm: object


def load_llama(path: str) -> LlamaModel:
    with BinFile(path) as f:
        if f.format != "LLRT":
            raise ValueError(f"{path}: a {f.format} file, not a Llama ('LLRT') file")
        h = f.header
        stage = _stage_for(f)
        layers = [LlamaLayer({nm: f.upload_wpk(f.find(nm, l), stage) for nm in PROJ},
                             f.upload_f16(f.find("attn_norm", l)), f.upload_f16(f.find("ffn_norm", l)))
                  for l in range(h.Nl)]
        hdr = {n: getattr(h, n) for n, _ in L.BinHeader._fields_}
        return LlamaModel(hdr, layers, f.upload_f16(f.find("token_embd")).view(h.V, h.H),
                          f.upload_f16(f.find("output_norm")))
