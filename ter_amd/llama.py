"""Llama single-token decode step on the fabric (the host side of the
reference's packed-trit Llama forward_token_dev,
cuda/ter_cuda_forward_packed.cu:505-560).

The reference runs, per layer: rmsnorm_quant_fp16_in_k on the fp16 hidden
stream, three GEMVs (Q, K, V), RoPE twice, the KV copy, attention_k,
quant_int8_k on the fp16 attention output, the O GEMV, add_k into the fp16
hidden stream, rmsnorm_quant_fp16_in_k, gate and up, silu_mul_quant_k, the
down GEMV and add_k again.  Here a layer is five launches: the Q/K/V plan
(fp16 RMSNorm prologue, fp16 outputs), the attention context (NORM RoPE,
cache write, attention), the O projection (absmax prologue on the fp16
attention output, fp16 residual epilogue), the gate/up plan and the down
projection (silu(gate) * up prologue, fp16 residual epilogue; the SiLU of
each gate value is computed once, by the gate GEMV's epilogue).

The token tail has two forms, as in the reference (:541-557):
  * bench mode, a ternary lm_head [H][V] (alloc_model, :446-472): the fp16
    RMSNorm prologue, the packed GEMV to fp16 logits, then the argmax;
  * tied weights (an 'LLRT' file, :588-664): RMSNorm to fp16, the fp16
    lm_head over token_embd and the argmax, in one launch.
Every buffer is preallocated, the position and token live on the device, and
the step replays from one HIP graph.
"""
from __future__ import annotations

import dataclasses
from typing import List, Optional

from . import fabric as F

PROJ = ("Wq", "Wk", "Wv", "Wo", "Wgate", "Wup", "Wdown")


@dataclasses.dataclass
class Shape:
    """Model shape (the reference's Cfg, cuda/ter_cuda_forward_packed.cu:22-25:
    Llama-3.2-1B)."""
    H: int = 2048
    F: int = 8192
    Nl: int = 16
    Nh: int = 32
    Nkv: int = 8
    Hd: int = 64
    V: int = 128256
    eps: float = 1e-5
    rope_theta: float = 500000.0


def proj_shapes(c: Shape):
    hkv = c.Nkv * c.Hd
    return {"Wq": (c.H, c.Nh * c.Hd), "Wk": (c.H, hkv), "Wv": (c.H, hkv), "Wo": (c.Nh * c.Hd, c.H),
            "Wgate": (c.H, c.F), "Wup": (c.H, c.F), "Wdown": (c.F, c.H)}


@dataclasses.dataclass
class Layer:
    W: dict            # name -> PackedTrits
    attn_norm: object  # fp16 [H]
    ffn_norm: object   # fp16 [H]


@dataclasses.dataclass
class Model:
    shape: Shape
    layers: List[Layer]
    token_embd: object      # fp16 [V][H]
    output_norm: object     # fp16 [H]
    lm_head: Optional[F.PackedTrits] = None  # ternary [H][V]; None: tied to token_embd


WEIGHT_SCALE = 0.05  # alloc_packed's per-matrix scale (cuda/ter_cuda_forward_packed.cu:443)


def weight_seed(seed: int, layer: int, i: int) -> int:
    """The splitmix64 seed of projection i of a layer (layer -1: the lm_head)."""
    return seed * 1_000_003 + (layer + 1) * 101 + i


def random_model(c: Shape, seed: int = 1, p_zero: float = 0.4, tied: bool = False) -> Model:
    """Random-init model of shape c (the reference's bench mode, alloc_model,
    cuda/ter_cuda_forward_packed.cu:446-472): seeded ternary projections with
    the scale 0.05, norms U[0.5, 1.5], token_embd N(0, 1) * 0.03, and a
    ternary lm_head unless `tied`."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    shapes = proj_shapes(c)

    def norm(n):
        return (torch.rand(n, generator=g, device="cuda") + 0.5).to(torch.float16)

    layers = []
    for l in range(c.Nl):
        W = {}
        for i, nm in enumerate(PROJ):
            K, N = shapes[nm]
            W[nm] = F.PackedTrits.from_v11(F.synth_v11(K, N, seed=weight_seed(seed, l, i), p_zero=p_zero), K, N,
                                           WEIGHT_SCALE)
        layers.append(Layer(W, norm(c.H), norm(c.H)))
    emb = (torch.randn(c.V, c.H, generator=g, device="cuda") * 0.03).to(torch.float16)
    out_norm = norm(c.H)
    head = None
    if not tied:
        head = F.PackedTrits.from_v11(F.synth_v11(c.H, c.V, seed=weight_seed(seed, -1, 0), p_zero=p_zero), c.H, c.V,
                                      WEIGHT_SCALE)
    return Model(c, layers, emb, out_norm, head)


def from_file(path: str) -> Model:
    """An 'LLRT' file (tools/convert_llama_to_packed.py) as a Model with the
    lm_head tied to token_embd, as load_model_from_bin does (:588-664)."""
    from . import modelfile
    m = modelfile.load_llama(path)
    h = m.header
    if h["H"] != h["Nh"] * h["Hd"] or h["Nh"] % h["Nkv"]:
        raise ValueError(f"{path}: H={h['H']} is not Nh*Hd={h['Nh']}*{h['Hd']}, or Nh % Nkv != 0")
    shape = Shape(H=h["H"], F=h["F"], Nl=h["Nl"], Nh=h["Nh"], Nkv=h["Nkv"], Hd=h["Hd"], V=h["V"],
                  eps=float(h["eps"]), rope_theta=float(h["rope_theta"]))
    layers = [Layer(l.W, l.attn_norm, l.ffn_norm) for l in m.layers]
    return Model(shape, layers, m.token_embd, m.output_norm, None)


class Decoder:
    """Scratch buffers, KV caches and launch plans for greedy decode (Scratch,
    cuda/ter_cuda_forward_packed.cu:474-487).  step() decodes the token in
    `token` at position `pos` (both device int32) and leaves the next token in
    `token` and pos + 1 in `pos`."""

    def __init__(self, model: Model, s_max: int):
        import torch
        c = model.shape
        self.model, self.s_max = model, s_max
        dev, f16 = "cuda", torch.float16
        hq, hkv = c.Nh * c.Hd, c.Nkv * c.Hd
        if hq != c.H:
            raise ValueError("the Llama forward needs H == Nh * Hd")
        self.hidden = torch.zeros(c.H, dtype=f16, device=dev)
        self.q = torch.empty(hq, dtype=f16, device=dev)
        self.k = torch.empty(hkv, dtype=f16, device=dev)
        self.v = torch.empty(hkv, dtype=f16, device=dev)
        self.attn_out = torch.empty(hq, dtype=f16, device=dev)
        self.gate_silu = torch.empty(c.F, dtype=torch.float32, device=dev)
        self.up = torch.empty(c.F, dtype=f16, device=dev)
        self.K = torch.zeros((c.Nl, s_max, c.Nkv, c.Hd), dtype=f16, device=dev)
        self.V = torch.zeros((c.Nl, s_max, c.Nkv, c.Hd), dtype=f16, device=dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.argmax = F.ArgmaxState(dev)
        self.attn = F.Attention(c.Nh, c.Nkv, c.Hd, s_max, c.rope_theta, neox=False)
        # every projection of the model in one allocation, each layer's in
        # the order Q, K, V, O, gate, up, down (views replace the model's
        # weights): the Q/K/V and gate/up plans then load the activation and
        # the weights from the launch's arguments (fabric.group_contiguous)
        order = [(lay.W, nm) for lay in model.layers for nm in PROJ]
        for (W, nm), w in zip(order, F.group_contiguous([W[nm] for W, nm in order])):
            W[nm] = w
        del order
        self.plans = []
        for lay in model.layers:
            W = lay.W
            qkv = F.Plan([dict(w=W["Wq"], x=self.hidden, gamma=lay.attn_norm, eps=c.eps, y16=self.q),
                          dict(w=W["Wk"], x=self.hidden, gamma=lay.attn_norm, eps=c.eps, y16=self.k),
                          dict(w=W["Wv"], x=self.hidden, gamma=lay.attn_norm, eps=c.eps, y16=self.v)])
            o = F.Plan([dict(w=W["Wo"], x=self.attn_out, resid16=self.hidden)])
            # silu_mul_quant_k split in two: the gate GEMV's epilogue writes
            # silu(half(gate)) once per element, the down projection's
            # prologue multiplies by up and quantizes (bit for bit the fused
            # form, without an exp per element in every down workgroup)
            gu = F.Plan([dict(w=W["Wgate"], x=self.hidden, gamma=lay.ffn_norm, eps=c.eps, silu=self.gate_silu),
                         dict(w=W["Wup"], x=self.hidden, gamma=lay.ffn_norm, eps=c.eps, y16=self.up)])
            dn = F.Plan([dict(w=W["Wdown"], x=self.gate_silu, up=self.up, resid16=self.hidden)])
            self.plans.append((qkv, o, gu, dn))
        self.logits = None
        self.head = None
        if model.lm_head is not None:
            if (model.lm_head.K, model.lm_head.N) != (c.H, c.V):
                raise ValueError("lm_head must be [H][V]")
            self.logits = torch.empty(c.V, dtype=f16, device=dev)
            self.head = F.Plan([dict(w=model.lm_head, x=self.hidden, gamma=model.output_norm, eps=c.eps,
                                     y16=self.logits)])
        self._graph = None

    def step(self, stream=None):
        """One token (launches only; nothing synchronizes)."""
        m, c = self.model, self.model.shape
        F.embed_h16(m.token_embd, self.token, self.hidden, stream=stream)
        for l, (qkv, o, gu, dn) in enumerate(self.plans):
            qkv.launch(stream)
            self.attn.decode(self.q, self.k, self.v, self.K[l], self.V[l], self.pos, self.attn_out, stream=stream)
            o.launch(stream)
            gu.launch(stream)
            dn.launch(stream)
        if self.head is None:
            F.lm_head_argmax(self.hidden, m.output_norm, m.token_embd, c.eps, token_out=self.token,
                             state=self.argmax, pos_advance=self.pos, stream=stream)
        else:
            self.head.launch(stream)
            F.argmax_f16(self.logits, self.token, self.argmax, pos_advance=self.pos, stream=stream)

    def capture(self):
        """The step as a HIP graph (position and token are read on the device,
        so one graph serves every token)."""
        import torch
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):  # records the launches; nothing runs
            self.step()
        torch.cuda.synchronize()
        self._graph = g
        return g

    def launches_per_token(self) -> int:
        return 2 + 5 * len(self.plans) + (1 if self.head is not None else 0)

    def close(self):
        for ps in self.plans:
            for p in ps:
                p.close()
        if self.head is not None:
            self.head.close()
        self.attn.close()
