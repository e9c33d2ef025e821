"""BitNet-b1.58 single-token decode step on the fabric (the host side of the
reference's forward_token_dev, cuda/ter_cuda_forward_bitnet.cu:848-913).

The reference launches ~15 kernels per layer (norms, quantizers, 7 GEMVs,
RoPE twice, the KV copy, attention, two residual adds).  Here a layer is five
launches: one work-list plan for Q/K/V with the RMSNorm prologue and fp16
outputs, the attention context (RoPE + cache write + attention), the
o-projection with the fp16 sub-norm prologue adding into the fp32 hidden
stream, gate/up, and the down projection with the relu^2 sub-norm prologue
adding into the hidden stream.  The token ends with the fused RMSNorm +
lm_head + argmax, which also advances the position; it starts with the
embedding lookup.  Every buffer is preallocated, the position and token live
on the device, and the whole step replays from one HIP graph.

Model structure (Model / Layer / Scratch, :615-650): fp16 norms and tied
fp16 token_embd, ternary projections packed as T16, KV caches
[layers][s_max][n_kv * head_dim] fp16.
"""
from __future__ import annotations

import dataclasses
from typing import List, Optional

from . import fabric as F


@dataclasses.dataclass
class Shape:
    """Model shape (the reference's Cfg, cuda/ter_cuda_forward_bitnet.cu:29-32)."""
    H: int = 2560
    F: int = 6912
    Nl: int = 30
    Nh: int = 20
    Nkv: int = 5
    Hd: int = 128
    V: int = 128256
    eps: float = 1e-5
    rope_theta: float = 500000.0


PROJ = ("Wq", "Wk", "Wv", "Wo", "Wgate", "Wup", "Wdown")


def proj_shapes(c: Shape):
    hkv = c.Nkv * c.Hd
    return {"Wq": (c.H, c.Nh * c.Hd), "Wk": (c.H, hkv), "Wv": (c.H, hkv), "Wo": (c.Nh * c.Hd, c.H),
            "Wgate": (c.H, c.F), "Wup": (c.H, c.F), "Wdown": (c.F, c.H)}


@dataclasses.dataclass
class Layer:
    W: dict                 # name -> PackedTrits
    attn_norm: object       # fp16 [H]
    attn_sub_norm: object   # fp16 [Nh * Hd]
    ffn_norm: object        # fp16 [H]
    ffn_sub_norm: object    # fp16 [F]


@dataclasses.dataclass
class Model:
    shape: Shape
    layers: List[Layer]
    token_embd: object      # fp16 [V][H] (tied lm_head)
    output_norm: object     # fp16 [H]


def random_model(c: Shape, seed: int = 1, p_zero: float = 0.4) -> Model:
    """Random-init model of shape c (the reference's bench mode, :786-823):
    seeded ternary projections with per-tensor scales, norms U[0.5, 1.5],
    token_embd N(0, 1) * 0.03."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    shapes = proj_shapes(c)
    layers = []
    for l in range(c.Nl):
        W = {}
        for i, nm in enumerate(PROJ):
            K, N = shapes[nm]
            s = seed * 1_000_003 + l * 101 + i
            scale = 0.01 + 0.09 * (((s * 2654435761) & 0xFFFFFFFF) / 2 ** 32)
            W[nm] = F.PackedTrits.from_v11(F.synth_v11(K, N, seed=s, p_zero=p_zero), K, N, scale)

        def norm(n):
            return (torch.rand(n, generator=g, device="cuda") + 0.5).to(torch.float16)
        layers.append(Layer(W, norm(c.H), norm(c.Nh * c.Hd), norm(c.H), norm(c.F)))
    emb = (torch.randn(c.V, c.H, generator=g, device="cuda") * 0.03).to(torch.float16)
    out_norm = (torch.rand(c.H, generator=g, device="cuda") + 0.5).to(torch.float16)
    return Model(c, layers, emb, out_norm)


class Decoder:
    """Scratch buffers, KV caches and launch plans for greedy decode
    (Scratch, :631-650).  step() decodes the token in `token` at position
    `pos` (both device int32) and leaves the next token in `token` and
    pos + 1 in `pos`."""

    def __init__(self, model: Model, s_max: int):
        import torch
        c = model.shape
        self.model, self.s_max = model, s_max
        dev, f16, f32 = "cuda", torch.float16, torch.float32
        hq, hkv = c.Nh * c.Hd, c.Nkv * c.Hd
        self.hidden = torch.zeros(c.H, dtype=f32, device=dev)
        self.q = torch.empty(hq, dtype=f16, device=dev)
        self.k = torch.empty(hkv, dtype=f16, device=dev)
        self.v = torch.empty(hkv, dtype=f16, device=dev)
        self.attn_out = torch.empty(hq, dtype=f16, device=dev)
        self.gate = torch.empty(c.F, dtype=f16, device=dev)
        self.up = torch.empty(c.F, dtype=f16, device=dev)
        self.K = torch.zeros((c.Nl, s_max, c.Nkv, c.Hd), dtype=f16, device=dev)
        self.V = torch.zeros((c.Nl, s_max, c.Nkv, c.Hd), dtype=f16, device=dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.argmax = F.ArgmaxState(dev)
        self.attn = F.Attention(c.Nh, c.Nkv, c.Hd, s_max, c.rope_theta, neox=True)
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
            o = F.Plan([dict(w=W["Wo"], x=self.attn_out, gamma=lay.attn_sub_norm, eps=c.eps, resid=self.hidden)])
            gu = F.Plan([dict(w=W["Wgate"], x=self.hidden, gamma=lay.ffn_norm, eps=c.eps, y16=self.gate),
                         dict(w=W["Wup"], x=self.hidden, gamma=lay.ffn_norm, eps=c.eps, y16=self.up)])
            dn = F.Plan([dict(w=W["Wdown"], x=self.gate, up=self.up, gamma=lay.ffn_sub_norm, eps=c.eps,
                              resid=self.hidden)])
            self.plans.append((qkv, o, gu, dn))
        self._graph = None

    def step(self, stream=None):
        """One token (launches only; nothing synchronizes)."""
        m, c = self.model, self.model.shape
        F.embed_f16(m.token_embd, self.token, self.hidden, stream=stream)
        for l, (qkv, o, gu, dn) in enumerate(self.plans):
            qkv.launch(stream)
            self.attn.decode(self.q, self.k, self.v, self.K[l], self.V[l], self.pos, self.attn_out, stream=stream)
            o.launch(stream)
            gu.launch(stream)
            dn.launch(stream)
        F.lm_head_argmax(self.hidden, m.output_norm, m.token_embd, c.eps, token_out=self.token, state=self.argmax,
                         pos_advance=self.pos, stream=stream)

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
        return 2 + 5 * len(self.plans)

    def close(self):
        for ps in self.plans:
            for p in ps:
                p.close()
        self.attn.close()
