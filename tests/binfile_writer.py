"""Writer of small packed model files for the loader tests: the byte
sequence of tools/convert_bitnet_to_packed.py ('TERT') and
tools/convert_llama_to_packed.py ('LLRT') -- the 64-byte header
(struct '<II' magic/version, '<IIIIIIII' H F Nl V Nh Nkv Hd Smax, '<ff'
rope_theta eps, zero padding), token_embd fp16, output_norm fp32, then per
layer the fp32 norms and the seven projections, each K*(N/4) v11 bytes and
its '<f' scale -- from arrays instead of a GGUF file.  Test infrastructure."""
import struct

import numpy as np

from oracle import oracle as O

TERT, LLRT = 0x54455254, 0x4C4C5254
PROJ = ("Wq", "Wk", "Wv", "Wo", "Wgate", "Wup", "Wdown")


def proj_shapes(H, F, Hkv):
    return {"Wq": (H, H), "Wk": (H, Hkv), "Wv": (H, Hkv), "Wo": (H, H), "Wgate": (H, F), "Wup": (H, F),
            "Wdown": (F, H)}


def random_model(magic, H, F, Nl, V, Nh, Nkv, Hd, Smax=64, theta=500000.0, eps=1e-5, seed=0):
    """Arrays of a random model: fp16 token_embd, fp32 norms, v11 projections
    with scales (trits with P(0) = 0.4)."""
    rng = np.random.default_rng(seed)
    hdr = dict(magic=magic, version=1, H=H, F=F, Nl=Nl, V=V, Nh=Nh, Nkv=Nkv, Hd=Hd, Smax=Smax, rope_theta=theta,
               eps=eps)
    emb = (rng.standard_normal((V, H)) * 0.05).astype(np.float16)
    out_norm = rng.uniform(0.5, 1.5, H).astype(np.float32)
    shapes = proj_shapes(H, F, Nkv * Hd)
    layers = []
    for l in range(Nl):
        lay = dict(attn_norm=rng.uniform(0.5, 1.5, H).astype(np.float32),
                   ffn_norm=rng.uniform(0.5, 1.5, H).astype(np.float32))
        if magic == TERT:
            lay["attn_sub_norm"] = rng.uniform(0.5, 1.5, H).astype(np.float32)
            lay["ffn_sub_norm"] = rng.uniform(0.5, 1.5, F).astype(np.float32)
        for i, nm in enumerate(PROJ):
            K, N = shapes[nm]
            lay[nm] = (O.v11_pack(O.rand_trits(seed * 1000 + l * 10 + i, K, N, 0.4)),
                       np.float32(0.01 + 0.005 * (l * 7 + i)))
        layers.append(lay)
    return dict(header=hdr, emb=emb, out_norm=out_norm, layers=layers)


def write(path, m, truncate=0, extra=b""):
    h = m["header"]
    blob = bytearray()
    blob += struct.pack("<II", h["magic"], h["version"])
    blob += struct.pack("<IIIIIIII", h["H"], h["F"], h["Nl"], h["V"], h["Nh"], h["Nkv"], h["Hd"], h["Smax"])
    blob += struct.pack("<ff", h["rope_theta"], h["eps"])
    blob += b"\x00" * (64 - 8 - 32 - 8)
    blob += np.ascontiguousarray(m["emb"], np.float16).tobytes()
    blob += np.ascontiguousarray(m["out_norm"], np.float32).tobytes()
    norms = ("attn_norm", "ffn_norm", "attn_sub_norm", "ffn_sub_norm") if h["magic"] == TERT else ("attn_norm",
                                                                                                   "ffn_norm")
    for lay in m["layers"]:
        for nm in norms:
            blob += np.ascontiguousarray(lay[nm], np.float32).tobytes()
        for nm in PROJ:
            v11, scale = lay[nm]
            blob += np.ascontiguousarray(v11, np.uint8).tobytes()
            blob += struct.pack("<f", float(scale))
    if truncate:
        blob = blob[:-truncate]
    with open(path, "wb") as f:
        f.write(bytes(blob) + extra)
    return path
