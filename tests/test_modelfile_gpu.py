"""GPU checks of the model loaders (ter_amd.modelfile over ter_hip_bin_*):
a 'TERT' file becomes a bitnet.Model whose decode is bit-exact against the
oracle chain built from the file's arrays (load_model_from_bin then
forward_token_dev, cuda/ter_cuda_forward_bitnet.cu:698-784, 848-913); an
'LLRT' file's projections, scales and norms arrive as written
(cuda/ter_cuda_forward_packed.cu:589-659).
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests import binfile_writer as BW
from tests.decode_ref import host, oracle_step

pytestmark = pytest.mark.gpu


def test_tert_file_decodes_like_the_oracle(cuda, tmp_path):
    import torch
    from ter_amd import bitnet as B
    from ter_amd.modelfile import load_bitnet
    m = BW.random_model(BW.TERT, H=256, F=512, Nl=2, V=1000, Nh=4, Nkv=2, Hd=64, seed=11)
    path = BW.write(tmp_path / "bitnet.bin", m)
    model = load_bitnet(str(path))
    c = model.shape
    assert (c.H, c.F, c.Nl, c.V, c.Nh, c.Nkv, c.Hd) == (256, 512, 2, 1000, 4, 2, 64)
    # the tensors as written (projections back to v11 bytes from the device layout)
    assert (host(model.token_embd).view(np.uint16) == m["emb"].view(np.uint16)).all()
    shapes = B.proj_shapes(c)
    for lay, want in zip(model.layers, m["layers"]):
        for nm in B.PROJ:
            v11, scale = want[nm]
            assert lay.W[nm].scale == scale
            assert (host(lay.W[nm].to_v11()) == v11).all(), nm
        assert (host(lay.ffn_sub_norm).view(np.uint16) == want["ffn_sub_norm"].astype(np.float16).view(np.uint16)).all()
    # decode four tokens from a pre-filled cache against the oracle chain of the file's arrays
    hm = dict(shape=c, emb=m["emb"], out_norm=m["out_norm"].astype(np.float16), layers=[
        dict({nm: (lw[nm][0], lw[nm][1], *shapes[nm]) for nm in B.PROJ},
             **{k: lw[k].astype(np.float16) for k in ("attn_norm", "attn_sub_norm", "ffn_norm", "ffn_sub_norm")})
        for lw in m["layers"]])
    s_max, start = 80, 60
    dec = B.Decoder(model, s_max)
    rng = np.random.default_rng(12)
    K = rng.standard_normal((c.Nl, s_max, c.Nkv, c.Hd)).astype(np.float16)
    V = rng.standard_normal((c.Nl, s_max, c.Nkv, c.Hd)).astype(np.float16)
    dec.K.copy_(torch.from_numpy(K))
    dec.V.copy_(torch.from_numpy(V))
    dec.pos.fill_(start)
    tok = 5
    dec.token.fill_(tok)
    table = O.rope_table(c.rope_theta, c.Hd, s_max)
    g = dec.capture()
    for step in range(4):
        want_tok, want_hidden = oracle_step(hm, tok, start + step, K, V, table)
        g.replay()
        assert (host(dec.hidden).view(np.uint32) == want_hidden.view(np.uint32)).all(), step
        assert int(host(dec.token)[0]) == want_tok, step
        tok = want_tok
    dec.close()


def test_llrt_file_tensors(cuda, tmp_path):
    from ter_amd.modelfile import load_llama
    m = BW.random_model(BW.LLRT, H=128, F=256, Nl=3, V=300, Nh=4, Nkv=2, Hd=32, seed=13)
    path = BW.write(tmp_path / "llama.bin", m)
    lm = load_llama(str(path))
    assert lm.header["magic"] == BW.LLRT and lm.header["Nl"] == 3
    assert (host(lm.output_norm).view(np.uint16) == m["out_norm"].astype(np.float16).view(np.uint16)).all()
    for lay, want in zip(lm.layers, m["layers"]):
        assert (host(lay.attn_norm).view(np.uint16) == want["attn_norm"].astype(np.float16).view(np.uint16)).all()
        for nm in BW.PROJ:
            v11, scale = want[nm]
            assert lay.W[nm].scale == scale
            assert (host(lay.W[nm].to_v11()) == v11).all(), nm
