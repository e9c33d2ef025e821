"""End-to-end greedy decode of a small random BitNet-shaped model
(ter_amd.bitnet: the fabric's plans, attention context and fused tail in the
reference's forward_token_dev order, cuda/ter_cuda_forward_bitnet.cu:848-913)
against the oracle chain of the same steps: the token of every step, the
fp32 hidden state and the KV-cache rows, bit for bit (the oracle's attention
is the GPU kernel's chunked order; its distance to the reference's sequential
order is pinned in tests/test_oracle.py and tests/test_attention_gpu.py).
Eager launches and a HIP-graph replay of the step give the same tokens.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.decode_ref import host, host_model, oracle_step

pytestmark = pytest.mark.gpu

SHAPE = dict(H=256, F=512, Nl=2, Nh=4, Nkv=2, Hd=64, V=1000)


@pytest.mark.parametrize("graph", [False, True], ids=["eager", "hip-graph"])
def test_small_bitnet_decode_matches_oracle(cuda, graph):
    import torch
    from ter_amd import bitnet as B
    c = B.Shape(**SHAPE)
    m = B.random_model(c, seed=3)
    s_max, start = 96, 70
    dec = B.Decoder(m, s_max)
    rng = np.random.default_rng(4)
    K = rng.standard_normal((c.Nl, s_max, c.Nkv, c.Hd)).astype(np.float16)   # a pre-filled cache
    V = rng.standard_normal((c.Nl, s_max, c.Nkv, c.Hd)).astype(np.float16)
    dec.K.copy_(torch.from_numpy(K))
    dec.V.copy_(torch.from_numpy(V))
    dec.pos.fill_(start)
    tok = 17
    dec.token.fill_(tok)
    hm = host_model(m)
    table = O.rope_table(c.rope_theta, c.Hd, s_max)
    g = dec.capture() if graph else None
    for step in range(4):
        pos = start + step
        want_tok, want_hidden = oracle_step(hm, tok, pos, K, V, table)
        if graph:
            g.replay()
        else:
            dec.step()
        got_tok = int(host(dec.token)[0])
        assert (host(dec.hidden).view(np.uint32) == want_hidden.view(np.uint32)).all(), step
        assert got_tok == want_tok, (step, got_tok, want_tok)
        assert int(host(dec.pos)[0]) == pos + 1
        assert (host(dec.K).view(np.uint16) == K.view(np.uint16)).all(), step
        assert (host(dec.V).view(np.uint16) == V.view(np.uint16)).all(), step
        tok = want_tok
    dec.close()
