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

pytestmark = pytest.mark.gpu

SHAPE = dict(H=256, F=512, Nl=2, Nh=4, Nkv=2, Hd=64, V=1000)


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def half_of(y):
    return O.float_to_half_bits(y).view(np.float16)


def oracle_step(hm, tok, pos, K, V, table):
    c = hm["shape"]
    hidden = hm["emb"][tok].astype(np.float32)
    for l, lay in enumerate(hm["layers"]):
        def mm(x_q, x_s, nm):
            v11, ws, Kd, Nd = lay[nm]
            return O.gemv_v11(x_q, x_s, v11, ws, Kd, Nd)[1]
        xq, xs, _ = O.rmsnorm_quant(hidden, lay["attn_norm"], c.eps)
        q = half_of(mm(xq, xs, "Wq")).reshape(c.Nh, c.Hd)
        k = half_of(mm(xq, xs, "Wk")).reshape(c.Nkv, c.Hd)
        v = half_of(mm(xq, xs, "Wv")).reshape(c.Nkv, c.Hd)
        qr = O.rope_f16(q, table[pos], True)
        K[l, pos] = O.rope_f16(k, table[pos], True)
        V[l, pos] = v
        att, _ = O.attention_splitk(qr, K[l, :pos + 1], V[l, :pos + 1])
        aq, as_, _ = O.rmsnorm_quant(att.reshape(-1), lay["attn_sub_norm"], c.eps)
        hidden = O.residual_add_f16(hidden, mm(aq, as_, "Wo"))
        fq, fs, _ = O.rmsnorm_quant(hidden, lay["ffn_norm"], c.eps)
        g16, u16 = half_of(mm(fq, fs, "Wgate")), half_of(mm(fq, fs, "Wup"))
        dq, ds, _ = O.relu2_rmsnorm_quant(g16, u16, lay["ffn_sub_norm"], c.eps)
        hidden = O.residual_add_f16(hidden, mm(dq, ds, "Wdown"))
    xn, _ = O.rmsnorm_f16(hidden, hm["out_norm"], c.eps)
    logits, _ = O.lm_head_f16(xn, hm["emb"])
    return O.argmax_f16(logits), hidden


def host_model(m):
    from ter_amd import bitnet as B
    shapes = B.proj_shapes(m.shape)
    layers = []
    for lay in m.layers:
        d = {nm: (host(lay.W[nm].to_v11()), lay.W[nm].scale, *shapes[nm]) for nm in B.PROJ}
        d.update(attn_norm=host(lay.attn_norm), attn_sub_norm=host(lay.attn_sub_norm), ffn_norm=host(lay.ffn_norm),
                 ffn_sub_norm=host(lay.ffn_sub_norm))
        layers.append(d)
    return dict(shape=m.shape, layers=layers, emb=host(m.token_embd), out_norm=host(m.output_norm))


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
