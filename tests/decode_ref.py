"""The oracle's chain of one BitNet decode step (the reference's
forward_token_dev order, cuda/ter_cuda_forward_bitnet.cu:848-913), shared by
the end-to-end decode tests: embedding, per layer the RMSNorm + quantization,
Q/K/V, RoPE, the chunked attention, the sub-norm, O with the residual add,
the FFN norm, gate/up, relu^2 sub-norm, down with the residual add; then the
final norm, the fp16 lm_head and the argmax.  Test infrastructure only."""
import numpy as np

from oracle import oracle as O


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
            w, ws, Kd, Nd = lay[nm]
            if w.dtype == np.int8:  # trits [K][N] (host_model_i8)
                return O.gemv_i8w(x_q, x_s, w, ws)[1]
            return O.gemv_v11(x_q, x_s, w, ws, Kd, Nd)[1]
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




def host_model_i8(m, seed, p_zero=0.4):
    """host_model for a random_model(shape, seed, p_zero): the projections as
    int8 trits [K][N] regenerated on the host from random_model's seeds (the
    splitmix64 stream ter_hip_synth_v11 draws), not read back from the
    device; norms and the token embedding copied from the device."""
    from ter_amd import bitnet as B
    shapes = B.proj_shapes(m.shape)
    layers = []
    for l, lay in enumerate(m.layers):
        d = {}
        for i, nm in enumerate(B.PROJ):
            K, N = shapes[nm]
            s = seed * 1_000_003 + l * 101 + i
            d[nm] = (O.rand_trits_c(s, K, N, p_zero), lay.W[nm].scale, K, N)
        d.update(attn_norm=host(lay.attn_norm), attn_sub_norm=host(lay.attn_sub_norm), ffn_norm=host(lay.ffn_norm),
                 ffn_sub_norm=host(lay.ffn_sub_norm))
        layers.append(d)
    return dict(shape=m.shape, layers=layers, emb=host(m.token_embd), out_norm=host(m.output_norm))
