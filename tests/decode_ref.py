"""The oracle's chain of one BitNet decode step (the reference's
forward_token_dev order, cuda/ter_cuda_forward_bitnet.cu:848-913), shared by
the end-to-end decode tests: embedding, per layer the RMSNorm + quantization,
Q/K/V, RoPE, the chunked attention, the sub-norm, O with the residual add,
the FFN norm, gate/up, relu^2 sub-norm, down with the residual add; then the
final norm, the fp16 lm_head and the argmax.  llama_oracle_step is the same
for the Llama forward (cuda/ter_cuda_forward_packed.cu:505-560).  Test
infrastructure only."""
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


def _mm(wt, x_q, x_s):
    w, ws, Kd, Nd = wt
    if w.dtype == np.int8:  # trits [K][N]
        return O.gemv_i8w(x_q, x_s, w, ws)[1]
    return O.gemv_v11(x_q, x_s, w, ws, Kd, Nd)[1]


def llama_oracle_step(hm, tok, pos, K, V, table):
    """The oracle's chain of one Llama decode step (forward_token_dev,
    cuda/ter_cuda_forward_packed.cu:505-560) on the fp16 hidden stream:
    embedding; per layer rmsnorm_quant_fp16_in_k, Q/K/V, NORM RoPE, the
    chunked attention, quant_int8_k of the fp16 attention output, O with
    add_k, rmsnorm_quant_fp16_in_k, gate/up, silu_mul_quant_k, down with
    add_k; then the tail: the ternary lm_head behind the fused norm + quant
    (bench mode, hm["lm_head"]) or rmsnorm_k + the fp16 lm_head over the
    tied token_embd; the argmax.  Writes the new cache rows into K and V."""
    c = hm["shape"]
    hidden = hm["emb"][tok].astype(np.float16)
    for l, lay in enumerate(hm["layers"]):
        xq, xs, _ = O.rmsnorm_quant(hidden, lay["attn_norm"], c.eps)
        q = half_of(_mm(lay["Wq"], xq, xs)).reshape(c.Nh, c.Hd)
        k = half_of(_mm(lay["Wk"], xq, xs)).reshape(c.Nkv, c.Hd)
        v = half_of(_mm(lay["Wv"], xq, xs)).reshape(c.Nkv, c.Hd)
        qr = O.rope_f16(q, table[pos], False)
        K[l, pos] = O.rope_f16(k, table[pos], False)
        V[l, pos] = v
        att, _ = O.attention_splitk(qr, K[l, :pos + 1], V[l, :pos + 1])
        aq, as_ = O.quant_int8(att.reshape(-1).astype(np.float32))
        hidden = O.residual_add_h16(hidden, _mm(lay["Wo"], aq, as_))
        fq, fs, _ = O.rmsnorm_quant(hidden, lay["ffn_norm"], c.eps)
        g16, u16 = half_of(_mm(lay["Wgate"], fq, fs)), half_of(_mm(lay["Wup"], fq, fs))
        dq, ds, _ = O.silu_mul_quant(g16, u16)
        hidden = O.residual_add_h16(hidden, _mm(lay["Wdown"], dq, ds))
    if hm.get("lm_head") is None:
        xn, _ = O.rmsnorm_f16(hidden.astype(np.float32), hm["out_norm"], c.eps)
        logits, _ = O.lm_head_f16(xn, hm["emb"])
    else:
        hq, hs, _ = O.rmsnorm_quant(hidden, hm["out_norm"], c.eps)
        logits = half_of(_mm(hm["lm_head"], hq, hs))
    return O.argmax_f16(logits), hidden


def llama_host_model(m, seed=None, p_zero=0.4):
    """The host copy of a llama.Model: projections read back as v11 bytes, or,
    with `seed` (a llama.random_model's), regenerated on the host as int8
    trits from the seeds the device drew (ter_hip_synth_v11's splitmix64
    stream); norms and the token embedding copied from the device."""
    from ter_amd import llama as LM
    shapes = LM.proj_shapes(m.shape)

    def wt(W, K, N, s):
        if seed is None:
            return (host(W.to_v11()), W.scale, K, N)
        return (O.rand_trits_c(s, K, N, p_zero), W.scale, K, N)

    layers = []
    for l, lay in enumerate(m.layers):
        d = {nm: wt(lay.W[nm], *shapes[nm], LM.weight_seed(seed or 0, l, i)) for i, nm in enumerate(LM.PROJ)}
        d.update(attn_norm=host(lay.attn_norm), ffn_norm=host(lay.ffn_norm))
        layers.append(d)
    head = None
    if m.lm_head is not None:
        head = wt(m.lm_head, m.shape.H, m.shape.V, LM.weight_seed(seed or 0, -1, 0))
    return dict(shape=m.shape, layers=layers, emb=host(m.token_embd), out_norm=host(m.output_norm), lm_head=head)
