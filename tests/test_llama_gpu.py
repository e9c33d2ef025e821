"""GPU parity of the Llama forward's steps on the fabric
(cuda/ter_cuda_forward_packed.cu:505-560):

* quant_int8_k on the fp16 attention output (:40-62) as the GEMV prologue
  TER_HIP_X_F16;
* silu_mul_quant_k (:312-344) as the GEMV prologue TER_HIP_X_SILU_MUL, and
  split in two: the gate GEMV's silu output (silu of its fp16 value) and the
  down projection's TER_HIP_X_SMUL prologue (times up, absmax);
* add_k into the fp16 hidden stream (:113-116) as the GEMV's resid16
  epilogue;
* one Llama layer's projection chain through work-list plans;
* the greedy decode of a small random Llama-shaped model (ter_amd.llama), in
  both tails (the bench mode's ternary lm_head, :541-545, and the tied fp16
  lm_head, :547-554), eagerly and from a HIP-graph replay, and of an 'LLRT'
  file (load_model_from_bin, :588-664);
* three tokens of the Llama-3.2-1B-shaped decode at full size.

Bar: int8 activations, scales, int32 accumulators, fp16 outputs, the fp16
hidden stream, KV-cache rows and tokens bit-exact against the oracle.  The
exp inside silu is the build's own (ter_expf, restated by orc_expf); its
distance to a float64 exp is pinned in tests/test_oracle.py.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.decode_ref import half_of, host, llama_host_model, llama_oracle_step

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def assert_f16_equal(got_t, want_f32):
    got = host(got_t).view(np.uint16)
    want = O.float_to_half_bits(want_f32).reshape(got.shape)
    assert (got == want).all(), np.flatnonzero(got.ravel() != want.ravel())[:8]


def weight(seed, K, N, s):
    import ter_amd as T
    v11 = O.v11_pack(O.rand_trits(seed, K, N, 0.4))
    return v11, T.PackedTrits.from_v11(v11, K, N, s)


def gate_up(seed, F, kind="normal"):
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal(F) * 2.0).astype(np.float16)
    u = (rng.standard_normal(F) * 2.0).astype(np.float16)
    if kind == "wide":  # saturated sigmoid on both sides, exp overflow at -g > 88.7
        g = rng.uniform(-120, 120, F).astype(np.float16)
        g[:4] = [-60000.0, 60000.0, 0.0, -0.0]
    return g, u


# ---------------------------------------------------------------------------
# Prologues and the fp16 residual
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("K,N", [(2048, 2048), (777, 20), (9000, 300), (2048, 512)])
def test_gemv_f16_absmax_prologue(cuda, K, N):
    """The O projection's input: quant_int8_k on an fp16 vector."""
    import torch
    import ter_amd as T
    x = (np.random.default_rng(K + N).standard_normal(K) * 0.7).astype(np.float16)
    v11, W = weight(K * 3 + N, K, N, 0.021)
    q = torch.empty(K, dtype=torch.int8, device="cuda")
    s = torch.empty(1, dtype=torch.float32, device="cuda")
    acc = torch.empty(N, dtype=torch.int32, device="cuda")
    y = torch.empty(N, dtype=torch.float32, device="cuda")
    T.gemv(W, dev(x), y=y, acc=acc, q_out=q, scale_out=s)
    rq, rs = O.quant_int8(x.astype(np.float32))
    assert (host(q) == rq).all()
    assert host(s)[0].view(np.int32) == np.float32(rs).view(np.int32)
    ra, ry = O.gemv_v11(rq, rs, v11, 0.021, K, N)
    assert (host(acc) == ra).all()
    assert (host(y).view(np.int32) == ry.view(np.int32)).all()


@pytest.mark.parametrize("K,N,kind", [(8192, 2048, "normal"), (769, 64, "normal"), (9000, 300, "wide"),
                                      (8192, 256, "wide")])
def test_gemv_silu_prologue(cuda, K, N, kind):
    """The down projection's input: silu(gate) * up, then quant_int8_k."""
    import torch
    import ter_amd as T
    g, u = gate_up(K + N, K, kind)
    v11, W = weight(K * 5 + N, K, N, 0.017)
    q = torch.empty(K, dtype=torch.int8, device="cuda")
    s = torch.empty(1, dtype=torch.float32, device="cuda")
    acc = torch.empty(N, dtype=torch.int32, device="cuda")
    y16 = torch.empty(N, dtype=torch.float16, device="cuda")
    T.gemv(W, dev(g), acc=acc, y16=y16, q_out=q, scale_out=s, up=dev(u))
    rq, rs, _ = O.silu_mul_quant(g, u)
    assert (host(q) == rq).all(), np.flatnonzero(host(q) != rq)[:8]
    assert host(s)[0].view(np.int32) == np.float32(rs).view(np.int32)
    ra, ry = O.gemv_v11(rq, rs, v11, 0.017, K, N)
    assert (host(acc) == ra).all()
    assert_f16_equal(y16, ry)


@pytest.mark.parametrize("K,N,ws", [(2048, 8192, 0.05), (777, 100, 0.3), (2048, 512, 3000.0)])
def test_gemv_silu_output(cuda, K, N, ws):
    """The gate projection's silu output: silu(float(half(y))) in fp32, beside
    its fp16 output (ws = 3000: outputs past 65504, half(y) = inf, silu = inf
    or -0)."""
    import torch
    import ter_amd as T
    v11, W = weight(K * 13 + N, K, N, ws)
    x8 = O.rand_int8(K + 3 * N, K)
    _, ry = O.gemv_v11(x8, np.float32(0.04), v11, ws, K, N)
    y16 = torch.empty(N, dtype=torch.float16, device="cuda")
    sl = torch.empty(N, dtype=torch.float32, device="cuda")
    T.gemv(W, dev(x8), x_scale=0.04, y16=y16, silu=sl)
    assert_f16_equal(y16, ry)
    want = O.silu_f16(half_of(ry))
    got = host(sl)
    assert (got.view(np.int32) == want.view(np.int32)).all(), np.flatnonzero(got.view(np.int32) != want.view(np.int32))[:8]
    if ws > 1000:
        assert np.isinf(half_of(ry).astype(np.float32)).any()
    T.gemv(W, dev(x8), x_scale=0.04, silu=sl)  # the silu output alone
    assert (host(sl).view(np.int32) == want.view(np.int32)).all()


@pytest.mark.parametrize("K,N", [(8192, 2048), (769, 64), (9000, 300)])
def test_gemv_smul_prologue(cuda, K, N):
    """The down projection's input from the split route: fp32 silu(gate)
    times fp16 up, then absmax -- the fused X_SILU_MUL prologue's int8
    vector, scale and outputs, bit for bit."""
    import torch
    import ter_amd as T
    g, u = gate_up(K * 3 + N, K)
    s = O.silu_f16(g)
    v11, W = weight(K * 7 + N, K, N, 0.019)
    outs = []
    for x in (dev(s), dev(g)):  # X_SMUL, then X_SILU_MUL
        q = torch.empty(K, dtype=torch.int8, device="cuda")
        sc = torch.empty(1, dtype=torch.float32, device="cuda")
        acc = torch.empty(N, dtype=torch.int32, device="cuda")
        T.gemv(W, x, acc=acc, q_out=q, scale_out=sc, up=dev(u))
        outs.append((host(q), host(sc)[0], host(acc)))
    rq, rs, _ = O.smul_quant(s, u)
    ra, _ = O.gemv_v11(rq, rs, v11, 0.019, K, N)
    for q, sc, acc in outs:
        assert (q == rq).all() and sc.view(np.int32) == np.float32(rs).view(np.int32)
        assert (acc == ra).all()


@pytest.mark.parametrize("K,N,ws", [(2048, 2048, 0.02), (8192, 2048, 0.05), (300, 20, 2000.0)])
def test_gemv_resid16_epilogue(cuda, K, N, ws):
    """hidden16 = half(float(hidden16) + float(half(y))), twice in a row
    (ws = 2000 drives the sum past 65504: inf, as add_k)."""
    import torch
    import ter_amd as T
    v11, W = weight(K + 11 * N, K, N, ws)
    x8 = O.rand_int8(K + N, K)
    ra, ry = O.gemv_v11(x8, np.float32(0.04), v11, ws, K, N)
    h0 = (np.random.default_rng(K).standard_normal(N) * 8).astype(np.float16)
    hid = dev(h0)
    y16 = torch.empty(N, dtype=torch.float16, device="cuda")
    T.gemv(W, dev(x8), x_scale=0.04, y16=y16, resid16=hid)
    assert_f16_equal(y16, ry)
    want = O.residual_add_h16(h0, ry)
    assert (host(hid).view(np.uint16) == want.view(np.uint16)).all()
    T.gemv(W, dev(x8), x_scale=0.04, resid16=hid)  # only the residual output
    want = O.residual_add_h16(want, ry)
    assert (host(hid).view(np.uint16) == want.view(np.uint16)).all()
    if ws > 1000:
        assert np.isinf(want.astype(np.float32)).any()


@pytest.mark.parametrize("kind,K,N", [("f16", 2048, 2048), ("f16", 4112, 256), ("f16", 777, 64),
                                      ("silu", 8192, 2048), ("silu", 9000, 512), ("silu", 1000, 128),
                                      ("silu", 512, 256), ("smul", 8192, 2048), ("smul", 9000, 512),
                                      ("smul", 1000, 128)],
                         ids=["f16-strided", "f16-beyond-strided", "f16-ragged", "silu-strided", "silu-beyond-strided",
                              "silu-ragged", "silu-small", "smul-strided", "smul-beyond-strided", "smul-ragged"])
def test_plan_absmax_prologues(cuda, kind, K, N):
    """Work-list plans of the fp16 absmax kinds: the strided strip prologue
    (K a multiple of 16 within its unit limit), and the general one past the
    limit or for ragged K; the quantized copy from the plan's owner."""
    import torch
    import ter_amd as T
    rng = np.random.default_rng(K * 7 + N)
    x = (rng.standard_normal(K) * 0.7).astype(np.float16)
    u = (rng.standard_normal(K) * 2.0).astype(np.float16)
    v11, W = weight(K * 11 + N, K, N, 0.03)
    q = torch.empty(K, dtype=torch.int8, device="cuda")
    s = torch.empty(1, dtype=torch.float32, device="cuda")
    y16 = torch.empty(N, dtype=torch.float16, device="cuda")
    it = dict(w=W, x=dev(x), y16=y16, q_out=q, scale_out=s)
    if kind == "silu":
        it["up"] = dev(u)
        rq, rs, _ = O.silu_mul_quant(x, u)
    elif kind == "smul":
        sl = O.silu_f16(x)
        it.update(x=dev(sl), up=dev(u))
        rq, rs, _ = O.smul_quant(sl, u)
    else:
        rq, rs = O.quant_int8(x.astype(np.float32))
    plan = T.Plan([it])
    for _ in range(2):  # a relaunch sees the same inputs
        plan.launch()
        assert (host(q) == rq).all(), np.flatnonzero(host(q) != rq)[:8]
        assert host(s)[0].view(np.int32) == np.float32(rs).view(np.int32)
        assert_f16_equal(y16, O.gemv_v11(rq, rs, v11, 0.03, K, N)[1])
    plan.close()


# ---------------------------------------------------------------------------
# One Llama layer's projection chain (:513-539)
# ---------------------------------------------------------------------------

def test_llama_layer_projection_chain(cuda):
    """hidden16 -> [fp16 RMSNorm prologue] Q, K, V ; synthetic fp16 attention
    output -> [absmax prologue] O, += hidden16 ; hidden16 -> [fp16 RMSNorm
    prologue] gate (fp16 and silu outputs), up -> [silu(gate) * up prologue
    from the gate's silu output] down, += hidden16.  Four plan launches;
    every output and the final hidden16 bit-exact."""
    import torch
    import ter_amd as T
    H, F, KV = 2048, 8192, 512
    rng = np.random.default_rng(2025)
    eps = 1e-5
    wq, Wq = weight(11, H, H, 0.05)
    wk, Wk = weight(12, H, KV, 0.05)
    wv, Wv = weight(13, H, KV, 0.05)
    wo, Wo = weight(14, H, H, 0.05)
    wg, Wg = weight(15, H, F, 0.05)
    wu, Wu = weight(16, H, F, 0.05)
    wd, Wd = weight(17, F, H, 0.05)
    n_attn = rng.uniform(0.5, 1.5, H).astype(np.float16)
    n_ffn = rng.uniform(0.5, 1.5, H).astype(np.float16)
    hidden0 = (rng.standard_normal(H) * 4).astype(np.float16)
    attn = (rng.standard_normal(H) * 0.5).astype(np.float16)  # stands in for attention_k's output

    f16 = dict(dtype=torch.float16, device="cuda")
    hid = dev(hidden0)
    q16, k16, v16 = torch.empty(H, **f16), torch.empty(KV, **f16), torch.empty(KV, **f16)
    g16, u16 = torch.empty(F, **f16), torch.empty(F, **f16)
    d_attn, d_na, d_nf = dev(attn), dev(n_attn), dev(n_ffn)
    qkv = T.Plan([dict(w=Wq, x=hid, gamma=d_na, eps=eps, y16=q16),
                  dict(w=Wk, x=hid, gamma=d_na, eps=eps, y16=k16),
                  dict(w=Wv, x=hid, gamma=d_na, eps=eps, y16=v16)])
    oproj = T.Plan([dict(w=Wo, x=d_attn, resid16=hid)])
    sl = torch.empty(F, dtype=torch.float32, device="cuda")
    gu = T.Plan([dict(w=Wg, x=hid, gamma=d_nf, eps=eps, y16=g16, silu=sl),
                 dict(w=Wu, x=hid, gamma=d_nf, eps=eps, y16=u16)])
    down = T.Plan([dict(w=Wd, x=sl, up=u16, resid16=hid)])
    for p in (qkv, oproj, gu, down):
        p.launch()

    xq, xs, _ = O.rmsnorm_quant(hidden0, n_attn, eps)
    ref_q = O.gemv_v11(xq, xs, wq, 0.05, H, H)[1]
    ref_k = O.gemv_v11(xq, xs, wk, 0.05, H, KV)[1]
    ref_v = O.gemv_v11(xq, xs, wv, 0.05, H, KV)[1]
    aq, as_ = O.quant_int8(attn.astype(np.float32))
    h1 = O.residual_add_h16(hidden0, O.gemv_v11(aq, as_, wo, 0.05, H, H)[1])
    fq, fs, _ = O.rmsnorm_quant(h1, n_ffn, eps)
    ref_g = O.gemv_v11(fq, fs, wg, 0.05, H, F)[1]
    ref_u = O.gemv_v11(fq, fs, wu, 0.05, H, F)[1]
    dq, ds, _ = O.silu_mul_quant(half_of(ref_g), half_of(ref_u))
    h2 = O.residual_add_h16(h1, O.gemv_v11(dq, ds, wd, 0.05, F, H)[1])

    assert_f16_equal(q16, ref_q)
    assert_f16_equal(k16, ref_k)
    assert_f16_equal(v16, ref_v)
    assert_f16_equal(g16, ref_g)
    assert_f16_equal(u16, ref_u)
    assert (host(sl).view(np.int32) == O.silu_f16(half_of(ref_g)).view(np.int32)).all()
    assert (host(hid).view(np.uint16) == h2.view(np.uint16)).all()
    for p in (qkv, oproj, gu, down):
        p.close()


# ---------------------------------------------------------------------------
# Greedy decode
# ---------------------------------------------------------------------------

SHAPE = dict(H=256, F=512, Nl=2, Nh=4, Nkv=2, Hd=64, V=1000)


def run_decode(dec, hm, c, s_max, start, tok, n_tok, graph, seed):
    import torch
    rng = np.random.default_rng(seed)
    K = rng.standard_normal((c.Nl, s_max, c.Nkv, c.Hd), dtype=np.float32).astype(np.float16)  # a pre-filled cache
    V = rng.standard_normal((c.Nl, s_max, c.Nkv, c.Hd), dtype=np.float32).astype(np.float16)
    dec.K.copy_(torch.from_numpy(K))
    dec.V.copy_(torch.from_numpy(V))
    dec.pos.fill_(start)
    dec.token.fill_(tok)
    table = O.rope_table(c.rope_theta, c.Hd, s_max)
    g = dec.capture() if graph else None
    for step in range(n_tok):
        pos = start + step
        print(f"llama decode ({'graph' if graph else 'eager'}): token {step} at position {pos}", flush=True)
        want_tok, want_hidden = llama_oracle_step(hm, tok, pos, K, V, table)
        assert np.isfinite(want_hidden.astype(np.float32)).all() and 0 <= want_tok < c.V  # not a degenerate chain
        if graph:
            g.replay()
        else:
            dec.step()
        got_tok = int(host(dec.token)[0])
        assert (host(dec.hidden).view(np.uint16) == want_hidden.view(np.uint16)).all(), step
        assert got_tok == want_tok, (step, got_tok, want_tok)
        assert int(host(dec.pos)[0]) == pos + 1
        assert (host(dec.K[:, pos]).view(np.uint16) == K[:, pos].view(np.uint16)).all(), step
        assert (host(dec.V[:, pos]).view(np.uint16) == V[:, pos].view(np.uint16)).all(), step
        tok = want_tok
    assert (host(dec.K).view(np.uint16) == K.view(np.uint16)).all()
    assert (host(dec.V).view(np.uint16) == V.view(np.uint16)).all()


@pytest.mark.parametrize("tied", [False, True], ids=["ternary-lm-head", "tied-lm-head"])
@pytest.mark.parametrize("graph", [False, True], ids=["eager", "hip-graph"])
def test_small_llama_decode_matches_oracle(cuda, graph, tied):
    from ter_amd import llama as LM
    c = LM.Shape(**SHAPE)
    m = LM.random_model(c, seed=3, tied=tied)
    dec = LM.Decoder(m, 96)
    assert dec.launches_per_token() == 2 + 5 * c.Nl + (0 if tied else 1)
    run_decode(dec, llama_host_model(m), c, 96, 70, 17, 4, graph, seed=4)
    dec.close()


def test_llrt_file_decodes_like_the_oracle(cuda, tmp_path):
    """An 'LLRT' file (tools/convert_llama_to_packed.py) through
    llama.from_file: the tied fp16 lm_head, the file's projections and norms;
    the decode against the oracle chain of the file's own arrays."""
    from tests import binfile_writer as BW
    from ter_amd import llama as LM
    m = BW.random_model(BW.LLRT, H=256, F=512, Nl=2, V=1000, Nh=4, Nkv=2, Hd=64, seed=21)
    path = BW.write(tmp_path / "llama.bin", m)
    model = LM.from_file(str(path))
    c = model.shape
    assert (c.H, c.F, c.Nl, c.V, c.Nh, c.Nkv, c.Hd) == (256, 512, 2, 1000, 4, 2, 64)
    assert model.lm_head is None
    shapes = LM.proj_shapes(c)
    hm = dict(shape=c, emb=m["emb"], out_norm=m["out_norm"].astype(np.float16), lm_head=None, layers=[
        dict({nm: (lw[nm][0], lw[nm][1], *shapes[nm]) for nm in LM.PROJ},
             **{k: lw[k].astype(np.float16) for k in ("attn_norm", "ffn_norm")})
        for lw in m["layers"]])
    dec = LM.Decoder(model, 80)
    run_decode(dec, hm, c, 80, 60, 5, 4, True, seed=22)
    dec.close()


@pytest.mark.parametrize("graph", [False, True], ids=["eager", "hip-graph"])
def test_llama_decode_full_size(cuda, graph):
    """The Llama-3.2-1B shape (16 layers, H 2048, F 8192, 32/8 heads of 64,
    V 128256, the ternary lm_head of the reference's bench mode): three greedy
    tokens from position 512 of a pre-filled cache; weights regenerated on
    the host from the device's seeds."""
    from ter_amd import llama as LM
    c = LM.Shape()
    seed = 7
    m = LM.random_model(c, seed=seed)
    s_max = 512 + 64
    dec = LM.Decoder(m, s_max)
    run_decode(dec, llama_host_model(m, seed=seed), c, s_max, 512, 1, 3, graph, seed=8)
    dec.close()
