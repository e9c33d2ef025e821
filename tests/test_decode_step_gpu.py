"""GPU parity of the decode-step neighbours of the packed GEMV:

* the fused relu^2(gate) * up + RMSNorm + int8 quantizer
  (relu2_mul_rmsnorm_quant_k, cuda/ter_cuda_forward_bitnet.cu:258-309) as a
  per-row kernel, as the GEMV prologue (TER_HIP_X_RELU2_RMS) and as the row
  step of batched GEMMs;
* the fp16 projection output out[j] = __float2half((float)acc * scale)
  (cuda/ter_cuda_forward_packed.cu:393, ter_cuda_forward_bitnet.cu:557,
  ter_cuda_addonly_batched.cu:120) and the residual add of that output into the
  fp32 hidden stream (add_k_f32, cuda/ter_cuda_forward_bitnet.cu:51-54), as
  epilogues of the GEMV and of every GEMM kernel;
* one BitNet layer's projection chain (:855-887, attention output synthetic)
  through work-list plans.

Bar: int8 activations, scales, int32 accumulators, fp32 and fp16 outputs and
the updated fp32 hidden stream bit-exact against the oracle (1e-5 relative
is the stated fp32 tolerance and is asserted on fp32 outputs too).
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu
REL_TOL = 1e-5


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def assert_f32_equal(got, want):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    fin = np.isfinite(want)
    rel = np.abs(got[fin].astype(np.float64) - want[fin]) / np.maximum(np.abs(want[fin].astype(np.float64)), 1e-30)
    assert rel.max(initial=0.0) <= REL_TOL
    assert (got.view(np.int32) == want.view(np.int32)).all()


def assert_f16_equal(got_t, want_f32):
    got = host(got_t).view(np.uint16)
    want = O.float_to_half_bits(want_f32).reshape(got.shape)
    assert (got == want).all(), np.flatnonzero(got.ravel() != want.ravel())[:8]


def ffn_inputs(seed, F, kind="normal"):
    """fp16 gate and up as the FFN produces them, fp16 gamma."""
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal(F) * 2.0).astype(np.float16)
    u = (rng.standard_normal(F) * 2.0).astype(np.float16)
    if kind == "negative":
        g = -np.abs(g)
        g[F // 2] = np.float16(3.0)
    elif kind == "order":  # v[0]^2 = 2^24, v[256]^2 = v[768]^2 = 1 (orders differ)
        g = np.zeros(F, np.float16)
        g[0], g[256], g[768] = 64.0, 1.0, 1.0
        u = np.ones(F, np.float16)
    elif kind == "large":  # relu^2 * up near 1e5 (fp32 math, as the reference notes)
        g = rng.uniform(15, 20, F).astype(np.float16)
        u = rng.uniform(-300, 300, F).astype(np.float16)
    gm = rng.uniform(0.25, 2.0, F).astype(np.float16)
    return g, u, gm


# ---------------------------------------------------------------------------
# relu^2 * up + RMSNorm + int8
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("F,kind", [(6912, "normal"), (6912, "negative"), (769, "order"), (1000, "normal"),
                                    (37, "normal"), (9000, "large"), (1024, "normal")])
def test_relu2_rmsnorm_quant_rows(cuda, F, kind):
    import ter_amd as T
    rows = [ffn_inputs(10 + r, F, kind) for r in range(3)]
    G = np.stack([r[0] for r in rows])
    U = np.stack([r[1] for r in rows])
    gm = rows[0][2]
    q, s = T.relu2_rmsnorm_quant(dev(G), dev(U), dev(gm), 1e-5)
    q, s = host(q), host(s)
    for r in range(3):
        rq, rs, _ = O.relu2_rmsnorm_quant(G[r], U[r], gm, 1e-5)
        assert (q[r] == rq).all(), (r, np.flatnonzero(q[r] != rq)[:8])
        assert s[r].view(np.int32) == np.float32(rs).view(np.int32)


@pytest.mark.parametrize("K,N,kind", [(6912, 2560, "normal"), (769, 64, "order"), (9000, 300, "large"),
                                      (777, 20, "negative")])
def test_gemv_relu2_prologue(cuda, K, N, kind):
    """relu^2 prologue of the down projection: K = 6912 (BitNet F), 769 (the
    summation-order case), 9000 (beyond the prefetched chunks), 777 ragged."""
    import torch
    import ter_amd as T
    g, u, gm = ffn_inputs(K + N, K, kind)
    v11 = O.v11_pack(O.rand_trits(K * 5 + N, K, N, 0.4))
    W = T.PackedTrits.from_v11(v11, K, N, 0.017)
    q = torch.empty(K, dtype=torch.int8, device="cuda")
    s = torch.empty(1, dtype=torch.float32, device="cuda")
    acc = torch.empty(N, dtype=torch.int32, device="cuda")
    y = torch.empty(N, dtype=torch.float32, device="cuda")
    T.gemv(W, dev(g), y=y, acc=acc, q_out=q, scale_out=s, gamma=dev(gm), up=dev(u), eps=1e-5)
    rq, rs, _ = O.relu2_rmsnorm_quant(g, u, gm, 1e-5)
    assert (host(q) == rq).all()
    assert host(s)[0].view(np.int32) == np.float32(rs).view(np.int32)
    ra, ry = O.gemv_v11(rq, rs, v11, 0.017, K, N)
    assert (host(acc) == ra).all()
    assert_f32_equal(host(y), ry)


@pytest.mark.parametrize("M", [3, 8, 32])
def test_gemm_relu2_rows(cuda, M):
    import torch
    import ter_amd as T
    K, N = 6912, 640
    rows = [ffn_inputs(900 + m, K) for m in range(M)]
    G = np.stack([r[0] for r in rows])
    U = np.stack([r[1] for r in rows])
    gm = rows[0][2]
    v11 = O.v11_pack(O.rand_trits(901, K, N, 0.4))
    W = T.PackedTrits.from_v11(v11, K, N, 0.02)
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    T.mm_batched(W, dev(G), y=y, acc=acc, gamma=dev(gm), up=dev(U), eps=1e-5)
    rq = np.empty((M, K), np.int8)
    rs = np.empty(M, np.float32)
    for m in range(M):
        rq[m], rs[m], _ = O.relu2_rmsnorm_quant(G[m], U[m], gm, 1e-5)
    ra, ry = O.gemm_v11(rq, rs, v11, 0.02, K, N)
    assert (host(acc) == ra).all()
    assert_f32_equal(host(y), ry)


# ---------------------------------------------------------------------------
# fp16 outputs and the residual add
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("K,N,ws", [(2560, 2560, 0.02), (2560, 640, 3000.0), (300, 20, 0.5)])
def test_gemv_f16_and_residual_outputs(cuda, K, N, ws):
    """y16 = half(y) (ws = 3000 drives |y| past 65504: inf, as __float2half),
    resid += float(half(y)) applied twice in a row."""
    import torch
    import ter_amd as T
    v11 = O.v11_pack(O.rand_trits(K + 7 * N, K, N, 0.4))
    W = T.PackedTrits.from_v11(v11, K, N, ws)
    x8 = O.rand_int8(K + N, K)
    ra, ry = O.gemv_v11(x8, np.float32(0.04), v11, ws, K, N)
    if ws > 1000:
        assert (np.abs(ry) > 65520).any()
    y16 = torch.empty(N, dtype=torch.float16, device="cuda")
    h0 = np.random.default_rng(K).standard_normal(N).astype(np.float32)
    hid = dev(h0)
    y = torch.empty(N, dtype=torch.float32, device="cuda")
    T.gemv(W, dev(x8), y=y, x_scale=0.04, y16=y16, resid=hid)
    assert_f32_equal(host(y), ry)
    assert_f16_equal(y16, ry)
    want = O.residual_add_f16(h0, ry)
    assert (host(hid).view(np.int32) == want.view(np.int32)).all()
    T.gemv(W, dev(x8), x_scale=0.04, resid=hid)  # only the residual output
    want = O.residual_add_f16(want, ry)
    assert (host(hid).view(np.int32) == want.view(np.int32)).all()


def test_mm_packed_dispatch_f16(cuda):
    """The reference launcher with its own fp16 output."""
    import torch
    import ter_amd as T
    K, N = 2560, 6912
    v11 = O.v11_pack(O.rand_trits(77, K, N, 0.4))
    W = T.PackedTrits.from_v11(v11, K, N, 0.013)
    x8 = O.rand_int8(78, K)
    out = torch.empty(N, dtype=torch.float16, device="cuda")
    T.mm_packed_dispatch_f16(dev(x8), dev(np.array([0.031], np.float32)), W, out, K, N)
    _, ry = O.gemv_v11(x8, np.float32(0.031), v11, 0.013, K, N)
    assert_f16_equal(out, ry)


@pytest.mark.parametrize("M,aligned", [(8, True), (8, False), (32, True), (32, False), (100, True)],
                         ids=["stream", "stream-bytewise", "lds-ring", "unit-major", "lds-ring-m100"])
def test_gemm_f16_and_residual_outputs(cuda, M, aligned):
    """Every GEMM kernel's epilogue: streaming (M <= 16), LDS ring (16-byte
    rows), unit-major (X not 16-byte aligned)."""
    import torch
    import ter_amd as T
    K, N = 2560, 640
    v11 = O.v11_pack(O.rand_trits(M * 11, K, N, 0.4))
    W = T.PackedTrits.from_v11(v11, K, N, 0.021)
    X = np.stack([O.rand_int8(M * 13 + m, K) for m in range(M)])
    xs = (np.arange(M, dtype=np.float32) + 1) * np.float32(0.01)
    buf = torch.empty(M * K + 16, dtype=torch.int8, device="cuda")
    off = 0 if aligned else 1
    Xd = buf[off:off + M * K].view(M, K)
    Xd.copy_(dev(X))
    y16 = torch.empty((M, N), dtype=torch.float16, device="cuda")
    h0 = np.random.default_rng(M).standard_normal((M, N)).astype(np.float32)
    hid = dev(h0)
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    T.mm_batched(W, Xd, acc=acc, x_scale_dev=dev(xs), y16=y16, resid=hid)
    ra, ry = O.gemm_v11(X, xs, v11, 0.021, K, N)
    assert (host(acc) == ra).all()
    assert_f16_equal(y16, ry)
    want = O.residual_add_f16(h0.ravel(), ry.ravel()).reshape(M, N)
    assert (host(hid).view(np.int32) == want.view(np.int32)).all()


def test_gemm_plan_f16_and_residual(cuda):
    import torch
    import ter_amd as T
    M = 16
    specs = [(2560, 2560), (2560, 640), (6912, 2560)]
    items, refs = [], []
    for i, (K, N) in enumerate(specs):
        v11 = O.v11_pack(O.rand_trits(40 + i, K, N, 0.4))
        W = T.PackedTrits.from_v11(v11, K, N, 0.01 * (i + 1))
        X = np.stack([O.rand_int8(50 + 16 * i + m, K) for m in range(M)])
        xs = np.full(M, 0.02, np.float32)
        h0 = np.random.default_rng(i).standard_normal((M, N)).astype(np.float32)
        it = dict(w=W, x=dev(X), x_scale_dev=dev(xs), y16=torch.empty((M, N), dtype=torch.float16, device="cuda"))
        if i != 1:
            it["resid"] = dev(h0)
        items.append(it)
        refs.append((O.gemm_v11(X, xs, v11, 0.01 * (i + 1), K, N)[1], h0))
    plan = T.GemmPlan(items)
    plan.launch()
    for i, (it, (ry, h0)) in enumerate(zip(items, refs)):
        assert_f16_equal(it["y16"], ry)
        if "resid" in it:
            want = O.residual_add_f16(h0.ravel(), ry.ravel()).reshape(h0.shape)
            assert (host(it["resid"]).view(np.int32) == want.view(np.int32)).all(), i


# ---------------------------------------------------------------------------
# One BitNet layer's projection chain (cuda/ter_cuda_forward_bitnet.cu:855-887)
# ---------------------------------------------------------------------------

def test_bitnet_layer_projection_chain(cuda):
    """hidden -> [RMSNorm+quant prologue] Q, K, V (fp16) ; synthetic fp16
    attention output -> [fp16 RMSNorm prologue] O, += hidden ; hidden ->
    [RMSNorm prologue] gate, up (fp16) -> [relu^2 prologue] down, += hidden.
    Four plan launches; the final fp32 hidden stream bit-exact against the
    oracle chain."""
    import torch
    import ter_amd as T
    H, F, KV = 2560, 6912, 640
    rng = np.random.default_rng(2024)
    eps = 1e-5

    def weight(seed, K, N, s):
        v11 = O.v11_pack(O.rand_trits(seed, K, N, 0.4))
        return v11, T.PackedTrits.from_v11(v11, K, N, s)

    wq, Wq = weight(1, H, H, 0.011)
    wk, Wk = weight(2, H, KV, 0.012)
    wv, Wv = weight(3, H, KV, 0.013)
    wo, Wo = weight(4, H, H, 0.014)
    wg, Wg = weight(5, H, F, 0.015)
    wu, Wu = weight(6, H, F, 0.016)
    wd, Wd = weight(7, F, H, 0.017)
    n_attn = rng.uniform(0.5, 1.5, H).astype(np.float16)
    n_sub = rng.uniform(0.5, 1.5, H).astype(np.float16)
    n_ffn = rng.uniform(0.5, 1.5, H).astype(np.float16)
    n_ffsub = rng.uniform(0.5, 1.5, F).astype(np.float16)
    hidden0 = (rng.standard_normal(H) * 4).astype(np.float32)
    attn = (rng.standard_normal(H) * 0.5).astype(np.float16)  # stands in for attention_k's output

    f16 = dict(dtype=torch.float16, device="cuda")
    hid = dev(hidden0)
    q16, k16, v16 = torch.empty(H, **f16), torch.empty(KV, **f16), torch.empty(KV, **f16)
    g16, u16 = torch.empty(F, **f16), torch.empty(F, **f16)
    d_attn, d_na, d_ns, d_nf, d_nfs = dev(attn), dev(n_attn), dev(n_sub), dev(n_ffn), dev(n_ffsub)
    qkv = T.Plan([dict(w=Wq, x=hid, gamma=d_na, eps=eps, y16=q16),
                  dict(w=Wk, x=hid, gamma=d_na, eps=eps, y16=k16),
                  dict(w=Wv, x=hid, gamma=d_na, eps=eps, y16=v16)])
    oproj = T.Plan([dict(w=Wo, x=d_attn, gamma=d_ns, eps=eps, resid=hid)])
    gate_up = T.Plan([dict(w=Wg, x=hid, gamma=d_nf, eps=eps, y16=g16),
                      dict(w=Wu, x=hid, gamma=d_nf, eps=eps, y16=u16)])
    down = T.Plan([dict(w=Wd, x=g16, up=u16, gamma=d_nfs, eps=eps, resid=hid)])
    qkv.launch()
    oproj.launch()
    gate_up.launch()
    down.launch()

    # oracle chain
    xq, xs, _ = O.rmsnorm_quant(hidden0, n_attn, eps)
    ref_q = O.gemv_v11(xq, xs, wq, 0.011, H, H)[1]
    ref_k = O.gemv_v11(xq, xs, wk, 0.012, H, KV)[1]
    ref_v = O.gemv_v11(xq, xs, wv, 0.013, H, KV)[1]
    aq, as_, _ = O.rmsnorm_quant(attn, n_sub, eps)
    h1 = O.residual_add_f16(hidden0, O.gemv_v11(aq, as_, wo, 0.014, H, H)[1])
    fq, fs, _ = O.rmsnorm_quant(h1, n_ffn, eps)
    ref_g = O.gemv_v11(fq, fs, wg, 0.015, H, F)[1]
    ref_u = O.gemv_v11(fq, fs, wu, 0.016, H, F)[1]
    g_h = O.float_to_half_bits(ref_g).view(np.float16)
    u_h = O.float_to_half_bits(ref_u).view(np.float16)
    dq, ds, _ = O.relu2_rmsnorm_quant(g_h, u_h, n_ffsub, eps)
    h2 = O.residual_add_f16(h1, O.gemv_v11(dq, ds, wd, 0.017, F, H)[1])

    assert_f16_equal(q16, ref_q)
    assert_f16_equal(k16, ref_k)
    assert_f16_equal(v16, ref_v)
    assert_f16_equal(g16, ref_g)
    assert_f16_equal(u16, ref_u)
    assert (host(hid).view(np.int32) == h2.view(np.int32)).all()
