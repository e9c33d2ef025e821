"""GPU parity of the fused RMSNorm + int8 quantizer (rmsnorm_quant_f32_in_k /
rmsnorm_quant_fp16_in_k, cuda/ter_cuda_forward_bitnet.cu:64-146): the
standalone per-row kernel, the GEMV prologue (activation kinds
TER_HIP_X_F32_RMS / TER_HIP_X_F16_RMS), work-list plans and batched GEMMs.

Bar: int8 activations, activation scales, int32 accumulators and fp32
outputs bit-exact against the oracle (orc_rmsnorm_quant, which follows the
reference's summation order; 1e-5 relative is the stated fp32 tolerance and
is asserted too).
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
    rel = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want.astype(np.float64)), 1e-30)
    assert rel.max(initial=0.0) <= REL_TOL
    assert (got.view(np.int32) == want.view(np.int32)).all()


def inputs(seed, K, f16, kind="normal"):
    rng = np.random.default_rng(seed)
    if kind == "normal":
        x = rng.standard_normal(K).astype(np.float32) * np.float32(3.0)
    elif kind == "spike":
        x = np.zeros(K, np.float32)
        x[K // 3] = -40.0
    elif kind == "zeros":
        x = np.zeros(K, np.float32)
    else:  # wide dynamic range
        x = (rng.standard_normal(K) * np.exp(rng.uniform(-6, 6, K))).astype(np.float32)
    if f16:
        x = x.astype(np.float16)
    g = rng.uniform(0.25, 2.0, K).astype(np.float16)
    return x, g


@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("K,kind", [(2560, "normal"), (6912, "normal"), (1000, "wide"), (37, "normal"),
                                    (2560, "spike"), (2560, "zeros"), (9000, "normal")])
def test_rmsnorm_quant_rows(cuda, f16, K, kind):
    import ter_amd as T
    rows = [inputs(100 + r, K, f16, kind) for r in range(3)]
    g = rows[0][1]
    X = np.stack([x for x, _ in rows])
    q, s = T.rmsnorm_quant(dev(X), dev(g), 1e-5)
    q, s = host(q), host(s)
    for r in range(3):
        rq, rs, _ = O.rmsnorm_quant(X[r], g, 1e-5)
        assert (q[r] == rq).all(), (r, np.flatnonzero(q[r] != rq)[:8])
        assert s[r].view(np.int32) == np.float32(rs).view(np.int32)


@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
@pytest.mark.parametrize("K,N", [(2560, 2560), (6912, 2560), (9000, 300), (777, 64)])
def test_gemv_rms_prologue(cuda, f16, K, N):
    """RMSNorm + quantization inside the GEMV prologue: K = 2560 (one chunk
    per thread), 6912 (two), 9000 (beyond the prefetched chunks), 777 (ragged)."""
    import torch
    import ter_amd as T
    x, g = inputs(K + N, K, f16)
    v11 = O.v11_pack(O.rand_trits(K * 3 + N, K, N, 0.4))
    W = T.PackedTrits.from_v11(v11, K, N, 0.021)
    q = torch.empty(K, dtype=torch.int8, device="cuda")
    s = torch.empty(1, dtype=torch.float32, device="cuda")
    acc = torch.empty(N, dtype=torch.int32, device="cuda")
    y = torch.empty(N, dtype=torch.float32, device="cuda")
    T.gemv(W, dev(x), y=y, acc=acc, q_out=q, scale_out=s, gamma=dev(g), eps=1e-5)
    rq, rs, _ = O.rmsnorm_quant(x, g, 1e-5)
    assert (host(q) == rq).all()
    assert host(s)[0].view(np.int32) == np.float32(rs).view(np.int32)
    ra, ry = O.gemv_v11(rq, rs, v11, 0.021, K, N)
    assert (host(acc) == ra).all()
    assert_f32_equal(host(y), ry)


def test_plan_mixes_rms_and_int8_items(cuda):
    """One work list: RMS fp32 and fp16 items (many workgroups each) beside
    int8 items, over 2 launch shapes, launched twice."""
    import torch
    import ter_amd as T
    specs = [(2560, 2560, "f32"), (2560, 640, "i8"), (6912, 2560, "f16"), (2048, 512, "f32"), (300, 20, "i8")]
    items, refs = [], []
    for i, (K, N, kind) in enumerate(specs):
        v11 = O.v11_pack(O.rand_trits(300 + i, K, N, 0.4))
        W = T.PackedTrits.from_v11(v11, K, N, 0.01 * (i + 1))
        y = torch.empty(N, dtype=torch.float32, device="cuda")
        acc = torch.empty(N, dtype=torch.int32, device="cuda")
        if kind == "i8":
            x8 = O.rand_int8(400 + i, K)
            items.append(dict(w=W, x=dev(x8), x_scale=0.05, y=y, acc=acc))
            refs.append(O.gemv_v11(x8, np.float32(0.05), v11, 0.01 * (i + 1), K, N))
        else:
            x, g = inputs(500 + i, K, kind == "f16")
            items.append(dict(w=W, x=dev(x), gamma=dev(g), eps=1e-6, y=y, acc=acc))
            rq, rs, _ = O.rmsnorm_quant(x, g, 1e-6)
            refs.append(O.gemv_v11(rq, rs, v11, 0.01 * (i + 1), K, N))
    for wg in (0, 1):
        plan = T.Plan(items, wg_per_cu=wg)
        for rep in range(2):
            for it in items:
                it["y"].fill_(-7)
                it["acc"].fill_(-7)
            plan.launch()
            for it, (ra, ry) in zip(items, refs):
                assert (host(it["acc"]) == ra).all(), (wg, rep, it["w"].K)
                assert_f32_equal(host(it["y"]), ry)


@pytest.mark.parametrize("M,f16", [(8, False), (32, True), (3, False)])
def test_gemm_rms_rows(cuda, M, f16):
    """Batched: rows RMS-normalized and quantized per token, then the GEMM."""
    import torch
    import ter_amd as T
    K, N = 2560, 640
    X = np.stack([inputs(700 + m, K, f16)[0] for m in range(M)])
    g = inputs(699, K, f16)[1]
    v11 = O.v11_pack(O.rand_trits(701, K, N, 0.4))
    W = T.PackedTrits.from_v11(v11, K, N, 0.03)
    q = torch.empty((M, K), dtype=torch.int8, device="cuda")
    s = torch.empty(M, dtype=torch.float32, device="cuda")
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    T.mm_batched(W, dev(X), y=y, acc=acc, q_out=q, scale_out=s, gamma=dev(g), eps=1e-5)
    rq = np.empty((M, K), np.int8)
    rs = np.empty(M, np.float32)
    for m in range(M):
        rq[m], rs[m], _ = O.rmsnorm_quant(X[m], g, 1e-5)
    assert (host(q) == rq).all()
    assert (host(s).view(np.int32) == rs.view(np.int32)).all()
    ra, ry = O.gemm_v11(rq, rs, v11, 0.03, K, N)
    assert (host(acc) == ra).all()
    assert_f32_equal(host(y), ry)
