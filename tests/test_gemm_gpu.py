"""GPU parity of the batched (M > 1) MFMA GEMM and the per-row quantizer.

Bar as for the GEMV: int32 accumulators and int8 quantized activations
bit-exact, fp32 outputs bit-exact (tolerance of the contract: 1e-5 relative).
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


CASES = [
    (2, 300, 20), (8, 2560, 640), (16, 2048, 512), (17, 257, 36), (32, 2560, 640),
    (64, 640, 128), (128, 2560, 640), (200, 512, 48), (256, 256, 16), (8, 6912, 256),
    (1, 2560, 640), (16, 6912, 64),  # M <= 16: streamed; M = 16 at K = 6912 exceeds its LDS and takes the row-block kernel
]


@pytest.mark.parametrize("M,K,N", CASES)
def test_gemm_int8(cuda, M, K, N):
    import torch
    import ter_amd as T
    w = O.rand_trits(M * 1000 + K, K, N, 0.4)
    v11 = O.v11_pack(w)
    X = O.rand_int8(M + K + N, M * K).reshape(M, K)
    xs = (0.001 * (np.arange(M) + 1)).astype(np.float32)
    W = T.PackedTrits.from_v11(v11, K, N, 0.043)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    T.mm_batched(W, dev(X), y=y, acc=acc, x_scale_dev=dev(xs))
    ra, ry = O.gemm_v11(X, xs, v11, 0.043, K, N)
    assert (host(acc) == ra).all()
    assert_f32_equal(host(y), ry)


@pytest.mark.parametrize("M,K,N", [(8, 2560, 640), (32, 6912, 64), (128, 2560, 128), (3, 100, 8)])
def test_gemm_fp32_rows_quantized(cuda, M, K, N):
    import torch
    import ter_amd as T
    w = O.rand_trits(K + N, K, N, 0.4)
    v11 = O.v11_pack(w)
    Xf = O.rand_normal_f32(M * 7 + 1, M * K).reshape(M, K)
    Xf[0] *= 50.0  # rows with very different ranges quantize independently
    W = T.PackedTrits.from_v11(v11, K, N, 0.021)
    q = torch.empty((M, K), dtype=torch.int8, device="cuda")
    s = torch.empty(M, dtype=torch.float32, device="cuda")
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    T.mm_batched(W, dev(Xf), y=y, acc=acc, q_out=q, scale_out=s)
    rq, rs = O.quant_int8_rows(Xf)
    assert (host(q) == rq).all()
    assert (host(s).view(np.int32) == rs.view(np.int32)).all()
    ra, ry = O.gemm_v11(rq, rs, v11, 0.021, K, N)
    assert (host(acc) == ra).all()
    assert_f32_equal(host(y), ry)


def test_gemm_generated_shapes(cuda):
    """Generated cases (hypothesis, derandomized): M from 2 to 256 (one to
    two 128-row pieces, every row-block configuration), K from 1 to 3000
    (16-byte aligned rows or not, so the LDS ring and the unaligned kernel
    both run), N a multiple of 4 up to 600; single launches and a two-GEMM
    plan; int32 and fp32 outputs against the oracle bit for bit."""
    import torch
    import ter_amd as T
    from hypothesis import given, settings, strategies as st

    def case(M, K, N, seed):
        v11 = O.v11_pack(O.rand_trits(seed, K, N, 0.4))
        X = O.rand_int8(seed + 1, M * K).reshape(M, K)
        xs = (0.001 * (np.arange(M) + 1)).astype(np.float32)
        return v11, X, xs, T.PackedTrits.from_v11(v11, K, N, 0.043)

    @settings(max_examples=30, deadline=None, derandomize=True)
    @given(M=st.integers(2, 256), K=st.integers(1, 3000), N=st.integers(1, 150).map(lambda v: 4 * v),
           seed=st.integers(0, 2 ** 20))
    def single(M, K, N, seed):
        v11, X, xs, W = case(M, K, N, seed)
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
        T.mm_batched(W, dev(X), y=y, acc=acc, x_scale_dev=dev(xs))
        ra, ry = O.gemm_v11(X, xs, v11, 0.043, K, N)
        assert (host(acc) == ra).all(), (M, K, N)
        assert_f32_equal(host(y), ry)

    @settings(max_examples=10, deadline=None, derandomize=True)
    @given(M=st.integers(2, 160), K1=st.integers(1, 100).map(lambda v: 16 * v),
           K2=st.integers(1, 100).map(lambda v: 16 * v), N1=st.integers(1, 100).map(lambda v: 4 * v),
           N2=st.integers(1, 100).map(lambda v: 4 * v), seed=st.integers(0, 2 ** 20))
    def plan(M, K1, K2, N1, N2, seed):
        items, refs = [], []
        for i, (K, N) in enumerate(((K1, N1), (K2, N2))):
            v11, X, xs, W = case(M, K, N, seed + 7 * i)
            y = torch.empty((M, N), dtype=torch.float32, device="cuda")
            acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
            items.append(dict(w=W, x=dev(X), x_scale_dev=dev(xs), y=y, acc=acc))
            refs.append(O.gemm_v11(X, xs, v11, 0.043, K, N))
        P = T.GemmPlan(items)
        P.launch()
        for it, (ra, ry) in zip(items, refs):
            assert (host(it["acc"]) == ra).all(), (M, K1, K2, N1, N2)
            assert_f32_equal(host(it["y"]), ry)
        P.close()

    single()
    plan()


def test_gemm_m1_rows_match_gemv(cuda):
    """Each row of the batched product equals the M = 1 GEMV of that row."""
    import torch
    import ter_amd as T
    M, K, N = 8, 2048, 512
    v11 = O.v11_pack(O.rand_trits(9, K, N))
    X = O.rand_int8(10, M * K).reshape(M, K)
    W = T.PackedTrits.from_v11(v11, K, N, 1.0)
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    T.mm_batched(W, dev(X), acc=acc, x_scale_dev=dev(np.ones(M, np.float32)))
    A = host(acc)
    for m in range(M):
        a1 = torch.empty(N, dtype=torch.int32, device="cuda")
        T.gemv(W, dev(X[m]), acc=a1, x_scale=1.0)
        assert (host(a1) == A[m]).all()


def test_quant_int8_kernel(cuda):
    import ter_amd as T
    x = O.rand_normal_f32(77, 5 * 6912).reshape(5, 6912)
    x[2] = 0.0
    x[3, 100] = 1e6
    q, s = T.quant_int8(dev(x))
    rq, rs = O.quant_int8_rows(x)
    assert (host(q) == rq).all()
    assert (host(s).view(np.int32) == rs.view(np.int32)).all()


def run_plan(specs, seed, wgs, with_acc=True):
    """Build a GemmPlan over `specs`, launch it twice per launch shape and
    compare every item with the oracle (outputs poisoned between launches).
    with_acc=False: fp32 outputs only (the kernels' store path for that form)."""
    import torch
    import ter_amd as T
    items, refs = [], []
    for i, (M, K, N) in enumerate(specs):
        v11 = O.v11_pack(O.rand_trits(seed + i, K, N, 0.4))
        X = O.rand_int8(seed + 50 + i, M * K).reshape(M, K)
        xs = (0.002 * (np.arange(M) + 1 + i)).astype(np.float32)
        W = T.PackedTrits.from_v11(v11, K, N, 0.03 + 0.01 * i)
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        acc = torch.empty((M, N), dtype=torch.int32, device="cuda") if with_acc else None
        items.append(dict(w=W, x=dev(X), x_scale_dev=dev(xs), y=y, acc=acc))
        refs.append(O.gemm_v11(X, xs, v11, 0.03 + 0.01 * i, K, N))
    for wg_per_cu in wgs:
        plan = T.GemmPlan(items, wg_per_cu=wg_per_cu)
        for rep in range(2):
            for it in items:
                if with_acc:
                    it["acc"].fill_(-9)
                it["y"].fill_(-9)
            plan.launch()
            for it, (ra, ry) in zip(items, refs):
                if with_acc:
                    assert (host(it["acc"]) == ra).all(), (wg_per_cu, rep, it["w"].K, it["w"].N)
                assert_f32_equal(host(it["y"]), ry)
        plan.close()


def test_gemm_plan_mixed(cuda):
    """Many GEMMs in one launch (GemmPlan): ragged shapes, different M per
    item, unaligned K (byte-wise X staging), launched twice."""
    run_plan([(8, 2560, 640), (32, 2560, 2560), (3, 300, 20), (17, 6912, 256), (8, 2048, 512), (1, 64, 16)],
             900, (0, 1))


@pytest.mark.parametrize("specs", [
    [(256, 2560, 640), (200, 512, 48), (130, 1024, 300), (8, 2048, 512)],
    [(256, 512, 64), (140, 300, 20)],
], ids=["row_pieces", "bytewise_x"])
def test_gemm_plan_prefill(cuda, specs):
    """M above 128: with every X 16-byte aligned (K a multiple of 16) each item
    is cut into pieces of 128 rows for the LDS-ring kernel (a piece may hold
    fewer rows); with a byte-wise X in the list the register-staged kernel
    takes all rows at once."""
    run_plan(specs, 500, (0,))


@pytest.mark.parametrize("specs", [
    [(8, 2560, 640), (3, 300, 20), (16, 2048, 512), (1, 64, 16), (5, 6912, 256), (12, 1000, 100)],
    [(8, 2560, 640), (8, 2560, 2560), (1, 256, 16), (16, 512, 4000), (4, 6912, 2560)],
], ids=["bytewise_x", "vector_x"])
def test_gemm_plan_small_m(cuda, specs):
    """Small-M plans with a K = 6912 item: 16 rows of it do not fit the
    streamed kernel's LDS, so these run the LDS-ring kernel (ragged M, K and
    N, byte-wise and vector X), at several launch shapes."""
    run_plan(specs, 700, (0, 1, 2))


@pytest.mark.parametrize("M", [16, 32, 100, 128])
@pytest.mark.parametrize("with_acc", [True, False], ids=["y_and_acc", "y_only"])
def test_gemm_plan_list_schedule(cuda, M, with_acc):
    """LDS-ring plans whose blocks the host deals out largest first: K = 6912
    blocks (27 units) first, then K = 2560, then many one-unit blocks (K =
    256) back to back at the end of each workgroup's list, partial blocks at
    every ragged N, ragged M (100 rows: lanes past the last row store
    nothing), with and without int32 outputs (fp32 outputs alone take the
    branch-free store path)."""
    run_plan([(M, 6912, 2560), (M, 256, 640), (M, 256, 48), (M, 512, 4000), (M, 256, 1024), (M, 2560, 256),
              (M, 256, 4096)], 1300 + M, (0,), with_acc)


@pytest.mark.parametrize("specs", [
    [(2, 256, 245760)],                    # Ku = 1: 16-strip output buffers, 12-tile chunks, 15 strips per wave
    [(8, 2560, 12000), (8, 6912, 2560)],   # M = 8 beside K = 6912: 5-strip buffers, 36-tile chunks, ragged last strip
    [(3, 2560, 6000), (7, 2048, 1000), (16, 512, 4096)],  # ragged M: lanes past the last row store nothing
    [(2, 256, 1 << 20)],                   # as long as these lists are, the LDS ring takes them (>= 4 blocks per CU)
    [(8, 2560, 262144), (8, 6912, 2560)],
], ids=["ku1_long_runs", "m8_bitnet_k", "ragged_m", "ring_ku1", "ring_m8"])
@pytest.mark.parametrize("with_acc", [True, False], ids=["y_and_acc", "y_only"])
def test_gemm_stream_chunks(cuda, specs, with_acc):
    """The streamed kernel (M <= 16 where the X image and the output buffers
    fit, and the list too short for the LDS ring): at one workgroup per CU each
    wave's run spans several chunks, so completed strips are buffered in LDS
    and written between chunks many times per wave; fp32 outputs alone take
    the branch-free store path.  The last two lists are long enough (at least
    4 ring blocks per CU on MI355X's 256 CUs) for the LDS ring."""
    run_plan(specs, 1300, (1,), with_acc)


@pytest.mark.parametrize("M", [8, 32, 128])
def test_gemm_plan_bitnet_layer(cuda, M):
    """One BitNet-2B layer (7 projections) at the C4 batch sizes in one launch."""
    import torch
    import ter_amd as T
    shapes = [(2560, 2560), (2560, 640), (2560, 640), (2560, 2560), (2560, 6912), (2560, 6912), (6912, 2560)]
    xs_of = {}
    items, refs = [], []
    for i, (K, N) in enumerate(shapes):
        v11 = O.v11_pack(O.rand_trits(70 + i, K, N, 0.4))
        if K not in xs_of:
            Xf = O.rand_normal_f32(K + M, M * K).reshape(M, K)
            q, s = O.quant_int8_rows(Xf)
            xs_of[K] = (q, s, dev(q), dev(s))
        q, s, qd, sd = xs_of[K]
        W = T.PackedTrits.from_v11(v11, K, N, 0.05)
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        items.append(dict(w=W, x=qd, x_scale_dev=sd, y=y))
        refs.append(O.gemm_v11(q, s, v11, 0.05, K, N)[1])
    T.GemmPlan(items).launch()
    for it, ry in zip(items, refs):
        assert_f32_equal(host(it["y"]), ry)


@pytest.mark.parametrize("M,K,N", [(8, 2560, 640), (32, 2560, 128), (128, 6912, 64), (200, 512, 48)])
def test_gemm_payload_magnitude(cuda, M, K, N):
    """{-m, 0, +m} payloads (m = 9841) on every GEMM kernel (streamed M <= 16,
    LDS ring, pieces of 128 rows) and in a GEMM plan: each row's fp32 output
    is the reference mm_row's float(int64 m * acc) * fl(xs * ws), bit for bit."""
    import torch
    import ter_amd as T
    m = 9841
    w = O.rand_trits(M + K + N, K, N, 0.4).astype(np.int32) * m
    X = O.rand_int8(M * K + 1, M * K).reshape(M, K)
    xs = (0.0007 * (np.arange(M) + 3)).astype(np.float32)
    ws = 0.00019
    W = T.PackedTrits.from_payload(w, ws)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    T.mm_batched(W, dev(X), y=y, acc=acc, x_scale_dev=dev(xs))
    ha, hy = host(acc), host(y)
    rows = [0, M // 2, M - 1]
    for r in rows:
        ra, ry = O.mm_row(X.astype(np.int32), r, float(xs[r]), w, ws)
        assert (ha[r].astype(np.int64) * m == ra).all(), r
        assert_f32_equal(hy[r], ry)
    assert np.abs(ha.astype(np.int64) * m).max() > 2 ** 24
    # every row through the closed form (the trit accumulators are checked above on sampled rows)
    want = (ha.astype(np.int64) * m).astype(np.float32) * (xs[:, None] * np.float32(ws)).astype(np.float32)
    assert_f32_equal(hy, want)
    # the same GEMM through a plan
    y2 = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    xd, sd = dev(X), dev(xs)
    p = T.GemmPlan([dict(w=W, x=xd, x_scale_dev=sd, y=y2)])
    p.launch()
    assert (host(y2).view(np.int32) == hy.view(np.int32)).all()
