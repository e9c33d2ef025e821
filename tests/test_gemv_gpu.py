"""GPU parity of the M = 1 packed-trit GEMV against the CPU oracle.

Bar: int32 accumulators bit-exact; fp32 outputs bit-exact (the kernel forms
float(acc) * (x_scale * w_scale) in the reference's order; the stated
tolerance of the contract is 1e-5 relative, REL_TOL below, and every fp32
comparison here also asserts it).
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
    assert (got.view(np.int32) == want.view(np.int32)).all(), "fp32 output not bit-identical"


def gemv_case(K, N, seed, p0=1 / 3, xs=0.0312, ws=0.05):
    import torch
    import ter_amd as T
    w = O.rand_trits(seed, K, N, p0)
    v11 = O.v11_pack(w)
    x = O.rand_int8(seed + 1, K)
    W = T.PackedTrits.from_v11(v11, K, N, ws)
    acc = torch.empty(N, dtype=torch.int32, device="cuda")
    y = torch.empty(N, dtype=torch.float32, device="cuda")
    T.gemv(W, dev(x), y=y, acc=acc, x_scale=xs)
    ra, ry = O.gemv_v11(x, xs, v11, ws, K, N)
    assert (host(acc) == ra).all(), f"int32 acc mismatch K={K} N={N}"
    assert_f32_equal(host(y), ry)


SHAPES = [
    (2048, 2048),   # C1 (Llama Wq/Wo)
    (2048, 512),    # Wk/Wv
    (2048, 8192),   # Wgate/Wup
    (8192, 2048),   # Wdown
    (2560, 2560), (2560, 640), (2560, 6912), (6912, 2560),  # BitNet-2B
    (128, 64),      # reference correctness-test shape
    (64, 16), (1, 4), (300, 20), (257, 4), (4112, 100), (255, 1028),
]


@pytest.mark.parametrize("K,N", SHAPES)
def test_gemv_shapes(cuda, K, N):
    gemv_case(K, N, seed=K * 7 + N)


def test_gemv_generated_shapes(cuda):
    """Generated cases (hypothesis, derandomized): K from 1 to 5000 and N
    from 1 to 700 (ragged units and strips, every launch form the size
    picks; v11 weights where N is a multiple of 4, the TritTensor payload
    otherwise), zero densities from none to all, single GEMVs and a
    three-GEMV work list of unrelated shapes; int32 and fp32 outputs against
    the oracle bit for bit."""
    import torch
    import ter_amd as T
    from hypothesis import given, settings, strategies as st

    @settings(max_examples=40, deadline=None, derandomize=True)
    @given(K=st.integers(1, 5000), N=st.integers(1, 700), p0=st.sampled_from([0.0, 0.4, 0.9, 1.0]),
           seed=st.integers(0, 2 ** 20))
    def single(K, N, p0, seed):
        if N % 4 == 0:  # the v11 layout packs 4 columns per byte
            gemv_case(K, N, seed=seed, p0=p0)
            return
        # any N: the TritTensor payload, against the restated mm_row
        w = O.rand_trits(seed, K, N, p0).astype(np.int32)
        x = O.rand_int8(seed + 1, K).astype(np.int32)
        W = T.PackedTrits.from_payload(w, 0.05)
        acc = torch.empty(N, dtype=torch.int32, device="cuda")
        y = torch.empty(N, dtype=torch.float32, device="cuda")
        T.gemv(W, dev(x.astype(np.int8)), y=y, acc=acc, x_scale=0.0312)
        ra, ry = O.mm_row(x[None], 0, 0.0312, w, 0.05)
        assert (host(acc).astype(np.int64) == ra).all(), (K, N)
        assert_f32_equal(host(y), ry)

    @settings(max_examples=12, deadline=None, derandomize=True)
    @given(shapes=st.lists(st.tuples(st.integers(1, 3000), st.integers(1, 100).map(lambda v: 4 * v)), min_size=3,
                           max_size=3),
           seed=st.integers(0, 2 ** 20))
    def plan(shapes, seed):
        items, refs = [], []
        for i, (K, N) in enumerate(shapes):
            v11 = O.v11_pack(O.rand_trits(seed + i, K, N, 0.4))
            x = O.rand_int8(seed + 10 + i, K)
            W = T.PackedTrits.from_v11(v11, K, N, 0.05 + 0.01 * i)
            acc = torch.empty(N, dtype=torch.int32, device="cuda")
            y = torch.empty(N, dtype=torch.float32, device="cuda")
            items.append(dict(w=W, x=dev(x), x_scale=0.03, y=y, acc=acc))
            refs.append(O.gemv_v11(x, 0.03, v11, 0.05 + 0.01 * i, K, N))
        P = T.Plan(items)
        P.launch()
        for it, (ra, ry) in zip(items, refs):
            assert (host(it["acc"]) == ra).all(), shapes
            assert_f32_equal(host(it["y"]), ry)
        P.close()

    single()
    plan()


def test_gemv_golden_reference_vectors(cuda, golden):
    """Vectors written by the reference mm_row itself (tests/golden)."""
    import torch
    import ter_amd as T
    g = golden("mm_row_random.npz")
    for i in range(int(g["n_cases"])):
        K, N = int(g[f"c{i}_K"]), int(g[f"c{i}_N"])
        row = int(g[f"c{i}_row"])
        x = g[f"c{i}_X"][row]
        xs, ws = float(g[f"c{i}_xs"]), float(g[f"c{i}_ws"])
        for W in (T.PackedTrits.from_v11(g[f"c{i}_v11"], K, N, ws),
                  T.PackedTrits.from_payload(g[f"c{i}_W"].astype(np.int32), ws)):
            acc = torch.empty(N, dtype=torch.int32, device="cuda")
            y = torch.empty(N, dtype=torch.float32, device="cuda")
            T.gemv(W, dev(x), y=y, acc=acc, x_scale=xs)
            assert (host(acc).astype(np.int64) == g[f"c{i}_acc"]).all(), i
            assert_f32_equal(host(y), g[f"c{i}_out"])


def test_gemv_reference_fixtures(cuda, golden):
    import torch
    import ter_amd as T
    f = golden("int4tc_fixture.npz")
    K, N = int(f["K"]), int(f["N"])
    W = T.PackedTrits.from_v11(f["v11"], K, N, 1.0)
    acc = torch.empty(N, dtype=torch.int32, device="cuda")
    T.gemv(W, dev(f["X"].astype(np.int8)), acc=acc, x_scale=1.0)
    assert (host(acc).astype(np.int64) == f["acc"]).all()
    # The closed-form fixtures of tests/test_kernel_matmul_b_small.cpp hold
    # format-B weights in {-2..2} (i % 5 - 2): not ternary, so the boundary
    # refuses them rather than computing them on the CPU.
    m = golden("matmul_b_small.npz")
    for wk in ("W1", "W2"):
        with pytest.raises(T._lib.TerHipError) as e:
            T.PackedTrits.from_payload(m[wk].astype(np.int32), 1.0)
        assert e.value.code == T._lib.ERR_PAYLOAD
    # Their ternary part (sign of W) goes through the payload path, K = 27 / 54, N = 1.
    for xk, wk in (("X1", "W1"), ("X2", "W2")):
        w = np.sign(m[wk]).astype(np.int32)
        W = T.PackedTrits.from_payload(w, 1.0)
        acc = torch.empty(1, dtype=torch.int32, device="cuda")
        T.gemv(W, dev(m[xk].astype(np.int8)), acc=acc, x_scale=1.0)
        assert int(host(acc)[0]) == int(m[xk].astype(np.int64) @ w[:, 0])


@pytest.mark.parametrize("K,N,m", [(100, 12, 9841), (2560, 640, 9841), (6912, 80, 9841), (2048, 48, 3)])
def test_gemv_payload_magnitude(cuda, K, N, m):
    """A ternary payload {-m,0,+m} (9-trit quantized BitNet weights,
    src/host/load_gguf.cpp:111) is packed as {-1,0,+1} with m kept as an
    integer: y = float(int64(m * acc)) * fl(xs * ws), bit for bit the
    reference mm_row (src/tx/forward.cpp:333-345), also where m * acc is
    beyond 2^24; every output form (fp32, fp16, residual) uses it."""
    import torch
    import ter_amd as T
    w = O.rand_trits(3 + K, K, N, 0.4).astype(np.int32) * m
    x = O.rand_int8(4 + K, K)
    xs, ws = 0.0173, 0.00071
    W = T.PackedTrits.from_payload(w, ws)
    assert W.magnitude == m and W.scale == np.float32(ws)
    acc = torch.empty(N, dtype=torch.int32, device="cuda")
    y = torch.empty(N, dtype=torch.float32, device="cuda")
    T.gemv(W, dev(x), y=y, acc=acc, x_scale=xs)
    ref_acc, ref_y = O.mm_row(x.astype(np.int32)[None], 0, xs, w, ws)
    assert (host(acc).astype(np.int64) * m == ref_acc).all()
    assert_f32_equal(host(y), ref_y)
    if K >= 2048 and m > 1000:
        assert np.abs(ref_acc).max() > 2 ** 24
    # the fp16 and residual epilogues take the same y
    y16 = torch.empty(N, dtype=torch.float16, device="cuda")
    resid = dev(O.rand_normal_f32(5 + K, N))
    r0 = host(resid).copy()
    T.gemv(W, dev(x), y16=y16, resid=resid, x_scale=xs)
    assert (host(y16).view(np.uint16) == O.float_to_half_bits(ref_y)).all()
    assert (host(resid).view(np.int32) == O.residual_add_f16(r0, ref_y).view(np.int32)).all()


def test_mm_row_bitnet9_golden(cuda, golden):
    """The reference host forward's own mm_row calls on BitNet weights
    (tests/golden/mm_row_bitnet9.npz, written by the reference build):
    payload {-9841, 0, +9841} and 9-trit activations (|x| <= 9841, the
    int16 GEMV) -- the fp32 outputs bit for bit."""
    import ter_amd as T
    g = golden("mm_row_bitnet9.npz")
    for i in range(int(g["n_cases"])):
        K, N = int(g[f"c{i}_K"]), int(g[f"c{i}_N"])
        m = int(g[f"c{i}_mag"])
        W = T.PackedTrits.from_payload(g[f"c{i}_trits"].astype(np.int32) * m, float(g[f"c{i}_ws"]))
        X = g[f"c{i}_X"].astype(np.int32)
        out = T.mm_row(np.stack([np.zeros(K, np.int32), X]), 1, float(g[f"c{i}_xs"]), W, K, N)
        assert_f32_equal(out, g[f"c{i}_out"])


def test_mm_row_blocked_golden(cuda, golden):
    """The per-block branch of mm_row (src/tx/forward.cpp:308-330) on the
    GPU against the reference build's outputs (tests/golden/mm_row_blocked.npz):
    block sizes that do and do not divide N, zero-scale blocks -- bit for bit."""
    import ter_amd as T
    g = golden("mm_row_blocked.npz")
    for i in range(int(g["n_cases"])):
        K, N, bs = int(g[f"c{i}_K"]), int(g[f"c{i}_N"]), int(g[f"c{i}_bs"])
        m = int(g[f"c{i}_mag"])
        W = T.PackedTrits.from_payload(g[f"c{i}_trits"].astype(np.int32) * m, 1.0)
        X = g[f"c{i}_X"].astype(np.int32)
        out = T.mm_row_blocked(np.stack([X, X[::-1]]), 0, float(g[f"c{i}_xs"]), W, K, N, g[f"c{i}_bsc"], bs)
        assert_f32_equal(out, g[f"c{i}_out"])


def test_mm_row_blocked_refuses_inexact_terms(cuda):
    """|x| * m at 2^29 or beyond would make the double terms round: refused."""
    import ter_amd as T
    K, N = 64, 16
    W = T.PackedTrits.from_payload(O.rand_trits(1, K, N).astype(np.int32) * 32767, 1.0)
    X = np.zeros((1, K), np.int32)
    X[0, 3] = 16385  # 16385 * 32767 >= 2^29
    with pytest.raises(T._lib.TerHipError) as e:
        T.mm_row_blocked(X, 0, 1.0, W, K, N, np.ones(K * N, np.float32), 1)
    assert e.value.code == T._lib.ERR_PAYLOAD


def int16_case(K, N, seed, x, p0=1 / 3, xs=0.00013, ws=0.05, x_scale_dev=False):
    import torch
    import ter_amd as T
    w = O.rand_trits(seed, K, N, p0).astype(np.int32)
    W = T.PackedTrits.from_payload(w, ws)
    acc = torch.empty(N, dtype=torch.int32, device="cuda")
    y = torch.empty(N, dtype=torch.float32, device="cuda")
    if x_scale_dev:
        T.gemv(W, dev(x.astype(np.int16)), y=y, acc=acc, x_scale_dev=dev(np.array([xs], np.float32)))
    else:
        T.gemv(W, dev(x.astype(np.int16)), y=y, acc=acc, x_scale=xs)
    ra, ry = O.mm_row(x.astype(np.int32)[None], 0, xs, w, ws)
    assert (host(acc).astype(np.int64) == ra).all(), f"int16 acc mismatch K={K} N={N}"
    assert_f32_equal(host(y), ry)


@pytest.mark.parametrize("K,N", [(2560, 2560), (2560, 640), (6912, 2560), (2048, 8192), (1, 4), (17, 33),
                                 (300, 20), (4112, 100), (32768, 48)])
def test_gemv_int16_activations(cuda, K, N):
    """int16 X (the host forward's 9-trit payloads, and the whole int16
    range) on the int16 GEMV: exact accumulators and fp32 outputs."""
    x = O.splitmix64(K * 31 + N, K)
    x9 = (x % np.uint64(2 * 9841 + 1)).astype(np.int64) - 9841
    int16_case(K, N, K + N, x9)
    full = (x % np.uint64(65536)).astype(np.int64) - 32768
    int16_case(K, N, K + N + 1, full, x_scale_dev=True)


def test_gemv_int16_extremes(cuda):
    """All -32768, all 32767 (the accumulator's largest magnitudes at
    K = 32768: 2^30), alternating, and a misaligned (odd-element) vector."""
    import torch
    import ter_amd as T
    K, N = 32768, 20
    for fill in (-32768, 32767):
        int16_case(K, N, 5, np.full(K, fill), p0=0.0)
    alt = np.where(np.arange(K) % 2 == 0, 32767, -32768)
    int16_case(K, N, 6, alt)
    # one element off 16-byte alignment: the element-wise staging path
    K2 = 1000
    x = ((O.splitmix64(7, K2 + 1) % np.uint64(65536)).astype(np.int64) - 32768).astype(np.int16)
    w = O.rand_trits(8, K2, N).astype(np.int32)
    W = T.PackedTrits.from_payload(w, 0.5)
    buf = dev(x)
    acc = torch.empty(N, dtype=torch.int32, device="cuda")
    T.gemv(W, buf[1:], acc=acc, x_scale=1.0)
    ra, _ = O.mm_row(x[1:].astype(np.int32)[None], 0, 1.0, w, 1.0)
    assert (host(acc).astype(np.int64) == ra).all()


def test_gemv_fp32_prologue(cuda):
    """fp32 X quantized by absmax inside the kernel (quant_int8_k steps)."""
    import torch
    import ter_amd as T
    for K, N, seed in ((2560, 2560, 1), (6912, 2560, 2), (300, 20, 3), (2560, 640, 4)):
        w = O.rand_trits(seed, K, N, 0.4)
        v11 = O.v11_pack(w)
        xf = O.rand_normal_f32(seed + 50, K)
        W = T.PackedTrits.from_v11(v11, K, N, 0.037)
        q = torch.empty(K, dtype=torch.int8, device="cuda")
        s = torch.empty(1, dtype=torch.float32, device="cuda")
        acc = torch.empty(N, dtype=torch.int32, device="cuda")
        y = torch.empty(N, dtype=torch.float32, device="cuda")
        T.gemv(W, dev(xf), y=y, acc=acc, q_out=q, scale_out=s)
        rq, rs = O.quant_int8(xf)
        assert (host(q) == rq).all(), "in-kernel quantization differs"
        assert host(s)[0].view(np.int32) == np.float32(rs).view(np.int32)
        ra, ry = O.gemv_v11(rq, rs, v11, 0.037, K, N)
        assert (host(acc) == ra).all()
        assert_f32_equal(host(y), ry)


def test_gemv_device_scale_and_dispatch(cuda):
    import torch
    import ter_amd as T
    K, N = 2048, 512
    w = O.rand_trits(21, K, N)
    v11 = O.v11_pack(w)
    x = O.rand_int8(22, K)
    W = T.PackedTrits.from_v11(v11, K, N, 0.061)
    sx = torch.tensor([0.0123], dtype=torch.float32, device="cuda")
    out = torch.empty(N, dtype=torch.float32, device="cuda")
    T.mm_packed_dispatch(dev(x), sx, W, out, K, N)
    _, ry = O.gemv_v11(x, np.float32(0.0123), v11, 0.061, K, N)
    assert_f32_equal(host(out), ry)


def test_mm_row_host_contract(cuda):
    import ter_amd as T
    K, N = 300, 24
    w = O.rand_trits(31, K, N).astype(np.int32)
    X = O.rand_int8(32, 2 * K).astype(np.int32).reshape(2, K)
    W = T.PackedTrits.from_payload(w, 0.02)
    out = T.mm_row(X, 1, 0.5, W, K, N)
    _, ref = O.mm_row(X, 1, 0.5, w, 0.02)
    assert_f32_equal(out, ref)


def test_mm_row_generated_host_calls(cuda):
    """Generated host mm_row calls (hypothesis, derandomized): the host
    forward's contract (int32 rows in host memory, a row index, outputs in
    host memory) with K from 1 to 4000, N from 1 to 400, payload magnitudes
    1, 3 and 9841, int8-range or 9-trit rows; every output bit for bit
    against the restated mm_row."""
    import ter_amd as T
    from hypothesis import given, settings, strategies as st

    @settings(max_examples=30, deadline=None, derandomize=True)
    @given(K=st.integers(1, 4000), N=st.integers(1, 400), m=st.sampled_from([1, 3, 9841]), wide=st.booleans(),
           row=st.integers(0, 2), seed=st.integers(0, 2 ** 20))
    def check(K, N, m, wide, row, seed):
        rng = np.random.default_rng(seed)
        w = (rng.integers(-1, 2, size=(K, N)) * m).astype(np.int32)
        lim = 9841 if wide else 127
        X = rng.integers(-lim, lim + 1, size=(3, K)).astype(np.int32)
        W = T.PackedTrits.from_payload(w, 0.02)
        out = T.mm_row(X, row, 0.5, W, K, N)
        _, ref = O.mm_row(X, row, 0.5, w, 0.02)
        assert_f32_equal(out, ref)

    check()


def test_gemv_edge_values(cuda):
    import torch
    import ter_amd as T
    K, N = 1024, 64
    w = O.rand_trits(41, K, N)
    v11 = O.v11_pack(w)
    W = T.PackedTrits.from_v11(v11, K, N, 1.0)
    for x in (np.zeros(K, np.int8), np.full(K, -128, np.int8), np.full(K, 127, np.int8),
              np.where(np.arange(K) % 2 == 0, -128, 127).astype(np.int8)):
        acc = torch.empty(N, dtype=torch.int32, device="cuda")
        T.gemv(W, dev(x), acc=acc, x_scale=1.0)
        ra, _ = O.gemv_v11(x, 1.0, v11, 1.0, K, N)
        assert (host(acc) == ra).all()
    # all-zero and all-reserved (code 11) weights
    for fill in (0x00, 0xFF):
        Wz = T.PackedTrits.from_v11(np.full((N // 4) * K, fill, np.uint8), K, N, 1.0)
        acc = torch.empty(N, dtype=torch.int32, device="cuda")
        T.gemv(Wz, dev(O.rand_int8(5, K)), acc=acc, x_scale=1.0)
        assert (host(acc) == 0).all()


def test_v11_roundtrip_on_device(cuda):
    import ter_amd as T
    for K, N in ((300, 20), (2048, 512), (7, 4)):
        v11 = O.v11_pack(O.rand_trits(K + N, K, N))
        W = T.PackedTrits.from_v11(v11, K, N, 1.0)
        assert (host(W.to_v11()) == v11).all()
    # code 11 is normalised to 00 (both decode as 0, include/ter/pack.hpp:18-19)
    W = T.PackedTrits.from_v11(np.full(8, 0xFF, np.uint8), 2, 16, 1.0)
    assert (host(W.to_v11()) == 0).all()


def test_synth_generator_matches_oracle(cuda):
    import ter_amd as T
    K, N = 96, 40
    for p0 in (1 / 3, 0.4):
        v = host(T.synth_v11(K, N, seed=1234, p_zero=p0))
        assert (O.v11_unpack(v, K, N) == O.rand_trits(1234, K, N, p0)).all()
    x = host(T.synth_i8(1000, seed=99))
    assert (x == O.rand_int8(99, 1000)).all()


@pytest.mark.parametrize("wg_per_cu", [1, 2, 3, 0])
def test_plan_worklist_mixed(cuda, wg_per_cu):
    """Many GEMVs in one launch: int8 and fp32 inputs, ragged shapes, strips
    split across waves/workgroups (fix-up path); launched twice to check the
    fix-up slots clean themselves."""
    import torch
    import ter_amd as T
    specs = [(2048, 512, "i8"), (300, 20, "f32"), (2560, 640, "f32"), (8192, 2048, "i8"),
             (64, 16, "i8"), (6912, 256, "f32"), (2048, 2048, "i8")]
    items, refs = [], []
    for i, (K, N, kind) in enumerate(specs):
        v11 = O.v11_pack(O.rand_trits(500 + i, K, N))
        W = T.PackedTrits.from_v11(v11, K, N, 0.01 * (i + 1))
        y = torch.empty(N, dtype=torch.float32, device="cuda")
        acc = torch.empty(N, dtype=torch.int32, device="cuda")
        if kind == "i8":
            x = O.rand_int8(600 + i, K)
            items.append(dict(w=W, x=dev(x), x_scale=0.5, y=y, acc=acc))
            ra, ry = O.gemv_v11(x, 0.5, v11, 0.01 * (i + 1), K, N)
        else:
            xf = O.rand_normal_f32(600 + i, K)
            items.append(dict(w=W, x=dev(xf), y=y, acc=acc))
            q, s = O.quant_int8(xf)
            ra, ry = O.gemv_v11(q, s, v11, 0.01 * (i + 1), K, N)
        refs.append((ra, ry))
    plan = T.Plan(items, wg_per_cu=wg_per_cu)
    for rep in range(2):
        for it in items:
            it["acc"].fill_(-7)
            it["y"].fill_(-7)
        plan.launch()
        for it, (ra, ry) in zip(items, refs):
            assert (host(it["acc"]) == ra).all(), (rep, it["w"].K, it["w"].N)
            assert_f32_equal(host(it["y"]), ry)
    for it in items:  # slots are zero at rest
        K, N = it["w"].K, it["w"].N
        fix = it["w"].buf[it["w"].buf.numel() - 8 * N:]
        assert int(host(fix).astype(np.int64).sum()) == 0


@pytest.mark.parametrize("K,N,count,wg_per_cu", [
    (6912, 1024, 20, 1),   # 34560 tiles / 256 workgroups: ranges on strip edges, waves' partials meet in LDS
    (20480, 496, 16, 1),   # 80-tile strips: too long to move range ends (LDS + global fix-up at range ends)
    (6912, 1024, 20, 2),   # 17 tiles per wave: each wave adds its partial strips to the global slots
])
def test_plan_partitions(cuda, K, N, count, wg_per_cu):
    """The three ways a work list's strips are completed (combine_mode and
    snap_ranges): bit-exact against the oracle on two launches in a row, and
    the global fix-up slots clean afterwards."""
    import torch
    import ter_amd as T
    items, refs = [], []
    for i in range(count):
        v11 = O.v11_pack(O.rand_trits(900 + i, K, N))
        W = T.PackedTrits.from_v11(v11, K, N, 0.02 * (i + 1))
        x = O.rand_int8(950 + i, K)
        acc = torch.empty(N, dtype=torch.int32, device="cuda")
        y = torch.empty(N, dtype=torch.float32, device="cuda")
        items.append(dict(w=W, x=dev(x), x_scale=0.25, y=y, acc=acc))
        refs.append(O.gemv_v11(x, 0.25, v11, 0.02 * (i + 1), K, N))
    plan = T.Plan(items, wg_per_cu=wg_per_cu)
    for rep in range(2):
        for it in items:
            it["acc"].fill_(-7)
            it["y"].fill_(-7)
        plan.launch()
        for it, (ra, ry) in zip(items, refs):
            assert (host(it["acc"]) == ra).all(), (rep, K, N, wg_per_cu)
            assert_f32_equal(host(it["y"]), ry)
    for it in items:
        fix = it["w"].buf[it["w"].buf.numel() - 8 * N:]
        assert int(host(fix).astype(np.int64).sum()) == 0


def test_single_gemv_ranges_on_strip_edges(cuda):
    """A single GEMV large enough that its workgroup ranges move to strip
    edges inside the kernel (K = 2048, N = 262144: 131072 tiles, 32 per wave
    at 1024 workgroups)."""
    gemv_case(2048, 262144, seed=4242)


def test_plan_keeps_its_tensors_alive(cuda):
    """A plan holds every tensor whose address it copied: outputs passed as
    temporaries stay allocated and receive the results."""
    import gc
    import weakref
    import torch
    import ter_amd as T
    K, N = 2048, 512
    v11 = O.v11_pack(O.rand_trits(77, K, N))
    x = O.rand_int8(78, K)
    W = T.PackedTrits.from_v11(v11, K, N, 0.5)
    plan = T.Plan([dict(w=W, x=dev(x), x_scale=1.0, acc=torch.empty(N, dtype=torch.int32, device="cuda"))])
    refs = [weakref.ref(t) for t in plan._keep if isinstance(t, torch.Tensor)]
    del W
    gc.collect()
    torch.cuda.empty_cache()
    assert all(r() is not None for r in refs)
    plan.launch()
    acc = [t for t in plan._keep if isinstance(t, torch.Tensor) and t.dtype == torch.int32][0]
    ra, _ = O.gemv_v11(x, 1.0, v11, 0.5, K, N)
    assert (host(acc) == ra).all()


def test_handle_native_slot_counts(cuda):
    import torch
    import ter_amd as T
    K, N = 2048, 512
    v11 = O.v11_pack(O.rand_trits(71, K, N))
    x = O.rand_int8(72, K)
    W = T.PackedTrits.from_v11(v11, K, N, 0.5)
    h = T.Handle(0)
    acc = torch.empty(N, dtype=torch.int32, device="cuda")
    assert h.matmul(W, dev(x), acc=acc, x_scale=1.0) == 0
    ra, _ = O.gemv_v11(x, 1.0, v11, 0.5, K, N)
    assert (host(acc) == ra).all()
    assert h.op_counts()["tvmac"] == O.mm_row_tvmac(K, N)  # src/tx/forward.cpp:349-350
    h.reset_counters()
    assert h.op_counts()["tvmac"] == 0


def test_llama_sweep_full_size_properties(cuda):
    """C2's shapes at full size (16 layers x 7 GEMVs, ~245 MB packed, one
    launch), with weights of other seeds than the bench's: linearity
    acc(x1) + acc(x2) == acc(x1 + x2) and acc(-x) == -acc(x) on every column,
    plus exact oracle values on sampled columns of every GEMV.  (The bench's
    own work list is checked column for column in test_fullsize_gpu.py.)"""
    import torch
    import ter_amd as T
    shapes = [(2048, 2048), (2048, 512), (2048, 512), (2048, 2048), (2048, 8192), (2048, 8192), (8192, 2048)]
    rng = np.random.default_rng(5)
    Ws, v11s, xs = [], [], []
    for layer in range(16):
        for i, (K, N) in enumerate(shapes):
            v = T.synth_v11(K, N, seed=10_000 + layer * 7 + i)
            Ws.append(T.PackedTrits.from_v11(v, K, N, 0.05))
            v11s.append(v)
    xa = {K: O.rand_int8(K, K, -63, 63) for K in (2048, 8192)}
    xb = {K: O.rand_int8(K + 1, K, -64, 64) for K in (2048, 8192)}

    def run(xmap):
        items, outs = [], []
        for W in Ws:
            acc = torch.empty(W.N, dtype=torch.int32, device="cuda")
            items.append(dict(w=W, x=dev(xmap[W.K]), x_scale=1.0, acc=acc))
            outs.append(acc)
        T.Plan(items).launch()
        torch.cuda.synchronize()
        return [o.cpu().numpy() for o in outs]

    a = run(xa)
    b = run(xb)
    s = run({K: (xa[K].astype(np.int16) + xb[K]).astype(np.int8) for K in xa})
    n = run({K: (-xa[K].astype(np.int16)).astype(np.int8) for K in xa})
    for i, W in enumerate(Ws):
        assert (a[i] + b[i] == s[i]).all() and (n[i] == -a[i]).all(), i
        jbs = rng.choice(W.N // 4, size=8, replace=False)
        cols, ra, _ = O.gemv_v11_cols(xa[W.K], 1.0, host(v11s[i]), 1.0, W.K, W.N, jbs)
        assert (a[i][cols] == ra).all(), i


@pytest.mark.parametrize("K,N", [(2560, 640), (6912, 2560), (128, 4), (64, 8), (384, 20)])
def test_pack_i2s_matches_oracle_repack(cuda, K, N):
    """Device repack of GGUF i2_s codes (tools/convert_bitnet_to_packed.py:85-157):
    its v11 bytes equal the oracle's i2s_to_v11 of the same codes, and a GEMV
    on it equals the oracle GEMV (K=384: ragged unit, N=20: ragged strip)."""
    import torch
    import ter_amd as T
    raw = (O.splitmix64(K * 7 + N, N * K // 4) & np.uint64(0xFF)).astype(np.uint8)
    W = T.PackedTrits.from_i2s(raw, K, N, 0.0271)
    want_v11 = O.i2s_to_v11(raw, K, N)
    assert (host(W.to_v11()) == want_v11).all()
    x = O.rand_int8(K + 1, K)
    acc = torch.empty(N, dtype=torch.int32, device="cuda")
    y = torch.empty(N, dtype=torch.float32, device="cuda")
    T.gemv(W, dev(x), y=y, acc=acc, x_scale=0.013)
    ra, ry = O.gemv_v11(x, np.float32(0.013), want_v11, 0.0271, K, N)
    assert (host(acc) == ra).all()
    assert_f32_equal(host(y), ry)
