"""GPU parity of the GEMV kernel's vector prologue: work lists whose GEMVs
share one activation kind, with K a multiple of 16 and 16-byte aligned x / up
/ gamma, run a kernel specialised on that kind (branch-free buffer loads of
the activations, issued before the weights).  The same items placed at an
unaligned offset take the general prologue.  Small lists run in strip mode
(whole strips per workgroup, partials reduced in LDS) unless wg_per_cu is
given, which selects the stream-K partition.

Bar: both placements give int32 accumulators, fp32 outputs, the int8
activation copy and its scale bit-exact against the oracle (quant_int8_k,
rmsnorm_quant_*_k and relu2_mul_rmsnorm_quant_k of
cuda/ter_cuda_forward_packed.cu:40-62 and cuda/ter_cuda_forward_bitnet.cu:64-146,
258-309, then mm_row's integer dot products).
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu
REL_TOL = 1e-5

KINDS = ["i8", "f32", "f32_rms", "f16_rms", "relu2"]


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def placed(a, offset):
    """Device copy of a starting `offset` elements into a fresh buffer (offset 0:
    256-byte aligned; 1: misaligned for 16-byte vectors)."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    buf = torch.zeros(a.size + 16, dtype=t.dtype, device="cuda")
    view = buf[offset:offset + a.size]
    view.copy_(t.cuda())
    return view


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


def make_case(kind, K, N, seed):
    """Host inputs of one item and the oracle's (int8 x, scale, acc, y)."""
    rng = np.random.default_rng(seed)
    v11 = O.v11_pack(O.rand_trits(seed, K, N, 0.4))
    ws = 0.01 + 0.001 * (seed % 50)
    host_in = {}
    if kind == "i8":
        x = O.rand_int8(seed + 1, K)
        host_in["x"] = x
        rq, rs = x, np.float32(0.037)
    elif kind == "f32":
        x = (rng.standard_normal(K) * 2).astype(np.float32)
        host_in["x"] = x
        rq, rs = O.quant_int8(x)
    elif kind in ("f32_rms", "f16_rms"):
        x = (rng.standard_normal(K) * 3).astype(np.float32)
        if kind == "f16_rms":
            x = x.astype(np.float16)
        g = rng.uniform(0.25, 2.0, K).astype(np.float16)
        host_in.update(x=x, gamma=g)
        rq, rs, _ = O.rmsnorm_quant(x, g, 1e-5)
    else:
        gate = rng.standard_normal(K).astype(np.float16)
        up = rng.standard_normal(K).astype(np.float16)
        g = rng.uniform(0.5, 1.5, K).astype(np.float16)
        host_in.update(x=gate, up=up, gamma=g)
        rq, rs, _ = O.relu2_rmsnorm_quant(gate, up, g, 1e-5)
    ra, ry = O.gemv_v11(rq, rs, v11, ws, K, N)
    return dict(v11=v11, ws=ws, host=host_in, rq=rq, rs=np.float32(rs), ra=ra, ry=ry)


def item_of(kind, case, K, N, offset):
    import torch
    import ter_amd as T
    W = T.PackedTrits.from_v11(case["v11"], K, N, case["ws"])
    it = dict(w=W, x=placed(case["host"]["x"], offset),
              y=torch.empty(N, dtype=torch.float32, device="cuda"),
              acc=torch.empty(N, dtype=torch.int32, device="cuda"))
    if kind == "i8":
        it["x_scale"] = float(case["rs"])
    else:
        it["q_out"] = torch.empty(K, dtype=torch.int8, device="cuda")
        it["scale_out"] = torch.empty(1, dtype=torch.float32, device="cuda")
    if "gamma" in case["host"]:
        it["gamma"] = placed(case["host"]["gamma"], offset)
        it["eps"] = 1e-5
    if "up" in case["host"]:
        it["up"] = placed(case["host"]["up"], offset)
    return it


def check(kind, it, case, what):
    assert (host(it["acc"]) == case["ra"]).all(), what
    assert_f32_equal(host(it["y"]), case["ry"])
    if kind != "i8":
        assert (host(it["q_out"]) == case["rq"]).all(), what
        assert host(it["scale_out"])[0].view(np.int32) == case["rs"].view(np.int32), what


@pytest.mark.parametrize("K,N", [(2560, 2560), (6912, 640), (9008, 300), (2064, 64)],
                         ids=["bitnet-h", "bitnet-f", "beyond-prefetch", "k-not-256"])
@pytest.mark.parametrize("kind", KINDS)
def test_vector_and_general_prologue(cuda, kind, K, N):
    """K = 2560 (one prefetched chunk per thread), 6912 (two), 9008 (chunks
    beyond the prefetched two), 2064 (units padded past K)."""
    import ter_amd as T
    case = make_case(kind, K, N, seed=K + N + len(kind))
    for offset in (0, 1):  # 0: vector prologue, 1: general prologue
        for wg in (0, 2):  # 0: strip mode (a small list), 2: stream-K
            it = item_of(kind, case, K, N, offset)
            plan = T.Plan([it], wg_per_cu=wg)
            for rep in range(2):
                it["acc"].fill_(-7)
                it["y"].fill_(-7)
                plan.launch()
                check(kind, it, case, (offset, wg, rep))
            plan.close()


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("wg", [0, 1, 3])
def test_vector_prologue_multi_item(cuda, kind, wg):
    """Three GEMVs of one kind in one work list (the decode step's Q/K/V
    shape), so workgroups stage several activation vectors in turn."""
    import ter_amd as T
    shapes = [(2560, 2560), (2560, 640), (2048, 640)]
    cases = [make_case(kind, K, N, seed=100 * i + wg + len(kind)) for i, (K, N) in enumerate(shapes)]
    items = [item_of(kind, c, K, N, 0) for c, (K, N) in zip(cases, shapes)]
    plan = T.Plan(items, wg_per_cu=wg)
    for rep in range(2):
        plan.launch()
        for it, c in zip(items, cases):
            check(kind, it, c, (wg, rep, it["w"].K, it["w"].N))
    plan.close()


@pytest.mark.parametrize("kind", ["f32_rms", "f16_rms", "relu2"])
def test_rms_prologue_at_k_max(cuda, kind):
    """K = 32768 (TER_HIP_K_MAX): the fp32 staging of the RMS prologue no
    longer fits beside the int8 activations in LDS, so the sums of squares
    re-read the inputs (same order); the list takes the general prologue."""
    import ter_amd as T
    K, N = 32768, 48
    case = make_case(kind, K, N, seed=4242 + len(kind))
    for wg in (0, 1):
        it = item_of(kind, case, K, N, 0)
        plan = T.Plan([it], wg_per_cu=wg)
        plan.launch()
        check(kind, it, case, wg)
        plan.close()
