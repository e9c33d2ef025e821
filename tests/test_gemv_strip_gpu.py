"""GPU parity of the GEMV kernel's strip mode: small work lists (fewer than
32 tiles per workgroup at two workgroups per CU, at most four strips per CU)
give each workgroup whole column strips, split each strip's 256-row units
over its four waves and add the waves' partial column sums in LDS; stream-K
fix-up slots are not used.

Bar: int32 accumulators and fp32 outputs bit-exact against the oracle
(mm_row's integer dot products, src/tx/forward.cpp:342-345), for strips
with fewer units than waves, partial last strips, many strips per
workgroup and workgroup ranges that cross GEMV boundaries.
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def run_list(specs, seed, launches=2, fp32=False):
    """specs: (K, N) per GEMV, int8 inputs (fp32 with the absmax prologue if
    fp32); checks acc and y after each launch."""
    import torch
    import ter_amd as T
    items, refs = [], []
    for i, (K, N) in enumerate(specs):
        v11 = O.v11_pack(O.rand_trits(seed + 17 * i, K, N, 0.4))
        ws = 0.01 + 0.003 * i
        W = T.PackedTrits.from_v11(v11, K, N, ws)
        out = dict(y=torch.empty(N, dtype=torch.float32, device="cuda"),
                   acc=torch.empty(N, dtype=torch.int32, device="cuda"))
        if fp32:
            x = (np.random.default_rng(seed + i).standard_normal(K) * 2).astype(np.float32)
            items.append(dict(w=W, x=dev(x), **out))
            rq, rs = O.quant_int8(x)
            refs.append(O.gemv_v11(rq, rs, v11, ws, K, N))
        else:
            x = O.rand_int8(seed + 31 * i, K)
            items.append(dict(w=W, x=dev(x), x_scale=0.02, **out))
            refs.append(O.gemv_v11(x, np.float32(0.02), v11, ws, K, N))
    plan = T.Plan(items)
    for rep in range(launches):
        for it in items:
            it["acc"].fill_(-7)
        plan.launch()
        for it, (ra, ry) in zip(items, refs):
            assert (host(it["acc"]) == ra).all(), (rep, it["w"].K, it["w"].N)
            assert (host(it["y"]).view(np.int32) == np.asarray(ry, np.float32).view(np.int32)).all()
    plan.close()


@pytest.mark.parametrize("K", [256, 512, 768, 1024, 2560, 6912], ids=lambda k: f"K{k}")
def test_units_per_wave(cuda, K):
    """Ku = 1, 2, 3 (waves without units write zero partials), 4, 10, 27."""
    run_list([(K, 300)], seed=K)


@pytest.mark.parametrize("K", [256, 2560])
def test_two_strips_per_workgroup(cuda, K):
    """512 strips with a prologue (one workgroup per CU): two strips per
    workgroup, one range crossing the boundary between the two GEMVs at an
    odd strip, ragged N."""
    run_list([(K, 16 * 255 - 4), (K, 16 * 257)], seed=5 + K, fp32=True)


@pytest.mark.parametrize("K", [512, 2560])
def test_four_strips_per_workgroup(cuda, K):
    """1000 strips with a prologue (one workgroup per CU): three or four
    strips per workgroup, ranges crossing the boundaries between three GEMVs
    at odd strips, ragged N."""
    run_list([(K, 16 * 333 - 4), (K, 16 * 334), (K, 16 * 333 + 4)], seed=7 + K, fp32=True)


@pytest.mark.parametrize("fp32", [False, True], ids=["int8", "fp32"])
def test_descriptor_table_lists(cuda, fp32):
    """Strip-mode lists of four, five and six GEMVs (descriptor table lookups
    across several GEMV boundaries), ragged N."""
    run_list([(2560, 640 + 16 * i - (4 if i % 2 else 0)) for i in range(4)], seed=21, fp32=fp32)
    run_list([(2560, 640 + 16 * i - (4 if i % 2 else 0)) for i in range(5)], seed=22, fp32=fp32)
    run_list([(1024, 300 + 32 * i) for i in range(6)], seed=23, fp32=fp32)


def test_decode_shaped_lists(cuda):
    """The decode step's lists: Q/K/V, O, gate/up (864 strips: strip mode),
    down (BitNet-2B shapes); and a list just past strip mode (1056 strips:
    stream-K)."""
    run_list([(2560, 2560), (2560, 640), (2560, 640)], seed=11)
    run_list([(2560, 2560)], seed=12)
    run_list([(2560, 6912), (2560, 6912)], seed=13)
    run_list([(2560, 6912), (2560, 6912)], seed=15, fp32=True)
    run_list([(6912, 2560)], seed=14)
    run_list([(2560, 8448), (2560, 8448)], seed=16)


@pytest.mark.parametrize("kind", ["f32-rms", "f16-rms", "relu2", "f16", "silu", "smul"])
@pytest.mark.parametrize("order", ["grouped", "reordered"])
def test_shared_activation_plans(cuda, kind, order):
    """Strided strip-mode lists whose GEMVs read one activation vector: with
    the weights grouped in one allocation in item order (fabric.group_contiguous)
    the plan takes the activation and weight streams from the launch's
    arguments (TER_HIP_PLAN_SHARED), workgroup ranges crossing GEMV
    boundaries included; listed in another order it runs the per-segment
    path.  Outputs, fp16 copies and accumulators bit-exact either way, over
    two launches."""
    import torch
    import ter_amd as T
    from ter_amd import _lib as L
    K = {"f32-rms": 2560, "f16-rms": 2048, "relu2": 6912, "f16": 2048, "silu": 8192, "smul": 8192}[kind]
    Ns = [4000, 48, 2000] if kind in ("f32-rms", "f16-rms") else [1024, 528]
    rng = np.random.default_rng(K + len(Ns))
    gm = rng.uniform(0.5, 1.5, K).astype(np.float16)
    if kind == "f32-rms":
        x = (rng.standard_normal(K) * 3).astype(np.float32)
    else:
        x = (rng.standard_normal(K) * 1.5).astype(np.float16)
    up = (rng.standard_normal(K) * 1.5).astype(np.float16)
    if kind in ("f32-rms", "f16-rms"):
        rq, rs, _ = O.rmsnorm_quant(x, gm, 1e-5)
    elif kind == "relu2":
        rq, rs, _ = O.relu2_rmsnorm_quant(x, up, gm, 1e-5)
    elif kind == "f16":
        rq, rs = O.quant_int8(x.astype(np.float32))
    elif kind == "silu":
        rq, rs, _ = O.silu_mul_quant(x, up)
    else:
        x = O.silu_f16(x)
        rq, rs, _ = O.smul_quant(x, up)
    v11s = [O.v11_pack(O.rand_trits(K * 3 + 7 * i, K, N, 0.4)) for i, N in enumerate(Ns)]
    Ws = [T.PackedTrits.from_v11(v, K, N, 0.01 * (i + 1)) for i, (v, N) in enumerate(zip(v11s, Ns))]
    Ws = T.group_contiguous(Ws)
    idx = list(range(len(Ns))) if order == "grouped" else list(range(len(Ns)))[::-1]
    dx, dg, du = dev(x), dev(gm), dev(up)
    items = []
    for i in idx:
        it = dict(w=Ws[i], x=dx, y=torch.empty(Ns[i], dtype=torch.float32, device="cuda"),
                  acc=torch.empty(Ns[i], dtype=torch.int32, device="cuda"),
                  y16=torch.empty(Ns[i], dtype=torch.float16, device="cuda"))
        if kind in ("f32-rms", "f16-rms", "relu2"):
            it.update(gamma=dg, eps=1e-5)
        if kind in ("relu2", "silu", "smul"):
            it["up"] = du
        items.append(it)
    plan = T.Plan(items)
    assert plan.mode & L.PLAN_STRIPS and plan.mode & L.PLAN_STRIDED, plan.mode
    assert bool(plan.mode & L.PLAN_SHARED) == (order == "grouped" or len(Ns) == 1), plan.mode
    for rep in range(2):
        for it in items:
            it["acc"].fill_(-7)
        plan.launch()
        for i, it in zip(idx, items):
            ra, ry = O.gemv_v11(rq, rs, v11s[i], 0.01 * (i + 1), K, Ns[i])
            assert (host(it["acc"]) == ra).all(), (rep, i)
            assert (host(it["y"]).view(np.int32) == ry.view(np.int32)).all(), (rep, i)
            assert (host(it["y16"]).view(np.uint16) == O.float_to_half_bits(ry)).all(), (rep, i)
    plan.close()


def test_prologue_plans_generated(cuda):
    """Generated decode-step plans (hypothesis, derandomized): one of the six
    prologue kinds, K a multiple of 16 up to the strided prologue's limit or
    any K (the general prologue), one to four GEMVs of N a multiple of 4
    reading one activation vector, weights grouped in one allocation or
    not; whichever launch form the plan picks, every output, fp16 copy and
    accumulator bit for bit against the oracle."""
    import torch
    import ter_amd as T
    from hypothesis import given, settings, strategies as st

    @settings(max_examples=36, deadline=None, derandomize=True)
    @given(kind=st.sampled_from(["f32-rms", "f16-rms", "relu2", "f16", "silu", "smul"]),
           ku16=st.integers(1, 256), ragged=st.booleans(),
           Ns=st.lists(st.integers(1, 600).map(lambda v: 4 * v), min_size=1, max_size=4),
           grouped=st.booleans(), seed=st.integers(0, 2 ** 20))
    def check(kind, ku16, ragged, Ns, grouped, seed):
        limit = 8192 if kind in ("relu2", "silu", "smul") else 4096
        K = min(16 * ku16, limit)
        if ragged:
            K = max(1, K - 5)
        rng = np.random.default_rng(seed)
        gm = rng.uniform(0.5, 1.5, K).astype(np.float16)
        x = (rng.standard_normal(K) * 3).astype(np.float32 if kind == "f32-rms" else np.float16)
        up = (rng.standard_normal(K) * 1.5).astype(np.float16)
        if kind in ("f32-rms", "f16-rms"):
            rq, rs, _ = O.rmsnorm_quant(x, gm, 1e-5)
        elif kind == "relu2":
            rq, rs, _ = O.relu2_rmsnorm_quant(x, up, gm, 1e-5)
        elif kind == "f16":
            rq, rs = O.quant_int8(x.astype(np.float32))
        elif kind == "silu":
            rq, rs, _ = O.silu_mul_quant(x, up)
        else:
            x = O.silu_f16(x)
            rq, rs, _ = O.smul_quant(x, up)
        v11s = [O.v11_pack(O.rand_trits(seed + 7 * i, K, N, 0.4)) for i, N in enumerate(Ns)]
        Ws = [T.PackedTrits.from_v11(v, K, N, 0.01 * (i + 1)) for i, (v, N) in enumerate(zip(v11s, Ns))]
        if grouped:
            Ws = T.group_contiguous(Ws)
        dx, dg, du = dev(x), dev(gm), dev(up)
        items = []
        for i, N in enumerate(Ns):
            it = dict(w=Ws[i], x=dx, y=torch.empty(N, dtype=torch.float32, device="cuda"),
                      acc=torch.empty(N, dtype=torch.int32, device="cuda"),
                      y16=torch.empty(N, dtype=torch.float16, device="cuda"))
            if kind in ("f32-rms", "f16-rms", "relu2"):
                it.update(gamma=dg, eps=1e-5)
            if kind in ("relu2", "silu", "smul"):
                it["up"] = du
            items.append(it)
        plan = T.Plan(items)
        plan.launch()
        for i, it in enumerate(items):
            ra, ry = O.gemv_v11(rq, rs, v11s[i], 0.01 * (i + 1), K, Ns[i])
            assert (host(it["acc"]) == ra).all(), (kind, K, Ns, i)
            assert (host(it["y"]).view(np.int32) == ry.view(np.int32)).all(), (kind, K, Ns, i)
            assert (host(it["y16"]).view(np.uint16) == O.float_to_half_bits(ry)).all(), (kind, K, Ns, i)
        plan.close()

    check()
