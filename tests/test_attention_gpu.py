"""GPU parity of the decode attention (RoPE + KV-cache write + attention in one
launch per layer; rope_k, kv_copy_k, attention_k of
cuda/ter_cuda_forward_bitnet.cu:185-214, 336-374 and the Llama forward's
NORM-pairing rope_k, cuda/ter_cuda_forward_packed.cu:64-76).

The cross-workgroup exchange runs in both of its forms (XCD-local and
device-wide).

Bar: the fp16 outputs bit-exact against the oracle's chunked order
(orc_attention_splitk), and within one fp16 ulp of the reference's sequential
order (orc_attention_ref; both orders' fp32 values are within 2e-6 of
float64 attention relative to sum_s p_s |v_sd|, tests/test_oracle.py); the
cache rows written at the new position bit-exact (RoPE'd k, v).
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


def bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


def run_decode(nh, nkv, hd, smax, theta, neox, positions, seed):
    import torch
    import ter_amd as T
    rng = np.random.default_rng(seed)
    A = T.Attention(nh, nkv, hd, smax, theta, neox)
    Kh = rng.standard_normal((smax, nkv, hd)).astype(np.float16)   # cache contents, incl. stale rows
    Vh = rng.standard_normal((smax, nkv, hd)).astype(np.float16)
    kc, vc = dev(Kh), dev(Vh)
    table = O.rope_table(theta, hd, smax)
    pos_dev = torch.zeros(1, dtype=torch.int32, device="cuda")
    for pos in positions:
        q = rng.standard_normal((nh, hd)).astype(np.float16)
        k = rng.standard_normal((nkv, hd)).astype(np.float16)
        v = rng.standard_normal((nkv, hd)).astype(np.float16)
        pos_dev.fill_(pos)
        out = host(A.decode(dev(q), dev(k), dev(v), kc, vc, pos_dev))
        qr = O.rope_f16(q, table[pos], neox)
        Kh[pos] = O.rope_f16(k, table[pos], neox)
        Vh[pos] = v
        want_s, _ = O.attention_splitk(qr, Kh[:pos + 1], Vh[:pos + 1])
        want_r, _ = O.attention_ref(qr, Kh[:pos + 1], Vh[:pos + 1])
        bad = np.flatnonzero(bits(out) != bits(want_s))
        assert bad.size == 0, (pos, bad[:8], out.ravel()[bad[:4]], want_s.ravel()[bad[:4]])
        ulps = np.abs(bits(out).astype(np.int64) - bits(want_r).astype(np.int64))
        assert ulps.max() <= 1, (pos, ulps.max())
        assert (bits(host(kc)[pos]) == bits(Kh[pos])).all(), pos   # the cache row of the new position
        assert (bits(host(vc)[pos]) == bits(Vh[pos])).all(), pos
    A.close()


@pytest.mark.parametrize("positions", [[0, 1, 2, 63, 64, 65], [127, 128, 200], [1500, 2047]],
                         ids=["first-tokens", "chunk-edges", "long"])
def test_bitnet_decode_attention(cuda, positions):
    """BitNet-2B: 20 query / 5 KV heads, head_dim 128, NEOX, theta 5e5,
    2048-position cache (the C5 context)."""
    run_decode(20, 5, 128, 2048, 500000.0, True, positions, seed=positions[0] + 1)


@pytest.mark.parametrize("form", ["xcd-local", "device-wide"])
def test_exchange_forms(cuda, monkeypatch, form):
    """Both forms of the cross-workgroup exchange (the context picks the
    XCD-local one when blocks land on XCD b % 8; TER_HIP_ATTN_DEVICE_WIDE=1
    keeps the device-wide one): BitNet shape, then Llama's 8 groups (one per
    XCD), over consecutive positions sharing one context."""
    if form == "device-wide":
        monkeypatch.setenv("TER_HIP_ATTN_DEVICE_WIDE", "1")
    else:
        monkeypatch.delenv("TER_HIP_ATTN_DEVICE_WIDE", raising=False)
    run_decode(20, 5, 128, 2048, 500000.0, True, [5, 6, 7, 2047], seed=31)
    run_decode(32, 8, 64, 1000, 500000.0, False, [0, 999], seed=32)


def test_llama_decode_attention(cuda):
    """Llama-3.2-1B: 32 query / 8 KV heads, head_dim 64, NORM pairing."""
    run_decode(32, 8, 64, 300, 500000.0, False, [0, 5, 64, 299], seed=7)


@pytest.mark.parametrize("nh,nkv,hd", [(4, 4, 128), (8, 4, 64), (16, 2, 128), (12, 2, 64)],
                         ids=["mha", "group-2", "group-8", "group-6"])
def test_head_groupings(cuda, nh, nkv, hd):
    """Groups of 1, 2, 8 (two workgroups per KV head) and 6 (a partial group)."""
    run_decode(nh, nkv, hd, 200, 10000.0, True, [0, 70, 199], seed=nh * 31 + nkv)


def test_rope_standalone(cuda):
    import torch
    import ter_amd as T
    A = T.Attention(20, 5, 128, 100, 500000.0, True)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((20, 128)).astype(np.float16)
    t = dev(x)
    A.rope(t, dev(np.array([77], np.int32)))
    want = O.rope_f16(x, O.rope_table(500000.0, 128, 100)[77], True)
    assert (bits(host(t)) == bits(want)).all()
    A.close()


def test_generated_attention_shapes(cuda):
    """Generated contexts (hypothesis, derandomized): 1 to 16 KV heads with
    1 to 12 query heads each, head_dim 64 or 128, either RoPE pairing,
    s_max from 1 to 4096 (up to 64 chunks), three positions each (the first,
    a random one and the last); outputs bit-exact against the chunked
    oracle and within one fp16 ulp of the sequential order, the new cache
    rows exact (run_decode's checks)."""
    from hypothesis import given, settings, strategies as st

    @settings(max_examples=16, deadline=None, derandomize=True)
    @given(nkv=st.integers(1, 16), g=st.integers(1, 12), hd=st.sampled_from([64, 128]), neox=st.booleans(),
           smax=st.integers(1, 4096), frac=st.floats(0.0, 1.0), seed=st.integers(0, 2 ** 20))
    def check(nkv, g, hd, neox, smax, frac, seed):
        positions = sorted({0, int(frac * (smax - 1)), smax - 1})
        run_decode(nkv * g, nkv, hd, smax, 10000.0, neox, positions, seed)

    check()
