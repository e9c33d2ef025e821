"""GPU parity of the decode step's tail (cuda/ter_cuda_forward_bitnet.cu:890-911):
the RMSNorm to fp16 (rmsnorm_f32_in_k, :37-47), the fp16 lm_head GEMV over the
tied token embedding (mm_fp16_lm_head_k, :388-429), the two-pass argmax
(argmax_local_k / argmax_final_k, :454-495), and the fused one-launch tail.

Bar: fp16 normalized inputs and fp16 logits bit-exact against the oracle
(which follows the reference's fp32 summation order), and the argmax index
identical, ties included.
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


def f16_bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


def embedding(seed, V, H, scale=0.05):
    """fp16 [V][H] drawn on the device (large tables), copied back for the oracle."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    E = (torch.randn(V, H, generator=g, device="cuda", dtype=torch.float32) * scale).to(torch.float16)
    return E, host(E)


@pytest.mark.parametrize("H", [2560, 2048, 37, 2561])
def test_rmsnorm_f16_rows(cuda, H):
    import ter_amd as T
    rng = np.random.default_rng(H)
    X = (rng.standard_normal((3, H)) * 4).astype(np.float32)
    g = rng.uniform(0.5, 1.5, H).astype(np.float16)
    y = host(T.rmsnorm_f16(dev(X), dev(g), 1e-5))
    for r in range(3):
        want, _ = O.rmsnorm_f16(X[r], g, 1e-5)
        assert (f16_bits(y[r]) == f16_bits(want)).all(), r


def test_rmsnorm_f16_double_rounding(cuda):
    """y = half(fp32((x * rms_inv) * gamma)): the product is rounded to fp32
    first, as the reference's __float2half of a float expression; rounding
    the exact product straight to fp16 differs where the fp32 value lands on
    an fp16 tie.  64 rows of 2560 hold such elements (counted here)."""
    import ter_amd as T
    rng = np.random.default_rng(77)
    H = 2560
    X = (rng.standard_normal((64, H)) * 3).astype(np.float32)
    g = rng.uniform(0.5, 1.5, H).astype(np.float16)
    y = host(T.rmsnorm_f16(dev(X), dev(g), 1e-5))
    sensitive = 0
    for r in range(64):
        want, rinv = O.rmsnorm_f16(X[r], g, 1e-5)
        assert (f16_bits(y[r]) == f16_bits(want)).all(), r
        a = (X[r] * rinv).astype(np.float32)
        exact = a.astype(np.float64) * g.astype(np.float64)
        sensitive += int((exact.astype(np.float16) != exact.astype(np.float32).astype(np.float16)).sum())
    assert sensitive > 0


@pytest.mark.parametrize("H,V", [(2560, 1000), (2560, 4097), (2048, 300), (64, 33), (1000, 300), (2056, 129),
                                 (100, 50), (2561, 77), (8200, 50), (2, 5)],
                         ids=["bitnet-h", "odd-v", "llama-h", "one-group", "masked-groups", "partial-group",
                              "h-not-8-generic", "odd-h-generic", "wide-h-generic", "tiny"])
def test_lm_head_logits(cuda, H, V):
    import torch
    import ter_amd as T
    E, Eh = embedding(H * 7 + V, V, H)
    x = (np.random.default_rng(H + V).standard_normal(H) * 2).astype(np.float16)
    lg = T.lm_head_f16(dev(x), E)
    want, _ = O.lm_head_f16(x, Eh)
    got = host(lg)
    bad = np.flatnonzero(f16_bits(got) != f16_bits(want))
    assert bad.size == 0, (bad[:8], got[bad[:4]], want[bad[:4]])


def test_lm_head_generated_shapes(cuda):
    """Generated tails (hypothesis, derandomized): H from 2 to 6000 (the
    octet path where H is a multiple of 8 and fits it, the generic one
    otherwise), V from 1 to 3000, fp32 or fp16 hidden stream; the fused
    RMSNorm + lm_head + argmax against the oracle (normalized input, every
    logit, the token), the argmax state left clean."""
    import torch
    import ter_amd as T
    from hypothesis import given, settings, strategies as st

    @settings(max_examples=24, deadline=None, derandomize=True)
    @given(H=st.integers(1, 3000).map(lambda v: 2 * v), V=st.integers(1, 3000), half=st.booleans(),
           seed=st.integers(0, 2 ** 20))
    def check(H, V, half, seed):
        E, Eh = embedding(seed, V, H)
        rng = np.random.default_rng(seed)
        gamma = rng.uniform(0.5, 1.5, H).astype(np.float16)
        hidden = (rng.standard_normal(H) * 3).astype(np.float16 if half else np.float32)
        state = T.ArgmaxState()
        x_out = torch.empty(H, dtype=torch.float16, device="cuda")
        lg_out = torch.empty(V, dtype=torch.float16, device="cuda")
        tok = T.lm_head_argmax(dev(hidden), dev(gamma), E, 1e-5, state=state, x_norm_out=x_out, logits_out=lg_out)
        xn, _ = O.rmsnorm_f16(hidden, gamma, 1e-5)
        assert (f16_bits(host(x_out)) == f16_bits(xn)).all(), (H, V, half)
        want_lg, _ = O.lm_head_f16(xn, Eh)
        assert (f16_bits(host(lg_out)) == f16_bits(want_lg)).all(), (H, V, half)
        assert int(host(tok)[0]) == O.argmax_f16(want_lg), (H, V, half)
        assert (host(state.t) == 0).all()

    check()


def test_lm_head_bitnet_full_size_and_fused_tail(cuda):
    """V = 128256, H = 2560 (BitNet-2B's tied lm_head): every logit, the
    normalized input and the token of the fused one-launch tail, over three
    tokens sharing one argmax state."""
    import torch
    import ter_amd as T
    V, H = 128256, 2560
    E, Eh = embedding(1234, V, H, 0.03)
    rng = np.random.default_rng(5)
    gamma = rng.uniform(0.5, 1.5, H).astype(np.float16)
    state = T.ArgmaxState()
    x_out = torch.empty(H, dtype=torch.float16, device="cuda")
    lg_out = torch.empty(V, dtype=torch.float16, device="cuda")
    for step in range(3):
        hidden = (rng.standard_normal(H) * (1 + 3 * step)).astype(np.float32)
        tok = T.lm_head_argmax(dev(hidden), dev(gamma), E, 1e-5, state=state, x_norm_out=x_out, logits_out=lg_out)
        xn, _ = O.rmsnorm_f16(hidden, gamma, 1e-5)
        assert (f16_bits(host(x_out)) == f16_bits(xn)).all(), step
        want_lg, _ = O.lm_head_f16(xn, Eh)
        got_lg = host(lg_out)
        assert (f16_bits(got_lg) == f16_bits(want_lg)).all(), step
        assert int(host(tok)[0]) == O.argmax_f16(want_lg), step
    assert (host(state.t) == 0).all()  # the last workgroup left the state clean


def test_fused_tail_ties_follow_the_reference(cuda):
    """Copies of the winning embedding row make equal logits; the fused
    argmax returns the index the reference's two trees pick."""
    import torch
    import ter_amd as T
    V, H = 20000, 2560
    E, Eh = embedding(99, V, H)
    rng = np.random.default_rng(6)
    gamma = rng.uniform(0.5, 1.5, H).astype(np.float16)
    hidden = rng.standard_normal(H).astype(np.float32)
    xn, _ = O.rmsnorm_f16(hidden, gamma, 1e-5)
    m = int(np.argmax(O.lm_head_f16(xn, Eh)[0].astype(np.float32)))
    state = T.ArgmaxState()
    for copies in ([3, 19999], [m - 1 if m else 1, 157, 12345], list(range(0, V, 997))):
        Et = Eh.copy()
        for c in copies:
            Et[c] = Eh[m]
        want_lg, _ = O.lm_head_f16(xn, Et)
        want = O.argmax_f16(want_lg)
        tok = T.lm_head_argmax(dev(hidden), dev(gamma), dev(Et), 1e-5, state=state)
        assert int(host(tok)[0]) == want, (copies, want)


def test_argmax_f16_matches_reference_rule(cuda):
    import ter_amd as T
    rng = np.random.default_rng(7)
    state = T.ArgmaxState()
    cases = []
    for N in (128256, 1000, 300, 100, 1, 3000):
        lg = rng.standard_normal(N).astype(np.float16)
        cases.append(lg)
        t = lg.copy()
        cand = rng.choice(N, size=min(N, 4), replace=False)
        t[cand] = np.float16(8.0)
        cases.append(t)
    z = np.full(1000, -np.inf, np.float16)
    cases.append(z.copy())          # nothing eligible: -1
    z[5], z[600] = np.float16(np.nan), np.float16(-65504.0)
    cases.append(z.copy())          # NaN never wins
    z[:] = np.float16(-1.0)
    z[[10, 300, 999]] = np.float16(0.0)
    z[300] = np.float16(-0.0)       # -0 ties with +0
    cases.append(z)
    # a last group of 8 that ends past N (read one by one): the maximum in it,
    # or values below every other (so a zero read there would win), or N = 1
    t = rng.standard_normal(1003).astype(np.float16)
    t[1001] = np.float16(8.5)
    cases.append(t)
    t = np.full(1003, -1.0, np.float16)
    t[1000:] = np.float16(-2.0)
    cases.append(t)
    cases.append(np.full(1, -np.inf, np.float16))
    cases.append(np.full(7, -3.0, np.float16))
    for i, lg in enumerate(cases):
        got = int(host(T.argmax_f16(dev(lg), state=state))[0])
        assert got == O.argmax_f16(lg), (i, lg.size)
        # logits 2 bytes past a 16-byte boundary: one logit per thread and round
        off = dev(np.concatenate([np.zeros(1, np.float16), lg]))[1:]
        got = int(host(T.argmax_f16(off, state=state))[0])
        assert got == O.argmax_f16(lg), ("unaligned", i, lg.size)
    assert (host(state.t) == 0).all()


@pytest.mark.parametrize("V,H", [(1000, 2560), (50, 77), (9, 8)])
def test_embedding_rows(cuda, V, H):
    """token_embed_lookup_k in both forms (fp32 hidden stream, fp16 hidden
    stream): the token's row exactly, for the first and last tokens, into an
    aligned and a misaligned output (one element past an aligned start); a
    token outside [0, V) writes nothing."""
    import torch
    import ter_amd as T
    rng = np.random.default_rng(V + H)
    Eh = (rng.standard_normal((V, H)) * 0.1).astype(np.float16)
    E = dev(Eh)
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    for t in (0, V - 1, V // 2):
        tok.fill_(t)
        for off in (0, 1):
            h32 = torch.full((H + off,), -7.0, dtype=torch.float32, device="cuda")
            T.embed_f16(E, tok, h32[off:])
            assert (host(h32[off:]) == Eh[t].astype(np.float32)).all(), (t, off)
            h16 = torch.full((H + off,), -7.0, dtype=torch.float16, device="cuda")
            T.embed_h16(E, tok, h16[off:])
            assert (host(h16[off:]).view(np.uint16) == Eh[t].view(np.uint16)).all(), (t, off)
    for t in (-1, V):
        tok.fill_(t)
        h32 = torch.full((H,), -7.0, dtype=torch.float32, device="cuda")
        T.embed_f16(E, tok, h32)
        h16 = torch.full((H,), -7.0, dtype=torch.float16, device="cuda")
        T.embed_h16(E, tok, h16)
        assert (host(h32) == -7.0).all() and (host(h16) == -7.0).all(), t
