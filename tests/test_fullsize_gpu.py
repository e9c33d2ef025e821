"""The benchmarked configurations checked at the size they are benchmarked.

C2: the Llama-3.2-1B sweep at M = 1 -- the exact 16 x 7 int8 work list that
    `bench.py` launches for its headline (bench.Sweep with the bench's own
    seeds, int8 activations over the full [-127, 127]), every output column
    of every one of the 112 GEMVs against the oracle.
C3: the BitNet-2B sweep at M = 1 -- the exact 30 x 7 fp32 work list that
    `bench.py --config bitnet` launches (bench.Sweep, bench's default launch
    shape), every output column of every GEMV against the oracle.
C4: the 210-GEMM plans at M = 8, 32 and 128 that `bench.py --config batched`
    launches (bench.Batched): the per-row quantized activations and every
    output of every GEMM against the oracle.
C5: the end-to-end greedy decode of the BitNet-2B-4T-shaped model that
    `bench.py --config decode` times (30 layers, H 2560, F 6912, 20/5 heads
    of 128, V 128256, KV cache pre-filled to 2048 positions): three tokens,
    eagerly and from a HIP-graph replay, the token, the fp32 hidden state and
    the new cache rows against the oracle's chain of the same steps.

The weights are regenerated on the host from the seeds the device used
(oracle.rand_trits_c: the splitmix64 stream of ter_hip_synth_v11), so the
check does not read the device's copy of them back.  The fast checkers
(orc_gemv_i8w / orc_gemm_i8w) are pinned to orc_mm_row in test_oracle.py.
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_llama_sweep_full_size(cuda):
    """C2: 112 GEMVs, int8 X, one launch (the headline's work list)."""
    import bench
    import ter_amd as T
    cfg = bench.LLAMA
    sw = bench.Sweep(cfg, 1, fp32_x=False)
    plan = T.Plan(sw.items(0))
    assert plan.bytes == bench.alg_bytes(cfg, False)
    first = None
    for rep in range(2):  # a second launch: fix-up slots left clean by the first
        plan.launch()
        ys = {(l, nm): host(sw.y[l][nm]).copy() for l in range(cfg["layers"]) for nm, _, _ in cfg["shapes"]}
        if first is None:
            first = ys
        else:
            assert all((ys[k].view(np.int32) == first[k].view(np.int32)).all() for k in ys), "relaunch differs"
    xs = {}
    for l in range(cfg["layers"]):
        for nm, K, N in cfg["shapes"]:
            W, _, seed = sw.copies[0][l][nm]
            key = (l, bench.X_OF[nm])
            if key not in xs:
                xs[key] = host(sw.x[l][bench.X_OF[nm]])
            x = xs[key]
            Wt = O.rand_trits_c(seed, K, N, cfg["p_zero"])
            _, want = O.gemv_i8w(x, 0.0312, Wt, W.scale)
            got = first[(l, nm)]
            assert (got.view(np.int32) == want.view(np.int32)).all(), (l, nm)
    allx = np.concatenate(list(xs.values()))
    assert allx.min() == -127 and allx.max() == 127  # the config's full activation range


def test_bitnet_sweep_full_size(cuda):
    """C3: 210 GEMVs, fp32 X quantized in the kernel prologue, one launch."""
    import bench
    import ter_amd as T
    cfg = bench.BITNET
    sw = bench.Sweep(cfg, 1, fp32_x=True)
    plan = T.Plan(sw.items(0))
    assert plan.bytes == bench.alg_bytes(cfg, True)
    first = None
    for rep in range(2):  # a second launch: fix-up slots left clean by the first
        plan.launch()
        ys = {(l, nm): host(sw.y[l][nm]).copy() for l in range(cfg["layers"]) for nm, _, _ in cfg["shapes"]}
        if first is None:
            first = ys
        else:
            assert all((ys[k].view(np.int32) == first[k].view(np.int32)).all() for k in ys), "relaunch differs"
    quant = {}
    for l in range(cfg["layers"]):
        for nm, K, N in cfg["shapes"]:
            W, _, seed = sw.copies[0][l][nm]
            key = (l, bench.X_OF[nm])
            if key not in quant:
                quant[key] = O.quant_int8(host(sw.x[l][bench.X_OF[nm]]))
            q, s = quant[key]
            Wt = O.rand_trits_c(seed, K, N, cfg["p_zero"])
            _, want = O.gemv_i8w(q, s, Wt, W.scale)
            got = first[(l, nm)]
            assert (got.view(np.int32) == want.view(np.int32)).all(), (l, nm)


@pytest.mark.parametrize("M", [8, 32, 128])
def test_bitnet_batched_full_size(cuda, M):
    """C4: 30 layers x 7 GEMMs at M rows in one plan launch (the LDS-ring
    kernel at every M: the 210-GEMM list holds more than 4 ring blocks per
    CU even at M = 8), after the per-row quantizers."""
    import torch
    import bench
    wl = bench.Batched(M)
    cfg = wl.cfg
    wl.step()
    torch.cuda.synchronize()
    qs = {}
    for k in wl.X:
        rq, rs = O.quant_int8_rows(host(wl.X[k]))
        assert (host(wl.q[k]) == rq).all(), k
        assert (host(wl.s[k]).view(np.int32) == rs.view(np.int32)).all(), k
        qs[k] = (rq, rs)
    first = {(l, nm): host(wl.Y[l][nm]).copy() for l in range(cfg["layers"]) for nm, _, _ in cfg["shapes"]}
    wl.step()
    for l in range(cfg["layers"]):
        for nm, K, N in cfg["shapes"]:
            W, seed = wl.layers[l][nm]
            rq, rs = qs[bench.X_OF[nm]]
            Wt = O.rand_trits_c(seed, K, N, cfg["p_zero"])
            _, want = O.gemm_i8w(rq, rs, Wt, W.scale)
            got = first[(l, nm)]
            assert (got.view(np.int32) == want.view(np.int32)).all(), (M, l, nm)
            assert (host(wl.Y[l][nm]).view(np.int32) == got.view(np.int32)).all(), ("relaunch", M, l, nm)
    del wl
    torch.cuda.empty_cache()


@pytest.mark.parametrize("graph", [False, True], ids=["eager", "hip-graph"])
def test_bitnet_decode_full_size(cuda, graph):
    """C5 at the benchmarked shape: three greedy tokens from position 2048."""
    import torch
    from ter_amd import bitnet as B
    from tests.decode_ref import host_model_i8, oracle_step
    c = B.Shape()
    seed = 5  # bench.py's random_model seed
    m = B.random_model(c, seed=seed)
    start, n_tok = 2048, 3
    s_max = start + 64
    dec = B.Decoder(m, s_max)
    rng = np.random.default_rng(6)
    K = rng.standard_normal((c.Nl, s_max, c.Nkv, c.Hd), dtype=np.float32).astype(np.float16)
    V = rng.standard_normal((c.Nl, s_max, c.Nkv, c.Hd), dtype=np.float32).astype(np.float16)
    dec.K.copy_(torch.from_numpy(K))
    dec.V.copy_(torch.from_numpy(V))
    dec.pos.fill_(start)
    tok = 1
    dec.token.fill_(tok)
    hm = host_model_i8(m, seed)
    table = O.rope_table(c.rope_theta, c.Hd, s_max)
    g = dec.capture() if graph else None
    for step in range(n_tok):
        pos = start + step
        print(f"C5 full-size decode ({'graph' if graph else 'eager'}): token {step} at position {pos}", flush=True)
        want_tok, want_hidden = oracle_step(hm, tok, pos, K, V, table)
        if graph:
            g.replay()
        else:
            dec.step()
        got_tok = int(host(dec.token)[0])
        assert (host(dec.hidden).view(np.uint32) == want_hidden.view(np.uint32)).all(), step
        assert got_tok == want_tok, (step, got_tok, want_tok)
        assert int(host(dec.pos)[0]) == pos + 1
        assert (host(dec.K[:, pos]).view(np.uint16) == K[:, pos].view(np.uint16)).all(), step
        assert (host(dec.V[:, pos]).view(np.uint16) == V[:, pos].view(np.uint16)).all(), step
        tok = want_tok
    # rows other than the written ones are untouched
    assert (host(dec.K).view(np.uint16) == K.view(np.uint16)).all()
    assert (host(dec.V).view(np.uint16) == V.view(np.uint16)).all()
    dec.close()
