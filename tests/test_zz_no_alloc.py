"""ter_hip_gemm_out_static: the GEMM entry point that allocates nothing.

It quantizes fp32 / fp16 / RMS activation rows into the library's static
device workspace instead of caller workspaces.  Checked through the C-ABI
against ter_hip_gemm_out (caller workspaces) and the oracle, on two calls
in a row, the second smaller, so stale workspace contents would show.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O
from ter_amd import _lib as L


def _act(kind, data, gamma=None, eps=1e-5, q_out=None, scale_out=None):
    a = L.Act()
    a.data = data
    a.kind = kind
    a.scale = 1.0
    a.gamma = gamma
    a.eps = eps
    a.q_out = q_out
    a.scale_out = scale_out
    return a


def test_static_gemm_validation_cpu():
    """Refusals happen on the host, before any device work."""
    lib = L.lib()
    w = L.WPK()
    fake = 1 << 20
    K, N = 32768, 16
    assert lib.ter_hip_wpk_init(C.byref(w), fake, lib.ter_hip_wpk_bytes(K, N), K, N, 1.0) == L.OK
    o = L.Out()
    o.y = fake
    a = _act(L.X_F32, fake)
    M = L.STATIC_Q_MAX // K + 1  # one row past the workspace
    assert lib.ter_hip_gemm_out_static(C.byref(w), C.byref(a), M, C.byref(o), None) == L.ERR_SHAPE
    assert b"static workspace" in lib.ter_hip_last_error()
    a2 = _act(L.X_F32, fake, q_out=fake)
    assert lib.ter_hip_gemm_out_static(C.byref(w), C.byref(a2), 4, C.byref(o), None) == L.ERR_SHAPE
    assert lib.ter_hip_gemm_out_static(C.byref(w), None, 4, C.byref(o), None) == L.ERR_NULL
    assert lib.ter_hip_gemm_out_static(C.byref(w), C.byref(a), 0, C.byref(o), None) == L.ERR_SHAPE


def _run(lib, fn, W, a, M, N):
    import torch
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    o = L.Out()
    o.y, o.acc = y.data_ptr(), acc.data_ptr()
    st = torch.cuda.current_stream().cuda_stream
    L.check(getattr(lib, fn)(C.byref(W.wpk), C.byref(a), M, C.byref(o), st), fn)
    torch.cuda.synchronize()
    return y.cpu().numpy(), acc.cpu().numpy()


def _capture_static(lib, W, a, M, N, y, acc):
    """A HIP graph holding one ter_hip_gemm_out_static call (torch's global
    capture mode, under which an allocation on any thread is an error)."""
    import torch
    o = L.Out()
    o.y, o.acc = y.data_ptr(), acc.data_ptr()
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(g, capture_error_mode="global"):
        st = torch.cuda.current_stream().cuda_stream
        rc = lib.ter_hip_gemm_out_static(C.byref(W.wpk), C.byref(a), M, C.byref(o), st)
    L.check(rc, "ter_hip_gemm_out_static under capture")
    return g


@pytest.mark.gpu
def test_static_gemm_under_graph_capture(cuda):
    """Captured into a HIP graph: first before any eager call of the entry
    point in this process (its first call on the device looks up the static
    workspace's address inside the capture; this test runs before the other
    GPU test of this file, and no other test file reaches that lookup), then
    again after eager calls.  Every replay, with eager calls of other inputs
    through the same workspace and synchronizations between the replays, is
    bit-identical to ter_hip_gemm_out with caller workspaces."""
    import torch
    import ter_amd as T
    lib = L.lib()
    M, K, N = 32, 2560, 640
    W = T.PackedTrits.from_v11(O.v11_pack(O.rand_trits(91, K, N, 0.4)), K, N, 0.023)
    X1 = torch.from_numpy(O.rand_normal_f32(92, M * K).reshape(M, K)).cuda()
    X2 = torch.from_numpy(O.rand_normal_f32(93, M * K).reshape(M, K) * 3).cuda()
    q = torch.empty((M, K), dtype=torch.int8, device="cuda")
    s = torch.empty(M, dtype=torch.float32, device="cuda")
    want1 = _run(lib, "ter_hip_gemm_out", W, _act(L.X_F32, X1.data_ptr(), q_out=q.data_ptr(),
                                                  scale_out=s.data_ptr()), M, N)
    want2 = _run(lib, "ter_hip_gemm_out", W, _act(L.X_F32, X2.data_ptr(), q_out=q.data_ptr(),
                                                  scale_out=s.data_ptr()), M, N)
    for phase in ("first call under capture", "after eager calls"):
        print(f"static GEMM capture: {phase}", flush=True)
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
        g = _capture_static(lib, W, _act(L.X_F32, X1.data_ptr()), M, N, y, acc)
        for rep in range(3):
            y.fill_(float("nan"))
            acc.fill_(-1)
            g.replay()
            torch.cuda.synchronize()
            assert (acc.cpu().numpy() == want1[1]).all(), (phase, rep)
            assert (y.cpu().numpy().view(np.int32) == want1[0].view(np.int32)).all(), (phase, rep)
            # eager work through the same static workspace between replays
            sy, sa = _run(lib, "ter_hip_gemm_out_static", W, _act(L.X_F32, X2.data_ptr()), M, N)
            assert (sa == want2[1]).all() and (sy.view(np.int32) == want2[0].view(np.int32)).all(), (phase, rep)
        del g


@pytest.mark.gpu
def test_static_gemm_matches_workspace_entry(cuda):
    import torch
    import ter_amd as T
    lib = L.lib()
    cases = [
        # (M, K, N, kind): the first call fills more of the workspace than the second
        (128, 6912, 640, L.X_F32),
        (8, 2048, 512, L.X_F32_RMS),
    ]
    for M, K, N, kind in cases:
        print(f"static GEMM case M={M} K={K} N={N} kind={kind}", flush=True)
        w = O.rand_trits(M + K, K, N, 0.4)
        v11 = O.v11_pack(w)
        W = T.PackedTrits.from_v11(v11, K, N, 0.031)
        Xf = O.rand_normal_f32(M * 3 + K, M * K).reshape(M, K)
        Xf[M // 2] *= 40.0
        xd = torch.from_numpy(Xf).cuda()
        gamma = None
        if kind == L.X_F32_RMS:
            g = (0.5 + O.rand_normal_f32(K + 9, K) * 0.1).astype(np.float16)
            gamma = torch.from_numpy(g).cuda()
        q = torch.empty((M, K), dtype=torch.int8, device="cuda")
        s = torch.empty(M, dtype=torch.float32, device="cuda")
        a_ws = _act(kind, xd.data_ptr(), gamma.data_ptr() if gamma is not None else None,
                    q_out=q.data_ptr(), scale_out=s.data_ptr())
        a_st = _act(kind, xd.data_ptr(), gamma.data_ptr() if gamma is not None else None)
        ry, ra = _run(lib, "ter_hip_gemm_out", W, a_ws, M, N)
        sy, sa = _run(lib, "ter_hip_gemm_out_static", W, a_st, M, N)
        assert (sa == ra).all()
        assert (sy.view(np.int32) == ry.view(np.int32)).all()
        # and the oracle
        if kind == L.X_F32:
            oq, os_ = O.quant_int8_rows(Xf)
        else:
            rows = [O.rmsnorm_quant(Xf[m], g, 1e-5) for m in range(M)]
            oq = np.stack([r[0] for r in rows])
            os_ = np.array([r[1] for r in rows], dtype=np.float32)
        oa, oy = O.gemm_v11(oq, os_, v11, 0.031, K, N)
        assert (sa == oa).all()
        assert (sy.view(np.int32) == oy.view(np.int32)).all()
