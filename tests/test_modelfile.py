"""CPU checks of the packed model-file reader (ter_hip_bin_*, modelfile.hip;
the formats of tools/convert_bitnet_to_packed.py and
tools/convert_llama_to_packed.py, read by load_model_from_bin,
cuda/ter_cuda_forward_bitnet.cu:698-784 and cuda/ter_cuda_forward_packed.cu:589-659).

Files are written from arrays in the converters' byte order
(tests/binfile_writer.py); the reader's directory, scales and host reads
must return those arrays, fp32 norms converted to fp16 by round to nearest
even (numpy's conversion; ties included), and malformed files are refused
at open.
"""
import ctypes as C
import struct

import numpy as np
import pytest

from ter_amd import _lib as L
from tests import binfile_writer as BW


def small(magic, **kw):
    args = dict(H=64, F=128, Nl=2, V=50, Nh=4, Nkv=2, Hd=16, seed=7)
    args.update(kw)
    return BW.random_model(magic, **args)


def open_bin(path):
    from ter_amd.modelfile import BinFile
    return BinFile(str(path))


@pytest.mark.parametrize("magic", [BW.TERT, BW.LLRT], ids=["TERT", "LLRT"])
def test_directory_and_host_reads(tmp_path, magic):
    m = small(magic)
    # fp16 rounding ties in a norm: 1 + 2^-11 and 1 + 3*2^-11 lie halfway between fp16 neighbours
    m["layers"][1]["attn_norm"][:4] = np.array([1 + 2 ** -11, 1 + 3 * 2 ** -11, -(1 + 2 ** -11), 65520.0],
                                               np.float32)
    path = BW.write(tmp_path / "m.bin", m)
    with open_bin(path) as f:
        h = f.header
        assert (h.magic, h.version, h.H, h.F, h.Nl, h.V, h.Nh, h.Nkv, h.Hd, h.Smax) == \
            (magic, 1, 64, 128, 2, 50, 4, 2, 16, 64)
        assert h.rope_theta == np.float32(500000.0) and h.eps == np.float32(1e-5)
        per_layer = (4 if magic == BW.TERT else 2) + 7
        assert len(f.tensors) == 2 + 2 * per_layer
        off = 64
        for t in f.tensors:  # contiguous, in file order
            assert t.offset == off
            off += t.bytes + (4 if t.kind == L.BIN_TRITS else 0)
        assert off == path.stat().st_size
        assert (f.read_host(f.find("token_embd")) == m["emb"].ravel()).all()
        assert (f.read_host(f.find("output_norm")).view(np.uint32) == m["out_norm"].view(np.uint32)).all()
        for l, lay in enumerate(m["layers"]):
            for nm in ("attn_norm", "ffn_norm") + (("attn_sub_norm", "ffn_sub_norm") if magic == BW.TERT else ()):
                i = f.find(nm, l)
                assert (f.read_host(i).view(np.uint32) == lay[nm].view(np.uint32)).all()
                h16 = f.read_host(i, as_f16=True)
                with np.errstate(over="ignore"):  # 65520 rounds to inf
                    want = lay[nm].astype(np.float16)
                assert (h16.view(np.uint16) == want.view(np.uint16)).all(), (l, nm)
            for nm in BW.PROJ:
                i = f.find(nm, l)
                t = f.tensors[i]
                v11, scale = lay[nm]
                assert (t.K, t.N) == BW.proj_shapes(64, 128, 32)[nm]
                assert t.scale == scale
                assert (f.read_host(i) == v11).all()
        ties = f.read_host(f.find("attn_norm", 1), as_f16=True)[:4]
        assert list(ties.astype(np.float32)) == [1.0, 1 + 2 ** -9, -1.0, np.inf]


def test_find_unknown_tensor(tmp_path):
    path = BW.write(tmp_path / "m.bin", small(BW.LLRT))
    with open_bin(path) as f:
        assert L.lib().ter_hip_bin_find(f._h, b"attn_sub_norm", 0) == L.ERR_NOTFOUND   # LLRT has no sub-norms
        assert L.lib().ter_hip_bin_find(f._h, b"Wq", 2) == L.ERR_NOTFOUND             # layer past Nl
        assert L.lib().ter_hip_bin_tensor(f._h, len(f.tensors), C.byref(L.BinTensor())) == L.ERR_NOTFOUND


def status_of(path):
    h = C.c_void_p()
    rc = L.lib().ter_hip_bin_open(str(path).encode(), C.byref(h), None)
    if rc == L.OK:
        L.lib().ter_hip_bin_close(h)
    return rc, L.lib().ter_hip_last_error().decode()


def test_malformed_files_are_refused(tmp_path):
    m = small(BW.TERT)
    assert status_of(tmp_path / "missing.bin")[0] == L.ERR_FILE
    assert status_of(BW.write(tmp_path / "ok.bin", m))[0] == L.OK
    rc, msg = status_of(BW.write(tmp_path / "short.bin", m, truncate=1))
    assert rc == L.ERR_FILE and "header implies" in msg
    assert status_of(BW.write(tmp_path / "long.bin", m, extra=b"\0"))[0] == L.ERR_FILE
    bad = dict(m, header=dict(m["header"], magic=0x12345678))
    assert status_of(BW.write(tmp_path / "magic.bin", bad))[0] == L.ERR_FILE
    bad = dict(m, header=dict(m["header"], version=2))
    assert status_of(BW.write(tmp_path / "version.bin", bad))[0] == L.ERR_FILE
    (tmp_path / "tiny.bin").write_bytes(struct.pack("<II", BW.TERT, 1))
    assert status_of(tmp_path / "tiny.bin")[0] == L.ERR_FILE
    # projections need N % 4 == 0: Nkv * Hd = 6 is not
    odd = BW.random_model(BW.LLRT, H=64, F=128, Nl=1, V=10, Nh=4, Nkv=2, Hd=16)
    odd["header"]["Hd"] = 3
    assert status_of(BW.write(tmp_path / "odd.bin", odd))[0] == L.ERR_SHAPE
