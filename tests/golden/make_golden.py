"""Write the golden fixtures of tests/golden/*.npz.

Expected outputs come from the reference's own code: oracle/_ref/libter_ref.so
is the reference mm_row / quantizers compiled from the reference sources
(oracle/Makefile), so this script needs the reference tree and a built
oracle/_ref.  The committed .npz files are data only (inputs + expected
outputs); the tests that read them run anywhere.

Fixtures:
  matmul_b_small.npz  closed-form dot products of tests/test_kernel_matmul_b_small.cpp:21-22,50-51
  int4tc_fixture.npz  the bit-exact fixture of cuda/ter_cuda_forward_packed_v13_int4tc.cu:512-547
                      (t = (7k + 13n) % 3, X = (11k + 3) % 15 - 7, K = 64, N = 16), v11 bytes
                      packed with the loop at :517-526
  i2s_block.npz       the hand-built i2_s block of tests/test_nt_dequant.cpp:37-61
  mm_row_random.npz   seeded random (X, W, scales) -> reference mm_row outputs, several shapes
  quantizers.npz      reference quantize(..., 9) and quantize_bitnet on seeded floats
  mm_row_blocked.npz  the per-block branch of the reference mm_row (src/tx/forward.cpp:308-330):
                      payload {-9841, 0, +9841}, per-block fp32 scales (some zero), block sizes
                      that do and do not divide N, 9-trit activations -> reference outputs
  mm_row_bitnet9.npz  the reference host forward's mm_row calls on BitNet weights: weights
                      through quantize_bitnet and quantize(..., 9) (src/host/load_gguf.cpp:64-111:
                      payload {-9841, 0, +9841}), activations through quantize(x, {1, K}, 9)
                      (src/tx/forward.cpp:400: |x| <= 9841) -> reference mm_row outputs

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402


def ref_mm(X: np.ndarray, xs: float, W: np.ndarray, ws: float, row: int = 0) -> np.ndarray:
    r = O.RefMmRow(X, xs, W, ws)
    out = r.run(row).copy()
    r.close()
    return out


def matmul_b_small():
    K1 = 27
    X1 = np.array([i - 13 for i in range(K1)], dtype=np.int32)
    W1 = np.array([(i % 5) - 2 for i in range(K1)], dtype=np.int32).reshape(K1, 1)
    K2 = 54
    X2 = np.array([(i * 7) % 19 - 9 for i in range(K2)], dtype=np.int32)
    W2 = np.array([(i * 5) % 13 - 6 for i in range(K2)], dtype=np.int32).reshape(K2, 1)
    e1 = ref_mm(X1, 1.0, W1, 1.0)
    e2 = ref_mm(X2, 1.0, W2, 1.0)
    np.savez(os.path.join(HERE, "matmul_b_small.npz"), X1=X1, W1=W1, out1=e1, X2=X2, W2=W2, out2=e2)


def int4tc_fixture():
    K, N = 64, 16
    v11 = np.zeros((N // 4) * K, dtype=np.uint8)
    trits = np.zeros((K, N), dtype=np.int32)
    for n in range(N):
        for k in range(K):
            code = (k * 7 + n * 13) % 3
            trits[k, n] = 1 if code == 1 else (-1 if code == 2 else 0)
            v11[(n // 4) * K + k] |= code << ((n % 4) * 2)
    X = np.array([(k * 11 + 3) % 15 - 7 for k in range(K)], dtype=np.int32)
    out = ref_mm(X, 1.0, trits, 1.0)  # scale 1: out == float(acc), exact
    np.savez(os.path.join(HERE, "int4tc_fixture.npz"), K=K, N=N, v11=v11, X=X, acc=out.astype(np.int64))


def i2s_block():
    buf = np.zeros(32 + 4, dtype=np.uint8)
    buf[:32] = 0x1B
    buf[32:] = np.frombuffer(np.float32(2.0).tobytes(), dtype=np.uint8)
    expected = np.concatenate([np.full(32, -2.0), np.zeros(32), np.full(32, 2.0), np.zeros(32)]).astype(np.float32)
    np.savez(os.path.join(HERE, "i2s_block.npz"), buf=buf, n=128, expected=expected)


# (K, N, seed, p_zero) -- small to medium shapes, incl. ragged K/N and the
# reference correctness-test shape 128 x 64 (tests/cuda_forward_correctness.cu:78).
RANDOM_CASES = [
    (128, 64, 42, 1 / 3),
    (300, 20, 7, 1 / 3),
    (1, 4, 9, 0.0),
    (27, 8, 11, 0.4),
    (513, 36, 13, 0.4),
    (2048, 32, 17, 1 / 3),
    (6912, 16, 19, 0.4),
]


def mm_row_random():
    arrays = {}
    for i, (K, N, seed, p0) in enumerate(RANDOM_CASES):
        W = O.rand_trits(seed, K, N, p0).astype(np.int32)
        X = O.rand_int8(seed + 1000, 3 * K).astype(np.int32).reshape(3, K)  # 3 rows; mm_row picks one
        row = 1
        xs = np.float32(0.0312)
        ws = np.float32(0.01 + 0.09 * ((seed * 2654435761) % 1000) / 1000.0)
        out = ref_mm(X, float(xs), W, float(ws), row)
        acc = ref_mm(X, 1.0, W, 1.0, row).astype(np.int64)
        arrays[f"c{i}_K"] = np.int32(K)
        arrays[f"c{i}_N"] = np.int32(N)
        arrays[f"c{i}_X"] = X.astype(np.int8)
        arrays[f"c{i}_row"] = np.int32(row)
        arrays[f"c{i}_v11"] = O.v11_pack(W.astype(np.int8)) if N % 4 == 0 else np.zeros(0, np.uint8)
        arrays[f"c{i}_W"] = W.astype(np.int8)
        arrays[f"c{i}_xs"] = xs
        arrays[f"c{i}_ws"] = ws
        arrays[f"c{i}_out"] = out
        arrays[f"c{i}_acc"] = acc
    arrays["n_cases"] = np.int32(len(RANDOM_CASES))
    np.savez_compressed(os.path.join(HERE, "mm_row_random.npz"), **arrays)


def quantizers():
    x = O.rand_normal_f32(123, 4096)
    x[7] = 0.0
    q9, s9 = O.ref_quantize(x, 9)
    qb, sb = O.ref_quantize_bitnet(x)
    np.savez(os.path.join(HERE, "quantizers.npz"), x=x, q9=q9, s9=s9, qb=qb, sb=sb)


# (K, N, seed): BitNet-2B's projection inputs (2560, 6912) and Llama's 2048.
BITNET9_CASES = [(2560, 64, 31), (6912, 32, 37), (2048, 48, 41)]


def mm_row_bitnet9():
    arrays = {}
    for i, (K, N, seed) in enumerate(BITNET9_CASES):
        wf = O.rand_normal_f32(seed, K * N) * np.float32(0.02)
        bn, sb = O.ref_quantize_bitnet(wf)                  # ternary {-1, 0, +1} and absmean scale
        tmp = bn.astype(np.float32) * sb                    # the bitnet round trip of tensor_to_trit
        W, ws = O.ref_quantize(tmp, 9)                      # payload {-9841, 0, +9841}
        W = W.reshape(K, N)
        mags = np.unique(np.abs(W[W != 0]))
        assert mags.size == 1, mags
        xf = O.rand_normal_f32(seed + 1, K)
        X, xs = O.ref_quantize(xf, 9)                       # |x| <= 9841
        out = ref_mm(X.reshape(1, K), float(xs), W, float(ws), 0)
        arrays[f"c{i}_K"] = np.int32(K)
        arrays[f"c{i}_N"] = np.int32(N)
        arrays[f"c{i}_trits"] = np.sign(W).astype(np.int8)
        arrays[f"c{i}_mag"] = np.int32(mags[0])
        arrays[f"c{i}_ws"] = np.float32(ws)
        arrays[f"c{i}_X"] = X.astype(np.int16)
        arrays[f"c{i}_xs"] = np.float32(xs)
        arrays[f"c{i}_out"] = out
    arrays["n_cases"] = np.int32(len(BITNET9_CASES))
    np.savez_compressed(os.path.join(HERE, "mm_row_bitnet9.npz"), **arrays)


# (K, N, block_size, seed)
BLOCKED_CASES = [(2560, 64, 4096, 51), (6912, 32, 1000, 53), (300, 20, 7, 57), (256, 16, 256 * 16, 59)]


def mm_row_blocked():
    arrays = {}
    for i, (K, N, bs, seed) in enumerate(BLOCKED_CASES):
        t = O.rand_trits(seed, K, N, 0.4)
        W = t.astype(np.int32) * 9841
        nb = -(-K * N // bs)
        u = (O.splitmix64(seed + 7, nb) >> np.uint64(40)).astype(np.float64) / float(1 << 24)
        bsc = (1e-6 + 2e-6 * u).astype(np.float32)
        bsc[::5] = 0.0  # blocks whose scale is zero (all-zero blocks of quantize_blocked)
        xf = O.rand_normal_f32(seed + 1, K)
        X, xs = O.ref_quantize(xf, 9)
        r = O.RefMmRow(X.reshape(1, K), float(xs), W, 1.0, bsc, bs)
        out = r.run(0).copy()
        r.close()
        arrays[f"c{i}_K"] = np.int32(K)
        arrays[f"c{i}_N"] = np.int32(N)
        arrays[f"c{i}_bs"] = np.int64(bs)
        arrays[f"c{i}_trits"] = t.astype(np.int8)
        arrays[f"c{i}_mag"] = np.int32(9841)
        arrays[f"c{i}_bsc"] = bsc
        arrays[f"c{i}_X"] = X.astype(np.int16)
        arrays[f"c{i}_xs"] = np.float32(xs)
        arrays[f"c{i}_out"] = out
    arrays["n_cases"] = np.int32(len(BLOCKED_CASES))
    np.savez_compressed(os.path.join(HERE, "mm_row_blocked.npz"), **arrays)


def main():
    if not O.ref_available():
        raise SystemExit("oracle/_ref is not built (make -C oracle ref needs the reference tree)")
    matmul_b_small()
    int4tc_fixture()
    i2s_block()
    mm_row_random()
    quantizers()
    mm_row_bitnet9()
    mm_row_blocked()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
