/*
 * ter_oracle.c -- CPU restatement of the reference ter hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP fabric in
 * ter_amd/ is compared against.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  The product never links it and
 * never falls back to it.
 *
 * Every function names the reference file:line it restates (paths relative
 * to the xaskasdf/ter source tree).  The arithmetic follows the reference
 * exactly: integer accumulation order does not matter (integer addition is
 * associative), but every floating-point step is kept in the same order and
 * precision as the reference so that fp32 outputs are bit-identical.
 *
 * Build: oracle/Makefile (gcc -O3 -mavx2 -mfma, the reference's own flags,
 * CMakeLists.txt:28-30).  No -ffast-math and no FMA contraction.
 *
 * Parity pins (what checks each function; all in tests/):
 *   orc_code_to_trit / orc_trit_to_code  -- tests/test_pack.cpp:8-15 and :29-33
 *                                           restated as known answers.
 *   orc_v11_pack / orc_v11_unpack        -- hand-derived byte known-answer tests,
 *                                           the int4tc fixture of
 *                                           cuda/ter_cuda_forward_packed_v13_int4tc.cu:512-547.
 *   orc_mm_row                           -- oracle/_ref (the reference mm_row itself)
 *                                           and the closed-form fixtures of
 *                                           tests/test_kernel_matmul_b_small.cpp.
 *   orc_mm_row_blocked                   -- oracle/_ref.
 *   orc_gemv_v11                         -- equality with orc_mm_row on unpacked W.
 *   orc_gemv_i8w / orc_gemm_i8w          -- equality with orc_mm_row (int64 accumulators,
 *                                           fp32 outputs) on random and ragged cases.
 *   orc_v11_to_i8                        -- equality with orc_v11_unpack.
 *   orc_rand_trits                       -- (an input generator, not a reference
 *                                           function) equality with oracle.rand_trits.
 *   orc_quant_int8                       -- closed-form tie / zero / amax cases.
 *   orc_float_to_half                    -- numpy's IEEE binary16 rounding on
 *                                           edge sets and random patterns.
 *   orc_relu2_rmsnorm_quant              -- closed forms (constant gate/up,
 *                                           negative gates), equality with
 *                                           orc_rmsnorm_quant where the
 *                                           1024-thread order reduces to it,
 *                                           a summation-order case.
 *   orc_residual_add_f16                 -- orc_float_to_half / orc_half_to_float.
 *   orc_residual_add_h16                 -- numpy's binary16 addition (one correctly
 *                                           rounded add) of hidden and half(y).
 *   orc_silu_f16 / orc_smul_quant        -- equal to orc_silu_mul_quant taken in one
 *                                           step (the split route), silu(g) equal to
 *                                           orc_silu_mul(g, 1).
 *   orc_silu_mul / orc_silu_mul_quant    -- closed forms (g = 0 or u = 0 gives 0,
 *                                           large g gives g * u exactly, very
 *                                           negative g gives 0), float64
 *                                           g * sigmoid(g) * u within the rounding
 *                                           bound, odd symmetry of silu(g) - g/2,
 *                                           the quantizer against orc_quant_int8.
 *   orc_rmsnorm_f16                      -- rms_inv equal to orc_rmsnorm_quant's (one
 *                                           reference order), constant-input closed
 *                                           form, fp16 rounding of the product.
 *   orc_lm_head_f16                      -- exact integer dot products, a case
 *                                           that separates the lane-strided order
 *                                           and butterfly from a sequential sum,
 *                                           odd H.
 *   orc_expf                             -- exp in double rounded to binary32 (max
 *                                           error measured over dense samples),
 *                                           exact special points.
 *   orc_rope_table, orc_rope_f16         -- identity at position 0, the NEOX
 *                                           pairing (k, k + hd/2) and the NORM
 *                                           pairing (2k, 2k+1) on unit vectors,
 *                                           norm preservation, table entries
 *                                           against numpy's double cos/sin.
 *   orc_attention_ref                    -- one position (out = v exactly), q = 0
 *                                           (out = mean of v), a dominant score,
 *                                           float64 softmax attention within the
 *                                           rounding bound.
 *   orc_attention_splitk                 -- orc_attention_ref within the rounding
 *                                           bound; equal to it where the chunked
 *                                           order reduces to the sequential one
 *                                           (one position).
 *   orc_argmax_f16                       -- numpy argmax on unique maxima; on
 *                                           ties the closed-form rule of the
 *                                           two reduction trees; NaN / -inf never
 *                                           win; all ineligible gives -1.
 *   orc_rmsnorm_quant                    -- closed forms (constant input, single
 *                                           spike), scale invariance, fp16
 *                                           widening of exact halves, the
 *                                           summation order against a
 *                                           double-precision bound.
 *   orc_quantize_bitnet, orc_quantize_nt -- oracle/_ref.
 *   orc_dequant_i2s                      -- tests/test_nt_dequant.cpp:37-61 block.
 *   orc_i2s_to_v11                       -- decode equality with orc_dequant_i2s.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#pragma STDC FP_CONTRACT OFF

/* ------------------------------------------------------------------------ */
/* 2-bit trit code map: include/ter/pack.hpp:8-21.                          */
/* 00 = 0, 01 = +1, 10 = -1, 11 = 0 (reserved, decodes as zero).            */
/* ------------------------------------------------------------------------ */
int orc_code_to_trit(unsigned c) {
    switch (c & 3u) {
        case 1u: return +1;
        case 2u: return -1;
        default: return 0;
    }
}

unsigned orc_trit_to_code(int t) { return t == 0 ? 0u : (t > 0 ? 1u : 2u); }

/* ------------------------------------------------------------------------ */
/* v11 column-major packed layout.                                          */
/*   W_col[j_byte*K + k] holds output columns 4*j_byte .. 4*j_byte+3 at      */
/*   input row k, column 4*j_byte+s at bits 2s..2s+1 (low bits = first col). */
/* Packer: tools/convert_llama_to_packed.py:128-140.                         */
/* Decoder: cuda/ter_cuda_forward_packed.cu:355-374 (byte at Wc = W_col +    */
/* j_byte*K, code (b >> 2*sub) & 3 for column j_base+sub).                   */
/* w_kn is the TritTensor payload orientation [K][N] row-major               */
/* (src/host/load_gguf.cpp transpose_2d, src/tx/forward.cpp:337).            */
/* ------------------------------------------------------------------------ */
int orc_v11_pack(const int8_t* w_kn, int K, int N, uint8_t* out) {
    if (K <= 0 || N <= 0 || (N % 4) != 0) return -5;
    const int NB = N / 4;
    for (int jb = 0; jb < NB; ++jb) {
        for (int k = 0; k < K; ++k) {
            unsigned b = 0;
            for (int s = 0; s < 4; ++s)
                b |= orc_trit_to_code(w_kn[(size_t)k * N + (size_t)(4 * jb + s)]) << (2 * s);
            out[(size_t)jb * K + k] = (uint8_t)b;
        }
    }
    return 0;
}

int orc_v11_unpack(const uint8_t* v11, int K, int N, int32_t* w_kn) {
    if (K <= 0 || N <= 0 || (N % 4) != 0) return -5;
    const int NB = N / 4;
    for (int jb = 0; jb < NB; ++jb) {
        const uint8_t* wc = v11 + (size_t)jb * K;
        for (int k = 0; k < K; ++k) {
            const unsigned b = wc[k];
            for (int s = 0; s < 4; ++s)
                w_kn[(size_t)k * N + (size_t)(4 * jb + s)] = orc_code_to_trit(b >> (2 * s));
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* mm_row, integer path: src/tx/forward.cpp:331-346.                         */
/*   acc[j] = sum_k int64(X[row*K+k]) * int64(W[k*N+j]), k-outer / j-inner,  */
/*   rows with X == 0 skipped (:334); s = Xt.scale * Wt.scale in fp32        */
/*   (:342); out[j] = float(acc[j]) * s (:344).                              */
/* acc_out (optional) receives the int64 accumulators.                      */
/* ------------------------------------------------------------------------ */
void orc_mm_row(const int32_t* X, int row, float xs, const int32_t* W, float ws,
                int K, int N, int64_t* acc_out, float* out) {
    int64_t* acc = acc_out ? acc_out : (int64_t*)malloc(sizeof(int64_t) * (size_t)N);
    memset(acc, 0, sizeof(int64_t) * (size_t)N);
    const int32_t* xp = X + (size_t)row * (size_t)K;
    for (int k = 0; k < K; ++k) {
        const int32_t xv = xp[k];
        if (xv == 0) continue;
        const int64_t xv64 = (int64_t)xv;
        const int32_t* w_row = W + (size_t)k * (size_t)N;
        for (int j = 0; j < N; ++j) acc[j] += xv64 * (int64_t)w_row[j];
    }
    const float s = xs * ws;
    for (int j = 0; j < N; ++j) out[j] = (float)acc[j] * s;
    if (!acc_out) free(acc);
}

/* ------------------------------------------------------------------------ */
/* mm_row, per-block branch: src/tx/forward.cpp:308-330.                     */
/* Double accumulation of xv * w * block_scales[(k*N+j)/bs]; out =           */
/* float(facc * double(Xt.scale)).  The HIP boundary rejects per-block       */
/* weights; this exists so the tests can state what is rejected.            */
/* ------------------------------------------------------------------------ */
void orc_mm_row_blocked(const int32_t* X, int row, float xs, const int32_t* W,
                        const float* block_scales, int block_size, int K, int N,
                        float* out) {
    double* facc = (double*)calloc((size_t)N, sizeof(double));
    const int32_t* xp = X + (size_t)row * (size_t)K;
    for (int k = 0; k < K; ++k) {
        const int32_t xv = xp[k];
        if (xv == 0) continue;
        const double xvd = (double)xv;
        const size_t base = (size_t)k * (size_t)N;
        const int32_t* w_row = W + base;
        for (int j = 0; j < N; ++j) {
            const size_t blk = (base + (size_t)j) / (size_t)block_size;
            facc[j] += xvd * (double)w_row[j] * (double)block_scales[blk];
        }
    }
    for (int j = 0; j < N; ++j) out[j] = (float)(facc[j] * (double)xs);
    free(facc);
}

/* ------------------------------------------------------------------------ */
/* Packed GEMV semantics of mm_packed_v4 (v11 production kernel):            */
/* cuda/ter_cuda_forward_packed.cu:346-397.  int8 X times v11-packed trits,  */
/* int32 accumulation; out = float(acc) * (x_scale * w_scale) (:353,:393).   */
/* The reference writes fp16; this fabric (and the oracle) keep fp32, which  */
/* is the mm_row output type (src/tx/forward.cpp:344).                       */
/* ------------------------------------------------------------------------ */
void orc_gemv_v11(const int8_t* x, float xs, const uint8_t* v11, float ws, int K, int N,
                  int32_t* acc_out, float* out) {
    const int NB = N / 4;
    const float s = xs * ws;
    for (int jb = 0; jb < NB; ++jb) {
        const uint8_t* wc = v11 + (size_t)jb * K;
        int32_t acc[4] = {0, 0, 0, 0};
        for (int k = 0; k < K; ++k) {
            const int xv = x[k];
            if (xv == 0) continue;
            const unsigned b = wc[k];
            for (int s2 = 0; s2 < 4; ++s2) acc[s2] += xv * orc_code_to_trit(b >> (2 * s2));
        }
        for (int s2 = 0; s2 < 4; ++s2) {
            if (acc_out) acc_out[4 * jb + s2] = acc[s2];
            if (out) out[4 * jb + s2] = (float)acc[s2] * s;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* mm_row's integer path (src/tx/forward.cpp:331-346) at int8 width: x int8  */
/* [K], W int8 [K][N] row-major (the payload orientation), the reference's   */
/* k-outer / j-inner loop with zero rows of x skipped, int32 accumulators    */
/* (exact: |acc| <= 128 * K < 2^31); out = float(acc) * (xs * ws).  The j    */
/* loop vectorizes as the reference's does; threads split the columns       */
/* (integer sums are exact in any split).  The checker of full-size lists.  */
/* ------------------------------------------------------------------------ */
void orc_gemv_i8w(const int8_t* x, float xs, const int8_t* W, float ws, int K, int N, int32_t* acc_out,
                  float* out) {
    const float s = xs * ws;
    enum { CB = 256 };  /* columns per thread chunk */
    #pragma omp parallel for schedule(static)
    for (int j0 = 0; j0 < N; j0 += CB) {
        const int j1 = j0 + CB < N ? j0 + CB : N;
        int32_t acc[CB];
        for (int j = j0; j < j1; ++j) acc[j - j0] = 0;
        for (int k = 0; k < K; ++k) {
            const int32_t xv = x[k];
            if (xv == 0) continue;
            const int8_t* w_row = W + (size_t)k * (size_t)N;
            for (int j = j0; j < j1; ++j) acc[j - j0] += xv * (int32_t)w_row[j];
        }
        for (int j = j0; j < j1; ++j) {
            if (acc_out) acc_out[j] = acc[j - j0];
            if (out) out[j] = (float)acc[j - j0] * s;
        }
    }
}

/* orc_gemv_i8w per row of X [M][K] with per-row scales xs[M] (the batched   */
/* semantics below); threads split the rows.                                 */
void orc_gemm_i8w(const int8_t* X, const float* xs, int M, const int8_t* W, float ws, int K, int N,
                  int32_t* acc_out, float* out) {
    const float* sx = xs;
    #pragma omp parallel for schedule(dynamic, 1)
    for (int m = 0; m < M; ++m) {
        const float s = sx[m] * ws;
        int32_t* acc = (int32_t*)calloc((size_t)N, sizeof(int32_t));
        const int8_t* xr = X + (size_t)m * (size_t)K;
        for (int k = 0; k < K; ++k) {
            const int32_t xv = xr[k];
            if (xv == 0) continue;
            const int8_t* w_row = W + (size_t)k * (size_t)N;
            for (int j = 0; j < N; ++j) acc[j] += xv * (int32_t)w_row[j];
        }
        for (int j = 0; j < N; ++j) {
            if (acc_out) acc_out[(size_t)m * N + j] = acc[j];
            if (out) out[(size_t)m * N + j] = (float)acc[j] * s;
        }
        free(acc);
    }
}

/* orc_v11_unpack at int8 width. */
int orc_v11_to_i8(const uint8_t* v11, int K, int N, int8_t* w_kn) {
    if (K <= 0 || N <= 0 || (N % 4) != 0) return -5;
    const int NB = N / 4;
    #pragma omp parallel for schedule(static)
    for (int k = 0; k < K; ++k)
        for (int jb = 0; jb < NB; ++jb) {
            const unsigned b = v11[(size_t)jb * K + k];
            for (int s2 = 0; s2 < 4; ++s2) w_kn[(size_t)k * N + (size_t)(4 * jb + s2)] = (int8_t)orc_code_to_trit(b >> (2 * s2));
        }
    return 0;
}

/* Test-input generator (not a reference function): trits [K][N] from the    */
/* counter-based splitmix64 stream of oracle.rand_trits, which             */
/* ter_hip_synth_v11 draws on the device -- element i = k*N + n takes state  */
/* seed + (i+1) * 0x9E3779B97F4A7C15; u = top 32 bits of the mixed value;   */
/* trit 0 if u < t0, +1 if u < t1, else -1.                                 */
void orc_rand_trits(uint64_t seed, int K, int N, uint64_t t0, uint64_t t1, int8_t* out) {
    const size_t n = (size_t)K * (size_t)N;
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        uint64_t z = seed + (uint64_t)(i + 1) * 0x9E3779B97F4A7C15ULL;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        z = z ^ (z >> 31);
        const uint64_t u = z >> 32;
        out[i] = (int8_t)(u < t0 ? 0 : (u < t1 ? 1 : -1));
    }
}

/* ------------------------------------------------------------------------ */
/* Batched semantics (M > 1): cuda/ter_cuda_addonly_batched.cu:31-124.        */
/* X[M][K] int8 row-major, per-row activation scale X_scale[m];              */
/* out[m*N+j] = float(acc[m][j]) * (X_scale[m] * w_scale) (:117-123).        */
/* ------------------------------------------------------------------------ */
void orc_gemm_v11(const int8_t* X, const float* xs, int M, const uint8_t* v11, float ws,
                  int K, int N, int32_t* acc_out, float* out) {
    for (int m = 0; m < M; ++m)
        orc_gemv_v11(X + (size_t)m * K, xs[m], v11, ws, K, N,
                     acc_out ? acc_out + (size_t)m * N : NULL,
                     out ? out + (size_t)m * N : NULL);
}

/* ------------------------------------------------------------------------ */
/* Activation absmax -> int8 quantizer: quant_int8_k,                        */
/* cuda/ter_cuda_forward_packed.cu:40-62 (same steps in the fused            */
/* rmsnorm_quant_* prologues, cuda/ter_cuda_forward_bitnet.cu:94-103).       */
/*   amax = max|x| + 1e-9f; scale = 127.f / amax;                            */
/*   q = __float2int_rn(x * scale) (round half to even), clamped [-128,127]; */
/*   act_scale = 1.f / scale.                                                */
/* ------------------------------------------------------------------------ */
void orc_quant_int8(const float* x, int n, int8_t* q, float* act_scale) {
    float local = 0.f;
    for (int i = 0; i < n; ++i) {
        const float v = fabsf(x[i]);
        if (v > local) local = v;
    }
    const float amax = local + 1e-9f;
    const float scale = 127.0f / amax;
    *act_scale = 1.0f / scale;
    for (int i = 0; i < n; ++i) {
        const float v = x[i] * scale;
        int qi = (int)nearbyintf(v); /* default rounding mode: nearest-even */
        if (qi > 127) qi = 127;
        if (qi < -128) qi = -128;
        q[i] = (int8_t)qi;
    }
}

/* Per-row (per-token) variant used by the batched path: each row of X[M][K]
 * is quantized independently with the quant_int8_k steps above
 * (per-row X_scale of cuda/ter_cuda_addonly_batched.cu:33-38). */
void orc_quant_int8_rows(const float* x, int M, int K, int8_t* q, float* act_scale) {
    for (int m = 0; m < M; ++m)
        orc_quant_int8(x + (size_t)m * K, K, q + (size_t)m * K, act_scale + m);
}

/* ------------------------------------------------------------------------ */
/* IEEE binary16 -> binary32 (exact), the __half2float of the reference.     */
/* ------------------------------------------------------------------------ */
float orc_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0x1Fu) {
        bits = sign | 0x7F800000u | (man << 13);           /* inf / nan */
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);  /* normal */
    } else if (man == 0) {
        bits = sign;                                       /* zero */
    } else {                                               /* subnormal: renormalize */
        exp = 113;
        while ((man & 0x400u) == 0) {
            man <<= 1;
            --exp;
        }
        bits = sign | (exp << 23) | ((man & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* ------------------------------------------------------------------------ */
/* Fused RMSNorm + int8 quantizer: rmsnorm_quant_f32_in_k and                 */
/* rmsnorm_quant_fp16_in_k, cuda/ter_cuda_forward_bitnet.cu:64-146, launched  */
/* with one block of 256 threads (:859, :873).  x is fp32 (x16 == NULL) or    */
/* fp16 (x32 == NULL); gamma is fp16.                                         */
/*   partial[t] = sum over i = t, t+256, ... (increasing) of x_i * x_i, each  */
/*                step one fused multiply-add (nvcc contracts                 */
/*                `local_sum += v * v` by default, -fmad=true);               */
/*   tree: for s = 128, 64, ..., 1: partial[t] += partial[t + s] (t < s);     */
/*   rms_inv = 1 / sqrt(partial[0] / H + eps).  The reference calls rsqrtf,   */
/*            an approximation; this restatement and the fabric both use the  */
/*            correctly rounded division and square root, so CPU and GPU      */
/*            agree bit for bit (a documented deviation of <= 2 ulp in        */
/*            rms_inv from the reference GPU build);                          */
/*   n_i = (x_i * rms_inv) * gamma_i;                                         */
/*   then the quant_int8_k steps on n (orc_quant_int8).                       */
/* ------------------------------------------------------------------------ */
void orc_rmsnorm_quant(const float* x32, const uint16_t* x16, const uint16_t* gamma, int H, float eps,
                       int8_t* q, float* act_scale, float* rms_inv_out) {
    float part[256];
    for (int t = 0; t < 256; ++t) {
        float acc = 0.f;
        for (int i = t; i < H; i += 256) {
            const float v = x32 ? x32[i] : orc_half_to_float(x16[i]);
            acc = fmaf(v, v, acc);
        }
        part[t] = acc;
    }
    for (int s = 128; s > 0; s >>= 1)
        for (int t = 0; t < s; ++t) part[t] += part[t + s];
    const float rms_inv = 1.0f / sqrtf(part[0] / (float)H + eps);
    if (rms_inv_out) *rms_inv_out = rms_inv;
    float* n = (float*)malloc(sizeof(float) * (size_t)(H > 0 ? H : 1));
    if (!n) return;
    for (int i = 0; i < H; ++i) {
        const float v = x32 ? x32[i] : orc_half_to_float(x16[i]);
        const float a = v * rms_inv;
        n[i] = a * orc_half_to_float(gamma[i]);
    }
    orc_quant_int8(n, H, q, act_scale);
    free(n);
}

/* ------------------------------------------------------------------------ */
/* binary32 -> binary16, round to nearest even (the reference's             */
/* __float2half of its fp16 outputs, cuda/ter_cuda_forward_packed.cu:393).  */
/* ------------------------------------------------------------------------ */
uint16_t orc_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u); /* nan / inf */
    if (ax >= 0x477FF000u) return sign | 0x7C00u;                               /* rounds past 65504 */
    if (ax < 0x38800000u) {                                                     /* half subnormal or zero */
        if (ax < 0x33000000u) return sign;                                       /* below half of 2^-24 */
        const uint32_t man = (ax & 0x7FFFFFu) | 0x800000u;
        const int shift = 126 - (int)(ax >> 23);                                 /* 14 .. 24 */
        const uint32_t q = man >> shift, rem = man & ((1u << shift) - 1u), half = 1u << (shift - 1);
        return sign | (uint16_t)(q + (rem > half || (rem == half && (q & 1u))));
    }
    const uint32_t e = (ax >> 23) - 112u, man = ax & 0x7FFFFFu;                  /* normal */
    const uint32_t q = (e << 10) | (man >> 13), rem = man & 0x1FFFu;
    return sign | (uint16_t)(q + (rem > 0x1000u || (rem == 0x1000u && (q & 1u))));
}

void orc_float_to_half_n(const float* f, uint16_t* h, size_t n) {
    for (size_t i = 0; i < n; ++i) h[i] = orc_float_to_half(f[i]);
}

/* ------------------------------------------------------------------------ */
/* Fused relu^2(gate) * up + RMSNorm + int8 quantizer:                       */
/* relu2_mul_rmsnorm_quant_k, cuda/ter_cuda_forward_bitnet.cu:258-309,       */
/* launched with one block of 1024 threads (:884).  gate, up, gamma fp16.    */
/*   v_i = (g_i > 0 ? g_i * g_i : 0) * u_i;                                 */
/*   partial[t] (t < 1024) = sum over i = t, t+1024, ... of v_i * v_i, each  */
/*   step a fused multiply-add; tree s = 512, ..., 1; rms_inv as in         */
/*   orc_rmsnorm_quant (correctly rounded); n_i = (v_i * rms_inv) * gamma_i; */
/*   then quant_int8_k.                                                      */
/* ------------------------------------------------------------------------ */
static float relu2_mul(uint16_t g16, uint16_t u16) {
    const float g = orc_half_to_float(g16), u = orc_half_to_float(u16);
    const float r = g > 0.f ? g * g : 0.f;
    return r * u;
}

void orc_relu2_rmsnorm_quant(const uint16_t* gate, const uint16_t* up, const uint16_t* gamma, int F, float eps,
                             int8_t* q, float* act_scale, float* rms_inv_out) {
    float part[1024];
    for (int t = 0; t < 1024; ++t) {
        float acc = 0.f;
        for (int i = t; i < F; i += 1024) {
            const float v = relu2_mul(gate[i], up[i]);
            acc = fmaf(v, v, acc);
        }
        part[t] = acc;
    }
    for (int s = 512; s > 0; s >>= 1)
        for (int t = 0; t < s; ++t) part[t] += part[t + s];
    const float rms_inv = 1.0f / sqrtf(part[0] / (float)F + eps);
    if (rms_inv_out) *rms_inv_out = rms_inv;
    float* n = (float*)malloc(sizeof(float) * (size_t)(F > 0 ? F : 1));
    if (!n) return;
    for (int i = 0; i < F; ++i) {
        const float a = relu2_mul(gate[i], up[i]) * rms_inv;
        n[i] = a * orc_half_to_float(gamma[i]);
    }
    orc_quant_int8(n, F, q, act_scale);
    free(n);
}

/* ------------------------------------------------------------------------ */
/* Residual add of an fp16-rounded projection output: add_k_f32,             */
/* cuda/ter_cuda_forward_bitnet.cu:51-54, after the GEMV wrote               */
/* __float2half((float)acc * scale): hidden[i] += float(half(y[i])).         */
/* ------------------------------------------------------------------------ */
void orc_residual_add_f16(float* hidden, const float* y, int n) {
    for (int i = 0; i < n; ++i) hidden[i] = hidden[i] + orc_half_to_float(orc_float_to_half(y[i]));
}

/* ------------------------------------------------------------------------ */
/* Residual add into an fp16 hidden state: add_k,                            */
/* cuda/ter_cuda_forward_packed.cu:113-116, after the GEMV wrote an fp16     */
/* output: hidden[i] = half(float(hidden[i]) + float(half(y[i]))).  binary32 */
/* has more than 2*11+1 significand bits, so the two roundings equal one     */
/* correctly rounded binary16 addition.                                      */
/* ------------------------------------------------------------------------ */
void orc_residual_add_h16(uint16_t* hidden, const float* y, int n) {
    for (int i = 0; i < n; ++i) {
        const float a = orc_half_to_float(hidden[i]);
        const float b = orc_half_to_float(orc_float_to_half(y[i]));
        hidden[i] = orc_float_to_half(a + b);
    }
}

/* ------------------------------------------------------------------------ */
/* SiLU(gate) * up + int8 quantizer: silu_mul_quant_k,                       */
/* cuda/ter_cuda_forward_packed.cu:312-344, launched <<<1,1024>>> (:535).    */
/* gate and up fp16; v_i = (g_i / (1 + expf(-g_i))) * u_i kept in binary32   */
/* (the kernel's shared-memory copy is float, never rounded to fp16); then   */
/* the quant_int8_k steps on v (amax + 1e-9f, 127 / amax, round to nearest   */
/* even, clamp).  expf is orc_expf.  v_out (may be NULL) receives v.         */
/* ------------------------------------------------------------------------ */
float orc_expf(float x); /* defined with the attention softmax below */

float orc_silu_mul(uint16_t g16, uint16_t u16) {
    const float g = orc_half_to_float(g16), u = orc_half_to_float(u16);
    const float d = 1.0f + orc_expf(-g);
    const float sg = g / d;
    return sg * u;
}

/* The same computation split in two, as the fabric's TER_HIP_X_SMUL route
 * runs it: orc_silu_f16 is the first step alone, silu(g) = g / (1 + expf(-g))
 * of each fp16 gate value; orc_smul_quant multiplies that fp32 value by the
 * fp16 up value and quantizes.  smul_quant(silu(g), u) is silu_mul_quant(g, u)
 * bit for bit (the same two rounded operations in the same order). */
void orc_silu_f16(const uint16_t* gate, int n, float* out) {
    for (int i = 0; i < n; ++i) {
        const float g = orc_half_to_float(gate[i]);
        const float d = 1.0f + orc_expf(-g);
        out[i] = g / d;
    }
}

void orc_smul_quant(const float* s, const uint16_t* up, int F, int8_t* q, float* act_scale, float* v_out) {
    float* v = (float*)malloc(sizeof(float) * (size_t)(F > 0 ? F : 1));
    if (!v) return;
    for (int i = 0; i < F; ++i) v[i] = s[i] * orc_half_to_float(up[i]);
    orc_quant_int8(v, F, q, act_scale);
    if (v_out) memcpy(v_out, v, sizeof(float) * (size_t)F);
    free(v);
}

void orc_silu_mul_quant(const uint16_t* gate, const uint16_t* up, int F, int8_t* q, float* act_scale, float* v_out) {
    float* v = (float*)malloc(sizeof(float) * (size_t)(F > 0 ? F : 1));
    if (!v) return;
    for (int i = 0; i < F; ++i) v[i] = orc_silu_mul(gate[i], up[i]);
    orc_quant_int8(v, F, q, act_scale);
    if (v_out) memcpy(v_out, v, sizeof(float) * (size_t)F);
    free(v);
}

/* ------------------------------------------------------------------------ */
/* RMSNorm with fp16 output: rmsnorm_f32_in_k, cuda/ter_cuda_forward_bitnet.cu */
/* :37-47, launched <<<1,256>>> before the lm_head (:890).  The sum of        */
/* squares is orc_rmsnorm_quant's (256 strided fused multiply-add partials,   */
/* the halving tree, correctly rounded rms_inv); y_i = half((x_i * rms_inv) * */
/* gamma_i).                                                                  */
/* ------------------------------------------------------------------------ */
void orc_rmsnorm_f16(const float* x, const uint16_t* gamma, int H, float eps, uint16_t* y, float* rms_inv_out) {
    float part[256];
    for (int t = 0; t < 256; ++t) {
        float acc = 0.f;
        for (int i = t; i < H; i += 256) acc = fmaf(x[i], x[i], acc);
        part[t] = acc;
    }
    for (int s = 128; s > 0; s >>= 1)
        for (int t = 0; t < s; ++t) part[t] += part[t + s];
    const float rms_inv = 1.0f / sqrtf(part[0] / (float)H + eps);
    if (rms_inv_out) *rms_inv_out = rms_inv;
    for (int i = 0; i < H; ++i) {
        const float a = x[i] * rms_inv;
        y[i] = orc_float_to_half(a * orc_half_to_float(gamma[i]));
    }
}

/* ------------------------------------------------------------------------ */
/* fp16 lm_head GEMV: mm_fp16_lm_head_k, cuda/ter_cuda_forward_bitnet.cu:     */
/* 388-429.  One 32-lane warp per vocabulary row v of token_embd [V][H]:      */
/*   H even: lane l sums pairs k = l, l+32, ... < H/2 in that order,          */
/*           acc += x[2k]*e[2k] + x[2k+1]*e[2k+1] (products of fp16 values    */
/*           are exact in fp32, so the one rounding per step is the sum's     */
/*           and no contraction choice can change it);                        */
/*   H odd:  lane l sums elements k = l, l+32, ... < H, acc += x[k]*e[k];     */
/*   then the xor butterfly o = 16, 8, 4, 2, 1 (acc_l += acc_{l^o} on every   */
/*   lane at once); lane 0's value, rounded to fp16, is logits[v].           */
/* acc_out (optional) receives lane 0's fp32 value.                          */
/* ------------------------------------------------------------------------ */
void orc_lm_head_f16(const uint16_t* x, const uint16_t* e, int H, int V, uint16_t* logits, float* acc_out) {
    #pragma omp parallel for schedule(static)  /* rows are independent; each keeps its own order */
    for (int v = 0; v < V; ++v) {
        const uint16_t* row = e + (size_t)v * (size_t)H;
        float lane[32];
        for (int l = 0; l < 32; ++l) {
            float acc = 0.f;
            if (H % 2 == 0) {
                for (int k = l; k < H / 2; k += 32) {
                    const float p0 = orc_half_to_float(x[2 * k]) * orc_half_to_float(row[2 * k]);
                    const float p1 = orc_half_to_float(x[2 * k + 1]) * orc_half_to_float(row[2 * k + 1]);
                    acc += p0 + p1;
                }
            } else {
                for (int k = l; k < H; k += 32) acc += orc_half_to_float(x[k]) * orc_half_to_float(row[k]);
            }
            lane[l] = acc;
        }
        for (int o = 16; o > 0; o >>= 1) {
            float next[32];
            for (int l = 0; l < 32; ++l) next[l] = lane[l] + lane[l ^ o];
            memcpy(lane, next, sizeof lane);
        }
        if (acc_out) acc_out[v] = lane[0];
        if (logits) logits[v] = orc_float_to_half(lane[0]);
    }
}

/* ------------------------------------------------------------------------ */
/* Two-pass argmax over fp16 logits: argmax_local_k / argmax_final_k,        */
/* cuda/ter_cuda_forward_bitnet.cu:454-495, launched with 128 parts of 256   */
/* threads and a 128-thread final block (:906-911).  Part b covers           */
/* [b*chunk, min(N, (b+1)*chunk)), chunk = ceil(N/128); thread t of a part   */
/* keeps its first strict maximum over i = start+t, +256, ...; each tree     */
/* level keeps the lower slot unless the upper is strictly greater.  Values  */
/* not above -1e30 (-inf) and NaN never win; with none eligible the result   */
/* is -1.                                                                    */
/* ------------------------------------------------------------------------ */
static void orc_tree_max(float* best, int* idx, int n) {
    for (int s = n / 2; s > 0; s >>= 1)
        for (int t = 0; t < s; ++t)
            if (best[t + s] > best[t]) {
                best[t] = best[t + s];
                idx[t] = idx[t + s];
            }
}

int orc_argmax_f16(const uint16_t* logits, int N) {
    enum { PARTS = 128, THREADS = 256 };
    float pmax[PARTS];
    int pidx[PARTS];
    const int chunk = (N + PARTS - 1) / PARTS;
    for (int b = 0; b < PARTS; ++b) {
        const int start = b * chunk;
        const int end = N < start + chunk ? N : start + chunk;
        float best[THREADS];
        int idx[THREADS];
        for (int t = 0; t < THREADS; ++t) {
            best[t] = -1e30f;
            idx[t] = -1;
            for (int i = start + t; i < end; i += THREADS) {
                const float v = orc_half_to_float(logits[i]);
                if (v > best[t]) {
                    best[t] = v;
                    idx[t] = i;
                }
            }
        }
        orc_tree_max(best, idx, THREADS);
        pmax[b] = best[0];
        pidx[b] = idx[0];
    }
    float best[PARTS];
    int idx[PARTS];
    for (int t = 0; t < PARTS; ++t) {
        best[t] = -1e30f;
        idx[t] = -1;
        if (pmax[t] > best[t]) {
            best[t] = pmax[t];
            idx[t] = pidx[t];
        }
    }
    orc_tree_max(best, idx, PARTS);
    return idx[0];
}

/* ------------------------------------------------------------------------ */
/* exp for the attention softmax.  The reference calls CUDA's expf, whose   */
/* exact results only its own GPU reproduces; this build uses one binary32  */
/* algorithm, the same operation for operation here and in the kernel:      */
/* Cody-Waite argument reduction x = n ln2 + r (ln2 split so that n ln2_hi  */
/* is exact), e^r by the degree-7 Taylor polynomial in Horner form with     */
/* fused multiply-adds (truncation < 6e-9 relative on |r| <= ln2/2), then   */
/* the scale 2^n applied in two exact-or-once-rounded steps.                */
/* ------------------------------------------------------------------------ */
static float orc_pow2i(int e) {  /* 2^e for -126 <= e <= 127 */
    const uint32_t b = (uint32_t)(e + 127) << 23;
    float f;
    memcpy(&f, &b, sizeof f);
    return f;
}

float orc_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.972084045410156f) return 0.0f;
    const float n = rintf(x * 1.44269502162933349609375f);
    float r = fmaf(-n, 0.693145751953125f, x);
    r = fmaf(-n, 1.42860676533018704e-06f, r);
    float p = 1.98412701e-04f;
    p = fmaf(p, r, 1.38888892e-03f);
    p = fmaf(p, r, 8.33333377e-03f);
    p = fmaf(p, r, 4.16666679e-02f);
    p = fmaf(p, r, 1.66666672e-01f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int ni = (int)n;
    const int n1 = ni / 2, n2 = ni - n1;
    return (p * orc_pow2i(n1)) * orc_pow2i(n2);
}

void orc_expf_n(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = orc_expf(x[i]);
}

/* ------------------------------------------------------------------------ */
/* NEOX RoPE: rope_k, cuda/ter_cuda_forward_bitnet.cu:185-200 (pairs        */
/* (v[k], v[k + hd/2]); tools/bitnet_pyfwd.py:83-94).  Table entry (p, k):  */
/* freq = fl(1 / fl(theta^(2k/hd))), a = fl(p * freq), c = fl(cos a),      */
/* s = fl(sin a): the reference's float steps, with its powf / cosf / sinf  */
/* replaced by libm in double rounded once to binary32.                     */
/* cs: [n_pos][hd/2][2] (cos, sin).                                         */
/* ------------------------------------------------------------------------ */
void orc_rope_table(float theta, int hd, int n_pos, float* cs) {
    const int half = hd / 2;
    for (int k = 0; k < half; ++k) {
        const float e = (2.0f * (float)k) / (float)hd;
        const float pw = (float)pow((double)theta, (double)e);
        const float freq = 1.0f / pw;
        for (int p = 0; p < n_pos; ++p) {
            const float a = (float)p * freq;
            cs[((size_t)p * half + k) * 2] = (float)cos((double)a);
            cs[((size_t)p * half + k) * 2 + 1] = (float)sin((double)a);
        }
    }
}

/* Rotate n_heads fp16 head vectors in place with one position's table row
 * cs_p [hd/2][2]: pair k is (v[k], v[k + hd/2]) for NEOX (BitNet, rope_k of
 * cuda/ter_cuda_forward_bitnet.cu:185-200) or (v[2k], v[2k+1]) for NORM (the
 * Llama forward's rope_k, cuda/ter_cuda_forward_packed.cu:64-76);
 * r0 = v0*c - v1*s, r1 = v0*s + v1*c, each contracted as one fused
 * multiply-add over the other product (fma(v0, c, -(v1 s)), fma(v0, s, v1 c):
 * the fold LLVM applies to the reference's expression), rounded to fp16. */
void orc_rope_f16(uint16_t* v, int n_heads, int hd, const float* cs_p, int neox) {
    const int half = hd / 2;
    for (int h = 0; h < n_heads; ++h)
        for (int k = 0; k < half; ++k) {
            uint16_t* a = v + (size_t)h * hd + (neox ? k : 2 * k);
            uint16_t* b = neox ? a + half : a + 1;
            const float c = cs_p[2 * k], sn = cs_p[2 * k + 1];
            const float v0 = orc_half_to_float(*a), v1 = orc_half_to_float(*b);
            const float r0 = fmaf(v0, c, -(v1 * sn));
            const float r1 = fmaf(v0, sn, v1 * c);
            *a = orc_float_to_half(r0);
            *b = orc_float_to_half(r1);
        }
}

/* ------------------------------------------------------------------------ */
/* Decode attention, reference order: attention_k,                           */
/* cuda/ter_cuda_forward_bitnet.cu:336-374, for one token over seq cached    */
/* positions.  q fp16 [nh][hd] (after RoPE); K, V fp16 [seq][nkv][hd]; query */
/* head h reads KV head h * nkv / nh.                                        */
/*   score_s = fl(dot_s * fl(1/sqrt(hd))), dot_s the fp32 sum over d in     */
/*     order (products of fp16 values are exact, so contraction is moot;    */
/*     the reference's rsqrtf is replaced by the correctly rounded value);   */
/*   one thread: mx = max_s score_s; e_s = orc_expf(score_s - mx); sum over  */
/*     s in order; p_s = e_s * (1 / sum);                                    */
/*   out[d] = half(acc), acc = fma(p_s, v_sd, acc) over s in order.         */
/* out32 (optional) receives acc.                                            */
/* ------------------------------------------------------------------------ */
static float orc_score(const uint16_t* q, const uint16_t* k, int hd, float inv_sqrt) {
    float dot = 0.f;
    for (int d = 0; d < hd; ++d) dot = fmaf(orc_half_to_float(q[d]), orc_half_to_float(k[d]), dot);
    return dot * inv_sqrt;
}

void orc_attention_ref(const uint16_t* q, const uint16_t* K, const uint16_t* V, int nh, int nkv, int hd, int seq,
                       uint16_t* out16, float* out32) {
    const float inv_sqrt = (float)(1.0 / sqrt((double)hd));
    float* p = (float*)malloc(sizeof(float) * (size_t)(seq > 0 ? seq : 1));
    if (!p) return;
    for (int h = 0; h < nh; ++h) {
        const int g = h * nkv / nh;
        for (int s = 0; s < seq; ++s)
            p[s] = orc_score(q + (size_t)h * hd, K + ((size_t)s * nkv + g) * hd, hd, inv_sqrt);
        float mx = p[0];
        for (int s = 1; s < seq; ++s)
            if (p[s] > mx) mx = p[s];
        float sum = 0.f;
        for (int s = 0; s < seq; ++s) {
            p[s] = orc_expf(p[s] - mx);
            sum += p[s];
        }
        const float inv = 1.f / sum;
        for (int s = 0; s < seq; ++s) p[s] *= inv;
        for (int d = 0; d < hd; ++d) {
            float acc = 0.f;
            for (int s = 0; s < seq; ++s) acc = fmaf(p[s], orc_half_to_float(V[((size_t)s * nkv + g) * hd + d]), acc);
            if (out32) out32[(size_t)h * hd + d] = acc;
            if (out16) out16[(size_t)h * hd + d] = orc_float_to_half(acc);
        }
    }
    free(p);
}

/* ------------------------------------------------------------------------ */
/* Decode attention in this build's chunked order (the GPU kernel's):        */
/* positions in chunks of 64; per chunk c and head: m_c = max score,         */
/* e_s = orc_expf(score_s - m_c), l_c = the xor butterfly (o = 32 .. 1) over */
/* the chunk's 64 lanes (lane i holds position 64c + i, 0 past seq),         */
/* o_c[d] = fma(e_s, v_sd, .) over the chunk's positions in order; then over */
/* chunks in order: w_c = orc_expf(m_c - M) (M = max_c m_c),                 */
/* L = fma(l_c, w_c, L), O[d] = fma(o_c[d], w_c, O[d]); out[d] = half(O/L).  */
/* Scores as orc_attention_ref.                                              */
/* ------------------------------------------------------------------------ */
void orc_attention_splitk(const uint16_t* q, const uint16_t* K, const uint16_t* V, int nh, int nkv, int hd, int seq,
                          uint16_t* out16, float* out32) {
    enum { CH = 64 };
    const float inv_sqrt = (float)(1.0 / sqrt((double)hd));
    const int nc = (seq + CH - 1) / CH;
    float* m = (float*)malloc(sizeof(float) * (size_t)nc);
    float* l = (float*)malloc(sizeof(float) * (size_t)nc);
    float* o = (float*)malloc(sizeof(float) * (size_t)nc * (size_t)hd);
    if (!m || !l || !o) {
        free(m), free(l), free(o);
        return;
    }
    for (int h = 0; h < nh; ++h) {
        const int g = h * nkv / nh;
        float M = -INFINITY;
        for (int c = 0; c < nc; ++c) {
            float sc[CH], e[CH], t[CH], u[CH];
            const int s0 = c * CH;
            const int n = seq - s0 < CH ? seq - s0 : CH;
            float mc = -INFINITY;
            for (int i = 0; i < n; ++i) {
                sc[i] = orc_score(q + (size_t)h * hd, K + ((size_t)(s0 + i) * nkv + g) * hd, hd, inv_sqrt);
                if (sc[i] > mc) mc = sc[i];
            }
            for (int i = 0; i < CH; ++i) e[i] = i < n ? orc_expf(sc[i] - mc) : 0.f;
            for (int d = 0; d < hd; ++d) {
                float acc = 0.f;
                for (int i = 0; i < n; ++i)
                    acc = fmaf(e[i], orc_half_to_float(V[((size_t)(s0 + i) * nkv + g) * hd + d]), acc);
                o[(size_t)c * hd + d] = acc;
            }
            memcpy(t, e, sizeof t);
            for (int w = CH / 2; w > 0; w >>= 1) {
                for (int i = 0; i < CH; ++i) u[i] = t[i] + t[i ^ w];
                memcpy(t, u, sizeof t);
            }
            m[c] = mc;
            l[c] = t[0];
            if (mc > M) M = mc;
        }
        float L = 0.f;
        for (int c = 0; c < nc; ++c) L = fmaf(l[c], orc_expf(m[c] - M), L);
        for (int d = 0; d < hd; ++d) {
            float O = 0.f;
            for (int c = 0; c < nc; ++c) O = fmaf(o[(size_t)c * hd + d], orc_expf(m[c] - M), O);
            const float r = O / L;
            if (out32) out32[(size_t)h * hd + d] = r;
            if (out16) out16[(size_t)h * hd + d] = orc_float_to_half(r);
        }
    }
    free(m), free(l), free(o);
}

/* ------------------------------------------------------------------------ */
/* BitNet absmean ternary quantizer: include/ter/bitnet.hpp:11-28.           */
/* ------------------------------------------------------------------------ */
float orc_quantize_bitnet(const float* in, size_t n, int8_t* out) {
    if (n == 0) return 0.0f;
    double sum_abs = 0.0;
    for (size_t i = 0; i < n; ++i) sum_abs += fabs((double)in[i]);
    const double scale = sum_abs / (double)n;
    if (scale == 0.0) {
        for (size_t i = 0; i < n; ++i) out[i] = 0;
        return 0.0f;
    }
    for (size_t i = 0; i < n; ++i) {
        const double q = (double)in[i] / scale;
        long r = lround(q);
        if (r > 1) r = 1;
        if (r < -1) r = -1;
        out[i] = (int8_t)r;
    }
    return (float)scale;
}

/* ------------------------------------------------------------------------ */
/* Format-B n-trit quantizer (TritTensor payload): src/numfmt/quantize.cpp:7-41 */
/* scale = max|x| / ((3^n - 1)/2); payload = clamp(lround(x / scale)).       */
/* Returns the scale (0 for an all-zero tensor; payload then all zero).      */
/* ------------------------------------------------------------------------ */
float orc_quantize_nt(const float* data, size_t n, int n_trits, int32_t* payload) {
    int64_t mti = 1;
    for (int i = 0; i < n_trits; ++i) mti *= 3;
    mti = (mti - 1) / 2;
    float max_abs = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        const float a = fabsf(data[i]);
        if (a > max_abs) max_abs = a;
    }
    if (max_abs == 0.0f) {
        memset(payload, 0, n * sizeof(int32_t));
        return 0.0f;
    }
    const float scale = max_abs / (float)mti;
    for (size_t i = 0; i < n; ++i) {
        const float q = data[i] / scale;
        int64_t r = (int64_t)lroundf(q);
        if (r > mti) r = mti;
        if (r < -mti) r = -mti;
        payload[i] = (int32_t)r;
    }
    return scale;
}

/* ------------------------------------------------------------------------ */
/* microsoft/BitNet i2_s decode: vendor/ntransformer/core/dequant.cpp:114-145 */
/* 128-element blocks of 32 bytes; byte p holds positions p+32g at shift     */
/* 6-2g; code map 0->-1, 1->0, 2->+1, 3->0; fp32 scale right after the codes. */
/* ------------------------------------------------------------------------ */
void orc_dequant_i2s(const uint8_t* src, size_t n_elems, float* out) {
    static const float LUT[4] = {-1.0f, 0.0f, +1.0f, 0.0f};
    float i2_scale = 1.0f;
    memcpy(&i2_scale, src + n_elems / 4, sizeof(float));
    const size_t n_blocks = n_elems / 128;
    for (size_t blk = 0; blk < n_blocks; ++blk) {
        const uint8_t* bb = src + blk * 32;
        for (int p = 0; p < 32; ++p) {
            const unsigned v = bb[p];
            for (int g = 0; g < 4; ++g)
                out[blk * 128 + (size_t)g * 32 + (size_t)p] = LUT[(v >> (6 - 2 * g)) & 3u] * i2_scale;
        }
    }
    for (size_t i = n_blocks * 128; i < n_elems; ++i) out[i] = 0.0f;
}

/* ------------------------------------------------------------------------ */
/* i2_s -> v11 repack: tools/convert_bitnet_to_packed.py:85-157.              */
/* The GGUF tensor is (N, K) row-major (each row one output column's         */
/* K-vector); microsoft codes are remapped with [2,0,1,0] to the ter code    */
/* map, then packed to v11 (out[j_byte*K + k], low bits = first column).     */
/* ------------------------------------------------------------------------ */
int orc_i2s_to_v11(const uint8_t* raw, int K, int N, uint8_t* out) {
    if (K <= 0 || N <= 0 || (K % 4) != 0 || (N % 4) != 0) return -5;
    const size_t total = (size_t)N * (size_t)K;
    if (total % 128 != 0) return -5;
    static const uint8_t remap[4] = {2, 0, 1, 0};
    memset(out, 0, total / 4);
    for (size_t e = 0; e < total; ++e) {
        const size_t blk = e / 128, pos = e % 128;
        const size_t g = pos / 32, p = pos % 32;
        const unsigned code = (raw[blk * 32 + p] >> (6 - 2 * g)) & 3u;
        const unsigned ours = remap[code];
        const size_t n = e / (size_t)K, k = e % (size_t)K;
        out[(n / 4) * (size_t)K + k] |= (uint8_t)(ours << (2 * (n % 4)));
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Reference TVMAC accounting of mm_row: src/tx/forward.cpp:349-350.         */
/* ------------------------------------------------------------------------ */
uint64_t orc_mm_row_tvmac(int K, int N) { return (uint64_t)((K + 26) / 27) * (uint64_t)N; }
