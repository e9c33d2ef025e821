// pack.hip -- device repack between the reference v11 layout and T16, the
// synthetic-data generators used by the benchmark, and the per-row int8
// activation quantizer of the batched path.
//
// v11 (reference wire format, tools/convert_llama_to_packed.py:128-140 and
// the decoder in cuda/ter_cuda_forward_packed.cu:355-374): byte
// W_col[j_byte * K + k] holds columns 4 j_byte + s at bits 2s..2s+1 with the
// code map of include/ter/pack.hpp:8-21 (00 = 0, 01 = +1, 10 = -1, 11 = 0).
// T16 is described in common.h.
#include "common.h"

namespace terhip {
namespace {

// 2-bit v11 code -> T16 field value u = w + 1 (code 11 decodes as 0 -> u = 1).
__device__ __forceinline__ unsigned code_to_u(unsigned c) {
    c &= 3u;
    return c == 1u ? 2u : (c == 2u ? 0u : 1u);
}

__device__ __forceinline__ unsigned u_to_code(unsigned u) {
    return u == 2u ? 1u : (u == 0u ? 2u : 0u);
}

// One thread per T16 dword: 16 trits of one column over 16 consecutive rows.
__global__ void pack_v11_kernel(const uint8_t* __restrict__ v11, uint32_t* __restrict__ t16, int K,
                                int N, int Ku, long long n_dwords) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_dwords) return;
    const int j = (int)(i & 3);
    const int lane = (int)((i >> 2) & 63);
    const long long tile = i >> 8;
    const int s = (int)(tile / Ku);
    const int u = (int)(tile - (long long)s * Ku);
    const int r = lane >> 4, q = lane & 15;
    const int n = s * kStripCols + r * 4 + j;
    const int k0 = u * kUnitK + q * 16;
    unsigned out = 0;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int k = k0 + e;
        unsigned uval = 1u;
        if (n < N && k < K) uval = code_to_u(v11[(long long)(n >> 2) * K + k] >> (2 * (n & 3)));
        const int f = e >> 2, b = e & 3;
        out |= uval << (8 * b + 2 * f);
    }
    t16[i] = out;
}

// One thread per T16 dword, from microsoft/BitNet i2_s bytes
// (tools/convert_bitnet_to_packed.py:85-157, vendor/ntransformer/core/dequant.cpp:114-145):
// the (N, K) tensor row-major (element e = n K + k) in blocks of 128 elements
// per 32 bytes; byte p of a block holds positions p, p+32, p+64, p+96 at
// shifts 6, 4, 2, 0; codes 0 -> -1, 1 -> 0, 2 -> +1, 3 -> 0, i.e. u = w + 1 =
// {0, 1, 2, 1}.  Padding rows / columns hold u = 1.
__global__ void pack_i2s_kernel(const uint8_t* __restrict__ raw, uint32_t* __restrict__ t16, int K, int N,
                                int Ku, long long n_dwords) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_dwords) return;
    const int j = (int)(i & 3);
    const int lane = (int)((i >> 2) & 63);
    const long long tile = i >> 8;
    const int s = (int)(tile / Ku);
    const int u = (int)(tile - (long long)s * Ku);
    const int r = lane >> 4, q = lane & 15;
    const int n = s * kStripCols + r * 4 + j;
    const int k0 = u * kUnitK + q * 16;
    unsigned out = 0;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int k = k0 + e;
        unsigned uval = 1u;
        if (n < N && k < K) {
            const long long el = (long long)n * K + k;
            const long long blk = el >> 7;
            const int pos = (int)(el & 127);
            const unsigned code = (raw[blk * 32 + (pos & 31)] >> (6 - 2 * (pos >> 5))) & 3u;
            uval = code == 3u ? 1u : code;  // w + 1 for w = {-1, 0, +1, 0}
        }
        const int f = e >> 2, b = e & 3;
        out |= uval << (8 * b + 2 * f);
    }
    t16[i] = out;
}

// One thread per v11 byte.
__global__ void unpack_v11_kernel(const uint32_t* __restrict__ t16, uint8_t* __restrict__ v11, int K,
                                  int N, int Ku) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)(N / 4) * K;
    if (i >= total) return;
    const int jb = (int)(i / K);
    const int k = (int)(i - (long long)jb * K);
    const int u = k / kUnitK;
    const int q = (k % kUnitK) / 16;
    const int e = k & 15;
    const int f = e >> 2, b = e & 3;
    unsigned byte = 0;
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
        const int n = jb * 4 + sub;
        const int s = n / kStripCols, r = (n % kStripCols) / 4, j = n & 3;
        const long long dw = (((long long)s * Ku + u) * 64 + (r * 16 + q)) * 4 + j;
        const unsigned uval = (t16[dw] >> (8 * b + 2 * f)) & 3u;
        byte |= u_to_code(uval) << (2 * sub);
    }
    v11[i] = (uint8_t)byte;
}

__device__ __forceinline__ uint64_t splitmix(uint64_t seed, uint64_t idx) {
    uint64_t z = seed + (idx + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// One thread per v11 byte: 4 trits of columns 4 jb .. 4 jb + 3 at row k.
__global__ void synth_v11_kernel(uint8_t* __restrict__ v11, int K, int N, uint64_t seed, uint32_t t0,
                                 uint32_t t1) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)(N / 4) * K;
    if (i >= total) return;
    const int jb = (int)(i / K);
    const int k = (int)(i - (long long)jb * K);
    unsigned byte = 0;
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
        const uint64_t idx = (uint64_t)k * (uint64_t)N + (uint64_t)(jb * 4 + sub);
        const uint32_t uu = (uint32_t)(splitmix(seed, idx) >> 32);
        const unsigned code = uu < t0 ? 0u : (uu < t1 ? 1u : 2u);
        byte |= code << (2 * sub);
    }
    v11[i] = (uint8_t)byte;
}

__global__ void synth_i8_kernel(int8_t* __restrict__ x, long long n, uint64_t seed, int lo, int hi) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t uu = splitmix(seed, (uint64_t)i) >> 32;
    const uint64_t span = (uint64_t)(hi - lo + 1);
    x[i] = (int8_t)(lo + (int)((uu * span) >> 32));
}

// One workgroup (256 threads) per row: quant_int8_k steps
// (cuda/ter_cuda_forward_packed.cu:40-62) on row m of x[M][K].
__global__ __launch_bounds__(256) void quant_rows_kernel(const float* __restrict__ x, int K,
                                                         int8_t* __restrict__ q,
                                                         float* __restrict__ scale_out) {
#pragma clang fp contract(off)
    __shared__ float red[4];
    const int m = blockIdx.x;
    const float* xr = x + (long long)m * K;
    float mx = 0.f;
    for (int k = threadIdx.x; k < K; k += 256) mx = fmaxf(mx, fabsf(xr[k]));
    mx = fmaxf(mx, __shfl_xor(mx, 1));
    mx = fmaxf(mx, __shfl_xor(mx, 2));
    mx = fmaxf(mx, __shfl_xor(mx, 4));
    mx = fmaxf(mx, __shfl_xor(mx, 8));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float amax = mx + 1e-9f;
    const float scale = 127.0f / amax;
    if (threadIdx.x == 0) scale_out[m] = 1.0f / scale;
    int8_t* qr = q + (long long)m * K;
    for (int k = threadIdx.x; k < K; k += 256) {
        const float v = xr[k] * scale;
        int qi = (int)__builtin_rintf(v);
        qi = qi > 127 ? 127 : (qi < -128 ? -128 : qi);
        qr[k] = (int8_t)qi;
    }
}

// One workgroup (256 threads) per row: the fused RMSNorm + int8 quantizer
// (rmsnorm_quant_f32_in_k / rmsnorm_quant_fp16_in_k,
// cuda/ter_cuda_forward_bitnet.cu:64-146) on row m of x[M][K]:
// per-thread strided partial sums of squares with fused multiply-adds (the
// reference build contracts `local_sum += v * v`), the reference's reduction
// tree, rms_inv = 1 / sqrt(ss / K + eps) correctly rounded (the reference's
// rsqrtf is an approximation), n = (x * rms_inv) * gamma, then quant_int8_k.
// X_RELU2_RMS is relu2_mul_rmsnorm_quant_k (ibid.:258-309, one 1024-thread
// block per row): x = relu^2(gate) * up and its 1024-strided sum order.
__global__ __launch_bounds__(256) void rmsnorm_quant_rows_kernel(const void* __restrict__ x,
                                                                 const uint16_t* __restrict__ up, int kind,
                                                                 const uint16_t* __restrict__ gamma, float eps,
                                                                 int K, int8_t* __restrict__ q,
                                                                 float* __restrict__ scale_out) {
#pragma clang fp contract(off)
    __shared__ float red[256];
    const int m = blockIdx.x, t = threadIdx.x;
    const long long row0 = (long long)m * K;
    auto xv = [&](int k) -> float {
        if (kind == TER_HIP_X_F32_RMS) return static_cast<const float*>(x)[row0 + k];
        const float h = half_bits_to_float(static_cast<const uint16_t*>(x)[row0 + k]);
        return kind == TER_HIP_X_F16_RMS ? h : relu2_mul(h, half_bits_to_float(up[row0 + k]));
    };
    float ss;
    if (kind == TER_HIP_X_RELU2_RMS) {
        ss = relu2_sum_sq_1024(static_cast<const uint16_t*>(x) + row0, up + row0, K, red);
    } else {
        float part = 0.f;
        for (int k = t; k < K; k += 256) {
            const float v = xv(k);
            part = __builtin_fmaf(v, v, part);
        }
        ss = tree_sum256(part, red);
    }
    const float rms_inv = 1.0f / __builtin_sqrtf(ss / (float)K + eps);
    float mx = 0.f;
    for (int k = t; k < K; k += 256) {
        const float n = (xv(k) * rms_inv) * half_bits_to_float(gamma[k]);
        mx = fmaxf(mx, fabsf(n));
    }
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) mx = fmaxf(mx, __shfl_xor(mx, s));
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float amax = mx + 1e-9f;
    const float scale = 127.0f / amax;
    if (t == 0) scale_out[m] = 1.0f / scale;
    int8_t* qr = q + row0;
    for (int k = t; k < K; k += 256) {
        const float n = (xv(k) * rms_inv) * half_bits_to_float(gamma[k]);
        int qi = (int)__builtin_rintf(n * scale);
        qi = qi > 127 ? 127 : (qi < -128 ? -128 : qi);
        qr[k] = (int8_t)qi;
    }
}

inline unsigned grid_of(long long n, int block) { return (unsigned)((n + block - 1) / block); }

}  // namespace

hipError_t launch_pack_v11(const uint8_t* v11, uint8_t* t16, int K, int N, hipStream_t st) {
    const int Ku = units_of(K);
    const long long n_dwords = (long long)strips_of(N) * Ku * (kTileBytes / 4);
    hipLaunchKernelGGL(pack_v11_kernel, dim3(grid_of(n_dwords, 256)), dim3(256), 0, st, v11,
                       reinterpret_cast<uint32_t*>(t16), K, N, Ku, n_dwords);
    return hipGetLastError();
}

hipError_t launch_pack_i2s(const uint8_t* raw, uint8_t* t16, int K, int N, hipStream_t st) {
    const int Ku = units_of(K);
    const long long n_dwords = (long long)strips_of(N) * Ku * (kTileBytes / 4);
    hipLaunchKernelGGL(pack_i2s_kernel, dim3(grid_of(n_dwords, 256)), dim3(256), 0, st, raw,
                       reinterpret_cast<uint32_t*>(t16), K, N, Ku, n_dwords);
    return hipGetLastError();
}

hipError_t launch_unpack_v11(const uint8_t* t16, uint8_t* v11, int K, int N, hipStream_t st) {
    const long long total = (long long)(N / 4) * K;
    hipLaunchKernelGGL(unpack_v11_kernel, dim3(grid_of(total, 256)), dim3(256), 0, st,
                       reinterpret_cast<const uint32_t*>(t16), v11, K, N, units_of(K));
    return hipGetLastError();
}

hipError_t launch_synth_v11(uint8_t* v11, int K, int N, uint64_t seed, uint32_t t0, uint32_t t1,
                            hipStream_t st) {
    const long long total = (long long)(N / 4) * K;
    hipLaunchKernelGGL(synth_v11_kernel, dim3(grid_of(total, 256)), dim3(256), 0, st, v11, K, N, seed,
                       t0, t1);
    return hipGetLastError();
}

hipError_t launch_synth_i8(int8_t* x, long long n, uint64_t seed, int lo, int hi, hipStream_t st) {
    hipLaunchKernelGGL(synth_i8_kernel, dim3(grid_of(n, 256)), dim3(256), 0, st, x, n, seed, lo, hi);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_quant_rows(const void* x, const uint16_t* up, int kind, const uint16_t* gamma, float eps,
                                     int M, int K,
                                     int8_t* q, float* s, hipStream_t st) {
    hipLaunchKernelGGL(rmsnorm_quant_rows_kernel, dim3(M), dim3(256), 0, st, x, up, kind, gamma, eps, K, q, s);
    return hipGetLastError();
}

hipError_t launch_quant_rows(const float* x, int M, int K, int8_t* q, float* s, hipStream_t st) {
    hipLaunchKernelGGL(quant_rows_kernel, dim3(M), dim3(256), 0, st, x, K, q, s);
    return hipGetLastError();
}

}  // namespace terhip
