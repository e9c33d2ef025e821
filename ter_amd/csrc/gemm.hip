// gemm.hip -- M > 1 packed-trit GEMM on gfx950 MFMA (v_mfma_i32_16x16x64_i8).
//
// Replaces the reference's batched kernels (mm_packed_batched,
// cuda/ter_cuda_packed_batched.cu:26-83; mm_bitnet_addonly_batched_k<M>,
// cuda/ter_cuda_addonly_batched.cu:31-124; the wmma s4 mm_int4_tc*).
// Semantics: acc[m][j] = sum_k X[m][k] w[k][j] (exact int32) and
// y[m][j] = float(acc[m][j]) * (x_scale[m] * w_scale)
// (cuda/ter_cuda_addonly_batched.cu:117-123).
//
// Input is the same T16 tile stream as the GEMV (common.h).  A workgroup of
// 4 waves owns 4 column strips (64 columns) and all M rows; for every
// 256-row unit it stages X[0:M, unit] (int8) in LDS once for the 4 waves,
// each wave gathers its strip's packed weights straight into the MFMA B
// operand layout (lane = column j + 16 * k-group g; one dword = 16 trits of
// column j), expands the 2-bit u = w + 1 codes to int8 with 7 bit operations
// per 16 trits, and runs one MFMA per 16-row block and 64-row slab.  The u
// encoding adds sum_k X[m][k] to every output; it is subtracted in the
// epilogue from row sums gathered while staging X.
//
// MFMA operand layout used (lane l, 16 bytes per lane): A lane l holds row
// l % 16, B lane l holds column l % 16, both for the 16 logical k values
// 16 * (l / 16) .. +15 of the 64-row slab (any lane/k bijection shared by A
// and B gives the same product); D lane l, element e holds row
// 4 * (l / 16) + e, column l % 16.
#include "common.h"

namespace terhip {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int row_sum16(int v) {
    v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);
    v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);
    v += __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true);
    v += __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true);
    return v;
}

__device__ __forceinline__ int sum_bytes(const u32x4& v) {
    int s = __builtin_amdgcn_sdot4((int)v.x, 0x01010101, 0, false);
    s = __builtin_amdgcn_sdot4((int)v.y, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4((int)v.z, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4((int)v.w, 0x01010101, s, false);
    return s;
}

constexpr int kLdRow = kUnitK + 16;  // padded LDS row of staged X (bytes)

template <int MB>
__global__ __launch_bounds__(kThreads) void gemm_t16_kernel(
    const uint8_t* __restrict__ w, int K, int N, int Ku, int n_strips,
    const int8_t* __restrict__ xq, const float* __restrict__ xs, int M, float w_scale,
    float* __restrict__ y, int32_t* __restrict__ acc) {
#pragma clang fp contract(off)
    constexpr int ROWS = MB * 16;
    __shared__ __align__(16) int8_t xl[ROWS * kLdRow];
    __shared__ int rsum[ROWS];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int st = blockIdx.x * kWaves + wave;
    const bool active = st < n_strips;
    const int g = lane >> 4, j = lane & 15;
    const bool xvec = ((reinterpret_cast<uintptr_t>(xq) & 15u) == 0) && ((K & 15) == 0);

    i32x4 C[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) C[mb] = i32x4{0, 0, 0, 0};
    int rs[MB];
#pragma unroll
    for (int p = 0; p < MB; ++p) rs[p] = 0;

    const uint8_t* wb = w + (size_t)(active ? st : 0) * Ku * kTileBytes + (j >> 2) * 256 + g * 16 +
                        (j & 3) * 4;
    for (int u = 0; u < Ku; ++u) {
        unsigned wd[4] = {0u, 0u, 0u, 0u};
        if (active) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                wd[ks] = __builtin_nontemporal_load(
                    reinterpret_cast<const unsigned*>(wb + (size_t)u * kTileBytes + ks * 64));
        }
        __syncthreads();  // previous unit's LDS reads are done
#pragma unroll
        for (int p = 0; p < MB; ++p) {
            const int row = p * 16 + (tid >> 4);
            const int ch = tid & 15;
            const int k = u * kUnitK + ch * 16;
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (row < M) {
                const int8_t* src = xq + (size_t)row * K + k;
                if (xvec && k + 16 <= K) {
                    v = *reinterpret_cast<const u32x4*>(src);
                } else {
                    unsigned wdd[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        unsigned a = 0;
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            const int kk = k + 4 * i + b;
                            a |= (kk < K ? (unsigned)(uint8_t)src[4 * i + b] : 0u) << (8 * b);
                        }
                        wdd[i] = a;
                    }
                    v = u32x4{wdd[0], wdd[1], wdd[2], wdd[3]};
                }
            }
            *reinterpret_cast<u32x4*>(xl + row * kLdRow + ch * 16) = v;
            const int s = row_sum16(sum_bytes(v));
            if (ch == 0) rs[p] += s;
        }
        __syncthreads();
        if (active) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const unsigned d = wd[ks];
                const i32x4 B = i32x4{(int)(d & 0x03030303u), (int)((d >> 2) & 0x03030303u),
                                      (int)((d >> 4) & 0x03030303u), (int)((d >> 6) & 0x03030303u)};
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    const i32x4 A =
                        *reinterpret_cast<const i32x4*>(xl + (mb * 16 + j) * kLdRow + ks * 64 + g * 16);
                    C[mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, C[mb], 0, 0, 0);
                }
            }
        }
    }
#pragma unroll
    for (int p = 0; p < MB; ++p)
        if ((tid & 15) == 0) rsum[p * 16 + (tid >> 4)] = rs[p];
    __syncthreads();
    if (!active) return;
    const int col = st * kStripCols + j;
    if (col >= N) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int row = mb * 16 + g * 4 + e;
            if (row < M) {
                const int val = C[mb][e] - rsum[row];
                if (acc) acc[(size_t)row * N + col] = val;
                if (y) y[(size_t)row * N + col] = (float)val * (xs[row] * w_scale);
            }
        }
    }
}

template <int MB>
hipError_t launch_mb(const uint8_t* w, int K, int N, const int8_t* xq, const float* xs, int M,
                     float w_scale, float* y, int32_t* acc, hipStream_t st) {
    const int Ku = units_of(K), ns = strips_of(N);
    const int grid = (ns + kWaves - 1) / kWaves;
    hipLaunchKernelGGL(gemm_t16_kernel<MB>, dim3(grid), dim3(kThreads), 0, st, w, K, N, Ku, ns, xq, xs,
                       M, w_scale, y, acc);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(const uint8_t* w, int K, int N, const int8_t* xq, const float* xs, int M,
                       float w_scale, float* y, int32_t* acc, hipStream_t st) {
    if (M <= 16) return launch_mb<1>(w, K, N, xq, xs, M, w_scale, y, acc, st);
    if (M <= 32) return launch_mb<2>(w, K, N, xq, xs, M, w_scale, y, acc, st);
    if (M <= 64) return launch_mb<4>(w, K, N, xq, xs, M, w_scale, y, acc, st);
    if (M <= 128) return launch_mb<8>(w, K, N, xq, xs, M, w_scale, y, acc, st);
    return launch_mb<16>(w, K, N, xq, xs, M, w_scale, y, acc, st);
}

}  // namespace terhip
