// probe.hip -- measurement utilities for the benchmark's floors.
//
//   noop_kernel        one wave that does nothing: the launch floor.
//   read_probe_kernel  a pure streaming read of a byte range with the GEMV's
//                      partition (equal contiguous ranges per workgroup,
//                      neighbouring ranges on one XCD, 4 waves per workgroup
//                      each streaming an equal contiguous piece with
//                      nontemporal buffer_load_dwordx4, two batches in
//                      flight): the ceiling the GEMV's streaming can reach
//                      on the same bytes.  Each wave folds what it read into
//                      one word of `sink` so the loads cannot be dropped.
#include "common.h"

namespace terhip {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ void noop_kernel() {}

constexpr int kProbeBatch = 5;

__global__ __launch_bounds__(kGemvThreads) void read_probe_kernel(const uint8_t* buf, long long tiles, int n_wg,
                                                                  unsigned* sink) {
    int g = blockIdx.x;
    if ((n_wg & 7) == 0) g = (g & 7) * (n_wg >> 3) + (g >> 3);
    const long long t0 = tiles * g / n_wg, t1 = tiles * (g + 1) / n_wg;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const long long a = t0 + (t1 - t0) * wave / kGemvWaves, b = t0 + (t1 - t0) * (wave + 1) / kGemvWaves;
    const int n = (int)(b - a);
    const int voff = (threadIdx.x & 63) * 16;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(buf + a * kTileBytes), 0, n * kTileBytes, 0x00020000);
    unsigned acc = 0;
    u32x4 wa[kProbeBatch], wb[kProbeBatch];
#pragma unroll
    for (int i = 0; i < kProbeBatch; ++i)
        wa[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + i * kTileBytes, 0, 2);
    for (int i0 = 0; i0 < n; i0 += 2 * kProbeBatch) {
#pragma unroll
        for (int i = 0; i < kProbeBatch; ++i)
            wb[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + (i0 + kProbeBatch + i) * kTileBytes, 0, 2);
#pragma unroll
        for (int i = 0; i < kProbeBatch; ++i) acc ^= wa[i].x ^ wa[i].y ^ wa[i].z ^ wa[i].w;
#pragma unroll
        for (int i = 0; i < kProbeBatch; ++i)
            wa[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + (i0 + 2 * kProbeBatch + i) * kTileBytes, 0, 2);
#pragma unroll
        for (int i = 0; i < kProbeBatch; ++i) acc ^= wb[i].x ^ wb[i].y ^ wb[i].z ^ wb[i].w;
    }
    acc = (unsigned)__builtin_amdgcn_readfirstlane((int)acc) ^ (unsigned)__shfl_xor((int)acc, 1);
    if ((threadIdx.x & 63) == 0) gptr(sink)[blockIdx.x * kGemvWaves + wave] = acc;
}

}  // namespace

hipError_t launch_noop(hipStream_t st) {
    hipLaunchKernelGGL(noop_kernel, dim3(1), dim3(64), 0, st);
    return hipGetLastError();
}

hipError_t launch_read_probe(const uint8_t* buf, long long tiles, int n_wg, unsigned* sink, hipStream_t st) {
    hipLaunchKernelGGL(read_probe_kernel, dim3(n_wg), dim3(kGemvThreads), 0, st, buf, tiles, n_wg, sink);
    return hipGetLastError();
}

}  // namespace terhip
