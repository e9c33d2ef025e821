// blocked.hip -- the per-block branch of mm_row on the GPU.
//
// src/tx/forward.cpp:308-330: when the weight TritTensor carries
// block_scales, mm_row accumulates in double,
//   facc[j] += double(x[k]) * double(W[k*N + j]) * double(block_scales[(k*N + j) / bs])
// over k in increasing order (x[k] == 0 skipped), and writes
//   out[j] = float(facc[j] * double(Xt.scale)).
// The weights here are the packed trits t with magnitude m (W = m * t).
// Each term is exact in double when |x| * m < 2^29 (the boundary checks it:
// 28 bits of integer product times the 24-bit scale mantissa), so the only
// roundings are the additions -- done here in the reference's order, one
// thread per column, k ascending -- and the final multiply and conversion.
// Whether the compiler fuses the multiply into the add makes no difference
// to an exact product, so the result is the reference's bit for bit.
#include "common.h"

namespace terhip {
namespace {

constexpr int kBlkThreads = 256;

__global__ __launch_bounds__(kBlkThreads) void mm_row_blocked_kernel(const uint8_t* __restrict__ w, int K, int N,
                                                                     int Ku, int mag, const int16_t* __restrict__ x,
                                                                     const float* __restrict__ bsc, long long bs,
                                                                     float xs, float* __restrict__ out) {
#pragma clang fp contract(off)
    const int j = blockIdx.x * kBlkThreads + threadIdx.x;
    if (j >= N) return;
    const int s = j / kStripCols, r = (j % kStripCols) / 4, d = j % 4;
    const TER_GLOBAL unsigned* wd = gptr(reinterpret_cast<const unsigned*>(w));
    double facc = 0.0;
    for (int k0 = 0; k0 < K; k0 += 16) {
        // the dword of column j over rows k0 .. k0 + 15 (T16 layout, common.h)
        const long long lane = (long long)r * 16 + (k0 % kUnitK) / 16;
        const unsigned dw = wd[(((long long)s * Ku + k0 / kUnitK) * 64 + lane) * 4 + d];
        const int e_end = K - k0 < 16 ? K - k0 : 16;
        for (int e = 0; e < e_end; ++e) {
            const int xv = gptr(x)[k0 + e];
            if (xv == 0) continue;  // the reference's zero skip (forward.cpp:314)
            const int t = (int)((dw >> (8 * (e & 3) + 2 * (e >> 2))) & 3u) - 1;
            const long long flat = (long long)(k0 + e) * N + j;
            const double term = ((double)xv * (double)(t * mag)) * (double)gptr(bsc)[flat / bs];
            facc = facc + term;
        }
    }
    gptr(out)[j] = (float)(facc * (double)xs);
}

}  // namespace

hipError_t launch_mm_row_blocked(const uint8_t* w, int K, int N, int mag, const int16_t* x, const float* bsc,
                                 long long bs, float xs, float* out, hipStream_t st) {
    hipLaunchKernelGGL(mm_row_blocked_kernel, dim3((N + kBlkThreads - 1) / kBlkThreads), dim3(kBlkThreads), 0, st, w,
                       K, N, units_of(K), mag, x, bsc, bs, xs, out);
    return hipGetLastError();
}

}  // namespace terhip
