// gemv_x16.hip -- M = 1 packed-trit GEMV with int16 activations.
//
// The reference host forward quantizes every activation vector to 9 trits
// before mm_row (quantize(x_norm, {1, H}, 9), src/tx/forward.cpp:400): the
// payload holds integers up to +-9841 (max_trit_int(9),
// src/numfmt/quantize.cpp:26-38), which do not fit the int8 lanes of
// v_dot4.  This kernel serves any int16 activation vector exactly: each
// value is split as x = 256 * hi + lo with hi = x >> 8 in [-128, 127]
// (signed, v_dot4c_i32_i8) and lo = x & 255 in [0, 255] (unsigned,
// v_dot4_u32_u8 against the unsigned trit codes u = w + 1).  Both products
// are exact, and the column sum is formed as
//   sum_k x_k w_kj = 256 * sum_k hi_k u_kj + sum_k lo_k u_kj - sum_k x_k
// in wrapping 32-bit arithmetic; the true result fits int32 (|x| <= 2^15,
// K <= 2^15), so it comes out exact.  The epilogue is the other kernels'
// (emit_out): y = float(m * acc) * (x_scale * w_scale).
//
// Work layout (the strip mode of gemv.hip, one GEMV): workgroup g owns whole
// column strips; its 4 waves split each strip's 256-row units, keep their
// partial column sums in LDS, and after a barrier one wave per strip adds the
// four partials and writes the outputs.  No fix-up slots, no atomics.
#include "common.h"

namespace terhip {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kX16Batch = 4;  // tiles per batch, two batches in flight per wave

__device__ __forceinline__ unsigned row_sum16_u(unsigned v) {
    v += (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true);   // quad_perm [1,0,3,2]
    v += (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true);   // quad_perm [2,3,0,1]
    v += (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, true);  // row_half_mirror
    v += (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, true);  // row_mirror
    return v;
}

// 16 int16 activations at k, read through a buffer resource that covers
// the K elements of X (elements past K read zeros), split into the hi plane
// (signed bytes x >> 8) and the lo plane (bytes x & 255); returns their sum.
// kVec (X 16-byte aligned, K a multiple of 16): two 16-byte loads, each
// chunk wholly inside X or wholly past it.  Otherwise 16 two-byte loads.
// Either way every load is unconditional: no branch joins loaded values
// (at such a join the compiler waited for every load in flight, the weight
// batch issued before the staging included).
template <bool kVec>
__device__ __forceinline__ int split16(__amdgpu_buffer_rsrc_t xr, int k, u32x4& hi, u32x4& lo) {
    int v[16];
    if constexpr (kVec) {
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(xr, 2 * k, 0, 0);
        const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(xr, 2 * k + 16, 0, 0);
        const unsigned w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[2 * i] = (int)(int16_t)(w[i] & 0xFFFFu);
            v[2 * i + 1] = (int)(int16_t)(w[i] >> 16);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            v[i] = (int)(int16_t)__builtin_amdgcn_raw_buffer_load_b16(xr, 2 * (k + i), 0, 0);
    }
    unsigned h[4], l[4];
    int sum = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        h[d] = l[d] = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int e = v[4 * d + b];
            h[d] |= ((unsigned)(e >> 8) & 0xFFu) << (8 * b);
            l[d] |= ((unsigned)e & 0xFFu) << (8 * b);
            sum += e;
        }
    }
    hi = u32x4{h[0], h[1], h[2], h[3]};
    lo = u32x4{l[0], l[1], l[2], l[3]};
    return sum;
}

// One tile (16 bytes of this lane): 4 columns x 16 rows against both planes.
__device__ __forceinline__ void dot_tile_x16(const u32x4& w, const u32x4& hi, const u32x4& lo, int (&h1)[4],
                                             int (&h4)[4], unsigned (&l1)[4], unsigned (&l4)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned dw = w[j];
        const unsigned d4 = dw >> 4;
        const unsigned f0 = dw & 0x03030303u, f1 = dw & 0x0C0C0C0Cu, f2 = d4 & 0x03030303u, f3 = d4 & 0x0C0C0C0Cu;
        h1[j] = __builtin_amdgcn_sdot4((int)hi.x, (int)f0, h1[j], false);
        h4[j] = __builtin_amdgcn_sdot4((int)hi.y, (int)f1, h4[j], false);
        h1[j] = __builtin_amdgcn_sdot4((int)hi.z, (int)f2, h1[j], false);
        h4[j] = __builtin_amdgcn_sdot4((int)hi.w, (int)f3, h4[j], false);
        l1[j] = __builtin_amdgcn_udot4(lo.x, f0, l1[j], false);
        l4[j] = __builtin_amdgcn_udot4(lo.y, f1, l4[j], false);
        l1[j] = __builtin_amdgcn_udot4(lo.z, f2, l1[j], false);
        l4[j] = __builtin_amdgcn_udot4(lo.w, f3, l4[j], false);
    }
}

template <bool kVec>
__global__ __launch_bounds__(kGemvThreads) void gemv_x16_kernel(GemvDesc d, int n_wg, int part_off) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    int g = blockIdx.x;
    if ((n_wg & 7) == 0) g = (g & 7) * (n_wg >> 3) + (g >> 3);  // neighbouring strips on one XCD
    const int s_begin = (int)((long long)d.n_strips * g / n_wg);
    const int s_end = (int)((long long)d.n_strips * (g + 1) / n_wg);
    if (s_begin >= s_end) return;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int voff = lane * 16;
    const int Ku = d.Ku;
    const int ns = s_end - s_begin;
    const int u0 = Ku * wave / kGemvWaves;
    const int nw = Ku * (wave + 1) / kGemvWaves - u0;  // units per strip of this wave
    const int n = nw * ns;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(d.w + (long long)s_begin * Ku * kTileBytes), 0, ns * Ku * kTileBytes, 0x00020000);
    // tile i of the wave's list: strip i / nw, unit u0 + i % nw; past n an
    // offset beyond the resource, which reads zeros
    int jl = 0, kl = 0;
    auto next_off = [&]() {
        const int off = jl < ns ? ((jl * Ku + u0 + kl) * kTileBytes) : 0x7FFFF000 - voff;
        if (++kl == nw) {
            kl = 0;
            ++jl;
        }
        return off;
    };
    auto load_b = [&](u32x4 (&w)[kX16Batch]) {
#pragma unroll
        for (int i = 0; i < kX16Batch; ++i) w[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + next_off(), 0, 2);
    };
    u32x4 wa[kX16Batch], wb[kX16Batch];
    if (nw > 0) load_b(wa);

    // Stage both planes (16-element chunks, 16 chunks per unit) and the
    // per-unit activation sums.
    int8_t* lds_hi = reinterpret_cast<int8_t*>(lds_raw);
    uint8_t* lds_lo = reinterpret_cast<uint8_t*>(lds_raw + Ku * kUnitK);
    int* usum = reinterpret_cast<int*>(lds_raw + 2 * Ku * kUnitK);
    int* part = reinterpret_cast<int*>(lds_raw + part_off);  // [strip][wave][16 columns]
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)d.x, 0, 2 * d.K, 0x00020000);
    const int nchunks = Ku * (kUnitK / 16);
    for (int c = tid; c < nchunks; c += kGemvThreads) {
        u32x4 hi, lo;
        const int sum = split16<kVec>(xr, c * 16, hi, lo);
        *reinterpret_cast<u32x4*>(lds_hi + c * 16) = hi;
        *reinterpret_cast<u32x4*>(lds_lo + c * 16) = lo;
        const unsigned us = row_sum16_u((unsigned)sum);
        if ((tid & 15) == 0) usum[c >> 4] = (int)us;
    }
    const float act = d.x_scale_dev ? *gptr(d.x_scale_dev) : d.x_scale;
    __syncthreads();
    const float s = act * d.w_scale;  // x_scale * w_scale (forward.cpp:342)

    const int q = lane & 15;
    const int pcol = (lane >> 4) * 4 + q;  // column within the strip of lanes q < 4
    if (nw == 0) {
        for (int j = 0; j < ns; ++j)
            if (q < 4) part[(j * kGemvWaves + wave) * 16 + pcol] = 0;
    } else {
        int h1[4] = {0, 0, 0, 0}, h4[4] = {0, 0, 0, 0};
        unsigned l1[4] = {0, 0, 0, 0}, l4[4] = {0, 0, 0, 0};
        unsigned corr = 0;
        int j = 0, k = 0;
        auto compute_b = [&](const u32x4 (&w)[kX16Batch], int i0) {
#pragma unroll
            for (int i = 0; i < kX16Batch; ++i) {
                if (i0 + i < n) {
                    const int u = u0 + k;
                    const u32x4 hv = *reinterpret_cast<const u32x4*>(lds_hi + u * kUnitK + q * 16);
                    const u32x4 lv = *reinterpret_cast<const u32x4*>(lds_lo + u * kUnitK + q * 16);
                    corr += (unsigned)usum[u];
                    dot_tile_x16(w[i], hv, lv, h1, h4, l1, l4);
                    if (++k == nw) {
                        unsigned v[4];
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            // fields f = 1, 3 were masked in place: their sums carry a factor 4
                            const unsigned hs = (unsigned)(h1[c] + (h4[c] >> 2));
                            const unsigned ls = l1[c] + (l4[c] >> 2);
                            v[c] = row_sum16_u(256u * hs + ls);
                            h1[c] = h4[c] = 0;
                            l1[c] = l4[c] = 0;
                        }
                        const unsigned vq = q == 0 ? v[0] : (q == 1 ? v[1] : (q == 2 ? v[2] : v[3]));
                        if (q < 4) part[(j * kGemvWaves + wave) * 16 + pcol] = (int)(vq - corr);
                        corr = 0;
                        k = 0;
                        ++j;
                    }
                }
            }
        };
        int i0 = 0;
        while (true) {
            load_b(wb);
            compute_b(wa, i0);
            i0 += kX16Batch;
            if (i0 >= n) break;
            load_b(wa);
            compute_b(wb, i0);
            i0 += kX16Batch;
            if (i0 >= n) break;
        }
    }
    __syncthreads();
    for (int j = wave; j < ns; j += kGemvWaves) {
        const int col = (s_begin + j) * kStripCols + lane;
        if (lane < 16 && col < d.N) {
            const int* pj = part + j * kGemvWaves * 16 + lane;
            emit_out(d, col, (int)((((unsigned)pj[0] + (unsigned)pj[16]) + (unsigned)pj[32]) + (unsigned)pj[48]), s);
        }
    }
}

}  // namespace

int gemv_x16_part_off(int K) { return (2 * units_of(K) * kUnitK + units_of(K) * 4 + 15) / 16 * 16; }

int gemv_x16_lds_bytes(int K, int strips_per_wg) {
    return gemv_x16_part_off(K) + strips_per_wg * kGemvWaves * kStripCols * 4;
}

hipError_t launch_gemv_x16(const GemvDesc& d, int n_wg, int lds_bytes, hipStream_t st) {
    if ((reinterpret_cast<uintptr_t>(d.x) & 15u) == 0 && d.K % 16 == 0)
        hipLaunchKernelGGL(gemv_x16_kernel<true>, dim3(n_wg), dim3(kGemvThreads), lds_bytes, st, d, n_wg,
                           gemv_x16_part_off(d.K));
    else
        hipLaunchKernelGGL(gemv_x16_kernel<false>, dim3(n_wg), dim3(kGemvThreads), lds_bytes, st, d, n_wg,
                           gemv_x16_part_off(d.K));
    return hipGetLastError();
}

}  // namespace terhip
