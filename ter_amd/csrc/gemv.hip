// gemv.hip -- M = 1 packed-trit GEMV for gfx950 (work-list, stream-K).
//
// Replaces the reference's CUDA GEMV family (mm_packed_v4 / v11,
// cuda/ter_cuda_forward_packed.cu:346-397; mm_bitnet_addonly_dev,
// cuda/ter_cuda_forward_bitnet.cu:497-559; v12/v13 variants) with one
// kernel that streams the T16 tile layout (common.h).  Results are the
// reference's: acc[j] = sum_k x[k] * w[k][j] in exact integers and
// y[j] = float(acc[j]) * (x_scale * w_scale) (src/tx/forward.cpp:342-345,
// cuda/ter_cuda_forward_packed.cu:353,393).
//
// Work distribution.  All GEMVs of a launch form one stream of 1 KiB tiles.
// The stream is cut into n_wg equal contiguous ranges, one per workgroup
// (4 waves); consecutive ranges are kept on one XCD.  A workgroup walks its
// range GEMV segment by GEMV segment: it stages that GEMV's int8 activation
// vector in LDS (quantizing an fp32 vector by absmax in this prologue), then
// its 4 waves split the segment's tiles into equal contiguous pieces.  A wave
// accumulates a column strip over its tiles; when a piece covers a whole
// strip the wave writes the outputs, otherwise it adds its partial sums into
// the strip's 64-bit fix-up slots with one atomic per column (high bits count
// the 256-row units seen, low 40 bits hold the signed partial sum); the wave
// whose atomic completes the count writes the outputs and clears the slot.
// Integer sums are order independent, so results are bit-exact whatever the
// split.
//
// Inner loop per tile and lane: one global_load_dwordx4 of packed weights
// (64 trits: 4 columns x 16 rows), one ds_read_b128 of the matching 16 int8
// activations, 5 bit operations + 4 v_dot4 per column dword.
#include "common.h"

namespace terhip {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Sum over the 16 lanes of a DPP row; every lane of the row gets the sum.
__device__ __forceinline__ int row_sum16(int v) {
    v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);   // quad_perm [1,0,3,2]
    v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);   // quad_perm [2,3,0,1]
    v += __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true);  // row_half_mirror
    v += __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true);  // row_mirror
    return v;
}

template <int kCtrl>
__device__ __forceinline__ float fmax_dpp(float v) {
    return fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xF, 0xF, true)));
}

// Max over the 64 lanes of a wave (all lanes get it).
__device__ __forceinline__ float wave_max(float v) {
    v = fmax_dpp<0xB1>(v);
    v = fmax_dpp<0x4E>(v);
    v = fmax_dpp<0x141>(v);
    v = fmax_dpp<0x140>(v);
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}

__device__ __forceinline__ int sum_bytes(const u32x4& v) {
    int s = __builtin_amdgcn_sdot4((int)v.x, 0x01010101, 0, false);
    s = __builtin_amdgcn_sdot4((int)v.y, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4((int)v.z, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4((int)v.w, 0x01010101, s, false);
    return s;
}

// Stage the activation vector of `d` into LDS as int8 [Ku*256] (zero padded)
// plus per-unit sums usum[Ku].  Returns the activation scale.  For fp32 input
// this is the absmax prologue of quant_int8_k (cuda/ter_cuda_forward_packed.cu:40-62):
// amax = max|x| + 1e-9f, scale = 127.f / amax, q = rint(x * scale) clamped to
// [-128, 127], act_scale = 1.f / scale.
__device__ float stage_x(const GemvDesc& d, int8_t* lds_x, int* usum, float* red, bool owner) {
#pragma clang fp contract(off)
    const int K = d.K;
    const int nchunks = d.Ku * (kUnitK / 16);
    const int tid = threadIdx.x;
    if (d.x_kind == TER_HIP_X_I8) {
        const int8_t* xp = static_cast<const int8_t*>(d.x);
        const bool vec_ok = ((reinterpret_cast<uintptr_t>(xp) & 15u) == 0);
        for (int c = tid; c < nchunks; c += kThreads) {
            const int k = c * 16;
            u32x4 v;
            if (vec_ok && k + 16 <= K) {
                v = *reinterpret_cast<const u32x4*>(xp + k);
            } else {
                unsigned wd[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    unsigned a = 0;
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const int kk = k + 4 * i + b;
                        const unsigned by = kk < K ? (unsigned)(uint8_t)xp[kk] : 0u;
                        a |= by << (8 * b);
                    }
                    wd[i] = a;
                }
                v = u32x4{wd[0], wd[1], wd[2], wd[3]};
            }
            *reinterpret_cast<u32x4*>(lds_x + k) = v;
            const int s = row_sum16(sum_bytes(v));
            if ((tid & 15) == 0) usum[c >> 4] = s;
        }
        return d.x_scale_dev ? *d.x_scale_dev : d.x_scale;
    }
    // fp32 input: absmax, then quantize.
    const float* xf = static_cast<const float*>(d.x);
    float m = 0.f;
    for (int k = tid; k < K; k += kThreads) m = fmaxf(m, fabsf(xf[k]));
    m = wave_max(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float amax = m + 1e-9f;
    const float scale = 127.0f / amax;
    const float act = 1.0f / scale;
    for (int c = tid; c < nchunks; c += kThreads) {
        const int k = c * 16;
        unsigned wd[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            unsigned a = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int kk = k + 4 * i + b;
                int qv = 0;
                if (kk < K) {
                    const float v = xf[kk] * scale;
                    qv = (int)__builtin_rintf(v);
                    qv = qv > 127 ? 127 : (qv < -128 ? -128 : qv);
                }
                a |= ((unsigned)qv & 0xFFu) << (8 * b);
            }
            wd[i] = a;
        }
        const u32x4 v = u32x4{wd[0], wd[1], wd[2], wd[3]};
        *reinterpret_cast<u32x4*>(lds_x + k) = v;
        const int s = row_sum16(sum_bytes(v));
        if ((tid & 15) == 0) usum[c >> 4] = s;
        if (owner && d.xq_out) {
            for (int i = 0; i < 16 && k + i < K; ++i)
                d.xq_out[k + i] = (int8_t)((wd[i >> 2] >> (8 * (i & 3))) & 0xFFu);
        }
    }
    if (owner && tid == 0 && d.xs_out) *d.xs_out = act;
    return act;
}

__device__ __forceinline__ void emit(const GemvDesc& d, int col, int val, float s) {
#pragma clang fp contract(off)
    if (d.acc) d.acc[col] = val;
    if (d.y) d.y[col] = (float)val * s;
}

// Accumulate 1 tile (16 bytes of this lane) into the 4 column accumulators.
__device__ __forceinline__ void dot_tile(const u32x4& w, const u32x4& x, int (&a1)[4], int (&a4)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned d = w[j];
        const unsigned d4 = d >> 4;
        a1[j] = __builtin_amdgcn_sdot4((int)x.x, (int)(d & 0x03030303u), a1[j], false);
        a4[j] = __builtin_amdgcn_sdot4((int)x.y, (int)(d & 0x0C0C0C0Cu), a4[j], false);
        a1[j] = __builtin_amdgcn_sdot4((int)x.z, (int)(d4 & 0x03030303u), a1[j], false);
        a4[j] = __builtin_amdgcn_sdot4((int)x.w, (int)(d4 & 0x0C0C0C0Cu), a4[j], false);
    }
}

constexpr int kBatch = 8;  // tiles in flight per wave

// One wave processes local tiles [la, lb) of GEMV d.
__device__ void run_wave(const GemvDesc& d, const int8_t* lds_x, const int* usum, float s,
                         long long la, long long lb) {
    const int lane = threadIdx.x & 63;
    const int q = lane & 15;
    const int r = lane >> 4;
    const int Ku = d.Ku;
    const uint8_t* wl = d.w + lane * 16;
    long long lt = la;
    while (lt < lb) {
        const int st = (int)(lt / Ku);
        const int u0 = (int)(lt - (long long)st * Ku);
        const int n = (int)min((long long)(Ku - u0), lb - lt);
        int a1[4] = {0, 0, 0, 0}, a4[4] = {0, 0, 0, 0};
        int corr = 0;
        const uint8_t* wt = wl + lt * kTileBytes;
        for (int i0 = 0; i0 < n; i0 += kBatch) {
            const int m = min(kBatch, n - i0);
            u32x4 wv[kBatch];
#pragma unroll
            for (int i = 0; i < kBatch; ++i)
                if (i < m)
                    wv[i] = __builtin_nontemporal_load(
                        reinterpret_cast<const u32x4*>(wt + (long long)(i0 + i) * kTileBytes));
#pragma unroll
            for (int i = 0; i < kBatch; ++i) {
                if (i < m) {
                    const int u = u0 + i0 + i;
                    const u32x4 xv = *reinterpret_cast<const u32x4*>(lds_x + u * kUnitK + q * 16);
                    corr += usum[u];
                    dot_tile(wv[i], xv, a1, a4);
                }
            }
        }
        int v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = row_sum16(a1[j] + (a4[j] >> 2));
        int val = q == 0 ? v[0] : (q == 1 ? v[1] : (q == 2 ? v[2] : v[3]));
        val -= corr;
        const int col = st * kStripCols + r * 4 + q;
        if (q < 4 && col < d.N) {
            if (u0 == 0 && n == Ku) {
                emit(d, col, val, s);
            } else {
                const unsigned long long add =
                    ((unsigned long long)n << 40) + (unsigned long long)(long long)val;
                const unsigned long long old = __hip_atomic_fetch_add(
                    d.fix + col, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const long long tot = (long long)(old + add);
                const long long units = (tot + (1LL << 39)) >> 40;
                if (units == (long long)Ku) {
                    const long long sum = tot - (units << 40);
                    __hip_atomic_store(d.fix + col, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    emit(d, col, (int)sum, s);
                }
            }
        }
        lt += n;
    }
}

__global__ __launch_bounds__(kThreads) void gemv_t16_kernel(GemvDesc single,
                                                            const GemvDesc* __restrict__ list,
                                                            int n_list, long long total, int n_wg) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    int g = blockIdx.x;
    if ((n_wg & 7) == 0) g = (g & 7) * (n_wg >> 3) + (g >> 3);  // keep neighbouring ranges on one XCD
    const long long t_begin = total * g / n_wg;
    const long long t_end = total * (g + 1) / n_wg;
    if (t_begin >= t_end) return;

    int di = 0;
    if (n_list > 0) {
        int lo = 0, hi = n_list - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (list[mid].tile0 <= t_begin) lo = mid; else hi = mid - 1;
        }
        di = lo;
    }
    long long t = t_begin;
    const int wave = threadIdx.x >> 6;
    while (t < t_end) {
        const GemvDesc d = n_list > 0 ? list[di] : single;
        const long long seg_end = min(t_end, d.tile0 + (long long)d.n_strips * d.Ku);
        int8_t* lds_x = reinterpret_cast<int8_t*>(lds_raw);
        int* usum = reinterpret_cast<int*>(lds_raw + d.Ku * kUnitK);
        float* red = reinterpret_cast<float*>(lds_raw + d.Ku * kUnitK + d.Ku * 4);
        __syncthreads();  // the previous segment is done with LDS
        const float act = stage_x(d, lds_x, usum, red, t == d.tile0);
        __syncthreads();
        const float s = act * d.w_scale;  // x_scale * w_scale, in this order (forward.cpp:342)
        const long long n = seg_end - t;
        const long long a = t + n * wave / kWaves;
        const long long b = t + n * (wave + 1) / kWaves;
        if (a < b) run_wave(d, lds_x, usum, s, a - d.tile0, b - d.tile0);
        t = seg_end;
        ++di;
    }
}

}  // namespace

int gemv_max_wg_per_cu(int lds_bytes) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_t16_kernel, kThreads, lds_bytes) != hipSuccess)
        return 0;
    return n;
}

hipError_t launch_gemv(const GemvDesc& single, const GemvDesc* list_dev, int n_list,
                       long long total_tiles, int n_wg, int lds_bytes, hipStream_t st) {
    hipLaunchKernelGGL(gemv_t16_kernel, dim3(n_wg), dim3(kThreads), lds_bytes, st, single, list_dev,
                       n_list, total_tiles, n_wg);
    return hipGetLastError();
}

}  // namespace terhip
