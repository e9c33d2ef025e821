// lm_head.hip -- the tail of a decode step on gfx950: RMSNorm of the fp32
// residual stream, the fp16 lm_head GEMV over the tied token embedding, and
// the argmax of the fp16 logits, fused into one launch; plus the standalone
// RMSNorm-to-fp16 and argmax kernels.
//
// Reference (cuda/ter_cuda_forward_bitnet.cu):
//   rmsnorm_f32_in_k     :37-47    <<<1,256>>> at :890
//   mm_fp16_lm_head_k    :388-429  one 32-lane warp per vocabulary row
//   argmax_local_k/_final_k :454-495  128 parts x 256 threads, then 128
//
// Summation order (bit-exact with the reference's fp32 arithmetic): for a
// row v of token_embd [V][H] (H even), "virtual lane" l = 0..31 sums the
// fp16 pairs k = l, l+32, ... < H/2, acc += x[2k]e[2k] + x[2k+1]e[2k+1]
// (products of fp16 values are exact in fp32), then the xor butterfly
// o = 16..1.  Here a wave64 runs two rows at once, one per 32-lane half,
// and each lane reads one dword (one fp16 pair) per group j of 32 pairs:
// every load instruction covers 128 contiguous bytes of each of two
// adjacent rows, so a wave streams its contiguous row range sequentially.
//
// Argmax without a second pass: the reference's winner is a total order on
// indices (value; then, among equal values, the smaller bit-reversed part
// index of its 128 parts, the smaller bit-reversed thread id of its 256
// threads, the first element of the thread; NaN and -inf never win).  Each
// logit gets a 64-bit key ordered that way; the launch keeps the maximum
// key with one 64-bit atomic max per workgroup, and the last workgroup to
// arrive decodes the index, writes it and returns the two state words to
// zero, so the next launch (or graph replay) starts clean.
#include "common.h"

namespace terhip {
namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kLmWaves = 4;
constexpr int kLmThreads = kLmWaves * 64;
constexpr unsigned kOob = 0x80000000u;  // voffset past any resource: the load returns 0

struct LmArgs {
    const float* hidden;        // fp32 [H] residual stream (RMSNorm prologue) or null
    const uint16_t* gamma;      // fp16 [H] RMSNorm weights (with hidden)
    const uint16_t* x16;        // fp16 [H] normalized input (without hidden)
    const uint16_t* emb;        // fp16 [V][H]
    uint16_t* x_out;            // fp16 [H] copy of the normalized input or null
    uint16_t* logits;           // fp16 [V] or null
    int32_t* token_out;         // argmax index or null
    unsigned long long* state;  // [2] zero at rest (argmax)
    float eps;
    int H, V;
};

// 64-bit argmax key of logit h at index i (0: never wins).
__device__ __forceinline__ unsigned long long argmax_key(uint16_t h, int i, int chunk) {
    const unsigned mag = h & 0x7FFFu;
    if (mag > 0x7C00u || h == 0xFC00u) return 0ull;  // NaN, -inf
    const unsigned ord = mag == 0u ? 0x8000u : ((h & 0x8000u) ? 0x7FFFu - mag : 0x8000u + mag);
    const int b = i / chunk;
    const int o = i - b * chunk;
    const unsigned rb = __builtin_bitreverse32((unsigned)b) >> 25;        // 7 bits
    const unsigned rt = __builtin_bitreverse32((unsigned)(o & 255)) >> 24;  // 8 bits
    const unsigned k = (unsigned)(o >> 8);
    return ((unsigned long long)ord << 40) | ((unsigned long long)(127u - rb) << 33) |
           ((unsigned long long)(255u - rt) << 25) | (unsigned long long)((1u << 25) - 1u - k);
}

__device__ __forceinline__ int argmax_index(unsigned long long key, int chunk) {
    if (key == 0ull) return -1;
    const unsigned rb = 127u - (unsigned)((key >> 33) & 127u);
    const unsigned rt = 255u - (unsigned)((key >> 25) & 255u);
    const unsigned k = (1u << 25) - 1u - (unsigned)(key & ((1u << 25) - 1u));
    const int b = (int)(__builtin_bitreverse32(rb) >> 25);
    const int t = (int)(__builtin_bitreverse32(rt) >> 24);
    return b * chunk + (int)k * 256 + t;
}

__device__ __forceinline__ int argmax_chunk(int n) { return (n + 127) / 128; }

__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) {
    return a > b ? a : b;
}

__device__ __forceinline__ unsigned long long wave_max64(unsigned long long k) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const unsigned lo = (unsigned)__shfl_xor((int)(unsigned)k, o);
        const unsigned hi = (unsigned)__shfl_xor((int)(unsigned)(k >> 32), o);
        k = umax64(k, ((unsigned long long)hi << 32) | lo);
    }
    return k;
}

// Workgroup maximum of the per-lane keys, then one atomic max per
// workgroup; the last workgroup to arrive writes the index and clears the
// state.  Every thread of the workgroup must call it.
__device__ void argmax_finish(unsigned long long key, unsigned long long* kred, unsigned long long* state,
                              int32_t* token_out, int chunk) {
    key = wave_max64(key);
    if ((threadIdx.x & 63) == 0) kred[threadIdx.x >> 6] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long m = kred[0];
#pragma unroll
        for (int w = 1; w < kLmWaves; ++w) m = umax64(m, kred[w]);
        if (m) atomicMax(state, m);
        __threadfence();
        const unsigned long long arrived = atomicAdd(state + 1, 1ull);
        if (arrived == (unsigned long long)gridDim.x - 1ull) {
            __threadfence();
            const unsigned long long best = atomicExch(state, 0ull);
            atomicExch(state + 1, 0ull);
            *gptr(token_out) = argmax_index(best, chunk);
        }
    }
}

// Stage the normalized input in LDS as fp16 pairs xs[0 .. npad), zero past
// H/2 (H even).  With hidden: rmsnorm_f32_in_k's steps (256 strided partial
// sums of squares with fused multiply-adds, the reference tree,
// rms_inv = 1 / sqrt(ss / H + eps) correctly rounded,
// y = half((x * rms_inv) * gamma)).  Workgroup 0 writes the optional copy.
__device__ void stage_x_pairs(const LmArgs& a, uint32_t* xs, int npad, float* red) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    const int n2 = a.H >> 1;
    const bool owner = blockIdx.x == 0 && a.x_out != nullptr;
    if (a.hidden) {
        const TER_GLOBAL float* h = gptr(a.hidden);
        float part = 0.f;
        for (int i = tid; i < a.H; i += kLmThreads) part = __builtin_fmaf(h[i], h[i], part);
        const float rms_inv = 1.0f / __builtin_sqrtf(tree_sum256(part, red) / (float)a.H + a.eps);
        for (int i = tid; i < npad; i += kLmThreads) {
            uint32_t w = 0;
            if (i < n2) {
                const f32x2 hv = *reinterpret_cast<const TER_GLOBAL f32x2*>(h + 2 * i);
                const uint32_t gw = gptr(reinterpret_cast<const uint32_t*>(a.gamma))[i];
                const uint16_t y0 = float_to_half_bits((hv.x * rms_inv) * half_bits_to_float((uint16_t)(gw & 0xFFFFu)));
                const uint16_t y1 = float_to_half_bits((hv.y * rms_inv) * half_bits_to_float((uint16_t)(gw >> 16)));
                w = (uint32_t)y0 | ((uint32_t)y1 << 16);
                if (owner) gptr(reinterpret_cast<uint32_t*>(a.x_out))[i] = w;
            }
            xs[i] = w;
        }
    } else {
        for (int i = tid; i < npad; i += kLmThreads)
            xs[i] = i < n2 ? gptr(reinterpret_cast<const uint32_t*>(a.x16))[i] : 0u;
    }
    __syncthreads();
}

// Row pair p of this wave (lanes 0-31: row 2p, lanes 32-63: row 2p + 1,
// relative to the wave's first row): one dword per group j.
template <int NJ>
__device__ __forceinline__ void load_pair(uint32_t (&w)[NJ], __amdgpu_buffer_rsrc_t rs, int p, int nrows, int rowb,
                                          int v, int half, int n2) {
    const int row = 2 * p + half;
    const bool row_ok = row < nrows;
    const unsigned base = (unsigned)(row * rowb + 4 * v);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const unsigned off = (row_ok && v + 32 * j < n2) ? base + 128u * j : kOob;
        w[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 2 /* nt */);
    }
}

template <int NJ>
__device__ __forceinline__ float dot_pair(const uint32_t (&w)[NJ], const uint32_t (&xr)[NJ]) {
#pragma clang fp contract(off)
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const float p0 = half_bits_to_float((uint16_t)(xr[j] & 0xFFFFu)) * half_bits_to_float((uint16_t)(w[j] & 0xFFFFu));
        const float p1 = half_bits_to_float((uint16_t)(xr[j] >> 16)) * half_bits_to_float((uint16_t)(w[j] >> 16));
        acc = acc + (p0 + p1);
    }
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) acc = acc + __shfl_xor(acc, o);
    return acc;
}

// Fast path, H even and H/2 <= 32 NJ: see the file comment.  The workgroup's
// 4 waves each own a contiguous range of row pairs (ranges of all waves of
// the grid in blockIdx order).
template <int NJ>
__global__ __launch_bounds__(kLmThreads) void lm_head_kernel(LmArgs a) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    uint32_t* xs = reinterpret_cast<uint32_t*>(lds_raw);
    float* red = reinterpret_cast<float*>(lds_raw + NJ * 32 * 4);
    unsigned long long* kred = reinterpret_cast<unsigned long long*>(red + kLmThreads);
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int v = lane & 31, half = lane >> 5;
    const int n2 = a.H >> 1;
    const int rowb = a.H * 2;
    const long long P = ((long long)a.V + 1) / 2;
    const long long W = (long long)gridDim.x * kLmWaves;
    const long long gw = (long long)blockIdx.x * kLmWaves + wave;
    const long long p0 = P * gw / W, p1 = P * (gw + 1) / W;
    const int np = (int)(p1 - p0);
    const long long r0 = 2 * p0;
    const long long r1 = 2 * p1 < (long long)a.V ? 2 * p1 : (long long)a.V;
    const int nrows = (int)(r1 - r0);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.emb + r0 * a.H), 0, nrows * rowb, 0x00020000);

    uint32_t wa[NJ], wb[NJ];
    if (np > 0) load_pair<NJ>(wa, rs, 0, nrows, rowb, v, half, n2);  // in flight during staging
    stage_x_pairs(a, xs, NJ * 32, red);
    uint32_t xr[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) xr[j] = xs[v + 32 * j];

    const int chunk = argmax_chunk(a.V);
    unsigned long long best = 0ull;
    uint16_t mine = 0;
    auto emit = [&](int p, float acc) {
        const uint16_t h = float_to_half_bits(acc);
        const int row = 2 * p + half;
        if (row < nrows) {
            if (a.token_out) best = umax64(best, argmax_key(h, (int)(r0 + row), chunk));
            if ((p & 31) == v) mine = h;
        }
        // one store per 32 pairs: lane v holds the logit of pair (p & ~31) + v
        if (a.logits && ((p & 31) == 31 || p == np - 1)) {
            const int rl = 2 * ((p & ~31) + v) + half;
            if (v <= (p & 31) && rl < nrows) gptr(a.logits)[r0 + rl] = mine;
        }
    };
    for (int p = 0; p < np; p += 2) {
        if (p + 1 < np) load_pair<NJ>(wb, rs, p + 1, nrows, rowb, v, half, n2);
        emit(p, dot_pair<NJ>(wa, xr));
        if (p + 1 >= np) break;
        if (p + 2 < np) load_pair<NJ>(wa, rs, p + 2, nrows, rowb, v, half, n2);
        emit(p + 1, dot_pair<NJ>(wb, xr));
    }
    if (a.token_out) argmax_finish(best, kred, a.state, a.token_out, chunk);
}

// Any H (odd, or H/2 above the fast path's 32 * 64 pairs): the reference's
// lane order with one load per element pair (or element), no pipelining.
__global__ __launch_bounds__(kLmThreads) void lm_head_generic_kernel(LmArgs a, int npad) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) unsigned char lds_raw[];
    uint32_t* xs = reinterpret_cast<uint32_t*>(lds_raw);
    float* red = reinterpret_cast<float*>(lds_raw + (size_t)npad * 4);
    unsigned long long* kred = reinterpret_cast<unsigned long long*>(red + kLmThreads);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int v = lane & 31, half = lane >> 5;
    const bool even = (a.H & 1) == 0;
    if (even) {
        stage_x_pairs(a, xs, npad, red);
    } else {  // odd H: no RMSNorm prologue (the host refuses it), elements as fp16 in LDS
        uint16_t* x1 = reinterpret_cast<uint16_t*>(xs);
        for (int i = tid; i < a.H; i += kLmThreads) x1[i] = gptr(a.x16)[i];
        __syncthreads();
    }
    const int chunk = argmax_chunk(a.V);
    unsigned long long best = 0ull;
    const long long W = (long long)gridDim.x * kLmWaves * 2;
    for (long long r = ((long long)blockIdx.x * kLmWaves + wave) * 2 + half; r < a.V; r += W) {
        const uint16_t* row = a.emb + r * a.H;
        float acc = 0.f;
        if (even) {
            for (int k = v; k < a.H / 2; k += 32) {
                const uint32_t w = gptr(reinterpret_cast<const uint32_t*>(row))[k];
                const float p0 = half_bits_to_float((uint16_t)(xs[k] & 0xFFFFu)) * half_bits_to_float((uint16_t)(w & 0xFFFFu));
                const float p1 = half_bits_to_float((uint16_t)(xs[k] >> 16)) * half_bits_to_float((uint16_t)(w >> 16));
                acc = acc + (p0 + p1);
            }
        } else {
            const uint16_t* x1 = reinterpret_cast<const uint16_t*>(xs);
            for (int k = v; k < a.H; k += 32) acc = acc + half_bits_to_float(x1[k]) * half_bits_to_float(gptr(row)[k]);
        }
        // xor butterfly within each 32-lane half (both halves run the loop in step)
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) acc = acc + __shfl_xor(acc, o);
        const uint16_t h = float_to_half_bits(acc);
        if (v == 0) {
            if (a.logits) gptr(a.logits)[r] = h;
            if (a.token_out) best = umax64(best, argmax_key(h, (int)r, chunk));
        }
    }
    if (a.token_out) argmax_finish(best, kred, a.state, a.token_out, chunk);
}

// argmax of fp16 logits [N] (argmax_local_k + argmax_final_k semantics).
__global__ __launch_bounds__(kLmThreads) void argmax_kernel(const uint16_t* __restrict__ logits, int n,
                                                            int32_t* token_out, unsigned long long* state) {
    __shared__ unsigned long long kred[kLmWaves];
    const int chunk = argmax_chunk(n);
    unsigned long long best = 0ull;
    for (long long i = (long long)blockIdx.x * kLmThreads + threadIdx.x; i < n; i += (long long)gridDim.x * kLmThreads)
        best = umax64(best, argmax_key(gptr(logits)[i], (int)i, chunk));
    argmax_finish(best, kred, state, token_out, chunk);
}

// rmsnorm_f32_in_k per row (256 threads): y = half((x * rms_inv) * gamma).
__global__ __launch_bounds__(256) void rmsnorm_f16_rows_kernel(const float* __restrict__ x,
                                                              const uint16_t* __restrict__ gamma, float eps, int H,
                                                              uint16_t* __restrict__ y) {
#pragma clang fp contract(off)
    __shared__ float red[256];
    const long long row0 = (long long)blockIdx.x * H;
    const TER_GLOBAL float* xr = gptr(x + row0);
    float part = 0.f;
    for (int i = threadIdx.x; i < H; i += 256) part = __builtin_fmaf(xr[i], xr[i], part);
    const float rms_inv = 1.0f / __builtin_sqrtf(tree_sum256(part, red) / (float)H + eps);
    for (int i = threadIdx.x; i < H; i += 256)
        gptr(y + row0)[i] = float_to_half_bits((xr[i] * rms_inv) * half_bits_to_float(gptr(gamma)[i]));
}

}  // namespace

int lm_head_fast_nj(int H) {
    if (H & 1) return 0;
    const int nj = (H / 2 + 31) / 32;
    const int r = (nj + 7) / 8 * 8;
    return r <= 64 ? r : 0;
}

int lm_head_lds_bytes(int H) {
    const int nj = lm_head_fast_nj(H);
    const int npad = nj ? nj * 32 : (H + 1) / 2;
    return npad * 4 + kLmThreads * 4 + kLmWaves * 8;
}

int lm_head_max_wg_per_cu(int H) {
    const int nj = lm_head_fast_nj(H), lds = lm_head_lds_bytes(H);
    int n = 0;
    hipError_t e;
    switch (nj) {
        case 8: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, lm_head_kernel<8>, kLmThreads, lds); break;
        case 16: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, lm_head_kernel<16>, kLmThreads, lds); break;
        case 24: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, lm_head_kernel<24>, kLmThreads, lds); break;
        case 32: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, lm_head_kernel<32>, kLmThreads, lds); break;
        case 40: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, lm_head_kernel<40>, kLmThreads, lds); break;
        case 48: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, lm_head_kernel<48>, kLmThreads, lds); break;
        case 56: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, lm_head_kernel<56>, kLmThreads, lds); break;
        case 64: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, lm_head_kernel<64>, kLmThreads, lds); break;
        default: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, lm_head_generic_kernel, kLmThreads, lds); break;
    }
    return e == hipSuccess ? n : 0;
}

hipError_t launch_lm_head(const float* hidden, const uint16_t* gamma, float eps, const uint16_t* x16,
                          const uint16_t* emb, int H, int V, uint16_t* x_out, uint16_t* logits, int32_t* token_out,
                          unsigned long long* state, int n_wg, hipStream_t st) {
    LmArgs a{};
    a.hidden = hidden;
    a.gamma = gamma;
    a.x16 = x16;
    a.emb = emb;
    a.x_out = x_out;
    a.logits = logits;
    a.token_out = token_out;
    a.state = state;
    a.eps = eps;
    a.H = H;
    a.V = V;
    const int nj = lm_head_fast_nj(H), lds = lm_head_lds_bytes(H);
    const dim3 g(n_wg), b(kLmThreads);
    switch (nj) {
        case 8: hipLaunchKernelGGL(lm_head_kernel<8>, g, b, lds, st, a); break;
        case 16: hipLaunchKernelGGL(lm_head_kernel<16>, g, b, lds, st, a); break;
        case 24: hipLaunchKernelGGL(lm_head_kernel<24>, g, b, lds, st, a); break;
        case 32: hipLaunchKernelGGL(lm_head_kernel<32>, g, b, lds, st, a); break;
        case 40: hipLaunchKernelGGL(lm_head_kernel<40>, g, b, lds, st, a); break;
        case 48: hipLaunchKernelGGL(lm_head_kernel<48>, g, b, lds, st, a); break;
        case 56: hipLaunchKernelGGL(lm_head_kernel<56>, g, b, lds, st, a); break;
        case 64: hipLaunchKernelGGL(lm_head_kernel<64>, g, b, lds, st, a); break;
        default: hipLaunchKernelGGL(lm_head_generic_kernel, g, b, lds, st, a, (H + 1) / 2); break;
    }
    return hipGetLastError();
}

hipError_t launch_argmax_f16(const uint16_t* logits, int n, int32_t* token_out, unsigned long long* state, int n_wg,
                             hipStream_t st) {
    hipLaunchKernelGGL(argmax_kernel, dim3(n_wg), dim3(kLmThreads), 0, st, logits, n, token_out, state);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_f16_rows(const float* x, const uint16_t* gamma, float eps, int M, int H, uint16_t* y,
                                   hipStream_t st) {
    hipLaunchKernelGGL(rmsnorm_f16_rows_kernel, dim3(M), dim3(256), 0, st, x, gamma, eps, H, y);
    return hipGetLastError();
}

}  // namespace terhip
