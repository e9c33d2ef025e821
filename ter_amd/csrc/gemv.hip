// gemv.hip -- M = 1 packed-trit GEMV for gfx950 (work-list, stream-K).
//
// Replaces the reference's CUDA GEMV family (mm_packed_v4 / v11,
// cuda/ter_cuda_forward_packed.cu:346-397; mm_bitnet_addonly_dev,
// cuda/ter_cuda_forward_bitnet.cu:497-559; v12/v13 variants) with one
// kernel that streams the T16 tile layout (common.h).  Results are the
// reference's: acc[j] = sum_k x[k] * w[k][j] in exact integers and
// y[j] = float(mag * acc[j]) * (x_scale * w_scale), mag the payload magnitude (src/tx/forward.cpp:342-345,
// cuda/ter_cuda_forward_packed.cu:353,393).
//
// Work distribution.  All GEMVs of a launch form one stream of 1 KiB tiles.
// The stream is cut into n_wg equal contiguous ranges, one per workgroup
// (4 waves); consecutive ranges are kept on one XCD.  A workgroup walks its
// range GEMV segment by GEMV segment: every wave first issues the loads of
// its first batch of weight tiles, then the workgroup stages that GEMV's
// int8 activation vector in LDS (quantizing an fp32 vector by absmax in this
// prologue), then the 4 waves stream equal contiguous pieces of the segment.
//
// A wave's piece is read through a buffer resource sized to the piece, with
// two batches of tiles in registers: the loads of batch i + 1 are in flight
// while batch i is reduced, and loads past the piece return zeros, so no
// load is predicated.  All control flow is wave-uniform (scalar registers).
// A wave accumulates a column strip over its tiles; a strip whose 256-row
// units all lie in the piece is written directly.  The (at most two) strips
// a piece shares with its neighbours are added, after the streaming loop,
// into per-column 64-bit fix-up slots with one atomic per column (high bits
// count the 256-row units seen, low 40 bits hold the signed partial sum);
// the wave whose atomic completes the count writes the outputs and clears
// the slot.  Integer sums are order independent, so results are bit-exact
// whatever the split.
//
// Inner loop per tile and lane: one buffer_load_dwordx4 of packed weights
// (64 trits: 4 columns x 16 rows), one ds_read_b128 of the matching 16 int8
// activations, 5 bit operations + 4 v_dot4 per column dword.
#include "common.h"

namespace terhip {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Tiles per batch (two batches per wave in flight): 6 for fp32 activations
// and for the general prologue, 5 for int8, 4 for the RMS kinds (the decode
// step's small lists).  Measured: the int8 C2 sweep 42.6 against 42.9 us and
// the decode step 1.168 against 1.194 ms per token with 5 rather than 6; the
// fp32 C3 sweep 90.5 against 92.2 us with 6 rather than 5; the decode step
// 1.166 against 1.171 ms with 4 rather than 5 for the RMS kinds.
template <int kKind>
constexpr int batch_of() {
    return kKind == TER_HIP_X_F32 || kKind < 0 ? 6 : (kKind >= TER_HIP_X_F32_RMS ? 4 : 5);
}

// Waves per SIMD the stream-K kernel is compiled for: 4 for int8 X (the
// workgroups of its default launch, kGemvWgPerCuI8 = 4 per CU, all resident),
// otherwise whatever the registers allow.
template <int kKind>
constexpr int gemv_waves_per_eu() {
    return kKind == TER_HIP_X_I8 ? 4 : 1;
}

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
    v = fmaxf(v, lane_xor16(v));
    v = fmaxf(v, lane_xor32(v));
    return v;
}

__device__ __forceinline__ int sum_bytes(const u32x4& v) {
    int s = __builtin_amdgcn_sdot4((int)v.x, 0x01010101, 0, false);
    s = __builtin_amdgcn_sdot4((int)v.y, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4((int)v.z, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4((int)v.w, 0x01010101, s, false);
    return s;
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// quant_int8_k element step (cuda/ter_cuda_forward_packed.cu:55-58):
// rint(x * scale) (round half to even), clamped to [-128, 127].
__device__ __forceinline__ unsigned quant_byte(float x, float scale) {
#pragma clang fp contract(off)
    int q = (int)__builtin_rintf(x * scale);
    q = q > 127 ? 127 : (q < -128 ? -128 : q);
    return (unsigned)q & 0xFFu;
}

// Store one 16-byte activation chunk (k = 16 c) in LDS and its unit sum.
__device__ __forceinline__ void put_chunk(int c, const u32x4& v, int8_t* lds_x, int* usum) {
    *reinterpret_cast<u32x4*>(lds_x + c * 16) = v;
    const int s = row_sum16(sum_bytes(v));
    if ((threadIdx.x & 15) == 0) usum[c >> 4] = s;
}

// 16 fp32 activations x[k .. k+15] (zeros past K).
__device__ __forceinline__ void load_f16(const float* xf, int k, int K, bool vec_ok, float (&v)[16]) {
    if (vec_ok && k + 16 <= K) {
        const TER_GLOBAL f32x4* p = gptr(reinterpret_cast<const f32x4*>(xf + k));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x4 f = p[i];
            v[4 * i] = f.x;
            v[4 * i + 1] = f.y;
            v[4 * i + 2] = f.z;
            v[4 * i + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = k + i < K ? gptr(xf)[k + i] : 0.f;
    }
}

__device__ __forceinline__ u32x4 pack_q16(const float (&v)[16], float scale) {
    unsigned wd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        wd[i] = quant_byte(v[4 * i], scale) | (quant_byte(v[4 * i + 1], scale) << 8) |
                (quant_byte(v[4 * i + 2], scale) << 16) | (quant_byte(v[4 * i + 3], scale) << 24);
    return u32x4{wd[0], wd[1], wd[2], wd[3]};
}

// int8 activations x[k .. k+15] (zeros past K).
__device__ __forceinline__ u32x4 load_i16(const int8_t* xp, int k, int K, bool vec_ok) {
    if (vec_ok && k + 16 <= K) return *gptr(reinterpret_cast<const u32x4*>(xp + k));
    unsigned wd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        unsigned a = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int kk = k + 4 * i + b;
            const unsigned by = kk < K ? (unsigned)(uint8_t)gptr(xp)[kk] : 0u;
            a |= by << (8 * b);
        }
        wd[i] = a;
    }
    return u32x4{wd[0], wd[1], wd[2], wd[3]};
}

// This thread's first two 16-element chunks of the activation vector
// (chunks tid and tid + kGemvThreads), loaded into registers before the
// weight batch is issued: a wave's loads return in issue order, so the
// activations (L2-resident, shared by many workgroups) then arrive without
// waiting behind the weight tiles from HBM.  That covers K <= 8192 with 256
// threads; chunks beyond are loaded during staging.
struct XPre {
    float v0[16], v1[16];  // fp32 / fp16 input (as fp32)
    u32x4 q0, q1;          // int8 input
};

// 16 fp16 activations x[k .. k+15] as fp32 (zeros past K).
__device__ __forceinline__ void load_h16(const uint16_t* xh, int k, int K, float (&v)[16]) {
    if (((reinterpret_cast<uintptr_t>(xh + k) & 15u) == 0) && k + 16 <= K) {
        const TER_GLOBAL u32x4* p = gptr(reinterpret_cast<const u32x4*>(xh + k));
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const u32x4 w = p[i];
            const unsigned wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[8 * i + 2 * j] = half_bits_to_float((uint16_t)(wd[j] & 0xFFFFu));
                v[8 * i + 2 * j + 1] = half_bits_to_float((uint16_t)(wd[j] >> 16));
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = k + i < K ? half_bits_to_float(gptr(xh)[k + i]) : 0.f;
    }
}

// 16 fp16 values at k as 8 packed dwords (zeros past K): half the registers
// of load_h16 while the values wait.
__device__ __forceinline__ void load_h16_raw(const uint16_t* xh, int k, int K, uint32_t (&w)[8]) {
    if (((reinterpret_cast<uintptr_t>(xh + k) & 15u) == 0) && k + 16 <= K) {
        const TER_GLOBAL u32x4* p = gptr(reinterpret_cast<const u32x4*>(xh + k));
        const u32x4 a = p[0], b = p[1];
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
        w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lo = k + 2 * i < K ? gptr(xh)[k + 2 * i] : 0u;
            const uint32_t hi = k + 2 * i + 1 < K ? gptr(xh)[k + 2 * i + 1] : 0u;
            w[i] = lo | (hi << 16);
        }
    }
}

// relu^2(gate) * up on 16 elements at k (zeros past K).
__device__ __forceinline__ void load_relu2_16(const uint16_t* g, const uint16_t* u, int k, int K, float (&v)[16]) {
    if ((((reinterpret_cast<uintptr_t>(g + k) | reinterpret_cast<uintptr_t>(u + k)) & 15u) == 0) && k + 16 <= K) {
        const TER_GLOBAL u32x4* pg = gptr(reinterpret_cast<const u32x4*>(g + k));
        const TER_GLOBAL u32x4* pu = gptr(reinterpret_cast<const u32x4*>(u + k));
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const u32x4 gw = pg[i], uw = pu[i];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[8 * i + 2 * j] = relu2_mul(half_bits_to_float((uint16_t)(gw[j] & 0xFFFFu)),
                                             half_bits_to_float((uint16_t)(uw[j] & 0xFFFFu)));
                v[8 * i + 2 * j + 1] = relu2_mul(half_bits_to_float((uint16_t)(gw[j] >> 16)),
                                                 half_bits_to_float((uint16_t)(uw[j] >> 16)));
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            v[i] = k + i < K ? relu2_mul(half_bits_to_float(gptr(g)[k + i]), half_bits_to_float(gptr(u)[k + i])) : 0.f;
    }
}

// silu(gate) * up on 16 elements at k (zeros past K).
__device__ __forceinline__ void load_silu16(const uint16_t* g, const uint16_t* u, int k, int K, float (&v)[16]) {
    float gv[16], uv[16];
    load_h16(g, k, K, gv);
    load_h16(u, k, K, uv);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = silu_mul(gv[i], uv[i]);  // past K: silu(0) * 0 = 0
}

// 16 activations of an fp32-family input (fp32, fp16 for X_F16 / X_F16_RMS,
// relu^2(gate) * up for X_RELU2_RMS, silu(gate) * up for X_SILU_MUL and
// X_SMUL) as fp32.
__device__ __forceinline__ void load_x16f(const GemvDesc& d, int k, float (&v)[16]) {
    if (d.x_kind == TER_HIP_X_SMUL) {
        // fp32 silu(gate) times fp16 up (zeros past K: 0 * 0)
#pragma clang fp contract(off)
        const float* xf = static_cast<const float*>(d.x);
        float u[16];
        load_f16(xf, k, d.K, (reinterpret_cast<uintptr_t>(xf) & 15u) == 0, v);
        load_h16(d.up, k, d.K, u);
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = v[i] * u[i];
    } else if (d.x_kind == TER_HIP_X_F16_RMS || d.x_kind == TER_HIP_X_F16) {
        load_h16(static_cast<const uint16_t*>(d.x), k, d.K, v);
    } else if (d.x_kind == TER_HIP_X_RELU2_RMS) {
        load_relu2_16(static_cast<const uint16_t*>(d.x), d.up, k, d.K, v);
    } else if (d.x_kind == TER_HIP_X_SILU_MUL) {
        load_silu16(static_cast<const uint16_t*>(d.x), d.up, k, d.K, v);
    } else {
        const float* xf = static_cast<const float*>(d.x);
        load_f16(xf, k, d.K, (reinterpret_cast<uintptr_t>(xf) & 15u) == 0, v);
    }
}

__device__ __forceinline__ float x_at(const GemvDesc& d, int i) {
    if (d.x_kind == TER_HIP_X_F32_RMS) return gptr(static_cast<const float*>(d.x))[i];
    const float h = half_bits_to_float(gptr(static_cast<const uint16_t*>(d.x))[i]);
    return d.x_kind == TER_HIP_X_F16_RMS ? h : relu2_mul(h, half_bits_to_float(gptr(d.up)[i]));  // (RMS kinds only)
}

// RMSNorm of the RMS kinds: n = (x * rms_inv) * gamma on 16 values at k.
__device__ __forceinline__ void rms_apply(const GemvDesc& d, int k, float rms_inv, float (&v)[16]) {
#pragma clang fp contract(off)
    float g[16];
    load_h16(d.gamma, k, d.K, g);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = (v[i] * rms_inv) * g[i];
}

__device__ __forceinline__ void x_prefetch(const GemvDesc& d, XPre& r) {
    const int nchunks = d.Ku * (kUnitK / 16);
    const int c0 = threadIdx.x, c1 = threadIdx.x + kGemvThreads;
    if (d.x_kind == TER_HIP_X_I8) {
        const int8_t* xp = static_cast<const int8_t*>(d.x);
        const bool vec_ok = ((reinterpret_cast<uintptr_t>(xp) & 15u) == 0);
        if (c0 < nchunks) r.q0 = load_i16(xp, c0 * 16, d.K, vec_ok);
        if (c1 < nchunks) r.q1 = load_i16(xp, c1 * 16, d.K, vec_ok);
    } else {
        if (c0 < nchunks) load_x16f(d, c0 * 16, r.v0);
        if (c1 < nchunks) load_x16f(d, c1 * 16, r.v1);
    }
}

// Stage the activation vector of `d` into LDS as int8 [Ku*256] (zero padded)
// plus per-unit sums usum[Ku], starting from the chunks prefetched in `r`.
// Returns the activation scale.  For fp32 input this is the absmax prologue
// of quant_int8_k (cuda/ter_cuda_forward_packed.cu:40-62): amax = max|x| +
// 1e-9f, scale = 127.f / amax, q = rint(x * scale) clamped to [-128, 127],
// act_scale = 1.f / scale.  The RMS kinds first apply the fused RMSNorm of
// rmsnorm_quant_{f32,fp16}_in_k (cuda/ter_cuda_forward_bitnet.cu:64-146):
// strided per-thread sums of squares (fused multiply-adds) reduced in the
// reference's tree order, rms_inv = 1 / sqrt(ss / K + eps) correctly rounded,
// x <- (x * rms_inv) * gamma.  X_RELU2_RMS is relu2_mul_rmsnorm_quant_k
// (cuda/ter_cuda_forward_bitnet.cu:258-309): x = relu^2(gate) * up and the
// sum of squares in its 1024-thread order.  `owner` (the workgroup that starts the GEMV)
// also writes the optional copies xq_out / xs_out.
__device__ __forceinline__ float stage_x(const GemvDesc& d, const XPre& r, int8_t* lds_x, int* usum, float* red, float* xs32,
                         bool owner) {
#pragma clang fp contract(off)
    const int K = d.K;
    const int nchunks = d.Ku * (kUnitK / 16);
    const int tid = threadIdx.x;
    const int c0 = tid, c1 = tid + kGemvThreads;
    if (d.x_kind == TER_HIP_X_I8) {
        const int8_t* xp = static_cast<const int8_t*>(d.x);
        const bool vec_ok = ((reinterpret_cast<uintptr_t>(xp) & 15u) == 0);
        if (c0 < nchunks) put_chunk(c0, r.q0, lds_x, usum);
        if (c1 < nchunks) put_chunk(c1, r.q1, lds_x, usum);
        for (int c = tid + 2 * kGemvThreads; c < nchunks; c += kGemvThreads)
            put_chunk(c, load_i16(xp, c * 16, K, vec_ok), lds_x, usum);
        return d.x_scale_dev ? *gptr(d.x_scale_dev) : d.x_scale;
    }
    const bool rms = d.x_kind == TER_HIP_X_F32_RMS || d.x_kind == TER_HIP_X_F16_RMS || d.x_kind == TER_HIP_X_RELU2_RMS;
    float rms_inv = 1.0f;
    uint32_t g0[8], g1[8];
    if (rms) {
        // gamma for the prefetched chunks, in flight during the reduction
        if (c0 < nchunks) load_h16_raw(d.gamma, c0 * 16, K, g0);
        if (c1 < nchunks) load_h16_raw(d.gamma, c1 * 16, K, g1);
        float ss;
        if (!d.stage32) {
            // K too large to stage fp32 activations beside the int8 ones: the
            // strided sums re-read the inputs (L2-resident) in the same order
            if (d.x_kind == TER_HIP_X_RELU2_RMS) {
                ss = relu2_sum_sq_1024(static_cast<const uint16_t*>(d.x), d.up, K, red);
            } else {
                float part = 0.f;
                for (int i = tid; i < K; i += kGemvThreads) {
                    const float v = x_at(d, i);
                    part = __builtin_fmaf(v, v, part);
                }
                ss = tree_sum256(part, red);
            }
        } else {
        // the (zero-padded) activations as fp32 in LDS, so the sum of squares
        // reads them in the reference's strided order without a second pass
        // over global memory
        auto put16 = [&](int c, const float (&v)[16]) {
#pragma unroll
            for (int i = 0; i < 16; i += 4)
                *reinterpret_cast<f32x4*>(xs32 + c * 16 + i) = f32x4{v[i], v[i + 1], v[i + 2], v[i + 3]};
        };
        if (c0 < nchunks) put16(c0, r.v0);
        if (c1 < nchunks) put16(c1, r.v1);
        for (int c = tid + 2 * kGemvThreads; c < nchunks; c += kGemvThreads) {
            float t[16];
            load_x16f(d, c * 16, t);
            put16(c, t);
        }
        __syncthreads();
        if (d.x_kind == TER_HIP_X_RELU2_RMS) {
            // 1024 virtual threads: element i goes to partial (i / 256) % 4 of thread i % 256
            float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
            for (int i = tid; i < K; i += 4 * kGemvThreads) {
                const float a = xs32[i];
                const float b = i + 256 < K ? xs32[i + 256] : 0.f;
                const float c = i + 512 < K ? xs32[i + 512] : 0.f;
                const float e = i + 768 < K ? xs32[i + 768] : 0.f;
                p0 = __builtin_fmaf(a, a, p0);
                p1 = __builtin_fmaf(b, b, p1);  // past K: +0, which changes no sum
                p2 = __builtin_fmaf(c, c, p2);
                p3 = __builtin_fmaf(e, e, p3);
            }
            ss = tree_sum256((p0 + p2) + (p1 + p3), red);
        } else {
            float part = 0.f;
            for (int i = tid; i < K; i += kGemvThreads) {
                const float v = xs32[i];
                part = __builtin_fmaf(v, v, part);
            }
            ss = tree_sum256(part, red);
        }
        }
        rms_inv = 1.0f / __builtin_sqrtf(ss / (float)K + d.eps);
    }
    float v0[16], v1[16];
    if (rms && !d.stage32) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int sh = 16 * (i & 1);
            v0[i] = (r.v0[i] * rms_inv) * half_bits_to_float((uint16_t)(g0[i >> 1] >> sh));
            v1[i] = (r.v1[i] * rms_inv) * half_bits_to_float((uint16_t)(g1[i >> 1] >> sh));
        }
    } else if (rms) {
        // the chunks come back from LDS, so the prefetch registers are free
        // during the reduction
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(xs32 + (c0 < nchunks ? c0 : 0) * 16 + i);
            const f32x4 b = *reinterpret_cast<const f32x4*>(xs32 + (c1 < nchunks ? c1 : 0) * 16 + i);
            v0[i] = a.x; v0[i + 1] = a.y; v0[i + 2] = a.z; v0[i + 3] = a.w;
            v1[i] = b.x; v1[i + 1] = b.y; v1[i + 2] = b.z; v1[i + 3] = b.w;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int sh = 16 * (i & 1);
            v0[i] = (v0[i] * rms_inv) * half_bits_to_float((uint16_t)(g0[i >> 1] >> sh));
            v1[i] = (v1[i] * rms_inv) * half_bits_to_float((uint16_t)(g1[i >> 1] >> sh));
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            v0[i] = r.v0[i];
            v1[i] = r.v1[i];
        }
    }
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if (c0 < nchunks) m = fmaxf(m, fabsf(v0[i]));
        if (c1 < nchunks) m = fmaxf(m, fabsf(v1[i]));
    }
    for (int c = tid + 2 * kGemvThreads; c < nchunks; c += kGemvThreads) {
        float t[16];
        if (rms && d.stage32) {
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const f32x4 f = *reinterpret_cast<const f32x4*>(xs32 + c * 16 + i);
                t[i] = f[0]; t[i + 1] = f[1]; t[i + 2] = f[2]; t[i + 3] = f[3];
            }
            rms_apply(d, c * 16, rms_inv, t);
        } else {
            load_x16f(d, c * 16, t);
            if (rms) rms_apply(d, c * 16, rms_inv, t);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(t[i]));
    }
    m = wave_max(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int i = 1; i < kGemvWaves; ++i) m = fmaxf(m, red[i]);
    const float amax = m + 1e-9f;
    const float scale = 127.0f / amax;
    const float act = 1.0f / scale;
    for (int c = tid; c < nchunks; c += kGemvThreads) {
        u32x4 q;
        if (c == c0) {
            q = pack_q16(v0, scale);
        } else if (c == c1) {
            q = pack_q16(v1, scale);
        } else {
            float t[16];
            load_x16f(d, c * 16, t);
            if (rms) rms_apply(d, c * 16, rms_inv, t);
            q = pack_q16(t, scale);
        }
        put_chunk(c, q, lds_x, usum);
        if (owner && d.xq_out) {
            const int k = c * 16;
            const unsigned qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (k + i < K) gptr(d.xq_out)[k + i] = (int8_t)((qw[i >> 2] >> (8 * (i & 3))) & 0xFFu);
        }
    }
    if (owner && tid == 0 && d.xs_out) *gptr(d.xs_out) = act;
    return act;
}

// ---------------------------------------------------------------------------
// Vector prologue.  When every GEMV of a launch has one activation kind, K a
// multiple of 16 and 16-byte aligned vectors (the decode step's case), the
// launch uses a kernel specialised on that kind: the activations (and gamma)
// are read through buffer resources sized to K elements, so a 16-element
// chunk is either loaded whole or reads as zeros past K, and no load sits
// behind a branch.  All of them are issued before the weight batch and stay
// raw in registers until staging, so the staging waits only for them and not
// for the weights (a wave's loads complete in issue order).  Results are those
// of stage_x.

// Raw chunk registers: for chunk c0 = tid and c1 = tid + 256, the x words
// (I8: a[0], a[1]; F16: a[0..1], a[2..3]; F32: a[0..3], a[4..7]; RELU2: gate
// a[0..1], a[2..3] and up a[4..5], a[6..7]) and gamma's (g[0..1], g[2..3]).
struct XRaw {
    u32x4 a[8];
    u32x4 g[4];
};

constexpr bool kind_rms(int kind) { return kind != TER_HIP_X_F32 && kind != TER_HIP_X_I8; }
// Bytes of one x element of a kind (gate's for X_RELU2_RMS).
constexpr int kind_bytes(int kind) {
    return kind == TER_HIP_X_I8 ? 1
                                : ((kind == TER_HIP_X_F32 || kind == TER_HIP_X_F32_RMS || kind == TER_HIP_X_SMUL) ? 4 : 2);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t vec_rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}

__device__ __forceinline__ u32x4 vload(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// Loads of chunk c into a[j0 ..] (x) and a[j0 + 4 ..] (up).
template <int kKind>
__device__ __forceinline__ void vload_chunk(__amdgpu_buffer_rsrc_t rx, __amdgpu_buffer_rsrc_t ru, int c, u32x4* a) {
    constexpr int L = kind_bytes(kKind);  // dwordx4 loads per 16 elements
#pragma unroll
    for (int j = 0; j < L; ++j) a[j] = vload(rx, c * 16 * L + 16 * j);
    if constexpr (kKind == TER_HIP_X_RELU2_RMS) {
#pragma unroll
        for (int j = 0; j < 2; ++j) a[4 + j] = vload(ru, c * 32 + 16 * j);
    }
}

__device__ __forceinline__ void halves_to_float(const u32x4* w, float (&v)[16]) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[8 * j + 2 * i] = half_bits_to_float((uint16_t)(w[j][i] & 0xFFFFu));
            v[8 * j + 2 * i + 1] = half_bits_to_float((uint16_t)(w[j][i] >> 16));
        }
}

// 16 activations of chunk registers a (layout of vload_chunk) as fp32.
template <int kKind>
__device__ __forceinline__ void unpack_chunk(const u32x4* a, float (&v)[16]) {
    if constexpr (kKind == TER_HIP_X_F32 || kKind == TER_HIP_X_F32_RMS) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const unsigned w = a[j][i];  // (bit_cast of the element lvalue itself reads element 0)
                v[4 * j + i] = __builtin_bit_cast(float, w);
            }
    } else if constexpr (kKind == TER_HIP_X_F16_RMS) {
        halves_to_float(a, v);
    } else {
        float g[16], u[16];
        halves_to_float(a, g);
        halves_to_float(a + 4, u);
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = relu2_mul(g[i], u[i]);
    }
}

template <int kKind>
__device__ __forceinline__ void x_prefetch_vec(const GemvDesc& d, XRaw& r) {
    const int c0 = threadIdx.x, c1 = threadIdx.x + kGemvThreads;
    const __amdgpu_buffer_rsrc_t rx = vec_rsrc(d.x, d.K * kind_bytes(kKind));
    if constexpr (kKind == TER_HIP_X_I8) {
        r.a[0] = vload(rx, c0 * 16);
        r.a[1] = vload(rx, c1 * 16);
        return;
    }
    const __amdgpu_buffer_rsrc_t ru = vec_rsrc(d.up, d.K * 2);
    if constexpr (kKind == TER_HIP_X_F32 || kKind == TER_HIP_X_F32_RMS) {
        vload_chunk<kKind>(rx, ru, c0, r.a);
        vload_chunk<kKind>(rx, ru, c1, r.a + 4);
    } else {
        // two-load chunks: x (gate) in a[0..3], up in a[4..7]
        u32x4 t[8];
        vload_chunk<kKind>(rx, ru, c0, t);
        r.a[0] = t[0];
        r.a[1] = t[1];
        if constexpr (kKind == TER_HIP_X_RELU2_RMS) {
            r.a[4] = t[4];
            r.a[5] = t[5];
        }
        vload_chunk<kKind>(rx, ru, c1, t);
        r.a[2] = t[0];
        r.a[3] = t[1];
        if constexpr (kKind == TER_HIP_X_RELU2_RMS) {
            r.a[6] = t[4];
            r.a[7] = t[5];
        }
    }
    if constexpr (kind_rms(kKind)) {
        const __amdgpu_buffer_rsrc_t rg = vec_rsrc(d.gamma, d.K * 2);
        r.g[0] = vload(rg, c0 * 32);
        r.g[1] = vload(rg, c0 * 32 + 16);
        r.g[2] = vload(rg, c1 * 32);
        r.g[3] = vload(rg, c1 * 32 + 16);
    }
}

// Chunk `which` (0: c0, 1: c1) of the prefetched registers as fp32.
template <int kKind>
__device__ __forceinline__ void prefetched_chunk(const XRaw& r, int which, float (&v)[16]) {
    if constexpr (kKind == TER_HIP_X_F32 || kKind == TER_HIP_X_F32_RMS) {
        unpack_chunk<kKind>(r.a + 4 * which, v);
    } else {
        u32x4 t[8];
        t[0] = r.a[2 * which];
        t[1] = r.a[2 * which + 1];
        if constexpr (kKind == TER_HIP_X_RELU2_RMS) {
            t[4] = r.a[4 + 2 * which];
            t[5] = r.a[5 + 2 * which];
        }
        unpack_chunk<kKind>(t, v);
    }
}

// Sum over 256 threads in the order of tree_sum256, with one barrier: every
// wave reads all 256 partials and reduces levels 128 and 64 as
// (v[l] + v[l + 128]) + (v[l + 64] + v[l + 192]), then the wave's own
// levels 32 .. 1.  `red` must not be written again before a later barrier.
__device__ __forceinline__ float tree_sum256_all(float v, float* red) {
    const int t = threadIdx.x, l = t & 63;
    red[t] = v;
    __syncthreads();
    return tree_down64((red[l] + red[l + 128]) + (red[l + 64] + red[l + 192]));
}

template <int kKind>
__device__ __forceinline__ float stage_x_vec(const GemvDesc& d, const XRaw& r, int8_t* lds_x, int* usum, float* red,
                                             float* xs32, bool owner) {
#pragma clang fp contract(off)
    const int K = d.K;
    const int nchunks = d.Ku * (kUnitK / 16);
    const int tid = threadIdx.x;
    const int c0 = tid, c1 = tid + kGemvThreads;
    const __amdgpu_buffer_rsrc_t rx = vec_rsrc(d.x, K * kind_bytes(kKind));
    if constexpr (kKind == TER_HIP_X_I8) {
        if (c0 < nchunks) put_chunk(c0, r.a[0], lds_x, usum);
        if (c1 < nchunks) put_chunk(c1, r.a[1], lds_x, usum);
        for (int c = tid + 2 * kGemvThreads; c < nchunks; c += kGemvThreads) put_chunk(c, vload(rx, c * 16), lds_x, usum);
        return d.x_scale_dev ? *gptr(d.x_scale_dev) : d.x_scale;
    } else {
        const __amdgpu_buffer_rsrc_t ru = vec_rsrc(d.up, K * 2);
        const __amdgpu_buffer_rsrc_t rg = vec_rsrc(d.gamma, K * 2);
        constexpr bool rms = kind_rms(kKind);
        float v0[16], v1[16];
        prefetched_chunk<kKind>(r, 0, v0);
        prefetched_chunk<kKind>(r, 1, v1);
        // chunk c (beyond the prefetched two) as fp32, normalized for the RMS kinds
        auto far_chunk = [&](int c, float rms_inv, float (&t)[16]) {
            if constexpr (rms) {
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    const f32x4 f = *reinterpret_cast<const f32x4*>(xs32 + c * 16 + i);
                    t[i] = f[0]; t[i + 1] = f[1]; t[i + 2] = f[2]; t[i + 3] = f[3];
                }
                const u32x4 gw[2] = {vload(rg, c * 32), vload(rg, c * 32 + 16)};
                float g[16];
                halves_to_float(gw, g);
#pragma unroll
                for (int i = 0; i < 16; ++i) t[i] = (t[i] * rms_inv) * g[i];
            } else {
                u32x4 a[8];
                vload_chunk<kKind>(rx, ru, c, a);
                unpack_chunk<kKind>(a, t);
            }
        };
        float rms_inv = 1.0f;
        if constexpr (rms) {
            auto put16 = [&](int c, const float (&v)[16]) {
#pragma unroll
                for (int i = 0; i < 16; i += 4)
                    *reinterpret_cast<f32x4*>(xs32 + c * 16 + i) = f32x4{v[i], v[i + 1], v[i + 2], v[i + 3]};
            };
            if (c0 < nchunks) put16(c0, v0);
            if (c1 < nchunks) put16(c1, v1);
            for (int c = tid + 2 * kGemvThreads; c < nchunks; c += kGemvThreads) {
                u32x4 a[8];
                vload_chunk<kKind>(rx, ru, c, a);
                float t[16];
                unpack_chunk<kKind>(a, t);
                put16(c, t);
            }
            __syncthreads();
            float ss;
            if constexpr (kKind == TER_HIP_X_RELU2_RMS) {
                // 1024 virtual threads (relu2_sum_sq_1024's order)
                float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
                for (int i = tid; i < K; i += 4 * kGemvThreads) {
                    const float a = xs32[i];
                    const float b = i + 256 < K ? xs32[i + 256] : 0.f;
                    const float c = i + 512 < K ? xs32[i + 512] : 0.f;
                    const float e = i + 768 < K ? xs32[i + 768] : 0.f;
                    p0 = __builtin_fmaf(a, a, p0);
                    p1 = __builtin_fmaf(b, b, p1);  // past K: +0, which changes no sum
                    p2 = __builtin_fmaf(c, c, p2);
                    p3 = __builtin_fmaf(e, e, p3);
                }
                ss = tree_sum256_all((p0 + p2) + (p1 + p3), red);
            } else {
                float part = 0.f;
                for (int i = tid; i < K; i += kGemvThreads) {
                    const float v = xs32[i];
                    part = __builtin_fmaf(v, v, part);
                }
                ss = tree_sum256_all(part, red);
            }
            rms_inv = 1.0f / __builtin_sqrtf(ss / (float)K + d.eps);
            float g0[16], g1[16];
            halves_to_float(r.g, g0);
            halves_to_float(r.g + 2, g1);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                v0[i] = (v0[i] * rms_inv) * g0[i];
                v1[i] = (v1[i] * rms_inv) * g1[i];
            }
        }
        float m = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) m = fmaxf(m, fmaxf(fabsf(v0[i]), fabsf(v1[i])));  // zeros past the chunks
        for (int c = tid + 2 * kGemvThreads; c < nchunks; c += kGemvThreads) {
            float t[16];
            far_chunk(c, rms_inv, t);
#pragma unroll
            for (int i = 0; i < 16; ++i) m = fmaxf(m, fabsf(t[i]));
        }
        m = wave_max(m);
        float* wmax = red + kGemvThreads;  // apart from the sum's slots, which other waves may still read
        if ((tid & 63) == 0) wmax[tid >> 6] = m;
        __syncthreads();
        m = wmax[0];
#pragma unroll
        for (int i = 1; i < kGemvWaves; ++i) m = fmaxf(m, wmax[i]);
        const float amax = m + 1e-9f;
        const float scale = 127.0f / amax;
        const float act = 1.0f / scale;
        for (int c = tid; c < nchunks; c += kGemvThreads) {
            u32x4 q;
            if (c == c0) {
                q = pack_q16(v0, scale);
            } else if (c == c1) {
                q = pack_q16(v1, scale);
            } else {
                float t[16];
                far_chunk(c, rms_inv, t);
                q = pack_q16(t, scale);
            }
            put_chunk(c, q, lds_x, usum);
            if (owner && d.xq_out) {
                const int k = c * 16;
                const unsigned qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (k + i < K) gptr(d.xq_out)[k + i] = (int8_t)((qw[i >> 2] >> (8 * (i & 3))) & 0xFFu);
            }
        }
        if (owner && tid == 0 && d.xs_out) *gptr(d.xs_out) = act;
        return act;
    }
}

// Strided prologue of the RMS kinds in strip mode (the decode step's plans).
// Thread t reads the values t + 256 j of x (and up) and gamma straight from
// memory (range-checked buffer loads: zeros past K), for j < kMaxStridedKu:
// those are exactly the values of its partial sum of squares in the
// reference's order (X_RELU2_RMS: virtual threads t + 256 (j mod 4)), so the
// sum needs no staging round.  The values also go to LDS (xs32, gs16) for the
// quantization.  Then, with two workgroup barriers where stage_x_vec has
// four: the partials meet in `red` (barrier), every wave forms the block tree
// (tree_sum256_all's operands) and the absmax of its threads' normalized
// values; the wave maxima meet (barrier); each wave quantizes only its own
// units [u0, u1), the ones its GEMV loop reads (rows r of the wave take units
// u0 + r, u0 + r + 4, ...), so a wave-level fence orders them before the loop.
// Results are stage_x_vec's bit for bit.  Needs Ku <= kMaxStridedKu and the
// fp32 staging (stage32); gs16: fp16 gamma [Ku*256] in LDS.
template <int kKind>
constexpr int max_strided_ku() {
    return kKind == TER_HIP_X_RELU2_RMS || kKind == TER_HIP_X_SILU_MUL || kKind == TER_HIP_X_SMUL ? 32 : 16;
}
// Waves per workgroup of the strided strip kernel: 8 for the down
// projections' kinds X_RELU2_RMS and X_SILU_MUL (their prologue over F values
// and the 27- or 32-unit strips keep one wave per SIMD busy for
// microseconds; a second wave per SIMD shares both), 4 for the 256-thread
// kinds, whose partials are the 256 threads'.
#ifndef TER_STRIDED_RELU2_WAVES
#define TER_STRIDED_RELU2_WAVES 8
#endif
template <int kKind>
constexpr int strided_waves() {
    return kKind == TER_HIP_X_RELU2_RMS || kKind == TER_HIP_X_SILU_MUL || kKind == TER_HIP_X_SMUL
               ? TER_STRIDED_RELU2_WAVES
               : 4;
}

// Registers of the strided prologue.  The 256-thread kinds: x and gamma of
// values t + T j.  X_RELU2_RMS: thread t owns the V = 1024 / T consecutive
// virtual threads V t .. V t + V - 1 and reads their values V t + 1024 j as
// one V-half vector each (gate, up and gamma: V = 4 a dwordx2, V = 2 a dword).
// The absmax kinds X_F16, X_SILU_MUL and X_SMUL (no sum, so no order to
// keep): x (and up) of values 8 t + 8 T j, 8 halves per dwordx4 (X_SMUL: 8
// fp32 x values in two).
template <int kKind, int kW>
struct XStrided {
    static constexpr int T = 64 * kW;
    static constexpr bool R2 = kKind == TER_HIP_X_RELU2_RMS;
    static constexpr bool ABS = kKind == TER_HIP_X_F16 || kKind == TER_HIP_X_SILU_MUL || kKind == TER_HIP_X_SMUL;
    static constexpr bool UP = R2 || kKind == TER_HIP_X_SILU_MUL || kKind == TER_HIP_X_SMUL;
    static constexpr int V = R2 ? 1024 / T : (ABS ? 8 : 1);                                  // values per load
    static constexpr int J = max_strided_ku<kKind>() * kUnitK / (R2 ? 1024 : (ABS ? 8 * T : T));  // loads per operand
    static constexpr int DW = R2 ? (V + 1) / 2 : (ABS ? 4 : 1);                               // dwords per load
    static constexpr int DX = kKind == TER_HIP_X_SMUL ? 8 : DW;                              // dwords of x per load
    unsigned x[J][DX];  // fp32 bits (X_F32_RMS, X_SMUL) or fp16 bits (X_F16_RMS, X_F16; the gate of X_RELU2_RMS / X_SILU_MUL)
    unsigned u[UP ? J : 1][DW];  // up (X_RELU2_RMS, X_SILU_MUL)
    unsigned g[ABS ? 1 : J][DW];  // gamma (fp16 bits; the RMS kinds)
};

template <int DW>
__device__ __forceinline__ void load_halves(__amdgpu_buffer_rsrc_t r, int off, unsigned (&o)[DW]) {
    if constexpr (DW == 4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
        o[0] = v.x;
        o[1] = v.y;
        o[2] = v.z;
        o[3] = v.w;
    } else if constexpr (DW == 2) {
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
        o[0] = v.x;
        o[1] = v.y;
    } else {
        o[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    }
}

template <int kKind, int kW>
__device__ __forceinline__ void x_prefetch_strided(const GemvDesc& d, XStrided<kKind, kW>& r) {
    using XS = XStrided<kKind, kW>;
    constexpr int J = XS::J, T = XS::T;
    const int t = threadIdx.x;
    const __amdgpu_buffer_rsrc_t rx = vec_rsrc(d.x, d.K * kind_bytes(kKind));
    if constexpr (XS::ABS) {
        // (K is a multiple of 16: a vector is either inside K or reads as zeros)
#pragma unroll
        for (int j = 0; j < J; ++j) {
            if constexpr (kKind == TER_HIP_X_SMUL) {
                const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rx, 4 * (8 * t + 8 * T * j), 0, 0);
                const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(rx, 4 * (8 * t + 8 * T * j) + 16, 0, 0);
                r.x[j][0] = a.x; r.x[j][1] = a.y; r.x[j][2] = a.z; r.x[j][3] = a.w;
                r.x[j][4] = b.x; r.x[j][5] = b.y; r.x[j][6] = b.z; r.x[j][7] = b.w;
            } else {
                load_halves(rx, 2 * (8 * t + 8 * T * j), r.x[j]);
            }
        }
        if constexpr (XS::UP) {
            const __amdgpu_buffer_rsrc_t ru = vec_rsrc(d.up, d.K * 2);
#pragma unroll
            for (int j = 0; j < J; ++j) load_halves(ru, 2 * (8 * t + 8 * T * j), r.u[j]);
        }
        return;
    }
    const __amdgpu_buffer_rsrc_t rg = vec_rsrc(d.gamma, d.K * 2);
    if constexpr (XS::R2) {
        // (a vector past K reads as zeros: K is a multiple of 16, so a vector
        // is either inside or wholly past it)
        const __amdgpu_buffer_rsrc_t ru = vec_rsrc(d.up, d.K * 2);
#pragma unroll
        for (int j = 0; j < J; ++j) load_halves(rx, 2 * (XS::V * t + 1024 * j), r.x[j]);
#pragma unroll
        for (int j = 0; j < J; ++j) load_halves(ru, 2 * (XS::V * t + 1024 * j), r.u[j]);
#pragma unroll
        for (int j = 0; j < J; ++j) load_halves(rg, 2 * (XS::V * t + 1024 * j), r.g[j]);
    } else {
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int i = t + T * j;
            if constexpr (kKind == TER_HIP_X_F32_RMS)
                r.x[j][0] = __builtin_amdgcn_raw_buffer_load_b32(rx, 4 * i, 0, 0);
            else
                r.x[j][0] = __builtin_amdgcn_raw_buffer_load_b16(rx, 2 * i, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < J; ++j) r.g[j][0] = __builtin_amdgcn_raw_buffer_load_b16(rg, 2 * (t + T * j), 0, 0);
    }
}

// Strided prologue of the RMS kinds in strip mode (the decode step's plans).
// Every thread reads straight from memory (range-checked buffer loads: zeros
// past K) the values of its own partial sums of squares in the reference's
// order: the 256 threads' partials for X_F32_RMS / X_F16_RMS (thread t: the
// values t + 256 j), the 1024 virtual threads' for X_RELU2_RMS (thread t of
// T: virtual threads V t .. V t + V - 1, V = 1024 / T, values v + 1024 j),
// each a fused multiply-add chain over increasing j.  So the sum needs no
// staging round; the values also go to LDS (xs32, gs16) for the
// quantization.  Then, with two workgroup barriers where stage_x_vec has
// four: the partials meet in `red` (barrier), every wave forms
// tree_sum256_all's operands (the 1024 virtual partials of a thread t' of 256
// paired as (p(t') + p(t' + 512)) + (p(t' + 256) + p(t' + 768)) first) and
// the absmax of its threads' normalized values; the wave maxima meet
// (barrier); each wave quantizes only its own units [u0, u1), the ones its
// GEMV loop reads (rows r of the wave take units u0 + r, u0 + r + 4, ...), so
// a wave-level fence orders them before the loop.  Results are stage_x_vec's
// bit for bit.  Needs Ku <= max_strided_ku and the fp32 staging (stage32);
// gs16: fp16 gamma [Ku*256], red: 1024 + 16 floats.
template <int kKind, int kW>
__device__ __forceinline__ float stage_x_strided(const GemvDesc& d, const XStrided<kKind, kW>& r, int8_t* lds_x,
                                                 int* usum, float* red, float* xs32, uint16_t* gs16, int u0, int u1,
                                                 bool owner) {
#pragma clang fp contract(off)
    using XS = XStrided<kKind, kW>;
    constexpr int J = XS::J, T = XS::T, V = XS::V;
    static_assert(XS::R2 ? (T == 256 || T == 512) : T == 256, "thread count");
    const int K = d.K, Ku = d.Ku;
    const int t = threadIdx.x, lane = t & 63;
    float x[J][V], gm[J][V];
    float P[V];
#pragma unroll
    for (int e = 0; e < V; ++e) P[e] = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
        for (int e = 0; e < V; ++e) {
            const uint16_t gh = (uint16_t)(r.g[j][e >> 1] >> (16 * (e & 1)));
            gm[j][e] = half_bits_to_float(XS::R2 ? gh : (uint16_t)r.g[j][0]);
            if constexpr (kKind == TER_HIP_X_F32_RMS) {
                x[j][e] = __builtin_bit_cast(float, r.x[j][0]);
            } else if constexpr (kKind == TER_HIP_X_F16_RMS) {
                x[j][e] = half_bits_to_float((uint16_t)r.x[j][0]);
            } else {
                const uint16_t xh = (uint16_t)(r.x[j][e >> 1] >> (16 * (e & 1)));
                const uint16_t uh = (uint16_t)(r.u[j][e >> 1] >> (16 * (e & 1)));
                x[j][e] = relu2_mul(half_bits_to_float(xh), half_bits_to_float(uh));
            }
            P[e] = __builtin_fmaf(x[j][e], x[j][e], P[e]);  // past K: fma(0, 0, p) = p
            const int i = XS::R2 ? V * t + e + 1024 * j : t + T * j;
            if (i < Ku * kUnitK) {  // the staged range
                xs32[i] = x[j][e];
                gs16[i] = XS::R2 ? gh : (uint16_t)r.g[j][0];
            }
        }
    }
#pragma unroll
    for (int e = 0; e < V; ++e) red[XS::R2 ? V * t + e : t] = P[e];
    __syncthreads();
    auto q = [&](int i) {
        if constexpr (XS::R2)
            return (red[i] + red[i + 512]) + (red[i + 256] + red[i + 768]);
        else
            return red[i];
    };
    const float ss = tree_down64((q(lane) + q(lane + 128)) + (q(lane + 64) + q(lane + 192)));
    const float rms_inv = 1.0f / __builtin_sqrtf(ss / (float)K + d.eps);
    float mx = 0.f;  // zeros past K
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
        for (int e = 0; e < V; ++e) mx = fmaxf(mx, fabsf((x[j][e] * rms_inv) * gm[j][e]));
    mx = wave_max(mx);
    float* wmax = red + (XS::R2 ? 1024 : T);  // apart from the partials, which other waves may still read
    if (lane == 0) wmax[t >> 6] = mx;
    __syncthreads();
    mx = wmax[0];
#pragma unroll
    for (int i = 1; i < kW; ++i) mx = fmaxf(mx, wmax[i]);
    const float amax = mx + 1e-9f;
    const float scale = 127.0f / amax;
    const float act = 1.0f / scale;
    const int row = lane >> 4, qd = lane & 15;
    for (int u = u0 + row; u < u1; u += 4) {
        const int c = u * 16 + qd;
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const f32x4 f = *reinterpret_cast<const f32x4*>(xs32 + c * 16 + i);
            v[i] = f[0]; v[i + 1] = f[1]; v[i + 2] = f[2]; v[i + 3] = f[3];
        }
        const u32x4 gw[2] = {*reinterpret_cast<const u32x4*>(gs16 + c * 16),
                             *reinterpret_cast<const u32x4*>(gs16 + c * 16 + 8)};
        float g[16];
        halves_to_float(gw, g);
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = (v[i] * rms_inv) * g[i];
        const u32x4 qv = pack_q16(v, scale);
        *reinterpret_cast<u32x4*>(lds_x + c * 16) = qv;
        const int su = row_sum16(sum_bytes(qv));
        if (qd == 0) usum[u] = su;
        if (owner && d.xq_out) {
            const int k = c * 16;
            const unsigned qw[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (k + i < K) gptr(d.xq_out)[k + i] = (int8_t)((qw[i >> 2] >> (8 * (i & 3))) & 0xFFu);
        }
    }
    if (owner && t == 0 && d.xs_out) *gptr(d.xs_out) = act;
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    return act;
}

// Strided prologue of the absmax kinds in strip mode: X_F16 (quant_int8_k on
// an fp16 vector, cuda/ter_cuda_forward_packed.cu:40-62) and X_SILU_MUL
// (silu_mul_quant_k, :312-344).  Each thread turns the 8 t + 8 T j values it
// loaded into fp32 (silu(gate) * up), writes them to LDS (xs32) and folds
// their absmax; the wave maxima meet (one workgroup barrier, which also
// publishes xs32); each wave quantizes only its own units [u0, u1), as in
// stage_x_strided.  The maximum is order-free, so the results are stage_x's
// bit for bit.  Needs Ku <= max_strided_ku and the fp32 staging; red: kW floats.
template <int kKind, int kW>
__device__ __forceinline__ float stage_x_abs_strided(const GemvDesc& d, const XStrided<kKind, kW>& r, int8_t* lds_x,
                                                     int* usum, float* red, float* xs32, int u0, int u1, bool owner) {
#pragma clang fp contract(off)
    using XS = XStrided<kKind, kW>;
    constexpr int J = XS::J, T = XS::T;
    const int K = d.K, Ku = d.Ku;
    const int t = threadIdx.x, lane = t & 63;
    float mx = 0.f;  // zeros past K
#pragma unroll
    for (int j = 0; j < J; ++j) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if constexpr (kKind == TER_HIP_X_SMUL) {
                // silu(gate) (fp32, from the gate GEMV) times up
                v[e] = __builtin_bit_cast(float, r.x[j][e]) *
                       half_bits_to_float((uint16_t)(r.u[j][e >> 1] >> (16 * (e & 1))));
            } else {
                const float x = half_bits_to_float((uint16_t)(r.x[j][e >> 1] >> (16 * (e & 1))));
                if constexpr (kKind == TER_HIP_X_SILU_MUL)
                    v[e] = silu_mul(x, half_bits_to_float((uint16_t)(r.u[j][e >> 1] >> (16 * (e & 1)))));
                else
                    v[e] = x;  // past K: silu(0) * 0 = 0
            }
            mx = fmaxf(mx, fabsf(v[e]));
        }
        const int i = 8 * t + 8 * T * j;
        if (i < Ku * kUnitK) {  // the staged range (a multiple of 8)
            *reinterpret_cast<f32x4*>(xs32 + i) = f32x4{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<f32x4*>(xs32 + i + 4) = f32x4{v[4], v[5], v[6], v[7]};
        }
    }
    mx = wave_max(mx);
    if (lane == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int i = 1; i < kW; ++i) mx = fmaxf(mx, red[i]);
    const float amax = mx + 1e-9f;
    const float scale = 127.0f / amax;
    const float act = 1.0f / scale;
    const int row = lane >> 4, qd = lane & 15;
    for (int u = u0 + row; u < u1; u += 4) {
        const int c = u * 16 + qd;
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const f32x4 f = *reinterpret_cast<const f32x4*>(xs32 + c * 16 + i);
            v[i] = f[0]; v[i + 1] = f[1]; v[i + 2] = f[2]; v[i + 3] = f[3];
        }
        const u32x4 qv = pack_q16(v, scale);
        *reinterpret_cast<u32x4*>(lds_x + c * 16) = qv;
        const int su = row_sum16(sum_bytes(qv));
        if (qd == 0) usum[u] = su;
        if (owner && d.xq_out) {
            const int k = c * 16;
            const unsigned qw[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (k + i < K) gptr(d.xq_out)[k + i] = (int8_t)((qw[i >> 2] >> (8 * (i & 3))) & 0xFFu);
        }
    }
    if (owner && t == 0 && d.xs_out) *gptr(d.xs_out) = act;
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    return act;
}

__device__ __forceinline__ void emit(const GemvDesc& d, int col, int val, float s) { emit_out(d, col, val, s); }

// Accumulate 1 tile (16 bytes of this lane) into the 4 column accumulators.
__device__ __forceinline__ void dot_tile(const u32x4& w, const u32x4& x, int (&a1)[4], int (&a4)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned dw = w[j];
        const unsigned d4 = dw >> 4;
        a1[j] = __builtin_amdgcn_sdot4((int)x.x, (int)(dw & 0x03030303u), a1[j], false);
        a4[j] = __builtin_amdgcn_sdot4((int)x.y, (int)(dw & 0x0C0C0C0Cu), a4[j], false);
        a1[j] = __builtin_amdgcn_sdot4((int)x.z, (int)(d4 & 0x03030303u), a1[j], false);
        a4[j] = __builtin_amdgcn_sdot4((int)x.w, (int)(d4 & 0x0C0C0C0Cu), a4[j], false);
    }
}

// Column value of a strip (lanes with q < 4 own column 4 r + q); clears the
// accumulators.  `corr` is the activation sum over the strip's units (the
// u = w + 1 encoding adds it to every column).
__device__ __forceinline__ int reduce_strip(int (&a1)[4], int (&a4)[4], int corr) {
    const int q = threadIdx.x & 15;
    int v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = row_sum16(a1[j] + (a4[j] >> 2));
#pragma unroll
    for (int j = 0; j < 4; ++j) a1[j] = a4[j] = 0;
    return (q == 0 ? v[0] : (q == 1 ? v[1] : (q == 2 ? v[2] : v[3]))) - corr;
}

__device__ __forceinline__ int strip_col(int st) {
    const int lane = threadIdx.x & 63;
    return st * kStripCols + (lane >> 4) * 4 + (lane & 15);
}

__device__ __forceinline__ bool col_owner(const GemvDesc& d, int st) {
    return (threadIdx.x & 15) < 4 && strip_col(st) < d.N;
}

// Fix-up slot word: units << 40 plus the signed partial sum.
__device__ __forceinline__ unsigned long long part_word(int units, int val) {
    return ((unsigned long long)units << 40) + (unsigned long long)(long long)val;
}

__device__ __forceinline__ unsigned long long part_add(const GemvDesc& d, int col, unsigned long long w) {
    return __hip_atomic_fetch_add(gptr(d.fix) + col, w,
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// After this wave's add: if the slot now counts all Ku units, write the
// column and clear the slot for the next launch.
__device__ __forceinline__ void part_complete(const GemvDesc& d, int col, unsigned long long tot_u, float s) {
    const long long tot = (long long)tot_u;
    const long long units = (tot + (1LL << 39)) >> 40;
    if (units == (long long)d.Ku) {
        __hip_atomic_store(gptr(d.fix) + col, 0ull, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        emit(d, col, (int)(tot - (units << 40)), s);
    }
}

// The tile offset goes into the vector offset: the buffer's range check
// covers the vector and immediate offsets but not the scalar one, and loads
// past the piece must read zeros rather than whatever memory follows it.
__device__ __forceinline__ u32x4 load_tile(__amdgpu_buffer_rsrc_t rs, int voff, int tile) {
    return __builtin_amdgcn_raw_buffer_load_b128(rs, voff + tile * kTileBytes, 0, 2 /* nt */);
}

template <int NB>
__device__ __forceinline__ void load_batch(u32x4 (&w)[NB], __amdgpu_buffer_rsrc_t rs, int voff, int i0) {
#pragma unroll
    for (int i = 0; i < NB; ++i) w[i] = load_tile(rs, voff, i0 + i);
}

struct Piece {
    int st, u, u_start, corr;
    int first_val, first_units, first_st;  // the leading partial strip, combined after the loop
    bool has_first;
    int nout;  // strips completed within the piece so far
    int a1[4], a4[4];
};

// Reduce tiles [i0, min(i0 + NB, n)) of the piece from registers `w`.
template <int NB>
__device__ __forceinline__ void compute_batch(const GemvDesc& d, const u32x4 (&w)[NB], int i0, int n,
                                              const int8_t* lds_x, const int* usum, float s, Piece& p, int* obuf) {
    const int q = threadIdx.x & 15;
    const int c = (threadIdx.x & 63) >> 4 << 2 | q;  // column within the strip of lanes q < 4
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        if (i0 + i < n) {
            const u32x4 xv = *reinterpret_cast<const u32x4*>(lds_x + p.u * kUnitK + q * 16);
            p.corr += usum[p.u];
            dot_tile(w[i], xv, p.a1, p.a4);
            ++p.u;
            if (p.u == d.Ku) {
                const int val = reduce_strip(p.a1, p.a4, p.corr);
                if (p.u_start == 0) {
                    if (q < 4) obuf[p.nout * kStripCols + c] = val;  // fewer than kGemvOutStrips per chunk
                    ++p.nout;
                } else {
                    p.first_val = val;
                    p.first_units = p.u - p.u_start;
                    p.first_st = p.st;
                    p.has_first = true;
                }
                p.st += 1;
                p.u = 0;
                p.u_start = 0;
                p.corr = 0;
            }
        }
    }
}

// The fix-up atomics of a piece's shared strips, issued but not yet checked:
// whether an add completed its column is examined only after the wave's next
// piece (or at its exit), so the atomics' round trip overlaps streaming.
struct Fixups {
    unsigned long long o_last, w_last, o_first, w_first;  // returned old values, added words
    int col_last, col_first;                              // -1: no add by this lane
    float s;
    float* y;
    int32_t* acc;
    uint16_t* y16;
    float* resid;
    uint16_t* resid16;
    unsigned long long* fix;
    int Ku, w_mag;
};

__device__ __forceinline__ void finish_fixups(const Fixups& f) {
#pragma clang fp contract(off)
    GemvDesc d{};
    d.y = f.y;
    d.acc = f.acc;
    d.y16 = f.y16;
    d.resid = f.resid;
    d.resid16 = f.resid16;
    d.fix = f.fix;
    d.Ku = f.Ku;
    d.w_mag = f.w_mag;
    if (f.col_last >= 0) part_complete(d, f.col_last, f.o_last + f.w_last, f.s);
    if (f.col_first >= 0) part_complete(d, f.col_first, f.o_first + f.w_first, f.s);
}

// The strips of a piece not complete within it (at most its first and its
// last), with the column sums of lanes q < 4; st = -1: none.
struct Partials {
    int st_first, units_first, val_first;
    int st_last, units_last, val_last;
};

// One wave streams local tiles [la, la + n) of GEMV d; `wa` holds the first
// batch already.  Strips complete within the piece are written; the others
// are returned.
template <int NB>
__device__ __forceinline__ Partials run_piece(const GemvDesc& d, const int8_t* lds_x, const int* usum, float s, int la,
                                              int n, __amdgpu_buffer_rsrc_t rs, int voff, u32x4 (&wa)[NB], int* obuf) {
    Piece p;
    p.st = la / d.Ku;
    p.u = la - p.st * d.Ku;
    p.u_start = p.u;
    p.corr = 0;
    p.first_val = p.first_units = p.first_st = 0;
    p.has_first = false;
    p.nout = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) p.a1[j] = p.a4[j] = 0;
    // The piece streams in chunks of C tiles, a whole number of double
    // batches and at most 15 Ku, so that a chunk completes at most 15 strips
    // (buffered in obuf); their outputs are written between chunks, and the
    // streaming loop itself issues no memory operation but the weight loads
    // (a store or another load among them makes the compiler drain every
    // load at the loop head).  The next chunk's first batch is in flight
    // meanwhile.
    const int C = 2 * NB * max(1, (kGemvOutStrips - 1) * d.Ku / (2 * NB));
    int st_full = p.u == 0 ? p.st : p.st + 1;  // strip of the next buffered completion
    u32x4 wb[NB];
    int i0 = 0;
    while (true) {
        const int cend = min(n, i0 + C);
        while (true) {
            load_batch(wb, rs, voff, i0 + NB);
            compute_batch(d, wa, i0, n, lds_x, usum, s, p, obuf);
            i0 += NB;
            if (i0 >= cend) break;  // only at the piece's end (cend < n is a whole double batch)
            load_batch(wa, rs, voff, i0 + NB);
            compute_batch(d, wb, i0, n, lds_x, usum, s, p, obuf);
            i0 += NB;
            if (i0 >= cend) break;
        }
        // the chunk's completed strips, four per store across the wave's 64
        // lanes (256 contiguous output bytes); a wave reads back only its own
        // LDS writes
        for (int j0 = 0; j0 < p.nout; j0 += 4) {
            const int j = j0 + ((threadIdx.x & 63) >> 4);
            const int col = (st_full + j) * kStripCols + (threadIdx.x & 15);
            if (j < p.nout && col < d.N) emit(d, col, obuf[j * kStripCols + (threadIdx.x & 15)], s);
        }
        p.nout = 0;
        st_full = p.u_start != 0 ? p.st + 1 : p.st;
        if (i0 >= n) break;
        // Another chunk: let the outputs (and a residual's read) complete
        // first, so the streaming loop never starts with them pending (the
        // compiler would then drain all loads at every loop head).
        __builtin_amdgcn_s_waitcnt(0);
    }
    Partials r;
    r.st_first = p.has_first ? p.first_st : -1;
    r.units_first = p.first_units;
    r.val_first = p.first_val;
    r.st_last = -1;
    r.units_last = r.val_last = 0;
    if (p.u != p.u_start) {
        r.st_last = p.st;
        r.units_last = p.u - p.u_start;
        r.val_last = reduce_strip(p.a1, p.a4, p.corr);
    }
    return r;
}

// After a segment: every wave has put its Partials in the slots (slot 2 w:
// first, 2 w + 1: last) and passed a barrier.  The first slot holding a strip
// adds the partials of every slot holding it (integer sums, so the result is
// the same in any order).  A strip with all Ku units is written; one that
// also spans another workgroup's range (a range end not on a strip edge) goes
// to the global fix-up slot with one atomic per column, whose result is
// examined later (finish_fixups).
__device__ __forceinline__ Fixups no_fixups(const GemvDesc& d, float s) {
    Fixups f;
    f.o_last = f.w_last = f.o_first = f.w_first = 0;
    f.col_last = f.col_first = -1;
    f.s = s;
    f.y = d.y;
    f.acc = d.acc;
    f.y16 = d.y16;
    f.resid = d.resid;
    f.resid16 = d.resid16;
    f.fix = d.fix;
    f.Ku = d.Ku;
    f.w_mag = d.w_mag;
    return f;
}

// Small pieces (no combine_mode): the wave adds its own partial strips to the
// global fix-up slots.
__device__ __forceinline__ Fixups partials_to_slots(const GemvDesc& d, const Partials& pr, float s) {
    Fixups f = no_fixups(d, s);
    if (pr.st_first >= 0 && col_owner(d, pr.st_first)) {
        f.col_first = strip_col(pr.st_first);
        f.w_first = part_word(pr.units_first, pr.val_first);
        f.o_first = part_add(d, f.col_first, f.w_first);
    }
    if (pr.st_last >= 0 && col_owner(d, pr.st_last)) {
        f.col_last = strip_col(pr.st_last);
        f.w_last = part_word(pr.units_last, pr.val_last);
        f.o_last = part_add(d, f.col_last, f.w_last);
    }
    return f;
}

// Combine mode: the strips a segment's waves share meet in LDS slots without
// a workgroup barrier.  The segment's boundaries b_0 .. b_4 (local tiles:
// the workgroup's start, the wave boundaries, its end) are known to every
// wave; a strip holding boundary b strictly inside gets slot b, or the slot
// of the lowest boundary inside the same strip.  Slot j = [unit count, 16
// column sums], zeroed while the activations are staged.  A wave adds its
// partial column sums (ds_add), then its unit count with one workgroup-scope
// acquire-release add; the add that brings the count to the strip's units
// within the segment completes it: that wave reads the sums and writes the
// column (all Ku units here), or adds it to the global fix-up slot (the strip
// continues in another workgroup's range).  Integer sums, so the result does
// not depend on which wave completes.
constexpr int kSlotInts = 1 + kStripCols;
static_assert((kGemvWaves + 1) * kSlotInts * 4 <= kGemvSlotBytes, "combine slots fit the slot area");

struct SegBounds {
    int b[kGemvWaves + 1];  // local tiles of the segment's boundaries
    int Ku;
};

// Slot of the partial strip `st` holding boundary `from` strictly inside it:
// the lowest boundary of the run of boundaries inside that strip.  (Constant
// indices only, so the bounds stay in scalar registers.)
__device__ __forceinline__ int strip_slot(const SegBounds& sb, int from, int st) {
    int j = from;
    bool run = true;
#pragma unroll
    for (int w = kGemvWaves - 1; w >= 0; --w) {
        if (w < from) {
            const bool in = sb.b[w] % sb.Ku != 0 && sb.b[w] / sb.Ku == st;
            if (run && in)
                j = w;
            else
                run = false;
        }
    }
    return j;
}

__device__ __forceinline__ void slot_finish(const GemvDesc& d, int* slots, const SegBounds& sb, int from, int st,
                                            int units, int val, float s, int& col_out, unsigned long long& w_out,
                                            unsigned long long& o_out) {
    const int lane = threadIdx.x & 63;
    const int c = (lane >> 4) * 4 + (lane & 15);  // column within the strip of lanes q < 4
    int* sl = slots + strip_slot(sb, from, st) * kSlotInts;
    const int lo = st * sb.Ku > sb.b[0] ? st * sb.Ku : sb.b[0];
    const int hi = (st + 1) * sb.Ku < sb.b[kGemvWaves] ? (st + 1) * sb.Ku : sb.b[kGemvWaves];
    const int expect = hi - lo;  // units of the strip within the segment
    if ((lane & 15) < 4) __hip_atomic_fetch_add(sl + 1 + c, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    int old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(sl, units, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    old = uniform(old);
    if (old + units != expect) return;
    const int tot = (lane & 15) < 4 ? __hip_atomic_load(sl + 1 + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) : 0;
    if (!col_owner(d, st)) return;
    if (expect == d.Ku) {
        emit(d, strip_col(st), tot, s);
    } else {
        col_out = strip_col(st);
        w_out = part_word(expect, tot);
        o_out = part_add(d, col_out, w_out);
    }
}

__device__ __forceinline__ Fixups combine_partials(const GemvDesc& d, int* slots, const SegBounds& sb,
                                                   const Partials& pr, float s) {
    const int wave = uniform(threadIdx.x >> 6);
    Fixups f = no_fixups(d, s);
    if (pr.st_first >= 0)
        slot_finish(d, slots, sb, wave, pr.st_first, pr.units_first, pr.val_first, s, f.col_first, f.w_first,
                    f.o_first);
    if (pr.st_last >= 0)
        slot_finish(d, slots, sb, wave + 1, pr.st_last, pr.units_last, pr.val_last, s, f.col_last, f.w_last,
                    f.o_last);
    return f;
}

// kList: GEMVs come from the device table `list` (plan launches) with the
// workgroup ranges `ranges`; otherwise the single descriptor is a kernel
// argument.  Two instantiations keep the descriptor in scalar registers
// either way.  kKind >= 0: every GEMV has that activation kind and qualifies
// for the vector prologue; -1: any kind.
template <bool kList, int kKind>
__global__ __launch_bounds__(kGemvThreads) __attribute__((amdgpu_waves_per_eu(gemv_waves_per_eu<kKind>())))
void gemv_t16_kernel(GemvDesc single,
                                                            const GemvDesc* __restrict__ list,
                                                            const int32_t* __restrict__ first,
                                                            const long long* __restrict__ ranges,
                                                            long long total, int n_wg) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    int g = blockIdx.x;
    if ((n_wg & 7) == 0) g = (g & 7) * (n_wg >> 3) + (g >> 3);  // keep neighbouring ranges on one XCD
    long long t_begin, t_end;
    int di = 0;  // the descriptor holding tile t_begin
    if constexpr (kList) {
        // all three loads issued together, ahead of the range test
        di = first[g];
        t_begin = ranges[g];
        t_end = ranges[g + 1];
    } else {
        t_begin = total * g / n_wg;
        t_end = total * (g + 1) / n_wg;
        if (snap_ranges(single.Ku, total, n_wg)) {
            t_begin = strip_edge_near(t_begin, single.Ku);
            t_end = strip_edge_near(t_end, single.Ku);
        }
    }
    // (di < 0, a null list and total < 0 never happen: they keep first[g]
    // among the loads above and the list pointer and total in the first
    // round of argument loads, so the descriptor is the third round)
    if (t_begin >= t_end || di < 0 || (kList && list == nullptr) || total < 0) return;

    const bool combine = combine_mode(total, n_wg);  // the waves' partial strips meet in LDS
    const int wave = uniform(threadIdx.x >> 6);
    const int voff = (threadIdx.x & 63) * 16;
    long long t = t_begin;
    Fixups prev;
    bool have_prev = false;
    while (t < t_end) {
        const GemvDesc d = kList ? list[di] : single;
        const long long seg_end = min(t_end, d.tile0 + (long long)d.n_strips * d.Ku);
        const long long nseg = seg_end - t;
        const int la = (int)(t + nseg * wave / kGemvWaves - d.tile0);
        const int lb = (int)(t + nseg * (wave + 1) / kGemvWaves - d.tile0);
        const int n = lb - la;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(d.w + (long long)la * kTileBytes), 0, n * kTileBytes, 0x00020000);
        XPre xpre;
        XRaw xraw;
        if constexpr (kKind < 0)
            x_prefetch(d, xpre);      // activations first (see XPre)
        else
            x_prefetch_vec<kKind>(d, xraw);
        u32x4 wa[batch_of<kKind>()];
        load_batch(wa, rs, voff, 0);  // in flight while the activations are staged
        int8_t* lds_x = reinterpret_cast<int8_t*>(lds_raw);
        int* usum = reinterpret_cast<int*>(lds_raw + d.Ku * kUnitK);
        float* red = reinterpret_cast<float*>(lds_raw + d.Ku * kUnitK + d.Ku * 4);
        float* xs32 = reinterpret_cast<float*>(lds_raw + gemv_lds_xs32_offset(d.K));
        int* slots = reinterpret_cast<int*>(lds_raw + gemv_lds_slots_offset(d.K, d.stage32 != 0));
        int* obuf = reinterpret_cast<int*>(lds_raw + gemv_lds_slots_offset(d.K, d.stage32 != 0) + kGemvSlotBytes) +
                    wave * kGemvOutStrips * kStripCols;
        __syncthreads();  // the previous segment is done with LDS
        float act;
        if constexpr (kKind < 0)
            act = stage_x(d, xpre, lds_x, usum, red, xs32, t == d.tile0);
        else
            act = stage_x_vec<kKind>(d, xraw, lds_x, usum, red, xs32, t == d.tile0);
        if (combine && threadIdx.x < (kGemvWaves + 1) * kSlotInts) slots[threadIdx.x] = 0;
        __syncthreads();
        const float s = act * d.w_scale;  // x_scale * w_scale (forward.cpp:342)
        Partials pr;
        pr.st_first = pr.st_last = -1;
        pr.units_first = pr.val_first = pr.units_last = pr.val_last = 0;
        if (n > 0) pr = run_piece(d, lds_x, usum, s, la, n, rs, voff, wa, obuf);
        Fixups f;
        if (!combine) {
            f = partials_to_slots(d, pr, s);
        } else {
            SegBounds sb;
            sb.Ku = d.Ku;
#pragma unroll
            for (int w = 0; w <= kGemvWaves; ++w) sb.b[w] = (int)(t + nseg * w / kGemvWaves - d.tile0);
            f = combine_partials(d, slots, sb, pr, s);
        }
        if (have_prev) finish_fixups(prev);
        prev = f;
        have_prev = true;
        t = seg_end;
        ++di;
    }
    if (have_prev) finish_fixups(prev);
}

// Strip mode, for work lists too small to keep the chip busy with whole
// strips per wave: workgroup g takes strips [S g / n_wg, S (g + 1) / n_wg) of
// the list's strip stream (S strips), and each strip's Ku units are split
// over the 4 waves (wave w: units [Ku w / 4, Ku (w + 1) / 4)).  A wave streams
// its units of every strip of a segment as one list of tiles, keeps each
// strip's partial column sums in LDS, and after a barrier wave j % 4 adds the
// four partials of strip j (integer sums, so the result is the stream-K
// kernel's) and writes the outputs.  No fix-up slots, no global atomics.
template <bool kList, int kKind, bool kStrided = false, int kW = kGemvWaves, bool kShared = false>
__global__ __launch_bounds__(64 * kW) void gemv_strip_kernel(GemvDesc single, const GemvDesc* __restrict__ list,
                                                                  const GemvDesc* __restrict__ wg_desc,
                                                                  long long total, int n_wg, int part_off) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    const int b = blockIdx.x;
    // kShared (strided lists): every GEMV of the list reads the one
    // activation vector `single` describes, and their tile streams follow
    // each other in memory from single.w (strip s at single.w + s Ku KiB).
    // Then the activation and weight loads need nothing but the kernel
    // arguments, and go out in the first round of loads after them, together
    // with the workgroup's descriptors, which only the outputs wait for.
    // The range is one segment; it spans at most two GEMVs, whose
    // descriptors wg_desc holds per block index (2 b: the first, 2 b + 1:
    // the next), so their loads need no argument but the table's address.
    static_assert(!kShared || (kList && kStrided), "shared lists run the strided prologue");
    GemvDesc e0{}, e1{};
    if constexpr (kShared) {
        e0 = wg_desc[2 * b];
        e1 = wg_desc[2 * b + 1];
        // every argument in one round of loads (an asm statement before the
        // descriptor loads would make them vector loads)
        asm volatile("" ::"s"(total), "s"(n_wg), "s"(single.w), "s"(single.x), "s"(single.gamma), "s"(single.up),
                     "s"(single.K), "s"(single.Ku), "s"(single.eps), "s"(single.stage32), "s"(single.strip0));
    }
    const int g = (n_wg & 7) == 0 ? (b & 7) * (n_wg >> 3) + (b >> 3) : b;  // neighbouring ranges on one XCD
    long long s_begin, s_end;
    if (total < (1LL << 20) && n_wg <= (1 << 11)) {
        // 32-bit division (a 64-bit one is about 150 scalar instructions)
        const unsigned t = (unsigned)total, n = (unsigned)n_wg;
        s_begin = t * (unsigned)g / n;
        s_end = t * (unsigned)(g + 1) / n;
    } else {
        s_begin = total * g / n_wg;
        s_end = total * (g + 1) / n_wg;
    }
    if (s_begin >= s_end) return;
    int di = 0;
    const int wave = uniform(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int voff = lane * 16;
    int* part = reinterpret_cast<int*>(lds_raw + part_off);  // [strip][wave][16 columns]
    long long sg = s_begin;
    while (sg < s_end) {
        // A plan's first segment reads the copy of its descriptor kept for
        // this workgroup (one round of loads instead of an index, then the
        // descriptor); later segments follow the list.
        const GemvDesc d = kShared ? single : (kList ? *(sg == s_begin ? wg_desc + g : list + di) : single);
        if constexpr (kList) di = d.self;
        const long long seg_end = kShared ? s_end : min(s_end, d.strip0 + (long long)d.n_strips);
        const int sa = (int)(sg - d.strip0);  // first strip of the segment within the GEMV
        const int ns = (int)(seg_end - sg);
        static_assert(kW == kGemvWaves || kStrided, "other wave counts run the strided prologue only");
        const int u0 = d.Ku * wave / kW;
        const int nw = d.Ku * (wave + 1) / kW - u0;  // units per strip of this wave
        const int n = nw * ns;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(d.w + (long long)sa * d.Ku * kTileBytes), 0, ns * d.Ku * kTileBytes, 0x00020000);
        // tile i of the wave's list: strip i / nw, unit u0 + i % nw; tracked
        // incrementally (jl, kl) for the loads, past n an out-of-range offset
        int jl = 0, kl = 0;
        auto next_off = [&]() {
            const int off = jl < ns ? ((jl * d.Ku + u0 + kl) * kTileBytes) : 0x7FFFF000 - voff;
            if (++kl == nw) {
                kl = 0;
                ++jl;
            }
            return off;
        };
        constexpr int NB = batch_of<kKind>();
        auto load_b = [&](u32x4 (&w)[NB]) {
#pragma unroll
            for (int i = 0; i < NB; ++i) w[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + next_off(), 0, 2);
        };
        XPre xpre;
        XRaw xraw;
        XStrided<kStrided ? kKind : TER_HIP_X_F32_RMS, kStrided ? kW : kGemvWaves> xst;
        if constexpr (kKind < 0)
            x_prefetch(d, xpre);
        else if constexpr (kStrided)
            x_prefetch_strided<kKind, kW>(d, xst);
        else
            x_prefetch_vec<kKind>(d, xraw);
        u32x4 wa[NB], wb[NB];
        if (nw > 0) load_b(wa);
        if constexpr (kShared) {
            // the descriptors the outputs need, in flight with the activation
            // and weight loads (left alone the compiler issues them at the
            // outputs, one more round trip at the end)
            asm volatile("" ::"s"(e0.y), "s"(e0.y16), "s"(e0.resid), "s"(e0.resid16), "s"(e0.acc),
                         "s"(e1.y), "s"(e1.y16), "s"(e1.resid), "s"(e1.resid16), "s"(e1.acc));
        }
        int8_t* lds_x = reinterpret_cast<int8_t*>(lds_raw);
        int* usum = reinterpret_cast<int*>(lds_raw + d.Ku * kUnitK);
        float* red = reinterpret_cast<float*>(lds_raw + d.Ku * kUnitK + d.Ku * 4);
        float* xs32 = reinterpret_cast<float*>(lds_raw + gemv_lds_xs32_offset(d.K));
        __syncthreads();  // the previous segment is done with LDS
        float act;
        if constexpr (kKind < 0) {
            act = stage_x(d, xpre, lds_x, usum, red, xs32, sg == d.strip0);
            __syncthreads();
        } else if constexpr (kStrided) {
            uint16_t* gs16 = reinterpret_cast<uint16_t*>(lds_raw + gemv_lds_slots_offset(d.K, true));
            float* red_s = reinterpret_cast<float*>(lds_raw + gemv_strip_red_offset(d.K));
            if constexpr (XStrided<kKind, kW>::ABS)
                act = stage_x_abs_strided<kKind, kW>(d, xst, lds_x, usum, red_s, xs32, u0, u0 + nw, sg == d.strip0);
            else
                act = stage_x_strided<kKind, kW>(d, xst, lds_x, usum, red_s, xs32, gs16, u0, u0 + nw,
                                                 sg == d.strip0);
        } else {
            act = stage_x_vec<kKind>(d, xraw, lds_x, usum, red, xs32, sg == d.strip0);
            __syncthreads();
        }
        const float s = act * d.w_scale;  // x_scale * w_scale (forward.cpp:342)
        const int q = lane & 15;
        const int pcol = (lane >> 4) * 4 + q;  // column within the strip of lanes q < 4
        if (nw == 0) {
            for (int j = 0; j < ns; ++j)
                if (q < 4) part[(j * kW + wave) * 16 + pcol] = 0;
        } else {
            int a1[4] = {0, 0, 0, 0}, a4[4] = {0, 0, 0, 0};
            int corr = 0, j = 0, k = 0;
            auto compute_b = [&](const u32x4 (&w)[NB], int i0) {
#pragma unroll
                for (int i = 0; i < NB; ++i) {
                    if (i0 + i < n) {
                        const int u = u0 + k;
                        const u32x4 xv = *reinterpret_cast<const u32x4*>(lds_x + u * kUnitK + q * 16);
                        corr += usum[u];
                        dot_tile(w[i], xv, a1, a4);
                        if (++k == nw) {
                            const int v = reduce_strip(a1, a4, corr);
                            if (q < 4) part[(j * kW + wave) * 16 + pcol] = v;
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
                i0 += NB;
                if (i0 >= n) break;
                load_b(wa);
                compute_b(wb, i0);
                i0 += NB;
                if (i0 >= n) break;
            }
        }
        __syncthreads();
        if constexpr (kShared) {
            // each strip's own GEMV: the workgroup's first or the next
            auto emit_strip = [&](const GemvDesc& e, int j) {
                const int col = (int)(sg + j - e.strip0) * kStripCols + lane;
                if (lane < 16 && col < e.N) {
                    const int* pj = part + j * kW * 16 + lane;
                    int v = pj[0];
#pragma unroll
                    for (int w = 1; w < kW; ++w) v += pj[16 * w];
                    emit(e, col, v, act * e.w_scale);
                }
            };
            const long long b = e0.strip0 + (long long)e0.n_strips;
            for (int j = wave; j < ns; j += kW) {
                if (sg + j < b)
                    emit_strip(e0, j);
                else
                    emit_strip(e1, j);
            }
        } else {
            for (int j = wave; j < ns; j += kW) {
                const int col = (sa + j) * kStripCols + lane;
                if (lane < 16 && col < d.N) {
                    const int* pj = part + j * kW * 16 + lane;
                    int v = pj[0];
#pragma unroll
                    for (int w = 1; w < kW; ++w) v += pj[16 * w];
                    emit(d, col, v, s);
                }
            }
        }
        sg = seg_end;
        ++di;
    }
}

}  // namespace

int gemv_max_wg_per_cu(int lds_bytes, int vec_kind) {
    int n = 0;
    hipError_t e;
    switch (vec_kind) {
    case TER_HIP_X_I8:
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_t16_kernel<true, TER_HIP_X_I8>, kGemvThreads,
                                                         lds_bytes);
        break;
    case TER_HIP_X_F32:
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_t16_kernel<true, TER_HIP_X_F32>, kGemvThreads,
                                                         lds_bytes);
        break;
    default:  // the general kernel needs the most registers of all
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_t16_kernel<true, -1>, kGemvThreads, lds_bytes);
    }
    return e == hipSuccess ? n : 0;
}

hipError_t launch_gemv(const GemvDesc& single, const GemvDesc* list_dev, const int32_t* first_dev,
                       const long long* ranges_dev, long long total_tiles, int n_wg, int lds_bytes, int vec_kind,
                       hipStream_t st) {
    const dim3 grid(n_wg), block(kGemvThreads);
    if (!list_dev) {
        hipLaunchKernelGGL((gemv_t16_kernel<false, -1>), grid, block, lds_bytes, st, single, list_dev, first_dev,
                           ranges_dev, total_tiles, n_wg);
        return hipGetLastError();
    }
    switch (vec_kind) {
    case TER_HIP_X_I8:
        hipLaunchKernelGGL((gemv_t16_kernel<true, TER_HIP_X_I8>), grid, block, lds_bytes, st, single, list_dev,
                           first_dev, ranges_dev, total_tiles, n_wg);
        break;
    case TER_HIP_X_F32:
        hipLaunchKernelGGL((gemv_t16_kernel<true, TER_HIP_X_F32>), grid, block, lds_bytes, st, single, list_dev,
                           first_dev, ranges_dev, total_tiles, n_wg);
        break;
    case TER_HIP_X_F32_RMS:
        hipLaunchKernelGGL((gemv_t16_kernel<true, TER_HIP_X_F32_RMS>), grid, block, lds_bytes, st, single,
                           list_dev, first_dev, ranges_dev, total_tiles, n_wg);
        break;
    case TER_HIP_X_F16_RMS:
        hipLaunchKernelGGL((gemv_t16_kernel<true, TER_HIP_X_F16_RMS>), grid, block, lds_bytes, st, single,
                           list_dev, first_dev, ranges_dev, total_tiles, n_wg);
        break;
    case TER_HIP_X_RELU2_RMS:
        hipLaunchKernelGGL((gemv_t16_kernel<true, TER_HIP_X_RELU2_RMS>), grid, block, lds_bytes, st, single,
                           list_dev, first_dev, ranges_dev, total_tiles, n_wg);
        break;
    default:
        hipLaunchKernelGGL((gemv_t16_kernel<true, -1>), grid, block, lds_bytes, st, single, list_dev, first_dev,
                           ranges_dev, total_tiles, n_wg);
    }
    return hipGetLastError();
}

hipError_t launch_gemv_strips(const GemvDesc* list_dev, const GemvDesc* wg_desc_dev, long long total_strips, int n_wg,
                              int lds_bytes, int part_off, int vec_kind, bool strided, const GemvDesc* shared,
                              hipStream_t st) {
    const dim3 grid(n_wg), block(kGemvThreads);
    if (strided && shared) {
        switch (vec_kind) {
        case TER_HIP_X_F32_RMS:
            hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_F32_RMS, true, kGemvWaves, true>), grid, block,
                               lds_bytes, st, *shared, list_dev, wg_desc_dev, total_strips, n_wg, part_off);
            return hipGetLastError();
        case TER_HIP_X_F16_RMS:
            hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_F16_RMS, true, kGemvWaves, true>), grid, block,
                               lds_bytes, st, *shared, list_dev, wg_desc_dev, total_strips, n_wg, part_off);
            return hipGetLastError();
        case TER_HIP_X_RELU2_RMS:
            hipLaunchKernelGGL(
                (gemv_strip_kernel<true, TER_HIP_X_RELU2_RMS, true, strided_waves<TER_HIP_X_RELU2_RMS>(), true>),
                grid, dim3(64 * strided_waves<TER_HIP_X_RELU2_RMS>()), lds_bytes, st, *shared, list_dev, wg_desc_dev,
                total_strips, n_wg, part_off);
            return hipGetLastError();
        case TER_HIP_X_F16:
            hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_F16, true, strided_waves<TER_HIP_X_F16>(), true>),
                               grid, dim3(64 * strided_waves<TER_HIP_X_F16>()), lds_bytes, st, *shared, list_dev,
                               wg_desc_dev, total_strips, n_wg, part_off);
            return hipGetLastError();
        case TER_HIP_X_SILU_MUL:
            hipLaunchKernelGGL(
                (gemv_strip_kernel<true, TER_HIP_X_SILU_MUL, true, strided_waves<TER_HIP_X_SILU_MUL>(), true>),
                grid, dim3(64 * strided_waves<TER_HIP_X_SILU_MUL>()), lds_bytes, st, *shared, list_dev, wg_desc_dev,
                total_strips, n_wg, part_off);
            return hipGetLastError();
        case TER_HIP_X_SMUL:
            hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_SMUL, true, strided_waves<TER_HIP_X_SMUL>(), true>),
                               grid, dim3(64 * strided_waves<TER_HIP_X_SMUL>()), lds_bytes, st, *shared, list_dev,
                               wg_desc_dev, total_strips, n_wg, part_off);
            return hipGetLastError();
        default:
            return hipErrorInvalidValue;
        }
    }
    if (strided) {
        const GemvDesc sh{};
        switch (vec_kind) {
        case TER_HIP_X_F32_RMS:
            hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_F32_RMS, true>), grid, block, lds_bytes, st,
                               sh, list_dev, wg_desc_dev, total_strips, n_wg, part_off);
            return hipGetLastError();
        case TER_HIP_X_F16_RMS:
            hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_F16_RMS, true>), grid, block, lds_bytes, st,
                               sh, list_dev, wg_desc_dev, total_strips, n_wg, part_off);
            return hipGetLastError();
        case TER_HIP_X_RELU2_RMS:
            hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_RELU2_RMS, true, strided_waves<TER_HIP_X_RELU2_RMS>()>),
                               grid, dim3(64 * strided_waves<TER_HIP_X_RELU2_RMS>()), lds_bytes, st, sh,
                               list_dev, wg_desc_dev, total_strips, n_wg, part_off);
            return hipGetLastError();
        case TER_HIP_X_F16:
            hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_F16, true, strided_waves<TER_HIP_X_F16>()>),
                               grid, dim3(64 * strided_waves<TER_HIP_X_F16>()), lds_bytes, st, sh,
                               list_dev, wg_desc_dev, total_strips, n_wg, part_off);
            return hipGetLastError();
        case TER_HIP_X_SILU_MUL:
            hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_SILU_MUL, true, strided_waves<TER_HIP_X_SILU_MUL>()>),
                               grid, dim3(64 * strided_waves<TER_HIP_X_SILU_MUL>()), lds_bytes, st, sh,
                               list_dev, wg_desc_dev, total_strips, n_wg, part_off);
            return hipGetLastError();
        case TER_HIP_X_SMUL:
            hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_SMUL, true, strided_waves<TER_HIP_X_SMUL>()>),
                               grid, dim3(64 * strided_waves<TER_HIP_X_SMUL>()), lds_bytes, st, sh,
                               list_dev, wg_desc_dev, total_strips, n_wg, part_off);
            return hipGetLastError();
        default:
            return hipErrorInvalidValue;
        }
    }
    switch (vec_kind) {
    case TER_HIP_X_I8:
        hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_I8>), grid, block, lds_bytes, st, GemvDesc{},
                           list_dev, wg_desc_dev, total_strips, n_wg, part_off);
        break;
    case TER_HIP_X_F32:
        hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_F32>), grid, block, lds_bytes, st, GemvDesc{},
                           list_dev, wg_desc_dev, total_strips, n_wg, part_off);
        break;
    case TER_HIP_X_F32_RMS:
        hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_F32_RMS>), grid, block, lds_bytes, st, GemvDesc{},
                           list_dev, wg_desc_dev, total_strips, n_wg, part_off);
        break;
    case TER_HIP_X_F16_RMS:
        hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_F16_RMS>), grid, block, lds_bytes, st, GemvDesc{},
                           list_dev, wg_desc_dev, total_strips, n_wg, part_off);
        break;
    case TER_HIP_X_RELU2_RMS:
        hipLaunchKernelGGL((gemv_strip_kernel<true, TER_HIP_X_RELU2_RMS>), grid, block, lds_bytes, st, GemvDesc{},
                           list_dev, wg_desc_dev, total_strips, n_wg, part_off);
        break;
    default:
        hipLaunchKernelGGL((gemv_strip_kernel<true, -1>), grid, block, lds_bytes, st, GemvDesc{},
                           list_dev, wg_desc_dev, total_strips, n_wg, part_off);
    }
    return hipGetLastError();
}

int gemv_strided_waves(int vec_kind) {
    switch (vec_kind) {
    case TER_HIP_X_RELU2_RMS: return strided_waves<TER_HIP_X_RELU2_RMS>();
    case TER_HIP_X_SILU_MUL: return strided_waves<TER_HIP_X_SILU_MUL>();
    case TER_HIP_X_SMUL: return strided_waves<TER_HIP_X_SMUL>();
    case TER_HIP_X_F16: return strided_waves<TER_HIP_X_F16>();
    default: return kGemvWaves;
    }
}

bool gemv_strided_ok(int vec_kind, int32_t K, bool stage32) {
    const int ku = units_of(K);
    switch (vec_kind) {
    case TER_HIP_X_F32_RMS: return stage32 && ku <= max_strided_ku<TER_HIP_X_F32_RMS>();
    case TER_HIP_X_F16_RMS: return stage32 && ku <= max_strided_ku<TER_HIP_X_F16_RMS>();
    case TER_HIP_X_RELU2_RMS: return stage32 && ku <= max_strided_ku<TER_HIP_X_RELU2_RMS>();
    case TER_HIP_X_F16: return stage32 && ku <= max_strided_ku<TER_HIP_X_F16>();
    case TER_HIP_X_SILU_MUL: return stage32 && ku <= max_strided_ku<TER_HIP_X_SILU_MUL>();
    case TER_HIP_X_SMUL: return stage32 && ku <= max_strided_ku<TER_HIP_X_SMUL>();
    default: return false;
    }
}

hipError_t launch_gemv_strips_single(const GemvDesc& d, long long total_strips, int n_wg, int lds_bytes, int part_off,
                                     hipStream_t st) {
    hipLaunchKernelGGL((gemv_strip_kernel<false, -1>), dim3(n_wg), dim3(kGemvThreads), lds_bytes, st, d, nullptr,
                       nullptr, total_strips, n_wg, part_off);
    return hipGetLastError();
}

}  // namespace terhip
