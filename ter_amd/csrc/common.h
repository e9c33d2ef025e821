// common.h -- shared definitions of the gfx950 packed-trit fabric.
//
// T16 tile layout (the HBM format every M=1 kernel streams):
//   A K x N ternary matrix is cut into column strips of 16 output columns and
//   units of 256 input rows.  Tile (strip s, unit u) is 1024 contiguous bytes
//   at offset (s * Ku + u) * 1024, Ku = ceil(K / 256); strips are stored one
//   after another, each strip's tiles in increasing u.
//   Inside a tile, lane L = 0..63 of a wave64 owns bytes [16L, 16L + 16):
//     row r = L / 16 -> output columns 16 s + 4 r + j   (j = 0..3, dword j)
//     q     = L % 16 -> input rows    k0 = 256 u + 16 q .. k0 + 15
//   Dword j holds 16 trits of column 16 s + 4 r + j: the trit of input row
//   k0 + 4 f + b sits in byte b (0..3), bits 2f..2f+1 (f = 0..3), encoded as
//   u = w + 1 in {0, 1, 2}.  Padding rows/columns hold u = 1 (w = 0).
//   With that order, (dword >> 2f) & 0x03030303 is an int8x4 of u for the
//   four consecutive rows k0 + 4f .. k0 + 4f + 3, which pair with the int8x4
//   activation dword X[k0 + 4f .. k0 + 4f + 3] in one v_dot4.
//   sum_k x_k w_kj = sum_k x_k u_kj - sum_k x_k, so the kernels subtract the
//   activation sum of each 256-row unit once per column strip.
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>
#include <stdint.h>

#include "ter_hip.h"

namespace terhip {

constexpr int kTileBytes = 1024;
constexpr int kStripCols = 16;
constexpr int kUnitK = 256;
constexpr int kWaves = 4;                 // waves per workgroup of the GEMM kernels
constexpr int kThreads = 64 * kWaves;
constexpr int kGemvWaves = 4;             // waves per workgroup of the GEMV kernel
constexpr int kGemvThreads = 64 * kGemvWaves;

__host__ __device__ inline int32_t units_of(int32_t K) { return (K + kUnitK - 1) / kUnitK; }
inline int32_t strips_of(int32_t N) { return (N + kStripCols - 1) / kStripCols; }
inline size_t tile_stream_bytes(int32_t K, int32_t N) {
    return (size_t)strips_of(N) * (size_t)units_of(K) * kTileBytes;
}
inline size_t fix_offset(int32_t K, int32_t N) { return tile_stream_bytes(K, N); }

// One GEMV of a work list, as the kernel reads it (device memory or kernarg).
struct alignas(16) GemvDesc {
    const uint8_t* w;            // T16 tile stream
    const void* x;               // int8 [K], fp32 [K] or fp16 [K] (x_kind; the gate for X_RELU2_RMS)
    const float* x_scale_dev;    // int8 input: device activation scale or null
    float* y;                    // fp32 [N] or null
    int32_t* acc;                // int32 [N] or null
    int8_t* xq_out;              // quantized input: int8 X copy or null
    float* xs_out;               // quantized input: activation scale copy or null
    const uint16_t* gamma;       // RMS kinds: fp16 RMSNorm weights [K]
    const uint16_t* up;          // X_RELU2_RMS: fp16 up projection [K]
    uint16_t* y16;               // fp16 [N] = half(y) or null
    float* resid;                // fp32 [N]: resid += float(half(y)), or null
    uint16_t* resid16;           // fp16 [N]: resid16 = half(float(resid16) + float(half(y))), or null
    float* silu;                 // fp32 [N]: silu(float(half(y))) (the X_SMUL kind's input), or null
    unsigned long long* fix;     // N fix-up slots, zero at rest
    long long tile0;             // first tile of this GEMV in the launch's stream
    long long strip0;            // first strip of this GEMV in the launch's strip stream (strip mode)
    int32_t stage32;             // RMS kinds: fp32 activations staged in LDS (else re-read for the sums)
    int32_t K, N, Ku, n_strips;
    float w_scale, x_scale;
    int32_t x_kind;
    float eps;                   // RMS kinds
    int32_t w_mag;               // trit magnitude m of a {-m, 0, +m} payload (1 for plain trits)
    int32_t self;                // index of this descriptor in its plan's list (strip-mode plans)
};

// One GEMM (M > 1) of a work list.  Its blocks (4 column strips x all K each)
// are numbered block0 .. block0 + n_blocks - 1 in the launch's block stream.
struct alignas(16) GemmDesc {
    const uint8_t* w;            // T16 tile stream
    const int8_t* x;             // int8 [M][ldx]
    const float* xs;             // per-row activation scales [M] (device)
    float* y;                    // fp32 [M][N] or null
    int32_t* acc;                // int32 [M][N] or null
    uint16_t* y16;               // fp16 [M][N] = half(y) or null
    float* resid;                // fp32 [M][N]: resid += float(half(y)), or null
    long long block0;            // first block (unit-major kernel)
    long long tile0;             // first tile in the launch's tile stream (streaming kernel)
    int32_t K, N, Ku, n_strips;
    int32_t M, ldx, n_blocks;
    float w_scale;
    int32_t w_mag;               // trit magnitude m of a {-m, 0, +m} payload (1 for plain trits)
};

// Host launchers (defined in the .hip files).  Work-list launches take the
// device descriptor table `list_dev` and `first_dev`, the index of each
// workgroup's first descriptor (range g starts at total * g / n_wg); single
// launches pass nullptr for both.
// Strip mode (small work lists): workgroups take whole column strips of the
// strip stream ([total_strips] over the list) and reduce the waves' partials
// in LDS at part_off; at most kStripModeMaxStrips strips per workgroup.
constexpr int kStripModeMaxStrips = 32;
// shared (strided lists only, else null): the activation every GEMV of the
// list reads and the base of their back-to-back tile streams (w, strip0 0,
// n_strips the list's), passed as the kernel argument so that the first
// loads need no descriptor.
hipError_t launch_gemv_strips(const GemvDesc* list_dev, const GemvDesc* wg_desc_dev, long long total_strips, int n_wg,
                              int lds_bytes, int part_off, int vec_kind, bool strided, const GemvDesc* shared,
                              hipStream_t st);
// Whether a strip-mode list of this activation kind and K runs the strided
// RMS prologue (gemv.hip: stage_x_strided).
bool gemv_strided_ok(int vec_kind, int32_t K, bool stage32);
// Waves per workgroup of that prologue's kernel (its strips' partial sums
// take [strip][waves][16] ints of LDS).
int gemv_strided_waves(int vec_kind);
// The same for one GEMV whose descriptor is a kernel argument (any activation kind).
hipError_t launch_gemv_strips_single(const GemvDesc& d, long long total_strips, int n_wg, int lds_bytes, int part_off,
                                     hipStream_t st);
// vec_kind: the activation kind of every GEMV of a work list that qualifies
// for the vector prologue (gemv_vec_kind), else -1.
// ranges_dev: [n_wg + 1] tile ranges of the workgroups of a work list (range
// g = [ranges[g], ranges[g + 1]), ends on strip edges where plan_ranges could
// put them there); single launches pass nullptr and cut total * g / n_wg,
// moved to the nearest strip edge under the same rule.
hipError_t launch_gemv(const GemvDesc& single, const GemvDesc* list_dev, const int32_t* first_dev,
                       const long long* ranges_dev, long long total_tiles, int n_wg, int lds_bytes, int vec_kind,
                       hipStream_t st);
// Single GEMV with int16 activations (gemv_x16.hip): whole strips per
// workgroup, at most kStripModeMaxStrips of them.
int gemv_x16_lds_bytes(int K, int strips_per_wg);
hipError_t launch_gemv_x16(const GemvDesc& d, int n_wg, int lds_bytes, hipStream_t st);
hipError_t launch_pack_v11(const uint8_t* v11, uint8_t* t16, int K, int N, hipStream_t st);
// The per-block branch of mm_row (blocked.hip): one thread per column.
hipError_t launch_mm_row_blocked(const uint8_t* w, int K, int N, int mag, const int16_t* x, const float* bsc,
                                 long long bs, float xs, float* out, hipStream_t st);
// Measurement kernels (probe.hip).
hipError_t launch_noop(hipStream_t st);
hipError_t launch_read_probe(const uint8_t* buf, long long tiles, int n_wg, unsigned* sink, hipStream_t st);
hipError_t launch_unpack_v11(const uint8_t* t16, uint8_t* v11, int K, int N, hipStream_t st);
hipError_t launch_pack_i2s(const uint8_t* raw, uint8_t* t16, int K, int N, hipStream_t st);
hipError_t launch_synth_v11(uint8_t* v11, int K, int N, uint64_t seed, uint32_t t0, uint32_t t1,
                            hipStream_t st);
hipError_t launch_synth_i8(int8_t* x, long long n, uint64_t seed, int lo, int hi, hipStream_t st);
hipError_t launch_quant_rows(const float* x, int M, int K, int8_t* q, float* s, hipStream_t st);
// One workgroup of 256 threads per row; kind is TER_HIP_X_F32_RMS,
// TER_HIP_X_F16_RMS or TER_HIP_X_RELU2_RMS (x = gate, up [M][K]).
hipError_t launch_rmsnorm_quant_rows(const void* x, const uint16_t* up, int kind, const uint16_t* gamma, float eps,
                                     int M, int K, int8_t* q, float* s, hipStream_t st);
// lm_head tail (lm_head.hip).  Fast path: H a multiple of 8 and at most
// 4096 (lm_head_fast_nb(H) > 0); any other H runs the generic kernel.  With
// `hidden` the launch normalizes it first (H even only); `state` (2 words,
// zero at rest) is needed when token_out is set.
int lm_head_fast_nb(int H);
int lm_head_max_wg_per_cu(int H);
// The RMSNorm prologue reads hidden (fp32) or hidden16 (fp16); with neither,
// x16 is the normalized input.
hipError_t launch_lm_head(const float* hidden, const uint16_t* hidden16, const uint16_t* gamma, float eps,
                          const uint16_t* x16, const uint16_t* emb, int H, int V, uint16_t* x_out, uint16_t* logits,
                          int32_t* token_out, unsigned long long* state, int32_t* pos_advance, int n_wg,
                          hipStream_t st);
hipError_t launch_embed_f16(const uint16_t* emb, int V, int H, const int32_t* token, float* hidden, hipStream_t st);
hipError_t launch_embed_h16(const uint16_t* emb, int V, int H, const int32_t* token, uint16_t* hidden16,
                            hipStream_t st);
hipError_t launch_argmax_f16(const uint16_t* logits, int n, int32_t* token_out, unsigned long long* state,
                             int32_t* pos_advance, int n_wg, hipStream_t st);
hipError_t launch_rmsnorm_f16_rows(const float* x, const uint16_t* gamma, float eps, int M, int H, uint16_t* y,
                                   hipStream_t st);
// Decode attention (attention.hip): head_dim 64 or 128, chunks of
// attn_chunk() positions, at most attn_max_chunks() chunks.
bool attn_supported_head_dim(int hd);
int attn_chunk();
int attn_max_chunks();
// Partial buffer [nh][n_chunks][attn_part_stride(hd)] floats; arrival
// counters [n_groups][attn_count_stride()] (zero at rest).
int attn_part_stride(int hd);
int attn_count_stride();
// Grid of the XCD-local launch, and whether blocks 0 .. n_blocks - 1 land on
// XCD b % 8 (probed with n_blocks ints of device scratch; false on any error).
int attn_local_blocks(int nh, int nkv, int smax);
int attn_head_groups(int nh, int nkv);  // workgroup head groups: query heads sharing a KV head, by kAttnWaves
bool attn_xcd_round_robin(int n_blocks, int* scratch, hipStream_t st);
hipError_t launch_attn_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* kc, uint16_t* vc,
                              const int32_t* pos, uint16_t* out, const float* rope, float* part, unsigned* count,
                              int nh, int nkv, int hd, int smax, bool neox, bool xcd_local, hipStream_t st);
// Positions outside [0, smax) write nothing (both kernels).
hipError_t launch_rope(uint16_t* v, int n_heads, int hd, const float* rope, const int32_t* pos, int smax, bool neox,
                       hipStream_t st);
// Rows per MFMA row block group: MB = 1, 2, 4, 8, 16 for M up to 16, 32, 64, 128, 256.
int gemm_mb_of(int M);
// vec: every x pointer 16-byte aligned and every ldx a multiple of 16.
hipError_t launch_gemm_list(const GemmDesc& single, const GemmDesc* list_dev, const int32_t* first_dev,
                            long long total_blocks, int n_wg, int mb, bool vec, hipStream_t st);
// Streaming GEMM for M <= 16 (whole X of a GEMM staged in LDS, whole strips
// per wave, no per-unit barrier).  Each GEMM segment lays out the launch's
// LDS for its own M and K: the X image, M rows of Ku * 16 chunks + one
// padding chunk each (16 bytes per chunk), at [0, gemm_stream_zero_off); a
// zero row of Ku * 256 bytes; 16 row sums; the waves' tile slots (each of the
// 4 waves turns its tiles into MFMA operand order through two 1 KiB slots);
// 16 row scales; then each wave's output buffer, as many whole strips as the
// rest of the launch's LDS holds (up to kGemmStreamOutMax): the int32 results
// of completed strips (M rows x 16 columns), written out between chunks of
// the wave's tiles, so that no store is issued among the weight loads.  A
// GEMM's X at K = 2560 leaves room for a whole run of strips (one write-out
// per run); the stores cost about 10 us at M = 8 on the BitNet sweep
// wherever they go, and 6 us more when split over five write-outs per run.
__host__ __device__ inline int gemm_stream_zero_off(int M, int K) { return M * (units_of(K) * (kUnitK / 16) + 1) * 16; }
constexpr int gemm_stream_slot_bytes() { return 4 * 2 * kTileBytes; }
__host__ __device__ inline int gemm_stream_out_off(int M, int K) {
    return gemm_stream_zero_off(M, K) + units_of(K) * kUnitK + 64 + gemm_stream_slot_bytes() + 64;
}
constexpr int kGemmStreamXMax = 64 * 1024;   // the X image (its staging registers hold 64 KiB)
constexpr int kGemmStreamLdsMax = 80 * 1024; // in all: two workgroups per CU
constexpr int kGemmStreamBatch = 6;          // tiles per batch (two batches per wave in flight)
constexpr int kGemmStreamOutMax = 32;        // strips per output buffer at most
// Strips of each wave's output buffer for a segment of this M and K in `lds` bytes.
__host__ __device__ inline int gemm_stream_out_strips(int M, int K, int lds) {
    const int left = lds - gemm_stream_out_off(M, K);
    const int s = left > 0 ? left / (4 * M * kStripCols * 4) : 0;
    return s < kGemmStreamOutMax ? s : kGemmStreamOutMax;
}
// A chunk is at least one double batch and completes at most
// floor(chunk / Ku) + 1 strips, so a buffer needs floor(2 batch / Ku) + 1.
__host__ __device__ inline int gemm_stream_out_need(int Ku) { return 2 * kGemmStreamBatch / Ku + 1; }
// The LDS a GEMM of this M and K would take (full buffers), capped.
inline int gemm_stream_lds_want(int M, int K) {
    const int w = gemm_stream_out_off(M, K) + 4 * kGemmStreamOutMax * M * kStripCols * 4;
    return w < kGemmStreamLdsMax ? w : kGemmStreamLdsMax;
}
// Whether a GEMM of this M and K streams in a launch of `lds` bytes.
inline bool gemm_stream_item_fits(int M, int K, int lds) {
    return M <= 16 && gemm_stream_zero_off(M, K) <= kGemmStreamXMax &&
           gemm_stream_out_strips(M, K, lds) >= gemm_stream_out_need(units_of(K));
}
// lds_bytes: the launch's LDS (the largest gemm_stream_lds_want of the list).
hipError_t launch_gemm_stream(const GemmDesc& single, const GemmDesc* list_dev, const int32_t* first_dev,
                              long long total_tiles, int n_wg, int lds_bytes, bool vec, hipStream_t st);
int gemm_stream_max_wg_per_cu(int lds_bytes);

// Resident GEMM workgroups per CU for row-block count mb (0 if the query fails).
int gemm_max_wg_per_cu(int mb);

// LDS-ring GEMM for M <= 128 (mb = 1, 2, 4, 8; gemm_lds.hip), used where the
// streaming kernel does not apply (M > 16, or M rows of X beyond its LDS).  Work is a
// list of blocks, each `gemm_lds_strips_per_block(mb)` strips of one GEMM;
// workgroup g (after the XCD remap) owns blocks [ranges[g], ranges[g+1]).
// Single launches pass null lists and split n_blocks of `single` evenly.
// Needs vec (16-byte aligned X rows).
struct GemmBlock {
    int32_t desc;    // index into the descriptor list
    int32_t strip0;  // first strip of the block
};
int gemm_lds_strips_per_block(int mb);  // 0: no LDS-ring configuration for mb
int gemm_lds_max_wg_per_cu(int mb);
hipError_t launch_gemm_lds(const GemmDesc& single, const GemmDesc* list_dev, const GemmBlock* blocks_dev,
                           const int32_t* ranges_dev, int n_blocks, int n_wg, int mb, hipStream_t st);
// Column strips per wave of the GEMM for row-block count mb (a block is
// kWaves * that many strips).
int gemm_strips_per_wave(int mb);

#if defined(__HIPCC__)
#define TER_GLOBAL __attribute__((address_space(1)))

// Generic -> global address space, so accesses compile to global_* / buffer
// instructions (flat ones also count against the LDS wait counter).
template <typename T>
__device__ __forceinline__ TER_GLOBAL T* gptr(T* p) {
    return (TER_GLOBAL T*)p;
}

__device__ inline float half_bits_to_float(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);  // exact widening
}

// binary32 -> binary16 in the default round-to-nearest-even mode (the
// reference's __float2half of its fp16 outputs); overflow gives inf.  The
// value is first pinned in a register as binary32: otherwise the compiler
// may fold the producing multiply / fma into the conversion
// (v_fma_mixlo_f16), rounding once to fp16 instead of to fp32 and then fp16.
__device__ inline uint16_t float_to_half_bits(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// The reference's accumulator as fp32: mm_row sums X * W in int64 over the
// payload {-m, 0, +m} and converts once (src/tx/forward.cpp:333-345), so
// float(acc) there is float(m * acc) here, rounded once from the exact int64
// product (acc is the trit accumulator, |acc| < 2^31).
__device__ __forceinline__ float acc_to_float(int val, int mag) {
    return mag == 1 ? (float)val : (float)((long long)val * (long long)mag);
}

// Output element o of a GEMV / GEMM (GemvDesc or GemmDesc): acc (the trit
// accumulator), y = float(m * acc) * s, y16 = half(y) (the reference's
// __float2half projection output), resid += float(half(y)) (BitNet's
// add_k_f32 residual step into its fp32 stream) and, for GEMVs, resid16 =
// half(float(resid16) + float(half(y))) (the Llama forward's add_k into its
// fp16 stream, cuda/ter_cuda_forward_packed.cu:115-118).
__device__ inline float silu_of(float g);

template <class D>
__device__ __forceinline__ void emit_out(const D& d, long long o, int val, float s) {
#pragma clang fp contract(off)
    if (d.acc) gptr(d.acc)[o] = val;
    const float y = acc_to_float(val, d.w_mag) * s;
    if (d.y) gptr(d.y)[o] = y;
    constexpr bool kR16 = std::is_same<D, GemvDesc>::value;  // the GEMV-only outputs
    bool half_out = d.y16 || d.resid;
    if constexpr (kR16) half_out = half_out || d.resid16 || d.silu;
    if (half_out) {
        const uint16_t h = float_to_half_bits(y);
        if (d.y16) gptr(d.y16)[o] = h;
        if (d.resid) gptr(d.resid)[o] = gptr(d.resid)[o] + half_bits_to_float(h);
        if constexpr (kR16) {
            if (d.resid16)
                gptr(d.resid16)[o] =
                    float_to_half_bits(half_bits_to_float(gptr(d.resid16)[o]) + half_bits_to_float(h));
            if (d.silu) gptr(d.silu)[o] = silu_of(half_bits_to_float(h));
        }
    }
}

// exp(x) of this build (the reference calls CUDA's expf): Cody-Waite
// reduction with a two-constant ln 2, degree-7 Taylor polynomial in Horner
// form, two-step scaling by 2^n.  Faithful (< 1 ulp from exp); the oracle's
// orc_expf runs the same operations, so both round identically.
__device__ inline float ter_pow2i(int e) { return __builtin_bit_cast(float, (unsigned)(e + 127) << 23); }

__device__ inline float ter_expf(float x) {
#pragma clang fp contract(off)
    if (x != x) return x;
    if (x > 88.72283935546875f) return __builtin_inff();
    if (x < -103.972084045410156f) return 0.0f;
    const float n = __builtin_rintf(x * 1.44269502162933349609375f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, x);
    r = __builtin_fmaf(-n, 1.42860676533018704e-06f, r);
    float p = 1.98412701e-04f;
    p = __builtin_fmaf(p, r, 1.38888892e-03f);
    p = __builtin_fmaf(p, r, 8.33333377e-03f);
    p = __builtin_fmaf(p, r, 4.16666679e-02f);
    p = __builtin_fmaf(p, r, 1.66666672e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int ni = (int)n;
    const int n1 = ni / 2, n2 = ni - n1;
    return (p * ter_pow2i(n1)) * ter_pow2i(n2);
}

// silu(gate) * up of silu_mul_quant_k (cuda/ter_cuda_forward_packed.cu:322-326):
// g / (1 + exp(-g)) with this build's exp, then the product, each rounded
// (the division correctly rounded, as nvcc's default division is).  silu_of
// is the first step alone (the gate GEMV's silu output; X_SMUL then forms
// the product), so both routes round identically.
__device__ inline float silu_of(float g) {
#pragma clang fp contract(off)
    return g / (1.0f + ter_expf(-g));
}

__device__ inline float silu_mul(float g, float u) {
#pragma clang fp contract(off)
    const float sg = silu_of(g);
    return sg * u;
}

// relu^2(gate) * up of relu2_mul_rmsnorm_quant_k
// (cuda/ter_cuda_forward_bitnet.cu:273-276): the square rounds first, then
// the product.
__device__ inline float relu2_mul(float g, float u) {
#pragma clang fp contract(off)
    const float r = g > 0.f ? g * g : 0.f;
    return r * u;
}

// Cross-row lane exchanges of gfx950 (no LDS round trip): the value of lane
// l ^ 32 (v_permlane32_swap) and of lane l ^ 16 (v_permlane16_swap).
__device__ __forceinline__ float lane_xor32(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor16(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __builtin_bit_cast(float, (threadIdx.x & 16) ? r[0] : r[1]);
}

template <int kCtrl>
__device__ __forceinline__ float dpp_move_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, true));
}

// The shuffle-down tree of a wave (for s = 32, 16, ..., 1: a[l] += a[l + s])
// as seen by lane 0, returned to every lane: the same two operands at each
// level for every lane that lane 0's sum depends on (lanes l < s), so the bits
// are those of the __shfl_down form.  Levels 32 and 16 use the permlane
// swaps, 8 .. 1 DPP row_shl inside the row.
__device__ __forceinline__ float tree_down64(float a) {
    a = a + lane_xor32(a);
    a = a + lane_xor16(a);
    a = a + dpp_move_f<0x108>(a);  // row_shl:8 (lane + 8)
    a = a + dpp_move_f<0x104>(a);  // row_shl:4
    a = a + dpp_move_f<0x102>(a);  // row_shl:2
    a = a + dpp_move_f<0x101>(a);  // row_shl:1
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 0));
}

// Sum of one value per thread of a 256-thread block, paired exactly as the
// reference's shared-memory tree (for s = 128, 64, ..., 1: partial[t] +=
// partial[t + s]): shared memory for the two cross-wave levels, lane shuffles
// within wave 0 below.  fp32 addition is commutative, so each level adds the
// same two operands and the result is bit-identical.  Every thread gets it.
__device__ inline float tree_sum256(float v, float* red) {
    const int t = threadIdx.x;
    red[t] = v;
    __syncthreads();
    if (t < 128) red[t] = red[t] + red[t + 128];
    __syncthreads();
    if (t < 64) {
        const float a = tree_down64(red[t] + red[t + 64]);
        if (t == 0) red[0] = a;
    }
    __syncthreads();
    const float r = red[0];
    __syncthreads();  // red may be reused
    return r;
}

// Sum of squares of v = relu2_mul(gate, up) over K elements in the order of
// a 1024-thread block (relu2_mul_rmsnorm_quant_k,
// cuda/ter_cuda_forward_bitnet.cu:270-284), computed by 256 threads: thread t
// keeps the strided partials of virtual threads t, t+256, t+512, t+768
// (fused multiply-adds), performs the tree's levels 512 and 256 itself, then
// tree_sum256 does 128 .. 1.
__device__ inline float relu2_sum_sq_1024(const uint16_t* gate, const uint16_t* up, int K, float* red) {
    const int t = threadIdx.x;
    float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
    for (int i = t; i < K; i += 1024) {
        float v = relu2_mul(half_bits_to_float(gptr(gate)[i]), half_bits_to_float(gptr(up)[i]));
        p0 = __builtin_fmaf(v, v, p0);
        if (i + 256 < K) {
            v = relu2_mul(half_bits_to_float(gptr(gate)[i + 256]), half_bits_to_float(gptr(up)[i + 256]));
            p1 = __builtin_fmaf(v, v, p1);
        }
        if (i + 512 < K) {
            v = relu2_mul(half_bits_to_float(gptr(gate)[i + 512]), half_bits_to_float(gptr(up)[i + 512]));
            p2 = __builtin_fmaf(v, v, p2);
        }
        if (i + 768 < K) {
            v = relu2_mul(half_bits_to_float(gptr(gate)[i + 768]), half_bits_to_float(gptr(up)[i + 768]));
            p3 = __builtin_fmaf(v, v, p3);
        }
    }
    p0 = p0 + p2;
    p1 = p1 + p3;
    return tree_sum256(p0 + p1, red);
}

#endif

// LDS bytes the GEMV kernel needs for a K: X (Ku*256 int8) + unit sums +
// reduction scratch (one float per thread, then one per wave).
__host__ __device__ inline int gemv_lds_bytes(int32_t K) {
    return units_of(K) * kUnitK + units_of(K) * 4 + (kGemvThreads + kGemvWaves) * 4;
}
// RMS activation kinds also stage the fp32 activations ([Ku*256] floats) at
// this 16-byte aligned offset.
__host__ __device__ inline int gemv_lds_xs32_offset(int32_t K) { return (gemv_lds_bytes(K) + 15) / 16 * 16; }
__host__ __device__ inline int gemv_lds_bytes_rms(int32_t K) {
    return gemv_lds_xs32_offset(K) + units_of(K) * kUnitK * 4;
}
// Workgroup ranges of the stream-K GEMV kernel end at strip edges where that
// moves them by at most a quarter of the mean range (2 Ku n_wg <= total):
// then the strips at a workgroup's range ends are not shared with another
// workgroup and need no global fix-up.  (Uneven ranges cost nothing here:
// the workgroups of a launch share the HBM stream, measured flat for ranges
// up to 3:1 apart.)  strip_edge_near: the strip edge nearest to local tile
// `local` of a GEMV (the upper edge is within the GEMV when local is).
// Both apply to launches whose waves stream at least kCombineMinTiles tiles
// each (combine_mode); for smaller pieces the workgroup barrier and the range
// imbalance cost more than the atomics, and each wave adds its partial strips
// to the global slots itself (decode-step lists: 34 tiles per workgroup,
// 7.55 against 8.17 us per launch).
constexpr long long kCombineMinTiles = 32;
__host__ __device__ inline bool combine_mode(long long total, int n_wg) {
    return total >= (long long)n_wg * kGemvWaves * kCombineMinTiles;
}
__host__ __device__ inline bool snap_ranges(int Ku, long long total, int n_wg) {
    return combine_mode(total, n_wg) && 2LL * Ku * n_wg <= total;
}
__host__ __device__ inline long long strip_edge_near(long long local, int Ku) {
    const long long lo = local - local % Ku;
    return local - lo <= Ku / 2 ? lo : lo + Ku;
}
// The stream-K kernel's slots, after the staging area, for the strips its
// waves share: per wave its first and last strip of a segment, each as a
// strip index, a unit count and the 16 column sums.
constexpr int kGemvSlotInts = 2 + kStripCols;
constexpr int kGemvSlotBytes = 2 * kGemvWaves * kGemvSlotInts * 4;
__host__ __device__ inline int gemv_lds_slots_offset(int32_t K, bool stage32) {
    return ((stage32 ? gemv_lds_bytes_rms(K) : gemv_lds_bytes(K)) + 15) / 16 * 16;
}
// Strip mode: the staging area, then (RMS kinds staging fp32) the fp16 gamma
// [Ku*256] and the partials of the strided prologue; the strips' partial
// sums follow.
__host__ __device__ inline int gemv_strip_red_offset(int32_t K) {
    return gemv_lds_slots_offset(K, true) + units_of(K) * kUnitK * 2;
}
constexpr int kStripRedBytes = (1024 + 16) * 4;  // the strided prologue's partials and wave maxima
__host__ __device__ inline int gemv_strip_part_off(int32_t K, bool stage32) {
    return stage32 ? gemv_strip_red_offset(K) + kStripRedBytes : gemv_lds_slots_offset(K, false);
}
// Then per wave the column sums of the first kGemvOutStrips strips completed
// within its piece (consecutive strips), written after its streaming loop so
// that no store is issued among the weight loads.
constexpr int kGemvOutStrips = 16;
constexpr int kGemvOutBytes = kGemvWaves * kGemvOutStrips * kStripCols * 4;
inline int gemv_t16_lds_bytes(int32_t K, bool stage32) {
    return gemv_lds_slots_offset(K, stage32) + kGemvSlotBytes + kGemvOutBytes;
}
// LDS of one workgroup on gfx950, and whether an RMS kind at this K stages
// its fp32 activations (the staging costs 4 bytes per element).
constexpr int kLdsMax = 160 * 1024;
inline bool gemv_stage32(int32_t K) { return gemv_t16_lds_bytes(K, true) <= kLdsMax; }

// Status helpers of the C-ABI (abi.hip): record the message returned by
// ter_hip_last_error() and return `code` (TER_HIP_ERR_HIP for hip_fail).
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char* what);

int device_cu_count(int device);
// Resident GEMV workgroups per CU at this LDS size (0 if the query fails).
int gemv_max_wg_per_cu(int lds_bytes, int vec_kind = -1);

}  // namespace terhip
