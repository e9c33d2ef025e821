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
#include <type_traits>

#include "common.h"

namespace terhip {
namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kLmWaves = 4;
constexpr int kLmThreads = kLmWaves * 64;
constexpr unsigned kOob = 0x80000000u;  // voffset past any resource: the load returns 0

struct LmArgs {
    const float* hidden;        // fp32 [H] residual stream (RMSNorm prologue) or null
    const uint16_t* hidden16;   // fp16 [H] residual stream (the Llama forward's; RMSNorm prologue) or null
    const uint16_t* gamma;      // fp16 [H] RMSNorm weights (with hidden)
    const uint16_t* x16;        // fp16 [H] normalized input (without hidden)
    const uint16_t* emb;        // fp16 [V][H]
    uint16_t* x_out;            // fp16 [H] copy of the normalized input or null
    uint16_t* logits;           // fp16 [V] or null
    int32_t* token_out;         // argmax index or null
    int32_t* pos_advance;       // position incremented after the token is written, or null
    unsigned long long* state;  // argmax state, zero at rest (kArgGroups + 1 pairs)
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

// Argmax state: kArgGroups groups of (key, count) words, 128 bytes apart,
// then the top (key, count); all zero at rest.
constexpr int kArgGroups = 128;
constexpr int kArgStride = 16;  // words (128 bytes) between groups
static_assert((kArgGroups + 1) * kArgStride * 8 == TER_HIP_ARGMAX_STATE_BYTES, "argmax state size");

__device__ __forceinline__ unsigned long long amax(unsigned long long* p, unsigned long long v) {
    return __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long aadd(unsigned long long* p, unsigned long long v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Fold key m into the (key, count) pair at p; true for the arrival that
// makes the count n, which also takes the pair's maximum into *best and
// clears the pair.  The max is performed (its old value returned) before
// the arrival is counted, so the arrival that counts last sees every max:
// read-modify-write atomics on one address are performed at one point, in
// order.  No fence: a device-scope fence writes back and invalidates the
// XCD's L2, which costs more than the whole argmax when every workgroup
// does it.
__device__ __forceinline__ bool arrive(unsigned long long* p, unsigned long long m, unsigned long long n,
                                       unsigned long long* best) {
    const unsigned long long old = amax(p, m);
    asm volatile("" ::"v"((unsigned)old) : "memory");
    if (aadd(p + 1, 1ull) != n - 1) return false;
    *best = __hip_atomic_exchange(p, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p + 1, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// Workgroup maximum of the per-lane keys, then two levels of atomics (a
// group of workgroups, then the groups) so that no address takes more than
// about n_wg / kArgGroups arrivals; the last arrival writes the index.
// Every thread of the workgroup must call it.
__device__ void argmax_finish(unsigned long long key, unsigned long long* kred, unsigned long long* state,
                              int32_t* token_out, int chunk, int32_t* pos_advance) {
    key = wave_max64(key);
    if ((threadIdx.x & 63) == 0) kred[threadIdx.x >> 6] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long m = kred[0];
#pragma unroll
        for (int w = 1; w < kLmWaves; ++w) m = umax64(m, kred[w]);
        const unsigned n_wg = gridDim.x, g = blockIdx.x % kArgGroups;
        const unsigned groups = n_wg < (unsigned)kArgGroups ? n_wg : (unsigned)kArgGroups;
        const unsigned in_group = (n_wg - g + kArgGroups - 1) / kArgGroups;
        unsigned long long bg, best;
        if (arrive(state + kArgStride * g, m, in_group, &bg) &&
            arrive(state + kArgStride * kArgGroups, bg, groups, &best)) {
            *gptr(token_out) = argmax_index(best, chunk);
            if (pos_advance) *gptr(pos_advance) += 1;  // inc_pos_k: the step's last use of the position is done
        }
    }
}

// Stage the normalized input in LDS as fp16 pairs xs[0 .. npad), zero past
// H/2 (H even).  With hidden: rmsnorm_f32_in_k's steps (256 strided partial
// sums of squares with fused multiply-adds, the reference tree,
// rms_inv = 1 / sqrt(ss / H + eps) correctly rounded,
// y = half((x * rms_inv) * gamma)).  With hidden16 the same steps on the
// fp16 values, widened exactly (rmsnorm_k, cuda/ter_cuda_forward_packed.cu:27-37).
// Workgroup 0 writes the optional copy.
__device__ void stage_x_pairs(const LmArgs& a, uint32_t* xs, int npad, float* red) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    const int n2 = a.H >> 1;
    const bool owner = blockIdx.x == 0 && a.x_out != nullptr;
    if (a.hidden16) {
        const TER_GLOBAL uint16_t* h = gptr(a.hidden16);
        float part = 0.f;
        for (int i = tid; i < a.H; i += kLmThreads) {
            const float v = half_bits_to_float(h[i]);
            part = __builtin_fmaf(v, v, part);
        }
        const float rms_inv = 1.0f / __builtin_sqrtf(tree_sum256(part, red) / (float)a.H + a.eps);
        for (int i = tid; i < npad; i += kLmThreads) {
            uint32_t w = 0;
            if (i < n2) {
                const uint32_t hw = gptr(reinterpret_cast<const uint32_t*>(a.hidden16))[i];
                const uint32_t gw = gptr(reinterpret_cast<const uint32_t*>(a.gamma))[i];
                const uint16_t y0 = float_to_half_bits((half_bits_to_float((uint16_t)(hw & 0xFFFFu)) * rms_inv) *
                                                       half_bits_to_float((uint16_t)(gw & 0xFFFFu)));
                const uint16_t y1 = float_to_half_bits((half_bits_to_float((uint16_t)(hw >> 16)) * rms_inv) *
                                                       half_bits_to_float((uint16_t)(gw >> 16)));
                w = (uint32_t)y0 | ((uint32_t)y1 << 16);
                if (owner) gptr(reinterpret_cast<uint32_t*>(a.x_out))[i] = w;
            }
            xs[i] = w;
        }
    } else if (a.hidden) {
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

// Fast path (H a multiple of 8, H/2 <= 32 * 8 * NB pairs).  A wave runs
// 8 vocabulary rows at once ("octet"): lane 8s + q serves row s of the octet
// and the reference's virtual lanes 4q .. 4q+3, whose pairs 4q+i + 32j are
// the 16 contiguous bytes 128j + 16q of the row.  So every load is a 16-byte
// buffer_load_dwordx4 covering, per instruction, 128 contiguous bytes of
// each of 8 adjacent rows, and each of the lane's 4 accumulators runs the
// reference's sequential chain over j.  The butterfly's steps o = 16, 8, 4
// pair lanes q ^ 4, q ^ 2, q ^ 1; o = 2, 1 pair accumulators i ^ 2, i ^ 1.
// Per fp16 pair: p1 = x_hi * e_hi (exact), t = x_lo * e_lo + p1 rounded
// once (exact products, so t equals the reference's rounding of the pair
// sum), acc += t.  Batches of 8 groups (8 loads of 16 bytes per lane) are
// double-buffered across the wave's whole sequence of octets.
constexpr int kGroupsPerBatch = 8;

// f(integral_constant<int, 0>) .. f(integral_constant<int, N - 1>), unrolled.
template <int N, int I = 0, class F>
__device__ __forceinline__ void unroll_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        unroll_for<N, I + 1>(f);
    }
}

// Batch jb (groups 8 jb .. 8 jb + 7) of octet `oct` of the wave's rows.
// Rows past the wave's range fall outside the buffer resource (the hardware
// range check returns zeros, and no memory is read); pairs past H/2 in a
// partial last group get an out-of-range offset.  Every lane issues every
// load and there is no branch, so the loads stay counted in order.
template <int JB, bool FULL>
__device__ __forceinline__ void load_batch16(u32x4 (&w)[kGroupsPerBatch], __amdgpu_buffer_rsrc_t rs, int oct, int rowb,
                                             int slot, int q, int n2) {
    const unsigned base = (unsigned)((8 * oct + slot) * rowb + 16 * q);
    const int lim = n2 - 4 * q;  // pairs of this lane's column that exist
#pragma unroll
    for (int g = 0; g < kGroupsPerBatch; ++g) {
        constexpr int j0 = JB * kGroupsPerBatch;
        const unsigned pen = FULL || 32 * (j0 + g) < lim ? 0u : kOob;
        w[g] = __builtin_amdgcn_raw_buffer_load_b128(rs, base + pen + 128u * (j0 + g), 0, 2 /* nt */);
    }
}

__device__ __forceinline__ float pair_term(unsigned x, unsigned e) {
    const float p1 = __builtin_fmaf((float)__builtin_bit_cast(_Float16, (uint16_t)(x >> 16)),
                                    (float)__builtin_bit_cast(_Float16, (uint16_t)(e >> 16)), 0.0f);
    return __builtin_fmaf((float)__builtin_bit_cast(_Float16, (uint16_t)(x & 0xFFFFu)),
                          (float)__builtin_bit_cast(_Float16, (uint16_t)(e & 0xFFFFu)), p1);
}

// FULL: H/2 == 256 NB, every group of every row exists (no masking).
template <int NB, bool FULL>
__global__ __launch_bounds__(kLmThreads) void lm_head_kernel(LmArgs a, int stage_rows) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) unsigned char lds_raw[];
    constexpr int NJ = NB * kGroupsPerBatch;
    uint32_t* xs = reinterpret_cast<uint32_t*>(lds_raw);
    float* red = reinterpret_cast<float*>(lds_raw + NJ * 32 * 4);
    unsigned long long* kred = reinterpret_cast<unsigned long long*>(red + kLmThreads);
    uint16_t* lg_stage = reinterpret_cast<uint16_t*>(kred + kLmWaves);
    const int tid = threadIdx.x;
    // wave-uniform in an SGPR, so the buffer resource built from it is too
    // (a resource in VGPRs turns every load into a readfirstlane loop)
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int slot = lane >> 3, q = lane & 7;
    const int n2 = a.H >> 1;
    const int rowb = a.H * 2;
    const long long O = ((long long)a.V + 7) / 8;
    const long long W = (long long)gridDim.x * kLmWaves;
    const long long gw = (long long)blockIdx.x * kLmWaves + wave;
    const long long o0 = O * gw / W, o1 = O * (gw + 1) / W;
    const int n_oct = (int)(o1 - o0);
    const long long r0 = 8 * o0;
    const long long r1 = 8 * o1 < (long long)a.V ? 8 * o1 : (long long)a.V;
    const int nrows = (int)(r1 - r0);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.emb + r0 * a.H), 0, nrows * rowb, 0x00020000);
    // logits of this wave's rows are staged in LDS and written at the end
    // (stores between the loads would make every wait drain the loads)
    const bool staged = a.logits && stage_rows > 0;
    uint16_t* my_stage = lg_stage + wave * stage_rows;

    u32x4 wa[kGroupsPerBatch], wb[kGroupsPerBatch];
    load_batch16<0, FULL>(wa, rs, 0, rowb, slot, q, n2);  // in flight during staging
    stage_x_pairs(a, xs, NJ * 32, red);

    const int chunk = argmax_chunk(a.V);
    unsigned long long best = 0ull;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    // Groups of batch JB of octet `oct` (w holds them), then for the last
    // batch the butterfly and the row's outputs.
    auto compute = [&](const u32x4 (&w)[kGroupsPerBatch], int oct, auto jb_tag) {
        constexpr int JB = decltype(jb_tag)::value;
        if constexpr (JB == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = 0.f;
        }
#pragma unroll
        for (int g = 0; g < kGroupsPerBatch; ++g) {
            const int j = JB * kGroupsPerBatch + g;
            const u32x4 x = *reinterpret_cast<const u32x4*>(xs + 32 * j + 4 * q);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = acc[i] + pair_term(x[i], w[g][i]);
        }
        if constexpr (JB == NB - 1) {
            float r[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) r[i] = acc[i];
#pragma unroll
            for (int m = 4; m >= 1; m >>= 1)
#pragma unroll
                for (int i = 0; i < 4; ++i) r[i] = r[i] + __shfl_xor(r[i], m);
            const float tot = (r[0] + r[2]) + (r[1] + r[3]);
            const int row = 8 * oct + slot;
            if (q == 0 && row < nrows) {
                const uint16_t h = float_to_half_bits(tot);
                if (a.token_out) best = umax64(best, argmax_key(h, (int)(r0 + row), chunk));
                if (staged) my_stage[row] = h;
                else if (a.logits) gptr(a.logits)[r0 + row] = h;
            }
        }
    };
    // Static two-buffer schedule over a block of OPS octets (OPS * NB batches,
    // an even count): batch t computes from buffer t & 1 while batch t + 1
    // (possibly the next block's first) loads into the other.  Loads past the
    // wave's octets read nothing (out of range); their computes are skipped.
    constexpr int OPS = NB % 2 ? 2 : 1;
    for (int o = 0; o < n_oct; o += OPS) {
        unroll_for<OPS * NB>([&](auto t_tag) {
            constexpr int t = decltype(t_tag)::value;
            constexpr int tn = t + 1;
            const int on = o + tn / NB;
            if constexpr (t % 2 == 0) {
                load_batch16<tn % NB, FULL>(wb, rs, on, rowb, slot, q, n2);
                if (o + t / NB < n_oct) compute(wa, o + t / NB, std::integral_constant<int, t % NB>{});
            } else {
                load_batch16<tn % NB, FULL>(wa, rs, on, rowb, slot, q, n2);
                if (o + t / NB < n_oct) compute(wb, o + t / NB, std::integral_constant<int, t % NB>{});
            }
        });
    }
    if (staged) {
        // LDS operations of one wave complete in order: the staged values are visible to its other lanes
        asm volatile("" ::: "memory");
        for (int i = lane; i < nrows; i += 64) gptr(a.logits)[r0 + i] = my_stage[i];
    }
    if (a.token_out) argmax_finish(best, kred, a.state, a.token_out, chunk, a.pos_advance);
}

// Any H off the fast path (not a multiple of 8, or above 4096): the reference's
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
    if (a.token_out) argmax_finish(best, kred, a.state, a.token_out, chunk, a.pos_advance);
}

// argmax of fp16 logits [N] (argmax_local_k + argmax_final_k semantics).
// kVec (logits 16-byte aligned): each thread reads 8 consecutive logits with
// one 16-byte load per round, so a launch sized at one round waits for one
// load; the one group that ends past n reads its logits one by one (no load
// straddles the end).  Otherwise one logit per thread and round.  The
// maximum key does not depend on who compares what, so both forms give the
// same index.
template <bool kVec>
__global__ __launch_bounds__(kLmThreads) void argmax_kernel(const uint16_t* __restrict__ logits, int n,
                                                            int32_t* token_out, unsigned long long* state,
                                                            int32_t* pos_advance) {
    __shared__ unsigned long long kred[kLmWaves];
    const int chunk = argmax_chunk(n);
    unsigned long long best = 0ull;
    if constexpr (kVec) {
        for (long long b = ((long long)blockIdx.x * kLmThreads + threadIdx.x) * 8; b < n;
             b += (long long)gridDim.x * kLmThreads * 8) {
            if (b + 8 <= n) {
                const u32x4 v = *reinterpret_cast<const TER_GLOBAL u32x4*>(gptr(logits) + b);
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    best = umax64(best, argmax_key((uint16_t)(v[e >> 1] >> (16 * (e & 1))), (int)b + e, chunk));
            } else {
                for (int i = (int)b; i < n; ++i) best = umax64(best, argmax_key(gptr(logits)[i], i, chunk));
            }
        }
    } else {
        for (long long i = (long long)blockIdx.x * kLmThreads + threadIdx.x; i < n;
             i += (long long)gridDim.x * kLmThreads)
            best = umax64(best, argmax_key(gptr(logits)[i], (int)i, chunk));
    }
    argmax_finish(best, kred, state, token_out, chunk, pos_advance);
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// The token through the scalar cache (invalidated at every launch; nothing
// in the launch writes it): one scalar load, not a vector load per thread.
__device__ __forceinline__ int token_of(const int32_t* token) {
    return *(const __attribute__((address_space(4))) int32_t*)(size_t)token;
}

// token_embed_lookup_k: hidden[i] = float(token_embd[token][i]) (exact
// widening); a token outside [0, V) writes nothing.  Thread j copies
// elements 8 j .. 8 j + 7 (one 16-byte load when H is a multiple of 8 and
// the table and the output are 16-byte aligned, else one by one).
__global__ void embed_kernel(const uint16_t* __restrict__ emb, int V, int H, const int32_t* __restrict__ token,
                             float* __restrict__ hidden) {
    const int i0 = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
    const int t = token_of(token);
    if (i0 >= H || t < 0 || t >= V) return;
    const uint16_t* row = emb + (long long)t * H;
    if (i0 + 8 <= H && (H & 7) == 0 && ((reinterpret_cast<uintptr_t>(emb) | reinterpret_cast<uintptr_t>(hidden)) & 15) == 0) {
        const u32x4 v = *reinterpret_cast<const TER_GLOBAL u32x4*>(gptr(row) + i0);
        f32x4_t lo, hi;
        for (int e = 0; e < 4; ++e) {
            lo[e] = half_bits_to_float((uint16_t)(v[e >> 1] >> (16 * (e & 1))));
            hi[e] = half_bits_to_float((uint16_t)(v[2 + (e >> 1)] >> (16 * (e & 1))));
        }
        *reinterpret_cast<TER_GLOBAL f32x4_t*>(gptr(hidden) + i0) = lo;
        *reinterpret_cast<TER_GLOBAL f32x4_t*>(gptr(hidden) + i0 + 4) = hi;
    } else {
        for (int i = i0; i < H && i < i0 + 8; ++i) gptr(hidden)[i] = half_bits_to_float(gptr(row)[i]);
    }
}

// token_embed_lookup_k (cuda/ter_cuda_forward_packed.cu:99-106): the token's
// fp16 row into the fp16 hidden stream (a token outside [0, V) writes
// nothing); 8 elements per thread as above.
__global__ void embed16_kernel(const uint16_t* __restrict__ emb, int V, int H, const int32_t* __restrict__ token,
                               uint16_t* __restrict__ hidden16) {
    const int i0 = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
    const int t = token_of(token);
    if (i0 >= H || t < 0 || t >= V) return;
    const uint16_t* row = emb + (long long)t * H;
    if (i0 + 8 <= H && (H & 7) == 0 &&
        ((reinterpret_cast<uintptr_t>(emb) | reinterpret_cast<uintptr_t>(hidden16)) & 15) == 0) {
        *reinterpret_cast<TER_GLOBAL u32x4*>(gptr(hidden16) + i0) =
            *reinterpret_cast<const TER_GLOBAL u32x4*>(gptr(row) + i0);
    } else {
        for (int i = i0; i < H && i < i0 + 8; ++i) gptr(hidden16)[i] = gptr(row)[i];
    }
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

int lm_head_fast_nb(int H) {
    if (H % 8) return 0;
    const int nb = (H / 2 + 32 * kGroupsPerBatch - 1) / (32 * kGroupsPerBatch);
    return nb <= 8 ? nb : 0;
}

int lm_head_stage_rows(int H, int V, int n_wg) {
    if (!lm_head_fast_nb(H)) return 0;
    const long long O = ((long long)V + 7) / 8, W = (long long)n_wg * kLmWaves;
    const long long rows = 8 * ((O + W - 1) / W);
    return rows <= 2048 ? (int)rows : 0;  // at most 16 KiB of LDS for the staged logits
}

int lm_head_lds_bytes(int H, int stage_rows) {
    const int nb = lm_head_fast_nb(H);
    const int npad = nb ? nb * kGroupsPerBatch * 32 : (H + 1) / 2;
    return npad * 4 + kLmThreads * 4 + kLmWaves * 8 + kLmWaves * stage_rows * 2;
}

namespace {

// The kernel for H: lm_head_kernel<NB, FULL> on the fast path, else the
// generic one (nullptr).
typedef void (*LmKernel)(LmArgs, int);

template <int NB>
LmKernel fast_kernel(bool full) {
    return full ? lm_head_kernel<NB, true> : lm_head_kernel<NB, false>;
}

LmKernel lm_kernel_of(int H) {
    const int nb = lm_head_fast_nb(H);
    const bool full = H / 2 == 32 * kGroupsPerBatch * nb;
    switch (nb) {
        case 1: return fast_kernel<1>(full);
        case 2: return fast_kernel<2>(full);
        case 3: return fast_kernel<3>(full);
        case 4: return fast_kernel<4>(full);
        case 5: return fast_kernel<5>(full);
        case 6: return fast_kernel<6>(full);
        case 7: return fast_kernel<7>(full);
        case 8: return fast_kernel<8>(full);
        default: return nullptr;
    }
}

}  // namespace

int lm_head_max_wg_per_cu(int H) {
    const int lds = lm_head_lds_bytes(H, 2048);
    const LmKernel k = lm_kernel_of(H);
    int n = 0;
    const hipError_t e =
        k ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, kLmThreads, lds)
          : hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, lm_head_generic_kernel, kLmThreads, lds);
    return e == hipSuccess ? n : 0;
}

hipError_t launch_lm_head(const float* hidden, const uint16_t* hidden16, const uint16_t* gamma, float eps,
                          const uint16_t* x16, const uint16_t* emb, int H, int V, uint16_t* x_out, uint16_t* logits,
                          int32_t* token_out, unsigned long long* state, int32_t* pos_advance, int n_wg,
                          hipStream_t st) {
    LmArgs a{};
    a.pos_advance = pos_advance;
    a.hidden = hidden;
    a.hidden16 = hidden16;
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
    const int srows = logits ? lm_head_stage_rows(H, V, n_wg) : 0;
    const int lds = lm_head_lds_bytes(H, srows);
    const LmKernel k = lm_kernel_of(H);
    if (k)
        hipLaunchKernelGGL(k, dim3(n_wg), dim3(kLmThreads), lds, st, a, srows);
    else
        hipLaunchKernelGGL(lm_head_generic_kernel, dim3(n_wg), dim3(kLmThreads), lds, st, a, (H + 1) / 2);
    return hipGetLastError();
}

hipError_t launch_argmax_f16(const uint16_t* logits, int n, int32_t* token_out, unsigned long long* state,
                             int32_t* pos_advance, int n_wg, hipStream_t st) {
    if ((reinterpret_cast<uintptr_t>(logits) & 15) == 0)
        hipLaunchKernelGGL(argmax_kernel<true>, dim3(n_wg), dim3(kLmThreads), 0, st, logits, n, token_out, state,
                           pos_advance);
    else
        hipLaunchKernelGGL(argmax_kernel<false>, dim3(n_wg), dim3(kLmThreads), 0, st, logits, n, token_out, state,
                           pos_advance);
    return hipGetLastError();
}

hipError_t launch_embed_f16(const uint16_t* emb, int V, int H, const int32_t* token, float* hidden, hipStream_t st) {
    hipLaunchKernelGGL(embed_kernel, dim3((H + 2047) / 2048), dim3(256), 0, st, emb, V, H, token, hidden);
    return hipGetLastError();
}

hipError_t launch_embed_h16(const uint16_t* emb, int V, int H, const int32_t* token, uint16_t* hidden16,
                            hipStream_t st) {
    hipLaunchKernelGGL(embed16_kernel, dim3((H + 2047) / 2048), dim3(256), 0, st, emb, V, H, token, hidden16);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_f16_rows(const float* x, const uint16_t* gamma, float eps, int M, int H, uint16_t* y,
                                   hipStream_t st) {
    hipLaunchKernelGGL(rmsnorm_f16_rows_kernel, dim3(M), dim3(256), 0, st, x, gamma, eps, H, y);
    return hipGetLastError();
}

}  // namespace terhip
