// attention.hip -- one decode step's attention for one layer on gfx950:
// RoPE of the new query and key, the KV-cache write of the new position, and
// attention over all cached positions, in one launch.
//
// Reference (cuda/ter_cuda_forward_bitnet.cu, BitNet; the Llama forward
// cuda/ter_cuda_forward_packed.cu has the same kernels with the NORM pairing):
//   rope_k       :185-200   NEOX pairs (k, k + hd/2) (NORM: (2k, 2k+1))
//   kv_copy_k    :204-214   K/V of the new position into [L][Smax][nkv*hd]
//   attention_k  :336-374   one block per head, whole sequence, one thread's softmax
//
// The reference kernel runs the softmax and every output element as single
// sequential chains over the sequence (2048 dependent steps at BitNet's
// C5 context).  Here the positions are split into chunks of 64:
//   - workgroup (head group, chunk): up to 4 query heads sharing one KV head
//     (GQA), 4 waves, wave i = query head i, lane = position in the chunk;
//   - scores exactly as the reference (fp32 dot over d in order, times
//     1/sqrt(hd)); chunk max m_c, e_s = exp(score - m_c), l_c the xor
//     butterfly over the wave, o_c[d] = sum over the chunk's positions in
//     order of e_s v_sd (fused multiply-adds);
//   - the last workgroup of a head group to finish combines the chunks in
//     order: w_c = exp(m_c - M), L = sum l_c w_c, O = sum o_c w_c, out = O/L
//     (while every position fits one chunk, that chunk's workgroup does it
//     at once, with no partials published or counted).
// The K and V rows of the chunk are staged in LDS with coalesced 16-byte
// loads issued before anything else; the new position's key and value come
// from the projection outputs (RoPE applied here), not from the cache, which
// this launch writes.
//
// Cross-workgroup exchange without fences.  Each thread waits for its
// partial stores to complete, then one arrival per workgroup is counted with
// an atomic add; the workgroup that counts last reads the partials.  The
// count returns to zero.  Two forms of it:
//   - XCD-local (the default where it holds): workgroups are dispatched to
//     the 8 XCDs round-robin by block index (checked once per context by
//     attn_xcd_round_robin), so the blocks of a head group are laid out on one
//     XCD and everything goes through that XCD's L2: plain stores, an L2
//     atomic, loads that bypass only L1.  Counters and partial rows are
//     padded to whole 256-byte lines so no line is shared by two XCDs.
//   - device-wide: agent-scope atomic stores (written through), an
//     agent-scope atomic add, system-coherent loads that bypass L2.
#include <type_traits>
#include <vector>

#include "common.h"

namespace terhip {
namespace {

constexpr int kAttnWaves = 4;  // query heads per workgroup (one wave each)
constexpr int kAttnThreads = kAttnWaves * 64;
constexpr int kChunk = 64;       // positions per chunk (one per lane)
constexpr int kMaxChunks = 64;   // combine: one lane per chunk
constexpr int kXcds = 8;         // XCDs of an MI355X, dispatched round-robin
constexpr int kCountStride = 64; // arrival counters, one per 256-byte line

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct AttnArgs {
    const uint16_t* q;      // fp16 [nh][hd], before RoPE
    const uint16_t* k;      // fp16 [nkv][hd], before RoPE
    const uint16_t* v;      // fp16 [nkv][hd]
    uint16_t* kc;           // fp16 [smax][nkv][hd] K cache of this layer
    uint16_t* vc;           // fp16 [smax][nkv][hd] V cache of this layer
    const int32_t* pos;     // device: the new token's position (< smax)
    uint16_t* out;          // fp16 [nh][hd]
    const float* rope;      // [smax][hd/2][2] (cos, sin)
    float* part;            // [nh][n_chunks][attn_part_stride(hd)]: o_c[hd], m_c, l_c
    unsigned* count;        // [n_groups][kCountStride], zero at rest
    int nh, nkv, smax, n_chunks, neox, groups_per_kv, n_groups;
    float inv_sqrt;
};

// The softmax exp is ter_expf (common.h), the same operations as the oracle's
// orc_expf, so both round identically.
__device__ __forceinline__ float attn_expf(float x) { return ter_expf(x); }

// RoPE of one pair (x0, x1) with table entry (c, s): the reference's
// v0*c - v1*s and v0*s + v1*c, each one fused multiply-add over the other
// product, rounded to fp16.
__device__ __forceinline__ void rope_pair(uint16_t& a, uint16_t& b, float c, float s) {
#pragma clang fp contract(off)
    const float v0 = half_bits_to_float(a), v1 = half_bits_to_float(b);
    const float r0 = __builtin_fmaf(v0, c, -(v1 * s));
    const float r1 = __builtin_fmaf(v0, s, v1 * c);
    a = float_to_half_bits(r0);
    b = float_to_half_bits(r1);
}

// Element indices of RoPE pair k of a head: NEOX (k, k + hd/2), NORM (2k, 2k+1).
__device__ __forceinline__ void pair_index(int k, int hd, bool neox, int& i0, int& i1) {
    i0 = neox ? k : 2 * k;
    i1 = neox ? k + hd / 2 : 2 * k + 1;
}

template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, true));
}

// Max over the 64 lanes (every lane gets it): DPP inside each row of 16
// lanes, then two cross-row exchanges (the max is exact in any order).
__device__ __forceinline__ float wave_max_f(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f<0x4E>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_f<0x140>(v));  // row_mirror
    v = fmaxf(v, lane_xor16(v));
    return fmaxf(v, lane_xor32(v));
}

// The xor butterfly sum  for o = 32, 16, ..., 1: v += v[lane ^ o]  (every
// lane ends with the same bits; each level adds the same two operands as the
// lane-shuffle form, so the result is that form's).  Levels 8 .. 1 use DPP
// inside a row of 16 lanes: xor 8 is a rotation by 8, xor 4 takes the row
// shifted by 4 in one direction or the other, xor 2 and 1 are quad
// permutations.
__device__ __forceinline__ float xor_sum64(float v) {
    v = v + lane_xor32(v);
    v = v + lane_xor16(v);
    v = v + dpp_f<0x128>(v);  // row_ror:8 (lane ^ 8 within the row)
    const float up = dpp_f<0x104>(v), down = dpp_f<0x114>(v);  // row_shl:4 (lane + 4), row_shr:4 (lane - 4)
    v = v + (((threadIdx.x & 4) == 0) ? up : down);
    v = v + dpp_f<0x4E>(v);   // quad_perm [2,3,0,1] (lane ^ 2)
    v = v + dpp_f<0xB1>(v);   // quad_perm [1,0,3,2] (lane ^ 1)
    return v;
}

// Floats per chunk partial (o_c[hd], m_c, l_c) rounded up to whole 256-byte lines.
constexpr int part_stride(int hd) { return (hd + 2 + 63) / 64 * 64; }

// kLocal: the XCD-local exchange (grid laid out by XCD), else device-wide.
template <int HD, bool kLocal>
__global__ __launch_bounds__(kAttnThreads) void attn_decode_kernel(AttnArgs a_in) {
#pragma clang fp contract(off)
    constexpr int PST = part_stride(HD);
    constexpr int KROW = HD * 2 + 16;  // padded K row in LDS (bytes): conflict-free 16-byte reads
    constexpr int VROW = HD * 2;
    constexpr int HALF = HD / 2;
    constexpr int DPT = HD / 64;       // output elements per thread
    static_assert(kAttnWaves * HALF <= kAttnThreads && HD <= kAttnThreads, "one RoPE pair / v element per thread");
    __shared__ __align__(16) unsigned char ks[kChunk * KROW];
    __shared__ __align__(16) unsigned char vs[kChunk * VROW];
    __shared__ __align__(16) uint16_t qs[kAttnWaves][HD];  // RoPE'd query heads (fp16, as the reference rounds them)
    __shared__ __align__(16) float es[kAttnWaves][kChunk];
    __shared__ int last_flag;

    // Every kernel argument in one round of scalar loads: left to itself the
    // compiler fetches them in several dependent rounds around the branches
    // below, each a scalar-cache miss on the launch's critical path.
    AttnArgs a = a_in;
    asm volatile("" : "+s"(a.q), "+s"(a.k), "+s"(a.v), "+s"(a.kc), "+s"(a.vc), "+s"(a.pos), "+s"(a.out),
                 "+s"(a.rope), "+s"(a.part), "+s"(a.count), "+s"(a.nh), "+s"(a.nkv), "+s"(a.smax),
                 "+s"(a.n_chunks), "+s"(a.neox), "+s"(a.groups_per_kv), "+s"(a.n_groups), "+s"(a.inv_sqrt));
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int grp, chunk;
    if constexpr (kLocal) {  // block b on XCD b % 8: group (r / n_chunks) * 8 + b % 8, r = b / 8
        const int x = blockIdx.x % kXcds, r = blockIdx.x / kXcds, gq = r / a.n_chunks;
        grp = gq * kXcds + x;
        chunk = r - gq * a.n_chunks;
        if (grp >= a.n_groups) return;
    } else {
        grp = blockIdx.x / a.n_chunks;
        chunk = blockIdx.x - grp * a.n_chunks;
    }
    const int g = grp / a.groups_per_kv;                      // KV head
    const int gs = a.nh / a.nkv;                              // query heads per KV head
    const int h0 = g * gs + (grp - g * a.groups_per_kv) * kAttnWaves;
    const int nhg = min(kAttnWaves, g * gs + gs - h0);        // query heads in this group
    const int s0 = chunk * kChunk;
    const long long row_stride = (long long)a.nkv * HD;        // halves between positions

    // 1. The chunk's K and V rows first (they do not depend on the position;
    // rows past smax are out of the buffers' range and read as zeros), with
    // the position as a scalar load beside them; then this position's RoPE
    // table entries and the new token's q pair, k pair and v element of this
    // thread (one each: nhg * hd/2 <= 256 query pairs).  These small loads
    // are unconditional, at clamped in-range addresses (values a thread does
    // not use are ignored), so no branch makes the compiler wait for them
    // early; they return right behind the cache rows.
    constexpr int kLoads = kChunk * VROW / 16 / kAttnThreads;  // 16-byte loads per thread per matrix
    const int cache_bytes = a.smax * (int)row_stride * 2;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(a.kc, 0, cache_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(a.vc, 0, cache_bytes, 0x00020000);
    u32x4 kreg[kLoads], vreg[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int idx = tid + i * kAttnThreads;               // 16-byte piece
        const int r = idx / (VROW / 16), cpart = idx - r * (VROW / 16);
        const int off = ((s0 + r) * (int)row_stride + g * HD + cpart * 8) * 2;
        kreg[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0);
        vreg[i] = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0);
    }
    asm volatile("" ::: "memory");  // keeps the row loads ahead of the branch on the position
    // the position through the scalar cache (invalidated at every launch;
    // nothing in this launch writes it), so waiting for it waits for no
    // vector load
    const int pos = *(const __attribute__((address_space(4))) int32_t*)(size_t)a.pos;
    const int pos_c = min(max(pos, 0), a.smax - 1);           // address only; checked below
    const int qi = tid / HALF, qk = tid - qi * HALF;          // query head of the group, pair
    int q0, q1;
    pair_index(qk, HD, a.neox != 0, q0, q1);
    const TER_GLOBAL float* tab = gptr(a.rope) + (long long)pos_c * HD;  // [hd/2][2] of this position
    const float rc = tab[2 * qk], rsn = tab[2 * qk + 1];
    const TER_GLOBAL uint16_t* qh = gptr(a.q) + (long long)min(h0 + qi, a.nh - 1) * HD;
    uint16_t qx0 = qh[q0], qx1 = qh[q1];
    const TER_GLOBAL uint16_t* kh = gptr(a.k) + (long long)g * HD;  // pair qk of the KV head's key
    uint16_t kx0 = kh[q0], kx1 = kh[q1];
    const uint16_t vx = gptr(a.v)[(long long)g * HD + min(tid, HD - 1)];
    if (pos < 0 || pos >= a.smax) return;                     // (the whole grid: no output, no count)
    const int seq = pos + 1;
    const int n = max(0, min(kChunk, seq - s0));              // positions in this chunk
    const bool has_pos = pos >= s0 && pos < s0 + kChunk;
    const bool writer = has_pos && grp == g * a.groups_per_kv;  // one workgroup per KV head writes the cache

    // 2. RoPE of the group's query heads into qs (as the fp16-rounded values).
    // (every thread: rows of heads past the group's hold values no wave reads,
    // and an unconditional use keeps the q loads ahead of the cache rows)
    rope_pair(qx0, qx1, rc, rsn);
    qs[qi][q0] = qx0;
    qs[qi][q1] = qx1;
    // stage K (padded rows) and V; rows past the sequence as zeros
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int idx = tid + i * kAttnThreads;
        const int r = idx / (VROW / 16), cpart = idx - r * (VROW / 16);
        const bool live = r < n;
        *reinterpret_cast<u32x4*>(ks + r * KROW + cpart * 16) = live ? kreg[i] : u32x4{0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(vs + r * VROW + cpart * 16) = live ? vreg[i] : u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();
    // the new position: RoPE(k) and v from the projections (the cache holds
    // the old contents until this launch writes it)
    if (has_pos) {
        const int r = pos - s0;
        uint16_t* krow = reinterpret_cast<uint16_t*>(ks + r * KROW);
        uint16_t* vrow = reinterpret_cast<uint16_t*>(vs + r * VROW);
        if (tid < HALF) {  // pair tid: the same table entry as query pair tid
            rope_pair(kx0, kx1, rc, rsn);
            krow[q0] = kx0;
            krow[q1] = kx1;
            if (writer) {
                uint16_t* kd = a.kc + (long long)pos * row_stride + (long long)g * HD;
                gptr(kd)[q0] = kx0;
                gptr(kd)[q1] = kx1;
            }
        }
        if (tid < HD) {
            vrow[tid] = vx;
            if (writer) gptr(a.vc + (long long)pos * row_stride + (long long)g * HD)[tid] = vx;
        }
    }
    __syncthreads();

    // 3. scores: wave i = query head i, lane = position (the reference's dot order)
    const bool head_ok = wave < nhg;
    float score = -__builtin_inff();
    if (head_ok && lane < n) {
        // blocks of 32 d: the block's K row and query values are read from
        // LDS into registers together, then the 32-step chain runs
        float dot = 0.f;
        const unsigned char* krow = ks + lane * KROW;
        const unsigned char* qrow = reinterpret_cast<const unsigned char*>(qs[wave]);
#pragma unroll
        for (int b = 0; b < HD; b += 32) {
            u32x4 kw[4], qw[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                kw[i] = *reinterpret_cast<const u32x4*>(krow + (b + 8 * i) * 2);
                qw[i] = *reinterpret_cast<const u32x4*>(qrow + (b + 8 * i) * 2);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    dot = __builtin_fmaf(half_bits_to_float((uint16_t)(qw[i][j] & 0xFFFFu)),
                                         half_bits_to_float((uint16_t)(kw[i][j] & 0xFFFFu)), dot);
                    dot = __builtin_fmaf(half_bits_to_float((uint16_t)(qw[i][j] >> 16)),
                                         half_bits_to_float((uint16_t)(kw[i][j] >> 16)), dot);
                }
        }
        score = dot * a.inv_sqrt;
    }
    // 4. chunk softmax statistics per head
    const float mc = wave_max_f(score);
    const float e = lane < n ? attn_expf(score - mc) : 0.f;
    float lsum = e;
    lsum = xor_sum64(lsum);
    es[wave][lane] = e;
    __syncthreads();

    // 5. output partials: thread (i, DPT consecutive d), positions in order.
    // All 64 rows: past n, e = 0 and the V row is zero, so those steps add +0
    // to an accumulator that is never -0 (exact no-ops), and the loop is
    // unrolled with its LDS reads scheduled ahead.
    float acc[DPT];
#pragma unroll
    for (int j = 0; j < DPT; ++j) acc[j] = 0.f;
    const int d0 = DPT * lane;
    if (head_ok) {
        // blocks of 16 positions: their weights and V values are read from
        // LDS into registers together, then the block's steps run in order
#pragma unroll
        for (int b = 0; b < kChunk; b += 16) {
            float wv[16];
            uint16_t vv[16][DPT];
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const float4 w4 = *reinterpret_cast<const float4*>(&es[wave][b + i]);
                wv[i] = w4.x;
                wv[i + 1] = w4.y;
                wv[i + 2] = w4.z;
                wv[i + 3] = w4.w;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint16_t* vrow = reinterpret_cast<const uint16_t*>(vs + (b + i) * VROW) + d0;
#pragma unroll
                for (int j = 0; j < DPT; ++j) vv[i][j] = vrow[j];
            }
#pragma unroll
            for (int i = 0; i < 16; ++i)
#pragma unroll
                for (int j = 0; j < DPT; ++j) acc[j] = __builtin_fmaf(wv[i], half_bits_to_float(vv[i][j]), acc[j]);
        }
    }
    // One chunk holds every position (seq <= kChunk): its workgroup combines
    // that chunk itself, with the combine's own operations (w = exp(m - M)
    // with M = m, so w = 1; L and O by the same fused multiply-adds), so the
    // same bits; no workgroup publishes or counts, and the counter stays zero.
    if (seq <= kChunk) {
        if (chunk != 0 || !head_ok) return;
        const float w = attn_expf(mc - mc);
        const float L = __builtin_fmaf(lsum, w, 0.f);
        uint16_t* oh = a.out + (long long)(h0 + wave) * HD + d0;
#pragma unroll
        for (int j = 0; j < DPT; ++j) gptr(oh)[j] = float_to_half_bits(__builtin_fmaf(acc[j], w, 0.f) / L);
        return;
    }

    // 6. publish the partials (written through), then count the arrival
    constexpr int kScope = kLocal ? __HIP_MEMORY_SCOPE_WORKGROUP : __HIP_MEMORY_SCOPE_AGENT;
    if (head_ok && n > 0) {
        float* P = a.part + ((long long)(h0 + wave) * a.n_chunks + chunk) * PST;
#pragma unroll
        for (int j = 0; j < DPT; ++j) __hip_atomic_store(P + d0 + j, acc[j], __ATOMIC_RELAXED, kScope);
        if (lane == 0) {
            __hip_atomic_store(P + HD, mc, __ATOMIC_RELAXED, kScope);
            __hip_atomic_store(P + HD + 1, lsum, __ATOMIC_RELAXED, kScope);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores are complete
    asm volatile("" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        unsigned* cnt = a.count + grp * kCountStride;
        const unsigned prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, kScope);
        last_flag = prev == (unsigned)a.n_chunks - 1u;
        if (last_flag) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, kScope);
    }
    __syncthreads();
    if (!last_flag || !head_ok) return;

    // 7. combine (last workgroup of the group): chunks in order.  The
    // partials are read with buffer loads that miss any stale copy (L1 for
    // the XCD-local exchange: SC0; L1 and this XCD's L2 otherwise: SC1);
    // chunks past nc are out of the buffer's range and read as zeros.  Lane c
    // holds chunk c's (m_c, l_c).  Every load is issued before the first
    // add (groups of 8 chunks, each group behind a wave-uniform test of nc),
    // so the chain waits for one round trip, not one per group.
    const int nc = (seq + kChunk - 1) / kChunk;
    const float* Ph = a.part + (long long)(h0 + wave) * a.n_chunks * PST;
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc((void*)Ph, 0, nc * PST * 4, 0x00020000);
    constexpr int kCoh = kLocal ? 1 : 16;  // cache policy: SC0 / SC1
    constexpr int G = 8;                   // chunks per group
    constexpr int NG = kMaxChunks / G;
    const unsigned long long ml =
        __builtin_bit_cast(unsigned long long, __builtin_amdgcn_raw_buffer_load_b64(pr, (lane * PST + HD) * 4, 0, kCoh));
    float pg[NG][G][DPT];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        if (gi * G < nc) {
#pragma unroll
            for (int c = 0; c < G; ++c) {
                const int off = ((gi * G + c) * PST + d0) * 4;
                if constexpr (DPT == 2) {
                    const unsigned long long w2 = __builtin_bit_cast(
                        unsigned long long, __builtin_amdgcn_raw_buffer_load_b64(pr, off, 0, kCoh));
                    pg[gi][c][0] = __builtin_bit_cast(float, (unsigned)w2);
                    pg[gi][c][1] = __builtin_bit_cast(float, (unsigned)(w2 >> 32));
                } else {
                    pg[gi][c][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pr, off, 0, kCoh));
                }
            }
        }
    }
    const float m_l = lane < nc ? __builtin_bit_cast(float, (unsigned)ml) : -__builtin_inff();
    const float M = wave_max_f(m_l);
    // lane c's weight and sum, read with v_readlane (a uniform lane per step)
    const int w_bits = __builtin_bit_cast(int, lane < nc ? attn_expf(m_l - M) : 0.f);
    const int l_bits = (int)(unsigned)(ml >> 32);
    float L = 0.f;
    float O[DPT];
#pragma unroll
    for (int j = 0; j < DPT; ++j) O[j] = 0.f;
    // chunks past nc in the last group have w = 0 and o = 0: exact no-ops;
    // at most 64 chunks, so every lane index read below is < 64
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        if (gi * G < nc) {
#pragma unroll
            for (int c = 0; c < G; ++c) {
                const int src = gi * G + c;
                const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(w_bits, src));
                L = __builtin_fmaf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(l_bits, src)), w, L);
#pragma unroll
                for (int j = 0; j < DPT; ++j) O[j] = __builtin_fmaf(pg[gi][c][j], w, O[j]);
            }
        }
    }
    uint16_t* oh = a.out + (long long)(h0 + wave) * HD + d0;
#pragma unroll
    for (int j = 0; j < DPT; ++j) gptr(oh)[j] = float_to_half_bits(O[j] / L);
}

// Standalone RoPE on fp16 head vectors in place (rope_k), one thread per pair.
__global__ void rope_kernel(uint16_t* v, int n_heads, int hd, const float* rope, const int32_t* pos_dev, int smax,
                            int neox) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    const int half = hd / 2;
    if (idx >= n_heads * half) return;
    const int h = idx / half, kk = idx - h * half;
    const int pos = *gptr(pos_dev);
    if (pos < 0 || pos >= smax) return;
    int i0, i1;
    pair_index(kk, hd, neox != 0, i0, i1);
    uint16_t* vh = v + (long long)h * hd;
    uint16_t x0 = gptr(vh)[i0], x1 = gptr(vh)[i1];
    const TER_GLOBAL float* t = gptr(rope) + ((long long)pos * half + kk) * 2;
    rope_pair(x0, x1, t[0], t[1]);
    gptr(vh)[i0] = x0;
    gptr(vh)[i1] = x1;
}

// Records the XCD of every block (XCC_ID hardware register).
__global__ void xcc_probe_kernel(int* out) {
    if (threadIdx.x == 0) {
        unsigned v;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
        out[blockIdx.x] = (int)(v & 0xFu);
    }
}

}  // namespace

bool attn_supported_head_dim(int hd) { return hd == 64 || hd == 128; }
int attn_part_stride(int hd) { return part_stride(hd); }
int attn_count_stride() { return kCountStride; }
int attn_head_groups(int nh, int nkv) { return nkv * ((nh / nkv + kAttnWaves - 1) / kAttnWaves); }

int attn_local_blocks(int nh, int nkv, int smax) {
    const int groups = attn_head_groups(nh, nkv);
    return kXcds * ((groups + kXcds - 1) / kXcds) * ((smax + kChunk - 1) / kChunk);
}

bool attn_xcd_round_robin(int n_blocks, int* scratch, hipStream_t st) {
    std::vector<int> h((size_t)n_blocks);
    for (int rep = 0; rep < 4; ++rep) {  // (a few launches: the mapping must hold every time)
        hipLaunchKernelGGL(xcc_probe_kernel, dim3(n_blocks), dim3(64), 0, st, scratch);
        if (hipGetLastError() != hipSuccess) return false;
        if (hipMemcpyAsync(h.data(), scratch, sizeof(int) * (size_t)n_blocks, hipMemcpyDeviceToHost, st) !=
                hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess)
            return false;
        for (int b = 0; b < n_blocks; ++b)
            if (h[(size_t)b] != b % kXcds) return false;
    }
    return true;
}

int attn_chunk() { return kChunk; }
int attn_max_chunks() { return kMaxChunks; }

hipError_t launch_attn_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* kc, uint16_t* vc,
                              const int32_t* pos, uint16_t* out, const float* rope, float* part, unsigned* count,
                              int nh, int nkv, int hd, int smax, bool neox, bool xcd_local, hipStream_t st) {
    AttnArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.kc = kc;
    a.vc = vc;
    a.pos = pos;
    a.out = out;
    a.rope = rope;
    a.part = part;
    a.count = count;
    a.nh = nh;
    a.nkv = nkv;
    a.smax = smax;
    a.n_chunks = (smax + kChunk - 1) / kChunk;
    a.neox = neox ? 1 : 0;
    a.groups_per_kv = (nh / nkv + kAttnWaves - 1) / kAttnWaves;
    a.n_groups = nkv * a.groups_per_kv;
    a.inv_sqrt = (float)(1.0 / __builtin_sqrt((double)hd));
    const dim3 block(kAttnThreads);
    if (xcd_local) {
        const dim3 grid(attn_local_blocks(nh, nkv, smax));
        if (hd == 128)
            hipLaunchKernelGGL((attn_decode_kernel<128, true>), grid, block, 0, st, a);
        else
            hipLaunchKernelGGL((attn_decode_kernel<64, true>), grid, block, 0, st, a);
    } else {
        const dim3 grid(a.n_groups * a.n_chunks);
        if (hd == 128)
            hipLaunchKernelGGL((attn_decode_kernel<128, false>), grid, block, 0, st, a);
        else
            hipLaunchKernelGGL((attn_decode_kernel<64, false>), grid, block, 0, st, a);
    }
    return hipGetLastError();
}

hipError_t launch_rope(uint16_t* v, int n_heads, int hd, const float* rope, const int32_t* pos, int smax, bool neox,
                       hipStream_t st) {
    const int n = n_heads * (hd / 2);
    hipLaunchKernelGGL(rope_kernel, dim3((n + 255) / 256), dim3(256), 0, st, v, n_heads, hd, rope, pos, smax,
                       neox ? 1 : 0);
    return hipGetLastError();
}

}  // namespace terhip
