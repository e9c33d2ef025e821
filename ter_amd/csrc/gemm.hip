// gemm.hip -- M > 1 packed-trit GEMM on gfx950 MFMA (v_mfma_i32_16x16x64_i8).
//
// Replaces the reference's batched kernels (mm_packed_batched,
// cuda/ter_cuda_packed_batched.cu:26-83; mm_bitnet_addonly_batched_k<M>,
// cuda/ter_cuda_addonly_batched.cu:31-124; the wmma s4 mm_int4_tc*).
// Semantics: acc[m][j] = sum_k X[m][k] w[k][j] (exact int32) and
// y[m][j] = float(mag * acc[m][j]) * (x_scale[m] * w_scale), mag the payload magnitude
// (cuda/ter_cuda_addonly_batched.cu:117-123).
//
// Input is the same T16 tile stream as the GEMV (common.h).  Work is a list
// of GEMMs cut into blocks of 4 column strips (64 columns) x all K; the
// blocks of the whole list form one stream, cut into equal contiguous ranges,
// one per workgroup of 4 waves (one strip per wave).  For every 256-row unit
// the workgroup stages X[0:M, unit] (int8) in LDS once for its 4 waves; the
// next unit's X and packed weights are loaded into registers while the
// current unit is multiplied, and the LDS copy of X is double-buffered, so a
// unit costs one barrier.  Each wave gathers its strip's packed weights
// straight into the MFMA B operand layout (lane = column j + 16 * k-group g;
// one dword = 16 trits of column j), expands the 2-bit u = w + 1 codes to
// int8 with 7 bit operations per 16 trits, and runs one MFMA per 16-row block
// and 64-row slab.  The u encoding adds sum_k X[m][k] to every output; it is
// subtracted in the epilogue from row sums gathered while staging X (rows and
// padding the kernel stages but the weights' padding rows hold u = 1, so any
// staged padding cancels exactly).
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
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

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

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

constexpr int kLdRow = kUnitK + 16;  // padded LDS row of staged X (bytes)

// X[row][k0 .. k0+15] of one GEMM (zeros past M; bytes past K are whatever
// the row holds there, or zero past the end of X -- both cancel, see above).
template <bool kVec>
__device__ __forceinline__ u32x4 load_x16(const GemmDesc& d, __amdgpu_buffer_rsrc_t xr, int row, int k0) {
    // Rows >= M lie past the buffer's M * ldx bytes and read as zeros, so the
    // vector load needs no branch (a divergent branch around a load forces
    // the wait counters to drain at the join).
    if (kVec) return __builtin_amdgcn_raw_buffer_load_b128(xr, row * d.ldx + k0, 0, 0);
    if (row >= d.M) return u32x4{0u, 0u, 0u, 0u};
    unsigned wd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        unsigned a = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int k = k0 + 4 * i + b;
            const unsigned by = k < d.K ? (unsigned)(uint8_t)gptr(d.x)[(long long)row * d.ldx + k] : 0u;
            a |= by << (8 * b);
        }
        wd[i] = a;
    }
    return u32x4{wd[0], wd[1], wd[2], wd[3]};
}

// Registers of one unit in flight: the wave's S strips x 4 gathered weight
// dwords, and this thread's MB staged activation chunks.
template <int MB, int S>
struct UnitRegs {
    unsigned w[S][4];
    u32x4 x[MB];
};

template <int MB, int S, bool kVec>
__device__ __forceinline__ void load_unit(UnitRegs<MB, S>& r, const GemmDesc& d, __amdgpu_buffer_rsrc_t wr,
                                          __amdgpu_buffer_rsrc_t xr, int woff, int srow, int sch, int u) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
        // tile offset in the range-checked vector offset (the scalar offset
        // is not range-checked), so loads past the wave's strips read zeros
        const int toff = woff + (s * d.Ku + u) * kTileBytes;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            r.w[s][ks] = __builtin_amdgcn_raw_buffer_load_b32(wr, toff + ks * 64, 0, 2 /* nt */);
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) r.x[i] = load_x16<kVec>(d, xr, srow + 16 * i, u * kUnitK + sch * 16);
}

// Stage unit u's activations (from registers) in LDS buffer u % 2, then
// multiply the wave's strips by them.
template <int MB, int S>
__device__ __forceinline__ void run_unit(const UnitRegs<MB, S>& r, int8_t (*xl)[MB * 16 * kLdRow], int u,
                                         int srow, int sch, int j, int g, bool act, int (&rs)[MB],
                                         i32x4 (&C)[S][MB]) {
    int8_t* xb = xl[u & 1];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        *reinterpret_cast<u32x4*>(xb + (srow + 16 * i) * kLdRow + sch * 16) = r.x[i];
        rs[i] += row_sum16(sum_bytes(r.x[i]));
    }
    __syncthreads();  // X[:, u] staged; buffer u % 2 was last read two units ago
    if (act) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            i32x4 A[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                A[mb] = *reinterpret_cast<const i32x4*>(xb + (mb * 16 + j) * kLdRow + ks * 64 + g * 16);
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const unsigned dw = r.w[s][ks];
                const i32x4 B = i32x4{(int)(dw & 0x03030303u), (int)((dw >> 2) & 0x03030303u),
                                      (int)((dw >> 4) & 0x03030303u), (int)((dw >> 6) & 0x03030303u)};
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    C[s][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[mb], B, C[s][mb], 0, 0, 0);
            }
        }
    }
}

template <int MB, int S, bool kList, bool kVec>
__global__ __launch_bounds__(kThreads) void gemm_t16_kernel(GemmDesc single, const GemmDesc* __restrict__ list,
                                                            const int32_t* __restrict__ first, long long total_blocks,
                                                            int n_wg) {
#pragma clang fp contract(off)
    constexpr int ROWS = MB * 16;
    __shared__ __align__(16) int8_t xl[2][ROWS * kLdRow];
    __shared__ int rsum[ROWS];
    int gi = blockIdx.x;
    if ((n_wg & 7) == 0) gi = (gi & 7) * (n_wg >> 3) + (gi >> 3);  // neighbouring ranges on one XCD
    const long long b_begin = total_blocks * gi / n_wg;
    const long long b_end = total_blocks * (gi + 1) / n_wg;
    if (b_begin >= b_end) return;
    int di = kList ? first[gi] : 0;  // the descriptor holding this range's start
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = uniform(tid >> 6);
    const int g = lane >> 4, j = lane & 15;
    // staging role: chunk c = tid + 256 i covers row tid / 16 + 16 i, bytes 16 (tid % 16)
    const int srow = tid >> 4, sch = tid & 15;
    // weight gather offset of this lane inside a tile (B operand layout)
    const int woff = (j >> 2) * 256 + g * 16 + (j & 3) * 4;

    for (long long b = b_begin; b < b_end; ++b) {
        if (kList) {
            while (b >= list[di].block0 + list[di].n_blocks) ++di;
        }
        const GemmDesc d = kList ? list[di] : single;
        // this wave's strips: st0 .. st0 + S - 1 (those < n_strips are active)
        const int st0 = ((int)(b - d.block0) * kWaves + wave) * S;
        const int n_act = min(S, d.n_strips - st0);  // may be <= 0
        const bool act = n_act > 0;
        const int Ku = d.Ku;
        const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(d.w + (long long)(act ? st0 : 0) * Ku * kTileBytes), 0, act ? n_act * Ku * kTileBytes : 0,
            0x00020000);
        const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)d.x, 0, d.M * d.ldx, 0x00020000);

        i32x4 C[S][MB];
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) C[s][mb] = i32x4{0, 0, 0, 0};
        int rs[MB];
#pragma unroll
        for (int i = 0; i < MB; ++i) rs[i] = 0;

        // kDepth units in flight: unit u is multiplied while the next
        // kDepth - 1 load (three for small M, two where the registers are
        // needed for row blocks).  Loads are unpredicated: past a strip they
        // read the next strip's first units (unused) or, past the last strip,
        // zeros.
        constexpr int kDepth = MB <= 2 ? 3 : 2;
        UnitRegs<MB, S> r0, r1, r2;
        load_unit<MB, S, kVec>(r0, d, wr, xr, woff, srow, sch, 0);
        if constexpr (kDepth == 3) {
            load_unit<MB, S, kVec>(r1, d, wr, xr, woff, srow, sch, 1);
            for (int u = 0; u < Ku; u += 3) {
                load_unit<MB, S, kVec>(r2, d, wr, xr, woff, srow, sch, u + 2);
                run_unit<MB, S>(r0, xl, u, srow, sch, j, g, act, rs, C);
                if (u + 1 >= Ku) break;
                load_unit<MB, S, kVec>(r0, d, wr, xr, woff, srow, sch, u + 3);
                run_unit<MB, S>(r1, xl, u + 1, srow, sch, j, g, act, rs, C);
                if (u + 2 >= Ku) break;
                load_unit<MB, S, kVec>(r1, d, wr, xr, woff, srow, sch, u + 4);
                run_unit<MB, S>(r2, xl, u + 2, srow, sch, j, g, act, rs, C);
            }
        } else {
            (void)r2;
            for (int u = 0; u < Ku; u += 2) {
                load_unit<MB, S, kVec>(r1, d, wr, xr, woff, srow, sch, u + 1);
                run_unit<MB, S>(r0, xl, u, srow, sch, j, g, act, rs, C);
                if (u + 1 >= Ku) break;
                load_unit<MB, S, kVec>(r0, d, wr, xr, woff, srow, sch, u + 2);
                run_unit<MB, S>(r1, xl, u + 1, srow, sch, j, g, act, rs, C);
            }
        }
#pragma unroll
        for (int i = 0; i < MB; ++i)
            if (sch == 0) rsum[srow + 16 * i] = rs[i];
        __syncthreads();
        // The output fields through an opaque copy: with one GEMM they are
        // loop-invariant, and the compiler would otherwise hoist every row's
        // output addresses and checks out of the block loop into registers.
        GemmDesc o_d = d;
        asm volatile("" : "+s"(o_d.N), "+s"(o_d.M), "+s"(o_d.y), "+s"(o_d.acc), "+s"(o_d.y16), "+s"(o_d.resid),
                     "+s"(o_d.xs), "+s"(o_d.w_scale), "+s"(o_d.w_mag));
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int col = (st0 + s) * kStripCols + j;
            if (s < n_act && col < o_d.N) {
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int row = mb * 16 + g * 4 + e;
                        if (row < o_d.M) {
                            const int val = C[s][mb][e] - rsum[row];
                            const long long o = (long long)row * o_d.N + col;
                            emit_out(o_d, o, val, gptr(o_d.xs)[row] * o_d.w_scale);
                        }
                    }
                }
            }
        }
        __syncthreads();  // rsum and the X buffers are reused by the next block
    }
}


// ---------------------------------------------------------------------------
// Streaming variant for M <= 16 (one MFMA row block).  The work list is one
// stream of tiles cut into equal contiguous ranges per workgroup, like the
// M = 1 GEMV; a workgroup owns the strips whose first tile lies in its range.
// Per GEMM segment it stages the whole X[0:M][0:Ku*256] in LDS once, then
// each wave streams the tiles of a contiguous run of whole strips with two
// batches of tiles in registers and no further barrier.  A strip's 16 x 16
// MFMA accumulator is written when its last unit is in.
//
// Staging.  The LDS image of X is a sequence of 16-byte chunks, row r's
// chunk c at index r * (Ku * 16 + 1) + c (one padding chunk per row, so the
// 16 rows an A operand reads fall on distinct banks).  Every thread loads
// its (at most kStageChunks) chunks into registers at once through a buffer
// resource (chunks past the end read zeros, so no load is predicated), then
// the segment's first weight batch is issued, then the chunks are written
// to LDS: the writes wait only for the X loads (older than the weights), in
// one L2 round trip for the whole X.  Row sums are gathered on the way (the
// u = w + 1 codes feed the MFMA as they are, 7 bit operations per 16 trits,
// and the epilogue subtracts sum_k X[m][k]); the lanes of rows >= M read a
// zero row kept after the X image instead of masking their A operands.
constexpr int kSWaves = 4;                  // waves per workgroup (all sharing one X image)
constexpr int kSThreads = 64 * kSWaves;
constexpr int kStageChunks = 65536 / 16 / kSThreads;  // chunks per thread: the 64 KiB LDS limit
constexpr int kSBatch = kGemmStreamBatch;   // tiles per batch, two batches per wave in flight

// Chunks of one staged row (Ku * 16) plus its padding chunk.
__device__ __forceinline__ int stream_row_chunks(int Ku) { return Ku * (kUnitK / 16) + 1; }

// This thread's chunks of X (16-byte aligned rows), in registers.
struct XStage {
    u32x4 v[kStageChunks];
};

__device__ __forceinline__ void stage_load(const GemmDesc& d, XStage& x) {
    const int per = stream_row_chunks(d.Ku) - 1;
    const int nch = d.M * per;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)d.x, 0, d.M * d.ldx, 0x00020000);
#pragma unroll
    for (int i = 0; i < kStageChunks; ++i) {
        const int c = threadIdx.x + kSThreads * i;
        const int row = c / per, ch = c - row * per;
        x.v[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, c < nch ? row * d.ldx + ch * 16 : 0x7FFFFFF0, 0, 0);
    }
}

// Write the staged chunks to LDS and add their bytes into rsum[row] (zero
// before the call).  per = Ku * 16 is a multiple of 16 and a thread's chunks
// are tid + 256 i, so the 16 lanes of a DPP row hold chunks of one row.
__device__ __forceinline__ void stage_store(const GemmDesc& d, const XStage& x, int8_t* lx, int* rsum) {
    const int rc = stream_row_chunks(d.Ku), per = rc - 1;
    const int nch = d.M * per;
#pragma unroll
    for (int i = 0; i < kStageChunks; ++i) {
        const int c = threadIdx.x + kSThreads * i;
        const int row = c / per, ch = c - row * per;
        if (c < nch) {
            *reinterpret_cast<u32x4*>(lx + (row * rc + ch) * 16) = x.v[i];
            const int sm = row_sum16(sum_bytes(x.v[i]));
            if ((threadIdx.x & 15) == 0) atomicAdd(rsum + row, sm);
        }
    }
}

// Byte-wise staging from registers (rows not 16-byte aligned), row sums too.
__device__ __forceinline__ void stage_rows_bytes(const GemmDesc& d, int8_t* lx, int* rsum) {
    const int rc = stream_row_chunks(d.Ku);
    const int nch = d.M * (rc - 1);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)d.x, 0, d.M * d.ldx, 0x00020000);
    for (int c = threadIdx.x; c < nch; c += kSThreads) {
        const int row = c / (rc - 1), ch = c - row * (rc - 1);
        const u32x4 v = load_x16<false>(d, xr, row, ch * 16);
        *reinterpret_cast<u32x4*>(lx + (row * rc + ch) * 16) = v;
        const int sm = row_sum16(sum_bytes(v));
        if ((threadIdx.x & 15) == 0) atomicAdd(rsum + row, sm);
    }
}

// A batch of NB tiles: one 16-byte load per lane and tile, lane L taking
// bytes [16 L, 16 L + 16) of the contiguous 1 KiB tile (the GEMV's loads).
template <int NB>
__device__ __forceinline__ void stream_load(u32x4 (&w)[NB], __amdgpu_buffer_rsrc_t rs, int i0) {
    const int voff = (threadIdx.x & 63) * 16;
#pragma unroll
    for (int i = 0; i < NB; ++i)  // range-checked: zeros past the wave's tiles
        w[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + (i0 + i) * kTileBytes, 0, 2 /* nt */);
}

struct StreamState {
    int strip, u;
    int nbuf;  // completed strips in the wave's output buffer
    i32x4 C;
};

// Reduce tiles [i0, min(i0 + NB, n)) of the wave's run.  Each tile goes
// through the wave's two 1 KiB LDS slots (tile order in, MFMA B order out):
// lane (j, g) takes, for slab ks, the dword of column j over rows
// 64 ks + 16 g .. +15 at tile offset (j >> 2) * 256 + (4 ks + g) * 16 + (j & 3) * 4.
// A wave's LDS operations run in order, so the slot written for tile i + 1
// while tile i is read back never overtakes the reads of tile i - 1.
template <int NB>
__device__ __forceinline__ void stream_compute(const GemmDesc& d, const u32x4 (&w)[NB], int i0, int n,
                                               const int8_t* arow, unsigned char* slot, int* obuf, int out_rows,
                                               const int (&rs)[4], StreamState& p) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, j = lane & 15;
    const int roff = (j >> 2) * 256 + g * 16 + (j & 3) * 4;
    *reinterpret_cast<u32x4*>(slot + lane * 16) = w[0];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        if (i + 1 < NB) *reinterpret_cast<u32x4*>(slot + ((i + 1) & 1) * kTileBytes + lane * 16) = w[i + 1];
        if (i0 + i < n) {
            const unsigned char* ts = slot + (i & 1) * kTileBytes + roff;
            const int8_t* ab = arow + p.u * kUnitK + g * 16;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const i32x4 A = *reinterpret_cast<const i32x4*>(ab + ks * 64);
                const unsigned dw = *reinterpret_cast<const unsigned*>(ts + ks * 64);
                const i32x4 B = i32x4{(int)(dw & 0x03030303u), (int)((dw >> 2) & 0x03030303u),
                                      (int)((dw >> 4) & 0x03030303u), (int)((dw >> 6) & 0x03030303u)};
                p.C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, p.C, 0, 0, 0);
            }
            if (++p.u == d.Ku) {
                // the strip's results into the output buffer (rows of 16 columns)
                int* ob = obuf + p.nbuf * out_rows * kStripCols;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int row = g * 4 + e;
                    if (row < d.M) ob[row * kStripCols + j] = p.C[e] - rs[e];
                }
                p.C = i32x4{0, 0, 0, 0};
                p.u = 0;
                ++p.strip;
                ++p.nbuf;
            }
        }
    }
}

template <bool kList, bool kVec>
__global__ __launch_bounds__(kSThreads) void gemm_stream_kernel(GemmDesc single, const GemmDesc* __restrict__ list,
                                                               const int32_t* __restrict__ first, long long total,
                                                               int n_wg, int lds_bytes) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    int gi = blockIdx.x;
    if ((n_wg & 7) == 0) gi = (gi & 7) * (n_wg >> 3) + (gi >> 3);
    const long long t_begin = total * gi / n_wg;
    const long long t_end = total * (gi + 1) / n_wg;
    if (t_begin >= t_end) return;
    int di = kList ? first[gi] : 0;  // the descriptor holding this range's start
    const int lane = threadIdx.x & 63;
    const int wave = uniform(threadIdx.x >> 6);
    const int g = lane >> 4, j = lane & 15;
    long long t = t_begin;
    while (t < t_end) {
        const GemmDesc d = kList ? list[di] : single;
        const long long seg_end = min(t_end, d.tile0 + (long long)d.n_strips * d.Ku);
        const int la = (int)(t - d.tile0), lb = (int)(seg_end - d.tile0);
        // the strips whose first tile lies in [la, lb)
        const int st_a = (la + d.Ku - 1) / d.Ku, st_b = (lb + d.Ku - 1) / d.Ku;
        const int ns = st_b - st_a;
        const int w_a = st_a + ns * wave / kSWaves, w_b = st_a + ns * (wave + 1) / kSWaves;
        const int n = (w_b - w_a) * d.Ku;  // this wave's tiles
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(d.w + (long long)w_a * d.Ku * kTileBytes), 0, n * kTileBytes, 0x00020000);
        const int rc = stream_row_chunks(d.Ku);
        unsigned char* lx = lds_raw;
        // this segment's LDS layout (common.h, gemm_stream_out_off)
        const int zero_off = gemm_stream_zero_off(d.M, d.K);
        const int out_off = gemm_stream_out_off(d.M, d.K);
        const int out_strips = gemm_stream_out_strips(d.M, d.K, lds_bytes);
        unsigned char* slot = lds_raw + zero_off + d.Ku * kUnitK + 64 + wave * 2 * kTileBytes;  // this wave's 2 tiles
        int* obuf = reinterpret_cast<int*>(lds_raw + out_off) + wave * out_strips * d.M * kStripCols;
        // rows 4g .. 4g + 3's scales in one load, rows past M reading zeros
        const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc((void*)d.xs, 0, d.M * 4, 0x00020000);
        const u32x4 xsw = __builtin_amdgcn_raw_buffer_load_b128(sr, g * 16, 0, 0);
        u32x4 wa[kSBatch], wb[kSBatch];
        int* rsum = reinterpret_cast<int*>(lds_raw + zero_off + d.Ku * kUnitK);
        // the zero row read by the A operands of rows >= M, and the row sums
        auto clear = [&]() {
            for (int c = threadIdx.x; c < d.Ku * (kUnitK / 16); c += kSThreads)
                *reinterpret_cast<u32x4*>(lds_raw + zero_off + c * 16) = u32x4{0u, 0u, 0u, 0u};
            if (threadIdx.x < 16) rsum[threadIdx.x] = 0;
        };
        if constexpr (kVec) {
            XStage xst;
            stage_load(d, xst);           // X first: its writes below wait for nothing else
            stream_load(wa, rs, 0);
            __syncthreads();              // the previous segment is done with LDS
            clear();
            __syncthreads();
            if (ns > 0) stage_store(d, xst, reinterpret_cast<int8_t*>(lx), rsum);
        } else {
            stream_load(wa, rs, 0);
            __syncthreads();
            clear();
            __syncthreads();
            if (ns > 0) stage_rows_bytes(d, reinterpret_cast<int8_t*>(lx), rsum);
        }
        // the rows' output scales x_scale[r] * w_scale for the flushes: lane
        // 16 g + e of wave 0 writes row 4 g + e (its xsw holds rows 4 g .. 4 g + 3)
        float* xs_l = reinterpret_cast<float*>(lds_raw + out_off - 64);
        if (wave == 0 && j < 4) {
            const unsigned b = j == 0 ? xsw[0] : (j == 1 ? xsw[1] : (j == 2 ? xsw[2] : xsw[3]));
            xs_l[g * 4 + j] = __builtin_bit_cast(float, b) * d.w_scale;
        }
        __syncthreads();
        if (n > 0) {
            // rows >= M read the zero row (their outputs are not written)
            const int8_t* arow = reinterpret_cast<const int8_t*>(lx) + (j < d.M ? j * rc * 16 : zero_off);
            int rsr[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) rsr[e] = rsum[g * 4 + e];
            StreamState p{0, 0, 0, i32x4{0, 0, 0, 0}};
            // Chunks of C tiles (whole double batches, at most (S - 1) Ku, so
            // at most S strips complete in one), their strips written between
            // chunks while the next chunk's first batch is in flight.
            const int C = 2 * kSBatch * max(1, (out_strips - 1) * d.Ku / (2 * kSBatch));
            int st_flush = 0;  // the run's strip index of the buffer's first strip
            int i0 = 0;
            while (true) {
                const int cend = min(n, i0 + C);
                while (true) {
                    stream_load(wb, rs, i0 + kSBatch);
                    stream_compute(d, wa, i0, n, arow, slot, obuf, d.M, rsr, p);
                    i0 += kSBatch;
                    if (i0 >= cend) break;  // only at the run's end (cend < n is a whole double batch)
                    stream_load(wa, rs, i0 + kSBatch);
                    stream_compute(d, wb, i0, n, arow, slot, obuf, d.M, rsr, p);
                    i0 += kSBatch;
                    if (i0 >= cend) break;
                }
                // The next chunk's first batch (wa) is in flight: wait for it
                // before the stores, so that no wait after them is for a load
                // issued before them (a load wait with stores pending drains
                // every store too; the one after these is for the batch
                // issued right behind them and overlaps their completion).
                if (i0 < n) {
#pragma unroll
                    for (int i = 0; i < kSBatch; ++i) asm volatile("" :: "v"(wa[i]));
                }
                // A wave reads back only its own LDS writes.  fp32 / int32
                // outputs with N a multiple of 4: lane (row r0 + lane / 16,
                // strip s0 + lane % 16 / 4, columns 4 (lane % 4) .. +3), 16
                // bytes per lane, four rows of four strips per store (the
                // address unit takes a store in about the same time whatever
                // its width).  Other forms: four strips of one row per store.
                const bool vec_out = !d.y16 && !d.resid && (d.N & 3) == 0 &&
                                     ((reinterpret_cast<uintptr_t>(d.y) | reinterpret_cast<uintptr_t>(d.acc)) & 15) == 0;
                // fp32 y only, payload magnitude 1, output of at most 2 GiB:
                // buffer stores at 32-bit offsets, lanes outside the matrix
                // sent to offset 2^31, past the buffer's range (dropped), so
                // no store needs a branch or a 64-bit address
                const bool fast_y = vec_out && d.y && !d.acc && d.w_mag == 1 && (long long)d.M * d.N <= (1LL << 29);
                if (fast_y) {
                    const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
                        (void*)d.y, 0, (int)((unsigned)d.M * (unsigned)d.N * 4u), 0x00020000);
                    for (int s0 = 0; s0 < p.nbuf; s0 += 4) {
                        const int sb = s0 + ((lane & 15) >> 2);
                        const int col = (w_a + st_flush + sb) * kStripCols + (lane & 3) * 4;
                        for (int r0 = 0; r0 < d.M; r0 += 4) {
                            const int row = r0 + (lane >> 4);
                            const bool ok = sb < p.nbuf && row < d.M && col < d.N;
                            const i32x4 v = *reinterpret_cast<const i32x4*>(
                                obuf + (min(sb, p.nbuf - 1) * d.M + min(row, d.M - 1)) * kStripCols + (lane & 3) * 4);
                            const float sc = xs_l[min(row, d.M - 1)];
                            const unsigned off = ok ? ((unsigned)row * (unsigned)d.N + (unsigned)col) * 4u : 0x80000000u;
                            const f32x4 y = f32x4{(float)v[0] * sc, (float)v[1] * sc, (float)v[2] * sc, (float)v[3] * sc};
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, y), yr, (int)off, 0, 0);
                        }
                    }
                } else if (vec_out) {
                    for (int s0 = 0; s0 < p.nbuf; s0 += 4) {
                        const int sb = s0 + ((lane & 15) >> 2);
                        const int col = (w_a + st_flush + sb) * kStripCols + (lane & 3) * 4;
                        for (int r0 = 0; r0 < d.M; r0 += 4) {
                            const int row = r0 + (lane >> 4);
                            if (sb < p.nbuf && row < d.M && col < d.N) {
                                const i32x4 v = *reinterpret_cast<const i32x4*>(obuf + (sb * d.M + row) * kStripCols +
                                                                                (lane & 3) * 4);
                                const long long o = (long long)row * d.N + col;
                                const float sc = xs_l[row];
                                if (d.acc) *reinterpret_cast<TER_GLOBAL i32x4*>(gptr(d.acc) + o) = v;
                                if (d.y)
                                    *reinterpret_cast<TER_GLOBAL f32x4*>(gptr(d.y) + o) =
                                        f32x4{acc_to_float(v[0], d.w_mag) * sc, acc_to_float(v[1], d.w_mag) * sc,
                                              acc_to_float(v[2], d.w_mag) * sc, acc_to_float(v[3], d.w_mag) * sc};
                            }
                        }
                    }
                } else {
                    for (int s0 = 0; s0 < p.nbuf; s0 += 4) {
                        const int sb = s0 + (lane >> 4);
                        const int col = (w_a + st_flush + sb) * kStripCols + (lane & 15);
                        if (sb < p.nbuf && col < d.N) {
                            const int* ob = obuf + sb * d.M * kStripCols + (lane & 15);
                            for (int row = 0; row < d.M; ++row)
                                emit_out(d, (long long)row * d.N + col, ob[row * kStripCols], xs_l[row]);
                        }
                    }
                }
                st_flush = p.strip;
                p.nbuf = 0;
                if (i0 >= n) break;
            }
        }
        t = seg_end;
        ++di;
    }
}

// Dynamic LDS above the 64 KiB default for every instantiation; once per process.
hipError_t allow_stream_lds() {
    static hipError_t done = [] {
        hipError_t e = hipSuccess;
        const void* fns[] = {reinterpret_cast<const void*>(&gemm_stream_kernel<true, true>),
                             reinterpret_cast<const void*>(&gemm_stream_kernel<true, false>),
                             reinterpret_cast<const void*>(&gemm_stream_kernel<false, true>),
                             reinterpret_cast<const void*>(&gemm_stream_kernel<false, false>)};
        for (const void* f : fns)
            if (e == hipSuccess) e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kGemmStreamLdsMax);
        return e;
    }();
    return done;
}

template <bool kList, bool kVec>
hipError_t launch_stream_t(const GemmDesc& single, const GemmDesc* list, const int32_t* first, long long total, int n_wg,
                           int lds_bytes, hipStream_t st) {
    const hipError_t e = allow_stream_lds();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((gemm_stream_kernel<kList, kVec>), dim3(n_wg), dim3(kSThreads), lds_bytes, st, single, list,
                       first, total, n_wg, lds_bytes);
    return hipGetLastError();
}

template <int MB, int S>
hipError_t launch_mbs(const GemmDesc& single, const GemmDesc* list, const int32_t* first, long long total_blocks, int n_wg,
                      bool vec, hipStream_t st) {
    if (list) {
        if (vec)
            hipLaunchKernelGGL((gemm_t16_kernel<MB, S, true, true>), dim3(n_wg), dim3(kThreads), 0, st, single, list,
                               first, total_blocks, n_wg);
        else
            hipLaunchKernelGGL((gemm_t16_kernel<MB, S, true, false>), dim3(n_wg), dim3(kThreads), 0, st, single, list,
                               first, total_blocks, n_wg);
    } else {
        if (vec)
            hipLaunchKernelGGL((gemm_t16_kernel<MB, S, false, true>), dim3(n_wg), dim3(kThreads), 0, st, single,
                               list, first, total_blocks, n_wg);
        else
            hipLaunchKernelGGL((gemm_t16_kernel<MB, S, false, false>), dim3(n_wg), dim3(kThreads), 0, st, single,
                               list, first, total_blocks, n_wg);
    }
    return hipGetLastError();
}

template <int MB, int S>
int occupancy_mbs() {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemm_t16_kernel<MB, S, true, true>, kThreads, 0) !=
        hipSuccess)
        return 0;
    return n;
}

}  // namespace

// Strips per wave (register blocking: one A operand read from LDS feeds S
// MFMAs; a block of 4 waves covers 64 S columns).  Measured on the BitNet-2B
// sweep: S = 1 at M <= 16 (more workgroups in flight), S = 2 up to M = 64,
// S = 4 at M = 128 (LDS-read bound below that), 1 above (registers).
constexpr int strips_for(int mb) { return mb <= 1 ? 1 : (mb <= 4 ? 2 : (mb <= 8 ? 4 : 1)); }
int gemm_strips_per_wave(int mb) { return strips_for(mb); }

int gemm_max_wg_per_cu(int mb) {
    switch (mb) {
        case 1: return occupancy_mbs<1, strips_for(1)>();
        case 2: return occupancy_mbs<2, strips_for(2)>();
        case 4: return occupancy_mbs<4, strips_for(4)>();
        case 8: return occupancy_mbs<8, strips_for(8)>();
        default: return occupancy_mbs<16, strips_for(16)>();
    }
}

int gemm_stream_max_wg_per_cu(int lds_bytes) {
    if (allow_stream_lds() != hipSuccess) return 0;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemm_stream_kernel<true, true>, kSThreads, lds_bytes) !=
        hipSuccess)
        return 0;
    return n;
}

hipError_t launch_gemm_stream(const GemmDesc& single, const GemmDesc* list_dev, const int32_t* first_dev,
                              long long total_tiles, int n_wg, int lds_bytes, bool vec, hipStream_t st) {
    if (list_dev)
        return vec ? launch_stream_t<true, true>(single, list_dev, first_dev, total_tiles, n_wg, lds_bytes, st)
                   : launch_stream_t<true, false>(single, list_dev, first_dev, total_tiles, n_wg, lds_bytes, st);
    return vec ? launch_stream_t<false, true>(single, list_dev, first_dev, total_tiles, n_wg, lds_bytes, st)
               : launch_stream_t<false, false>(single, list_dev, first_dev, total_tiles, n_wg, lds_bytes, st);
}

int gemm_mb_of(int M) {
    if (M <= 16) return 1;
    if (M <= 32) return 2;
    if (M <= 64) return 4;
    if (M <= 128) return 8;
    return 16;
}

hipError_t launch_gemm_list(const GemmDesc& single, const GemmDesc* list_dev, const int32_t* first_dev,
                            long long total_blocks, int n_wg, int mb, bool vec, hipStream_t st) {
    switch (mb) {
        case 1: return launch_mbs<1, strips_for(1)>(single, list_dev, first_dev, total_blocks, n_wg, vec, st);
        case 2: return launch_mbs<2, strips_for(2)>(single, list_dev, first_dev, total_blocks, n_wg, vec, st);
        case 4: return launch_mbs<4, strips_for(4)>(single, list_dev, first_dev, total_blocks, n_wg, vec, st);
        case 8: return launch_mbs<8, strips_for(8)>(single, list_dev, first_dev, total_blocks, n_wg, vec, st);
        default: return launch_mbs<16, strips_for(16)>(single, list_dev, first_dev, total_blocks, n_wg, vec, st);
    }
}

}  // namespace terhip
