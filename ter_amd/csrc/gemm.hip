// gemm.hip -- M > 1 packed-trit GEMM on gfx950 MFMA (v_mfma_i32_16x16x64_i8).
//
// Replaces the reference's batched kernels (mm_packed_batched,
// cuda/ter_cuda_packed_batched.cu:26-83; mm_bitnet_addonly_batched_k<M>,
// cuda/ter_cuda_addonly_batched.cu:31-124; the wmma s4 mm_int4_tc*).
// Semantics: acc[m][j] = sum_k X[m][k] w[k][j] (exact int32) and
// y[m][j] = float(acc[m][j]) * (x_scale[m] * w_scale)
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
#define TER_GLOBAL __attribute__((address_space(1)))

template <typename T>
__device__ __forceinline__ TER_GLOBAL T* gptr(T* p) {
    return (TER_GLOBAL T*)p;
}

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
        const int soff = uniform((s * d.Ku + u) * kTileBytes);  // scalar offset: no waterfall loop
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            r.w[s][ks] = __builtin_amdgcn_raw_buffer_load_b32(wr, woff + ks * 64, soff, 2 /* nt */);
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
                                                            int n_list, long long total_blocks, int n_wg) {
#pragma clang fp contract(off)
    constexpr int ROWS = MB * 16;
    __shared__ __align__(16) int8_t xl[2][ROWS * kLdRow];
    __shared__ int rsum[ROWS];
    int gi = blockIdx.x;
    if ((n_wg & 7) == 0) gi = (gi & 7) * (n_wg >> 3) + (gi >> 3);  // neighbouring ranges on one XCD
    const long long b_begin = total_blocks * gi / n_wg;
    const long long b_end = total_blocks * (gi + 1) / n_wg;
    if (b_begin >= b_end) return;
    int di = 0;
    if (kList) {
        int lo = 0, hi = n_list - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (list[mid].block0 <= b_begin) lo = mid; else hi = mid - 1;
        }
        di = lo;
    }
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
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int col = (st0 + s) * kStripCols + j;
            if (s < n_act && col < d.N) {
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int row = mb * 16 + g * 4 + e;
                        if (row < d.M) {
                            const int val = C[s][mb][e] - rsum[row];
                            const long long o = (long long)row * d.N + col;
                            if (d.acc) gptr(d.acc)[o] = val;
                            if (d.y) gptr(d.y)[o] = (float)val * (gptr(d.xs)[row] * d.w_scale);
                        }
                    }
                }
            }
        }
        __syncthreads();  // rsum and the X buffers are reused by the next block
    }
}

template <int MB, int S>
hipError_t launch_mbs(const GemmDesc& single, const GemmDesc* list, int n_list, long long total_blocks, int n_wg,
                      bool vec, hipStream_t st) {
    if (list) {
        if (vec)
            hipLaunchKernelGGL((gemm_t16_kernel<MB, S, true, true>), dim3(n_wg), dim3(kThreads), 0, st, single, list,
                               n_list, total_blocks, n_wg);
        else
            hipLaunchKernelGGL((gemm_t16_kernel<MB, S, true, false>), dim3(n_wg), dim3(kThreads), 0, st, single, list,
                               n_list, total_blocks, n_wg);
    } else {
        if (vec)
            hipLaunchKernelGGL((gemm_t16_kernel<MB, S, false, true>), dim3(n_wg), dim3(kThreads), 0, st, single,
                               list, n_list, total_blocks, n_wg);
        else
            hipLaunchKernelGGL((gemm_t16_kernel<MB, S, false, false>), dim3(n_wg), dim3(kThreads), 0, st, single,
                               list, n_list, total_blocks, n_wg);
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
int gemm_strips_per_wave(int mb) { return mb <= 1 ? 1 : (mb <= 4 ? 2 : (mb <= 8 ? 4 : 1)); }

int gemm_max_wg_per_cu(int mb) {
    const int s = gemm_strips_per_wave(mb);
#define TER_OCC(MBV)                                              \
    case MBV:                                                     \
        return s == 1 ? occupancy_mbs<MBV, 1>() : (s == 2 ? occupancy_mbs<MBV, 2>() : occupancy_mbs<MBV, 4>());
    switch (mb) {
        TER_OCC(1)
        TER_OCC(2)
        TER_OCC(4)
        TER_OCC(8)
        default:
            return s == 1 ? occupancy_mbs<16, 1>() : (s == 2 ? occupancy_mbs<16, 2>() : occupancy_mbs<16, 4>());
    }
#undef TER_OCC
}

int gemm_mb_of(int M) {
    if (M <= 16) return 1;
    if (M <= 32) return 2;
    if (M <= 64) return 4;
    if (M <= 128) return 8;
    return 16;
}

hipError_t launch_gemm_list(const GemmDesc& single, const GemmDesc* list_dev, int n_list, long long total_blocks,
                            int n_wg, int mb, bool vec, hipStream_t st) {
    const int s = gemm_strips_per_wave(mb);
#define TER_LAUNCH(MBV)                                                                                         \
    case MBV:                                                                                                   \
        if (s == 1) return launch_mbs<MBV, 1>(single, list_dev, n_list, total_blocks, n_wg, vec, st);           \
        if (s == 2) return launch_mbs<MBV, 2>(single, list_dev, n_list, total_blocks, n_wg, vec, st);           \
        return launch_mbs<MBV, 4>(single, list_dev, n_list, total_blocks, n_wg, vec, st);
    switch (mb) {
        TER_LAUNCH(1)
        TER_LAUNCH(2)
        TER_LAUNCH(4)
        TER_LAUNCH(8)
        default:
            if (s == 1) return launch_mbs<16, 1>(single, list_dev, n_list, total_blocks, n_wg, vec, st);
            if (s == 2) return launch_mbs<16, 2>(single, list_dev, n_list, total_blocks, n_wg, vec, st);
            return launch_mbs<16, 4>(single, list_dev, n_list, total_blocks, n_wg, vec, st);
    }
#undef TER_LAUNCH
}

}  // namespace terhip
