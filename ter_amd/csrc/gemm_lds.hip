// gemm_lds.hip -- batched packed-trit GEMM for M <= 128 on gfx950 MFMA,
// fed through an LDS ring by direct global->LDS loads.
//
// Same semantics as gemm.hip (cuda/ter_cuda_addonly_batched.cu:117-123):
// acc[m][j] = sum_k X[m][k] w[k][j] in exact int32, y = float(mag * acc) * (xs[m] * w_scale).
//
// Work.  A block is BS consecutive column strips of one GEMM (all M rows,
// all K).  The host deals the blocks of a launch out to the workgroups by
// list scheduling (upload_lds_plan in abi.hip: largest estimated cost first,
// each to the workgroup free first; the pieces of a GEMM cut into 128-row
// pieces side by side, so they read the same weights at the same time), and
// stores each workgroup's blocks as one range of the block list in the order
// it runs them; workgroups with neighbouring ranges sit on one XCD.  A single
// GEMM (no list) splits its blocks into equal contiguous ranges.  A
// workgroup (8 compute waves) walks its blocks unit by unit: for unit u of
// block b it needs X[0:M, u] (M x 256 int8) and the BS weight tiles
// (strip, u) of the block, 1 KiB each.
//
// Pipeline.  NST stages of LDS, each holding one unit's X rows and weight
// tiles, are filled by buffer_load_dwordx4 ... lds (64 lanes x 16 bytes = one
// 1 KiB LDS run per instruction; no registers involved) NST - 1 units ahead
// of the MFMAs.  Per unit: the issuing waves wait for their loads of the unit
// (explicit vmcnt), barrier (every load landed, and every compute wave is
// done reading the stage about to be refilled), the issuing waves issue the
// loads of unit + NST - 1, the compute waves run the MFMAs.  A wave's loads
// complete in issue order, so waiting until no more operations are
// outstanding than the younger stages' loads guarantees the stage has landed.
// That holds with the epilogue's stores in flight too (stores may complete
// out of order with respect to loads, but a wait that leaves only the younger
// loads outstanding waits for them as well), so a block's epilogue needs no
// drain.  Four producer waves (PW > 0) issue all the loads and the 8 compute
// waves issue none: the memory pipeline accepts only so many loads in
// flight, and a wave that stalls at its loads holds back nothing behind it
// in issue order (measured at M = 32: 154 -> 145 us per C4 launch).  With
// PW = 0 the compute waves issue the loads themselves after the barrier.
//
// Operands.  X rows sit in LDS as 256-byte rows whose 16-byte chunks are
// XOR-swizzled by the row's low 4 bits (chunk c of row r at position
// c ^ (r & 15)), so the 16 rows an MFMA A operand reads hit distinct banks.
// The wave grid is RS row groups x (CW / RS) strip groups; a wave holds
// MBW x S accumulators (MBW row blocks of 16 x S strips).  Per 64-row slab a
// wave reads MBW A operands (ds_read_b128) and S weight dwords (ds_read_b32,
// lane = column j + 16 * k-group g, one dword = 16 trits of column j) and
// issues v_mfma_i32_16x16x64_i8.  From 3 row blocks per wave on, each 2-bit
// code u = w + 1 becomes the signed int8 w with one v_perm_b32 per 4 trits
// (a byte table {-1, 0, +1, 0} indexed by u) and needs no correction.  Up to
// 2 row blocks (C::UC) the MFMAs take the unsigned codes u themselves (7 bit
// operations per 16 trits instead of 11), and the epilogue subtracts the row
// sums of X (sum_k x u = sum_k x w + sum_k x, and the padding rows past K,
// which hold u = 1, cancel the same way): formed by the producer waves from
// the X runs they load (C::PRS), or without producers by one more MFMA per A
// operand against all-ones.  The A operands are read a few steps ahead of
// their MFMAs.
//
// Epilogue.  The common output form (fp32 y only, payload magnitude 1, N a
// multiple of 4) transposes each accumulator in quads of lanes (DPP), pairs
// the two strips of a wave with v_permlane16_swap so that every store covers
// whole 128-byte lines (8 rows x 2 strips), and stores them nontemporally
// through a buffer resource at 32-bit offsets (lanes outside the matrix
// store past its range, which the hardware drops: no branch).  Other fp32 /
// int32 outputs with N a multiple of 4 store 4 consecutive columns of one
// row per lane; fp16 and residual outputs go element by element.
#include <type_traits>

#include "common.h"

namespace terhip {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
#define TER_LDS __attribute__((address_space(3)))

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

constexpr int kLWaves = 8;

// PW producer waves (0: the compute waves issue the loads themselves), CW
// compute waves.
template <int MBW_, int S_, int RS_, int NST_, int PW_ = 0, int FS_ = 0, int CW_ = kLWaves>
struct LCfg {
    static constexpr int MBW = MBW_, S = S_, RS = RS_, NST = NST_, PW = PW_, CW = CW_;
    // FS: stage hand-over through LDS counters instead of a workgroup
    // barrier per unit (needs producer waves)
    static constexpr bool FS = FS_ != 0 && PW > 0;
    static constexpr int THREADS = 64 * (CW + PW);
    static constexpr int IW = PW > 0 ? PW : CW;       // waves that issue the loads
    static constexpr int MB = RS * MBW;               // row blocks of 16
    static constexpr int SG = CW / RS;                // strip groups
    static constexpr int BS = SG * S;                 // strips per block
    static constexpr int XB = MB * 16 * kUnitK;       // X bytes per stage
    static constexpr int STB = XB + BS * kTileBytes;  // bytes per stage
    static constexpr int XSO = NST * STB;             // row-scale slots: NST x 1 KiB
    static constexpr int FLO = XSO + NST * 1024;      // stage counters: ready[NST], freed[NST]
    static constexpr int RSO = FLO + 64;              // (PRS) row sums of X per block: NST slots x MB*16 ints
    static constexpr int LDS = RSO + NST * MB * 16 * 4;
    static constexpr int XI = XB / 1024;              // 1 KiB load runs of X per stage
    static constexpr int NI = XI + BS;                // load runs per stage, run q issued by issuer q % IW
    static constexpr int NIW = NI / IW;               // runs of issuers >= NR ...
    static constexpr int NR = NI % IW;                // ... and issuers < NR issue one more
    // Weight tiles transposed by 16-byte chunks in LDS: conflict-free operand
    // reads, but each quarter-wave's load spans four 256-byte runs instead of
    // one.  Measured on the BitNet-2B sweep: 2.8% faster at M = 128 (8 row
    // blocks, bound by LDS reads), 2.7% slower at M = 16 (bound by the loads).
    // Without it the tiles keep their runs with the row groups XOR-swizzled
    // (see issue_run), also conflict-free; from 4 row blocks on the transposed
    // layout is still 1-3% faster (C4 M = 64 162.4 against 167.4 us, M = 128
    // 259.3 against 262.4, M = 256 488.8 against 498.1).
#ifndef TER_LDS_TW_MB
#define TER_LDS_TW_MB 4
#endif
    static constexpr bool TW = MBW >= TER_LDS_TW_MB;
    // Up to 2 row blocks the weights enter the MFMAs as their unsigned codes
    // u = w + 1 (7 bit operations per 16 trits instead of 11 for the signed
    // table lookup) and the row sums of X are subtracted in the epilogue:
    // there each weight dword feeds only MBW MFMAs, and its unpacking bounds
    // the compute waves.  (At 4 and 8 row blocks, with the producers' row
    // sums: M = 128 272-273 against 260-261 us, M = 256 515-520 against 491
    // us; the producers' eight X runs per unit delay the barrier.)
#ifndef TER_LDS_UC_MB
#define TER_LDS_UC_MB 2
#endif
    static constexpr bool UC = MBW <= TER_LDS_UC_MB;
    // With producer waves, the producers form those row sums from the X rows
    // they load (v_dot4 against ones) and hand them over in LDS once per
    // block; the compute waves then issue no row-sum MFMA (at 2 row blocks, 8
    // of a wave's 40 MFMAs per stage; without producers they do).  Measured, alternating builds on one
    // box: M = 32 119.7-121.1 -> 117.8-118.3 us, M = 16 95.8-96.2 -> 95.3-95.5
    // us, provided only a block's last unit adds before its ready count.
    static constexpr bool PRS = UC && PW > 0;
    static_assert(NST >= 2 && NST <= 8, "stage count");
    static_assert(S % 2 == 0, "the fp32 epilogue stores strips in pairs");
    static_assert(LDS <= kLdsMax, "LDS budget");
};

// The configuration per row-block count (M <= 16, 32, 64, 128) as
// (MBW, S, RS, NST, PW), measured on the BitNet-2B sweep (C4): every wave
// covers all rows (RS = 1) and four producer waves issue the loads.  At 64
// and 128 rows the blocks are 16 strips (2 per wave): the compute waves'
// accumulators then fit 168 VGPRs, which leaves room for the producers, and
// the smaller stages a third ring stage (M = 128: 325 -> 284 us against
// 32-strip blocks of 8 compute waves that issued their own loads; M = 64:
// 200 -> 180 us); 32-strip blocks at M = 32 (2 per wave: 142 against 138 us);
// four stages at M = 16 (124 -> 120 us).  FS (the sixth field): at M = 32
// the stages change hands through LDS counters instead of a barrier per unit
// (123.2 -> 117.4 us); at 8, 16, 64, 128 and 256 rows the barrier is as fast
// or 1-2% faster.  (Each can be overridden at build time.)
#ifndef TER_LDS_PW
#define TER_LDS_PW 4
#endif
#ifndef TER_LDS_CFG1
#define TER_LDS_CFG1 1, 2, 1, 4, TER_LDS_PW
#endif
#ifndef TER_LDS_CFG2
#define TER_LDS_CFG2 2, 4, 1, 3, TER_LDS_PW, 1
#endif
using Cfg1 = LCfg<TER_LDS_CFG1>;
using Cfg2 = LCfg<TER_LDS_CFG2>;
#ifndef TER_LDS_CFG4
#define TER_LDS_CFG4 4, 2, 1, 3, 4
#endif
#ifndef TER_LDS_CFG8
#define TER_LDS_CFG8 8, 2, 1, 3, 4
#endif
using Cfg4 = LCfg<TER_LDS_CFG4>;
using Cfg8 = LCfg<TER_LDS_CFG8>;

// s_waitcnt immediate (gfx9 family): vmcnt(n), expcnt and lgkmcnt not waited on.
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Barrier that orders memory for the compiler but adds no wait of its own
// (the waits are explicit above it).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Stage hand-over without a workgroup barrier (PW > 0).  Two monotonic
// counters per ring stage in LDS: ready[s] counts the producers' "my loads
// of the unit in stage s have landed" signals (PW per use of the stage),
// freed[s] the compute waves' "done reading stage s" signals (C::CW per
// use).  A compute wave waits for ready of its next unit only; a producer
// waits for freed of the stage it is about to refill only.  So no wave
// waits for the slowest of the others at every stage, and a stage is freed
// as soon as its last operand is read, before the MFMAs on it finish.  LDS
// operations of one wave execute in order, and a producer signals only
// after its direct-to-LDS loads have landed (vmcnt), so a wave that sees a
// count has the data (or the free slot) it stands for.  Every wait gives up
// after kSpinCap polls (the kernel then ends with wrong results instead of
// hanging; the parity tests would show it).
//
// The counter accesses are written as inline ds instructions: for a plain
// LDS access the compiler first waits for every direct-to-LDS load in
// flight (it cannot tell that the counters do not alias the ring), which in
// a producer would drain the whole pipeline at every signal.
constexpr int kSpinCap = 1 << 18;

__device__ __forceinline__ unsigned lds_off(unsigned char* p) {
    return (unsigned)reinterpret_cast<uintptr_t>((TER_LDS unsigned char*)p);
}

__device__ __forceinline__ void spin_ge(unsigned char* lds_byte, unsigned target) {
    const unsigned a = lds_off(lds_byte);
    for (int n = 0; n < kSpinCap; ++n) {
        unsigned v;
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
        if ((unsigned)__builtin_amdgcn_readfirstlane((int)v) >= target) break;
        __builtin_amdgcn_s_sleep(1);
    }
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ void signal_one(unsigned char* lds_byte, int lane) {
    const unsigned a = lds_off(lds_byte);
    asm volatile("" ::: "memory");
    if (lane == 0) asm volatile("ds_add_u32 %0, %1" : : "v"(a), "v"(1u) : "memory");
}

// (PRS) A producer's LDS accesses for the row sums, inline for the same
// reason as the counters: 16 bytes of a landed X run, and a row sum.
__device__ __forceinline__ u32x4_t lds_read16(unsigned char* p) {
    u32x4_t v;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_off(p)) : "memory");
    return v;
}

__device__ __forceinline__ void lds_write4(unsigned char* p, int v) {
    asm volatile("ds_write_b32 %0, %1" : : "v"(lds_off(p)), "v"(v) : "memory");
}

// Sum over each row of 16 lanes (every lane gets its row's total): xor 1 and
// 2 within quads, then the half-row and row mirrors (DPP, no LDS).
__device__ __forceinline__ int row_total16(int v) {
    v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    v += __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false);  // row_half_mirror
    v += __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false);  // row_mirror
    return v;
}

// (PRS) The producer's share of a unit's row sums: its X runs q = issuer +
// IW r (rows 4 q .. 4 q + 3, lane l: row 4 q + l / 16, one 16-byte chunk) of
// the landed stage, added into rsp[r]; at the block's last unit each row's
// total goes to the block's slot (row 4 q + l / 16 by lane 16 (l / 16)).
template <class C>
__device__ __forceinline__ void producer_row_sums(unsigned char* stage, unsigned char* slot, int issuer, int lane,
                                                  bool last, int (&rsp)[C::XI / C::IW + 1]) {
#pragma unroll
    for (int r = 0; r < C::XI / C::IW + 1; ++r) {
        const int q = issuer + C::IW * r;  // wave-uniform
        if (q < C::XI) {
            const u32x4_t c = lds_read16(stage + q * 1024 + lane * 16);
            int v = rsp[r];
            v = __builtin_amdgcn_sdot4((int)c.x, 0x01010101, v, false);
            v = __builtin_amdgcn_sdot4((int)c.y, 0x01010101, v, false);
            v = __builtin_amdgcn_sdot4((int)c.z, 0x01010101, v, false);
            v = __builtin_amdgcn_sdot4((int)c.w, 0x01010101, v, false);
            rsp[r] = v;
            if (last) {
                const int t = row_total16(v);
                if ((lane & 15) == 0) lds_write4(slot + (4 * q + (lane >> 4)) * 4, t);
                rsp[r] = 0;
            }
        }
    }
}

// Wait until this wave's loads of the unit `behind` stages older than the
// newest issued one have landed: `behind` = stages issued after it (0..NST-2),
// each holding N of this wave's loads.
template <class C, int N, int B = C::NST - 2>
__device__ __forceinline__ void wait_stage_n(int behind) {
    if constexpr (B == 0) {
        wait_vm<0>();
    } else {
        if (behind >= B)
            wait_vm<B * N>();
        else
            wait_stage_n<C, N, B - 1>(behind);
    }
}

template <class C>
__device__ __forceinline__ void wait_stage(int behind, int issuer) {
    if (C::NR != 0 && issuer < C::NR)
        wait_stage_n<C, C::NIW + 1>(behind);
    else
        wait_stage_n<C, C::NIW>(behind);
}

// Load runs an issuing wave issues per stage (at most; run q of the stage is
// issued by issuer q % IW).
template <class C>
constexpr int runs_per_wave() { return C::NIW + (C::NR != 0); }

// Issue the issuing wave's r-th load run of unit u of the block starting at strip
// st0 into `stage`.  xr covers X (M * ldx bytes: rows >= M read zeros); wr
// covers the block's strips (strips past the matrix read zeros).
template <class C>
__device__ __forceinline__ void issue_run(int r, int ldx, int Ku, int u, unsigned char* stage,
                                          __amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t wr, int issuer, int lane) {
    const int q = issuer + C::IW * r;  // wave-uniform
    if (C::NR != 0 && q >= C::NI) return;
    if (q < C::XI) {
        // rows 4q .. 4q+3: lane -> row 4q + lane / 16, stored chunk lane % 16
        const int row = 4 * q + (lane >> 4);
        const int chunk = (lane & 15) ^ (row & 15);
        // (resource, LDS run, bytes per lane, vector offset, scalar offset, immediate offset, cache policy)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (TER_LDS void*)(stage + q * 1024), 16,
                                                 row * ldx + u * kUnitK + chunk * 16, 0, 0, 0);
    } else {
        // tile (strip t of the block, unit u); its 16-byte chunk (column quad
        // cq, row group rq) at tile offset cq * 256 + rq * 16 lands at LDS
        // chunk 4 rq + cq with C::TW, else at chunk 16 cq + (rq ^ 4 cq) (each
        // quarter-wave still loads one contiguous 256-byte run; see
        // compute_stage)
        const int t = q - C::XI;
        const int src = C::TW ? (lane & 3) * 256 + (lane >> 2) * 16
                              : (lane >> 4) * 256 + ((lane & 15) ^ (4 * (lane >> 4))) * 16;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (TER_LDS void*)(stage + C::XB + t * 1024), 16,
                                                 (t * Ku + u) * kTileBytes + src, 0, 0, 2 /* nt */);
    }
}

// Signed int8 weights of 16 trits (one T16 dword) in MFMA B operand order:
// byte b of word f is the trit of row 4 f + b; u = w + 1 -> w by table lookup.
__device__ __forceinline__ i32x4 unpack_signed(unsigned dw) {
    const unsigned kM = 0x03030303u, kT = 0x000100FFu;  // bytes: u=0 -> -1, 1 -> 0, 2 -> +1, 3 -> 0
    return i32x4{(int)__builtin_amdgcn_perm(0u, kT, dw & kM), (int)__builtin_amdgcn_perm(0u, kT, (dw >> 2) & kM),
                 (int)__builtin_amdgcn_perm(0u, kT, (dw >> 4) & kM), (int)__builtin_amdgcn_perm(0u, kT, (dw >> 6) & kM)};
}

// The 16 trits of one T16 dword as their unsigned codes u = w + 1 in MFMA B
// operand order (byte b of word f: row 4 f + b); T16 fields hold 0, 1 or 2.
__device__ __forceinline__ i32x4 unpack_u(unsigned dw) {
    const unsigned kM = 0x03030303u;
    return i32x4{(int)(dw & kM), (int)((dw >> 2) & kM), (int)((dw >> 4) & kM), (int)((dw >> 6) & kM)};
}

// 4 x 4 transpose within each quad of lanes: lane 4 a + b returns element c
// = element b of lane 4 a + c (two exchange rounds, partner lane b ^ 1 then
// b ^ 2, each taking the elements whose index bit differs from the lane's).
__device__ __forceinline__ i32x4 quad_transpose(i32x4 v, int lane) {
    const bool o1 = lane & 1, o2 = lane & 2;
    const int p0 = __builtin_amdgcn_mov_dpp(v[1], 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    const int p1 = __builtin_amdgcn_mov_dpp(v[0], 0xB1, 0xF, 0xF, false);
    const int p2 = __builtin_amdgcn_mov_dpp(v[3], 0xB1, 0xF, 0xF, false);
    const int p3 = __builtin_amdgcn_mov_dpp(v[2], 0xB1, 0xF, 0xF, false);
    const int a0 = o1 ? p0 : v[0], a1 = o1 ? v[1] : p1, a2 = o1 ? p2 : v[2], a3 = o1 ? v[3] : p3;
    const int q0 = __builtin_amdgcn_mov_dpp(a2, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    const int q1 = __builtin_amdgcn_mov_dpp(a3, 0x4E, 0xF, 0xF, false);
    const int q2 = __builtin_amdgcn_mov_dpp(a0, 0x4E, 0xF, 0xF, false);
    const int q3 = __builtin_amdgcn_mov_dpp(a1, 0x4E, 0xF, 0xF, false);
    return i32x4{o2 ? q0 : a0, o2 ? q1 : a1, o2 ? a2 : q2, o2 ? a3 : q3};
}

// A operands read this many (slab, row block) steps ahead of their MFMAs.
#ifndef TER_LDS_APF
#define TER_LDS_APF 3
#endif
constexpr int kAPrefetch = TER_LDS_APF;

// One stage: 4 slabs of 64 rows x MBW row blocks = 4 MBW steps, each one A
// operand (ds_read_b128) feeding S MFMAs.  The stage's weight dwords (4 x S
// ds_read_b32) are read first; then step t's MFMAs run while the A operand of
// step t + kAPrefetch is in flight (a wave's LDS reads return in order, so
// the wait before step t's MFMAs leaves the younger reads outstanding).  The
// scheduling fences keep the compiler from pulling the reads down next to
// their MFMAs, which exposed the LDS latency on every step.
template <class C>
__device__ __forceinline__ void compute_stage(const unsigned char* stage, int rg, int sg, int lane,
                                              i32x4 (&acc)[C::S][C::MBW], i32x4 (&rsum)[C::MBW],
                                              unsigned char* freed) {
    const int j = lane & 15, g = lane >> 4;
    // (two steps ahead at 8 row blocks, whose accumulators leave no room for a third)
    constexpr int KS = 4, T = KS * C::MBW, P = C::MBW >= 8 ? 2 : (kAPrefetch < T ? kAPrefetch : T);
    unsigned dw[KS][C::S];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int s = 0; s < C::S; ++s) {
            // column j, rows (4 ks + g) * 16 .. +15: tile offset (j >> 2) * 256 +
            // (4 ks + g) * 16 + (j & 3) * 4.  With C::TW the load placed it at
            // ks * 256 + lane * 4: the 64 lanes read 256 contiguous bytes.
            // Otherwise the row groups of column quad cq sit XOR-swizzled by
            // 4 cq, so the four quads' dwords of one row group fall on
            // different banks: the 64 lanes hit 64 banks, where in tile order
            // four lanes shared each (C4 M = 16 99.0 -> 95.5 us, M = 32
            // 120.0 -> 118.3 us; M = 8 unchanged).
            const int off = C::TW ? ks * 256 + lane * 4
                                  : (j >> 2) * 256 + ((4 * ks + g) ^ (4 * (j >> 2))) * 16 + (j & 3) * 4;
            dw[ks][s] = *reinterpret_cast<const unsigned*>(stage + C::XB + (sg * C::S + s) * kTileBytes + off);
        }
    auto a_at = [&](int t) {
        const int ks = t / C::MBW, mb = t % C::MBW;
        const int row = (rg * C::MBW + mb) * 16 + j;  // row % 16 == j
        return *reinterpret_cast<const i32x4*>(stage + row * kUnitK + (((ks * 4 + g) ^ j) * 16));
    };
    i32x4 A[P];
#pragma unroll
    for (int t = 0; t < P; ++t) A[t] = a_at(t);
    // the stage's last operand read issued: hand the stage back (freed is
    // null where the caller signals later)
    if (P >= T && freed) signal_one(freed, lane);
    i32x4 B[C::S];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int ks = t / C::MBW, mb = t % C::MBW;
        if (mb == 0) {
#pragma unroll
            for (int s = 0; s < C::S; ++s) B[s] = C::UC ? unpack_u(dw[ks][s]) : unpack_signed(dw[ks][s]);
        }
        const i32x4 a = A[t % P];
        if (t + P < T) A[t % P] = a_at(t + P);
        if (t + P == T - 1 && freed) signal_one(freed, lane);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < C::S; ++s)
            acc[s][mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, B[s], acc[s][mb], 0, 0, 0);
        if constexpr (C::UC && !C::PRS) {
            const i32x4 ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
            rsum[mb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, ones, rsum[mb], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

struct BlockRef {
    GemmDesc d;
    int st0;
};

template <bool kList>
__device__ __forceinline__ BlockRef block_at(const GemmDesc& single, const GemmDesc* list,
                                             const GemmBlock* blocks, int b, int bs) {
    BlockRef r;
    if (kList) {
        const GemmBlock gb = blocks[b];
        r.d = list[gb.desc];
        r.st0 = gb.strip0;
    } else {
        r.d = single;
        r.st0 = b * bs;
    }
    return r;
}

template <class C, bool kList>
__global__ __launch_bounds__(C::THREADS) void gemm_lds_kernel(GemmDesc single, const GemmDesc* __restrict__ list,
                                                             const GemmBlock* __restrict__ blocks,
                                                             const int32_t* __restrict__ ranges, int n_blocks,
                                                             int n_wg) {
#pragma clang fp contract(off)
    extern __shared__ __align__(1024) unsigned char lds[];
    int gi = blockIdx.x;
    if ((n_wg & 7) == 0) gi = (gi & 7) * (n_wg >> 3) + (gi >> 3);  // neighbouring ranges on one XCD
    int b_lo, b_hi;
    if (kList) {
        b_lo = ranges[gi];
        b_hi = ranges[gi + 1];
    } else {
        b_lo = (int)((long long)n_blocks * gi / n_wg);
        b_hi = (int)((long long)n_blocks * (gi + 1) / n_wg);
    }
    if (b_lo >= b_hi) return;
    const int lane = threadIdx.x & 63;
    const int wave = uniform(threadIdx.x >> 6);
    const bool producer = C::PW > 0 && wave >= C::CW;  // wave-uniform
    const int issuer = C::PW > 0 ? wave - C::CW : wave;  // index among the issuing waves
    const int rg = wave / C::SG, sg = wave % C::SG;
    const int j = lane & 15, g = lane >> 4;

    // issue side: the next unit to load
    int ib = b_lo, iu = 0, n_issued = 0, i_stage = 0;
    BlockRef bi = block_at<kList>(single, list, blocks, ib, C::BS);
    auto rsrc_x = [](const GemmDesc& d) {
        return __builtin_amdgcn_make_buffer_rsrc((void*)d.x, 0, d.M * d.ldx, 0x00020000);
    };
    auto rsrc_w = [](const BlockRef& r) {
        const int ns = min(C::BS, r.d.n_strips - r.st0);
        return __builtin_amdgcn_make_buffer_rsrc((void*)(r.d.w + (long long)r.st0 * r.d.Ku * kTileBytes), 0,
                                                 ns * r.d.Ku * kTileBytes, 0x00020000);
    };
    __amdgpu_buffer_rsrc_t xr = rsrc_x(bi.d), wr = rsrc_w(bi);
    // Block ib's row scales go to LDS slot ib % NST with its first unit
    // (issuer 0, one extra load: an extra operation only makes the stage waits
    // stricter).  The issue side runs at most NST - 1 units ahead, so a slot
    // is refilled only after the block that used it has finished.
    auto issue_scales = [&]() {
        if (iu == 0 && issuer == 0) {
            const __amdgpu_buffer_rsrc_t sr =
                __builtin_amdgcn_make_buffer_rsrc((void*)bi.d.xs, 0, bi.d.M * 4, 0x00020000);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (TER_LDS void*)(lds + C::XSO + (ib % C::NST) * 1024), 16,
                                                     lane * 16, 0, 0, 0);
        }
    };
    // this wave's loads of the next stage, then advance to the stage after it
    auto issue_next = [&]() {
        issue_scales();
#pragma unroll
        for (int r = 0; r < runs_per_wave<C>(); ++r)
            issue_run<C>(r, bi.d.ldx, bi.d.Ku, iu, lds + i_stage * C::STB, xr, wr, issuer, lane);
        ++n_issued;
        i_stage = i_stage + 1 == C::NST ? 0 : i_stage + 1;
        if (++iu == bi.d.Ku) {
            iu = 0;
            if (++ib < b_hi) {
                bi = block_at<kList>(single, list, blocks, ib, C::BS);
                xr = rsrc_x(bi.d);
                wr = rsrc_w(bi);
            }
        }
    };
    unsigned char* const ready = lds + C::FLO;             // ready[NST]
    unsigned char* const freed = lds + C::FLO + 4 * C::NST;  // freed[NST]
    if (C::FS) {
        if (threadIdx.x < 2 * C::NST) reinterpret_cast<unsigned*>(ready)[threadIdx.x] = 0u;
        __syncthreads();
    }
    if (C::PW == 0 || producer) {
#pragma unroll
        for (int p = 0; p < C::NST - 1; ++p)
            if (ib < b_hi) issue_next();
    }
    if (C::FS && producer) {
        // Producer waves, unit j: wait for their loads of unit j (vmcnt) and
        // signal it ready; then refill the stage unit j - 1 used with unit
        // j + NST - 1 once every compute wave has freed it.  A producer that
        // stalls at its loads (the memory pipeline accepts only so many in
        // flight) holds back no MFMA; the compute waves wait only when the
        // data is late.
        int cb = b_lo, cu = 0, j = 0, js = 0, cku = block_at<kList>(single, list, blocks, cb, C::BS).d.Ku;
        int rsp[C::XI / C::IW + 1] = {};
        while (true) {
            wait_stage<C>(n_issued - j - 1, issuer);
            // (the block's row sums written before its last unit's ready count,
            // which the epilogue waits behind; the other units' added after
            // their count, off the compute waves' path)
            const bool last_u = cu + 1 == cku;
            if constexpr (C::PRS)
                if (last_u)
                    producer_row_sums<C>(lds + js * C::STB, lds + C::RSO + (cb % C::NST) * C::MB * 64, issuer, lane,
                                         true, rsp);
            signal_one(ready + 4 * js, lane);
            if constexpr (C::PRS)
                if (!last_u) producer_row_sums<C>(lds + js * C::STB, nullptr, issuer, lane, false, rsp);
            if (ib < b_hi) {
                if (j >= 1) {
                    const int jp = j - 1, sp = js == 0 ? C::NST - 1 : js - 1;
                    spin_ge(freed + 4 * sp, (unsigned)(C::CW * (jp / C::NST + 1)));
                }
                issue_next();
            }
            ++j;
            js = js + 1 == C::NST ? 0 : js + 1;
            if (++cu == cku) {
                if (++cb >= b_hi) break;
                cku = block_at<kList>(single, list, blocks, cb, C::BS).d.Ku;
                cu = 0;
            }
        }
        return;
    }
    if (producer) {
        // Producer waves with a workgroup barrier per unit: wait for their
        // loads of unit it, meet the compute waves at the unit's barrier, then
        // issue the unit that refills the stage the compute waves have just
        // left.  Same unit count and barrier count as the compute waves.
        int cb = b_lo, cu = 0, it = 0, cku = block_at<kList>(single, list, blocks, cb, C::BS).d.Ku;
        int rsp[C::XI / C::IW + 1] = {};
        while (true) {
            wait_stage<C>(n_issued - it - 1, issuer);
            if constexpr (C::PRS) {
                producer_row_sums<C>(lds + (it % C::NST) * C::STB, lds + C::RSO + (cb % C::NST) * C::MB * 64, issuer,
                                     lane, cu + 1 == cku, rsp);
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the row sums written before the barrier
            }
            lds_barrier();
            if (ib < b_hi) issue_next();
            ++it;
            if (++cu == cku) {
                if (++cb >= b_hi) break;
                cku = block_at<kList>(single, list, blocks, cb, C::BS).d.Ku;
                cu = 0;
            }
        }
        return;
    }

    // compute side
    int cb = b_lo, cu = 0, it = 0, c_stage = 0;
    BlockRef bc = block_at<kList>(single, list, blocks, cb, C::BS);
    i32x4 acc[C::S][C::MBW];
    i32x4 rsum[C::MBW];  // row sums of X (C::UC only)
#pragma unroll
    for (int s = 0; s < C::S; ++s)
#pragma unroll
        for (int mb = 0; mb < C::MBW; ++mb) acc[s][mb] = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int mb = 0; mb < C::MBW; ++mb) rsum[mb] = i32x4{0, 0, 0, 0};
    while (true) {
        const bool last_unit = cu + 1 == bc.d.Ku;
        if constexpr (C::FS) {
            spin_ge(ready + 4 * c_stage, (unsigned)(C::PW * (it / C::NST + 1)));
            // the block's last unit is freed after its epilogue has read the
            // row scales (the slot they sit in is refilled NST blocks on)
            compute_stage<C>(lds + c_stage * C::STB, rg, sg, lane, acc, rsum,
                             last_unit ? nullptr : freed + 4 * c_stage);
        } else {
            if (C::PW == 0) wait_stage<C>(n_issued - it - 1, issuer);
            lds_barrier();
            if (C::PW == 0 && ib < b_hi) issue_next();
            compute_stage<C>(lds + c_stage * C::STB, rg, sg, lane, acc, rsum, nullptr);
        }
        const int done_stage = c_stage;
        ++it;
        c_stage = c_stage + 1 == C::NST ? 0 : c_stage + 1;
        if (++cu == bc.d.Ku) {
            // epilogue of block cb.  The output fields through an opaque copy:
            // with one GEMM they are loop-invariant, and the compiler would
            // otherwise hoist every row's output addresses and checks out of
            // the loop (at 8 row blocks, 136 VGPRs spilled to scratch)
            if constexpr (C::UC) {
                // sum_k x u = sum_k x w + sum_k x (padding rows hold u = 1 and
                // cancel too); the row sums are the same in every column
                if constexpr (C::PRS) {
                    // the producers' sums of this block (slot cb % NST): lane (j, g)
                    // holds rows 4 g .. 4 g + 3 of each row block
                    const int* rs = reinterpret_cast<const int*>(lds + C::RSO + (cb % C::NST) * C::MB * 64);
#pragma unroll
                    for (int mb = 0; mb < C::MBW; ++mb)
                        rsum[mb] = *reinterpret_cast<const i32x4*>(rs + (rg * C::MBW + mb) * 16 + 4 * g);
                }
#pragma unroll
                for (int s = 0; s < C::S; ++s)
#pragma unroll
                    for (int mb = 0; mb < C::MBW; ++mb) acc[s][mb] -= rsum[mb];
#pragma unroll
                for (int mb = 0; mb < C::MBW; ++mb) rsum[mb] = i32x4{0, 0, 0, 0};
            }
            GemmDesc d = bc.d;
            asm volatile("" : "+s"(d.N), "+s"(d.M), "+s"(d.y), "+s"(d.acc), "+s"(d.y16), "+s"(d.resid),
                         "+s"(d.w_scale), "+s"(d.w_mag));
            const float* xs_l = reinterpret_cast<const float*>(lds + C::XSO + (cb % C::NST) * 1024);
            // fp32 / int32 outputs with N a multiple of 4 go out 16 bytes per
            // lane: the address unit takes a store in about the same time
            // whatever its width (4 lanes per cycle), and dword stores of a
            // block's outputs cost more of it than the block's loads.
            const bool vec_out = !d.y16 && !d.resid && (d.N & 3) == 0 &&
                                 ((reinterpret_cast<uintptr_t>(d.y) | reinterpret_cast<uintptr_t>(d.acc)) & 15) == 0;
            // The common form, fp32 y only with payload magnitude 1 and an
            // output of at most 2 GiB: buffer stores at 32-bit offsets, lanes
            // outside the matrix sent to offset 2^31, past the buffer's range
            // (the hardware drops them), so no store needs a branch or a
            // 64-bit address (the general form below takes 20 or more
            // instructions a store, and the matrix cores idle meanwhile).
            const bool fast_y = vec_out && d.y && !d.acc && d.w_mag == 1 && (long long)d.M * d.N <= (1LL << 29);
            bool freed_early = false;  // (FS) the stage freed before the stores
            if (fast_y) {
                // Strips in pairs (2 t, 2 t + 1), whole 128-byte lines per
                // store: after the transpose lane (j, g) holds row 4 g + j % 4
                // of the row block, columns 4 (j / 4) .. +3 of a strip; the
                // swap of 16-lane rows between the pair (odd rows of the
                // first with even rows of the second) leaves in the first
                // rows 8 (g / 2) + j % 4 and in the second 8 (g / 2) + 4 +
                // j % 4, of strip 2 t + g % 2, so a store covers 8 rows x 2
                // strips.  Nontemporal: with whole lines it pays at every row
                // count (C4: M = 128 265.3 -> 255.0 us, M = 32 121.1 -> 119.7,
                // M = 16 98.1 -> 96.1, M = 8 90.4 -> 89.8), where half lines
                // made it cost from two row blocks per wave on.
                const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
                    (void*)d.y, 0, (int)((unsigned)d.M * (unsigned)d.N * 4u), 0x00020000);
                // this lane's row scales first, then the stage is free
                float scl[C::MBW][2];
#pragma unroll
                for (int mb = 0; mb < C::MBW; ++mb)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        scl[mb][h] = xs_l[(rg * C::MBW + mb) * 16 + (g >> 1) * 8 + h * 4 + (lane & 3)] * d.w_scale;
                if constexpr (C::FS) {
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    signal_one(freed + 4 * done_stage, lane);
                    freed_early = true;
                }
#pragma unroll
                for (int mb = 0; mb < C::MBW; ++mb) {
#pragma unroll
                    for (int t = 0; t < C::S / 2; ++t) {
                        i32x4 v[2] = {quad_transpose(acc[2 * t][mb], lane), quad_transpose(acc[2 * t + 1][mb], lane)};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const auto sw = __builtin_amdgcn_permlane16_swap((unsigned)v[0][e], (unsigned)v[1][e],
                                                                             false, false);
                            v[0][e] = (int)sw[0];
                            v[1][e] = (int)sw[1];
                        }
                        const int col = (bc.st0 + sg * C::S + 2 * t + (g & 1)) * kStripCols + (j & ~3);
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const int row = (rg * C::MBW + mb) * 16 + (g >> 1) * 8 + h * 4 + (lane & 3);
                            const float sc = scl[mb][h];
                            const unsigned off = row < d.M && col < d.N
                                                     ? ((unsigned)row * (unsigned)d.N + (unsigned)col) * 4u
                                                     : 0x80000000u;
                            const f32x4 y = f32x4{(float)v[h][0] * sc, (float)v[h][1] * sc, (float)v[h][2] * sc,
                                                  (float)v[h][3] * sc};
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, y), yr, (int)off, 0,
                                                                   2 /* nt */);
                        }
                    }
                }
            } else if (vec_out) {
#pragma unroll
                for (int mb = 0; mb < C::MBW; ++mb) {
                    // after the transpose lane (j, g) holds row 4 g + j % 4 of
                    // the row block, columns 4 (j / 4) .. +3 of each strip
                    const int row = (rg * C::MBW + mb) * 16 + g * 4 + (lane & 3);
                    const float sc = xs_l[row] * d.w_scale;
#pragma unroll
                    for (int s = 0; s < C::S; ++s) {
                        i32x4 v = quad_transpose(acc[s][mb], lane);
                        const int col = (bc.st0 + sg * C::S + s) * kStripCols + (j & ~3);
                        if (row < d.M && col < d.N) {
                            const long long o = (long long)row * d.N + col;
                            if (d.acc) *reinterpret_cast<TER_GLOBAL i32x4*>(gptr(d.acc) + o) = v;
                            if (d.y)
                                *reinterpret_cast<TER_GLOBAL f32x4*>(gptr(d.y) + o) =
                                    f32x4{acc_to_float(v[0], d.w_mag) * sc, acc_to_float(v[1], d.w_mag) * sc,
                                          acc_to_float(v[2], d.w_mag) * sc, acc_to_float(v[3], d.w_mag) * sc};
                        }
                    }
                }
            } else {
#pragma unroll
                for (int mb = 0; mb < C::MBW; ++mb) {
                    const f32x4 xq = *reinterpret_cast<const f32x4*>(xs_l + (rg * C::MBW + mb) * 16 + g * 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int row = (rg * C::MBW + mb) * 16 + g * 4 + e;
                        if (row < d.M) {
                            const float sc = xq[e] * d.w_scale;
#pragma unroll
                            for (int s = 0; s < C::S; ++s) {
                                const int col = (bc.st0 + sg * C::S + s) * kStripCols + j;
                                if (col < d.N) emit_out(d, (long long)row * d.N + col, acc[s][mb][e], sc);
                            }
                        }
                    }
                }
            }
            if (C::FS && !freed_early) signal_one(freed + 4 * done_stage, lane);
#pragma unroll
            for (int s = 0; s < C::S; ++s)
#pragma unroll
                for (int mb = 0; mb < C::MBW; ++mb) acc[s][mb] = i32x4{0, 0, 0, 0};
            if (++cb >= b_hi) break;
            bc = block_at<kList>(single, list, blocks, cb, C::BS);
            cu = 0;
        }
    }
}

// Allow the configuration's dynamic LDS (above the 64 KiB default) for both
// instantiations; once per process (repeating it is harmless).
template <class C>
hipError_t allow_lds() {
    static hipError_t done = [] {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_lds_kernel<C, true>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e == hipSuccess)
            e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_lds_kernel<C, false>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        return e;
    }();
    return done;
}

template <class C>
hipError_t launch_cfg(const GemmDesc& single, const GemmDesc* list, const GemmBlock* blocks, const int32_t* ranges,
                      int n_blocks, int n_wg, hipStream_t st) {
    const hipError_t e = allow_lds<C>();
    if (e != hipSuccess) return e;
    if (list)
        hipLaunchKernelGGL((gemm_lds_kernel<C, true>), dim3(n_wg), dim3(C::THREADS), C::LDS, st, single, list, blocks,
                           ranges, n_blocks, n_wg);
    else
        hipLaunchKernelGGL((gemm_lds_kernel<C, false>), dim3(n_wg), dim3(C::THREADS), C::LDS, st, single, list,
                           blocks, ranges, n_blocks, n_wg);
    return hipGetLastError();
}

template <class C>
int occupancy_cfg() {
    if (allow_lds<C>() != hipSuccess) return 0;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemm_lds_kernel<C, true>, C::THREADS, C::LDS) != hipSuccess)
        return 0;
    return n;
}

}  // namespace

int gemm_lds_strips_per_block(int mb) {
    switch (mb) {
        case 1: return Cfg1::BS;
        case 2: return Cfg2::BS;
        case 4: return Cfg4::BS;
        case 8: return Cfg8::BS;
        default: return 0;
    }
}

int gemm_lds_max_wg_per_cu(int mb) {
    switch (mb) {
        case 1: return occupancy_cfg<Cfg1>();
        case 2: return occupancy_cfg<Cfg2>();
        case 4: return occupancy_cfg<Cfg4>();
        case 8: return occupancy_cfg<Cfg8>();
        default: return 0;
    }
}

hipError_t launch_gemm_lds(const GemmDesc& single, const GemmDesc* list_dev, const GemmBlock* blocks_dev,
                           const int32_t* ranges_dev, int n_blocks, int n_wg, int mb, hipStream_t st) {
    switch (mb) {
        case 1: return launch_cfg<Cfg1>(single, list_dev, blocks_dev, ranges_dev, n_blocks, n_wg, st);
        case 2: return launch_cfg<Cfg2>(single, list_dev, blocks_dev, ranges_dev, n_blocks, n_wg, st);
        case 4: return launch_cfg<Cfg4>(single, list_dev, blocks_dev, ranges_dev, n_blocks, n_wg, st);
        case 8: return launch_cfg<Cfg8>(single, list_dev, blocks_dev, ranges_dev, n_blocks, n_wg, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace terhip
