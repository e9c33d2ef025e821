// abi.hip -- the extern "C" boundary (include/ter_hip.h).
//
// Validates every argument on the host before touching the device and
// returns ter_k4-style status codes (src/k4/ter_k4.cpp:38,52-55); never
// aborts.  There is no CPU compute path: a request the HIP kernels cannot
// serve is an error.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cmath>
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <queue>
#include <new>
#include <string>
#include <vector>

#include "common.h"

namespace terhip {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(TER_HIP_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

namespace {

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int check_wpk(const ter_hip_wpk_t* w) {
    if (!w || !w->data || !w->fix) return fail(TER_HIP_ERR_NULL, "null weight handle or buffer");
    if (w->layout != TER_HIP_LAYOUT_T16) return fail(TER_HIP_ERR_PAYLOAD, "unknown weight layout %d", w->layout);
    if (w->K < 1 || w->K > TER_HIP_K_MAX || w->N < 1 || w->N > TER_HIP_N_MAX)
        return fail(TER_HIP_ERR_SHAPE, "weight shape K=%d N=%d out of range", w->K, w->N);
    if (w->bytes < ter_hip_wpk_bytes(w->K, w->N)) return fail(TER_HIP_ERR_SHAPE, "weight buffer too small");
    if (w->mag < 1) return fail(TER_HIP_ERR_PAYLOAD, "trit magnitude %d < 1", w->mag);
    return TER_HIP_OK;
}

bool is_rms(int kind) {
    return kind == TER_HIP_X_F32_RMS || kind == TER_HIP_X_F16_RMS || kind == TER_HIP_X_RELU2_RMS;
}

// Kinds whose GEMV descriptor stages fp32 activations in LDS where K allows:
// the RMS kinds (their sum of squares reads them) and the fp16 absmax kinds
// (the strided strip prologue quantizes from them).
bool stages32(int kind) {
    return is_rms(kind) || kind == TER_HIP_X_F16 || kind == TER_HIP_X_SILU_MUL || kind == TER_HIP_X_SMUL;
}

// The gated kinds: `up` multiplies the activation.
bool gated(int kind) {
    return kind == TER_HIP_X_RELU2_RMS || kind == TER_HIP_X_SILU_MUL || kind == TER_HIP_X_SMUL;
}

// Kinds whose prologue runs only inside the GEMV kernels (no batched row
// quantizer): int16 rows, the fp16 absmax and the silu(gate) * up kinds.
bool gemv_only_kind(int kind) {
    return kind == TER_HIP_X_I16 || kind == TER_HIP_X_F16 || kind == TER_HIP_X_SILU_MUL || kind == TER_HIP_X_SMUL;
}

int check_act(const ter_hip_act_t* x, int M) {
    if (!x || !x->data) return fail(TER_HIP_ERR_NULL, "null activation");
    if (x->kind != TER_HIP_X_I8 && x->kind != TER_HIP_X_F32 && !gemv_only_kind(x->kind) && !is_rms(x->kind))
        return fail(TER_HIP_ERR_PAYLOAD, "unknown activation kind %d", x->kind);
    if (gemv_only_kind(x->kind) && M != 1)
        return fail(TER_HIP_ERR_PAYLOAD, "activation kind %d runs as single GEMVs and GEMV work lists only (M=%d)",
                    x->kind, M);
    if (x->kind == TER_HIP_X_I16 && !aligned(x->data, 2)) return fail(TER_HIP_ERR_ALIGN, "int16 X misaligned");
    if ((x->kind == TER_HIP_X_F32 || x->kind == TER_HIP_X_F32_RMS || x->kind == TER_HIP_X_SMUL) &&
        !aligned(x->data, 4))
        return fail(TER_HIP_ERR_ALIGN, "fp32 X misaligned");
    if ((x->kind == TER_HIP_X_F16_RMS || x->kind == TER_HIP_X_RELU2_RMS || x->kind == TER_HIP_X_F16 ||
         x->kind == TER_HIP_X_SILU_MUL) &&
        !aligned(x->data, 2))
        return fail(TER_HIP_ERR_ALIGN, "fp16 X misaligned");
    if (gated(x->kind)) {
        if (!x->up) return fail(TER_HIP_ERR_NULL, "gated activation without up");
        if (!aligned(x->up, 2)) return fail(TER_HIP_ERR_ALIGN, "fp16 up misaligned");
    }
    if (is_rms(x->kind)) {
        if (!x->gamma) return fail(TER_HIP_ERR_NULL, "RMSNorm activation without gamma");
        if (!aligned(x->gamma, 2)) return fail(TER_HIP_ERR_ALIGN, "gamma misaligned");
        if (!(x->eps >= 0.f)) return fail(TER_HIP_ERR_SHAPE, "RMSNorm eps must be >= 0");
    }
    if (M > 1 && x->kind == TER_HIP_X_I8 && !x->scale_dev)
        return fail(TER_HIP_ERR_NULL, "batched int8 X needs per-row device scales");
    return TER_HIP_OK;
}

int check_out(const ter_hip_out_t* o) {
    if (!o || (!o->y && !o->acc && !o->y16 && !o->resid && !o->resid16 && !o->silu))
        return fail(TER_HIP_ERR_NULL, "no output buffer");
    if (!aligned(o->y, 4) || !aligned(o->acc, 4) || !aligned(o->y16, 2) || !aligned(o->resid, 4) ||
        !aligned(o->resid16, 2) || !aligned(o->silu, 4))
        return fail(TER_HIP_ERR_ALIGN, "output buffer misaligned");
    return TER_HIP_OK;
}

// Algorithmic bytes per activation element (inputs, gamma included) and per
// output element (a residual is read and written).
unsigned act_bytes(int kind) {
    switch (kind) {
        case TER_HIP_X_F32: return 4;
        case TER_HIP_X_F32_RMS: return 6;
        case TER_HIP_X_F16_RMS: return 4;
        case TER_HIP_X_RELU2_RMS: return 6;
        case TER_HIP_X_I16: return 2;
        case TER_HIP_X_F16: return 2;
        case TER_HIP_X_SILU_MUL: return 4;
        case TER_HIP_X_SMUL: return 6;
        default: return 1;
    }
}
unsigned out_bytes(const ter_hip_out_t& o) {
    return (o.y ? 4u : 0u) + (o.acc ? 4u : 0u) + (o.y16 ? 2u : 0u) + (o.resid ? 8u : 0u) + (o.resid16 ? 4u : 0u) +
           (o.silu ? 4u : 0u);
}

typedef std::vector<std::pair<uintptr_t, uintptr_t>> Ranges;

bool overlaps(const std::pair<uintptr_t, uintptr_t>& a, const std::pair<uintptr_t, uintptr_t>& b) {
    return a.first < b.second && b.first < a.second;
}

// Device byte ranges an activation operand reads (M rows of K elements).
void act_ranges(const ter_hip_act_t* x, int M, int K, Ranges* out) {
    const size_t n = (size_t)M * (size_t)K;
    const size_t el = x->kind == TER_HIP_X_I8
                          ? 1
                          : (x->kind == TER_HIP_X_F32 || x->kind == TER_HIP_X_F32_RMS || x->kind == TER_HIP_X_SMUL
                                 ? 4
                                 : 2);  // I16, fp16: 2
    out->emplace_back((uintptr_t)x->data, (uintptr_t)x->data + n * el);
    if (gated(x->kind) && x->up)
        out->emplace_back((uintptr_t)x->up, (uintptr_t)(x->up + n));
}

// Residual targets of one launch must not overlap one another or any input
// the launch reads: each element is a plain read-modify-write by the one
// thread that finishes its column, while other workgroups may still be
// reading their activations.
int check_resid_overlap(const Ranges& resid, const Ranges& inputs) {
    for (size_t i = 0; i < resid.size(); ++i) {
        for (size_t k = 0; k < i; ++k)
            if (overlaps(resid[i], resid[k]))
                return fail(TER_HIP_ERR_CONFLICT, "residual outputs %zu and %zu overlap", i, k);
        for (const auto& in : inputs)
            if (overlaps(resid[i], in))
                return fail(TER_HIP_ERR_CONFLICT, "residual output %zu overlaps an activation input", i);
    }
    return TER_HIP_OK;
}

std::mutex g_cu_mu;
std::vector<int> g_cu;

GemvDesc make_desc(const ter_hip_wpk_t* w, const ter_hip_act_t* x, const ter_hip_out_t& o, long long tile0) {
    GemvDesc d{};
    d.w = w->data;
    d.x = x->data;
    d.x_scale_dev = x->kind == TER_HIP_X_I8 || x->kind == TER_HIP_X_I16 ? x->scale_dev : nullptr;
    d.y = o.y;
    d.acc = o.acc;
    d.y16 = o.y16;
    d.resid = o.resid;
    d.resid16 = o.resid16;
    d.silu = o.silu;
    const bool quantized = x->kind != TER_HIP_X_I8 && x->kind != TER_HIP_X_I16;
    d.xq_out = quantized ? x->q_out : nullptr;
    d.xs_out = quantized ? x->scale_out : nullptr;
    d.gamma = is_rms(x->kind) ? x->gamma : nullptr;
    d.up = gated(x->kind) ? x->up : nullptr;
    d.eps = x->eps;
    d.fix = reinterpret_cast<unsigned long long*>(w->fix);
    d.tile0 = tile0;
    d.K = w->K;
    d.N = w->N;
    d.Ku = units_of(w->K);
    d.n_strips = strips_of(w->N);
    d.w_scale = w->scale;
    d.w_mag = w->mag;
    d.x_scale = x->scale;
    d.x_kind = x->kind;
    d.stage32 = stages32(x->kind) && gemv_stage32(w->K) ? 1 : 0;
    return d;
}

// Workgroups of one GEMV launch: kGemvWgPerCu per CU (measured best for the
// layer sweeps), capped by what fits at once (occupancy query) so the static
// partition runs as a single wave of resident workgroups, and raised if a
// wave's piece would exceed kMaxPieceTiles (its buffer resource spans at most
// 2^31 bytes).  wg_per_cu > 0 overrides (tuning).
constexpr int kGemvWgPerCu = 2;
// Work lists of int8 GEMVs qualifying for the vector prologue run the int8
// kernel (96 VGPRs): four workgroups per CU hide more latency there (C2
// Llama sweep: 42.6 against 43.3 us at two); the other kinds keep two.
constexpr int kGemvWgPerCuI8 = 4;
// fp32 activations (the in-kernel absmax prologue; that kernel fits three
// waves per SIMD): three workgroups per CU (C3 BitNet sweep: 86.3 against
// 87.0 us at two, 91.4 at four, the fourth waiting for a free slot).
constexpr int kGemvWgPerCuF32 = 3;
// A launch whose activations need a prologue (any kind but X_I8) and that
// has fewer tiles than this per workgroup at kGemvWgPerCu uses one workgroup
// per CU: every workgroup repeats the prologue, and below this size halving
// the repeats gains more than the second workgroup's overlap (decode-step
// plans: 1600 - 8640 tiles).
constexpr long long kSmallPlanTilesPerWg = 32;
constexpr long long kMaxPieceTiles = 1 << 20;

// The activation kind shared by every item of a GEMV work list when each
// qualifies for the kernel's vector prologue (K a multiple of 16; x, up and
// gamma 16-byte aligned; the staged kinds' fp32 staging fits), else -1 (the
// general prologue).  X_F16 and X_SILU_MUL have a vector prologue only in
// strip mode (strided); elsewhere their kind launches the general kernel.
int gemv_vec_kind(const ter_hip_gemv_item_t* items, int n) {
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    const int kind = items[0].x.kind;
    for (int i = 0; i < n; ++i) {
        const ter_hip_act_t& x = items[i].x;
        if (x.kind != kind || items[i].w->K % 16 != 0 || !a16(x.data)) return -1;
        if (x.kind == TER_HIP_X_I16) return -1;  // the general prologue
        if (stages32(x.kind) && !gemv_stage32(items[i].w->K)) return -1;  // the vector prologues always stage
        if (gated(x.kind) && !a16(x.up)) return -1;
        if (is_rms(x.kind) && !a16(x.gamma)) return -1;
    }
    return kind;
}

// Strip mode for work lists below kSmallPlanTilesPerWg tiles per workgroup at
// the default occupancy and with at most four strips per CU (the decode
// step's gate/up list, 2 x 432 strips of 10 units, included: 1.168 -> 1.147 ms
// per C5 token against its stream-K partition): one workgroup per strip up to
// one per CU (two for int8 inputs, which have no prologue to repeat).
int pick_strip_mode(long long total_tiles, long long total_strips, bool prologue, bool* strip_mode, int* n_wg) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    const int cus = device_cu_count(dev);
    if (cus <= 0) return fail(TER_HIP_ERR_HIP, "cannot query CU count");
    *strip_mode = total_tiles < (long long)cus * kGemvWgPerCu * kSmallPlanTilesPerWg &&
                  total_strips <= (long long)cus * 4;
    if (!*strip_mode) return TER_HIP_OK;
    long long g = (long long)cus * (prologue ? 1 : kGemvWgPerCu);
    if (g > total_strips) g = total_strips;
    const long long min_g = (total_strips + kStripModeMaxStrips - 1) / kStripModeMaxStrips;
    if (g < min_g) g = min_g;
    if (g < 1) g = 1;
    *n_wg = (int)g;
    return TER_HIP_OK;
}

int pick_wg(long long total_tiles, int wg_per_cu, int lds_bytes, bool prologue, int vec_kind, int* n_wg) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    const int cus = device_cu_count(dev);
    if (cus <= 0) return fail(TER_HIP_ERR_HIP, "cannot query CU count");
    const int fit = gemv_max_wg_per_cu(lds_bytes, vec_kind);
    if (fit <= 0) return fail(TER_HIP_ERR_SHAPE, "GEMV workgroup does not fit a CU (LDS %d bytes)", lds_bytes);
    const int dflt = vec_kind == TER_HIP_X_I8 ? kGemvWgPerCuI8
                     : (vec_kind == TER_HIP_X_F32 ? kGemvWgPerCuF32 : kGemvWgPerCu);
    int per_cu = wg_per_cu > 0 ? wg_per_cu : (dflt < fit ? dflt : fit);
    if (wg_per_cu <= 0 && prologue && total_tiles < (long long)cus * kGemvWgPerCu * kSmallPlanTilesPerWg) per_cu = 1;
    long long g = (long long)cus * per_cu;
    const long long min_g = (total_tiles + kMaxPieceTiles * kGemvWaves - 1) / (kMaxPieceTiles * kGemvWaves);
    if (g < min_g) g = min_g;
    if (g > total_tiles) g = total_tiles;
    if (g < 1) g = 1;
    if (g > 0x7fffffffLL) return fail(TER_HIP_ERR_SHAPE, "work list too large");
    *n_wg = (int)g;
    return TER_HIP_OK;
}

// per_block: strips per block of the launch (kWaves * strips per wave for its row-block count).
GemmDesc make_gemm_desc(const ter_hip_wpk_t* w, const int8_t* x, const float* xs, int M, const ter_hip_out_t& o,
                        long long block0, int per_block, long long tile0) {
    GemmDesc d{};
    d.w = w->data;
    d.x = x;
    d.xs = xs;
    d.y = o.y;
    d.acc = o.acc;
    d.y16 = o.y16;
    d.resid = o.resid;
    d.block0 = block0;
    d.tile0 = tile0;
    d.K = w->K;
    d.N = w->N;
    d.Ku = units_of(w->K);
    d.n_strips = strips_of(w->N);
    d.M = M;
    d.ldx = w->K;
    d.n_blocks = (d.n_strips + per_block - 1) / per_block;
    d.w_scale = w->scale;
    d.w_mag = w->mag;
    return d;
}

bool gemm_vec_ok(const GemmDesc& d) { return aligned(d.x, 16) && d.ldx % 16 == 0; }

// Rows per piece of the LDS-ring GEMM (8 row blocks).  A GEMM with more rows
// (prefill) whose X rows are 16-byte aligned is cut into pieces of this many
// rows over the same weights, so the ring kernel serves it instead of the
// register-staged kernel (M = 256 on the BitNet-2B sweep: about 2x the
// M = 128 time, against 11x).
constexpr int kRingRows = 128;

bool ring_rows_ok(const int8_t* x, int K) { return aligned(x, 16) && K % 16 == 0; }

// The outputs of rows r0.. of an [M][N] output set.
ter_hip_out_t out_rows(const ter_hip_out_t& o, int r0, int N) {
    const size_t off = (size_t)r0 * (size_t)N;
    return ter_hip_out_t{o.y ? o.y + off : nullptr, o.acc ? o.acc + off : nullptr, o.y16 ? o.y16 + off : nullptr,
                         o.resid ? o.resid + off : nullptr, o.resid16 ? o.resid16 + off : nullptr,
                         o.silu ? o.silu + off : nullptr};
}

// GEMM workgroups: up to kGemmWgPerCu per CU (more weight bytes in flight
// for the HBM-bound small-M blocks), capped by occupancy and by the block count.
constexpr int kGemmWgPerCu = 8;

// Streaming GEMM (M <= 16): kGemmWgPerCuStream workgroups per CU, capped by
// occupancy at this LDS size.
constexpr int kGemmWgPerCuStream = 2;

int pick_stream_wg(long long tiles, int lds, int wg_per_cu, int* n_wg) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    const int cus = device_cu_count(dev);
    if (cus <= 0) return fail(TER_HIP_ERR_HIP, "cannot query CU count");
    const int fit = gemm_stream_max_wg_per_cu(lds);
    if (fit <= 0) return fail(TER_HIP_ERR_HIP, "GEMM occupancy query failed");
    const int per_cu = wg_per_cu > 0 ? wg_per_cu : (kGemmWgPerCuStream < fit ? kGemmWgPerCuStream : fit);
    long long g = (long long)cus * per_cu;
    if (g > tiles) g = tiles;
    if (g < 1) g = 1;
    *n_wg = (int)g;
    return TER_HIP_OK;
}

int pick_gemm_wg(long long blocks, int mb, int wg_per_cu, int* n_wg) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    const int cus = device_cu_count(dev);
    if (cus <= 0) return fail(TER_HIP_ERR_HIP, "cannot query CU count");
    const int fit = gemm_max_wg_per_cu(mb);
    if (fit <= 0) return fail(TER_HIP_ERR_HIP, "GEMM occupancy query failed");
    const int per_cu = wg_per_cu > 0 ? wg_per_cu : (kGemmWgPerCu < fit ? kGemmWgPerCu : fit);
    long long g = (long long)cus * per_cu;
    if (g > blocks) g = blocks;
    if (g < 1) g = 1;
    *n_wg = (int)g;
    return TER_HIP_OK;
}

}  // namespace

int device_cu_count(int device) {
    std::lock_guard<std::mutex> lk(g_cu_mu);
    if (device < 0) return -1;
    if ((int)g_cu.size() <= device) g_cu.resize(device + 1, 0);
    if (g_cu[device] == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return -1;
        g_cu[device] = v;
    }
    return g_cu[device];
}

}  // namespace terhip

using namespace terhip;

struct ter_hip_plan {
    void* descs_dev = nullptr;   // GemvDesc[n] (GEMV plan) or GemmDesc[n] (GEMM plan), then first_dev
    const int32_t* first_dev = nullptr;  // [n_wg] first descriptor of each workgroup's range
    int n = 0;
    bool gemm = false;
    long long total = 0;         // tiles (GEMV) or blocks (GEMM) of one launch
    int n_wg = 0;
    int lds_bytes = 0;           // GEMV
    int vec_kind = -1;           // GEMV: common activation kind for the vector prologue, or -1
    bool strip_mode = false;     // GEMV: strip-mode kernel, total counts strips
    int part_off = 0;            // GEMV strip mode: LDS offset of the partial sums
    bool strided = false;        // GEMV strip mode: the strided RMS prologue (gemv_strided_ok for every item)
    bool shared = false;         // GEMV strided strip mode: one activation, back-to-back tile streams
    GemvDesc shared_desc{};      //   its kernel argument (shared_plan_desc)
    int mb = 0;                  // GEMM row-block count
    bool vec = false;            // GEMM: 16-byte X rows
    bool stream = false;         // GEMM: streaming kernel (M <= 16), total counts tiles

    bool lds = false;            // GEMM: LDS-ring kernel (M <= 128 where streaming does not apply)
    const GemmBlock* blocks_dev = nullptr;  // LDS-ring: [n_blocks] blocks, then
    const int32_t* ranges_dev = nullptr;    //   [n_wg + 1] block ranges per workgroup
    const long long* wg_ranges_dev = nullptr;  // GEMV stream-K: [n_wg + 1] tile ranges per workgroup
    const void* wg_desc_dev = nullptr;         // GEMV strip mode: [n_wg] copies of each workgroup's first descriptor
    int n_blocks = 0;
    uint64_t bytes = 0, macs = 0;
};

struct ter_hip_attn {
    int nh = 0, nkv = 0, hd = 0, smax = 0;
    bool neox = true;
    bool xcd_local = false;     // the XCD-local exchange (dispatch checked at creation)
    float* rope = nullptr;      // [smax][hd/2][2]
    float* part = nullptr;      // [nh][n_chunks][attn_part_stride(hd)]
    unsigned* count = nullptr;  // [n_groups][attn_count_stride()], zero at rest
};

struct ter_hip_handle {
    int device = 0;
    struct Slot {
        char name[32];
        ter_hip_native_fn fn;
        bool used;
    } slots[32];
    ter_hip_op_counts_t counts;
};

// Device copy of a plan: the descriptors, followed by the index of each
// workgroup's first descriptor.  The kernels cut `total` units into n_wg
// ranges, range g starting at total * g / n_wg, or at ranges[g] when a range
// table is given (then uploaded after `first`); starts[i] is descriptor i's
// first unit, strictly increasing.
template <typename Desc>
int upload_plan(ter_hip_plan* p, const std::vector<Desc>& ds, const std::vector<long long>& starts, long long total,
                int n_wg, const std::vector<long long>* ranges = nullptr, int wg_copies = 0) {
    std::vector<int32_t> first((size_t)n_wg);
    size_t di = 0;
    for (int g = 0; g < n_wg; ++g) {
        const long long t = ranges ? (*ranges)[(size_t)g] : total * g / n_wg;
        while (di + 1 < starts.size() && starts[di + 1] <= t) ++di;
        first[(size_t)g] = (int32_t)di;
    }
    const size_t db = sizeof(Desc) * ds.size();
    const size_t fb = (sizeof(int32_t) * (size_t)n_wg + 7) / 8 * 8;
    const size_t rb = ranges ? sizeof(long long) * ranges->size() : 0;
    // wg_copies 1: then each workgroup's first descriptor once more, in
    // workgroup order; 2: its first and the next (the last one repeated), in
    // block order (block b runs workgroup range (b % 8) (n_wg / 8) + b / 8
    // when 8 divides n_wg, else b)
    const size_t cb0 = (db + fb + rb + 15) / 16 * 16;
    std::vector<Desc> copies;
    for (int b = 0; wg_copies > 0 && b < n_wg; ++b) {
        const int g = wg_copies > 1 && n_wg % 8 == 0 ? (b % 8) * (n_wg / 8) + b / 8 : b;
        const size_t f = (size_t)first[(size_t)g];
        copies.push_back(ds[f]);
        if (wg_copies > 1) copies.push_back(ds[f + 1 < ds.size() ? f + 1 : f]);
    }
    const size_t cb = sizeof(Desc) * copies.size();
    hipError_t e = hipMalloc(&p->descs_dev, cb0 + cb);
    if (e != hipSuccess) {
        p->descs_dev = nullptr;
        return hip_fail(e, "plan descriptor allocation");
    }
    char* base = static_cast<char*>(p->descs_dev);
    e = hipMemcpy(base, ds.data(), db, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(base + db, first.data(), sizeof(int32_t) * (size_t)n_wg, hipMemcpyHostToDevice);
    if (e == hipSuccess && ranges) e = hipMemcpy(base + db + fb, ranges->data(), rb, hipMemcpyHostToDevice);
    if (e == hipSuccess && cb) e = hipMemcpy(base + cb0, copies.data(), cb, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(p->descs_dev);
        p->descs_dev = nullptr;
        return hip_fail(e, "plan descriptor upload");
    }
    p->first_dev = reinterpret_cast<const int32_t*>(base + db);
    p->wg_ranges_dev = ranges ? reinterpret_cast<const long long*>(base + db + fb) : nullptr;
    p->wg_desc_dev = cb ? base + cb0 : nullptr;
    return TER_HIP_OK;
}

// Workgroup tile ranges of a stream-K GEMV plan: range g nominally starts at
// total * g / n_wg; each interior start moves to the nearest strip edge of
// the GEMV holding it when snap_ranges allows (common.h), so that most
// workgroups share no strip with a neighbour.  Nondecreasing, ranges[0] = 0,
// ranges[n_wg] = total.
std::vector<long long> plan_ranges(const std::vector<GemvDesc>& ds, const std::vector<long long>& starts,
                                   long long total, int n_wg) {
    std::vector<long long> r((size_t)n_wg + 1);
    size_t di = 0;
    r[0] = 0;
    r[(size_t)n_wg] = total;
    for (int g = 1; g < n_wg; ++g) {
        long long t = total * g / n_wg;
        while (di + 1 < starts.size() && starts[di + 1] <= t) ++di;
        const int Ku = ds[di].Ku;
        if (snap_ranges(Ku, total, n_wg)) t = starts[di] + strip_edge_near(t - starts[di], Ku);
        r[(size_t)g] = t < r[(size_t)g - 1] ? r[(size_t)g - 1] : t;
    }
    return r;
}

// LDS-ring GEMM (M <= 128, 16-byte aligned X): resident workgroups per
// CU times the CU count, capped by the block count.
int pick_lds_wg(long long blocks, int mb, int* n_wg) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    const int cus = device_cu_count(dev);
    if (cus <= 0) return fail(TER_HIP_ERR_HIP, "cannot query CU count");
    const int fit = gemm_lds_max_wg_per_cu(mb);
    if (fit <= 0) return fail(TER_HIP_ERR_HIP, "GEMM occupancy query failed");
    long long g = (long long)cus * fit;
    if (g > blocks) g = blocks;
    if (g < 1) g = 1;
    *n_wg = (int)g;
    return TER_HIP_OK;
}

// Int16-activation GEMV: whole strips per workgroup, two workgroups per CU
// (one strip each for small N), at most kStripModeMaxStrips strips each.
int launch_x16(const GemvDesc& d, hipStream_t st) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    const int cus = device_cu_count(dev);
    if (cus <= 0) return fail(TER_HIP_ERR_HIP, "cannot query CU count");
    long long g = std::min<long long>((long long)cus * 2, d.n_strips);
    const long long min_g = ((long long)d.n_strips + kStripModeMaxStrips - 1) / kStripModeMaxStrips;
    if (g < min_g) g = min_g;
    if (g >= 8) g -= g % 8;  // a multiple of 8 keeps neighbouring strips on one XCD
    if (g < min_g) g += 8;
    const int per_wg = (int)(((long long)d.n_strips + g - 1) / g);
    const int lds = gemv_x16_lds_bytes(d.K, per_wg);
    if (lds > kLdsMax) return fail(TER_HIP_ERR_SHAPE, "int16 GEMV needs %d bytes of LDS", lds);
    e = launch_gemv_x16(d, (int)g, lds, st);
    if (e != hipSuccess) return hip_fail(e, "int16 gemv launch");
    return TER_HIP_OK;
}

// Workspace of ter_hip_gemm_out_static: the quantized rows (int8
// [M][K], at most TER_HIP_STATIC_Q_MAX bytes) followed by their scales
// (fp32 [M], M <= TER_HIP_M_MAX).  One copy per GPU, held until the process
// ends; host code reaches it only through the address hipGetSymbolAddress
// returns for the current device (the array's name is a host-side stand-in).
constexpr size_t kScratchScaleOff = TER_HIP_STATIC_Q_MAX;
constexpr size_t kScratchBytes = kScratchScaleOff + TER_HIP_M_MAX * sizeof(float);
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

static std::mutex g_scratch_mu;
static std::vector<void*> g_scratch_ptr;  // per device; null until looked up on it

// The current device's address of `scratch`, looked up once per device.
static int scratch_of_current_device(unsigned char** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize((size_t)dev + 1, nullptr);
    if (!g_scratch_ptr[(size_t)dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(TER_HIP_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
        g_scratch_ptr[(size_t)dev] = p;
    }
    *out = static_cast<unsigned char*>(g_scratch_ptr[(size_t)dev]);
    return TER_HIP_OK;
}

// Host staging of the synchronous mm_row calls: page-locked buffers, one
// pair per device, grown on demand and held until the process ends.  The
// row is narrowed straight into page-locked memory, so its upload is one DMA
// with no bounce through the runtime's own staging, and the GEMV writes its
// fp32 outputs straight into page-locked host memory (coherent: the writes
// reach host memory by the end of the kernel), so no download copy follows.
// Callers hold g_stage_mu for the whole call (the reference's mm_row is never
// called concurrently; calls from several threads are serialized).
struct MmRowStage {
    void* x = nullptr;
    size_t xcap = 0;
    float* y = nullptr;      // host address
    float* y_dev = nullptr;  // the same memory as the device addresses it
    size_t ycap = 0;
};
static std::mutex g_stage_mu;
static std::vector<MmRowStage> g_stage;

static size_t grown(size_t want) {
    size_t c = 64 * 1024;
    while (c < want) c *= 2;
    return c;
}

// The device's staging with room for xbytes and ybytes; false when pinned
// memory cannot be had (the caller then takes the pageable path).
static bool mm_row_stage(int dev, size_t xbytes, size_t ybytes, MmRowStage** out) {
    if ((int)g_stage.size() <= dev) g_stage.resize((size_t)dev + 1);
    MmRowStage& s = g_stage[(size_t)dev];
    if (s.xcap < xbytes) {
        if (s.x) (void)hipHostFree(s.x);
        s.x = nullptr;
        s.xcap = 0;
        const size_t c = grown(xbytes);
        if (hipHostMalloc(&s.x, c, hipHostMallocDefault) != hipSuccess) {
            s.x = nullptr;
            return false;
        }
        s.xcap = c;
    }
    if (s.ycap < ybytes) {
        if (s.y) (void)hipHostFree(s.y);
        s.y = s.y_dev = nullptr;
        s.ycap = 0;
        const size_t c = grown(ybytes);
        void* h = nullptr;
        void* d = nullptr;
        if (hipHostMalloc(&h, c, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) return false;
        if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess || !d || ((uintptr_t)d & 15u) != 0) {
            (void)hipHostFree(h);
            return false;
        }
        s.y = static_cast<float*>(h);
        s.y_dev = static_cast<float*>(d);
        s.ycap = c;
    }
    *out = &s;
    return true;
}

// Device copy of an LDS-ring GEMM plan: descriptors, the block list in
// workgroup order, and the per-workgroup block ranges.  Range g holds
// workgroup g's blocks in the order it runs them.  The blocks are dealt out
// largest first, each to the workgroup that would be free first (list
// scheduling; ties to the lowest workgroup).  The order is a stable sort by
// estimated cost, so blocks of one size stay in list order, and neighbouring
// blocks run at about the same time on neighbouring workgroups, which the
// kernel places on one XCD: the weight runs and output rows in flight at
// any moment lie close together in memory.  The cost of a block of ns
// strips over Ku 256-row units, in units of one full stage: Ku (0.3 + 0.7 ns
// / bs) (a stage's barrier and X rows cost the same at any width), plus one
// for the epilogue.  Against contiguous ranges balanced by units (the
// largest range 15% above the mean at 16 rows, 37% at 32 rows) this keeps
// every range within about 5% of the mean.
constexpr long long kRingMinBlocksPerCu = 4;
int upload_lds_plan(ter_hip_plan* p, const std::vector<GemmDesc>& ds, const std::vector<GemmBlock>& blocks_in,
                    int bs, int n_wg) {
    const size_t nb = blocks_in.size();
    std::vector<double> cost(nb);
    for (size_t b = 0; b < nb; ++b) {
        const GemmDesc& d = ds[(size_t)blocks_in[b].desc];
        const int ns = std::min(bs, d.n_strips - blocks_in[b].strip0);
        cost[b] = d.Ku * (0.3 + 0.7 * ns / bs) + 1.0;
    }
    std::vector<int32_t> order(nb);
    for (size_t b = 0; b < nb; ++b) order[b] = (int32_t)b;
    std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) { return cost[(size_t)a] > cost[(size_t)b]; });
    std::vector<std::vector<int32_t>> per_wg((size_t)n_wg);
    using Slot = std::pair<double, int>;  // (time the workgroup is free, workgroup)
    std::priority_queue<Slot, std::vector<Slot>, std::greater<Slot>> free_at;
    for (int g = 0; g < n_wg; ++g) free_at.push(Slot{0.0, g});
    for (const int32_t b : order) {
        Slot s = free_at.top();
        free_at.pop();
        per_wg[(size_t)s.second].push_back(b);
        s.first += cost[(size_t)b];
        free_at.push(s);
    }
    std::vector<GemmBlock> blocks;
    blocks.reserve(nb);
    std::vector<int32_t> ranges((size_t)n_wg + 1);
    for (int g = 0; g < n_wg; ++g) {
        ranges[(size_t)g] = (int32_t)blocks.size();
        for (const int32_t b : per_wg[(size_t)g]) blocks.push_back(blocks_in[(size_t)b]);
    }
    ranges[(size_t)n_wg] = (int32_t)blocks.size();
    const size_t db = sizeof(GemmDesc) * ds.size(), bb = sizeof(GemmBlock) * blocks.size();
    hipError_t e = hipMalloc(&p->descs_dev, db + bb + sizeof(int32_t) * ranges.size());
    if (e != hipSuccess) {
        p->descs_dev = nullptr;
        return hip_fail(e, "plan descriptor allocation");
    }
    char* base = static_cast<char*>(p->descs_dev);
    e = hipMemcpy(base, ds.data(), db, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(base + db, blocks.data(), bb, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = hipMemcpy(base + db + bb, ranges.data(), sizeof(int32_t) * ranges.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(p->descs_dev);
        p->descs_dev = nullptr;
        return hip_fail(e, "plan descriptor upload");
    }
    p->blocks_dev = reinterpret_cast<const GemmBlock*>(base + db);
    p->ranges_dev = reinterpret_cast<const int32_t*>(base + db + bb);
    p->n_blocks = (int)blocks.size();
    return TER_HIP_OK;
}

extern "C" {

const char* ter_hip_version(void) { return "ter_hip 0.1.0 (gfx950, T16 layout)"; }

const char* ter_hip_last_error(void) { return g_last_error.c_str(); }

size_t ter_hip_wpk_bytes(int32_t K, int32_t N) {
    if (K < 1 || N < 1) return 0;
    return tile_stream_bytes(K, N) + (size_t)N * sizeof(uint64_t);
}

int ter_hip_wpk_init(ter_hip_wpk_t* w, void* dev_buf, size_t buf_bytes, int32_t K, int32_t N, float scale) {
    if (!w || !dev_buf) return fail(TER_HIP_ERR_NULL, "null weight handle or buffer");
    if (K < 1 || K > TER_HIP_K_MAX || N < 1 || N > TER_HIP_N_MAX)
        return fail(TER_HIP_ERR_SHAPE, "shape K=%d N=%d out of range (K<=%d)", K, N, TER_HIP_K_MAX);
    if (!aligned(dev_buf, 256)) return fail(TER_HIP_ERR_ALIGN, "weight buffer must be 256-byte aligned");
    const size_t need = ter_hip_wpk_bytes(K, N);
    if (buf_bytes < need) return fail(TER_HIP_ERR_SHAPE, "weight buffer %zu < %zu bytes", buf_bytes, need);
    w->data = static_cast<uint8_t*>(dev_buf);
    w->bytes = need;
    w->fix = reinterpret_cast<uint64_t*>(w->data + fix_offset(K, N));
    w->K = K;
    w->N = N;
    w->scale = scale;
    w->layout = TER_HIP_LAYOUT_T16;
    w->mag = 1;
    return TER_HIP_OK;
}

int ter_hip_pack_v11(ter_hip_wpk_t* w, const uint8_t* v11_dev, void* stream) {
    int rc = check_wpk(w);
    if (rc) return rc;
    if (!v11_dev) return fail(TER_HIP_ERR_NULL, "null v11 buffer");
    if (w->N % 4) return fail(TER_HIP_ERR_SHAPE, "v11 needs N %% 4 == 0 (N=%d)", w->N);
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = launch_pack_v11(v11_dev, w->data, w->K, w->N, st);
    if (e != hipSuccess) return hip_fail(e, "pack_v11 launch");
    e = hipMemsetAsync(w->fix, 0, (size_t)w->N * sizeof(uint64_t), st);
    if (e != hipSuccess) return hip_fail(e, "fix-up slot clear");
    return TER_HIP_OK;
}

int ter_hip_pack_i2s(ter_hip_wpk_t* w, const uint8_t* i2s_dev, void* stream) {
    int rc = check_wpk(w);
    if (rc) return rc;
    if (!i2s_dev) return fail(TER_HIP_ERR_NULL, "null i2_s buffer");
    if (w->K % 4 || w->N % 4 || ((long long)w->K * w->N) % 128)
        return fail(TER_HIP_ERR_SHAPE, "i2_s needs K, N multiples of 4 and N*K a multiple of 128 (K=%d N=%d)", w->K,
                    w->N);
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = launch_pack_i2s(i2s_dev, w->data, w->K, w->N, st);
    if (e != hipSuccess) return hip_fail(e, "pack_i2s launch");
    e = hipMemsetAsync(w->fix, 0, (size_t)w->N * sizeof(uint64_t), st);
    if (e != hipSuccess) return hip_fail(e, "fix-up slot clear");
    return TER_HIP_OK;
}

int ter_hip_unpack_v11(const ter_hip_wpk_t* w, uint8_t* v11_dev, void* stream) {
    int rc = check_wpk(w);
    if (rc) return rc;
    if (!v11_dev) return fail(TER_HIP_ERR_NULL, "null v11 buffer");
    if (w->N % 4) return fail(TER_HIP_ERR_SHAPE, "v11 needs N %% 4 == 0 (N=%d)", w->N);
    hipError_t e = launch_unpack_v11(w->data, v11_dev, w->K, w->N, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "unpack_v11 launch");
    return TER_HIP_OK;
}

int ter_hip_pack_payload(ter_hip_wpk_t* w, const int32_t* payload, float scale, int32_t* magnitude_out,
                         void* stream) {
    int rc = check_wpk(w);
    if (rc) return rc;
    if (!payload) return fail(TER_HIP_ERR_NULL, "null payload");
    const int K = w->K, N = w->N;
    const size_t n = (size_t)K * (size_t)N;
    int64_t m = 0;
    for (size_t i = 0; i < n; ++i) {
        const int64_t a = payload[i] < 0 ? -(int64_t)payload[i] : (int64_t)payload[i];
        if (a == 0) continue;
        if (a > 0x7FFFFFFFLL) return fail(TER_HIP_ERR_PAYLOAD, "payload magnitude %lld does not fit int32", (long long)a);
        if (m == 0) m = a;
        else if (a != m)
            return fail(TER_HIP_ERR_PAYLOAD, "payload not ternary: |%lld| vs |%lld| at %zu", (long long)a,
                        (long long)m, i);
    }
    const int Ku = units_of(K), ns = strips_of(N);
    std::vector<uint32_t> host;
    try {
        host.assign(tile_stream_bytes(K, N) / 4, 0u);
    } catch (...) {
        return fail(TER_HIP_ERR_ALLOC, "host staging allocation");
    }
    for (int s = 0; s < ns; ++s)
        for (int u = 0; u < Ku; ++u)
            for (int lane = 0; lane < 64; ++lane)
                for (int j = 0; j < 4; ++j) {
                    const int r = lane >> 4, q = lane & 15;
                    const int col = s * kStripCols + r * 4 + j;
                    const int k0 = u * kUnitK + q * 16;
                    uint32_t out = 0;
                    for (int e = 0; e < 16; ++e) {
                        const int k = k0 + e;
                        uint32_t uv = 1u;
                        if (col < N && k < K) {
                            const int32_t p = payload[(size_t)k * N + col];
                            uv = p > 0 ? 2u : (p < 0 ? 0u : 1u);
                        }
                        out |= uv << (8 * (e & 3) + 2 * (e >> 2));
                    }
                    host[(((size_t)s * Ku + u) * 64 + lane) * 4 + j] = out;
                }
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(w->data, host.data(), host.size() * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipMemsetAsync(w->fix, 0, (size_t)N * sizeof(uint64_t), st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "payload upload");
    w->scale = scale;
    w->mag = (int32_t)(m == 0 ? 1 : m);
    if (magnitude_out) *magnitude_out = w->mag;
    return TER_HIP_OK;
}

int ter_hip_gemv(const ter_hip_wpk_t* w, const ter_hip_act_t* x, float* y, int32_t* acc, void* stream) {
    const ter_hip_out_t o{y, acc, nullptr, nullptr, nullptr};
    return ter_hip_gemv_out(w, x, &o, stream);
}

int ter_hip_gemv_out(const ter_hip_wpk_t* w, const ter_hip_act_t* x, const ter_hip_out_t* out, void* stream) {
    int rc = check_wpk(w);
    if (rc) return rc;
    rc = check_act(x, 1);
    if (rc) return rc;
    rc = check_out(out);
    if (rc) return rc;
    if (out->resid || out->resid16) {
        Ranges in, rr;
        act_ranges(x, 1, w->K, &in);
        if (out->resid) rr.emplace_back((uintptr_t)out->resid, (uintptr_t)(out->resid + w->N));
        if (out->resid16) rr.emplace_back((uintptr_t)out->resid16, (uintptr_t)(out->resid16 + w->N));
        rc = check_resid_overlap(rr, in);
        if (rc) return rc;
    }
    const GemvDesc d = make_desc(w, x, *out, 0);
    if (x->kind == TER_HIP_X_I16) return launch_x16(d, static_cast<hipStream_t>(stream));
    const long long total = (long long)d.n_strips * d.Ku;
    int n_wg = 0;
    const bool prologue = x->kind != TER_HIP_X_I8;
    // small GEMVs: strip mode, as for a plan (whole strips per workgroup,
    // the waves' partials added in LDS, no fix-up slots)
    bool strip_mode = false;
    rc = pick_strip_mode(total, d.n_strips, prologue, &strip_mode, &n_wg);
    if (rc) return rc;
    if (strip_mode) {
        const int part_off = (gemv_strip_part_off(w->K, d.stage32 != 0) + 15) / 16 * 16;
        const long long per_wg = (d.n_strips + n_wg - 1) / n_wg;
        const int lds_strip = part_off + (int)per_wg * kGemvWaves * kStripCols * 4;
        if (gemv_max_wg_per_cu(lds_strip) > 0) {
            const hipError_t e = launch_gemv_strips_single(d, d.n_strips, n_wg, lds_strip, part_off,
                                                           static_cast<hipStream_t>(stream));
            if (e != hipSuccess) return hip_fail(e, "gemv launch");
            return TER_HIP_OK;
        }
    }
    const int lds = gemv_t16_lds_bytes(w->K, d.stage32 != 0);
    rc = pick_wg(total, 0, lds, prologue, -1, &n_wg);
    if (rc) return rc;
    hipError_t e = launch_gemv(d, nullptr, nullptr, nullptr, total, n_wg, lds, -1, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "gemv launch");
    return TER_HIP_OK;
}

int ter_hip_mm_packed_dispatch(const int8_t* X, const float* scale_x_dev, const ter_hip_wpk_t* W, float* out,
                               int32_t K, int32_t N, void* stream) {
    if (!X || !scale_x_dev || !W || !out) return fail(TER_HIP_ERR_NULL, "null argument");
    if (W->K != K || W->N != N) return fail(TER_HIP_ERR_SHAPE, "K/N (%d,%d) do not match W (%d,%d)", K, N, W->K, W->N);
    ter_hip_act_t x{};
    x.data = X;
    x.kind = TER_HIP_X_I8;
    x.scale_dev = scale_x_dev;
    return ter_hip_gemv(W, &x, out, nullptr, stream);
}

int ter_hip_mm_packed_dispatch_f16(const int8_t* X, const float* scale_x_dev, const ter_hip_wpk_t* W, uint16_t* out,
                                   int32_t K, int32_t N, void* stream) {
    if (!X || !scale_x_dev || !W || !out) return fail(TER_HIP_ERR_NULL, "null argument");
    if (W->K != K || W->N != N) return fail(TER_HIP_ERR_SHAPE, "K/N (%d,%d) do not match W (%d,%d)", K, N, W->K, W->N);
    ter_hip_act_t x{};
    x.data = X;
    x.kind = TER_HIP_X_I8;
    x.scale_dev = scale_x_dev;
    const ter_hip_out_t o{nullptr, nullptr, out, nullptr, nullptr};
    return ter_hip_gemv_out(W, &x, &o, stream);
}

int ter_hip_mm_row(const int32_t* X, int32_t row, int32_t K, float x_scale, const ter_hip_wpk_t* W, int32_t N,
                   float* out, void* x_stage_dev, float* y_stage_dev, void* stream) {
    if (!X || !W || !out || !x_stage_dev || !y_stage_dev) return fail(TER_HIP_ERR_NULL, "null argument");
    if (row < 0) return fail(TER_HIP_ERR_SHAPE, "negative row");
    if (W->K != K || W->N != N) return fail(TER_HIP_ERR_SHAPE, "K/N (%d,%d) do not match W (%d,%d)", K, N, W->K, W->N);
    if (!aligned(x_stage_dev, 16)) return fail(TER_HIP_ERR_ALIGN, "x_stage_dev must be 16-byte aligned");
    const int32_t* xr = X + (size_t)row * (size_t)K;
    int32_t lo = 0, hi = 0;
    for (int k = 0; k < K; ++k) {
        lo = std::min(lo, xr[k]);
        hi = std::max(hi, xr[k]);
    }
    if (lo < -32768 || hi > 32767)
        return fail(TER_HIP_ERR_PAYLOAD, "X values [%d, %d] do not fit int16 (no CPU fallback)", lo, hi);
    const bool wide = lo < -128 || hi > 127;
    const size_t xbytes = (size_t)K * (wide ? 2 : 1);
    hipStream_t st = static_cast<hipStream_t>(stream);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    ter_hip_act_t x{};
    x.data = x_stage_dev;
    x.kind = wide ? TER_HIP_X_I16 : TER_HIP_X_I8;
    x.scale = x_scale;
    std::lock_guard<std::mutex> lk(g_stage_mu);
    MmRowStage* sg = nullptr;
    if (mm_row_stage(dev, xbytes, (size_t)N * sizeof(float), &sg)) {
        // pinned path: the row narrowed straight into page-locked memory, one
        // DMA up, the GEMV's outputs written into page-locked host memory
        if (wide)
            for (int k = 0; k < K; ++k) static_cast<int16_t*>(sg->x)[k] = (int16_t)xr[k];
        else
            for (int k = 0; k < K; ++k) static_cast<int8_t*>(sg->x)[k] = (int8_t)xr[k];
        e = hipMemcpyAsync(x_stage_dev, sg->x, xbytes, hipMemcpyHostToDevice, st);
        if (e != hipSuccess) return hip_fail(e, "X upload");
        int rc = ter_hip_gemv(W, &x, sg->y_dev, nullptr, stream);
        if (rc) return rc;
        e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, "mm_row synchronize");
        std::memcpy(out, sg->y, (size_t)N * sizeof(float));
        return TER_HIP_OK;
    }
    // no pinned staging: pageable copies through the caller's device buffers
    std::vector<int8_t> xb;
    std::vector<int16_t> xw;
    try {
        if (wide)
            xw.assign(xr, xr + K);
        else
            xb.assign(xr, xr + K);
    } catch (...) {
        return fail(TER_HIP_ERR_ALLOC, "host staging allocation");
    }
    e = wide ? hipMemcpyAsync(x_stage_dev, xw.data(), xbytes, hipMemcpyHostToDevice, st)
             : hipMemcpyAsync(x_stage_dev, xb.data(), xbytes, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return hip_fail(e, "X upload");
    int rc = ter_hip_gemv(W, &x, y_stage_dev, nullptr, stream);
    if (rc) return rc;
    e = hipMemcpyAsync(out, y_stage_dev, (size_t)N * sizeof(float), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "y download");
    return TER_HIP_OK;
}

int ter_hip_mm_row_blocked(const int32_t* X, int32_t row, int32_t K, float x_scale, const ter_hip_wpk_t* W, int32_t N,
                           const float* block_scales_dev, int64_t block_size, float* out, void* x_stage_dev,
                           float* y_stage_dev, void* stream) {
    if (!X || !W || !out || !x_stage_dev || !y_stage_dev || !block_scales_dev)
        return fail(TER_HIP_ERR_NULL, "null argument");
    int rc = check_wpk(W);
    if (rc) return rc;
    if (row < 0) return fail(TER_HIP_ERR_SHAPE, "negative row");
    if (W->K != K || W->N != N) return fail(TER_HIP_ERR_SHAPE, "K/N (%d,%d) do not match W (%d,%d)", K, N, W->K, W->N);
    if (block_size < 1) return fail(TER_HIP_ERR_SHAPE, "block_size %lld < 1", (long long)block_size);
    if (!aligned(x_stage_dev, 16) || !aligned(y_stage_dev, 4) || !aligned(block_scales_dev, 4))
        return fail(TER_HIP_ERR_ALIGN, "misaligned staging or scale buffer");
    const int32_t* xr = X + (size_t)row * (size_t)K;
    int32_t lo = 0, hi = 0;
    for (int k = 0; k < K; ++k) {
        lo = std::min(lo, xr[k]);
        hi = std::max(hi, xr[k]);
    }
    if (lo < -32768 || hi > 32767)
        return fail(TER_HIP_ERR_PAYLOAD, "X values [%d, %d] do not fit int16 (no CPU fallback)", lo, hi);
    const long long amax = std::max(-(long long)lo, (long long)hi);
    if (amax * (long long)W->mag >= (1LL << 29))
        return fail(TER_HIP_ERR_PAYLOAD, "|x| * m = %lld * %d reaches 2^29: the double terms would round", amax, W->mag);
    std::vector<int16_t> xw;
    try {
        xw.assign(xr, xr + K);
    } catch (...) {
        return fail(TER_HIP_ERR_ALLOC, "host staging allocation");
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(x_stage_dev, xw.data(), (size_t)K * 2, hipMemcpyHostToDevice, st);
    if (e == hipSuccess)
        e = launch_mm_row_blocked(W->data, K, N, W->mag, static_cast<const int16_t*>(x_stage_dev), block_scales_dev,
                                  (long long)block_size, x_scale, y_stage_dev, st);
    if (e == hipSuccess) e = hipMemcpyAsync(out, y_stage_dev, (size_t)N * sizeof(float), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "blocked mm_row");
    return TER_HIP_OK;
}

// A strided strip-mode list whose GEMVs all read one activation vector (same
// pointers, kind, K, norm) with no quantized copies requested, whose tile
// streams follow each other in memory in list order, and where no
// workgroup's range spans more than two GEMVs: the descriptor the kernel
// takes as its argument (the activation, the first stream's base, strip0 0,
// the list's strip count).  Returns false for any other list.
bool shared_plan_desc(const std::vector<GemvDesc>& ds, long long strips, int n_wg, GemvDesc* out) {
    const GemvDesc& a = ds[0];
    // every workgroup's strips [S g / n_wg, S (g + 1) / n_wg) within two GEMVs
    size_t di = 0;
    for (int g = 0; g < n_wg; ++g) {
        const long long s0 = strips * g / n_wg, s1 = strips * (g + 1) / n_wg;
        if (s0 >= s1) continue;
        while (di + 1 < ds.size() && ds[di + 1].strip0 <= s0) ++di;
        size_t dl = di;
        while (dl + 1 < ds.size() && ds[dl + 1].strip0 <= s1 - 1) ++dl;
        if (dl > di + 1) return false;
    }
    for (const GemvDesc& d : ds) {
        if (d.x != a.x || d.x_kind != a.x_kind || d.up != a.up || d.gamma != a.gamma || d.eps != a.eps ||
            d.K != a.K || d.Ku != a.Ku || d.stage32 != a.stage32 || d.xq_out || d.xs_out || d.x_scale_dev)
            return false;
        if (d.w != a.w + d.strip0 * (long long)a.Ku * kTileBytes) return false;
    }
    GemvDesc s{};
    s.w = a.w;
    s.x = a.x;
    s.up = a.up;
    s.gamma = a.gamma;
    s.eps = a.eps;
    s.K = a.K;
    s.Ku = a.Ku;
    s.N = a.N;
    s.stage32 = a.stage32;
    s.x_kind = a.x_kind;
    s.x_scale = a.x_scale;
    s.w_mag = a.w_mag;
    s.strip0 = 0;
    s.n_strips = (int32_t)strips;
    *out = s;
    return true;
}

int ter_hip_plan_create(ter_hip_plan_t** plan, const ter_hip_gemv_item_t* items, int32_t n, int32_t wg_per_cu) {
    if (!plan || !items) return fail(TER_HIP_ERR_NULL, "null plan or items");
    *plan = nullptr;
    if (n < 1) return fail(TER_HIP_ERR_SHAPE, "empty work list");
    std::vector<GemvDesc> ds((size_t)n);
    std::vector<long long> starts((size_t)n), strip_starts((size_t)n);
    long long tile = 0, strips = 0;
    uint64_t bytes = 0, macs = 0;
    int lds = 0;        // the stream-K kernel's (staging, slots and output buffers)
    int lds_stage = 0;  // the staging area, all the strip-mode kernel needs beside its partial sums
    Ranges resid, inputs;
    for (int i = 0; i < n; ++i) {
        const ter_hip_gemv_item_t& it = items[i];
        int rc = check_wpk(it.w);
        if (rc) return rc;
        rc = check_act(&it.x, 1);
        if (rc) return rc;
        if (it.x.kind == TER_HIP_X_I16)
            return fail(TER_HIP_ERR_PAYLOAD, "item %d: int16 activations run as single GEMVs only", i);
        const ter_hip_out_t o{it.y, it.acc, it.y16, it.resid, it.resid16, it.silu};
        rc = check_out(&o);
        if (rc) return rc;
        for (int k = 0; k < i; ++k)
            if (items[k].w->fix == it.w->fix)
                return fail(TER_HIP_ERR_CONFLICT, "weight of item %d repeats item %d", i, k);
        if (it.resid) resid.emplace_back((uintptr_t)it.resid, (uintptr_t)(it.resid + it.w->N));
        if (it.resid16) resid.emplace_back((uintptr_t)it.resid16, (uintptr_t)(it.resid16 + it.w->N));
        act_ranges(&it.x, 1, it.w->K, &inputs);
        ds[(size_t)i] = make_desc(it.w, &it.x, o, tile);
        ds[(size_t)i].strip0 = strips;
        starts[(size_t)i] = tile;
        strip_starts[(size_t)i] = strips;
        tile += (long long)ds[(size_t)i].n_strips * ds[(size_t)i].Ku;
        strips += ds[(size_t)i].n_strips;
        const int lb = gemv_t16_lds_bytes(it.w->K, ds[(size_t)i].stage32 != 0);
        if (lb > lds) lds = lb;
        const int ls = gemv_strip_part_off(it.w->K, ds[(size_t)i].stage32 != 0);  // the staging area alone
        if (ls > lds_stage) lds_stage = ls;
        bytes += (uint64_t)it.w->K * (uint64_t)it.w->N / 4 + (uint64_t)it.w->K * act_bytes(it.x.kind) +
                 (uint64_t)it.w->N * out_bytes(o);
        macs += (uint64_t)it.w->K * (uint64_t)it.w->N;
    }
    int rc = check_resid_overlap(resid, inputs);
    if (rc) return rc;
    int n_wg = 0;
    bool prologue = false;
    for (int i = 0; i < n; ++i) prologue = prologue || items[i].x.kind != TER_HIP_X_I8;
    const int vec_kind = gemv_vec_kind(items, n);
    bool strip_mode = false;
    int part_off = 0;
    if (wg_per_cu <= 0) {
        rc = pick_strip_mode(tile, strips, prologue, &strip_mode, &n_wg);
        if (rc) return rc;
    }
    bool strided = false;
    if (strip_mode) {
        part_off = (lds_stage + 15) / 16 * 16;
        strided = vec_kind >= 0;
        for (const GemvDesc& d : ds) strided = strided && gemv_strided_ok(vec_kind, d.K, d.stage32 != 0);
        const int waves = strided ? gemv_strided_waves(vec_kind) : kGemvWaves;
        const long long per_wg = (strips + n_wg - 1) / n_wg;
        const int lds_strip = part_off + (int)per_wg * waves * kStripCols * 4;
        if (gemv_max_wg_per_cu(lds_strip) > 0)
            lds = lds_strip;
        else
            strip_mode = false;  // partial sums do not fit beside the activations: stream-K
    }
    if (!strip_mode) {
        rc = pick_wg(tile, wg_per_cu, lds, prologue, vec_kind, &n_wg);
        if (rc) return rc;
    }
    ter_hip_plan* p = new (std::nothrow) ter_hip_plan();
    if (!p) return fail(TER_HIP_ERR_ALLOC, "plan allocation");
    GemvDesc shared_desc{};
    const bool shared = strip_mode && strided && shared_plan_desc(ds, strips, n_wg, &shared_desc);
    if (strip_mode) {
        for (size_t i = 0; i < ds.size(); ++i) ds[i].self = (int32_t)i;
        rc = upload_plan(p, ds, strip_starts, strips, n_wg, nullptr, shared ? 2 : 1);
    } else {
        const std::vector<long long> ranges = plan_ranges(ds, starts, tile, n_wg);
        rc = upload_plan(p, ds, starts, tile, n_wg, &ranges);
    }
    if (rc) {
        delete p;
        return rc;
    }
    p->n = n;
    p->total = strip_mode ? strips : tile;
    p->strip_mode = strip_mode;
    p->part_off = part_off;
    p->strided = strip_mode && strided;
    p->shared = shared;
    p->shared_desc = shared_desc;
    p->n_wg = n_wg;
    p->lds_bytes = lds;
    p->vec_kind = vec_kind;
    p->bytes = bytes;
    p->macs = macs;
    *plan = p;
    return TER_HIP_OK;
}

int ter_hip_plan_launch(const ter_hip_plan_t* plan, void* stream) {
    if (!plan) return fail(TER_HIP_ERR_NULL, "null plan");
    hipError_t e;
    if (plan->gemm && plan->lds) {
        GemmDesc none{};
        e = launch_gemm_lds(none, static_cast<const GemmDesc*>(plan->descs_dev), plan->blocks_dev, plan->ranges_dev,
                            plan->n_blocks, plan->n_wg, plan->mb, static_cast<hipStream_t>(stream));
    } else if (plan->gemm && plan->stream) {
        GemmDesc none{};
        e = launch_gemm_stream(none, static_cast<const GemmDesc*>(plan->descs_dev), plan->first_dev, plan->total,
                               plan->n_wg, plan->lds_bytes, plan->vec, static_cast<hipStream_t>(stream));
    } else if (plan->gemm) {
        GemmDesc none{};
        e = launch_gemm_list(none, static_cast<const GemmDesc*>(plan->descs_dev), plan->first_dev, plan->total,
                             plan->n_wg, plan->mb, plan->vec, static_cast<hipStream_t>(stream));
    } else {
        GemvDesc none{};
        if (plan->strip_mode)
            e = launch_gemv_strips(static_cast<const GemvDesc*>(plan->descs_dev),
                                   static_cast<const GemvDesc*>(plan->wg_desc_dev), plan->total,
                                   plan->n_wg, plan->lds_bytes, plan->part_off, plan->vec_kind, plan->strided,
                                   plan->shared ? &plan->shared_desc : nullptr, static_cast<hipStream_t>(stream));
        else
            e = launch_gemv(none, static_cast<const GemvDesc*>(plan->descs_dev), plan->first_dev,
                            plan->wg_ranges_dev, plan->total, plan->n_wg, plan->lds_bytes, plan->vec_kind,
                            static_cast<hipStream_t>(stream));
    }
    if (e != hipSuccess) return hip_fail(e, "plan launch");
    return TER_HIP_OK;
}

int ter_hip_plan_mode(const ter_hip_plan_t* plan, int32_t* mode) {
    if (!plan || !mode) return fail(TER_HIP_ERR_NULL, "null plan or mode");
    *mode = plan->gemm ? 0
                       : (plan->strip_mode ? TER_HIP_PLAN_STRIPS : 0) | (plan->strided ? TER_HIP_PLAN_STRIDED : 0) |
                             (plan->shared ? TER_HIP_PLAN_SHARED : 0);
    return TER_HIP_OK;
}

int ter_hip_plan_stats(const ter_hip_plan_t* plan, uint64_t* bytes, uint64_t* macs, int32_t* n_wg) {
    if (!plan) return fail(TER_HIP_ERR_NULL, "null plan");
    if (bytes) *bytes = plan->bytes;
    if (macs) *macs = plan->macs;
    if (n_wg) *n_wg = plan->n_wg;
    return TER_HIP_OK;
}

void ter_hip_plan_destroy(ter_hip_plan_t* plan) {
    if (!plan) return;
    (void)hipFree(plan->descs_dev);
    delete plan;
}

int ter_hip_rmsnorm_quant(const void* x, int32_t kind, const uint16_t* gamma, float eps, int32_t M, int32_t K,
                          int8_t* q, float* scale_out, void* stream) {
    if (!x || !gamma || !q || !scale_out) return fail(TER_HIP_ERR_NULL, "null argument");
    if (!is_rms(kind)) return fail(TER_HIP_ERR_PAYLOAD, "kind %d is not an RMSNorm kind", kind);
    if (M < 1 || K < 1 || K > TER_HIP_K_MAX || M > 65535) return fail(TER_HIP_ERR_SHAPE, "M=%d K=%d out of range", M, K);
    if (!aligned(x, kind == TER_HIP_X_F32_RMS ? 4 : 2) || !aligned(gamma, 2))
        return fail(TER_HIP_ERR_ALIGN, "x or gamma misaligned");
    if (!(eps >= 0.f)) return fail(TER_HIP_ERR_SHAPE, "RMSNorm eps must be >= 0");
    if (kind == TER_HIP_X_RELU2_RMS) return fail(TER_HIP_ERR_PAYLOAD, "relu2 rows: use ter_hip_relu2_rmsnorm_quant");
    hipError_t e = launch_rmsnorm_quant_rows(x, nullptr, kind, gamma, eps, M, K, q, scale_out,
                                             static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "rmsnorm quant launch");
    return TER_HIP_OK;
}

int ter_hip_relu2_rmsnorm_quant(const uint16_t* gate, const uint16_t* up, const uint16_t* gamma, float eps, int32_t M,
                                int32_t F, int8_t* q, float* scale_out, void* stream) {
    if (!gate || !up || !gamma || !q || !scale_out) return fail(TER_HIP_ERR_NULL, "null argument");
    if (M < 1 || F < 1 || F > TER_HIP_K_MAX || M > 65535) return fail(TER_HIP_ERR_SHAPE, "M=%d F=%d out of range", M, F);
    if (!aligned(gate, 2) || !aligned(up, 2) || !aligned(gamma, 2))
        return fail(TER_HIP_ERR_ALIGN, "gate, up or gamma misaligned");
    if (!(eps >= 0.f)) return fail(TER_HIP_ERR_SHAPE, "RMSNorm eps must be >= 0");
    hipError_t e = launch_rmsnorm_quant_rows(gate, up, TER_HIP_X_RELU2_RMS, gamma, eps, M, F, q, scale_out,
                                             static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "relu2 rmsnorm quant launch");
    return TER_HIP_OK;
}

int ter_hip_quant_int8(const float* x, int32_t M, int32_t K, int8_t* q, float* scale_out, void* stream) {
    if (!x || !q || !scale_out) return fail(TER_HIP_ERR_NULL, "null argument");
    if (M < 1 || K < 1 || K > TER_HIP_K_MAX || M > 65535) return fail(TER_HIP_ERR_SHAPE, "M=%d K=%d out of range", M, K);
    if (!aligned(x, 4)) return fail(TER_HIP_ERR_ALIGN, "fp32 X misaligned");
    hipError_t e = launch_quant_rows(x, M, K, q, scale_out, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "quant launch");
    return TER_HIP_OK;
}

int ter_hip_gemm(const ter_hip_wpk_t* w, const ter_hip_act_t* x, int32_t M, float* y, int32_t* acc, void* stream) {
    const ter_hip_out_t o{y, acc, nullptr, nullptr, nullptr};
    return ter_hip_gemm_out(w, x, M, &o, stream);
}

// ter_hip_gemm_out with the quantized rows of fp32 / fp16 activations in
// q_ws [M][K] and s_ws [M] (unused for int8 X).
static int gemm_out_ws(const ter_hip_wpk_t* w, const ter_hip_act_t* x, int32_t M, const ter_hip_out_t* out,
                       int8_t* q_ws, float* s_ws, void* stream) {
    int rc = check_wpk(w);
    if (rc) return rc;
    if (M < 1 || M > TER_HIP_M_MAX) return fail(TER_HIP_ERR_SHAPE, "M=%d out of range [1,%d]", M, TER_HIP_M_MAX);
    rc = check_act(x, M);
    if (rc) return rc;
    if (gemv_only_kind(x->kind))  // the GEMM kernels take int8 rows from the batched quantizers
        return fail(TER_HIP_ERR_PAYLOAD, "activation kind %d runs as single GEMVs and GEMV work lists only", x->kind);
    rc = check_out(out);
    if (rc) return rc;
    if (out->resid16) return fail(TER_HIP_ERR_PAYLOAD, "fp16 residual outputs: GEMVs only");
    if (out->silu) return fail(TER_HIP_ERR_PAYLOAD, "silu outputs: GEMVs only");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int8_t* xq = static_cast<const int8_t*>(x->data);
    const float* xs = x->scale_dev;
    if (out->resid) {  // the GEMM reads int8 rows: X itself or the q_out workspace
        const int8_t* xr = x->kind == TER_HIP_X_I8 ? xq : q_ws;
        const size_t mk = (size_t)M * (size_t)w->K;
        rc = check_resid_overlap({{(uintptr_t)out->resid, (uintptr_t)(out->resid + (size_t)M * w->N)}},
                                 {{(uintptr_t)xr, (uintptr_t)(xr + mk)}});
        if (rc) return rc;
    }
    if (x->kind != TER_HIP_X_I8) {
        if (!q_ws || !s_ws)
            return fail(TER_HIP_ERR_NULL, "fp32/fp16 batched X needs q_out and scale_out workspaces");
        if (x->kind == TER_HIP_X_F32)
            rc = ter_hip_quant_int8(static_cast<const float*>(x->data), M, w->K, q_ws, s_ws, stream);
        else if (x->kind == TER_HIP_X_RELU2_RMS)
            rc = ter_hip_relu2_rmsnorm_quant(static_cast<const uint16_t*>(x->data), x->up, x->gamma, x->eps, M, w->K,
                                             q_ws, s_ws, stream);
        else
            rc = ter_hip_rmsnorm_quant(x->data, x->kind, x->gamma, x->eps, M, w->K, q_ws, s_ws, stream);
        if (rc) return rc;
        xq = q_ws;
        xs = s_ws;
    }
    if (M > kRingRows && ring_rows_ok(xq, w->K)) {
        // pieces of kRingRows rows, one LDS-ring launch each
        const int mb = gemm_mb_of(kRingRows), lbs = gemm_lds_strips_per_block(mb);
        for (int r0 = 0; r0 < M; r0 += kRingRows) {
            const int m = std::min(kRingRows, M - r0);
            const GemmDesc d = make_gemm_desc(w, xq + (size_t)r0 * w->K, xs + r0, m, out_rows(*out, r0, w->N), 0,
                                              kWaves * gemm_strips_per_wave(mb), 0);
            const int nb = (d.n_strips + lbs - 1) / lbs;
            int n_wg = 0;
            rc = pick_lds_wg(nb, mb, &n_wg);
            if (rc) return rc;
            const hipError_t e = launch_gemm_lds(d, nullptr, nullptr, nullptr, nb, n_wg, mb, st);
            if (e != hipSuccess) return hip_fail(e, "gemm launch");
        }
        return TER_HIP_OK;
    }
    const int mb = gemm_mb_of(M);
    const GemmDesc d = make_gemm_desc(w, xq, xs, M, *out, 0, kWaves * gemm_strips_per_wave(mb), 0);
    int n_wg = 0;
    hipError_t e;
    const int slds = gemm_stream_lds_want(M, w->K);
    const int lbs = gemm_vec_ok(d) ? gemm_lds_strips_per_block(mb) : 0;
    if (gemm_stream_item_fits(M, w->K, slds)) {
        const long long tiles = (long long)d.n_strips * d.Ku;
        rc = pick_stream_wg(tiles, slds, 0, &n_wg);
        if (rc) return rc;
        e = launch_gemm_stream(d, nullptr, nullptr, tiles, n_wg, slds, gemm_vec_ok(d), st);
    } else if (lbs > 0) {
        const int nb = (d.n_strips + lbs - 1) / lbs;
        rc = pick_lds_wg(nb, mb, &n_wg);
        if (rc) return rc;
        e = launch_gemm_lds(d, nullptr, nullptr, nullptr, nb, n_wg, mb, st);
    } else {
        rc = pick_gemm_wg(d.n_blocks, mb, 0, &n_wg);
        if (rc) return rc;
        e = launch_gemm_list(d, nullptr, nullptr, d.n_blocks, n_wg, mb, gemm_vec_ok(d), st);
    }
    if (e != hipSuccess) return hip_fail(e, "gemm launch");
    return TER_HIP_OK;
}

int ter_hip_gemm_out(const ter_hip_wpk_t* w, const ter_hip_act_t* x, int32_t M, const ter_hip_out_t* out,
                     void* stream) {
    if (!x) return fail(TER_HIP_ERR_NULL, "null activation");
    return gemm_out_ws(w, x, M, out, x->q_out, x->scale_out, stream);
}

int ter_hip_gemm_out_static(const ter_hip_wpk_t* w, const ter_hip_act_t* x, int32_t M, const ter_hip_out_t* out,
                            void* stream) {
    int rc = check_wpk(w);
    if (rc) return rc;
    if (!x) return fail(TER_HIP_ERR_NULL, "null activation");
    if (x->q_out || x->scale_out)
        return fail(TER_HIP_ERR_SHAPE, "ter_hip_gemm_out_static takes no q_out / scale_out (its workspace is static)");
    if (M < 1 || M > TER_HIP_M_MAX) return fail(TER_HIP_ERR_SHAPE, "M=%d out of range [1,%d]", M, TER_HIP_M_MAX);
    if ((long long)M * w->K > (long long)TER_HIP_STATIC_Q_MAX)
        return fail(TER_HIP_ERR_SHAPE, "M*K = %lld exceeds the static workspace (%d bytes)", (long long)M * w->K,
                    TER_HIP_STATIC_Q_MAX);
    if (x->kind == TER_HIP_X_I8 || x->kind == TER_HIP_X_I16)  // no workspace used (int16 rows are refused there)
        return gemm_out_ws(w, x, M, out, nullptr, nullptr, stream);
    unsigned char* ws = nullptr;
    rc = scratch_of_current_device(&ws);
    if (rc) return rc;
    return gemm_out_ws(w, x, M, out, reinterpret_cast<int8_t*>(ws), reinterpret_cast<float*>(ws + kScratchScaleOff),
                       stream);
}

int ter_hip_gemm_plan_create(ter_hip_plan_t** plan, const ter_hip_gemm_item_t* items, int32_t n,
                             int32_t wg_per_cu) {
    if (!plan || !items) return fail(TER_HIP_ERR_NULL, "null plan or items");
    *plan = nullptr;
    if (n < 1) return fail(TER_HIP_ERR_SHAPE, "empty work list");
    std::vector<GemmDesc> ds((size_t)n);
    long long blocks = 0;
    uint64_t bytes = 0, macs = 0;
    int max_m = 1;
    bool vec = true;
    Ranges resid, inputs;
    for (int i = 0; i < n; ++i) {
        const ter_hip_gemm_item_t& it = items[i];
        int rc = check_wpk(it.w);
        if (rc) return rc;
        if (!it.x || !it.x_scale_dev) return fail(TER_HIP_ERR_NULL, "item %d: null X or X scales", i);
        if (it.M < 1 || it.M > TER_HIP_M_MAX)
            return fail(TER_HIP_ERR_SHAPE, "item %d: M=%d out of range [1,%d]", i, it.M, TER_HIP_M_MAX);
        const ter_hip_out_t o{it.y, it.acc, it.y16, it.resid, nullptr, nullptr};
        rc = check_out(&o);
        if (rc) return rc;
        if (it.resid16) return fail(TER_HIP_ERR_PAYLOAD, "item %d: fp16 residual outputs: GEMVs only", i);
        if (it.silu) return fail(TER_HIP_ERR_PAYLOAD, "item %d: silu outputs: GEMVs only", i);
        if (it.resid) resid.emplace_back((uintptr_t)it.resid, (uintptr_t)(it.resid + (size_t)it.M * it.w->N));
        inputs.emplace_back((uintptr_t)it.x, (uintptr_t)(it.x + (size_t)it.M * it.w->K));
        if (it.M > max_m) max_m = it.M;
    }
    if (int rc = check_resid_overlap(resid, inputs)) return rc;
    // Items with more than kRingRows rows become pieces of kRingRows rows
    // (one descriptor each) when every X qualifies for the LDS-ring kernel.
    bool ring_all = true;
    for (int i = 0; i < n; ++i) ring_all = ring_all && ring_rows_ok(items[i].x, items[i].w->K);
    const int rows = max_m > kRingRows && ring_all ? kRingRows : TER_HIP_M_MAX;
    const int mb = gemm_mb_of(std::min(max_m, rows));  // one row-block count (and block width) per launch
    const int per_block = kWaves * gemm_strips_per_wave(mb);
    long long tiles = 0;
    ds.clear();
    std::vector<long long> block_starts, tile_starts;
    std::vector<int> piece0;  // first descriptor of each item (its pieces follow)
    for (int i = 0; i < n; ++i) {
        const ter_hip_gemm_item_t& it = items[i];
        const ter_hip_out_t o{it.y, it.acc, it.y16, it.resid, nullptr, nullptr};
        piece0.push_back((int)ds.size());
        for (int r0 = 0; r0 < it.M; r0 += rows) {
            const int m = std::min(rows, it.M - r0);
            const GemmDesc d = make_gemm_desc(it.w, it.x + (size_t)r0 * it.w->K, it.x_scale_dev + r0, m,
                                              out_rows(o, r0, it.w->N), blocks, per_block, tiles);
            ds.push_back(d);
            block_starts.push_back(blocks);
            tile_starts.push_back(tiles);
            blocks += d.n_blocks;
            tiles += (long long)d.n_strips * d.Ku;
            vec = vec && gemm_vec_ok(d);
        }
        bytes += (uint64_t)it.w->K * (uint64_t)it.w->N / 4 + (uint64_t)it.M * it.w->K +
                 (uint64_t)it.M * it.w->N * out_bytes(o);
        macs += (uint64_t)it.M * (uint64_t)it.w->K * (uint64_t)it.w->N;
    }
    n = (int)ds.size();
    int n_wg = 0;
    int slds = 0;  // the streaming kernel's LDS: the most any item wants
    for (int i = 0; i < n; ++i) slds = std::max(slds, gemm_stream_lds_want(ds[(size_t)i].M, ds[(size_t)i].K));
    bool stream = true;
    for (int i = 0; i < n && stream; ++i) stream = gemm_stream_item_fits(ds[(size_t)i].M, ds[(size_t)i].K, slds);
    // The LDS-ring kernel where the streamed one does not fit, and also
    // where the list holds at least kRingMinBlocksPerCu of its blocks per CU:
    // dealt out by list scheduling it beats the streamed kernel on large
    // lists (C4 at 8 rows: 95.3 against 101.7 us; at 4 rows 88.7 against
    // 95.5 us), while a short list needs the streamed kernel's split of K
    // to fill the GPU (a ring block covers all of K for its strips).
    int lbs = vec ? gemm_lds_strips_per_block(mb) : 0;
    if (lbs > 0 && stream) {
        long long ring_blocks = 0;
        for (int i = 0; i < n; ++i) ring_blocks += (ds[(size_t)i].n_strips + lbs - 1) / lbs;
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return fail(TER_HIP_ERR_HIP, "hipGetDevice");
        const int cus = device_cu_count(dev);
        if (cus <= 0) return fail(TER_HIP_ERR_HIP, "cannot query CU count");
        if (ring_blocks < (long long)cus * kRingMinBlocksPerCu) lbs = 0;
    }
    ter_hip_plan* p = new (std::nothrow) ter_hip_plan();
    if (!p) return fail(TER_HIP_ERR_ALLOC, "plan allocation");
    int rc;
    if (lbs > 0) {
        // LDS-ring kernel: blocks of lbs strips, dealt out by list scheduling.
        // The pieces of an item read the same weights: their blocks of one
        // strip range are listed next to each other, so the scheduler hands
        // them out together to neighbouring workgroups on one XCD (equal cost,
        // adjacent in the stable order) and the pieces after the first find
        // the weight runs in that XCD's L2 instead of reading them again.
        std::vector<GemmBlock> bl;
        piece0.push_back(n);
        for (size_t it = 0; it + 1 < piece0.size(); ++it) {
            const int d0 = piece0[it], d1 = piece0[it + 1];
            for (int st = 0; st < ds[(size_t)d0].n_strips; st += lbs)
                for (int i = d0; i < d1; ++i) bl.push_back(GemmBlock{i, st});
        }
        rc = pick_lds_wg((long long)bl.size(), mb, &n_wg);
        if (!rc) rc = upload_lds_plan(p, ds, bl, lbs, n_wg);
    } else {
        rc = stream ? pick_stream_wg(tiles, slds, wg_per_cu, &n_wg) : pick_gemm_wg(blocks, mb, wg_per_cu, &n_wg);
        if (!rc) rc = stream ? upload_plan(p, ds, tile_starts, tiles, n_wg) : upload_plan(p, ds, block_starts, blocks, n_wg);
    }
    if (rc) {
        delete p;
        return rc;
    }
    p->lds = lbs > 0;
    p->n = n;
    p->gemm = true;
    p->stream = stream;
    p->total = stream ? tiles : blocks;
    p->lds_bytes = stream ? slds : 0;

    p->n_wg = n_wg;
    p->mb = mb;
    p->vec = vec;
    p->bytes = bytes;
    p->macs = macs;
    *plan = p;
    return TER_HIP_OK;
}

int ter_hip_rmsnorm_f16(const float* x, const uint16_t* gamma, float eps, int32_t M, int32_t H, uint16_t* y,
                        void* stream) {
    if (!x || !gamma || !y) return fail(TER_HIP_ERR_NULL, "null argument");
    if (M < 1 || M > 65535 || H < 1 || H > TER_HIP_K_MAX) return fail(TER_HIP_ERR_SHAPE, "M=%d H=%d out of range", M, H);
    if (!aligned(x, 4) || !aligned(gamma, 2) || !aligned(y, 2)) return fail(TER_HIP_ERR_ALIGN, "x, gamma or y misaligned");
    if (!(eps >= 0.f)) return fail(TER_HIP_ERR_SHAPE, "RMSNorm eps must be >= 0");
    hipError_t e = launch_rmsnorm_f16_rows(x, gamma, eps, M, H, y, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "rmsnorm f16 launch");
    return TER_HIP_OK;
}

namespace {

// Workgroups of an lm_head launch: resident workgroups per CU times the CU
// count, raised so no wave's row range spans 2^31 bytes (its buffer
// resource), capped by the row pairs.
int pick_lm_head_wg(int H, int V, int* n_wg) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    const int cus = device_cu_count(dev);
    if (cus <= 0) return fail(TER_HIP_ERR_HIP, "cannot query CU count");
    const int fit = lm_head_max_wg_per_cu(H);
    if (fit <= 0) return fail(TER_HIP_ERR_SHAPE, "lm_head workgroup does not fit a CU (H=%d)", H);
    long long g = (long long)cus * fit;
    const long long bytes = (long long)V * H * 2;
    const long long min_g = bytes / ((1LL << 30) * 4) + 1;  // 4 waves per workgroup, < 1 GiB per wave
    if (g < min_g) g = min_g;
    const long long pairs = ((long long)V + 1) / 2;
    if (g > pairs) g = pairs;
    if (g < 1) g = 1;
    *n_wg = (int)g;
    return TER_HIP_OK;
}

int check_lm_head(const uint16_t* emb, int H, int V) {
    if (!emb) return fail(TER_HIP_ERR_NULL, "null token_embd");
    if (H < 1 || H > TER_HIP_K_MAX || V < 1 || V > TER_HIP_N_MAX)
        return fail(TER_HIP_ERR_SHAPE, "H=%d V=%d out of range", H, V);
    if (H % 2 == 0 && !aligned(emb, 4)) return fail(TER_HIP_ERR_ALIGN, "token_embd must be 4-byte aligned");
    if (!aligned(emb, 2)) return fail(TER_HIP_ERR_ALIGN, "token_embd misaligned");
    return TER_HIP_OK;
}

}  // namespace

int ter_hip_lm_head_f16(const uint16_t* x_norm, const uint16_t* token_embd, uint16_t* logits, int32_t H, int32_t V,
                        void* stream) {
    if (!x_norm || !logits) return fail(TER_HIP_ERR_NULL, "null argument");
    int rc = check_lm_head(token_embd, H, V);
    if (rc) return rc;
    if (!aligned(x_norm, H % 2 == 0 ? 4 : 2) || !aligned(logits, 2)) return fail(TER_HIP_ERR_ALIGN, "x_norm or logits misaligned");
    int n_wg = 0;
    rc = pick_lm_head_wg(H, V, &n_wg);
    if (rc) return rc;
    hipError_t e = launch_lm_head(nullptr, nullptr, nullptr, 0.f, x_norm, token_embd, H, V, nullptr, logits, nullptr, nullptr,
                                  nullptr, n_wg, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "lm_head launch");
    return TER_HIP_OK;
}

static int argmax_any(const uint16_t* logits, int32_t N, int32_t* out_idx, uint64_t* state, int32_t* pos_advance,
                      void* stream) {
    if (!logits || !out_idx || !state) return fail(TER_HIP_ERR_NULL, "null argument");
    if (N < 1 || N > TER_HIP_N_MAX) return fail(TER_HIP_ERR_SHAPE, "N=%d out of range", N);
    if (!aligned(logits, 2) || !aligned(out_idx, 4) || !aligned(state, 8) || !aligned(pos_advance, 4))
        return fail(TER_HIP_ERR_ALIGN, "misaligned argument");
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    const int cus = device_cu_count(dev);
    if (cus <= 0) return fail(TER_HIP_ERR_HIP, "cannot query CU count");
    // one round per thread: 8 logits each (16-byte aligned logits), else 4
    const long long per_wg = aligned(logits, 16) ? 8 * 256 : 1024;
    long long g = ((long long)N + per_wg - 1) / per_wg;
    if (g > cus) g = cus;
    e = launch_argmax_f16(logits, N, out_idx, reinterpret_cast<unsigned long long*>(state), pos_advance, (int)g,
                          static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "argmax launch");
    return TER_HIP_OK;
}

int ter_hip_argmax_f16(const uint16_t* logits, int32_t N, int32_t* out_idx, uint64_t* state, void* stream) {
    return argmax_any(logits, N, out_idx, state, nullptr, stream);
}

int ter_hip_argmax_f16_step(const uint16_t* logits, int32_t N, int32_t* out_idx, uint64_t* state,
                            int32_t* pos_advance, void* stream) {
    if (!pos_advance) return fail(TER_HIP_ERR_NULL, "null argument");
    return argmax_any(logits, N, out_idx, state, pos_advance, stream);
}

int ter_hip_embed_f16(const uint16_t* token_embd, int32_t V, int32_t H, const int32_t* token_dev, float* hidden,
                      void* stream) {
    if (!token_embd || !token_dev || !hidden) return fail(TER_HIP_ERR_NULL, "null argument");
    if (V < 1 || H < 1 || V > TER_HIP_N_MAX || H > TER_HIP_K_MAX) return fail(TER_HIP_ERR_SHAPE, "V=%d H=%d", V, H);
    if (!aligned(token_embd, 2) || !aligned(token_dev, 4) || !aligned(hidden, 4))
        return fail(TER_HIP_ERR_ALIGN, "misaligned argument");
    hipError_t e = launch_embed_f16(token_embd, V, H, token_dev, hidden, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "embedding launch");
    return TER_HIP_OK;
}

// The fused tail over an fp32 (hidden) or fp16 (hidden16) residual stream.
static int lm_head_argmax_any(const float* hidden, const uint16_t* hidden16, const uint16_t* gamma, float eps,
                              const uint16_t* token_embd, int32_t H, int32_t V, uint16_t* x_norm_out,
                              uint16_t* logits_out, int32_t* token_out, uint64_t* state, int32_t* pos_advance,
                              void* stream) {
    if ((!hidden && !hidden16) || !gamma || !token_out || !state) return fail(TER_HIP_ERR_NULL, "null argument");
    int rc = check_lm_head(token_embd, H, V);
    if (rc) return rc;
    if (H % 2) return fail(TER_HIP_ERR_SHAPE, "the fused RMSNorm prologue needs an even H (H=%d)", H);
    if (!aligned(hidden, 8) || !aligned(hidden16, 4) || !aligned(gamma, 4) || !aligned(x_norm_out, 4) ||
        !aligned(logits_out, 2) || !aligned(token_out, 4) || !aligned(state, 8) || !aligned(pos_advance, 4))
        return fail(TER_HIP_ERR_ALIGN, "misaligned argument");
    if (!(eps >= 0.f)) return fail(TER_HIP_ERR_SHAPE, "RMSNorm eps must be >= 0");
    int n_wg = 0;
    rc = pick_lm_head_wg(H, V, &n_wg);
    if (rc) return rc;
    hipError_t e = launch_lm_head(hidden, hidden16, gamma, eps, nullptr, token_embd, H, V, x_norm_out, logits_out,
                                  token_out, reinterpret_cast<unsigned long long*>(state), pos_advance, n_wg,
                                  static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "lm_head launch");
    return TER_HIP_OK;
}

int ter_hip_lm_head_argmax(const float* hidden, const uint16_t* gamma, float eps, const uint16_t* token_embd, int32_t H,
                           int32_t V, uint16_t* x_norm_out, uint16_t* logits_out, int32_t* token_out, uint64_t* state,
                           int32_t* pos_advance, void* stream) {
    if (!hidden) return fail(TER_HIP_ERR_NULL, "null argument");
    return lm_head_argmax_any(hidden, nullptr, gamma, eps, token_embd, H, V, x_norm_out, logits_out, token_out, state,
                              pos_advance, stream);
}

int ter_hip_lm_head_argmax_h16(const uint16_t* hidden16, const uint16_t* gamma, float eps, const uint16_t* token_embd,
                               int32_t H, int32_t V, uint16_t* x_norm_out, uint16_t* logits_out, int32_t* token_out,
                               uint64_t* state, int32_t* pos_advance, void* stream) {
    if (!hidden16) return fail(TER_HIP_ERR_NULL, "null argument");
    return lm_head_argmax_any(nullptr, hidden16, gamma, eps, token_embd, H, V, x_norm_out, logits_out, token_out,
                              state, pos_advance, stream);
}

int ter_hip_embed_h16(const uint16_t* token_embd, int32_t V, int32_t H, const int32_t* token_dev, uint16_t* hidden16,
                      void* stream) {
    if (!token_embd || !token_dev || !hidden16) return fail(TER_HIP_ERR_NULL, "null argument");
    if (V < 1 || H < 1 || V > TER_HIP_N_MAX || H > TER_HIP_K_MAX) return fail(TER_HIP_ERR_SHAPE, "V=%d H=%d", V, H);
    if (!aligned(token_embd, 2) || !aligned(token_dev, 4) || !aligned(hidden16, 2))
        return fail(TER_HIP_ERR_ALIGN, "misaligned argument");
    hipError_t e = launch_embed_h16(token_embd, V, H, token_dev, hidden16, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "embedding launch");
    return TER_HIP_OK;
}

int ter_hip_attn_create(ter_hip_attn_t** out, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int32_t s_max,
                        float theta, int32_t rope_type) {
    if (!out) return fail(TER_HIP_ERR_NULL, "null context pointer");
    *out = nullptr;
    if (n_heads < 1 || n_kv_heads < 1 || n_heads % n_kv_heads || !attn_supported_head_dim(head_dim) || s_max < 1 ||
        s_max > attn_chunk() * attn_max_chunks() || (long long)s_max * n_kv_heads * head_dim * 2 > 0x7FFFFFFFLL)
        return fail(TER_HIP_ERR_SHAPE, "attention shape nh=%d nkv=%d hd=%d smax=%d unsupported", n_heads, n_kv_heads,
                    head_dim, s_max);
    if (rope_type != TER_HIP_ROPE_NORM && rope_type != TER_HIP_ROPE_NEOX)
        return fail(TER_HIP_ERR_PAYLOAD, "unknown RoPE type %d", rope_type);
    if (!(theta > 0.f)) return fail(TER_HIP_ERR_SHAPE, "RoPE theta must be > 0");
    const int half = head_dim / 2;
    const int n_chunks = (s_max + attn_chunk() - 1) / attn_chunk();
    const int groups = attn_head_groups(n_heads, n_kv_heads);
    // RoPE table: the reference's float steps (rope_k), powf / cosf / sinf
    // replaced by libm in double rounded once to binary32
    std::vector<float> tab;
    try {
        tab.resize((size_t)s_max * half * 2);
    } catch (...) {
        return fail(TER_HIP_ERR_ALLOC, "RoPE table");
    }
    for (int k = 0; k < half; ++k) {
        const float e = (2.0f * (float)k) / (float)head_dim;
        const float pw = (float)std::pow((double)theta, (double)e);
        const float freq = 1.0f / pw;
        for (int p = 0; p < s_max; ++p) {
            const float ang = (float)p * freq;
            tab[((size_t)p * half + k) * 2] = (float)std::cos((double)ang);
            tab[((size_t)p * half + k) * 2 + 1] = (float)std::sin((double)ang);
        }
    }
    ter_hip_attn* a = new (std::nothrow) ter_hip_attn();
    if (!a) return fail(TER_HIP_ERR_ALLOC, "attention context");
    a->nh = n_heads;
    a->nkv = n_kv_heads;
    a->hd = head_dim;
    a->smax = s_max;
    a->neox = rope_type == TER_HIP_ROPE_NEOX;
    const size_t tb = tab.size() * sizeof(float);
    const size_t pb = (size_t)n_heads * n_chunks * attn_part_stride(head_dim) * sizeof(float);
    const size_t cb = (size_t)groups * attn_count_stride() * sizeof(unsigned);
    hipError_t e = hipMalloc(&a->rope, tb);
    if (e == hipSuccess) e = hipMalloc(&a->part, pb);
    if (e == hipSuccess) e = hipMalloc(&a->count, cb);
    if (e == hipSuccess) e = hipMemcpy(a->rope, tab.data(), tb, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    // the XCD-local exchange needs blocks on XCD b % 8; the partial buffer
    // serves as the probe's scratch (it holds no state between launches)
    const int nb = attn_local_blocks(n_heads, n_kv_heads, s_max);
    // (TER_HIP_ATTN_DEVICE_WIDE=1 in the environment keeps the device-wide form)
    const char* dw = std::getenv("TER_HIP_ATTN_DEVICE_WIDE");
    const bool want_local = !(dw && dw[0] == '1');
    if (e == hipSuccess && want_local && (size_t)nb * sizeof(int) <= pb)
        a->xcd_local = attn_xcd_round_robin(nb, reinterpret_cast<int*>(a->part), nullptr);
    if (e == hipSuccess) e = hipGetLastError();
    if (e == hipSuccess) e = hipMemset(a->count, 0, cb);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        ter_hip_attn_destroy(a);
        return hip_fail(e, "attention context allocation");
    }
    *out = a;
    return TER_HIP_OK;
}

int ter_hip_attn_decode(const ter_hip_attn_t* a, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                        uint16_t* k_cache, uint16_t* v_cache, const int32_t* pos_dev, uint16_t* out, void* stream) {
    if (!a || !q || !k || !v || !k_cache || !v_cache || !pos_dev || !out) return fail(TER_HIP_ERR_NULL, "null argument");
    if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(q, 2) || !aligned(k, 2) || !aligned(v, 2) ||
        !aligned(out, 2) || !aligned(pos_dev, 4))
        return fail(TER_HIP_ERR_ALIGN, "misaligned argument (caches need 16 bytes)");
    hipError_t e = launch_attn_decode(q, k, v, k_cache, v_cache, pos_dev, out, a->rope, a->part, a->count, a->nh,
                                      a->nkv, a->hd, a->smax, a->neox, a->xcd_local, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "attention launch");
    return TER_HIP_OK;
}

int ter_hip_rope(const ter_hip_attn_t* a, uint16_t* x, int32_t n_heads, const int32_t* pos_dev, void* stream) {
    if (!a || !x || !pos_dev) return fail(TER_HIP_ERR_NULL, "null argument");
    if (n_heads < 1) return fail(TER_HIP_ERR_SHAPE, "n_heads=%d", n_heads);
    if (!aligned(x, 2) || !aligned(pos_dev, 4)) return fail(TER_HIP_ERR_ALIGN, "misaligned argument");
    hipError_t e =
        launch_rope(x, n_heads, a->hd, a->rope, pos_dev, a->smax, a->neox, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "rope launch");
    return TER_HIP_OK;
}

void ter_hip_attn_destroy(ter_hip_attn_t* a) {
    if (!a) return;
    (void)hipFree(a->rope);
    (void)hipFree(a->part);
    (void)hipFree(a->count);
    delete a;
}

int ter_hip_synth_v11(uint8_t* v11_dev, int32_t K, int32_t N, uint64_t seed, uint32_t t0, uint32_t t1, void* stream) {
    if (!v11_dev) return fail(TER_HIP_ERR_NULL, "null buffer");
    if (K < 1 || N < 4 || N % 4) return fail(TER_HIP_ERR_SHAPE, "K=%d N=%d", K, N);
    hipError_t e = launch_synth_v11(v11_dev, K, N, seed, t0, t1, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "synth launch");
    return TER_HIP_OK;
}

int ter_hip_synth_i8(int8_t* x_dev, int64_t n, uint64_t seed, int32_t lo, int32_t hi, void* stream) {
    if (!x_dev) return fail(TER_HIP_ERR_NULL, "null buffer");
    if (n < 1 || lo > hi || lo < -128 || hi > 127) return fail(TER_HIP_ERR_SHAPE, "bad range");
    hipError_t e = launch_synth_i8(x_dev, n, seed, lo, hi, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "synth launch");
    return TER_HIP_OK;
}

int ter_hip_noop(void* stream) {
    hipError_t e = launch_noop(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "noop launch");
    return TER_HIP_OK;
}

int ter_hip_read_probe(const void* buf, size_t bytes, int32_t n_wg, uint32_t* sink, void* stream) {
    if (!buf || !sink) return fail(TER_HIP_ERR_NULL, "null argument");
    if (bytes == 0 || bytes % kTileBytes || bytes / kTileBytes > (size_t)n_wg * kGemvWaves * (1u << 20))
        return fail(TER_HIP_ERR_SHAPE, "bytes %zu: a nonzero multiple of 1024, at most 1 GiB per wave", bytes);
    if (n_wg < 1) return fail(TER_HIP_ERR_SHAPE, "n_wg=%d", n_wg);
    if (!aligned(buf, 16) || !aligned(sink, 4)) return fail(TER_HIP_ERR_ALIGN, "misaligned argument");
    hipError_t e = launch_read_probe(static_cast<const uint8_t*>(buf), (long long)(bytes / kTileBytes), n_wg,
                                     reinterpret_cast<unsigned*>(sink), static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "read probe launch");
    return TER_HIP_OK;
}

// ---- K4-style handle + KernelTable native slot -------------------------

static int native_matmul(ter_hip_handle_t* h, const int64_t* args, size_t n_args) {
    if (n_args < 6) return fail(TER_HIP_ERR_FEWARGS, TER_HIP_SLOT_MATMUL " takes 6 args, got %zu", n_args);
    const ter_hip_wpk_t* w = reinterpret_cast<const ter_hip_wpk_t*>(static_cast<intptr_t>(args[0]));
    const ter_hip_act_t* x = reinterpret_cast<const ter_hip_act_t*>(static_cast<intptr_t>(args[1]));
    float* y = reinterpret_cast<float*>(static_cast<intptr_t>(args[2]));
    int32_t* acc = reinterpret_cast<int32_t*>(static_cast<intptr_t>(args[3]));
    void* stream = reinterpret_cast<void*>(static_cast<intptr_t>(args[4]));
    const int64_t M = args[5];
    if (!w) return fail(TER_HIP_ERR_NULL, "null weight");
    if (M < 1 || M > TER_HIP_M_MAX) return fail(TER_HIP_ERR_SHAPE, "M=%lld", (long long)M);
    const int rc = M == 1 ? ter_hip_gemv(w, x, y, acc, stream) : ter_hip_gemm(w, x, (int32_t)M, y, acc, stream);
    if (rc == TER_HIP_OK) {
        const uint64_t n = (uint64_t)((w->K + 26) / 27) * (uint64_t)w->N * (uint64_t)M;
        h->counts.tvmac += n;
        h->counts.total_ops += n;
    }
    return rc;
}

ter_hip_handle_t* ter_hip_create(int32_t device) {
    ter_hip_handle_t* h = new (std::nothrow) ter_hip_handle_t();
    if (!h) return nullptr;
    std::memset(h, 0, sizeof *h);
    h->device = device;
    if (ter_hip_install_native(h, TER_HIP_SLOT_MATMUL, native_matmul) != TER_HIP_OK) {
        delete h;
        return nullptr;
    }
    return h;
}

void ter_hip_destroy(ter_hip_handle_t* h) { delete h; }

int ter_hip_install_native(ter_hip_handle_t* h, const char* name, ter_hip_native_fn fn) {
    if (!h || !name || !fn) return fail(TER_HIP_ERR_NULL, "null handle, name or function");
    for (auto& s : h->slots)
        if (s.used && std::strncmp(s.name, name, sizeof s.name - 1) == 0) {
            s.fn = fn;
            return TER_HIP_OK;
        }
    for (auto& s : h->slots) {
        if (s.used) continue;
        std::strncpy(s.name, name, sizeof s.name - 1);
        s.name[sizeof s.name - 1] = '\0';
        s.fn = fn;
        s.used = true;
        return TER_HIP_OK;
    }
    return fail(TER_HIP_ERR_FULL, "kernel table full (32 slots)");
}

int ter_hip_call(ter_hip_handle_t* h, const char* name, const int64_t* args, size_t n_args) {
    if (!h || !name) return fail(TER_HIP_ERR_NULL, "null handle or name");
    if (n_args > 7) return fail(TER_HIP_ERR_NARGS, "at most 7 args (R1..R7), got %zu", n_args);
    if (n_args > 0 && !args) return fail(TER_HIP_ERR_NULL, "null args");
    for (auto& s : h->slots)
        if (s.used && std::strncmp(s.name, name, sizeof s.name) == 0) {
            if (h->device >= 0) {
                hipError_t e = hipSetDevice(h->device);
                if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
            }
            return s.fn(h, args, n_args);
        }
    return fail(TER_HIP_ERR_NOTFOUND, "no kernel named '%s'", name);
}

void ter_hip_op_counts(const ter_hip_handle_t* h, ter_hip_op_counts_t* out) {
    if (!h || !out) return;
    *out = h->counts;
}

void ter_hip_reset_counters(ter_hip_handle_t* h) {
    if (h) std::memset(&h->counts, 0, sizeof h->counts);
}

}  // extern "C"
