/*
 * ter_hip.h -- C-ABI of the MI355X (gfx950) packed-trit matmul fabric.
 *
 * Drop-in boundary for ter's packed-trit GEMV/GEMM.  Plain C types only:
 * device pointers are `void*`/typed pointers, a HIP stream is passed as
 * `void*` (a hipStream_t; NULL = the null stream).  Every entry point returns
 * an int status in the ter_k4 style (0 = ok, negative = error) and never
 * aborts the process.
 *
 * Reference interfaces this header replaces (paths in the xaskasdf/ter tree):
 *   - the packed weight handle  WPK{uint8_t* data; float scale; size_t bytes}
 *       cuda/ter_cuda_forward_packed.cu:400
 *   - the GPU GEMV launcher     mm_packed_dispatch(X, scale_x_dev, W, out, K, N, stream)
 *       cuda/ter_cuda_forward_packed.cu:493-500
 *   - the CPU GEMV contract     mm_row(sim, kt, id, Xt, row, Wt, K, N, out)
 *       src/tx/forward.cpp:299-352 (internal linkage: bound through the KernelTable slot below)
 *   - the batched launchers     mm_bitnet_addonly_batched_k<M>(X, X_scale, W_col, K, N, w_scale, out)
 *       cuda/ter_cuda_addonly_batched.cu:31-38
 *   - the activation quantizer  quant_int8_k(x, y, scale_out, N)
 *       cuda/ter_cuda_forward_packed.cu:40-62
 *   - the K4 C-ABI              ter_k4_create/destroy/install_kernel/call/op_counts/reset_counters
 *       include/ter_k4/ter_k4.h:29-55, src/k4/ter_k4.cpp:14-73
 *   - the KernelTable slot      KernelTable::install/find, 32 slots, names < 32 chars
 *       include/ter/kernels.hpp:21-38, src/sim/call_kernel.cpp:24-61
 */
#ifndef TER_HIP_H
#define TER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (ter_k4 values kept: src/k4/ter_k4.cpp:38,52-55) ---- */
#define TER_HIP_OK             0
#define TER_HIP_ERR_NULL      -1  /* null handle / pointer argument            */
#define TER_HIP_ERR_NOTFOUND  -2  /* unknown kernel name                       */
#define TER_HIP_ERR_ALLOC     -3  /* allocation failure                        */
#define TER_HIP_ERR_NARGS     -4  /* more than 7 kernel-call arguments         */
#define TER_HIP_ERR_SHAPE     -5  /* K/N/M out of range or buffer too small    */
#define TER_HIP_ERR_PAYLOAD   -6  /* payload not ternary / X not int8 / blocked scales */
#define TER_HIP_ERR_HIP       -7  /* HIP runtime error (launch, copy, device)  */
#define TER_HIP_ERR_ALIGN     -8  /* device pointer misaligned                  */
#define TER_HIP_ERR_FULL      -9  /* kernel table has no free slot             */
#define TER_HIP_ERR_CONFLICT -10  /* a plan names one weight twice (shared fix-up slots) */
#define TER_HIP_ERR_FILE     -11  /* model file: cannot open, bad header, size mismatch, short read */
#define TER_HIP_ERR_FEWARGS  -12  /* a native slot got fewer arguments than it takes */

/* ---- limits ---- */
#define TER_HIP_K_MAX      32768  /* activation vector staged in LDS (int8)    */
#define TER_HIP_N_MAX  (1 << 24)
#define TER_HIP_M_MAX        256  /* batched rows per call                      */

/* ---- activation kinds ---- */
#define TER_HIP_X_I8   0  /* int8 X[K] with a host or device activation scale       */
#define TER_HIP_X_F32  1  /* fp32 X[K]: absmax -> int8 inside the kernel prologue    */
/* RMSNorm (fp16 gamma, eps) then absmax -> int8 inside the kernel prologue:
 * the fused rmsnorm_quant_f32_in_k / rmsnorm_quant_fp16_in_k steps
 * (cuda/ter_cuda_forward_bitnet.cu:64-146), with fp32 or fp16 X[K]. */
#define TER_HIP_X_F32_RMS 2
#define TER_HIP_X_F16_RMS 3
/* relu^2(gate) * up, RMSNorm (fp16 gamma, eps), then absmax -> int8: the
 * fused relu2_mul_rmsnorm_quant_k step in front of the FFN down projection
 * (cuda/ter_cuda_forward_bitnet.cu:258-309, launched <<<1,1024>>> at :884).
 * `data` is the fp16 gate [K], `up` the fp16 up projection [K]. */
#define TER_HIP_X_RELU2_RMS 4
/* int16 X[K] with a host or device activation scale: the reference host
 * forward's 9-trit payloads (quantize(x_norm, {1,H}, 9) gives |x| <= 9841,
 * src/tx/forward.cpp:400, src/numfmt/quantize.cpp:26-38); any int16 value is
 * exact.  Single GEMVs only (ter_hip_gemv, ter_hip_gemv_out, ter_hip_mm_row);
 * work lists and batched GEMMs refuse it (TER_HIP_ERR_PAYLOAD). */
#define TER_HIP_X_I16 5
/* fp16 X[K]: absmax -> int8 inside the kernel prologue, the Llama forward's
 * quant_int8_k on its fp16 attention output before Wo
 * (cuda/ter_cuda_forward_packed.cu:40-62, launched at :536). */
#define TER_HIP_X_F16 6
/* silu(gate) * up, then absmax -> int8: the Llama forward's fused
 * silu_mul_quant_k in front of the FFN down projection
 * (cuda/ter_cuda_forward_packed.cu:312-344, launched <<<1,1024>>> at :545).
 * `data` is the fp16 gate [K], `up` the fp16 up projection [K].  The exp is
 * this build's (faithful, the oracle's orc_expf), not CUDA's expf.
 * TER_HIP_X_F16 and TER_HIP_X_SILU_MUL are single GEMVs and work lists
 * only; batched GEMMs refuse them (TER_HIP_ERR_PAYLOAD). */
#define TER_HIP_X_SILU_MUL 7
/* The second half of silu_mul_quant_k (cuda/ter_cuda_forward_packed.cu:325-343):
 * `data` is fp32 silu(gate) [K], as the gate GEMV's `silu` output writes it
 * (ter_hip_out_t), `up` the fp16 up projection [K]; v = data * float(up),
 * then absmax -> int8.  With the gate GEMV's silu output this is
 * TER_HIP_X_SILU_MUL bit for bit, with the exp computed once per element
 * instead of in every workgroup of the down projection.  Single GEMVs and
 * work lists only, like TER_HIP_X_SILU_MUL. */
#define TER_HIP_X_SMUL 8

/*
 * Packed ternary weight (replaces WPK, cuda/ter_cuda_forward_packed.cu:400).
 *
 * `data` holds the "T16" tile stream the kernels read: 1 KiB tiles of
 * 16 output columns x 256 input rows, 2 bits per trit, stored as u = w + 1
 * (dword 4L+j of a tile holds column 4(L/16)+j of the tile's strip over rows
 * 16(L%16)+e, e = 4f+b at bits 8b+2f), followed by `N` 64-bit fix-up slots
 * (`fix`, zero at rest) used to combine split column strips.  The whole
 * buffer is `ter_hip_wpk_bytes(K, N)` bytes of device memory owned by the
 * caller.  `scale` is the per-tensor weight scale (Wt.scale).  A ternary
 * payload {-m,0,+m} is stored as trits {-1,0,+1} with m in `mag` (1 for
 * plain trits): the kernels keep the trit accumulator acc in int32 and form
 * the reference's float((int64)(m * acc)) in the epilogue, so the fp32
 * outputs are mm_row's bit for bit (src/tx/forward.cpp:333-345).
 */
typedef struct ter_hip_wpk {
    uint8_t*  data;    /* device: tile stream, then fix-up slots            */
    size_t    bytes;   /* total device bytes (== ter_hip_wpk_bytes(K, N))    */
    uint64_t* fix;     /* device: N fix-up slots inside `data`               */
    int32_t   K, N;
    float     scale;
    int32_t   layout;  /* TER_HIP_LAYOUT_T16                                */
    int32_t   mag;     /* trit magnitude m >= 1 (ter_hip_wpk_init sets 1)    */
} ter_hip_wpk_t;

#define TER_HIP_LAYOUT_T16 16

/* Activation operand of one GEMV / GEMM. */
typedef struct ter_hip_act {
    const void*  data;       /* device: int8 (X_I8), int16 (X_I16), fp32 (X_F32, X_F32_RMS)
                                or fp16 (X_F16, X_F16_RMS; the gate for X_RELU2_RMS and
                                X_SILU_MUL) [M][K]                                       */
    int32_t      kind;       /* TER_HIP_X_*                                            */
    float        scale;      /* X_I8, X_I16: host activation scale, used when scale_dev NULL */
    const float* scale_dev;  /* X_I8, X_I16: device activation scale(s) ([M]), or NULL */
    int8_t*      q_out;      /* X_F32: optional device copy of the quantized X [M][K]  */
    float*       scale_out;  /* X_F32: optional device act scale(s) 1/scale ([M])     */
    const uint16_t* gamma;   /* RMS kinds: device fp16 RMSNorm weights [K]             */
    float        eps;        /* RMS kinds: RMSNorm epsilon                             */
    const uint16_t* up;      /* X_RELU2_RMS, X_SILU_MUL: device fp16 up projection [M][K] */
} ter_hip_act_t;

/* Outputs of one GEMV / GEMM; any subset, at least one non-NULL.  With
 * y = float(m * acc) * (x_scale * w->scale), m = w->mag (1 for plain trits):
 *   y     fp32 [M][N]
 *   acc   int32 [M][N]
 *   y16   fp16 bits [M][N] = half(y), round to nearest even: the reference's
 *         projection output out[j] = __float2half((float)acc * scale)
 *         (cuda/ter_cuda_forward_packed.cu:393, ter_cuda_forward_bitnet.cu:557,
 *         ter_cuda_addonly_batched.cu:120)
 *   resid fp32 [M][N], updated in place: resid += float(half(y)), the
 *         projection followed by add_k_f32 into the residual stream
 *         (cuda/ter_cuda_forward_bitnet.cu:51-54, :876, :887).  A plain
 *         read-modify-write: no other work of the same launch may target the
 *         same elements.
 *   resid16 fp16 bits [M][N], updated in place: resid16 = half(float(resid16)
 *         + float(half(y))), the projection followed by add_k into the Llama
 *         forward's fp16 residual stream (cuda/ter_cuda_forward_packed.cu:115-118,
 *         :538, :548); the same rule as resid.  GEMVs and GEMV work lists
 *         only: the batched GEMMs refuse it (TER_HIP_ERR_PAYLOAD).
 *   silu  fp32 [N] = h / (1 + exp(-h)), h = float(half(y)): the gate
 *         projection's fp16 output taken through the first half of
 *         silu_mul_quant_k (cuda/ter_cuda_forward_packed.cu:322-324, this
 *         build's exp), for the TER_HIP_X_SMUL activation of the down
 *         projection.  GEMVs and GEMV work lists only, like resid16. */
typedef struct ter_hip_out {
    float*    y;
    int32_t*  acc;
    uint16_t* y16;
    float*    resid;
    uint16_t* resid16;
    float*    silu;
} ter_hip_out_t;

/* ---------------------------------------------------------------------- */
/* Packed payload (TritTensor -> device tile stream)                       */
/* ---------------------------------------------------------------------- */

/* Device bytes needed for a K x N packed weight (tile stream + fix-up slots). */
size_t ter_hip_wpk_bytes(int32_t K, int32_t N);

/* Fill `w` for a caller-owned device buffer `dev_buf` of `buf_bytes` bytes
 * (256-byte aligned).  Does not touch the device. */
int ter_hip_wpk_init(ter_hip_wpk_t* w, void* dev_buf, size_t buf_bytes,
                     int32_t K, int32_t N, float scale);

/* Device repack of reference v11 bytes (W_col[j_byte*K + k], 4 columns per
 * byte, code map 00=0 01=+1 10=-1 11=0; tools/convert_llama_to_packed.py:128-140)
 * into `w`, and zero of its fix-up slots.  v11_dev: (N/4)*K device bytes;
 * N must be a multiple of 4 (the v11 format's own requirement). */
int ter_hip_pack_v11(ter_hip_wpk_t* w, const uint8_t* v11_dev, void* stream);

/* Inverse of ter_hip_pack_v11 (device): write v11 bytes of `w` to v11_dev. */
int ter_hip_unpack_v11(const ter_hip_wpk_t* w, uint8_t* v11_dev, void* stream);

/* Device repack of a microsoft/BitNet GGUF i2_s tensor (the codes of the
 * (N, K) tensor, N*K/4 device bytes; replaces the host converter
 * i2s_to_col_packed, tools/convert_bitnet_to_packed.py:85-157) into `w`, and
 * zero of its fix-up slots.  The per-tensor scale is the fp32 that follows
 * the codes in the file (read_i2s_scale, ibid.:85-91): pass it to
 * ter_hip_wpk_init.  K and N must be multiples of 4 and N*K a multiple of
 * 128 (whole i2_s blocks), as the converter requires. */
int ter_hip_pack_i2s(ter_hip_wpk_t* w, const uint8_t* i2s_dev, void* stream);

/* Host pack of a TritTensor payload (int32 [K][N] row-major, the orientation
 * mm_row reads, src/tx/forward.cpp:337) into `w` (synchronous upload).  The
 * payload must be ternary {-m, 0, +m} for one m > 0 (or all zero; then
 * m = 1); `w->scale` becomes `scale` and `w->mag` m.  Returns
 * TER_HIP_ERR_PAYLOAD otherwise.  `magnitude_out` (optional) receives m. */
int ter_hip_pack_payload(ter_hip_wpk_t* w, const int32_t* payload_host, float scale,
                         int32_t* magnitude_out, void* stream);

/* ---------------------------------------------------------------------- */
/* M = 1 decode GEMV                                                       */
/* ---------------------------------------------------------------------- */

/* y[j] = float(m * acc[j]) * (x_scale * w->scale), acc[j] = sum_k x[k] * w[k][j], m = w->mag.
 * y (fp32 [N]) and acc (int32 [N]) are optional device outputs (at least one). */
int ter_hip_gemv(const ter_hip_wpk_t* w, const ter_hip_act_t* x, float* y, int32_t* acc,
                 void* stream);
/* ter_hip_gemv with every output form (ter_hip_out_t). */
int ter_hip_gemv_out(const ter_hip_wpk_t* w, const ter_hip_act_t* x, const ter_hip_out_t* out,
                     void* stream);

/* Drop-in for mm_packed_dispatch (cuda/ter_cuda_forward_packed.cu:493-500):
 * int8 X, device activation scale, fp32 out[N].  K, N must match W. */
int ter_hip_mm_packed_dispatch(const int8_t* X, const float* scale_x_dev,
                               const ter_hip_wpk_t* W, float* out, int32_t K, int32_t N,
                               void* stream);
/* mm_packed_dispatch with the reference's own output type: fp16 out[N] =
 * __float2half((float)acc * scale) (cuda/ter_cuda_forward_packed.cu:493-500,
 * ter_cuda_forward_bitnet.cu:837-845). */
int ter_hip_mm_packed_dispatch_f16(const int8_t* X, const float* scale_x_dev,
                                   const ter_hip_wpk_t* W, uint16_t* out, int32_t K, int32_t N,
                                   void* stream);

/* Host-side mm_row contract (src/tx/forward.cpp:299-352): X is the host
 * TritTensor payload (int32 [rows][K]), `row` selects the row; out (host
 * fp32 [N]) = float(W.mag * acc) * (x_scale * W.scale), bit for bit the
 * reference's float(int64 acc) * (Xt.scale * Wt.scale).  A row whose values
 * fit int8 runs the int8 GEMV; one that fits int16 (the reference forward's
 * 9-trit activations, |x| <= 9841) runs the int16 GEMV (TER_HIP_X_I16);
 * anything wider is TER_HIP_ERR_PAYLOAD (no CPU fallback).  Synchronous.
 * `x_stage_dev` (2*K bytes, 16-byte aligned) receives the row on the device.
 * The library narrows the row into its own page-locked host buffer and the
 * GEMV writes its outputs into another (one pair per device, grown on demand
 * and held until the process ends; calls are serialized on them), so a call
 * is one upload, one kernel and one synchronize; `y_stage_dev` (N fp32) is
 * used only where page-locked memory cannot be had (pageable copies). */
int ter_hip_mm_row(const int32_t* X, int32_t row, int32_t K, float x_scale,
                   const ter_hip_wpk_t* W, int32_t N, float* out,
                   void* x_stage_dev, float* y_stage_dev, void* stream);

/* The per-block branch of mm_row (src/tx/forward.cpp:308-330), for weights
 * whose TritTensor carries block_scales: W is the payload {-m, 0, +m} packed
 * by ter_hip_pack_payload, block_scales_dev the device fp32 scales
 * [ceil(K*N / block_size)] (block b covers the row-major payload elements
 * [b*bs, (b+1)*bs), as the reference indexes them).  out (host fp32 [N]) =
 * float(facc * double(x_scale)), facc the reference's double sum over k in
 * increasing order of x[k] * W[k][j] * block_scales[(k*N + j) / bs], bit for
 * bit.  W.scale is not used (the reference's branch ignores Wt.scale).  X as
 * ter_hip_mm_row (the row must fit int16), and every |x| * W.mag must be
 * below 2^29 so each term is exact in double (TER_HIP_ERR_PAYLOAD
 * otherwise; the reference's 9-trit activations and weights give at most
 * 9841^2).  Synchronous; x_stage_dev 2*K bytes (16-byte aligned),
 * y_stage_dev N fp32. */
int ter_hip_mm_row_blocked(const int32_t* X, int32_t row, int32_t K, float x_scale,
                           const ter_hip_wpk_t* W, int32_t N, const float* block_scales_dev,
                           int64_t block_size, float* out, void* x_stage_dev, float* y_stage_dev,
                           void* stream);

/* ---------------------------------------------------------------------- */
/* Work lists: many independent GEMVs in ONE launch (layer sweeps)          */
/* ---------------------------------------------------------------------- */
typedef struct ter_hip_gemv_item {
    const ter_hip_wpk_t* w;
    ter_hip_act_t        x;
    float*               y;    /* fp32 [N] or NULL */
    int32_t*             acc;  /* int32 [N] or NULL */
    uint16_t*            y16;  /* fp16 [N] or NULL (ter_hip_out_t)            */
    float*               resid;/* fp32 [N] residual, += half(y), or NULL      */
    uint16_t*            resid16; /* fp16 [N] residual, += half(y), or NULL   */
    float*               silu; /* fp32 [N] silu(half(y)) or NULL (ter_hip_out_t) */
} ter_hip_gemv_item_t;

typedef struct ter_hip_plan ter_hip_plan_t;

/* Build a launch plan for `n` GEMVs (descriptor table copied to the device).
 * wg_per_cu <= 0 picks the default launch shape (2 workgroups per CU, 4 for
 * int8 lists that take the vector prologue; small lists: whole strips per
 * workgroup, or 1 workgroup per CU when their activations need a prologue).  When every item has the
 * same activation kind, K % 16 == 0 and 16-byte aligned x / up / gamma, the
 * plan launches the kernel specialised on that kind.  Items sharing a weight must not
 * appear twice in one plan, and no two items may write overlapping `resid`
 * ranges (TER_HIP_ERR_CONFLICT). */
int ter_hip_plan_create(ter_hip_plan_t** plan, const ter_hip_gemv_item_t* items, int32_t n,
                        int32_t wg_per_cu);
int ter_hip_plan_launch(const ter_hip_plan_t* plan, void* stream);
/* Algorithmic bytes (packed W + X + Y) and MACs of one launch of the plan. */
int ter_hip_plan_stats(const ter_hip_plan_t* plan, uint64_t* bytes, uint64_t* macs,
                       int32_t* n_wg);
/* How a GEMV plan runs (no counterpart in the reference; for tuning and
 * tests): *mode = TER_HIP_PLAN_STRIPS (whole column strips per workgroup)
 * | TER_HIP_PLAN_STRIDED (the strided prologue) | TER_HIP_PLAN_SHARED (one
 * activation vector and back-to-back tile streams, e.g. weights grouped in
 * one allocation in item order: the first loads need no descriptor); 0 for
 * the stream-K partition and for GEMM plans. */
#define TER_HIP_PLAN_STRIPS 1
#define TER_HIP_PLAN_STRIDED 2
#define TER_HIP_PLAN_SHARED 4
int ter_hip_plan_mode(const ter_hip_plan_t* plan, int32_t* mode);
void ter_hip_plan_destroy(ter_hip_plan_t* plan);

/* ---------------------------------------------------------------------- */
/* M > 1 batched GEMM (replaces mm_bitnet_addonly_batched_k /              */
/* mm_packed_batched, cuda/ter_cuda_addonly_batched.cu:31-124)              */
/* ---------------------------------------------------------------------- */

/* Y[m][j] = float(w->mag * acc[m][j]) * (x_scale[m] * w->scale).  x->data is [M][K];
 * for X_F32 each row is quantized by absmax (quant_int8_k steps) into
 * `x->q_out` / `x->scale_out` (both REQUIRED for X_F32, [M][K] / [M]).  For
 * X_I8, x->scale_dev ([M]) is required.  M up to TER_HIP_M_MAX; above 128
 * rows, with the int8 rows 16-byte aligned and K % 16 == 0, the rows run in
 * pieces of 128 (one launch each, on the same stream). */
int ter_hip_gemm(const ter_hip_wpk_t* w, const ter_hip_act_t* x, int32_t M, float* y,
                 int32_t* acc, void* stream);
/* ter_hip_gemm with every output form (ter_hip_out_t, [M][N] each). */
int ter_hip_gemm_out(const ter_hip_wpk_t* w, const ter_hip_act_t* x, int32_t M,
                     const ter_hip_out_t* out, void* stream);

/* ter_hip_gemm_out that allocates nothing and takes no workspace.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  fp32 / fp16 / RMS activations are quantized into a
 * static device array of the library (one per GPU, TER_HIP_STATIC_Q_MAX
 * bytes of rows plus TER_HIP_M_MAX scales, held until the process ends)
 * instead of x->q_out / x->scale_out, which must be NULL; int8 X uses no
 * workspace.  M * K above TER_HIP_STATIC_Q_MAX is TER_HIP_ERR_SHAPE.  Every
 * call on a GPU shares that GPU's array: calls that overlap in time on one
 * GPU (other streams, other threads) race on it.  Results are
 * ter_hip_gemm_out's.  No hipMalloc, hipFree or allocating library call. */
#define TER_HIP_STATIC_Q_MAX (4 << 20)
int ter_hip_gemm_out_static(const ter_hip_wpk_t* w, const ter_hip_act_t* x, int32_t M,
                            const ter_hip_out_t* out, void* stream);

/* Many independent GEMMs in ONE launch (batched decode / prefill over a
 * layer sweep; replaces one mm_bitnet_addonly_batched_k launch per
 * projection).  X is int8 [M][K] (row stride K) with per-row device scales
 * x_scale_dev[M] (quantize fp32 rows with ter_hip_quant_int8 first).  The
 * plan is launched, queried and destroyed with ter_hip_plan_launch /
 * ter_hip_plan_stats / ter_hip_plan_destroy.  When some item has more than
 * 128 rows and every x is 16-byte aligned with K % 16 == 0, each item is cut
 * into pieces of 128 rows (one descriptor each, still one launch). */
typedef struct ter_hip_gemm_item {
    const ter_hip_wpk_t* w;
    const int8_t*        x;            /* device int8 [M][K]                 */
    const float*         x_scale_dev;  /* device fp32 [M]                    */
    int32_t              M;
    float*               y;            /* fp32 [M][N] or NULL                */
    int32_t*             acc;          /* int32 [M][N] or NULL               */
    uint16_t*            y16;          /* fp16 [M][N] or NULL                */
    float*               resid;        /* fp32 [M][N] residual or NULL       */
    uint16_t*            resid16;      /* NULL: fp16 residuals are GEMV-only */
    float*               silu;         /* NULL: the silu output is GEMV-only */
} ter_hip_gemm_item_t;

int ter_hip_gemm_plan_create(ter_hip_plan_t** plan, const ter_hip_gemm_item_t* items, int32_t n,
                             int32_t wg_per_cu);

/* Per-row absmax int8 quantizer (quant_int8_k, cuda/ter_cuda_forward_packed.cu:40-62):
 * q[m][k] = rn(x[m][k] * 127/(max_k|x[m][k]| + 1e-9)), scale_out[m] = 1/that. */
int ter_hip_quant_int8(const float* x, int32_t M, int32_t K, int8_t* q, float* scale_out,
                       void* stream);

/* Per-row fused RMSNorm + int8 quantizer, the drop-in for
 * rmsnorm_quant_f32_in_k / rmsnorm_quant_fp16_in_k
 * (cuda/ter_cuda_forward_bitnet.cu:64-146, launched <<<1,256>>> per row):
 * kind TER_HIP_X_F32_RMS (x fp32 [M][K]) or TER_HIP_X_F16_RMS (x fp16 bits [M][K]);
 * gamma fp16 bits [K].  Sum of squares in the reference's order (256 strided
 * partials with fused multiply-adds, then the halving tree);
 * rms_inv = 1 / sqrt(ss / K + eps), correctly rounded (the reference's rsqrtf
 * is an approximation); n = (x * rms_inv) * gamma; then the quant_int8_k steps. */
int ter_hip_rmsnorm_quant(const void* x, int32_t kind, const uint16_t* gamma, float eps, int32_t M,
                          int32_t K, int8_t* q, float* scale_out, void* stream);
/* Per-row fused relu^2(gate) * up + RMSNorm + int8 quantizer, the drop-in for
 * relu2_mul_rmsnorm_quant_k (cuda/ter_cuda_forward_bitnet.cu:258-309,
 * <<<1,1024>>> per row at :884): gate, up fp16 bits [M][F], gamma fp16 [F].
 * v = (g > 0 ? g*g : 0) * u; sum of squares in the 1024-thread order (1024
 * strided partials with fused multiply-adds, tree from s = 512);
 * rms_inv = 1 / sqrt(ss / F + eps), correctly rounded; n = (v * rms_inv) *
 * gamma; then the quant_int8_k steps. */
int ter_hip_relu2_rmsnorm_quant(const uint16_t* gate, const uint16_t* up, const uint16_t* gamma,
                                float eps, int32_t M, int32_t F, int8_t* q, float* scale_out,
                                void* stream);

/* ---------------------------------------------------------------------- */
/* Decode-step tail: final RMSNorm, fp16 lm_head over the tied token       */
/* embedding, argmax (cuda/ter_cuda_forward_bitnet.cu:890-911)             */
/* ---------------------------------------------------------------------- */
/* Per-row RMSNorm with fp16 output, the drop-in for rmsnorm_f32_in_k
 * (cuda/ter_cuda_forward_bitnet.cu:37-47, <<<1,256>>> per row): x fp32 [M][H],
 * gamma fp16 [H], y fp16 [M][H] = half((x * rms_inv) * gamma); the sum of
 * squares and rms_inv as ter_hip_rmsnorm_quant. */
int ter_hip_rmsnorm_f16(const float* x, const uint16_t* gamma, float eps, int32_t M, int32_t H,
                        uint16_t* y, void* stream);
/* fp16 lm_head GEMV, the drop-in for mm_fp16_lm_head_k
 * (cuda/ter_cuda_forward_bitnet.cu:388-429): logits[v] = half(sum_k x[k] *
 * token_embd[v][k]) in the reference's fp32 order (32 strided lane partials
 * over fp16 pairs, then the xor butterfly).  token_embd fp16 [V][H] row-major;
 * x, token_embd 4-byte aligned for even H. */
int ter_hip_lm_head_f16(const uint16_t* x_norm, const uint16_t* token_embd, uint16_t* logits,
                        int32_t H, int32_t V, void* stream);
/* argmax of fp16 logits [N], the drop-in for argmax_local_k + argmax_final_k
 * (cuda/ter_cuda_forward_bitnet.cu:454-495, 128 parts): the same index,
 * ties included (among equal maxima the reference's two reduction trees
 * decide: smallest bit-reversed part, then smallest bit-reversed thread,
 * then the first element); NaN and -inf never win; -1 if nothing is
 * eligible.  One launch.  `state`: TER_HIP_ARGMAX_STATE_BYTES of device
 * memory (8-byte aligned), zero before the first call (hipMemset) and left
 * zero by every call; calls that share a state must not overlap in time. */
#define TER_HIP_ARGMAX_STATE_BYTES 16512
int ter_hip_argmax_f16(const uint16_t* logits, int32_t N, int32_t* out_idx, uint64_t* state,
                       void* stream);
/* ter_hip_argmax_f16 followed by inc_pos_k: the tail of the Llama forward's
 * bench mode (cuda/ter_cuda_forward_packed.cu:555-559, after the packed
 * lm_head GEMV of :541-545).  pos_advance (device int32, required) is
 * incremented once the token is written. */
int ter_hip_argmax_f16_step(const uint16_t* logits, int32_t N, int32_t* out_idx, uint64_t* state,
                            int32_t* pos_advance, void* stream);
/* The whole tail in ONE launch (rmsnorm_f32_in_k + mm_fp16_lm_head_k +
 * argmax, :890-911): hidden fp32 [H] -> x_norm -> logits -> *token_out.
 * x_norm_out (fp16 [H]) and logits_out (fp16 [V]) are optional copies;
 * token_out and state (as ter_hip_argmax_f16) are required.  pos_advance
 * (optional, device int32) is incremented once the token is written: the
 * step's inc_pos_k (:912).  H even; hidden 8-byte and gamma 4-byte aligned. */
int ter_hip_lm_head_argmax(const float* hidden, const uint16_t* gamma, float eps,
                           const uint16_t* token_embd, int32_t H, int32_t V, uint16_t* x_norm_out,
                           uint16_t* logits_out, int32_t* token_out, uint64_t* state,
                           int32_t* pos_advance, void* stream);
/* The step's first kernel, token_embed_lookup_k (:220-231): hidden fp32 [H] =
 * token_embd[*token_dev] widened (a token outside [0, V) writes nothing). */
int ter_hip_embed_f16(const uint16_t* token_embd, int32_t V, int32_t H, const int32_t* token_dev,
                      float* hidden, void* stream);
/* The Llama forward's tail and first kernel, on its fp16 residual stream
 * (cuda/ter_cuda_forward_packed.cu:505-560): ter_hip_lm_head_argmax_h16 is
 * ter_hip_lm_head_argmax with hidden16 fp16 [H] (rmsnorm_k, :27-37, then
 * mm_fp16_lm_head_k and the argmax, :550-557; hidden16 4-byte aligned), and
 * ter_hip_embed_h16 writes hidden16 fp16 [H] = token_embd[*token_dev]
 * (token_embed_lookup_k, :99-106; a token outside [0, V) writes nothing). */
int ter_hip_lm_head_argmax_h16(const uint16_t* hidden16, const uint16_t* gamma, float eps,
                               const uint16_t* token_embd, int32_t H, int32_t V, uint16_t* x_norm_out,
                               uint16_t* logits_out, int32_t* token_out, uint64_t* state,
                               int32_t* pos_advance, void* stream);
int ter_hip_embed_h16(const uint16_t* token_embd, int32_t V, int32_t H, const int32_t* token_dev,
                      uint16_t* hidden16, void* stream);

/* ---------------------------------------------------------------------- */
/* Decode attention: RoPE + KV-cache write + attention, one launch per      */
/* layer (rope_k, kv_copy_k, attention_k: cuda/ter_cuda_forward_bitnet.cu   */
/* :185-214, 336-374, launched at :864-871; cuda/ter_cuda_forward_packed.cu  */
/* :64-157 for the Llama forward)                                           */
/* ---------------------------------------------------------------------- */
#define TER_HIP_ROPE_NORM 0  /* pairs (2k, 2k+1): the Llama forward's rope_k  */
#define TER_HIP_ROPE_NEOX 1  /* pairs (k, k + hd/2): BitNet (LLAMA_ROPE_TYPE_NEOX) */
typedef struct ter_hip_attn ter_hip_attn_t;
/* A decode-attention context for one model shape: n_heads query heads,
 * n_kv_heads KV heads (n_heads a multiple of it; query head h reads KV head
 * h * n_kv_heads / n_heads), head_dim 64 or 128, caches of s_max <= 4096
 * positions laid out [s_max][n_kv_heads][head_dim] fp16 per layer (the
 * reference's K_cache / V_cache slice of one layer), RoPE base theta.
 * Holds the RoPE table (fl(1/fl(theta^(2k/hd))), positions times that, cos
 * and sin in double rounded once to binary32) and the chunk workspace.
 * Creation runs a probe kernel once: when blocks are dispatched to the 8 XCDs
 * round-robin by index, launches keep each head group's partial exchange in
 * one XCD's L2; otherwise (or with TER_HIP_ATTN_DEVICE_WIDE=1 in the
 * environment) they use a device-wide exchange.  Same results either way.
 * Contexts are not shared between streams: launches of one context must not
 * overlap in time. */
int ter_hip_attn_create(ter_hip_attn_t** a, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                        int32_t s_max, float theta, int32_t rope_type);
/* One token of one layer: q fp16 [n_heads][hd], k, v fp16 [n_kv_heads][hd]
 * (projection outputs, before RoPE), *pos_dev the token's position
 * (device int32, < s_max; a position outside [0, s_max) makes the launch
 * write nothing).  Applies RoPE to q and k, writes k and v at
 * position pos of k_cache / v_cache, and writes out fp16 [n_heads][hd] =
 * softmax(q K^T / sqrt(hd)) V over positions 0 .. pos.  Scores are the
 * reference's bit for bit; the softmax runs over chunks of 64 positions
 * combined in order (fp16 outputs within one ulp of the reference's
 * sequential order).  Caches 16-byte aligned. */
int ter_hip_attn_decode(const ter_hip_attn_t* a, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                        uint16_t* k_cache, uint16_t* v_cache, const int32_t* pos_dev, uint16_t* out,
                        void* stream);
/* RoPE in place on fp16 head vectors x [n_heads][hd] at *pos_dev (rope_k). */
int ter_hip_rope(const ter_hip_attn_t* a, uint16_t* x, int32_t n_heads, const int32_t* pos_dev, void* stream);
void ter_hip_attn_destroy(ter_hip_attn_t* a);

/* ---------------------------------------------------------------------- */
/* Packed model files: the flat .bin blobs of tools/convert_bitnet_to_packed.py */
/* ('TERT', read by load_model_from_bin, cuda/ter_cuda_forward_bitnet.cu     */
/* :698-784) and tools/convert_llama_to_packed.py ('LLRT', read by           */
/* load_model_from_bin, cuda/ter_cuda_forward_packed.cu:589-659).  Little     */
/* endian: a 64-byte header, token_embd fp16 [V][H], output_norm fp32 [H],    */
/* then per layer the fp32 norms (attn_norm [H], ffn_norm [H]; TERT also      */
/* attn_sub_norm [H], ffn_sub_norm [F]) and the seven projections Wq Wk Wv Wo */
/* Wgate Wup Wdown, each K*(N/4) v11 bytes followed by its fp32 scale.        */
/* ---------------------------------------------------------------------- */
#define TER_HIP_BIN_TERT 0x54455254u  /* BitNet b1.58 (sub-norms, relu^2 FFN) */
#define TER_HIP_BIN_LLRT 0x4C4C5254u  /* Llama, ternarized per tensor         */

typedef struct ter_hip_bin_header {
    uint32_t magic, version;           /* TER_HIP_BIN_*, 1                    */
    uint32_t H, F, Nl, V, Nh, Nkv, Hd, Smax;
    float    rope_theta, eps;
} ter_hip_bin_header_t;

#define TER_HIP_BIN_F16   0  /* fp16 [n]: token_embd                          */
#define TER_HIP_BIN_F32   1  /* fp32 [n]: a norm (the loaders convert to fp16) */
#define TER_HIP_BIN_TRITS 2  /* v11 packed trits [K*(N/4)] + fp32 scale        */

typedef struct ter_hip_bin_tensor {
    char     name[24];   /* token_embd, output_norm, attn_norm, ffn_norm,
                            attn_sub_norm, ffn_sub_norm, Wq .. Wdown          */
    int32_t  layer;      /* -1 for token_embd and output_norm                  */
    int32_t  kind;       /* TER_HIP_BIN_*                                      */
    int64_t  offset;     /* file offset of the data                            */
    int64_t  bytes;      /* data bytes (trits: without the scale)              */
    int64_t  n;          /* elements (F16 / F32)                               */
    int32_t  K, N;       /* TRITS: input rows, output columns                   */
    float    scale;      /* TRITS: the per-tensor scale that follows the data   */
} ter_hip_bin_tensor_t;

typedef struct ter_hip_bin ter_hip_bin_t;

/* Open a model file: checks magic and version (as the reference loaders),
 * shapes (N a multiple of 4 for every projection), and that the file holds
 * exactly the tensors the header implies; reads the projection scales and
 * builds the tensor directory.  Host only (no device work). */
int ter_hip_bin_open(const char* path, ter_hip_bin_t** bin, ter_hip_bin_header_t* header);
/* Number of tensors and entry i of the directory (file order). */
int32_t ter_hip_bin_count(const ter_hip_bin_t* bin);
int ter_hip_bin_tensor(const ter_hip_bin_t* bin, int32_t i, ter_hip_bin_tensor_t* out);
/* Index of the tensor `name` of `layer` (-1 for the model-level tensors),
 * or TER_HIP_ERR_NOTFOUND. */
int32_t ter_hip_bin_find(const ter_hip_bin_t* bin, const char* name, int32_t layer);
/* Tensor i into host memory: F16 and TRITS as stored (TRITS without the
 * scale); F32 as stored, or, with as_f16, rounded to fp16 (to nearest even,
 * the loaders' __float2half of read_f32_to_half_device). */
int ter_hip_bin_read_host(const ter_hip_bin_t* bin, int32_t i, void* dst, int32_t as_f16);
/* Tensor i (F16, or F32 as fp16) into device memory [n] fp16. */
int ter_hip_bin_upload_f16(const ter_hip_bin_t* bin, int32_t i, uint16_t* dst_dev, void* stream);
/* Projection i into `w` (initialised by ter_hip_wpk_init for its K x N; the
 * scale is set from the file): the v11 bytes go through v11_stage_dev
 * (K*(N/4) device bytes) and ter_hip_pack_v11. */
int ter_hip_bin_upload_wpk(const ter_hip_bin_t* bin, int32_t i, ter_hip_wpk_t* w, uint8_t* v11_stage_dev,
                           void* stream);
void ter_hip_bin_close(ter_hip_bin_t* bin);

/* ---------------------------------------------------------------------- */
/* K4-style handle + KernelTable native slot                               */
/* (include/ter_k4/ter_k4.h:29-55; include/ter/kernels.hpp:21-38)           */
/* ---------------------------------------------------------------------- */
typedef struct ter_hip_handle ter_hip_handle_t;

/* A native kernel: receives the handle and up to 7 int64 register args
 * (the R1..R7 convention of Sim::call_kernel, src/sim/call_kernel.cpp:64-78). */
typedef int (*ter_hip_native_fn)(ter_hip_handle_t* h, const int64_t* args, size_t n_args);

typedef struct {
    uint64_t total_ops;
    uint64_t tvmac;
    uint64_t tvadd;
    uint64_t tvsub;
    uint64_t tvmul;
} ter_hip_op_counts_t;  /* same fields as ter_k4_op_counts_t */

/* Name of the native packed GEMV/GEMM slot.  It is not the reference's
 * "tk_matmul_b_9t" (src/kernels/registry.cpp:18-20): that name belongs to the
 * 3-argument Sim kernel (R1 = X, R2 = W, R3 = Y, src/kernels/tk_matmul_b_9t.tasm),
 * whose calls must keep reaching the Sim (ter_hip_call returns
 * TER_HIP_ERR_NOTFOUND for it, the router's cue to fall through). */
#define TER_HIP_SLOT_MATMUL "tk_matmul_t16"

/* Creates a handle bound to HIP device `device` (-1: calls select no device)
 * with the slot TER_HIP_SLOT_MATMUL installed as the native packed GEMV.
 * Returns NULL on failure. */
ter_hip_handle_t* ter_hip_create(int32_t device);
void ter_hip_destroy(ter_hip_handle_t* h);
/* Install (or replace) a named native slot.  Names longer than 31 chars are
 * truncated (KernelTable::kNameMax = 32).  TER_HIP_ERR_FULL after 32 slots. */
int ter_hip_install_native(ter_hip_handle_t* h, const char* name, ter_hip_native_fn fn);
/* Call a slot by name: -1 null, -2 unknown name, -4 n_args > 7
 * (src/k4/ter_k4.cpp:52-55); otherwise the slot's return value
 * (TER_HIP_ERR_FEWARGS when a slot gets fewer arguments than it takes). */
int ter_hip_call(ter_hip_handle_t* h, const char* name, const int64_t* args, size_t n_args);
void ter_hip_op_counts(const ter_hip_handle_t* h, ter_hip_op_counts_t* out);
void ter_hip_reset_counters(ter_hip_handle_t* h);

/* Argument convention of the TER_HIP_SLOT_MATMUL native slot:
 *   args[0] = (const ter_hip_wpk_t*) W
 *   args[1] = (const ter_hip_act_t*) X
 *   args[2] = (float*)   y   (device, may be 0)
 *   args[3] = (int32_t*) acc (device, may be 0)
 *   args[4] = (hipStream_t) stream
 *   args[5] = M (rows; 1 = GEMV)
 * It bumps tvmac by ceil(K/27) * N * M, the analytic count mm_row reports
 * (src/tx/forward.cpp:349-350). */

/* ---------------------------------------------------------------------- */
/* Utilities                                                                */
/* ---------------------------------------------------------------------- */

/* Library version string. */
const char* ter_hip_version(void);
/* Text of the last error recorded by this thread (never NULL). */
const char* ter_hip_last_error(void);

/* Synthetic benchmark data, generated on the device from a counter-based
 * splitmix64 stream (element i = k*N + n of the [K][N] trit matrix draws
 * state seed + (i+1) * 0x9E3779B97F4A7C15).  u = top 32 bits; trit = 0 if
 * u < t0, +1 if u < t1, else -1.  Writes reference v11 bytes. */
int ter_hip_synth_v11(uint8_t* v11_dev, int32_t K, int32_t N, uint64_t seed,
                      uint32_t t0, uint32_t t1, void* stream);
/* int8 draws: x[i] = lo + ((u * (hi - lo + 1)) >> 32) with u as above. */
int ter_hip_synth_i8(int8_t* x_dev, int64_t n, uint64_t seed, int32_t lo, int32_t hi,
                     void* stream);

/* Measurement utilities (the floors bench.py reports beside the GEMV).
 * ter_hip_noop: one launch of an empty kernel (the launch floor).
 * ter_hip_read_probe: a pure streaming read of `bytes` (a multiple of 1024)
 * of device memory at `buf`, split as the GEMV splits its tile stream (n_wg
 * equal contiguous ranges, neighbouring ranges on one XCD, 4 waves per
 * workgroup with nontemporal 16-byte loads); `sink` receives 4 * n_wg
 * device words folded from the data.  No arithmetic: the ceiling of the
 * GEMV's streaming on the same bytes. */
int ter_hip_noop(void* stream);
int ter_hip_read_probe(const void* buf, size_t bytes, int32_t n_wg, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TER_HIP_H */
