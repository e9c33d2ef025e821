// ref_shim.cpp -- C entry points into the reference's own CPU code.
//
// TEST INFRASTRUCTURE ONLY (see ter_oracle.c).  oracle/Makefile compiles this
// file together with the reference sources where they lie under the reference
// tree (nothing is copied) into oracle/_ref/libter_ref.so.  The reference's
// mm_row has internal linkage (anonymous namespace, src/tx/forward.cpp:16-354),
// so this translation unit includes src/tx/forward.cpp itself; every other
// reference function it calls is linked from the reference's own objects.
//
// Entry points:
//   ter_ref_ctx_*          -- the reference mm_row (src/tx/forward.cpp:299-352)
//                             over caller-provided int32 payloads; the context
//                             builds the TritTensors once so timing covers
//                             mm_row only.
//   ter_ref_quantize       -- ter::quantize (src/numfmt/quantize.cpp:7-41).
//   ter_ref_quantize_bitnet-- ter::quantize_bitnet (include/ter/bitnet.hpp:11-28).
#include "tx/forward.cpp"

#include <ter/bitnet.hpp>

#include <cstdint>
#include <new>
#include <vector>

struct ter_ref_ctx {
    ter::TritTensor xt, wt;
    ter::Sim sim{64};
    ter::KernelTable kt;
    std::vector<float> out;
    int K = 0, N = 0, rows = 0;
};

extern "C" {

// X: int32 [rows][K]; W: int32 [K][N] (TritTensor payload orientation).
// block_size > 0 selects the per-block branch with block_scales.
ter_ref_ctx* ter_ref_ctx_new(const int32_t* X, int rows, int K, float xs,
                             const int32_t* W, int N, float ws,
                             const float* block_scales, int block_size) {
    ter_ref_ctx* c = new (std::nothrow) ter_ref_ctx();
    if (!c) return nullptr;
    c->K = K; c->N = N; c->rows = rows;
    c->xt.scale = xs;
    c->xt.shape = {rows, K};
    c->xt.payload.assign(X, X + static_cast<size_t>(rows) * static_cast<size_t>(K));
    c->wt.scale = ws;
    c->wt.shape = {K, N};
    c->wt.payload.assign(W, W + static_cast<size_t>(K) * static_cast<size_t>(N));
    if (block_size > 0) {
        const size_t nb = (static_cast<size_t>(K) * static_cast<size_t>(N) +
                           static_cast<size_t>(block_size) - 1) / static_cast<size_t>(block_size);
        c->wt.block_size = block_size;
        c->wt.block_scales.assign(block_scales, block_scales + nb);
    }
    return c;
}

int ter_ref_ctx_run(ter_ref_ctx* c, int row, float* out) {
    if (!c || !out || row < 0 || row >= c->rows) return -1;
    ter::tx::mm_row(c->sim, c->kt, ter::KernelId{}, c->xt, row, c->wt, c->K, c->N, c->out);
    for (int j = 0; j < c->N; ++j) out[j] = c->out[static_cast<size_t>(j)];
    return 0;
}

uint64_t ter_ref_ctx_tvmac(const ter_ref_ctx* c) {
    return c ? c->sim.counters().get(ter::Opcode::TVMAC) : 0;
}

void ter_ref_ctx_free(ter_ref_ctx* c) { delete c; }

float ter_ref_quantize(const float* data, int n, int n_trits, int32_t* payload) {
    ter::TritTensor t = ter::quantize(data, {n}, n_trits);
    for (int i = 0; i < n; ++i) payload[i] = t.payload[static_cast<size_t>(i)];
    return t.scale;
}

float ter_ref_quantize_bitnet(const float* in, int n, int8_t* out) {
    return ter::quantize_bitnet(in, static_cast<size_t>(n), out);
}

}  // extern "C"
