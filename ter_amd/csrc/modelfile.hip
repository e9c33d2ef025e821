// modelfile.hip -- host reader of the packed model files (.bin).
//
// Formats (written by tools/convert_bitnet_to_packed.py and
// tools/convert_llama_to_packed.py; read by the two load_model_from_bin,
// cuda/ter_cuda_forward_bitnet.cu:698-784 and
// cuda/ter_cuda_forward_packed.cu:589-659), little endian:
//   header, 64 bytes: magic, version (1), H, F, Nl, V, Nh, Nkv, Hd, Smax
//                     (uint32), rope_theta, eps (fp32), zero padding
//   token_embd        fp16 [V][H]
//   output_norm       fp32 [H]
//   per layer         fp32 attn_norm [H], ffn_norm [H]
//                     ('TERT' only: attn_sub_norm [H], ffn_sub_norm [F])
//                     Wq (K=H, N=H), Wk (H, Nkv*Hd), Wv (H, Nkv*Hd), Wo (H, H),
//                     Wgate (H, F), Wup (H, F), Wdown (F, H): each K*(N/4)
//                     v11 bytes, then its fp32 scale
// The reference loaders read the blob front to back and trust the header;
// this reader builds the tensor directory from the header first and refuses
// a file whose size differs from what the header implies, so a truncated or
// mismatched file fails at open rather than midway through a load.
#include <cstdio>
#include <cstring>
#include <vector>

#include "common.h"

struct ter_hip_bin {
    std::FILE* fp = nullptr;
    ter_hip_bin_header_t hdr{};
    std::vector<ter_hip_bin_tensor_t> dir;
};

namespace terhip {
namespace {

bool read_at(std::FILE* fp, int64_t off, void* dst, size_t n) {
    if (fseeko(fp, (off_t)off, SEEK_SET) != 0) return false;
    return std::fread(dst, 1, n, fp) == n;
}

// fp32 -> fp16, round to nearest even (the loaders' __float2half on the host).
uint16_t half_of(float f) {
    const _Float16 h = (_Float16)f;
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

void add(std::vector<ter_hip_bin_tensor_t>& dir, int64_t& off, const char* name, int layer, int kind, int64_t n,
         int K = 0, int N = 0) {
    ter_hip_bin_tensor_t t{};
    std::snprintf(t.name, sizeof t.name, "%s", name);
    t.layer = layer;
    t.kind = kind;
    t.offset = off;
    t.n = n;
    t.K = K;
    t.N = N;
    t.bytes = kind == TER_HIP_BIN_F16 ? 2 * n : (kind == TER_HIP_BIN_F32 ? 4 * n : (int64_t)K * (N / 4));
    off += t.bytes + (kind == TER_HIP_BIN_TRITS ? 4 : 0);
    dir.push_back(t);
}

int check_index(const ter_hip_bin_t* bin, int32_t i) {
    if (!bin) return fail(TER_HIP_ERR_NULL, "null model file");
    if (i < 0 || i >= (int32_t)bin->dir.size()) return fail(TER_HIP_ERR_NOTFOUND, "tensor index %d out of range", i);
    return TER_HIP_OK;
}

}  // namespace
}  // namespace terhip

using namespace terhip;

extern "C" {

int ter_hip_bin_open(const char* path, ter_hip_bin_t** out, ter_hip_bin_header_t* header) {
    if (!path || !out) return fail(TER_HIP_ERR_NULL, "null path or handle");
    *out = nullptr;
    std::FILE* fp = std::fopen(path, "rb");
    if (!fp) return fail(TER_HIP_ERR_FILE, "cannot open %s", path);
    unsigned char raw[64];
    if (std::fread(raw, 1, sizeof raw, fp) != sizeof raw) {
        std::fclose(fp);
        return fail(TER_HIP_ERR_FILE, "%s: shorter than the 64-byte header", path);
    }
    ter_hip_bin_header_t h{};
    uint32_t u[10];
    std::memcpy(u, raw, sizeof u);
    h.magic = u[0];
    h.version = u[1];
    h.H = u[2];
    h.F = u[3];
    h.Nl = u[4];
    h.V = u[5];
    h.Nh = u[6];
    h.Nkv = u[7];
    h.Hd = u[8];
    h.Smax = u[9];
    std::memcpy(&h.rope_theta, raw + 40, 4);
    std::memcpy(&h.eps, raw + 44, 4);
    const bool tert = h.magic == TER_HIP_BIN_TERT;
    if ((!tert && h.magic != TER_HIP_BIN_LLRT) || h.version != 1) {
        std::fclose(fp);
        return fail(TER_HIP_ERR_FILE, "%s: bad magic/version 0x%08x v%u (expected 'TERT' or 'LLRT' v1)", path,
                    h.magic, h.version);
    }
    const uint32_t hkv = h.Nkv * h.Hd;
    if (h.H < 4 || h.F < 4 || h.Nl < 1 || h.V < 1 || h.Nh < 1 || h.Nkv < 1 || h.Hd < 1 || h.H % 4 || h.F % 4 ||
        hkv % 4 || h.H > (1u << 20) || h.F > (1u << 20) || hkv > (1u << 20) || h.Nl > 4096 || h.V > (1u << 24)) {
        std::fclose(fp);
        return fail(TER_HIP_ERR_SHAPE, "%s: unsupported shape H=%u F=%u Nl=%u V=%u Nh=%u Nkv=%u Hd=%u", path, h.H,
                    h.F, h.Nl, h.V, h.Nh, h.Nkv, h.Hd);
    }
    ter_hip_bin* b = new (std::nothrow) ter_hip_bin();
    if (!b) {
        std::fclose(fp);
        return fail(TER_HIP_ERR_ALLOC, "model file handle");
    }
    b->fp = fp;
    b->hdr = h;
    const int H = (int)h.H, F = (int)h.F, Hkv = (int)hkv;
    int64_t off = 64;
    add(b->dir, off, "token_embd", -1, TER_HIP_BIN_F16, (int64_t)h.V * H);
    add(b->dir, off, "output_norm", -1, TER_HIP_BIN_F32, H);
    for (int l = 0; l < (int)h.Nl; ++l) {
        add(b->dir, off, "attn_norm", l, TER_HIP_BIN_F32, H);
        add(b->dir, off, "ffn_norm", l, TER_HIP_BIN_F32, H);
        if (tert) {
            add(b->dir, off, "attn_sub_norm", l, TER_HIP_BIN_F32, H);
            add(b->dir, off, "ffn_sub_norm", l, TER_HIP_BIN_F32, F);
        }
        add(b->dir, off, "Wq", l, TER_HIP_BIN_TRITS, 0, H, H);
        add(b->dir, off, "Wk", l, TER_HIP_BIN_TRITS, 0, H, Hkv);
        add(b->dir, off, "Wv", l, TER_HIP_BIN_TRITS, 0, H, Hkv);
        add(b->dir, off, "Wo", l, TER_HIP_BIN_TRITS, 0, H, H);
        add(b->dir, off, "Wgate", l, TER_HIP_BIN_TRITS, 0, H, F);
        add(b->dir, off, "Wup", l, TER_HIP_BIN_TRITS, 0, H, F);
        add(b->dir, off, "Wdown", l, TER_HIP_BIN_TRITS, 0, F, H);
    }
    int64_t size = -1;
    if (fseeko(fp, 0, SEEK_END) == 0) size = (int64_t)ftello(fp);
    if (size != off) {
        ter_hip_bin_close(b);
        return fail(TER_HIP_ERR_FILE, "%s: %lld bytes, the header implies %lld", path, (long long)size,
                    (long long)off);
    }
    for (auto& t : b->dir) {
        if (t.kind != TER_HIP_BIN_TRITS) continue;
        if (!read_at(fp, t.offset + t.bytes, &t.scale, 4)) {
            ter_hip_bin_close(b);
            return fail(TER_HIP_ERR_FILE, "%s: cannot read the scale of %s (layer %d)", path, t.name, t.layer);
        }
    }
    if (header) *header = h;
    *out = b;
    return TER_HIP_OK;
}

int32_t ter_hip_bin_count(const ter_hip_bin_t* bin) {
    if (!bin) return fail(TER_HIP_ERR_NULL, "null model file");
    return (int32_t)bin->dir.size();
}

int ter_hip_bin_tensor(const ter_hip_bin_t* bin, int32_t i, ter_hip_bin_tensor_t* out) {
    int rc = check_index(bin, i);
    if (rc) return rc;
    if (!out) return fail(TER_HIP_ERR_NULL, "null output");
    *out = bin->dir[(size_t)i];
    return TER_HIP_OK;
}

int32_t ter_hip_bin_find(const ter_hip_bin_t* bin, const char* name, int32_t layer) {
    if (!bin || !name) return fail(TER_HIP_ERR_NULL, "null model file or name");
    for (size_t i = 0; i < bin->dir.size(); ++i)
        if (bin->dir[i].layer == layer && std::strcmp(bin->dir[i].name, name) == 0) return (int32_t)i;
    return fail(TER_HIP_ERR_NOTFOUND, "no tensor %s in layer %d", name, layer);
}

int ter_hip_bin_read_host(const ter_hip_bin_t* bin, int32_t i, void* dst, int32_t as_f16) {
    int rc = check_index(bin, i);
    if (rc) return rc;
    if (!dst) return fail(TER_HIP_ERR_NULL, "null destination");
    const ter_hip_bin_tensor_t& t = bin->dir[(size_t)i];
    if (t.kind == TER_HIP_BIN_F32 && as_f16) {
        std::vector<float> f((size_t)t.n);
        if (!read_at(bin->fp, t.offset, f.data(), (size_t)t.bytes))
            return fail(TER_HIP_ERR_FILE, "short read of %s (layer %d)", t.name, t.layer);
        uint16_t* o = static_cast<uint16_t*>(dst);
        for (size_t k = 0; k < f.size(); ++k) o[k] = half_of(f[k]);
        return TER_HIP_OK;
    }
    if (!read_at(bin->fp, t.offset, dst, (size_t)t.bytes))
        return fail(TER_HIP_ERR_FILE, "short read of %s (layer %d)", t.name, t.layer);
    return TER_HIP_OK;
}

int ter_hip_bin_upload_f16(const ter_hip_bin_t* bin, int32_t i, uint16_t* dst_dev, void* stream) {
    int rc = check_index(bin, i);
    if (rc) return rc;
    if (!dst_dev) return fail(TER_HIP_ERR_NULL, "null destination");
    const ter_hip_bin_tensor_t& t = bin->dir[(size_t)i];
    if (t.kind == TER_HIP_BIN_TRITS) return fail(TER_HIP_ERR_PAYLOAD, "%s is a projection, not an fp16 vector", t.name);
    std::vector<uint16_t> h((size_t)t.n);
    rc = ter_hip_bin_read_host(bin, i, h.data(), 1);
    if (rc) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(dst_dev, h.data(), h.size() * 2, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);  // (the staging vector ends here)
    if (e != hipSuccess) return hip_fail(e, "model tensor upload");
    return TER_HIP_OK;
}

int ter_hip_bin_upload_wpk(const ter_hip_bin_t* bin, int32_t i, ter_hip_wpk_t* w, uint8_t* v11_stage_dev,
                           void* stream) {
    int rc = check_index(bin, i);
    if (rc) return rc;
    if (!w || !v11_stage_dev) return fail(TER_HIP_ERR_NULL, "null weight or staging buffer");
    const ter_hip_bin_tensor_t& t = bin->dir[(size_t)i];
    if (t.kind != TER_HIP_BIN_TRITS) return fail(TER_HIP_ERR_PAYLOAD, "%s is not a projection", t.name);
    if (w->K != t.K || w->N != t.N)
        return fail(TER_HIP_ERR_SHAPE, "%s (layer %d) is %d x %d, the weight handle %d x %d", t.name, t.layer, t.K,
                    t.N, w->K, w->N);
    std::vector<uint8_t> h((size_t)t.bytes);
    rc = ter_hip_bin_read_host(bin, i, h.data(), 0);
    if (rc) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(v11_stage_dev, h.data(), h.size(), hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return hip_fail(e, "projection upload");
    w->scale = t.scale;
    rc = ter_hip_pack_v11(w, v11_stage_dev, stream);
    if (rc) return rc;
    e = hipStreamSynchronize(st);  // (the staging vector ends here)
    if (e != hipSuccess) return hip_fail(e, "projection repack");
    return TER_HIP_OK;
}

void ter_hip_bin_close(ter_hip_bin_t* bin) {
    if (!bin) return;
    if (bin->fp) std::fclose(bin->fp);
    delete bin;
}

}  // extern "C"
