// bin_loader.cpp — the reference's fp32 checkpoint (.bin) into this library's
// MoE buffers, one layer at a time (host code; the MXFP4 quantisation runs on
// the GPU through gptoss_moe_quantize_mxfp4).
//
// File layout (run.cpp:206-296, load_checkpoint + memory_map_weights): the
// Config struct (run.cpp:25-45, 15 x 4 bytes), then fp32 arrays back to back:
// token embedding [V][H], unembedding [V][H], rms_attn_w [L][H], rms_ffn_w
// [L][H], rms_out_w [H], w_qkv [L][H][(nh + 2 nkv) hd], b_qkv, w_o, b_o [L][H],
// attn_sinks [L][nh], w_router [L][E][H], b_router [L][E], w_mlp1
// [L][E][2D][H] (gate/up rows interleaved), b_mlp1 [L][E][2D], w_mlp2
// [L][E][H][D], b_mlp2 [L][E][H].
//
// The reference's GPU loader converts the router, biases and RMSNorm weight
// to bf16 with __float2bfloat16 (getp_run.cpp:818-830, utils.hpp:23-29) and
// quantises w_mlp1 / w_mlp2 per layer with quantize_pack_mxfp4_block32_kernel
// in chunks through pinned + device staging (getp_run.cpp:1140-1240); this
// loader does the same with caller-owned staging buffers.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "../../include/gptoss_moe.h"

namespace {

// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN with its sign.
uint16_t host_f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

struct Mapped {
    const uint8_t *p = nullptr;
    size_t n = 0;
    int fd = -1;
    ~Mapped() {
        if (p) munmap(const_cast<uint8_t *>(p), n);
        if (fd >= 0) close(fd);
    }
    bool open_file(const char *path) {
        fd = ::open(path, O_RDONLY);
        if (fd < 0) return false;
        struct stat st;
        if (fstat(fd, &st) != 0 || st.st_size <= 0) return false;
        n = (size_t)st.st_size;
        void *m = mmap(nullptr, n, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) return false;
        p = static_cast<const uint8_t *>(m);
        return true;
    }
};

int hip_rc(hipError_t e) { return e == hipSuccess ? GPTOSS_MOE_OK : GPTOSS_MOE_ERR_HIP; }

// fp32 elements [src, src + n) -> bf16 at dst (device), through the staging.
int upload_bf16(const float *src, size_t n, uint16_t *dst, void *stage_host, size_t stage_bytes,
                hipStream_t st) {
    const size_t chunk = stage_bytes / 2;
    uint16_t *h = static_cast<uint16_t *>(stage_host);
    for (size_t o = 0; o < n; o += chunk) {
        const size_t m = n - o < chunk ? n - o : chunk;
        for (size_t i = 0; i < m; ++i) h[i] = host_f2bf(src[o + i]);
        int rc = hip_rc(hipMemcpyAsync(dst + o, h, m * 2, hipMemcpyHostToDevice, st));
        if (!rc) rc = hip_rc(hipStreamSynchronize(st));  // the host staging is reused
        if (rc) return rc;
    }
    return GPTOSS_MOE_OK;
}

// fp32 elements [src, src + n) (n a multiple of 32) -> MXFP4 at packed / scales.
int upload_mxfp4(const float *src, size_t n, uint8_t *packed, uint8_t *scales, void *stage_host,
                 void *stage_dev, size_t stage_bytes, hipStream_t st) {
    const size_t chunk = stage_bytes / 4 / 32 * 32;
    for (size_t o = 0; o < n; o += chunk) {
        const size_t m = n - o < chunk ? n - o : chunk;
        memcpy(stage_host, src + o, m * 4);
        int rc = hip_rc(hipMemcpyAsync(stage_dev, stage_host, m * 4, hipMemcpyHostToDevice, st));
        if (rc) return rc;
        rc = gptoss_moe_quantize_mxfp4(static_cast<const float *>(stage_dev), (int64_t)m,
                                       packed + o / 2, scales + o / 32, st);
        if (!rc) rc = hip_rc(hipStreamSynchronize(st));
        if (rc) return rc;
    }
    return GPTOSS_MOE_OK;
}

}  // namespace

extern "C" {

int gptoss_moe_bin_read_config(const char *path, gptoss_moe_bin_config *cfg) {
    if (!path || !cfg) return GPTOSS_MOE_ERR_INVALID_ARG;
    Mapped m;
    if (!m.open_file(path) || m.n < sizeof(gptoss_moe_bin_config)) return GPTOSS_MOE_ERR_INVALID_ARG;
    memcpy(cfg, m.p, sizeof(gptoss_moe_bin_config));
    return GPTOSS_MOE_OK;
}

int gptoss_moe_bin_layer_offsets(const gptoss_moe_bin_config *c, int layer,
                                 gptoss_moe_bin_layer *o) {
    if (!c || !o) return GPTOSS_MOE_ERR_INVALID_ARG;
    if (c->vocab_size <= 0 || c->hidden_dim <= 0 || c->n_experts <= 0 || c->intermediate_dim <= 0 ||
        c->n_layers <= 0 || c->head_dim <= 0 || c->n_attn_heads <= 0 || c->n_kv_heads < 0 ||
        layer < 0 || layer >= c->n_layers)
        return GPTOSS_MOE_ERR_INVALID_ARG;
    const int64_t V = c->vocab_size, H = c->hidden_dim, E = c->n_experts, D = c->intermediate_dim;
    const int64_t L = c->n_layers, hd = c->head_dim, nh = c->n_attn_heads, nkv = c->n_kv_heads;
    const int64_t qkv = hd * nh + 2 * hd * nkv;
    int64_t f = 0;  // fp32 elements after the header
    f += V * H;                                // token_embedding_table
    f += V * H;                                // out
    f += L * H;                                // rms_attn_w
    const int64_t rms_ffn = f;
    f += L * H;                                // rms_ffn_w
    f += H;                                    // rms_out_w
    f += L * H * qkv;                          // w_qkv
    f += L * qkv;                              // b_qkv
    f += L * (hd * nh) * H;                    // w_o
    f += L * H;                                // b_o
    f += L * nh;                               // attn_sinks
    const int64_t w_router = f;
    f += L * H * E;
    const int64_t b_router = f;
    f += L * E;
    const int64_t w_mlp1 = f;
    f += L * E * 2 * D * H;
    const int64_t b_mlp1 = f;
    f += L * E * 2 * D;
    const int64_t w_mlp2 = f;
    f += L * E * H * D;
    const int64_t b_mlp2 = f;
    f += L * E * H;
    const int64_t hdr = (int64_t)sizeof(gptoss_moe_bin_config), l = layer;
    o->rms_ffn_w = hdr + 4 * (rms_ffn + l * H);
    o->w_router = hdr + 4 * (w_router + l * E * H);
    o->b_router = hdr + 4 * (b_router + l * E);
    o->w_mlp1 = hdr + 4 * (w_mlp1 + l * E * 2 * D * H);
    o->b_mlp1 = hdr + 4 * (b_mlp1 + l * E * 2 * D);
    o->w_mlp2 = hdr + 4 * (w_mlp2 + l * E * H * D);
    o->b_mlp2 = hdr + 4 * (b_mlp2 + l * E * H);
    o->file_bytes = hdr + 4 * f;
    return GPTOSS_MOE_OK;
}

int gptoss_moe_load_bin_layer(const char *path, int layer, const gptoss_moe_bin_dest *dst,
                              void *stage_host, void *stage_dev, size_t stage_bytes,
                              hipStream_t stream) {
    if (!path || !dst || !stage_host || !stage_dev || stage_bytes < 4096 || stage_bytes % 128)
        return GPTOSS_MOE_ERR_INVALID_ARG;
    if (!dst->w1 || !dst->w1_scales || !dst->b1 || !dst->w2 || !dst->w2_scales || !dst->b2 ||
        !dst->router_w || !dst->router_b)
        return GPTOSS_MOE_ERR_INVALID_ARG;
    Mapped m;
    if (!m.open_file(path) || m.n < sizeof(gptoss_moe_bin_config)) return GPTOSS_MOE_ERR_INVALID_ARG;
    gptoss_moe_bin_config c;
    memcpy(&c, m.p, sizeof(c));
    gptoss_moe_bin_layer o;
    int rc = gptoss_moe_bin_layer_offsets(&c, layer, &o);
    if (rc) return rc;
    if ((size_t)o.file_bytes > m.n) return GPTOSS_MOE_ERR_INVALID_ARG;  // truncated file
    const size_t H = c.hidden_dim, E = c.n_experts, D = c.intermediate_dim;
    if (H % 64 || D % 64) return GPTOSS_MOE_ERR_UNSUPPORTED;
    auto at = [&](int64_t off) { return reinterpret_cast<const float *>(m.p + off); };
    if ((rc = upload_mxfp4(at(o.w_mlp1), E * 2 * D * H, dst->w1, dst->w1_scales, stage_host,
                           stage_dev, stage_bytes, stream)) != 0)
        return rc;
    if ((rc = upload_mxfp4(at(o.w_mlp2), E * H * D, dst->w2, dst->w2_scales, stage_host, stage_dev,
                           stage_bytes, stream)) != 0)
        return rc;
    if ((rc = upload_bf16(at(o.b_mlp1), E * 2 * D, dst->b1, stage_host, stage_bytes, stream)) != 0)
        return rc;
    if ((rc = upload_bf16(at(o.b_mlp2), E * H, dst->b2, stage_host, stage_bytes, stream)) != 0)
        return rc;
    if ((rc = upload_bf16(at(o.w_router), E * H, dst->router_w, stage_host, stage_bytes, stream)) != 0)
        return rc;
    if ((rc = upload_bf16(at(o.b_router), E, dst->router_b, stage_host, stage_bytes, stream)) != 0)
        return rc;
    if (dst->rms_ffn_w &&
        (rc = upload_bf16(at(o.rms_ffn_w), H, dst->rms_ffn_w, stage_host, stage_bytes, stream)) != 0)
        return rc;
    return GPTOSS_MOE_OK;
}

}  // extern "C"
