// moe_gpu_shim.hpp — the reference's MoE entry point on this library.
//
// Drop-in for `void moe_gpu(GPUTransformer *, int layer_idx, int batch_size,
// int row_offset, hipStream_t)` (getp-csrc/getp_run.cpp:2540, called from
// forward_batch_gpu at getp_run.cpp:3337 and :3353): x += MoE(RMSNorm(x)) on
// rows [row_offset, row_offset + batch_size) of the run state, in place, on
// the given stream (TP = 1).  getp_run.cpp includes this header in place of
// its own moe_gpu and calls moe_gpu_init once at warm-up; the batch loop is
// unchanged.  Header-only and templated on the transformer type, so it
// compiles against the reference's GPUTransformer (getp_run.cpp:46-212) or
// any type with the same member names: config.{hidden_dim,
// intermediate_dim, n_experts, experts_per_token, n_layers, swiglu_limit},
// weights.{rms_ffn_w, w_router, b_router, w_mlp1, w_mlp2, b_mlp1, b_mlp2,
// w_mlp1_mxfp4, w_mlp1_scales, w_mlp2_mxfp4, w_mlp2_scales},
// state.{x, t}.
//
// Weights.  The 120B path keeps MXFP4 MoE weights (w_mlp*_mxfp4 + scales,
// getp_run.cpp:704-721); they are packed once (gptoss_moe_pack_weights) and
// the forward reads only the packed copy.  The 20B path keeps bf16 MoE
// weights (w_mlp1 / w_mlp2, getp_run.cpp:833-972), which are exact
// dequantisations of the checkpoint's MXFP4 blocks: moe_gpu_init
// re-quantises them on the device with the reference's rule
// (gptoss_moe_quantize_mxfp4, mxfp4.hpp:112-217; lossless for such values),
// packs them and frees the temporaries, so each layer holds one packed copy.
//
// Errors: as the reference's HIP_CHECK (utils.hpp:11-20), a failed call
// prints and exits.  One state per device (the reference runs one host
// thread per GPU, getp_run.cpp:3514).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <vector>

#include "gptoss_moe.h"

namespace gptoss_moe_shim {

struct State {
    gptoss_moe_shape shape{};
    void *ws = nullptr;
    size_t ws_bytes = 0;
    int max_tokens = 0;
    bool mxfp4 = false;               // weights come from w_mlp*_mxfp4 (120B path)
    std::vector<uint8_t *> packed;    // one packed copy per layer
    bool ready = false;
};

inline State &state() {
    static State s[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    return s[dev];
}

inline void fail(const char *what, int rc) {
    fprintf(stderr, "moe_gpu: %s failed: %d (hip error %d)\n", what, rc, gptoss_moe_last_hip_error());
    exit(EXIT_FAILURE);
}

inline void hip_or_fail(hipError_t e, const char *what) {
    if (e != hipSuccess) {
        fprintf(stderr, "moe_gpu: %s: %s\n", what, hipGetErrorString(e));
        exit(EXIT_FAILURE);
    }
}

// bf16 -> fp32 (exact), for the 20B weights' re-quantisation.
__global__ void bf16_to_f32_kernel(const uint16_t *__restrict__ in, float *__restrict__ out, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = __uint_as_float((uint32_t)in[i] << 16);
}

// bf16 [n] -> MXFP4 nibbles [n / 2] + e8m0 [n / 32], through an fp32 staging
// buffer of `chunk` floats (a multiple of 32).
inline void quantize_bf16(const uint16_t *src, size_t n, uint8_t *q, uint8_t *s, float *stage,
                          size_t chunk, hipStream_t st) {
    for (size_t o = 0; o < n; o += chunk) {
        const size_t c = n - o < chunk ? n - o : chunk;
        hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(1024), dim3(256), 0, st, src + o, stage, c);
        hip_or_fail(hipGetLastError(), "bf16_to_f32_kernel");
        const int rc = gptoss_moe_quantize_mxfp4(stage, (int64_t)c, q + o / 2, s + o / 32, st);
        if (rc != GPTOSS_MOE_OK) fail("gptoss_moe_quantize_mxfp4", rc);
    }
}

// The library's weight view of layer l (per-layer strides of
// GPUTransformerWeights, getp_run.cpp:46-82): router [E][H] + [E], MXFP4 W1
// [E][2D][H] and W2 [E][H][D] (for the 120B path; NULL otherwise), biases.
template <class GPUTransformer>
gptoss_moe_weights layer_weights(GPUTransformer *gpu_t, int l, const State &S) {
    auto *w = &gpu_t->weights;
    const size_t H = S.shape.hidden, D = S.shape.intermediate, E = S.shape.n_experts;
    const size_t n1 = E * 2 * D * H, n2 = E * H * D;  // MoE weight elements per layer
    gptoss_moe_weights mw{};
    mw.router_w = reinterpret_cast<const uint16_t *>(w->w_router) + (size_t)l * E * H;
    mw.router_b = reinterpret_cast<const uint16_t *>(w->b_router) + (size_t)l * E;
    mw.b1 = reinterpret_cast<const uint16_t *>(w->b_mlp1) + (size_t)l * E * 2 * D;
    mw.b2 = reinterpret_cast<const uint16_t *>(w->b_mlp2) + (size_t)l * E * H;
    if (S.mxfp4) {
        mw.w1 = w->w_mlp1_mxfp4 + (size_t)l * (n1 / 2);
        mw.w1_scales = w->w_mlp1_scales + (size_t)l * (n1 / 32);
        mw.w2 = w->w_mlp2_mxfp4 + (size_t)l * (n2 / 2);
        mw.w2_scales = w->w_mlp2_scales + (size_t)l * (n2 / 32);
    }
    if (!S.packed.empty()) mw.packed = S.packed[l];
    return mw;
}

// Warm-up: workspace for up to max_tokens rows per call, and one packed copy
// of every layer's expert weights (weights_mxfp4: the 120B fields; else the
// 20B bf16 fields, re-quantised).  Allocates (warm-up only); synchronises.
template <class GPUTransformer>
void moe_gpu_init(GPUTransformer *gpu_t, int max_tokens, bool weights_mxfp4, hipStream_t st) {
    auto *p = &gpu_t->config;
    auto *w = &gpu_t->weights;
    State &S = state();
    S.shape = gptoss_moe_shape{p->hidden_dim, p->intermediate_dim, p->n_experts, p->experts_per_token,
                               p->swiglu_limit, 1.702f};
    S.mxfp4 = weights_mxfp4;
    S.max_tokens = max_tokens;
    S.ws_bytes = gptoss_moe_workspace_size(&S.shape, max_tokens);
    if (S.ws_bytes == 0) fail("gptoss_moe_workspace_size", GPTOSS_MOE_ERR_INVALID_ARG);
    hip_or_fail(hipMalloc(&S.ws, S.ws_bytes), "hipMalloc(workspace)");
    int rc = gptoss_moe_workspace_init(S.ws, S.ws_bytes, st);
    if (rc != GPTOSS_MOE_OK) fail("gptoss_moe_workspace_init", rc);

    const size_t H = S.shape.hidden, D = S.shape.intermediate, E = S.shape.n_experts;
    const size_t n1 = E * 2 * D * H, n2 = E * H * D;
    const size_t pbytes = gptoss_moe_packed_size(&S.shape);
    uint8_t *q1 = nullptr, *s1 = nullptr, *q2 = nullptr, *s2 = nullptr;
    float *stage = nullptr;
    const size_t chunk = (size_t)1 << 24;  // 64 MB of fp32 staging
    if (!S.mxfp4) {
        hip_or_fail(hipMalloc(&q1, n1 / 2), "hipMalloc");
        hip_or_fail(hipMalloc(&s1, n1 / 32), "hipMalloc");
        hip_or_fail(hipMalloc(&q2, n2 / 2), "hipMalloc");
        hip_or_fail(hipMalloc(&s2, n2 / 32), "hipMalloc");
        hip_or_fail(hipMalloc(&stage, chunk * sizeof(float)), "hipMalloc");
    }
    S.packed.assign(p->n_layers, nullptr);
    std::vector<uint8_t *> packed(p->n_layers, nullptr);
    for (int l = 0; l < p->n_layers; ++l) {
        gptoss_moe_weights mw = layer_weights(gpu_t, l, S);  // S.packed still all NULL
        mw.packed = nullptr;
        if (!S.mxfp4) {
            quantize_bf16(reinterpret_cast<const uint16_t *>(w->w_mlp1) + (size_t)l * n1, n1, q1, s1,
                          stage, chunk, st);
            quantize_bf16(reinterpret_cast<const uint16_t *>(w->w_mlp2) + (size_t)l * n2, n2, q2, s2,
                          stage, chunk, st);
            mw.w1 = q1;
            mw.w1_scales = s1;
            mw.w2 = q2;
            mw.w2_scales = s2;
        }
        hip_or_fail(hipMalloc(&packed[l], pbytes), "hipMalloc(packed)");
        rc = gptoss_moe_pack_weights(&S.shape, &mw, packed[l], pbytes, st);
        if (rc != GPTOSS_MOE_OK) fail("gptoss_moe_pack_weights", rc);
        // the temporaries are reused by the next layer
        hip_or_fail(hipStreamSynchronize(st), "hipStreamSynchronize");
    }
    if (!S.mxfp4) {
        (void)hipFree(q1);
        (void)hipFree(s1);
        (void)hipFree(q2);
        (void)hipFree(s2);
        (void)hipFree(stage);
    }
    S.packed = packed;
    S.ready = true;
}

}  // namespace gptoss_moe_shim

// The reference's signature (getp_run.cpp:2540).
template <class GPUTransformer>
void moe_gpu(GPUTransformer *gpu_t, int layer_idx, int batch_size, int row_offset, hipStream_t sMoe) {
    using namespace gptoss_moe_shim;
    if (batch_size <= 0) return;
    State &S = state();
    if (!S.ready) {
        fprintf(stderr, "moe_gpu: moe_gpu_init was not called on this device\n");
        exit(EXIT_FAILURE);
    }
    auto *s = &gpu_t->state;
    auto *w = &gpu_t->weights;
    const size_t H = S.shape.hidden;
    const gptoss_moe_weights mw = layer_weights(gpu_t, layer_idx, S);
    uint16_t *x = reinterpret_cast<uint16_t *>(s->x) + (size_t)row_offset * H;
    uint16_t *t = reinterpret_cast<uint16_t *>(s->t) + (size_t)row_offset * H;
    const uint16_t *rms = reinterpret_cast<const uint16_t *>(w->rms_ffn_w) + (size_t)layer_idx * H;
    const int rc = gptoss_moe_layer(&S.shape, &mw, rms, x, t, batch_size, S.ws, S.ws_bytes,
                                    S.max_tokens, sMoe);
    if (rc != GPTOSS_MOE_OK) fail("gptoss_moe_layer", rc);
}
