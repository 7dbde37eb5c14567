// attn_gpu_shim.hpp — steps 5 and 6 of the reference's attention_gpu_120b /
// attention_gpu on this library.
//
// Drop-in for the block of attention_gpu_120b (getp-csrc/getp_run.cpp:
// 2311-2470: quantize_kv_cache_kernel_int8 / _bf16 and the int8 flash-decoding
// kernels) or of attention_gpu (:2096-2160, the 20B path: update_kv_cache_kernel
// and ..._full_bf16kv_okay on the bf16 cache) that updates the KV cache and
// runs the fused flash-decoding kernel: `attention_cache_and_decode(gpu_t,
// layer_idx, batch_size, row_offset, stream)` does both for rows
// [row_offset, row_offset + batch_size) of the run state, reading the query,
// key and value that steps 1-4 left in state.{q, k, v} and writing state.tb,
// in stream order.  The rest of attention_gpu (RMSNorm, QKV, bias, RoPE,
// output projection) is unchanged.  Header-only and templated on the
// transformer type, so it compiles against the reference's GPUTransformer
// (getp_run.cpp:46-212) or any type with the same member names:
// config.{n_layers, n_attn_heads, n_kv_heads, head_dim, sliding_window},
// weights.attn_sinks, state.{q, k, v, tb, positions, key_cache, value_cache,
// key_cache_scales, value_cache_scales, key_cache_recent_bf16,
// value_cache_recent_bf16, key_cache_bf16, value_cache_bf16}.
//
// The caches keep the reference's allocations and per-layer offsets
// (getp_run.cpp:2195-2230); the byte order inside each 16-row block is this
// library's (gptoss_attn.h), so the shim must be the only code that touches
// them, as attention_gpu's two kernels are in the reference.
//
// Errors: as the reference's HIP_CHECK (utils.hpp:11-20), a failed call prints
// and exits.  One state per device.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "gptoss_attn.h"

namespace gptoss_attn_shim {

struct State {
    gptoss_attn_shape shape{};
    int max_seq_len = 0;   // MAX_SEQ_LEN: rows of odd layers
    int sw_window = 0;     // SW_WINDOW: rows of even layers (sliding_window > 0)
    void *ws = nullptr;    // token-split workspace (small batches)
    size_t ws_bytes = 0;
    bool ready = false;
};

inline State &state() {
    static State s[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    return s[dev];
}

inline void fail(const char *what, int rc) {
    fprintf(stderr, "attention: %s failed: %d (hip error %d)\n", what, rc, gptoss_attn_last_hip_error());
    exit(EXIT_FAILURE);
}

// Warm-up: the model's shape, the reference's compile-time MAX_SEQ_LEN,
// SW_WINDOW and KV_BF16_KEEP_TOKENS, the token source rule of the kept
// tokens (GPTOSS_ATTN_PREFIX_*), the cache kind (GPTOSS_ATTN_CACHE_INT8 for
// attention_gpu_120b's caches, GPTOSS_ATTN_CACHE_BF16 for attention_gpu's
// key_cache_bf16 / value_cache_bf16), and a workspace for up to max_batch
// sequences.  Allocates (warm-up only).
template <class GPUTransformer>
void attn_gpu_init(GPUTransformer *gpu_t, int max_batch, int max_seq_len, int sw_window, int keep,
                   int prefix_rule, int cache_kind = GPTOSS_ATTN_CACHE_INT8) {
    auto *p = &gpu_t->config;
    State &S = state();
    S.shape = gptoss_attn_shape{p->n_attn_heads, p->n_kv_heads, p->head_dim, p->n_layers,
                                p->sliding_window > 0 ? sw_window : 0,
                                cache_kind == GPTOSS_ATTN_CACHE_BF16 ? 0 : keep, prefix_rule, cache_kind};
    S.max_seq_len = max_seq_len;
    S.sw_window = sw_window;
    S.ws_bytes = gptoss_attn_workspace_size(&S.shape, max_seq_len, max_batch);
    if (S.ws_bytes && hipMalloc(&S.ws, S.ws_bytes) != hipSuccess) fail("hipMalloc(workspace)", GPTOSS_ATTN_ERR_HIP);
    S.ready = true;
}

}  // namespace gptoss_attn_shim

// Steps 5) and 6) of attention_gpu_120b (getp_run.cpp:2311-2470) or
// attention_gpu (:2096-2160).
template <class GPUTransformer>
void attention_cache_and_decode(GPUTransformer *gpu_t, int layer_idx, int batch_size, int row_offset,
                                hipStream_t sAttn) {
    using namespace gptoss_attn_shim;
    if (batch_size <= 0) return;
    State &S = state();
    if (!S.ready) {
        fprintf(stderr, "attention: attn_gpu_init was not called on this device\n");
        exit(EXIT_FAILURE);
    }
    auto *p = &gpu_t->config;
    auto *s = &gpu_t->state;
    auto *w = &gpu_t->weights;
    const int KV = p->head_dim * p->n_kv_heads;
    const int NA = p->n_attn_heads;
    // per-sequence rows of every layer and this layer's offset (getp_run.cpp:2195-2220)
    const int even_cap = p->sliding_window > 0 ? S.sw_window : S.max_seq_len;
    size_t layers_capacity = 0, layer_pos_offset = 0;
    for (int L = 0; L < p->n_layers; ++L) {
        const size_t cap = (L & 1) == 0 ? (size_t)even_cap : (size_t)S.max_seq_len;
        if (L < layer_idx) layer_pos_offset += cap;
        layers_capacity += cap;
    }
    const size_t kv_slice = layers_capacity * (size_t)KV;
    const size_t recent_slice = (size_t)p->n_layers * (size_t)S.shape.keep * (size_t)KV;
    gptoss_attn_cache cache{};
    if (S.shape.cache_kind == GPTOSS_ATTN_CACHE_BF16) {  // attention_gpu's bf16 rows (getp_run.cpp:2052-2053)
        cache.key_codes = reinterpret_cast<int8_t *>(s->key_cache_bf16 + (size_t)row_offset * kv_slice);
        cache.value_codes = reinterpret_cast<int8_t *>(s->value_cache_bf16 + (size_t)row_offset * kv_slice);
    } else {
        cache.key_codes = reinterpret_cast<int8_t *>(s->key_cache) + (size_t)row_offset * kv_slice;
        cache.value_codes = reinterpret_cast<int8_t *>(s->value_cache) + (size_t)row_offset * kv_slice;
        cache.key_scales = reinterpret_cast<uint16_t *>(s->key_cache_scales) + (size_t)row_offset * layers_capacity;
        cache.value_scales = reinterpret_cast<uint16_t *>(s->value_cache_scales) + (size_t)row_offset * layers_capacity;
    }
    if (S.shape.keep > 0) {
        cache.key_bf16 = reinterpret_cast<uint16_t *>(s->key_cache_recent_bf16) + (size_t)row_offset * recent_slice;
        cache.value_bf16 = reinterpret_cast<uint16_t *>(s->value_cache_recent_bf16) + (size_t)row_offset * recent_slice;
    }
    cache.batch_kv_stride = kv_slice;
    cache.batch_scale_stride = layers_capacity;
    gptoss_attn_layer lay{};
    lay.layer_idx = layer_idx;
    lay.cap = (layer_idx & 1) == 0 ? even_cap : S.max_seq_len;
    lay.layer_kv_offset = layer_pos_offset * (size_t)KV;
    lay.layer_scale_offset = layer_pos_offset;
    const int32_t *pos = s->positions + row_offset;
    int rc = gptoss_attn_kv_update(&S.shape, &cache, &lay,
                                   reinterpret_cast<const uint16_t *>(s->k) + (size_t)row_offset * KV,
                                   reinterpret_cast<const uint16_t *>(s->v) + (size_t)row_offset * KV, pos,
                                   batch_size, sAttn);
    if (rc != GPTOSS_ATTN_OK) fail("gptoss_attn_kv_update", rc);
    const size_t qd = (size_t)NA * p->head_dim;
    rc = gptoss_attn_decode(&S.shape, &cache, &lay,
                            reinterpret_cast<const uint16_t *>(s->q) + (size_t)row_offset * qd,
                            reinterpret_cast<const uint16_t *>(w->attn_sinks) + (size_t)layer_idx * NA, pos,
                            batch_size, reinterpret_cast<uint16_t *>(s->tb) + (size_t)row_offset * qd, S.ws,
                            S.ws_bytes, sAttn);
    if (rc != GPTOSS_ATTN_OK) fail("gptoss_attn_decode", rc);
}
