/*
 * gptoss_attn.h — C ABI of the MI355X (gfx950) decode attention over an int8
 * KV cache: the attention half of a gpt-oss decoder layer, next to the MoE
 * layer of gptoss_moe.h.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream,
 * returns an int status (0 = ok, negative = error), never exits, allocates
 * nothing and does not synchronise the host.
 *
 * Scope (what the reference's GPU decode paths compute per layer): the
 * KV-cache update of the current token and the attention of one query token
 * per sequence with learned sinks, a sliding window on even layers and GQA,
 * over either cache the reference keeps:
 *   int8 (attention_gpu_120b, getp-csrc/getp_run.cpp:2181-2481):
 *     quantize_kv_cache_kernel_{int8,bf16} (kernels/attention.hpp:536-720)
 *     and flashdecoding_fused_fastmerge_nostage_1warp8q_bf16q_bf16out
 *     {,_bf16kv} (kernels/attention_mfma.hpp:1113-1460);
 *   bf16 (attention_gpu, getp_run.cpp:2008-2180, the 20B model):
 *     update_kv_cache_kernel (attention.hpp:756-778) and
 *     flashdecoding_fused_fastmerge_nostage_1warp8q_bf16q_bf16out_full_bf16kv
 *     _okay (attention_mfma.hpp:1679-1900).
 * gpt-oss shapes only: 64 query heads, 8 KV heads, head_dim 64.
 *
 * Cache memory.  The allocations, strides and per-layer offsets are the
 * reference's (GPURunState.key_cache / value_cache / key_cache_scales /
 * value_cache_scales / key_cache_recent_bf16 / value_cache_recent_bf16,
 * getp_run.cpp:104-112, :443-486): per sequence b, layer l owns `cap` rows of
 * kv_dim = 512 values (int8 codes, or bf16 with GPTOSS_ATTN_CACHE_BF16) at
 * element offset
 *     b * batch_kv_stride + layer_kv_offset,
 * one fp16 scale per row at  b * batch_scale_stride + layer_scale_offset,
 * and (odd layers, keep > 0) `keep` bf16 rows at
 *     ((b * n_layers + l) * keep) * kv_dim.
 * Row of the token at position pos: pos % sliding_window on even layers when
 * sliding_window > 0 (a ring), pos otherwise (getp_run.cpp:2316-2318,
 * attention.hpp:582).  Inside a layer's rows the bytes are grouped in blocks
 * of 16 rows, one 1 KiB tile per KV head, ordered so that one 16-byte load
 * per lane brings a wave a whole tile in the register layout of its matrix
 * instructions (the reference keeps [row][kv_dim]):
 *     key   (row r, head g, dim d):  ((r/16)*8 + g)*1024 + (r%16)*64 + d
 *     value (row r, head g, dim d):  ((r/16)*8 + g)*1024 + (d%16)*64
 *                                     + ((r%16)/4)*16 + (d/16)*4 + r%4
 * in bytes for the int8 codes and in elements for the bf16 rows.  Only
 * gptoss_attn_kv_update writes these caches and only gptoss_attn_decode
 * reads them, as in the reference, where the quantize and attention kernels
 * are the only users of GPURunState's caches.
 *
 * Values: bf16 and fp16 are passed as uint16_t bit patterns.
 */
#ifndef GPTOSS_ATTN_H
#define GPTOSS_ATTN_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GPTOSS_ATTN_OK 0
#define GPTOSS_ATTN_ERR_INVALID_ARG (-1)   /* bad shape, pointer, stride or flag */
#define GPTOSS_ATTN_ERR_WORKSPACE (-2)     /* workspace misaligned */
#define GPTOSS_ATTN_ERR_HIP (-3)           /* a HIP call failed; see gptoss_attn_last_hip_error */

/* Token source of odd layers' first `keep` tokens.
 * REFERENCE: every token comes from the bf16 rows while pos < keep, from the
 *   int8 rows once pos >= keep (attention_mfma.hpp:1160-1172, the rule of
 *   getp_run.cpp:2253-2276).
 * MIXED: tokens t < keep always come from the bf16 rows, later ones from
 *   int8 (keeps the first tokens exact at every position). */
#define GPTOSS_ATTN_PREFIX_REFERENCE 0
#define GPTOSS_ATTN_PREFIX_MIXED 1

/* Cache kind.  INT8: codes + fp16 scales per row (+ the bf16-kept rows of
 * odd layers).  BF16: the rows themselves in bf16 (key_codes / value_codes
 * then point to uint16_t bf16 elements, same element offsets and tile
 * order; scales, keep and the bf16-kept rows are not used). */
#define GPTOSS_ATTN_CACHE_INT8 0
#define GPTOSS_ATTN_CACHE_BF16 1

/* Model shape (run.cpp Config fields; getp_run.cpp's compile-time
 * SW_WINDOW and KV_BF16_KEEP_TOKENS). */
typedef struct gptoss_attn_shape {
    int n_heads;         /* Config.n_attn_heads: 64 */
    int n_kv_heads;      /* Config.n_kv_heads: 8 */
    int head_dim;        /* Config.head_dim: 64 */
    int n_layers;        /* Config.n_layers (strides the bf16 rows) */
    int sliding_window;  /* Config.sliding_window (ring rows of even layers): 0 or a multiple of 16 */
    int keep;            /* bf16-kept tokens of odd layers: 0 or a multiple of 16 */
    int prefix_rule;     /* GPTOSS_ATTN_PREFIX_* */
    int cache_kind;      /* GPTOSS_ATTN_CACHE_* */
} gptoss_attn_shape;

/* The caches of all sequences and layers (GPURunState fields).  Device
 * pointers; key/value codes 16-byte aligned, scales 8-byte aligned, bf16
 * rows 16-byte aligned (NULL when keep == 0).  With GPTOSS_ATTN_CACHE_BF16
 * only key_codes / value_codes (bf16 elements) are read. */
typedef struct gptoss_attn_cache {
    int8_t *key_codes;
    int8_t *value_codes;
    uint16_t *key_scales;     /* fp16 */
    uint16_t *value_scales;   /* fp16 */
    uint16_t *key_bf16;
    uint16_t *value_bf16;
    size_t batch_kv_stride;   /* elements per sequence; a multiple of 1024 */
    size_t batch_scale_stride;/* scales per sequence; a multiple of 16 */
} gptoss_attn_cache;

/* One layer's slice of the caches. */
typedef struct gptoss_attn_layer {
    int layer_idx;
    int cap;                  /* rows of this layer: sliding_window for even layers
                                 when sliding_window > 0, else the max context;
                                 a multiple of 16 */
    size_t layer_kv_offset;   /* elements; a multiple of 1024 */
    size_t layer_scale_offset;/* scales; a multiple of 16 */
} gptoss_attn_layer;

/* KV-cache update of the current token of n_seqs sequences
 * (quantize_kv_cache_kernel_int8 / _bf16, attention.hpp:536-720, launched at
 * getp_run.cpp:2326-2360; with a bf16 cache update_kv_cache_kernel,
 * attention.hpp:756-778, launched at getp_run.cpp:2096-2105): k, v bf16
 * [n_seqs][n_kv_heads * head_dim] (after RoPE), pos int32 [n_seqs] (device).
 * int8: writes each row's codes with an fp16 scale max(max|x|, 1e-6) / 127
 * and codes rint(x * 127 / that max) clamped to +-127; on odd layers with
 * pos < keep also the bf16 row.  bf16: writes the row.  A sequence with
 * pos < 0, or pos >= cap where rows are not a ring, is skipped
 * (attention.hpp:557-558). */
int gptoss_attn_kv_update(const gptoss_attn_shape *shape, const gptoss_attn_cache *cache,
                          const gptoss_attn_layer *layer, const uint16_t *k, const uint16_t *v,
                          const int32_t *pos, int n_seqs, hipStream_t stream);

/* Bytes of workspace that let gptoss_attn_decode split each sequence's
 * tokens over several waves (flash-decoding) for n_seqs sequences of up to
 * `cap` rows.  With a smaller workspace (or none) the split is smaller (or
 * there is none); results agree within fp32 rounding either way. */
size_t gptoss_attn_workspace_size(const gptoss_attn_shape *shape, int cap, int n_seqs);

/* Decode attention (flashdecoding_fused_fastmerge_nostage_1warp8q_bf16q_
 * bf16out{,_bf16kv}, attention_mfma.hpp:1113-1460, launched at
 * getp_run.cpp:2362-2470; with a bf16 cache ..._full_bf16kv_okay,
 * attention_mfma.hpp:1679-1900, launched at getp_run.cpp:2107-2135) for the
 * token at pos[b] of each sequence, whose
 * row gptoss_attn_kv_update has written:
 *     out[b][h] = sum_t softmax_t(q[b][h] . k_t / sqrt(64) | sink[h]) v_t
 * over t in [max(0, pos - sliding_window + 1), pos] on even layers (when
 * sliding_window > 0) and [0, pos] on odd ones, the sink logit taking part in
 * the softmax denominator only (run.cpp:598-643); query head h reads KV head
 * h / 8.  The softmax is exact (every token weighs in; the reference GPU
 * kernel drops tokens 8 or more below its running maximum).
 * q bf16 [n_seqs][n_heads][head_dim]; sinks bf16 [n_heads] (this layer's);
 * out bf16 [n_seqs][n_heads][head_dim].  A skipped sequence (see
 * gptoss_attn_kv_update) gets zeros.  ws may be NULL (ws_bytes 0); else
 * 256-byte aligned. */
int gptoss_attn_decode(const gptoss_attn_shape *shape, const gptoss_attn_cache *cache,
                       const gptoss_attn_layer *layer, const uint16_t *q, const uint16_t *sinks,
                       const int32_t *pos, int n_seqs, uint16_t *out, void *ws, size_t ws_bytes,
                       hipStream_t stream);

/* hipError_t of the last failed HIP call in this thread (0 if none), for
 * the entry points of gptoss_attn.h and gptoss_decoder.h. */
int gptoss_attn_last_hip_error(void);

#ifdef __cplusplus
}
#endif

#endif /* GPTOSS_ATTN_H */
