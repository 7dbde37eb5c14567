// C++ caller of the attention shim (gpt-oss_amd/csrc/attn_gpu_shim.hpp), run
// by tests/wip_gpu_attn.py: a mock of the reference's state with its
// member names, T decode steps of every layer through
// attention_cache_and_decode, then the last step again in two row ranges.
//
// usage: attn_gpu_test <in.bin> <out.bin>
// in.bin : int32 B, L, max_seq, window, keep, rule, T, kind (GPTOSS_ATTN_CACHE_*);
//          then per step t < T:
//          k bf16 [B][512], v bf16 [B][512]; then q bf16 [B][64][64]; sinks
//          bf16 [L][64].  Positions: t for every sequence at step t.
// out.bin: bf16 [2][L][B][64][64]: state.tb after each layer's call of the
//          last step, whole batch, then rows [0, B/2) and [B/2, B) apart.
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <vector>

#include "attn_gpu_shim.hpp"

// The members of the reference's structs the shim reads (getp_run.cpp:46-212).
typedef struct {
    int n_layers, n_attn_heads, n_kv_heads, head_dim, sliding_window;
} Config;
typedef struct {
    __hip_bfloat16 *attn_sinks;
} GPUTransformerWeights;
typedef struct {
    __hip_bfloat16 *q, *k, *v, *tb;
    int *positions;
    __hip_bfloat16 *key_cache_bf16, *value_cache_bf16;
    int8_t *key_cache, *value_cache;
    __half *key_cache_scales, *value_cache_scales;
    __hip_bfloat16 *key_cache_recent_bf16, *value_cache_recent_bf16;
} GPURunState;
typedef struct {
    Config config;
    GPUTransformerWeights weights;
    GPURunState state;
} GPUTransformer;

template <class T>
static T *dalloc(size_t n) {
    T *d = nullptr;
    if (hipMalloc(&d, n * sizeof(T) + 256) != hipSuccess || hipMemset(d, 0, n * sizeof(T)) != hipSuccess) {
        fprintf(stderr, "hipMalloc failed\n");
        exit(2);
    }
    return d;
}

static void rd(FILE *f, void *p, size_t bytes) {
    if (fread(p, 1, bytes, f) != bytes) {
        fprintf(stderr, "short input\n");
        exit(2);
    }
}

static void h2d(void *d, const void *h, size_t bytes) {
    if (hipMemcpy(d, h, bytes, hipMemcpyHostToDevice) != hipSuccess) exit(2);
}

int main(int argc, char **argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: %s in.bin out.bin\n", argv[0]);
        return 2;
    }
    FILE *f = fopen(argv[1], "rb");
    if (!f) return 2;
    int32_t hd[8];
    rd(f, hd, sizeof hd);
    const int B = hd[0], L = hd[1], max_seq = hd[2], window = hd[3], keep = hd[4], rule = hd[5], T = hd[6];
    const int kind = hd[7];
    const int KV = 512, QD = 64 * 64;
    std::vector<uint16_t> kh((size_t)T * B * KV), vh((size_t)T * B * KV), qh((size_t)B * QD), sh((size_t)L * 64);
    for (int t = 0; t < T; ++t) {
        rd(f, kh.data() + (size_t)t * B * KV, (size_t)B * KV * 2);
        rd(f, vh.data() + (size_t)t * B * KV, (size_t)B * KV * 2);
    }
    rd(f, qh.data(), qh.size() * 2);
    rd(f, sh.data(), sh.size() * 2);
    fclose(f);

    GPUTransformer gt{};
    gt.config = Config{L, 64, 8, 64, window};
    size_t cap_all = 0;
    for (int l = 0; l < L; ++l) cap_all += (l & 1) == 0 && window > 0 ? window : max_seq;
    GPURunState &s = gt.state;
    s.q = dalloc<__hip_bfloat16>((size_t)B * QD);
    s.k = dalloc<__hip_bfloat16>((size_t)B * KV);
    s.v = dalloc<__hip_bfloat16>((size_t)B * KV);
    s.tb = dalloc<__hip_bfloat16>((size_t)B * QD);
    s.positions = dalloc<int>(B);
    s.key_cache_bf16 = dalloc<__hip_bfloat16>((size_t)B * cap_all * KV);
    s.value_cache_bf16 = dalloc<__hip_bfloat16>((size_t)B * cap_all * KV);
    s.key_cache = dalloc<int8_t>((size_t)B * cap_all * KV);
    s.value_cache = dalloc<int8_t>((size_t)B * cap_all * KV);
    s.key_cache_scales = dalloc<__half>((size_t)B * cap_all);
    s.value_cache_scales = dalloc<__half>((size_t)B * cap_all);
    s.key_cache_recent_bf16 = dalloc<__hip_bfloat16>((size_t)B * L * (keep > 0 ? keep : 1) * KV);
    s.value_cache_recent_bf16 = dalloc<__hip_bfloat16>((size_t)B * L * (keep > 0 ? keep : 1) * KV);
    gt.weights.attn_sinks = dalloc<__hip_bfloat16>((size_t)L * 64);
    h2d(gt.weights.attn_sinks, sh.data(), sh.size() * 2);
    h2d(s.q, qh.data(), qh.size() * 2);

    hipStream_t st;
    if (hipStreamCreate(&st) != hipSuccess) return 2;
    gptoss_attn_shim::attn_gpu_init(&gt, B, max_seq, window, keep, rule, kind);
    std::vector<int> pos(B);
    std::vector<uint16_t> out((size_t)2 * L * B * QD);
    for (int t = 0; t < T; ++t) {
        for (int b = 0; b < B; ++b) pos[b] = t;
        h2d(s.positions, pos.data(), B * 4);
        h2d(s.k, kh.data() + (size_t)t * B * KV, (size_t)B * KV * 2);
        h2d(s.v, vh.data() + (size_t)t * B * KV, (size_t)B * KV * 2);
        for (int l = 0; l < L; ++l) {
            attention_cache_and_decode(&gt, l, B, 0, st);
            if (t == T - 1) {
                if (hipStreamSynchronize(st) != hipSuccess ||
                    hipMemcpy(out.data() + (size_t)l * B * QD, s.tb, (size_t)B * QD * 2,
                              hipMemcpyDeviceToHost) != hipSuccess)
                    return 2;
            }
        }
    }
    // the last step again, as two row ranges (rewrites the same cache rows)
    for (int l = 0; l < L; ++l) {
        attention_cache_and_decode(&gt, l, B / 2, 0, st);
        attention_cache_and_decode(&gt, l, B - B / 2, B / 2, st);
        if (hipStreamSynchronize(st) != hipSuccess ||
            hipMemcpy(out.data() + (size_t)(L + l) * B * QD, s.tb, (size_t)B * QD * 2,
                      hipMemcpyDeviceToHost) != hipSuccess)
            return 2;
    }
    FILE *o = fopen(argv[2], "wb");
    if (!o || fwrite(out.data(), 2, out.size(), o) != out.size()) return 2;
    fclose(o);
    printf("attn_gpu_test: B %d L %d T %d kind %d ok\n", B, L, T, kind);
    return 0;
}
