/*
 * attn_oracle.c — CPU restatement of the reference's decode attention with an
 * int8 KV cache (the attention half of a gpt-oss decoder layer).
 *
 * TEST INFRASTRUCTURE ONLY.  The parity tests and bench.py's cpu_baseline
 * leg compare the HIP attention path against these functions.  The product
 * (gpt-oss_amd/) never links, loads or calls them.
 *
 * Restated:
 *   - KV quantisation of one token row (quantize_kv_cache_kernel_impl,
 *     getp-csrc/kernels/attention.hpp:536-628): a per-row fp16 scale
 *     max(max|x|, 1e-6) / 127, codes rint(x * (127 / safe)) clamped to
 *     [-127, 127].
 *   - Cache addressing (getp_run.cpp:2195-2230, attention.hpp:582): even
 *     layers keep a ring of `sliding_window` rows (row = pos % window), odd
 *     layers keep row = pos; the first `keep` tokens of odd layers are also
 *     kept in bf16 (attention.hpp:559-566, :630-652).
 *   - The attention itself, in two semantics:
 *       phi_splits == 0: the CPU engine's math (run.cpp:598-643): score =
 *         (double sum of fp32 products) / sqrtf(head_dim), the sink logit
 *         appended to the softmax, softmax with a double max and sum,
 *         fp32 weighted sum of V.
 *       phi_splits  > 0: the reference GPU kernel
 *         flashdecoding_fused_fastmerge_nostage_1warp8q_body
 *         (attention_mfma.hpp:1113-1395): `phi_splits` contiguous token
 *         splits, each a streaming softmax that drops tokens whose score is
 *         8 (SOFTMAX_PHI, attention.hpp:14) or more below the running max,
 *         merged, with the sink in the denominator only and
 *         1e-9 (SOFTMAX_EPS, attention.hpp:22) added to it.  Order-faithful
 *         in fp32 with libm expf (the GPU uses __expf).
 *   The token source on odd layers follows `prefix_rule`:
 *       0: the reference's (attention_mfma.hpp:1160-1172): every token is
 *          read from the bf16 copy while pos < keep, from int8 otherwise;
 *       1: tokens t < keep are read from the bf16 copy, later ones from int8.
 *
 * Caches are in the reference's logical layout: kq/vq [B][cap][kv_dim] int8,
 * ks/vs [B][cap] fp16 bit patterns, kb/vb [B][keep][kv_dim] bf16 bit
 * patterns; q [B][n_heads][head_dim] bf16; sinks [n_heads] bf16.  With
 * cache_bf16 (the 20B path: update_kv_cache_kernel, attention.hpp:756-778,
 * and ..._full_bf16kv_okay, attention_mfma.hpp:1679-1900) kb/vb are the
 * whole caches, bf16 rows [B][cap][kv_dim] at the same rows as the int8
 * codes, and kq/vq/ks/vs/keep are not used.
 *
 * Build: oracle/Makefile (-ffp-contract=off: no implicit fused multiply-add).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

uint16_t orc_f2bf(float f);
float orc_bf2f(uint16_t h);

/* ---------------------------------------------------------------- fp16 -- */

/* fp32 -> IEEE binary16, round to nearest even (as __float2half). */
uint16_t orc_f2h(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);      /* NaN */
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);     /* rounds to >= 65520: Inf */
    if (a < 0x38800000u) {                                       /* below 2^-14: subnormal */
        /* value = a_float; subnormal unit 2^-24: code = rne(value * 2^24) */
        const int e = (int)(a >> 23);                            /* biased exponent */
        if (e < 102) return sign;                                /* < 2^-25: rounds to 0 */
        const uint32_t m = (a & 0x7fffffu) | 0x800000u;          /* 24-bit significand */
        const int shift = 126 - e;                               /* 14..24 */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    /* normal: rebias 127 -> 15, keep 10 mantissa bits, RNE (carry may bump the exponent) */
    uint32_t r = a - 0x38000000u;                                /* exponent - 112 */
    r += 0xfffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}

float orc_h2f(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t u;
    if (e == 0) {
        float f = ldexpf((float)m, -24);
        memcpy(&u, &f, 4);
        u |= sign;
    } else if (e == 31) {
        u = sign | 0x7f800000u | (m << 13);
    } else {
        u = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ------------------------------------------------------ KV quantisation -- */

/* One token row (quantize_kv_cache_kernel_impl, attention.hpp:582-628). */
void orc_kv_quantize_row(const uint16_t *x, int kv_dim, int8_t *q, uint16_t *scale) {
    float mx = 0.f;
    for (int i = 0; i < kv_dim; ++i) mx = fmaxf(mx, fabsf(orc_bf2f(x[i])));
    const float safe = fmaxf(mx, 1e-6f);
    const float inv = 127.f / safe;
    *scale = orc_f2h(safe / 127.f);
    for (int i = 0; i < kv_dim; ++i) {
        float c = rintf(orc_bf2f(x[i]) * inv);    /* __float2int_rn: nearest, ties to even */
        if (c > 127.f) c = 127.f;
        if (c < -127.f) c = -127.f;
        q[i] = (int8_t)c;
    }
}

/* --------------------------------------------------------- attention -- */

typedef struct {
    int n_heads, n_kv_heads, head_dim, cap, layer_idx, window, keep, prefix_rule, cache_bf16;
} orc_attn_cfg;

/* The dequantised key or value row of token t (run.cpp reads fp32 caches;
 * the GPU path dequantises as float(code) * float(scale),
 * attention_mfma.hpp:1236-1243). */
static void orc_kv_row(const orc_attn_cfg *c, int b, int t, int pos, const int8_t *cq,
                       const uint16_t *cs, const uint16_t *cb, int kvh, float *out) {
    const int kv_dim = c->n_kv_heads * c->head_dim;
    const int odd = c->layer_idx & 1;
    if (c->cache_bf16) { /* the 20B path's cache: bf16 rows [B][cap][kv_dim] (attention.hpp:756-778) */
        const int row = (!odd && c->window > 0) ? t % c->window : t;
        const uint16_t *r = cb + ((size_t)b * c->cap + row) * kv_dim + (size_t)kvh * c->head_dim;
        for (int i = 0; i < c->head_dim; ++i) out[i] = orc_bf2f(r[i]);
        return;
    }
    int bf16 = 0;
    if (odd && c->keep > 0 && cb)
        bf16 = c->prefix_rule == 0 ? (pos < c->keep) : (t < c->keep);
    if (bf16) {
        const uint16_t *r = cb + ((size_t)b * c->keep + t) * kv_dim + (size_t)kvh * c->head_dim;
        for (int i = 0; i < c->head_dim; ++i) out[i] = orc_bf2f(r[i]);
        return;
    }
    const int row = (!odd && c->window > 0) ? t % c->window : t;
    const int8_t *r = cq + ((size_t)b * c->cap + row) * kv_dim + (size_t)kvh * c->head_dim;
    const float s = orc_h2f(cs[(size_t)b * c->cap + row]);
    for (int i = 0; i < c->head_dim; ++i) out[i] = (float)r[i] * s;
}

/* First token of the attended range: the sliding-window mask of run.cpp:170-176
 * (-inf where pos - t >= window) applied on even layers (run.cpp:617). */
static int orc_t_start(const orc_attn_cfg *c, int pos) {
    if (c->window > 0 && (c->layer_idx & 1) == 0) return pos - (c->window - 1) > 0 ? pos - (c->window - 1) : 0;
    return 0;
}

/* run.cpp:598-643 for head h of sequence b. */
static void orc_head_exact(const orc_attn_cfg *c, int b, int h, int pos, const uint16_t *qbf,
                           const int8_t *kq, const int8_t *vq, const uint16_t *ks,
                           const uint16_t *vs, const uint16_t *kb, const uint16_t *vb, float sink,
                           float *att, float *row, float *out) {
    const int hd = c->head_dim, kvh = h / (c->n_heads / c->n_kv_heads);
    const int t0 = orc_t_start(c, pos), n = pos - t0 + 1;
    float q[256];
    for (int i = 0; i < hd; ++i) q[i] = orc_bf2f(qbf[((size_t)b * c->n_heads + h) * hd + i]);
    for (int j = 0; j < n; ++j) {
        orc_kv_row(c, b, t0 + j, pos, kq, ks, kb, kvh, row);
        double score = 0.0;
        for (int i = 0; i < hd; ++i) score += q[i] * row[i];
        score /= sqrtf((float)hd);
        att[j] = (float)score;
    }
    att[n] = sink;
    /* softmax (run.cpp:335-353) */
    double mx = att[0];
    for (int j = 1; j <= n; ++j)
        if (att[j] > mx) mx = att[j];
    double sum = 0.0;
    for (int j = 0; j <= n; ++j) {
        att[j] = expf((float)(att[j] - mx));
        sum += att[j];
    }
    for (int j = 0; j <= n; ++j) att[j] = (float)(att[j] / sum);
    for (int i = 0; i < hd; ++i) out[i] = 0.f;
    for (int j = 0; j < n; ++j) {
        orc_kv_row(c, b, t0 + j, pos, vq, vs, vb, kvh, row);
        const float a = att[j];
        for (int i = 0; i < hd; ++i) out[i] += a * row[i];
    }
}

/* attention_mfma.hpp:1199-1395 for head h of sequence b (head_dim 64). */
static void orc_head_phi(const orc_attn_cfg *c, int b, int h, int pos, int splits,
                         const uint16_t *qbf, const int8_t *kq, const int8_t *vq,
                         const uint16_t *ks, const uint16_t *vs, const uint16_t *kb,
                         const uint16_t *vb, float sink, float *row, float *out) {
    const int hd = c->head_dim, kvh = h / (c->n_heads / c->n_kv_heads);
    const int t0 = orc_t_start(c, pos), n = pos - t0 + 1;
    const float phi = 8.0f, eps = 1e-9f;
    float qs[64];
    for (int i = 0; i < 64; ++i) qs[i] = orc_bf2f(qbf[((size_t)b * c->n_heads + h) * hd + i]) * (1.0f / sqrtf(64.f));
    float m_w[64], l_w[64], o_w[64][64];
    for (int w = 0; w < splits; ++w) {
        const int tb = (int)((int64_t)n * w / splits), te = (int)((int64_t)n * (w + 1) / splits);
        float m = -INFINITY, l = 0.f, o[64];
        for (int i = 0; i < 64; ++i) o[i] = 0.f;
        for (int j = tb; j < te; ++j) {
            orc_kv_row(c, b, t0 + j, pos, kq, ks, kb, kvh, row);
            float part[8];
            for (int li = 0; li < 8; ++li) {
                float p = 0.f;
                for (int s = 0; s < 8; ++s) p = fmaf(qs[li + 8 * s], row[li + 8 * s], p);
                part[li] = p;
            }
            const float s = ((part[0] + part[4]) + (part[2] + part[6])) +
                            ((part[1] + part[5]) + (part[3] + part[7]));
            const float mn = fmaxf(m, s);
            const float alpha = expf(m - mn);
            const float dm = s - mn;
            const float wgt = dm > -phi ? expf(dm) : 0.f;
            l = fmaf(l, alpha, wgt);
            m = mn;
            orc_kv_row(c, b, t0 + j, pos, vq, vs, vb, kvh, row);
            for (int i = 0; i < 64; ++i) o[i] = fmaf(wgt, row[i], o[i] * alpha);
        }
        m_w[w] = m;
        l_w[w] = l;
        memcpy(o_w[w], o, sizeof o);
    }
    float mmax = -INFINITY;
    for (int w = 0; w < splits; ++w) mmax = fmaxf(mmax, m_w[w]);
    float lsum = 0.f, num[64];
    for (int i = 0; i < 64; ++i) num[i] = 0.f;
    for (int w = 0; w < splits; ++w) {
        const float sc = m_w[w] == -INFINITY ? 0.f : expf(m_w[w] - mmax);
        lsum = fmaf(l_w[w], sc, lsum);
        for (int i = 0; i < 64; ++i) num[i] = fmaf(o_w[w][i], sc, num[i]);
    }
    const float mnew = fmaxf(mmax, sink);
    const float alpha = expf(mmax - mnew);
    const float lf = lsum * alpha + expf(sink - mnew);
    for (int i = 0; i < 64; ++i) out[i] = (num[i] * alpha) / (lf + eps);
}

/* Decode attention of B sequences at positions pos[b] (the current token's
 * row already written), one layer.  out: fp32 [B][n_heads][head_dim].
 * Returns 0, or -1 for shapes outside what the restatement handles. */
int orc_attn_decode(int B, int n_heads, int n_kv_heads, int head_dim, int cap, int layer_idx,
                    int sliding_window, int keep, int prefix_rule, int phi_splits, int cache_bf16,
                    const uint16_t *q, const int8_t *kq, const int8_t *vq, const uint16_t *ks,
                    const uint16_t *vs, const uint16_t *kb, const uint16_t *vb,
                    const uint16_t *sinks, const int32_t *pos, float *out) {
    if (B < 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || head_dim <= 0 || head_dim > 256)
        return -1;
    if (phi_splits > 64 || (phi_splits > 0 && head_dim != 64)) return -1;
    const orc_attn_cfg c = {n_heads, n_kv_heads, head_dim, cap, layer_idx, sliding_window, keep,
                            prefix_rule, cache_bf16};
    for (int b = 0; b < B; ++b) {
        const int odd = layer_idx & 1;
        const int rows = (!odd && sliding_window > 0) ? sliding_window : pos[b] + 1;
        if (pos[b] < 0 || rows > cap) return -1;
    }
    int bad = 0;
#pragma omp parallel for schedule(dynamic) reduction(| : bad)
    for (int bh = 0; bh < B * n_heads; ++bh) {
        const int b = bh / n_heads, h = bh % n_heads;
        float *att = (float *)malloc(sizeof(float) * ((size_t)pos[b] + 2));
        float row[256];
        if (!att) {
            bad = 1;
            continue;
        }
        float *o = out + ((size_t)b * n_heads + h) * head_dim;
        const float sink = orc_bf2f(sinks[h]);
        if (phi_splits > 0)
            orc_head_phi(&c, b, h, pos[b], phi_splits, q, kq, vq, ks, vs, kb, vb, sink, row, o);
        else
            orc_head_exact(&c, b, h, pos[b], q, kq, vq, ks, vs, kb, vb, sink, att, row, o);
        free(att);
    }
    return bad ? -1 : 0;
}

/* ------------------------------------------------- decoder-step pieces -- */

/* RoPE tables with YaRN (compute_concentration_and_inv_freq and
 * compute_cos_sin, run.cpp:422-503; the reference GPU path fills its
 * cos/sin tables on the host with them, getp_run.cpp:1876-1890):
 * cos_out/sin_out [n_pos][head_dim / 2].  ntk_beta 32, ntk_alpha 1
 * (run.cpp:576-577).  Returns -1 where run.cpp's assert would fail. */
int orc_rope_table(float base, int head_dim, float scaling_factor, float initial_context_length,
                   int n_pos, float *cos_out, float *sin_out) {
    const int d_half = head_dim / 2;
    const float ntk_beta = 32.0f, ntk_alpha = 1.0f;
    float inv_freq[512];
    if (d_half > 512) return -1;
    float concentration = 1.0f;
    if (scaling_factor > 1.0f) {
        concentration = 0.1f * logf(scaling_factor) + 1.0f;
        /* M_PI is a double there: the quotient is taken in double and
         * rounded to float by logf's parameter */
        const double pi = 3.14159265358979323846;
        const float low = d_half * logf((float)(initial_context_length / (ntk_beta * 2.0f * pi))) / logf(base);
        const float high = d_half * logf((float)(initial_context_length / (ntk_alpha * 2.0f * pi))) / logf(base);
        if (!(0 < low && low < high && high < d_half - 1)) return -1;
        for (int i = 0; i < d_half; i++) {
            const float freq = powf(base, ((float)(2 * i)) / (float)head_dim);
            const float interpolation = 1.0f / (scaling_factor * freq);
            const float extrapolation = 1.0f / freq;
            float ramp = ((float)i - low) / (high - low);
            if (ramp < 0) ramp = 0;
            if (ramp > 1) ramp = 1;
            const float mask = 1.0f - ramp;
            inv_freq[i] = interpolation * (1.0f - mask) + extrapolation * mask;
        }
    } else {
        for (int i = 0; i < d_half; i++) inv_freq[i] = 1.0f / powf(base, ((float)(2 * i)) / (float)head_dim);
    }
    for (int p = 0; p < n_pos; ++p)
        for (int j = 0; j < d_half; j++) {
            const float val = (float)p * inv_freq[j];
            cos_out[(size_t)p * d_half + j] = cosf(val) * concentration;
            sin_out[(size_t)p * d_half + j] = sinf(val) * concentration;
        }
    return 0;
}

/* Bias add + split + RoPE of the QKV projection (add_bias_kernel,
 * other_kernels.hpp:53-61, then split_qkv_apply_rotary_kernel_vec_bf16,
 * rope.hpp:209-330): qkv bf16 [B][(nq + 2 nkv) hd] (the GEMM output,
 * already bf16), bias bf16; each element first bf16(x + b); then for head
 * element pairs (i, i + hd/2) at position pos: y0 = a c - b s,
 * y1 = b c + a s in fp32, rounded to bf16.  The fp32 rotation is evaluated
 * as fmaf(a, c, -(b * s)) and fmaf(b, c, a * s) (the reference leaves the
 * contraction to its compiler).  v is copied. */
void orc_qkv_bias_rope(const uint16_t *qkv, const uint16_t *bias, const float *cos_t,
                       const float *sin_t, const int32_t *pos, int B, int nq, int nkv, int hd,
                       uint16_t *q, uint16_t *k, uint16_t *v) {
    const int width = (nq + 2 * nkv) * hd, half = hd / 2;
    for (int b = 0; b < B; ++b) {
        const uint16_t *row = qkv + (size_t)b * width;
        const float *cs = cos_t + (size_t)pos[b] * half, *sn = sin_t + (size_t)pos[b] * half;
        for (int h = 0; h < nq + nkv; ++h) {
            uint16_t *dst = h < nq ? q + ((size_t)b * nq + h) * hd : k + ((size_t)b * nkv + h - nq) * hd;
            for (int i = 0; i < half; ++i) {
                const int e0 = h * hd + i, e1 = e0 + half;
                const float a = orc_bf2f(orc_f2bf(orc_bf2f(row[e0]) + orc_bf2f(bias[e0])));
                const float c2 = orc_bf2f(orc_f2bf(orc_bf2f(row[e1]) + orc_bf2f(bias[e1])));
                dst[i] = orc_f2bf(fmaf(a, cs[i], -(c2 * sn[i])));
                dst[i + half] = orc_f2bf(fmaf(c2, cs[i], a * sn[i]));
            }
        }
        for (int i = 0; i < nkv * hd; ++i) {
            const int e = (nq + nkv) * hd + i;
            v[(size_t)b * nkv * hd + i] = orc_f2bf(orc_bf2f(row[e]) + orc_bf2f(bias[e]));
        }
    }
}

/* Output projection epilogue (store_and_fuse_tile_bf16, matmul.hpp:121-139):
 * x = bf16(bf16(proj + bias) + x), proj the GEMM output already in bf16. */
void orc_bias_residual(uint16_t *x, const uint16_t *proj, const uint16_t *bias, int B, int H) {
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h) {
            const size_t i = (size_t)b * H + h;
            const float v = orc_bf2f(orc_f2bf(orc_bf2f(proj[i]) + orc_bf2f(bias[h])));
            x[i] = orc_f2bf(v + orc_bf2f(x[i]));
        }
}

/* Dense bf16 GEMM out[m][n] = bf16(sum_k a[m][k] w[n][k]) with a double
 * accumulator (the limit of any fp32 MFMA order). */
void orc_matmul_bf16(const uint16_t *a, const uint16_t *w, int M, int N, int K, uint16_t *out) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double acc = 0.0;
            const uint16_t *ar = a + (size_t)m * K, *wr = w + (size_t)n * K;
            for (int k = 0; k < K; ++k) acc += (double)orc_bf2f(ar[k]) * (double)orc_bf2f(wr[k]);
            out[(size_t)m * N + n] = orc_f2bf((float)acc);
        }
}

/* Greedy sampling (sample_argmax_kernel_bf16, softmax.hpp:236-290): the
 * first index of the largest bf16 value of each row. */
void orc_argmax_bf16(const uint16_t *logits, int B, int n, int32_t *out) {
    for (int b = 0; b < B; ++b) {
        float best = -INFINITY;
        int bi = 0x7fffffff;
        for (int i = 0; i < n; ++i) {
            const float p = orc_bf2f(logits[(size_t)b * n + i]);
            if (p > best || (p == best && i < bi)) {
                best = p;
                bi = i;
            }
        }
        out[b] = bi;
    }
}
