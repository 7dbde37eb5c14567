/*
 * moe_oracle.c — CPU restatement of the reference's MXFP4 MoE layer.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the parity tests, the
 * smoke check and bench.py's cpu_baseline leg compare the HIP path against.
 * The product (gpt-oss_amd/) never links, loads or calls it.
 *
 * Two semantics are restated:
 *   (i)  "getp" — the reference GPU batch path at TP = 1
 *        (getp-csrc/getp_run.cpp:2540-2887), with bf16 rounding at the same
 *        points: router logits bf16, scores fp32 = logit + bias, top-k with
 *        the epsilon tie rule, softmax weights bf16, MLP1 out bf16,
 *        SwiGLU out bf16, MLP2 out bf16, weighted reduction fp32 -> bf16.
 *        Dot products are accumulated in double (the exact limit of the
 *        reference's fp32 MFMA accumulation, whose internal order is not
 *        specified), except the router GEMM, whose fp32 order is pinned
 *        (see orc_router_logits).
 *   (ii) "fp32" — the CPU engine's MoE block (run.cpp:657-748), used as the
 *        CPU baseline that bench.py times (OpenMP over output rows, as
 *        run.cpp:355-368).
 *
 * Build: see oracle/Makefile (-ffp-contract=off: every fused multiply-add
 * here is an explicit fmaf()).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- bf16 -- */

/* fp32 -> bf16, round to nearest even; NaN -> quiet NaN (sign kept).
 * Matches __float2bfloat16 / pack2_bf16_bits_f32 (matmul.hpp:144-148). */
uint16_t orc_f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf2f(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* -------------------------------------------------------------- MXFP4 -- */

/* E2M1 magnitudes, memory/mxfp4.hpp:7-10 (== FP4_VALUES in
 * export_model_bin/gpt-oss-20b/export_model_bin.py:66-83). */
static const float kE2M1[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

/* Scale X = 2^(e-127) by placing e in the fp32 exponent field
 * (mxfp4.hpp:53: __uint_as_float(uint32_t(e) << 23)); e = 0 gives 0.0. */
float orc_e8m0_to_f32(uint8_t e) {
    uint32_t u = (uint32_t)e << 23;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Element i of one segment (mxfp4.hpp:42-57): byte i>>1, low nibble for even
 * i (export_model_bin.py:112-117), scale i>>5, value = code * X in fp32. */
float orc_mxfp4_elem(const uint8_t *packed, const uint8_t *scales, int64_t i) {
    uint8_t byte = packed[i >> 1];
    uint8_t nib = (uint8_t)((byte >> ((i & 1) << 2)) & 0xF);
    return kE2M1[nib] * orc_e8m0_to_f32(scales[i >> 5]);
}

/* One segment of n elements -> bf16 (dequant_mxfp4_pairs_to_bf16_kernel,
 * mxfp4.hpp:223-275). */
void orc_dequant_mxfp4(const uint8_t *packed, const uint8_t *scales, int64_t n, uint16_t *out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f2bf(orc_mxfp4_elem(packed, scales, i));
}

/* Same, to fp32 (the CPU engine's dequantised weights). */
void orc_dequant_mxfp4_f32(const uint8_t *packed, const uint8_t *scales, int64_t n, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = orc_mxfp4_elem(packed, scales, i);
}

/*
 * fp32 -> MXFP4 quantisation (quantize_pack_mxfp4_block32_kernel,
 * mxfp4.hpp:112-217): per 32-element block of the flattened array (the tail
 * block zero-filled), maxabs = max |v| over the block (NaN never wins: the
 * reference's `a > maxabs` is false for NaN); exp = ilogb(maxabs) - 2 via
 * frexpf (e - 1 - 2), 0 for an all-zero block; scale byte = clamp(exp + 127,
 * 0, 255); each element the nearest E2M1 code to v / 2^exp by a brute-force
 * scan with strict `<` (ties to the lower code index; NaN -> 0); two codes per
 * byte, low nibble = even element.  packed: ceil(n/32) * 16 bytes,
 * scales: ceil(n/32) bytes.
 */
void orc_quantize_mxfp4(const float *src, int64_t n, uint8_t *packed, uint8_t *scales) {
    const int64_t nb = (n + 31) / 32;
    for (int64_t b = 0; b < nb; ++b) {
        float v[32];
        for (int l = 0; l < 32; ++l) v[l] = (b * 32 + l < n) ? src[b * 32 + l] : 0.0f;
        float maxabs = 0.0f;
        for (int l = 0; l < 32; ++l) {
            const float a = fabsf(v[l]);
            if (a > maxabs) maxabs = a;
        }
        int exp_scale = 0;
        if (maxabs > 0.0f) {
            int e;
            frexpf(maxabs, &e);
            exp_scale = (e - 1) - 2;
        }
        int eb = exp_scale + 127;
        scales[b] = (uint8_t)(eb < 0 ? 0 : (eb > 255 ? 255 : eb));
        const float X = ldexpf(1.0f, exp_scale);
        uint8_t nib[32];
        for (int l = 0; l < 32; ++l) {
            const float x = v[l] / X;
            uint8_t best = 0;
            float best_diff = fabsf(x - kE2M1[0]);
            for (uint8_t i = 1; i < 16; ++i) {
                const float dd = fabsf(x - kE2M1[i]);
                if (dd < best_diff) {
                    best_diff = dd;
                    best = i;
                }
            }
            nib[l] = best;
        }
        for (int q = 0; q < 16; ++q)
            packed[b * 16 + q] = (uint8_t)((nib[2 * q + 1] << 4) | (nib[2 * q] & 0xF));
    }
}

/* ------------------------------------------------------------- router -- */

/*
 * Router logits, logits[t][e] = bf16(sum_k x[t][k] * wr[e][k]) with fp32
 * accumulation and no bias (matmul_vec128_singlebuf_Abf16, matmul.hpp:1344,
 * called at getp_run.cpp:2612-2620).  The reference accumulates inside MFMA
 * tiles in an unspecified order; this build pins one fp32 order so router
 * indices can be compared bit for bit: 16 partial sums p[l], each a chain of
 * fmaf over k = 128*i + 8*l + j (i ascending, then j = 0..7), then a
 * butterfly p[l] = p[l] + p[l ^ s] for s = 8, 4, 2, 1.
 * H must be a multiple of 8.
 */
void orc_router_logits(const uint16_t *x, const uint16_t *wr, int T, int H, int E,
                       uint16_t *out) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
        float p[16], q[16];
        for (int e = 0; e < E; ++e) {
            const uint16_t *xr = x + (int64_t)t * H;
            const uint16_t *wrow = wr + (int64_t)e * H;
            for (int l = 0; l < 16; ++l) {
                float acc = 0.0f;
                for (int base = 8 * l; base < H; base += 128)
                    for (int j = 0; j < 8; ++j)
                        acc = fmaf(orc_bf2f(xr[base + j]), orc_bf2f(wrow[base + j]), acc);
                p[l] = acc;
            }
            for (int s = 8; s >= 1; s >>= 1) {
                for (int l = 0; l < 16; ++l) q[l] = p[l] + p[l ^ s];
                memcpy(p, q, sizeof(p));
            }
            out[(int64_t)t * E + e] = orc_f2bf(p[0]);
        }
    }
}

/* ---------------------------------------------------------- top-k ------ */

typedef struct {
    float v;
    int i;
} orc_pick;

/* better_pick (moe.hpp:333-342): larger wins unless within eps*max(|a|,|b|),
 * then the lower index wins. */
static int orc_better(orc_pick a, orc_pick b, float eps) {
    float thr = eps * fmaxf(fabsf(a.v), fabsf(b.v));
    if (a.v > b.v + thr) return 1;
    if (fabsf(a.v - b.v) <= thr && a.i < b.i) return 1;
    return 0;
}

/*
 * route_select_softmax_kernel_bf16io + run_route_select_softmax_fused
 * (moe.hpp:465-599) for one token: scores fp32 = logit + bias, K rounds of a
 * block arg-max over nthreads = clamp(nextpow2(E), 64, 512) threads (thread
 * tid scans i = tid, tid + nthreads, ...; then a halving tree), softmax over
 * the K selected (expf, 1/(sum + 1e-20)), weights rounded to bf16.  The
 * reference only instantiates K = 4; the same rule is used for any K <= 8.
 * A round that finds no finite candidate yields index -1 (the reference
 * writes E there).
 */
void orc_topk_softmax(const uint16_t *logits, const uint16_t *bias, int T, int E, int K,
                      int32_t *topk_i, uint16_t *topk_w) {
    int nthreads = 1;
    while (nthreads < E) nthreads <<= 1;
    if (nthreads < 64) nthreads = 64;
    if (nthreads > 512) nthreads = 512;
    const float eps = 1e-6f;
    orc_pick *red = (orc_pick *)malloc(sizeof(orc_pick) * nthreads);
    float *sc = (float *)malloc(sizeof(float) * E);
    unsigned char *vis = (unsigned char *)malloc(E);
    for (int t = 0; t < T; ++t) {
        for (int i = 0; i < E; ++i) {
            sc[i] = orc_bf2f(logits[(int64_t)t * E + i]) + orc_bf2f(bias[i]);
            vis[i] = 0;
        }
        int sel_i[8] = {0};
        float sel_v[8] = {0};
        for (int s = 0; s < K; ++s) {
            for (int tid = 0; tid < nthreads; ++tid) {
                orc_pick best = {-INFINITY, E};
                for (int i = tid; i < E; i += nthreads) {
                    if (vis[i]) continue;
                    orc_pick c = {sc[i], i};
                    if (orc_better(c, best, eps)) best = c;
                }
                red[tid] = best;
            }
            for (int st = nthreads >> 1; st > 0; st >>= 1)
                for (int tid = 0; tid < st; ++tid)
                    if (orc_better(red[tid + st], red[tid], eps)) red[tid] = red[tid + st];
            sel_i[s] = red[0].i;
            sel_v[s] = red[0].v;
            if (red[0].i < E) vis[red[0].i] = 1;
        }
        float mx = sel_v[0];
        for (int s = 1; s < K; ++s) mx = fmaxf(mx, sel_v[s]);
        float ex[8], sum = 0.0f;
        for (int s = 0; s < K; ++s) {
            ex[s] = expf(sel_v[s] - mx);
            sum += ex[s];
        }
        const float inv = 1.0f / (sum + 1e-20f);
        for (int s = 0; s < K; ++s) {
            topk_w[(int64_t)t * K + s] = orc_f2bf(ex[s] * inv);
            topk_i[(int64_t)t * K + s] = sel_i[s] < E ? sel_i[s] : -1;
        }
    }
    free(red);
    free(sc);
    free(vis);
}

/* ----------------------------------------------------- routing index -- */

/* Slot (t, k) is live iff its expert is in [0, E) and not already taken by
 * an earlier slot of the same token. */
static int orc_slot_live(const int32_t *ti, int t, int K, int k, int E) {
    int e = ti[(int64_t)t * K + k];
    if (e < 0 || e >= E) return 0;
    for (int j = 0; j < k; ++j)
        if (ti[(int64_t)t * K + j] == e) return 0;
    return 1;
}

/*
 * Histogram (count_tokens_per_expert_kernel, moe.hpp:744-760), exclusive
 * prefix (host loop, getp_run.cpp:2651-2657) and the compact row map of
 * route_build_index_kernel_bf16wts (moe.hpp:1173-1270): rows of expert e are
 * offsets[e] .. offsets[e+1]-1 in ascending token order.  Returns the number
 * of dropped (dead) slots.
 */
int orc_route_index(const int32_t *ti, const uint16_t *tw, int T, int K, int E, int32_t *counts,
                    int32_t *offsets, int32_t *local_ids, int32_t *row_token, float *row_w) {
    int dropped = 0;
    for (int e = 0; e < E; ++e) counts[e] = 0;
    for (int t = 0; t < T; ++t)
        for (int k = 0; k < K; ++k) {
            if (orc_slot_live(ti, t, K, k, E))
                counts[ti[(int64_t)t * K + k]]++;
            else
                dropped++;
        }
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    for (int64_t i = 0; i < (int64_t)T * K; ++i) local_ids[i] = -1;
    for (int e = 0; e < E; ++e) {
        int row = offsets[e];
        for (int t = 0; t < T; ++t)
            for (int k = 0; k < K; ++k)
                if (orc_slot_live(ti, t, K, k, E) && ti[(int64_t)t * K + k] == e) {
                    local_ids[(int64_t)t * K + k] = row;
                    row_token[row] = t;
                    row_w[row] = orc_bf2f(tw[(int64_t)t * K + k]);
                    row++;
                }
    }
    return dropped;
}

/* ------------------------------------------- MXFP8 activations (variant) -- */
/*
 * Activation quantiser of the block-scaled FP4 MFMA variant (no counterpart in
 * the reference, whose GEMMs take bf16 activations; the variant's own rule):
 * per 32-element block along K, e = floor(log2 max|x|) - 7 clamped to
 * [-123, 120] (0 for an all-zero block); hi = e4m3_rne(x * 2^-e), and for two
 * terms lo = e4m3_rne((x * 2^-e - hi) * 16); e8m0 scales e + 127 (hi) and
 * e + 123 (lo).  x = hi * 2^e + lo * 2^(e-4) up to the rounding of lo.
 * Layout per row: ceil(K/512) stages of 1 KB (512 B hi, then 512 B lo); in a
 * stage, k step kp (128 k) is 128 bytes whose byte 32 g + 16 h + j is
 * k = 128 kp + 64 h + 16 g + j (the MFMA's A-operand order: lane group g
 * holds k 16 g .. + 15 and 64 + 16 g .. + 15).  Scales per row and stage:
 * 16 B hi then 16 B lo; byte 4 g + b is 32-k group 4 b + g.  k >= K: code 0.
 */

/* OCP e4m3 (bias 7, no infinities) of a finite v with |v| < 464, round to
 * nearest even; the sign is kept (a negative value rounding to 0 is 0x80). */
static uint8_t orc_e4m3_rne(float v) {
    const uint8_t sgn = signbit(v) ? 0x80 : 0;
    const float a = fabsf(v);
    if (a < 0x1p-6f) return sgn | (uint8_t)(int)rintf(a * 512.0f); /* multiples of 2^-9; 8 = 2^-6 */
    int E;
    frexpf(a, &E);
    E -= 1; /* a in [2^E, 2^(E+1)) */
    int q = (int)rintf(ldexpf(a, 3 - E)); /* 8 .. 16 */
    if (q == 16) {
        q = 8;
        E += 1;
    }
    return sgn | (uint8_t)(((E + 7) << 3) | (q - 8));
}

float orc_e4m3_dec(uint8_t c) {
    const int e = (c >> 3) & 15, m = c & 7;
    const float v = e == 0 ? ldexpf((float)m, -9) : ldexpf((float)(8 + m), e - 10);
    return (c & 0x80) ? -v : v;
}

static int64_t orc_aq_pos(int k) {
    const int j = k / 512, kk = k % 512, kp = kk / 128, kin = kk % 128;
    const int g = (kin % 64) / 16, h = kin / 64, jj = kin % 16;
    return (int64_t)j * 1024 + kp * 128 + 32 * g + 16 * h + jj;
}
static int64_t orc_aq_spos(int b) { /* 32-k group b -> scale byte of its row */
    const int j = b / 16, bs = b % 16;
    return (int64_t)j * 32 + 4 * (bs % 4) + bs / 4;
}

void orc_quantize_act(const uint16_t *x, int rows, int K, int terms, uint8_t *q, uint8_t *s) {
    const int KS = (K + 511) / 512;
    memset(q, 0, (size_t)rows * KS * 1024);
    for (int r = 0; r < rows; ++r) {
        const uint16_t *xr = x + (int64_t)r * K;
        uint8_t *qr = q + (int64_t)r * KS * 1024, *sr = s + (int64_t)r * KS * 32;
        for (int b = 0; b < KS * 16; ++b) {
            float amax = 0.0f;
            for (int k = 32 * b; k < 32 * b + 32 && k < K; ++k) amax = fmaxf(amax, fabsf(orc_bf2f(xr[k])));
            int e = 0;
            if (amax > 0.0f) {
                int E;
                frexpf(amax, &E);
                e = E - 1 - 7;
                e = e < -123 ? -123 : (e > 120 ? 120 : e);
            }
            sr[orc_aq_spos(b)] = (uint8_t)(e + 127);
            sr[orc_aq_spos(b) + 16] = (uint8_t)(e + 123);
            for (int k = 32 * b; k < 32 * b + 32 && k < K; ++k) {
                const float v = ldexpf(orc_bf2f(xr[k]), -e);
                const uint8_t hi = orc_e4m3_rne(v);
                qr[orc_aq_pos(k)] = hi;
                qr[orc_aq_pos(k) + 512] = terms == 2 ? orc_e4m3_rne((v - orc_e4m3_dec(hi)) * 16.0f) : 0;
            }
        }
    }
}

/* The values the variant's GEMM sees: hi * 2^(sh-127) + lo * 2^(sl-127). */
void orc_dequant_act(const uint8_t *q, const uint8_t *s, int rows, int K, float *out) {
    const int KS = (K + 511) / 512;
    for (int r = 0; r < rows; ++r) {
        const uint8_t *qr = q + (int64_t)r * KS * 1024, *sr = s + (int64_t)r * KS * 32;
        for (int k = 0; k < K; ++k) {
            const int64_t sp = orc_aq_spos(k / 32);
            const double v = (double)orc_e4m3_dec(qr[orc_aq_pos(k)]) * ldexp(1.0, sr[sp] - 127) +
                             (double)orc_e4m3_dec(qr[orc_aq_pos(k) + 512]) * ldexp(1.0, sr[sp + 16] - 127);
            out[(int64_t)r * K + k] = (float)v;
        }
    }
}

/* Rows of bf16 x [rows][K] replaced in place (as float) by what the variant's
 * GEMM sees for activation mode aq (0 = bf16 as is, 1 = one MXFP8 term,
 * 2 = two). */
static void orc_act_as_seen(const uint16_t *x, int rows, int K, int aq, float *out) {
    if (aq == 0) {
        for (int64_t i = 0; i < (int64_t)rows * K; ++i) out[i] = orc_bf2f(x[i]);
        return;
    }
    const int KS = (K + 511) / 512;
    uint8_t *q = (uint8_t *)malloc((size_t)rows * KS * 1024 + 1);
    uint8_t *s = (uint8_t *)malloc((size_t)rows * KS * 32 + 1);
    orc_quantize_act(x, rows, K, aq, q, s);
    orc_dequant_act(q, s, rows, K, out);
    free(q);
    free(s);
}

/* ------------------------------------------------------------ experts -- */

static double orc_dot(const float *a, const float *b, int n) {
    double s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int k = 0;
    for (; k + 8 <= n; k += 8)
        for (int j = 0; j < 8; ++j) s[j] += (double)a[k + j] * (double)b[k + j];
    for (; k < n; ++k) s[0] += (double)a[k] * (double)b[k];
    return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

/* Clamped SwiGLU of the reference GPU path (moe.hpp:1472-1496): both gate
 * and up clamped to [-limit, limit], out = g*sigma(alpha*g)*(u+1) as
 * fmaf(g*sig, u, g*sig).  (The CPU engine clamps the gate only from above,
 * run.cpp:706-724; see orc_moe_fp32_token.) */
static float orc_swiglu(float g, float u, float limit, float alpha) {
    g = fminf(fmaxf(g, -limit), limit);
    u = fminf(fmaxf(u, -limit), limit);
    const float sig = 1.0f / (1.0f + expf(-alpha * g));
    g = g * sig;
    return fmaf(g, u, g);
}

/*
 * Expert MLPs and weighted reduction, getp semantics, for given routing.
 *   x_norm bf16 [T][H]; weights MXFP4 as in include/gptoss_moe.h.
 *   e_agg  bf16 [T][H] out.  act bf16 [P][D] out (optional, compact rows).
 * MLP1 (moe.hpp:2783-2858): bf16(acc + b1); SwiGLU -> bf16; MLP2: bf16(acc +
 * b2) (TP = 1, getp_run.cpp:951-967); reduction (moe.hpp:700-730): fmaf over
 * the k slots in slot order, fp32, then bf16.
 */
static void orc_moe_experts_aq(int H, int D, int E, int K, float limit, float alpha,
                               const uint16_t *x_norm, const uint8_t *w1, const uint8_t *s1,
                               const uint16_t *b1, const uint8_t *w2, const uint8_t *s2,
                               const uint16_t *b2, const int32_t *ti, const uint16_t *tw, int T,
                               uint16_t *e_agg, uint16_t *act_out, int aq) {
    const int N1 = 2 * D;
    int32_t *counts = (int32_t *)malloc(sizeof(int32_t) * E);
    int32_t *offsets = (int32_t *)malloc(sizeof(int32_t) * (E + 1));
    int32_t *local_ids = (int32_t *)malloc(sizeof(int32_t) * (size_t)T * K + 4);
    int32_t *row_token = (int32_t *)malloc(sizeof(int32_t) * (size_t)T * K + 4);
    float *row_w = (float *)malloc(sizeof(float) * (size_t)T * K + 4);
    orc_route_index(ti, tw, T, K, E, counts, offsets, local_ids, row_token, row_w);
    const int P = offsets[E];
    uint16_t *y = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)P * H + 2);
    uint16_t *act = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)P * D + 2);
    float *xf = (float *)malloc(sizeof(float) * (size_t)T * H + 4);
    orc_act_as_seen(x_norm, T, H, aq, xf);
    float *W = (float *)malloc(sizeof(float) * (size_t)N1 * H);
    float *hrow = (float *)malloc(sizeof(float) * (size_t)(P > 0 ? P : 1) * D);
    for (int e = 0; e < E; ++e) {
        const int r0 = offsets[e], nr = counts[e];
        if (nr == 0) continue;
        /* MLP1 + SwiGLU */
        const int64_t seg1 = (int64_t)N1 * H;
        orc_dequant_mxfp4_f32(w1 + e * (seg1 / 2), s1 + e * (seg1 / 32), seg1, W);
        for (int r = 0; r < nr; ++r) {
            const float *xr = xf + (int64_t)row_token[r0 + r] * H;
#pragma omp parallel for schedule(static)
            for (int j = 0; j < D; ++j) {
                float g = (float)orc_dot(W + (int64_t)(2 * j) * H, xr, H);
                float u = (float)orc_dot(W + (int64_t)(2 * j + 1) * H, xr, H);
                g = orc_bf2f(orc_f2bf(g + orc_bf2f(b1[(int64_t)e * N1 + 2 * j])));
                u = orc_bf2f(orc_f2bf(u + orc_bf2f(b1[(int64_t)e * N1 + 2 * j + 1])));
                uint16_t a = orc_f2bf(orc_swiglu(g, u, limit, alpha));
                act[(int64_t)(r0 + r) * D + j] = a;
            }
        }
        orc_act_as_seen(act + (int64_t)r0 * D, nr, D, aq, hrow);
        /* MLP2 */
        const int64_t seg2 = (int64_t)H * D;
        orc_dequant_mxfp4_f32(w2 + e * (seg2 / 2), s2 + e * (seg2 / 32), seg2, W);
        for (int r = 0; r < nr; ++r) {
#pragma omp parallel for schedule(static)
            for (int h = 0; h < H; ++h) {
                float v = (float)orc_dot(W + (int64_t)h * D, hrow + (int64_t)r * D, D);
                y[(int64_t)(r0 + r) * H + h] = orc_f2bf(v + orc_bf2f(b2[(int64_t)e * H + h]));
            }
        }
    }
    for (int t = 0; t < T; ++t)
        for (int h = 0; h < H; ++h) {
            float acc = 0.0f;
            for (int k = 0; k < K; ++k) {
                int ci = local_ids[(int64_t)t * K + k];
                if (ci >= 0) acc = fmaf(row_w[ci], orc_bf2f(y[(int64_t)ci * H + h]), acc);
            }
            e_agg[(int64_t)t * H + h] = orc_f2bf(acc);
        }
    if (act_out) memcpy(act_out, act, sizeof(uint16_t) * (size_t)P * D);
    free(counts); free(offsets); free(local_ids); free(row_token); free(row_w);
    free(y); free(act); free(xf); free(W); free(hrow);
}

void orc_moe_experts(int H, int D, int E, int K, float limit, float alpha, const uint16_t *x_norm,
                     const uint8_t *w1, const uint8_t *s1, const uint16_t *b1, const uint8_t *w2,
                     const uint8_t *s2, const uint16_t *b2, const int32_t *ti, const uint16_t *tw,
                     int T, uint16_t *e_agg, uint16_t *act_out) {
    orc_moe_experts_aq(H, D, E, K, limit, alpha, x_norm, w1, s1, b1, w2, s2, b2, ti, tw, T, e_agg,
                       act_out, 0);
}

/* ----------------------------------------------------- layer boundary -- */

/* rmsnorm_kernel_bf16_io (rmsnorm.hpp:113-164) with its 256-thread layout:
 * per-thread strided double partials, halving tree, inv = 1/sqrt(mean+1e-5)
 * in double, y = bf16(w * (float(inv) * x)). */
void orc_rmsnorm(const uint16_t *x, const uint16_t *w, int rows, int size, uint16_t *out) {
    double part[256];
    for (int r = 0; r < rows; ++r) {
        const uint16_t *xr = x + (int64_t)r * size;
        for (int tid = 0; tid < 256; ++tid) {
            double ss = 0.0;
            for (int i = tid; i < size; i += 256) {
                double v = (double)orc_bf2f(xr[i]);
                ss += v * v;
            }
            part[tid] = ss;
        }
        for (int s = 128; s > 0; s >>= 1)
            for (int tid = 0; tid < s; ++tid) part[tid] += part[tid + s];
        const double inv = 1.0 / sqrt(part[0] / (double)size + 1e-5);
        const float invf = (float)inv;
        for (int i = 0; i < size; ++i) {
            float v = invf * orc_bf2f(xr[i]);
            out[(int64_t)r * size + i] = orc_f2bf(orc_bf2f(w[i]) * v);
        }
    }
}

/* accumulate_kernel_bf16 with factor 1 (other_kernels.hpp:17-35). */
void orc_residual_add(uint16_t *x, const uint16_t *e, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = orc_f2bf(orc_bf2f(x[i]) + orc_bf2f(e[i]) * 1.0f);
}

/* Whole MoE on normalised rows, getp semantics: router (or forced routing
 * when ti_in != NULL), experts, reduction.  Optional outputs may be NULL. */
/* aq: activations as the FP4-MFMA variant sees them (0 = bf16 path). */
void orc_moe_forward_aq(int H, int D, int E, int K, float limit, float alpha,
                        const uint16_t *x_norm, const uint16_t *wr, const uint16_t *br,
                        const uint8_t *w1, const uint8_t *s1, const uint16_t *b1,
                        const uint8_t *w2, const uint8_t *s2, const uint16_t *b2, int T,
                        const int32_t *ti_in, const uint16_t *tw_in, uint16_t *e_agg,
                        uint16_t *logits_out, int32_t *ti_out, uint16_t *tw_out, int aq) {
    int32_t *ti = (int32_t *)malloc(sizeof(int32_t) * (size_t)T * K + 4);
    uint16_t *tw = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)T * K + 4);
    if (ti_in) {
        memcpy(ti, ti_in, sizeof(int32_t) * (size_t)T * K);
        memcpy(tw, tw_in, sizeof(uint16_t) * (size_t)T * K);
    } else {
        uint16_t *lg = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)T * E + 2);
        orc_router_logits(x_norm, wr, T, H, E, lg);
        orc_topk_softmax(lg, br, T, E, K, ti, tw);
        if (logits_out) memcpy(logits_out, lg, sizeof(uint16_t) * (size_t)T * E);
        free(lg);
    }
    orc_moe_experts_aq(H, D, E, K, limit, alpha, x_norm, w1, s1, b1, w2, s2, b2, ti, tw, T, e_agg,
                       NULL, aq);
    if (ti_out) memcpy(ti_out, ti, sizeof(int32_t) * (size_t)T * K);
    if (tw_out) memcpy(tw_out, tw, sizeof(uint16_t) * (size_t)T * K);
    free(ti);
    free(tw);
}

void orc_moe_forward(int H, int D, int E, int K, float limit, float alpha, const uint16_t *x_norm,
                     const uint16_t *wr, const uint16_t *br, const uint8_t *w1, const uint8_t *s1,
                     const uint16_t *b1, const uint8_t *w2, const uint8_t *s2, const uint16_t *b2,
                     int T, const int32_t *ti_in, const uint16_t *tw_in, uint16_t *e_agg,
                     uint16_t *logits_out, int32_t *ti_out, uint16_t *tw_out) {
    orc_moe_forward_aq(H, D, E, K, limit, alpha, x_norm, wr, br, w1, s1, b1, w2, s2, b2, T, ti_in,
                       tw_in, e_agg, logits_out, ti_out, tw_out, 0);
}

/* ------------------------------------------------- fp32 CPU engine ----- */

/* matmul (run.cpp:355-368): OpenMP over output rows, double accumulation of
 * fp32 products. */
static void orc_matmul_f32(float *xout, const float *x, const float *w, int n, int d) {
    int i;
#pragma omp parallel for private(i)
    for (i = 0; i < d; i++) {
        double val = 0.0;
        for (int j = 0; j < n; j++) val += (double)(w[(int64_t)i * n + j] * x[j]);
        xout[i] = (float)val;
    }
}

typedef struct {
    float value;
    int index;
} orc_pair;

/* topk (run.cpp:387-420) sorts (value, index) pairs descending with qsort;
 * a stable insertion sort reproduces glibc's (merge-sort) order, ties keeping
 * ascending index. */
static void orc_topk_f32(float *vals, int *idx, const float *score, int E, int K) {
    orc_pair p[256];
    for (int i = 0; i < E; ++i) {
        p[i].value = score[i];
        p[i].index = i;
        int j = i;
        while (j > 0 && p[j - 1].value < p[j].value) {
            orc_pair tmp = p[j - 1];
            p[j - 1] = p[j];
            p[j] = tmp;
            --j;
        }
    }
    for (int i = 0; i < K; ++i) {
        vals[i] = p[i].value;
        idx[i] = p[i].index;
    }
}

/*
 * One token through the CPU engine's MoE block (run.cpp:657-748) with fp32
 * weights (w1f [E][2D][H], w2f [E][H][D]) and fp32 router.  x is the
 * normalised token row; e_agg (fp32 [H]) is the MoE output.  scratch needs
 * 2D + 3D + H + E floats.  Experts are visited in ascending index order as in
 * run.cpp:689-747.
 */
void orc_moe_fp32_token(int H, int D, int E, int K, float limit, const float *x, const float *wr,
                        const float *br, const float *w1f, const float *b1f, const float *w2f,
                        const float *b2f, float *e_agg, float *scratch) {
    float *mlp1 = scratch, *gate = mlp1 + 2 * D, *up = gate + D, *gu = up + D;
    float *tb2 = gu + D, *score = tb2 + H;
    float topv[8];
    int topi[8];
    orc_matmul_f32(score, x, wr, H, E);
    for (int i = 0; i < E; ++i) score[i] += br[i];
    orc_topk_f32(topv, topi, score, E, K);
    /* softmax (run.cpp:335-353) over the K selected */
    double mx = topv[0];
    for (int i = 1; i < K; ++i)
        if (topv[i] > mx) mx = topv[i];
    double sum = 0.0;
    for (int i = 0; i < K; ++i) {
        topv[i] = expf((float)(topv[i] - mx));
        sum += topv[i];
    }
    for (int i = 0; i < K; ++i) topv[i] = (float)(topv[i] / sum);
    memset(e_agg, 0, sizeof(float) * H);
    const float alpha = 1.702f;
    for (int e = 0; e < E; ++e) {
        float ew = 0.0f;
        int in = 0;
        for (int i = 0; i < K; ++i)
            if (topi[i] == e) {
                in = 1;
                ew = topv[i];
                break;
            }
        if (!in) continue;
        orc_matmul_f32(mlp1, x, w1f + (int64_t)e * 2 * D * H, H, 2 * D);
        for (int i = 0; i < 2 * D; ++i) mlp1[i] += b1f[(int64_t)e * 2 * D + i];
        for (int j = 0; j < D; ++j) {
            gate[j] = mlp1[2 * j];
            up[j] = mlp1[2 * j + 1];
        }
        for (int i = 0; i < D; ++i) {
            float v = gate[i], u = up[i];
            if (v > limit) v = limit;
            if (u > limit) u = limit;
            if (u < -limit) u = -limit;
            v *= (1.0f / (1.0f + expf(-alpha * v)));
            v *= (u + 1.0f);
            gu[i] = v;
        }
        orc_matmul_f32(tb2, gu, w2f + (int64_t)e * H * D, D, H);
        for (int i = 0; i < H; ++i) tb2[i] += b2f[(int64_t)e * H + i];
        for (int i = 0; i < H; ++i) e_agg[i] += tb2[i] * ew;
    }
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
