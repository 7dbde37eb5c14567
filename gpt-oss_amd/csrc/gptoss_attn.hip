// gptoss_attn.hip — decode attention over an int8 KV cache for gfx950.
//
// Two kernels per layer and decode step, as in the reference's attention_gpu
// (getp-csrc/getp_run.cpp:2311-2470):
//   kv_update_kernel   the current token's K/V row -> int8 codes + fp16 scale
//                      (+ a bf16 copy of odd layers' first `keep` tokens)
//                      (attention.hpp:536-720);
//   attn_decode_kernel one wave per (sequence, KV head, token split): the 8
//                      query heads of the KV head against 32 tokens per step
//                      on the matrix cores, online softmax in the log2
//                      domain, sink in the denominator (run.cpp:598-643;
//                      attention_mfma.hpp:1113-1460);
//   attn_combine_kernel merges the splits when there are several.
//
// Matrix-core mapping (v_mfma_f32_16x16x32_bf16, lane = c + 16 g):
//   scores  S[token][head] = K[16 tokens][64 dims] . Q^T, two k-steps; lane
//           (c, g) supplies key row c, dims 16g..16g+15 (one 16-byte load of
//           the tile, int8 -> bf16 exactly) and query head c, the same dims;
//           query heads 8..15 of the instruction are zero.  The result gives
//           lane (c, g) head c at tokens 4g..4g+3.
//   output  O[head][dim] += P'[head][32 tokens] . V[32 tokens][16 dims] for
//           4 dim tiles; P' = p * value_scale (bf16) is exactly the score
//           layout of two 16-token blocks, and the value tile order gives
//           lane (c, g) dims 16 dt + c at tokens 4g..4g+3 of a block in one
//           16-byte load.  Rows 4g..4g+3 of the result are heads (g < 2).
// Keys and values are exact in bf16 (|code| <= 127); q . k is accumulated in
// fp32 and scaled by the token's key scale / 8 afterwards.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>

#include "gptoss_attn.h"

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

constexpr int kKvHeads = 8;      // n_kv_heads
constexpr int kGqa = 8;          // query heads per KV head
constexpr int kHd = 64;          // head_dim
constexpr int kKvDim = kKvHeads * kHd;
constexpr int kTile = 1024;      // elements of one (16-row block, KV head) tile
constexpr int kPartFloats = 2 * kGqa + kGqa * kHd;  // m[8], l[8], o[8][64] of a split
constexpr int kMaxSplits = 64;
constexpr int kTargetWaves = 2048;  // 256 CUs x 8 waves
constexpr float kLog2e = 1.4426950408889634f;

thread_local int g_last_hip_error = 0;

int hip_fail(hipError_t e) {
    g_last_hip_error = (int)e;
    return GPTOSS_ATTN_ERR_HIP;
}

__device__ inline float bf2f(uint32_t h) { return __uint_as_float(h << 16); }

__device__ inline uint32_t f2bf(float f) {  // round to nearest even; finite inputs
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ inline float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

__device__ inline uint16_t f2h(float f) {  // round to nearest even (the default mode)
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Two signed bytes (bits sh..sh+7 and sh+8..sh+15 of w) -> bf16x2, exactly.
__device__ inline uint32_t i8x2_bf16(uint32_t w, int sh) {
    const float a = (float)(int)(int8_t)(w >> sh);
    const float b = (float)(int)(int8_t)(w >> (sh + 8));
    return (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xffff0000u);
}

__device__ inline u32x4 i8x8_bf16(uint32_t lo, uint32_t hi) {
    return u32x4{i8x2_bf16(lo, 0), i8x2_bf16(lo, 16), i8x2_bf16(hi, 0), i8x2_bf16(hi, 16)};
}

__device__ inline bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ inline u32x4 ld16(const void *p) { return *(const u32x4 *)p; }
__device__ inline u32x4 ld16_nt(const void *p) { return __builtin_nontemporal_load((const u32x4 *)p); }

// ---------------------------------------------------------------------------
// KV-cache update (attention.hpp:536-652): one wave per sequence, lane l owns
// elements 8l..8l+7 of the row (KV head l/8, dims 8(l%8)..8(l%8)+7).
struct KvArgs {
    int8_t *kc, *vc;
    uint16_t *ks, *vs, *kb, *vb;
    size_t bks, bss, lko, lso;
    const uint16_t *k, *v;
    const int32_t *pos;
    int cap, window, ring, odd, keep, n_layers, layer;
};

__device__ inline int v_tile_off(int r, int d) {  // value element (row r % 16, dim d) in a tile
    return (d & 15) * 64 + ((r & 15) >> 2) * 16 + (d >> 4) * 4 + (r & 3);
}

__global__ __launch_bounds__(64) void kv_update_kernel(KvArgs a) {
    const int b = blockIdx.x, l = threadIdx.x;
    const int pos = a.pos[b];
    if (pos < 0 || (!a.ring && pos >= a.cap)) return;
    const int r = a.ring ? pos % a.window : pos;
    const int kvh = l >> 3, d0 = 8 * (l & 7);
    const u32x4 kr = ld16(a.k + (size_t)b * kKvDim + 8 * l);
    const u32x4 vr = ld16(a.v + (size_t)b * kKvDim + 8 * l);
    float kf[8], vf[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        kf[2 * j] = bf2f(kr[j] & 0xffffu);
        kf[2 * j + 1] = bf2f(kr[j] >> 16);
        vf[2 * j] = bf2f(vr[j] & 0xffffu);
        vf[2 * j + 1] = bf2f(vr[j] >> 16);
    }
    float mk = 0.f, mv = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        mk = fmaxf(mk, fabsf(kf[j]));
        mv = fmaxf(mv, fabsf(vf[j]));
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        mk = fmaxf(mk, __shfl_xor(mk, o));
        mv = fmaxf(mv, __shfl_xor(mv, o));
    }
    const float safe_k = fmaxf(mk, 1e-6f), safe_v = fmaxf(mv, 1e-6f);
    const float inv_k = 127.f / safe_k, inv_v = 127.f / safe_v;
    uint32_t kq[2] = {0u, 0u};
    uint8_t vq[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int ck = min(max(__float2int_rn(kf[j] * inv_k), -127), 127);
        const int cv = min(max(__float2int_rn(vf[j] * inv_v), -127), 127);
        kq[j >> 2] |= (uint32_t)(uint8_t)ck << (8 * (j & 3));
        vq[j] = (uint8_t)cv;
    }
    const size_t tile = (size_t)b * a.bks + a.lko + (size_t)((r >> 4) * kKvHeads + kvh) * kTile;
    *(u32x2 *)(a.kc + tile + (r & 15) * 64 + d0) = u32x2{kq[0], kq[1]};
#pragma unroll
    for (int j = 0; j < 8; ++j) a.vc[tile + v_tile_off(r, d0 + j)] = (int8_t)vq[j];
    if (l == 0) {
        const size_t so = (size_t)b * a.bss + a.lso + r;
        a.ks[so] = f2h(safe_k / 127.f);
        a.vs[so] = f2h(safe_v / 127.f);
    }
    if (a.odd && pos < a.keep) {  // the bf16 copy (attention.hpp:630-652)
        const size_t slab = ((size_t)b * a.n_layers + a.layer) * a.keep * kKvDim;
        const size_t bt = slab + (size_t)((pos >> 4) * kKvHeads + kvh) * kTile;
        *(u32x4 *)(a.kb + bt + (pos & 15) * 64 + d0) = kr;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            a.vb[bt + v_tile_off(pos, d0 + j)] = (uint16_t)(j & 1 ? vr[j >> 1] >> 16 : vr[j >> 1] & 0xffffu);
    }
}

// ---------------------------------------------------------------------------
// Decode attention.
struct DecArgs {
    const int8_t *kc, *vc;
    const uint16_t *ks, *vs, *kb, *vb;
    size_t bks, bss, lko, lso;
    const uint16_t *q, *sinks;
    const int32_t *pos;
    uint16_t *out;
    float *ws;
    int cap, window, ring, odd, keep, rule, n_layers, layer, splits;
};

// One 16-row block in matrix-instruction operand form.
struct BlkOp {
    u32x4 k0, k1;     // key rows: bf16 dims 16g..16g+7, 16g+8..16g+15 of row c
    u32x2 v[4];       // per dim tile: bf16 values of tokens 4g..4g+3 at dim 16 dt + c
    float ksc[4];     // key scale * log2(e) / 8 of tokens 4g..4g+3
    float vsc[4];     // value scale
};

struct RawI8 {        // an int8 block as loaded
    u32x4 k, v;
    u32x2 ks, vs;
};

__device__ inline void load_i8(const DecArgs &a, size_t kv_base, size_t sc_base, int kvh, int blk,
                               int c, int g, RawI8 &r) {
    const size_t t = kv_base + (size_t)(blk * kKvHeads + kvh) * kTile;
    r.k = ld16_nt(a.kc + t + c * 64 + 16 * g);
    r.v = ld16_nt(a.vc + t + c * 64 + 16 * g);
    const size_t s = sc_base + blk * 16 + 4 * g;
    r.ks = *(const u32x2 *)(a.ks + s);
    r.vs = *(const u32x2 *)(a.vs + s);
}

__device__ inline void op_from_i8(const RawI8 &r, BlkOp &o) {
    o.k0 = i8x8_bf16(r.k[0], r.k[1]);
    o.k1 = i8x8_bf16(r.k[2], r.k[3]);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o.v[dt] = u32x2{i8x2_bf16(r.v[dt], 0), i8x2_bf16(r.v[dt], 16)};
    const float C = 0.125f * kLog2e;
    o.ksc[0] = h2f(r.ks[0] & 0xffffu) * C;
    o.ksc[1] = h2f(r.ks[0] >> 16) * C;
    o.ksc[2] = h2f(r.ks[1] & 0xffffu) * C;
    o.ksc[3] = h2f(r.ks[1] >> 16) * C;
    o.vsc[0] = h2f(r.vs[0] & 0xffffu);
    o.vsc[1] = h2f(r.vs[0] >> 16);
    o.vsc[2] = h2f(r.vs[1] & 0xffffu);
    o.vsc[3] = h2f(r.vs[1] >> 16);
}

__device__ inline void op_from_bf16(const DecArgs &a, size_t slab, int kvh, int blk, int c, int g,
                                    BlkOp &o) {
    const size_t t = slab + (size_t)(blk * kKvHeads + kvh) * kTile;
    o.k0 = ld16(a.kb + t + c * 64 + 16 * g);
    o.k1 = ld16(a.kb + t + c * 64 + 16 * g + 8);
    const u32x4 v0 = ld16(a.vb + t + c * 64 + 16 * g);
    const u32x4 v1 = ld16(a.vb + t + c * 64 + 16 * g + 8);
    o.v[0] = u32x2{v0[0], v0[1]};
    o.v[1] = u32x2{v0[2], v0[3]};
    o.v[2] = u32x2{v1[0], v1[1]};
    o.v[3] = u32x2{v1[2], v1[3]};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o.ksc[i] = 0.125f * kLog2e;
        o.vsc[i] = 1.f;
    }
}

__device__ inline void op_zero(BlkOp &o) {
    o.k0 = o.k1 = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o.v[dt] = u32x2{0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) o.ksc[i] = o.vsc[i] = 0.f;
}

struct SoftState {
    float m, l;       // running max (log2 domain) and this lane's part of the sum, for head c
    f32x4 o[4];       // O[head 4g+i][dim 16 dt + c]
};

// Two blocks (32 tokens) starting at block `blk`; `nb` of them present (1 or 2).
// Rows at or past `nvalid` weigh nothing.  `zero_v` clears value elements of
// such rows (bf16 rows past the written ones may hold anything).
__device__ inline void pair_step(const BlkOp &A, const BlkOp &B, int blk, int nb, int nvalid, int g,
                                 int lane, bf16x8 q0, bf16x8 q1, bool zero_v, SoftState &st) {
    f32x4 s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(A.k0), q0, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(A.k1), q1, s0, 0, 0, 0);
    f32x4 s1 = f32x4{0.f, 0.f, 0.f, 0.f};
    if (nb > 1) {
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(B.k0), q0, s1, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(B.k1), q1, s1, 0, 0, 0);
    }
    float sv[8];
    bool ok[8];
    const int row0 = blk * 16 + 4 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ok[i] = row0 + i < nvalid;
        ok[4 + i] = nb > 1 && row0 + 16 + i < nvalid;
        sv[i] = ok[i] ? s0[i] * A.ksc[i] : -INFINITY;
        sv[4 + i] = ok[4 + i] ? s1[i] * B.ksc[i] : -INFINITY;
    }
    float bm = sv[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) bm = fmaxf(bm, sv[j]);
    bm = fmaxf(bm, __shfl_xor(bm, 16));
    bm = fmaxf(bm, __shfl_xor(bm, 32));
    const float mn = fmaxf(st.m, bm);
    const float alpha = __builtin_amdgcn_exp2f(st.m - mn);
    float p[8], ps = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        p[j] = __builtin_amdgcn_exp2f(sv[j] - mn);
        ps += p[j];
    }
    st.l = st.l * alpha + ps;
    st.m = mn;
    uint32_t pw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float lo = ok[2 * j] ? p[2 * j] * (j < 2 ? A.vsc[2 * j] : B.vsc[2 * j - 4]) : 0.f;
        const float hi = ok[2 * j + 1] ? p[2 * j + 1] * (j < 2 ? A.vsc[2 * j + 1] : B.vsc[2 * j - 3]) : 0.f;
        pw[j] = f2bf(lo) | (f2bf(hi) << 16);
    }
    const bf16x8 pop = as_bf16x8(u32x4{pw[0], pw[1], pw[2], pw[3]});
    float ar[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ar[i] = __shfl(alpha, 4 * g + i);
    (void)lane;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
        u32x2 va = A.v[dt], vb = nb > 1 ? B.v[dt] : u32x2{0u, 0u};
        if (zero_v) {
            va[0] &= (ok[0] ? 0xffffu : 0u) | (ok[1] ? 0xffff0000u : 0u);
            va[1] &= (ok[2] ? 0xffffu : 0u) | (ok[3] ? 0xffff0000u : 0u);
            vb[0] &= (ok[4] ? 0xffffu : 0u) | (ok[5] ? 0xffff0000u : 0u);
            vb[1] &= (ok[6] ? 0xffffu : 0u) | (ok[7] ? 0xffff0000u : 0u);
        }
        f32x4 acc = st.o[dt];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] *= ar[i];
        st.o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pop, as_bf16x8(u32x4{va[0], va[1], vb[0], vb[1]}),
                                                          acc, 0, 0, 0);
    }
}

__device__ inline bool seq_valid(const DecArgs &a, int pos) { return pos >= 0 && (a.ring || pos < a.cap); }

__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(4, 8))) void attn_decode_kernel(DecArgs a) {
    __shared__ float red[kGqa * kHd];
    const int S = a.splits;
    const int s = blockIdx.x % S;
    const int bk = blockIdx.x / S;
    const int kvh = bk % kKvHeads, b = bk / kKvHeads;
    const int lane = threadIdx.x, c = lane & 15, g = lane >> 4;
    const int pos = a.pos[b];
    uint16_t *out = a.out + ((size_t)b * kKvHeads * kGqa + kvh * kGqa) * kHd;
    if (!seq_valid(a, pos)) {
        if (S == 1) *(u32x4 *)(out + 8 * lane) = u32x4{0u, 0u, 0u, 0u};
        return;  // with splits, the combine kernel writes the zeros
    }
    const int nvalid = a.ring ? min(pos + 1, a.window) : pos + 1;
    const int nblk = (nvalid + 15) >> 4;
    int nb16 = 0;
    if (a.odd && a.keep > 0) nb16 = a.rule == GPTOSS_ATTN_PREFIX_REFERENCE ? (pos < a.keep ? nblk : 0)
                                                                         : min(nblk, a.keep >> 4);
    const int blk0 = (int)((int64_t)nblk * s / S), blk1 = (int)((int64_t)nblk * (s + 1) / S);

    bf16x8 q0 = as_bf16x8(u32x4{0u, 0u, 0u, 0u}), q1 = q0;
    if (c < kGqa) {
        const uint16_t *qp = a.q + ((size_t)b * kKvHeads * kGqa + kvh * kGqa + c) * kHd + 16 * g;
        q0 = as_bf16x8(ld16(qp));
        q1 = as_bf16x8(ld16(qp + 8));
    }
    SoftState st;
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) st.o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // bf16 rows first (odd layers' kept tokens), then the int8 rows
    const int e16 = min(blk1, nb16);
    if (blk0 < e16) {
        const size_t slab = ((size_t)b * a.n_layers + a.layer) * a.keep * kKvDim;
        for (int blk = blk0; blk < e16; blk += 2) {
            const int nb = min(2, e16 - blk);
            BlkOp A, B;
            op_from_bf16(a, slab, kvh, blk, c, g, A);
            if (nb > 1) op_from_bf16(a, slab, kvh, blk + 1, c, g, B);
            else op_zero(B);
            pair_step(A, B, blk, nb, nvalid, g, lane, q0, q1, true, st);
        }
    }
    const int i0 = max(blk0, nb16);
    if (i0 < blk1) {
        const size_t kv_base = (size_t)b * a.bks + a.lko;
        const size_t sc_base = (size_t)b * a.bss + a.lso;
        RawI8 nA, nB;
        load_i8(a, kv_base, sc_base, kvh, i0, c, g, nA);
        if (i0 + 1 < blk1) load_i8(a, kv_base, sc_base, kvh, i0 + 1, c, g, nB);
        for (int blk = i0; blk < blk1; blk += 2) {
            const int nb = min(2, blk1 - blk);
            const RawI8 rA = nA, rB = nB;
            if (blk + 2 < blk1) load_i8(a, kv_base, sc_base, kvh, blk + 2, c, g, nA);
            if (blk + 3 < blk1) load_i8(a, kv_base, sc_base, kvh, blk + 3, c, g, nB);
            BlkOp A, B;
            op_from_i8(rA, A);
            if (nb > 1) op_from_i8(rB, B);
            else op_zero(B);
            pair_step(A, B, blk, nb, nvalid, g, lane, q0, q1, false, st);
        }
    }

    // this head's sum over the four lane groups
    float l = st.l;
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (S == 1) {
        const float sk = c < kGqa ? bf2f(a.sinks[kvh * kGqa + c]) * kLog2e : 0.f;
        const float mf = fmaxf(st.m, sk);
        const float al = __builtin_amdgcn_exp2f(st.m - mf);
        const float f = al / (l * al + __builtin_amdgcn_exp2f(sk - mf));
        float fr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) fr[i] = __shfl(f, 4 * g + i);
        if (g < 2) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) red[(4 * g + i) * kHd + 16 * dt + c] = st.o[dt][i] * fr[i];
        }
        __syncthreads();
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = f2bf(red[8 * lane + 2 * j]) | (f2bf(red[8 * lane + 2 * j + 1]) << 16);
        *(u32x4 *)(out + 8 * lane) = u32x4{w[0], w[1], w[2], w[3]};
    } else {
        float *part = a.ws + ((size_t)bk * S + s) * kPartFloats;
        if (g == 0 && c < kGqa) {
            part[c] = st.m;
            part[kGqa + c] = l;
        }
        if (g < 2) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) red[(4 * g + i) * kHd + 16 * dt + c] = st.o[dt][i];
        }
        __syncthreads();
        float *po = part + 2 * kGqa + 8 * lane;
        *(f32x4 *)po = f32x4{red[8 * lane], red[8 * lane + 1], red[8 * lane + 2], red[8 * lane + 3]};
        *(f32x4 *)(po + 4) = f32x4{red[8 * lane + 4], red[8 * lane + 5], red[8 * lane + 6], red[8 * lane + 7]};
    }
}

// Merge of the splits: lane l owns head l/8, dims 8(l%8)..8(l%8)+7.
__global__ __launch_bounds__(64) void attn_combine_kernel(DecArgs a) {
    const int bk = blockIdx.x, kvh = bk % kKvHeads, b = bk / kKvHeads;
    const int lane = threadIdx.x, hh = lane >> 3;
    uint16_t *out = a.out + ((size_t)b * kKvHeads * kGqa + kvh * kGqa) * kHd + 8 * lane;
    if (!seq_valid(a, a.pos[b])) {
        *(u32x4 *)out = u32x4{0u, 0u, 0u, 0u};
        return;
    }
    const float *base = a.ws + (size_t)bk * a.splits * kPartFloats;
    float mm = -INFINITY;
    for (int s = 0; s < a.splits; ++s) mm = fmaxf(mm, base[s * kPartFloats + hh]);
    float L = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < a.splits; ++s) {
        const float *p = base + s * kPartFloats;
        const float w = __builtin_amdgcn_exp2f(p[hh] - mm);  // empty split: exp2(-inf) = 0
        L += p[kGqa + hh] * w;
        const f32x4 x0 = *(const f32x4 *)(p + 2 * kGqa + 8 * lane);
        const f32x4 x1 = *(const f32x4 *)(p + 2 * kGqa + 8 * lane + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            o[j] += x0[j] * w;
            o[4 + j] += x1[j] * w;
        }
    }
    const float sk = bf2f(a.sinks[kvh * kGqa + hh]) * kLog2e;
    const float mf = fmaxf(mm, sk);
    const float al = __builtin_amdgcn_exp2f(mm - mf);
    const float f = al / (L * al + __builtin_amdgcn_exp2f(sk - mf));
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = f2bf(o[2 * j] * f) | (f2bf(o[2 * j + 1] * f) << 16);
    *(u32x4 *)out = u32x4{w[0], w[1], w[2], w[3]};
}

// ---------------------------------------------------------------------------
// Host side.
bool aligned(const void *p, size_t n) { return ((uintptr_t)p % n) == 0; }

bool shape_ok(const gptoss_attn_shape *s) {
    return s && s->n_heads == kKvHeads * kGqa && s->n_kv_heads == kKvHeads && s->head_dim == kHd &&
           s->n_layers >= 1 && s->sliding_window >= 0 && s->sliding_window % 16 == 0 &&
           s->keep >= 0 && s->keep % 16 == 0 &&
           (s->prefix_rule == GPTOSS_ATTN_PREFIX_REFERENCE || s->prefix_rule == GPTOSS_ATTN_PREFIX_MIXED);
}

bool ring_layer(const gptoss_attn_shape *s, const gptoss_attn_layer *l) {
    return (l->layer_idx & 1) == 0 && s->sliding_window > 0;
}

// Rows a sequence can attend to in this layer.
int layer_rows(const gptoss_attn_shape *s, const gptoss_attn_layer *l) {
    return ring_layer(s, l) ? s->sliding_window : l->cap;
}

bool layer_ok(const gptoss_attn_shape *s, const gptoss_attn_cache *c, const gptoss_attn_layer *l) {
    if (!c || !l) return false;
    if (l->layer_idx < 0 || l->layer_idx >= s->n_layers || l->cap <= 0 || l->cap % 16) return false;
    if (ring_layer(s, l) && l->cap < s->sliding_window) return false;
    if (l->layer_kv_offset % kTile || l->layer_scale_offset % 16) return false;
    if (c->batch_kv_stride % kTile || c->batch_scale_stride % 16) return false;
    if (c->batch_kv_stride < l->layer_kv_offset + (size_t)l->cap * kKvDim) return false;
    if (c->batch_scale_stride < l->layer_scale_offset + (size_t)l->cap) return false;
    if (!c->key_codes || !c->value_codes || !c->key_scales || !c->value_scales) return false;
    if (!aligned(c->key_codes, 16) || !aligned(c->value_codes, 16) || !aligned(c->key_scales, 8) ||
        !aligned(c->value_scales, 8))
        return false;
    if ((l->layer_idx & 1) && s->keep > 0) {
        if (s->keep > l->cap) return false;
        if (!c->key_bf16 || !c->value_bf16 || !aligned(c->key_bf16, 16) || !aligned(c->value_bf16, 16))
            return false;
    }
    return true;
}

void fill_common(const gptoss_attn_shape *s, const gptoss_attn_layer *l, int &window, int &ring,
                 int &odd, int &keep) {
    ring = ring_layer(s, l) ? 1 : 0;
    window = s->sliding_window;
    odd = l->layer_idx & 1;
    keep = odd ? s->keep : 0;
}

int splits_for(const gptoss_attn_shape *s, int rows, int n_seqs) {
    if (n_seqs <= 0) return 1;
    const int waves = n_seqs * kKvHeads;
    int S = (kTargetWaves + waves - 1) / waves;
    S = std::min(S, std::max(1, rows / 16 / 4));  // at least 4 blocks of 16 rows per split
    return std::max(1, std::min(S, kMaxSplits));
}

}  // namespace

extern "C" {

int gptoss_attn_kv_update(const gptoss_attn_shape *shape, const gptoss_attn_cache *cache,
                          const gptoss_attn_layer *layer, const uint16_t *k, const uint16_t *v,
                          const int32_t *pos, int n_seqs, hipStream_t stream) {
    if (!shape_ok(shape) || !layer_ok(shape, cache, layer) || n_seqs < 0) return GPTOSS_ATTN_ERR_INVALID_ARG;
    if (n_seqs == 0) return GPTOSS_ATTN_OK;
    if (!k || !v || !pos || !aligned(k, 16) || !aligned(v, 16) || !aligned(pos, 4))
        return GPTOSS_ATTN_ERR_INVALID_ARG;
    KvArgs a{};
    a.kc = cache->key_codes;
    a.vc = cache->value_codes;
    a.ks = cache->key_scales;
    a.vs = cache->value_scales;
    a.kb = cache->key_bf16;
    a.vb = cache->value_bf16;
    a.bks = cache->batch_kv_stride;
    a.bss = cache->batch_scale_stride;
    a.lko = layer->layer_kv_offset;
    a.lso = layer->layer_scale_offset;
    a.k = k;
    a.v = v;
    a.pos = pos;
    a.cap = layer->cap;
    fill_common(shape, layer, a.window, a.ring, a.odd, a.keep);
    a.n_layers = shape->n_layers;
    a.layer = layer->layer_idx;
    hipLaunchKernelGGL(kv_update_kernel, dim3(n_seqs), dim3(64), 0, stream, a);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? GPTOSS_ATTN_OK : hip_fail(e);
}

size_t gptoss_attn_workspace_size(const gptoss_attn_shape *shape, int cap, int n_seqs) {
    if (!shape_ok(shape) || cap <= 0 || n_seqs <= 0) return 0;
    const int S = splits_for(shape, cap, n_seqs);
    if (S <= 1) return 0;
    return (size_t)n_seqs * kKvHeads * S * kPartFloats * sizeof(float);
}

int gptoss_attn_decode(const gptoss_attn_shape *shape, const gptoss_attn_cache *cache,
                       const gptoss_attn_layer *layer, const uint16_t *q, const uint16_t *sinks,
                       const int32_t *pos, int n_seqs, uint16_t *out, void *ws, size_t ws_bytes,
                       hipStream_t stream) {
    if (!shape_ok(shape) || !layer_ok(shape, cache, layer) || n_seqs < 0) return GPTOSS_ATTN_ERR_INVALID_ARG;
    if (n_seqs == 0) return GPTOSS_ATTN_OK;
    if (!q || !sinks || !pos || !out || !aligned(q, 16) || !aligned(out, 16) || !aligned(pos, 4) ||
        !aligned(sinks, 2))
        return GPTOSS_ATTN_ERR_INVALID_ARG;
    if (ws && !aligned(ws, 256)) return GPTOSS_ATTN_ERR_WORKSPACE;
    DecArgs a{};
    a.kc = cache->key_codes;
    a.vc = cache->value_codes;
    a.ks = cache->key_scales;
    a.vs = cache->value_scales;
    a.kb = cache->key_bf16;
    a.vb = cache->value_bf16;
    a.bks = cache->batch_kv_stride;
    a.bss = cache->batch_scale_stride;
    a.lko = layer->layer_kv_offset;
    a.lso = layer->layer_scale_offset;
    a.q = q;
    a.sinks = sinks;
    a.pos = pos;
    a.out = out;
    a.cap = layer->cap;
    fill_common(shape, layer, a.window, a.ring, a.odd, a.keep);
    a.rule = shape->prefix_rule;
    a.n_layers = shape->n_layers;
    a.layer = layer->layer_idx;
    int S = splits_for(shape, layer_rows(shape, layer), n_seqs);
    const size_t per_split = (size_t)n_seqs * kKvHeads * kPartFloats * sizeof(float);
    if (!ws) S = 1;
    else S = (int)std::min<size_t>((size_t)S, ws_bytes / per_split);
    if (S < 1) S = 1;
    a.splits = S;
    a.ws = (float *)ws;
    hipLaunchKernelGGL(attn_decode_kernel, dim3(n_seqs * kKvHeads * S), dim3(64), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e);
    if (S > 1) {
        hipLaunchKernelGGL(attn_combine_kernel, dim3(n_seqs * kKvHeads), dim3(64), 0, stream, a);
        e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(e);
    }
    return GPTOSS_ATTN_OK;
}

int gptoss_attn_last_hip_error(void) { return g_last_hip_error; }

}  // extern "C"
