// gptoss_attn.hip — decode attention over an int8 (or bf16) KV cache for
// gfx950.
//
// Two kernels per layer and decode step, as in the reference's
// attention_gpu_120b (getp-csrc/getp_run.cpp:2311-2470; the bf16-cache kind
// is attention_gpu's, :2096-2160):
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
// Matrix-core mapping (lane = c + 16 g; every instruction is 16x16, lane
// (c, g) receives rows 4g..4g+3 of column c of the result):
//   scores  S[token][head] = K[16 tokens][64 dims] . Q^T on
//           v_mfma_i32_16x16x64_i8: lane (c, g) supplies key row c, dims
//           16g..16g+15 (the 16 raw bytes of the tile, no conversion) and
//           query head c, the same dims, as Q = rint(q 2^E) = 256 hi + lo
//           (two instructions, exact in int32; |Q| < 2^14, E per head, so Q
//           carries q to 2^-14 of the head's largest element).  Heads 8..15
//           of the instruction are zero.  Lane (c, g) gets head c at tokens
//           4g..4g+3; the score is S * key scale * 2^-E * log2(e) / 8.
//   output  O[head][dim] += P'[head][32 tokens] . V[32 tokens][16 dims] on
//           v_mfma_f32_16x16x32_bf16 for 4 dim tiles: P' = p * value scale
//           (bf16) is the score layout of two 16-token blocks, and the value
//           tile order gives lane (c, g) dims 16 dt + c at tokens 4g..4g+3 of
//           a block in one 16-byte load (int8 -> bf16 exactly).  Rows 4g..4g+3
//           of the result are heads (g < 2).
// bf16-kept blocks use v_mfma_f32_16x16x32_bf16 for the scores with the bf16
// query itself.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>

#include "gptoss_attn.h"

// The last failed HIP call of this thread, for every entry point of the
// library (gptoss_decoder.hip records its own here too).
namespace gptoss_attn_detail {
thread_local int last_hip_error = 0;
}

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(4))) int i32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

constexpr int kKvHeads = 8;      // n_kv_heads
constexpr int kGqa = 8;          // query heads per KV head
constexpr int kHd = 64;          // head_dim
constexpr int kKvDim = kKvHeads * kHd;
constexpr int kTile = 1024;      // elements of one (16-row block, KV head) tile
constexpr int kPartFloats = 2 * kGqa + kGqa * kHd;  // m[8], l[8], o[8][64] of a split
constexpr int kMaxSplits = 64;
constexpr int kTargetWaves = 2048;  // 256 CUs x 8 waves
constexpr float kLog2e = 1.4426950408889634f;

int hip_fail(hipError_t e) {
    gptoss_attn_detail::last_hip_error = (int)e;
    return GPTOSS_ATTN_ERR_HIP;
}

__device__ inline float bf2f(uint32_t h) { return __uint_as_float(h << 16); }

__device__ inline float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

__device__ inline uint16_t f2h(float f) {  // round to nearest even (the default mode)
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ inline bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ inline u32x4 ld16(const void *p) { return *(const u32x4 *)p; }

// ---- global -> LDS loads (lane l writes lds + l * size; lds wave-uniform),
// vmcnt waits and LDS reads as inline asm.  The compiler cannot tell which
// in-flight global -> LDS load a plain LDS read may alias and would drain
// them all before it; here each read follows an explicit vmcnt wait for the
// stage it reads, and each result is tied to an lgkmcnt wait before use.
__device__ inline void lds_dma16_nt(const void *src, void *lds) {
    __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 2);  // nontemporal: streamed once
}
__device__ inline void lds_dma4(const void *src, void *lds) { __builtin_amdgcn_global_load_lds(src, lds, 4, 0, 0); }

template <int N>
__device__ inline void wait_vmcnt() {  // s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding)
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ inline void wait_vmcnt_le(int n) {  // at most n of this wave's loads outstanding, n <= 10
    switch (n) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<1>(); break;
        case 2: wait_vmcnt<2>(); break;
        case 3: wait_vmcnt<3>(); break;
        case 4: wait_vmcnt<4>(); break;
        case 5: wait_vmcnt<5>(); break;
        case 6: wait_vmcnt<6>(); break;
        case 7: wait_vmcnt<7>(); break;
        case 8: wait_vmcnt<8>(); break;
        case 9: wait_vmcnt<9>(); break;
        default: wait_vmcnt<10>(); break;
    }
}
__device__ inline uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
__device__ inline u32x4 lds_read_b128(uint32_t addr) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}
__device__ inline u32x2 lds_read_b64(uint32_t addr) {
    u32x2 v;
    asm volatile("ds_read_b64 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}
__device__ inline void lds_wait_all(u32x4 &a, u32x4 &b, u32x4 &c, u32x4 &d, u32x2 &e, u32x2 &f, u32x2 &g,
                                    u32x2 &h) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e), "+v"(f), "+v"(g), "+v"(h));
}

// ---------------------------------------------------------------------------
// KV-cache update (attention.hpp:536-652): one wave per sequence, lane l owns
// elements 8l..8l+7 of the row (KV head l/8, dims 8(l%8)..8(l%8)+7).
struct KvArgs {
    int8_t *kc, *vc;
    uint16_t *ks, *vs, *kb, *vb;
    size_t bks, bss, lko, lso;
    const uint16_t *k, *v;
    const int32_t *pos;
    int cap, window, ring, odd, keep, n_layers, layer, bf16cache;
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
    if (a.bf16cache) {  // the rows themselves (update_kv_cache_kernel, attention.hpp:756-778)
        uint16_t *kc = reinterpret_cast<uint16_t *>(a.kc), *vc = reinterpret_cast<uint16_t *>(a.vc);
        const size_t tile = (size_t)b * a.bks + a.lko + (size_t)((r >> 4) * kKvHeads + kvh) * kTile;
        *(u32x4 *)(kc + tile + (r & 15) * 64 + d0) = kr;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            vc[tile + v_tile_off(r, d0 + j)] = (uint16_t)(j & 1 ? vr[j >> 1] >> 16 : vr[j >> 1] & 0xffffu);
        return;
    }
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
    int cap, window, ring, odd, keep, rule, n_layers, layer, splits, bf16cache;
};

struct RawI8 {        // an int8 block as loaded: key tile, value tile, scales of tokens 4g..4g+3
    u32x4 k, v;
    u32x2 ks, vs;
};

struct BlkBf {        // a bf16 block (odd layers' kept tokens) in operand form
    u32x4 k0, k1;     // key row c: dims 16g..16g+7 and 16g+8..16g+15
    u32x2 v[4];       // per dim tile: tokens 4g..4g+3 at dim 16 dt + c
};

// One stage of the int8 ring: two blocks' key and value tiles of this
// wave's KV head, and their scales (lane-ordered as the loads write them).
constexpr int kStages = 3;
struct AttnStage {
    u32x4 k[2][64];
    u32x4 v[2][64];
    uint32_t sc[64];
};

struct SoftState {
    float m, l;       // running max (log2 domain) and this lane's part of the sum, for head c
    f32x4 o[4];       // O[head 4g+i][dim 16 dt + c]
};

__device__ inline void load_bf(const DecArgs &a, size_t slab, int kvh, int blk, int c, int g, BlkBf &o) {
    const size_t t = slab + (size_t)(blk * kKvHeads + kvh) * kTile + c * 64 + 16 * g;
    o.k0 = ld16(a.kb + t);
    o.k1 = ld16(a.kb + t + 8);
    const u32x4 v0 = ld16(a.vb + t), v1 = ld16(a.vb + t + 8);
    o.v[0] = u32x2{v0[0], v0[1]};
    o.v[1] = u32x2{v0[2], v0[3]};
    o.v[2] = u32x2{v1[0], v1[1]};
    o.v[3] = u32x2{v1[2], v1[3]};
}

__device__ inline uint32_t pk_bf16(float a, float b) {  // two floats -> bf16x2, nearest even
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// Four signed bytes -> four bf16 (exact).
__device__ inline u32x2 i8x4_bf16(uint32_t w) {
    return u32x2{pk_bf16((float)(int8_t)w, (float)(int8_t)(w >> 8)),
                 pk_bf16((float)(int8_t)(w >> 16), (float)(int8_t)(w >> 24))};
}

__device__ inline void unpack_h4(u32x2 h, float mul, float *out) {  // four fp16 -> float * mul
    out[0] = h2f(h[0] & 0xffffu) * mul;
    out[1] = h2f(h[0] >> 16) * mul;
    out[2] = h2f(h[1] & 0xffffu) * mul;
    out[3] = h2f(h[1] >> 16) * mul;
}

// Online-softmax update and O += P'.V for 32 tokens.  sv: scores (log2
// domain; -inf where masked); vsc(j): value scale of token slot j (0 where
// masked); vop(dt): the value operand of dim tile dt (tokens of the first
// block, then the second).  Both are called where their results are used,
// which keeps them out of the registers live across the softmax.
template <class VScale, class VOp>
__device__ inline void softmax_pv(const float (&sv)[8], VScale vsc, VOp vop, int g, SoftState &st) {
    float bm = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                     fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
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
    const bf16x8 pop = __builtin_bit_cast(
        bf16x8, u32x4{pk_bf16(p[0] * vsc(0), p[1] * vsc(1)), pk_bf16(p[2] * vsc(2), p[3] * vsc(3)),
                      pk_bf16(p[4] * vsc(4), p[5] * vsc(5)), pk_bf16(p[6] * vsc(6), p[7] * vsc(7))});
    // rescale the output rows only when some head's maximum moved (alpha != 1)
    if (__ballot(alpha != 1.f)) {
        float ar[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) ar[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) st.o[dt][i] *= ar[i];
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
        st.o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pop, as_bf16x8(vop(dt)), st.o[dt], 0, 0, 0);
}

// Scores of one int8 key tile: the query as Q = 256 hi + lo (int8 each),
// exact in int32.
__device__ inline i32x4 qk_i8(u32x4 k, i32x4 qh, i32x4 ql) {
    const i32x4 kk = __builtin_bit_cast(i32x4, k);
    i32x4 s = __builtin_amdgcn_mfma_i32_16x16x64_i8(kk, qh, i32x4{0, 0, 0, 0}, 0, 0, 0);
    s = s << 8;
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(kk, ql, s, 0, 0, 0);
}

// Two int8 blocks (32 tokens) from block `blk`, `nb` (1 or 2) present.
// kMask: some row is at or past `nvalid` (else every row counts).
template <bool kMask>
__device__ inline void pair_i8(const RawI8 &A, const RawI8 &B, int blk, int nb, int nvalid, int g,
                               i32x4 qh, i32x4 ql, float qf, SoftState &st) {
    const i32x4 sa = qk_i8(A.k, qh, ql);
    const i32x4 sb = (!kMask || nb > 1) ? qk_i8(B.k, qh, ql) : i32x4{0, 0, 0, 0};
    float sv[8];
    {
        float ksc[8];
        unpack_h4(A.ks, qf, ksc);
        unpack_h4(B.ks, qf, ksc + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sv[i] = (float)sa[i] * ksc[i];
            sv[4 + i] = (float)sb[i] * ksc[4 + i];
        }
    }
    const int row0 = blk * 16 + 4 * g;
    if (kMask) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sv[i] = row0 + i < nvalid ? sv[i] : -INFINITY;
            sv[4 + i] = nb > 1 && row0 + 16 + i < nvalid ? sv[4 + i] : -INFINITY;
        }
    }
    auto vsc = [&](int j) {
        const u32x2 h = j < 4 ? A.vs : B.vs;
        const float v = h2f((j & 2 ? h[1] : h[0]) >> (j & 1 ? 16 : 0) & 0xffffu);
        if (!kMask) return v;
        const bool ok = j < 4 ? row0 + j < nvalid : (nb > 1 && row0 + 12 + j < nvalid);
        return ok ? v : 0.f;
    };
    auto vop = [&](int dt) {
        const u32x2 x = i8x4_bf16(A.v[dt]), y = i8x4_bf16(B.v[dt]);
        return u32x4{x[0], x[1], y[0], y[1]};
    };
    softmax_pv(sv, vsc, vop, g, st);
}

// Two bf16 blocks from block `blk` (`nb` present); values of masked rows
// are cleared, since rows past the written ones may hold anything.
__device__ inline void pair_bf(const BlkBf &A, const BlkBf &B, int blk, int nb, int nvalid, int g,
                               bf16x8 q0, bf16x8 q1, SoftState &st) {
    const f32x4 z = f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 sa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(A.k0), q0, z, 0, 0, 0);
    sa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(A.k1), q1, sa, 0, 0, 0);
    f32x4 sb = z;
    if (nb > 1) {
        sb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(B.k0), q0, z, 0, 0, 0);
        sb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(B.k1), q1, sb, 0, 0, 0);
    }
    const float C = 0.125f * kLog2e;
    const int row0 = blk * 16 + 4 * g;
    float sv[8];
    uint32_t keep[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sv[i] = row0 + i < nvalid ? sa[i] * C : -INFINITY;
        sv[4 + i] = nb > 1 && row0 + 16 + i < nvalid ? sb[i] * C : -INFINITY;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
        keep[j] = (sv[2 * j] != -INFINITY ? 0xffffu : 0u) | (sv[2 * j + 1] != -INFINITY ? 0xffff0000u : 0u);
    auto vsc = [&](int j) { return sv[j] != -INFINITY ? 1.f : 0.f; };
    auto vop = [&](int dt) {
        const u32x2 y = nb > 1 ? B.v[dt] : u32x2{0u, 0u};
        return u32x4{A.v[dt][0] & keep[0], A.v[dt][1] & keep[1], y[0] & keep[2], y[1] & keep[3]};
    };
    softmax_pv(sv, vsc, vop, g, st);
}

__device__ inline bool seq_valid(const DecArgs &a, int pos) { return pos >= 0 && (a.ring || pos < a.cap); }

__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3, 8))) void attn_decode_kernel(DecArgs a) {
    __shared__ AttnStage ring[kStages];
    float *red = reinterpret_cast<float *>(&ring[0]);  // after the loop: the output rows
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
    int nb16 = 0;  // leading blocks read as bf16 rows
    if (a.bf16cache) nb16 = nblk;
    else if (a.odd && a.keep > 0) nb16 = a.rule == GPTOSS_ATTN_PREFIX_REFERENCE ? (pos < a.keep ? nblk : 0)
                                                                              : min(nblk, a.keep >> 4);
    const int blk0 = (int)((int64_t)nblk * s / S), blk1 = (int)((int64_t)nblk * (s + 1) / S);

    // The query of head c (heads 8..15 of the instruction are zero), dims
    // 16g..16g+15: as bf16 for the kept blocks, and as Q = rint(q 2^E) =
    // 256 hi + lo with |Q| < 2^14 (E per head) for the int8 blocks.
    u32x4 qa = u32x4{0u, 0u, 0u, 0u}, qb = qa;
    if (c < kGqa) {
        const uint16_t *qp = a.q + ((size_t)b * kKvHeads * kGqa + kvh * kGqa + c) * kHd + 16 * g;
        qa = ld16(qp);
        qb = ld16(qp + 8);
    }
    const bf16x8 q0 = as_bf16x8(qa), q1 = as_bf16x8(qb);
    float qv[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        qv[2 * j] = bf2f(qa[j] & 0xffffu);
        qv[2 * j + 1] = bf2f(qa[j] >> 16);
        qv[8 + 2 * j] = bf2f(qb[j] & 0xffffu);
        qv[8 + 2 * j + 1] = bf2f(qb[j] >> 16);
    }
    float qm = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) qm = fmaxf(qm, fabsf(qv[j]));
    qm = fmaxf(qm, __shfl_xor(qm, 16));
    qm = fmaxf(qm, __shfl_xor(qm, 32));
    const int E = 14 - __builtin_amdgcn_frexp_expf(qm);  // qm 2^E in [2^13, 2^14)
    uint32_t hw[4] = {0u, 0u, 0u, 0u}, lw[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int Q = (int)__builtin_rintf(__builtin_ldexpf(qv[j], E));
        const int hi = (Q + 128) >> 8, lo = Q - (hi << 8);
        hw[j >> 2] |= (uint32_t)(uint8_t)hi << (8 * (j & 3));
        lw[j >> 2] |= (uint32_t)(uint8_t)lo << (8 * (j & 3));
    }
    const i32x4 qh = __builtin_bit_cast(i32x4, u32x4{hw[0], hw[1], hw[2], hw[3]});
    const i32x4 ql = __builtin_bit_cast(i32x4, u32x4{lw[0], lw[1], lw[2], lw[3]});
    const float qf = __builtin_ldexpf(0.125f * kLog2e, -E);

    SoftState st;
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) st.o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // bf16 rows first (odd layers' kept tokens), then the int8 rows
    const int e16 = min(blk1, nb16);
    if (blk0 < e16) {
        // the kept-token slab of (sequence, layer), or with the bf16 cache the
        // layer's rows of the sequence (the same base kv_update_kernel writes)
        const size_t slab = a.bf16cache ? (size_t)b * a.bks + a.lko
                                        : ((size_t)b * a.n_layers + a.layer) * a.keep * kKvDim;
        // Two register buffers, one pair ahead: the next pair's loads are in
        // flight while this pair computes.  Block indices are clamped to the
        // last block, so every load is of a valid block (a partner past the
        // end is masked by nb, a pair past the end is never computed), and no
        // buffer is ever copied (a copy would wait for its loads).
        auto load_pair = [&](int blk, BlkBf &X, BlkBf &Y) {
            load_bf(a, slab, kvh, min(blk, e16 - 1), c, g, X);
            load_bf(a, slab, kvh, min(blk + 1, e16 - 1), c, g, Y);
        };
        BlkBf A0, B0, A1, B1;
        load_pair(blk0, A0, B0);
        for (int blk = blk0; blk < e16; blk += 4) {
            load_pair(blk + 2, A1, B1);
            pair_bf(A0, B0, blk, min(2, e16 - blk), nvalid, g, q0, q1, st);
            if (blk + 2 >= e16) break;
            load_pair(blk + 4, A0, B0);
            pair_bf(A1, B1, blk + 2, min(2, e16 - blk - 2), nvalid, g, q0, q1, st);
        }
    }
    const int i0 = max(blk0, nb16);
    if (i0 < blk1) {
        // int8 blocks, two per stage, through a ring of kStages LDS slots:
        // stage p (blocks i0 + 2p, +1) lands while earlier stages compute.
        const char *kb = reinterpret_cast<const char *>(a.kc + (size_t)b * a.bks + a.lko) + kvh * kTile;
        const char *vb = reinterpret_cast<const char *>(a.vc + (size_t)b * a.bks + a.lko) + kvh * kTile;
        const char *ksb = reinterpret_cast<const char *>(a.ks + (size_t)b * a.bss + a.lso);
        const char *vsb = reinterpret_cast<const char *>(a.vs + (size_t)b * a.bss + a.lso);
        const int npairs = (blk1 - i0 + 1) >> 1;
        const int last = i0 + 2 * (npairs - 1);
        const int nfull = (blk1 - last == 2 && (last + 2) * 16 <= nvalid) ? npairs : npairs - 1;
        // scale lanes: 0..7 key scales of the first block, 8..15 of the second,
        // 16..23 / 24..31 value scales; lanes 32..63 repeat 0..31
        const int sl = lane & 31;
        const char *sbase = (sl < 16 ? ksb : vsb) + (sl & 7) * 4;
        const int sblk = (sl >> 3) & 1;
        auto loads = [&](int p) { return i0 + 2 * p + 1 < blk1 ? 5 : 3; };  // global -> LDS loads of stage p
        auto issue = [&](int p) {
            AttnStage &sg = ring[p % kStages];
            const int blk = i0 + 2 * p;
            const bool two = blk + 1 < blk1;
            const size_t t0 = (size_t)blk * kKvHeads * kTile;
            const size_t t1 = t0 + (two ? (size_t)kKvHeads * kTile : 0);
            lds_dma16_nt(kb + t0 + 16 * lane, &sg.k[0][0]);
            lds_dma16_nt(vb + t0 + 16 * lane, &sg.v[0][0]);
            if (two) {
                lds_dma16_nt(kb + t1 + 16 * lane, &sg.k[1][0]);
                lds_dma16_nt(vb + t1 + 16 * lane, &sg.v[1][0]);
            }
            lds_dma4(sbase + (size_t)(blk + (two ? sblk : 0)) * 32, &sg.sc[0]);
        };
        for (int p = 0; p < min(kStages - 1, npairs); ++p) issue(p);
        for (int p = 0; p < npairs; ++p) {
            if (p + kStages - 1 < npairs) issue(p + kStages - 1);
            // loads of the stages after p may stay in flight
            int after = 0;
            for (int q = p + 1; q < min(p + kStages, npairs); ++q) after += loads(q);
            wait_vmcnt_le(after);
            const AttnStage &sg = ring[p % kStages];
            const uint32_t ka = lds_addr(&sg.k[0][0]) + c * 64 + 16 * g;
            RawI8 A, B;
            A.k = lds_read_b128(ka);
            A.v = lds_read_b128(ka + (uint32_t)(offsetof(AttnStage, v) - offsetof(AttnStage, k)));
            B.k = lds_read_b128(ka + 1024u);
            B.v = lds_read_b128(ka + 1024u + (uint32_t)(offsetof(AttnStage, v) - offsetof(AttnStage, k)));
            const uint32_t sa = lds_addr(&sg.sc[0]) + 8 * g;
            A.ks = lds_read_b64(sa);
            B.ks = lds_read_b64(sa + 32);
            A.vs = lds_read_b64(sa + 64);
            B.vs = lds_read_b64(sa + 96);
            lds_wait_all(A.k, A.v, B.k, B.v, A.ks, B.ks, A.vs, B.vs);
            asm volatile("" ::: "memory");  // the slot is free for a later stage's loads
            const int blk = i0 + 2 * p;
            if (p < nfull) pair_i8<false>(A, B, blk, 2, nvalid, g, qh, ql, qf, st);
            else pair_i8<true>(A, B, blk, min(2, blk1 - blk), nvalid, g, qh, ql, qf, st);
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
        for (int j = 0; j < 4; ++j) w[j] = pk_bf16(red[8 * lane + 2 * j], red[8 * lane + 2 * j + 1]);
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
    for (int j = 0; j < 4; ++j) w[j] = pk_bf16(o[2 * j] * f, o[2 * j + 1] * f);
    *(u32x4 *)out = u32x4{w[0], w[1], w[2], w[3]};
}

// ---------------------------------------------------------------------------
// Host side.
bool aligned(const void *p, size_t n) { return ((uintptr_t)p % n) == 0; }

bool shape_ok(const gptoss_attn_shape *s) {
    return s && s->n_heads == kKvHeads * kGqa && s->n_kv_heads == kKvHeads && s->head_dim == kHd &&
           s->n_layers >= 1 && s->sliding_window >= 0 && s->sliding_window % 16 == 0 &&
           s->keep >= 0 && s->keep % 16 == 0 &&
           (s->prefix_rule == GPTOSS_ATTN_PREFIX_REFERENCE || s->prefix_rule == GPTOSS_ATTN_PREFIX_MIXED) &&
           (s->cache_kind == GPTOSS_ATTN_CACHE_INT8 || s->cache_kind == GPTOSS_ATTN_CACHE_BF16);
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
    if (!c->key_codes || !c->value_codes || !aligned(c->key_codes, 16) || !aligned(c->value_codes, 16))
        return false;
    if (s->cache_kind == GPTOSS_ATTN_CACHE_BF16) return true;  // rows only: no scales, no kept rows
    if (!c->key_scales || !c->value_scales || !aligned(c->key_scales, 8) || !aligned(c->value_scales, 8))
        return false;
    if ((l->layer_idx & 1) && s->keep > 0) {
        if (s->keep > l->cap) return false;
        if (!c->key_bf16 || !c->value_bf16 || !aligned(c->key_bf16, 16) || !aligned(c->value_bf16, 16))
            return false;
    }
    return true;
}

void fill_common(const gptoss_attn_shape *s, const gptoss_attn_layer *l, int &window, int &ring,
                 int &odd, int &keep, int &bf16cache) {
    ring = ring_layer(s, l) ? 1 : 0;
    window = s->sliding_window;
    odd = l->layer_idx & 1;
    bf16cache = s->cache_kind == GPTOSS_ATTN_CACHE_BF16 ? 1 : 0;
    keep = odd && !bf16cache ? s->keep : 0;
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
    fill_common(shape, layer, a.window, a.ring, a.odd, a.keep, a.bf16cache);
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
    fill_common(shape, layer, a.window, a.ring, a.odd, a.keep, a.bf16cache);
    a.rule = shape->prefix_rule;
    if (a.bf16cache) {  // the blocks are the cache's own bf16 rows
        a.kb = reinterpret_cast<const uint16_t *>(cache->key_codes);
        a.vb = reinterpret_cast<const uint16_t *>(cache->value_codes);
    }
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

int gptoss_attn_last_hip_error(void) { return gptoss_attn_detail::last_hip_error; }

}  // extern "C"
