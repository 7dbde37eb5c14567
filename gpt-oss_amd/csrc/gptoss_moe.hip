// gptoss_moe.hip — MI355X (gfx950) MXFP4 mixture-of-experts layer.
//
// Kernels (one stream, no host round trip):
//   route_kernel   router GEMM (pinned fp32 order) + top-k/softmax + expert
//                  histogram; the last workgroup scans the histogram and
//                  writes the per-expert tile list.
//   index_kernel   per-expert ballot compaction: compact row -> token map.
//   mlp1_kernel    grouped GEMM x[token(row)] . W1[e]^T, MXFP4 dequantised
//                  in registers (v_cvt_scalef32_pk_bf16_fp4) into bf16 MFMA
//                  operands; epilogue: bias + clamped SwiGLU on the
//                  interleaved gate/up rows, bf16 out.
//   mlp2_kernel    grouped GEMM act . W2[e]^T; epilogue: bias, bf16 round,
//                  scatter of each row to its token-order slot [t][k][h].
//   finalize_kernel  router-weighted k-way sum of the slots in slot order
//                  (fmaf, fp32) -> bf16, optionally + residual.
//
// The C ABI (include/gptoss_moe.h) is at the bottom of this file.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/gptoss_moe.h"

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;

constexpr int kWave = 64;
constexpr int kMaxExperts = 256;
constexpr int kMaxTopK = 8;
constexpr int kMaxHidden = 4096;    // router keeps x rows in registers
constexpr int kTileRows = 64;       // rows per grouped-GEMM tile (4 x 16)
constexpr int kBlockN = 128;        // weight rows per workgroup (4 waves x 32)
constexpr int kChunkK = 256;        // k per LDS chunk of activations
constexpr int kUnits = kChunkK / 8; // 16-byte units per LDS row
constexpr int kPipe = 4;            // k-groups (128 k) of weights in flight

// ----------------------------------------------------------------- bf16 --
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {
    __bf16 b = (__bf16)f;  // round to nearest even (v_cvt_pk_bf16_f32)
    return __builtin_bit_cast(uint16_t, b);
}
__device__ __forceinline__ float bf16_round(float f) { return bf2f(f2bf(f)); }

// e8m0 scale byte -> fp32 2^(e-127) (e = 0 -> 0.0), memory/mxfp4.hpp:53.
__device__ __forceinline__ float e8m0_to_f32(uint32_t e) { return __uint_as_float(e << 23); }

// 8 E2M1 codes (one dword, low nibble first) * scale -> 8 bf16.
__device__ __forceinline__ bf16x8 dequant8(uint32_t q, float scale) {
    bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, scale, 0);
    bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, scale, 1);
    bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, scale, 2);
    bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, scale, 3);
    bf16x8 r = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    return r;
}

// The hardware reads the scale operand's exponent field as an OCP e8m0
// (0 -> 2^-127, 255 -> NaN); the reference maps 0 -> 0.0 and 255 -> +Inf.
// For e = 0 keep only the sign bits of the codes, so every element converts
// to +-0 exactly as code * 0.0 does.
__device__ __forceinline__ uint32_t zero_scale_fix(uint32_t q, uint32_t e) {
    return e == 0 ? (q & 0x88888888u) : q;
}

// ------------------------------------------------------- workspace map --
struct WsLayout {
    size_t hdr, counts_hot, counts, offsets, tiles, logits, topk_i, topk_w, local_ids, row_token,
        row_w, row_slot, act, slots, total;
    int max_tiles;
};

// hdr ints: DONE = workgroups finished (reset by the last one), NTILES = tile
// count, STATUS_HOT = dropped slots of the running call, STATUS = last call's.
enum { HDR_DONE = 0, HDR_NTILES = 1, HDR_STATUS_HOT = 2, HDR_STATUS = 4, HDR_INTS = 64 };

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

WsLayout ws_layout(const gptoss_moe_shape &s, int max_tokens) {
    WsLayout L;
    const size_t T = (size_t)(max_tokens > 0 ? max_tokens : 1);
    const size_t E = (size_t)s.n_experts, K = (size_t)s.top_k;
    const size_t P = T * K;
    L.max_tiles = (int)(P / 16 + E + 1);
    size_t o = 0;
    auto take = [&](size_t bytes) {
        size_t at = o;
        o = align_up(o + bytes, 256);
        return at;
    };
    L.hdr = take(HDR_INTS * 4);
    L.counts_hot = take(E * 4);
    L.counts = take(E * 4);
    L.offsets = take((E + 1) * 4);
    L.tiles = take((size_t)L.max_tiles * 16);
    L.logits = take(T * E * 2);
    L.topk_i = take(P * 4);
    L.topk_w = take(P * 2);
    L.local_ids = take(P * 4);
    L.row_token = take(P * 4);
    L.row_w = take(P * 4);
    L.row_slot = take(P * 4);
    L.act = take(P * (size_t)s.intermediate * 2);
    L.slots = take(P * (size_t)s.hidden * 2);
    L.total = o;
    return L;
}

struct Tile {
    int expert, row0, rows, pad;
};

// ------------------------------------------------------------- routing --
// better_pick of moe.hpp:333-342 with the multiplies and adds kept unfused
// so the comparison rounds exactly as written.
__device__ __forceinline__ bool better_pick(float av, int ai, float bv, int bi) {
    const float eps = 1e-6f;
    const float thr = __fmul_rn(eps, fmaxf(fabsf(av), fabsf(bv)));
    if (av > __fadd_rn(bv, thr)) return true;
    if (fabsf(__fsub_rn(av, bv)) <= thr && ai < bi) return true;
    return false;
}

constexpr int kRouteTokens = 2;  // tokens per route workgroup

// One workgroup of 256 threads per kRouteTokens tokens.
//  - router: wave w computes experts e = w, w+4, ... for the tokens; each
//    logit is 64 lane-partial fmaf chains over k = 512 i + 8 l + j plus an
//    xor butterfly, rounded to bf16 (the order the oracle restates);
//  - top-k: wave tt selects for token tt, reproducing the reference's
//    halving-tree arg-max over clamp(nextpow2(E), 64, 512) threads
//    (moe.hpp:465-599) with 64 lanes x R slots;
//  - histogram via device atomics; the last workgroup to finish scans the
//    histogram (and resets it) and writes offsets and the tile list.
__global__ __launch_bounds__(256) void route_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ wr, const uint16_t *__restrict__ br,
    const int32_t *__restrict__ forced_i, const uint16_t *__restrict__ forced_w, int T, int H, int E,
    int K, uint16_t *__restrict__ logits, int32_t *__restrict__ topk_i, uint16_t *__restrict__ topk_w,
    int32_t *__restrict__ local_ids, int32_t *counts_hot, int32_t *__restrict__ counts,
    int32_t *__restrict__ offsets, Tile *__restrict__ tiles, int32_t *hdr, int nthreads_ref) {
    __shared__ float s_score[kRouteTokens][kMaxExperts];
    __shared__ int s_last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.x * kRouteTokens;

    if (forced_i == nullptr) {
        // ---- router logits
        constexpr int NI = kMaxHidden / 512;
        float xf[kRouteTokens][NI][8];
        const int ni = (H + 511) / 512;
#pragma unroll
        for (int tt = 0; tt < kRouteTokens; ++tt) {
            const int t = min(t0 + tt, T - 1);
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int k = 512 * i + 8 * lane;
                uint4 v = make_uint4(0, 0, 0, 0);
                if (i < ni && k < H) v = *reinterpret_cast<const uint4 *>(x + (size_t)t * H + k);
                const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    xf[tt][i][2 * j] = __uint_as_float(d[j] << 16);
                    xf[tt][i][2 * j + 1] = __uint_as_float(d[j] & 0xffff0000u);
                }
            }
        }
        for (int e = wave; e < E; e += 4) {
            float p[kRouteTokens];
#pragma unroll
            for (int tt = 0; tt < kRouteTokens; ++tt) p[tt] = 0.f;
            const uint16_t *wrow = wr + (size_t)e * H;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int k = 512 * i + 8 * lane;
                if (i < ni && k < H) {
                    const uint4 v = *reinterpret_cast<const uint4 *>(wrow + k);
                    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float w0 = __uint_as_float(d[j] << 16);
                        const float w1 = __uint_as_float(d[j] & 0xffff0000u);
#pragma unroll
                        for (int tt = 0; tt < kRouteTokens; ++tt) {
                            p[tt] = __builtin_fmaf(xf[tt][i][2 * j], w0, p[tt]);
                            p[tt] = __builtin_fmaf(xf[tt][i][2 * j + 1], w1, p[tt]);
                        }
                    }
                }
            }
#pragma unroll
            for (int tt = 0; tt < kRouteTokens; ++tt) {
                float v = p[tt];
#pragma unroll
                for (int s = 32; s >= 1; s >>= 1) v = __fadd_rn(v, __shfl_xor(v, s, 64));
                const int t = t0 + tt;
                if (lane == 0 && t < T) {
                    const uint16_t lb = f2bf(v);
                    logits[(size_t)t * E + e] = lb;
                    s_score[tt][e] = __fadd_rn(bf2f(lb), bf2f(br[e]));
                }
            }
        }
        __syncthreads();

        // ---- top-k + softmax, one wave per token
        if (wave < kRouteTokens && t0 + wave < T) {
            const int t = t0 + wave;
            const int R = nthreads_ref / 64;  // 1, 2 or 4 slots per lane
            float sv[4];
            int si[4];
            uint32_t visited = 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = lane + 64 * r;
                const bool ok = r < R && i < E;
                sv[r] = ok ? s_score[wave][i] : -INFINITY;
                si[r] = ok ? i : E;
            }
            int sel_i[kMaxTopK];
            float sel_v[kMaxTopK];
            for (int s = 0; s < K; ++s) {
                float cv[4];
                int ci[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bool live = (si[r] < E) && !((visited >> r) & 1u);
                    cv[r] = live ? sv[r] : -INFINITY;
                    ci[r] = live ? si[r] : E;
                }
                // tree strides >= 64 of the reference: combine slots
                for (int q = R >> 1; q >= 1; q >>= 1)
                    for (int r = 0; r < q; ++r)
                        if (better_pick(cv[r + q], ci[r + q], cv[r], ci[r])) {
                            cv[r] = cv[r + q];
                            ci[r] = ci[r + q];
                        }
                float bv = cv[0];
                int bi = ci[0];
                // tree strides 32..1: lanes l < s take lane l+s's pick if better
#pragma unroll
                for (int st = 32; st >= 1; st >>= 1) {
                    const float ov = __shfl_down(bv, st, 64);
                    const int oi = __shfl_down(bi, st, 64);
                    if (lane < st && better_pick(ov, oi, bv, bi)) {
                        bv = ov;
                        bi = oi;
                    }
                }
                bv = __shfl(bv, 0, 64);
                bi = __shfl(bi, 0, 64);
                sel_i[s] = bi;
                sel_v[s] = bv;
                if (bi < E && (bi & 63) == lane) visited |= 1u << (bi >> 6);
            }
            if (lane == 0) {
                float mx = sel_v[0];
                for (int s = 1; s < K; ++s) mx = fmaxf(mx, sel_v[s]);
                float ex[kMaxTopK], sum = 0.f;
                for (int s = 0; s < K; ++s) {
                    ex[s] = expf(__fsub_rn(sel_v[s], mx));
                    sum = __fadd_rn(sum, ex[s]);
                }
                const float inv = 1.f / __fadd_rn(sum, 1e-20f);
                for (int s = 0; s < K; ++s) {
                    const int e = sel_i[s] < E ? sel_i[s] : -1;
                    topk_i[(size_t)t * K + s] = e;
                    topk_w[(size_t)t * K + s] = f2bf(__fmul_rn(ex[s], inv));
                    if (e >= 0) {
                        atomicAdd(&counts_hot[e], 1);
                    } else {
                        local_ids[(size_t)t * K + s] = -1;
                        atomicAdd(&hdr[HDR_STATUS_HOT], 1);
                    }
                }
            }
        }
    } else {
        // ---- forced routing: copy, validate, count
        if (tid < kRouteTokens * K) {
            const int tt = tid / K, s = tid % K, t = t0 + tt;
            if (t < T) {
                const int e = forced_i[(size_t)t * K + s];
                bool live = e >= 0 && e < E;
                for (int j = 0; j < s; ++j)
                    if (forced_i[(size_t)t * K + j] == e) live = false;
                topk_i[(size_t)t * K + s] = e;
                topk_w[(size_t)t * K + s] = forced_w[(size_t)t * K + s];
                if (live) {
                    atomicAdd(&counts_hot[e], 1);
                } else {
                    local_ids[(size_t)t * K + s] = -1;
                    atomicAdd(&hdr[HDR_STATUS_HOT], 1);
                }
            }
        }
    }

    // ---- last workgroup: scan, reset histogram, tile list
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = (atomicAdd(&hdr[HDR_DONE], 1) == (int)gridDim.x - 1);
    __syncthreads();
    if (!s_last || wave != 0) return;
    __threadfence();
    // lane l owns experts 4l .. 4l+3
    int c[4], nt[4];
    int csum = 0, tsum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = 4 * lane + j;
        c[j] = e < E ? atomicExch(&counts_hot[e], 0) : 0;
        nt[j] = (c[j] + kTileRows - 1) / kTileRows;
        csum += c[j];
        tsum += nt[j];
    }
    int cinc = csum, tinc = tsum;
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) {
        const int oc = __shfl_up(cinc, s, 64), ot = __shfl_up(tinc, s, 64);
        if (lane >= s) {
            cinc += oc;
            tinc += ot;
        }
    }
    int off = cinc - csum, toff = tinc - tsum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = 4 * lane + j;
        if (e < E) {
            counts[e] = c[j];
            offsets[e] = off;
            for (int m = 0; m < nt[j]; ++m) {
                Tile tl;
                tl.expert = e;
                tl.row0 = off + m * kTileRows;
                tl.rows = min(kTileRows, c[j] - m * kTileRows);
                tl.pad = 0;
                tiles[toff + m] = tl;
            }
        }
        off += c[j];
        toff += nt[j];
    }
    if (lane == 63) {
        offsets[E] = off;
        hdr[HDR_NTILES] = toff;
        hdr[HDR_STATUS] = atomicExch(&hdr[HDR_STATUS_HOT], 0);
        hdr[HDR_DONE] = 0;
    }
}

// Compact row map (route_build_index_kernel_bf16wts, moe.hpp:1173-1270):
// one workgroup per expert; rows of expert e are assigned in ascending
// token order with wave ballots.
__global__ __launch_bounds__(256) void index_kernel(const int32_t *__restrict__ topk_i,
                                                   const uint16_t *__restrict__ topk_w, int T, int K,
                                                   int E, const int32_t *__restrict__ offsets,
                                                   int32_t *__restrict__ local_ids,
                                                   int32_t *__restrict__ row_token,
                                                   float *__restrict__ row_w,
                                                   int32_t *__restrict__ row_slot) {
    __shared__ int s_wcount[4];
    const int e = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int carry = 0;
    const int base_row = offsets[e];
    for (int base = 0; base < T; base += 256) {
        const int t = base + tid;
        int kk = -1;
        if (t < T) {
            for (int s = 0; s < K; ++s) {
                const int v = topk_i[(size_t)t * K + s];
                if (v == e) {
                    bool dup = false;
                    for (int j = 0; j < s; ++j) dup |= topk_i[(size_t)t * K + j] == e;
                    if (!dup) kk = s;
                    break;
                }
            }
        }
        const uint64_t m = __ballot(kk >= 0);
        const int rank = __popcll(m & ((1ull << lane) - 1ull));
        if (lane == 0) s_wcount[wave] = __popcll(m);
        __syncthreads();
        int wbase = 0, total = 0;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            if (w < wave) wbase += s_wcount[w];
            total += s_wcount[w];
        }
        if (kk >= 0) {
            const int row = base_row + carry + wbase + rank;
            local_ids[(size_t)t * K + kk] = row;
            row_token[row] = t;
            row_w[row] = bf2f(topk_w[(size_t)t * K + kk]);
            row_slot[row] = t * K + kk;
        }
        carry += total;
        __syncthreads();
    }
}

// ---------------------------------------------------- grouped GEMM core --
//
// Workgroup = 4 waves; a tile of up to 64 activation rows against 128 weight
// rows (32 per wave).  Weights go HBM -> registers (16 B per lane = one
// 32-element e8m0 block of one weight row) with kPipe k-groups in flight and
// are dequantised in registers straight into the bf16 MFMA B operand.
// Activation rows are staged through LDS in chunks of 256 k with an XOR
// swizzle (16-byte unit c of row r stored at unit c ^ (r & 15)).
//
// MFMA v_mfma_f32_16x16x32_bf16: lane l = (n = l & 15, g = l >> 4).  For
// k-group kg (128 k) the lane's weight bytes cover k = 128 kg + 32 g .. +31;
// MFMA step s (0..3) takes k = 128 kg + 32 g + 8 s + (0..7) from both the A
// rows (LDS) and the weight row, which is a permutation of k shared by both
// operands.  Output: lane holds C[m = 4 g + v][n] for v = 0..3.

struct GemmArgs {
    const uint16_t *A;          // activations (x for MLP1, act for MLP2)
    const int32_t *row_token;   // compact row -> token
    const int32_t *row_slot;    // compact row -> token-order slot t*k + j
    const uint8_t *Wq;          // MXFP4 nibbles, all experts
    const uint8_t *Ws;          // e8m0 scales, all experts
    const uint16_t *bias;       // bf16 [E][N]
    const Tile *tiles;
    const int32_t *hdr;
    uint16_t *out_act;          // MLP1: bf16 [P][N/2]
    uint16_t *out_slots;        // MLP2: bf16 [T*k][N]
    int N, K;                   // weight rows / reduction length
    float limit, alpha;
};

// Weight row of tile t (0/1) for this lane: MLP1 pairs gate (t = 0) and up
// (t = 1) rows of the same output column in the same lane; MLP2 is plain.
template <bool kMlp1>
__device__ __forceinline__ int weight_row(int wcol0, int n, int t) {
    return kMlp1 ? wcol0 + 2 * n + t : wcol0 + 16 * t + n;
}

template <int MT, bool kMlp1>
__device__ __forceinline__ void gemm_tile(const GemmArgs &a, const Tile &tl, int nb,
                                          uint4 *__restrict__ lds) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n_l = lane & 15, g = lane >> 4;
    const int N = a.N, K = a.K;
    const int e = tl.expert;
    const int wcol0 = nb * kBlockN + wave * 32;
    const bool wave_active = wcol0 < N;  // N is a multiple of 32
    const int KG = (K + 127) / 128;
    const int NCH = (K + kChunkK - 1) / kChunkK;

    // ---- weight stream setup
    const size_t seg_el = (size_t)N * K;
    const uint8_t *wq = a.Wq + (size_t)e * (seg_el / 2);
    const uint8_t *ws = a.Ws + (size_t)e * (seg_el / 32);
    const uint8_t *qptr[2];
    const uint8_t *sptr[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int row = wave_active ? weight_row<kMlp1>(wcol0, n_l, t) : 0;
        qptr[t] = wq + ((size_t)row * K + 32 * g) / 2;
        sptr[t] = ws + ((size_t)row * K + 32 * g) / 32;
    }
    uint4 q[kPipe][2];
    uint32_t sc[kPipe][2];
    auto load_group = [&](int kg, int stage) {
        const bool ok = wave_active && (kg * 128 + 32 * g < K);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            if (ok) {
                q[stage][t] = *reinterpret_cast<const uint4 *>(qptr[t] + kg * 64);
                sc[stage][t] = sptr[t][kg * 4];
            } else {
                q[stage][t] = make_uint4(0, 0, 0, 0);
                sc[stage][t] = 0;
            }
        }
    };

    // ---- activation staging: thread owns units u = tid + 256 i
    constexpr int UPT = MT * 16 * kUnits / 256;  // units per thread (2 MT)
    const uint16_t *arow[UPT];
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
        const int r = (tid + 256 * i) / kUnits;
        if (r < tl.rows) {
            const int grow = tl.row0 + r;
            const size_t src_row = kMlp1 ? (size_t)a.row_token[grow] : (size_t)grow;
            arow[i] = a.A + src_row * K;
        } else {
            arow[i] = nullptr;
        }
    }
    uint4 stage_a[UPT];
    auto load_a = [&](int ch) {
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
            const int c = (tid + 256 * i) % kUnits;
            const int k = ch * kChunkK + 8 * c;
            stage_a[i] = (arow[i] != nullptr && k < K)
                             ? *reinterpret_cast<const uint4 *>(arow[i] + k)
                             : make_uint4(0, 0, 0, 0);
        }
    };
    auto store_a = [&]() {
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
            const int u = tid + 256 * i;
            const int r = u / kUnits, c = u % kUnits;
            lds[r * kUnits + (c ^ (r & 15))] = stage_a[i];
        }
    };

    f32x4 acc[MT][2];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[m][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // ---- prologue
    load_a(0);
#pragma unroll
    for (int u = 0; u < kPipe; ++u)
        if (u < KG) load_group(u, u);
    store_a();
    __syncthreads();
    if (NCH > 1) load_a(1);

    // ---- main loop over k-groups, kPipe at a time so stages are static
    for (int kg0 = 0; kg0 < KG; kg0 += kPipe) {
#pragma unroll
        for (int u = 0; u < kPipe; ++u) {
            const int kg = kg0 + u;
            if (kg < KG) {
                const int cbase = (kg & 1) * 16 + 4 * g;  // LDS unit of step 0
                if (wave_active) {
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const uint32_t d0 = (s == 0)   ? q[u][0].x
                                            : (s == 1) ? q[u][0].y
                                            : (s == 2) ? q[u][0].z
                                                       : q[u][0].w;
                        const uint32_t d1 = (s == 0)   ? q[u][1].x
                                            : (s == 1) ? q[u][1].y
                                            : (s == 2) ? q[u][1].z
                                                       : q[u][1].w;
                        const bf16x8 b0 = dequant8(zero_scale_fix(d0, sc[u][0]), e8m0_to_f32(sc[u][0]));
                        const bf16x8 b1 = dequant8(zero_scale_fix(d1, sc[u][1]), e8m0_to_f32(sc[u][1]));
#pragma unroll
                        for (int m = 0; m < MT; ++m) {
                            const int r = m * 16 + n_l;
                            const uint4 av = lds[r * kUnits + ((cbase + s) ^ n_l)];
                            const bf16x8 af = __builtin_bit_cast(bf16x8, av);
                            acc[m][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, b0, acc[m][0], 0, 0, 0);
                            acc[m][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, b1, acc[m][1], 0, 0, 0);
                        }
                    }
                }
                if (kg + kPipe < KG) load_group(kg + kPipe, u);
                // end of an activation chunk: swap in the next one
                if ((kg & 1) == 1 && kg + 1 < KG) {
                    const int next = (kg >> 1) + 1;
                    __syncthreads();
                    store_a();
                    __syncthreads();
                    if (next + 1 < NCH) load_a(next + 1);
                }
            }
        }
    }

    // ---- epilogues
    if (!wave_active) return;
    if (kMlp1) {
        const int D = N / 2;
        const int j = wcol0 / 2 + n_l;
        const float bg = bf2f(a.bias[(size_t)e * N + 2 * j]);
        const float bu = bf2f(a.bias[(size_t)e * N + 2 * j + 1]);
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int r = m * 16 + 4 * g + v;
                if (r < tl.rows) {
                    float gt = bf16_round(acc[m][0][v] + bg);
                    float up = bf16_round(acc[m][1][v] + bu);
                    gt = fminf(fmaxf(gt, -a.limit), a.limit);
                    up = fminf(fmaxf(up, -a.limit), a.limit);
                    const float sig = 1.0f / (1.0f + __expf(-a.alpha * gt));
                    gt = gt * sig;
                    a.out_act[(size_t)(tl.row0 + r) * D + j] = f2bf(__builtin_fmaf(gt, up, gt));
                }
            }
    } else {
        const int H = N;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int h = wcol0 + 16 * t + n_l;
            const float bb = bf2f(a.bias[(size_t)e * N + h]);
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int r = m * 16 + 4 * g + v;
                    if (r < tl.rows) {
                        const int row = tl.row0 + r;
                        a.out_slots[(size_t)a.row_slot[row] * H + h] = f2bf(acc[m][t][v] + bb);
                    }
                }
        }
    }
}

// Persistent grouped GEMM: workgroups stride over (tile, 128-row weight block)
// items; the tile count comes from the device-side tile list.
template <bool kMlp1>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(GemmArgs a) {
    __shared__ uint4 lds[kTileRows * kUnits];
    const int ntiles = a.hdr[HDR_NTILES];
    const int nblk = (a.N + kBlockN - 1) / kBlockN;
    const int items = ntiles * nblk;
    for (int it = blockIdx.x; it < items; it += gridDim.x) {
        const Tile tl = a.tiles[it / nblk];
        const int nb = it % nblk;
        const int mt = (tl.rows + 15) / 16;
        __syncthreads();  // previous item finished with LDS
        switch (mt) {
            case 1: gemm_tile<1, kMlp1>(a, tl, nb, lds); break;
            case 2: gemm_tile<2, kMlp1>(a, tl, nb, lds); break;
            case 3: gemm_tile<3, kMlp1>(a, tl, nb, lds); break;
            default: gemm_tile<4, kMlp1>(a, tl, nb, lds); break;
        }
    }
}

// Weighted top-k reduction (reduce_tokenwise_expert_outputs_bf16_bf16wts,
// moe.hpp:700-730): e_agg[t][h] = bf16(sum over live slots j, in slot order,
// of fmaf(w[t][j], y[t][j][h], acc)); with residual, out = bf16(out + e_agg)
// (other_kernels.hpp:17-35).  Thread per (token, 8 columns).
__global__ __launch_bounds__(256) void finalize_kernel(const uint16_t *__restrict__ slots,
                                                      const int32_t *__restrict__ local_ids,
                                                      const uint16_t *__restrict__ topk_w,
                                                      uint16_t *__restrict__ out, int T, int H,
                                                      int K, int residual) {
    const int h8 = H / 8;
    const size_t n = (size_t)T * h8;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const int t = (int)(i / h8), c = (int)(i % h8);
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j < K; ++j) {
            if (local_ids[(size_t)t * K + j] < 0) continue;
            const float w = bf2f(topk_w[(size_t)t * K + j]);
            const uint4 y = *reinterpret_cast<const uint4 *>(slots + ((size_t)t * K + j) * H + 8 * c);
            const uint32_t d[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[2 * q] = __builtin_fmaf(w, __uint_as_float(d[q] << 16), acc[2 * q]);
                acc[2 * q + 1] = __builtin_fmaf(w, __uint_as_float(d[q] & 0xffff0000u), acc[2 * q + 1]);
            }
        }
        uint4 *po = reinterpret_cast<uint4 *>(out + (size_t)t * H + 8 * c);
        uint32_t r[4];
        if (residual) {
            const uint4 p = *po;
            const uint32_t pd[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t lo = f2bf(__fadd_rn(__uint_as_float(pd[q] << 16), bf16_round(acc[2 * q])));
                const uint32_t hi = f2bf(__fadd_rn(__uint_as_float(pd[q] & 0xffff0000u), bf16_round(acc[2 * q + 1])));
                r[q] = lo | (hi << 16);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                r[q] = (uint32_t)f2bf(acc[2 * q]) | ((uint32_t)f2bf(acc[2 * q + 1]) << 16);
        }
        *po = make_uint4(r[0], r[1], r[2], r[3]);
    }
}

// rmsnorm_kernel_bf16_io (rmsnorm.hpp:113-164): 256 threads per row, double
// partial sums with a halving tree.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t *__restrict__ x,
                                                     const uint16_t *__restrict__ w,
                                                     uint16_t *__restrict__ out, int size) {
    __shared__ double ss[256];
    const int r = blockIdx.x, tid = threadIdx.x;
    const uint16_t *xr = x + (size_t)r * size;
    double s = 0.0;
    for (int i = tid; i < size; i += 256) {
        const double v = (double)bf2f(xr[i]);
        s = __dadd_rn(s, __dmul_rn(v, v));
    }
    ss[tid] = s;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if (tid < st) ss[tid] = __dadd_rn(ss[tid], ss[tid + st]);
        __syncthreads();
    }
    const double inv = 1.0 / sqrt(ss[0] / (double)size + 1e-5);
    const float invf = (float)inv;
    for (int i = tid; i < size; i += 256)
        out[(size_t)r * size + i] = f2bf(__fmul_rn(bf2f(w[i]), __fmul_rn(invf, bf2f(xr[i]))));
}

// MXFP4 -> bf16 with the GEMMs' conversion (dequant8 + zero_scale_fix),
// thread per 8 elements.  Scale byte 255 (X = +Inf in the reference) is
// written as the reference's code * Inf: +-Inf, NaN for the +-0 codes.
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ packed,
                                                     const uint8_t *__restrict__ scales,
                                                     int64_t seg, uint16_t *__restrict__ out) {
    const int e = blockIdx.y;
    const uint8_t *pq = packed + (size_t)e * ((seg + 1) / 2);
    const uint8_t *ps = scales + (size_t)e * ((seg + 31) / 32);
    uint16_t *po = out + (size_t)e * seg;
    const int64_t n8 = (seg + 7) / 8;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8;
         i += (int64_t)gridDim.x * 256) {
        const int64_t el = i * 8;
        const int nv = (int)min<int64_t>(8, seg - el);
        uint32_t q = 0;
        for (int b = 0; b < (nv + 1) / 2; ++b) q |= (uint32_t)pq[el / 2 + b] << (8 * b);
        const uint32_t sc = ps[el >> 5];
        uint4 v = __builtin_bit_cast(uint4, dequant8(zero_scale_fix(q, sc), e8m0_to_f32(sc)));
        if (sc == 255) {
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t code = (q >> (4 * j)) & 0xFu;
                const uint32_t bits = (code & 7u) == 0 ? 0x7fc0u : ((code & 8u) ? 0xff80u : 0x7f80u);
                if (j & 1) w[j >> 1] |= bits << 16; else w[j >> 1] = bits;
            }
            v = make_uint4(w[0], w[1], w[2], w[3]);
        }
        if (nv == 8 && (((uintptr_t)(po + el)) & 15) == 0) {
            *reinterpret_cast<uint4 *>(po + el) = v;
        } else {
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            for (int j = 0; j < nv; ++j) po[el + j] = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
        }
    }
}

// ------------------------------------------------------------ host side --
thread_local int g_last_hip_error = 0;

int hip_status(hipError_t err) {
    if (err == hipSuccess) return GPTOSS_MOE_OK;
    g_last_hip_error = (int)err;
    return GPTOSS_MOE_ERR_HIP;
}

int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
            v = 256;
        cus[dev] = v;
    }
    return cus[dev];
}

bool shape_ok(const gptoss_moe_shape *s) {
    if (!s) return false;
    if (s->hidden <= 0 || s->intermediate <= 0) return false;
    if (s->hidden % 32 || s->intermediate % 32) return false;
    if (s->n_experts < 1 || s->n_experts > kMaxExperts) return false;
    if (s->top_k < 1 || s->top_k > kMaxTopK || s->top_k > s->n_experts) return false;
    if (!(s->swiglu_limit > 0.f) || !(s->swiglu_alpha > 0.f)) return false;
    return true;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

struct Ptrs {
    int32_t *hdr, *counts_hot, *counts, *offsets, *topk_i, *local_ids, *row_token;
    Tile *tiles;
    uint16_t *logits, *topk_w, *act, *slots;
    int32_t *row_slot;
    float *row_w;
};

Ptrs ws_ptrs(const WsLayout &L, void *ws) {
    char *b = (char *)ws;
    Ptrs p;
    p.hdr = (int32_t *)(b + L.hdr);
    p.counts_hot = (int32_t *)(b + L.counts_hot);
    p.counts = (int32_t *)(b + L.counts);
    p.offsets = (int32_t *)(b + L.offsets);
    p.tiles = (Tile *)(b + L.tiles);
    p.logits = (uint16_t *)(b + L.logits);
    p.topk_i = (int32_t *)(b + L.topk_i);
    p.topk_w = (uint16_t *)(b + L.topk_w);
    p.local_ids = (int32_t *)(b + L.local_ids);
    p.row_token = (int32_t *)(b + L.row_token);
    p.row_w = (float *)(b + L.row_w);
    p.row_slot = (int32_t *)(b + L.row_slot);
    p.act = (uint16_t *)(b + L.act);
    p.slots = (uint16_t *)(b + L.slots);
    return p;
}

int check_common(const gptoss_moe_shape *shape, const gptoss_moe_weights *w, int n_tokens,
                 const int32_t *fi, const uint16_t *fw, void *ws, size_t ws_bytes, int max_tokens) {
    if (!shape_ok(shape) || !w) return GPTOSS_MOE_ERR_INVALID_ARG;
    if (shape->hidden > kMaxHidden) return GPTOSS_MOE_ERR_UNSUPPORTED;
    if (n_tokens < 0 || max_tokens < 0 || n_tokens > max_tokens) return GPTOSS_MOE_ERR_INVALID_ARG;
    if ((fi == nullptr) != (fw == nullptr)) return GPTOSS_MOE_ERR_INVALID_ARG;
    if (fi == nullptr && (!w->router_w || !w->router_b || !aligned16(w->router_w)))
        return GPTOSS_MOE_ERR_INVALID_ARG;
    if (!ws || !aligned16(ws)) return GPTOSS_MOE_ERR_WORKSPACE;
    if (ws_bytes < ws_layout(*shape, max_tokens).total) return GPTOSS_MOE_ERR_WORKSPACE;
    return GPTOSS_MOE_OK;
}

// Optional event marks between kernels for gptoss_moe_forward_profiled.
struct Marks {
    hipEvent_t ev[8];
    int n = 0;
    bool on = false;
    void mark(hipStream_t st) {
        if (on && n < 8) (void)hipEventRecord(ev[n++], st);
    }
};

int launch_route(const gptoss_moe_shape *s, const gptoss_moe_weights *w, const uint16_t *x,
                 int T, const int32_t *fi, const uint16_t *fw, const Ptrs &p, hipStream_t st,
                 Marks *mk = nullptr) {
    int nthreads_ref = 1;
    while (nthreads_ref < s->n_experts) nthreads_ref <<= 1;
    nthreads_ref = nthreads_ref < 64 ? 64 : (nthreads_ref > 512 ? 512 : nthreads_ref);
    const int grid = (T + kRouteTokens - 1) / kRouteTokens;
    hipLaunchKernelGGL(route_kernel, dim3(grid), dim3(256), 0, st, x, w->router_w, w->router_b,
                       fi, fw, T, s->hidden, s->n_experts, s->top_k, p.logits, p.topk_i, p.topk_w,
                       p.local_ids, p.counts_hot, p.counts, p.offsets, p.tiles, p.hdr,
                       nthreads_ref);
    if (mk) mk->mark(st);
    hipLaunchKernelGGL(index_kernel, dim3(s->n_experts), dim3(256), 0, st, p.topk_i, p.topk_w, T,
                       s->top_k, s->n_experts, p.offsets, p.local_ids, p.row_token, p.row_w,
                       p.row_slot);
    if (mk) mk->mark(st);
    return hip_status(hipGetLastError());
}

int launch_experts(const gptoss_moe_shape *s, const gptoss_moe_weights *w, const uint16_t *x,
                   uint16_t *out, int T, unsigned flags, const WsLayout &L, const Ptrs &p,
                   hipStream_t st, Marks *mk = nullptr) {
    const int H = s->hidden, D = s->intermediate;
    const int occupancy = 2;
    const int cap = device_cus() * occupancy;

    GemmArgs a1;
    memset(&a1, 0, sizeof(a1));
    a1.A = x;
    a1.row_token = p.row_token;
    a1.row_slot = p.row_slot;
    a1.Wq = w->w1;
    a1.Ws = w->w1_scales;
    a1.bias = w->b1;
    a1.tiles = p.tiles;
    a1.hdr = p.hdr;
    a1.out_act = p.act;
    a1.N = 2 * D;
    a1.K = H;
    a1.limit = s->swiglu_limit;
    a1.alpha = s->swiglu_alpha;
    const int max_tiles = (int)((size_t)T * s->top_k / 16 + s->n_experts + 1);
    const int items1 = max_tiles * ((2 * D + kBlockN - 1) / kBlockN);
    hipLaunchKernelGGL(grouped_gemm_kernel<true>, dim3(items1 < cap ? items1 : cap), dim3(256), 0,
                       st, a1);
    if (mk) mk->mark(st);

    GemmArgs a2 = a1;
    a2.A = p.act;
    a2.Wq = w->w2;
    a2.Ws = w->w2_scales;
    a2.bias = w->b2;
    a2.out_act = nullptr;
    a2.out_slots = p.slots;
    a2.N = H;
    a2.K = D;
    const int items2 = max_tiles * ((H + kBlockN - 1) / kBlockN);
    hipLaunchKernelGGL(grouped_gemm_kernel<false>, dim3(items2 < cap ? items2 : cap), dim3(256), 0,
                       st, a2);
    if (mk) mk->mark(st);

    const size_t n8 = (size_t)T * H / 8;
    int fgrid = (int)((n8 + 255) / 256);
    if (fgrid > 4 * device_cus()) fgrid = 4 * device_cus();
    hipLaunchKernelGGL(finalize_kernel, dim3(fgrid), dim3(256), 0, st, p.slots, p.local_ids,
                       p.topk_w, out, T, H, s->top_k,
                       (flags & GPTOSS_MOE_FLAG_RESIDUAL_ADD) ? 1 : 0);
    if (mk) mk->mark(st);
    (void)L;
    return hip_status(hipGetLastError());
}

}  // namespace

// ================================================================ C ABI ==
extern "C" {

size_t gptoss_moe_workspace_size(const gptoss_moe_shape *shape, int max_tokens) {
    if (!shape_ok(shape) || max_tokens < 0) return 0;
    return ws_layout(*shape, max_tokens).total;
}

int gptoss_moe_workspace_init(void *workspace, size_t ws_bytes, hipStream_t stream) {
    if (!workspace) return GPTOSS_MOE_ERR_WORKSPACE;
    return hip_status(hipMemsetAsync(workspace, 0, ws_bytes, stream));
}

int gptoss_moe_workspace_views(const gptoss_moe_shape *shape, int max_tokens, void *workspace,
                               size_t ws_bytes, gptoss_moe_views *v) {
    if (!shape_ok(shape) || !v || max_tokens < 0) return GPTOSS_MOE_ERR_INVALID_ARG;
    const WsLayout L = ws_layout(*shape, max_tokens);
    if (!workspace || ws_bytes < L.total) return GPTOSS_MOE_ERR_WORKSPACE;
    const Ptrs p = ws_ptrs(L, workspace);
    v->logits = p.logits;
    v->topk_i = p.topk_i;
    v->topk_w = p.topk_w;
    v->counts = p.counts;
    v->offsets = p.offsets;
    v->local_ids = p.local_ids;
    v->row_token = p.row_token;
    v->row_weight = p.row_w;
    v->act = p.act;
    v->slots = p.slots;
    v->row_slot = p.row_slot;
    v->status = p.hdr + HDR_STATUS;
    return GPTOSS_MOE_OK;
}

int gptoss_moe_route(const gptoss_moe_shape *shape, const gptoss_moe_weights *w,
                     const uint16_t *x_norm, int n_tokens, const int32_t *forced_topk_i,
                     const uint16_t *forced_topk_w, void *workspace, size_t ws_bytes,
                     int max_tokens, hipStream_t stream) {
    int rc = check_common(shape, w, n_tokens, forced_topk_i, forced_topk_w, workspace, ws_bytes,
                          max_tokens);
    if (rc) return rc;
    if (n_tokens == 0) return GPTOSS_MOE_OK;
    if (!x_norm || !aligned16(x_norm)) return GPTOSS_MOE_ERR_INVALID_ARG;
    const WsLayout L = ws_layout(*shape, max_tokens);
    return launch_route(shape, w, x_norm, n_tokens, forced_topk_i, forced_topk_w,
                        ws_ptrs(L, workspace), stream);
}

int gptoss_moe_forward(const gptoss_moe_shape *shape, const gptoss_moe_weights *w,
                       const uint16_t *x_norm, uint16_t *out, int n_tokens,
                       const int32_t *forced_topk_i, const uint16_t *forced_topk_w,
                       unsigned flags, void *workspace, size_t ws_bytes, int max_tokens,
                       hipStream_t stream) {
    int rc = check_common(shape, w, n_tokens, forced_topk_i, forced_topk_w, workspace, ws_bytes,
                          max_tokens);
    if (rc) return rc;
    if (flags & ~(unsigned)GPTOSS_MOE_FLAG_RESIDUAL_ADD) return GPTOSS_MOE_ERR_INVALID_ARG;
    if (!w->w1 || !w->w1_scales || !w->b1 || !w->w2 || !w->w2_scales || !w->b2)
        return GPTOSS_MOE_ERR_INVALID_ARG;
    if (!aligned16(w->w1) || !aligned16(w->w2)) return GPTOSS_MOE_ERR_INVALID_ARG;
    if (n_tokens == 0) return GPTOSS_MOE_OK;
    if (!x_norm || !out || !aligned16(x_norm) || !aligned16(out)) return GPTOSS_MOE_ERR_INVALID_ARG;
    const WsLayout L = ws_layout(*shape, max_tokens);
    const Ptrs p = ws_ptrs(L, workspace);
    rc = launch_route(shape, w, x_norm, n_tokens, forced_topk_i, forced_topk_w, p, stream);
    if (rc) return rc;
    return launch_experts(shape, w, x_norm, out, n_tokens, flags, L, p, stream);
}

int gptoss_moe_forward_profiled(const gptoss_moe_shape *shape, const gptoss_moe_weights *w,
                                const uint16_t *x_norm, uint16_t *out, int n_tokens,
                                const int32_t *forced_topk_i, const uint16_t *forced_topk_w,
                                unsigned flags, void *workspace, size_t ws_bytes, int max_tokens,
                                hipStream_t stream, float *kernel_ms) {
    int rc = check_common(shape, w, n_tokens, forced_topk_i, forced_topk_w, workspace, ws_bytes,
                          max_tokens);
    if (rc) return rc;
    if (!kernel_ms || n_tokens == 0 || !x_norm || !out) return GPTOSS_MOE_ERR_INVALID_ARG;
    if (flags & ~(unsigned)GPTOSS_MOE_FLAG_RESIDUAL_ADD) return GPTOSS_MOE_ERR_INVALID_ARG;
    Marks mk;
    mk.on = true;
    for (int i = 0; i < 6; ++i)
        if ((rc = hip_status(hipEventCreate(&mk.ev[i]))) != 0) return rc;
    const WsLayout L = ws_layout(*shape, max_tokens);
    const Ptrs p = ws_ptrs(L, workspace);
    mk.mark(stream);
    rc = launch_route(shape, w, x_norm, n_tokens, forced_topk_i, forced_topk_w, p, stream, &mk);
    if (!rc) rc = launch_experts(shape, w, x_norm, out, n_tokens, flags, L, p, stream, &mk);
    if (!rc) rc = hip_status(hipEventSynchronize(mk.ev[5]));
    for (int i = 0; i < 5 && !rc; ++i)
        rc = hip_status(hipEventElapsedTime(&kernel_ms[i], mk.ev[i], mk.ev[i + 1]));
    for (int i = 0; i < 6; ++i) (void)hipEventDestroy(mk.ev[i]);
    return rc;
}

int gptoss_moe_rmsnorm(const uint16_t *x, const uint16_t *weight, uint16_t *out, int n_rows,
                       int size, hipStream_t stream) {
    if (!x || !weight || !out || n_rows < 0 || size <= 0) return GPTOSS_MOE_ERR_INVALID_ARG;
    if (n_rows == 0) return GPTOSS_MOE_OK;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(n_rows), dim3(256), 0, stream, x, weight, out, size);
    return hip_status(hipGetLastError());
}

int gptoss_moe_layer(const gptoss_moe_shape *shape, const gptoss_moe_weights *w,
                     const uint16_t *rms_w, uint16_t *x, uint16_t *t_scratch, int n_tokens,
                     void *workspace, size_t ws_bytes, int max_tokens, hipStream_t stream) {
    if (!rms_w || !x || !t_scratch) return GPTOSS_MOE_ERR_INVALID_ARG;
    int rc = check_common(shape, w, n_tokens, nullptr, nullptr, workspace, ws_bytes, max_tokens);
    if (rc) return rc;
    if (n_tokens == 0) return GPTOSS_MOE_OK;
    rc = gptoss_moe_rmsnorm(x, rms_w, t_scratch, n_tokens, shape->hidden, stream);
    if (rc) return rc;
    return gptoss_moe_forward(shape, w, t_scratch, x, n_tokens, nullptr, nullptr,
                              GPTOSS_MOE_FLAG_RESIDUAL_ADD, workspace, ws_bytes, max_tokens,
                              stream);
}

int gptoss_moe_dequant_mxfp4(const uint8_t *packed, const uint8_t *scales, int n_experts,
                             int64_t n_rows, int64_t k_cols, uint16_t *out, hipStream_t stream) {
    if (!packed || !scales || !out || n_experts < 1 || n_experts > 65535 || n_rows < 0 || k_cols < 0)
        return GPTOSS_MOE_ERR_INVALID_ARG;
    const int64_t seg = n_rows * k_cols;
    if (seg == 0) return GPTOSS_MOE_OK;
    int64_t blocks = (seg / 8 + 255) / 256 + 1;
    if (blocks > 1024) blocks = 1024;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)blocks, n_experts), dim3(256), 0, stream,
                       packed, scales, seg, out);
    return hip_status(hipGetLastError());
}

int gptoss_moe_last_hip_error(void) { return g_last_hip_error; }

const char *gptoss_moe_version(void) { return "gptoss_moe 0.1 gfx950"; }

}  // extern "C"
