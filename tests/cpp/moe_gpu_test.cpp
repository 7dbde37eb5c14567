// C++ caller of the C ABI and of the moe_gpu shim, run by
// tests/test_gpu_cpp_shim.py on one small layer.
//
// usage: moe_gpu_test <in.bin> <out.bin>
// in.bin : int32 H, D, E, K, T, then x bf16 [T][H], rms bf16 [H], router_w bf16
//          [E][H], router_b bf16 [E], w1 u8 [E*2D*H/2], s1 u8 [E*2D*H/32], b1 bf16
//          [E][2D], w2 u8 [E*H*D/2], s2 u8 [E*H*D/32], b2 bf16 [E][H], w1 bf16
//          [E][2D][H], w2 bf16 [E][H][D] (the MXFP4 weights dequantised)
// out.bin: bf16 [T][H] each of
//   e_agg  gptoss_moe_forward(x) on a caller workspace
//   x_q    moe_gpu (120B path: MXFP4 fields) on all T rows
//   x_b    moe_gpu (20B path: bf16 fields, re-quantised at init) on all T rows
//   x_o    moe_gpu (120B path) on rows 3 .. T - 1 only (row_offset 3)
#include <hip/hip_bf16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <vector>

#include "gptoss_moe.h"
#include "moe_gpu_shim.hpp"

// The members of the reference's structs the shim reads (getp_run.cpp:46-212,
// run.cpp:25-45), under the reference's names.
typedef struct {
    int hidden_dim, intermediate_dim, n_experts, experts_per_token, n_layers;
    float swiglu_limit;
} Config;
typedef struct {
    __hip_bfloat16 *rms_ffn_w, *w_router, *b_router, *w_mlp1, *w_mlp2, *b_mlp1, *b_mlp2;
    uint8_t *w_mlp1_mxfp4, *w_mlp2_mxfp4, *w_mlp1_scales, *w_mlp2_scales;
} GPUTransformerWeights;
typedef struct {
    __hip_bfloat16 *x, *t;
} GPURunState;
typedef struct {
    Config config;
    GPUTransformerWeights weights;
    GPURunState state;
} GPUTransformer;

#define CK(e)                                                                     \
    do {                                                                          \
        hipError_t err_ = (e);                                                    \
        if (err_ != hipSuccess) {                                                 \
            fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(err_)); \
            return 2;                                                             \
        }                                                                         \
    } while (0)

template <class T>
static T *upload(FILE *f, size_t n) {
    std::vector<T> h(n);
    if (fread(h.data(), sizeof(T), n, f) != n) {
        fprintf(stderr, "short input\n");
        exit(2);
    }
    T *d = nullptr;
    if (hipMalloc(&d, n * sizeof(T) + 256) != hipSuccess ||
        hipMemcpy(d, h.data(), n * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) {
        fprintf(stderr, "upload failed\n");
        exit(2);
    }
    return d;
}

int main(int argc, char **argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: %s in.bin out.bin\n", argv[0]);
        return 2;
    }
    FILE *f = fopen(argv[1], "rb");
    if (!f) return 2;
    int32_t hd[5];
    if (fread(hd, 4, 5, f) != 5) return 2;
    const int H = hd[0], D = hd[1], E = hd[2], K = hd[3], T = hd[4];
    const size_t n1 = (size_t)E * 2 * D * H, n2 = (size_t)E * H * D;
    uint16_t *x0 = upload<uint16_t>(f, (size_t)T * H);
    uint16_t *rms = upload<uint16_t>(f, H);
    uint16_t *rw = upload<uint16_t>(f, (size_t)E * H);
    uint16_t *rb = upload<uint16_t>(f, E);
    uint8_t *w1 = upload<uint8_t>(f, n1 / 2);
    uint8_t *s1 = upload<uint8_t>(f, n1 / 32);
    uint16_t *b1 = upload<uint16_t>(f, (size_t)E * 2 * D);
    uint8_t *w2 = upload<uint8_t>(f, n2 / 2);
    uint8_t *s2 = upload<uint8_t>(f, n2 / 32);
    uint16_t *b2 = upload<uint16_t>(f, (size_t)E * H);
    uint16_t *w1b = upload<uint16_t>(f, n1);
    uint16_t *w2b = upload<uint16_t>(f, n2);
    fclose(f);

    hipStream_t st;
    CK(hipStreamCreate(&st));
    const size_t xb = (size_t)T * H * 2;
    std::vector<uint16_t> out(4 * (size_t)T * H, 0);

    // (1) gptoss_moe_forward on a caller workspace, with a packed copy
    {
        gptoss_moe_shape shape{H, D, E, K, 7.0f, 1.702f};
        gptoss_moe_weights w{rw, rb, w1, s1, b1, w2, s2, b2, nullptr, nullptr};
        const size_t pbytes = gptoss_moe_packed_size(&shape);
        uint8_t *packed = nullptr;
        CK(hipMalloc(&packed, pbytes));
        if (gptoss_moe_pack_weights(&shape, &w, packed, pbytes, st) != GPTOSS_MOE_OK) return 3;
        w.packed = packed;
        const size_t ws_bytes = gptoss_moe_workspace_size(&shape, T);
        void *ws = nullptr;
        CK(hipMalloc(&ws, ws_bytes));
        if (gptoss_moe_workspace_init(ws, ws_bytes, st) != GPTOSS_MOE_OK) return 3;
        uint16_t *e = nullptr;
        CK(hipMalloc(&e, xb));
        const int rc = gptoss_moe_forward(&shape, &w, x0, e, T, nullptr, nullptr, 0, ws, ws_bytes, T, st);
        if (rc != GPTOSS_MOE_OK) {
            fprintf(stderr, "gptoss_moe_forward: %d\n", rc);
            return 3;
        }
        CK(hipMemcpyAsync(out.data(), e, xb, hipMemcpyDeviceToHost, st));
        CK(hipStreamSynchronize(st));
    }

    // (2)-(4) the moe_gpu shim on a one-layer transformer
    GPUTransformer gt{};
    gt.config = Config{H, D, E, K, 1, 7.0f};
    auto bf = [](void *p) { return reinterpret_cast<__hip_bfloat16 *>(p); };
    gt.weights.rms_ffn_w = bf(rms);
    gt.weights.w_router = bf(rw);
    gt.weights.b_router = bf(rb);
    gt.weights.b_mlp1 = bf(b1);
    gt.weights.b_mlp2 = bf(b2);
    gt.weights.w_mlp1 = bf(w1b);
    gt.weights.w_mlp2 = bf(w2b);
    gt.weights.w_mlp1_mxfp4 = w1;
    gt.weights.w_mlp1_scales = s1;
    gt.weights.w_mlp2_mxfp4 = w2;
    gt.weights.w_mlp2_scales = s2;
    uint16_t *x = nullptr, *t = nullptr;
    CK(hipMalloc(&x, xb));
    CK(hipMalloc(&t, xb));
    gt.state.x = bf(x);
    gt.state.t = bf(t);
    struct Run {
        bool mxfp4;
        int row_offset;
        size_t slot;
    } runs[3] = {{true, 0, 1}, {false, 0, 2}, {true, 3, 3}};
    for (const Run &r : runs) {
        if (r.row_offset >= T) continue;
        gptoss_moe_shim::moe_gpu_init(&gt, T, r.mxfp4, st);
        CK(hipMemcpyAsync(x, x0, xb, hipMemcpyDeviceToDevice, st));
        moe_gpu(&gt, 0, T - r.row_offset, r.row_offset, st);
        CK(hipMemcpyAsync(out.data() + r.slot * T * H, x, xb, hipMemcpyDeviceToHost, st));
        CK(hipStreamSynchronize(st));
    }
    FILE *o = fopen(argv[2], "wb");
    if (!o || fwrite(out.data(), 2, out.size(), o) != out.size()) return 2;
    fclose(o);
    printf("moe_gpu_test ok H=%d D=%d E=%d K=%d T=%d\n", H, D, E, K, T);
    return 0;
}
