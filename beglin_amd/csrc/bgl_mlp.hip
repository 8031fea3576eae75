// bgl_mlp.hip -- the dense MLP block of one decode step on the device (forward_token,
// qwen_infer.c:1560-1573): gate and up in one launch over the same activation rows, the SwiGLU
// (swiglu, qwen_infer.c:726-733), then the down projection -- three launches on the context's
// stream, no host copy between them, so the block can be captured in a HIP graph.
//
//   g, u = W_gate x, W_up x      bgl_matmul_group_dev over {gate, up} (one fused launch)
//   h = silu(g) * u              k_swiglu: h = (g / (1 + exp(-g))) * u in fp32, exp rounded once
//                                (several W4A8 columns whose down projection quantizes them up front:
//                                that quantization launch forms h itself, so no k_swiglu launch)
//                                (>= 16 fp32 columns on the matrix cores: the GEMM's reduce launch
//                                forms h with the same arithmetic, from the K-split sums or, for a
//                                tensor whose K did not split, from the g / u the GEMM stored)
//   y = W_down h                 bgl_matmul_dev (W4A8: h quantized to int8 as any activation)
//
// The exponential is evaluated in double and rounded once to float: a correctly rounded expf in
// all but double-rounding cases, so h is a function of g and u alone (the CPU restatement gives
// the same bits), and the W4A8 down projection's int8 codes follow bit for bit.  The division and
// the product round as written (-ffp-contract=off).
#include <math.h>

#include "../../include/beglin_qgemv.h"
#include "bgl_internal.h"

#define HIPCHK(expr)                                                                             \
    do {                                                                                         \
        hipError_t e_ = (expr);                                                                  \
        if (e_ != hipSuccess) return bgl_fail(BGL_E_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

// h[m][i] = silu(g[m][i]) * u[m][i] over n = M * I values; 4 per thread.
__global__ __launch_bounds__(256) void k_swiglu(const float *__restrict__ g, const float *__restrict__ u,
                                                float *__restrict__ h, long n) {
    const long i0 = ((long)blockIdx.x * blockDim.x + threadIdx.x) * 4;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const long i = i0 + j;
        if (i < n) {
            const float gv = g[i];
            const float e = (float)exp(-(double)gv);
            h[i] = (gv / (1.0f + e)) * u[i];
        }
    }
}

extern "C" int bgl_mlp_dev(bgl_ctx *c, const bgl_tensor *gate, const bgl_tensor *up, const bgl_tensor *down, int act,
                           const float *x_dev, float *y_dev, int M, float *h_dev) {
    if (!c || !gate || !up || !down || !x_dev || !y_dev || M < 1) return bgl_fail(BGL_E_ARG, "bgl_mlp_dev: bad argument");
    if (!gate->experts.empty() || !up->experts.empty() || !down->experts.empty())
        return bgl_fail(BGL_E_ARG, "bgl_mlp_dev: dense tensors only (expert stacks go through bgl_moe_ffn_dev)");
    const int H = gate->T.K, I = gate->T.N;
    if (up->T.K != H || up->T.N != I || down->T.K != I || down->T.N != H)
        return bgl_fail(BGL_E_ARG, "bgl_mlp_dev: gate/up [%d x %d], up [%d x %d] and down [%d x %d] do not form an MLP", I, H,
                        up->T.N, up->T.K, down->T.N, down->T.K);
    const size_t n = (size_t)M * I;
    // the scratch belongs to the context's device: select it before any allocation
    HIPCHK(hipSetDevice(c->device));
    // one W4A8 column: the whole block in one launch (bgl_mlp_q.hip)
    if (act == BGL_ACT_W4A8 && M == 1 && !c->no_fused_mlp && !c->no_fused && mlp_q_ok(c, gate->T, up->T, down->T)) {
        float *hq = h_dev;
        if (!hq) {
            if (dbuf_reserve(c, c->mlp, n * 4, false)) return bgl_last_code();
            hq = (float *)c->mlp.p;
        }
        return run_mlp_q(c, gate->T, up->T, down->T, x_dev, hq, y_dev);
    }
    // g and u side by side, then h unless the caller keeps it
    if (dbuf_reserve(c, c->mlp, n * 4 * (h_dev ? 2 : 3), false)) return bgl_last_code();
    float *g = (float *)c->mlp.p, *u = g + n, *h = h_dev ? h_dev : u + n;
    const bgl_tensor *gu[2] = {gate, up};
    const float *nob[2] = {nullptr, nullptr};
    float *ys[2] = {g, u};
    // M >= BGL_MFMA_MIN_M fp32 columns on the matrix cores: the K-split reduce forms h itself
    if (act == BGL_ACT_F32 && M >= BGL_MFMA_MIN_M && !c->no_mfma && gate->T.fmt == up->T.fmt &&
        gate->T.bits == up->T.bits && bgl_mfma_ok(gate->T.fmt, gate->T.bits)) {
        const BglDevTensor Ts[2] = {gate->T, up->T};
        int rc = run_gemm_mfma(c, 2, Ts, x_dev, M, nob, ys, nullptr, h);
        if (rc) return rc;
        return bgl_matmul_dev(c, down, act, h, nullptr, y_dev, M);
    }
    int rc = bgl_matmul_group_dev(c, 2, gu, act, x_dev, nob, ys, M);
    if (rc) return rc;
    // several W4A8 columns whose down projection quantizes them up front: that launch forms h too
    if (act == BGL_ACT_W4A8) {
        rc = run_down_swiglu_w4a8(c, down->T, g, u, h, M, y_dev);
        if (rc <= 0) return rc;
    }
    int tok = prof_begin(c, 2);
    hipLaunchKernelGGL(k_swiglu, dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, c->stream, g, u, h, (long)n);
    prof_end(c, tok);
    HIPCHK(hipGetLastError());
    return bgl_matmul_dev(c, down, act, h, nullptr, y_dev, M);
}
