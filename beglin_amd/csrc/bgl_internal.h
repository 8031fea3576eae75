// bgl_internal.h -- host-side context and tensor records behind the opaque C-ABI handles.
#pragma once
#include <hip/hip_runtime.h>

#include <mutex>
#include <unordered_map>
#include <vector>

#include "bgl_kernels.h"

struct DevBuf {
    void *p = nullptr;
    size_t bytes = 0;
};

struct bgl_tensor {
    BglDevTensor T{};                     // single tensor (experts.empty())
    std::vector<void *> owned;            // device allocations owned by this tensor
    size_t device_bytes = 0;
    std::vector<bgl_tensor *> experts;    // E-stacked expert tensor: one bound tensor per expert
    void *dev_table = nullptr;            // device copy of the experts' BglDevTensor records
};

struct bgl_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    int max_waves = 16;                   // wavefronts per GEMV workgroup cap (BGL_MAX_WAVES)
    bool no_fused = false;                // BGL_NO_FUSED_Q=1: W4A8 M=1 through the separate prep kernel
    bool no_mfma = false;                 // BGL_NO_MFMA=1: fp32-activation M >= 16 through the dot4 kernels
    int min_blocks = 256;                 // fused W4A8: split tiles until at least this many workgroups
    float mf_pcap = 1.0f;                 // matrix-core K split: partials (written + read) at most this x the weight bytes
    int force_tr = 0;                     // BGL_FORCE_TR: fixed rows per workgroup (tuning)
    bool no_gemv_x = false;               // BGL_NO_GEMV_X=1: fp32-activation M=1 through the tile kernel (k_gemv)
    int x_waves = 0;                      // BGL_X_WAVES: wavefronts per k_gemv_x workgroup (tuning)
    int q_prep = -1;                      // BGL_Q_PREP: 0 never / 1 always quantize W4A8 columns up front; -1 by M and K
    bool no_moe_x = false;                // BGL_NO_MOE_X=1: MoE gathers through the prep kernel + k_moe_gemv
    int x_fuse = -1;                      // BGL_X_FUSE: 0 never / 1 always make the digits inside k_gemv_x; -1 by K
    int moe_merge = -1;                   // BGL_MOE_MERGE: 0 never / 1 always run the routed and shared gate+up in one launch; -1 by shape
    int moe_cap = 0;                      // BGL_MOE_CAP: 4 / 8 token columns of records per k_moe_x chunk; 0 by LDS fit (tuning)
    DevBuf act_w, act_s, act_sum;         // activation operands of the current call
    int prep_act = -1, prep_gq = 0, prep_M = 0, prep_K = 0;   // what act_* currently hold
    const float *prep_x = nullptr;        // the raw fp32 columns they were made from (non-finite slow path)
    const float *prep_u = nullptr;        // set around run_down_swiglu_w4a8: the prep launch forms h = SwiGLU(x, prep_u)
    float *prep_h = nullptr;              //   into prep_h
    bool prep_reuse = false;              // act_* come from bgl_prep_act_dev (or a host drop-in): bgl_matmul_prepped_dev may use them
    DevBuf prep_xc;                       // bgl_prep_act_dev's own copy of the fp32 columns (prep_x points here)
    DevBuf part;                          // K-split partial sums [ks][M][N]
    DevBuf hx, hy, hb;                    // staging for the host-pointer entry points
    DevBuf moe_a, moe_b, moe_c, moe_d, moe_e, moe_f, moe_g, moe_meta;   // MoE digits x2, fp32 h/down, bucket scratch
    DevBuf moe_route;                     // routing of bgl_moe_layer_dev: idx [T][K] + w [T][K]
    DevBuf moe_scores;                    // router scores [T][E]
    DevBuf mlp;                           // bgl_mlp_dev: gate and up outputs [M][I] each, then h [M][I]
    std::unordered_map<uint64_t, DevBuf> mlp_sync;   // single-launch MLP, per shape (in << 32 | down workgroups): counters, generations, flag
    bool no_qmfma = false;                // BGL_NO_QMFMA=1: W4A8 at 2..16 columns through the dot4 kernel (k_gemv_q)
    int qm_rb = 0, qm_s = 0;              // BGL_QM_RB / BGL_QM_S: k_gemv_qm row blocks / unit slices per workgroup (tuning; 0 by shape)
    int qm_prb = 0, qm_ps = 0;            // BGL_QM_PRB / BGL_QM_PS: the same for its launches over prepared codes
    int mlp_gu = 0;                       // BGL_MLP_GU: gate+up workgroups of the single-launch MLP (tuning; 0 by shape)
    bool no_fused_mlp = false;            // BGL_NO_FUSED_MLP=1: the MLP block as three launches at every M
    int mlp_spin = 1 << 20;               // BGL_MLP_SPIN: polls of the single-launch MLP's bounded wait
    int mlp_delay = -1;                   // BGL_MLP_DELAY: ns the single-launch MLP's down waves wait before loading their weights (tuning; -1 by shape)
    int mlp_waves = 0;                    // BGL_MLP_WAVES: wavefronts per single-launch MLP workgroup (tuning; 0 by shape)
    int mlp_test_timeout = 0;             // BGL_MLP_TEST_TIMEOUT=n: the next n such launches wait for a count never reached (tests of the give-up path)
    std::vector<void *> retired;          // outgrown scratch, kept for captured graphs until destroy / epoch reset
    uint8_t *fixed_base = nullptr;        // set during bgl_matmul_group_noalloc_dev: scratch comes from here
    size_t fixed_cap = 0, fixed_used = 0;
    bool prof = false;                    // bracket launches with events (bgl_prof_enable)
    std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> prof_ev;
    std::vector<hipEvent_t> ev_pool;
    std::mutex mu;
    std::unordered_map<const void *, bgl_tensor *> host_cache;
};

int bgl_fail(int code, const char *fmt, ...);
int bgl_last_code(void);             // the code of this thread's last bgl_fail (BGL_E_NOMEM if none)
// The device layout's version: bump when any format's device bytes change, so caches of the
// repacked layout written before the change are rejected.  (2: signed-nibble g256sf with one
// 8-byte scale word per unit.)
#define BGL_DEVICE_LAYOUT_VERSION 3
void device_layout(int kind, int bits, int out, int in, BglDevTensor &T, size_t bytes[3]);
bgl_tensor *tensor_from_parts(const BglDevTensor &T, void *w, void *s0, void *s1, size_t device_bytes);
// Profiling brackets: prof_begin returns a token (or -1 when profiling is off).
int prof_begin(bgl_ctx *c, int phase);
void prof_end(bgl_ctx *c, int token);
int dbuf_reserve(bgl_ctx *c, DevBuf &b, size_t bytes, bool zero);
// Bytes of per-call scratch the context holds; with release, frees it (the caller synchronizes).
size_t ctx_scratch(bgl_ctx *c, bool release);
int check_wt(int kind, int bits, int out, int in);
int prep_act(bgl_ctx *c, int act, int gq, const float *x_dev, int M, int K, GemvAct &A);
void f32_act_ptrs(const void *xw, const void *xs, const void *xsum, int M, int K, const float *x_dev, GemvAct &A);
int pick_waves(bgl_ctx *c, int nunits);
int run_gemv(bgl_ctx *c, int n, const BglDevTensor *Ts, int act, const GemvAct &A, int M,
             const float *const *bias, float *const *y, const int *ystride);
// Batched fp32-activation GEMM on the matrix cores (bgl_mfma.hip): formats it takes, and the call.
#define BGL_MFMA_MIN_M 16
bool bgl_mfma_ok(int fmt, int bits);
// glu_h (n == 2, a gate/up pair of one shape): the reduce launch also forms h = silu(gate) * up
// into glu_h [M][N] (k_swiglu's arithmetic), so the caller needs no SwiGLU launch.
int run_gemm_mfma(bgl_ctx *c, int n, const BglDevTensor *Ts, const float *x_dev, int M, const float *const *bias,
                  float *const *y, const int *ystride, float *glu_h = nullptr);
// The dense MLP block at one W4A8 column in one launch (bgl_mlp_q.hip): the formats it takes, and the call.
int run_down_swiglu_w4a8(bgl_ctx *c, const BglDevTensor &down, const float *g, const float *u, float *h, int M, float *y);
bool mlp_q_ok(bgl_ctx *c, const BglDevTensor &gate, const BglDevTensor &up, const BglDevTensor &down);
int run_mlp_q(bgl_ctx *c, const BglDevTensor &gate, const BglDevTensor &up, const BglDevTensor &down, const float *x,
              float *h, float *y);
