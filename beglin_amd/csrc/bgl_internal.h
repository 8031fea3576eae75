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
    int target_blocks = 1024;
    DevBuf act_w, act_s, act_sum;         // activation operands of the current call
    DevBuf tbuf, ctr;                     // split-K partials and arrival counters (counters zeroed)
    DevBuf hx, hy, hb;                    // staging for the host-pointer entry points
    DevBuf moe_a, moe_b, moe_c, moe_d, moe_meta;
    std::mutex mu;
    std::unordered_map<const void *, bgl_tensor *> host_cache;
};

int bgl_fail(int code, const char *fmt, ...);
int dbuf_reserve(bgl_ctx *c, DevBuf &b, size_t bytes, bool zero);
int check_wt(int kind, int bits, int out, int in);
int prep_act(bgl_ctx *c, int act, int gq, const float *x_dev, int M, int K, GemvAct &A);
void plan_task(bgl_ctx *c, const BglDevTensor &T, int total_tiles, int &ks, int &gpb);
int run_gemv(bgl_ctx *c, int n, const BglDevTensor *Ts, int act, const GemvAct &A, int M,
             const float *const *bias, float *const *y, const int *ystride);
