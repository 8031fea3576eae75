// bgl_moe.hip -- expert-stacked tensors and the expert-sorted MoE gather.
#include "../../include/beglin_qgemv.h"
#include "bgl_internal.h"

extern "C" int bgl_bind_experts(bgl_ctx *c, int E, const bgl_wt *experts, bgl_tensor **out) {
    (void)c; (void)E; (void)experts; (void)out;
    return bgl_fail(BGL_E_UNSUPPORTED, "bgl_bind_experts: not built yet");
}
extern "C" int bgl_experts_from_tensors(bgl_ctx *c, int E, bgl_tensor *const *experts, bgl_tensor **out) {
    (void)c; (void)E; (void)experts; (void)out;
    return bgl_fail(BGL_E_UNSUPPORTED, "bgl_experts_from_tensors: not built yet");
}
extern "C" int bgl_gather_matvec_dev(bgl_ctx *c, const bgl_tensor *experts, const float *x_dev, const int32_t *idx, int N, float *y) {
    (void)c; (void)experts; (void)x_dev; (void)idx; (void)N; (void)y;
    return bgl_fail(BGL_E_UNSUPPORTED, "bgl_gather_matvec_dev: not built yet");
}
extern "C" int bgl_moe_ffn_dev(bgl_ctx *c, const bgl_tensor *g, const bgl_tensor *u, const bgl_tensor *d, const bgl_tensor *sg,
                               const bgl_tensor *su, const bgl_tensor *sd, const float *x, const int32_t *idx, const float *w,
                               int T, int K, float *out) {
    (void)c; (void)g; (void)u; (void)d; (void)sg; (void)su; (void)sd; (void)x; (void)idx; (void)w; (void)T; (void)K; (void)out;
    return bgl_fail(BGL_E_UNSUPPORTED, "bgl_moe_ffn_dev: not built yet");
}
