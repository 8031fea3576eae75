/* beglin_qgemv.h -- C-ABI of the MI355X (gfx950) quantized GEMV / MoE-gather backend.
 *
 * Plain C: pointers, sizes and ints only.  Implemented by beglin_amd/libbeglin_hip.so (HIP).
 * Each entry point names the reference interface it replaces (paths relative to the reference
 * repository root).  Conventions:
 *   - return 0 on success, a negative BGL_E_* code on failure (bgl_last_error() has the text).
 *     The reference's GEMV entries FATAL+exit(1) on misuse (q4gemv.h:675, :704, :783;
 *     q4gemv_g256.h:342-343); an engine-side shim that turns a non-zero return into that same
 *     FATAL keeps the behaviour at the engine boundary unchanged.  The bgl_gpu_* (MLX boundary)
 *     functions below keep MLX's convention instead: 1 = ok, 0 = failure.
 *   - weights: "kind" ids 1..4 are the engine's WT kinds (qwen_infer.c:207): 1 K_Q4G64, 2 K_Q8G64,
 *     3 K_Q4G256SF, 4 K_QNG64; 5 is BGL_K_Q4G32H (int4 group-32, fp16 scale, q4gemv nibble pairing).
 *     6..8 are the AF expert kinds the MoE boundary binds (mlx_gpu_bind_af bits=4/16/32,
 *     mlx_moe.cpp:146-367): 6 BGL_K_Q4G64A int4 affine (nib*s + b, group 64), 7 BGL_K_F16 and
 *     8 BGL_K_F32 dense rows.  9 BGL_K_MXFP4 is the AF kind bits = MOE_BITS_GGUF_MXFP4 (40) of the CPU
 *     MoE path (moe_decode_af / moe_matvec_af_row, qwen_infer.c:2584-2595, :2702-2725): GGUF MXFP4
 *     blocks of 32, an E8M0 exponent byte then 16 bytes of E2M1 nibbles (gguf_quants.c:284-327).
 *     Kinds 6..9 run in the MoE gather only (fp32 activations).  10 BGL_K_Q4G256P is the plain-g256
 *     diagnostic of q4gemv_g256.h:102-130 (q4 nibbles, one fp32 scale per 256 values, W4A8 only).
 *   - *_dev entry points take DEVICE pointers and are asynchronous on the context's stream;
 *     host-pointer entry points (the drop-ins with the reference's exact argument lists) copy
 *     x in and y out and return after y is on the host.
 *   - one context = one HIP stream; calls on one context are serialised by that stream.  Two
 *     threads must not use the same context concurrently (the q4pool contract, q4gemv.h:721).
 *   - graph capture: the *_dev calls may be captured from the context's stream once the same
 *     call has run outside a capture at the same or larger sizes (that sizes the context's
 *     per-call scratch).  A captured call that would need more scratch returns BGL_E_CAPTURE and
 *     enqueues nothing.  Scratch a graph uses stays allocated until bgl_ctx_destroy or
 *     bgl_gpu_reset_runtime_epoch (after which graphs must be captured again), even when a
 *     later, larger call outgrows it.
 */
#ifndef BEGLIN_QGEMV_H
#define BEGLIN_QGEMV_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { BGL_K_Q4G64 = 1, BGL_K_Q8G64 = 2, BGL_K_Q4G256SF = 3, BGL_K_QNG64 = 4, BGL_K_Q4G32H = 5,
       BGL_K_Q4G64A = 6, BGL_K_F16 = 7, BGL_K_F32 = 8, BGL_K_MXFP4 = 9, BGL_K_Q4G256P = 10 };
enum { BGL_ACT_F32 = 0, BGL_ACT_W4A8 = 1 };
enum { BGL_OK = 0, BGL_E_ARG = -1, BGL_E_UNSUPPORTED = -2, BGL_E_HIP = -3, BGL_E_NODEV = -4, BGL_E_NOMEM = -5,
       BGL_E_CAPTURE = -6 /* per-call scratch would have to grow inside a stream capture */,
       BGL_E_TIMEOUT = -7 /* a bounded wait inside a kernel gave up (bgl_ctx_check) */ };

typedef struct bgl_ctx bgl_ctx;
typedef struct bgl_tensor bgl_tensor;

/* Weight descriptor: the fields of the engine's WT (qwen_infer.c:208-222).
 *   packed: K_Q4G64/K_Q4G256SF/Q4G32H/Q4G64A nibbles [out][in/2] (low nibble = even column; the
 *           AF int4 u32 words [out][in/8] are the same bytes, mlx_moe.cpp:238-257);
 *           K_Q8G64 int8 codes [out][in]; K_QNG64 bit planes [out][in/64][n][8];
 *           F16 / F32: dense fp16 / fp32 rows [out][in]; MXFP4: the GGUF blocks [out][in/32][17].
 *   scales: fp32 [out][in/64] (K_Q4G64, K_Q8G64, K_QNG64, Q4G64A); fp32 wsuper [out][in/256]
 *           (K_Q4G256SF; the plain scale for Q4G256P); fp16 bits [out][in/32] (Q4G32H); unused (may be NULL) for F16 / F32 / MXFP4.
 *   sub:    K_Q4G256SF: sub-codes u8 [out][in/64]; Q4G64A: fp32 biases [out][in/64] (read as bytes).
 *   bits:   K_QNG64 only: n in 2..15. */
typedef struct {
    int kind, bits, out, in;
    const void *packed;
    const void *scales;
    const uint8_t *sub;
} bgl_wt;

/* ---------------- runtime (mlx_moe.h:24-36 analogues) ---------------- */
int  bgl_available(void);                                   /* mlx_gpu_available (mlx_moe.h:24) */
const char *bgl_last_error(void);
int  bgl_ctx_create(int device, void *hip_stream, bgl_ctx **out);   /* q4pool_init+start (q4gemv.h:580-620); stream NULL = own stream */
void bgl_ctx_destroy(bgl_ctx *ctx);                         /* q4pool_destroy (q4gemv.h:623-637) */
int  bgl_synchronize(bgl_ctx *ctx);                         /* mlx_gpu_synchronize (mlx_moe.h:29) */
/* Synchronize the context's stream, then report (and clear) a bounded in-kernel wait that gave up
 * since the last check: BGL_E_TIMEOUT means the outputs of that call are invalid.  No counterpart in
 * the reference (its CPU kernels never wait on each other); the single-launch MLP block of
 * bgl_mlp_dev is the call that waits. */
int  bgl_ctx_check(bgl_ctx *ctx);
void *bgl_ctx_stream(bgl_ctx *ctx);                          /* the hipStream_t work is queued on */

/* ---------------- profiling (the QWEN_PROF phase buckets, qwen_infer.c:1231, :1851-1895) ----------------
 * While enabled, every kernel the context launches is bracketed by HIP events on its stream.
 * bgl_prof_read synchronises and reports, per phase (0 = activation prep, 1 = GEMV/gather, 2 = other),
 * the summed kernel time in ms and the launch count, then clears the records. */
int  bgl_prof_enable(bgl_ctx *ctx, int on);
int  bgl_prof_read(bgl_ctx *ctx, double *ms_by_phase, int *launches_by_phase, int nphase);

/* ---------------- weight binding: upload + repack into the tiled device layout ----------------
 * mlx_gpu_bind_af (mlx_moe.h:48-50) / kai_repack_one_lazy (qwen_infer.c:473-487).  Host buffers
 * are read once; the device copy is owned by the returned tensor. */
int  bgl_bind(bgl_ctx *ctx, const bgl_wt *w, bgl_tensor **out);
/* Mixed per-cell qNg64 (MixedQNg64Tensor, mlx_moe.cpp:87-93): one width n = bits[cell] (2..15) per
 * (row, 64-group) cell, n bit-planes of 8 bytes at planes + offsets[cell] (the qng64_dense.c plane
 * layout), value (u - 2^(n-1)) * scales[cell].  offsets has out*in/64 + 1 entries; the checks of
 * mlx_moe.cpp:1750-1758 apply.  The cells are re-biased to the tensor's widest n on the device, so
 * the result is a K_QNG64 tensor of that width with bit-identical values. */
int  bgl_bind_qng64_mixed(bgl_ctx *ctx, const uint8_t *planes, long planes_bytes, const uint32_t *offsets,
                          const uint8_t *bits, const float *scales, int out, int in, bgl_tensor **res);
/* Quantize fp32 weights already on the device with the reference packer of `kind`, straight into
 * the device layout (load-time transcode: gguf_quantize_q4g64_error_feedback / gguf_quantize_q8g64 /
 * gguf_quantize_qNg64 (gguf_transcode.c:24-162), qng64_quantize_f32 (qng64_dense.c:29-68,
 * qng64_encoder=1), gguf_w_quantize_q4_0 re-paired (gguf_write_quants.c:34-62), g256sf build packer).
 * If ref_packed/ref_scales/ref_sub are non-NULL the reference-layout bytes are copied back there
 * (host pointers) for byte-exact checks or caching. */
int  bgl_quantize_dev(bgl_ctx *ctx, int kind, int bits, int qng64_encoder, const float *w_dev, int out, int in,
                      bgl_tensor **t, void *ref_packed, void *ref_scales, uint8_t *ref_sub);
void bgl_tensor_free(bgl_tensor *t);
int  bgl_tensor_info(const bgl_tensor *t, int *kind, int *bits, int *out, int *in, size_t *device_bytes);
/* mlx_gpu_dequant_probe (mlx_moe.h:78-79): decode rows [row0,row0+nrows) from the device layout. */
int  bgl_dequant_dev(bgl_ctx *ctx, const bgl_tensor *t, int row0, int nrows, float *out_dev);

/* ---------------- GEMV / small-M GEMM on device pointers ----------------
 * y[m][r] = bias[r] + sum_c W[r][c] x[m][c], m < M.
 *   act = BGL_ACT_F32: fp32 activations (gemv_q4g64_mt / gemv_q8g64_mt / gemm_qXg64_mt,
 *         q4gemv.h:672-769; qng64_matvec_f32 / qng64_matmul_f32, qng64_dense.c:70-100).
 *   act = BGL_ACT_W4A8: the reference's dynamic int8 activations (gemv_q4g64_sdot_mt,
 *         gemv_q8g64_sdot_mt, gemm_qXg64_sdot_mt, q4gemv.h:701-791; gemv/gemm_q4g256sf_sdot_mt,
 *         q4gemv_g256.h:339-383).  K_Q4G256SF accepts only this mode (qwen_infer.c:697-702).
 * This is the matvec_t / matmul_t / matmul_sdot backend switch (qwen_infer.c:687-708,
 * :1608-1655, :1852-1900) with the format taken from the bound tensor. */
int  bgl_matmul_dev(bgl_ctx *ctx, const bgl_tensor *w, int act, const float *x_dev, const float *bias_dev,
                    float *y_dev, int M);
/* Several tensors that share one activation (fused q/k/v or gate+up, QWEN_FUSED_DISPATCH,
 * qwen_infer.c:1276-1306) in ONE launch.  All must have the same `in` and kind; n <= 4. */
int  bgl_matmul_group_dev(bgl_ctx *ctx, int n, const bgl_tensor *const *w, int act, const float *x_dev,
                          const float *const *bias_dev, float *const *y_dev, int M);
/* The dense MLP block of forward_token (qwen_infer.c:1560-1573) on the device: g = W_gate x and
 * u = W_up x in one fused launch, h = silu(g) * u (swiglu, qwen_infer.c:726-733: g / (1 + exp(-g)),
 * then * u, in fp32; the exponential rounded once from double), y = W_down h.  gate / up [I][H],
 * down [H][I], x_dev [M][H], y_dev [M][H]; act as bgl_matmul_dev (W4A8 quantizes x and h).  h_dev:
 * optional [M][I] that receives h (NULL: it stays in the context's scratch).  No host round trip;
 * capturable under the same scratch rule as the other *_dev calls.  One W4A8 column in q4g64,
 * q8g64 or g256sf (plain g256 included) runs the whole block as ONE launch whose down-projection
 * workgroups wait, bounded, for the gate+up workgroups (bgl_ctx_check reports a wait that gave up);
 * the values are the three-launch path's, bit for bit.  Calls on one context run in its stream's
 * order; two streams running this context's MLP calls at once would share its counters. */
int  bgl_mlp_dev(bgl_ctx *ctx, const bgl_tensor *gate, const bgl_tensor *up, const bgl_tensor *down, int act,
                 const float *x_dev, float *y_dev, int M, float *h_dev);
/* bgl_matmul_group_dev that allocates nothing: no counterpart in the reference.  For callers that
 * cannot allocate device memory -- code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc.  The same kernels and results as bgl_matmul_group_dev; the per-call
 * scratch (activation digits / codes, K-split partials) comes from a fixed per-GPU device array of
 * BGL_NOALLOC_SCRATCH_BYTES, held until the process ends.  A call that needs more returns
 * BGL_E_NOMEM (e.g. fp32 activations: about 116 KB per column at K = 16384).  The array is shared
 * by every call on the GPU: calls that overlap on one GPU (two contexts or streams) race. */
#define BGL_NOALLOC_SCRATCH_BYTES (32u << 20)
int  bgl_matmul_group_noalloc_dev(bgl_ctx *ctx, int n, const bgl_tensor *const *w, int act, const float *x_dev,
                                  const float *const *bias_dev, float *const *y_dev, int M);
/* Streaming read of up to 64 bound tensors' device bytes (packed chunks, scales, biases) on the
 * context's stream, in one launch: no counterpart in the reference -- a measurement aid that gives
 * the plain-read floor for exactly the bytes a GEMV call or a MoE gather launch streams.  The
 * tensors are single (not expert stacks).  nblocks / nthreads <= 0: 1024 x 256. */
int  bgl_read_probe_dev(bgl_ctx *ctx, int n, const bgl_tensor *const *w, int nblocks, int nthreads);
/* Prepare activation operands once and reuse them for several GEMVs with the same input (the
 * caller-side quantization of matmul_sdot, qwen_infer.c:1870-1889, feeding gemm_qXg64_sdot_mt's
 * xq/ascale arguments, q4gemv.h:779-791).  `kind` selects the activation grouping (g256sf: 256).
 * The prepared operands live in the context until the next prep or GEMV call that prepares. */
int  bgl_prep_act_dev(bgl_ctx *ctx, int act, int kind, const float *x_dev, int M, int in);
int  bgl_matmul_prepped_dev(bgl_ctx *ctx, const bgl_tensor *w, int act, const float *bias_dev, float *y_dev, int M);
/* W4A8 activation quantizer on device (q4_quant_act_i8, q4gemv.h:177-213; _g256,
 * q4gemv_g256.h:72-99): xq [M][in] int8, ascale [M][in/gsize]. */
int  bgl_quant_act_i8_dev(bgl_ctx *ctx, const float *x_dev, int M, int in, int gsize, int8_t *xq_dev, float *ascale_dev);

/* ---------------- host-pointer drop-ins with the reference's argument lists ----------------
 * The q4pool* argument becomes the context.  The weight pointer identifies the tensor: the first
 * call binds it (lazy repack), later calls reuse the device copy (keyed by the packed pointer).
 * Synchronous: y is valid on return. */
int bgl_gemv_q4g64_mt(bgl_ctx *p, const uint8_t *packed, const float *scales, const float *x,
                      const float *bias, float *y, int out, int in);                     /* q4gemv.h:672 */
int bgl_gemv_q4g64_mt_fused(bgl_ctx *p, const uint8_t *packed, const float *scales, const float *x,
                            const float *bias, float *y, int out, int in);               /* q4gemv.h:686 (same values as :672) */
int bgl_gemv_q4g64_sdot_mt(bgl_ctx *p, const uint8_t *packed, const float *scales, const float *x,
                           const float *bias, float *y, int out, int in);                /* q4gemv.h:701 */
int bgl_gemv_q8g64_mt(bgl_ctx *p, const uint8_t *packed, const float *scales, const float *x,
                      const float *bias, float *y, int out, int in);                     /* q4gemv.h:748 */
int bgl_gemv_q8g64_sdot_mt(bgl_ctx *p, const uint8_t *packed, const float *scales, const float *x,
                           const float *bias, float *y, int out, int in);                /* q4gemv.h:726 */
int bgl_gemm_qXg64_mt(bgl_ctx *p, int bits, const uint8_t *packed, const float *scales, const float *x,
                      const float *bias, float *y, int out, int in, int M);              /* q4gemv.h:761 */
/* Caller-quantized int8 columns (matmul_sdot's serve path, qwen_infer.c:1870-1898): xq [M][in] as
 * q4_quant_act_i8 produced it -- for bits=4 in q4_split_act's split order ([even16][odd16] per 32
 * bytes, q4gemv.h:298-312), for bits=8 in natural order -- and ascale [M][in/64]. */
int bgl_gemm_qXg64_sdot_mt(bgl_ctx *p, int bits, const uint8_t *packed, const float *scales, const int8_t *xq,
                           const float *ascale, const float *bias, float *y, int out, int in, int M);   /* q4gemv.h:779 */
/* g256sf with caller-quantized columns: xq split order, ascale [M][in/256] (q4gemv_g256.h:366-383). */
int bgl_gemm_q4g256sf_sdot_mt(bgl_ctx *p, const uint8_t *packed, const float *wsuper, const uint8_t *subcode,
                              const int8_t *xq, const float *ascale, const float *bias, float *y, int out, int in,
                              int M);                                                    /* q4gemv_g256.h:368 */
int bgl_gemv_q4g256sf_sdot_mt(bgl_ctx *p, const uint8_t *packed, const float *wsuper, const uint8_t *subcode,
                              const float *x, const float *bias, float *y, int out, int in);   /* q4gemv_g256.h:339 */
int bgl_gemm_q4g256sf_mt(bgl_ctx *p, const uint8_t *packed, const float *wsuper, const uint8_t *subcode,
                         const float *x, const float *bias, float *y, int out, int in, int M); /* matmul_sdot g256sf arm, qwen_infer.c:1880-1898 */
int bgl_qng64_matvec_f32(bgl_ctx *p, const uint8_t *packed, const float *scales, int n, const float *x,
                         const float *bias, float *y, int out, int in);                  /* qng64_dense.c:81 */
int bgl_qng64_matmul_f32(bgl_ctx *p, const uint8_t *packed, const float *scales, int n, const float *x,
                         const float *bias, float *y, int out, int in, int M);           /* qng64_dense.c:70 */
int bgl_gemv_q4g32h_mt(bgl_ctx *p, const uint8_t *packed, const uint16_t *scales16, const float *x,
                       const float *bias, float *y, int out, int in);                    /* no reference kernel: Q4_0 values (gguf_quants.c:118-130) */
/* Drop the cached device copy bound to `packed` (rebind after the caller changes the bytes). */
int bgl_forget(bgl_ctx *p, const void *packed);

/* ---------------- int4-mode loader and the repacked-layout cache ----------------
 * load_int4 (qwen_infer.c:554-615): the layout manifest, one line "name kind doff out in ng soff
 * [soff2]" per tensor over the weight blob; kinds q4g64, q8g64, q4g256sf (8th field: sub-code offset)
 * and f32.  Every check of the reference loader applies (ng and in divisibility, 64-byte alignment of
 * the int4 offsets, extents inside the blob, unknown kinds, duplicate names, at most 512 tensors);
 * a failed check loads nothing.  Quantized tensors are bound on the device (the model owns them:
 * do not free what bgl_model_find returns); f32 tensors stay in the read-only mapped blob.
 * bgl_int4_layout_check runs the parse and the checks only (no device work). */
typedef struct bgl_model bgl_model;
int bgl_int4_layout_check(const char *layout_path, const char *blob_path, int *n_tensors);
int bgl_model_load_int4(bgl_ctx *ctx, const char *layout_path, const char *blob_path, bgl_model **out);
int bgl_model_count(const bgl_model *m);
/* kind: BGL_K_* of a bound tensor (then *t is set) or 0 for f32 (then *f32 points into the blob). */
int bgl_model_find(const bgl_model *m, const char *name, int *kind, int *out, int *in, bgl_tensor **t, const float **f32);
int bgl_model_free(bgl_model *m);
/* The repacked device layout on disk (the .beglin cache pattern, gguf_cache.c): valid only for the
 * same blob and manifest (size and mtime), device architecture and device-layout version; opened
 * without following symlinks; a directory pointing outside the file is an error. */
int bgl_model_save_cache(const bgl_model *m, const char *cache_path, const char *layout_path, const char *blob_path);
int bgl_model_cache_valid(const char *cache_path, const char *layout_path, const char *blob_path);   /* 1 / 0 */
int bgl_model_load_cache(bgl_ctx *ctx, const char *cache_path, const char *layout_path, const char *blob_path,
                         bgl_model **out);

/* ---------------- MoE: expert-sorted gather ----------------
 * An E-stacked expert tensor (MoeAFTensor, qwen_infer.c:2358-2444; per-expert widths like
 * st_register_moe_experts_mixed_as, :16439-16564): E descriptors, each expert with its own kind.
 * All experts share out/in. */
int bgl_bind_experts(bgl_ctx *ctx, int E, const bgl_wt *experts, bgl_tensor **out);
int bgl_experts_from_tensors(bgl_ctx *ctx, int E, bgl_tensor *const *experts, bgl_tensor **out);  /* takes ownership */
/* Explicit pairs: y[z] = W[expert_idx[z]] x[z] for z < N (mlx_gpu_qng64_gather_probe, mlx_moe.h:89-91;
 * ffn_gather canonical form, mlx_moe.cpp:1577-1589, :1901-1916).  Pairs are sorted by expert on
 * the device so each expert's weights stream once per call.  fp32 activations. */
int bgl_gather_matvec_dev(bgl_ctx *ctx, const bgl_tensor *experts, const float *x_dev, const int32_t *expert_idx_dev,
                          int N, float *y_dev);
/* Routed SwiGLU FFN for T tokens with top-K routing given (moe_ffn_batched, qwen_infer.c:5238-5350):
 * out[t] = sum_k w[t][k] * down_e(silu(gate_e x_t) * up_e x_t) + shared(x_t), e = idx[t][k];
 * the weighted sum runs in ascending expert order per token like the reference's bucket loop.
 * shared_* may be NULL (no shared experts). x_dev [T][in], idx/w [T][K] on device, out [T][in]. */
int bgl_moe_ffn_dev(bgl_ctx *ctx, const bgl_tensor *gate, const bgl_tensor *up, const bgl_tensor *down,
                    const bgl_tensor *shared_gate, const bgl_tensor *shared_up, const bgl_tensor *shared_down,
                    const float *x_dev, const int32_t *topk_idx_dev, const float *topk_w_dev, int T, int K,
                    float *out_dev);
/* Router of the routed FFN (moe_ffn_batched's routing, qwen_infer.c:5243-5257, :5275): per token,
 * scores = W_r x (+ b) accumulated in double (moe_matvec_f32, :3460-3466), softmax
 * (moe_softmax_full, :3467-3472), top-K by repeated strict maximum with ties to the lowest expert id
 * (moe_top_k_select, :3514-3521), and with renorm != 0 the K weights divided by their sum
 * (moe_topk_renorm, :3529-3534; MOE_NORM_TOPK_PROB).  router_w_dev fp32 [E][in] (16-byte aligned,
 * in % 4 == 0), router_b_dev [E] or NULL, x_dev [T][in]; writes topk_idx_dev / topk_w_dev [T][K].
 * E <= 256, K <= min(E, 16). */
int bgl_moe_route_dev(bgl_ctx *ctx, const float *router_w_dev, const float *router_b_dev, int E, int in,
                      const float *x_dev, int T, int K, int renorm, int32_t *topk_idx_dev, float *topk_w_dev);
/* The whole routed FFN step on the device (moe_ffn_batched, qwen_infer.c:5238-5350): bgl_moe_route_dev
 * then bgl_moe_ffn_dev, with the routing kept in the context's scratch.  E = the experts in gate. */
int bgl_moe_layer_dev(bgl_ctx *ctx, const float *router_w_dev, const float *router_b_dev, int renorm,
                      const bgl_tensor *gate, const bgl_tensor *up, const bgl_tensor *down,
                      const bgl_tensor *shared_gate, const bgl_tensor *shared_up, const bgl_tensor *shared_down,
                      const float *x_dev, int T, int K, float *out_dev);

/* ---------------- name-keyed MoE registry: the mlx_moe.h GPU boundary ----------------
 * One process-wide registry on device 0 (own stream, like MLX's default stream).  Each function
 * has the argument list and the return convention of the mlx_gpu_* function it replaces:
 * 1 = ok, 0 = failure (bgl_last_error() says why), unless stated otherwise.  Weights are COPIED
 * into the device layout at bind (the reference wraps the blob zero-copy); the blob may be
 * released after bgl_gpu_bind_af returns. */
int bgl_gpu_available(void);                                           /* mlx_moe.h:24 */
int bgl_gpu_synchronize(void);                                         /* mlx_moe.h:29 */
/* Synchronizes and releases per-call scratch; bindings stay (mlx_moe.h:36, mlx_moe.cpp:3167-3200). */
int bgl_gpu_reset_runtime_epoch(void);
/* E experts [out][in], groups of 64 (ng = in/64), read from blob at the byte offsets.  bits:
 * 4 int4 affine (scale_off, bias_off), 8 q8g64 (no bias), 2/3/5/6/7/9..15 qNg64 planes,
 * 16 / 32 dense fp16 / fp32 (no scales); n=8 planes and other widths are refused (mlx_moe.cpp:
 * 146-367).  Rebinding a name replaces it. */
int bgl_gpu_bind_af(const uint8_t *blob, long blob_bytes, const char *name, long E, long out, long in, long ng,
                    long packed_off, long scale_off, long bias_off, int bits);           /* mlx_moe.h:48-50 */
/* The AF layout manifest over an AF blob (moe_load_layout_af, qwen_infer.c:2496-2515): one record per
 * tensor, "name E out in ng packed_off packed_bytes scale_off bias_off", whitespace-separated; every
 * tensor is E experts of [out][in] int4 affine weights (bits = 4: nib * scale + bias, groups of 64).
 * Each record is checked (in % 64 == 0 and ng == in/64; packed_bytes at least the E*out*in/2 code
 * bytes; codes, scales [E][out][ng] and biases inside the blob; no duplicate names; at most 1024
 * records; names under 128 characters) before anything is bound, then every tensor is bound by name
 * through bgl_gpu_bind_af.  A record cut short ends the manifest, as the reference's fscanf loop
 * ends.  Returns the number of tensors bound, or -1 (bgl_last_error() says why; on a device failure
 * the tensors before it stay bound).  The reference exits where this returns -1. */
int bgl_gpu_load_layout_af(const char *layout_path, const uint8_t *blob, long blob_bytes);
/* The same parse and checks with no device work: 0 and the record count, or a BGL_E_* code. */
int bgl_af_layout_check(const char *layout_path, long blob_bytes, int *n_tensors);
/* 0 missing, 1 quantized (bits 2..6, 8), 2 dense (16/32), 3 qNg64 planes n=7, 9..15 (mlx_moe.h:57). */
int bgl_gpu_binding_kind(const char *name, int *bits_out);
int bgl_gpu_snapshot_binding(const char *name, uint64_t *snapshot_id);  /* mlx_moe.h:63 */
int bgl_gpu_restore_binding_snapshot(uint64_t snapshot_id);           /* mlx_moe.h:64 */
int bgl_gpu_drop_binding_snapshot(uint64_t snapshot_id);              /* mlx_moe.h:65 */
int bgl_gpu_binding_snapshot_count(void);                             /* mlx_moe.h:66: returns the count */
/* Every binding is an explicit copy: zero_copy = 0, copied = bytes_copied's tensor count; returns
 * the number of binds performed (mlx_moe.h:72). */
int bgl_gpu_zerocopy_count(int *zero_copy, int *copied, size_t *bytes_copied);
/* Decoded weights of expert e, row `row`, columns [col0, col0+ncols) read back from the device
 * layout (mlx_moe.h:78-79). */
int bgl_gpu_dequant_probe(const char *name, long e, long row, long col0, int ncols, float *out);
/* Explicit-pair gather with raw host buffers (mlx_moe.h:89-91): planes [E][out][ng*n*8],
 * scales [E][out][ng], x [N][in], expert_idx [N], out_buf [N][out]. */
int bgl_gpu_qng64_gather_probe(const uint8_t *planes, long E, long out, long in, long ng, int n, const float *scales,
                               const float *x, int N, const int32_t *expert_idx, float *out_buf);
/* Bind one caller-owned qNg64 tensor (n in {2,3,5,6}) as a single-expert binding (mlx_moe.h:97-98). */
int bgl_gpu_bind_qng64_dense_probe(const uint8_t *packed, const float *scales, const char *name, long out, long in, int n);
/* Mixed per-cell qNg64 probes (mlx_moe.h:104-116): the one-shot GEMV out_buf [batch][out] = W x for
 * x [batch][in] (registry untouched), and the binder (kind 4, bits 0 in bgl_gpu_binding_kind; served by
 * bgl_gpu_matvec_probe with e = 0; bgl_gpu_dequant_probe refuses it, as the reference's does). */
int bgl_gpu_qng64_mixed_dense_probe(const uint8_t *planes, long planes_bytes, const uint32_t *offsets, const uint8_t *bits,
                                    const float *scales, long out, long in, const float *x, int batch, float *out_buf);
int bgl_gpu_bind_qng64_mixed_dense_probe(const uint8_t *planes, long planes_bytes, const uint32_t *offsets,
                                         const uint8_t *bits, const float *scales, const char *name, long out, long in);
/* y[out] = W_e x for one expert of a bound tensor, host x / y (mlx_moe.h:121). */
int bgl_gpu_matvec_probe(const char *name, long e, const float *x, float *y);
/* Device bytes held by bindings (active), the high-water mark (peak) and per-call scratch (cache). */
void bgl_gpu_report_memory(size_t *active, size_t *peak, size_t *cache);    /* mlx_moe.h:125 */
int bgl_gpu_set_batch(int B);                                          /* mlx_moe.h:255: 1 <= B <= 64 */
/* Recorded for the caller; the gather always sorts pairs by expert, which gives the same values
 * as the unsorted form (mlx_moe.h:264). */
int bgl_gpu_set_sort_threshold(int threshold);
/* 1 uniform, 0 mixed dense / quantized / qNg64-plane roles, -1 a name is not bound (mlx_moe.h:334). */
int bgl_gpu_test_ffn_uniform(const char *gate_name, const char *up_name, const char *down_name);
/* The gather itself by name, host buffers: y[z] = W_{idx[z]} x[z] for z < N (ffn_gather's explicit-pair
 * canonical form, mlx_moe.cpp:1577-1589, :1901-1916). */
int bgl_gpu_ffn_gather(const char *name, const float *x, int N, const int32_t *expert_idx, float *y);
/* Routed SwiGLU FFN over bound gate/up/down names (+ optional shared-expert names, NULL for none)
 * with top-K routing given, host buffers (routed-FFN composition mlx_moe.cpp:2155-2232 /
 * moe_ffn_batched qwen_infer.c:5238-5350). */
/* The router of a MoE layer, registered by name: fp32 [E][in] (the engine's router weights,
 * qwen_infer.c:5244) and an optional bias [E] (:5247-5250), copied to the device.  No mlx_moe.h
 * counterpart (the MLX path wraps the host router per call, mlx_moe.cpp:2534): it lets
 * bgl_gpu_moe_layer run moe_ffn_batched whole.  1 = ok, 0 = failure. */
int bgl_gpu_bind_router(const char *name, const float *w, const float *bias, long E, long in);
/* moe_ffn_batched (qwen_infer.c:5238-5350) by names, routing included: bgl_moe_layer_dev on the
 * registry's context with host x [T][in] / out [T][in]; renorm = MOE_NORM_TOPK_PROB.  topk_idx /
 * topk_w [T][K] (either may be NULL) receive the routing (the engine's routing capture, :5274-5278).
 * 1 = ok, 0 = failure. */
int bgl_gpu_moe_layer(const char *router, const char *gate, const char *up, const char *down,
                      const char *shared_gate, const char *shared_up, const char *shared_down, const float *x, int T,
                      int K, int renorm, float *out, int32_t *topk_idx, float *topk_w);
int bgl_gpu_moe_ffn(const char *gate, const char *up, const char *down, const char *shared_gate,
                    const char *shared_up, const char *shared_down, const float *x, int T, const int32_t *topk_idx,
                    const float *topk_w, int K, float *out);
/* The registry's context, for device-pointer calls on registered tensors. */
bgl_ctx *bgl_gpu_context(void);
/* The registry's current device tensor for `name` (NULL if missing). */
const bgl_tensor *bgl_gpu_lookup(const char *name);

#ifdef __cplusplus
}
#endif
#endif
