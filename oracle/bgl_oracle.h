/* bgl_oracle.h -- CPU oracle for the quantized GEMV / MoE-gather path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference engine's
 * packers, decoders and GEMV/gather arithmetic, used as the checker by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg.  Nothing in the product
 * (beglin_amd/) links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to the
 * reference repository root).  Build: oracle/Makefile, compiled with -ffp-contract=off
 * so every fp32 expression rounds exactly as written (the literal C semantics).
 *
 * Parity status (what pins each function; tests/test_oracle.py):
 *   - or_quantize_q4g64_ef / _q8g64 / _qng64_gguf / _qng64_dense / _q4_0, or_decode_*,
 *     or_qng64_decode_code, or_qng64_matvec_f32: byte-exact against the reference's own C
 *     (oracle/_ref, built from the reference sources), the tiny_st control constants and the
 *     qng64_dense_test KAT.
 *   - or_f32_to_f16 / or_f16_to_f32: exhaustive over all 2^16 halves / IEEE RNE cases.
 *   - or_gemm_f32, or_moe_row, or_moe_decode, or_moe_matvec: equal to the double product over
 *     independently decoded weights; the reference's vDSP_dotpr summation order (closed
 *     Accelerate library) is parity unpinned beyond the 1e-5 tolerance.
 *   - or_quant_act_i8, or_gemm_*_sdot, or_matmul_sdot: reference rounding cases + the identity
 *     against the de-quantized product + batched == per-column.
 *   - or_quantize_g256sf: build-defined (the reference ships no g256sf emitter).  Pinned where
 *     it reduces to the reference: with the four 64-subgroups of every 256-group sharing their
 *     max |w| it must be gguf_quantize_q4g64_error_feedback (oracle/_ref) byte for byte, sub = 63;
 *     plus the minimality of sub (smallest code whose effective scale covers max|w|/7) and
 *     wsuper = the largest subgroup scale.
 *   - or_moe_router_logits: a pure-Python sequential double loop (the reference order), bit for bit.
 *   - or_decode_qng64_mixed: equal to or_decode_qng64 when every cell has the same n, and to an
 *     independent Python bit-plane decode for random per-cell widths.
 *   - or_moe_route / _softmax_full / _top_k_select / _topk_renorm: brute force; or_moe_ffn_*:
 *     bucketed == naive and a dense float64 pipeline over decoded weights.
 *   - or_mx_scale / or_mx_value and the MXFP4 arms of or_moe_decode / or_moe_row: bit for bit
 *     against oracle/_ref's gguf_quants.c (every exponent byte, every code, gguf_dequant_row).
 *   - or_gemm_g256plain_sdot: at power-of-two scales, where every term is exact, equal to a float32
 *     running sum of integer sums computed independently from the nibbles.
 *   - or_swiglu: numpy's float64 exp rounded once, then the float steps; special values; within
 *     2 ulp of the reference's float-expf form.
 *   - or_pool_* (the CPU baseline): equal to the single-threaded restatements they split.
 * This file and its .c are test infrastructure: only tests/, smoke() and bench.py's CPU leg use
 * them, as the checker, never as the thing measured or shipped.
 */
#ifndef BGL_ORACLE_H
#define BGL_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- IEEE binary16 helpers (round-to-nearest-even) ---------------- */
uint16_t or_f32_to_f16(float f);
float    or_f16_to_f32(uint16_t h);

/* ---------------- packers ---------------- */
void or_quantize_q4g64_ef(const float *w, int out, int in, uint8_t *packed, float *scales);
void or_quantize_q8g64(const float *w, int out, int in, int8_t *codes, float *scales);
void or_quantize_qng64_gguf(const float *w, int out, int in, int n, uint8_t *planes, float *scales);
int  or_quantize_qng64_dense(const float *w, int out, int in, int n, uint8_t *planes, float *scales);
void or_quantize_q4_0(const float *w, int64_t n, uint8_t *blocks);
void or_q4_0_to_q4g32h(const uint8_t *blocks, int out, int in, uint8_t *packed, uint16_t *scales16);
void or_quantize_q4g32h(const float *w, int out, int in, uint8_t *packed, uint16_t *scales16);
void or_quantize_g256sf(const float *w, int out, int in, uint8_t *packed, float *wsuper, uint8_t *sub);
size_t or_qng64_group_bytes(int n);

/* ---------------- decoders: full [out][in] fp32 ---------------- */
void or_decode_q4g64(const uint8_t *packed, const float *scales, int out, int in, float *w);
void or_decode_q8g64(const int8_t *codes, const float *scales, int out, int in, float *w);
void or_decode_qng64(const uint8_t *planes, const float *scales, int n, int out, int in, float *w);
void or_decode_q4_0(const uint8_t *blocks, int64_t n, float *w);
void or_decode_q4g32h(const uint8_t *packed, const uint16_t *scales16, int out, int in, float *w);
void or_decode_g256sf(const uint8_t *packed, const float *wsuper, const uint8_t *sub, int out, int in, float *w);
float or_qng64_decode_code(const uint8_t *group, int n, int index);
void or_decode_qng64_mixed(const uint8_t *planes, const uint32_t *offsets, const uint8_t *bits, const float *scales,
                           int out, int in, float *w);

/* ---------------- fp32-activation GEMV (y = W x + bias), x [M][in], y [M][out] ----------------
 * kind: 1 q4g64, 2 q8g64, 4 qNg64 (bits=n), 5 q4g32h (packed + fp16 scales in `scales`). */
void or_gemm_f32(int kind, int bits, const void *packed, const void *scales,
                 const float *x, const float *bias, float *y, int out, int in, int M);
void or_qng64_matvec_f32(const uint8_t *planes, const float *scales, int n, const float *x,
                         const float *bias, float *y, int out, int in);

/* ---------------- W4A8 / W8A8 (int8-activation) path ---------------- */
void or_quant_act_i8(const float *x, int in, int gsize, int8_t *xq, float *ascale);
void or_gemm_q4g64_sdot(const uint8_t *packed, const float *wscale, const int8_t *xq, const float *ascale,
                        const float *bias, float *y, int out, int in, int M);
void or_gemm_q8g64_sdot(const int8_t *codes, const float *wscale, const int8_t *xq, const float *ascale,
                        const float *bias, float *y, int out, int in, int M);
void or_gemm_g256sf_sdot(const uint8_t *packed, const float *wsuper, const uint8_t *sub,
                         const int8_t *xq, const float *ascale, const float *bias, float *y,
                         int out, int in, int M);
/* the plain-g256 diagnostic row (q4gemv_g256.h:102-130), unwired in the reference too */
void or_gemm_g256plain_sdot(const uint8_t *packed, const float *wscale, const int8_t *xq, const float *ascale,
                            const float *bias, float *y, int out, int in, int M);
/* convenience: quantize each column of x then run the sdot GEMM (matmul_sdot, qwen_infer.c:1852-1900);
 * kind 1 q4g64, 2 q8g64, 3 g256sf, 10 plain g256 */
void or_matmul_sdot(int kind, const void *packed, const float *scales, const uint8_t *sub,
                    const float *x, const float *bias, float *y, int out, int in, int M);

/* ---------------- MoE ---------------- */
typedef struct {
    int kind;            /* 1 q4g64 (sym), 2 q8g64, 4 qNg64, 5 q4g32h, 6 int4 affine, 7 fp16, 8 fp32,
                            9 MXFP4 (GGUF blocks [out][in/32][17]) */
    int bits;            /* qNg64 n */
    const void *packed;
    const void *scales;  /* fp32, or fp16 bits for q4g32h; unused for 7 / 8 */
    const void *bias;    /* kind 6: fp32 biases [out][in/64] */
} or_expert;

double or_moe_row(const or_expert *w, int in, long row, const float *x);
float or_mx_scale(uint8_t b);
int or_mx_value(int code);
float or_moe_decode(const or_expert *w, int in, long row, long col);
void or_moe_matvec(const or_expert *w, int out, int in, const float *x, float *y);
void or_moe_softmax_full(float *x, int n);
void or_moe_top_k_select(const float *scores, int n, int k, int *out_idx);
void or_moe_topk_renorm(float *scores, const int *idx, int k);
void or_moe_swiglu_inplace(float *gate, const float *up, int n);
void or_swiglu(const float *g, const float *u, float *out, int n);
void or_moe_route(const float *logits, int T, int E, int K, int renorm, int *top_idx, float *top_w);
void or_moe_router_logits(const float *w, const float *bias, const float *x, int T, int E, int H, float *logits);
void or_moe_ffn_bucketed(const or_expert *gate, const or_expert *up, const or_expert *down, int E,
                         const or_expert *sh_gate, const or_expert *sh_up, const or_expert *sh_down,
                         int H, int I, int Ish, int T, int K, const float *x,
                         const int *top_idx, const float *top_w, float *out);
void or_moe_ffn_naive(const or_expert *gate, const or_expert *up, const or_expert *down, int E,
                      const or_expert *sh_gate, const or_expert *sh_up, const or_expert *sh_down,
                      int H, int I, int Ish, int T, int K, const float *x,
                      const int *top_idx, const float *top_w, float *out);

/* ---------------- CPU baseline: pthread row-block pool (q4gemv.h:408-670 semantics) ---------------- */
typedef struct or_pool or_pool;
or_pool *or_pool_create(int nthreads, int max_in);
void or_pool_destroy(or_pool *p);
int  or_pool_threads(const or_pool *p);
void or_pool_gemv_g256sf_sdot(or_pool *p, const uint8_t *packed, const float *wsuper, const uint8_t *sub,
                              const float *x, const float *bias, float *y, int out, int in);
void or_pool_gemv_q4g64_sdot(or_pool *p, const uint8_t *packed, const float *scales,
                             const float *x, const float *bias, float *y, int out, int in);
void or_pool_gemv_f32(or_pool *p, int kind, int bits, const void *packed, const void *scales,
                      const float *x, const float *bias, float *y, int out, int in);
void or_pool_moe_ffn_bucketed(or_pool *p, const or_expert *gate, const or_expert *up, const or_expert *down, int E,
                              const or_expert *sh_gate, const or_expert *sh_up, const or_expert *sh_down,
                              int H, int I, int Ish, int T, int K, const float *x,
                              const int *top_idx, const float *top_w, float *out);

#ifdef __cplusplus
}
#endif
#endif
