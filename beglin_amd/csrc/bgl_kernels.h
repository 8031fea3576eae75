// bgl_kernels.h -- device tensor descriptor and kernel entry points (internal to the library).
#pragma once
#include "bgl_device.h"

// A bound tensor in the tiled device layout.  Work unit per format (one wave iteration):
//   Q4G64   64 elements, 2 chunks, s0 = fp32 scale
//   Q4G32H  64 elements, 2 chunks, s0 = u32 holding the two fp16 group-32 scales (low = first)
//   G256SF  256 elements, 8 chunks, s0 = u32x2 (x = fp32 wsuper bits, y = the 4 sub-codes, byte s =
//           sub s), one load per unit; codes stored as signed nibbles (code ^ 8)
//   Q8G64   64 elements, 4 chunks, s0 = fp32 scale
//   QNG64   128 elements (a pair of 64-groups), n chunks, s0 = float2 (the two group scales)
struct BglDevTensor {
    int fmt, bits, N, K, ntiles, cpr, nunits, cpu;   // cpu: chunks per unit
    const uint8_t *w;
    const void *s0;
    const uint32_t *s1;
};

#define BGL_MAX_TASKS 4

// One GEMV "task" = one tensor of a (possibly fused) launch.  Blocks [blk0, blk0 + ntiles) of the
// grid belong to it; block b computes tile b-blk0 over the whole K range.
struct GemvTask {
    BglDevTensor T;
    float *y;                 // [M][N] (row stride ystride)
    const float *bias;        // [N] or null
    int ystride;
    int blk0;
    int ks, gpb;              // K split over ks workgroups of gpb units each (ks == 1: no split)
    float *part;              // ks > 1: partials [ks][M][N], summed by k_splitk_reduce
};

// Activation operands (shared by every task of a launch; all tasks have the same K).
struct GemvAct {
    const int *xw;            // W4A8: xq dwords [M][K/4];       F32: digits [M][K/64][48]
    const float *xs;          // W4A8: ascale [M][K/gq];          F32: 2^(e-21) [M][K/64]
    const int *xsum;          // W4A8: sum xq per 64 [M][K/64];   F32: digit sums [M][K/32][4]
    const int *colmap;        // optional: column m of this launch reads activation row colmap[m]
    const float *xf;          // F32: the raw rows [M][K] (dense fp16 / fp32 weights read these)
    int gq;                   // W4A8 activation group (64 or 256)
};

struct GemvLaunch {
    GemvTask t[BGL_MAX_TASKS];
    int ntasks;
    GemvAct a;                // prepared activation operands (k_gemv)
    const float *x;           // raw fp32 activations [M][K] (k_gemv_q quantizes them itself)
    int m0, mcols;            // columns [m0, m0+mcols) of the activation (mcols <= MB)
    int mtot;                 // total columns of the call (partial buffer stride)
};

#define MOE_MAX_K 16        // top-K limit of the combine

// One expert-sorted gather launch (bgl_moe.hip, bgl_moe_x.hip).
struct MoeTask {
    const BglDevTensor *ta;      // expert table [E] (gate, or the only projection); null: use da
    const BglDevTensor *tb;      // up table [E] in SwiGLU mode
    BglDevTensor da, db;         // by-value single tensor(s) when ta is null (shared experts)
    int E, tpe;                  // grid = E * tpe workgroups (tpe: 64-row tiles per expert)
    const int *off;              // [E+1] sorted segment starts; null: one segment [0, ncols), or with
    int ncols, seg;              // seg > 0 runs of seg columns (E = ncols / seg rounded up, one tensor)
    const int *cols;             // activation row of sorted position s (null: s)
    const int *ymap;             // output row of sorted position s (null: s)
    GemvAct a;                   // k_moe_gemv: exact-digit activations (k_act_x24 layout); k_moe_x: a.xf, the raw rows
    float *y;
    int ystride;
    int swiglu;                  // y = silu(A x) * (B x)
    // k_moe_x only (the shared down projection of a routed FFN, column = token): when cout is set,
    // the store is the whole combine, cout[t] = sum over t's experts in ascending id of
    // w * cdown[pos] + this launch's value (k_moe_combine's arithmetic)
    float *cout;
    const float *cdown, *cw;
    const int *cpos;
    const int32_t *cidx;
    int ck;
};

// ---- kernels (bgl_prep.hip) ----
__global__ void k_act_w4a8(const float *x, int M, int K, int gsize, int8_t *xq, float *ascale, int *xqsum64);
__global__ void k_act_x24(const float *x, int M, int K, int8_t *xd, float *xs, int *dsum);
__global__ void k_act_import_i8(const int8_t *xq, const float *ascale, int M, int K, int gq, int split, int8_t *xw,
                                float *xs, int *xsum64);
__global__ void k_quant_q4g64(const float *w, int N, int K, uint8_t *packed, float *scales);
__global__ void k_quant_q8g64(const float *w, int N, int K, int8_t *codes, float *scales);
__global__ void k_quant_qng64(const float *w, int N, int K, int n, int dense_floor, uint8_t *planes, float *scales);
__global__ void k_quant_q4g32h(const float *w, int N, int K, uint8_t *packed, uint16_t *scales16);
__global__ void k_quant_g256sf(const float *w, int N, int K, uint8_t *packed, float *wsuper, uint8_t *sub);
__global__ void k_repack_nib(const uint8_t *src, int N, int K, uint32_t flip, uint8_t *dst);
__global__ void k_repack_q8(const int8_t *src, int N, int K, uint8_t *dst);
__global__ void k_repack_qng(const uint8_t *src, int N, int K, int n, uint8_t *dst);
__global__ void k_repack_u32(const uint32_t *src, int N, int U, uint32_t *dst);
__global__ void k_repack_u64(const uint64_t *src, int N, int U, uint64_t *dst);
__global__ void k_repack_zip_u32(const uint32_t *a, const uint32_t *b, int N, int U, uint2 *dst);
__global__ void k_mixed_qng_to_dense(const uint8_t *planes, const uint32_t *offsets, const uint8_t *bits, long cells, int W,
                                     uint8_t *dst);
__global__ void k_repack_qng_scales(const float *src, int N, int ng, float2 *dst);
__global__ void k_dequant(BglDevTensor T, int row0, int nrows, float *out);
__global__ void k_splitk_reduce(const float *part, int ks, int M, int N, const float *bias, float *y, int ystride);

// ---- host-side launchers (bgl_gemv.hip) ----
int bgl_launch_gemv(int act, int MB, const GemvLaunch &L, int nblocks, int nw, hipStream_t st);
int bgl_launch_gemv_q(const GemvLaunch &L, int ntiles, int TR, int nw, int MB, hipStream_t st);
size_t bgl_gemv_q_lds(int fmt, int K, int TR, int MB);
// ---- bgl_gemv_x.hip: one-column fp32-activation GEMV over prepared digits ----
int bgl_launch_gemv_x(const GemvLaunch &L, bool fuse, int nblocks, int TR, int nw, hipStream_t st);
size_t bgl_gemv_x_lds(int K, int TR, int nw);
// ---- bgl_moe_x.hip: the MoE gather over records made in the kernel ----
bool bgl_moe_x_fmt(int fmt);
size_t bgl_moe_x_lds(int K, int nw, int TR);
void bgl_moe_x_shape(int K, long active_wgs, int tr_force, int nw_cap, int *TR, int *nw);
int bgl_launch_moe_x(const MoeTask &Mt, int K, int TR, int nw, hipStream_t st);
// Two gathers over the same activation rows in one launch (workgroups [0, nb0) run t[0], the rest
// t[1]); whole 64-row tiles; t[1] may be segmented (seg > 0 without off).
struct MoePair {
    MoeTask t[2];
    int nb0;
};
int bgl_launch_moe_x2(const MoeTask &a, const MoeTask &b, int K, int nw, hipStream_t st);
