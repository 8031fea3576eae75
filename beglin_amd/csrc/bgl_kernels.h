// bgl_kernels.h -- device tensor descriptor and kernel entry points (internal to the library).
#pragma once
#include "bgl_device.h"

// A bound tensor in the tiled device layout.  Work unit per format (one wave iteration):
//   Q4G64   64 elements, 2 chunks, s0 = fp32 scale
//   Q4G32H  64 elements, 2 chunks, s0 = u32 holding the two fp16 group-32 scales (low = first)
//   G256SF  256 elements, 8 chunks, s0 = u32x2 (x = fp32 wsuper bits, y = the 4 sub-codes, byte s =
//           sub s), one load per unit; codes stored as signed nibbles (code ^ 8).  The plain-g256
//           diagnostic kind is this layout with every sub-code 1 and gmul 1 instead of 1/63.
//   Q8G64   64 elements, 4 chunks, s0 = fp32 scale
//   QNG64   128 elements (a pair of 64-groups), n chunks, s0 = float2 (the two group scales)
//   MXFP4   64 elements (two GGUF blocks), 2 chunks (Q4G64's nibble order), s0 = u32 holding the
//           two E8M0 exponent bytes (low = first block)
struct BglDevTensor {
    int fmt, bits, N, K, ntiles, cpr, nunits, cpu;   // cpu: chunks per unit
    float gmul;                                      // G256SF: the fold's factor, 1/63 (subfold) or 1 (plain g256)
    const uint8_t *w;
    const void *s0;
    const uint32_t *s1;
};

// The biased code u = code + 2^(n-1) of qNg64 weight (r, c) in the tiled layout (fields widest first,
// device nibble / crumb / bit orders: bgl_prep.hip k_repack_qng).
__device__ __forceinline__ uint32_t qng_u_at(const BglDevTensor &T, int r, int c) {
    const int tile = r / BGL_TILE, lane = r % BGL_TILE;
    const QngFields f = qng_fields(T.bits);
    const int pr = c / 128, e = c % 128, h = e / 64, p64 = e % 64;
    const size_t base = (size_t)tile * T.cpr + (size_t)pr * T.bits;
    auto chunkp = [&](int k) { return T.w + ((base + k) * BGL_TILE + lane) * 16; };
    uint32_t u = 0;
    int k = 0;
    if (f.has8) { u |= (uint32_t)((chunkp(k + e / 16)[e % 16] ^ 0x80) & 255); k += 8; }
    if (f.has4) {
        const int ck = e / 32, el = e % 32, j = el / 8, q = el % 8;
        const uint8_t *b = chunkp(k + ck) + 4 * j;
        const uint32_t nib = q < 4 ? (b[q] & 15) : (b[q - 4] >> 4);
        u |= nib << f.sh4; k += 4;
    }
    if (f.has2) {
        const int j = p64 / 16, rem = p64 % 16, q = rem / 4, i = rem % 4;
        const uint8_t *b = chunkp(k + h) + 4 * j;
        u |= (uint32_t)((b[i] >> (2 * q)) & 3) << f.sh2; k += 2;
    }
    if (f.has1) {
        const int j = e / 32, rem = e % 32, q = rem / 4, i = rem % 4;
        const uint8_t *b = chunkp(k) + 4 * j;
        u |= (uint32_t)((b[i] >> q) & 1) << f.sh1;
    }
    return u;
}

// The fp32 value of weight (r, c) of a bound tensor in the tiled layout: code * scale (nib * s + b for
// the affine int4 kind), the product the reference decoders form (moe_decode_af, qwen_infer.c:2554-2655;
// dequant_row_q4_0, gguf_quants.c:118-130; qng64_decode_code, qng64_dense.c:19-27).  One element per
// call: used by k_dequant and by the GEMVs' slow path for non-finite activations.
__device__ __forceinline__ float w_at(const BglDevTensor &T, int r, int c) {
    int tile = r / BGL_TILE, lane = r % BGL_TILE;
    float v = 0.0f;
    if (T.fmt == BGL_F16 || T.fmt == BGL_F32) {
        const int esz = T.fmt == BGL_F16 ? 2 : 4, per = 16 / esz;
        const uint8_t *p = T.w + (((size_t)tile * T.cpr + c / per) * BGL_TILE + lane) * 16 + (c % per) * esz;
        if (T.fmt == BGL_F16) v = __half2float(__ushort_as_half(*reinterpret_cast<const unsigned short *>(p)));
        else v = *reinterpret_cast<const float *>(p);
    } else if (T.fmt == BGL_Q4G64 || T.fmt == BGL_Q4G32H || T.fmt == BGL_Q4G256SF || T.fmt == BGL_Q4G64A || T.fmt == BGL_MXFP4) {
        int chunk = c / 32, e = c % 32, j = e / 8, q = e % 8;
        const uint8_t *p = T.w + (((size_t)tile * T.cpr + chunk) * BGL_TILE + lane) * 16 + 4 * j;
        int nib = q < 4 ? (p[q] & 15) : (p[q - 4] >> 4);
        if (T.fmt == BGL_Q4G256SF) nib ^= 8;                 // stored as signed nibbles
        if (T.fmt == BGL_Q4G64A) {
            // moe_decode_af's affine arm (qwen_infer.c:2649-2652): (float)nib * s + b
            size_t o = ((size_t)tile * T.nunits + c / 64) * BGL_TILE + lane;
            v = __fadd_rn(__fmul_rn((float)nib, reinterpret_cast<const float *>(T.s0)[o]),
                          reinterpret_cast<const float *>(T.s1)[o]);
        } else if (T.fmt == BGL_Q4G64) {
            float s = reinterpret_cast<const float *>(T.s0)[((size_t)tile * T.nunits + c / 64) * BGL_TILE + lane];
            v = (float)(nib - 8) * s;
        } else if (T.fmt == BGL_Q4G32H) {
            uint32_t s2 = reinterpret_cast<const uint32_t *>(T.s0)[((size_t)tile * T.nunits + c / 64) * BGL_TILE + lane];
            uint16_t h = (uint16_t)(((c / 32) & 1) ? (s2 >> 16) : (s2 & 0xffff));
            v = (float)(nib - 8) * __half2float(__ushort_as_half(h));
        } else if (T.fmt == BGL_MXFP4) {
            // moe_decode_af's MXFP4 arm (qwen_infer.c:2584-2595): kvalues[nib] * e8m0_half(block byte)
            uint32_t s2 = reinterpret_cast<const uint32_t *>(T.s0)[((size_t)tile * T.nunits + c / 64) * BGL_TILE + lane];
            v = (float)(int8_t)(mx_codes((uint32_t)nib) & 255) * mx_scale((s2 >> (8 * ((c / 32) & 1))) & 255u);
        } else {
            size_t o = ((size_t)tile * T.nunits + c / 256) * BGL_TILE + lane;
            const uint2 wsub = reinterpret_cast<const uint2 *>(T.s0)[o];
            float ws = __uint_as_float(wsub.x);
            uint32_t sub4 = wsub.y;
            float sc = (float)((sub4 >> (8 * ((c / 64) & 3))) & 255);
            v = T.gmul == 1.0f ? (float)(nib - 8) * ws : (float)(nib - 8) * __fmul_rn(ws, __fdiv_rn(sc, 63.0f));
        }
    } else if (T.fmt == BGL_Q8G64) {
        const int8_t *p = reinterpret_cast<const int8_t *>(T.w) + (((size_t)tile * T.cpr + c / 16) * BGL_TILE + lane) * 16;
        float s = reinterpret_cast<const float *>(T.s0)[((size_t)tile * T.nunits + c / 64) * BGL_TILE + lane];
        v = (float)p[c % 16] * s;
    } else {
        const int n = T.bits, pr = c / 128, h = (c % 128) / 64;
        const uint32_t u = qng_u_at(T, r, c);
        float2 s2 = reinterpret_cast<const float2 *>(T.s0)[((size_t)tile * T.nunits + pr) * BGL_TILE + lane];
        float s = h ? s2.y : s2.x;
        v = (float)((int)u - (1 << (n - 1))) * s;
    }
    return v;
}

// w_at for a format known at compile time (the GEMVs' cold paths): 32-bit offsets, no format switch.
template <int FMT, int NB>
__device__ __forceinline__ float w_at_t(const BglDevTensor &T, int r, int c) {
    const uint32_t tile = (uint32_t)r / BGL_TILE, lane = (uint32_t)r % BGL_TILE;
    if constexpr (FMT == BGL_Q4G64 || FMT == BGL_Q4G32H || FMT == BGL_Q4G64A || FMT == BGL_MXFP4) {
        const uint32_t e = (uint32_t)c % 32u, j = e / 8u, q = e % 8u;
        const uint8_t b = T.w[((tile * (uint32_t)T.cpr + (uint32_t)c / 32u) * BGL_TILE + lane) * 16u + 4u * j + (q & 3u)];
        const int nib = q < 4 ? (b & 15) : (b >> 4);
        const uint32_t so = (tile * (uint32_t)T.nunits + (uint32_t)c / 64u) * BGL_TILE + lane;
        if constexpr (FMT == BGL_Q4G64A)
            return __fadd_rn(__fmul_rn((float)nib, reinterpret_cast<const float *>(T.s0)[so]), reinterpret_cast<const float *>(T.s1)[so]);
        else if constexpr (FMT == BGL_Q4G64)
            return (float)(nib - 8) * reinterpret_cast<const float *>(T.s0)[so];
        else if constexpr (FMT == BGL_MXFP4)
            return (float)(int8_t)(mx_codes((uint32_t)nib) & 255) *
                   mx_scale((reinterpret_cast<const uint32_t *>(T.s0)[so] >> (8u * (((uint32_t)c / 32u) & 1u))) & 255u);
        else {
            const uint32_t s2 = reinterpret_cast<const uint32_t *>(T.s0)[so];
            return (float)(nib - 8) * __half2float(__ushort_as_half((unsigned short)((((uint32_t)c / 32u) & 1u) ? (s2 >> 16) : (s2 & 0xffffu))));
        }
    } else if constexpr (FMT == BGL_Q8G64) {
        const int8_t v = reinterpret_cast<const int8_t *>(T.w)[((tile * (uint32_t)T.cpr + (uint32_t)c / 16u) * BGL_TILE + lane) * 16u + (uint32_t)c % 16u];
        return (float)v * reinterpret_cast<const float *>(T.s0)[(tile * (uint32_t)T.nunits + (uint32_t)c / 64u) * BGL_TILE + lane];
    } else if constexpr (FMT == BGL_QNG64) {
        const uint32_t u = qng_u_at(T, r, c);
        const float2 s2 = reinterpret_cast<const float2 *>(T.s0)[(tile * (uint32_t)T.nunits + (uint32_t)c / 128u) * BGL_TILE + lane];
        return (float)((int)u - (1 << (NB - 1))) * (((c % 128) / 64) ? s2.y : s2.x);
    } else {
        return w_at(T, r, c);
    }
}

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
    const float *xs;          // W4A8: ascale [M][K/gq];          F32: 2^(e-22) [M][K/64]
    const int *xsum;          // W4A8: sum xq per 64 [M][K/64];   F32: digit sums [M][K/32][4], the
                              //   4th int of a group's first half = its flags (BGL_XF_*)
    const int *xw1;           // F32 level 1 (groups flagged BGL_XF_L1): residual digits [M][K/64][48]
    const float *xs1;         // F32 level 1: 2^(e1-22) relative to the level-0 scale, 0 without level 1 [M][K/64]
    const int *xsum1;         // F32 level 1: digit sums [M][K/32][4]
    const int *colmap;        // optional: column m of this launch reads activation row colmap[m]
    const float *xf;          // F32: the raw rows [M][K] (dense fp16 / fp32 weights and the non-finite
                              //   slow path read these)
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
    int mbx;                     // k_moe_x: token columns of records the launch's LDS holds (4 or 8)
};

// ---- kernels (bgl_prep.hip) ----
__global__ void k_act_w4a8(const float *x, int M, int K, int gsize, int8_t *xq, float *ascale, int *xqsum64, const float *u,
                           float *h);
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
// bgl_gemv_qm.hip: W4A8 at 2..16 columns on the matrix cores; nblk workgroups of RB 16-row blocks
// and S unit slices; prep: L.a holds prepared codes
int bgl_launch_gemv_qm(const GemvLaunch &L, int nblk, int RB, int S, bool prep, hipStream_t st);
size_t bgl_gemv_qm_lds(int fmt, int K, int MC, int RB, bool prep);
size_t bgl_gemv_q_lds(int fmt, int K, int TR, int MB);
// ---- bgl_gemv_x.hip: one-column fp32-activation GEMV over prepared digits ----
int bgl_launch_gemv_x(const GemvLaunch &L, bool fuse, int nblocks, int TR, int nw, hipStream_t st);
size_t bgl_gemv_x_lds(int K, int TR, int nw, bool fuse);
// ---- bgl_moe_x.hip: the MoE gather over records made in the kernel ----
bool bgl_moe_x_fmt(int fmt);
size_t bgl_moe_x_lds(int K, int nw, int TR, int cap);
int bgl_moe_x_cap(int K, int nw, int TR);
void bgl_moe_x_shape(int K, long active_wgs, int tr_force, int nw_cap, int *TR, int *nw);
int bgl_launch_moe_x(const MoeTask &Mt, int K, int TR, int nw, int cap, hipStream_t st);
// Two gathers over the same activation rows in one launch (workgroups [0, nb0) run t[0], the rest
// t[1]); whole 64-row tiles; t[1] may be segmented (seg > 0 without off).
struct MoePair {
    MoeTask t[2];
    int nb0;
};
int bgl_launch_moe_x2(const MoeTask &a, const MoeTask &b, int K, int nw, int cap, hipStream_t st);
