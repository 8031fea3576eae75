// bgl_gemv_impl.h -- device building blocks shared by the GEMV and MoE-gather kernels: per-format
// raw unit loads from the tiled layout and the per-unit dot/fold against prepared activations
// (SGPR operands).  Included by bgl_gemv.hip and bgl_moe.hip only.
#pragma once
#include "bgl_kernels.h"

#define C63 (1.0f / 63.0f)
#define MAXW 16

template <int MB>
struct Cols {
    int am[MB];
};

template <int MB>
__device__ __forceinline__ Cols<MB> col_rows(const GemvAct &A, int m0, int mcols) {
    Cols<MB> c;
#pragma unroll
    for (int m = 0; m < MB; m++) {
        int mm = m < mcols ? m : mcols - 1;                 // padded columns repeat the last one
        c.am[m] = A.colmap ? uni(A.colmap)[m0 + mm] : m0 + mm;
    }
    return c;
}

// digit sums of one 32-element half (3 ints; the 4th: the group's BGL_XF_* flags in its first half)
__device__ __forceinline__ int4 ld_dsum(const int *xsum, int am, int K, int half) {
    ucint p = uni(xsum) + ((size_t)am * (K >> 5) + half) * 4;
    return make_int4(p[0], p[1], p[2], p[3]);
}
__device__ __forceinline__ int4 ld_dsum(const GemvAct &A, int am, int K, int half) { return ld_dsum(A.xsum, am, K, half); }
// the BGL_XF_* flags of group g of prepared column am
__device__ __forceinline__ int ld_xflags(const GemvAct &A, int am, int K, int g) {
    return uni(A.xsum)[((size_t)am * (K >> 5) + 2 * g) * 4 + 3];
}

// The products code * scale * x of a group's non-finite activations, one element at a time
// (IEEE: NaN and +-Inf propagate as in the reference's fp32-product sums).  Only groups flagged
// BGL_XF_NF take this path; their finite part comes from the digits.
template <int FMT, int NB>
__device__ __forceinline__ float x_nonfinite(const BglDevTensor &T, int row, int g, const float *xr) {
    float acc = 0.0f;
#pragma unroll 1
    for (int j = 0; j < 64; j++) {
        const float v = xr[g * 64 + j];
        if (!isfinite(v)) acc += w_at_t<FMT, NB>(T, row, g * 64 + j) * v;
    }
    return acc;
}

// The weight row a lane computes (for the non-finite slow path).
struct WRow {
    const BglDevTensor *T;
    int row;
};

__device__ __forceinline__ float fold_digits(int t0, int t1, int t2) {
    return (float)t0 + 256.0f * (float)t1 + 65536.0f * (float)t2;
}

// ================================================================================== raw unit loads
template <int FMT, int NB> struct Raw;
template <int NB> struct Raw<BGL_Q4G64, NB> { uint4 c[2]; float s; };
template <int NB> struct Raw<BGL_Q4G32H, NB> { uint4 c[2]; uint32_t s; };
template <int NB> struct Raw<BGL_Q4G256SF, NB> { uint4 c[8]; float s; uint32_t sub; float gm; };
template <int NB> struct Raw<BGL_Q8G64, NB> { uint4 c[4]; float s; };
template <int NB> struct Raw<BGL_QNG64, NB> { uint4 c[NB]; float2 s; };
template <int NB> struct Raw<BGL_Q4G64A, NB> { uint4 c[2]; float s; float b; };
template <int NB> struct Raw<BGL_F16, NB> { uint4 c[8]; };
template <int NB> struct Raw<BGL_F32, NB> { uint4 c[16]; };

template <int FMT> constexpr int chunks_per_unit(int nb) {
    return FMT == BGL_Q4G256SF ? 8 : FMT == BGL_Q8G64 ? 4 : FMT == BGL_QNG64 ? nb : FMT == BGL_F16 ? 8 : FMT == BGL_F32 ? 16 : 2;
}

// Weight planes live in global memory; the explicit address space keeps these global (not flat)
// loads when the tensor record itself was read from a device table.
// (native vector types: HIP's uint4/float2 classes cannot be assigned from such references)
#define BGL_GLOBAL __attribute__((address_space(1)))
typedef unsigned int bgl_u32x4 __attribute__((ext_vector_type(4)));
typedef float bgl_f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int bgl_u32x2 __attribute__((ext_vector_type(2)));
typedef float bgl_f32x4 __attribute__((ext_vector_type(4)));

template <int FMT, int NB>
__device__ __forceinline__ void load_raw(Raw<FMT, NB> &r, const BglDevTensor &T, int tile, int lane, int u) {
    constexpr int CPU = chunks_per_unit<FMT>(NB);
    const BGL_GLOBAL bgl_u32x4 *cp =
        (const BGL_GLOBAL bgl_u32x4 *)(T.w) + ((size_t)tile * T.cpr + (size_t)u * CPU) * BGL_TILE + lane;
#pragma unroll
    for (int k = 0; k < CPU; k++) {
        const bgl_u32x4 v = cp[k * BGL_TILE];
        r.c[k] = make_uint4(v.x, v.y, v.z, v.w);
    }
    if constexpr (FMT != BGL_F16 && FMT != BGL_F32) {                 // dense rows carry no scales
    const size_t so = ((size_t)tile * T.nunits + u) * BGL_TILE + lane;
    if constexpr (FMT == BGL_Q4G64A) {
        r.s = ((const BGL_GLOBAL float *)T.s0)[so];
        r.b = ((const BGL_GLOBAL float *)T.s1)[so];
    } else if constexpr (FMT == BGL_QNG64) {
        const bgl_f32x2 v = ((const BGL_GLOBAL bgl_f32x2 *)T.s0)[so];
        r.s = make_float2(v.x, v.y);
    } else if constexpr (FMT == BGL_Q4G32H) r.s = ((const BGL_GLOBAL uint32_t *)T.s0)[so];
    else if constexpr (FMT == BGL_Q4G256SF) {
        const bgl_u32x2 w = ((const BGL_GLOBAL bgl_u32x2 *)T.s0)[so];
        r.s = __uint_as_float(w.x);
        r.sub = w.y;
        r.gm = T.gmul;
    } else r.s = ((const BGL_GLOBAL float *)T.s0)[so];
    }
}

// ================================================================================== path A compute
// x operands: ucint (scalar-loaded) pointers into the prepared activation buffers.

template <int ACT, int MB, int NB>
__device__ __forceinline__ void comp_q4g64(const Raw<BGL_Q4G64, NB> &r, int K, int u, const GemvAct &A,
                                           const Cols<MB> &C, float (&acc)[MB]) {
    int lo[8], hi[8];
    uint32_t raw[8] = {r.c[0].x, r.c[0].y, r.c[0].z, r.c[0].w, r.c[1].x, r.c[1].y, r.c[1].z, r.c[1].w};
#pragma unroll
    for (int q = 0; q < 8; q++) { lo[q] = nib_lo(raw[q]); hi[q] = nib_hi(raw[q]); }
    const int ng = K >> 6;
#pragma unroll
    for (int m = 0; m < MB; m++) {
        const int am = C.am[m];
        if constexpr (ACT == BGL_ACT_F32) {
            ucint xg = uni(A.xw) + ((size_t)am * ng + u) * BGL_XD_DW;
            int t0 = 0, t1 = 0, t2 = 0;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                t0 = dot4(lo[q], xg[2 * q], t0);      t0 = dot4(hi[q], xg[2 * q + 1], t0);
                t1 = dot4(lo[q], xg[16 + 2 * q], t1); t1 = dot4(hi[q], xg[16 + 2 * q + 1], t1);
                t2 = dot4(lo[q], xg[32 + 2 * q], t2); t2 = dot4(hi[q], xg[32 + 2 * q + 1], t2);
            }
            int4 d0 = ld_dsum(A, am, K, 2 * u), d1 = ld_dsum(A, am, K, 2 * u + 1);
            t0 -= 8 * (d0.x + d1.x); t1 -= 8 * (d0.y + d1.y); t2 -= 8 * (d0.z + d1.z);
            acc[m] += r.s * (fold_digits(t0, t1, t2) * uni(A.xs)[(size_t)am * ng + u]);
        } else {
            ucint xq = uni(A.xw) + (size_t)am * (K >> 2) + (size_t)u * 16;
            int isum = 0;
#pragma unroll
            for (int q = 0; q < 8; q++) { isum = dot4(lo[q], xq[2 * q], isum); isum = dot4(hi[q], xq[2 * q + 1], isum); }
            isum -= 8 * uni(A.xsum)[(size_t)am * ng + u];
            acc[m] = __fadd_rn(acc[m], __fmul_rn(__fmul_rn((float)isum, r.s), uni(A.xs)[(size_t)am * ng + u]));
        }
    }
}

template <int MB, int NB>
__device__ __forceinline__ void comp_q4g32h(const Raw<BGL_Q4G32H, NB> &r, int K, int u, const GemvAct &A,
                                            const Cols<MB> &C, float (&acc)[MB]) {
    float sa = __half2float(__ushort_as_half((unsigned short)(r.s & 0xffffu)));
    float sb = __half2float(__ushort_as_half((unsigned short)(r.s >> 16)));
    int lo[8], hi[8];
    uint32_t raw[8] = {r.c[0].x, r.c[0].y, r.c[0].z, r.c[0].w, r.c[1].x, r.c[1].y, r.c[1].z, r.c[1].w};
#pragma unroll
    for (int q = 0; q < 8; q++) { lo[q] = nib_lo(raw[q]); hi[q] = nib_hi(raw[q]); }
    const int ng = K >> 6;
#pragma unroll
    for (int m = 0; m < MB; m++) {
        const int am = C.am[m];
        ucint xg = uni(A.xw) + ((size_t)am * ng + u) * BGL_XD_DW;
        int a0 = 0, a1 = 0, a2 = 0, b0 = 0, b1 = 0, b2 = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            a0 = dot4(lo[q], xg[2 * q], a0);      a0 = dot4(hi[q], xg[2 * q + 1], a0);
            a1 = dot4(lo[q], xg[16 + 2 * q], a1); a1 = dot4(hi[q], xg[16 + 2 * q + 1], a1);
            a2 = dot4(lo[q], xg[32 + 2 * q], a2); a2 = dot4(hi[q], xg[32 + 2 * q + 1], a2);
        }
#pragma unroll
        for (int q = 4; q < 8; q++) {
            b0 = dot4(lo[q], xg[2 * q], b0);      b0 = dot4(hi[q], xg[2 * q + 1], b0);
            b1 = dot4(lo[q], xg[16 + 2 * q], b1); b1 = dot4(hi[q], xg[16 + 2 * q + 1], b1);
            b2 = dot4(lo[q], xg[32 + 2 * q], b2); b2 = dot4(hi[q], xg[32 + 2 * q + 1], b2);
        }
        int4 d0 = ld_dsum(A, am, K, 2 * u), d1 = ld_dsum(A, am, K, 2 * u + 1);
        float Va = fold_digits(a0 - 8 * d0.x, a1 - 8 * d0.y, a2 - 8 * d0.z);
        float Vb = fold_digits(b0 - 8 * d1.x, b1 - 8 * d1.y, b2 - 8 * d1.z);
        float xs = uni(A.xs)[(size_t)am * ng + u];
        acc[m] += sa * (Va * xs) + sb * (Vb * xs);
    }
}

// g256sf codes are stored as signed nibbles (code ^ 8): (w << 4) & 0xF0F0F0F0 and w & 0xF0F0F0F0 are
// 16*(code-8) as int8, so the dot4 sums are exactly 16x the reference's isum (no sum(xq) term).
template <int MB, int NB>
__device__ __forceinline__ void comp_g256sf(const Raw<BGL_Q4G256SF, NB> &r, int K, int u, const GemvAct &A,
                                            const Cols<MB> &C, float (&acc)[MB]) {
    int lo[32], hi[32];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t d[4] = {r.c[k].x, r.c[k].y, r.c[k].z, r.c[k].w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            lo[4 * k + j] = (int)((d[j] << 4) & 0xF0F0F0F0u);
            hi[4 * k + j] = (int)(d[j] & 0xF0F0F0F0u);
        }
    }
#pragma unroll
    for (int m = 0; m < MB; m++) {
        const int am = C.am[m];
        ucint xq = uni(A.xw) + (size_t)am * (K >> 2) + (size_t)u * 64;
        int comb16 = 0;
#pragma unroll
        for (int sg = 0; sg < 4; sg++) {
            int isum16 = 0;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                isum16 = dot4(lo[8 * sg + q], xq[16 * sg + 2 * q], isum16);
                isum16 = dot4(hi[8 * sg + q], xq[16 * sg + 2 * q + 1], isum16);
            }
            comb16 += isum16 * (int)((r.sub >> (8 * sg)) & 255u);
        }
        float t = __fmul_rn(__fmul_rn(__fmul_rn((float)(comb16 >> 4), r.s), r.gm), uni(A.xs)[(size_t)am * (K >> 8) + u]);
        acc[m] = __fadd_rn(acc[m], t);
    }
}

template <int ACT, int MB, int NB>
__device__ __forceinline__ void comp_q8g64(const Raw<BGL_Q8G64, NB> &r, int K, int u, const GemvAct &A,
                                           const Cols<MB> &C, float (&acc)[MB]) {
    int w[16];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        w[4 * k] = (int)r.c[k].x; w[4 * k + 1] = (int)r.c[k].y; w[4 * k + 2] = (int)r.c[k].z; w[4 * k + 3] = (int)r.c[k].w;
    }
    const int ng = K >> 6;
#pragma unroll
    for (int m = 0; m < MB; m++) {
        const int am = C.am[m];
        if constexpr (ACT == BGL_ACT_F32) {
            ucint xg = uni(A.xw) + ((size_t)am * ng + u) * BGL_XD_DW;
            int t0 = 0, t1 = 0, t2 = 0;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                t0 = dot4(w[q], xg[q], t0); t1 = dot4(w[q], xg[16 + q], t1); t2 = dot4(w[q], xg[32 + q], t2);
            }
            acc[m] += r.s * (fold_digits(t0, t1, t2) * uni(A.xs)[(size_t)am * ng + u]);
        } else {
            ucint xq = uni(A.xw) + (size_t)am * (K >> 2) + (size_t)u * 16;
            int isum = 0;
#pragma unroll
            for (int q = 0; q < 16; q++) isum = dot4(w[q], xq[q], isum);
            acc[m] = __fadd_rn(acc[m], __fmul_rn(__fmul_rn((float)isum, r.s), uni(A.xs)[(size_t)am * ng + u]));
        }
    }
}

template <int MB, int NB>
__device__ __forceinline__ void comp_qng64(const Raw<BGL_QNG64, NB> &r, int K, int u, const GemvAct &A,
                                           const Cols<MB> &C, float (&acc)[MB]) {
    constexpr int H8 = (NB >> 3) & 1, H4 = (NB >> 2) & 1, H2 = (NB >> 1) & 1, H1 = NB & 1;
    constexpr int K4 = 8 * H8, K2 = K4 + 4 * H4, K1 = K2 + 2 * H2;
    constexpr int SH4 = 8 * H8, SH2 = SH4 + 4 * H4, SH1 = SH2 + 2 * H2;
    constexpr int CORR = 128 * H8 - (1 << (NB - 1));
    const int ng = K >> 6;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int g = 2 * u + h;
        if (g >= ng) break;
        const float s = h ? r.s.y : r.s.x;
        int f8[16], f4[16], f2[16], f1[16];
        if constexpr (H8) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                uint4 c = r.c[4 * h + k];
                f8[4 * k] = (int)c.x; f8[4 * k + 1] = (int)c.y; f8[4 * k + 2] = (int)c.z; f8[4 * k + 3] = (int)c.w;
            }
        }
        if constexpr (H4) {
#pragma unroll
            for (int k = 0; k < 2; k++) {
                uint4 c = r.c[K4 + 2 * h + k];
                uint32_t r4[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
                for (int j = 0; j < 4; j++) { f4[8 * k + 2 * j] = nib_lo(r4[j]); f4[8 * k + 2 * j + 1] = nib_hi(r4[j]); }
            }
        }
        if constexpr (H2) {
            uint4 c = r.c[K2 + h];
            uint32_t r2[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int t = 0; t < 4; t++) f2[4 * j + t] = (int)((r2[j] >> (2 * t)) & 0x03030303u);
        }
        if constexpr (H1) {
            uint4 c = r.c[K1];
            uint32_t r1[2] = {h ? c.z : c.x, h ? c.w : c.y};
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int t = 0; t < 8; t++) f1[8 * j + t] = (int)((r1[j] >> t) & 0x01010101u);
        }
#pragma unroll
        for (int m = 0; m < MB; m++) {
            const int am = C.am[m];
            ucint xg = uni(A.xw) + ((size_t)am * ng + g) * BGL_XD_DW;
            int td[3];
#pragma unroll
            for (int d = 0; d < 3; d++) {
                ucint xd = xg + 16 * d;
                int tot = 0;
                if constexpr (H8) {
                    int a = 0;
#pragma unroll
                    for (int q = 0; q < 16; q++) a = dot4(f8[q], xd[q], a);
                    tot += a;
                }
                if constexpr (H4) {
                    int a = 0;
#pragma unroll
                    for (int q = 0; q < 16; q++) a = dot4(f4[q], xd[q], a);
                    tot += a * (1 << SH4);
                }
                if constexpr (H2) {
                    int a = 0;
#pragma unroll
                    for (int q = 0; q < 16; q++) a = dot4(f2[q], xd[q], a);
                    tot += a * (1 << SH2);
                }
                if constexpr (H1) {
                    int a = 0;
#pragma unroll
                    for (int q = 0; q < 16; q++) a = dot4(f1[q], xd[q], a);
                    tot += a * (1 << SH1);
                }
                td[d] = tot;
            }
            int4 d0 = ld_dsum(A, am, K, 2 * g), d1 = ld_dsum(A, am, K, 2 * g + 1);
            td[0] += CORR * (d0.x + d1.x); td[1] += CORR * (d0.y + d1.y); td[2] += CORR * (d0.z + d1.z);
            acc[m] += s * (fold_digits(td[0], td[1], td[2]) * uni(A.xs)[(size_t)am * ng + g]);
        }
    }
}

// int4 affine (AF int4, value = nib*s + b): sum = s * sum(nib*x) + b * sum(x), both sums exact
// integers over the activation digits, so only the fold rounds.
template <int MB, int NB>
__device__ __forceinline__ void comp_q4g64a(const Raw<BGL_Q4G64A, NB> &r, int K, int u, const GemvAct &A,
                                            const Cols<MB> &C, float (&acc)[MB]) {
    int lo[8], hi[8];
    uint32_t raw[8] = {r.c[0].x, r.c[0].y, r.c[0].z, r.c[0].w, r.c[1].x, r.c[1].y, r.c[1].z, r.c[1].w};
#pragma unroll
    for (int q = 0; q < 8; q++) { lo[q] = nib_lo(raw[q]); hi[q] = nib_hi(raw[q]); }
    const int ng = K >> 6;
#pragma unroll
    for (int m = 0; m < MB; m++) {
        const int am = C.am[m];
        ucint xg = uni(A.xw) + ((size_t)am * ng + u) * BGL_XD_DW;
        int t0 = 0, t1 = 0, t2 = 0;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            t0 = dot4(lo[q], xg[2 * q], t0);      t0 = dot4(hi[q], xg[2 * q + 1], t0);
            t1 = dot4(lo[q], xg[16 + 2 * q], t1); t1 = dot4(hi[q], xg[16 + 2 * q + 1], t1);
            t2 = dot4(lo[q], xg[32 + 2 * q], t2); t2 = dot4(hi[q], xg[32 + 2 * q + 1], t2);
        }
        int4 d0 = ld_dsum(A, am, K, 2 * u), d1 = ld_dsum(A, am, K, 2 * u + 1);
        const float xs = uni(A.xs)[(size_t)am * ng + u];
        const float sx = fold_digits(d0.x + d1.x, d0.y + d1.y, d0.z + d1.z) * xs;
        acc[m] += r.s * (fold_digits(t0, t1, t2) * xs) + r.b * sx;
    }
}

// Dense fp16 / fp32 rows against the raw fp32 activation (scalar-loaded), fp32 FMA in column
// order; each 16-byte chunk is converted where it is used so few weights are live at once.
template <int FMT, int MB, int NB>
__device__ __forceinline__ void comp_dense(const Raw<FMT, NB> &r, int K, int u, const GemvAct &A, const Cols<MB> &C,
                                           float (&acc)[MB]) {
    constexpr int NCH = FMT == BGL_F16 ? 8 : 16, EPC = 64 / NCH;    // chunks per unit, elements per chunk
    float a[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) a[m] = 0.0f;
#pragma unroll
    for (int k = 0; k < NCH; k++) {
        const uint32_t v[4] = {r.c[k].x, r.c[k].y, r.c[k].z, r.c[k].w};
        float w[EPC];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if constexpr (FMT == BGL_F16) {
                w[2 * j] = __half2float(__ushort_as_half((unsigned short)(v[j] & 0xffffu)));
                w[2 * j + 1] = __half2float(__ushort_as_half((unsigned short)(v[j] >> 16)));
            } else {
                w[j] = __uint_as_float(v[j]);
            }
        }
#pragma unroll
        for (int m = 0; m < MB; m++) {
            ucfloat xr = uni(A.xf) + (size_t)C.am[m] * K + (size_t)u * 64 + k * EPC;
#pragma unroll
            for (int i = 0; i < EPC; i++) a[m] = __fmaf_rn(w[i], xr[i], a[m]);
        }
    }
#pragma unroll
    for (int m = 0; m < MB; m++) acc[m] += a[m];
}

// ======================================================================== flagged groups (cold path)
// The terms the level-0 digits leave out, for the groups of unit u flagged in some column of the
// launch: the level-1 residual s * ((V1 * 2^(e1-22)) * 2^(e-22)) and the non-finite products.  Run
// after the main loop over units whose flags are set (the unit's weights are loaded again), so the
// hot loop keeps its registers.
template <int FMT, int NB>
__device__ __forceinline__ int unit_flags(const GemvAct &A, int am, int K, int u) {
    if constexpr (FMT == BGL_QNG64) {
        const int g = 2 * u;
        return ld_xflags(A, am, K, g) | (g + 1 < (K >> 6) ? ld_xflags(A, am, K, g + 1) : 0);
    } else {
        return ld_xflags(A, am, K, u);
    }
}

template <int FMT, int NB, int MB>
__device__ __forceinline__ void comp_fix(const Raw<FMT, NB> &r, const WRow &W, int u, const GemvAct &A, const Cols<MB> &C,
                                         float (&acc)[MB]) {
    const int K = W.T->K, ng = K >> 6;
    if constexpr (FMT == BGL_Q4G64 || FMT == BGL_Q4G32H || FMT == BGL_Q4G64A) {
        int lo[8], hi[8];
        const uint32_t raw[8] = {r.c[0].x, r.c[0].y, r.c[0].z, r.c[0].w, r.c[1].x, r.c[1].y, r.c[1].z, r.c[1].w};
#pragma unroll
        for (int q = 0; q < 8; q++) { lo[q] = nib_lo(raw[q]); hi[q] = nib_hi(raw[q]); }
#pragma unroll
        for (int m = 0; m < MB; m++) {
            const int am = C.am[m];
            const size_t gi = (size_t)am * ng + u;
            const int fl = ld_xflags(A, am, K, u);
            if (!fl) continue;
            float t = 0.0f;
            if (fl & BGL_XF_L1) {
                ucint xg = uni(A.xw1) + gi * BGL_XD_DW;
                int a[3] = {0, 0, 0}, b[3] = {0, 0, 0};
#pragma unroll
                for (int d = 0; d < 3; d++) {
#pragma unroll
                    for (int q = 0; q < 4; q++) { a[d] = dot4(lo[q], xg[16 * d + 2 * q], a[d]); a[d] = dot4(hi[q], xg[16 * d + 2 * q + 1], a[d]); }
#pragma unroll
                    for (int q = 4; q < 8; q++) { b[d] = dot4(lo[q], xg[16 * d + 2 * q], b[d]); b[d] = dot4(hi[q], xg[16 * d + 2 * q + 1], b[d]); }
                }
                const int4 d0 = ld_dsum(A.xsum1, am, K, 2 * u), d1 = ld_dsum(A.xsum1, am, K, 2 * u + 1);
                const float rt = uni(A.xs1)[gi], xs = uni(A.xs)[gi];
                if constexpr (FMT == BGL_Q4G64) {
                    const float V = fold_digits(a[0] + b[0] - 8 * (d0.x + d1.x), a[1] + b[1] - 8 * (d0.y + d1.y),
                                                a[2] + b[2] - 8 * (d0.z + d1.z));
                    t = r.s * ((V * rt) * xs);
                } else if constexpr (FMT == BGL_Q4G32H) {
                    const float sa = __half2float(__ushort_as_half((unsigned short)(r.s & 0xffffu)));
                    const float sb = __half2float(__ushort_as_half((unsigned short)(r.s >> 16)));
                    const float Va = fold_digits(a[0] - 8 * d0.x, a[1] - 8 * d0.y, a[2] - 8 * d0.z);
                    const float Vb = fold_digits(b[0] - 8 * d1.x, b[1] - 8 * d1.y, b[2] - 8 * d1.z);
                    t = sa * ((Va * rt) * xs) + sb * ((Vb * rt) * xs);
                } else {                                         // affine: s * sum(nib X1) + b * sum(X1)
                    const float V = fold_digits(a[0] + b[0], a[1] + b[1], a[2] + b[2]);
                    const float sx = fold_digits(d0.x + d1.x, d0.y + d1.y, d0.z + d1.z);
                    t = r.s * ((V * rt) * xs) + r.b * ((sx * rt) * xs);
                }
            }
            if (fl & BGL_XF_NF) t += x_nonfinite<FMT, NB>(*W.T, W.row, u, A.xf + (size_t)am * K);
            acc[m] += t;
        }
    } else if constexpr (FMT == BGL_Q8G64) {
        int w[16];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            w[4 * k] = (int)r.c[k].x; w[4 * k + 1] = (int)r.c[k].y; w[4 * k + 2] = (int)r.c[k].z; w[4 * k + 3] = (int)r.c[k].w;
        }
#pragma unroll
        for (int m = 0; m < MB; m++) {
            const int am = C.am[m];
            const size_t gi = (size_t)am * ng + u;
            const int fl = ld_xflags(A, am, K, u);
            if (!fl) continue;
            float t = 0.0f;
            if (fl & BGL_XF_L1) {
                ucint xg = uni(A.xw1) + gi * BGL_XD_DW;
                int t0 = 0, t1 = 0, t2 = 0;
#pragma unroll
                for (int q = 0; q < 16; q++) {
                    t0 = dot4(w[q], xg[q], t0); t1 = dot4(w[q], xg[16 + q], t1); t2 = dot4(w[q], xg[32 + q], t2);
                }
                t = r.s * ((fold_digits(t0, t1, t2) * uni(A.xs1)[gi]) * uni(A.xs)[gi]);
            }
            if (fl & BGL_XF_NF) t += x_nonfinite<FMT, NB>(*W.T, W.row, u, A.xf + (size_t)am * K);
            acc[m] += t;
        }
    } else if constexpr (FMT == BGL_QNG64) {
        // per element: the row's code (read from the tiled layout) times each level-1 digit (cold path)
#pragma unroll 1
        for (int h = 0; h < 2; h++) {
            const int g = 2 * u + h;
            if (g >= ng) break;
            const float s = h ? r.s.y : r.s.x;
#pragma unroll
            for (int m = 0; m < MB; m++) {
                const int am = C.am[m];
                const size_t gi = (size_t)am * ng + g;
                const int fl = ld_xflags(A, am, K, g);
                if (!fl) continue;
                float t = 0.0f;
                if (fl & BGL_XF_L1) {
                    ucint xg = uni(A.xw1) + gi * BGL_XD_DW;
                    int td[3] = {0, 0, 0};
#pragma unroll 1
                    for (int j = 0; j < 64; j++) {
                        const int code = (int)qng_u_at(*W.T, W.row, g * 64 + j) - (1 << (NB - 1));
#pragma unroll
                        for (int d = 0; d < 3; d++) td[d] += code * (int)(int8_t)(xg[16 * d + (j >> 2)] >> (8 * (j & 3)));
                    }
                    t = s * ((fold_digits(td[0], td[1], td[2]) * uni(A.xs1)[gi]) * uni(A.xs)[gi]);
                }
                if (fl & BGL_XF_NF) t += x_nonfinite<FMT, NB>(*W.T, W.row, g, A.xf + (size_t)am * K);
                acc[m] += t;
            }
        }
    }
}

template <int FMT, int ACT, int NB, int MB>
__device__ __forceinline__ void comp_dispatch(const Raw<FMT, NB> &r, int K, int u, const GemvAct &A,
                                              const Cols<MB> &C, float (&acc)[MB]) {
    if constexpr (FMT == BGL_Q4G64) comp_q4g64<ACT, MB, NB>(r, K, u, A, C, acc);
    else if constexpr (FMT == BGL_Q4G32H) comp_q4g32h<MB, NB>(r, K, u, A, C, acc);
    else if constexpr (FMT == BGL_Q4G256SF) comp_g256sf<MB, NB>(r, K, u, A, C, acc);
    else if constexpr (FMT == BGL_Q8G64) comp_q8g64<ACT, MB, NB>(r, K, u, A, C, acc);
    else if constexpr (FMT == BGL_Q4G64A) comp_q4g64a<MB, NB>(r, K, u, A, C, acc);
    else if constexpr (FMT == BGL_F16 || FMT == BGL_F32) comp_dense<FMT, MB, NB>(r, K, u, A, C, acc);
    else comp_qng64<MB, NB>(r, K, u, A, C, acc);
}

