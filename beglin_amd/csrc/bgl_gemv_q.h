// bgl_gemv_q.h -- building blocks of the W4A8 kernels that quantize their fp32 activations
// themselves (k_gemv_q in bgl_gemv.hip, k_mlp_q in bgl_mlp_q.hip): the reference's activation
// quantizer in passes of 256 values into LDS, a lane's share of a weight unit, its exact integer
// dot product against the int8 codes, and the reference's per-group fp32 term.
#pragma once
#include "bgl_gemv_impl.h"

// ================================================================================== path B kernel (W4A8, fused quantization)
// A workgroup owns TR rows (a 1/(64/TR) slice of a 64-row tile) and the whole K range.  Lane l of a
// wave handles row l % TR and unit kq = l / TR of each group of KQ = 64/TR consecutive units, so a
// wave-wide load is KQ runs of TR*16 >= 128 bytes.  Activation bytes come from LDS (each lane reads
// its own unit's slice; units are padded by 16 bytes so neighbouring units fall in different banks).
//
// The activations are quantized in passes of 256 consecutive values, lane l holding values 4l..4l+3
// (one float4 load, one packed dword store): a pass is one g256 group (wave-wide max) or four g64
// groups (one per 16-lane row, row-wide max and sum).  A wave's first QP passes are loaded before its
// first weight units and the quantization is branch-free, so it waits only for the x loads (vector
// memory loads retire in order) and runs while the weight bytes are still arriving.  Lanes past K
// store into a dummy slot after the real ones.
// Dynamic LDS: [xq: (U+1) x (unit bytes + 16)][ascale: K/gq + 1][xqsum: K/64 + 1][t: U x TR floats].

template <int FMT> struct QUnit {
    static constexpr int GQ = FMT == BGL_Q4G256SF ? 256 : 64;        // activation quantization group
    static constexpr int ELEMS = FMT == BGL_Q4G256SF ? 256 : 64;     // elements per work unit
    static constexpr int STRIDE = ELEMS + 16;                       // padded LDS bytes per unit
    static constexpr bool XSUM = FMT == BGL_Q4G64;                  // unsigned nibbles: needs sum(xq) per 64
};

// A lane's share of one work unit: H lanes (lane l and its partner l ^ TR when H == 2) split the
// unit's chunks, part h holding chunks [h*CP, (h+1)*CP).  Partners read the same scale words.
template <int FMT, int H> struct RawPart {
    static constexpr int CP = chunks_per_unit<FMT>(0) / H;
    uint4 c[CP];
    float s;
    uint32_t sub;             // g256sf: this part's sub-codes, from the low byte up
};

template <int FMT, int H>
__device__ __forceinline__ void load_part(RawPart<FMT, H> &r, const BglDevTensor &T, int tile, int rr, int u, int h) {
    constexpr int CPU = chunks_per_unit<FMT>(0), CP = CPU / H;
    // global address space: flat loads would also count against the LDS wait counter
    const BGL_GLOBAL bgl_u32x4 *cp =
        (const BGL_GLOBAL bgl_u32x4 *)(T.w) + ((size_t)tile * T.cpr + (size_t)u * CPU + h * CP) * BGL_TILE + rr;
#pragma unroll
    for (int k = 0; k < CP; k++) {
        const bgl_u32x4 v = cp[k * BGL_TILE];
        r.c[k] = make_uint4(v.x, v.y, v.z, v.w);
    }
    const size_t so = ((size_t)tile * T.nunits + u) * BGL_TILE + rr;
    if constexpr (FMT == BGL_Q4G256SF) {
        const bgl_u32x2 w = ((const BGL_GLOBAL bgl_u32x2 *)T.s0)[so];
        r.s = __uint_as_float(w.x);
        r.sub = w.y >> (h * 8 * (4 / H));
    } else {
        r.s = ((const BGL_GLOBAL float *)T.s0)[so];
    }
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) { return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false); }
__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint32_t abs_bits(float x) { return __float_as_uint(x) & 0x7fffffffu; }

// q4_quant_act_i8's rounding (q4gemv.h:199-206): q = (int)(x*inv + (x*inv >= 0 ? 0.5 : -0.5)),
// clamped to [-128, 127].  copysign(0.5, p) differs from the comparison only at p = -0, where both
// truncate to 0.  nf: the group's |x| maximum is NaN or +-Inf, where the reference's FMAX carries it
// into mx and every code comes out 0 (FCVTZS maps the NaN products to 0, inv = 0 makes the finite
// ones +-0), so the product is replaced by 0.
__device__ __forceinline__ uint32_t quant_byte(float x, float inv, bool nf) {
    const float p = nf ? 0.0f : __fmul_rn(x, inv);
    int q = (int)__fadd_rn(p, __builtin_copysignf(0.5f, p));   // |.| <= 128.5: no int32 overflow
    q = q > 127 ? 127 : (q < -128 ? -128 : q);
    return (uint32_t)q & 255u;
}

// Quantizes QP passes into LDS.  The MB columns of a launch are one run of passes: pass p is values
// 256*(p % NP) .. +255 of column p / NP (NP passes per column, NPT = MB*NP in all); pass i of the
// call is pp[i], lane l holding values 4l..4l+3 of it in v[i].  The passes are processed in
// lockstep so their dependency chains interleave.  Column m's operands live at xq + m*XQS,
// asc + m*(NGQ+1), xsum + m*(K/64+1); passes past NPT and lanes past K store into each region's dummy
// slot.  |x| is maximised on its bit pattern (the same order as the float values for non-NaN inputs).
// GQ=256: one pass is one group; its four row maxima are combined with readlane, and one IEEE
// division pair serves every pass (lane i computes pass i's scale and reciprocal).  GQ=64: one pass
// is four groups, one per 16-lane row.
template <int FMT, int QP, int MB>
__device__ __forceinline__ void quant_passes_at(const float4 (&v)[QP], const int (&pp)[QP], int K, int NP, int NPT, int NGQ,
                                                int U, int lane, int8_t *xq, float *asc, int *xsum) {
    using QU = QUnit<FMT>;
    const int XQS = (U + 1) * QU::STRIDE;
    uint32_t m[QP];
#pragma unroll
    for (int i = 0; i < QP; i++)
        m[i] = umax(umax(abs_bits(v[i].x), abs_bits(v[i].y)), umax(abs_bits(v[i].z), abs_bits(v[i].w)));
#pragma unroll
    for (int i = 0; i < QP; i++) m[i] = umax(m[i], dpp_u<0xB1>(m[i]));
#pragma unroll
    for (int i = 0; i < QP; i++) m[i] = umax(m[i], dpp_u<0x4E>(m[i]));
#pragma unroll
    for (int i = 0; i < QP; i++) m[i] = umax(m[i], dpp_u<0x141>(m[i]));
#pragma unroll
    for (int i = 0; i < QP; i++) m[i] = umax(m[i], dpp_u<0x140>(m[i]));   // row maxima in every lane
    // pass i: column col[i] (clamped), value offset e[i] within the column, whether it is real
    int col[QP], e[QP];
    bool ok[QP];
#pragma unroll
    for (int i = 0; i < QP; i++) {
        const int p = pp[i];
        if constexpr (MB == 1) {                       // one column: passes past K land past K
            col[i] = 0;
            e[i] = 256 * p + 4 * lane;
            ok[i] = e[i] < K;
        } else {
            const int pc = p < NPT ? p : NPT - 1;
            col[i] = pc / NP;
            e[i] = 256 * (pc - col[i] * NP) + 4 * lane;
            ok[i] = p < NPT && e[i] < K;               // K % 64 == 0: whole 16-lane rows are in or out
        }
    }
    float inv[QP];
    bool nf[QP];                                       // the pass's group maximum is NaN or +-Inf
    if constexpr (QU::GQ == 256) {
        uint32_t mb = 0u;
#pragma unroll
        for (int i = 0; i < QP; i++) {
            const uint32_t M = umax(umax((uint32_t)__builtin_amdgcn_readlane((int)m[i], 0), (uint32_t)__builtin_amdgcn_readlane((int)m[i], 16)),
                                    umax((uint32_t)__builtin_amdgcn_readlane((int)m[i], 32), (uint32_t)__builtin_amdgcn_readlane((int)m[i], 48)));
            mb = (i == 0 || lane == i) ? M : mb;
            nf[i] = M >= 0x7f800000u;
        }
        // mx starts at 1e-8 (q4gemv_g256.h:78); on bit patterns a NaN stays NaN, as FMAX keeps it
        const float mx = __uint_as_float(umax(mb, __float_as_uint(1e-8f)));
        const float sc = __fdiv_rn(mx, 127.0f), iv = __fdiv_rn(1.0f, sc);
#pragma unroll
        for (int i = 0; i < QP; i++) inv[i] = rlane_f(iv, i);
        if (lane < QP) {
            int p = pp[0];
#pragma unroll
            for (int i = 1; i < QP; i++) p = lane == i ? pp[i] : p;
            if constexpr (MB == 1) {
                asc[256 * p < K ? p : NGQ] = sc;
            } else {
                const int pc = p < NPT ? p : NPT - 1, cm = pc / NP, pp = pc - cm * NP;
                asc[cm * (NGQ + 1) + (p < NPT && 256 * pp < K ? pp : NGQ)] = sc;
            }
        }
    } else {
        float sc[QP];
#pragma unroll
        for (int i = 0; i < QP; i++) {                 // mx starts at 1e-8 (q4gemv.h:182); NaN bits stay NaN
            sc[i] = __fdiv_rn(__uint_as_float(umax(m[i], __float_as_uint(1e-8f))), 127.0f);
            nf[i] = m[i] >= 0x7f800000u;
        }
#pragma unroll
        for (int i = 0; i < QP; i++) inv[i] = __fdiv_rn(1.0f, sc[i]);
        if ((lane & 15) == 0) {
#pragma unroll
            for (int i = 0; i < QP; i++) asc[col[i] * (NGQ + 1) + (ok[i] ? e[i] / 64 : NGQ)] = sc[i];
        }
    }
    uint32_t word[QP];
#pragma unroll
    for (int i = 0; i < QP; i++)
        word[i] = quant_byte(v[i].x, inv[i], nf[i]) | (quant_byte(v[i].y, inv[i], nf[i]) << 8) |
                  (quant_byte(v[i].z, inv[i], nf[i]) << 16) | (quant_byte(v[i].w, inv[i], nf[i]) << 24);
#pragma unroll
    for (int i = 0; i < QP; i++)
        *reinterpret_cast<uint32_t *>(xq + col[i] * XQS + (ok[i] ? e[i] / QU::ELEMS : U) * QU::STRIDE + e[i] % QU::ELEMS) = word[i];
    if constexpr (QU::XSUM) {
        int sm[QP];
#pragma unroll
        for (int i = 0; i < QP; i++) {
            const uint32_t w = word[i];
            sm[i] = (int)(int8_t)(w & 255u) + (int)(int8_t)((w >> 8) & 255u) + (int)(int8_t)((w >> 16) & 255u) + (int)(int8_t)(w >> 24);
        }
#pragma unroll
        for (int i = 0; i < QP; i++) sm[i] = row_sum_i32(sm[i]);
        if ((lane & 15) == 0) {
#pragma unroll
            for (int i = 0; i < QP; i++) xsum[col[i] * (K / 64 + 1) + (ok[i] ? e[i] / 64 : K / 64)] = sm[i];
        }
    }
}

// passes p0, p0 + nw, p0 + 2 nw, ...
template <int FMT, int QP, int MB>
__device__ __forceinline__ void quant_passes(const float4 (&v)[QP], int p0, int nw, int K, int NP, int NPT, int NGQ, int U,
                                             int lane, int8_t *xq, float *asc, int *xsum) {
    int pp[QP];
#pragma unroll
    for (int i = 0; i < QP; i++) pp[i] = p0 + i * nw;
    quant_passes_at<FMT, QP, MB>(v, pp, K, NP, NPT, NGQ, U, lane, xq, asc, xsum);
}

// x values of QP passes (see quant_passes); addresses are clamped, so every load is valid.
template <int QP, int MB>
__device__ __forceinline__ void load_xpass(float4 (&v)[QP], const float *x, int p0, int nw, int K, int NP, int NPT, int lane) {
#pragma unroll
    for (int i = 0; i < QP; i++) {
        const float *xp;
        if constexpr (MB == 1) {
            xp = x + min(256 * (p0 + i * nw) + 4 * lane, K - 4);
        } else {
            const int p = min(p0 + i * nw, NPT - 1), cm = p / NP;
            xp = x + (size_t)cm * K + min(256 * (p - cm * NP) + 4 * lane, K - 4);
        }
        const bgl_f32x4 t = *((const BGL_GLOBAL bgl_f32x4 *)xp);
        v[i] = make_float4(t.x, t.y, t.z, t.w);
    }
}

// g256sf codes are stored as signed nibbles (code ^ 8 = the 4-bit two's complement of code-8), so
// masking a nibble into the high half of a byte gives 16*(code-8) as an int8 and dot4 sums come out
// as exactly 16x the reference's integer sums.
__device__ __forceinline__ int snib_lo16(uint32_t w) { return (int)((w << 4) & 0xF0F0F0F0u); }
__device__ __forceinline__ int snib_hi16(uint32_t w) { return (int)(w & 0xF0F0F0F0u); }

// The exact integer part of a unit's dot product over this lane's chunks (partners' parts add up
// to the reference's integer sum): g256sf 16 * sum_sg isum_sg * sub_sg over its sub-groups, |.| < 2^29;
// q4g64 sum code*xq (the -8*sum(xq) term is applied once, in unit_float); q8g64 sum code*xq.
template <int FMT, int H>
__device__ __forceinline__ int unit_part(const RawPart<FMT, H> &r, const int8_t *xq, int u, int h) {
    constexpr int CP = RawPart<FMT, H>::CP;
    const int4 *x4 = reinterpret_cast<const int4 *>(xq + (size_t)u * QUnit<FMT>::STRIDE);
    if constexpr (FMT == BGL_Q4G256SF) {
        x4 += h * CP * 2;                              // 32 activation bytes per chunk
        int comb16 = 0;
#pragma unroll
        for (int sg = 0; sg < CP / 2; sg++) {
            int ia = 0, ib = 0;                        // two independent dot chains; exact int32 sums
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const uint4 c = r.c[2 * sg + k];
                const int4 xa = x4[sg * 4 + 2 * k], xb = x4[sg * 4 + 2 * k + 1];
                ia = dot4(snib_lo16(c.x), xa.x, ia); ib = dot4(snib_hi16(c.x), xa.y, ib);
                ia = dot4(snib_lo16(c.y), xa.z, ia); ib = dot4(snib_hi16(c.y), xa.w, ib);
                ia = dot4(snib_lo16(c.z), xb.x, ia); ib = dot4(snib_hi16(c.z), xb.y, ib);
                ia = dot4(snib_lo16(c.w), xb.z, ia); ib = dot4(snib_hi16(c.w), xb.w, ib);
            }
            comb16 += (ia + ib) * (int)((r.sub >> (8 * sg)) & 255u);
        }
        return comb16;
    } else if constexpr (FMT == BGL_Q4G64) {
        x4 += h * CP * 2;
        int isum = 0;
#pragma unroll
        for (int k = 0; k < CP; k++) {
            const uint4 c = r.c[k];
            const int4 xa = x4[2 * k], xb = x4[2 * k + 1];
            isum = dot4(nib_lo(c.x), xa.x, isum); isum = dot4(nib_hi(c.x), xa.y, isum);
            isum = dot4(nib_lo(c.y), xa.z, isum); isum = dot4(nib_hi(c.y), xa.w, isum);
            isum = dot4(nib_lo(c.z), xb.x, isum); isum = dot4(nib_hi(c.z), xb.y, isum);
            isum = dot4(nib_lo(c.w), xb.z, isum); isum = dot4(nib_hi(c.w), xb.w, isum);
        }
        return isum;
    } else {
        x4 += h * CP;                                  // 16 activation bytes per chunk
        int isum = 0;
#pragma unroll
        for (int k = 0; k < CP; k++) {
            const uint4 c = r.c[k];
            const int4 xa = x4[k];
            isum = dot4((int)c.x, xa.x, isum); isum = dot4((int)c.y, xa.y, isum);
            isum = dot4((int)c.z, xa.z, isum); isum = dot4((int)c.w, xa.w, isum);
        }
        return isum;
    }
}

// The unit's fp32 term, exactly the reference's per-group expression (q4gemv_g256.h:154,
// q4gemv.h:241): g256sf ((comb * wsuper) * (1/63)) * ascale -- plain g256 (q4gemv_g256.h:125) has
// sub-codes 1 and gm = 1, an exact multiply, so (isum * wscale) * ascale; q4g64 / q8g64
// (isum * wscale) * ascale.
template <int FMT>
__device__ __forceinline__ float unit_float(int isum, float s, float gm, const float *asc, const int *xsum, int u) {
    if constexpr (FMT == BGL_Q4G256SF) return __fmul_rn(__fmul_rn(__fmul_rn((float)(isum >> 4), s), gm), asc[u]);
    else if constexpr (FMT == BGL_Q4G64) return __fmul_rn(__fmul_rn((float)(isum - 8 * xsum[u]), s), asc[u]);
    else return __fmul_rn(__fmul_rn((float)isum, s), asc[u]);
}
