// bgl_gemv_x.h -- device building blocks of the fp32-activation GEMVs over LDS activation records
// (k_gemv_x in bgl_gemv_x.hip, k_moe_x in bgl_moe_x.hip): per-format weight loads through buffer
// resources, the decode of a lane's 64-group, its exact integer dot products against a record and
// the fp32 fold, and the in-kernel making of the records from raw fp32 values.
//
// A record (one per 64-group and activation column, 240 bytes in LDS): the three balanced int8
// digits of X = rint(x * 2^(22-e)) (e = exponent of the group's largest finite |x|) as 48 dwords,
// the digit sums of the two 32-element halves (the first half's 4th int holds the group's BGL_XF_*
// flags), the scale 2^(e-22) and the level-1 ratio 2^(e1-22) -- k_act_x24's operands
// (bgl_prep.hip), so every product is an exact int32 dot4 sum and fp32 only enters in the
// per-group fold.  A group flagged BGL_XF_L1 also has a level-1 record (the residual's digits and
// sums) at a fixed dword offset l1 from its level-0 record; its ratio is 0 otherwise, so a level-1
// fold over a stale record adds exactly 0.  The 60-dword stride puts the <= 8 records one read
// touches in disjoint banks.
//
// qNg64 bit planes: the 8-bit field (stored as f ^ 0x80, a signed byte f - 128) is one dot4
// operand; the 4-, 2- and 1-bit fields of an element are merged into one byte (their values sit at
// bit 0, 4*has4 and 4*has4 + 2*has2 of it, < 128) with one shift and one v_and_or per field, so a
// group costs two dot4 operands per digit instead of one per field.
#pragma once
#include "bgl_gemv_impl.h"

#define XREC_DW 60            // LDS dwords per 64-group record
#define XREC_DSUM 48          // digit sums of the two halves: [half][digit 0..2, flags / pad]
#define XREC_SCALE 56         // 2^(e-22), then the level-1 ratio 2^(e1-22)
#define X_PRE 4               // record pieces (16 bytes) per thread loaded ahead of the weights

// (a & m) | o in one v_and_or_b32 (gfx9's three-operand encoding takes no literal constant and
// reads at most one scalar register: m in a scalar register, o in a vector register).
__device__ __forceinline__ uint32_t x_and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(o));
    return r;
}

// A lane's weights for one 64-group.
template <int FMT, int NB> struct XRaw;
template <int NB> struct XRaw<BGL_Q4G64, NB> { uint4 c[2]; float s; };
template <int NB> struct XRaw<BGL_Q4G32H, NB> { uint4 c[2]; uint32_t s; };
template <int NB> struct XRaw<BGL_MXFP4, NB> { uint4 c[2]; uint32_t s; };
template <int NB> struct XRaw<BGL_Q8G64, NB> { uint4 c[4]; float s; };
template <int NB> struct XRaw<BGL_QNG64, NB> {
    static constexpr int H8 = (NB >> 3) & 1, H4 = (NB >> 2) & 1, H2 = (NB >> 1) & 1, H1 = NB & 1;
    uint4 p8[H8 ? 4 : 1], p4[H4 ? 2 : 1], p2;
    uint2 p1;
    float s;
};

// Buffer resources over a tensor's chunks and its per-unit scales, and an empty one: every load
// through it returns zeros without touching memory.  A wave issues the loads of slots it does not
// have through the empty resource, so every load is unconditional and each wait counts exactly the
// loads issued after the one it needs.  Offsets: a lane-constant part in a vector register, the
// slot's part in a scalar one.
#define X_RSRC_W3 0x00020000  // buffer resource word 3 on gfx9: 32-bit data format, raw addressing
#define X_OOB 0x80000000u     // a lane offset past any resource (resources are < 2^31 bytes)
typedef unsigned int x_u32x2 __attribute__((ext_vector_type(2)));
template <int FMT> constexpr int x_scale_bytes() { return FMT == BGL_QNG64 ? 8 : 4; }
struct XRes {
    __amdgpu_buffer_rsrc_t w, s, z;
    uint32_t wtile, stile;    // byte offsets of this workgroup's tile in w and s
};
template <int FMT>
__device__ __forceinline__ XRes x_res(const BglDevTensor &T, int tile) {
    XRes r;
    const uint32_t wb = (uint32_t)T.ntiles * (uint32_t)T.cpr * 1024u;
    const uint32_t sb = (uint32_t)T.ntiles * (uint32_t)T.nunits * 64u * x_scale_bytes<FMT>();
    r.w = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(T.w), (short)0, (int)wb, X_RSRC_W3);
    r.s = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(T.s0), (short)0, (int)sb, X_RSRC_W3);
    r.z = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(T.w), (short)0, 0, X_RSRC_W3);
    r.wtile = (uint32_t)tile * (uint32_t)T.cpr * 1024u;
    r.stile = (uint32_t)tile * (uint32_t)T.nunits * 64u * x_scale_bytes<FMT>();
    return r;
}

// Lane-constant byte offsets of a lane's group inside a slot: row rr, group kq of the slot's KQ.
// qNg64 units are pairs of groups: with KQ >= 2 the lane's half h = kq & 1 is fixed, with KQ == 1
// it alternates with the slot (and goes into the slot's scalar offset).
template <int NB> struct XPlanes {
    static constexpr int H8 = (NB >> 3) & 1, H4 = (NB >> 2) & 1, H2 = (NB >> 1) & 1;
    static constexpr int K4 = 8 * H8, K2 = K4 + 4 * H4, K1 = K2 + 2 * H2;
};
struct XLane {
    uint32_t p8, p4, p2, p1, s;   // qNg64 fields (p8 is the chunk base of the other formats)
};
template <int FMT, int NB, int KQ>
__device__ __forceinline__ XLane x_lane(int rr, int kq) {
    constexpr int CPU = chunks_per_unit<FMT>(NB);
    XLane l;
    if constexpr (FMT == BGL_QNG64) {
        using P = XPlanes<NB>;
        const uint32_t ub = KQ >= 2 ? (uint32_t)kq >> 1 : 0u, h = KQ >= 2 ? (uint32_t)kq & 1u : 0u;
        const uint32_t base = ub * CPU * 1024u + (uint32_t)rr * 16u;
        l.p8 = base + 4096u * h;
        l.p4 = base + 2048u * h + P::K4 * 1024u;
        l.p2 = base + 1024u * h + P::K2 * 1024u;
        l.p1 = base + 8u * h + P::K1 * 1024u;
        l.s = (ub * 64u + (uint32_t)rr) * 8u + 4u * h;
    } else {
        l.p8 = (uint32_t)kq * CPU * 1024u + (uint32_t)rr * 16u;
        l.p4 = l.p2 = l.p1 = 0u;
        l.s = ((uint32_t)kq * 64u + (uint32_t)rr) * 4u;
    }
    return l;
}

// Slot sl's weights (zeros when !ok).
template <int FMT, int NB, int KQ>
__device__ __forceinline__ void x_load(XRaw<FMT, NB> &r, const XRes &R, const XLane &l, int sl, bool ok) {
    constexpr int CPU = chunks_per_unit<FMT>(NB);
    const __amdgpu_buffer_rsrc_t W = ok ? R.w : R.z, S = ok ? R.s : R.z;
    auto ld = [&](uint32_t lane_off, uint32_t soff) {
        const bgl_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(W, lane_off, soff, 0);
        return make_uint4(v.x, v.y, v.z, v.w);
    };
    uint32_t sv;
    if constexpr (FMT == BGL_QNG64) {
        using X = XRaw<FMT, NB>;
        const uint32_t su = KQ >= 2 ? (uint32_t)sl * (KQ / 2) : (uint32_t)sl >> 1;   // first unit of the slot
        const uint32_t hh = KQ >= 2 ? 0u : (uint32_t)sl & 1u;                        // KQ == 1: the slot's half
        const uint32_t wo = R.wtile + su * CPU * 1024u;
        if constexpr (X::H8) {
#pragma unroll
            for (int k = 0; k < 4; k++) r.p8[k] = ld(l.p8, wo + 4096u * hh + 1024u * k);
        }
        if constexpr (X::H4) {
#pragma unroll
            for (int k = 0; k < 2; k++) r.p4[k] = ld(l.p4, wo + 2048u * hh + 1024u * k);
        }
        if constexpr (X::H2) r.p2 = ld(l.p2, wo + 1024u * hh);
        if constexpr (X::H1) {
            const x_u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(W, l.p1, wo + 8u * hh, 0);
            r.p1 = make_uint2(v.x, v.y);
        }
        sv = __builtin_amdgcn_raw_buffer_load_b32(S, l.s, R.stile + su * 512u + 4u * hh, 0);
    } else {
        const uint32_t su = (uint32_t)sl * KQ;
        const uint32_t wo = R.wtile + su * CPU * 1024u;
#pragma unroll
        for (int k = 0; k < CPU; k++) r.c[k] = ld(l.p8, wo + 1024u * k);
        sv = __builtin_amdgcn_raw_buffer_load_b32(S, l.s, R.stile + su * 256u, 0);
    }
    if constexpr (FMT == BGL_Q4G32H || FMT == BGL_MXFP4) r.s = sv;
    else r.s = __uint_as_float(sv);
}

// Slots a wave keeps in flight: as many as fit beside the decode registers.
template <int FMT, int NB> constexpr int x_depth() {
    return FMT == BGL_QNG64 ? (NB <= 4 ? 4 : NB <= 8 ? 3 : 2) : FMT == BGL_Q8G64 ? 3 : 4;
}

// Digit d of the group record as 16 dwords (element 4q..4q+3 in dword q).
struct XDig {
    int v[16];
};
__device__ __forceinline__ XDig x_digit(const int *rec, int d) {
    XDig x;
    const int4 *p = reinterpret_cast<const int4 *>(rec + 16 * d);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int4 t = p[k];
        x.v[4 * k] = t.x; x.v[4 * k + 1] = t.y; x.v[4 * k + 2] = t.z; x.v[4 * k + 3] = t.w;
    }
    return x;
}

// A lane's 64-group decoded into dot4 operands (element 4q..4q+3 in dword q) and its scales.
template <int FMT, int NB> struct XDec;
template <int NB> struct XDec<BGL_Q4G64, NB> { int lo[8], hi[8]; float s; };
template <int NB> struct XDec<BGL_Q4G32H, NB> { int lo[8], hi[8]; float sa, sb; };
template <int NB> struct XDec<BGL_MXFP4, NB> { int lo[8], hi[8]; float sa, sb; };   // codes as signed int8
template <int NB> struct XDec<BGL_Q8G64, NB> { int w[16]; float s; };
template <int NB> struct XDec<BGL_QNG64, NB> {
    static constexpr int H8 = (NB >> 3) & 1, H4 = (NB >> 2) & 1, H2 = (NB >> 1) & 1, H1 = NB & 1;
    static constexpr bool HI = H4 || H2 || H1;       // fields merged into the second operand
    int lo[H8 ? 16 : 1], hi[HI ? 16 : 1];
    float s;
};

template <int FMT, int NB>
__device__ __forceinline__ XDec<FMT, NB> x_decode(const XRaw<FMT, NB> &r) {
    XDec<FMT, NB> d;
    if constexpr (FMT == BGL_MXFP4) {
        const uint32_t raw[8] = {r.c[0].x, r.c[0].y, r.c[0].z, r.c[0].w, r.c[1].x, r.c[1].y, r.c[1].z, r.c[1].w};
#pragma unroll
        for (int q = 0; q < 8; q++) { d.lo[q] = mx_codes((uint32_t)nib_lo(raw[q])); d.hi[q] = mx_codes((uint32_t)nib_hi(raw[q])); }
        d.sa = mx_scale(r.s & 255u);
        d.sb = mx_scale((r.s >> 8) & 255u);
    } else if constexpr (FMT == BGL_Q4G64 || FMT == BGL_Q4G32H) {
        const uint32_t raw[8] = {r.c[0].x, r.c[0].y, r.c[0].z, r.c[0].w, r.c[1].x, r.c[1].y, r.c[1].z, r.c[1].w};
#pragma unroll
        for (int q = 0; q < 8; q++) { d.lo[q] = nib_lo(raw[q]); d.hi[q] = nib_hi(raw[q]); }
        if constexpr (FMT == BGL_Q4G64) d.s = r.s;
        else {
            d.sa = __half2float(__ushort_as_half((unsigned short)(r.s & 0xffffu)));
            d.sb = __half2float(__ushort_as_half((unsigned short)(r.s >> 16)));
        }
    } else if constexpr (FMT == BGL_Q8G64) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            d.w[4 * k] = (int)r.c[k].x; d.w[4 * k + 1] = (int)r.c[k].y; d.w[4 * k + 2] = (int)r.c[k].z; d.w[4 * k + 3] = (int)r.c[k].w;
        }
        d.s = r.s;
    } else {
        using X = XDec<FMT, NB>;
        constexpr int H8 = X::H8, H4 = X::H4, H2 = X::H2, H1 = X::H1;
        constexpr int S2 = 4 * H4, S1 = 4 * H4 + 2 * H2;     // bit offsets of the 2- and 1-bit fields in the merged byte
        if constexpr (H8) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                d.lo[4 * k] = (int)r.p8[k].x; d.lo[4 * k + 1] = (int)r.p8[k].y; d.lo[4 * k + 2] = (int)r.p8[k].z; d.lo[4 * k + 3] = (int)r.p8[k].w;
            }
        }
        if constexpr (X::HI) {
#pragma unroll
            for (int q = 0; q < 16; q++) {
                uint32_t h = 0;
                if constexpr (H4) {
                    // element 4q+i's 4-bit field: chunk q/8, dword (q/2)%4, byte i, low nibble for even q
                    const uint4 &c = r.p4[q >> 3];
                    const uint32_t w = ((q >> 1) & 3) == 0 ? c.x : ((q >> 1) & 3) == 1 ? c.y : ((q >> 1) & 3) == 2 ? c.z : c.w;
                    h = ((q & 1) ? w >> 4 : w) & 0x0F0F0F0Fu;
                }
                if constexpr (H2) {
                    // element 4q+i's 2-bit field: dword q/4, byte i, bits 2(q%4)..+1
                    const uint32_t w = (q >> 2) == 0 ? r.p2.x : (q >> 2) == 1 ? r.p2.y : (q >> 2) == 2 ? r.p2.z : r.p2.w;
                    const int sh = 2 * (q & 3) - S2;
                    const uint32_t v = sh >= 0 ? w >> sh : w << -sh;
                    h = H4 ? x_and_or(v, 0x03030303u << S2, h) : (v & (0x03030303u << S2));
                }
                if constexpr (H1) {
                    // element 4q+i's 1-bit field: dword q/8, byte i, bit q%8
                    const uint32_t w = (q >> 3) ? r.p1.y : r.p1.x;
                    const int sh = (q & 7) - S1;
                    const uint32_t v = sh >= 0 ? w >> sh : w << -sh;
                    h = (H4 || H2) ? x_and_or(v, 0x01010101u << S1, h) : (v & (0x01010101u << S1));
                }
                d.hi[q] = (int)h;
            }
        }
        d.s = r.s;
    }
    return d;
}

// The exact integer dot products of a lane's decoded group with one record's digits, bias
// corrections included: o[0..2] per digit (Q4G32H: the first half; o[3..5] the second).
template <int FMT, int NB>
__device__ __forceinline__ void x_ints(const XDec<FMT, NB> &w, const int *rec, const int4 &ds0, const int4 &ds1, int (&o)[6]) {
    // cold path only: one digit at a time (unrolled, the three digits' LDS reads are hoisted together)
    if constexpr (FMT == BGL_Q4G64 || FMT == BGL_Q4G32H || FMT == BGL_MXFP4) {
        int ta[3], tb[3];
#pragma unroll 1
        for (int d = 0; d < 3; d++) {
            const XDig x = x_digit(rec, d);
            int a = 0, b = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) { a = dot4(w.lo[q], x.v[2 * q], a); a = dot4(w.hi[q], x.v[2 * q + 1], a); }
#pragma unroll
            for (int q = 4; q < 8; q++) { b = dot4(w.lo[q], x.v[2 * q], b); b = dot4(w.hi[q], x.v[2 * q + 1], b); }
            ta[d] = a; tb[d] = b;
        }
        if constexpr (FMT == BGL_Q4G64) {
            o[0] = ta[0] + tb[0] - 8 * (ds0.x + ds1.x); o[1] = ta[1] + tb[1] - 8 * (ds0.y + ds1.y);
            o[2] = ta[2] + tb[2] - 8 * (ds0.z + ds1.z);
        } else if constexpr (FMT == BGL_MXFP4) {     // signed codes: no bias correction
            o[0] = ta[0]; o[1] = ta[1]; o[2] = ta[2]; o[3] = tb[0]; o[4] = tb[1]; o[5] = tb[2];
        } else {
            o[0] = ta[0] - 8 * ds0.x; o[1] = ta[1] - 8 * ds0.y; o[2] = ta[2] - 8 * ds0.z;
            o[3] = tb[0] - 8 * ds1.x; o[4] = tb[1] - 8 * ds1.y; o[5] = tb[2] - 8 * ds1.z;
        }
    } else if constexpr (FMT == BGL_Q8G64) {
#pragma unroll 1
        for (int d = 0; d < 3; d++) {
            const XDig x = x_digit(rec, d);
            int a = 0;
#pragma unroll
            for (int q = 0; q < 16; q++) a = dot4(w.w[q], x.v[q], a);
            o[d] = a;
        }
    } else {
        using X = XDec<FMT, NB>;
        constexpr int CORR = 128 * X::H8 - (1 << (NB - 1));     // code = u - 2^(n-1); the 8-bit field is stored as f - 128
#pragma unroll 1
        for (int d = 0; d < 3; d++) {
            const XDig x = x_digit(rec, d);
            int a = 0, b = 0;
            if constexpr (X::H8) {
#pragma unroll
                for (int q = 0; q < 16; q++) a = dot4(w.lo[q], x.v[q], a);
            }
            if constexpr (X::HI) {
#pragma unroll
                for (int q = 0; q < 16; q++) b = dot4(w.hi[q], x.v[q], b);
            }
            o[d] = X::H8 ? a + b * 256 : b;
        }
        o[0] += CORR * (ds0.x + ds1.x); o[1] += CORR * (ds0.y + ds1.y); o[2] += CORR * (ds0.z + ds1.z);
    }
}

// Where the raw values of a lane's group are, for the non-finite slow path.
struct XRow {
    const BglDevTensor *T;
    int row;                  // the lane's weight row
    const float *xr;          // the activation column's raw values
};

// The group's fp32 term against one record: the exact integer dot product per digit, folded as
// s * ((t0 + 256 t1 + 65536 t2) * 2^(e-22)).
template <int FMT, int NB>
__device__ __forceinline__ float x_dot(const XDec<FMT, NB> &w, const int *rec) {
    const int4 ds0 = *reinterpret_cast<const int4 *>(rec + XREC_DSUM);
    const int4 ds1 = *reinterpret_cast<const int4 *>(rec + XREC_DSUM + 4);
    const float xs = *reinterpret_cast<const float *>(rec + XREC_SCALE);
    if constexpr (FMT == BGL_Q4G64 || FMT == BGL_Q4G32H || FMT == BGL_MXFP4) {
        int ta[3], tb[3];
#pragma unroll
        for (int d = 0; d < 3; d++) {
            const XDig x = x_digit(rec, d);
            int a = 0, b = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) { a = dot4(w.lo[q], x.v[2 * q], a); a = dot4(w.hi[q], x.v[2 * q + 1], a); }
#pragma unroll
            for (int q = 4; q < 8; q++) { b = dot4(w.lo[q], x.v[2 * q], b); b = dot4(w.hi[q], x.v[2 * q + 1], b); }
            ta[d] = a; tb[d] = b;
        }
        if constexpr (FMT == BGL_Q4G64) {
            const float V = fold_digits(ta[0] + tb[0] - 8 * (ds0.x + ds1.x), ta[1] + tb[1] - 8 * (ds0.y + ds1.y),
                                        ta[2] + tb[2] - 8 * (ds0.z + ds1.z));
            return w.s * (V * xs);
        } else if constexpr (FMT == BGL_MXFP4) {
            return w.sa * (fold_digits(ta[0], ta[1], ta[2]) * xs) + w.sb * (fold_digits(tb[0], tb[1], tb[2]) * xs);
        } else {
            const float Va = fold_digits(ta[0] - 8 * ds0.x, ta[1] - 8 * ds0.y, ta[2] - 8 * ds0.z);
            const float Vb = fold_digits(tb[0] - 8 * ds1.x, tb[1] - 8 * ds1.y, tb[2] - 8 * ds1.z);
            return w.sa * (Va * xs) + w.sb * (Vb * xs);
        }
    } else if constexpr (FMT == BGL_Q8G64) {
        int t[3];
#pragma unroll
        for (int d = 0; d < 3; d++) {
            const XDig x = x_digit(rec, d);
            int a = 0;
#pragma unroll
            for (int q = 0; q < 16; q++) a = dot4(w.w[q], x.v[q], a);
            t[d] = a;
        }
        return w.s * (fold_digits(t[0], t[1], t[2]) * xs);
    } else {
        using X = XDec<FMT, NB>;
        constexpr int CORR = 128 * X::H8 - (1 << (NB - 1));     // code = u - 2^(n-1); the 8-bit field is stored as f - 128
        int t[3];
#pragma unroll
        for (int d = 0; d < 3; d++) {
            const XDig x = x_digit(rec, d);
            int a = 0, b = 0;
            if constexpr (X::H8) {
#pragma unroll
                for (int q = 0; q < 16; q++) a = dot4(w.lo[q], x.v[q], a);
            }
            if constexpr (X::HI) {
#pragma unroll
                for (int q = 0; q < 16; q++) b = dot4(w.hi[q], x.v[q], b);
            }
            t[d] = X::H8 ? a + b * 256 : b;
        }
        t[0] += CORR * (ds0.x + ds1.x); t[1] += CORR * (ds0.y + ds1.y); t[2] += CORR * (ds0.z + ds1.z);
        return w.s * (fold_digits(t[0], t[1], t[2]) * xs);
    }
}

// The terms the level-0 digits leave out, for a lane's group flagged BGL_XF_L1 or BGL_XF_NF (0 for
// the lanes of the wave whose groups are not): the level-1 residual
// s * ((V1 * 2^(e1-22)) * 2^(e-22)) against the level-1 digits at r1 (48 dwords, LDS or global)
// with their half sums e0 / e1, and the non-finite products.  Cold path: the GEMVs run it after
// their main loop for the slots whose records carry flags, with the weights loaded again.
template <int FMT, int NB>
__device__ __forceinline__ float x_fix(const XDec<FMT, NB> &w, const int *rec, const int *r1, int4 e0, int4 e1,
                                       const XRow &xrow, int g) {
    const int fl = rec[XREC_DSUM + 3];
    const float2 xs = *reinterpret_cast<const float2 *>(rec + XREC_SCALE);
    float t = 0.0f;
    if (__builtin_amdgcn_ballot_w64(fl & BGL_XF_L1)) {
        int p[6];
        x_ints<FMT, NB>(w, r1, e0, e1, p);
        const float rt = (fl & BGL_XF_L1) ? xs.y : 0.0f;      // other lanes' level-1 data is not theirs: 0
        if constexpr (FMT == BGL_Q4G32H || FMT == BGL_MXFP4)
            t = w.sa * ((fold_digits(p[0], p[1], p[2]) * rt) * xs.x) + w.sb * ((fold_digits(p[3], p[4], p[5]) * rt) * xs.x);
        else
            t = w.s * ((fold_digits(p[0], p[1], p[2]) * rt) * xs.x);
    }
    if (fl & BGL_XF_NF) t += x_nonfinite<FMT, NB>(*xrow.T, xrow.row, g, xrow.xr);
    return t;
}

template <int FMT, int NB>
__device__ __forceinline__ float x_group(const XRaw<FMT, NB> &r, const int *rec) { return x_dot<FMT, NB>(x_decode<FMT, NB>(r), rec); }

// ---- fused activation digits (k_act_x24's arithmetic, bgl_prep.hip): one pass is 256 consecutive
// values, lane l holding values 4l..4l+3 (one float4), a 16-lane row one 64-group g = 4p + l/16.
// Per group e = exponent of the largest finite |x| (frexp), X = rint(x * 2^(22-e)) split into
// balanced int8 digits X = d0 + 256 d1 + 65536 d2; the record gets the digits, their sums per
// 32-element half, the flags, 2^(e-22) and the level-1 ratio.  Groups that bgl_x_level1 selects
// (many elements more than 2^BGL_X_SPIKE_BITS below the max) also get the level-1 record of the
// residual at rec + l1; non-finite elements count as 0 and flag the group.
template <int CTRL>
__device__ __forceinline__ uint32_t x_dpp(uint32_t v) { return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false); }
__device__ __forceinline__ uint32_t x_umax(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint32_t x_row_umax(uint32_t v) {
    v = x_umax(v, x_dpp<0xB1>(v));
    v = x_umax(v, x_dpp<0x4E>(v));
    v = x_umax(v, x_dpp<0x141>(v));
    return x_umax(v, x_dpp<0x140>(v));            // the 16-lane row's max in all its lanes
}

__device__ __forceinline__ float4 x_pass_load(const float *x, int p, int lane, int K) {
    const bgl_f32x4 t = *((const BGL_GLOBAL bgl_f32x4 *)(x + min(256 * p + 4 * lane, K - 4)));
    return make_float4(t.x, t.y, t.z, t.w);
}

// Three balanced digits of 4 integers |X| <= 2^22, packed one byte per element, and their sums
// over the lane's 8-lane half of the row (32 elements).
struct XPack {
    uint32_t D[3];
    int s[3];
};
__device__ __forceinline__ XPack x_pack3(const int (&X)[4]) {
    XPack p;
    p.D[0] = p.D[1] = p.D[2] = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int d0 = (int)(int8_t)(X[i] & 255);
        const int X1 = (X[i] - d0) >> 8;
        const int d1 = (int)(int8_t)(X1 & 255);
        const int d2 = (X1 - d1) >> 8;
        p.D[0] |= ((uint32_t)d0 & 255u) << (8 * i);
        p.D[1] |= ((uint32_t)d1 & 255u) << (8 * i);
        p.D[2] |= ((uint32_t)d2 & 255u) << (8 * i);
    }
#pragma unroll
    for (int d = 0; d < 3; d++) {
        int t = dot4((int)p.D[d], 0x01010101, 0);
        t += (int)x_dpp<0xB1>((uint32_t)t);
        t += (int)x_dpp<0x4E>((uint32_t)t);
        t += (int)x_dpp<0x141>((uint32_t)t);
        p.s[d] = t;
    }
    return p;
}
__device__ __forceinline__ void x_store3(int *rec, int q, const XPack &p, int flags) {
    rec[q] = (int)p.D[0]; rec[16 + q] = (int)p.D[1]; rec[32 + q] = (int)p.D[2];
    if ((q & 7) == 0) {
        int4 *ds = reinterpret_cast<int4 *>(rec + XREC_DSUM + 4 * (q >> 3));
        *ds = make_int4(p.s[0], p.s[1], p.s[2], q == 0 ? flags : 0);
    }
}

// A 16-lane row's 64-group (4 values per lane): non-finite values zeroed (rare: only when the
// row's largest |x| bits are Inf/NaN), e = exponent of the largest finite |x| (frexp), whether the
// group needs level 1, and the level-0 integers X = rint(x * 2^(22-e)) with their exact residuals.
struct XStat {
    float mx;                  // the group's largest finite |x|
    int e, nnf;                // exponent of mx; non-finite values in the row
    bool spiky;                // bgl_x_level1 over the nonzero |x| below / at or above 2^(e - BGL_X_SPIKE_BITS)
    int X[4];
    float r[4];                // x * 2^(22-e) - X, exact, |r| <= 1/2
};
__device__ __forceinline__ XStat x_stat(const float4 &v) {
    XStat st;
    float f[4] = {v.x, v.y, v.z, v.w};
    uint32_t b[4];
#pragma unroll
    for (int i = 0; i < 4; i++) b[i] = __float_as_uint(f[i]) & 0x7fffffffu;
    uint32_t mb = x_row_umax(x_umax(x_umax(b[0], b[1]), x_umax(b[2], b[3])));   // the group's max |x| bits
    st.nnf = 0;
    if (__builtin_amdgcn_ballot_w64(mb >= 0x7f800000u)) {   // NaN / +-Inf somewhere in the wave: 0 in the digits
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (b[i] >= 0x7f800000u) { f[i] = 0.0f; b[i] = 0u; st.nnf++; }
        mb = x_row_umax(x_umax(x_umax(b[0], b[1]), x_umax(b[2], b[3])));
        st.nnf = row_sum_i32(st.nnf);
    }
    st.mx = __uint_as_float(mb);
    st.e = 0;
    if (st.mx > 0.0f) frexpf(st.mx, &st.e);
    st.e = max(st.e, BGL_X_EMIN);
    const uint32_t thr = st.mx > 0.0f ? __float_as_uint(ldexpf(1.0f, st.e - BGL_X_SPIKE_BITS)) : 0u;
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) cnt += (b[i] != 0u ? 256 : 0) + (b[i] >= thr ? 1 : 0);
    cnt = row_sum_i32(cnt);
    st.spiky = bgl_x_level1((cnt >> 8) - (cnt & 255), cnt & 255);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float xp = st.mx > 0.0f ? ldexpf(f[i], BGL_X_FRAC - st.e) : 0.0f;   // power-of-two scaling: exact
        const float Xf = rintf(xp);
        st.X[i] = (int)Xf;
        st.r[i] = xp - Xf;
    }
    return st;
}
// exponent e1 of the row's largest |residual| (0 when all are 0), in every lane of the row
__device__ __forceinline__ int x_resid_exp(const XStat &st, float &mr) {
    const uint32_t rb = x_row_umax(x_umax(x_umax(__float_as_uint(st.r[0]) & 0x7fffffffu, __float_as_uint(st.r[1]) & 0x7fffffffu),
                                          x_umax(__float_as_uint(st.r[2]) & 0x7fffffffu, __float_as_uint(st.r[3]) & 0x7fffffffu)));
    mr = __uint_as_float(rb);
    int e1 = 0;
    if (mr > 0.0f) frexpf(mr, &e1);
    return e1;
}

// Pass p's level-0 records: digits, sums, flags, the scale 2^(e-22) and the level-1 ratio
// 2^(e1-22) (0 unless the group needs level 1).  The level-1 digits themselves are made only where
// a GEMV needs them (x_pass_l1, cold path).
__device__ __forceinline__ void x_pass_digits(const float4 &v, int p, int lane, int G, int *xl) {
    const int g = 4 * p + (lane >> 4), q = lane & 15;
    const XStat st = x_stat(v);
    const XPack P0 = x_pack3(st.X);
    int flags = st.nnf ? BGL_XF_NF : 0;
    float ratio = 0.0f;
    if (__builtin_amdgcn_ballot_w64(st.spiky)) {    // uniform branch: some row of the wave has an outlier
        float mr;
        const int e1 = x_resid_exp(st, mr);
        if (st.spiky && mr > 0.0f) { ratio = ldexpf(1.0f, e1 - BGL_X_FRAC); flags |= BGL_XF_L1; }
    }
    if (g < G) {
        int *rec = xl + g * XREC_DW;
        x_store3(rec, q, P0, flags);
        if (q == 0) *reinterpret_cast<float2 *>(rec + XREC_SCALE) = make_float2(st.mx > 0.0f ? ldexpf(1.0f, st.e - BGL_X_FRAC) : 0.0f, ratio);
    }
}

// The level-1 records (the residual's digits and sums) of pass p's groups in [g0, g1), written to
// dst + (g - g0) * XREC_DW: the same arithmetic as x_pass_digits, so they match its ratios.
__device__ __forceinline__ void x_pass_l1(const float4 &v, int p, int lane, int g0, int g1, int *dst) {
    const int g = 4 * p + (lane >> 4), q = lane & 15;
    const XStat st = x_stat(v);
    float mr;
    const int e1 = x_resid_exp(st, mr);
    int X1[4];
#pragma unroll
    for (int i = 0; i < 4; i++) X1[i] = mr > 0.0f ? (int)rintf(ldexpf(st.r[i], BGL_X_FRAC - e1)) : 0;
    const XPack P1 = x_pack3(X1);
    if (g >= g0 && g < g1) x_store3(dst + (g - g0) * XREC_DW, q, P1, 0);
}
