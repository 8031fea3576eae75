// bgl_gemv_x.hip -- the one-column fp32-activation GEMV (q4gemv.h:761-769 gemm_qXg64_mt at M=1,
// qng64_dense.c:70-79 qng64_matvec_f32; int4 g64, int4 g32 fp16-scale, int8 g64, qNg64 n=2..15).
//
// Activations arrive prepared by k_act_x24 (bgl_prep.hip): per 64-group three balanced int8 digits
// of X = rint(x * 2^(21-e)), the digit sums per 32-element half and the scale 2^(e-21), so every
// product below is an exact int32 dot4 sum and fp32 only enters in the per-group fold.
//
// Work decomposition (the shape of the fused W4A8 kernel): a workgroup owns TR rows of a 64-row
// tile and the whole K range, so no launch needs a K split or a second reduction kernel.  Lane l
// of a wave handles row l % TR and group kq = l / TR of each slot of KQ = 64/TR consecutive
// 64-groups, so each wave-wide weight load is KQ runs of TR*16 >= 128 contiguous bytes.  The
// workgroup's waves take the slots in turn; a wave's next slot is loaded before the current one is
// used.
//
// The activation operands of the whole K range are copied into LDS once per workgroup (one 240-byte
// record per group: 48 digit dwords, two 4-dword digit-sum words, the scale), issued before the
// first weight loads so the copy's latency hides under theirs.  Lanes of one group read the same
// record (a broadcast); the 60-dword record stride puts the KQ <= 8 records a read touches in
// disjoint banks.
//
// qNg64 bit planes: the 8-bit field (stored as f ^ 0x80, a signed byte f - 128) is one dot4
// operand; the 4-, 2- and 1-bit fields of an element are merged into one byte (their values sit at
// bit 0, 4*has4 and 4*has4 + 2*has2 of it, < 128) with one shift and one v_and_or per field, so a
// group costs two dot4 operands per digit instead of one per field.
#include "bgl_gemv_impl.h"

#define XREC_DW 60            // LDS dwords per 64-group record
#define XREC_DSUM 48          // digit sums of the two halves: [half][digit 0..2, pad]
#define XREC_SCALE 56         // 2^(e-21)
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
    if constexpr (FMT == BGL_Q4G32H) r.s = sv;
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

// The group's fp32 term: the exact integer dot product per digit, folded as
// s * ((t0 + 256 t1 + 65536 t2) * 2^(e-21)).
template <int FMT, int NB>
__device__ __forceinline__ float x_group(const XRaw<FMT, NB> &r, const int *rec) {
    const int4 ds0 = *reinterpret_cast<const int4 *>(rec + XREC_DSUM);
    const int4 ds1 = *reinterpret_cast<const int4 *>(rec + XREC_DSUM + 4);
    const float xs = *reinterpret_cast<const float *>(rec + XREC_SCALE);
    if constexpr (FMT == BGL_Q4G64 || FMT == BGL_Q4G32H) {
        const uint32_t raw[8] = {r.c[0].x, r.c[0].y, r.c[0].z, r.c[0].w, r.c[1].x, r.c[1].y, r.c[1].z, r.c[1].w};
        int lo[8], hi[8];
#pragma unroll
        for (int q = 0; q < 8; q++) { lo[q] = nib_lo(raw[q]); hi[q] = nib_hi(raw[q]); }
        int ta[3], tb[3];
#pragma unroll
        for (int d = 0; d < 3; d++) {
            const XDig x = x_digit(rec, d);
            int a = 0, b = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) { a = dot4(lo[q], x.v[2 * q], a); a = dot4(hi[q], x.v[2 * q + 1], a); }
#pragma unroll
            for (int q = 4; q < 8; q++) { b = dot4(lo[q], x.v[2 * q], b); b = dot4(hi[q], x.v[2 * q + 1], b); }
            ta[d] = a; tb[d] = b;
        }
        if constexpr (FMT == BGL_Q4G64) {
            const float V = fold_digits(ta[0] + tb[0] - 8 * (ds0.x + ds1.x), ta[1] + tb[1] - 8 * (ds0.y + ds1.y),
                                        ta[2] + tb[2] - 8 * (ds0.z + ds1.z));
            return r.s * (V * xs);
        } else {
            const float sa = __half2float(__ushort_as_half((unsigned short)(r.s & 0xffffu)));
            const float sb = __half2float(__ushort_as_half((unsigned short)(r.s >> 16)));
            const float Va = fold_digits(ta[0] - 8 * ds0.x, ta[1] - 8 * ds0.y, ta[2] - 8 * ds0.z);
            const float Vb = fold_digits(tb[0] - 8 * ds1.x, tb[1] - 8 * ds1.y, tb[2] - 8 * ds1.z);
            return sa * (Va * xs) + sb * (Vb * xs);
        }
    } else if constexpr (FMT == BGL_Q8G64) {
        const int w[16] = {(int)r.c[0].x, (int)r.c[0].y, (int)r.c[0].z, (int)r.c[0].w, (int)r.c[1].x, (int)r.c[1].y,
                           (int)r.c[1].z, (int)r.c[1].w, (int)r.c[2].x, (int)r.c[2].y, (int)r.c[2].z, (int)r.c[2].w,
                           (int)r.c[3].x, (int)r.c[3].y, (int)r.c[3].z, (int)r.c[3].w};
        int t[3];
#pragma unroll
        for (int d = 0; d < 3; d++) {
            const XDig x = x_digit(rec, d);
            int a = 0;
#pragma unroll
            for (int q = 0; q < 16; q++) a = dot4(w[q], x.v[q], a);
            t[d] = a;
        }
        return r.s * (fold_digits(t[0], t[1], t[2]) * xs);
    } else {
        using R = XRaw<FMT, NB>;
        constexpr int H8 = R::H8, H4 = R::H4, H2 = R::H2, H1 = R::H1;
        constexpr bool HI = H4 || H2 || H1;                  // fields merged into the second operand
        constexpr int S2 = 4 * H4, S1 = 4 * H4 + 2 * H2;     // their bit offsets inside it
        constexpr int CORR = 128 * H8 - (1 << (NB - 1));     // code = u - 2^(n-1); the 8-bit field is stored as f - 128
        int lo[16], hi[16];
        if constexpr (H8) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                lo[4 * k] = (int)r.p8[k].x; lo[4 * k + 1] = (int)r.p8[k].y; lo[4 * k + 2] = (int)r.p8[k].z; lo[4 * k + 3] = (int)r.p8[k].w;
            }
        }
        if constexpr (HI) {
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
                hi[q] = (int)h;
            }
        }
        int t[3];
#pragma unroll
        for (int d = 0; d < 3; d++) {
            const XDig x = x_digit(rec, d);
            int a = 0, b = 0;
            if constexpr (H8) {
#pragma unroll
                for (int q = 0; q < 16; q++) a = dot4(lo[q], x.v[q], a);
            }
            if constexpr (HI) {
#pragma unroll
                for (int q = 0; q < 16; q++) b = dot4(hi[q], x.v[q], b);
            }
            t[d] = H8 ? a + b * 256 : b;
        }
        t[0] += CORR * (ds0.x + ds1.x); t[1] += CORR * (ds0.y + ds1.y); t[2] += CORR * (ds0.z + ds1.z);
        return r.s * (fold_digits(t[0], t[1], t[2]) * xs);
    }
}

// ---- fused activation digits (k_act_x24's arithmetic, bgl_prep.hip): one pass is 256 consecutive
// values, lane l holding values 4l..4l+3 (one float4), a 16-lane row one 64-group g = 4p + l/16.
// Per group e = exponent of max|x| (frexp), X = rint(x * 2^(21-e)) split into balanced int8 digits
// X = d0 + 256 d1 + 65536 d2; the record gets the digits, their sums per 32-element half and 2^(e-21).
template <int CTRL>
__device__ __forceinline__ uint32_t x_dpp(uint32_t v) { return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false); }
__device__ __forceinline__ uint32_t x_umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

__device__ __forceinline__ float4 x_pass_load(const float *x, int p, int lane, int K) {
    const bgl_f32x4 t = *((const BGL_GLOBAL bgl_f32x4 *)(x + min(256 * p + 4 * lane, K - 4)));
    return make_float4(t.x, t.y, t.z, t.w);
}

__device__ __forceinline__ void x_pass_digits(const float4 &v, int p, int lane, int G, int *xl) {
    const int g = 4 * p + (lane >> 4), q = lane & 15;
    uint32_t mb = x_umax(x_umax(__float_as_uint(v.x) & 0x7fffffffu, __float_as_uint(v.y) & 0x7fffffffu),
                         x_umax(__float_as_uint(v.z) & 0x7fffffffu, __float_as_uint(v.w) & 0x7fffffffu));
    mb = x_umax(mb, x_dpp<0xB1>(mb));
    mb = x_umax(mb, x_dpp<0x4E>(mb));
    mb = x_umax(mb, x_dpp<0x141>(mb));
    mb = x_umax(mb, x_dpp<0x140>(mb));             // the group's max |x| bits in all 16 lanes
    const float mx = __uint_as_float(mb);
    int e = 0;
    if (mx > 0.0f) frexpf(mx, &e);
    const float f[4] = {v.x, v.y, v.z, v.w};
    uint32_t D0 = 0, D1 = 0, D2 = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int X = mx > 0.0f ? (int)rintf(ldexpf(f[i], 21 - e)) : 0;
        const int d0 = (int)(int8_t)(X & 255);
        const int X1 = (X - d0) >> 8;
        const int d1 = (int)(int8_t)(X1 & 255);
        const int d2 = (X1 - d1) >> 8;
        D0 |= ((uint32_t)d0 & 255u) << (8 * i);
        D1 |= ((uint32_t)d1 & 255u) << (8 * i);
        D2 |= ((uint32_t)d2 & 255u) << (8 * i);
    }
    // digit sums of the lane's 4 values, then of its 8-lane half (32 values)
    int s0 = dot4((int)D0, 0x01010101, 0), s1 = dot4((int)D1, 0x01010101, 0), s2 = dot4((int)D2, 0x01010101, 0);
    s0 += (int)x_dpp<0xB1>((uint32_t)s0); s1 += (int)x_dpp<0xB1>((uint32_t)s1); s2 += (int)x_dpp<0xB1>((uint32_t)s2);
    s0 += (int)x_dpp<0x4E>((uint32_t)s0); s1 += (int)x_dpp<0x4E>((uint32_t)s1); s2 += (int)x_dpp<0x4E>((uint32_t)s2);
    s0 += (int)x_dpp<0x141>((uint32_t)s0); s1 += (int)x_dpp<0x141>((uint32_t)s1); s2 += (int)x_dpp<0x141>((uint32_t)s2);
    if (g < G) {
        int *rec = xl + g * XREC_DW;
        rec[q] = (int)D0; rec[16 + q] = (int)D1; rec[32 + q] = (int)D2;
        if ((q & 7) == 0) {
            int4 *ds = reinterpret_cast<int4 *>(rec + XREC_DSUM + 4 * (q >> 3));
            *ds = make_int4(s0, s1, s2, 0);
        }
        if (q == 0) rec[XREC_SCALE] = __float_as_int(mx > 0.0f ? ldexpf(1.0f, e - 21) : 0.0f);
    }
}

template <int FMT, int NB, int TR, bool FUSE>
__global__ __launch_bounds__(MAXW * BGL_TILE) void k_gemv_x(GemvLaunch L) {
    extern __shared__ __align__(16) int xl[];
    constexpr int KQ = BGL_TILE / TR, SUBS = BGL_TILE / TR;
    const int b = blockIdx.x;
    int ti = 0;
#pragma unroll
    for (int i = 1; i < BGL_MAX_TASKS; i++) if (i < L.ntasks && b >= L.t[i].blk0) ti = i;
    GemvTask task = L.t[0];
#pragma unroll
    for (int i = 1; i < BGL_MAX_TASKS; i++) if (i == ti) task = L.t[i];
    const BglDevTensor &T = task.T;
    const int lb = b - task.blk0, tile = lb / SUBS, r0 = (lb % SUBS) * TR;
    const int nthr = blockDim.x, nw = nthr >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int K = T.K, G = K >> 6, m = L.m0;
    const int *xw = L.a.xw + (size_t)m * G * BGL_XD_DW;
    const int *xsum = L.a.xsum + (size_t)m * (K >> 5) * 4;
    const float *xsc = L.a.xs + (size_t)m * G;
    const float *xr = L.x + (size_t)m * K;
    const int NPX = (K + 255) >> 8;               // fused: passes of 256 values

    // ---- activation records (or the raw values they are made from): the first loads go out ahead
    // of the weights
    const int npc = G * 14;                       // 16-byte pieces: 12 of digits, 2 of digit sums per group
    auto piece_src = [&](int i) -> const bgl_u32x4 * {
        const int g = i / 14, p = i - g * 14;
        return p < 12 ? reinterpret_cast<const bgl_u32x4 *>(xw + (size_t)g * BGL_XD_DW + 4 * p)
                      : reinterpret_cast<const bgl_u32x4 *>(xsum + ((size_t)2 * g + (p - 12)) * 4);
    };
    auto piece_dst = [&](int i) -> bgl_u32x4 * {
        const int g = i / 14, p = i - g * 14;
        return reinterpret_cast<bgl_u32x4 *>(xl + g * XREC_DW + (p < 12 ? 4 * p : XREC_DSUM + 4 * (p - 12)));
    };
    bgl_u32x4 pre0, pre1, pre2, pre3;
    float xs0 = 0.0f;
    float4 xv;
    if constexpr (FUSE) {
        xv = x_pass_load(xr, wave, lane, K);
    } else {
        pre0 = *piece_src(min((int)threadIdx.x, npc - 1));
        pre1 = *piece_src(min((int)threadIdx.x + nthr, npc - 1));
        pre2 = *piece_src(min((int)threadIdx.x + 2 * nthr, npc - 1));
        pre3 = *piece_src(min((int)threadIdx.x + 3 * nthr, npc - 1));
        xs0 = xsc[min((int)threadIdx.x, G - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- the first slots' weights: a wave's slots are wave, wave + nw, ...; D of them in flight
    const int r = lane % TR, kq = lane / TR, rr = r0 + r;
    const int S = (G + KQ - 1) / KQ;               // slots of KQ groups (records past G are zero)
    constexpr int D = x_depth<FMT, NB>();
    const int ns = (S - 1 - wave) / nw + 1;        // nw <= S: every wave has a slot
    XRaw<FMT, NB> c[D];
    const XRes R = x_res<FMT>(T, tile);
    // lanes whose group of the last slot lies past K read nothing there (an offset past every
    // resource); their zero records make the term zero
    const XLane xlane = x_lane<FMT, NB, KQ>(rr, kq);
    XLane xlast = xlane;
    if (kq >= G - (S - 1) * KQ) xlast = XLane{X_OOB, X_OOB, X_OOB, X_OOB, X_OOB};
    auto lane_of = [&](int sl) { return sl == S - 1 ? xlast : xlane; };
#pragma unroll
    for (int j = 0; j < D; j++) x_load<FMT, NB, KQ>(c[j], R, lane_of(wave + j * nw), wave + j * nw, j < ns);
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (FUSE) {
        for (int p = wave; p < NPX; p += nw) {
            if (p != wave) xv = x_pass_load(xr, p, lane, K);
            x_pass_digits(xv, p, lane, G, xl);
        }
    } else {
        if ((int)threadIdx.x < npc) *piece_dst(threadIdx.x) = pre0;
        if ((int)threadIdx.x + nthr < npc) *piece_dst(threadIdx.x + nthr) = pre1;
        if ((int)threadIdx.x + 2 * nthr < npc) *piece_dst(threadIdx.x + 2 * nthr) = pre2;
        if ((int)threadIdx.x + 3 * nthr < npc) *piece_dst(threadIdx.x + 3 * nthr) = pre3;
        if ((int)threadIdx.x < G) xl[threadIdx.x * XREC_DW + XREC_SCALE] = __float_as_int(xs0);
        for (int i = threadIdx.x + X_PRE * nthr; i < npc; i += nthr) *piece_dst(i) = *piece_src(i);
        for (int g = threadIdx.x + nthr; g < G; g += nthr) xl[g * XREC_DW + XREC_SCALE] = __float_as_int(xsc[g]);
    }
    // records of the last slot's groups past K: zero digits, sums and scale (a zero term for any weight)
    for (int i = G * XREC_DW + threadIdx.x; i < S * KQ * XREC_DW; i += nthr) xl[i] = 0;
    __syncthreads();

    float acc = 0.0f;
    const int *xk = xl + kq * XREC_DW;
    for (int i0 = 0; i0 < ns; i0 += D) {
#pragma unroll
        for (int j = 0; j < D; j++) {
            const int i = i0 + j, sl = wave + i * nw;
            if (i < ns) acc += x_group<FMT, NB>(c[j], xk + sl * (KQ * XREC_DW));
            x_load<FMT, NB, KQ>(c[j], R, lane_of(sl + D * nw), sl + D * nw, i + D < ns);
        }
    }
    // rows' partials: over the KQ lanes of a row, then over the waves in order
#pragma unroll
    for (int o = TR; o < BGL_TILE; o <<= 1) acc += __shfl_xor(acc, o);
    float *red = reinterpret_cast<float *>(xl + S * KQ * XREC_DW);
    if (lane < TR) red[wave * TR + lane] = acc;
    __syncthreads();
    if (threadIdx.x < TR) {
        const int row = tile * BGL_TILE + r0 + threadIdx.x;
        if (row < T.N) {
            float v = red[threadIdx.x];
            for (int w = 1; w < nw; w++) v += red[w * TR + threadIdx.x];
            task.y[(size_t)m * task.ystride + row] = (task.bias ? task.bias[row] : 0.0f) + v;
        }
    }
}

// Records of every slot's groups (K/64 rounded up to the slot width 64/TR) and the row partials.
size_t bgl_gemv_x_lds(int K, int TR, int nw) {
    const int KQ = 64 / TR, S = (K / 64 + KQ - 1) / KQ;
    return (size_t)S * KQ * XREC_DW * 4 + (size_t)nw * TR * 4;
}

template <int FMT, int NB, bool FUSE>
static int launch_x_tr(int TR, const GemvLaunch &L, int nblocks, int nw, hipStream_t st) {
    dim3 g(nblocks), b(nw * BGL_TILE);
    const size_t lds = bgl_gemv_x_lds(L.t[0].T.K, TR, nw);
    switch (TR) {
    case 8: hipLaunchKernelGGL((k_gemv_x<FMT, NB, 8, FUSE>), g, b, lds, st, L); return 0;
    case 16: hipLaunchKernelGGL((k_gemv_x<FMT, NB, 16, FUSE>), g, b, lds, st, L); return 0;
    case 32: hipLaunchKernelGGL((k_gemv_x<FMT, NB, 32, FUSE>), g, b, lds, st, L); return 0;
    case 64: hipLaunchKernelGGL((k_gemv_x<FMT, NB, 64, FUSE>), g, b, lds, st, L); return 0;
    default: return -1;
    }
}

template <int FMT, int NB>
static int launch_x_fuse(bool fuse, int TR, const GemvLaunch &L, int nblocks, int nw, hipStream_t st) {
    return fuse ? launch_x_tr<FMT, NB, true>(TR, L, nblocks, nw, st) : launch_x_tr<FMT, NB, false>(TR, L, nblocks, nw, st);
}

// One activation column (L.m0) of up to BGL_MAX_TASKS tensors sharing K; nblocks = workgroups of
// TR rows over every task (task i's first workgroup is L.t[i].blk0).  fuse: every workgroup makes
// the activation records from the raw column L.x itself; otherwise they come prepared in L.a.
int bgl_launch_gemv_x(const GemvLaunch &L, bool fuse, int nblocks, int TR, int nw, hipStream_t st) {
    const BglDevTensor &T = L.t[0].T;
    if (T.K < 64 || T.K % 64 || nw < 1 || nw > MAXW) return -1;
    switch (T.fmt) {
    case BGL_Q4G64: return launch_x_fuse<BGL_Q4G64, 0>(fuse, TR, L, nblocks, nw, st);
    case BGL_Q4G32H: return launch_x_fuse<BGL_Q4G32H, 0>(fuse, TR, L, nblocks, nw, st);
    case BGL_Q8G64: return launch_x_fuse<BGL_Q8G64, 0>(fuse, TR, L, nblocks, nw, st);
    case BGL_QNG64:
        switch (T.bits) {
        case 2: return launch_x_fuse<BGL_QNG64, 2>(fuse, TR, L, nblocks, nw, st);
        case 3: return launch_x_fuse<BGL_QNG64, 3>(fuse, TR, L, nblocks, nw, st);
        case 4: return launch_x_fuse<BGL_QNG64, 4>(fuse, TR, L, nblocks, nw, st);
        case 5: return launch_x_fuse<BGL_QNG64, 5>(fuse, TR, L, nblocks, nw, st);
        case 6: return launch_x_fuse<BGL_QNG64, 6>(fuse, TR, L, nblocks, nw, st);
        case 7: return launch_x_fuse<BGL_QNG64, 7>(fuse, TR, L, nblocks, nw, st);
        case 8: return launch_x_fuse<BGL_QNG64, 8>(fuse, TR, L, nblocks, nw, st);
        case 9: return launch_x_fuse<BGL_QNG64, 9>(fuse, TR, L, nblocks, nw, st);
        case 10: return launch_x_fuse<BGL_QNG64, 10>(fuse, TR, L, nblocks, nw, st);
        case 11: return launch_x_fuse<BGL_QNG64, 11>(fuse, TR, L, nblocks, nw, st);
        case 12: return launch_x_fuse<BGL_QNG64, 12>(fuse, TR, L, nblocks, nw, st);
        case 13: return launch_x_fuse<BGL_QNG64, 13>(fuse, TR, L, nblocks, nw, st);
        case 14: return launch_x_fuse<BGL_QNG64, 14>(fuse, TR, L, nblocks, nw, st);
        case 15: return launch_x_fuse<BGL_QNG64, 15>(fuse, TR, L, nblocks, nw, st);
        default: return -2;
        }
    default: return -2;
    }
}
