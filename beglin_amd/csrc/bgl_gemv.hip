// bgl_gemv.hip -- the quantized GEMV / small-M GEMM kernel family (one kernel template per format).
//
// Work decomposition: one workgroup owns one 64-row tile and the whole K range (no cross-workgroup
// reduction); its nw wavefronts (1..16) split the work units along K.  lane = row, so every
// wave-wide weight load is a contiguous 1 KB run and every lane needs the same activation bytes.
// Each wave prefetches its next unit's chunks before consuming the current one.
//
// Two activation paths:
//   k_gemv   (fp32 activations, and batched W4A8): the activation operands were prepared by a
//            separate kernel (bgl_prep.hip) and are read with scalar loads straight into SGPRs,
//            which feed v_dot4 directly.  Waves' fp32 partials are combined in LDS in fixed order.
//   k_gemv_q (W4A8, one column): the workgroup quantizes x itself into LDS (the reference's
//            q4_quant_act_i8 / _g256 arithmetic, bit for bit), so one call is one launch, and the
//            per-group fp32 terms are folded in group order exactly as the reference's row loop
//            does (q4gemv.h:241, q4gemv_g256.h:154): the result is bit-identical to the oracle.
//
// Arithmetic: weight codes are exact integers; fp32 activations arrive as three int8 digits of an
// exact fixed-point value (bgl_device.h), W4A8 activations as the reference's int8 codes; every
// product is an exact int32 dot4 sum and fp32 only enters in the per-unit scale fold.
#include "bgl_gemv_impl.h"

__device__ __forceinline__ int pick_task(const GemvLaunch &L, int b) {
    int ti = 0;
#pragma unroll
    for (int i = 1; i < BGL_MAX_TASKS; i++) if (i < L.ntasks && b >= L.t[i].blk0) ti = i;
    return ti;
}

// The task of workgroup b, its weight pointers and the activation row.  Every task's blk0 and
// pointers are read from the kernel arguments in one round of independent scalar loads: the single
// empty asm statement makes all of them opaque at once, so the compiler can neither split the loads
// into rounds nor turn the selects into a second load through a selected address (each dependent
// round trip to the kernel arguments delays the first weight loads).
struct TaskSel {
    int ti, blk0;
    const uint8_t *w;
    const void *s0;
    const uint32_t *s1;
    const float *x;           // activation row m0 of the launch
    int cpr, nunits, nthreads;
};
static_assert(BGL_MAX_TASKS == 4, "select_task names four tasks");
__device__ __forceinline__ TaskSel select_task(const GemvLaunch &L, int b) {
    const uint8_t *w0 = L.t[0].T.w, *w1 = L.t[1].T.w, *w2 = L.t[2].T.w, *w3 = L.t[3].T.w;
    const void *a0 = L.t[0].T.s0, *a1 = L.t[1].T.s0, *a2 = L.t[2].T.s0, *a3 = L.t[3].T.s0;
    const uint32_t *c0 = L.t[0].T.s1, *c1 = L.t[1].T.s1, *c2 = L.t[2].T.s1, *c3 = L.t[3].T.s1;
    int b0 = L.t[0].blk0, b1 = L.t[1].blk0, b2 = L.t[2].blk0, b3 = L.t[3].blk0, nt = L.ntasks;
    const float *x = L.x + (size_t)L.m0 * L.t[0].T.K;
    int cpr = L.t[0].T.cpr, nu = L.t[0].T.nunits, nth = blockDim.x;
    asm volatile("" : "+s"(w0), "+s"(w1), "+s"(w2), "+s"(w3), "+s"(a0), "+s"(a1), "+s"(a2), "+s"(a3), "+s"(c0), "+s"(c1),
                 "+s"(c2), "+s"(c3), "+s"(b0), "+s"(b1), "+s"(b2), "+s"(b3), "+s"(nt), "+s"(x), "+s"(cpr), "+s"(nu), "+s"(nth));
    TaskSel r{0, b0, w0, a0, c0, x, cpr, nu, nth};
    if (nt > 1 && b >= b1) r = TaskSel{1, b1, w1, a1, c1, x, cpr, nu, nth};
    if (nt > 2 && b >= b2) r = TaskSel{2, b2, w2, a2, c2, x, cpr, nu, nth};
    if (nt > 3 && b >= b3) r = TaskSel{3, b3, w3, a3, c3, x, cpr, nu, nth};
    return r;
}

// ================================================================================== path A kernel
template <int FMT, int ACT, int NB, int MB>
__global__ __launch_bounds__(MAXW * BGL_TILE) void k_gemv(GemvLaunch L) {
    __shared__ float red[MAXW][MB][BGL_TILE];
    const int b = blockIdx.x, ti = pick_task(L, b);
    GemvTask task = L.t[0];
#pragma unroll
    for (int i = 1; i < BGL_MAX_TASKS; i++) if (i == ti) task = L.t[i];
    const BglDevTensor &T = task.T;
    const int lb = b - task.blk0, tile = lb / task.ks, split = lb % task.ks;
    const int nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const Cols<MB> C = col_rows<MB>(L.a, L.m0, L.mcols);
    const int K = T.K;
    const int ubeg = split * task.gpb, U = min(ubeg + task.gpb, T.nunits);

    float acc[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) acc[m] = 0.0f;
    constexpr bool PREFETCH = chunks_per_unit<FMT>(NB) <= 8;
    int u = ubeg + wave;
    Raw<FMT, NB> r0, r1;
    if (u < U) load_raw<FMT, NB>(r0, T, tile, lane, u);
    while (u < U) {
        const int un = u + nw;
        if constexpr (PREFETCH) {
            if (un < U) load_raw<FMT, NB>(r1, T, tile, lane, un);
            comp_dispatch<FMT, ACT, NB, MB>(r0, K, u, L.a, C, acc);
            r0 = r1;
        } else {
            comp_dispatch<FMT, ACT, NB, MB>(r0, K, u, L.a, C, acc);
            if (un < U) load_raw<FMT, NB>(r0, T, tile, lane, un);
        }
        u = un;
    }
    // groups whose fp32 activations carry a level-1 residual or non-finite values (cold path)
    if constexpr (ACT == BGL_ACT_F32 && FMT != BGL_F16 && FMT != BGL_F32 && FMT != BGL_Q4G256SF) {
        const WRow W{&T, tile * BGL_TILE + lane};
        for (int uu = ubeg + wave; uu < U; uu += nw) {
            int fl = 0;
#pragma unroll
            for (int m = 0; m < MB; m++) fl |= unit_flags<FMT, NB>(L.a, C.am[m], K, uu);
            if (fl) {
                Raw<FMT, NB> rf;
                load_raw<FMT, NB>(rf, T, tile, lane, uu);
                comp_fix<FMT, NB, MB>(rf, W, uu, L.a, C, acc);
            }
        }
    }

#pragma unroll
    for (int m = 0; m < MB; m++) red[wave][m][lane] = acc[m];
    __syncthreads();
    if (wave != 0) return;
    const int row = tile * BGL_TILE + lane;
    if (row >= T.N) return;
    if (task.ks > 1) {                     // partial of this K slice; k_splitk_reduce adds the slices
#pragma unroll
        for (int m = 0; m < MB; m++) {
            float v = red[0][m][lane];
            for (int w = 1; w < nw; w++) v += red[w][m][lane];
            if (m < L.mcols) task.part[((size_t)split * L.mtot + L.m0 + m) * T.N + row] = v;
        }
        return;
    }
    const float bb = task.bias ? task.bias[row] : 0.0f;
#pragma unroll
    for (int m = 0; m < MB; m++) {
        float v = red[0][m][lane];
        for (int w = 1; w < nw; w++) v += red[w][m][lane];
        if (m < L.mcols) task.y[(size_t)(L.m0 + m) * task.ystride + row] = bb + v;
    }
}

// Sums the K-slice partials in slice order: y[m][r] = bias[r] + sum_s part[s][m][r].
__global__ void k_splitk_reduce(const float *__restrict__ part, int ks, int M, int N, const float *__restrict__ bias,
                                float *__restrict__ y, int ystride) {
    const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)M * N) return;
    const int m = (int)(t / N), r = (int)(t % N);
    float v = part[t];
    for (int s = 1; s < ks; s++) v += part[(size_t)s * M * N + t];
    y[(size_t)m * ystride + r] = (bias ? bias[r] : 0.0f) + v;
}

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
// truncate to 0.
__device__ __forceinline__ uint32_t quant_byte(float x, float inv) {
    const float p = __fmul_rn(x, inv);
    int q = (int)__fadd_rn(p, __builtin_copysignf(0.5f, p));   // |.| <= 128.5: no int32 overflow
    q = q > 127 ? 127 : (q < -128 ? -128 : q);
    return (uint32_t)q & 255u;
}

// Quantizes QP passes into LDS.  The MB columns of a launch are one run of passes: pass p is values
// 256*(p % NP) .. +255 of column p / NP (NP passes per column, NPT = MB*NP in all); pass i of the
// call is p0 + i*nw, lane l holding values 4l..4l+3 of it in v[i].  The passes are processed in
// lockstep so their dependency chains interleave.  Column m's operands live at xq + m*XQS,
// asc + m*(NGQ+1), xsum + m*(K/64+1); passes past NPT and lanes past K store into each region's dummy
// slot.  |x| is maximised on its bit pattern (the same order as the float values for non-NaN inputs).
// GQ=256: one pass is one group; its four row maxima are combined with readlane, and one IEEE
// division pair serves every pass (lane i computes pass i's scale and reciprocal).  GQ=64: one pass
// is four groups, one per 16-lane row.
template <int FMT, int QP, int MB>
__device__ __forceinline__ void quant_passes(const float4 (&v)[QP], int p0, int nw, int K, int NP, int NPT, int NGQ, int U,
                                             int lane, int8_t *xq, float *asc, int *xsum) {
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
        const int p = p0 + i * nw;
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
    if constexpr (QU::GQ == 256) {
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < QP; i++) {
            const uint32_t M = umax(umax((uint32_t)__builtin_amdgcn_readlane((int)m[i], 0), (uint32_t)__builtin_amdgcn_readlane((int)m[i], 16)),
                                    umax((uint32_t)__builtin_amdgcn_readlane((int)m[i], 32), (uint32_t)__builtin_amdgcn_readlane((int)m[i], 48)));
            mx = (i == 0 || lane == i) ? __uint_as_float(M) : mx;
        }
        mx = fmaxf(1e-8f, mx);                         // mx starts at 1e-8 (q4gemv_g256.h:78)
        const float sc = __fdiv_rn(mx, 127.0f), iv = __fdiv_rn(1.0f, sc);
#pragma unroll
        for (int i = 0; i < QP; i++) inv[i] = rlane_f(iv, i);
        if (lane < QP) {
            const int p = p0 + lane * nw;
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
        for (int i = 0; i < QP; i++) sc[i] = __fdiv_rn(fmaxf(1e-8f, __uint_as_float(m[i])), 127.0f);   // mx starts at 1e-8 (q4gemv.h:182)
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
        word[i] = quant_byte(v[i].x, inv[i]) | (quant_byte(v[i].y, inv[i]) << 8) | (quant_byte(v[i].z, inv[i]) << 16) |
                  (quant_byte(v[i].w, inv[i]) << 24);
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
            int isum16 = 0;
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const uint4 c = r.c[2 * sg + k];
                const int4 xa = x4[sg * 4 + 2 * k], xb = x4[sg * 4 + 2 * k + 1];
                isum16 = dot4(snib_lo16(c.x), xa.x, isum16); isum16 = dot4(snib_hi16(c.x), xa.y, isum16);
                isum16 = dot4(snib_lo16(c.y), xa.z, isum16); isum16 = dot4(snib_hi16(c.y), xa.w, isum16);
                isum16 = dot4(snib_lo16(c.z), xb.x, isum16); isum16 = dot4(snib_hi16(c.z), xb.y, isum16);
                isum16 = dot4(snib_lo16(c.w), xb.z, isum16); isum16 = dot4(snib_hi16(c.w), xb.w, isum16);
            }
            comb16 += isum16 * (int)((r.sub >> (8 * sg)) & 255u);
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

template <int FMT, int TR, int QP, int MB, bool PREP>
__global__ __launch_bounds__(MAXW * BGL_TILE) void k_gemv_q(GemvLaunch L) {
    extern __shared__ __align__(16) unsigned char lds[];
    constexpr int KQ = BGL_TILE / TR, SUBS = BGL_TILE / TR;
    using QU = QUnit<FMT>;
    const int b = blockIdx.x;
    const TaskSel sel = select_task(L, b);
    BglDevTensor T = L.t[0].T;                          // fmt, K, cpr, nunits are shared by all tasks
    T.w = sel.w; T.s0 = sel.s0; T.s1 = sel.s1; T.cpr = sel.cpr; T.nunits = sel.nunits;
    const int lb = b - sel.blk0, tile = lb / SUBS, r0 = (lb % SUBS) * TR;
    const int nw = sel.nthreads >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    // passes run over the launch's real columns only (a launch of MB columns may carry fewer)
    const int K = T.K, U = T.nunits, NGQ = K / QU::GQ, NP = (K + 255) / 256, NPT = (MB == 1 ? 1 : L.mcols) * NP;
    const int XQS = (U + 1) * QU::STRIDE;               // LDS bytes of one column's codes
    int8_t *xq = reinterpret_cast<int8_t *>(lds);
    float *asc = reinterpret_cast<float *>(lds + (size_t)MB * XQS);
    int *xsum = reinterpret_cast<int *>(asc + MB * (NGQ + 1));
    float *tl = reinterpret_cast<float *>(xsum + MB * (K / 64 + 1));
    const float *x = sel.x;

    // ---- x loads of the first pass (PREP: of the first prepared codes), then the first weight
    // units (unconditional, clamped)
    float4 v[QP];
    const int8_t *pq = L.a.xw ? reinterpret_cast<const int8_t *>(L.a.xw) + (size_t)L.m0 * K : nullptr;
    const int npq = L.mcols * (K >> 4);           // PREP: 16-byte pieces of the columns' codes
    bgl_u32x4 pre[4];
    if constexpr (PREP) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = min((int)threadIdx.x + j * sel.nthreads, npq - 1);
            pre[j] = *(const BGL_GLOBAL bgl_u32x4 *)(pq + (size_t)(i / (K >> 4)) * K + (size_t)(i % (K >> 4)) * 16);
        }
    } else {
        load_xpass<QP, MB>(v, x, wave, nw, K, NP, NPT, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    // PREP: the prepared codes, scales and code sums into the per-column LDS regions
    auto copy_prep = [&]() {
        const int nthr = sel.nthreads;
        auto dst = [&](int i) {
            const int m = i / (K >> 4), o = (i % (K >> 4)) * 16;
            return reinterpret_cast<bgl_u32x4 *>(xq + m * XQS + (o / QU::ELEMS) * QU::STRIDE + o % QU::ELEMS);
        };
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = threadIdx.x + j * nthr;
            if (i < npq) *dst(i) = pre[j];
        }
        for (int i = threadIdx.x + 4 * nthr; i < npq; i += nthr)
            *dst(i) = *(const BGL_GLOBAL bgl_u32x4 *)(pq + (size_t)(i / (K >> 4)) * K + (size_t)(i % (K >> 4)) * 16);
        for (int i = threadIdx.x; i < L.mcols * NGQ; i += nthr)
            asc[(i / NGQ) * (NGQ + 1) + i % NGQ] = L.a.xs[(size_t)(L.m0 + i / NGQ) * NGQ + i % NGQ];
        if constexpr (QU::XSUM) {
            const int n64 = K / 64;
            for (int i = threadIdx.x; i < L.mcols * n64; i += nthr)
                xsum[(i / n64) * (n64 + 1) + i % n64] = L.a.xsum[(size_t)(L.m0 + i / n64) * n64 + i % n64];
        }
    };
    // Waves [0, nwl) own weight units; any further waves of the launch only quantize.  The two
    // roles are separate branches so the weight waves' wait for x is not merged with a path that
    // issued no weight loads.
    constexpr int H = TR <= 32 ? 2 : 1;                  // lanes sharing one unit
    constexpr int UPI = KQ / H;                          // units per wave and iteration
    const int nwl = min(nw, (U + UPI - 1) / UPI);
    if (wave < nwl) {
        const int r = lane % TR, j = lane / TR, kq = j / H, h = j % H, rr = r0 + r;
        int ub = wave * UPI;
        RawPart<FMT, H> c0, c1;
        load_part<FMT, H>(c0, T, tile, rr, min(ub + kq, U - 1), h);
        __builtin_amdgcn_sched_barrier(0);
        // quantize x (q4gemv.h:177-213 / q4gemv_g256.h:72-99).  The first passes stay outside the
        // loop: a loop header joining the back edge (whose x loads are the newest) would make the
        // compiler wait for the weight loads as well.
        if constexpr (PREP) {
            copy_prep();
        } else {
            quant_passes<FMT, QP, MB>(v, wave, nw, K, NP, NPT, NGQ, U, lane, xq, asc, xsum);
            for (int p0 = wave + QP * nw; p0 < NPT; p0 += QP * nw) {
                load_xpass<QP, MB>(v, x, p0, nw, K, NP, NPT, lane);
                quant_passes<FMT, QP, MB>(v, p0, nw, K, NP, NPT, NGQ, U, lane, xq, asc, xsum);
            }
        }
        __syncthreads();
        // per-unit fold terms t[m][u][row]; every lane computes (the partner exchange is wave-wide).
        // One unit's weights serve every column.
        auto emit = [&](const RawPart<FMT, H> &c, int u) {
#pragma unroll
            for (int m = 0; m < MB; m++) {
                int p = unit_part<FMT, H>(c, xq + m * XQS, min(u, U - 1), h);
                if constexpr (H == 2) p += __shfl_xor(p, TR);
                if (h == 0 && u < U)
                    tl[(m * U + u) * TR + r] = unit_float<FMT>(p, c.s, T.gmul, asc + m * (NGQ + 1), xsum + m * (K / 64 + 1), u);
            }
        };
        for (;;) {
            const int un = ub + nwl * UPI, u = ub + kq;
            if (un >= U) {                  // last iteration: no prefetch, so no join before the wait
                emit(c0, u);
                break;
            }
            load_part<FMT, H>(c1, T, tile, rr, min(un + kq, U - 1), h);
            emit(c0, u);
            c0 = c1;
            ub = un;
        }
    } else {
        if constexpr (PREP) {
            copy_prep();
        } else {
            quant_passes<FMT, QP, MB>(v, wave, nw, K, NP, NPT, NGQ, U, lane, xq, asc, xsum);
            for (int p0 = wave + QP * nw; p0 < NPT; p0 += QP * nw) {
                load_xpass<QP, MB>(v, x, p0, nw, K, NP, NPT, lane);
                quant_passes<FMT, QP, MB>(v, p0, nw, K, NP, NPT, NGQ, U, lane, xq, asc, xsum);
            }
        }
        __syncthreads();
    }
    __syncthreads();
    // sequential fold of each (column, row) in group order; the LDS reads go out 8 at a time, one
    // batch ahead of the adds
    const GemvTask &task = L.t[sel.ti];
    auto fold = [&](int m, int rl) {
        const int row = tile * BGL_TILE + r0 + rl;
        if (row >= task.T.N) return;
        float acc = 0.0f;
        const float *tr = tl + (size_t)m * U * TR + rl;
        const int U8 = U & ~7;
        float t8[8], n8[8];
        if (U8) {
#pragma unroll
            for (int i = 0; i < 8; i++) t8[i] = tr[i * TR];
        }
        for (int g = 0; g < U8; g += 8) {
            if (g + 8 < U8) {
#pragma unroll
                for (int i = 0; i < 8; i++) n8[i] = tr[(g + 8 + i) * TR];
            }
#pragma unroll
            for (int i = 0; i < 8; i++) acc = __fadd_rn(acc, t8[i]);
#pragma unroll
            for (int i = 0; i < 8; i++) t8[i] = n8[i];
        }
        for (int g = U8; g < U; g++) acc = __fadd_rn(acc, tr[g * TR]);
        const float bb = task.bias ? task.bias[row] : 0.0f;
        task.y[(size_t)(L.m0 + m) * task.ystride + row] = __fadd_rn(bb, acc);
    };
    if constexpr (MB == 1) {
        if (threadIdx.x < TR) fold(0, threadIdx.x);
    } else {
        for (int t = threadIdx.x; t < MB * TR; t += sel.nthreads)
            if (t / TR < L.mcols) fold(t / TR, t % TR);
    }
}

// ================================================================================== launchers
template <int FMT, int ACT, int NB>
static int launch_mb(int MB, const GemvLaunch &L, int nblocks, int nw, hipStream_t st) {
    dim3 g(nblocks), b(nw * BGL_TILE);
    switch (MB) {
    case 1: hipLaunchKernelGGL((k_gemv<FMT, ACT, NB, 1>), g, b, 0, st, L); break;
    case 4: hipLaunchKernelGGL((k_gemv<FMT, ACT, NB, 4>), g, b, 0, st, L); break;
    case 8: hipLaunchKernelGGL((k_gemv<FMT, ACT, NB, 8>), g, b, 0, st, L); break;
    default: return -1;
    }
    return 0;
}

template <int NB>
static int launch_qng(int MB, const GemvLaunch &L, int nblocks, int nw, hipStream_t st) {
    return launch_mb<BGL_QNG64, BGL_ACT_F32, NB>(MB, L, nblocks, nw, st);
}

int bgl_launch_gemv(int act, int MB, const GemvLaunch &L, int nblocks, int nw, hipStream_t st) {
    const int fmt = L.t[0].T.fmt;
    if (fmt == BGL_Q4G64)
        return act == BGL_ACT_F32 ? launch_mb<BGL_Q4G64, BGL_ACT_F32, 0>(MB, L, nblocks, nw, st)
                                  : launch_mb<BGL_Q4G64, BGL_ACT_W4A8, 0>(MB, L, nblocks, nw, st);
    if (fmt == BGL_Q8G64)
        return act == BGL_ACT_F32 ? launch_mb<BGL_Q8G64, BGL_ACT_F32, 0>(MB, L, nblocks, nw, st)
                                  : launch_mb<BGL_Q8G64, BGL_ACT_W4A8, 0>(MB, L, nblocks, nw, st);
    if (fmt == BGL_Q4G32H) return act == BGL_ACT_F32 ? launch_mb<BGL_Q4G32H, BGL_ACT_F32, 0>(MB, L, nblocks, nw, st) : -2;
    if (fmt == BGL_Q4G256SF) return act == BGL_ACT_W4A8 ? launch_mb<BGL_Q4G256SF, BGL_ACT_W4A8, 0>(MB, L, nblocks, nw, st) : -2;
    if (fmt == BGL_QNG64 && act == BGL_ACT_F32) {
        switch (L.t[0].T.bits) {
        case 2: return launch_qng<2>(MB, L, nblocks, nw, st);
        case 3: return launch_qng<3>(MB, L, nblocks, nw, st);
        case 4: return launch_qng<4>(MB, L, nblocks, nw, st);
        case 5: return launch_qng<5>(MB, L, nblocks, nw, st);
        case 6: return launch_qng<6>(MB, L, nblocks, nw, st);
        case 7: return launch_qng<7>(MB, L, nblocks, nw, st);
        case 8: return launch_qng<8>(MB, L, nblocks, nw, st);
        case 9: return launch_qng<9>(MB, L, nblocks, nw, st);
        case 10: return launch_qng<10>(MB, L, nblocks, nw, st);
        case 11: return launch_qng<11>(MB, L, nblocks, nw, st);
        case 12: return launch_qng<12>(MB, L, nblocks, nw, st);
        case 13: return launch_qng<13>(MB, L, nblocks, nw, st);
        case 14: return launch_qng<14>(MB, L, nblocks, nw, st);
        case 15: return launch_qng<15>(MB, L, nblocks, nw, st);
        default: return -2;
        }
    }
    return -2;
}

size_t bgl_gemv_q_lds(int fmt, int K, int TR, int MB) {
    const int GQ = fmt == BGL_Q4G256SF ? 256 : 64;
    const int ELEMS = fmt == BGL_Q4G256SF ? 256 : 64;
    const int U = K / ELEMS;
    return (size_t)MB * ((size_t)(U + 1) * (ELEMS + 16) + 4 * (size_t)(K / GQ + 1) + 4 * (size_t)(K / 64 + 1) + 4 * (size_t)U * TR);
}

template <int FMT, int QP, int MB, bool PREP = false>
static int launch_q_tr(int TR, const GemvLaunch &L, int nblocks, int nw, size_t lds, hipStream_t st) {
    dim3 g(nblocks), b(nw * BGL_TILE);
    switch (TR) {
    case 64: hipLaunchKernelGGL((k_gemv_q<FMT, 64, QP, MB, PREP>), g, b, lds, st, L); return 0;
    case 32: hipLaunchKernelGGL((k_gemv_q<FMT, 32, QP, MB, PREP>), g, b, lds, st, L); return 0;
    case 16: hipLaunchKernelGGL((k_gemv_q<FMT, 16, QP, MB, PREP>), g, b, lds, st, L); return 0;
    case 8: hipLaunchKernelGGL((k_gemv_q<FMT, 8, QP, MB, PREP>), g, b, lds, st, L); return 0;
    default: return -1;
    }
}

template <int FMT, int MB>
static int launch_q_qp(int QP, int TR, const GemvLaunch &L, int nblocks, int nw, size_t lds, hipStream_t st) {
    switch (QP) {
    case 1: return launch_q_tr<FMT, 1, MB>(TR, L, nblocks, nw, lds, st);
    case 2: return launch_q_tr<FMT, 2, MB>(TR, L, nblocks, nw, lds, st);
    default: return launch_q_tr<FMT, 4, MB>(TR, L, nblocks, nw, lds, st);
    }
}

template <int FMT>
static int launch_q_mb(int MB, int QP, int TR, const GemvLaunch &L, int nblocks, int nw, size_t lds, hipStream_t st) {
    if (L.a.xw) {                                  // prepared codes (QP is unused)
        switch (MB) {
        case 4: return launch_q_tr<FMT, 1, 4, true>(TR, L, nblocks, nw, lds, st);
        case 8: return launch_q_tr<FMT, 1, 8, true>(TR, L, nblocks, nw, lds, st);
        default: return -1;
        }
    }
    switch (MB) {
    case 1: return launch_q_qp<FMT, 1>(QP, TR, L, nblocks, nw, lds, st);
    case 4: return launch_q_qp<FMT, 4>(QP, TR, L, nblocks, nw, lds, st);
    case 8: return launch_q_qp<FMT, 8>(QP, TR, L, nblocks, nw, lds, st);
    default: return -1;
    }
}

// ntiles counts 64-row tiles; each is split into 64/TR workgroups.  MB columns (1, 4 or 8) per
// launch, L.mcols of them real.  With L.a.xw set (MB 4 or 8) the workgroups copy the columns' int8
// codes, scales and code sums prepared by k_act_w4a8 (the same codes the fused quantization makes)
// instead of quantizing every column themselves.  QP (quantization passes per wave loaded up front) covers a wave's
// whole share of the MB*ceil(K/256) passes when that is <= 4.  (8 passes up front for the 4- and
// 8-column launches measured no faster.)
int bgl_launch_gemv_q(const GemvLaunch &L, int ntiles, int TR, int nw, int MB, hipStream_t st) {
    const int fmt = L.t[0].T.fmt, K = L.t[0].T.K;
    if (K < 64 || K % 64) return -1;
    const size_t lds = bgl_gemv_q_lds(fmt, K, TR, MB);
    const int nblocks = ntiles * (BGL_TILE / TR);
    const int pw = (MB * ((K + 255) / 256) + nw - 1) / nw;
    const int QP = pw <= 1 ? 1 : pw <= 2 ? 2 : 4;
    switch (fmt) {
    case BGL_Q4G256SF: return launch_q_mb<BGL_Q4G256SF>(MB, QP, TR, L, nblocks, nw, lds, st);
    case BGL_Q4G64: return launch_q_mb<BGL_Q4G64>(MB, QP, TR, L, nblocks, nw, lds, st);
    case BGL_Q8G64: return launch_q_mb<BGL_Q8G64>(MB, QP, TR, L, nblocks, nw, lds, st);
    default: return -2;
    }
}
