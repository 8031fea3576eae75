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
// Dynamic LDS: [xq: U x (unit bytes + 16)][ascale: K/gq][xqsum: K/64][t: U x TR floats].

template <int FMT> struct QUnit {
    static constexpr int GQ = FMT == BGL_Q4G256SF ? 256 : 64;        // activation quantization group
    static constexpr int ELEMS = FMT == BGL_Q4G256SF ? 256 : 64;     // elements per work unit
    static constexpr int STRIDE = ELEMS + 16;                       // padded LDS bytes per unit
};

template <int FMT>
__device__ __forceinline__ void load_raw_row(Raw<FMT, 0> &r, const BglDevTensor &T, int tile, int rr, int u) {
    constexpr int CPU = chunks_per_unit<FMT>(0);
    const uint4 *cp = reinterpret_cast<const uint4 *>(T.w) + ((size_t)tile * T.cpr + (size_t)u * CPU) * BGL_TILE + rr;
#pragma unroll
    for (int k = 0; k < CPU; k++) r.c[k] = cp[k * BGL_TILE];
    const size_t so = ((size_t)tile * T.nunits + u) * BGL_TILE + rr;
    r.s = reinterpret_cast<const float *>(T.s0)[so];
    if constexpr (FMT == BGL_Q4G256SF) r.sub = T.s1[so];
}

template <int FMT>
__device__ __forceinline__ float unit_term(const Raw<FMT, 0> &r, const int8_t *xq, const float *asc, const int *xsum, int u) {
    const int4 *x4 = reinterpret_cast<const int4 *>(xq + (size_t)u * QUnit<FMT>::STRIDE);
    if constexpr (FMT == BGL_Q4G256SF) {
        int comb = 0;
#pragma unroll
        for (int sg = 0; sg < 4; sg++) {
            int isum = 0;
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const uint4 c = r.c[2 * sg + k];
                const int4 xa = x4[sg * 4 + 2 * k], xb = x4[sg * 4 + 2 * k + 1];
                isum = dot4(nib_lo(c.x), xa.x, isum); isum = dot4(nib_hi(c.x), xa.y, isum);
                isum = dot4(nib_lo(c.y), xa.z, isum); isum = dot4(nib_hi(c.y), xa.w, isum);
                isum = dot4(nib_lo(c.z), xb.x, isum); isum = dot4(nib_hi(c.z), xb.y, isum);
                isum = dot4(nib_lo(c.w), xb.z, isum); isum = dot4(nib_hi(c.w), xb.w, isum);
            }
            isum -= 8 * xsum[u * 4 + sg];
            comb += isum * (int)((r.sub >> (8 * sg)) & 255u);
        }
        return __fmul_rn(__fmul_rn(__fmul_rn((float)comb, r.s), C63), asc[u]);
    } else if constexpr (FMT == BGL_Q4G64) {
        int isum = 0;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint4 c = r.c[k];
            const int4 xa = x4[2 * k], xb = x4[2 * k + 1];
            isum = dot4(nib_lo(c.x), xa.x, isum); isum = dot4(nib_hi(c.x), xa.y, isum);
            isum = dot4(nib_lo(c.y), xa.z, isum); isum = dot4(nib_hi(c.y), xa.w, isum);
            isum = dot4(nib_lo(c.z), xb.x, isum); isum = dot4(nib_hi(c.z), xb.y, isum);
            isum = dot4(nib_lo(c.w), xb.z, isum); isum = dot4(nib_hi(c.w), xb.w, isum);
        }
        isum -= 8 * xsum[u];
        return __fmul_rn(__fmul_rn((float)isum, r.s), asc[u]);
    } else {
        int isum = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint4 c = r.c[k];
            const int4 xa = x4[k];
            isum = dot4((int)c.x, xa.x, isum); isum = dot4((int)c.y, xa.y, isum);
            isum = dot4((int)c.z, xa.z, isum); isum = dot4((int)c.w, xa.w, isum);
        }
        return __fmul_rn(__fmul_rn((float)isum, r.s), asc[u]);
    }
}

template <int FMT, int TR>
__global__ __launch_bounds__(MAXW * BGL_TILE) void k_gemv_q(GemvLaunch L) {
    extern __shared__ __align__(16) unsigned char lds[];
    constexpr int KQ = BGL_TILE / TR, SUBS = BGL_TILE / TR;
    using QU = QUnit<FMT>;
    const int b = blockIdx.x, ti = pick_task(L, b);
    GemvTask task = L.t[0];
#pragma unroll
    for (int i = 1; i < BGL_MAX_TASKS; i++) if (i == ti) task = L.t[i];
    const BglDevTensor &T = task.T;
    const int lb = b - task.blk0, tile = lb / SUBS, r0 = (lb % SUBS) * TR;
    const int nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int K = T.K, U = T.nunits;
    int8_t *xq = reinterpret_cast<int8_t *>(lds);
    float *asc = reinterpret_cast<float *>(lds + (size_t)U * QU::STRIDE);
    int *xsum = reinterpret_cast<int *>(asc + K / QU::GQ);
    float *tl = reinterpret_cast<float *>(xsum + K / 64);

    // ---- first weight loads go out before the activation work (they do not depend on it)
    const int r = lane % TR, kq = lane / TR, rr = r0 + r;
    int ub = wave * KQ;
    Raw<FMT, 0> c0, c1;
    if (ub + kq < U) load_raw_row<FMT>(c0, T, tile, rr, ub + kq);

    // ---- quantize x (q4gemv.h:177-213 / q4gemv_g256.h:72-99), one wave per group; each wave
    // first loads every group it owns (up to 4 per pass) so the loads overlap
    const float *x = L.x + (size_t)L.m0 * K;
    constexpr int PER = QU::GQ / 64;
    const int NGQ = K / QU::GQ;
    for (int g0 = wave; g0 < NGQ; g0 += 4 * nw) {
        float v[4][PER];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int g = g0 + i * nw;
#pragma unroll
            for (int j = 0; j < PER; j++) v[i][j] = g < NGQ ? x[g * QU::GQ + 64 * j + lane] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int g = g0 + i * nw;
            if (g >= NGQ) break;
            float mx = 1e-8f;
#pragma unroll
            for (int j = 0; j < PER; j++) mx = fmaxf(mx, fabsf(v[i][j]));
            mx = wave_max_f32(mx);
            const float sc = __fdiv_rn(mx, 127.0f), inv = __fdiv_rn(1.0f, sc);
            if (lane == 0) asc[g] = sc;
#pragma unroll
            for (int j = 0; j < PER; j++) {
                const float p = __fmul_rn(v[i][j], inv);
                const float t = __fadd_rn(p, p >= 0.0f ? 0.5f : -0.5f);
                int q = (int)t;                                // |t| <= 128: no int32 overflow
                q = q > 127 ? 127 : (q < -128 ? -128 : q);
                const int e = g * QU::GQ + 64 * j + lane;      // element index
                xq[(e / QU::ELEMS) * QU::STRIDE + e % QU::ELEMS] = (int8_t)q;
                const int s = wave_sum_i32(q);
                if (lane == 0) xsum[g * PER + j] = s;
            }
        }
    }
    __syncthreads();

    // ---- per-unit fold terms t[u][row], exactly the reference's per-group expression
    while (ub < U) {
        const int un = ub + nw * KQ;
        if (un + kq < U) load_raw_row<FMT>(c1, T, tile, rr, un + kq);
        const int u = ub + kq;
        if (u < U) tl[u * TR + r] = unit_term<FMT>(c0, xq, asc, xsum, u);
        c0 = c1;
        ub = un;
    }
    __syncthreads();
    if (threadIdx.x >= TR) return;
    const int row = tile * BGL_TILE + r0 + threadIdx.x;
    if (row >= T.N) return;
    // sequential fold in group order; the LDS reads are batched 8 at a time
    float acc = 0.0f;
    const float *tr = tl + threadIdx.x;
    int g = 0;
    for (; g + 8 <= U; g += 8) {
        float t8[8];
#pragma unroll
        for (int i = 0; i < 8; i++) t8[i] = tr[(g + i) * TR];
#pragma unroll
        for (int i = 0; i < 8; i++) acc = __fadd_rn(acc, t8[i]);
    }
    for (; g < U; g++) acc = __fadd_rn(acc, tr[g * TR]);
    const float bb = task.bias ? task.bias[row] : 0.0f;
    task.y[(size_t)L.m0 * task.ystride + row] = __fadd_rn(bb, acc);
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

size_t bgl_gemv_q_lds(int fmt, int K, int TR) {
    const int GQ = fmt == BGL_Q4G256SF ? 256 : 64;
    const int ELEMS = fmt == BGL_Q4G256SF ? 256 : 64;
    const int U = K / ELEMS;
    return (size_t)U * (ELEMS + 16) + 4 * (K / GQ) + 4 * (K / 64) + 4 * (size_t)U * TR;
}

template <int FMT>
static int launch_q_tr(int TR, const GemvLaunch &L, int nblocks, int nw, size_t lds, hipStream_t st) {
    dim3 g(nblocks), b(nw * BGL_TILE);
    switch (TR) {
    case 64: hipLaunchKernelGGL((k_gemv_q<FMT, 64>), g, b, lds, st, L); return 0;
    case 32: hipLaunchKernelGGL((k_gemv_q<FMT, 32>), g, b, lds, st, L); return 0;
    case 16: hipLaunchKernelGGL((k_gemv_q<FMT, 16>), g, b, lds, st, L); return 0;
    case 8: hipLaunchKernelGGL((k_gemv_q<FMT, 8>), g, b, lds, st, L); return 0;
    default: return -1;
    }
}

// nblocks counts 64-row tiles; each is split into 64/TR workgroups.
int bgl_launch_gemv_q(const GemvLaunch &L, int ntiles, int TR, int nw, hipStream_t st) {
    const int fmt = L.t[0].T.fmt;
    const size_t lds = bgl_gemv_q_lds(fmt, L.t[0].T.K, TR);
    const int nblocks = ntiles * (BGL_TILE / TR);
    switch (fmt) {
    case BGL_Q4G256SF: return launch_q_tr<BGL_Q4G256SF>(TR, L, nblocks, nw, lds, st);
    case BGL_Q4G64: return launch_q_tr<BGL_Q4G64>(TR, L, nblocks, nw, lds, st);
    case BGL_Q8G64: return launch_q_tr<BGL_Q8G64>(TR, L, nblocks, nw, lds, st);
    default: return -2;
    }
}
