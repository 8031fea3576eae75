// bgl_gemv.hip -- the quantized GEMV / small-M GEMM kernel family (one kernel template per format).
//
// Work decomposition: a workgroup of 4 wavefronts owns one 64-row tile and a contiguous range of
// work units along K; lane = row, so every wave-wide weight load is a contiguous 1 KB run and the
// activation operands are wave-uniform (scalar loads, SGPR operands of v_dot4).  Each wave walks
// units w, w+4, ... of the range, folding each unit's contribution into per-column fp32
// accumulators; the 4 waves are combined in LDS in fixed order.  When K is split over several
// workgroups (ks > 1) each writes its partial to a scratch buffer and the last one to arrive
// (device-scope counter, reset by that same block) sums them in block order, so results are
// deterministic run to run.
//
// Arithmetic: weight codes are exact integers.  fp32 activations arrive as three int8 digits of an
// exact fixed-point value (see bgl_device.h), W4A8 activations as the reference's int8 codes; all
// products are exact int32 dot4 sums, and fp32 only enters in the per-unit scale fold.
#include "bgl_kernels.h"

#define C63 (1.0f / 63.0f)

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

// digit sums of one 32-element half (3 ints, padded to 4)
__device__ __forceinline__ int4 ld_dsum(const GemvAct &A, int am, int K, int half) {
    ucint p = uni(A.xsum) + ((size_t)am * (K >> 5) + half) * 4;
    return make_int4(p[0], p[1], p[2], p[3]);
}

__device__ __forceinline__ float fold_digits(int t0, int t1, int t2) {
    return (float)t0 + 256.0f * (float)t1 + 65536.0f * (float)t2;
}

// ---------------------------------------------------------------------------------- Q4G64
template <int ACT, int MB>
__device__ __forceinline__ void unit_q4g64(const BglDevTensor &T, int tile, int lane, int u, const GemvAct &A,
                                           const Cols<MB> &C, float (&acc)[MB]) {
    const uint4 *cp = reinterpret_cast<const uint4 *>(T.w) + ((size_t)tile * T.cpr + (size_t)u * 2) * BGL_TILE + lane;
    uint4 c0 = cp[0], c1 = cp[BGL_TILE];
    float s = reinterpret_cast<const float *>(T.s0)[((size_t)tile * T.nunits + u) * BGL_TILE + lane];
    int lo[8], hi[8];
    uint32_t raw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
    for (int q = 0; q < 8; q++) { lo[q] = nib_lo(raw[q]); hi[q] = nib_hi(raw[q]); }
    const int K = T.K, ng = K >> 6;
#pragma unroll
    for (int m = 0; m < MB; m++) {
        int am = C.am[m];
        if (ACT == BGL_ACT_F32) {
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
            float V = fold_digits(t0, t1, t2);
            acc[m] += s * (V * uni(A.xs)[(size_t)am * ng + u]);
        } else {
            ucint xq = uni(A.xw) + (size_t)am * (K >> 2) + (size_t)u * 16;
            int isum = 0;
#pragma unroll
            for (int q = 0; q < 8; q++) { isum = dot4(lo[q], xq[2 * q], isum); isum = dot4(hi[q], xq[2 * q + 1], isum); }
            isum -= 8 * uni(A.xsum)[(size_t)am * ng + u];
            float t = __fmul_rn(__fmul_rn((float)isum, s), uni(A.xs)[(size_t)am * ng + u]);
            acc[m] = __fadd_rn(acc[m], t);
        }
    }
}

// ---------------------------------------------------------------------------------- Q4G32H (fp32 act)
template <int MB>
__device__ __forceinline__ void unit_q4g32h(const BglDevTensor &T, int tile, int lane, int u, const GemvAct &A,
                                            const Cols<MB> &C, float (&acc)[MB]) {
    const uint4 *cp = reinterpret_cast<const uint4 *>(T.w) + ((size_t)tile * T.cpr + (size_t)u * 2) * BGL_TILE + lane;
    uint4 c0 = cp[0], c1 = cp[BGL_TILE];
    uint32_t s2 = reinterpret_cast<const uint32_t *>(T.s0)[((size_t)tile * T.nunits + u) * BGL_TILE + lane];
    float sa = __half2float(__ushort_as_half((unsigned short)(s2 & 0xffffu)));
    float sb = __half2float(__ushort_as_half((unsigned short)(s2 >> 16)));
    int lo[8], hi[8];
    uint32_t raw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
    for (int q = 0; q < 8; q++) { lo[q] = nib_lo(raw[q]); hi[q] = nib_hi(raw[q]); }
    const int K = T.K, ng = K >> 6;
#pragma unroll
    for (int m = 0; m < MB; m++) {
        int am = C.am[m];
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

// ---------------------------------------------------------------------------------- G256SF (W4A8)
template <int MB>
__device__ __forceinline__ void unit_g256sf(const BglDevTensor &T, int tile, int lane, int u, const GemvAct &A,
                                            const Cols<MB> &C, float (&acc)[MB]) {
    const uint4 *cp = reinterpret_cast<const uint4 *>(T.w) + ((size_t)tile * T.cpr + (size_t)u * 8) * BGL_TILE + lane;
    uint4 ch[8];
#pragma unroll
    for (int k = 0; k < 8; k++) ch[k] = cp[k * BGL_TILE];
    size_t so = ((size_t)tile * T.nunits + u) * BGL_TILE + lane;
    float ws = reinterpret_cast<const float *>(T.s0)[so];
    uint32_t sub4 = T.s1[so];
    int lo[32], hi[32];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        lo[4 * k] = nib_lo(ch[k].x); hi[4 * k] = nib_hi(ch[k].x);
        lo[4 * k + 1] = nib_lo(ch[k].y); hi[4 * k + 1] = nib_hi(ch[k].y);
        lo[4 * k + 2] = nib_lo(ch[k].z); hi[4 * k + 2] = nib_hi(ch[k].z);
        lo[4 * k + 3] = nib_lo(ch[k].w); hi[4 * k + 3] = nib_hi(ch[k].w);
    }
    const int K = T.K;
#pragma unroll
    for (int m = 0; m < MB; m++) {
        int am = C.am[m];
        ucint xq = uni(A.xw) + (size_t)am * (K >> 2) + (size_t)u * 64;
        ucint xs = uni(A.xsum) + (size_t)am * (K >> 6) + (size_t)u * 4;
        int comb = 0;
#pragma unroll
        for (int sg = 0; sg < 4; sg++) {
            int isum = 0;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                isum = dot4(lo[8 * sg + q], xq[16 * sg + 2 * q], isum);
                isum = dot4(hi[8 * sg + q], xq[16 * sg + 2 * q + 1], isum);
            }
            isum -= 8 * xs[sg];
            comb += isum * (int)((sub4 >> (8 * sg)) & 255u);
        }
        float t = __fmul_rn(__fmul_rn(__fmul_rn((float)comb, ws), C63), uni(A.xs)[(size_t)am * (K >> 8) + u]);
        acc[m] = __fadd_rn(acc[m], t);
    }
}

// ---------------------------------------------------------------------------------- Q8G64
template <int ACT, int MB>
__device__ __forceinline__ void unit_q8g64(const BglDevTensor &T, int tile, int lane, int u, const GemvAct &A,
                                           const Cols<MB> &C, float (&acc)[MB]) {
    const uint4 *cp = reinterpret_cast<const uint4 *>(T.w) + ((size_t)tile * T.cpr + (size_t)u * 4) * BGL_TILE + lane;
    int w[16];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint4 c = cp[k * BGL_TILE];
        w[4 * k] = (int)c.x; w[4 * k + 1] = (int)c.y; w[4 * k + 2] = (int)c.z; w[4 * k + 3] = (int)c.w;
    }
    float s = reinterpret_cast<const float *>(T.s0)[((size_t)tile * T.nunits + u) * BGL_TILE + lane];
    const int K = T.K, ng = K >> 6;
#pragma unroll
    for (int m = 0; m < MB; m++) {
        int am = C.am[m];
        if (ACT == BGL_ACT_F32) {
            ucint xg = uni(A.xw) + ((size_t)am * ng + u) * BGL_XD_DW;
            int t0 = 0, t1 = 0, t2 = 0;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                t0 = dot4(w[q], xg[q], t0); t1 = dot4(w[q], xg[16 + q], t1); t2 = dot4(w[q], xg[32 + q], t2);
            }
            float V = fold_digits(t0, t1, t2);
            acc[m] += s * (V * uni(A.xs)[(size_t)am * ng + u]);
        } else {
            ucint xq = uni(A.xw) + (size_t)am * (K >> 2) + (size_t)u * 16;
            int isum = 0;
#pragma unroll
            for (int q = 0; q < 16; q++) isum = dot4(w[q], xq[q], isum);
            float t = __fmul_rn(__fmul_rn((float)isum, s), uni(A.xs)[(size_t)am * ng + u]);
            acc[m] = __fadd_rn(acc[m], t);
        }
    }
}

// ---------------------------------------------------------------------------------- QNG64 (fp32 act)
template <int NB, int MB>
__device__ __forceinline__ void unit_qng64(const BglDevTensor &T, int tile, int lane, int u, const GemvAct &A,
                                           const Cols<MB> &C, float (&acc)[MB]) {
    constexpr int H8 = (NB >> 3) & 1, H4 = (NB >> 2) & 1, H2 = (NB >> 1) & 1, H1 = NB & 1;
    constexpr int K4 = 8 * H8, K2 = K4 + 4 * H4, K1 = K2 + 2 * H2;
    constexpr int SH4 = 8 * H8, SH2 = SH4 + 4 * H4, SH1 = SH2 + 2 * H2;
    constexpr int CORR = 128 * H8 - (1 << (NB - 1));
    const uint4 *cp = reinterpret_cast<const uint4 *>(T.w) + ((size_t)tile * T.cpr + (size_t)u * NB) * BGL_TILE + lane;
    uint4 ch[NB];
#pragma unroll
    for (int k = 0; k < NB; k++) ch[k] = cp[k * BGL_TILE];
    float2 s2 = reinterpret_cast<const float2 *>(T.s0)[((size_t)tile * T.nunits + u) * BGL_TILE + lane];
    const int K = T.K, ng = K >> 6;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int g = 2 * u + h;
        if (g >= ng) break;
        const float s = h ? s2.y : s2.x;
        // unpack this half's fields into byte lanes (element order = x dword order)
        int f8[16], f4[16], f2[16], f1[16];
        if (H8) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                uint4 c = ch[4 * h + k];
                f8[4 * k] = (int)c.x; f8[4 * k + 1] = (int)c.y; f8[4 * k + 2] = (int)c.z; f8[4 * k + 3] = (int)c.w;
            }
        }
        if (H4) {
#pragma unroll
            for (int k = 0; k < 2; k++) {
                uint4 c = ch[K4 + 2 * h + k];
                uint32_t r4[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
                for (int j = 0; j < 4; j++) { f4[8 * k + 2 * j] = nib_lo(r4[j]); f4[8 * k + 2 * j + 1] = nib_hi(r4[j]); }
            }
        }
        if (H2) {
            uint4 c = ch[K2 + h];
            uint32_t r2[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int t = 0; t < 4; t++) f2[4 * j + t] = (int)((r2[j] >> (2 * t)) & 0x03030303u);
        }
        if (H1) {
            uint4 c = ch[K1];
            uint32_t r1[2] = {h ? c.z : c.x, h ? c.w : c.y};
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int t = 0; t < 8; t++) f1[8 * j + t] = (int)((r1[j] >> t) & 0x01010101u);
        }
#pragma unroll
        for (int m = 0; m < MB; m++) {
            int am = C.am[m];
            ucint xg = uni(A.xw) + ((size_t)am * ng + g) * BGL_XD_DW;
            int td[3];
#pragma unroll
            for (int d = 0; d < 3; d++) {
                ucint xd = xg + 16 * d;
                int tot = 0;
                if (H8) {
                    int a = 0;
#pragma unroll
                    for (int q = 0; q < 16; q++) a = dot4(f8[q], xd[q], a);
                    tot += a;
                }
                if (H4) {
                    int a = 0;
#pragma unroll
                    for (int q = 0; q < 16; q++) a = dot4(f4[q], xd[q], a);
                    tot += a * (1 << SH4);
                }
                if (H2) {
                    int a = 0;
#pragma unroll
                    for (int q = 0; q < 16; q++) a = dot4(f2[q], xd[q], a);
                    tot += a * (1 << SH2);
                }
                if (H1) {
                    int a = 0;
#pragma unroll
                    for (int q = 0; q < 16; q++) a = dot4(f1[q], xd[q], a);
                    tot += a * (1 << SH1);
                }
                td[d] = tot;
            }
            int4 d0 = ld_dsum(A, am, K, 2 * g), d1 = ld_dsum(A, am, K, 2 * g + 1);
            td[0] += CORR * (d0.x + d1.x); td[1] += CORR * (d0.y + d1.y); td[2] += CORR * (d0.z + d1.z);
            float V = fold_digits(td[0], td[1], td[2]);
            acc[m] += s * (V * uni(A.xs)[(size_t)am * ng + g]);
        }
    }
}

// ---------------------------------------------------------------------------------- kernel
template <int FMT, int ACT, int NB, int MB>
__device__ __forceinline__ void unit_dispatch(const BglDevTensor &T, int tile, int lane, int u, const GemvAct &A,
                                              const Cols<MB> &C, float (&acc)[MB]) {
    if constexpr (FMT == BGL_Q4G64) unit_q4g64<ACT, MB>(T, tile, lane, u, A, C, acc);
    else if constexpr (FMT == BGL_Q4G32H) unit_q4g32h<MB>(T, tile, lane, u, A, C, acc);
    else if constexpr (FMT == BGL_Q4G256SF) unit_g256sf<MB>(T, tile, lane, u, A, C, acc);
    else if constexpr (FMT == BGL_Q8G64) unit_q8g64<ACT, MB>(T, tile, lane, u, A, C, acc);
    else unit_qng64<NB, MB>(T, tile, lane, u, A, C, acc);
}

template <int FMT, int ACT, int NB, int MB>
__global__ __launch_bounds__(BGL_WAVES * BGL_TILE) void k_gemv(GemvLaunch L) {
    __shared__ float red[BGL_WAVES][MB][BGL_TILE];
    const int b = blockIdx.x;
    int ti = 0;
#pragma unroll
    for (int i = 1; i < BGL_MAX_TASKS; i++) if (i < L.ntasks && b >= L.t[i].blk0) ti = i;
    GemvTask task = L.t[0];
#pragma unroll
    for (int i = 1; i < BGL_MAX_TASKS; i++) if (i == ti) task = L.t[i];
    const BglDevTensor &T = task.T;
    const int lb = b - task.blk0, tile = lb / task.ks, s = lb % task.ks;
    const int ubeg = s * task.gpb;
    const int uend = min(ubeg + task.gpb, T.nunits);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const Cols<MB> C = col_rows<MB>(L.a, L.m0, L.mcols);

    float acc[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) acc[m] = 0.0f;
    for (int u = ubeg + wave; u < uend; u += BGL_WAVES) unit_dispatch<FMT, ACT, NB, MB>(T, tile, lane, u, L.a, C, acc);

#pragma unroll
    for (int m = 0; m < MB; m++) red[wave][m][lane] = acc[m];
    __syncthreads();
    if (wave != 0) return;
    float p[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) {
        float v = red[0][m][lane];
#pragma unroll
        for (int w = 1; w < BGL_WAVES; w++) v += red[w][m][lane];
        p[m] = v;
    }
    const int row = tile * BGL_TILE + lane;
    if (task.ks > 1) {
        float *tb = L.tbuf + task.tb_off + ((size_t)tile * task.ks + s) * MB * BGL_TILE;
#pragma unroll
        for (int m = 0; m < MB; m++) tb[m * BGL_TILE + lane] = p[m];
        __threadfence();
        unsigned old = 0;
        if (lane == 0) old = atomicAdd(&L.ctr[task.ctr_off + tile], 1u);
        old = __shfl(old, 0, 64);
        if (old != (unsigned)(task.ks - 1)) return;
        __threadfence();
        const float *tb0 = L.tbuf + task.tb_off + (size_t)tile * task.ks * MB * BGL_TILE;
#pragma unroll
        for (int m = 0; m < MB; m++) {
            float v = __hip_atomic_load(tb0 + m * BGL_TILE + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (int s2 = 1; s2 < task.ks; s2++)
                v += __hip_atomic_load(tb0 + ((size_t)s2 * MB + m) * BGL_TILE + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            p[m] = v;
        }
        if (lane == 0) __hip_atomic_store(&L.ctr[task.ctr_off + tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (row < T.N) {
        const float bb = task.bias ? task.bias[row] : 0.0f;
#pragma unroll
        for (int m = 0; m < MB; m++)
            if (m < L.mcols) task.y[(size_t)(L.m0 + m) * task.ystride + row] = bb + p[m];
    }
}

// ---------------------------------------------------------------------------------- launcher
template <int FMT, int ACT, int NB>
static int launch_mb(int MB, const GemvLaunch &L, int nblocks, hipStream_t st) {
    dim3 g(nblocks), b(BGL_WAVES * BGL_TILE);
    switch (MB) {
    case 1: hipLaunchKernelGGL((k_gemv<FMT, ACT, NB, 1>), g, b, 0, st, L); break;
    case 4: hipLaunchKernelGGL((k_gemv<FMT, ACT, NB, 4>), g, b, 0, st, L); break;
    case 8: hipLaunchKernelGGL((k_gemv<FMT, ACT, NB, 8>), g, b, 0, st, L); break;
    default: return -1;
    }
    return 0;
}

template <int NB>
static int launch_qng(int MB, const GemvLaunch &L, int nblocks, hipStream_t st) {
    return launch_mb<BGL_QNG64, BGL_ACT_F32, NB>(MB, L, nblocks, st);
}

int bgl_launch_gemv(int act, int MB, const GemvLaunch &L, int nblocks, hipStream_t st) {
    const int fmt = L.t[0].T.fmt;
    if (fmt == BGL_Q4G64)
        return act == BGL_ACT_F32 ? launch_mb<BGL_Q4G64, BGL_ACT_F32, 0>(MB, L, nblocks, st)
                                  : launch_mb<BGL_Q4G64, BGL_ACT_W4A8, 0>(MB, L, nblocks, st);
    if (fmt == BGL_Q8G64)
        return act == BGL_ACT_F32 ? launch_mb<BGL_Q8G64, BGL_ACT_F32, 0>(MB, L, nblocks, st)
                                  : launch_mb<BGL_Q8G64, BGL_ACT_W4A8, 0>(MB, L, nblocks, st);
    if (fmt == BGL_Q4G32H) return act == BGL_ACT_F32 ? launch_mb<BGL_Q4G32H, BGL_ACT_F32, 0>(MB, L, nblocks, st) : -2;
    if (fmt == BGL_Q4G256SF) return act == BGL_ACT_W4A8 ? launch_mb<BGL_Q4G256SF, BGL_ACT_W4A8, 0>(MB, L, nblocks, st) : -2;
    if (fmt == BGL_QNG64 && act == BGL_ACT_F32) {
        switch (L.t[0].T.bits) {
        case 2: return launch_qng<2>(MB, L, nblocks, st);
        case 3: return launch_qng<3>(MB, L, nblocks, st);
        case 4: return launch_qng<4>(MB, L, nblocks, st);
        case 5: return launch_qng<5>(MB, L, nblocks, st);
        case 6: return launch_qng<6>(MB, L, nblocks, st);
        case 7: return launch_qng<7>(MB, L, nblocks, st);
        case 8: return launch_qng<8>(MB, L, nblocks, st);
        case 9: return launch_qng<9>(MB, L, nblocks, st);
        case 10: return launch_qng<10>(MB, L, nblocks, st);
        case 11: return launch_qng<11>(MB, L, nblocks, st);
        case 12: return launch_qng<12>(MB, L, nblocks, st);
        case 13: return launch_qng<13>(MB, L, nblocks, st);
        case 14: return launch_qng<14>(MB, L, nblocks, st);
        case 15: return launch_qng<15>(MB, L, nblocks, st);
        default: return -2;
        }
    }
    return -2;
}
