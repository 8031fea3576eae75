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
#include "bgl_gemv_q.h"

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
// (building blocks in bgl_gemv_q.h)

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
