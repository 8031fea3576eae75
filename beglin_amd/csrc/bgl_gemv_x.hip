// bgl_gemv_x.hip -- the one-column fp32-activation GEMV (q4gemv.h:761-769 gemm_qXg64_mt at M=1,
// qng64_dense.c:70-79 qng64_matvec_f32; int4 g64, int4 g32 fp16-scale, int8 g64, qNg64 n=2..15).
//
// Work decomposition (the shape of the fused W4A8 kernel): a workgroup owns TR rows of a 64-row
// tile and the whole K range, so no launch needs a K split or a second reduction kernel.  Lane l
// of a wave handles row l % TR and group kq = l / TR of each slot of KQ = 64/TR consecutive
// 64-groups, so each wave-wide weight load is KQ runs of TR*16 >= 128 contiguous bytes.  The
// workgroup's waves take the slots in turn, each keeping up to D of its slots in flight.
//
// The activation records of the whole K range (bgl_gemv_x.h) sit in LDS: copied from the prep
// kernel's output, or (FUSE) made by the workgroup itself from the raw column; the first loads go
// out before the weights' so their latency hides under the weights'.  Lanes of one group read the
// same record (a broadcast).
#include "bgl_gemv_x.h"

// dwords of the row-partial area: nw waves x TR rows, rounded to 4 (16-byte alignment after it)
__host__ __device__ constexpr int x_red_dw(int TR, int nw) { return (nw * TR + 3) & ~3; }

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
    const float *xr = (FUSE ? L.x : L.a.xf) + (size_t)m * K;
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
        // the level-1 ratio of every group (its digits stay in global memory: only the cold path reads them)
        const float *xsc1 = L.a.xs1 + (size_t)m * G;
        for (int g = threadIdx.x; g < G; g += nthr) xl[g * XREC_DW + XREC_SCALE + 1] = __float_as_int(xsc1[g]);
    }
    // records of the last slot's groups past K: zero digits, sums, flags and scales (a zero term for
    // any weight)
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
    // slots whose records carry a level-1 residual or non-finite values: their weights again (cold)
    {
        int fl = 0;
        for (int i = 0; i < ns; i++) fl |= xk[(wave + i * nw) * (KQ * XREC_DW) + XREC_DSUM + 3];
        if (__builtin_amdgcn_ballot_w64(fl != 0)) {
            const XRow xrow{&T, tile * BGL_TILE + rr, xr};
            int *scr = xl + S * KQ * XREC_DW + x_red_dw(TR, nw) + wave * KQ * XREC_DW;   // this wave's level-1 records
            for (int i = 0; i < ns; i++) {
                const int sl = wave + i * nw, gl = min(sl * KQ + kq, G - 1);
                const int *rec = xk + sl * (KQ * XREC_DW);
                const int f2 = rec[XREC_DSUM + 3];
                if (!__builtin_amdgcn_ballot_w64(f2 != 0)) continue;
                const int *r1;
                int4 e0, e1;
                if constexpr (FUSE) {
                    // the slot's level-1 records, made from the raw column into this wave's scratch
                    if (__builtin_amdgcn_ballot_w64(f2 & BGL_XF_L1)) {
                        const int g0 = sl * KQ, g1 = min(g0 + KQ, G);
                        for (int p = g0 >> 2; p <= (g1 - 1) >> 2; p++) x_pass_l1(x_pass_load(xr, p, lane, K), p, lane, g0, g1, scr);
                        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                        __builtin_amdgcn_wave_barrier();
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    }
                    r1 = scr + kq * XREC_DW;
                    e0 = *reinterpret_cast<const int4 *>(r1 + XREC_DSUM);
                    e1 = *reinterpret_cast<const int4 *>(r1 + XREC_DSUM + 4);
                } else {
                    // the prep kernel's level-1 digits, read from global memory
                    r1 = L.a.xw1 + ((size_t)m * G + gl) * BGL_XD_DW;
                    const int *d1 = L.a.xsum1 + ((size_t)m * (K >> 5) + 2 * gl) * 4;
                    e0 = *reinterpret_cast<const int4 *>(d1);
                    e1 = *reinterpret_cast<const int4 *>(d1 + 4);
                }
                XRaw<FMT, NB> rf;
                x_load<FMT, NB, KQ>(rf, R, lane_of(sl), sl, true);
                acc += x_fix<FMT, NB>(x_decode<FMT, NB>(rf), rec, r1, e0, e1, xrow, gl);
            }
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

// Records of every slot's groups (K/64 rounded up to the slot width 64/TR), the row partials, and
// with in-kernel digits one slot of level-1 records per wave (cold path).
size_t bgl_gemv_x_lds(int K, int TR, int nw, bool fuse) {
    const int KQ = 64 / TR, S = (K / 64 + KQ - 1) / KQ;
    return ((size_t)S * KQ * XREC_DW + x_red_dw(TR, nw) + (fuse ? (size_t)nw * KQ * XREC_DW : 0)) * 4;
}

template <int FMT, int NB, bool FUSE>
static int launch_x_tr(int TR, const GemvLaunch &L, int nblocks, int nw, hipStream_t st) {
    dim3 g(nblocks), b(nw * BGL_TILE);
    const size_t lds = bgl_gemv_x_lds(L.t[0].T.K, TR, nw, FUSE);
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
