// bgl_moe_x.h -- device code of the expert-sorted MoE gather over LDS activation records
// (the kernels k_moe_x and k_moe_x2; their launchers are in bgl_moe_x.hip).  The kernel
// instances are compiled in separate translation units (bgl_moe_x_i*.hip, one instance each)
// so the build compiles them in parallel; each unit defines moe_x_go / moe_x2_go for its instances.
//
// The expert-sorted MoE gather GEMV over LDS activation records (the gate+up with
// SwiGLU and down projections of moe_ffn_batched, qwen_infer.c:5238-5350, and the routed gather
// of mlx_moe.cpp's gather_qmm), for experts in int4 g64, int4 g32 fp16-scale, int8 g64, qNg64 or
// MXFP4.
//
// A workgroup owns one 64-row tile of one expert (gate and up rows together in SwiGLU mode; lane =
// row) and walks the expert's sorted segment in chunks of up to 4 token columns, or up to 8 where
// the launch's LDS holds 8 columns of records (MoeTask.mbx): then the waves form two column groups
// of up to 4 columns each that take the same weight items in the same order, so the chunk's
// weights come from HBM once and the second group's loads hit the L2.  Per chunk it
// makes the columns' activation records (bgl_gemv_x.h) from the raw fp32 rows itself -- so a routed
// FFN needs no activation-prep launches -- while its waves' first weight loads are in flight; then
// the waves take the 64-groups in turn (each group once per tensor, two in flight): each lane
// decodes its row's group once and folds it against every column (the records are read as
// broadcasts).  Row sums go over the waves in order; SwiGLU
// (moe_swiglu_inplace, qwen_infer.c:3475-3481) is applied before the store.
#pragma once
#include "bgl_gemv_x.h"

#define MX_MB 4                  // token columns per chunk
#define MX_DEPTH 2               // items (a group of one tensor) a wave keeps in flight
#define MX_MAXW 16               // waves per workgroup (instances of 8 and 16)

// out[t][c] = (((0 + w_a d_a) + w_b d_b) + ...) over t's experts in ascending expert id (then k), then
// + the shared value: k_moe_combine's order (bgl_moe.hip), the order in which moe_ffn_batched's
// bucket loop adds into mlp_out_batch.
__device__ __forceinline__ void moe_x_combine(const MoeTask &Mt, int t, int c, float shared) {
    const int K = Mt.ck;
    const int32_t *it = Mt.cidx + (size_t)t * K;
    int order[MOE_MAX_K];
    for (int k = 0; k < K; k++) order[k] = k;
    for (int a = 1; a < K; a++)
        for (int b = a; b > 0 && it[order[b]] < it[order[b - 1]]; b--) {
            const int tmp = order[b]; order[b] = order[b - 1]; order[b - 1] = tmp;
        }
    float acc = 0.0f;
    for (int a = 0; a < K; a++) {
        const int p = t * K + order[a];
        const int s = Mt.cpos[p];
        if (s >= 0) acc += Mt.cw[p] * Mt.cdown[(size_t)s * Mt.ystride + c];
    }
    Mt.cout[(size_t)t * Mt.ystride + c] = acc + shared;
}

// mc columns from sorted position base; cgn column groups (1, or 2 with nw even and mc <= 2 MB):
// group g = waves [g nwg, (g+1) nwg) takes columns [g mc0, g mc0 + mcg) -- mc0 = ceil(mc / cgn) --
// over every item of the tile.
template <int FMT, int NB, int MB, int TR>
__device__ __forceinline__ void moe_x_chunk(const MoeTask &Mt, const BglDevTensor &Ta, const BglDevTensor &Tb, bool glu,
                                            int tile, int r0, int base, int mc, int cgn, int *xl) {
    constexpr int KQ = BGL_TILE / TR;              // groups per slot: lane = (row lane % TR, group lane / TR)
    const int nthr = blockDim.x, nw = nthr >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int K = Ta.K, G = K >> 6, S = (G + KQ - 1) / KQ, RC = S * KQ * XREC_DW, NPX = (K + 255) >> 8;
    const int r = lane % TR, kq = lane / TR;
    const int nwg = nw / cgn, cg = wave / nwg, wv = wave - cg * nwg;
    const int mc0 = (mc + cgn - 1) / cgn, cb = cg * mc0, mcg = cg ? mc - mc0 : mc0;

    // ---- a wave's items: its slots wv, wv + nwg, ... -- each once per tensor in SwiGLU mode
    // (gate then up) -- MX_DEPTH in flight; the first ones go out ahead of the activation work.
    // Lanes whose group of the last slot lies past K read nothing there; their records are zero.
    const XRes Ra = x_res<FMT>(Ta, tile), Rb = x_res<FMT>(Tb, tile);
    const XLane xlane = x_lane<FMT, NB, KQ>(r0 + r, kq);
    XLane xlast = xlane;
    if (kq >= G - (S - 1) * KQ) xlast = XLane{X_OOB, X_OOB, X_OOB, X_OOB, X_OOB};
    const int ns = (S - 1 - wv) / nwg + 1, NI = glu ? 2 * ns : ns;     // nwg <= nw <= S: every wave has a slot
    auto item_load = [&](XRaw<FMT, NB> &rw, int j) {
        const int sl = wv + (glu ? j >> 1 : j) * nwg;
        x_load<FMT, NB, KQ>(rw, glu && (j & 1) ? Rb : Ra, sl == S - 1 ? xlast : xlane, sl, j < NI);
    };
    XRaw<FMT, NB> c[MX_DEPTH];
#pragma unroll
    for (int j = 0; j < MX_DEPTH; j++) item_load(c[j], j);
    __builtin_amdgcn_sched_barrier(0);

    // ---- the chunk's records, made from the raw rows: pass pi = column pi / NPX, values
    // 256 * (pi % NPX) ..
    for (int pi = wave; pi < mc * NPX; pi += nw) {
        const int m = pi / NPX, p = pi - m * NPX;
        const int row = Mt.cols ? uni(Mt.cols)[base + m] : base + m;
        const float4 v = x_pass_load(Mt.a.xf + (size_t)row * K, p, lane, K);
        x_pass_digits(v, p, lane, G, xl + m * RC);
    }
    if (KQ > 1) {
        const int per = (S * KQ - G) * XREC_DW;
        for (int i = threadIdx.x; i < mc * per; i += nthr) {
            const int m = i / per;
            xl[m * RC + G * XREC_DW + (i - m * per)] = 0;
        }
    }
    __syncthreads();

    float acc[MB], accb[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) { acc[m] = 0.0f; accb[m] = 0.0f; }
    const int *xk = xl + kq * XREC_DW;
    for (int j0 = 0; j0 < NI; j0 += MX_DEPTH) {
#pragma unroll
        for (int jj = 0; jj < MX_DEPTH; jj++) {
            const int j = j0 + jj;
            if (j < NI) {
                const bool up = glu && (j & 1);
                const int *rec = xk + (wv + (glu ? j >> 1 : j) * nwg) * (KQ * XREC_DW) + cb * RC;
                const XDec<FMT, NB> d = x_decode<FMT, NB>(c[jj]);
                // columns one loop iteration at a time (not unrolled: the scheduler would hoist every
                // column's record reads, and their registers, to the front); the accumulator is
                // picked by wave-uniform branches
#pragma unroll 1
                for (int m = 0; m < mcg; m++) {
                    const float v = x_dot<FMT, NB>(d, rec + m * RC);
#pragma unroll
                    for (int q = 0; q < MB; q++) {
                        if (q == m && !up) acc[q] += v;
                        if (q == m && up) accb[q] += v;
                    }
                }
            }
            item_load(c[jj], j + MX_DEPTH);
        }
    }
    // items whose records carry a level-1 residual or non-finite values in some column: their
    // weights again, and the column's level-1 records made from its raw row (cold path)
    {
        int fl = 0;
        for (int i = 0; i < ns; i++)
            for (int m = 0; m < mcg; m++) fl |= xk[(wv + i * nwg) * (KQ * XREC_DW) + (cb + m) * RC + XREC_DSUM + 3];
        if (__builtin_amdgcn_ballot_w64(fl != 0)) {
            int *scr = xl + Mt.mbx * RC + nw * 2 * MX_MB * TR + wave * KQ * XREC_DW;   // this wave's level-1 records
            const int *r1 = scr + kq * XREC_DW;
            for (int j = 0; j < NI; j++) {
                const int sl = wv + (glu ? j >> 1 : j) * nwg, gl = min(sl * KQ + kq, G - 1);
                const bool up = glu && (j & 1);
                const int *rec = xk + sl * (KQ * XREC_DW) + cb * RC;
                int f2 = 0;
                for (int m = 0; m < mcg; m++) f2 |= rec[m * RC + XREC_DSUM + 3];
                if (!__builtin_amdgcn_ballot_w64(f2 != 0)) continue;
                // the item's weights once for all its flagged columns, loaded first so their latency
                // runs under the first column's level-1 records
                XRaw<FMT, NB> rf;
                x_load<FMT, NB, KQ>(rf, up ? Rb : Ra, sl == S - 1 ? xlast : xlane, sl, true);
                const XDec<FMT, NB> df = x_decode<FMT, NB>(rf);   // decoded once for all its flagged columns
#pragma unroll 1
                for (int m = 0; m < mcg; m++) {
                    const int f3 = rec[m * RC + XREC_DSUM + 3];
                    if (!__builtin_amdgcn_ballot_w64(f3 != 0)) continue;
                    const int xrow_m = Mt.cols ? uni(Mt.cols)[base + cb + m] : base + cb + m;
                    const float *xr = Mt.a.xf + (size_t)xrow_m * K;
                    if (__builtin_amdgcn_ballot_w64(f3 & BGL_XF_L1)) {
                        __builtin_amdgcn_wave_barrier();      // the previous column's reads of scr are done
                        const int g0 = sl * KQ, g1 = min(g0 + KQ, G);
                        for (int p = g0 >> 2; p <= (g1 - 1) >> 2; p++) x_pass_l1(x_pass_load(xr, p, lane, K), p, lane, g0, g1, scr);
                        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                        __builtin_amdgcn_wave_barrier();
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    }
                    const XRow xrow{up ? &Tb : &Ta, tile * BGL_TILE + r0 + r, xr};
                    const float v = x_fix<FMT, NB>(df, rec + m * RC, r1, *reinterpret_cast<const int4 *>(r1 + XREC_DSUM),
                                                   *reinterpret_cast<const int4 *>(r1 + XREC_DSUM + 4), xrow, gl);
#pragma unroll
                    for (int q = 0; q < MB; q++) {
                        if (q == m && !up) acc[q] += v;
                        if (q == m && up) accb[q] += v;
                    }
                }
            }
        }
    }

    // ---- row sums: over the KQ lanes of a row, then over the column group's waves in order
#pragma unroll
    for (int m = 0; m < MB; m++) {
#pragma unroll
        for (int o = TR; o < BGL_TILE; o <<= 1) {
            acc[m] += __shfl_xor(acc[m], o);
            accb[m] += __shfl_xor(accb[m], o);
        }
    }
    float *red = reinterpret_cast<float *>(xl + Mt.mbx * RC);     // [wave][2][MB][TR]
    if (lane < TR) {
#pragma unroll
        for (int m = 0; m < MB; m++) {
            red[((wave * 2 + 0) * MB + m) * TR + lane] = acc[m];
            red[((wave * 2 + 1) * MB + m) * TR + lane] = accb[m];
        }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < mc * TR; t += nthr) {
        const int m = t / TR, rl = t % TR, row = tile * BGL_TILE + r0 + rl;
        if (row < Ta.N) {
            const int g = m >= mc0, mm = m - g * mc0, w0 = g * nwg;
            float va = red[((w0 * 2 + 0) * MB + mm) * TR + rl], vb = red[((w0 * 2 + 1) * MB + mm) * TR + rl];
            for (int w = w0 + 1; w < w0 + nwg; w++) {
                va += red[((w * 2 + 0) * MB + mm) * TR + rl];
                vb += red[((w * 2 + 1) * MB + mm) * TR + rl];
            }
            const float out = glu ? (va / (1.0f + expf(-va))) * vb : va;
            const int yr = Mt.ymap ? Mt.ymap[base + m] : base + m;
            if (Mt.cout) moe_x_combine(Mt, yr, row, out);
            else Mt.y[(size_t)yr * Mt.ystride + row] = out;
        }
    }
    __syncthreads();                                               // the next chunk reuses the LDS
}

template <int FMT, int NB, int TR>
__device__ __forceinline__ void moe_x_tile(const MoeTask &Mt, const BglDevTensor &Ta, const BglDevTensor &Tb, bool glu,
                                           int tile, int r0, int seg0, int ncols, int *xl) {
    int c0 = 0;
    if (Mt.mbx > MX_MB && !((blockDim.x >> 6) & 1))            // chunks of 5..8 columns: two column groups
        for (; ncols - c0 > MX_MB; c0 += 2 * MX_MB) {
            const int rem = ncols - c0;
            moe_x_chunk<FMT, NB, MX_MB, TR>(Mt, Ta, Tb, glu, tile, r0, seg0 + c0, rem < 2 * MX_MB ? rem : 2 * MX_MB, 2, xl);
        }
    for (; ncols - c0 >= 2; c0 += MX_MB) {
        const int rem = ncols - c0;
        moe_x_chunk<FMT, NB, MX_MB, TR>(Mt, Ta, Tb, glu, tile, r0, seg0 + c0, rem < MX_MB ? rem : MX_MB, 1, xl);
    }
    if (c0 < ncols) moe_x_chunk<FMT, NB, 1, TR>(Mt, Ta, Tb, glu, tile, r0, seg0 + c0, 1, 1, xl);
}

// Expert record through the constant address space (scalar loads, wave-uniform addresses).
__device__ __forceinline__ BglDevTensor mx_tensor(const BglDevTensor *p) {
    static_assert(sizeof(BglDevTensor) % 4 == 0, "BglDevTensor is loaded as dwords");
    int w[sizeof(BglDevTensor) / 4];
    ucint q = uni(reinterpret_cast<const int *>(p));
#pragma unroll
    for (int i = 0; i < (int)(sizeof(BglDevTensor) / 4); i++) w[i] = q[i];
    BglDevTensor t;
    __builtin_memcpy(&t, w, sizeof t);
    return t;
}

// Grid: E x tpe workgroups.  SEG: the segments are consecutive runs of Mt.seg columns of
// one by-value tensor (the shared experts).
template <bool SEG, int TR>
__device__ __forceinline__ void moe_x_body(const MoeTask &Mt, int bid, int *xl) {
    constexpr int SUBS = BGL_TILE / TR;
    const int e = bid / (Mt.tpe * SUBS), rem = bid - e * Mt.tpe * SUBS;
    const int tile = rem / SUBS, r0 = (rem % SUBS) * TR;
    int seg0 = 0, ncols = Mt.ncols;
    if constexpr (SEG) { seg0 = e * Mt.seg; ncols = min(Mt.seg, Mt.ncols - seg0); }
    else if (Mt.off) { seg0 = uni(Mt.off)[e]; ncols = uni(Mt.off)[e + 1] - seg0; }
    if (ncols <= 0) return;                                   // expert not routed to by any pair
    const BglDevTensor Ta = Mt.ta ? mx_tensor(Mt.ta + e) : Mt.da;
    if (tile >= Ta.ntiles) return;
    const bool glu = Mt.swiglu != 0;
    const BglDevTensor Tb = glu ? (Mt.tb ? mx_tensor(Mt.tb + e) : Mt.db) : Ta;
    switch (Ta.fmt) {
    case BGL_Q4G32H: moe_x_tile<BGL_Q4G32H, 0, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
    case BGL_MXFP4: moe_x_tile<BGL_MXFP4, 0, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
    case BGL_Q4G64: moe_x_tile<BGL_Q4G64, 0, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
    case BGL_Q8G64: moe_x_tile<BGL_Q8G64, 0, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
    case BGL_QNG64:
        switch (Ta.bits) {
        case 2: moe_x_tile<BGL_QNG64, 2, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
        case 3: moe_x_tile<BGL_QNG64, 3, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
        case 4: moe_x_tile<BGL_QNG64, 4, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
        case 5: moe_x_tile<BGL_QNG64, 5, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
        case 6: moe_x_tile<BGL_QNG64, 6, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
        case 7: moe_x_tile<BGL_QNG64, 7, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
        case 8: moe_x_tile<BGL_QNG64, 8, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
        case 9: moe_x_tile<BGL_QNG64, 9, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
        case 10: moe_x_tile<BGL_QNG64, 10, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
        case 11: moe_x_tile<BGL_QNG64, 11, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
        case 12: moe_x_tile<BGL_QNG64, 12, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
        case 13: moe_x_tile<BGL_QNG64, 13, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
        case 14: moe_x_tile<BGL_QNG64, 14, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
        case 15: moe_x_tile<BGL_QNG64, 15, TR>(Mt, Ta, Tb, glu, tile, r0, seg0, ncols, xl); break;
        default: break;
        }
        break;
    default: break;
    }
}

// Whole-tile instances are held to 4 waves per SIMD (128 VGPRs: two 8-wave workgroups per CU, the
// occupancy the hot loop fits in); the 16-row instance runs only where fewer workgroups than CUs
// have work, so 3 waves per SIMD leave its widest formats room without spilling.
template <bool SEG, int NWMAX, int TR>
__global__ __launch_bounds__(NWMAX * BGL_TILE, TR == BGL_TILE ? 4 : 3) void k_moe_x(MoeTask Mt) {
    extern __shared__ __align__(16) int xl[];
    moe_x_body<SEG, TR>(Mt, blockIdx.x, xl);
}

// The routed experts' and the shared experts' gate+up of the same token rows in one launch: the
// shared tiles run beside the routed ones instead of after them.  SEG1: the second task's columns
// are cut into segments (the shared experts over more than 4 tokens).
template <int NWMAX, bool SEG1>
__global__ __launch_bounds__(NWMAX * BGL_TILE, 4) void k_moe_x2(MoePair P) {
    extern __shared__ __align__(16) int xl[];
    if ((int)blockIdx.x < P.nb0) moe_x_body<false, BGL_TILE>(P.t[0], blockIdx.x, xl);
    else moe_x_body<SEG1, BGL_TILE>(P.t[1], (int)blockIdx.x - P.nb0, xl);
}

// Launch one kernel instance (defined, and explicitly instantiated, in the unit that holds it).
template <bool SEG, int NWMAX, int TR>
void moe_x_go(dim3 g, dim3 b, size_t lds, hipStream_t st, const MoeTask &Mt);
template <int NWMAX, bool SEG1>
void moe_x2_go(dim3 g, dim3 b, size_t lds, hipStream_t st, const MoePair &P);
