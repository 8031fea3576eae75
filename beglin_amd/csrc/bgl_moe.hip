// bgl_moe.hip -- expert-stacked tensors and the expert-sorted MoE gather.
//
// One routed FFN call (moe_ffn_batched, qwen_infer.c:5238-5350, routing supplied by the caller):
//   k_moe_bucket   sort the T*K (token, k) pairs by expert, stable in pair order (the reference's
//                  bucket fill order) -> segment offsets, permutation, inverse permutation
//   k_act_x24      exact activation digits of the T token rows, shared by every expert
//   k_moe_gemv     gate+up of every touched expert with SwiGLU fused, h[s] = silu(g) * u; one
//                  workgroup per (expert, 64-row tile) so each expert's weights stream once for
//                  all of its tokens; experts may differ in format (runtime switch per workgroup)
//   k_moe_gemv     shared-expert gate+up over all T tokens (one by-value pseudo-expert)
//   k_act_x24      digits of the routed h rows -> k_moe_gemv down projection
//   k_act_x24      digits of the shared h rows -> k_moe_gemv shared down projection
//   k_moe_combine  out[t] = sum over t's experts in ascending expert order of w * down, + shared
// No host->device copies happen inside a call, so the sequence can be captured in a HIP graph.
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "bgl_gemv_impl.h"
#include "bgl_internal.h"

#define HIPCHK(expr)                                                                             \
    do {                                                                                         \
        hipError_t e_ = (expr);                                                                  \
        if (e_ != hipSuccess) return bgl_fail(BGL_E_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

#define MOE_MB 4            // token columns per weight pass of one tile
#define MOE_MAXW 8          // waves per workgroup: 512 threads leave 256 VGPRs for the widest formats

static inline unsigned nblk(long n, int bs = 256) { return (unsigned)((n + bs - 1) / bs); }

// ====================================================================================== bucketing
// start[0..E) holds per-expert counts; rewrites them as exclusive segment starts and sets
// start[E] to the total.  The first wave scans 256 experts per round (4 per lane, then a wave
// prefix over the lanes); the caller synchronizes before and after.
__device__ __forceinline__ void bucket_scan(int *start, int E) {
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    int carry = 0;
    for (int e0 = 0; e0 < E; e0 += 256) {
        int c[4], sum = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = e0 + 4 * lane + j;
            c[j] = e < E ? start[e] : 0;
            sum += c[j];
        }
        int incl = sum;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int n = __shfl_up(incl, o);
            if (lane >= o) incl += n;
        }
        int run = carry + incl - sum;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = e0 + 4 * lane + j;
            if (e < E) start[e] = run;
            run += c[j];
        }
        carry += __shfl(incl, 63);
    }
    if (lane == 0) start[E] = carry;
}

// One workgroup.  off[E+1]: segment starts in sorted order; perm[s]: pair at sorted position s;
// pos[p]: sorted position of pair p (-1 for an expert id outside [0, E), which is skipped);
// tok[s] = perm[s] / K, the token row that feeds sorted position s.
__global__ __launch_bounds__(1024) void k_moe_bucket(const int32_t *__restrict__ idx, int P, int K, int E,
                                                     int *__restrict__ off, int *__restrict__ perm,
                                                     int *__restrict__ pos, int *__restrict__ tok) {
    extern __shared__ int sm[];
    int *start = sm;               // [E + 1]
    int *ids = sm + E + 1;         // [P]
    for (int e = threadIdx.x; e <= E; e += blockDim.x) start[e] = 0;
    __syncthreads();
    for (int p = threadIdx.x; p < P; p += blockDim.x) {
        int e = idx[p];
        if (e < 0 || e >= E) e = -1;
        ids[p] = e;
        if (e >= 0) atomicAdd(&start[e], 1);
    }
    __syncthreads();
    bucket_scan(start, E);
    __syncthreads();
    for (int e = threadIdx.x; e <= E; e += blockDim.x) off[e] = start[e];
    for (int p = threadIdx.x; p < P; p += blockDim.x) {
        const int e = ids[p];
        if (e < 0) { pos[p] = -1; continue; }
        int rank = 0;
        for (int q = 0; q < p; q++) rank += ids[q] == e;
        const int s = start[e] + rank;
        perm[s] = p;
        pos[p] = s;
        tok[s] = p / K;
    }
}

// ====================================================================================== gather GEMV


template <int FMT, int NB, int MB>
__device__ __forceinline__ void moe_chunk(const MoeTask &Mt, const BglDevTensor &Ta, const BglDevTensor &Tb, bool glu,
                                          int tile, int base, int mc, float (*red)[2][MOE_MB][BGL_TILE]) {
    const int nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    Cols<MB> C;
#pragma unroll
    for (int m = 0; m < MB; m++) {
        const int mm = m < mc ? m : mc - 1;              // padded columns repeat the last one
        C.am[m] = Mt.cols ? uni(Mt.cols)[base + mm] : base + mm;
    }
    float acc[MB], accb[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) { acc[m] = 0.0f; accb[m] = 0.0f; }
    const int K = Ta.K, U = Ta.nunits;
    for (int u = wave; u < U; u += nw) {
        Raw<FMT, NB> r;
        load_raw<FMT, NB>(r, Ta, tile, lane, u);
        comp_dispatch<FMT, BGL_ACT_F32, NB, MB>(r, K, u, Mt.a, C, acc);
        if (glu) {
            load_raw<FMT, NB>(r, Tb, tile, lane, u);
            comp_dispatch<FMT, BGL_ACT_F32, NB, MB>(r, K, u, Mt.a, C, accb);
        }
    }
    // groups whose activations carry a level-1 residual or non-finite values (cold path)
    if constexpr (FMT != BGL_F16 && FMT != BGL_F32) {
        const WRow Wa{&Ta, tile * BGL_TILE + lane}, Wb{&Tb, tile * BGL_TILE + lane};
        for (int u = wave; u < U; u += nw) {
            int fl = 0;
#pragma unroll
            for (int m = 0; m < MB; m++) fl |= unit_flags<FMT, NB>(Mt.a, C.am[m], K, u);
            if (fl) {
                Raw<FMT, NB> r;
                load_raw<FMT, NB>(r, Ta, tile, lane, u);
                comp_fix<FMT, NB, MB>(r, Wa, u, Mt.a, C, acc);
                if (glu) {
                    load_raw<FMT, NB>(r, Tb, tile, lane, u);
                    comp_fix<FMT, NB, MB>(r, Wb, u, Mt.a, C, accb);
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MB; m++) { red[wave][0][m][lane] = acc[m]; red[wave][1][m][lane] = accb[m]; }
    __syncthreads();
    const int row = tile * BGL_TILE + lane;
    if (wave == 0 && row < Ta.N) {
#pragma unroll
        for (int m = 0; m < MB; m++) {
            if (m < mc) {
                float va = red[0][0][m][lane], vb = red[0][1][m][lane];
                for (int w = 1; w < nw; w++) { va += red[w][0][m][lane]; vb += red[w][1][m][lane]; }
                float out = va;
                if (glu) out = (va / (1.0f + expf(-va))) * vb;   // moe_swiglu_inplace, qwen_infer.c:3475-3481
                const int yr = Mt.ymap ? Mt.ymap[base + m] : base + m;
                Mt.y[(size_t)yr * Mt.ystride + row] = out;
            }
        }
    }
    __syncthreads();
}

template <int FMT, int NB>
__device__ __forceinline__ void moe_tile(const MoeTask &Mt, const BglDevTensor &Ta, const BglDevTensor &Tb, bool glu,
                                         int tile, int seg0, int ncols, float (*red)[2][MOE_MB][BGL_TILE]) {
    int c0 = 0;
    for (; ncols - c0 >= 2; c0 += MOE_MB) {
        const int rem = ncols - c0;
        moe_chunk<FMT, NB, MOE_MB>(Mt, Ta, Tb, glu, tile, seg0 + c0, rem < MOE_MB ? rem : MOE_MB, red);
    }
    if (c0 < ncols) moe_chunk<FMT, NB, 1>(Mt, Ta, Tb, glu, tile, seg0 + c0, 1, red);
}

// Expert record through the constant address space: scalar loads, so every address derived from
// it stays wave-uniform (a plain global load would be treated as divergent).
__device__ __forceinline__ BglDevTensor ld_tensor(const BglDevTensor *p) {
    static_assert(sizeof(BglDevTensor) % 4 == 0, "BglDevTensor is loaded as dwords");
    int w[sizeof(BglDevTensor) / 4];
    ucint q = uni(reinterpret_cast<const int *>(p));
#pragma unroll
    for (int i = 0; i < (int)(sizeof(BglDevTensor) / 4); i++) w[i] = q[i];
    BglDevTensor t;
    __builtin_memcpy(&t, w, sizeof t);
    return t;
}

// WIDE: also the dense fp16 / fp32 cases, whose 64-register units would raise every format's
// register count (and lower occupancy) if they shared one instantiation.
// SEG: the segments are consecutive runs of Mt.seg columns (the shared experts).  A separate
// instantiation, so the routed kernel's register allocation (and occupancy) stays its own.
template <bool WIDE, bool SEG>
__global__ __launch_bounds__(MOE_MAXW * BGL_TILE, WIDE || SEG ? 2 : 4) void k_moe_gemv(MoeTask Mt) {
    __shared__ float red[MOE_MAXW][2][MOE_MB][BGL_TILE];
    const int e = blockIdx.x / Mt.tpe, tile = blockIdx.x % Mt.tpe;
    int seg0 = 0, ncols = Mt.ncols;
    if constexpr (SEG) { seg0 = e * Mt.seg; ncols = min(Mt.seg, Mt.ncols - seg0); }
    else if (Mt.off) { seg0 = uni(Mt.off)[e]; ncols = uni(Mt.off)[e + 1] - seg0; }
    if (ncols <= 0) return;                                   // expert not routed to by any pair
    const BglDevTensor Ta = Mt.ta ? ld_tensor(Mt.ta + e) : Mt.da;
    if (tile >= Ta.ntiles) return;
    const bool glu = Mt.swiglu != 0;
    const BglDevTensor Tb = glu ? (Mt.tb ? ld_tensor(Mt.tb + e) : Mt.db) : Ta;
    switch (Ta.fmt) {
    case BGL_Q4G32H: moe_tile<BGL_Q4G32H, 0>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
    case BGL_Q4G64: moe_tile<BGL_Q4G64, 0>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
    case BGL_Q8G64: moe_tile<BGL_Q8G64, 0>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
    case BGL_Q4G64A: moe_tile<BGL_Q4G64A, 0>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
    case BGL_F16: if constexpr (WIDE) moe_tile<BGL_F16, 0>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
    case BGL_F32: if constexpr (WIDE) moe_tile<BGL_F32, 0>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
    case BGL_QNG64:
        switch (Ta.bits) {
        case 2: moe_tile<BGL_QNG64, 2>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
        case 3: moe_tile<BGL_QNG64, 3>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
        case 4: moe_tile<BGL_QNG64, 4>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
        case 5: moe_tile<BGL_QNG64, 5>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
        case 6: moe_tile<BGL_QNG64, 6>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
        case 7: moe_tile<BGL_QNG64, 7>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
        case 8: moe_tile<BGL_QNG64, 8>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
        case 9: moe_tile<BGL_QNG64, 9>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
        case 10: moe_tile<BGL_QNG64, 10>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
        case 11: moe_tile<BGL_QNG64, 11>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
        case 12: moe_tile<BGL_QNG64, 12>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
        case 13: moe_tile<BGL_QNG64, 13>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
        case 14: moe_tile<BGL_QNG64, 14>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
        case 15: moe_tile<BGL_QNG64, 15>(Mt, Ta, Tb, glu, tile, seg0, ncols, red); break;
        default: break;
        }
        break;
    default: break;
    }
}

// ====================================================================================== combine
// out[t][c] = (((0 + w_a d_a) + w_b d_b) + ...) over t's experts in ascending expert id, then
// + shared[t][c]: the order in which moe_ffn_batched's bucket loop adds into mlp_out_batch.
__global__ __launch_bounds__(256) void k_moe_combine(const float *__restrict__ D, const int *__restrict__ pos,
                                                     const int32_t *__restrict__ idx, const float *__restrict__ w,
                                                     int T, int K, int H, const float *__restrict__ shared,
                                                     float *__restrict__ out) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)T * H) return;
    const int t = (int)(i / H), c = (int)(i % H);
    const int32_t *it = idx + (size_t)t * K;
    int order[MOE_MAX_K];
    for (int k = 0; k < K; k++) order[k] = k;
    for (int a = 1; a < K; a++)                               // insertion sort: expert id, then k
        for (int b = a; b > 0 && it[order[b]] < it[order[b - 1]]; b--) {
            const int tmp = order[b]; order[b] = order[b - 1]; order[b - 1] = tmp;
        }
    float acc = 0.0f;
    for (int a = 0; a < K; a++) {
        const int p = t * K + order[a];
        const int s = pos[p];
        if (s >= 0) acc += w[p] * D[(size_t)s * H + c];
    }
    if (shared) acc += shared[i];
    out[i] = acc;
}

// ====================================================================================== host side
extern "C" int bgl_experts_from_tensors(bgl_ctx *c, int E, bgl_tensor *const *experts, bgl_tensor **out) {
    if (!c || E < 1 || !experts || !out) return bgl_fail(BGL_E_ARG, "bgl_experts_from_tensors: bad argument");
    std::vector<BglDevTensor> tab(E);
    for (int e = 0; e < E; e++) {
        if (!experts[e] || !experts[e]->experts.empty())
            return bgl_fail(BGL_E_ARG, "bgl_experts_from_tensors: expert %d is not a single bound tensor", e);
        if (experts[e]->T.N != experts[0]->T.N || experts[e]->T.K != experts[0]->T.K)
            return bgl_fail(BGL_E_ARG, "bgl_experts_from_tensors: expert %d shape differs from expert 0", e);
        if (experts[e]->T.fmt == BGL_Q4G256SF)
            return bgl_fail(BGL_E_UNSUPPORTED, "bgl_experts_from_tensors: g256sf experts take W4A8 activations only");
        tab[e] = experts[e]->T;
    }
    HIPCHK(hipSetDevice(c->device));
    void *d = nullptr;
    HIPCHK(hipMalloc(&d, sizeof(BglDevTensor) * E));
    hipError_t err = hipMemcpy(d, tab.data(), sizeof(BglDevTensor) * E, hipMemcpyHostToDevice);
    if (err != hipSuccess) {
        (void)hipFree(d);
        return bgl_fail(BGL_E_HIP, "bgl_experts_from_tensors: table copy: %s", hipGetErrorString(err));
    }
    bgl_tensor *t = new bgl_tensor();
    t->T = tab[0];
    t->dev_table = d;
    t->owned.push_back(d);
    t->experts.assign(experts, experts + E);
    *out = t;
    return 0;
}

extern "C" int bgl_bind_experts(bgl_ctx *c, int E, const bgl_wt *experts, bgl_tensor **out) {
    if (!c || E < 1 || !experts || !out) return bgl_fail(BGL_E_ARG, "bgl_bind_experts: bad argument");
    std::vector<bgl_tensor *> ts(E, nullptr);
    int rc = 0;
    for (int e = 0; e < E && !rc; e++) {
        if (experts[e].out != experts[0].out || experts[e].in != experts[0].in)
            rc = bgl_fail(BGL_E_ARG, "bgl_bind_experts: expert %d shape differs from expert 0", e);
        else
            rc = bgl_bind(c, &experts[e], &ts[e]);
    }
    if (!rc) rc = bgl_experts_from_tensors(c, E, ts.data(), out);
    if (rc)
        for (bgl_tensor *t : ts) bgl_tensor_free(t);
    return rc;
}

struct MoeScratch {
    int *off, *perm, *pos, *tok;
};

// The bucketing outputs in the context's scratch: off [E+1], perm [P], pos [P], tok [P].
static int moe_scratch(bgl_ctx *c, int P, int E, MoeScratch &S) {
    const size_t lds = ((size_t)E + 1 + P) * 4;
    if (lds > 64 * 1024)
        return bgl_fail(BGL_E_ARG, "MoE bucketing: %d pairs over %d experts exceed one workgroup's LDS", P, E);
    if (dbuf_reserve(c, c->moe_meta, ((size_t)E + 1 + 3 * (size_t)P) * 4, false)) return bgl_last_code();
    int *b = (int *)c->moe_meta.p;
    S.off = b; S.perm = b + E + 1; S.pos = S.perm + P; S.tok = S.pos + P;
    return 0;
}

static int moe_bucket(bgl_ctx *c, const int32_t *idx_dev, int P, int K, int E, MoeScratch &S) {
    int rc = moe_scratch(c, P, E, S);
    if (rc) return rc;
    const size_t lds = ((size_t)E + 1 + P) * 4;
    int tok = prof_begin(c, 2);
    hipLaunchKernelGGL(k_moe_bucket, dim3(1), dim3(1024), lds, c->stream, idx_dev, P, K, E, S.off, S.perm, S.pos, S.tok);
    prof_end(c, tok);
    HIPCHK(hipGetLastError());
    return 0;
}

// Exact activation digits of M rows of length K into digit slot 0 or 1.
static int moe_prep(bgl_ctx *c, int slot, const float *x_dev, int M, int K, GemvAct &A) {
    DevBuf &w = slot ? c->moe_d : c->moe_a;
    DevBuf &s = slot ? c->moe_e : c->moe_b;
    DevBuf &d = slot ? c->moe_f : c->moe_c;
    const int ng = K / 64;
    if (dbuf_reserve(c, w, (size_t)2 * M * ng * 192, false) || dbuf_reserve(c, s, (size_t)2 * M * ng * 4, false) ||
        dbuf_reserve(c, d, (size_t)2 * M * (K / 32) * 16, false))
        return bgl_last_code();
    int tok = prof_begin(c, 0);
    hipLaunchKernelGGL(k_act_x24, dim3(nblk((long)M * ng * 64)), dim3(256), 0, c->stream, x_dev, M, K, (int8_t *)w.p,
                       (float *)s.p, (int *)d.p);
    prof_end(c, tok);
    HIPCHK(hipGetLastError());
    memset(&A, 0, sizeof A);
    f32_act_ptrs(w.p, s.p, d.p, M, K, x_dev, A);
    return 0;
}

static bool dense_fmt(int fmt) { return fmt == BGL_F16 || fmt == BGL_F32; }

// Whether a launch meets dense experts: the stack's experts, or the by-value tensors.
static bool task_wide(const bgl_tensor *stack, const MoeTask &Mt) {
    if (stack)
        for (const bgl_tensor *e : stack->experts)
            if (dense_fmt(e->T.fmt)) return true;
    return !Mt.ta && (dense_fmt(Mt.da.fmt) || (Mt.swiglu && dense_fmt(Mt.db.fmt)));
}

// The shared experts' T columns are cut into segments, one pseudo-expert each (every one reads
// the same tensor), so the chunks run on separate workgroups instead of one after another on each
// tile's workgroup.  Every segment reads the whole tensor, so segments are as long as one weight
// pass serves: MOE_MB columns in k_moe_gemv; in k_moe_x 8 (two column groups) beyond 8 tokens and
// 4 between 5 and 8 tokens, which keeps twice the workgroups where the tensors are small.
// Routed experts keep one workgroup per tile, which walks its segment in chunks.
static int shared_seg(int T, bool xpath) {
    if (!xpath) return T > MOE_MB ? MOE_MB : 0;
    return T > 8 ? 8 : T > 4 ? 4 : 0;
}

// Token columns of records one k_moe_x chunk holds: 8 where the launch's LDS allows (BGL_MOE_CAP
// forces 4 or 8).
static int moe_cap(const bgl_ctx *c, int K, int nw, int TR) { return c->moe_cap ? c->moe_cap : bgl_moe_x_cap(K, nw, TR); }

static int moe_launch(bgl_ctx *c, const MoeTask &Mt, int units, bool wide) {
    int nw = units < c->max_waves ? units : c->max_waves;
    if (nw > MOE_MAXW) nw = MOE_MAXW;
    if (nw < 1) nw = 1;
    int tok = prof_begin(c, 1);
    const bool seg = !Mt.off && Mt.seg > 0;
    const dim3 g(Mt.E * Mt.tpe), b(nw * BGL_TILE);
    if (wide) {
        if (seg) hipLaunchKernelGGL((k_moe_gemv<true, true>), g, b, 0, c->stream, Mt);
        else hipLaunchKernelGGL((k_moe_gemv<true, false>), g, b, 0, c->stream, Mt);
    } else {
        if (seg) hipLaunchKernelGGL((k_moe_gemv<false, true>), g, b, 0, c->stream, Mt);
        else hipLaunchKernelGGL((k_moe_gemv<false, false>), g, b, 0, c->stream, Mt);
    }
    prof_end(c, tok);
    HIPCHK(hipGetLastError());
    return 0;
}

// Whether a gather launch can run k_moe_x (bgl_moe_x.hip): every tensor it meets in a format that
// kernel takes, addressable through 32-bit buffer offsets, and the chunk's records fit LDS.
static bool x_tensor_ok(const BglDevTensor &T) {
    return bgl_moe_x_fmt(T.fmt) && (size_t)T.ntiles * T.cpr * 1024 < (1ull << 31) && (size_t)T.ntiles * T.nunits * 512 < (1ull << 31);
}
static bool moe_x_ok(bgl_ctx *c, const bgl_tensor *sa, const bgl_tensor *sb, const MoeTask &Mt, int K) {
    if (c->no_moe_x || bgl_moe_x_lds(K, 16, 64, 4) > 160 * 1024 || bgl_moe_x_lds(K, 8, 16, 4) > 160 * 1024) return false;
    for (const bgl_tensor *st : {sa, sb})
        if (st)
            for (const bgl_tensor *e : st->experts)
                if (!x_tensor_ok(e->T)) return false;
    if (!Mt.ta && (!x_tensor_ok(Mt.da) || (Mt.swiglu && !x_tensor_ok(Mt.db)))) return false;
    return true;
}

// Activation digits already made in this call (reused by the launches that read the same rows).
struct PrepMemo {
    const float *x = nullptr;
    int K = 0;
    GemvAct A{};
};

// One gather launch over the activation rows x_rows ([nrows][K]): through k_moe_x, which makes the
// records from the raw rows itself, when every tensor takes it; else k_act_x24 into digit slot
// `slot` (once per rows) and k_moe_gemv.
static int moe_run(bgl_ctx *c, MoeTask &Mt, const bgl_tensor *sa, const bgl_tensor *sb, int units, int slot,
                   PrepMemo &memo, const float *x_rows, int nrows, int K, long active_wgs) {
    if (Mt.cout && !moe_x_ok(c, sa, sb, Mt, K)) return bgl_fail(BGL_E_ARG, "internal: a fused combine needs k_moe_x");
    if (moe_x_ok(c, sa, sb, Mt, K)) {
        memset(&Mt.a, 0, sizeof Mt.a);
        Mt.a.xf = x_rows;
        int tok = prof_begin(c, 1);
        int TR, nw;
        bgl_moe_x_shape(K, active_wgs, c->force_tr, c->x_waves, &TR, &nw);
        int rc = bgl_launch_moe_x(Mt, K, TR, nw, moe_cap(c, K, nw, TR), c->stream);
        prof_end(c, tok);
        if (rc) return bgl_fail(BGL_E_ARG, "k_moe_x launch: in=%d", K);
        HIPCHK(hipGetLastError());
        return 0;
    }
    // k_moe_gemv has no MXFP4 arm: such a launch (an MXFP4 expert beside an AF int4 or dense one, or
    // BGL_NO_MOE_X) is refused rather than run with that expert's tiles skipped
    bool mx = !Mt.ta && (Mt.da.fmt == BGL_MXFP4 || (Mt.swiglu && Mt.db.fmt == BGL_MXFP4));
    for (const bgl_tensor *st : {sa, sb})
        if (st)
            for (const bgl_tensor *e : st->experts) mx = mx || e->T.fmt == BGL_MXFP4;
    if (mx)
        return bgl_fail(BGL_E_UNSUPPORTED, "MXFP4 experts run in the in-kernel-digit gather only; this launch also holds "
                        "AF int4 / dense experts (or BGL_NO_MOE_X is set)");
    if (memo.x != x_rows || memo.K != K) {
        int rc = moe_prep(c, slot, x_rows, nrows, K, memo.A);
        if (rc) return rc;
        memo.x = x_rows; memo.K = K;
    }
    Mt.a = memo.A;
    return moe_launch(c, Mt, units, task_wide(sa, Mt) || task_wide(sb, Mt));
}

static int expert_check(const bgl_tensor *t, const char *what) {
    if (!t || t->experts.empty() || !t->dev_table)
        return bgl_fail(BGL_E_ARG, "%s must be an expert tensor (bgl_bind_experts / bgl_experts_from_tensors)", what);
    if (t->T.K % 64) return bgl_fail(BGL_E_ARG, "%s: in=%d is not a multiple of 64", what, t->T.K);
    return 0;
}

static void max_units(const bgl_tensor *t, int &tiles, int &units) {
    tiles = 0; units = 0;
    for (const bgl_tensor *e : t->experts) {
        if (e->T.ntiles > tiles) tiles = e->T.ntiles;
        if (e->T.nunits > units) units = e->T.nunits;
    }
}

extern "C" int bgl_gather_matvec_dev(bgl_ctx *c, const bgl_tensor *experts, const float *x_dev,
                                     const int32_t *idx_dev, int N, float *y_dev) {
    if (!c || !x_dev || !idx_dev || !y_dev || N < 1) return bgl_fail(BGL_E_ARG, "bgl_gather_matvec_dev: bad argument");
    int rc = expert_check(experts, "bgl_gather_matvec_dev: experts");
    if (rc) return rc;
    HIPCHK(hipSetDevice(c->device));
    const int E = (int)experts->experts.size();
    MoeScratch S;
    if ((rc = moe_bucket(c, idx_dev, N, 1, E, S))) return rc;
    MoeTask Mt;
    memset(&Mt, 0, sizeof Mt);
    int units;
    max_units(experts, Mt.tpe, units);
    Mt.ta = (const BglDevTensor *)experts->dev_table; Mt.E = E; Mt.off = S.off;
    Mt.cols = S.perm; Mt.ymap = S.perm; Mt.y = y_dev; Mt.ystride = experts->T.N;
    PrepMemo memo;
    return moe_run(c, Mt, experts, nullptr, units, 0, memo, x_dev, N, experts->T.K, (long)std::min(E, N) * Mt.tpe);
}

// The routed FFN; pre: the pairs' bucketing when the caller already made it (the whole-layer entry).
static int moe_ffn(bgl_ctx *c, const bgl_tensor *gate, const bgl_tensor *up, const bgl_tensor *down, const bgl_tensor *sg,
                   const bgl_tensor *su, const bgl_tensor *sd, const float *x_dev, const int32_t *idx_dev, const float *w_dev,
                   int T, int K, float *out_dev, const MoeScratch *pre) {
    if (!c || !x_dev || !idx_dev || !w_dev || !out_dev || T < 1 || K < 1 || K > MOE_MAX_K)
        return bgl_fail(BGL_E_ARG, "bgl_moe_ffn_dev: bad argument (T=%d, K=%d; 1 <= K <= %d)", T, K, MOE_MAX_K);
    int rc;
    if ((rc = expert_check(gate, "bgl_moe_ffn_dev: gate")) || (rc = expert_check(up, "bgl_moe_ffn_dev: up")) ||
        (rc = expert_check(down, "bgl_moe_ffn_dev: down")))
        return rc;
    const int E = (int)gate->experts.size();
    if ((int)up->experts.size() != E || (int)down->experts.size() != E)
        return bgl_fail(BGL_E_ARG, "bgl_moe_ffn_dev: gate/up/down expert counts differ");
    const int H = gate->T.K, I = gate->T.N;
    if (up->T.K != H || up->T.N != I || down->T.K != I || down->T.N != H)
        return bgl_fail(BGL_E_ARG, "bgl_moe_ffn_dev: gate/up [%d x %d] and down [%d x %d] disagree", I, H, down->T.N, down->T.K);
    for (int e = 0; e < E; e++)
        if (gate->experts[e]->T.fmt != up->experts[e]->T.fmt || gate->experts[e]->T.bits != up->experts[e]->T.bits)
            return bgl_fail(BGL_E_ARG, "bgl_moe_ffn_dev: expert %d gate and up differ in format", e);
    const int nsh = (sg != nullptr) + (su != nullptr) + (sd != nullptr);
    if (nsh != 0 && nsh != 3) return bgl_fail(BGL_E_ARG, "bgl_moe_ffn_dev: give all three shared tensors or none");
    int Ish = 0;
    if (nsh) {
        if (!sg->experts.empty() || !su->experts.empty() || !sd->experts.empty())
            return bgl_fail(BGL_E_ARG, "bgl_moe_ffn_dev: shared experts are single tensors");
        Ish = sg->T.N;
        if (sg->T.K != H || su->T.K != H || su->T.N != Ish || sd->T.K != Ish || sd->T.N != H)
            return bgl_fail(BGL_E_ARG, "bgl_moe_ffn_dev: shared shapes disagree with hidden=%d", H);
        if (sg->T.fmt != su->T.fmt || sg->T.bits != su->T.bits)
            return bgl_fail(BGL_E_ARG, "bgl_moe_ffn_dev: shared gate and up differ in format");
        if (sg->T.fmt == BGL_Q4G256SF || sd->T.fmt == BGL_Q4G256SF || Ish % 64)
            return bgl_fail(BGL_E_UNSUPPORTED, "bgl_moe_ffn_dev: shared experts need fp32-activation formats, in %% 64 == 0");
    }
    HIPCHK(hipSetDevice(c->device));
    const int P = T * K;
    MoeScratch S;
    if (pre) S = *pre;
    else if ((rc = moe_bucket(c, idx_dev, P, K, E, S))) return rc;
    // fp32 work rows: h [P][I], shared h [T][Ish], routed down [P][H], shared down [T][H]
    const size_t nh = (size_t)P * I, nsh_h = (size_t)T * Ish, nd = (size_t)P * H, nsd = (size_t)T * H;
    if (dbuf_reserve(c, c->moe_g, (nh + nsh_h + nd + nsd) * 4, false)) return bgl_last_code();
    float *h = (float *)c->moe_g.p, *shh = h + nh, *dd = shh + nsh_h, *sdd = dd + nd;

    MoeTask Mr, Ms;
    PrepMemo mx, mh, ms;                      // digits of x (slot 0), of h (slot 1), of the shared h (slot 0)
    memset(&Mr, 0, sizeof Mr);
    int units;
    max_units(gate, Mr.tpe, units);
    Mr.ta = (const BglDevTensor *)gate->dev_table; Mr.tb = (const BglDevTensor *)up->dev_table;
    Mr.E = E; Mr.off = S.off; Mr.cols = S.tok; Mr.y = h; Mr.ystride = I; Mr.swiglu = 1;
    // workgroups with work: at most one expert per pair, every tile of it
    const long act_r = (long)std::min(E, P);
    if (nsh) {
        memset(&Ms, 0, sizeof Ms);
        Ms.da = sg->T; Ms.db = su->T; Ms.tpe = sg->T.ntiles; Ms.ncols = T;
        Ms.y = shh; Ms.ystride = Ish; Ms.swiglu = 1;
        Ms.seg = shared_seg(T, moe_x_ok(c, nullptr, nullptr, Ms, H)); Ms.E = Ms.seg ? (T + Ms.seg - 1) / Ms.seg : 1;
    }
    // Shared experts over >= BGL_MFMA_MIN_M tokens, in formats the matrix cores decode exactly, run
    // as a dense MLP block on the matrix cores (bgl_mlp_dev: gate+up, SwiGLU, down) instead of in
    // the gathers, whose exact-digit work grows with the token count; the combine adds their rows.
    const bool shm = nsh && T >= BGL_MFMA_MIN_M && !c->no_mfma && bgl_mfma_ok(sg->T.fmt, sg->T.bits) &&
                     bgl_mfma_ok(sd->T.fmt, sd->T.bits);
    // The shared gate+up joins the routed launch when that launch runs whole-tile workgroups
    // (BGL_MOE_MERGE=1 forces whole tiles, 0 keeps two launches).
    bool merged = false;
    if (nsh && !shm && c->moe_merge != 0 && moe_x_ok(c, gate, up, Mr, H) && moe_x_ok(c, nullptr, nullptr, Ms, H)) {
        int TR, nw;
        bgl_moe_x_shape(H, act_r * Mr.tpe + (long)Ms.E * Ms.tpe, c->moe_merge == 1 ? BGL_TILE : c->force_tr, c->x_waves, &TR,
                        &nw);
        if (TR == BGL_TILE) {
            memset(&Mr.a, 0, sizeof Mr.a);
            memset(&Ms.a, 0, sizeof Ms.a);
            Mr.a.xf = x_dev;
            Ms.a.xf = x_dev;
            int tok = prof_begin(c, 1);
            rc = bgl_launch_moe_x2(Mr, Ms, H, nw, moe_cap(c, H, nw, BGL_TILE), c->stream);
            prof_end(c, tok);
            if (rc) return bgl_fail(BGL_E_ARG, "k_moe_x2 launch: in=%d", H);
            HIPCHK(hipGetLastError());
            merged = true;
        }
    }
    if (!merged) {
        if ((rc = moe_run(c, Mr, gate, up, units, 0, mx, x_dev, T, H, act_r * Mr.tpe))) return rc;
        if (nsh && !shm && (rc = moe_run(c, Ms, nullptr, nullptr, sg->T.nunits, 0, mx, x_dev, T, H, (long)Ms.E * Ms.tpe)))
            return rc;
    }
    memset(&Mr, 0, sizeof Mr);
    max_units(down, Mr.tpe, units);
    Mr.ta = (const BglDevTensor *)down->dev_table; Mr.E = E; Mr.off = S.off; Mr.y = dd; Mr.ystride = H;
    if ((rc = moe_run(c, Mr, down, nullptr, units, 1, mh, h, P, I, act_r * Mr.tpe))) return rc;
    bool combined = false;
    if (shm) {
        if ((rc = bgl_mlp_dev(c, sg, su, sd, BGL_ACT_F32, x_dev, sdd, T, shh))) return rc;
    } else if (nsh) {
        memset(&Ms, 0, sizeof Ms);
        Ms.da = sd->T; Ms.tpe = sd->T.ntiles; Ms.ncols = T; Ms.y = sdd; Ms.ystride = H;
        const bool sdx = moe_x_ok(c, nullptr, nullptr, Ms, Ish);
        Ms.seg = shared_seg(T, sdx); Ms.E = Ms.seg ? (T + Ms.seg - 1) / Ms.seg : 1;
        if (sdx) {      // the combine rides on the shared down's store
            Ms.cout = out_dev; Ms.cdown = dd; Ms.cw = w_dev; Ms.cpos = S.pos; Ms.cidx = idx_dev; Ms.ck = K;
            combined = true;
        }
        if ((rc = moe_run(c, Ms, nullptr, nullptr, sd->T.nunits, 0, ms, shh, T, Ish, (long)Ms.E * Ms.tpe))) return rc;
    }
    if (combined) return 0;
    int tok = prof_begin(c, 2);
    hipLaunchKernelGGL(k_moe_combine, dim3(nblk((long)T * H)), dim3(256), 0, c->stream, dd, S.pos, idx_dev, w_dev, T, K, H,
                       nsh ? sdd : nullptr, out_dev);
    prof_end(c, tok);
    HIPCHK(hipGetLastError());
    return 0;
}

extern "C" int bgl_moe_ffn_dev(bgl_ctx *c, const bgl_tensor *gate, const bgl_tensor *up, const bgl_tensor *down,
                               const bgl_tensor *sg, const bgl_tensor *su, const bgl_tensor *sd, const float *x_dev,
                               const int32_t *idx_dev, const float *w_dev, int T, int K, float *out_dev) {
    return moe_ffn(c, gate, up, down, sg, su, sd, x_dev, idx_dev, w_dev, T, K, out_dev, nullptr);
}

// ================================================================================== router
// The routing of moe_ffn_batched (qwen_infer.c:5243-5257, :5275), in two kernels: the scores
// (one wave per token and expert, so the router matrix streams through many CUs), then the
// softmax / top-K / renorm of each token (one wave per token):
//   scores[e] = (float)(sum_c (double)W[e][c] * x[c]) (+ b[e])       moe_matvec_f32, :3460-3466
//   softmax: max, expf(s - max) in float, double sum, (float)(e / sum)  moe_softmax_full, :3467-3472
//   top-K: repeated strict maximum, ties to the lowest expert id       moe_top_k_select, :3514-3521
//   optional renorm: the K weights over their double sum               moe_topk_renorm, :3529-3534
// The router dot products run in double on every lane (fma with exact float products) and are
// combined across the wave; the softmax sum runs sequentially in expert order as the reference's.
// exp is evaluated in double and rounded once to float.
#define ROUTE_MAXE 256
#define ROUTE_EPW 4          // experts per scores workgroup: one per wave

// scores[t][e] = (float)(sum_c (double)W[e][c] * x[t][c]) (+ b[e]); grid (T, ceil(E/4)), one wave
// per expert so the router matrix is read by many CUs at once.  Each lane sums its elements
// 4*lane + 256*i in ascending order; a round's 8 row and 8 x loads all go out before the first fma
// (buffer loads: the ones past H return zero, so none is conditional and one round trip serves
// H <= 2048).
#define ROUTE_RND 8
__global__ __launch_bounds__(ROUTE_EPW * 64) void k_moe_router_scores(const float *__restrict__ W, const float *__restrict__ bias,
                                                                      int E, int H, const float *__restrict__ x,
                                                                      float *__restrict__ scores) {
    const int t = blockIdx.x, e = blockIdx.y * ROUTE_EPW + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (e >= E) return;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(W + (size_t)e * H), (short)0, H * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(x + (size_t)t * H), (short)0, H * 4, 0x00020000);
    typedef float rf4 __attribute__((ext_vector_type(4)));
    double acc = 0.0;
    for (int c0 = 0; c0 < H; c0 += ROUTE_RND * 256) {
        rf4 wv[ROUTE_RND], xv[ROUTE_RND];
#pragma unroll
        for (int i = 0; i < ROUTE_RND; i++) {
            const int off = (c0 + 256 * i + 4 * lane) * 4;
            wv[i] = __builtin_bit_cast(rf4, __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0));
            xv[i] = __builtin_bit_cast(rf4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < ROUTE_RND; i++) {
            acc = fma((double)wv[i].x, (double)xv[i].x, acc);
            acc = fma((double)wv[i].y, (double)xv[i].y, acc);
            acc = fma((double)wv[i].z, (double)xv[i].z, acc);
            acc = fma((double)wv[i].w, (double)xv[i].w, acc);
        }
    }
    for (int o = 32; o; o >>= 1) acc += __shfl_xor(acc, o);
    if (lane == 0) scores[(size_t)t * E + e] = bias ? __fadd_rn((float)acc, bias[e]) : (float)acc;
}

// Softmax, top-K and renorm of one token's E scores by one wave; lane 0 returns the K picks.
__device__ __forceinline__ void route_topk_wave(const float *__restrict__ sc_t, int E, int K, int renorm, int lane,
                                                int *sel_i, float *sel_w, float *lbuf) {
    constexpr int PL = ROUTE_MAXE / 64;                      // scores per lane: expert lane + 64j
    float v[PL];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PL; j++) {
        const int e = lane + 64 * j;
        v[j] = e < E ? sc_t[e] : 0.0f;
        if (e < E) mx = fmaxf(mx, v[j]);
    }
    mx = wave_max_f32(mx);
#pragma unroll
    for (int j = 0; j < PL; j++) {
        const int e = lane + 64 * j;
        if (e < E) v[j] = (float)exp((double)__fsub_rn(v[j], mx));
    }
    // the double sum in expert order: the values go through the wave's LDS row (lbuf, 16-byte
    // aligned, ROUTE_MAXE floats) and every lane reads them all at the same addresses (broadcast
    // reads, 16 values per round); a wave's LDS accesses complete in order
#pragma unroll
    for (int j = 0; j < PL; j++)
        if (lane + 64 * j < E) lbuf[lane + 64 * j] = v[j];
    __builtin_amdgcn_wave_barrier();
    typedef float lf4 __attribute__((ext_vector_type(4)));
    const lf4 *l4 = reinterpret_cast<const lf4 *>(lbuf);
    double sum = 0.0;
    int e16 = 0;
    for (; e16 + 16 <= E; e16 += 16) {
        const lf4 q0 = l4[e16 / 4], q1 = l4[e16 / 4 + 1], q2 = l4[e16 / 4 + 2], q3 = l4[e16 / 4 + 3];
        sum += (double)q0.x; sum += (double)q0.y; sum += (double)q0.z; sum += (double)q0.w;
        sum += (double)q1.x; sum += (double)q1.y; sum += (double)q1.z; sum += (double)q1.w;
        sum += (double)q2.x; sum += (double)q2.y; sum += (double)q2.z; sum += (double)q2.w;
        sum += (double)q3.x; sum += (double)q3.y; sum += (double)q3.z; sum += (double)q3.w;
    }
    for (; e16 < E; e16++) sum += (double)lbuf[e16];
    unsigned used = 0;                                       // bit j: expert lane + 64j selected
#pragma unroll
    for (int j = 0; j < PL; j++) v[j] = (float)((double)v[j] / sum);
    for (int k = 0; k < K; k++) {
        // this lane's best unselected expert (lowest id first among equal values), then the wave's
        float bv = -1.0f;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < PL; j++) {
            const int e = lane + 64 * j;
            if (e < E && !((used >> j) & 1u) && v[j] > bv) { bv = v[j]; bi = e; }
        }
        wave_argmax(bv, bi);                                  // DPP and readlane: no LDS round trips
        if ((bi & 63) == lane) used |= 1u << (bi >> 6);
        sel_w[k] = bv;
        sel_i[k] = bi;
    }
    if (lane == 0 && renorm) {
        double s = 0.0;
        for (int k = 0; k < K; k++) s += (double)sel_w[k];
        if (s > 0.0)
            for (int k = 0; k < K; k++) sel_w[k] = (float)((double)sel_w[k] / s);
    }
}

// softmax, top-K and renorm of one token per wave (grid T, 64 threads).
__global__ __launch_bounds__(64) void k_moe_route_topk(const float *__restrict__ scores, int E, int K, int renorm,
                                                       int32_t *__restrict__ idx_out, float *__restrict__ w_out) {
    __shared__ __align__(16) float lbuf[ROUTE_MAXE];
    const int t = blockIdx.x, lane = threadIdx.x;
    float sel_w[MOE_MAX_K];
    int sel_i[MOE_MAX_K];
    route_topk_wave(scores + (size_t)t * E, E, K, renorm, lane, sel_i, sel_w, lbuf);
    if (lane != 0) return;
    for (int k = 0; k < K; k++) {
        idx_out[(size_t)t * K + k] = sel_i[k];
        w_out[(size_t)t * K + k] = sel_w[k];
    }
}

// The top-K of every token (one wave per token in turn) and the bucketing of the T*K pairs by
// expert (k_moe_bucket's outputs, stable in pair order) in one workgroup: the whole routing after
// the scores is one launch.
__global__ __launch_bounds__(1024) void k_moe_route_bucket(const float *__restrict__ scores, int T, int E, int K, int renorm,
                                                           int32_t *__restrict__ idx_out, float *__restrict__ w_out,
                                                           int *__restrict__ off, int *__restrict__ perm,
                                                           int *__restrict__ pos, int *__restrict__ tok) {
    extern __shared__ int sm[];
    __shared__ __align__(16) float lbuf[16][ROUTE_MAXE];   // a row per wave
    int *start = sm;               // [E + 1]
    int *ids = sm + E + 1;         // [P]
    const int P = T * K, wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    for (int e = threadIdx.x; e <= E; e += blockDim.x) start[e] = 0;
    for (int t = wave; t < T; t += nw) {
        float sel_w[MOE_MAX_K];
        int sel_i[MOE_MAX_K];
        route_topk_wave(scores + (size_t)t * E, E, K, renorm, lane, sel_i, sel_w, lbuf[wave]);
        if (lane == 0)
            for (int k = 0; k < K; k++) {
                idx_out[(size_t)t * K + k] = sel_i[k];
                w_out[(size_t)t * K + k] = sel_w[k];
                ids[t * K + k] = sel_i[k] < E ? sel_i[k] : -1;   // a slot no score filled
            }
    }
    __syncthreads();
    for (int p = threadIdx.x; p < P; p += blockDim.x)
        if (ids[p] >= 0) atomicAdd(&start[ids[p]], 1);
    __syncthreads();
    bucket_scan(start, E);
    __syncthreads();
    for (int e = threadIdx.x; e <= E; e += blockDim.x) off[e] = start[e];
    for (int p = threadIdx.x; p < P; p += blockDim.x) {
        const int e = ids[p];
        if (e < 0) { pos[p] = -1; continue; }
        int rank = 0;
        for (int q = 0; q < p; q++) rank += ids[q] == e;
        const int s = start[e] + rank;
        perm[s] = p;
        pos[p] = s;
        tok[s] = p / K;
    }
}

// The router's checks and its scores kernel; *scores: the [T][E] scores in the context's scratch.
static int route_scores(bgl_ctx *c, const char *who, const float *rw_dev, const float *rb_dev, int E, int in,
                        const float *x_dev, int T, int K, float **scores) {
    if (!c || !rw_dev || !x_dev || T < 1) return bgl_fail(BGL_E_ARG, "%s: bad argument", who);
    if (E < 1 || E > ROUTE_MAXE || K < 1 || K > E || K > MOE_MAX_K)
        return bgl_fail(BGL_E_ARG, "%s: need 1 <= K <= min(E, %d) and E <= %d (E=%d, K=%d)", who, MOE_MAX_K, ROUTE_MAXE, E, K);
    if (in < 4 || in % 4 || ((uintptr_t)rw_dev | (uintptr_t)x_dev) % 16)
        return bgl_fail(BGL_E_ARG, "%s: in=%d must be a multiple of 4 with 16-byte aligned rows", who, in);
    HIPCHK(hipSetDevice(c->device));
    if (dbuf_reserve(c, c->moe_scores, (size_t)T * E * 4, false)) return bgl_last_code();
    *scores = (float *)c->moe_scores.p;
    int tok = prof_begin(c, 2);
    hipLaunchKernelGGL(k_moe_router_scores, dim3(T, (E + ROUTE_EPW - 1) / ROUTE_EPW), dim3(ROUTE_EPW * 64), 0, c->stream, rw_dev,
                       rb_dev, E, in, x_dev, *scores);
    prof_end(c, tok);
    HIPCHK(hipGetLastError());
    return 0;
}

extern "C" int bgl_moe_route_dev(bgl_ctx *c, const float *rw_dev, const float *rb_dev, int E, int in, const float *x_dev,
                                 int T, int K, int renorm, int32_t *idx_dev, float *w_dev) {
    if (!idx_dev || !w_dev) return bgl_fail(BGL_E_ARG, "bgl_moe_route_dev: bad argument");
    float *scores = nullptr;
    int rc = route_scores(c, "bgl_moe_route_dev", rw_dev, rb_dev, E, in, x_dev, T, K, &scores);
    if (rc) return rc;
    int tok = prof_begin(c, 2);
    hipLaunchKernelGGL(k_moe_route_topk, dim3(T), dim3(64), 0, c->stream, (const float *)scores, E, K, renorm ? 1 : 0, idx_dev, w_dev);
    prof_end(c, tok);
    HIPCHK(hipGetLastError());
    return 0;
}

extern "C" int bgl_moe_layer_dev(bgl_ctx *c, const float *rw_dev, const float *rb_dev, int renorm, const bgl_tensor *gate,
                                 const bgl_tensor *up, const bgl_tensor *down, const bgl_tensor *sg, const bgl_tensor *su,
                                 const bgl_tensor *sd, const float *x_dev, int T, int K, float *out_dev) {
    if (!c || !gate || T < 1 || K < 1) return bgl_fail(BGL_E_ARG, "bgl_moe_layer_dev: bad argument");
    int rc;
    if ((rc = expert_check(gate, "bgl_moe_layer_dev: gate"))) return rc;
    const int E = (int)gate->experts.size(), H = gate->T.K;
    HIPCHK(hipSetDevice(c->device));
    if (dbuf_reserve(c, c->moe_route, (size_t)T * K * 8, false)) return bgl_last_code();
    int32_t *idx = (int32_t *)c->moe_route.p;
    float *w = (float *)(idx + (size_t)T * K);
    float *scores = nullptr;
    if ((rc = route_scores(c, "bgl_moe_layer_dev", rw_dev, rb_dev, E, H, x_dev, T, K, &scores))) return rc;
    // up to 16 tokens (one per wave): top-K and bucketing in one launch, then the FFN without its
    // own bucketing; more tokens: a wave per token in parallel (one workgroup walking 64 tokens'
    // top-K measured 35 us slower per layer at T = 64)
    if (T > 16) {
        int tok = prof_begin(c, 2);
        hipLaunchKernelGGL(k_moe_route_topk, dim3(T), dim3(64), 0, c->stream, (const float *)scores, E, K, renorm ? 1 : 0, idx, w);
        prof_end(c, tok);
        HIPCHK(hipGetLastError());
        return moe_ffn(c, gate, up, down, sg, su, sd, x_dev, idx, w, T, K, out_dev, nullptr);
    }
    MoeScratch S;
    if ((rc = moe_scratch(c, T * K, E, S))) return rc;
    int tok = prof_begin(c, 2);
    hipLaunchKernelGGL(k_moe_route_bucket, dim3(1), dim3(1024), ((size_t)E + 1 + (size_t)T * K) * 4, c->stream,
                       (const float *)scores, T, E, K, renorm ? 1 : 0, idx, w, S.off, S.perm, S.pos, S.tok);
    prof_end(c, tok);
    HIPCHK(hipGetLastError());
    return moe_ffn(c, gate, up, down, sg, su, sd, x_dev, idx, w, T, K, out_dev, &S);
}
