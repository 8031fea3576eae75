// bgl_mlp_q.hip -- the dense MLP block of one decode step (forward_token, qwen_infer.c:1560-1573)
// at one W4A8 column in a single launch: g = W_gate x and u = W_up x, h = silu(g) * u (swiglu,
// qwen_infer.c:726-733), y = W_down h.
//
// The grid holds two roles.  Workgroups [0, ngu) run gate+up: each quantizes x into LDS once (the
// reference's q4_quant_act_i8 / _g256, bit for bit), and each of its waves then runs one item of 8
// rows of BOTH gate and up (the same rows): the units of the two tensors, the fold of each row in
// the reference's group order (q4gemv.h:241, q4gemv_g256.h:154) and h for its rows.  With one item
// per wave, a CU's share of the gate+up bytes is at most its waves' items (a whole-workgroup row
// slice of 32 rows left some CUs with two slices and the launch waiting on them).  Workgroups
// [ngu, ngu + nd) each own 8 rows of down.  Each of their waves first waits a fixed delay (about
// the time the gate+up weights take to stream, so that the gate+up role's x and weights are not
// queued behind the down weights), then loads ALL its weight units at once (they do not depend on
// h), then loads the 256-value groups of h its own units read until they are complete: as soon as
// the groups of one of its unit iterations are, it quantizes exactly those (every unit's codes are
// made by the wave that uses them, so no workgroup barrier comes between the quantization and the
// dot products) and runs that iteration's units.  A last barrier and the fold follow.  So the
// block is one launch instead of three (gate+up, SwiGLU, down), the down weights stream while
// gate+up computes, and when the last h rows land only their iteration is left.  Every value is
// the one the three-launch path computes: g, u and y bit for bit, h with the same arithmetic.
//
// Publishing h across workgroups (which run on different XCDs, each with its own L2): h is written
// and read with device-scope (sc1) buffer accesses, which the L2s do not hold stale, so no cache
// maintenance is needed, and the data carries its own "not yet" mark.  h has two buffers, used in
// turn by successive launches of one shape; a slot of the buffer a launch reads holds a sentinel (a
// signalling-NaN bit pattern, which no arithmetic produces: every NaN an operation returns is
// quiet) until its gate+up wave stores the value, and that wave also puts the sentinel back into
// its rows of the other buffer for the next launch.  A producer stores its rows and moves on: no
// wait for the stores to complete, no atomic read-modify-write.  Each workgroup keeps its own
// count of the launches it has run on this shape (which buffer is current is its parity; every
// workgroup of a launch has the same count), read at its start and stored +1 at its end, so graph
// replays need no memset.  The wait is bounded: after `spin` rounds a wave gives up, sets the
// host-visible flag and finishes with whatever h holds (bgl_ctx_check reports it); the buffers
// stay consistent because every producer resets its rows of the other buffer in every launch.  No
// workgroup waits on one that is not yet running: the gate+up workgroups have the lower ids, so
// the dispatcher starts every one of them before any down workgroup, and they wait on nothing.
#include <string.h>

#include <algorithm>

#include "../../include/beglin_qgemv.h"
#include "bgl_gemv_q.h"
#include "bgl_internal.h"

#define HIPCHK(expr)                                                                             \
    do {                                                                                         \
        hipError_t e_ = (expr);                                                                  \
        if (e_ != hipSuccess) return bgl_fail(BGL_E_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

// The sync buffer of one MLP shape: [the timeout flag, padded to 64 bytes][h buffer 0: I floats]
// [h buffer 1: I floats][launch count of each gate+up workgroup: ngu ints][of each down workgroup:
// nd ints].
#define MLP_TRD 8             // rows of down per workgroup
#define MLP_MAXQ 8            // 256-value passes of h a down wave may quantize (its units' groups)
#define MLP_MAXW 12           // waves per workgroup; at most 168 VGPRs (3 waves per SIMD), so a CU
                              // holds a gate+up and a down workgroup of 6 waves together
#define MLP_EMPTY 0x7F800001u // the sentinel of an h slot not yet written (a signalling NaN)

struct MlpQLaunch {
    BglDevTensor gate, up, down;   // gate / up [I][H], down [H][I], one format
    const float *x;                // [H]
    float *hb;                     // [2][I] the two h buffers
    float *hout;                   // [I] the caller's copy of h, or null
    float *y;                      // [H]
    int *gen_gu, *gen_d;           // [ngu], [nd] launches each workgroup has run on this shape
    int *flag;                     // the timeout flag
    int ngu, nd;                   // workgroups of each role
    int never;                     // 1: the down waves' wait is never satisfied (tests of the give-up path)
    int spin;                      // polls before a down wave gives up
    int delay;                     // 10 ns ticks a down wave waits before it loads its weights (0: none)
};

// buffer-resource word 3 for raw 32-bit accesses, and the cache-policy bit that makes a buffer
// access device-scope coherent (sc1)
#define MLP_RSRC_W3 0x00020000
#define MLP_SC1 16

__device__ __forceinline__ __amdgpu_buffer_rsrc_t mlp_rsrc(const void *p, int n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, n * 4, MLP_RSRC_W3);
}

// the SwiGLU of k_swiglu (bgl_mlp.hip): g / (1 + exp(-g)) * u, the exponential rounded once from double
__device__ __forceinline__ float mlp_swiglu(float g, float u) {
    const float e = (float)exp(-(double)g);
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, e)), u);
}

// a row's sequential fold of U fp32 terms at stride TR (k_gemv_q's order: u ascending).  The LDS
// reads go out 16 at a time, a batch ahead of the adds, so the adds do not wait on one read each.
template <int TR>
__device__ __forceinline__ float mlp_fold(const float *tr, int U) {
    float acc = 0.0f, t[16], n[16];
    const int U16 = U & ~15;
    if (U16) {
#pragma unroll
        for (int i = 0; i < 16; i++) t[i] = tr[i * TR];
    }
    for (int g = 0; g < U16; g += 16) {
        if (g + 16 < U16) {
#pragma unroll
            for (int i = 0; i < 16; i++) n[i] = tr[(g + 16 + i) * TR];
        }
#pragma unroll
        for (int i = 0; i < 16; i++) acc = __fadd_rn(acc, t[i]);
#pragma unroll
        for (int i = 0; i < 16; i++) t[i] = n[i];
    }
    const int R = U - U16;
    // the tail: every load unconditional (clamped to a real term), the adds selected, so no
    // branch per term
#pragma unroll
    for (int i = 0; i < 16; i++) t[i] = tr[max(U16 + min(i, R - 1), 0) * TR];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float s = __fadd_rn(acc, t[i]);
        acc = i < R ? s : acc;
    }
    return acc;
}

// The x values of QP passes p0, p0 + stride, ... (lane l: values 4l..4l+3 of each; addresses
// clamped, so every load is valid).  COH: device-scope loads (h, written by other workgroups).
template <int QP, bool COH>
__device__ __forceinline__ void mlp_xload(float4 (&v)[QP], const float *x, int p0, int stride, int K, int lane) {
    const __amdgpu_buffer_rsrc_t R = mlp_rsrc(x, K);
#pragma unroll
    for (int i = 0; i < QP; i++) {
        const int off = min(256 * (p0 + i * stride) + 4 * lane, K - 4);
        bgl_f32x4 t;
        if constexpr (COH) t = __builtin_bit_cast(bgl_f32x4, __builtin_amdgcn_raw_buffer_load_b128(R, off * 4, 0, MLP_SC1));
        else t = *((const BGL_GLOBAL bgl_f32x4 *)(x + off));
        v[i] = make_float4(t.x, t.y, t.z, t.w);
    }
}

template <int FMT, int GP, int NIT>
__global__ __launch_bounds__(MLP_MAXW * BGL_TILE, 4) void k_mlp_q(MlpQLaunch L) {
    extern __shared__ __align__(16) unsigned char lds[];
    using QU = QUnit<FMT>;
    const int nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if ((int)blockIdx.x < L.ngu) {
        // ------------------------------------------------------------ gate + up: items of 8 rows
        // An item is 8 consecutive rows of BOTH gate and up; a wave runs whole items (item k = rows
        // 8k .. 8k+7), the workgroup only shares the quantized x.  Lane l: row l % 8 and, of each
        // unit iteration's UPI = 4 units, unit (l / 8) / 2 (two lanes share a unit, half its chunks
        // each); unit v < U is gate's unit v, v >= U up's unit v - U (the same shape and layout).
        // The unit iterations are loaded GP at a time: GP >= 3 means every iteration of an item in
        // one group (the host picks it only then), else the next group loads while one computes.
        constexpr int TRI = MLP_TRD, IPT = BGL_TILE / TRI, KQ = BGL_TILE / TRI, H = 2, UPI = KQ / H;
        const int b = blockIdx.x;
        const BglDevTensor &T = L.gate;
        const int K = T.K, U = T.nunits, U2 = 2 * U, NGQ = K / QU::GQ, NP = (K + 255) / 256;
        const int NG = ((U2 + UPI - 1) / UPI + GP - 1) / GP;
        const int nitems = (T.N + TRI - 1) / TRI;
        const unsigned gen = (unsigned)L.gen_gu[b];          // this shape's launches so far: its parity picks the buffer
        int8_t *xq = reinterpret_cast<int8_t *>(lds);
        float *asc = reinterpret_cast<float *>(lds + (size_t)(U + 1) * QU::STRIDE);
        int *xsum = reinterpret_cast<int *>(asc + NGQ + 1);
        float *tw = reinterpret_cast<float *>(xsum + K / 64 + 1) + (size_t)wave * U2 * TRI;   // this wave's terms [v][8]
        const int r = lane % TRI, j = lane / TRI, kq = j / H, hh = j % H;
        auto ld = [&](RawPart<FMT, H>(&c)[GP], int item, int g) {
            const int tile = item / IPT, rr = (item % IPT) * TRI + r;
#pragma unroll
            for (int i = 0; i < GP; i++) {
                const int v = min((g * GP + i) * UPI + kq, U2 - 1);
                BglDevTensor Tv = L.gate;
                if (v >= U) { Tv.w = L.up.w; Tv.s0 = L.up.s0; }
                load_part<FMT, H>(c[i], Tv, tile, rr, v >= U ? v - U : v, hh);
            }
        };
        auto em = [&](const RawPart<FMT, H>(&c)[GP], int g) {
#pragma unroll
            for (int i = 0; i < GP; i++) {
                const int v = (g * GP + i) * UPI + kq, vc = min(v, U2 - 1), u = vc >= U ? vc - U : vc;
                int p = unit_part<FMT, H>(c[i], xq, u, hh);
                p += __shfl_xor(p, TRI);
                if (hh == 0 && v < U2) tw[v * TRI + r] = unit_float<FMT>(p, c[i].s, T.gmul, asc, xsum, u);
            }
        };
        // x loads first, then the first item's first weight units: vector loads retire in order, so
        // the quantization waits only for x while the weight bytes are in flight.  Both unconditional
        // (a wave without an item loads the last one's), so no wait merges paths.
        const int item = b + wave * L.ngu;                  // ngu * nw >= items: one item per wave at most
        float4 xv[2];
        mlp_xload<2, false>(xv, L.x, wave, nw, K, lane);
        constexpr bool ONE = GP >= 3;
        RawPart<FMT, H> ca[GP], cb[ONE ? 1 : GP];
        ld(ca, min(item, nitems - 1), 0);
        __builtin_amdgcn_sched_barrier(0);
        if (wave < NP) quant_passes<FMT, 2, 1>(xv, wave, nw, K, NP, 1, NGQ, U, lane, xq, asc, xsum);
        for (int p0 = wave + 2 * nw; p0 < NP; p0 += 2 * nw) {
            mlp_xload<2, false>(xv, L.x, p0, nw, K, lane);
            quant_passes<FMT, 2, 1>(xv, p0, nw, K, NP, 1, NGQ, U, lane, xq, asc, xsum);
        }
        __syncthreads();
        const __amdgpu_buffer_rsrc_t HB = mlp_rsrc(L.hb, 2 * T.N);
        if (item < nitems) {
            if constexpr (ONE) {
                em(ca, 0);
            } else {
                for (int g = 0;; g++) {
                    if (g + 1 >= NG) {
                        em(ca, g);
                        break;
                    }
                    ld(cb, item, g + 1);
                    em(ca, g);
#pragma unroll
                    for (int i = 0; i < GP; i++) ca[i] = cb[i];
                }
            }
            // the terms were written by this wave's lanes: LDS operations of a wave are in order
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const int row = item * TRI + lane;
            if (lane < TRI && row < T.N) {
                const float g = mlp_fold<TRI>(tw + lane, U), u = mlp_fold<TRI>(tw + U * TRI + lane, U);
                const float hv = mlp_swiglu(g, u);
                // the value into this launch's buffer, the sentinel back into the other one's row
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(hv), HB, ((gen & 1u) * T.N + row) * 4, 0, MLP_SC1);
                __builtin_amdgcn_raw_buffer_store_b32(MLP_EMPTY, HB, ((~gen & 1u) * T.N + row) * 4, 0, MLP_SC1);
                if (L.hout) L.hout[row] = hv;
            }
        }
        __syncthreads();                                       // every wave has read gen
        if (threadIdx.x == 0) L.gen_gu[b] = (int)(gen + 1u);   // read by this workgroup's next launch only
        return;
    }
    // ---------------------------------------------------------------- down: MLP_TRD rows
    // Lane l: row l % 8 and, of each wave iteration's UPI = 4 units, unit (l / 8) / 2 (two lanes
    // share a unit, half its chunks each).  Wave w takes the wave iterations it * nwl + w, it < NIT;
    // the UPI units of one iteration are PPI whole 256-value passes of h (g256sf: 4, g64: 1).
    constexpr int TRD = MLP_TRD, SUBS = BGL_TILE / TRD, KQ = BGL_TILE / TRD, H = 2, UPI = KQ / H;
    constexpr int PPI = UPI * QU::ELEMS / 256, NQ = NIT * PPI;
    static_assert(NQ <= MLP_MAXQ, "a down wave quantizes at most MLP_MAXQ passes");
    const int d = blockIdx.x - L.ngu, tile = d / SUBS, r0 = (d % SUBS) * TRD;
    const BglDevTensor &T = L.down;
    const int K = T.K, U = T.nunits, NGQ = K / QU::GQ, NP = K / 256;
    const int UIT = (U + UPI - 1) / UPI, nwl = min(nw, UIT);
    int8_t *xq = reinterpret_cast<int8_t *>(lds);
    float *asc = reinterpret_cast<float *>(lds + (size_t)(U + 1) * QU::STRIDE);
    int *xsum = reinterpret_cast<int *>(asc + NGQ + 1);
    float *tl = reinterpret_cast<float *>(xsum + K / 64 + 1);
    const int r = lane % TRD, j = lane / TRD, kq = j / H, hh = j % H, rr = r0 + r;
    const unsigned gen = (unsigned)L.gen_d[d];                   // this shape's launches so far
    const float *hc = L.hb + (size_t)(gen & 1u) * K;
    if (wave < nwl) {
        // First `delay` (about the time the gate+up weights take to stream), so that the gate+up
        // role's x and weights are not queued behind these, then every weight unit of this wave,
        // before anything depends on h.
        if (L.delay > 0) {
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            while (__builtin_amdgcn_s_memrealtime() - t0 < (uint64_t)L.delay) __builtin_amdgcn_s_sleep(8);
        }
        RawPart<FMT, H> cw[NIT];
#pragma unroll
        for (int it = 0; it < NIT; it++) load_part<FMT, H>(cw[it], T, tile, rr, min((it * nwl + wave) * UPI + kq, U - 1), hh);
        // The wave's passes of h, loaded again while any is incomplete (a sentinel left): an
        // iteration's PPI passes are quantized into LDS and its dot products run as soon as all of
        // them are complete, so once the last gate+up rows land only their iteration remains.  The
        // wait is bounded: after `spin` rounds one more round runs with whatever h holds and the
        // flag is set.  ipend: iterations still to do (wave-uniform).
        uint32_t ipend = 0u;
#pragma unroll
        for (int it = 0; it < NIT; it++)
            if (it * nwl + wave < UIT) ipend |= 1u << it;
        bool ok = true;
        for (int s = 0;;) {
#pragma unroll
            for (int it = 0; it < NIT; it++) {
                if (!(ipend >> it & 1u)) continue;
                const int p0 = (it * nwl + wave) * PPI;
                float4 hv[PPI];
                mlp_xload<PPI, true>(hv, hc, p0, 1, K, lane);
                bool e = false;
#pragma unroll
                for (int k = 0; k < PPI; k++)
                    if (p0 + k < NP)
                        e |= __float_as_uint(hv[k].x) == MLP_EMPTY || __float_as_uint(hv[k].y) == MLP_EMPTY ||
                             __float_as_uint(hv[k].z) == MLP_EMPTY || __float_as_uint(hv[k].w) == MLP_EMPTY;
                if ((__builtin_amdgcn_ballot_w64(e) != 0 || L.never) && ok) continue;
                quant_passes<FMT, PPI, 1>(hv, p0, 1, K, NP, 1, NGQ, U, lane, xq, asc, xsum);
                // the codes this wave reads were written by this wave: LDS operations of a wave are in order
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const int u = (it * nwl + wave) * UPI + kq;
                int p = unit_part<FMT, H>(cw[it], xq, min(u, U - 1), hh);
                p += __shfl_xor(p, TRD);
                if (hh == 0 && u < U) tl[u * TRD + r] = unit_float<FMT>(p, cw[it].s, T.gmul, asc, xsum, u);
                ipend &= ~(1u << it);
            }
            if (ipend == 0u) break;
            if (++s >= L.spin) ok = false;
            else __builtin_amdgcn_s_sleep(2);
        }
        if (!ok && lane == 0) __hip_atomic_store(L.flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (threadIdx.x < TRD) {
        const int row = tile * BGL_TILE + r0 + threadIdx.x;
        if (row < T.N) L.y[row] = mlp_fold<TRD>(tl + threadIdx.x, U);
    }
    if (threadIdx.x == 0) L.gen_d[d] = (int)(gen + 1u);  // read by this workgroup's next launch only
}

// LDS bytes of one role: the column's codes, scales and code sums, and nterm x TR fp32 terms.
static size_t mlp_role_lds(int fmt, int K, int U, int nterm, int TR) {
    const int GQ = fmt == BGL_Q4G256SF ? 256 : 64, ELEMS = fmt == BGL_Q4G256SF ? 256 : 64;
    return (size_t)(U + 1) * (ELEMS + 16) + 4 * (size_t)(K / GQ + 1) + 4 * (size_t)(K / 64 + 1) + 4 * (size_t)nterm * TR;
}

template <int FMT, int GP>
static int mlp_launch_nit(int NIT, const MlpQLaunch &L, dim3 g, dim3 b, size_t lds, hipStream_t st) {
    switch (NIT) {
    case 1: hipLaunchKernelGGL((k_mlp_q<FMT, GP, 1>), g, b, lds, st, L); return 0;
    case 2: hipLaunchKernelGGL((k_mlp_q<FMT, GP, 2>), g, b, lds, st, L); return 0;
    default: break;
    }
    if constexpr (FMT != BGL_Q4G256SF) {              // one pass per iteration: up to 8 iterations
        switch (NIT) {
        case 4: hipLaunchKernelGGL((k_mlp_q<FMT, GP, 4>), g, b, lds, st, L); return 0;
        case 8: hipLaunchKernelGGL((k_mlp_q<FMT, GP, 8>), g, b, lds, st, L); return 0;
        default: break;
        }
    }
    return -1;
}

// The launch shape of one MLP: waves per workgroup (the fewest from 6 up that keep every down wave
// at <= MLP_MAXQ passes of h), wave iterations per down wave (the instantiated 1, 2, 4 or 8 >= what
// the shape needs), the gate+up workgroups (one 8-row item per wave: Qwen2.5-1.5B's 1120 items in
// 187 workgroups of 6 waves) and the down workgroups (8 rows each).  False if the shape cannot run
// in one launch.
struct MlpShape {
    int nw, NIT, ngu, nd;
};
static bool mlp_shape(bgl_ctx *c, const BglDevTensor &gate, const BglDevTensor &down, MlpShape &s) {
    const int ppi = gate.fmt == BGL_Q4G256SF ? 4 : 1;
    const int U = down.nunits, UIT = (U + 3) / 4;
    const int nitems = (gate.N + MLP_TRD - 1) / MLP_TRD;
    s.nd = down.ntiles * (BGL_TILE / MLP_TRD);
    int nw0 = c->mlp_waves ? c->mlp_waves : 6;
    for (int nw = nw0; nw <= MLP_MAXW; nw++) {
        const int nwl = std::min(nw, UIT), nit = (UIT + nwl - 1) / nwl;
        const int NIT = nit <= 1 ? 1 : nit <= 2 ? 2 : nit <= 4 ? 4 : 8;
        if (nit <= NIT && NIT * ppi <= MLP_MAXQ) {      // every wave iteration covered, <= MLP_MAXQ passes
            s.nw = nw;
            s.NIT = NIT;
            s.ngu = std::max(c->mlp_gu, (nitems + nw - 1) / nw);
            return nw <= c->max_waves;
        }
        if (c->mlp_waves) break;
    }
    return false;
}

// LDS of the single-launch kernel: the larger of the two roles'
static size_t mlp_lds(const BglDevTensor &gate, const BglDevTensor &down, const MlpShape &s) {
    return std::max(mlp_role_lds(gate.fmt, gate.K, gate.nunits, 2 * gate.nunits, MLP_TRD * s.nw),
                    mlp_role_lds(down.fmt, down.K, down.nunits, down.nunits, MLP_TRD));
}

bool mlp_q_ok(bgl_ctx *c, const BglDevTensor &g, const BglDevTensor &u, const BglDevTensor &d) {
    const int f = g.fmt;
    if (f != BGL_Q4G256SF && f != BGL_Q4G64 && f != BGL_Q8G64) return false;
    if (u.fmt != f || d.fmt != f || u.gmul != g.gmul || d.gmul != g.gmul) return false;
    if (g.K % 256 || d.K % 256) return false;              // whole 256-value groups of x and of h
    MlpShape s;
    if (!mlp_shape(c, g, d, s)) return false;
    return mlp_lds(g, d, s) <= 65536;
}

// One column through the single-launch block.  Shapes as bgl_mlp_dev checked them, and mlp_q_ok.
int run_mlp_q(bgl_ctx *c, const BglDevTensor &gate, const BglDevTensor &up, const BglDevTensor &down, const float *x,
              float *h, float *y) {
    MlpShape s;
    if (!mlp_shape(c, gate, down, s)) return bgl_fail(BGL_E_UNSUPPORTED, "single-launch MLP: no launch shape");
    // the sync buffer of this shape: its h buffers and its workgroups' launch counts only mean
    // something between launches of one shape (made once: counts 0, both h buffers empty)
    const int I = down.K;
    DevBuf &sb = c->mlp_sync[((uint64_t)(uint32_t)I << 32) | (uint32_t)s.nd];
    const bool fresh = sb.p == nullptr;
    const size_t bytes = (16 + 2 * (size_t)I + s.ngu + s.nd) * 4;
    if (dbuf_reserve(c, sb, bytes, true)) return bgl_last_code();
    if (fresh) {
        HIPCHK(hipMemsetD32Async((hipDeviceptr_t)((int *)sb.p + 16), (int)MLP_EMPTY, 2 * (size_t)I, c->stream));
        HIPCHK(hipStreamSynchronize(c->stream));
    }
    MlpQLaunch L;
    memset(&L, 0, sizeof L);
    L.gate = gate; L.up = up; L.down = down;
    L.x = x; L.hout = h; L.y = y;
    L.flag = (int *)sb.p;
    L.hb = (float *)sb.p + 16;
    L.gen_gu = (int *)(L.hb + 2 * (size_t)I);
    L.gen_d = L.gen_gu + s.ngu;
    L.ngu = s.ngu;
    L.nd = s.nd;
    L.never = c->mlp_test_timeout > 0 ? 1 : 0;                  // a test's launch whose wait must give up
    if (c->mlp_test_timeout > 0) c->mlp_test_timeout--;
    L.spin = c->mlp_spin;
    // the down waves' delay: the time the gate+up weight bytes take at 5 TB/s, about what a
    // streaming read sustains here (5000 bytes per ns; Qwen2.5-1.5B: 14.6 MB, 2.9 us: 10.9 us per
    // block against 12.7 at 2.0 us and 11.3 at 3.5 us), in 10 ns ticks
    const long gu_bytes = (long)2 * gate.ntiles * BGL_TILE * gate.nunits * (long)(gate.fmt == BGL_Q4G256SF ? 136 : gate.fmt == BGL_Q4G64 ? 36 : 68);
    L.delay = (c->mlp_delay >= 0 ? c->mlp_delay : (int)std::min(gu_bytes / 5000, 100000L)) / 10;
    const int fmt = gate.fmt;
    const size_t lds = mlp_lds(gate, down, s);
    const dim3 g(L.ngu + L.nd), b(s.nw * BGL_TILE);
    int tok = prof_begin(c, 1);
    int rc;
    // unit iterations of a gate+up item loaded per group: all of them when they are <= 3 (g256sf at
    // K <= 1536: Qwen2.5-1.5B's 12 units of gate+up), else 2 at a time, double-buffered
    const int git = (2 * gate.nunits + 3) / 4;
    switch (fmt) {
    case BGL_Q4G256SF:
        rc = git <= 3 ? mlp_launch_nit<BGL_Q4G256SF, 3>(s.NIT, L, g, b, lds, c->stream)
                      : mlp_launch_nit<BGL_Q4G256SF, 2>(s.NIT, L, g, b, lds, c->stream);
        break;
    case BGL_Q4G64: rc = mlp_launch_nit<BGL_Q4G64, 2>(s.NIT, L, g, b, lds, c->stream); break;
    default: rc = mlp_launch_nit<BGL_Q8G64, 2>(s.NIT, L, g, b, lds, c->stream); break;
    }
    prof_end(c, tok);
    if (rc) return bgl_fail(BGL_E_UNSUPPORTED, "single-launch MLP: no kernel for %d iterations", s.NIT);
    HIPCHK(hipGetLastError());
    return 0;
}

extern "C" int bgl_ctx_check(bgl_ctx *c) {
    if (!c) return bgl_fail(BGL_E_ARG, "bgl_ctx_check: NULL context");
    HIPCHK(hipSetDevice(c->device));
    HIPCHK(hipStreamSynchronize(c->stream));
    bool gave_up = false;
    for (auto &kv : c->mlp_sync) {
        const DevBuf &sb = kv.second;
        if (!sb.p) continue;
        int *flag = (int *)sb.p;
        int f = 0;
        HIPCHK(hipMemcpy(&f, flag, sizeof f, hipMemcpyDeviceToHost));
        if (!f) continue;
        const int zero = 0;
        HIPCHK(hipMemcpy(flag, &zero, sizeof zero, hipMemcpyHostToDevice));
        gave_up = true;
    }
    if (gave_up)
        return bgl_fail(BGL_E_TIMEOUT, "a single-launch MLP block stopped waiting for its gate+up workgroups: its outputs are invalid");
    return 0;
}
