// bgl_mfma.hip -- batched GEMM for M >= 16 activation rows on the gfx950 fp16 matrix cores
// (the M-column case of gemm_qXg64_mt / qng64_matmul_f32, q4gemv.h:761-769, qng64_dense.c:70-79).
//
// Numerics.  Weight codes are exact in fp16 (int4 and int8 codes, qNg64 codes for n <= 10), so
// the decode is exact.  Each activation column is scaled by a power of two so its largest
// magnitude lies in [2^13, 2^14), then split as hi = fp16(x'), lo = fp16(x' - hi): hi + lo holds
// x' to about 2^-22 of the column maximum.  v_mfma_f32_16x16x32_f16 multiplies exactly and
// accumulates in fp32; each quantization group's partial sum is folded with its fp32 scale (one
// FMA per output per group) and the column factor 2^-(14-e) is applied at the end.
//
// Layout.  A (weights, 16 rows x 32 k per instruction): lane l holds row l%16 and the 8 elements
// 8*(l/16)..+7 of the 32-element K-step -- with the device's 16-byte chunk layout that is one
// dword (int4) or two (int8) per lane and row block, and a wave's load covers 256 contiguous
// bytes.  The int4 nibble order (byte i: element i low, element 4+i high) decodes into halves in
// the order {0,2,1,3,4,6,5,7}; the activation fragments are stored in that same order, since the
// MFMA only needs A and B to agree element for element.  B (activations, 32 k x 16 columns):
// lane l holds column l%16, elements 8*(l/16)..+7.  D: lane l holds column l%16, rows
// 4*(l/16)..+3 of the 16-row block.
//
// Work split.  A workgroup = 4 waves = 4 consecutive 64-row weight tiles (256 rows) over one
// K range; the 4 waves share the activation fragments of that range, staged through LDS in
// blocks of MF_KC K-steps (double buffered).  Each wave computes its tile's 4 row blocks x CT
// column tiles.  Shapes with few tiles split K over blockIdx.y into fp32 partials that
// k_splitk_reduce adds in split order (deterministic; no atomics).
#include <string.h>

#include "bgl_gemv_impl.h"
#include "bgl_internal.h"

#define HIPCHK(expr)                                                                             \
    do {                                                                                         \
        hipError_t e_ = (expr);                                                                  \
        if (e_ != hipSuccess) return bgl_fail(BGL_E_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

typedef _Float16 mf_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 mf_h2 __attribute__((ext_vector_type(2)));
typedef float mf_f4 __attribute__((ext_vector_type(4)));
typedef unsigned int mf_u4 __attribute__((ext_vector_type(4)));

#define MF_TILES 4           // 64-row weight tiles per workgroup (they share the staged activations)
#define MF_RBW 2             // 16-row blocks per wave: two waves per tile
#define MF_WAVES (MF_TILES * 4 / MF_RBW)
#define MF_KC 4              // K-steps (32 elements each) per staged activation block
#define MF_MAXCT 4           // column tiles (16 columns each) per launch: up to 64 columns
#define MF_MAXN 10           // qNg64 widths whose codes are exact in fp16 via the 1024+u trick
#ifndef MF_WPE_INT4
#define MF_WPE_INT4 0      // 1: ask for 4 waves per SIMD on the int4 kernels of up to 32 columns
#endif

static inline unsigned nblk(long n, int bs = 256) { return (unsigned)((n + bs - 1) / bs); }

struct MfmaLaunch {
    BglDevTensor T;
    const uint4 *xf;         // activation fragments [K/32][CT][2][64] x 16 B
    const float *colinv;     // [16*CT] column factors 2^(e-14)
    const float *bias;       // [N] or null
    float *y;                // y[m][n] at y + m*ystride + n
    int ystride;
    float *part;             // K-split partials [S][M][N] (S > 1)
    int M;                   // valid columns (<= 16*CT)
    int kps;                 // K-steps per split
};

// ==================================================================================== activations
// Grid (16*CT columns, K/2048 chunks); columns >= M are zero.  x: [M][K] rows of this launch.
// Every chunk's workgroup reduces its column's max over all of K (the column is L2-resident), so
// the split needs no second pass.
#define MF_PREP_CHUNK 2048
__global__ __launch_bounds__(256) void k_act_frag(const float *__restrict__ x, int M, int K, int CT,
                                                  uint4 *__restrict__ xf, float *__restrict__ colinv) {
    __shared__ float wmax[4];
    const int m = blockIdx.x, t = threadIdx.x;
    const float *xr = x + (size_t)m * K;
    float mx = 0.0f;
    if (m < M) {                                         // K % 64 == 0: whole float4s, 4 in flight per thread
        const float4 *x4 = reinterpret_cast<const float4 *>(xr);
        const int n4 = K >> 2;
        int k = t;
        for (; k + 3 * 256 < n4; k += 4 * 256) {
            const float4 a = x4[k], b = x4[k + 256], c = x4[k + 512], d = x4[k + 768];
            mx = fmaxf(mx, fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                                 fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w)))));
            mx = fmaxf(mx, fmaxf(fmaxf(fmaxf(fabsf(c.x), fabsf(c.y)), fmaxf(fabsf(c.z), fabsf(c.w))),
                                 fmaxf(fmaxf(fabsf(d.x), fabsf(d.y)), fmaxf(fabsf(d.z), fabsf(d.w)))));
        }
        for (; k < n4; k += 256) {
            const float4 a = x4[k];
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
        }
    }
    mx = wave_max_f32(mx);
    if ((t & 63) == 0) wmax[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int e = 0;
    if (mx > 0.0f) frexpf(mx, &e);                       // mx in [2^(e-1), 2^e)
    const float sc = mx > 0.0f ? ldexpf(1.0f, 14 - e) : 1.0f;
    if (t == 0 && blockIdx.y == 0) colinv[m] = mx > 0.0f ? ldexpf(1.0f, e - 14) : 1.0f;
    const int ct = m >> 4, ml = m & 15;
    const int g = blockIdx.y * (MF_PREP_CHUNK / 8) + t;  // one 8-element slot per thread
    if (g >= K / 8) return;
    const int k0 = 8 * g, s = k0 >> 5, q = (k0 & 31) >> 3;
    const int perm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    _Float16 hi[8], lo[8];
#pragma unroll
    for (int p = 0; p < 8; p++) {
        const float v = m < M ? xr[k0 + perm[p]] * sc : 0.0f;   // power-of-two scaling: exact
        const _Float16 h = (_Float16)v;
        hi[p] = h;
        lo[p] = (_Float16)(v - (float)h);
    }
    uint4 H, L;
    memcpy(&H, hi, 16);
    memcpy(&L, lo, 16);
    const size_t base = ((size_t)s * CT + ct) * 2 * 64 + ml + 16 * q;
    xf[base] = H;
    xf[base + 64] = L;
}

// ==================================================================================== weights
// Raw A-fragment words of one K-step for one lane (row 16*rb + lane%16, slot q = lane/16).
template <int FMT, int NB> struct ARaw { uint32_t w[1]; };
template <int NB> struct ARaw<BGL_Q8G64, NB> { uint32_t w[2]; };
template <int NB> struct ARaw<BGL_QNG64, NB> {
    static constexpr int H8 = (NB >> 3) & 1, H4 = (NB >> 2) & 1, H2 = (NB >> 1) & 1, H1 = NB & 1;
    uint32_t w[2 * H8 + H4 + H2 + H1 > 0 ? 2 * H8 + H4 + H2 + H1 : 1];
};

template <int FMT> constexpr int ksteps_per_unit() { return FMT == BGL_QNG64 ? 4 : 2; }

template <int FMT, int NB>
__device__ __forceinline__ void ld_a(ARaw<FMT, NB> &a, const BglDevTensor &T, int tile, int rb, int s, int lane) {
    const int row = 16 * rb + (lane & 15), q = lane >> 4;
    constexpr int SPU = ksteps_per_unit<FMT>();
    const int u = s / SPU, j = s % SPU;
    const BGL_GLOBAL uint8_t *base = (const BGL_GLOBAL uint8_t *)T.w;
    auto chunk = [&](int c) { return base + (((size_t)tile * T.cpr + (size_t)u * T.cpu + c) * BGL_TILE + row) * 16; };
    if constexpr (FMT == BGL_Q8G64) {
        const BGL_GLOBAL uint32_t *p = (const BGL_GLOBAL uint32_t *)(chunk(2 * j + (q >> 1)) + 8 * (q & 1));
        a.w[0] = p[0]; a.w[1] = p[1];
    } else if constexpr (FMT == BGL_QNG64) {
        constexpr int H8 = ARaw<FMT, NB>::H8, H4 = ARaw<FMT, NB>::H4, H2 = ARaw<FMT, NB>::H2, H1 = ARaw<FMT, NB>::H1;
        constexpr int K4 = 8 * H8, K2 = K4 + 4 * H4, K1 = K2 + 2 * H2;
        int i = 0;
        if constexpr (H8) {
            const BGL_GLOBAL uint32_t *p = (const BGL_GLOBAL uint32_t *)(chunk(2 * j + (q >> 1)) + 8 * (q & 1));
            a.w[i++] = p[0]; a.w[i++] = p[1];
        }
        if constexpr (H4) a.w[i++] = *(const BGL_GLOBAL uint32_t *)(chunk(K4 + j) + 4 * q);
        if constexpr (H2) a.w[i++] = *(const BGL_GLOBAL uint32_t *)(chunk(K2 + (j >> 1)) + 4 * (2 * (j & 1) + (q >> 1)));
        if constexpr (H1) a.w[i++] = *(const BGL_GLOBAL uint32_t *)(chunk(K1) + 4 * j);
    } else {                                             // int4: chunk j of the unit, dword q
        a.w[0] = *(const BGL_GLOBAL uint32_t *)(chunk(j) + 4 * q);
    }
}

__device__ __forceinline__ uint32_t sub_h2(uint32_t p, _Float16 c) {
    mf_h2 v = __builtin_bit_cast(mf_h2, p);
    const mf_h2 cc = {c, c};
    v = v + cc;                                          // exact: both operands and the result are fp16 integers
    return __builtin_bit_cast(uint32_t, v);
}

// Codes of the lane's 8 elements as halves in the order {0,2,1,3,4,6,5,7}.
template <int FMT, int NB>
__device__ __forceinline__ mf_h8 dec_a(const ARaw<FMT, NB> &a, int q) {
    constexpr uint32_t MAG = 0x64006400u;                // fp16 1024.0 in both halves
    uint32_t p02, p13, p46, p57;
    _Float16 off;
    if constexpr (FMT == BGL_Q8G64) {
        const uint32_t x0 = a.w[0] ^ 0x80808080u, x1 = a.w[1] ^ 0x80808080u;   // u = code + 128
        p02 = (x0 & 0x00FF00FFu) | MAG; p13 = ((x0 >> 8) & 0x00FF00FFu) | MAG;
        p46 = (x1 & 0x00FF00FFu) | MAG; p57 = ((x1 >> 8) & 0x00FF00FFu) | MAG;
        off = (_Float16)-1152.0f;
    } else if constexpr (FMT == BGL_QNG64) {
        constexpr int H8 = ARaw<FMT, NB>::H8, H4 = ARaw<FMT, NB>::H4, H2 = ARaw<FMT, NB>::H2, H1 = ARaw<FMT, NB>::H1;
        constexpr int SH4 = 8 * H8, SH2 = SH4 + 4 * H4, SH1 = SH2 + 2 * H2;
        uint32_t u02 = 0, u13 = 0, u46 = 0, u57 = 0;
        int i = 0;
        if constexpr (H8) {
            const uint32_t x0 = a.w[i] ^ 0x80808080u, x1 = a.w[i + 1] ^ 0x80808080u;
            u02 = x0 & 0x00FF00FFu; u13 = (x0 >> 8) & 0x00FF00FFu;
            u46 = x1 & 0x00FF00FFu; u57 = (x1 >> 8) & 0x00FF00FFu;
            i += 2;
        }
        if constexpr (H4) {
            const uint32_t w = a.w[i++];
            u02 |= (w & 0x000F000Fu) << SH4; u13 |= ((w >> 8) & 0x000F000Fu) << SH4;
            u46 |= ((w >> 4) & 0x000F000Fu) << SH4; u57 |= ((w >> 12) & 0x000F000Fu) << SH4;
        }
        if constexpr (H2) {
            const uint32_t w = a.w[i++] >> (4 * (q & 1));   // crumbs 2(q%2) (elements 0..3) and +1 (4..7)
            u02 |= (w & 0x00030003u) << SH2; u13 |= ((w >> 8) & 0x00030003u) << SH2;
            u46 |= ((w >> 2) & 0x00030003u) << SH2; u57 |= ((w >> 10) & 0x00030003u) << SH2;
        }
        if constexpr (H1) {
            const uint32_t w = a.w[i++] >> (2 * q);          // bits 2q (elements 0..3) and 2q+1 (4..7)
            u02 |= (w & 0x00010001u) << SH1; u13 |= ((w >> 8) & 0x00010001u) << SH1;
            u46 |= ((w >> 1) & 0x00010001u) << SH1; u57 |= ((w >> 9) & 0x00010001u) << SH1;
        }
        p02 = u02 | MAG; p13 = u13 | MAG; p46 = u46 | MAG; p57 = u57 | MAG;
        off = (_Float16)(-(1024.0f + (float)(1 << (NB - 1))));
    } else {
        const uint32_t w = a.w[0];
        p02 = (w & 0x000F000Fu) | MAG; p13 = ((w >> 8) & 0x000F000Fu) | MAG;
        p46 = ((w >> 4) & 0x000F000Fu) | MAG; p57 = ((w >> 12) & 0x000F000Fu) | MAG;
        off = (_Float16)-1032.0f;
    }
    mf_u4 r = {sub_h2(p02, off), sub_h2(p13, off), sub_h2(p46, off), sub_h2(p57, off)};
    return __builtin_bit_cast(mf_h8, r);
}

// Raw A words per K-step and row block.  A block is 4 K-steps; two blocks of weights are in
// registers per wave (the ring), and two workgroups share a CU where the registers allow.
template <int FMT, int NB> constexpr int a_words() {
    return FMT == BGL_Q8G64 ? 2 : FMT == BGL_QNG64 ? 2 * ((NB >> 3) & 1) + ((NB >> 2) & 1) + ((NB >> 1) & 1) + (NB & 1) : 1;
}
template <int FMT, int NB, int CT> constexpr int block_ksteps() { return 4; }
// Occupancy asked of the compiler: 4 waves per SIMD (two 8-wave workgroups per CU, <= 128 VGPRs)
// where the kernel fits without spilling -- up to 32 columns of one-word (int4) weights; the
// others keep their registers.
template <int FMT, int NB, int CT> constexpr int mfma_waves_per_eu() { return MF_WPE_INT4 && CT <= 2 && a_words<FMT, NB>() == 1 ? 4 : 1; }
// bytes of scale data per row and unit in the device layout
template <int FMT> constexpr int scale_bytes() { return FMT == BGL_QNG64 ? 8 : 4; }

// ==================================================================================== GEMM kernel
template <int FMT, int NB, int CT>
__global__ __launch_bounds__(MF_WAVES * 64) __attribute__((amdgpu_waves_per_eu(mfma_waves_per_eu<FMT, NB, CT>()))) void
k_gemm_mfma(MfmaLaunch L) {
    constexpr int KC = block_ksteps<FMT, NB, CT>();
    constexpr int SPU = ksteps_per_unit<FMT>();
    constexpr int UPB = KC / SPU;                                  // units per block
    constexpr int SCW = scale_bytes<FMT>();
    // in LDS every format keeps fp32 scales; Q4G32H's fp16 pair becomes a float2 per row (as qNg64)
    constexpr int SCL = FMT == BGL_Q4G32H ? 8 : SCW;
    constexpr int BF = KC * CT * 2 * 64;                           // activation uint4 per block
    constexpr int SF = MF_TILES * UPB * 64 * SCW / 16;             // scale uint4 per block in global layout
    constexpr int SFL = MF_TILES * UPB * 64 * SCL / 16;            // ... and in LDS
    constexpr int NT = MF_WAVES * 64;
    constexpr int PER_B = BF / NT, PER_S = (SF + NT - 1) / NT;
    constexpr int SPG = FMT == BGL_Q4G32H ? 1 : 2;                 // K-steps per scale group
    __shared__ uint4 stage[2][BF + SFL];

    const BglDevTensor &T = L.T;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, q = lane >> 4;
    const int wt = wave / (4 / MF_RBW), rbase = (wave % (4 / MF_RBW)) * MF_RBW;   // tile in the group, first row block
    const int tile0 = blockIdx.x * MF_TILES, tile = tile0 + wt;
    const bool active = tile < T.ntiles;
    const int KS = T.K >> 5;
    const int s0 = blockIdx.y * L.kps, s1 = min(s0 + L.kps, KS);
    const int nblocks = (s1 - s0 + KC - 1) / KC;
    const int u0 = s0 / SPU;

    mf_f4 acc[MF_RBW][CT], cg[MF_RBW][CT];
#pragma unroll
    for (int r = 0; r < MF_RBW; r++)
#pragma unroll
        for (int c = 0; c < CT; c++) { acc[r][c] = mf_f4{0, 0, 0, 0}; cg[r][c] = mf_f4{0, 0, 0, 0}; }

    // ---- staged data of block b (activation fragments + the 4 tiles' scales) ----
    struct SR { uint4 b[PER_B], s[PER_S]; };
    // Every global load below is unconditional, from an address clamped into the tensor, and the
    // unwanted values are dropped by a select: conditional loads would keep the compiler from
    // counting outstanding loads, and it would then wait for all of them before each block.
    auto load_stage = [&](SR &R, int b) {
        const int sb = s0 + b * KC;
#pragma unroll
        for (int i = 0; i < PER_B; i++) {
            const int e = threadIdx.x + i * NT;
            const int s = sb + e / (CT * 2 * 64);
            const int sc = s < s1 ? s : s1 - 1;
            const bgl_u32x4 g = ((const BGL_GLOBAL bgl_u32x4 *)L.xf)[((size_t)sc * CT * 2 * 64) + e % (CT * 2 * 64)];
            R.b[i] = make_uint4(g.x, g.y, g.z, g.w);             // out-of-range steps are zeroed at the store
        }
#pragma unroll
        for (int i = 0; i < PER_S; i++) {
            const int e = threadIdx.x + i * NT;                    // uint4 index: [wt][ub][row*SCW/16]
            const int per_tile = UPB * 64 * SCW / 16;
            const int ec = e < SF ? e : SF - 1;
            const int st = ec / per_tile, rem = ec % per_tile;
            const int ub = rem / (64 * SCW / 16);
            const int t = tile0 + st, u = u0 + b * UPB + ub;
            const int tc = t < T.ntiles ? t : T.ntiles - 1, uc = u < T.nunits ? u : T.nunits - 1;
            const bgl_u32x4 g = ((const BGL_GLOBAL bgl_u32x4 *)T.s0)[((size_t)tc * T.nunits + uc) * (64 * SCW / 16) +
                                                                      rem % (64 * SCW / 16)];
            R.s[i] = make_uint4(g.x, g.y, g.z, g.w);             // rows past the tensor never reach y
        }
    };
    auto store_stage = [&](int buf, const SR &R, int b) {
#pragma unroll
        for (int i = 0; i < PER_B; i++) {
            const int e = threadIdx.x + i * NT;
            const bool in = s0 + b * KC + e / (CT * 2 * 64) < s1;
            stage[buf][e] = in ? R.b[i] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < PER_S; i++) {
            const int e = threadIdx.x + i * NT;
            if (e < SF) {
                if constexpr (FMT == BGL_Q4G32H) {                  // 4 rows x (fp16 lo, fp16 hi) -> 4 float2
                    const uint32_t w[4] = {R.s[i].x, R.s[i].y, R.s[i].z, R.s[i].w};
                    float f[8];
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        f[2 * v] = __half2float(__ushort_as_half((unsigned short)(w[v] & 0xffffu)));
                        f[2 * v + 1] = __half2float(__ushort_as_half((unsigned short)(w[v] >> 16)));
                    }
                    uint4 a, b;
                    memcpy(&a, f, 16);
                    memcpy(&b, f + 4, 16);
                    stage[buf][BF + 2 * e] = a;
                    stage[buf][BF + 2 * e + 1] = b;
                } else {
                    stage[buf][BF + e] = R.s[i];
                }
            }
        }
    };

    // ---- weights of block b for this wave: the register ring ----
    struct WR { ARaw<FMT, NB> a[KC][MF_RBW]; };
    const int tile_c = active ? tile : T.ntiles - 1;               // inactive waves read a real tile
    auto load_w = [&](WR &W, int b) {
#pragma unroll
        for (int j = 0; j < KC; j++) {
            const int s = s0 + b * KC + j;
            const int sc = s < s1 ? s : s1 - 1;                     // past the split: reread, unused
#pragma unroll
            for (int r = 0; r < MF_RBW; r++) ld_a<FMT, NB>(W.a[j][r], T, tile_c, rbase + r, sc, lane);
        }
    };

    auto compute = [&](const WR &W, int b) {
        const uint4 *stg = stage[b & 1];
        const float *scl = reinterpret_cast<const float *>(stg + BF);
        // K-steps past the split still run: their staged activations are zero and their weights
        // are rereads of real codes, so they add exact zeros, and the block stays one straight-line
        // region the scheduler can interleave (a per-step exit made every step its own block).
#pragma unroll
        for (int j = 0; j < KC; j++) {
            mf_h8 A[MF_RBW];
#pragma unroll
            for (int r = 0; r < MF_RBW; r++) A[r] = dec_a<FMT, NB>(W.a[j][r], q);
            const bool gstart = j % SPG == 0;                       // first K-step of a scale group
#pragma unroll
            for (int c = 0; c < CT; c++) {
                const mf_h8 Bh = __builtin_bit_cast(mf_h8, stg[((j * CT + c) * 2 + 0) * 64 + lane]);
                const mf_h8 Bl = __builtin_bit_cast(mf_h8, stg[((j * CT + c) * 2 + 1) * 64 + lane]);
#pragma unroll
                for (int r = 0; r < MF_RBW; r++) {
                    cg[r][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[r], Bh, gstart ? mf_f4{0, 0, 0, 0} : cg[r][c], 0, 0, 0);
                    cg[r][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[r], Bl, cg[r][c], 0, 0, 0);
                }
            }
            if ((j + 1) % SPG == 0) {                                // group complete: fold with its scales
                const int ub = j / SPU;
                const int g = FMT == BGL_Q4G32H ? (j & 1) : (FMT == BGL_QNG64 ? ((j % SPU) >> 1) : 0);
#pragma unroll
                for (int rb = 0; rb < MF_RBW; rb++) {
                    const int r0 = 16 * (rbase + rb) + 4 * q;
                    mf_f4 sc;
                    if constexpr (FMT == BGL_QNG64 || FMT == BGL_Q4G32H) {   // float2 per row: group g
                        const float *p = scl + ((wt * UPB + ub) * 64 + r0) * 2 + g;
                        sc = mf_f4{p[0], p[2], p[4], p[6]};
                    } else {
                        const float *p = scl + (wt * UPB + ub) * 64 + r0;
                        sc = mf_f4{p[0], p[1], p[2], p[3]};
                    }
#pragma unroll
                    for (int c = 0; c < CT; c++) {
#pragma unroll
                        for (int v = 0; v < 4; v++) acc[rb][c][v] = __fmaf_rn(cg[rb][c][v], sc[v], acc[rb][c][v]);
                    }
                }
            }
        }
    };

    // Pipeline: block b is computed while block b+2's weights and staged data (activation
    // fragments and scales) are loading and block b+1's staged data goes to LDS -- both streams
    // have a full block of compute between issue and use.  Iteration b uses weight registers w[b%3]
    // and loads w[(b+2)%3]; it stores staged set (b+1)%2 and refills set b%2.  Every load is issued
    // on every path (past the end they reread the last K-step and are never used), so the number
    // of loads in flight is the same everywhere and each wait covers only its own block.
    WR w0, w1, w2;
    SR r0, r1;
    load_stage(r0, 0);
    load_w(w0, 0);
    load_stage(r1, 1);
    load_w(w1, 1);
    store_stage(0, r0, 0);
    __syncthreads();
    auto iter = [&](WR &wc, WR &wl, SR &rs, SR &rl, int b) {
        load_stage(rl, b + 2);
        load_w(wl, b + 2);
        if (active) compute(wc, b);
        store_stage((b + 1) & 1, rs, b + 1);   // past the end it fills a buffer nobody reads again
        __syncthreads();
        return b + 1 < nblocks;
    };
    for (int b = 0; b < nblocks; b += 6) {
        if (!iter(w0, w2, r1, r0, b)) break;
        if (!iter(w1, w0, r0, r1, b + 1)) break;
        if (!iter(w2, w1, r1, r0, b + 2)) break;
        if (!iter(w0, w2, r0, r1, b + 3)) break;
        if (!iter(w1, w0, r1, r0, b + 4)) break;
        if (!iter(w2, w1, r0, r1, b + 5)) break;
    }
    if (!active) return;

    const int nsplit = gridDim.y;
#pragma unroll
    for (int rb = 0; rb < MF_RBW; rb++) {
        const int n0 = tile * BGL_TILE + 16 * (rbase + rb) + 4 * q;
#pragma unroll
        for (int c = 0; c < CT; c++) {
            const int m = 16 * c + (lane & 15);
            if (m >= L.M) continue;
            const float ci = L.colinv[m];
            float *dst = nsplit > 1 ? L.part + ((size_t)blockIdx.y * L.M + m) * T.N : L.y + (size_t)m * L.ystride;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int n = n0 + v;
                if (n < T.N) {
                    float o = acc[rb][c][v] * ci;
                    if (nsplit == 1 && L.bias) o += L.bias[n];
                    dst[n] = o;
                }
            }
        }
    }
}

// ==================================================================================== host side
bool bgl_mfma_ok(int fmt, int bits) {
    if (fmt == BGL_Q4G64 || fmt == BGL_Q4G32H || fmt == BGL_Q8G64) return true;
    return fmt == BGL_QNG64 && bits >= 2 && bits <= MF_MAXN;
}

template <int FMT, int NB>
static int launch_fmt(const MfmaLaunch &L, int CT, dim3 grid, hipStream_t st) {
    switch (CT) {
    case 1: hipLaunchKernelGGL((k_gemm_mfma<FMT, NB, 1>), grid, dim3(MF_WAVES * 64), 0, st, L); return 0;
    case 2: hipLaunchKernelGGL((k_gemm_mfma<FMT, NB, 2>), grid, dim3(MF_WAVES * 64), 0, st, L); return 0;
    case 3: hipLaunchKernelGGL((k_gemm_mfma<FMT, NB, 3>), grid, dim3(MF_WAVES * 64), 0, st, L); return 0;
    case 4: hipLaunchKernelGGL((k_gemm_mfma<FMT, NB, 4>), grid, dim3(MF_WAVES * 64), 0, st, L); return 0;
    default: return -1;
    }
}

static int launch_any(const MfmaLaunch &L, int CT, dim3 grid, hipStream_t st) {
    switch (L.T.fmt) {
    case BGL_Q4G64: return launch_fmt<BGL_Q4G64, 0>(L, CT, grid, st);
    case BGL_Q4G32H: return launch_fmt<BGL_Q4G32H, 0>(L, CT, grid, st);
    case BGL_Q8G64: return launch_fmt<BGL_Q8G64, 0>(L, CT, grid, st);
    case BGL_QNG64:
        switch (L.T.bits) {
        case 2: return launch_fmt<BGL_QNG64, 2>(L, CT, grid, st);
        case 3: return launch_fmt<BGL_QNG64, 3>(L, CT, grid, st);
        case 4: return launch_fmt<BGL_QNG64, 4>(L, CT, grid, st);
        case 5: return launch_fmt<BGL_QNG64, 5>(L, CT, grid, st);
        case 6: return launch_fmt<BGL_QNG64, 6>(L, CT, grid, st);
        case 7: return launch_fmt<BGL_QNG64, 7>(L, CT, grid, st);
        case 8: return launch_fmt<BGL_QNG64, 8>(L, CT, grid, st);
        case 9: return launch_fmt<BGL_QNG64, 9>(L, CT, grid, st);
        case 10: return launch_fmt<BGL_QNG64, 10>(L, CT, grid, st);
        default: return -1;
        }
    default: return -1;
    }
}

// y[m][n] = bias[n] + sum_k W[n][k] x[m][k] for the n tensors of a group sharing x, M >= 1 columns
// (the caller routes M >= 16 here).  Columns go in launches of up to 64.
int run_gemm_mfma(bgl_ctx *c, int n, const BglDevTensor *Ts, const float *x_dev, int M, const float *const *bias,
                  float *const *y, const int *ystride) {
    const int K = Ts[0].K;
    if (K % 64) return bgl_fail(BGL_E_ARG, "MFMA path: in=%d %% 64 != 0", K);
    for (int i = 0; i < n; i++)
        if (!bgl_mfma_ok(Ts[i].fmt, Ts[i].bits)) return bgl_fail(BGL_E_UNSUPPORTED, "MFMA path: kind %d", Ts[i].fmt);
    const int KS = K / 32;
    for (int m0 = 0; m0 < M; m0 += 16 * MF_MAXCT) {
        const int Mc = M - m0 < 16 * MF_MAXCT ? M - m0 : 16 * MF_MAXCT;
        const int CT = (Mc + 15) / 16;
        const size_t fbytes = (size_t)KS * CT * 2 * 64 * 16;
        if (dbuf_reserve(c, c->act_w, fbytes, false) || dbuf_reserve(c, c->act_s, (size_t)16 * CT * 4, false)) return BGL_E_NOMEM;
        int tok = prof_begin(c, 0);
        hipLaunchKernelGGL(k_act_frag, dim3(16 * CT, (K + MF_PREP_CHUNK - 1) / MF_PREP_CHUNK), dim3(256), 0, c->stream,
                           x_dev + (size_t)m0 * K, Mc, K, CT, (uint4 *)c->act_w.p, (float *)c->act_s.p);
        prof_end(c, tok);
        HIPCHK(hipGetLastError());
        c->prep_act = -1;                                 // the activation buffers now hold fragments
        for (int i = 0; i < n; i++) {
            const BglDevTensor &T = Ts[i];
            const int wgr = (T.ntiles + MF_TILES - 1) / MF_TILES;
            const int spu = T.fmt == BGL_QNG64 ? 4 : 2;
            int S = (c->min_blocks + wgr - 1) / wgr;     // split K until the grid has ~min_blocks workgroups
            int maxS = KS / (2 * MF_KC);                  // at least two staged blocks per split
            if (maxS > 16) maxS = 16;
            // the partials (written and read back once each) stay under half the weight bytes
            const double wbytes = (double)T.N * T.K * (T.fmt == BGL_Q8G64 ? 1.0625 : T.fmt == BGL_QNG64 ? T.bits / 8.0 + 0.0625 : 0.5625);
            const int capS = (int)(0.5 * wbytes / (8.0 * Mc * T.N));
            if (maxS > capS) maxS = capS;
            if (S > maxS) S = maxS;
            if (S < 1) S = 1;
            int kps = (KS + S - 1) / S;
            kps = (kps + spu - 1) / spu * spu;            // splits end on unit boundaries
            S = (KS + kps - 1) / kps;
            MfmaLaunch L;
            memset(&L, 0, sizeof L);
            L.T = T; L.xf = (const uint4 *)c->act_w.p; L.colinv = (const float *)c->act_s.p;
            L.bias = bias ? bias[i] : nullptr;
            const int ys = ystride ? ystride[i] : T.N;
            L.y = y[i] + (size_t)m0 * ys; L.ystride = ys; L.M = Mc; L.kps = kps;
            if (S > 1) {
                if (dbuf_reserve(c, c->part, (size_t)S * Mc * T.N * 4, false)) return BGL_E_NOMEM;
                L.part = (float *)c->part.p;
            }
            tok = prof_begin(c, 1);
            if (launch_any(L, CT, dim3(wgr, S), c->stream)) return bgl_fail(BGL_E_UNSUPPORTED, "MFMA path: format");
            prof_end(c, tok);
            HIPCHK(hipGetLastError());
            if (S > 1) {
                tok = prof_begin(c, 2);
                hipLaunchKernelGGL(k_splitk_reduce, dim3(nblk((long)Mc * T.N)), dim3(256), 0, c->stream,
                                   (const float *)c->part.p, S, Mc, T.N, L.bias, L.y, ys);
                prof_end(c, tok);
                HIPCHK(hipGetLastError());
            }
        }
    }
    return 0;
}
