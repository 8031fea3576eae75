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
// Work split.  A workgroup = 8 waves = 4 consecutive 64-row weight tiles (256 rows) over one K
// range; two waves share a tile (two 16-row blocks each).  The activation fragments and scales of
// 4 consecutive K-steps (a block) are staged through LDS, double buffered, and shared by every
// wave.  Shapes with few tiles split K over workgroups into fp32 partials that k_mfma_reduce adds
// in split order (deterministic; no atomics).  All tensors of a group (same format and K, one
// activation) run in one launch and one reduce.
//
// Memory access.  Weights, fragments and scales are read with buffer loads: the per-lane part of
// every address is fixed for the whole kernel and the per-step part is a scalar offset, so the
// loads cost no vector ALU work.  The fragment buffer is zero-padded to whole blocks and the weight
// and scale offsets are clamped into the tensor, so no load is conditional (a conditional load
// makes the compiler wait for every load in flight) and steps past K add exact zeros.
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
typedef unsigned int mf_u2 __attribute__((ext_vector_type(2)));

#define MF_TILES 4           // 64-row weight tiles per workgroup (they share the staged activations)
#define MF_RBW 2             // 16-row blocks per wave: two waves per tile
#define MF_WAVES (MF_TILES * 4 / MF_RBW)
#define MF_KC 4              // K-steps (32 elements each) per staged block
#define MF_MAXCT 4           // column tiles (16 columns each) per launch: up to 64 columns
#define MF_MAXN 10           // qNg64 widths whose codes are exact in fp16 via the 1024+u trick
#define MF_MAXS 16           // K splits per tensor
#define MF_RSRC_W3 0x00020000   // buffer resource word 3 on gfx9: 32-bit data format, raw addressing

static inline unsigned nblk(long n, int bs = 256) { return (unsigned)((n + bs - 1) / bs); }

struct MfmaTask {
    BglDevTensor T;
    const float *bias;       // [N] or null
    float *y;                // y[m][n] at y + m*ystride + n
    float *part;             // K-split partials [S][M][N] (S > 1)
    int ystride;
    int wg0;                 // first workgroup of this task in the launch
    int wgr;                 // workgroups along the rows (groups of 4 tiles)
    int kps;                 // K-steps per split, a multiple of the block size
};

struct MfmaLaunch {
    MfmaTask t[BGL_MAX_TASKS];
    int ntasks;
    int M;                   // valid columns (<= 16*CT)
    const uint4 *xf;         // activation fragments [KSP][CT][2][64] x 16 B, zero past K
    const float *colinv;     // [16*CT] column factors 2^(e-14)
    int xf_steps;            // KSP: K-steps held in xf (K/32 rounded up to whole blocks)
};

// ==================================================================================== activations
// Grid (16*CT columns, KSP*4/256 chunks of 256 8-element slots), 256 threads; columns >= M and
// slots past K are zero.  x: [M][K] rows of this launch.  Every chunk's workgroup reduces its
// column's max over all of K (the column is L2-resident), so no second pass is needed; a thread's
// own 8 values and its share of the column are loaded in one round before any is used.
#define MF_PREP_SLOTS 256
#define MF_PREP_BATCH 16
__global__ __launch_bounds__(256) void k_act_frag(const float *__restrict__ x, int M, int K, int KSP, int CT,
                                                  uint4 *__restrict__ xf, float *__restrict__ colinv) {
    __shared__ float wmax[4];
    const int m = blockIdx.x, t = threadIdx.x;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)(m < M ? m : 0) * K);   // K % 64 == 0
    const int n4 = K >> 2;
    const int g = blockIdx.y * MF_PREP_SLOTS + t;                                        // this thread's slot
    const bool own = m < M && g < (K >> 3);
    const int gc = own ? g : 0;
    const float4 a = x4[2 * gc], b = x4[2 * gc + 1];
    float mx = 0.0f;
    if (m < M) {                                                                         // uniform per workgroup
        for (int k0 = 0; k0 < n4; k0 += MF_PREP_BATCH * 256) {
            float4 v[MF_PREP_BATCH];
#pragma unroll
            for (int i = 0; i < MF_PREP_BATCH; i++) {
                const int k = k0 + t + i * 256;
                v[i] = x4[k < n4 ? k : n4 - 1];
            }
#pragma unroll
            for (int i = 0; i < MF_PREP_BATCH; i++) {
                const float mm = fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w)));
                mx = k0 + t + i * 256 < n4 ? fmaxf(mx, mm) : mx;
            }
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
    if (g >= KSP * 4) return;
    const int ct = m >> 4, ml = m & 15;
    const int s = g >> 2, q = g & 3;
    const float v8[8] = {a.x, a.z, a.y, a.w, b.x, b.z, b.y, b.w};   // element order {0,2,1,3,4,6,5,7}
    _Float16 hi[8], lo[8];
#pragma unroll
    for (int p = 0; p < 8; p++) {
        const float v = own ? v8[p] * sc : 0.0f;         // power-of-two scaling: exact
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
// quantization groups per unit: two for the fp16-pair (Q4G32H) and float2 (qNg64) scale words
template <int FMT> constexpr int groups_per_unit() { return FMT == BGL_Q4G32H || FMT == BGL_QNG64 ? 2 : 1; }
// bytes of scale data per row and unit in the device layout
template <int FMT> constexpr int scale_bytes() { return FMT == BGL_QNG64 ? 8 : 4; }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t mf_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, MF_RSRC_W3);
}

// Per-lane byte offsets of a wave's A fragments within a tile's chunk (row block rb0; row block
// rb0+r adds 256 bytes), fixed for the kernel.  ld_a adds the K-step's scalar offset.
struct AOff { uint32_t o8, o4, o2, o1; };

__device__ __forceinline__ AOff a_offsets(int rb0, int lane) {
    const uint32_t row = 16 * rb0 + (lane & 15), q = lane >> 4;
    AOff o;
    o.o8 = (q >> 1) * 1024 + row * 16 + 8 * (q & 1);     // byte codes: chunk 2j + q/2, bytes 8(q%2)..+7
    o.o4 = row * 16 + 4 * q;                             // nibble chunk: dword q
    o.o2 = row * 16 + 4 * (q >> 1);                      // crumb chunk: dword 2(j%2) + q/2
    o.o1 = row * 16;                                     // bit chunk: dword j
    return o;
}

// A words of K-step sc (already clamped into the tensor) for row block r of the wave; tchunk is
// the first chunk of the wave's tile.
template <int FMT, int NB>
__device__ __forceinline__ void ld_a(ARaw<FMT, NB> &a, __amdgpu_buffer_rsrc_t rs, const AOff &o, uint32_t tchunk,
                                     int sc, int r) {
    const uint32_t rofs = 256u * r;
    if constexpr (FMT == BGL_Q8G64) {                    // 4 chunks per 64-element unit: K-step s is chunks 2s, 2s+1
        const mf_u2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, o.o8 + rofs, (tchunk + 2u * sc) * 1024u, 0);
        a.w[0] = v[0]; a.w[1] = v[1];
    } else if constexpr (FMT == BGL_QNG64) {
        constexpr int H8 = ARaw<FMT, NB>::H8, H4 = ARaw<FMT, NB>::H4, H2 = ARaw<FMT, NB>::H2, H1 = ARaw<FMT, NB>::H1;
        constexpr int K4 = 8 * H8, K2 = K4 + 4 * H4, K1 = K2 + 2 * H2;
        const uint32_t u = (uint32_t)sc >> 2, j = (uint32_t)sc & 3, c0 = tchunk + u * NB;
        int i = 0;
        if constexpr (H8) {
            const mf_u2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, o.o8 + rofs, (c0 + 2 * j) * 1024u, 0);
            a.w[i++] = v[0]; a.w[i++] = v[1];
        }
        if constexpr (H4) a.w[i++] = __builtin_amdgcn_raw_buffer_load_b32(rs, o.o4 + rofs, (c0 + K4 + j) * 1024u, 0);
        if constexpr (H2) a.w[i++] = __builtin_amdgcn_raw_buffer_load_b32(rs, o.o2 + rofs, (c0 + K2 + (j >> 1)) * 1024u + 8 * (j & 1), 0);
        if constexpr (H1) a.w[i++] = __builtin_amdgcn_raw_buffer_load_b32(rs, o.o1 + rofs, (c0 + K1) * 1024u + 4 * j, 0);
    } else {                                             // int4: 2 chunks per unit, K-step s is chunk s
        a.w[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, o.o4 + rofs, (tchunk + (uint32_t)sc) * 1024u, 0);
    }
}

__device__ __forceinline__ uint32_t sub_h2(uint32_t p, _Float16 c) {
    mf_h2 v = __builtin_bit_cast(mf_h2, p);
    const mf_h2 cc = {c, c};
    v = v + cc;                                          // exact: both operands and the result are fp16 integers
    return __builtin_bit_cast(uint32_t, v);
}

// (a & m) | o in one v_and_or_b32.  gfx9's three-operand encoding takes no literal constant and
// reads at most one scalar register, so m comes in a scalar register and o in a vector register.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(o));
    return r;
}

// Codes of the lane's 8 elements as halves in the order {0,2,1,3,4,6,5,7}.
template <int FMT, int NB>
__device__ __forceinline__ mf_h8 dec_a(const ARaw<FMT, NB> &a, int q) {
    constexpr uint32_t MAG = 0x64006400u;                // fp16 1024.0 in both halves
    uint32_t p02, p13, p46, p57;
    _Float16 off;
    if constexpr (FMT == BGL_Q8G64) {
        const uint32_t x0 = a.w[0] ^ 0x80808080u, x1 = a.w[1] ^ 0x80808080u;   // u = code + 128
        p02 = and_or(x0, 0x00FF00FFu, MAG); p13 = and_or(x0 >> 8, 0x00FF00FFu, MAG);
        p46 = and_or(x1, 0x00FF00FFu, MAG); p57 = and_or(x1 >> 8, 0x00FF00FFu, MAG);
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
        p02 = and_or(w, 0x000F000Fu, MAG); p13 = and_or(w >> 8, 0x000F000Fu, MAG);
        p46 = and_or(w >> 4, 0x000F000Fu, MAG); p57 = and_or(w >> 12, 0x000F000Fu, MAG);
        off = (_Float16)-1032.0f;
    }
    mf_u4 r = {sub_h2(p02, off), sub_h2(p13, off), sub_h2(p46, off), sub_h2(p57, off)};
    return __builtin_bit_cast(mf_h8, r);
}

// ==================================================================================== GEMM kernel
// Task of this workgroup: the last task whose first workgroup is <= blockIdx.x (uniform).
__device__ __forceinline__ int mf_task(const MfmaLaunch &L) {
    int ti = 0;
#pragma unroll
    for (int i = 1; i < BGL_MAX_TASKS; i++)
        if (i < L.ntasks && (int)blockIdx.x >= L.t[i].wg0) ti = i;
    return ti;
}

// Raw A words per K-step and row block.
template <int FMT, int NB> constexpr int a_words() {
    return FMT == BGL_Q8G64 ? 2 : FMT == BGL_QNG64 ? 2 * ((NB >> 3) & 1) + ((NB >> 2) & 1) + ((NB >> 1) & 1) + (NB & 1) : 1;
}

template <int FMT, int NB, int CT>
__global__ __launch_bounds__(MF_WAVES * 64) void k_gemm_mfma(MfmaLaunch L) {
    constexpr int NT = MF_WAVES * 64;
    constexpr int KC = MF_KC;                                      // K-steps per staged block
    constexpr int SPU = ksteps_per_unit<FMT>();
    constexpr int UPB = KC / SPU;                                  // units per block
    constexpr int GPU = groups_per_unit<FMT>();
    constexpr int SCW = scale_bytes<FMT>();
    constexpr int SPG = SPU / GPU;                                 // K-steps per scale group
    constexpr int BF = KC * CT * 2 * 64;                           // activation uint4 per block
    constexpr int SUT = UPB * 64 * SCW / 16;                       // scale uint4 per tile and block (global layout)
    constexpr int SF = MF_TILES * SUT;
    constexpr int SFL = MF_TILES * UPB * GPU * 64 / 4;             // ... in LDS: fp32 [tile][unit][group][row]
    constexpr int PER_B = BF / NT, PER_S = (SF + NT - 1) / NT;
    static_assert(BF % NT == 0, "staged block must split evenly over the threads");
    __shared__ uint4 stage[2][BF + SFL];

    const int ti = mf_task(L);
    const MfmaTask &tk = L.t[ti];
    const BglDevTensor &T = tk.T;
    // the wave index is uniform: in a scalar register, every offset derived from it is scalar too
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, q = lane >> 4;
    const int wt = wave / (4 / MF_RBW), rbase = (wave % (4 / MF_RBW)) * MF_RBW;   // tile in the group, first row block
    const int local = (int)blockIdx.x - tk.wg0;
    const int split = local / tk.wgr, tg = local % tk.wgr;
    const int tile0 = tg * MF_TILES, tile = tile0 + wt;
    const int KS = T.K >> 5;
    const int s0 = split * tk.kps, s1 = min(s0 + tk.kps, KS);
    const int nblocks = (s1 - s0 + KC - 1) / KC;
    const int u0 = s0 / SPU;

    const __amdgpu_buffer_rsrc_t rw = mf_rsrc(T.w, (uint32_t)T.ntiles * T.cpr * 1024u);
    const __amdgpu_buffer_rsrc_t rx = mf_rsrc(L.xf, (uint32_t)L.xf_steps * CT * 2048u);
    const __amdgpu_buffer_rsrc_t rsc = mf_rsrc(T.s0, (uint32_t)T.ntiles * T.nunits * 64 * SCW);

    mf_f4 acc[MF_RBW][CT], cg[MF_RBW][CT];
#pragma unroll
    for (int r = 0; r < MF_RBW; r++)
#pragma unroll
        for (int c = 0; c < CT; c++) { acc[r][c] = mf_f4{0, 0, 0, 0}; cg[r][c] = mf_f4{0, 0, 0, 0}; }

    // ---- staged data of block b (activation fragments + the 4 tiles' scales) ----
    // Blocks past the split reread its last block (the prefetch runs two ahead); their buffers are
    // never read.  Fragment K-steps past K are zeros in xf.
    struct SR { uint4 b[PER_B], s[PER_S]; };
    const uint32_t xo = threadIdx.x * 16u;
    // scale uint4 e = threadIdx.x + i*NT: tile st = e / SUT (clamped into the tensor), offset rem
    uint32_t so[PER_S];
    int sub[PER_S];
#pragma unroll
    for (int i = 0; i < PER_S; i++) {
        const int e = threadIdx.x + i * NT, ec = e < SF ? e : SF - 1;
        const int st = ec / SUT, rem = ec % SUT;
        const int tc = min(tile0 + st, T.ntiles - 1);
        sub[i] = rem / (64 * SCW / 16);                              // unit within the block
        so[i] = ((uint32_t)tc * T.nunits) * (64 * SCW) + (uint32_t)(rem % (64 * SCW / 16)) * 16u;
    }
    auto load_stage = [&](SR &R, int b) {
        const int bc = min(b, nblocks - 1);
        const uint32_t xs = (uint32_t)(s0 + bc * KC) * CT * 2048u;
#pragma unroll
        for (int i = 0; i < PER_B; i++) {
            const mf_u4 g = __builtin_amdgcn_raw_buffer_load_b128(rx, xo + i * NT * 16u, xs, 0);
            R.b[i] = make_uint4(g[0], g[1], g[2], g[3]);
        }
#pragma unroll
        for (int i = 0; i < PER_S; i++) {
            const int uc = min(u0 + bc * UPB + sub[i], T.nunits - 1);
            const mf_u4 g = __builtin_amdgcn_raw_buffer_load_b128(rsc, so[i] + (uint32_t)uc * (64 * SCW), 0, 0);
            R.s[i] = make_uint4(g[0], g[1], g[2], g[3]);
        }
    };
    // Scales go to LDS as fp32 [tile][unit][group][64 rows], so a lane's 4 rows of one group are
    // one 16-byte read.
    auto store_stage = [&](int buf, const SR &R) {
#pragma unroll
        for (int i = 0; i < PER_B; i++) stage[buf][threadIdx.x + i * NT] = R.b[i];
        float *sl = reinterpret_cast<float *>(&stage[buf][BF]);
#pragma unroll
        for (int i = 0; i < PER_S; i++) {
            const int e = threadIdx.x + i * NT;
            if (e < SF) {
                const int tu = e / (64 * SCW / 16), rr = e % (64 * SCW / 16);   // (tile, unit) pair, uint4 within its rows
                float *d = sl + tu * GPU * 64;
                if constexpr (FMT == BGL_Q4G32H) {              // 4 rows x (fp16 group 0, fp16 group 1)
                    const uint32_t w[4] = {R.s[i].x, R.s[i].y, R.s[i].z, R.s[i].w};
                    float4 g0, g1;
                    g0.x = __half2float(__ushort_as_half((unsigned short)(w[0] & 0xffffu)));
                    g0.y = __half2float(__ushort_as_half((unsigned short)(w[1] & 0xffffu)));
                    g0.z = __half2float(__ushort_as_half((unsigned short)(w[2] & 0xffffu)));
                    g0.w = __half2float(__ushort_as_half((unsigned short)(w[3] & 0xffffu)));
                    g1.x = __half2float(__ushort_as_half((unsigned short)(w[0] >> 16)));
                    g1.y = __half2float(__ushort_as_half((unsigned short)(w[1] >> 16)));
                    g1.z = __half2float(__ushort_as_half((unsigned short)(w[2] >> 16)));
                    g1.w = __half2float(__ushort_as_half((unsigned short)(w[3] >> 16)));
                    *reinterpret_cast<float4 *>(d + 4 * rr) = g0;
                    *reinterpret_cast<float4 *>(d + 64 + 4 * rr) = g1;
                } else if constexpr (FMT == BGL_QNG64) {        // 2 rows x (group 0, group 1)
                    *reinterpret_cast<float2 *>(d + 2 * rr) = make_float2(__uint_as_float(R.s[i].x), __uint_as_float(R.s[i].z));
                    *reinterpret_cast<float2 *>(d + 64 + 2 * rr) = make_float2(__uint_as_float(R.s[i].y), __uint_as_float(R.s[i].w));
                } else {
                    reinterpret_cast<uint4 *>(d)[rr] = R.s[i];
                }
            }
        }
    };

    // ---- weights of block b for this wave: the register ring ----
    struct WR { ARaw<FMT, NB> a[KC][MF_RBW]; };
    const int tile_c = min(tile, T.ntiles - 1);                    // waves past the tensor read a real tile
    const uint32_t tchunk = (uint32_t)tile_c * T.cpr;
    const AOff ao = a_offsets(rbase, lane);
    auto load_w = [&](WR &W, int b) {
        const int bc = min(b, nblocks - 1);
#pragma unroll
        for (int j = 0; j < KC; j++) {
            const int sc = min(s0 + bc * KC + j, KS - 1);
#pragma unroll
            for (int r = 0; r < MF_RBW; r++) ld_a<FMT, NB>(W.a[j][r], rw, ao, tchunk, sc, r);
        }
    };

    auto compute = [&](const WR &W, int b) {
        const uint4 *stg = stage[b & 1];
        const float *scl = reinterpret_cast<const float *>(stg + BF);
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
                const int ub = j / SPU, g = (j % SPU) / SPG;
#pragma unroll
                for (int rb = 0; rb < MF_RBW; rb++) {
                    const mf_f4 sc = *reinterpret_cast<const mf_f4 *>(scl + ((wt * UPB + ub) * GPU + g) * 64 +
                                                                     16 * (rbase + rb) + 4 * q);
#pragma unroll
                    for (int c = 0; c < CT; c++) {
#pragma unroll
                        for (int v = 0; v < 4; v++) acc[rb][c][v] = __fmaf_rn(cg[rb][c][v], sc[v], acc[rb][c][v]);
                    }
                }
            }
        }
    };

    // Pipeline: block b is computed while block b+2's weights and staged data are loading and
    // block b+1's staged data goes to LDS, so both streams have a block of compute between issue
    // and use.  Weights use a ring of three register sets (block b in w[b%3]); staged data uses
    // two (the set of block b is free once b is in LDS).  Every load is issued on every path, so
    // each wait covers only its own block.
    // With 48-64 columns, or three or more A words per K-step, two weight sets are all that fit
    // beside the accumulators: the weights then load one block ahead.
    constexpr int WD = CT <= 2 && a_words<FMT, NB>() <= 2 ? 2 : 1;   // weight prefetch distance in blocks
    WR w0, w1, w2;
    SR r0, r1;
    load_stage(r0, 0);
    load_w(w0, 0);
    load_stage(r1, 1);
    if constexpr (WD == 2) load_w(w1, 1);
    store_stage(0, r0);
    __syncthreads();
    auto iter = [&](WR &wc, WR &wl, SR &rs, SR &rl, int b) {
        load_stage(rl, b + 2);
        load_w(wl, b + WD);
        compute(wc, b);
        store_stage((b + 1) & 1, rs);                // past the end it fills a buffer nobody reads again
        __syncthreads();
        return b + 1 < nblocks;
    };
    if constexpr (WD == 2) {
        for (int b = 0; b < nblocks; b += 6) {
            if (!iter(w0, w2, r1, r0, b)) break;
            if (!iter(w1, w0, r0, r1, b + 1)) break;
            if (!iter(w2, w1, r1, r0, b + 2)) break;
            if (!iter(w0, w2, r0, r1, b + 3)) break;
            if (!iter(w1, w0, r1, r0, b + 4)) break;
            if (!iter(w2, w1, r0, r1, b + 5)) break;
        }
    } else {
        for (int b = 0; b < nblocks; b += 2) {
            if (!iter(w0, w1, r1, r0, b)) break;
            if (!iter(w1, w0, r0, r1, b + 1)) break;
        }
    }

    if (tile >= T.ntiles) return;
    const int S = (KS + tk.kps - 1) / tk.kps;
#pragma unroll
    for (int rb = 0; rb < MF_RBW; rb++) {
        const int n0 = tile * BGL_TILE + 16 * (rbase + rb) + 4 * q;
#pragma unroll
        for (int c = 0; c < CT; c++) {
            const int m = 16 * c + (lane & 15);
            if (m >= L.M) continue;
            const float ci = L.colinv[m];
            float *dst = S > 1 ? tk.part + ((size_t)split * L.M + m) * T.N : tk.y + (size_t)m * tk.ystride;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int n = n0 + v;
                if (n < T.N) {
                    float o = acc[rb][c][v] * ci;
                    if (S == 1 && tk.bias) o += tk.bias[n];
                    dst[n] = o;
                }
            }
        }
    }
}

// ==================================================================================== K-split reduce
// y[m][n] = bias[n] + sum_s part[s][m][n], s in order, for every task of a launch with S > 1.  A
// thread owns 4 consecutive n of one m and loads all S partials before adding them.
struct MfmaReduceTask {
    const float *part;
    const float *bias;
    float *y;
    int N, S, ystride, q0;   // q0: first quad of this task in the grid
};
struct MfmaReduce {
    MfmaReduceTask t[BGL_MAX_TASKS];
    int ntasks, M, nquads;
};

__global__ __launch_bounds__(256) void k_mfma_reduce(MfmaReduce R) {
    const int qd = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (qd >= R.nquads) return;
    int ti = 0;
#pragma unroll
    for (int i = 1; i < BGL_MAX_TASKS; i++)
        if (i < R.ntasks && qd >= R.t[i].q0) ti = i;
    const MfmaReduceTask &t = R.t[ti];
    const int nq = (t.N + 3) >> 2, lq = qd - t.q0;
    const int m = lq / nq, n = 4 * (lq % nq);
    const size_t plane = (size_t)R.M * t.N;
    const float *p = t.part + (size_t)m * t.N + n;
    float v[MF_MAXS][4];
    if ((t.N & 3) == 0) {
#pragma unroll
        for (int s = 0; s < MF_MAXS; s++)
            if (s < t.S) {
                const float4 f = *reinterpret_cast<const float4 *>(p + s * plane);
                v[s][0] = f.x; v[s][1] = f.y; v[s][2] = f.z; v[s][3] = f.w;
            }
    } else {
#pragma unroll
        for (int s = 0; s < MF_MAXS; s++)
            if (s < t.S)
#pragma unroll
                for (int e = 0; e < 4; e++) v[s][e] = n + e < t.N ? p[s * plane + e] : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
        if (n + e >= t.N) break;
        float a = v[0][e];
#pragma unroll
        for (int s = 1; s < MF_MAXS; s++)
            if (s < t.S) a += v[s][e];
        t.y[(size_t)m * t.ystride + n + e] = (t.bias ? t.bias[n + e] : 0.0f) + a;
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

static int launch_any(const MfmaLaunch &L, int fmt, int bits, int CT, dim3 grid, hipStream_t st) {
    switch (fmt) {
    case BGL_Q4G64: return launch_fmt<BGL_Q4G64, 0>(L, CT, grid, st);
    case BGL_Q4G32H: return launch_fmt<BGL_Q4G32H, 0>(L, CT, grid, st);
    case BGL_Q8G64: return launch_fmt<BGL_Q8G64, 0>(L, CT, grid, st);
    case BGL_QNG64:
        switch (bits) {
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

static double mf_weight_bytes(const BglDevTensor &T) {
    const double per = T.fmt == BGL_Q8G64 ? 1.0625 : T.fmt == BGL_QNG64 ? T.bits / 8.0 + 0.0625 : 0.5625;
    return per * T.N * T.K;
}

// y[m][n] = bias[n] + sum_k W[n][k] x[m][k] for the n tensors of a group sharing x (same format,
// width and K), M >= 1 columns (the caller routes M >= 16 here).  Columns go in launches of up to
// 64: one fragment prep, one GEMM over every tensor, and one reduce when any tensor splits K.
int run_gemm_mfma(bgl_ctx *c, int n, const BglDevTensor *Ts, const float *x_dev, int M, const float *const *bias,
                  float *const *y, const int *ystride) {
    const int K = Ts[0].K;
    if (K % 64) return bgl_fail(BGL_E_ARG, "MFMA path: in=%d %% 64 != 0", K);
    if (n < 1 || n > BGL_MAX_TASKS) return bgl_fail(BGL_E_ARG, "MFMA path: %d tensors in a group (1..%d)", n, BGL_MAX_TASKS);
    for (int i = 0; i < n; i++) {
        if (!bgl_mfma_ok(Ts[i].fmt, Ts[i].bits)) return bgl_fail(BGL_E_UNSUPPORTED, "MFMA path: kind %d", Ts[i].fmt);
        if (Ts[i].fmt != Ts[0].fmt || Ts[i].bits != Ts[0].bits || Ts[i].K != K)
            return bgl_fail(BGL_E_ARG, "MFMA path: a group shares kind, bits and in");
        const double wb = (double)Ts[i].ntiles * Ts[i].cpr * 1024.0;
        if (wb >= 2147483648.0) return bgl_fail(BGL_E_UNSUPPORTED, "MFMA path: tensor %d holds >= 2 GiB (32-bit buffer offsets)", i);
    }
    const int KS = K / 32;
    for (int m0 = 0; m0 < M; m0 += 16 * MF_MAXCT) {
        const int Mc = M - m0 < 16 * MF_MAXCT ? M - m0 : 16 * MF_MAXCT;
        const int CT = (Mc + 15) / 16;
        const int KC = MF_KC;
        const int KSP = (KS + KC - 1) / KC * KC;
        const size_t fbytes = (size_t)KSP * CT * 2 * 64 * 16;
        if (dbuf_reserve(c, c->act_w, fbytes, false) || dbuf_reserve(c, c->act_s, (size_t)16 * CT * 4, false)) return BGL_E_NOMEM;
        int tok = prof_begin(c, 0);
        hipLaunchKernelGGL(k_act_frag, dim3(16 * CT, (KSP * 4 + MF_PREP_SLOTS - 1) / MF_PREP_SLOTS), dim3(256), 0, c->stream,
                           x_dev + (size_t)m0 * K, Mc, K, KSP, CT, (uint4 *)c->act_w.p, (float *)c->act_s.p);
        prof_end(c, tok);
        HIPCHK(hipGetLastError());
        c->prep_act = -1;                                 // the activation buffers now hold fragments

        MfmaLaunch L;
        memset(&L, 0, sizeof L);
        L.ntasks = n; L.M = Mc; L.xf = (const uint4 *)c->act_w.p; L.colinv = (const float *)c->act_s.p; L.xf_steps = KSP;
        MfmaReduce R;
        memset(&R, 0, sizeof R);
        R.M = Mc;
        int wgs = 0;
        size_t poff[BGL_MAX_TASKS], pfl = 0;              // partial offsets (floats) in the shared buffer
        int S_[BGL_MAX_TASKS];
        for (int i = 0; i < n; i++) {
            const BglDevTensor &T = Ts[i];
            const int wgr = (T.ntiles + MF_TILES - 1) / MF_TILES;
            int S = (c->min_blocks + wgr - 1) / wgr;     // split K until the grid has ~min_blocks workgroups
            int maxS = KS / (2 * KC);                     // at least two staged blocks per split
            if (maxS > MF_MAXS) maxS = MF_MAXS;
            // the partials (written and read back once each) stay under half the weight bytes
            const int capS = (int)(0.5 * mf_weight_bytes(T) / (8.0 * Mc * T.N));
            if (maxS > capS) maxS = capS;
            if (S > maxS) S = maxS;
            if (S < 1) S = 1;
            int kps = (KS + S - 1) / S;
            kps = (kps + KC - 1) / KC * KC;               // splits end on block boundaries
            S = (KS + kps - 1) / kps;
            S_[i] = S;
            MfmaTask &t = L.t[i];
            t.T = T; t.bias = bias ? bias[i] : nullptr;
            t.ystride = ystride ? ystride[i] : T.N;
            t.y = y[i] + (size_t)m0 * t.ystride;
            t.wg0 = wgs; t.wgr = wgr; t.kps = kps;
            wgs += wgr * S;
            poff[i] = pfl;
            if (S > 1) pfl += (size_t)S * Mc * T.N;
        }
        if (pfl) {
            if (dbuf_reserve(c, c->part, pfl * 4, false)) return BGL_E_NOMEM;
            int nq = 0;
            for (int i = 0; i < n; i++) {
                if (S_[i] == 1) continue;
                MfmaTask &t = L.t[i];
                t.part = (float *)c->part.p + poff[i];
                MfmaReduceTask &rt = R.t[R.ntasks++];
                rt.part = t.part; rt.bias = t.bias; rt.y = t.y; rt.N = t.T.N; rt.S = S_[i]; rt.ystride = t.ystride;
                rt.q0 = nq;
                nq += Mc * ((t.T.N + 3) / 4);
            }
            R.nquads = nq;
        }
        tok = prof_begin(c, 1);
        if (launch_any(L, Ts[0].fmt, Ts[0].bits, CT, dim3(wgs), c->stream)) return bgl_fail(BGL_E_UNSUPPORTED, "MFMA path: format");
        prof_end(c, tok);
        HIPCHK(hipGetLastError());
        if (R.ntasks) {
            tok = prof_begin(c, 2);
            hipLaunchKernelGGL(k_mfma_reduce, dim3(nblk(R.nquads)), dim3(256), 0, c->stream, R);
            prof_end(c, tok);
            HIPCHK(hipGetLastError());
        }
    }
    return 0;
}
