// bgl_mfma.hip -- batched GEMM for M >= 16 activation rows on the gfx950 fp16 matrix cores
// (the M-column case of gemm_qXg64_mt / qng64_matmul_f32, q4gemv.h:761-769, qng64_dense.c:70-79).
//
// Numerics.  Weight codes are exact in fp16 (int4 and int8 codes, qNg64 codes for n <= 10), so
// the decode is exact.  Each activation column is scaled by a power of two so its largest
// magnitude lies in [2^13, 2^14), then split as hi = fp16(x') and lo = fp16(x' - hi), both rounded
// toward zero (x' - hi is exact in fp32): hi + lo holds x' to about 2^-21 of the column maximum.  v_mfma_f32_16x16x32_f16 multiplies exactly and
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
// Work split.  A workgroup owns 4 consecutive 64-row weight tiles (256 rows) over one K range (a
// split) and has KW K-slices of 8 waves; in a slice two waves share a tile (two 16-row blocks
// each).  The split's activation fragments and the 4 tiles' scales are staged in LDS once (up to
// 152 KB, which bounds the split's length), then each wave streams its own weights with no further
// barrier: a register ring keeps the next K-steps' loads in flight.  Splits are sized so the grid
// fills the chip; k_mfma_reduce adds their fp32 partials in split order (deterministic; no
// atomics).  All tensors of a group (same format and K, one activation) run in one launch and one
// reduce.  (A reduce inside the GEMM by the last workgroup of each row group -- an agent-scope
// ticket -- measured slower: the cache write-back and the serial tail cost more than the launch.)
//
// Memory access.  Weights are read a whole 16-byte chunk row per lane (buffer_load_dwordx4: each
// quarter-wave reads 256 contiguous bytes) and the operand layout above -- four lanes per row -- is
// rebuilt with v_permlane16/32_swap; the per-lane part of every address is fixed for the kernel and
// the per-step part is a scalar offset, so the loads cost no vector ALU work.  Offsets are clamped
// into the tensors, so no load is conditional (a conditional load makes the compiler wait for
// every load in flight), and steps past K meet zero fragments.
//
// Schedule.  The fold is software-pipelined: a group's MFMA sums are folded while the next group's
// MFMAs run, so the vector ALUs and the matrix cores overlap.
//
// Output.  The sums leave through LDS (the stage is free by then): stored straight from the MFMA
// layout, each store instruction would write 4 bytes to each of 16 output rows, and the partials
// of a 14336 x 4096 tensor at M = 32 took 3.8 us to write that way; staged, every lane writes 16
// consecutive bytes and each wave 1 KB runs (2 us faster per such launch).
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
#define MF_KSTEP_PAD 16      // split length granularity in K-steps (every ring depth divides it)
#define MF_MAXCT 4           // column tiles (16 columns each) per launch: up to 64 columns
#define MF_MAXN 10           // qNg64 widths whose codes are exact in fp16 via the 1024+u trick
#define MF_RSRC_W3 0x00020000   // buffer resource word 3 on gfx9: 32-bit data format, raw addressing

struct MfmaTask {
    BglDevTensor T;
    const float *bias;       // [N] or null
    float *y;                // y[m][n] at y + m*ystride + n
    float *part;             // K-split partials [S][M][N] (S > 1)
    int ystride;
    int wg0;                 // first workgroup of this task in the launch
    int wgr;                 // workgroups along the rows (groups of 4 tiles)
    int kps;                 // K-steps per split, a multiple of MF_KSTEP_PAD
};

struct MfmaLaunch {
    MfmaTask t[BGL_MAX_TASKS];
    int ntasks;
    int M;                   // valid columns (<= 16*CT)
    const float *x;          // activations x[m][k], M rows of K floats
};

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

// Code planes of a format: byte codes (q8g64; qNg64 with n >= 8), nibbles (int4; qNg64 bit 2 of
// n), crumbs and single bits (qNg64).
template <int FMT, int NB> struct Planes {
    static constexpr int P8 = FMT == BGL_Q8G64 ? 1 : FMT == BGL_QNG64 ? (NB >> 3) & 1 : 0;
    static constexpr int P4 = FMT == BGL_Q4G64 || FMT == BGL_Q4G32H ? 1 : FMT == BGL_QNG64 ? (NB >> 2) & 1 : 0;
    static constexpr int P2 = FMT == BGL_QNG64 ? (NB >> 1) & 1 : 0;
    static constexpr int P1 = FMT == BGL_QNG64 ? NB & 1 : 0;
    static constexpr int WORDS = 8 * P8 + 4 * P4 + 4 * P2 + 4 * P1;   // per lane and K-step pair
};

// Raw words of one K-step pair (s, s+1) for a wave's two 16-row blocks, as loaded.
//  - byte codes and nibbles are read a whole 16-byte chunk row per lane (one buffer_load_dwordx4
//    covers 32 rows of two chunks: lanes 32..63 take the second), so each quarter-wave reads 256
//    contiguous bytes; the MFMA operand layout (4 lanes per row) is rebuilt with lane swaps;
//  - crumbs and bits (2/n and 1/n of a qNg64 tensor's bytes) are read as the operand's own dword.
template <int FMT, int NB> struct PRaw {
    using P = Planes<FMT, NB>;
    uint32_t w8[P::P8 ? 8 : 1];      // byte codes: K-step j of the pair in words 4j..4j+3
    uint32_t w4[P::P4 ? 4 : 1];      // nibbles: lanes < 32 K-step s, lanes >= 32 K-step s+1
    uint32_t w2[P::P2 ? 4 : 1];      // crumb operand word of [j][rb]
    uint32_t w1[P::P1 ? 4 : 1];      // bit operand word of [j][rb]
};

// Per-lane byte offsets within a tile's chunk, fixed for the kernel: the chunk-row reads (rows
// 16*rb0 + lane%32 of chunk lane/32) and the operand-dword reads of row block rb0 (rb0+1 adds
// 256 bytes).
struct AOff { uint32_t op, o2, o1; };

__device__ __forceinline__ AOff a_offsets(int rb0, int lane) {
    AOff o;
    o.op = (uint32_t)(lane >> 5) * 1024u + (uint32_t)(16 * rb0 + (lane & 31)) * 16u;
    const uint32_t row = 16 * rb0 + (lane & 15), q = lane >> 4;
    o.o2 = row * 16 + 4 * (q >> 1);                      // crumb chunk: dword 2(j%2) + q/2
    o.o1 = row * 16;                                     // bit chunk: dword j
    return o;
}

// Loads K-steps s, s+1 (s even, already clamped into the tensor) of the wave's rows; tchunk is the
// first chunk of the wave's tile.
template <int FMT, int NB>
__device__ __forceinline__ void ld_pair(PRaw<FMT, NB> &p, __amdgpu_buffer_rsrc_t rs, const AOff &o, uint32_t tchunk, int s) {
    using P = Planes<FMT, NB>;
    // both are wave-uniform; said so explicitly, so every offset below is a scalar operand (a value
    // the compiler cannot prove uniform would wrap each load in a loop over the lanes' values)
    tchunk = __builtin_amdgcn_readfirstlane(tchunk);
    s = __builtin_amdgcn_readfirstlane(s);
    if constexpr (FMT == BGL_Q8G64) {                    // K-step s is chunks 2s, 2s+1
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const mf_u4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, o.op, (tchunk + 2u * (s + j)) * 1024u, 0);
            p.w8[4 * j] = v[0]; p.w8[4 * j + 1] = v[1]; p.w8[4 * j + 2] = v[2]; p.w8[4 * j + 3] = v[3];
        }
    } else if constexpr (FMT == BGL_QNG64) {
        constexpr int K4 = 8 * P::P8, K2 = K4 + 4 * P::P4, K1 = K2 + 2 * P::P2;
        const uint32_t u = (uint32_t)s >> 2, j0 = (uint32_t)s & 3, c0 = tchunk + u * NB;
        if constexpr (P::P8) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const mf_u4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, o.op, (c0 + 2 * (j0 + j)) * 1024u, 0);
                p.w8[4 * j] = v[0]; p.w8[4 * j + 1] = v[1]; p.w8[4 * j + 2] = v[2]; p.w8[4 * j + 3] = v[3];
            }
        }
        if constexpr (P::P4) {
            const mf_u4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, o.op, (c0 + K4 + j0) * 1024u, 0);
            p.w4[0] = v[0]; p.w4[1] = v[1]; p.w4[2] = v[2]; p.w4[3] = v[3];
        }
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const uint32_t jj = j0 + j;
                if constexpr (P::P2)
                    p.w2[2 * j + r] = __builtin_amdgcn_raw_buffer_load_b32(rs, o.o2 + 256u * r, (c0 + K2 + (jj >> 1)) * 1024u + 8 * (jj & 1), 0);
                if constexpr (P::P1)
                    p.w1[2 * j + r] = __builtin_amdgcn_raw_buffer_load_b32(rs, o.o1 + 256u * r, (c0 + K1) * 1024u + 4 * jj, 0);
            }
    } else {                                             // int4: K-step s is chunk s
        const mf_u4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, o.op, (tchunk + (uint32_t)s) * 1024u, 0);
        p.w4[0] = v[0]; p.w4[1] = v[1]; p.w4[2] = v[2]; p.w4[3] = v[3];
    }
}

// Operand words of both K-steps and row blocks from a loaded pair.  Nibble chunks: a 4x4 transpose
// of (quarter-wave, word) -- quarter-wave 2j+rb holds rows 16rb..+15 of K-step j -- puts word q of
// row 16rb + r into lane (r, q), register 2j+rb.  Byte chunks: quarter-wave 2c+rb holds chunk c of
// rows 16rb..+15; swapping odd with even quarter-waves puts bytes 8q..8q+7 of the row (chunk q/2,
// words 2(q%2), +1) into lane (r, q), registers (2rb, 2rb+1).
template <int FMT, int NB>
__device__ __forceinline__ void exch(const PRaw<FMT, NB> &p, ARaw<FMT, NB> (&a)[2][MF_RBW]) {
    using P = Planes<FMT, NB>;
    int i = 0;
    if constexpr (P::P8) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const auto e = __builtin_amdgcn_permlane16_swap(p.w8[4 * j], p.w8[4 * j + 2], false, false);
            const auto f = __builtin_amdgcn_permlane16_swap(p.w8[4 * j + 1], p.w8[4 * j + 3], false, false);
            a[j][0].w[i] = e[0]; a[j][0].w[i + 1] = f[0];
            a[j][1].w[i] = e[1]; a[j][1].w[i + 1] = f[1];
        }
        i += 2;
    }
    if constexpr (P::P4) {
        const auto x = __builtin_amdgcn_permlane32_swap(p.w4[0], p.w4[2], false, false);
        const auto y = __builtin_amdgcn_permlane32_swap(p.w4[1], p.w4[3], false, false);
        const auto c = __builtin_amdgcn_permlane16_swap(x[0], y[0], false, false);
        const auto d = __builtin_amdgcn_permlane16_swap(x[1], y[1], false, false);
        a[0][0].w[i] = c[0]; a[0][1].w[i] = c[1]; a[1][0].w[i] = d[0]; a[1][1].w[i] = d[1];
        i += 1;
    }
    if constexpr (P::P2) {
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 2; r++) a[j][r].w[i] = p.w2[2 * j + r];
        i += 1;
    }
    if constexpr (P::P1) {
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 2; r++) a[j][r].w[i] = p.w1[2 * j + r];
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
// K-steps of weights a wave keeps in flight: a ring of depth/2 K-step pairs, Planes::WORDS
// registers each.
template <int FMT, int NB> constexpr int ring_depth() { return Planes<FMT, NB>::WORDS <= 4 ? 16 : Planes<FMT, NB>::WORDS <= 8 ? 8 : 4; }
// LDS bytes per staged K-step: activation fragments (CT x hi/lo x 1 KB, + 16 B of row padding) +
// the 4 tiles' scale words in the device layout (512 B for every format).
constexpr int mf_step_lds(int CT) { return CT * 2048 + 16 + 512; }
// K-steps one workgroup stages (its split's whole K range): as many as fit 152 KB, a multiple of
// 16 (every ring depth divides it).
constexpr int mf_kps_max(int CT) { return (155648 / mf_step_lds(CT)) / 16 * 16; }

// Sum of code * scale * x over the non-finite x[k], k in [k0, k1), for weight row n (the rare path
// of a column that holds NaN or +-Inf).
template <int FMT, int NB>
__device__ __forceinline__ float mf_nonfinite(const BglDevTensor &T, int n, const float *x, int k0, int k1) {
    float acc = 0.0f;
#pragma unroll 1
    for (int k = k0; k < k1; k++) {
        const float v = x[k];
        if (!isfinite(v)) acc += w_at_t<FMT, NB>(T, n, k) * v;
    }
    return acc;
}

template <int FMT, int NB, int CT, int KW>
__global__ __launch_bounds__(MF_WAVES * KW * 64) void k_gemm_mfma(MfmaLaunch L) {
    constexpr int NT = MF_WAVES * KW * 64;
    constexpr int KPM = mf_kps_max(CT);                             // staged K-steps (max)
    constexpr int SPU = ksteps_per_unit<FMT>();
    constexpr int GPU = groups_per_unit<FMT>();
    constexpr int SCW = scale_bytes<FMT>();
    constexpr int SPG = SPU / GPU;                                 // K-steps per scale group
    constexpr int BST = CT * 2 * 64;                               // activation uint4 per K-step
    constexpr int XS = BST + 1;                                    // their row stride in the stage
    constexpr int UMAX = KPM / SPU;                                // staged units (max)
    constexpr int SUT = 64 * SCW / 16;                             // scale uint4 per tile and unit
    // ring depth: halved with two slices (each wave runs half the split, and 16 waves share the
    // registers); at least 4 so that a unit's groups keep their parity pattern
    constexpr int D = KW == 1 || ring_depth<FMT, NB>() == 4 ? ring_depth<FMT, NB>() : ring_depth<FMT, NB>() / 2;
    static_assert(KPM % D == 0 && KPM % SPU == 0 && D % SPU == 0, "staged range must hold whole rings and units");
    __shared__ uint4 xs[KPM * XS];                                 // [step][CT][hi/lo][64 lanes], rows XS apart
    __shared__ uint4 ss[MF_TILES * UMAX * SUT];                    // [tile][unit][64 rows] scale words

    const int ti = mf_task(L);
    const MfmaTask &tk = L.t[ti];
    const BglDevTensor &T = tk.T;
    // the wave index is uniform: in a scalar register, every offset derived from it is scalar too
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, q = lane >> 4;
    const int kw = wave / MF_WAVES, w8 = wave % MF_WAVES;          // K-slice, wave within the slice
    const int wt = w8 / (4 / MF_RBW), rbase = (w8 % (4 / MF_RBW)) * MF_RBW;   // tile in the group, first row block
    const int local = (int)blockIdx.x - tk.wg0;
    const int split = local / tk.wgr, tg = local % tk.wgr;
    const int tile0 = tg * MF_TILES, tile = tile0 + wt;
    const int KS = T.K >> 5;
    const int s0 = split * tk.kps, ns = min(tk.kps, KS - s0);      // this split: K-steps [s0, s0 + ns)
    const int nrings = (ns + D - 1) / D;                           // whole rings (steps past ns are zeros)
    const int nsr = nrings * D;
    const int u0 = s0 / SPU, nu = nsr / SPU;
    // slice kw runs rings [r0, r1) of the split
    const int rsplit = (nrings + KW - 1) / KW;
    const int ls0 = min(kw * rsplit, nrings) * D, ls1 = min((kw + 1) * rsplit, nrings) * D;

    const __amdgpu_buffer_rsrc_t rw = mf_rsrc(T.w, (uint32_t)T.ntiles * T.cpr * 1024u);
    const __amdgpu_buffer_rsrc_t rx = mf_rsrc(L.x, (uint32_t)L.M * (uint32_t)T.K * 4u);
    const __amdgpu_buffer_rsrc_t rsc = mf_rsrc(T.s0, (uint32_t)T.ntiles * T.nunits * 64 * SCW);

    // ---- activations of the split: each wave loads 8-element slots of its columns ----
    // Column m belongs to wave m % NW; lane l takes slots l, l+64, ... (slot g = K elements
    // 8g..8g+7 of the split).  Loads are unconditional (clamped) and issued before the weights, so
    // the conversion below waits for them alone.
    constexpr int NW = MF_WAVES * KW;                              // waves
    constexpr int CPW = (16 * CT + NW - 1) / NW;                   // columns per wave
    constexpr int SPL = KPM / 16;                                  // slots per lane (4 per K-step)
    float4 xv[CPW][SPL][2];
#pragma unroll
    for (int ci = 0; ci < CPW; ci++)
#pragma unroll
        for (int j = 0; j < SPL; j++) {
            const int m = ci * NW + wave, g = lane + 64 * j;
            const bool ok = m < L.M && g < 4 * ns;
            const uint32_t off = ((uint32_t)(ok ? m : 0) * (uint32_t)T.K + (uint32_t)s0 * 32u + 8u * (uint32_t)(ok ? g : 0)) * 4u;
            const mf_u4 a = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
            const mf_u4 b = __builtin_amdgcn_raw_buffer_load_b128(rx, off + 16u, 0, 0);
            xv[ci][j][0] = make_float4(__uint_as_float(a[0]), __uint_as_float(a[1]), __uint_as_float(a[2]), __uint_as_float(a[3]));
            xv[ci][j][1] = make_float4(__uint_as_float(b[0]), __uint_as_float(b[1]), __uint_as_float(b[2]), __uint_as_float(b[3]));
        }

    // ---- the 4 tiles' scales of the split: loaded now (a fixed count per thread, clamped), put
    // into LDS after the conversion below, so that nothing waits for them before the weights are
    // requested ----
    // (up to 32 columns, where that is one per thread; other shapes stage them here, before the
    // weights, as holding them through the conversion made the compiler spill in their main loops)
    constexpr int SLT = (MF_TILES * UMAX * SUT + NT - 1) / NT;     // scale uint4 per thread (max)
    constexpr bool EARLY = SLT == 1 && CT <= 2;
    const int nsu = nu * SUT;                                      // scale uint4 per tile in this split
    auto scale_ld = [&](int e) -> mf_u4 {
        e = min(e, MF_TILES * nsu - 1);                            // clamped: every load is real
        const int st = e / nsu, rem = e % nsu, uu = rem / SUT;
        const int tc = min(tile0 + st, T.ntiles - 1), uc = min(u0 + uu, T.nunits - 1);
        return __builtin_amdgcn_raw_buffer_load_b128(rsc, ((uint32_t)tc * T.nunits + uc) * (64 * SCW) + (uint32_t)(rem % SUT) * 16u, 0, 0);
    };
    auto scale_st = [&](int e, const mf_u4 &g) {
        const int st = e / nsu, rem = e % nsu, uu = rem / SUT;
        ss[(st * UMAX + uu) * SUT + rem % SUT] = uu * SPU < ns ? make_uint4(g[0], g[1], g[2], g[3]) : make_uint4(0, 0, 0, 0);
    };
    mf_u4 sreg;
    if constexpr (EARLY) sreg = scale_ld((int)threadIdx.x);
    else
        for (int e = threadIdx.x; e < MF_TILES * nsu; e += NT) scale_st(e, scale_ld(e));

    // ---- the weight ring: local K-step s lives in slot (s - ls0) % D until it is computed ----
    const int tile_c = min(tile, T.ntiles - 1);                    // waves past the tensor read a real tile
    const uint32_t tchunk = (uint32_t)tile_c * T.cpr;
    const AOff ao = a_offsets(rbase, lane);
    PRaw<FMT, NB> ring[D / 2];
    auto load_w = [&](PRaw<FMT, NB> &slot, int s) {             // local K-steps s, s+1 (s even)
        const int sc = min(s0 + s, KS - 2);                        // past the split: reread, multiplied by zeros
        ld_pair<FMT, NB>(slot, rw, ao, tchunk, sc);
    };
    // the activation and scale loads go out first: the conversion below waits for them by the
    // in-order load counter, which would also wait for any weight load issued before them
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 0; d < D / 2; d++) load_w(ring[d], ls0 + 2 * d);

    // ---- activation fragments: each column is scaled by a power of two so its largest magnitude
    // over the split lies in [2^13, 2^14), then split into hi = fp16(x') and lo = fp16(x' - hi) in
    // the MFMA operand order; the split's column factor 2^(e-14) is applied to its partial sums ----
    // Non-finite values (NaN, +-Inf) enter the fragments as 0 and flag the column; the store adds
    // their products code * scale * x one element at a time (IEEE propagation, as the reference's
    // fp32-product sums).
    __shared__ int cex[16 * MF_MAXCT];
    __shared__ int cnf[16 * MF_MAXCT];
#pragma unroll
    for (int ci = 0; ci < CPW; ci++) {
        const int m = ci * NW + wave;
        if (m >= 16 * CT) break;                                   // uniform
        // the column's largest |x| bits over the split; Inf / NaN bits exceed every finite value's, so
        // only then (rare) are they zeroed and the maximum taken again
        uint32_t mb = 0u;
#pragma unroll
        for (int j = 0; j < SPL; j++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const float4 v = xv[ci][j][h];
                const uint32_t t = max(max(__float_as_uint(v.x) & 0x7fffffffu, __float_as_uint(v.y) & 0x7fffffffu),
                                       max(__float_as_uint(v.z) & 0x7fffffffu, __float_as_uint(v.w) & 0x7fffffffu));
                mb = m < L.M && lane + 64 * j < 4 * ns ? max(mb, t) : mb;
            }
        mb = wave_max_u32(mb);
        if (lane == 0) cnf[m] = 0;
        if (mb >= 0x7f800000u) {                                   // uniform: Inf or NaN in this column's split
            mb = 0u;
#pragma unroll
            for (int j = 0; j < SPL; j++)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    float4 &v = xv[ci][j][h];
                    const bool in = m < L.M && lane + 64 * j < 4 * ns;
                    auto screen = [&](float &e) {
                        const uint32_t ab = __float_as_uint(e) & 0x7fffffffu;
                        const bool bad = ab >= 0x7f800000u;
                        e = bad ? 0.0f : e;
                        mb = (!bad && in && ab > mb) ? ab : mb;
                    };
                    screen(v.x); screen(v.y); screen(v.z); screen(v.w);
                }
            mb = wave_max_u32(mb);
            if (lane == 0) cnf[m] = 1;
        }
        const float mx = __uint_as_float(mb);
        int e = 0;
        if (mx > 0.0f) frexpf(mx, &e);                             // mx in [2^(e-1), 2^e)
        // x' = x * 2^(14-e), applied to each value (the factor alone leaves fp32's range for
        // e < -113, columns whose largest |x| is below 2^-114); the sums are unscaled by 2^(e-14)
        const int sh = mx > 0.0f ? 14 - e : 0;
        if (lane == 0) cex[m] = -sh;
        const int ct = m >> 4, ml = m & 15;
#pragma unroll
        for (int j = 0; j < SPL; j++) {
            const int g = lane + 64 * j;
            if (g >= 4 * nsr) break;
            const bool ok = m < L.M && g < 4 * ns;
            const float4 a = xv[ci][j][0], b = xv[ci][j][1];
            const float v8[8] = {a.x, a.z, a.y, a.w, b.x, b.z, b.y, b.w};   // element order {0,2,1,3,4,6,5,7}
            // hi = fp16(x') rounded toward zero, two at a time; x' - hi is exact in fp32 (hi is x'
            // cut to 11 bits); lo = fp16 of that, toward zero
            uint32_t H[4], Lo[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float v0 = ldexpf(v8[2 * k], sh), v1 = ldexpf(v8[2 * k + 1], sh);   // power-of-two scaling: exact
                const mf_h2 hh = __builtin_bit_cast(mf_h2, __builtin_amdgcn_cvt_pkrtz(v0, v1));
                const float r0 = v0 - (float)hh[0], r1 = v1 - (float)hh[1];
                const uint32_t hw = __builtin_bit_cast(uint32_t, hh);
                const uint32_t lw = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(r0, r1));
                H[k] = ok ? hw : 0u;                               // K-steps past the split: zero fragments
                Lo[k] = ok ? lw : 0u;
            }
            // step rows are XS = BST + 1 uint4 apart: the lanes of one store hold 16 steps of one
            // column, which then fall on 16 different bank groups instead of one
            uint4 *d = xs + (g >> 2) * XS + ct * 128 + ml + 16 * (g & 3);
            d[0] = make_uint4(H[0], H[1], H[2], H[3]);
            d[64] = make_uint4(Lo[0], Lo[1], Lo[2], Lo[3]);
        }
    }
    // the scales, into LDS (scale units past the split are zeroed)
    if constexpr (EARLY)
        if ((int)threadIdx.x < MF_TILES * nsu) scale_st((int)threadIdx.x, sreg);
    __syncthreads();

    mf_f4 acc[MF_RBW][CT];
#pragma unroll
    for (int r = 0; r < MF_RBW; r++)
#pragma unroll
        for (int c = 0; c < CT; c++) acc[r][c] = mf_f4{0, 0, 0, 0};

    // Scale words of this lane's 4 rows (16*(rbase+rb) + 4q .. +3) for staged unit u: one uint4
    // (4 rows x one fp32, or x an fp16 pair), or for qNg64 the two groups' float2s split into one
    // mf_f4 per group.
    struct SW { uint4 w; mf_f4 g0, g1; };
    auto scale_words = [&](int u, int rb) -> SW {
        const int row = 16 * (rbase + rb) + 4 * q;
        const uint4 *base = ss + (wt * UMAX + u) * SUT;
        SW r;
        if constexpr (SCW == 8) {
            const uint4 a = base[row >> 1], b = base[(row >> 1) + 1];
            r.g0 = mf_f4{__uint_as_float(a.x), __uint_as_float(a.z), __uint_as_float(b.x), __uint_as_float(b.z)};
            r.g1 = mf_f4{__uint_as_float(a.y), __uint_as_float(a.w), __uint_as_float(b.y), __uint_as_float(b.w)};
        } else {
            r.w = base[row >> 2];
        }
        return r;
    };
    auto scale_of = [&](const SW &r, int g) -> mf_f4 {
        if constexpr (FMT == BGL_Q4G32H) {                         // fp16 pairs: group g is half g of each word
            const uint32_t sh = 16 * g;
            return mf_f4{__half2float(__ushort_as_half((unsigned short)(r.w.x >> sh))),
                         __half2float(__ushort_as_half((unsigned short)(r.w.y >> sh))),
                         __half2float(__ushort_as_half((unsigned short)(r.w.z >> sh))),
                         __half2float(__ushort_as_half((unsigned short)(r.w.w >> sh)))};
        } else if constexpr (FMT == BGL_QNG64) {
            return g == 0 ? r.g0 : r.g1;
        } else {
            return mf_f4{__uint_as_float(r.w.x), __uint_as_float(r.w.y), __uint_as_float(r.w.z), __uint_as_float(r.w.w)};
        }
    };
    // Activation fragments of local step s (clamped into the staged range).
    struct BF { mf_h8 h[CT], l[CT]; };
    auto load_b = [&](int s) -> BF {
        const uint4 *p = xs + min(s, nsr - 1) * XS + lane;
        BF r;
#pragma unroll
        for (int c = 0; c < CT; c++) {
            r.h[c] = __builtin_bit_cast(mf_h8, p[c * 128]);
            r.l[c] = __builtin_bit_cast(mf_h8, p[c * 128 + 64]);
        }
        return r;
    };

    // ---- main loop: no barriers; each wave streams its own weights D K-steps ahead, and the next
    // step's fragments and the unit's scales are read from LDS a step ahead of their use.  The
    // fold is software-pipelined: a group's MFMA sums (cg[g % 2]) are folded into acc while the
    // next group's MFMAs run, so the matrix cores and the vector ALUs work at the same time ----
    static_assert((D / SPG) % 2 == 0, "group parity must repeat every ring");
    mf_f4 cg[2][MF_RBW][CT], scp[MF_RBW];
#pragma unroll
    for (int r = 0; r < MF_RBW; r++) {
        scp[r] = mf_f4{0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < CT; c++) { cg[0][r][c] = mf_f4{0, 0, 0, 0}; cg[1][r][c] = mf_f4{0, 0, 0, 0}; }
    }
    auto fold = [&](const mf_f4 (&g)[MF_RBW][CT]) {
#pragma unroll
        for (int rb = 0; rb < MF_RBW; rb++)
#pragma unroll
            for (int c = 0; c < CT; c++)
#pragma unroll
                for (int v = 0; v < 4; v++) acc[rb][c][v] = __fmaf_rn(g[rb][c][v], scp[rb][v], acc[rb][c][v]);
    };
    BF bnext;
    if constexpr (KW == 1) bnext = load_b(ls0);
    for (int sb = ls0; sb < ls1; sb += D) {
        SW swd[MF_RBW];
        ARaw<FMT, NB> apair[2][MF_RBW];
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int s = sb + d, par = (d / SPG) & 1;
            if (d % SPU == 0) {
#pragma unroll
                for (int rb = 0; rb < MF_RBW; rb++) swd[rb] = scale_words(s / SPU, rb);
            }
            // one slice (2 waves per SIMD) reads the next step's fragments ahead; two slices read
            // them in place (the other waves cover the LDS latency, and the registers are needed)
            BF bc;
            if constexpr (KW == 1) { bc = bnext; bnext = load_b(s + 1); }
            else bc = load_b(s);
            if (d % 2 == 0) {                                       // a new K-step pair: exchange, refill the slot
                exch<FMT, NB>(ring[d / 2], apair);
                load_w(ring[d / 2], s + D);                         // unconditional, clamped
            }
            mf_h8 A[MF_RBW];
#pragma unroll
            for (int r = 0; r < MF_RBW; r++) A[r] = dec_a<FMT, NB>(apair[d % 2][r], q);
            const bool gstart = d % SPG == 0;                       // first K-step of a scale group
#pragma unroll
            for (int h = 0; h < 2; h++)                             // all hi products, then the lo ones
#pragma unroll
                for (int c = 0; c < CT; c++)
#pragma unroll
                    for (int r = 0; r < MF_RBW; r++)
                        cg[par][r][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            A[r], h ? bc.l[c] : bc.h[c], gstart && !h ? mf_f4{0, 0, 0, 0} : cg[par][r][c], 0, 0, 0);
            if (gstart) fold(cg[par ^ 1]);                          // the previous group, while these run
            if ((d + 1) % SPG == 0) {                                // group complete: its scales for the next fold
                const int g = (d % SPU) / SPG;
#pragma unroll
                for (int rb = 0; rb < MF_RBW; rb++) scp[rb] = scale_of(swd[rb], g);
            }
        }
    }
    fold(cg[((D / SPG) - 1) & 1]);                                  // the last group

    // ---- outputs through LDS: a lane's sums lie on rows 16 apart per column (stored directly, each
    // store instruction would touch 16 output rows), so every wave puts its sums into
    // ob[slice][column][256 rows of the workgroup] and the stores below write runs of consecutive
    // rows, 16 bytes per lane.  Row index nl of column m sits at nl ^ 4*(m % 16) (a swizzle of whole
    // float4s that spreads a wave's writes over the banks).  The K-slices' sums are added there,
    // slice 0 + slice 1 ----
    constexpr int OBR = MF_TILES * BGL_TILE;                        // rows per workgroup
    static_assert(KW * 16 * CT * OBR * 4 <= (int)sizeof(xs), "output staging must fit the stage");
    __syncthreads();                                                // every wave is done with the staged data
    float *ob = reinterpret_cast<float *>(xs);
#pragma unroll
    for (int rb = 0; rb < MF_RBW; rb++)
#pragma unroll
        for (int c = 0; c < CT; c++) {
            // the lane's 4 sums of column m are rows nl..nl+3: one 16-byte write
            const int m = 16 * c + (lane & 15), nl = wt * BGL_TILE + 16 * (rbase + rb) + 4 * q;
            *reinterpret_cast<float4 *>(ob + (kw * 16 * CT + m) * OBR + (nl ^ ((m & 15) << 2))) =
                make_float4(acc[rb][c][0], acc[rb][c][1], acc[rb][c][2], acc[rb][c][3]);
        }
    __syncthreads();

    const int S = (KS + tk.kps - 1) / tk.kps;
    const int nb = tile0 * BGL_TILE;                                // first row of the workgroup
    for (int i = threadIdx.x; i < 16 * CT * (OBR / 4); i += NT) {
        const int m = i / (OBR / 4), nl = (i % (OBR / 4)) * 4, n = nb + nl;
        if (m >= L.M || n >= T.N) continue;
        const int sw = nl ^ ((m & 15) << 2);
        const float4 a = *reinterpret_cast<const float4 *>(ob + m * OBR + sw);
        float o[4] = {a.x, a.y, a.z, a.w};
        if constexpr (KW == 2) {
            const float4 b = *reinterpret_cast<const float4 *>(ob + (16 * CT + m) * OBR + sw);
            o[0] += b.x; o[1] += b.y; o[2] += b.z; o[3] += b.w;
        }
        const int ce = cex[m];
        float *dst = (S > 1 ? tk.part + ((size_t)split * L.M + m) * T.N : tk.y + (size_t)m * tk.ystride) + n;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            o[e] = ldexpf(o[e], ce);
            if (n + e < T.N) {
                if (cnf[m]) o[e] += mf_nonfinite<FMT, NB>(T, n + e, L.x + (size_t)m * T.K, 32 * s0, min(32 * (s0 + ns), T.K));
                if (S == 1 && tk.bias) o[e] += tk.bias[n + e];
            }
        }
        if (n + 3 < T.N && ((uintptr_t)dst & 15) == 0) {
            *reinterpret_cast<float4 *>(dst) = make_float4(o[0], o[1], o[2], o[3]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (n + e < T.N) dst[e] = o[e];
        }
    }
}

// ==================================================================================== K-split reduce
// y[m][n] = bias[n] + sum_s part[s][m][n], s in order, for every task of a launch with S > 1.  A
// thread owns 4 consecutive n of one m and keeps MF_RED_BATCH partials in flight.
// SwiGLU pair mode (glu_h set; tasks 0 and 1 are gate and up of one shape): a thread forms both
// tasks' values at its (m, n) -- the split sums as above, or y as the GEMM stored it when the task
// did not split -- and stores h = silu(g) * u (k_swiglu's arithmetic: exp in double, rounded once)
// instead of g and u.
#define MF_RED_BATCH 8
struct MfmaReduceTask {
    const float *part;
    const float *bias;
    float *y;
    int N, S, ystride, q0;   // q0: first quad of this task in the grid
};
struct MfmaReduce {
    MfmaReduceTask t[BGL_MAX_TASKS];
    int ntasks, M, nquads;
    float *glu_h;            // SwiGLU pair mode: h [M][glu_stride]
    int glu_stride;
};

// bias[n] + sum_s part[s][m][n] for the 4 values n.. of row m, s in order
__device__ __forceinline__ void mf_red_quad(const MfmaReduceTask &t, int M, int m, int n, float (&a)[4]) {
    const size_t plane = (size_t)M * t.N;
    const float *p = t.part + (size_t)m * t.N + n;
    const bool vec = (t.N & 3) == 0;
#pragma unroll
    for (int e = 0; e < 4; e++) a[e] = 0.0f;
    for (int s0 = 0; s0 < t.S; s0 += MF_RED_BATCH) {               // a batch of partials in flight, added in order
        float v[MF_RED_BATCH][4];
#pragma unroll
        for (int i = 0; i < MF_RED_BATCH; i++) {
            const int s = s0 + i;
            if (s >= t.S) break;
            if (vec) {
                const float4 f = *reinterpret_cast<const float4 *>(p + s * plane);
                v[i][0] = f.x; v[i][1] = f.y; v[i][2] = f.z; v[i][3] = f.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) v[i][e] = n + e < t.N ? p[s * plane + e] : 0.0f;
            }
        }
#pragma unroll
        for (int i = 0; i < MF_RED_BATCH; i++) {
            if (s0 + i >= t.S) break;
#pragma unroll
            for (int e = 0; e < 4; e++) a[e] = s0 + i == 0 ? v[i][e] : a[e] + v[i][e];
        }
    }
#pragma unroll
    for (int e = 0; e < 4; e++) a[e] = (t.bias && n + e < t.N ? t.bias[n + e] : 0.0f) + a[e];
}

__global__ __launch_bounds__(256) void k_mfma_reduce(MfmaReduce R) {
    const int qd = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (qd >= R.nquads) return;
    if (R.glu_h) {
        const MfmaReduceTask &tg = R.t[0], &tu = R.t[1];
        const int nq = (tg.N + 3) >> 2, m = qd / nq, n = 4 * (qd % nq);
        float g[4], u[4];
        if (tg.S > 1) mf_red_quad(tg, R.M, m, n, g);
        else {
#pragma unroll
            for (int e = 0; e < 4; e++) g[e] = n + e < tg.N ? tg.y[(size_t)m * tg.ystride + n + e] : 0.0f;
        }
        if (tu.S > 1) mf_red_quad(tu, R.M, m, n, u);
        else {
#pragma unroll
            for (int e = 0; e < 4; e++) u[e] = n + e < tu.N ? tu.y[(size_t)m * tu.ystride + n + e] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            if (n + e >= tg.N) break;
            const float ex = (float)exp(-(double)g[e]);
            R.glu_h[(size_t)m * R.glu_stride + n + e] = (g[e] / (1.0f + ex)) * u[e];
        }
        return;
    }
    int ti = 0;
#pragma unroll
    for (int i = 1; i < BGL_MAX_TASKS; i++)
        if (i < R.ntasks && qd >= R.t[i].q0) ti = i;
    const MfmaReduceTask &t = R.t[ti];
    const int nq = (t.N + 3) >> 2, lq = qd - t.q0;
    const int m = lq / nq, n = 4 * (lq % nq);
    float a[4];
    mf_red_quad(t, R.M, m, n, a);
#pragma unroll
    for (int e = 0; e < 4; e++) {
        if (n + e >= t.N) break;
        t.y[(size_t)m * t.ystride + n + e] = a[e];
    }
}

// ==================================================================================== host side
bool bgl_mfma_ok(int fmt, int bits) {
    if (fmt == BGL_Q4G64 || fmt == BGL_Q4G32H || fmt == BGL_Q8G64) return true;
    return fmt == BGL_QNG64 && bits >= 2 && bits <= MF_MAXN;
}

// Two K-slices (16 waves, <= 128 VGPRs) where that instance compiles without private memory --
// which instances fit depends on the register allocator, so it is read from the code object --
// else one slice (8 waves, <= 256 VGPRs), unless that one needs even more private memory.
template <int FMT, int NB, int CT>
static void launch_ct(const MfmaLaunch &L, dim3 grid, hipStream_t st) {
    static int kw2 = -1;
    if (kw2 < 0) {
        hipFuncAttributes a2, a1;
        const bool ok2 = hipFuncGetAttributes(&a2, reinterpret_cast<const void *>(&k_gemm_mfma<FMT, NB, CT, 2>)) == hipSuccess;
        const bool ok1 = hipFuncGetAttributes(&a1, reinterpret_cast<const void *>(&k_gemm_mfma<FMT, NB, CT, 1>)) == hipSuccess;
        // two slices unless they need private memory and one slice needs less
        kw2 = ok2 && (a2.localSizeBytes == 0 || !ok1 || a2.localSizeBytes <= a1.localSizeBytes);
    }
    if (kw2) hipLaunchKernelGGL((k_gemm_mfma<FMT, NB, CT, 2>), grid, dim3(MF_WAVES * 2 * 64), 0, st, L);
    else hipLaunchKernelGGL((k_gemm_mfma<FMT, NB, CT, 1>), grid, dim3(MF_WAVES * 64), 0, st, L);
}

template <int FMT, int NB>
static int launch_fmt(const MfmaLaunch &L, int CT, dim3 grid, hipStream_t st) {
    switch (CT) {
    case 1: launch_ct<FMT, NB, 1>(L, grid, st); return 0;
    case 2: launch_ct<FMT, NB, 2>(L, grid, st); return 0;
    case 3: launch_ct<FMT, NB, 3>(L, grid, st); return 0;
    case 4: launch_ct<FMT, NB, 4>(L, grid, st); return 0;
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
                  float *const *y, const int *ystride, float *glu_h) {
    const int K = Ts[0].K;
    if (glu_h && (n != 2 || Ts[1].N != Ts[0].N))
        return bgl_fail(BGL_E_ARG, "MFMA path: the SwiGLU pair needs two tensors of one shape");
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
    // The chunks run in stream order, so each reuses the same K-split partials.  In a no-alloc call
    // the fixed array is handed out by a bump pointer: rewind it to this mark before every chunk,
    // so the first (largest) chunk's reservation bounds the whole call.
    const size_t fixed_mark = c->fixed_used;
    for (int m0 = 0; m0 < M; m0 += 16 * MF_MAXCT) {
        const int Mc = M - m0 < 16 * MF_MAXCT ? M - m0 : 16 * MF_MAXCT;
        if (c->fixed_base) c->fixed_used = fixed_mark;
        const int CT = (Mc + 15) / 16;
        const int kpm = CT == 1 ? mf_kps_max(1) : CT == 2 ? mf_kps_max(2) : CT == 3 ? mf_kps_max(3) : mf_kps_max(4);
        MfmaLaunch L;
        memset(&L, 0, sizeof L);
        L.ntasks = n; L.M = Mc; L.x = x_dev + (size_t)m0 * K;
        int wgs = 0;
        size_t poff[BGL_MAX_TASKS], pfl = 0;              // partial offsets (floats) in the shared buffer
        int S_[BGL_MAX_TASKS];
        for (int i = 0; i < n; i++) {
            const BglDevTensor &T = Ts[i];
            const int wgr = (T.ntiles + MF_TILES - 1) / MF_TILES;
            // A split's K range must fit the workgroup's LDS (kpm steps); beyond that, split K until
            // the grid has ~min_blocks workgroups while the partials (written and read back once
            // each) stay under mf_pcap x the weight bytes (1 by default: at 0.5 the 4096 x 4096
            // qNg64 n=5 tensors of a 32-column launch ran 64 workgroups, 19.3 us, against 128 and
            // 15.0 us; finer splits than 16 K-steps measured no faster).
            const int smin = (KS + kpm - 1) / kpm;
            int S = (c->min_blocks + wgr - 1) / wgr;
            const int capS = (int)(c->mf_pcap * mf_weight_bytes(T) / (8.0 * Mc * T.N));
            if (S > capS) S = capS;
            if (S < smin) S = smin;
            if (S < 1) S = 1;
            int kps = (KS + S - 1) / S;
            kps = (kps + MF_KSTEP_PAD - 1) / MF_KSTEP_PAD * MF_KSTEP_PAD;
            if (kps > kpm) kps = kpm;
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
        MfmaReduce R;
        memset(&R, 0, sizeof R);
        R.M = Mc;
        if (pfl) {
            if (dbuf_reserve(c, c->part, pfl * 4, false)) return bgl_last_code();
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
        if (glu_h) {                    // SwiGLU pair: both tasks, split or not, one quad grid
            for (int i = 0; i < 2; i++) {
                const MfmaTask &t = L.t[i];
                MfmaReduceTask &rt = R.t[i];
                rt.part = S_[i] > 1 ? t.part : nullptr; rt.bias = t.bias; rt.y = t.y;
                rt.N = t.T.N; rt.S = S_[i]; rt.ystride = t.ystride; rt.q0 = 0;
            }
            R.ntasks = 2;
            R.glu_h = glu_h + (size_t)m0 * Ts[0].N;
            R.glu_stride = Ts[0].N;
            R.nquads = Mc * ((Ts[0].N + 3) / 4);
        }
        int tok = prof_begin(c, 1);
        if (launch_any(L, Ts[0].fmt, Ts[0].bits, CT, dim3(wgs), c->stream)) return bgl_fail(BGL_E_UNSUPPORTED, "MFMA path: format");
        prof_end(c, tok);
        HIPCHK(hipGetLastError());
        if (R.ntasks) {
            tok = prof_begin(c, 2);
            hipLaunchKernelGGL(k_mfma_reduce, dim3((R.nquads + 255) / 256), dim3(256), 0, c->stream, R);
            prof_end(c, tok);
            HIPCHK(hipGetLastError());
        }
    }
    return 0;
}
