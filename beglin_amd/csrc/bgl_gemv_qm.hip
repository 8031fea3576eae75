// bgl_gemv_qm.hip -- the W4A8 GEMV at 2..16 columns on the matrix cores (q4gemv_g256.h:230-262
// q4_gemv_g256_sdot_mt, q4gemv.h:87-133 q4_gemm_sdot_mt at M > 1 columns; q4g64, q8g64, g256sf and
// plain g256).
//
// One v_mfma_i32_16x16x64_i8 multiplies 16 weight rows by 64 activation codes of up to 16 columns
// (one MFMA column per activation column): a 64-value sub-group of a g256 unit, or a whole q4g64 /
// q8g64 unit.  Its int32 results are exactly the reference's integer dot products of those 64
// values (every product and sum is exact in int32), so each (row, column) then takes the
// reference's own fp32 terms: g256sf comb = sum_sg isum_sg * sub_sg and ((comb * wsuper) * (1/63))
// * ascale (q4gemv_g256.h:154), q4g64 ((isum - 8 * sum(xq)) * wscale) * ascale and q8g64
// (isum * wscale) * ascale (q4gemv.h:241), folded in group order: the outputs are bit-identical to
// the dot4 kernels' and the oracle's.  The dot4 path issues one 4-value product per lane and column;
// here one instruction covers 16 rows x 64 values x 16 columns, so the per-column VALU work that
// bounds k_gemv_q at 4-8 columns is gone.
//
// Operand layouts (measured on gfx950 with an in-bounds probe): lane l holds A[row l % 16]
// [k 16 (l / 16) .. +16], B[k 16 (l / 16) .. +16][column l % 16] and D[row 4 (l / 16) + v]
// [column l % 16], v = 0..3.  The k order inside a 64-value sub-group is the natural element order:
// lane group g = l / 16 takes elements 16g .. 16g + 15, i.e. bytes 8 (g % 2) .. +8 of the sub-group's
// chunk g / 2 for int4 (each byte i of a dword carries element i in its low and i + 4 in its high
// nibble: lo, hi, lo, hi of two dwords give elements 0-3, 4-7, 8-11, 12-15) and chunk g for int8.
// g256sf nibbles are signed (code ^ 8), so a nibble masked into the high half of a byte is
// 16 (code - 8) as an int8 and the MFMA sums come out 16x the reference's (shifted back exactly).
//
// Work split: a workgroup owns RB 16-row blocks of one 64-row tile and S slices of the units
// (wave = (block, slice); slice s takes units s, s + S, ...).  Without prepared codes the workgroup
// first quantizes its columns into LDS (the reference's q4_quant_act_i8 / _g256, bit for bit, the
// k_gemv_q passes), while the first weight loads are in flight; with prepared codes (k_act_w4a8)
// the B operand comes straight from global memory (L2-resident: M x K bytes).  Each unit's
// fp32 terms go to LDS as t[block][unit][row][column]; after one barrier every (row, column) folds
// its terms in unit order.
#include "bgl_gemv_q.h"

#define QM_MAXC 16   // columns per launch (the MFMA's N)

typedef int bgl_i32x4 __attribute__((ext_vector_type(4)));

template <int FMT> struct QmFmt {
    static constexpr int ELEMS = QUnit<FMT>::ELEMS;        // values per unit
    static constexpr int SG = ELEMS / 64;                  // 64-value sub-groups (MFMAs) per unit
    static constexpr int CPU = FMT == BGL_Q8G64 ? 4 : FMT == BGL_Q4G64 ? 2 : 8;   // 16-byte chunks per unit
};

// A operand of sub-group sg of unit u for row `row` of the tile, lane group g
template <int FMT>
__device__ __forceinline__ bgl_i32x4 qm_load_a(const uint8_t *w, int cpr, int tile, int u, int sg, int row, int g) {
    using F = QmFmt<FMT>;
    const size_t chunk = (size_t)tile * cpr + (size_t)u * F::CPU;
    if constexpr (FMT == BGL_Q8G64) {
        const bgl_u32x4 v = ((const BGL_GLOBAL bgl_u32x4 *)w)[(chunk + g) * BGL_TILE + row];
        return bgl_i32x4{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
    } else {
        const bgl_u32x2 v = ((const BGL_GLOBAL bgl_u32x2 *)w)[((chunk + 2 * sg + g / 2) * BGL_TILE + row) * 2 + (g & 1)];
        if constexpr (FMT == BGL_Q4G256SF)
            return bgl_i32x4{snib_lo16(v.x), snib_hi16(v.x), snib_lo16(v.y), snib_hi16(v.y)};
        else
            return bgl_i32x4{nib_lo(v.x), nib_hi(v.x), nib_lo(v.y), nib_hi(v.y)};
    }
}

template <int FMT, bool PREP, int QP>
__global__ __launch_bounds__(MAXW * BGL_TILE) void k_gemv_qm(GemvLaunch L, int RB, int S) {
    extern __shared__ __align__(16) unsigned char lds[];
    using QU = QUnit<FMT>;
    using F = QmFmt<FMT>;
    const int b = blockIdx.x;
    int ti = 0;
#pragma unroll
    for (int i = 1; i < BGL_MAX_TASKS; i++) if (i < L.ntasks && b >= L.t[i].blk0) ti = i;
    GemvTask task = L.t[0];
#pragma unroll
    for (int i = 1; i < BGL_MAX_TASKS; i++) if (i == ti) task = L.t[i];
    const BglDevTensor &T = task.T;
    const int SUBS = 4 / RB;                            // workgroups per 64-row tile
    const int lb = b - task.blk0, tile = lb / SUBS, rb0 = (lb % SUBS) * RB;
    const int nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int rb = wave / S, sl = wave % S;              // this wave's 16-row block and unit slice
    const int K = T.K, U = T.nunits, NGQ = K / QU::GQ, NP = (K + 255) / 256, MC = L.mcols, NPT = MC * NP;
    const int g = lane >> 4, col = min(lane & 15, MC - 1);   // B / D column (clamped past the launch's columns)
    const int arow = (rb0 + rb) * 16 + (lane & 15);      // A row within the tile
    // LDS: [xq: MC x XQS][ascale: MC x (NGQ+1)][xsum: MC x (K/64+1)] (quantized here) then the terms
    const int XQS = (U + 1) * QU::STRIDE;
    int8_t *xq = reinterpret_cast<int8_t *>(lds);
    float *asc = reinterpret_cast<float *>(lds + (PREP ? 0 : (size_t)MC * XQS));
    int *xsum = reinterpret_cast<int *>(asc + (PREP ? 0 : MC * (NGQ + 1)));
    float *tl = reinterpret_cast<float *>(xsum + (PREP ? 0 : MC * (K / 64 + 1)));

    // x loads of the first passes, then this wave's first weights (unconditional, clamped)
    // QP passes per wave and round: the host picks QP >= passes / waves where it can, so every x
    // load goes out in the first round (each further round would wait for its own loads)
    float4 xv[QP];
    const float *x = L.x + (size_t)L.m0 * K;
    if constexpr (!PREP) load_xpass<QP, QM_MAXC>(xv, x, wave, nw, K, NP, NPT, lane);
    // this wave's units go in batches of UB (a batch's weight loads all in flight at once); the first
    // batch is loaded before the quantization
    // (with prepared codes the B operands come from global memory and are loaded with the batch too)
    constexpr int UB = FMT == BGL_Q4G256SF ? 2 : 4;
    constexpr int SCW = FMT == BGL_Q4G256SF ? 2 : 1;     // 16-byte scale records of the lane's 4 D rows per unit
    bgl_i32x4 a[UB][F::SG], bq[PREP ? UB : 1][F::SG];
    bgl_u32x4 sr[UB][SCW];
    const int8_t *pq = PREP ? reinterpret_cast<const int8_t *>(L.a.xw) + (size_t)(L.m0 + col) * K : nullptr;
    auto load_batch = [&](int ub) {
#pragma unroll
        for (int i = 0; i < UB; i++) {
            const int u = min(ub + i * S, U - 1);
#pragma unroll
            for (int s = 0; s < F::SG; s++) a[i][s] = qm_load_a<FMT>(T.w, T.cpr, tile, u, s, arow, g);
            // scales of the 4 D rows of this lane: rows 4g .. 4g+3 of the block
            const size_t so = ((size_t)tile * T.nunits + u) * BGL_TILE + (rb0 + rb) * 16 + 4 * g;
#pragma unroll
            for (int k = 0; k < SCW; k++) sr[i][k] = ((const BGL_GLOBAL bgl_u32x4 *)T.s0)[so / (4 / SCW) + k];
            if constexpr (PREP) {
#pragma unroll
                for (int s = 0; s < F::SG; s++) {
                    const bgl_u32x4 v = *(const BGL_GLOBAL bgl_u32x4 *)(pq + (size_t)u * F::ELEMS + s * 64 + 16 * g);
                    bq[i][s] = bgl_i32x4{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
                }
            }
        }
    };
    load_batch(sl);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!PREP) {
        quant_passes<FMT, QP, QM_MAXC>(xv, wave, nw, K, NP, NPT, NGQ, U, lane, xq, asc, xsum);
        for (int p0 = wave + QP * nw; p0 < NPT; p0 += QP * nw) {
            load_xpass<QP, QM_MAXC>(xv, x, p0, nw, K, NP, NPT, lane);
            quant_passes<FMT, QP, QM_MAXC>(xv, p0, nw, K, NP, NPT, NGQ, U, lane, xq, asc, xsum);
        }
        __syncthreads();
    }
    // the B operand of sub-group s of batch slot i, unit u (16 codes of column `col`)
    auto load_b = [&](int i, int u, int s) -> bgl_i32x4 {
        if constexpr (PREP) return bq[i][s];
        else return *reinterpret_cast<const bgl_i32x4 *>(xq + col * XQS + u * QU::STRIDE + s * 64 + 16 * g);
    };
    for (int ub = sl;;) {
#pragma unroll
        for (int i = 0; i < UB; i++) {
            const int u = ub + i * S;
            if (u >= U) break;
            int comb[4] = {0, 0, 0, 0};
            float ws[4];
            if constexpr (FMT == BGL_Q4G256SF) {
                const bgl_u32x4 s01 = sr[i][0], s23 = sr[i][SCW - 1];
                const uint32_t sc[4] = {s01.x, s01.z, s23.x, s23.z}, sb[4] = {s01.y, s01.w, s23.y, s23.w};
#pragma unroll
                for (int s = 0; s < F::SG; s++) {
                    const bgl_i32x4 d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i][s], load_b(i, u, s), bgl_i32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 4; v++) comb[v] += d[v] * (int)((sb[v] >> (8 * s)) & 255u);
                }
#pragma unroll
                for (int v = 0; v < 4; v++) ws[v] = __uint_as_float(sc[v]);
            } else {
                const bgl_u32x4 s4u = sr[i][0];
                const bgl_f32x4 s4 = {__uint_as_float(s4u.x), __uint_as_float(s4u.y), __uint_as_float(s4u.z), __uint_as_float(s4u.w)};
                const bgl_i32x4 d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i][0], load_b(i, u, 0), bgl_i32x4{0, 0, 0, 0}, 0, 0, 0);
                comb[0] = d[0]; comb[1] = d[1]; comb[2] = d[2]; comb[3] = d[3];
                ws[0] = s4.x; ws[1] = s4.y; ws[2] = s4.z; ws[3] = s4.w;
            }
            // the unit's fp32 terms (unit_float's arithmetic), column `col`
            float as;
            int xs = 0;
            if constexpr (PREP) {
                as = L.a.xs[(size_t)(L.m0 + col) * NGQ + u];
                if constexpr (QU::XSUM) xs = L.a.xsum[(size_t)(L.m0 + col) * (K / 64) + u];
            } else {
                as = asc[col * (NGQ + 1) + u];
                if constexpr (QU::XSUM) xs = xsum[col * (K / 64 + 1) + u];
            }
            float *tu = tl + ((size_t)rb * U + u) * 256 + 4 * g * 16 + (lane & 15);
#pragma unroll
            for (int v = 0; v < 4; v++) {
                float t;
                if constexpr (FMT == BGL_Q4G256SF) t = __fmul_rn(__fmul_rn(__fmul_rn((float)(comb[v] >> 4), ws[v]), T.gmul), as);
                else if constexpr (FMT == BGL_Q4G64) t = __fmul_rn(__fmul_rn((float)(comb[v] - 8 * xs), ws[v]), as);
                else t = __fmul_rn(__fmul_rn((float)comb[v], ws[v]), as);
                tu[v * 16] = t;
            }
        }
        ub += UB * S;
        if (ub >= U) break;
        load_batch(ub);
    }
    __syncthreads();
    // each (block, row, column) folds its terms in unit order (the reference's group loop)
    for (int t = threadIdx.x; t < RB * 16 * MC; t += nw * 64) {
        const int bl = t / (16 * MC), r = (t / MC) % 16, c = t % MC;
        const int row = tile * BGL_TILE + (rb0 + bl) * 16 + r;
        if (row >= T.N) continue;
        const float *tr = tl + (size_t)bl * U * 256 + r * 16 + c;
        float acc = 0.0f, t8[8];
        const int U8 = U & ~7;
        for (int g0 = 0; g0 < U8; g0 += 8) {
#pragma unroll
            for (int i = 0; i < 8; i++) t8[i] = tr[(g0 + i) * 256];
#pragma unroll
            for (int i = 0; i < 8; i++) acc = __fadd_rn(acc, t8[i]);
        }
        for (int g0 = U8; g0 < U; g0++) acc = __fadd_rn(acc, tr[g0 * 256]);
        const float bb = task.bias ? task.bias[row] : 0.0f;
        task.y[(size_t)(L.m0 + c) * task.ystride + row] = __fadd_rn(bb, acc);
    }
}

size_t bgl_gemv_qm_lds(int fmt, int K, int MC, int RB, bool prep) {
    const int ELEMS = fmt == BGL_Q4G256SF ? 256 : 64, GQ = ELEMS, U = K / ELEMS;
    const size_t xs = prep ? 0 : (size_t)MC * ((U + 1) * (ELEMS + 16) + 4 * (K / GQ + 1) + 4 * (K / 64 + 1));
    return xs + (size_t)RB * U * 256 * 4;
}

template <int FMT>
static int qm_launch(bool prep, const GemvLaunch &L, int nblk, int RB, int S, size_t lds, hipStream_t st) {
    const dim3 g(nblk), b(RB * S * BGL_TILE);
    const int NP = (L.t[0].T.K + 255) / 256, ppw = (L.mcols * NP + RB * S - 1) / (RB * S);
    if (prep) hipLaunchKernelGGL((k_gemv_qm<FMT, true, 1>), g, b, lds, st, L, RB, S);
    else if (ppw <= 2) hipLaunchKernelGGL((k_gemv_qm<FMT, false, 2>), g, b, lds, st, L, RB, S);
    else if (ppw <= 4) hipLaunchKernelGGL((k_gemv_qm<FMT, false, 4>), g, b, lds, st, L, RB, S);
    else hipLaunchKernelGGL((k_gemv_qm<FMT, false, 8>), g, b, lds, st, L, RB, S);
    return 0;
}

// L: tasks with blk0 in workgroup units (4 / RB per tile), mcols in [2, 16]; prep: L.a holds the
// launch's prepared codes.
int bgl_launch_gemv_qm(const GemvLaunch &L, int nblk, int RB, int S, bool prep, hipStream_t st) {
    const int fmt = L.t[0].T.fmt;
    if (L.mcols < 1 || L.mcols > QM_MAXC || (RB != 1 && RB != 2 && RB != 4) || S < 1 || RB * S > MAXW) return -1;
    const size_t lds = bgl_gemv_qm_lds(fmt, L.t[0].T.K, L.mcols, RB, prep);
    switch (fmt) {
    case BGL_Q4G256SF: return qm_launch<BGL_Q4G256SF>(prep, L, nblk, RB, S, lds, st);
    case BGL_Q4G64: return qm_launch<BGL_Q4G64>(prep, L, nblk, RB, S, lds, st);
    case BGL_Q8G64: return qm_launch<BGL_Q8G64>(prep, L, nblk, RB, S, lds, st);
    default: return -2;
    }
}
