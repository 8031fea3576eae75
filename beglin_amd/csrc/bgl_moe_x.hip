// bgl_moe_x.hip -- host side of the expert-sorted MoE gather over LDS activation records: the
// LDS sizing, the launch shape and the launchers of k_moe_x / k_moe_x2 (device code in
// bgl_moe_x.h, kernel instances in bgl_moe_x_i*.hip).
#include "bgl_moe_x.h"

bool bgl_moe_x_fmt(int fmt) {
    return fmt == BGL_Q4G64 || fmt == BGL_Q4G32H || fmt == BGL_Q8G64 || fmt == BGL_QNG64 || fmt == BGL_MXFP4;
}

// LDS: cap columns of records (K/64 rounded up to whole slots of 64/TR groups), the wave partials
// (MX_MB columns per wave), and one slot of level-1 records per wave (cold path).
size_t bgl_moe_x_lds(int K, int nw, int TR, int cap) {
    const int KQ = BGL_TILE / TR, S = (K / 64 + KQ - 1) / KQ;
    return (size_t)cap * S * KQ * XREC_DW * 4 + (size_t)nw * 2 * MX_MB * TR * 4 + (size_t)nw * KQ * XREC_DW * 4;
}

// Record columns a launch's LDS holds: 8 where that fits the workgroups the launch keeps per CU
// (two of 64 rows, one of 16 rows), else 4.
int bgl_moe_x_cap(int K, int nw, int TR) {
    return bgl_moe_x_lds(K, nw, TR, 2 * MX_MB) <= (TR == BGL_TILE ? 80 : 160) * 1024 ? 2 * MX_MB : MX_MB;
}

int bgl_launch_moe_x2(const MoeTask &a, const MoeTask &b, int K, int nw, int cap, hipStream_t st) {
    if (K < 64 || K % 64 || nw < 1 || nw > MX_MAXW || (cap != MX_MB && cap != 2 * MX_MB)) return -1;
    if (a.seg > 0 && !a.off) return -1;                     // the first task is never segmented
    const bool seg1 = !b.off && b.seg > 0;
    const size_t lds = bgl_moe_x_lds(K, nw, BGL_TILE, cap);
    if (lds > 160 * 1024) return -1;
    MoePair P;
    P.t[0] = a; P.t[1] = b;
    P.t[0].mbx = cap; P.t[1].mbx = cap;
    P.nb0 = a.E * a.tpe;
    const dim3 g(P.nb0 + b.E * b.tpe), bl(nw * BGL_TILE);
    if (nw <= 8) {
        if (seg1) moe_x2_go<8, true>(g, bl, lds, st, P);
        else moe_x2_go<8, false>(g, bl, lds, st, P);
    } else {
        if (seg1) moe_x2_go<16, true>(g, bl, lds, st, P);
        else moe_x2_go<16, false>(g, bl, lds, st, P);
    }
    return 0;
}

// Mt.a.xf: the raw fp32 activation rows (row stride K = the tensors' in).  TR rows per workgroup
// (64 or 16), nw waves (<= 16, at most one per slot of 64/TR groups).
int bgl_launch_moe_x(const MoeTask &Mt0, int K, int TR, int nw, int cap, hipStream_t st) {
    if (K < 64 || K % 64 || nw < 1 || nw > MX_MAXW || (TR != 64 && TR != 16) || (cap != MX_MB && cap != 2 * MX_MB)) return -1;
    const size_t lds = bgl_moe_x_lds(K, nw, TR, cap);
    if (lds > 160 * 1024) return -1;
    MoeTask Mt = Mt0;
    Mt.mbx = cap;
    const dim3 g(Mt.E * Mt.tpe * (BGL_TILE / TR)), b(nw * BGL_TILE);
    const bool seg = !Mt.off && Mt.seg > 0;
#define MX_GO(S_, W_, T_) moe_x_go<S_, W_, T_>(g, b, lds, st, Mt)
    if (TR == 64) {
        if (nw <= 8) { if (seg) MX_GO(true, 8, 64); else MX_GO(false, 8, 64); }
        else { if (seg) MX_GO(true, 16, 64); else MX_GO(false, 16, 64); }
    } else {
        if (seg) MX_GO(true, 8, 16); else MX_GO(false, 8, 16);
    }
#undef MX_GO
    return 0;
}

// Shape of a launch with active_wgs workgroups of whole tiles: very few (< 128: the shared experts
// at a few tokens) -> 16-row workgroups (4x as many) of up to 8 waves; few (< 256: the routed
// experts of one token) -> whole tiles of 12 waves; else whole tiles of 8 waves.  tr_force /
// nw_cap: tuning overrides.
void bgl_moe_x_shape(int K, long active_wgs, int tr_force, int nw_cap, int *TR, int *nw) {
    int tr = active_wgs < 128 ? 16 : 64;
    if (tr_force == 16 || tr_force == 64) tr = tr_force;
    const int KQ = BGL_TILE / tr, S = (K / 64 + KQ - 1) / KQ;
    int w = active_wgs < 256 ? 12 : 8;
    if (nw_cap > 0) w = nw_cap < MX_MAXW ? nw_cap : MX_MAXW;
    if (tr == 16 && w > 8) w = 8;
    *TR = tr;
    *nw = S < w ? S : w;
}
