// bgl_prep.hip -- activation preparation, device packers, and repack into the tiled layout.
//
// Every fp32 operation that must reproduce the reference bit for bit is a separate IEEE operation:
// the library is compiled with -ffp-contract=off (no multiply-add is fused), divisions are
// correctly rounded, and rintf is round-half-even -- each step rounds exactly as the reference's C
// expression does.
#include "bgl_device.h"
#include "bgl_kernels.h"


// ------------------------------------------------------------------ W4A8 activation quantizer
// q4gemv.h:177-213 / q4gemv_g256.h:72-99: mx = max(1e-8, max|x|); sc = mx/127; inv = 1/sc;
// q = sat8(trunc(x*inv +/- 0.5)).  One wave per (column, group); gsize is 64 or 256 (lane handles
// gsize/64 elements, element l + 64*j).  Also writes the exact sum of xq per 64-subgroup (used for
// the nibble bias correction) and xq itself as packed int8.
// |x| is maximised on its bit pattern, where every NaN lies above +Inf and +Inf above every finite
// value: that is the reference's FMAX (vmaxq_f32 / vmaxvq_f32), which carries a NaN into mx.  A group
// whose maximum is NaN or +-Inf gets sc = NaN or +Inf and every code 0 (FCVTZS maps the NaN products
// to 0; with inv = 0 the finite ones are +-0), so the fold's 0 * sc makes its outputs NaN.
// u != null: the column is h = silu(x) * u of the MLP block (swiglu, qwen_infer.c:726-733, the
// arithmetic of k_swiglu in bgl_mlp.hip: x / (1 + exp(-x)) * u, the exponential rounded once from
// double), formed here and also written to h, so the SwiGLU costs no launch of its own.
__global__ __launch_bounds__(256) void k_act_w4a8(const float *__restrict__ x, int M, int K, int gsize,
                                                  int8_t *__restrict__ xq, float *__restrict__ ascale,
                                                  int *__restrict__ xqsum64, const float *__restrict__ u,
                                                  float *__restrict__ h) {
    int wid = (blockIdx.x * blockDim.x + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    int ng = K / gsize;
    if (wid >= M * ng) return;
    int m = wid / ng, g = wid % ng, per = gsize >> 6;
    const size_t o = (size_t)m * K + (size_t)g * gsize;
    const float *xp = x + o;
    float v[4];
    uint32_t mb = __float_as_uint(1e-8f);                  // mx starts at 1e-8 (q4gemv.h:182)
    // all four slots unconditionally (per < 4 repeats the last element, which leaves the maximum
    // unchanged), so the SwiGLU exponentials of a lane overlap
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int jj = j < per ? j : per - 1;
        v[j] = xp[lane + 64 * jj];
        if (u) {
            const float e = (float)exp(-(double)v[j]);
            v[j] = __fmul_rn(__fdiv_rn(v[j], __fadd_rn(1.0f, e)), u[o + lane + 64 * jj]);
            if (j < per) h[o + lane + 64 * j] = v[j];
        }
        mb = max(mb, __float_as_uint(v[j]) & 0x7fffffffu);
    }
    mb = wave_max_u32(mb);
    const bool nf = mb >= 0x7f800000u;                    // NaN or +-Inf in the group: every code 0
    float sc = __fdiv_rn(__uint_as_float(mb), 127.0f), inv = __fdiv_rn(1.0f, sc);
    if (lane == 0) ascale[(size_t)m * ng + g] = sc;
    for (int j = 0; j < per; j++) {
        float p = nf ? 0.0f : __fmul_rn(v[j], inv);
        float t = __fadd_rn(p, p >= 0.0f ? 0.5f : -0.5f);
        int q;
        if (t >= 2147483647.0f) q = 2147483647;
        else if (t <= -2147483648.0f) q = -2147483647 - 1;
        else q = (int)t;                                   // truncation toward zero
        q = q > 127 ? 127 : (q < -128 ? -128 : q);
        xq[(size_t)m * K + (size_t)g * gsize + lane + 64 * j] = (int8_t)q;
        int s = wave_sum_i32(q);
        if (lane == 0) xqsum64[(size_t)m * (K >> 6) + (size_t)g * per + j] = s;
    }
}

// ------------------------------------------------------------------ fp32 activation digits
// One wave per (column, 64-group), lane = element.  Level 0: e = exponent of the group's largest
// finite |x| (frexp, at least BGL_X_EMIN), X = rint(x * 2^(22-e)), |X| <= 2^22, as X = d0 + 256*d1 + 65536*d2 with
// balanced int8 digits.  Level 1 (bgl_x_level1: groups with BGL_X_SMALL_MAX or more nonzero
// elements below 2^(e-BGL_X_SPIKE_BITS), or more of them than elements above): the exact residual
// r = x * 2^(22-e) - X in the same form relative to its own maximum, X1 = rint(r * 2^(22-e1)).
// Non-finite elements count as 0 and flag the group.  Each buffer holds level 0 for all M columns,
// then level 1:
//   xd   [m][g][digit][64] bytes, then the level-1 digits;
//   xs   [m][g] = 2^(e-22), then [m][g] = 2^(e1-22) (0 without level 1);
//   dsum [m][K/32][4] per-half digit sums (the 4th int: the group's BGL_XF_* flags), then level 1's.
__device__ __forceinline__ int x_balanced3(int X, int &d0, int &d1) {
    d0 = (int)(int8_t)(X & 255);
    const int X1 = (X - d0) >> 8;
    d1 = (int)(int8_t)(X1 & 255);
    return (X1 - d1) >> 8;
}

__global__ __launch_bounds__(256) void k_act_x24(const float *__restrict__ x, int M, int K,
                                                 int8_t *__restrict__ xd, float *__restrict__ xs,
                                                 int *__restrict__ dsum) {
    int wid = (blockIdx.x * blockDim.x + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    int ng = K >> 6;
    if (wid >= M * ng) return;
    int m = wid / ng, g = wid % ng;
    float v = x[(size_t)m * K + (size_t)g * 64 + lane];
    uint32_t ab = __float_as_uint(v) & 0x7fffffffu;
    const bool nf = ab >= 0x7f800000u;                     // NaN or +-Inf: 0 in the digits
    if (nf) { v = 0.0f; ab = 0u; }
    float mx = wave_max_f32(__uint_as_float(ab));
    int e = 0;
    if (mx > 0.0f) frexpf(mx, &e);
    e = max(e, BGL_X_EMIN);
    const float thr = mx > 0.0f ? ldexpf(1.0f, e - BGL_X_SPIKE_BITS) : 0.0f;
    const int cnt = wave_sum_i32((ab != 0u && __uint_as_float(ab) >= thr ? 1 : 0) + (ab != 0u ? 256 : 0) + (nf ? 65536 : 0));
    const int nlarge = cnt & 255, nnz = (cnt >> 8) & 255, nnf = cnt >> 16;
    const float xp = mx > 0.0f ? ldexpf(v, BGL_X_FRAC - e) : 0.0f;   // power-of-two scaling: exact
    const float Xf = rintf(xp);
    int d0, d1;
    int d2 = x_balanced3((int)Xf, d0, d1);
    int8_t *dst = xd + ((size_t)m * ng + g) * 192;
    dst[lane] = (int8_t)d0; dst[64 + lane] = (int8_t)d1; dst[128 + lane] = (int8_t)d2;
    int flags = nnf ? BGL_XF_NF : 0;
    float ratio = 0.0f;
    if (bgl_x_level1(nnz - nlarge, nlarge)) {              // wave-uniform: one group per wave
        const float r = xp - Xf;                           // exact: xp and rint(xp) differ by <= 1/2
        const float mr = wave_max_f32(fabsf(r));
        if (mr > 0.0f) {
            int e1 = 0;
            frexpf(mr, &e1);
            int c0, c1;
            const int c2 = x_balanced3((int)rintf(ldexpf(r, BGL_X_FRAC - e1)), c0, c1);
            int8_t *d1p = xd + ((size_t)M * ng + (size_t)m * ng + g) * 192;
            d1p[lane] = (int8_t)c0; d1p[64 + lane] = (int8_t)c1; d1p[128 + lane] = (int8_t)c2;
            const int2 t0 = half_sums_i32(c0), t1 = half_sums_i32(c1), t2 = half_sums_i32(c2);
            if ((lane & 31) == 0) {
                const int h = lane >> 5;
                int *ds = dsum + ((size_t)M * (K >> 5) + (size_t)m * (K >> 5) + (size_t)g * 2 + h) * 4;
                ds[0] = h ? t0.y : t0.x; ds[1] = h ? t1.y : t1.x; ds[2] = h ? t2.y : t2.x; ds[3] = 0;
            }
            ratio = ldexpf(1.0f, e1 - BGL_X_FRAC);
            flags |= BGL_XF_L1;
        }
    }
    if (lane == 0) {
        xs[(size_t)m * ng + g] = (mx > 0.0f) ? ldexpf(1.0f, e - BGL_X_FRAC) : 0.0f;
        xs[(size_t)M * ng + (size_t)m * ng + g] = ratio;
    }
    int2 s0 = half_sums_i32(d0), s1 = half_sums_i32(d1), s2 = half_sums_i32(d2);
    if ((lane & 31) == 0) {
        const int h = lane >> 5;
        int *ds = dsum + ((size_t)m * (K >> 5) + (size_t)g * 2 + h) * 4;
        ds[0] = h ? s0.y : s0.x; ds[1] = h ? s1.y : s1.x; ds[2] = h ? s2.y : s2.x; ds[3] = flags;
    }
}

// ------------------------------------------------------------------ caller-quantized int8 columns
// q4_quant_act_i8 output handed over by the caller (gemm_qXg64_sdot_mt / gemm_q4g256sf_sdot_mt,
// q4gemv.h:779, q4gemv_g256.h:368) -> the W4A8 operand layout: natural-order codes, the scales
// per gq-group and the per-64 code sums.  One wave per (column, 64-group), lane = element.
// split=1: the source is in q4_split_act order (per 32 bytes: the 16 even then the 16 odd
// elements, q4gemv.h:306-312).
__global__ __launch_bounds__(256) void k_act_import_i8(const int8_t *__restrict__ xq, const float *__restrict__ ascale,
                                                       int M, int K, int gq, int split, int8_t *__restrict__ xw,
                                                       float *__restrict__ xs, int *__restrict__ xsum64) {
    const int wid = (blockIdx.x * blockDim.x + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    const int ng = K >> 6;
    if (wid >= M * ng) return;
    const int m = wid / ng, g = wid % ng;
    const int i = lane & 31, half = lane >> 5;
    const int src = split ? half * 32 + ((i & 1) ? 16 : 0) + (i >> 1) : lane;
    const int v = xq[(size_t)m * K + (size_t)g * 64 + src];
    xw[(size_t)m * K + (size_t)g * 64 + lane] = (int8_t)v;
    const int sum = wave_sum_i32(v);
    const int per = gq >> 6;
    if (lane == 0) {
        xsum64[(size_t)m * ng + g] = sum;
        if (g % per == 0) xs[(size_t)m * (K / gq) + g / per] = ascale[(size_t)m * (K / gq) + g / per];
    }
}

// ------------------------------------------------------------------ device packers (reference byte layouts)
// One thread per (row, group).  Arithmetic identical to the reference packers.

// gguf_transcode.c:24-68 (q4g64 with error feedback).
__global__ void k_quant_q4g64(const float *__restrict__ w, int N, int K, uint8_t *__restrict__ packed,
                              float *__restrict__ scales) {
    int ng = K / 64;
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)N * ng) return;
    int r = (int)(t / ng), g = (int)(t % ng);
    const float *grp = w + (size_t)r * K + (size_t)g * 64;
    float maxabs = 0.0f;
    for (int p = 0; p < 64; p++) maxabs = fmaxf(maxabs, fabsf(grp[p]));
    float scale = __fdiv_rn(maxabs, 7.0f);
    if (scale < 1e-12f) scale = 1.0f;
    scales[t] = scale;
    float inv = __fdiv_rn(1.0f, scale), err = 0.0f;
    uint8_t *prow = packed + (size_t)r * (K / 2) + (size_t)g * 32;
    for (int p = 0; p < 64; p += 2) {
        int nib[2];
        for (int h = 0; h < 2; h++) {
            float xv = __fadd_rn(grp[p + h], err);
            float qf = rintf(__fmul_rn(xv, inv));
            qf = fminf(fmaxf(qf, -8.0f), 7.0f);
            err = __fsub_rn(xv, __fmul_rn(qf, scale));
            nib[h] = ((int)qf + 8) & 15;
        }
        prow[p / 2] = (uint8_t)(nib[0] | (nib[1] << 4));
    }
}

// gguf_transcode.c:70-101 (q8g64: direct division, no error feedback).
__global__ void k_quant_q8g64(const float *__restrict__ w, int N, int K, int8_t *__restrict__ codes,
                              float *__restrict__ scales) {
    int ng = K / 64;
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)N * ng) return;
    int r = (int)(t / ng), g = (int)(t % ng);
    const float *grp = w + (size_t)r * K + (size_t)g * 64;
    float maxabs = 0.0f;
    for (int p = 0; p < 64; p++) maxabs = fmaxf(maxabs, fabsf(grp[p]));
    float scale = __fdiv_rn(maxabs, 127.0f);
    if (scale < 1e-12f) scale = 1.0f;
    scales[t] = scale;
    int8_t *c = codes + (size_t)r * K + (size_t)g * 64;
    for (int p = 0; p < 64; p++) {
        float qf = rintf(__fdiv_rn(grp[p], scale));
        qf = fminf(fmaxf(qf, -127.0f), 127.0f);
        c[p] = (int8_t)qf;
    }
}

// gguf_transcode.c:108-162 (dense_floor=0) or qng64_dense.c:29-68 (dense_floor=1): the two
// qNg64 encoders differ only in the scale floor test.
__global__ void k_quant_qng64(const float *__restrict__ w, int N, int K, int n, int dense_floor,
                              uint8_t *__restrict__ planes, float *__restrict__ scales) {
    int ng = K / 64;
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)N * ng) return;
    int r = (int)(t / ng), g = (int)(t % ng);
    int qmax = (1 << (n - 1)) - 1, qmin = -(1 << (n - 1)), bias = 1 << (n - 1), mask = (1 << n) - 1;
    const float *grp = w + (size_t)r * K + (size_t)g * 64;
    float maxabs = 0.0f;
    for (int p = 0; p < 64; p++) maxabs = fmaxf(maxabs, fabsf(grp[p]));
    float scale;
    if (dense_floor) scale = maxabs > 1e-12f ? __fdiv_rn(maxabs, (float)qmax) : 1.0f;
    else { scale = __fdiv_rn(maxabs, (float)qmax); if (scale < 1e-12f) scale = 1.0f; }
    scales[t] = scale;
    float inv = __fdiv_rn(1.0f, scale), err = 0.0f;
    uint32_t pl[15][2];
    for (int j = 0; j < 15; j++) { pl[j][0] = 0; pl[j][1] = 0; }
    for (int p = 0; p < 64; p++) {
        float xv = __fadd_rn(grp[p], err);
        float qf = rintf(__fmul_rn(xv, inv));
        qf = fminf(fmaxf(qf, (float)qmin), (float)qmax);
        err = __fsub_rn(xv, __fmul_rn(qf, scale));
        uint32_t u = (uint32_t)(((int)qf + bias) & mask);
        for (int j = 0; j < n; j++) pl[j][p >> 5] |= ((u >> j) & 1u) << (p & 31);
    }
    uint32_t *dst = reinterpret_cast<uint32_t *>(planes + ((size_t)r * ng + g) * (size_t)n * 8);
    for (int j = 0; j < n; j++) { dst[2 * j] = pl[j][0]; dst[2 * j + 1] = pl[j][1]; }
}

// gguf_write_quants.c:34-62 (Q4_0 encoder: fp32 scale inside the loop, fp16 stored), written in
// the Q4G32H pairing (byte b low = element 2b, high = 2b+1) with the fp16 scale beside it.
__global__ void k_quant_q4g32h(const float *__restrict__ w, int N, int K, uint8_t *__restrict__ packed,
                               uint16_t *__restrict__ scales16) {
    int nb = K / 32;
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)N * nb) return;
    int r = (int)(t / nb), b = (int)(t % nb);
    const float *grp = w + (size_t)r * K + (size_t)b * 32;
    float maxabs = 0.0f;
    for (int p = 0; p < 32; p++) maxabs = fmaxf(maxabs, fabsf(grp[p]));
    float scale = __fdiv_rn(maxabs, 7.0f);
    if (scale < 1e-12f) scale = 1.0f;
    scales16[t] = __half_as_ushort(__float2half_rn(scale));
    float inv = __fdiv_rn(1.0f, scale), err = 0.0f;
    uint8_t *dst = packed + (size_t)r * (K / 2) + (size_t)b * 16;
    for (int p = 0; p < 32; p += 2) {
        int nib[2];
        for (int h = 0; h < 2; h++) {
            float xv = __fadd_rn(grp[p + h], err);
            float qf = rintf(__fmul_rn(xv, inv));
            qf = fminf(fmaxf(qf, -8.0f), 7.0f);
            err = __fsub_rn(xv, __fmul_rn(qf, scale));
            nib[h] = ((int)qf + 8) & 15;
        }
        dst[p / 2] = (uint8_t)(nib[0] | (nib[1] << 4));
    }
}

// q4g256sf (build-defined packer; same arithmetic as the oracle's or_quantize_g256sf): one thread
// per (row, superblock).
__global__ void k_quant_g256sf(const float *__restrict__ w, int N, int K, uint8_t *__restrict__ packed,
                               float *__restrict__ wsuper, uint8_t *__restrict__ sub) {
    int ns = K / 256;
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)N * ns) return;
    int r = (int)(t / ns), gs = (int)(t % ns);
    const float *row = w + (size_t)r * K;
    float s64[4], ws = 0.0f;
    for (int k = 0; k < 4; k++) {
        const float *grp = row + (size_t)(gs * 4 + k) * 64;
        float maxabs = 0.0f;
        for (int p = 0; p < 64; p++) maxabs = fmaxf(maxabs, fabsf(grp[p]));
        s64[k] = __fdiv_rn(maxabs, 7.0f);
        ws = fmaxf(ws, s64[k]);
    }
    if (ws < 1e-12f) ws = 1.0f;
    wsuper[t] = ws;
    for (int k = 0; k < 4; k++) {
        int g = gs * 4 + k;
        int sc = (int)ceilf(__fdiv_rn(__fmul_rn(63.0f, s64[k]), ws));
        sc = sc < 1 ? 1 : (sc > 63 ? 63 : sc);
        sub[(size_t)r * (K / 64) + g] = (uint8_t)sc;
        float scale = __fmul_rn(ws, __fdiv_rn((float)sc, 63.0f));
        float inv = __fdiv_rn(1.0f, scale), err = 0.0f;
        const float *grp = row + (size_t)g * 64;
        uint8_t *dst = packed + (size_t)r * (K / 2) + (size_t)g * 32;
        for (int p = 0; p < 64; p += 2) {
            int nib[2];
            for (int h = 0; h < 2; h++) {
                float xv = __fadd_rn(grp[p + h], err);
                float qf = rintf(__fmul_rn(xv, inv));
                qf = fminf(fmaxf(qf, -8.0f), 7.0f);
                err = __fsub_rn(xv, __fmul_rn(qf, scale));
                nib[h] = ((int)qf + 8) & 15;
            }
            dst[p / 2] = (uint8_t)(nib[0] | (nib[1] << 4));
        }
    }
}

// ------------------------------------------------------------------ repack: reference layout -> tiles
// int4 nibbles: one thread per (row, 16-byte chunk).  Reference byte b holds element 2b (low) and
// 2b+1 (high); the device chunk's dword j byte i holds element 8j+i (low) and 8j+4+i (high).
__global__ void k_repack_nib(const uint8_t *__restrict__ src, int N, int K, uint32_t flip, uint8_t *__restrict__ dst) {
    int cpr = K / 32;
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long ntiles = (N + BGL_TILE - 1) / BGL_TILE;
    if (t >= ntiles * BGL_TILE * cpr) return;
    int r = (int)(t / cpr), c = (int)(t % cpr);
    uint32_t outw[4] = {0, 0, 0, 0};
    if (r < N) {
        const uint8_t *s = src + (size_t)r * (K / 2) + (size_t)c * 16;
        uint8_t b[16];
        for (int i = 0; i < 16; i++) b[i] = s[i];
        for (int j = 0; j < 4; j++)
            for (int i = 0; i < 4; i++) {
                int e0 = 8 * j + i, e1 = 8 * j + 4 + i;
                uint32_t n0 = (e0 & 1) ? (b[e0 >> 1] >> 4) : (b[e0 >> 1] & 15);
                uint32_t n1 = (e1 & 1) ? (b[e1 >> 1] >> 4) : (b[e1 >> 1] & 15);
                outw[j] |= (n0 | (n1 << 4)) << (8 * i);
            }
        for (int j = 0; j < 4; j++) outw[j] ^= flip;     // 0x88888888: signed-nibble layout (g256sf)
    }
    int tile = r / BGL_TILE, lane = r % BGL_TILE;
    uint4 *d = reinterpret_cast<uint4 *>(dst + (((size_t)tile * cpr + c) * BGL_TILE + lane) * 16);
    *d = make_uint4(outw[0], outw[1], outw[2], outw[3]);
}

// int8 codes: natural order, only the tiling changes.
__global__ void k_repack_q8(const int8_t *__restrict__ src, int N, int K, uint8_t *__restrict__ dst) {
    int cpr = K / 16;
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long ntiles = (N + BGL_TILE - 1) / BGL_TILE;
    if (t >= ntiles * BGL_TILE * cpr) return;
    int r = (int)(t / cpr), c = (int)(t % cpr);
    uint4 v = make_uint4(0, 0, 0, 0);
    if (r < N) v = *reinterpret_cast<const uint4 *>(src + (size_t)r * K + (size_t)c * 16);
    int tile = r / BGL_TILE, lane = r % BGL_TILE;
    *reinterpret_cast<uint4 *>(dst + (((size_t)tile * cpr + c) * BGL_TILE + lane) * 16) = v;
}

// qNg64 bit planes -> field chunks.  One thread per (row, pair of 64-groups).  Per pair (128
// elements) the device stores n chunks: the 8-bit field (8 chunks, element 16k+i in byte i of chunk
// k, stored as f ^ 0x80 i.e. f-128 as a signed byte), the 4-bit field (4 chunks, int4 device nibble
// order), the 2-bit field (2 chunks; dword j byte i crumb t = element 16j+4t+i of the 64-group) and
// the 1-bit field (1 chunk; dword j byte i bit t = element 32j+4t+i of the pair).  A missing second
// group (odd K/64) is padded with u = 0.
__global__ void k_repack_qng(const uint8_t *__restrict__ src, int N, int K, int n, uint8_t *__restrict__ dst) {
    int ng = K / 64, np = (ng + 1) / 2;
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long ntiles = (N + BGL_TILE - 1) / BGL_TILE;
    if (t >= ntiles * BGL_TILE * np) return;
    int r = (int)(t / np), pr = (int)(t % np);
    QngFields f = qng_fields(n);
    uint16_t u[128];
    for (int e = 0; e < 128; e++) u[e] = 0;
    if (r < N)
        for (int h = 0; h < 2; h++) {
            int g = 2 * pr + h;
            if (g >= ng) break;
            const uint8_t *grp = src + ((size_t)r * ng + g) * (size_t)n * 8;
            for (int p = 0; p < 64; p++) {
                uint32_t v = 0;
                for (int j = 0; j < n; j++) v |= (uint32_t)((grp[j * 8 + (p >> 3)] >> (p & 7)) & 1) << j;
                u[64 * h + p] = (uint16_t)v;
            }
        }
    int tile = r / BGL_TILE, lane = r % BGL_TILE;
    int cpr = np * n, c = pr * n;
    auto put = [&](int chunk, const uint32_t *wv) {
        uint4 *d = reinterpret_cast<uint4 *>(dst + (((size_t)tile * cpr + chunk) * BGL_TILE + lane) * 16);
        *d = make_uint4(wv[0], wv[1], wv[2], wv[3]);
    };
    uint32_t wv[4];
    if (f.has8)
        for (int k = 0; k < 8; k++, c++) {
            for (int j = 0; j < 4; j++) {
                wv[j] = 0;
                for (int i = 0; i < 4; i++) wv[j] |= (uint32_t)(((u[16 * k + 4 * j + i]) & 255) ^ 0x80) << (8 * i);
            }
            put(c, wv);
        }
    if (f.has4)
        for (int k = 0; k < 4; k++, c++) {
            for (int j = 0; j < 4; j++) {
                wv[j] = 0;
                for (int i = 0; i < 4; i++) {
                    uint32_t lo = (u[32 * k + 8 * j + i] >> f.sh4) & 15, hi = (u[32 * k + 8 * j + 4 + i] >> f.sh4) & 15;
                    wv[j] |= (lo | (hi << 4)) << (8 * i);
                }
            }
            put(c, wv);
        }
    if (f.has2)
        for (int k = 0; k < 2; k++, c++) {
            for (int j = 0; j < 4; j++) {
                wv[j] = 0;
                for (int i = 0; i < 4; i++)
                    for (int q = 0; q < 4; q++)
                        wv[j] |= (uint32_t)((u[64 * k + 16 * j + 4 * q + i] >> f.sh2) & 3) << (8 * i + 2 * q);
            }
            put(c, wv);
        }
    if (f.has1) {
        for (int j = 0; j < 4; j++) {
            wv[j] = 0;
            for (int i = 0; i < 4; i++)
                for (int q = 0; q < 8; q++)
                    wv[j] |= (uint32_t)((u[32 * j + 4 * q + i] >> f.sh1) & 1) << (8 * i + q);
        }
        put(c, wv);
        c++;
    }
}

// Per-(row, unit) scalars [N][U] (32-bit words) -> [tile][U][lane]; padded rows get 0.
__global__ void k_repack_u32(const uint32_t *__restrict__ src, int N, int U, uint32_t *__restrict__ dst) {
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long ntiles = (N + BGL_TILE - 1) / BGL_TILE;
    if (t >= ntiles * BGL_TILE * U) return;
    int r = (int)(t / U), u = (int)(t % U);
    int tile = r / BGL_TILE, lane = r % BGL_TILE;
    dst[((size_t)tile * U + u) * BGL_TILE + lane] = r < N ? src[(size_t)r * U + u] : 0u;
}

// Two per-(row, unit) u32 arrays [N][U] -> one 8-byte word per unit in the tile layout
// [tile][u][lane] (x from a, y from b): the g256sf wsuper and its four sub-codes travel together.
__global__ void k_repack_zip_u32(const uint32_t *__restrict__ a, const uint32_t *__restrict__ b, int N, int U,
                                 uint2 *__restrict__ dst) {
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long ntiles = (N + BGL_TILE - 1) / BGL_TILE;
    if (t >= ntiles * BGL_TILE * U) return;
    int r = (int)(t / U), u = (int)(t % U);
    int tile = r / BGL_TILE, lane = r % BGL_TILE;
    const size_t i = (size_t)r * U + u;
    dst[((size_t)tile * U + u) * BGL_TILE + lane] = r < N ? make_uint2(a[i], b[i]) : make_uint2(0u, 0u);
}

// Per-(row, unit) pairs of 16-bit fp16 scales or 8-byte float pairs, and 4 sub-codes -> one word.
__global__ void k_repack_u64(const uint64_t *__restrict__ src, int N, int U, uint64_t *__restrict__ dst) {
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long ntiles = (N + BGL_TILE - 1) / BGL_TILE;
    if (t >= ntiles * BGL_TILE * U) return;
    int r = (int)(t / U), u = (int)(t % U);
    int tile = r / BGL_TILE, lane = r % BGL_TILE;
    dst[((size_t)tile * U + u) * BGL_TILE + lane] = r < N ? src[(size_t)r * U + u] : 0ull;
}

// Mixed per-cell qNg64 (MixedQNg64Tensor, mlx_moe.cpp:87-93) -> the dense width-W plane layout
// (qng64_dense.c:19-27): one thread per (row, 64-group) cell.  A cell holds n = bits[cell] planes of
// 8 bytes at planes + offsets[cell] (plane j: bit j of element p at byte p>>3, bit p&7, i.e. bit p of
// the little-endian u64) and decodes to (u - 2^(n-1)) * scale (mlx_moe.cpp:1708-1722).  Re-biasing
// u' = u + 2^(W-1) - 2^(n-1) keeps every code (u' - 2^(W-1) = u - 2^(n-1)); the add runs bit-sliced
// over the 64 elements, one u64 per plane.
__global__ void k_mixed_qng_to_dense(const uint8_t *__restrict__ planes, const uint32_t *__restrict__ offsets,
                                     const uint8_t *__restrict__ bits, long cells, int W, uint8_t *__restrict__ dst) {
    const long cell = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (cell >= cells) return;
    const int n = bits[cell];
    const uint64_t *src = reinterpret_cast<const uint64_t *>(planes + offsets[cell]);   // offsets are multiples of 8
    uint64_t *out = reinterpret_cast<uint64_t *>(dst + (size_t)cell * W * 8);
    const uint32_t D = (1u << (W - 1)) - (1u << (n - 1));
    uint64_t carry = 0;
    for (int j = 0; j < W; j++) {
        const uint64_t a = j < n ? src[j] : 0ull, d = ((D >> j) & 1u) ? ~0ull : 0ull;
        out[j] = a ^ d ^ carry;
        carry = (a & d) | (carry & (a ^ d));
    }
}

// qNg64 scales [N][ng] fp32 -> [tile][pair][lane] float2 (odd ng: second scale 0).
__global__ void k_repack_qng_scales(const float *__restrict__ src, int N, int ng, float2 *__restrict__ dst) {
    int np = (ng + 1) / 2;
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long ntiles = (N + BGL_TILE - 1) / BGL_TILE;
    if (t >= ntiles * BGL_TILE * np) return;
    int r = (int)(t / np), p = (int)(t % np);
    int tile = r / BGL_TILE, lane = r % BGL_TILE;
    float a = 0.0f, b = 0.0f;
    if (r < N) {
        a = src[(size_t)r * ng + 2 * p];
        if (2 * p + 1 < ng) b = src[(size_t)r * ng + 2 * p + 1];
    }
    dst[((size_t)tile * np + p) * BGL_TILE + lane] = make_float2(a, b);
}

// ------------------------------------------------------------------ dequant probe (tiled layout)
// Decodes rows [row0, row0+nrows) of a bound tensor straight from the device layout, one thread
// per element -- the device analogue of moe_decode_af (qwen_infer.c:2554-2655) used to prove that
// the repacked layout decodes bit-exactly.
__global__ void k_dequant(BglDevTensor T, int row0, int nrows, float *__restrict__ out) {
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long)nrows * T.K) return;
    out[t] = w_at(T, row0 + (int)(t / T.K), (int)(t % T.K));
}
