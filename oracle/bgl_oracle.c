/* bgl_oracle.c -- CPU oracle (TEST INFRASTRUCTURE ONLY; see bgl_oracle.h).
 *
 * Plain-C restatement of the reference's packers, decoders and GEMV / MoE arithmetic.
 * Compiled with -ffp-contract=off: each fp32 expression below rounds exactly as written.
 * Where the reference relies on a closed vendor routine (Accelerate vDSP_dotpr in
 * q4gemv.h:82/165/533) the oracle sums in double (the "brute force" reading); callers
 * compare GPU output against it with a relative tolerance, never for bit equality.
 */
#include "bgl_oracle.h"
#include <math.h>
#include <string.h>
#include <stdlib.h>

#define G64 64

/* ============================ IEEE binary16 ============================
 * The reference converts with the compiler's __fp16 (gguf_write_quants.c:19-23,
 * gguf_quants.c:96-101): IEEE round-to-nearest-even.  Restated bit by bit here because
 * gcc 11 on x86 has no half type.  Pinned exhaustively against numpy float16 in tests. */
uint16_t or_f32_to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                                  /* inf / nan */
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);    /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                    /* below 2^-14: subnormal half */
        if (ax < 0x33000000u) return (uint16_t)sign;           /* < 2^-25 rounds to 0 */
        uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t sh = 126u - e;                                /* 14..24 */
        uint32_t q = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = ax - 0x38000000u;                             /* rebias 127 -> 15 */
    uint32_t q = r >> 13, rem = r & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu, out;
    if (e == 0) {
        if (m == 0) out = sign;
        else {                                                 /* subnormal: m * 2^-24 */
            float v = (float)m * 5.9604644775390625e-08f;
            memcpy(&out, &v, 4); out |= sign;
        }
    } else if (e == 31) out = sign | 0x7f800000u | (m << 13);
    else out = sign | ((e + 112u) << 23) | (m << 13);
    float f; memcpy(&f, &out, 4); return f;
}

/* ============================ packers ============================ */

/* gguf_transcode.c:24-68 (gguf_quantize_q4g64_error_feedback): per (row, g64) s = maxabs/7
 * (1.0 if < 1e-12); reciprocal + rintf; clamp [-8,7]; error feedback within the group;
 * nibble = code+8, low nibble = even column, high nibble = odd column. */
void or_quantize_q4g64_ef(const float *w, int out, int in, uint8_t *packed, float *scales) {
    int ng = in / G64;
    for (int r = 0; r < out; r++) {
        const float *row = w + (size_t)r * in;
        uint8_t *prow = packed + (size_t)r * (in / 2);
        float *srow = scales + (size_t)r * ng;
        for (int g = 0; g < ng; g++) {
            const float *grp = row + (size_t)g * G64;
            float maxabs = 0.0f;
            for (int p = 0; p < G64; p++) { float a = fabsf(grp[p]); if (a > maxabs) maxabs = a; }
            float scale = maxabs / 7.0f;
            if (scale < 1e-12f) scale = 1.0f;
            srow[g] = scale;
            float inv = 1.0f / scale, err = 0.0f;
            for (int p = 0; p < G64; p++) {
                float x = grp[p] + err;
                float qf = rintf(x * inv);
                if (qf > 7.0f) qf = 7.0f;
                if (qf < -8.0f) qf = -8.0f;
                float deq = qf * scale;
                err = x - deq;
                int nib = ((int)qf + 8) & 0x0F, idx = g * G64 + p;
                if ((idx & 1) == 0) prow[idx / 2] = (uint8_t)nib;
                else prow[idx / 2] = (uint8_t)(prow[idx / 2] | (nib << 4));
            }
        }
    }
}

/* gguf_transcode.c:70-101 (gguf_quantize_q8g64): s = maxabs/127 (1.0 if < 1e-12); DIRECT
 * division w/s (no reciprocal), rintf, clamp [-127,127], no error feedback. */
void or_quantize_q8g64(const float *w, int out, int in, int8_t *codes, float *scales) {
    int ng = in / G64;
    for (int r = 0; r < out; r++) {
        const float *row = w + (size_t)r * in;
        int8_t *crow = codes + (size_t)r * in;
        float *srow = scales + (size_t)r * ng;
        for (int g = 0; g < ng; g++) {
            const float *grp = row + (size_t)g * G64;
            float maxabs = 0.0f;
            for (int p = 0; p < G64; p++) { float a = fabsf(grp[p]); if (a > maxabs) maxabs = a; }
            float scale = maxabs / 127.0f;
            if (scale < 1e-12f) scale = 1.0f;
            srow[g] = scale;
            for (int p = 0; p < G64; p++) {
                float qf = rintf(grp[p] / scale);
                if (qf > 127.0f) qf = 127.0f;
                if (qf < -127.0f) qf = -127.0f;
                crow[g * G64 + p] = (int8_t)qf;
            }
        }
    }
}

size_t or_qng64_group_bytes(int n) { return (n >= 2 && n <= 15) ? (size_t)n * 8 : 0; }

static void qng64_set_code(uint8_t *grp, int n, int p, unsigned u) {
    for (int j = 0; j < n; j++)
        if ((u >> j) & 1u) grp[(size_t)j * 8 + (p >> 3)] |= (uint8_t)(1u << (p & 7));
}

/* gguf_transcode.c:108-162 (gguf_quantize_qNg64): q4g64's loop with qmax = 2^(n-1)-1,
 * clamp [-2^(n-1), qmax], bias-then-extract bit planes (plane j = bit j of u = code + 2^(n-1),
 * element p -> byte p>>3, bit p&7 of each 8-byte plane, gguf_transcode.h:217-235).  No n gate. */
void or_quantize_qng64_gguf(const float *w, int out, int in, int n, uint8_t *planes, float *scales) {
    int ng = in / G64, qmax = (1 << (n - 1)) - 1, qmin = -(1 << (n - 1)), bias = 1 << (n - 1);
    int mask = (1 << n) - 1;
    size_t gb = (size_t)n * 8, rb = (size_t)ng * gb;
    for (int r = 0; r < out; r++) {
        const float *row = w + (size_t)r * in;
        for (int g = 0; g < ng; g++) {
            const float *grp = row + (size_t)g * G64;
            uint8_t *pg = planes + (size_t)r * rb + (size_t)g * gb;
            memset(pg, 0, gb);
            float maxabs = 0.0f;
            for (int p = 0; p < G64; p++) { float a = fabsf(grp[p]); if (a > maxabs) maxabs = a; }
            float scale = maxabs / (float)qmax;
            if (scale < 1e-12f) scale = 1.0f;
            scales[(size_t)r * ng + g] = scale;
            float inv = 1.0f / scale, err = 0.0f;
            for (int p = 0; p < G64; p++) {
                float x = grp[p] + err;
                float qf = rintf(x * inv);
                if (qf > (float)qmax) qf = (float)qmax;
                if (qf < (float)qmin) qf = (float)qmin;
                float deq = qf * scale;
                err = x - deq;
                qng64_set_code(pg, n, p, (unsigned)(((int)qf + bias) & mask));
            }
        }
    }
}

/* qng64_dense.c:29-68 (qng64_quantize_f32): rejects n=4 (qng64_dense.c:9); scale = maxabs >
 * 1e-12 ? maxabs/qmax : 1 (a different floor test than gguf_quantize_qNg64); lrintf; err computed
 * as v - (float)qi*scale in one (non-contracted) expression. */
int or_quantize_qng64_dense(const float *w, int out, int in, int n, uint8_t *planes, float *scales) {
    if (!w || !planes || !scales || out <= 0 || in <= 0 || (in % G64) || n < 2 || n > 15 || n == 4) return -1;
    int ng = in / G64, qmax = (1 << (n - 1)) - 1, qmin = -(1 << (n - 1)), bias = 1 << (n - 1);
    size_t gb = (size_t)n * 8;
    memset(planes, 0, (size_t)out * ng * gb);
    for (int r = 0; r < out; r++)
        for (int g = 0; g < ng; g++) {
            const float *grp = w + (size_t)r * in + (size_t)g * G64;
            float maxabs = 0.0f;
            for (int p = 0; p < G64; p++) { float a = fabsf(grp[p]); if (a > maxabs) maxabs = a; }
            float scale = maxabs > 1e-12f ? maxabs / (float)qmax : 1.0f;
            float inv = 1.0f / scale;
            scales[(size_t)r * ng + g] = scale;
            uint8_t *dst = planes + ((size_t)r * ng + g) * gb;
            float err = 0.0f;
            for (int p = 0; p < G64; p++) {
                float v = grp[p] + err;
                long qi = lrintf(v * inv);
                if (qi > qmax) qi = qmax;
                if (qi < qmin) qi = qmin;
                err = v - (float)qi * scale;
                unsigned u = ((unsigned)((int)qi + bias)) & ((1u << n) - 1u);
                qng64_set_code(dst, n, p, u);
            }
        }
    return 0;
}

/* gguf_write_quants.c:34-62 (gguf_w_quantize_q4_0): 32-element blocks {fp16 d; 16 B qs}.
 * The loop quantizes with the fp32 scale s = maxabs/7 and stores d = fp16(s); byte j holds
 * element j (low nibble) and element j+16 (high nibble). */
void or_quantize_q4_0(const float *w, int64_t n, uint8_t *blocks) {
    int64_t nb = n / 32;
    for (int64_t b = 0; b < nb; b++) {
        const float *grp = w + b * 32;
        uint8_t *blk = blocks + b * 18;
        float maxabs = 0.0f;
        for (int p = 0; p < 32; p++) { float a = fabsf(grp[p]); if (a > maxabs) maxabs = a; }
        float scale = maxabs / 7.0f;
        if (scale < 1e-12f) scale = 1.0f;
        uint16_t d = or_f32_to_f16(scale);
        blk[0] = (uint8_t)(d & 0xff); blk[1] = (uint8_t)(d >> 8);
        float inv = 1.0f / scale, err = 0.0f;
        int8_t codes[32];
        for (int p = 0; p < 32; p++) {
            float x = grp[p] + err;
            float qf = rintf(x * inv);
            if (qf > 7.0f) qf = 7.0f;
            if (qf < -8.0f) qf = -8.0f;
            float deq = qf * scale;
            err = x - deq;
            codes[p] = (int8_t)qf;
        }
        for (int j = 0; j < 16; j++) {
            uint8_t lo = (uint8_t)((codes[j] + 8) & 0x0F), hi = (uint8_t)((codes[j + 16] + 8) & 0x0F);
            blk[2 + j] = (uint8_t)(lo | (hi << 4));
        }
    }
}

/* Q4G32H (build-defined format, no reference kernel): the Q4_0 block's codes and fp16 scale,
 * re-paired into q4gemv's nibble convention (q4gemv.h:6-8: byte b low = element 2b,
 * high = element 2b+1).  A lossless permutation of the Q4_0 bytes (gguf_quants.c:118-130). */
void or_q4_0_to_q4g32h(const uint8_t *blocks, int out, int in, uint8_t *packed, uint16_t *scales16) {
    int nb = in / 32;
    for (int r = 0; r < out; r++)
        for (int b = 0; b < nb; b++) {
            const uint8_t *blk = blocks + ((size_t)r * nb + b) * 18;
            scales16[(size_t)r * nb + b] = (uint16_t)(blk[0] | (blk[1] << 8));
            uint8_t nib[32];
            for (int j = 0; j < 16; j++) { nib[j] = blk[2 + j] & 0x0F; nib[j + 16] = blk[2 + j] >> 4; }
            uint8_t *dst = packed + (size_t)r * (in / 2) + (size_t)b * 16;
            for (int j = 0; j < 16; j++) dst[j] = (uint8_t)(nib[2 * j] | (nib[2 * j + 1] << 4));
        }
}

void or_quantize_q4g32h(const float *w, int out, int in, uint8_t *packed, uint16_t *scales16) {
    size_t nblk = (size_t)out * (in / 32);
    uint8_t *blocks = (uint8_t *)malloc(nblk * 18);
    or_quantize_q4_0(w, (int64_t)out * in, blocks);
    or_q4_0_to_q4g32h(blocks, out, in, packed, scales16);
    free(blocks);
}

/* q4g256sf packer -- BUILD-DEFINED.  The reference ships only the format (q4gemv_g256.h:31-38:
 * effective per-64 scale = wsuper * sub/63, sub in [0,63]) and the kernel; its offline emitter is
 * not in the tree.  This packer: s64 = maxabs/7 per 64-subgroup, wsuper = max s64 over the 4
 * subgroups (1.0 if < 1e-12), sub = clamp(ceil(63*s64/wsuper), 1, 63), then the q4g64 error-feedback
 * quantizer (gguf_transcode.c:24-68 arithmetic) run with the effective scale wsuper*(sub/63). */
void or_quantize_g256sf(const float *w, int out, int in, uint8_t *packed, float *wsuper, uint8_t *sub) {
    int ng256 = in / 256, ng64 = in / 64;
    for (int r = 0; r < out; r++) {
        const float *row = w + (size_t)r * in;
        uint8_t *prow = packed + (size_t)r * (in / 2);
        for (int gs = 0; gs < ng256; gs++) {
            float s64[4], ws = 0.0f;
            for (int k = 0; k < 4; k++) {
                const float *grp = row + (size_t)(gs * 4 + k) * G64;
                float maxabs = 0.0f;
                for (int p = 0; p < G64; p++) { float a = fabsf(grp[p]); if (a > maxabs) maxabs = a; }
                s64[k] = maxabs / 7.0f;
                if (s64[k] > ws) ws = s64[k];
            }
            if (ws < 1e-12f) ws = 1.0f;
            wsuper[(size_t)r * ng256 + gs] = ws;
            for (int k = 0; k < 4; k++) {
                int g = gs * 4 + k;
                int sc = (int)ceilf(63.0f * s64[k] / ws);
                if (sc < 1) sc = 1;
                if (sc > 63) sc = 63;
                sub[(size_t)r * ng64 + g] = (uint8_t)sc;
                float scale = ws * ((float)sc / 63.0f);
                float inv = 1.0f / scale, err = 0.0f;
                const float *grp = row + (size_t)g * G64;
                for (int p = 0; p < G64; p++) {
                    float x = grp[p] + err;
                    float qf = rintf(x * inv);
                    if (qf > 7.0f) qf = 7.0f;
                    if (qf < -8.0f) qf = -8.0f;
                    float deq = qf * scale;
                    err = x - deq;
                    int nib = ((int)qf + 8) & 0x0F, idx = g * G64 + p;
                    if ((idx & 1) == 0) prow[idx / 2] = (uint8_t)nib;
                    else prow[idx / 2] = (uint8_t)(prow[idx / 2] | (nib << 4));
                }
            }
        }
    }
}

/* ============================ decoders ============================ */

/* q4gemv.h:40-73 (q4_unpack_row): value = (float)(nib-8) * s[row, col/64]. */
void or_decode_q4g64(const uint8_t *packed, const float *scales, int out, int in, float *w) {
    int ng = in / G64;
    for (int r = 0; r < out; r++)
        for (int c = 0; c < in; c++) {
            uint8_t b = packed[(size_t)r * (in / 2) + c / 2];
            int nib = (c & 1) ? (b >> 4) : (b & 0x0F);
            w[(size_t)r * in + c] = (float)(nib - 8) * scales[(size_t)r * ng + c / G64];
        }
}

/* q4gemv.h:140-156 (q8_unpack_row): value = (float)code * s. */
void or_decode_q8g64(const int8_t *codes, const float *scales, int out, int in, float *w) {
    int ng = in / G64;
    for (int r = 0; r < out; r++)
        for (int c = 0; c < in; c++)
            w[(size_t)r * in + c] = (float)codes[(size_t)r * in + c] * scales[(size_t)r * ng + c / G64];
}

/* qng64_dense.c:19-27 (qng64_decode_code). */
float or_qng64_decode_code(const uint8_t *group, int n, int index) {
    if (!group || !or_qng64_group_bytes(n) || index < 0 || index >= G64) return 0.0f;
    int u = 0;
    for (int j = 0; j < n; ++j)
        if ((group[(size_t)j * 8 + (index >> 3)] >> (index & 7)) & 1u) u |= 1 << j;
    return (float)(u - (1 << (n - 1)));
}

/* qng64_dense.c:94-96: value = decode_code * scale (fp32 product). */
void or_decode_qng64(const uint8_t *planes, const float *scales, int n, int out, int in, float *w) {
    int ng = in / G64;
    size_t gb = (size_t)n * 8;
    for (int r = 0; r < out; r++)
        for (int c = 0; c < in; c++) {
            const uint8_t *grp = planes + ((size_t)r * ng + c / G64) * gb;
            w[(size_t)r * in + c] = or_qng64_decode_code(grp, n, c % G64) * scales[(size_t)r * ng + c / G64];
        }
}

/* gguf_quants.c:118-130 (dequant_row_q4_0): y = (nib-8) * fp32(d), split-half nibbles. */
void or_decode_q4_0(const uint8_t *blocks, int64_t n, float *w) {
    int64_t nb = n / 32;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *blk = blocks + i * 18;
        float d = or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int j = 0; j < 16; j++) {
            int x0 = (blk[2 + j] & 0x0F) - 8, x1 = (blk[2 + j] >> 4) - 8;
            w[i * 32 + j] = x0 * d;
            w[i * 32 + j + 16] = x1 * d;
        }
    }
}

/* Q4G32H decode = dequant_row_q4_0's value on the re-paired nibbles: (nib-8) * fp32(d). */
void or_decode_q4g32h(const uint8_t *packed, const uint16_t *scales16, int out, int in, float *w) {
    int nb = in / 32;
    for (int r = 0; r < out; r++)
        for (int c = 0; c < in; c++) {
            uint8_t b = packed[(size_t)r * (in / 2) + c / 2];
            int nib = (c & 1) ? (b >> 4) : (b & 0x0F);
            w[(size_t)r * in + c] = (nib - 8) * or_f16_to_f32(scales16[(size_t)r * nb + c / 32]);
        }
}

/* q4gemv_g256.h:31-38 (D2): effective per-64 scale = wsuper * (sub / 63.0f); value = (nib-8)*that. */
void or_decode_g256sf(const uint8_t *packed, const float *wsuper, const uint8_t *sub, int out, int in, float *w) {
    int ng256 = in / 256, ng64 = in / 64;
    for (int r = 0; r < out; r++)
        for (int c = 0; c < in; c++) {
            uint8_t b = packed[(size_t)r * (in / 2) + c / 2];
            int nib = (c & 1) ? (b >> 4) : (b & 0x0F);
            float s = wsuper[(size_t)r * ng256 + c / 256] * ((float)sub[(size_t)r * ng64 + c / 64] / 63.0f);
            w[(size_t)r * in + c] = (float)(nib - 8) * s;
        }
}

/* ============================ fp32-activation GEMV ============================ */

/* qng64_dense.c:81-100 (qng64_matvec_f32), restated exactly: double sum = bias; sum +=
 * (double)(decode*scale) * x; y = (float)sum. */
void or_qng64_matvec_f32(const uint8_t *planes, const float *scales, int n, const float *x,
                         const float *bias, float *y, int out, int in) {
    int ng = in / G64;
    size_t gb = (size_t)n * 8;
    for (int r = 0; r < out; r++) {
        double sum = bias ? bias[r] : 0.0;
        for (int g = 0; g < ng; g++) {
            const uint8_t *grp = planes + ((size_t)r * ng + g) * gb;
            float scale = scales[(size_t)r * ng + g];
            const float *xg = x + g * G64;
            for (int p = 0; p < G64; p++)
                sum += (double)(or_qng64_decode_code(grp, n, p) * scale) * xg[p];
        }
        y[r] = (float)sum;
    }
}

/* q4gemv.h:75-85 / 158-168 / 761-769 (gemv_q4g64, gemv_q8g64, gemm_qXg64_mt): decode the row to
 * fp32 then vDSP_dotpr; y = bias + dot.  vDSP's summation order is closed, so the dot is taken in
 * double here.  qNg64 (matmul_t -> qng64_matmul_f32, qwen_infer.c:1612-1613) uses the exact
 * restatement above; Q4G32H decodes per dequant_row_q4_0 and sums like q4g64. */
void or_gemm_f32(int kind, int bits, const void *packed, const void *scales,
                 const float *x, const float *bias, float *y, int out, int in, int M) {
    if (kind == 4) {
        for (int m = 0; m < M; m++)
            or_qng64_matvec_f32((const uint8_t *)packed, (const float *)scales, bits,
                                x + (size_t)m * in, bias, y + (size_t)m * out, out, in);
        return;
    }
    float *row = (float *)malloc(sizeof(float) * (size_t)in);
    for (int r = 0; r < out; r++) {
        if (kind == 1)
            or_decode_q4g64((const uint8_t *)packed + (size_t)r * (in / 2), (const float *)scales + (size_t)r * (in / 64), 1, in, row);
        else if (kind == 2)
            or_decode_q8g64((const int8_t *)packed + (size_t)r * in, (const float *)scales + (size_t)r * (in / 64), 1, in, row);
        else
            or_decode_q4g32h((const uint8_t *)packed + (size_t)r * (in / 2), (const uint16_t *)scales + (size_t)r * (in / 32), 1, in, row);
        float b = bias ? bias[r] : 0.0f;
        for (int m = 0; m < M; m++) {
            const float *xm = x + (size_t)m * in;
            double dot = 0.0;
            for (int c = 0; c < in; c++) dot += (double)row[c] * xm[c];
            y[(size_t)m * out + r] = b + (float)dot;
        }
    }
    free(row);
}

/* ============================ W4A8 / W8A8 ============================ */

/* AArch64 FMAX (vmaxq_f32 / vmaxvq_f32): a NaN operand gives NaN; otherwise the larger value. */
static float or_fmax_nan(float a, float b) {
    if (isnan(a) || isnan(b)) return NAN;
    return a > b ? a : b;
}

/* AArch64 FCVTZS to int32 (vcvtq_s32_f32): toward zero, NaN -> 0, out of range saturates. */
static int32_t or_fcvtzs(float t) {
    if (isnan(t)) return 0;
    if (t >= 2147483648.0f) return INT32_MAX;
    if (t <= -2147483648.0f) return INT32_MIN;
    return (int32_t)t;
}

/* q4gemv.h:177-213 (q4_quant_act_i8) and q4gemv_g256.h:72-99 (q4_quant_act_i8_g256):
 * mx = FMAX(1e-8, |x|...); sc = mx/127; inv = 1/sc; q = sat8(FCVTZS(x*inv +/- 0.5))
 * (round half away from zero, saturating narrow through int16).
 * Non-finite groups follow the NEON instructions: FMAX carries a NaN into mx, so a group holding a
 * NaN gets sc = NaN, inv = NaN, every x*inv NaN and every code FCVTZS(NaN) = 0; a group holding
 * +-Inf (and no NaN) gets mx = +Inf, sc = +Inf, inv = 0, x*inv = +-0 (NaN at the Inf) and again
 * every code 0.  The fold then multiplies 0 by a NaN or +Inf scale: every output row is NaN. */
void or_quant_act_i8(const float *x, int in, int gsize, int8_t *xq, float *ascale) {
    int ng = in / gsize;
    for (int gi = 0; gi < ng; gi++) {
        const float *xp = x + (size_t)gi * gsize;
        float mx = 1e-8f;
        for (int b = 0; b < gsize; b++) mx = or_fmax_nan(mx, fabsf(xp[b]));
        float sc = mx / 127.0f, inv = 1.0f / sc;
        ascale[gi] = sc;
        for (int b = 0; b < gsize; b++) {
            float p = xp[b] * inv;
            float t = p + (p >= 0.0f ? 0.5f : -0.5f);       /* vcgeq(NaN, 0) is false: NaN - 0.5 */
            int32_t q = or_fcvtzs(t);
            if (q > 127) q = 127;                             /* vqmovn_s32 then vqmovn_s16 */
            if (q < -128) q = -128;
            xq[(size_t)gi * gsize + b] = (int8_t)q;
        }
    }
}

/* q4gemv.h:226-244 (q4_dot_sdot_row) and :313-339 (batched, bit-identical per column):
 * per g64 isum = sum (nib-8)*xq exactly; acc += (float)isum * ws * as, groups ascending. */
void or_gemm_q4g64_sdot(const uint8_t *packed, const float *wscale, const int8_t *xq, const float *ascale,
                        const float *bias, float *y, int out, int in, int M) {
    int ng = in / G64;
    for (int r = 0; r < out; r++) {
        const uint8_t *pr = packed + (size_t)r * (in / 2);
        const float *ws = wscale + (size_t)r * ng;
        float b = bias ? bias[r] : 0.0f;
        for (int m = 0; m < M; m++) {
            const int8_t *xm = xq + (size_t)m * in;
            const float *am = ascale + (size_t)m * ng;
            float acc = 0.0f;
            for (int g = 0; g < ng; g++) {
                int32_t isum = 0;
                for (int p = 0; p < G64; p++) {
                    int c = g * G64 + p;
                    int nib = (c & 1) ? (pr[c / 2] >> 4) : (pr[c / 2] & 0x0F);
                    isum += (nib - 8) * (int32_t)xm[c];
                }
                acc += (float)isum * ws[g] * am[g];
            }
            y[(size_t)m * out + r] = b + acc;
        }
    }
}

/* q4gemv.h:247-258 (q8_dot_sdot_row) and :344-364 (batched). */
void or_gemm_q8g64_sdot(const int8_t *codes, const float *wscale, const int8_t *xq, const float *ascale,
                        const float *bias, float *y, int out, int in, int M) {
    int ng = in / G64;
    for (int r = 0; r < out; r++) {
        const int8_t *pr = codes + (size_t)r * in;
        const float *ws = wscale + (size_t)r * ng;
        float b = bias ? bias[r] : 0.0f;
        for (int m = 0; m < M; m++) {
            const int8_t *xm = xq + (size_t)m * in;
            const float *am = ascale + (size_t)m * ng;
            float acc = 0.0f;
            for (int g = 0; g < ng; g++) {
                int32_t isum = 0;
                for (int p = 0; p < G64; p++) isum += (int32_t)pr[g * G64 + p] * (int32_t)xm[g * G64 + p];
                acc += (float)isum * ws[g] * am[g];
            }
            y[(size_t)m * out + r] = b + acc;
        }
    }
}

/* q4gemv_g256.h:134-157 (q4_dot_sdot_row_g256sf_v) and :230-262 (batched V-form): per 256
 * combined = sum_sub isum64 * sub_code (exact int32); acc += (float)combined * wsuper * (1/63) * as. */
void or_gemm_g256sf_sdot(const uint8_t *packed, const float *wsuper, const uint8_t *sub,
                         const int8_t *xq, const float *ascale, const float *bias, float *y,
                         int out, int in, int M) {
    int ng256 = in / 256, ng64 = in / 64;
    for (int r = 0; r < out; r++) {
        const uint8_t *pr = packed + (size_t)r * (in / 2);
        float b = bias ? bias[r] : 0.0f;
        for (int m = 0; m < M; m++) {
            const int8_t *xm = xq + (size_t)m * in;
            const float *am = ascale + (size_t)m * ng256;
            float acc = 0.0f;
            for (int gs = 0; gs < ng256; gs++) {
                int32_t combined = 0;
                for (int s = 0; s < 4; s++) {
                    int g = gs * 4 + s;
                    int32_t isum = 0;
                    for (int p = 0; p < G64; p++) {
                        int c = g * G64 + p;
                        int nib = (c & 1) ? (pr[c / 2] >> 4) : (pr[c / 2] & 0x0F);
                        isum += (nib - 8) * (int32_t)xm[c];
                    }
                    combined += isum * (int32_t)sub[(size_t)r * ng64 + g];
                }
                acc += (float)combined * wsuper[(size_t)r * ng256 + gs] * (1.0f / 63.0f) * am[gs];
            }
            y[(size_t)m * out + r] = b + acc;
        }
    }
}

/* q4gemv_g256.h:102-130 (q4_dot_sdot_row_g256plain) and :196-220 (batched): the plain-g256
 * diagnostic, one fp32 scale per 256 weights and no sub-codes: per 256 the exact int32 sum of
 * (nib - 8) * xq, then acc += (float)sum * wscale256 * ascale256, left to right. */
void or_gemm_g256plain_sdot(const uint8_t *packed, const float *wscale, const int8_t *xq, const float *ascale,
                            const float *bias, float *y, int out, int in, int M) {
    int ng256 = in / 256;
    for (int r = 0; r < out; r++) {
        const uint8_t *pr = packed + (size_t)r * (in / 2);
        float b = bias ? bias[r] : 0.0f;
        for (int m = 0; m < M; m++) {
            const int8_t *xm = xq + (size_t)m * in;
            const float *am = ascale + (size_t)m * ng256;
            float acc = 0.0f;
            for (int gs = 0; gs < ng256; gs++) {
                int32_t sum = 0;
                for (int c = gs * 256; c < gs * 256 + 256; c++) {
                    int nib = (c & 1) ? (pr[c / 2] >> 4) : (pr[c / 2] & 0x0F);
                    sum += (nib - 8) * (int32_t)xm[c];
                }
                acc += (float)sum * wscale[(size_t)r * ng256 + gs] * am[gs];
            }
            y[(size_t)m * out + r] = b + acc;
        }
    }
}

void or_matmul_sdot(int kind, const void *packed, const float *scales, const uint8_t *sub,
                    const float *x, const float *bias, float *y, int out, int in, int M) {
    int gsize = (kind == 3 || kind == 10) ? 256 : 64, ng = in / gsize;
    int8_t *xq = (int8_t *)malloc((size_t)M * in);
    float *as = (float *)malloc(sizeof(float) * (size_t)M * ng);
    for (int m = 0; m < M; m++) or_quant_act_i8(x + (size_t)m * in, in, gsize, xq + (size_t)m * in, as + (size_t)m * ng);
    if (kind == 1) or_gemm_q4g64_sdot((const uint8_t *)packed, scales, xq, as, bias, y, out, in, M);
    else if (kind == 2) or_gemm_q8g64_sdot((const int8_t *)packed, scales, xq, as, bias, y, out, in, M);
    else if (kind == 10) or_gemm_g256plain_sdot((const uint8_t *)packed, scales, xq, as, bias, y, out, in, M);
    else or_gemm_g256sf_sdot((const uint8_t *)packed, scales, sub, xq, as, bias, y, out, in, M);
    free(xq); free(as);
}

/* ============================ MoE ============================ */

/* qwen_infer.c:2668-2801 (moe_matvec_af_row): one (expert,row) dot, double accumulation,
 * columns left to right; the per-format weight value is the fp32 decode (q4 sym:
 * ((float)nib - 8.0f) * scale; int8: (float)code * scale; qNg64: (float)(u - 2^(n-1)) * scale).
 * Q4G32H has no MoE decoder in the reference; its value is dequant_row_q4_0's. */
/* MXFP4 (gguf_quants.c:284-312): E2M1 values doubled, and the E8M0 exponent byte as 2^(b-128)
 * (b < 2: the subnormal bit patterns 2^-128, 2^-127). */
static const int8_t or_mx_values[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
float or_mx_scale(uint8_t b) {
    uint32_t bits = b < 2 ? 0x00200000u << b : (uint32_t)(b - 1) << 23;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
int or_mx_value(int code) { return or_mx_values[code & 15]; }

double or_moe_row(const or_expert *w, int in, long row, const float *x) {
    int ng = in / G64;
    double acc = 0.0;
    if (w->kind == 9) {                        /* MXFP4 arm, qwen_infer.c:2702-2725 */
        const long rb = (long)(in / 32) * 17;
        const uint8_t *pr = (const uint8_t *)w->packed + (size_t)row * rb;
        for (long b = 0; b < in / 32; b++) {
            const uint8_t *blk = pr + b * 17;
            float scale = or_mx_scale(blk[0]);
            long c0 = b * 32;
            for (int j = 0; j < 16; j++) {
                float w0 = (float)or_mx_value(blk[1 + j] & 15) * scale, w1 = (float)or_mx_value(blk[1 + j] >> 4) * scale;
                acc += (double)w0 * x[c0 + j] + (double)w1 * x[c0 + j + 16];
            }
        }
        return acc;
    }
    if (w->kind == 8) {                        /* bits==32 arm, qwen_infer.c:2674-2682 */
        const float *pr = (const float *)w->packed + (size_t)row * in;
        for (int c = 0; c < in; c++) acc += (double)pr[c] * x[c];
        return acc;
    }
    if (w->kind == 7) {                        /* bits==16 arm, qwen_infer.c:2683-2691 */
        const uint16_t *pr = (const uint16_t *)w->packed + (size_t)row * in;
        for (int c = 0; c < in; c++) acc += (double)or_f16_to_f32(pr[c]) * x[c];
        return acc;
    }
    if (w->kind == 6) {                        /* int4 affine arm, qwen_infer.c:2780-2798 (no LUT) */
        const uint8_t *pr = (const uint8_t *)w->packed + (size_t)row * (in / 2);
        const float *sc = (const float *)w->scales + (size_t)row * ng;
        const float *bi = (const float *)w->bias + (size_t)row * ng;
        for (int g = 0; g < ng; g++) {
            float scale = sc[g], bias = bi[g];
            for (int ci = 0; ci < G64; ci++) {
                int c = g * G64 + ci;
                uint8_t b = pr[c / 2];
                int nib = (c % 2 == 0) ? (b & 0xF) : ((b >> 4) & 0xF);
                float wv = (float)nib * scale + bias;
                acc += (double)wv * x[c];
            }
        }
        return acc;
    }
    if (w->kind == 2) {
        const int8_t *pr = (const int8_t *)w->packed + (size_t)row * in;
        const float *sc = (const float *)w->scales + (size_t)row * ng;
        for (int g = 0; g < ng; g++) {
            float scale = sc[g];
            for (int ci = 0; ci < G64; ci++) acc += (double)((float)pr[g * G64 + ci] * scale) * x[g * G64 + ci];
        }
        return acc;
    }
    if (w->kind == 4) {
        int n = w->bits, bias_code = 1 << (n - 1);
        size_t gb = (size_t)n * 8;
        const uint8_t *pr = (const uint8_t *)w->packed + (size_t)row * ng * gb;
        const float *sc = (const float *)w->scales + (size_t)row * ng;
        for (int g = 0; g < ng; g++) {
            float scale = sc[g];
            const uint8_t *grp = pr + (size_t)g * gb;
            for (int p = 0; p < G64; p++) {
                int u = 0;
                for (int j = 0; j < n; j++)
                    if ((grp[(size_t)j * 8 + (p >> 3)] >> (p & 7)) & 1) u |= (1 << j);
                float wv = (float)(u - bias_code) * scale;
                acc += (double)wv * x[g * G64 + p];
            }
        }
        return acc;
    }
    const uint8_t *pr = (const uint8_t *)w->packed + (size_t)row * (in / 2);
    for (int c = 0; c < in; c++) {
        uint8_t b = pr[c / 2];
        int nib = (c % 2 == 0) ? (b & 0xF) : ((b >> 4) & 0xF);
        float wv;
        if (w->kind == 5) wv = (nib - 8) * or_f16_to_f32(((const uint16_t *)w->scales)[(size_t)row * (in / 32) + c / 32]);
        else wv = ((float)nib - 8.0f) * ((const float *)w->scales)[(size_t)row * ng + c / G64];
        acc += (double)wv * x[c];
    }
    return acc;
}

/* moe_decode_af (qwen_infer.c:2554-2655): one decoded weight, every kind or_moe_row knows.
 * The int4 arms address the packed row as bytes (the AF u32 words hold the same bytes). */
float or_moe_decode(const or_expert *w, int in, long row, long col) {
    int ng = in / G64;
    long g = col / G64;
    if (w->kind == 9) {                        /* MXFP4 arm, qwen_infer.c:2584-2595 */
        const uint8_t *blk = (const uint8_t *)w->packed + (size_t)row * (in / 32) * 17 + (size_t)(col / 32) * 17;
        int p = (int)(col % 32), q = blk[1 + (p & 15)];
        return (float)or_mx_value(p < 16 ? q & 15 : q >> 4) * or_mx_scale(blk[0]);
    }
    if (w->kind == 8) return ((const float *)w->packed)[(size_t)row * in + col];
    if (w->kind == 7) return or_f16_to_f32(((const uint16_t *)w->packed)[(size_t)row * in + col]);
    if (w->kind == 2)
        return (float)((const int8_t *)w->packed)[(size_t)row * in + col] * ((const float *)w->scales)[(size_t)row * ng + g];
    if (w->kind == 4) {
        int n = w->bits;
        const uint8_t *grp = (const uint8_t *)w->packed + ((size_t)row * ng + g) * n * 8;
        int p = (int)(col % G64), u = 0;
        for (int j = 0; j < n; j++)
            if ((grp[j * 8 + (p >> 3)] >> (p & 7)) & 1) u |= 1 << j;
        return (float)(u - (1 << (n - 1))) * ((const float *)w->scales)[(size_t)row * ng + g];
    }
    uint8_t b = ((const uint8_t *)w->packed)[(size_t)row * (in / 2) + col / 2];
    int nib = (col % 2 == 0) ? (b & 0xF) : ((b >> 4) & 0xF);
    if (w->kind == 5) return (float)(nib - 8) * or_f16_to_f32(((const uint16_t *)w->scales)[(size_t)row * (in / 32) + col / 32]);
    float scale = ((const float *)w->scales)[(size_t)row * ng + g];
    if (w->kind == 6) return (float)nib * scale + ((const float *)w->bias)[(size_t)row * ng + g];
    return ((float)nib - 8.0f) * scale;
}

/* qwen_infer.c:3223-3225 (moe_matvec_af): y[r] = (float)row_dot. */
void or_moe_matvec(const or_expert *w, int out, int in, const float *x, float *y) {
    for (long r = 0; r < out; r++) y[r] = (float)or_moe_row(w, in, r, x);
}

/* qwen_infer.c:3467-3472 (moe_softmax_full). */
void or_moe_softmax_full(float *x, int n) {
    float mx_v = x[0];
    for (int i = 1; i < n; i++) if (x[i] > mx_v) mx_v = x[i];
    double sum = 0.0;
    for (int i = 0; i < n; i++) { x[i] = expf(x[i] - mx_v); sum += x[i]; }
    for (int i = 0; i < n; i++) x[i] = (float)(x[i] / sum);
}

/* qwen_infer.c:3514-3521 (moe_top_k_select): repeated strict-'>' max, ties -> lowest index. */
void or_moe_top_k_select(const float *scores, int n, int k, int *out_idx) {
    int *used = (int *)calloc((size_t)n, sizeof(int));
    for (int i = 0; i < k; i++) {
        int best = -1; float bestv = -1e30f;
        for (int j = 0; j < n; j++) if (!used[j] && scores[j] > bestv) { bestv = scores[j]; best = j; }
        used[best] = 1; out_idx[i] = best;
    }
    free(used);
}

/* qwen_infer.c:3529-3534 (moe_topk_renorm). */
void or_moe_topk_renorm(float *scores, const int *idx, int k) {
    double s = 0.0;
    for (int i = 0; i < k; i++) s += scores[idx[i]];
    if (!(s > 0.0)) return;
    for (int i = 0; i < k; i++) scores[idx[i]] = (float)(scores[idx[i]] / s);
}

/* qwen_infer.c:3475-3481 (moe_swiglu_inplace): g/(1+expf(-g)) * u. */
void or_moe_swiglu_inplace(float *gate, const float *up, int n) {
    for (int i = 0; i < n; i++) {
        float g = gate[i];
        float silu = g / (1.0f + expf(-g));
        gate[i] = silu * up[i];
    }
}

/* qwen_infer.c:726-733 (swiglu, the dense MLP's): out = (g / (1 + e)) * u, e = exp(-g), each step
 * rounded to float as the reference's vDSP sequence rounds it (negate, vvexpf, +1, divide,
 * multiply).  e is exp evaluated in double and rounded once: the correctly rounded expf in all but
 * double-rounding cases, where the reference's vvexpf is only faithful -- the choice that makes h
 * a function of g and u alone. */
void or_swiglu(const float *g, const float *u, float *out, int n) {
    for (int i = 0; i < n; i++) {
        const float e = (float)exp(-(double)g[i]);
        out[i] = (g[i] / (1.0f + e)) * u[i];
    }
}

/* Mixed per-cell qNg64 (MixedQNg64Tensor, mlx_moe.cpp:87-93) decoded as the QT-4 GEMV kernel does
 * (mlx_moe.cpp:1708-1722): cell (r, g) has n = bits[cell] planes of 8 bytes at planes + offsets[cell];
 * element p's bit j is bit (p & 7) of byte j*8 + (p >> 3); value (u - 2^(n-1)) * scales[cell]. */
void or_decode_qng64_mixed(const uint8_t *planes, const uint32_t *offsets, const uint8_t *bits, const float *scales,
                           int out, int in, float *w) {
    const int ng = in / 64;
    for (int r = 0; r < out; r++)
        for (int g = 0; g < ng; g++) {
            const size_t cell = (size_t)r * ng + g;
            const int n = bits[cell];
            const uint8_t *pl = planes + offsets[cell];
            for (int p = 0; p < 64; p++) {
                int u = 0;
                for (int j = 0; j < n; j++) u |= ((pl[j * 8 + (p >> 3)] >> (p & 7)) & 1) << j;
                w[(size_t)r * in + g * 64 + p] = (float)(u - (1 << (n - 1))) * scales[cell];
            }
        }
}

/* Router scores of moe_ffn_batched (qwen_infer.c:5243-5250): moe_matvec_f32 (:3460-3466), a
 * sequential double accumulation per expert row cast to float, then + the router bias in float. */
void or_moe_router_logits(const float *w, const float *bias, const float *x, int T, int E, int H, float *logits) {
    for (int t = 0; t < T; t++)
        for (int e = 0; e < E; e++) {
            double acc = 0.0;
            for (int c = 0; c < H; c++) acc += (double)w[(long)e * H + c] * x[(long)t * H + c];
            float s = (float)acc;
            if (bias) s += bias[e];
            logits[(long)t * E + e] = s;
        }
}

/* Routing of moe_ffn_batched (qwen_infer.c:5251-5257, 5275): softmax over the router scores,
 * top-k, optional renorm; the per-token weight is the (renormalised) softmax probability. */
void or_moe_route(const float *logits, int T, int E, int K, int renorm, int *top_idx, float *top_w) {
    float *s = (float *)malloc(sizeof(float) * (size_t)E);
    for (int t = 0; t < T; t++) {
        memcpy(s, logits + (size_t)t * E, sizeof(float) * (size_t)E);
        or_moe_softmax_full(s, E);
        or_moe_top_k_select(s, E, K, top_idx + (size_t)t * K);
        if (renorm) or_moe_topk_renorm(s, top_idx + (size_t)t * K, K);
        for (int k = 0; k < K; k++) top_w[(size_t)t * K + k] = s[top_idx[(size_t)t * K + k]];
    }
    free(s);
}

static void moe_shared(const or_expert *sg, const or_expert *su, const or_expert *sd, int H, int Ish,
                       const float *xt, float *out_t, float *tg, float *tu, float *td) {
    or_moe_matvec(sg, Ish, H, xt, tg);
    or_moe_matvec(su, Ish, H, xt, tu);
    or_moe_swiglu_inplace(tg, tu, Ish);
    or_moe_matvec(sd, H, Ish, tg, td);
    for (int c = 0; c < H; c++) out_t[c] += td[c];
}

/* qwen_infer.c:5238-5350 (moe_ffn_batched) with routing supplied: bucket (token,k) pairs by expert
 * in token order; experts ascending: gate/up matvec per member, SwiGLU, down, out[b] += wgt*down;
 * then the shared experts for every token. */
void or_moe_ffn_bucketed(const or_expert *gate, const or_expert *up, const or_expert *down, int E,
                         const or_expert *sh_gate, const or_expert *sh_up, const or_expert *sh_down,
                         int H, int I, int Ish, int T, int K, const float *x,
                         const int *top_idx, const float *top_w, float *out) {
    int *cnt = (int *)calloc((size_t)E, sizeof(int));
    int *mtok = (int *)malloc(sizeof(int) * (size_t)E * T);
    float *mw = (float *)malloc(sizeof(float) * (size_t)E * T);
    for (int b = 0; b < T; b++)
        for (int k = 0; k < K; k++) {
            int e = top_idx[(size_t)b * K + k];
            mtok[(size_t)e * T + cnt[e]] = b; mw[(size_t)e * T + cnt[e]] = top_w[(size_t)b * K + k]; cnt[e]++;
        }
    for (size_t i = 0; i < (size_t)T * H; i++) out[i] = 0.0f;
    int Imax = I > Ish ? I : Ish;
    float *g = (float *)malloc(sizeof(float) * (size_t)Imax), *u = (float *)malloc(sizeof(float) * (size_t)Imax);
    float *d = (float *)malloc(sizeof(float) * (size_t)H);
    for (int e = 0; e < E; e++)
        for (int m = 0; m < cnt[e]; m++) {
            int b = mtok[(size_t)e * T + m];
            float wgt = mw[(size_t)e * T + m];
            or_moe_matvec(&gate[e], I, H, x + (size_t)b * H, g);
            or_moe_matvec(&up[e], I, H, x + (size_t)b * H, u);
            or_moe_swiglu_inplace(g, u, I);
            or_moe_matvec(&down[e], H, I, g, d);
            for (int c = 0; c < H; c++) out[(size_t)b * H + c] += wgt * d[c];
        }
    if (sh_gate)
        for (int b = 0; b < T; b++) moe_shared(sh_gate, sh_up, sh_down, H, Ish, x + (size_t)b * H, out + (size_t)b * H, g, u, d);
    free(cnt); free(mtok); free(mw); free(g); free(u); free(d);
}

/* qwen_infer.c:5356-5400 (moe_ffn_naive_batched): same math, pairs in router-selection order. */
void or_moe_ffn_naive(const or_expert *gate, const or_expert *up, const or_expert *down, int E,
                      const or_expert *sh_gate, const or_expert *sh_up, const or_expert *sh_down,
                      int H, int I, int Ish, int T, int K, const float *x,
                      const int *top_idx, const float *top_w, float *out) {
    (void)E;
    int Imax = I > Ish ? I : Ish;
    float *g = (float *)malloc(sizeof(float) * (size_t)Imax), *u = (float *)malloc(sizeof(float) * (size_t)Imax);
    float *d = (float *)malloc(sizeof(float) * (size_t)H);
    for (int b = 0; b < T; b++) {
        float *ob = out + (size_t)b * H;
        for (int c = 0; c < H; c++) ob[c] = 0.0f;
        for (int k = 0; k < K; k++) {
            int e = top_idx[(size_t)b * K + k];
            float wgt = top_w[(size_t)b * K + k];
            or_moe_matvec(&gate[e], I, H, x + (size_t)b * H, g);
            or_moe_matvec(&up[e], I, H, x + (size_t)b * H, u);
            or_moe_swiglu_inplace(g, u, I);
            or_moe_matvec(&down[e], H, I, g, d);
            for (int c = 0; c < H; c++) ob[c] += wgt * d[c];
        }
        if (sh_gate) moe_shared(sh_gate, sh_up, sh_down, H, Ish, x + (size_t)b * H, ob, g, u, d);
    }
    free(g); free(u); free(d);
}
