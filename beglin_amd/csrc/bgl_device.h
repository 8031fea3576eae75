// bgl_device.h -- device-side layout constants and helpers shared by the HIP kernels.
//
// Device weight layout ("row-interleaved tiles"): rows are grouped in tiles of 64 (one row per
// lane of a wavefront).  A row's packed bytes are cut into 16-byte chunks in K order; the tile
// stores chunk c of all 64 rows contiguously: byte offset ((tile*cpr + c)*64 + lane)*16.  Every
// wave-wide load is one contiguous 1 KB run, and all lanes of a wave work on the same K range,
// so the activation values they need are wave-uniform (scalar loads, SGPR operands).
// Per-group scales are stored the same way: [tile][group][lane].
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define BGL_TILE 64            // rows per tile == lanes per wavefront
#define BGL_WAVES 4            // wavefronts per workgroup in the GEMV kernels

#include "../../include/beglin_qgemv.h"

// Format ids: 1..4 are the reference engine's WT kinds (qwen_infer.c:207); 5 is the
// build-defined int4 group-32 fp16-scale format.  Activation modes BGL_ACT_F32 (fp32 activations,
// exact fixed-point digits) and BGL_ACT_W4A8 (the reference's dynamic int8 quantization,
// QWEN_W4A8=1, qwen_infer.c:625-629) come from the public header.
#define BGL_Q4G64 BGL_K_Q4G64
#define BGL_Q8G64 BGL_K_Q8G64
#define BGL_Q4G256SF BGL_K_Q4G256SF
#define BGL_QNG64 BGL_K_QNG64
#define BGL_Q4G32H BGL_K_Q4G32H
#define BGL_Q4G64A BGL_K_Q4G64A
#define BGL_F16 BGL_K_F16
#define BGL_F32 BGL_K_F32
#define BGL_MXFP4 BGL_K_MXFP4

// fp32 activations as exact integers, per 64-group:
//   level 0: X = rint(x * 2^(22-e)), e = exponent of the group's largest finite |x| (|X| <= 2^22),
//            at least -127 (an all-subnormal group then has X = x * 2^149, exact), as three balanced base-256 int8 digits X = d0 + 256*d1 + 65536*d2 (|d2| <= 64).  An
//            element's error is at most 2^(e-23): relative to any |x| >= 2^(e-6), at most 2^-17.
//   level 1: in groups holding at least BGL_X_SMALL_MAX nonzero elements below 2^(e-6), or more
//            such small elements than elements at or above it (an outlier, or a cluster of large
//            channels, would otherwise leave the small elements with few bits): the residual
//            r = x * 2^(22-e) - X (exact) as X1 = rint(r * 2^(22-e1)), e1 = exponent of the group's
//            largest |r|, in the same three digits.  x = (X + X1 * 2^(e1-22)) * 2^(e-22) to about
//            2^-46 of the group maximum.
//   So a level-0 group's dot product errs by at most 2^-17 * sum |w| * max(|x|, 2^(e-6)), where at
//   most BGL_X_SMALL_MAX - 1 nonzero elements take the 2^(e-6) floor.
// Non-finite elements (NaN, +-Inf) enter both levels as 0; the group is flagged and the GEMVs add
// their products code * scale * x one element at a time, so NaN and +-Inf propagate as in IEEE
// arithmetic.  Per column the prep kernel writes [group][digit][64 bytes] (48 dwords per group),
// the power-of-two scale 2^(e-22) per group and the exact integer sum of the digits per
// 32-element half-group; level 1 the same beside it, plus the ratio 2^(e1-22) (0 without level 1).
#define BGL_XD_DW 48
#define BGL_XF_L1 1            // group flags: the group has level-1 digits
#define BGL_XF_NF 2            //              the group holds a non-finite element
#define BGL_X_FRAC 22          // level-0 / level-1 fixed point: X = rint(x * 2^(BGL_X_FRAC - e))
#define BGL_X_EMIN (BGL_X_FRAC - 149)   // e is at least this, so the scale 2^(e-22) is >= 2^-149, a float;
                                  // groups below it (|x| < 2^-128, subnormal) get X = x * 2^149 exactly
#define BGL_X_SPIKE_BITS 6     // "small": a nonzero |x| below 2^(e-6)
#define BGL_X_SMALL_MAX 22     // level 1 from this many small elements (or more small than large)

// The level-1 trigger from a group's count of small (nonzero, below 2^(e-6)) and large elements.
__host__ __device__ __forceinline__ bool bgl_x_level1(int nsmall, int nlarge) {
    return nsmall > nlarge || nsmall >= BGL_X_SMALL_MAX;
}

// Wave-uniform read-only operands (activations, column maps) are read through the constant address
// space so the compiler emits scalar loads (s_load_dwordx16) and feeds v_dot4 from SGPRs.
typedef const int __attribute__((address_space(4))) *ucint;
typedef const float __attribute__((address_space(4))) *ucfloat;
__device__ __forceinline__ ucint uni(const int *p) { return (ucint)p; }
__device__ __forceinline__ ucfloat uni(const float *p) { return (ucfloat)p; }

// Wavefront reductions through DPP (quad_perm 1032 / 2301, row_half_mirror, row_mirror reduce each
// 16-lane row), then readlane of the four row results.  Every lane gets the (uniform) result.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) { return __int_as_float(dpp_i<CTRL>(__float_as_int(v))); }
__device__ __forceinline__ float rlane_f(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }

__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return fmaxf(fmaxf(rlane_f(v, 0), rlane_f(v, 16)), fmaxf(rlane_f(v, 32), rlane_f(v, 48)));
}
// unsigned max over the wave (NaN bit patterns compare as large integers, unlike fmaxf)
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)dpp_i<0xB1>((int)v));
    v = max(v, (uint32_t)dpp_i<0x4E>((int)v));
    v = max(v, (uint32_t)dpp_i<0x141>((int)v));
    v = max(v, (uint32_t)dpp_i<0x140>((int)v));
    return max(max((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16)),
               max((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48)));
}
// (value, index) maximum over the wave, ties to the lower index, in every lane.  The order is total
// for non-NaN values, so any pairing gives the same winner: DPP within each row, then the four row
// winners by readlane.
__device__ __forceinline__ void arg_take(float &bv, int &bi, float ov, int oi) {
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}
template <int CTRL>
__device__ __forceinline__ void arg_dpp(float &bv, int &bi) { arg_take(bv, bi, dpp_f<CTRL>(bv), dpp_i<CTRL>(bi)); }
__device__ __forceinline__ void wave_argmax(float &bv, int &bi) {
    arg_dpp<0xB1>(bv, bi);
    arg_dpp<0x4E>(bv, bi);
    arg_dpp<0x141>(bv, bi);
    arg_dpp<0x140>(bv, bi);
    float v = rlane_f(bv, 0);
    int i = __builtin_amdgcn_readlane(bi, 0);
    arg_take(v, i, rlane_f(bv, 16), __builtin_amdgcn_readlane(bi, 16));
    arg_take(v, i, rlane_f(bv, 32), __builtin_amdgcn_readlane(bi, 32));
    arg_take(v, i, rlane_f(bv, 48), __builtin_amdgcn_readlane(bi, 48));
    bv = v;
    bi = i;
}
// returns the per-row (16-lane) sums in every lane of that row
__device__ __forceinline__ int row_sum_i32(int v) {
    v += dpp_i<0xB1>(v);
    v += dpp_i<0x4E>(v);
    v += dpp_i<0x141>(v);
    v += dpp_i<0x140>(v);
    return v;
}
__device__ __forceinline__ int wave_sum_i32(int v) {
    v = row_sum_i32(v);
    return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
           (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}
// sums over lanes 0..31 and 32..63
__device__ __forceinline__ int2 half_sums_i32(int v) {
    v = row_sum_i32(v);
    return make_int2(__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16),
                     __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// int4 chunk dword -> two dwords of 4 unsigned nibble bytes (device nibble order: byte i of the
// dword holds element i in its low nibble and element 4+i in its high nibble).
__device__ __forceinline__ int nib_lo(uint32_t w) { return (int)(w & 0x0F0F0F0Fu); }
__device__ __forceinline__ int nib_hi(uint32_t w) { return (int)((w >> 4) & 0x0F0F0F0Fu); }

__device__ __forceinline__ uint4 ldg16(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }

// MXFP4 (OCP microscaling FP4 in GGUF blocks of 32): an E2M1 nibble's value doubled -- 0, 1, 2, 3,
// 4, 6, 8, 12 for codes 0..7 and the same negated for 8..15 -- times an E8M0 exponent byte b read
// as 2^(b-128), i.e. the exponent halved to undo the doubling (gguf_quants.c:284-305).  Both
// factors are exact, so every weight is an exact float.
__device__ __forceinline__ float mx_scale(uint32_t b) { return __uint_as_float(b < 2u ? (0x00200000u << b) : (b - 1u) << 23); }
// Four codes (one per byte, bits 0..3) -> their four doubled values as int8: magnitude and
// negated magnitude by byte permutes over the low three bits, picked per byte by the fourth.
__device__ __forceinline__ int mx_codes(uint32_t c) {
    const uint32_t idx = c & 0x07070707u;
    const uint32_t pos = __builtin_amdgcn_perm(0x0C080604u, 0x03020100u, idx);
    const uint32_t neg = __builtin_amdgcn_perm(0xF4F8FAFCu, 0xFDFEFF00u, idx);
    const uint32_t m = ((c >> 3) & 0x01010101u) * 0xFFu;
    return (int)((neg & m) | (pos & ~m));
}

// qNg64 field decomposition: n = 8a + 4b + 2c + d; field widths in descending order occupy
// consecutive bits of the biased code u = code + 2^(n-1) from bit 0 upwards.
struct QngFields {
    int has8, has4, has2, has1;
    int sh4, sh2, sh1;         // bit offsets of the 4-, 2-, 1-bit fields inside u
};
__host__ __device__ inline QngFields qng_fields(int n) {
    QngFields f;
    f.has8 = (n >> 3) & 1; f.has4 = (n >> 2) & 1; f.has2 = (n >> 1) & 1; f.has1 = n & 1;
    f.sh4 = 8 * f.has8; f.sh2 = f.sh4 + 4 * f.has4; f.sh1 = f.sh2 + 2 * f.has2;
    return f;
}
