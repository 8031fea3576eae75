// bgl_api.hip -- the C-ABI (include/beglin_qgemv.h): contexts, binding/repack, GEMV dispatch.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "../../include/beglin_qgemv.h"
#include "bgl_kernels.h"
#include "bgl_internal.h"

static thread_local char g_err[512];
static thread_local int g_code;

int bgl_last_code(void) { return g_code ? g_code : BGL_E_NOMEM; }

int bgl_fail(int code, const char *fmt, ...) {
    g_code = code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}
#define HIPCHK(expr)                                                                             \
    do {                                                                                         \
        hipError_t e_ = (expr);                                                                  \
        if (e_ != hipSuccess) return bgl_fail(BGL_E_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

extern "C" const char *bgl_last_error(void) { return g_err; }

extern "C" int bgl_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, 0) != hipSuccess) return 0;
    return strncmp(p.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

// ------------------------------------------------------------------ device buffers
// Per-call scratch grows on demand.  A graph captured from the context's stream keeps the raw
// addresses of the scratch its calls used, so a buffer that has to grow is not freed: it is
// retired and freed with the context (bgl_ctx_destroy) or an epoch reset.  Growing inside a
// stream capture would put allocation into the captured region: refused with BGL_E_CAPTURE
// (the caller runs the call once eagerly at that size first).
int dbuf_reserve(bgl_ctx *c, DevBuf &b, size_t bytes, bool zero) {
    if (c->fixed_base) {                    // bgl_matmul_group_noalloc_dev: a slice of the fixed array, never an allocation
        const size_t off = (c->fixed_used + 255) & ~(size_t)255;
        if (zero) return bgl_fail(BGL_E_UNSUPPORTED, "no-alloc call: no path here needs zeroed scratch");
        if (off + bytes > c->fixed_cap)
            return bgl_fail(BGL_E_NOMEM, "no-alloc call needs more than the fixed %zu B of device scratch (BGL_NOALLOC_SCRATCH_BYTES): "
                            "use fewer columns or the allocating entry point", c->fixed_cap);
        b.p = c->fixed_base + off;
        b.bytes = bytes;
        c->fixed_used = off + bytes;
        return 0;
    }
    if (b.bytes >= bytes) return 0;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIPCHK(hipStreamIsCapturing(c->stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return bgl_fail(BGL_E_CAPTURE, "per-call scratch would have to grow to %zu B inside a stream capture: run the call "
                        "once without capture at this size (or larger) first", bytes);
    if (b.p) {
        c->retired.push_back(b.p);          // a captured graph may still use it
        b.p = nullptr; b.bytes = 0;
    }
    size_t want = bytes + bytes / 4 + 4096;
    HIPCHK(hipSetDevice(c->device));        // the context's device, whatever the calling thread had selected
    HIPCHK(hipMalloc(&b.p, want));
    b.bytes = want;
    if (zero) {
        HIPCHK(hipMemsetAsync(b.p, 0, want, c->stream));
        HIPCHK(hipStreamSynchronize(c->stream));
    }
    return 0;
}

static void dbuf_free(DevBuf &b) {
    if (b.p) (void)hipFree(b.p);
    b.p = nullptr; b.bytes = 0;
}

size_t ctx_scratch(bgl_ctx *c, bool release) {
    DevBuf *bufs[] = {&c->act_w, &c->act_s, &c->act_sum, &c->part, &c->hx, &c->hy, &c->hb,
                      &c->moe_a, &c->moe_b, &c->moe_c, &c->moe_d, &c->moe_e, &c->moe_f, &c->moe_g, &c->moe_meta,
                      &c->moe_route, &c->moe_scores, &c->mlp, &c->prep_xc};
    size_t total = 0;
    for (DevBuf *b : bufs) {
        total += b->bytes;
        if (release) dbuf_free(*b);
    }
    for (auto &kv : c->mlp_sync) {
        total += kv.second.bytes;
        if (release) dbuf_free(kv.second);
    }
    if (release) c->mlp_sync.clear();
    if (release) {
        for (void *p : c->retired) (void)hipFree(p);
        c->retired.clear();
        c->prep_act = -1; c->prep_M = 0; c->prep_K = 0; c->prep_reuse = false; c->prep_x = nullptr;
    }
    return total;
}

// ------------------------------------------------------------------ fixed scratch (no-alloc entry)
// The scratch of bgl_matmul_group_noalloc_dev: a file-scope device array, so the call allocates
// nothing.  Each GPU the library runs on holds its own copy (BGL_NOALLOC_SCRATCH_BYTES) until the
// process ends.  In host code `scratch` names a host-side stand-in, not the device array: its
// device address comes from hipGetSymbolAddress, once per device, and only that address is used.
static __device__ __align__(256) uint8_t scratch[BGL_NOALLOC_SCRATCH_BYTES];
#define BGL_MAX_DEVICES 64
static std::mutex g_scratch_mu;
static uint8_t *g_scratch_ptr[BGL_MAX_DEVICES];

// The device address of this device's fixed scratch (the caller has made `device` current).
static int scratch_setup(int device) {
    if (device < 0 || device >= BGL_MAX_DEVICES) return bgl_fail(BGL_E_NODEV, "fixed scratch: device %d out of range", device);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[device]) return 0;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return bgl_fail(BGL_E_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[device] = (uint8_t *)ptr;
    return 0;
}

extern "C" int bgl_ctx_create(int device, void *hip_stream, bgl_ctx **out) {
    if (!out) return bgl_fail(BGL_E_ARG, "bgl_ctx_create: out is NULL");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n)
        return bgl_fail(BGL_E_NODEV, "bgl_ctx_create: no HIP device %d", device);
    HIPCHK(hipSetDevice(device));
    int rc = scratch_setup(device);
    if (rc) return rc;
    bgl_ctx *c = new bgl_ctx();
    c->device = device;
    if (hip_stream) { c->stream = (hipStream_t)hip_stream; c->own_stream = false; }
    else {
        hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
        if (e != hipSuccess) { delete c; return bgl_fail(BGL_E_HIP, "hipStreamCreate: %s", hipGetErrorString(e)); }
        c->own_stream = true;
    }
    const char *mw = getenv("BGL_MAX_WAVES");
    c->max_waves = mw ? atoi(mw) : 16;
    if (c->max_waves < 1 || c->max_waves > 16) c->max_waves = 16;
    const char *mb = getenv("BGL_MIN_BLOCKS");
    c->min_blocks = mb ? atoi(mb) : 256;
    const char *pc = getenv("BGL_MF_PCAP");
    c->mf_pcap = pc ? (float)atof(pc) : 1.0f;
    if (!(c->mf_pcap >= 0.0f && c->mf_pcap <= 64.0f)) c->mf_pcap = 1.0f;
    const char *ft = getenv("BGL_FORCE_TR");
    c->force_tr = ft ? atoi(ft) : 0;
    if (c->force_tr != 0 && c->force_tr != 8 && c->force_tr != 16 && c->force_tr != 32 && c->force_tr != 64) c->force_tr = 0;
    const char *nf = getenv("BGL_NO_FUSED_Q");
    c->no_fused = nf && atoi(nf) != 0;
    const char *nm = getenv("BGL_NO_MFMA");
    c->no_mfma = nm && atoi(nm) != 0;
    const char *nx = getenv("BGL_NO_GEMV_X");
    c->no_gemv_x = nx && atoi(nx) != 0;
    const char *xw = getenv("BGL_X_WAVES");
    c->x_waves = xw ? atoi(xw) : 0;
    if (c->x_waves < 0 || c->x_waves > 16) c->x_waves = 0;
    const char *qp = getenv("BGL_Q_PREP");
    c->q_prep = qp ? (atoi(qp) != 0) : -1;
    const char *nmx = getenv("BGL_NO_MOE_X");
    c->no_moe_x = nmx && atoi(nmx) != 0;
    const char *xf = getenv("BGL_X_FUSE");
    c->x_fuse = xf ? (atoi(xf) != 0) : -1;
    const char *mm = getenv("BGL_MOE_MERGE");
    c->moe_merge = mm ? (atoi(mm) != 0) : -1;
    const char *mcap = getenv("BGL_MOE_CAP");
    c->moe_cap = mcap ? atoi(mcap) : 0;
    if (c->moe_cap != 4 && c->moe_cap != 8) c->moe_cap = 0;
    const char *nfm = getenv("BGL_NO_FUSED_MLP");
    c->no_fused_mlp = nfm && atoi(nfm) != 0;
    const char *ms = getenv("BGL_MLP_SPIN");
    if (ms && atoi(ms) > 0) c->mlp_spin = atoi(ms);
    const char *mwv = getenv("BGL_MLP_WAVES");
    c->mlp_waves = mwv ? atoi(mwv) : 0;
    if (c->mlp_waves < 0 || c->mlp_waves > 16) c->mlp_waves = 0;
    const char *mdl = getenv("BGL_MLP_DELAY");
    c->mlp_delay = mdl ? atoi(mdl) : -1;
    if (c->mlp_delay < -1 || c->mlp_delay > 100000) c->mlp_delay = -1;
    const char *nqm = getenv("BGL_NO_QMFMA");
    c->no_qmfma = nqm && atoi(nqm) != 0;
    const char *qrb = getenv("BGL_QM_RB");
    c->qm_rb = qrb ? atoi(qrb) : 0;
    const char *qs = getenv("BGL_QM_S");
    c->qm_s = qs ? atoi(qs) : 0;
    if (c->qm_s < 0 || c->qm_s > 16) c->qm_s = 0;
    const char *qprb = getenv("BGL_QM_PRB");
    c->qm_prb = qprb ? atoi(qprb) : 0;
    const char *qps = getenv("BGL_QM_PS");
    c->qm_ps = qps ? atoi(qps) : 0;
    if (c->qm_ps < 0 || c->qm_ps > 16) c->qm_ps = 0;
    const char *mgu = getenv("BGL_MLP_GU");
    c->mlp_gu = mgu ? atoi(mgu) : 0;
    if (c->mlp_gu < 0 || c->mlp_gu > 4096) c->mlp_gu = 0;
    const char *mt = getenv("BGL_MLP_TEST_TIMEOUT");
    c->mlp_test_timeout = mt && atoi(mt) > 0 ? atoi(mt) : 0;
    *out = c;
    return 0;
}

// ------------------------------------------------------------------ profiling
static hipEvent_t ev_get(bgl_ctx *c) {
    if (!c->ev_pool.empty()) { hipEvent_t e = c->ev_pool.back(); c->ev_pool.pop_back(); return e; }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

int prof_begin(bgl_ctx *c, int phase) {
    if (!c->prof) return -1;
    hipEvent_t a = ev_get(c), b = ev_get(c);
    if (!a || !b) return -1;
    (void)hipEventRecord(a, c->stream);
    c->prof_ev.push_back({phase, {a, b}});
    return (int)c->prof_ev.size() - 1;
}

void prof_end(bgl_ctx *c, int token) {
    if (token < 0) return;
    (void)hipEventRecord(c->prof_ev[token].second.second, c->stream);
}

extern "C" int bgl_prof_enable(bgl_ctx *c, int on) {
    if (!c) return bgl_fail(BGL_E_ARG, "bgl_prof_enable: NULL context");
    c->prof = on != 0;
    return 0;
}

extern "C" int bgl_prof_read(bgl_ctx *c, double *ms, int *cnt, int nphase) {
    if (!c) return bgl_fail(BGL_E_ARG, "bgl_prof_read: NULL context");
    HIPCHK(hipStreamSynchronize(c->stream));
    for (int i = 0; i < nphase; i++) { if (ms) ms[i] = 0.0; if (cnt) cnt[i] = 0; }
    int bad = 0;
    for (auto &r : c->prof_ev) {
        float t = 0.0f;
        if (hipEventElapsedTime(&t, r.second.first, r.second.second) == hipSuccess) {
            if (r.first < nphase) {
                if (ms) ms[r.first] += t;
                if (cnt) cnt[r.first] += 1;
            }
        } else {
            bad++;
        }
        c->ev_pool.push_back(r.second.first);
        c->ev_pool.push_back(r.second.second);
    }
    c->prof_ev.clear();
    (void)hipGetLastError();             // an unreadable event pair must not poison the next call
    if (bad) return bgl_fail(BGL_E_HIP, "bgl_prof_read: %d event pairs had no timing", bad);
    return 0;
}

extern "C" void bgl_ctx_destroy(bgl_ctx *c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    for (auto &r : c->prof_ev) { c->ev_pool.push_back(r.second.first); c->ev_pool.push_back(r.second.second); }
    for (hipEvent_t e : c->ev_pool) (void)hipEventDestroy(e);
    for (auto &kv : c->host_cache) bgl_tensor_free(kv.second);
    c->host_cache.clear();
    ctx_scratch(c, true);
    if (c->own_stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

extern "C" int bgl_synchronize(bgl_ctx *c) {
    if (!c) return bgl_fail(BGL_E_ARG, "bgl_synchronize: NULL context");
    HIPCHK(hipStreamSynchronize(c->stream));
    return 0;
}

extern "C" void *bgl_ctx_stream(bgl_ctx *c) { return c ? (void *)c->stream : nullptr; }

// ------------------------------------------------------------------ tensors
static int units_of(int kind, int in) {
    switch (kind) {
    case BGL_Q4G64: case BGL_Q4G32H: case BGL_Q8G64: case BGL_Q4G64A: case BGL_F16: case BGL_F32: case BGL_MXFP4: return in / 64;
    case BGL_Q4G256SF: return in / 256;
    case BGL_QNG64: return (in / 64 + 1) / 2;
    default: return 0;
    }
}

int check_wt(int kind, int bits, int out, int in) {
    if (out <= 0 || in <= 0) return bgl_fail(BGL_E_ARG, "bad shape out=%d in=%d", out, in);
    switch (kind) {
    case BGL_Q4G64: case BGL_Q8G64: case BGL_QNG64:
        if (in % 64) return bgl_fail(BGL_E_ARG, "in=%d %% 64 != 0", in);
        if (kind == BGL_QNG64 && (bits < 2 || bits > 15)) return bgl_fail(BGL_E_ARG, "qNg64 n=%d outside 2..15", bits);
        return 0;
    case BGL_Q4G32H: case BGL_Q4G64A: case BGL_F16: case BGL_F32: case BGL_MXFP4:
        // MXFP4 blocks hold 32 values; the gather works in 64-groups (two blocks)
        if (in % 64) return bgl_fail(BGL_E_ARG, "kind %d: in=%d %% 64 != 0", kind, in);
        return 0;
    case BGL_Q4G256SF: case BGL_K_Q4G256P:
        if (in % 256) return bgl_fail(BGL_E_ARG, "g256 in=%d %% 256 != 0", in);
        return 0;
    default: return bgl_fail(BGL_E_UNSUPPORTED, "unknown weight kind %d", kind);
    }
}

static size_t ref_packed_bytes(int kind, int bits, int out, int in) {
    switch (kind) {
    case BGL_Q4G64: case BGL_Q4G256SF: case BGL_Q4G32H: case BGL_Q4G64A: case BGL_K_Q4G256P: return (size_t)out * in / 2;
    case BGL_Q8G64: return (size_t)out * in;
    case BGL_F16: return (size_t)out * in * 2;
    case BGL_F32: return (size_t)out * in * 4;
    case BGL_QNG64: return (size_t)out * (in / 64) * bits * 8;
    case BGL_MXFP4: return (size_t)out * (in / 32) * 17;
    default: return 0;
    }
}
static size_t ref_scale_bytes(int kind, int out, int in) {
    switch (kind) {
    case BGL_Q4G64: case BGL_Q8G64: case BGL_QNG64: case BGL_Q4G64A: return (size_t)out * (in / 64) * 4;
    case BGL_Q4G256SF: case BGL_K_Q4G256P: return (size_t)out * (in / 256) * 4;
    case BGL_Q4G32H: return (size_t)out * (in / 32) * 2;
    default: return 0;
    }
}

static inline unsigned nblk(long n, int bs = 256) { return (unsigned)((n + bs - 1) / bs); }

// The tiled device layout of a (kind, bits, out, in) tensor: its record and the byte sizes of its
// three allocations (chunks, per-unit scales, per-unit second word; 0 when absent).
void device_layout(int kind, int bits, int out, int in, BglDevTensor &T, size_t bytes[3]) {
    T = BglDevTensor{};
    T.fmt = kind;
    T.bits = kind == BGL_QNG64 ? bits : kind == BGL_Q8G64 ? 8 : kind == BGL_F16 ? 16 : kind == BGL_F32 ? 32 : 4;
    T.N = out; T.K = in; T.ntiles = (out + BGL_TILE - 1) / BGL_TILE;
    T.gmul = kind == BGL_Q4G256SF ? 1.0f / 63.0f : 1.0f;
    T.nunits = units_of(kind, in);
    T.cpu = kind == BGL_Q4G256SF ? 8 : kind == BGL_Q8G64 ? 4 : kind == BGL_QNG64 ? bits : kind == BGL_F16 ? 8
          : kind == BGL_F32 ? 16 : 2;
    T.cpr = T.nunits * T.cpu;
    const long rows = (long)T.ntiles * BGL_TILE;
    const bool dense = kind == BGL_F16 || kind == BGL_F32;
    bytes[0] = (size_t)rows * T.cpr * 16;
    bytes[1] = dense ? 0 : (size_t)rows * T.nunits * (kind == BGL_QNG64 || kind == BGL_Q4G256SF ? 8 : 4);
    bytes[2] = kind == BGL_Q4G64A ? (size_t)rows * T.nunits * 4 : 0;
}

bgl_tensor *tensor_from_parts(const BglDevTensor &T, void *w, void *s0, void *s1, size_t device_bytes) {
    bgl_tensor *t = new bgl_tensor();
    t->T = T;
    t->T.w = (const uint8_t *)w; t->T.s0 = s0; t->T.s1 = (const uint32_t *)s1;
    t->owned = {w, s0, s1};
    t->device_bytes = device_bytes;
    return t;
}

// Repack reference-layout device buffers into a new tensor.
static int repack_into(bgl_ctx *c, int kind, int bits, int out, int in, const void *dpk, const void *dsc,
                       const uint8_t *dsub, bgl_tensor **res) {
    switch (kind) {
    case BGL_Q4G64: case BGL_Q4G32H: case BGL_Q4G256SF: case BGL_Q4G64A: case BGL_MXFP4:
    case BGL_Q8G64: case BGL_F16: case BGL_F32: case BGL_QNG64:
        break;
    default:
        return bgl_fail(BGL_E_ARG, "repack: kind %d has no device layout of its own", kind);
    }
    bgl_tensor *t = new bgl_tensor();
    BglDevTensor &T = t->T;
    size_t lb[3];
    device_layout(kind, bits, out, in, T, lb);
    const long rows = (long)T.ntiles * BGL_TILE;
    const size_t wbytes = lb[0], s0bytes = lb[1];
    const bool has_s1 = lb[2] != 0;
    void *w = nullptr, *s0 = nullptr, *s1 = nullptr;
    hipError_t e = hipMalloc(&w, wbytes);
    if (e == hipSuccess && s0bytes) e = hipMalloc(&s0, s0bytes);
    if (e == hipSuccess && has_s1) e = hipMalloc(&s1, (size_t)rows * T.nunits * 4);
    if (e != hipSuccess) {
        if (w) (void)hipFree(w);
        if (s0) (void)hipFree(s0);
        delete t;
        return bgl_fail(BGL_E_NOMEM, "hipMalloc for tensor (%zu B): %s", wbytes, hipGetErrorString(e));
    }
    t->owned = {w, s0, s1};
    T.w = (const uint8_t *)w; T.s0 = s0; T.s1 = (const uint32_t *)s1;
    t->device_bytes = wbytes + s0bytes + (s1 ? (size_t)rows * T.nunits * 4 : 0);
    long nch = rows * T.cpr;
    switch (kind) {
    case BGL_Q4G64: case BGL_Q4G32H: case BGL_Q4G256SF: case BGL_Q4G64A: case BGL_MXFP4:
        // g256sf is only read by the int8-activation kernels, which take its codes as signed nibbles
        hipLaunchKernelGGL(k_repack_nib, dim3(nblk(nch)), dim3(256), 0, c->stream, (const uint8_t *)dpk, out, in,
                           kind == BGL_Q4G256SF ? 0x88888888u : 0u, (uint8_t *)w);
        break;
    case BGL_Q8G64: case BGL_F16: case BGL_F32:      // plain 16-byte chunk interleave of the row bytes
        hipLaunchKernelGGL(k_repack_q8, dim3(nblk(nch)), dim3(256), 0, c->stream, (const int8_t *)dpk, out,
                           in * (kind == BGL_F16 ? 2 : kind == BGL_F32 ? 4 : 1), (uint8_t *)w);
        break;
    case BGL_QNG64:
        hipLaunchKernelGGL(k_repack_qng, dim3(nblk(rows * T.nunits, 64)), dim3(64), 0, c->stream, (const uint8_t *)dpk, out, in, bits, (uint8_t *)w);
        break;
    }
    long nu = rows * T.nunits;
    switch (kind) {
    case BGL_Q4G64: case BGL_Q8G64: case BGL_Q4G32H: case BGL_Q4G64A: case BGL_MXFP4:
        // Q4G32H: two fp16 per unit read as one u32; MXFP4: the two exponent bytes; the others one fp32.
        hipLaunchKernelGGL(k_repack_u32, dim3(nblk(nu)), dim3(256), 0, c->stream, (const uint32_t *)dsc, out, T.nunits, (uint32_t *)s0);
        if (has_s1)   // Q4G64A: the fp32 bias per unit
            hipLaunchKernelGGL(k_repack_u32, dim3(nblk(nu)), dim3(256), 0, c->stream, (const uint32_t *)dsub, out, T.nunits, (uint32_t *)s1);
        break;
    case BGL_Q4G256SF:   // wsuper and the unit's 4 sub-codes in one 8-byte word
        hipLaunchKernelGGL(k_repack_zip_u32, dim3(nblk(nu)), dim3(256), 0, c->stream, (const uint32_t *)dsc, (const uint32_t *)dsub,
                           out, T.nunits, (uint2 *)s0);
        break;
    case BGL_QNG64:
        hipLaunchKernelGGL(k_repack_qng_scales, dim3(nblk(nu)), dim3(256), 0, c->stream, (const float *)dsc, out, in / 64, (float2 *)s0);
        break;
    }
    e = hipGetLastError();
    if (e != hipSuccess) { bgl_tensor_free(t); return bgl_fail(BGL_E_HIP, "repack launch: %s", hipGetErrorString(e)); }
    *res = t;
    return 0;
}

// MXFP4 blocks [out][in/32][17] (exponent byte, then 16 bytes whose byte j holds value j in its
// low nibble and value j+16 in its high nibble) -> codes [out][in/2] in the reference q4 order
// (byte b: value 2b low, 2b+1 high) and one u32 per 64-unit with its two exponent bytes; then
// the q4 repacks.
__global__ void k_split_mxfp4(const uint8_t *__restrict__ blk, int out, int in, uint8_t *__restrict__ codes,
                              uint32_t *__restrict__ ex) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x, nu = (long)out * (in / 64);
    if (i >= nu) return;
    const uint8_t *b = blk + i * 34;                 // two blocks per unit, consecutive within a row
    uint8_t *d = codes + i * 32;
    auto code = [&](int h, int p) {                  // value p (0..31) of block h
        const uint8_t q = b[17 * h + 1 + (p & 15)];
        return p < 16 ? q & 15 : q >> 4;
    };
    for (int h = 0; h < 2; h++)
        for (int j = 0; j < 16; j++) d[16 * h + j] = (uint8_t)(code(h, 2 * j) | (code(h, 2 * j + 1) << 4));
    ex[i] = (uint32_t)b[0] | ((uint32_t)b[17] << 8);
}

static int bind_mxfp4(bgl_ctx *c, const bgl_wt *w, bgl_tensor **out) {
    HIPCHK(hipSetDevice(c->device));
    const size_t pb = ref_packed_bytes(BGL_MXFP4, 4, w->out, w->in), nu = (size_t)w->out * (w->in / 64);
    void *dblk = nullptr, *dcodes = nullptr, *dex = nullptr;
    HIPCHK(hipMalloc(&dblk, pb));
    HIPCHK(hipMalloc(&dcodes, nu * 32));
    HIPCHK(hipMalloc(&dex, nu * 4));
    HIPCHK(hipMemcpyAsync(dblk, w->packed, pb, hipMemcpyHostToDevice, c->stream));
    hipLaunchKernelGGL(k_split_mxfp4, dim3(nblk((long)nu)), dim3(256), 0, c->stream, (const uint8_t *)dblk, w->out, w->in,
                       (uint8_t *)dcodes, (uint32_t *)dex);
    int rc = repack_into(c, BGL_MXFP4, 4, w->out, w->in, dcodes, dex, nullptr, out);
    hipError_t e = hipStreamSynchronize(c->stream);
    (void)hipFree(dblk); (void)hipFree(dcodes); (void)hipFree(dex);
    if (rc) return rc;
    if (e != hipSuccess) return bgl_fail(BGL_E_HIP, "bind sync: %s", hipGetErrorString(e));
    return 0;
}

// The plain-g256 diagnostic (q4gemv_g256.h:102-130): q4 nibbles and one fp32 scale per 256 values,
// bound as the g256sf layout with every sub-code 1 and the fold factor 1 instead of 1/63.
static int bind_g256plain(bgl_ctx *c, const bgl_wt *w, bgl_tensor **out) {
    if (!w->scales) return bgl_fail(BGL_E_ARG, "bgl_bind: plain g256 needs scales");
    HIPCHK(hipSetDevice(c->device));
    const size_t pb = (size_t)w->out * w->in / 2, sb = (size_t)w->out * (w->in / 256) * 4, nsub = (size_t)w->out * (w->in / 64);
    void *dpk = nullptr, *dsc = nullptr, *dsub = nullptr;
    HIPCHK(hipMalloc(&dpk, pb));
    HIPCHK(hipMalloc(&dsc, sb));
    HIPCHK(hipMalloc(&dsub, nsub));
    HIPCHK(hipMemcpyAsync(dpk, w->packed, pb, hipMemcpyHostToDevice, c->stream));
    HIPCHK(hipMemcpyAsync(dsc, w->scales, sb, hipMemcpyHostToDevice, c->stream));
    HIPCHK(hipMemsetAsync(dsub, 1, nsub, c->stream));
    int rc = repack_into(c, BGL_Q4G256SF, 4, w->out, w->in, dpk, dsc, (const uint8_t *)dsub, out);
    hipError_t e = hipStreamSynchronize(c->stream);
    (void)hipFree(dpk); (void)hipFree(dsc); (void)hipFree(dsub);
    if (rc) return rc;
    if (e != hipSuccess) return bgl_fail(BGL_E_HIP, "bind sync: %s", hipGetErrorString(e));
    (*out)->T.gmul = 1.0f;
    return 0;
}

extern "C" int bgl_bind(bgl_ctx *c, const bgl_wt *w, bgl_tensor **out) {
    if (!c || !w || !out || !w->packed) return bgl_fail(BGL_E_ARG, "bgl_bind: NULL argument");
    int rc = check_wt(w->kind, w->bits, w->out, w->in);
    if (rc) return rc;
    const bool dense = w->kind == BGL_F16 || w->kind == BGL_F32;
    if (w->kind == BGL_MXFP4) return bind_mxfp4(c, w, out);
    if (w->kind == BGL_K_Q4G256P) return bind_g256plain(c, w, out);
    if (!dense && !w->scales) return bgl_fail(BGL_E_ARG, "bgl_bind: kind %d needs scales", w->kind);
    if (w->kind == BGL_Q4G256SF && !w->sub) return bgl_fail(BGL_E_ARG, "bgl_bind: g256sf needs sub-codes");
    if (w->kind == BGL_Q4G64A && !w->sub) return bgl_fail(BGL_E_ARG, "bgl_bind: int4 affine needs biases (sub)");
    HIPCHK(hipSetDevice(c->device));
    size_t pb = ref_packed_bytes(w->kind, w->bits, w->out, w->in), sb = ref_scale_bytes(w->kind, w->out, w->in);
    size_t subb = w->kind == BGL_Q4G256SF ? (size_t)w->out * (w->in / 64)
                : w->kind == BGL_Q4G64A ? (size_t)w->out * (w->in / 64) * 4 : 0;
    void *dpk = nullptr, *dsc = nullptr, *dsub = nullptr;
    HIPCHK(hipMalloc(&dpk, pb));
    if (sb) HIPCHK(hipMalloc(&dsc, sb));
    if (subb) HIPCHK(hipMalloc(&dsub, subb));
    HIPCHK(hipMemcpyAsync(dpk, w->packed, pb, hipMemcpyHostToDevice, c->stream));
    if (sb) HIPCHK(hipMemcpyAsync(dsc, w->scales, sb, hipMemcpyHostToDevice, c->stream));
    if (subb) HIPCHK(hipMemcpyAsync(dsub, w->sub, subb, hipMemcpyHostToDevice, c->stream));
    rc = repack_into(c, w->kind, w->bits, w->out, w->in, dpk, dsc, (const uint8_t *)dsub, out);
    hipError_t e = hipStreamSynchronize(c->stream);
    (void)hipFree(dpk); (void)hipFree(dsc);
    if (dsub) (void)hipFree(dsub);
    if (rc) return rc;
    if (e != hipSuccess) return bgl_fail(BGL_E_HIP, "bind sync: %s", hipGetErrorString(e));
    return 0;
}

// The checks of the mixed binders (mlx_moe.cpp:1750-1758 / :1790-1798): offsets[0] = 0,
// offsets[cells] = planes_bytes, each cell exactly n*8 bytes with 2 <= n <= 15, scales finite and > 0.
static int mixed_check(const uint8_t *planes, long planes_bytes, const uint32_t *offsets, const uint8_t *bits,
                       const float *scales, long out, long in, int *W) {
    if (!planes || !offsets || !bits || !scales || planes_bytes <= 0 || out <= 0 || in <= 0 || in % 64)
        return bgl_fail(BGL_E_ARG, "mixed qNg64: bad argument (in %% 64 == 0, buffers non-NULL)");
    const long ng = in / 64;
    const size_t cells = (size_t)out * (size_t)ng;
    if (offsets[0] != 0 || (long)offsets[cells] != planes_bytes)
        return bgl_fail(BGL_E_ARG, "mixed qNg64: offsets[0] must be 0 and offsets[%zu] = planes_bytes", cells);
    int w = 2;
    for (size_t i = 0; i < cells; ++i) {
        const int n = (int)bits[i];
        if (n < 2 || n > 15) return bgl_fail(BGL_E_ARG, "mixed qNg64: cell %zu has n=%d (2..15)", i, n);
        if (offsets[i + 1] < offsets[i] || (size_t)(offsets[i + 1] - offsets[i]) != (size_t)n * 8u)
            return bgl_fail(BGL_E_ARG, "mixed qNg64: cell %zu spans %u bytes, not n*8", i, offsets[i + 1] - offsets[i]);
        if (!std::isfinite(scales[i]) || scales[i] <= 0.0f) return bgl_fail(BGL_E_ARG, "mixed qNg64: cell %zu scale", i);
        if (n > w) w = n;
    }
    *W = w;
    return 0;
}

extern "C" int bgl_bind_qng64_mixed(bgl_ctx *c, const uint8_t *planes, long planes_bytes, const uint32_t *offsets,
                                    const uint8_t *bits, const float *scales, int out, int in, bgl_tensor **res) {
    if (!c || !res) return bgl_fail(BGL_E_ARG, "bgl_bind_qng64_mixed: NULL argument");
    int W = 0, rc = mixed_check(planes, planes_bytes, offsets, bits, scales, out, in, &W);
    if (rc) return rc;
    HIPCHK(hipSetDevice(c->device));
    const size_t cells = (size_t)out * (in / 64);
    void *dpl = nullptr, *doff = nullptr, *dbits = nullptr, *dsc = nullptr, *dense = nullptr;
    hipError_t e = hipMalloc(&dpl, planes_bytes);
    if (e == hipSuccess) e = hipMalloc(&doff, (cells + 1) * 4);
    if (e == hipSuccess) e = hipMalloc(&dbits, cells);
    if (e == hipSuccess) e = hipMalloc(&dsc, cells * 4);
    if (e == hipSuccess) e = hipMalloc(&dense, cells * W * 8);
    if (e == hipSuccess) e = hipMemcpyAsync(dpl, planes, planes_bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(doff, offsets, (cells + 1) * 4, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(dbits, bits, cells, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(dsc, scales, cells * 4, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(k_mixed_qng_to_dense, dim3(nblk((long)cells)), dim3(256), 0, c->stream, (const uint8_t *)dpl,
                           (const uint32_t *)doff, (const uint8_t *)dbits, (long)cells, W, (uint8_t *)dense);
        e = hipGetLastError();
    }
    rc = e == hipSuccess ? repack_into(c, BGL_QNG64, W, out, in, dense, dsc, nullptr, res)
                         : bgl_fail(BGL_E_HIP, "bgl_bind_qng64_mixed: %s", hipGetErrorString(e));
    const hipError_t es = hipStreamSynchronize(c->stream);
    for (void *p : {dpl, doff, dbits, dsc, dense})
        if (p) (void)hipFree(p);
    if (rc) return rc;
    if (es != hipSuccess) return bgl_fail(BGL_E_HIP, "bgl_bind_qng64_mixed sync: %s", hipGetErrorString(es));
    return 0;
}

extern "C" int bgl_quantize_dev(bgl_ctx *c, int kind, int bits, int qng64_encoder, const float *w_dev, int out, int in,
                                bgl_tensor **t, void *ref_packed, void *ref_scales, uint8_t *ref_sub) {
    if (!c || !w_dev || !t) return bgl_fail(BGL_E_ARG, "bgl_quantize_dev: NULL argument");
    int rc = check_wt(kind, bits, out, in);
    if (rc) return rc;
    if (kind == BGL_Q4G64A || kind == BGL_F16 || kind == BGL_F32 || kind == BGL_MXFP4 || kind == BGL_K_Q4G256P)
        return bgl_fail(BGL_E_UNSUPPORTED, "bgl_quantize_dev: kind %d has no packer here (bind its bytes with bgl_bind)", kind);
    if (kind == BGL_QNG64 && qng64_encoder && bits == 4)
        return bgl_fail(BGL_E_ARG, "qng64_quantize_f32 rejects n=4 (qng64_dense.c:9)");
    HIPCHK(hipSetDevice(c->device));
    size_t pb = ref_packed_bytes(kind, bits, out, in), sb = ref_scale_bytes(kind, out, in);
    size_t subb = kind == BGL_Q4G256SF ? (size_t)out * (in / 64) : 0;
    void *dpk = nullptr, *dsc = nullptr, *dsub = nullptr;
    HIPCHK(hipMalloc(&dpk, pb));
    HIPCHK(hipMalloc(&dsc, sb));
    if (subb) HIPCHK(hipMalloc(&dsub, subb));
    long units;
    switch (kind) {
    case BGL_Q4G64:
        units = (long)out * (in / 64);
        hipLaunchKernelGGL(k_quant_q4g64, dim3(nblk(units)), dim3(256), 0, c->stream, w_dev, out, in, (uint8_t *)dpk, (float *)dsc);
        break;
    case BGL_Q8G64:
        units = (long)out * (in / 64);
        hipLaunchKernelGGL(k_quant_q8g64, dim3(nblk(units)), dim3(256), 0, c->stream, w_dev, out, in, (int8_t *)dpk, (float *)dsc);
        break;
    case BGL_QNG64:
        units = (long)out * (in / 64);
        hipLaunchKernelGGL(k_quant_qng64, dim3(nblk(units, 64)), dim3(64), 0, c->stream, w_dev, out, in, bits, qng64_encoder ? 1 : 0,
                           (uint8_t *)dpk, (float *)dsc);
        break;
    case BGL_Q4G32H:
        units = (long)out * (in / 32);
        hipLaunchKernelGGL(k_quant_q4g32h, dim3(nblk(units)), dim3(256), 0, c->stream, w_dev, out, in, (uint8_t *)dpk, (uint16_t *)dsc);
        break;
    case BGL_Q4G256SF:
        units = (long)out * (in / 256);
        hipLaunchKernelGGL(k_quant_g256sf, dim3(nblk(units, 64)), dim3(64), 0, c->stream, w_dev, out, in, (uint8_t *)dpk, (float *)dsc,
                           (uint8_t *)dsub);
        break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) rc = bgl_fail(BGL_E_HIP, "quantize launch: %s", hipGetErrorString(e));
    if (!rc) rc = repack_into(c, kind, bits, out, in, dpk, dsc, (const uint8_t *)dsub, t);
    if (!rc && ref_packed) rc = hipMemcpyAsync(ref_packed, dpk, pb, hipMemcpyDeviceToHost, c->stream) ? BGL_E_HIP : 0;
    if (!rc && ref_scales) rc = hipMemcpyAsync(ref_scales, dsc, sb, hipMemcpyDeviceToHost, c->stream) ? BGL_E_HIP : 0;
    if (!rc && ref_sub && subb) rc = hipMemcpyAsync(ref_sub, dsub, subb, hipMemcpyDeviceToHost, c->stream) ? BGL_E_HIP : 0;
    e = hipStreamSynchronize(c->stream);
    (void)hipFree(dpk); (void)hipFree(dsc);
    if (dsub) (void)hipFree(dsub);
    if (rc) return rc == BGL_E_HIP ? bgl_fail(BGL_E_HIP, "quantize copy-back failed") : rc;
    if (e != hipSuccess) return bgl_fail(BGL_E_HIP, "quantize sync: %s", hipGetErrorString(e));
    return 0;
}

extern "C" void bgl_tensor_free(bgl_tensor *t) {
    if (!t) return;
    for (void *p : t->owned) if (p) (void)hipFree(p);
    for (bgl_tensor *e : t->experts) bgl_tensor_free(e);
    delete t;
}

extern "C" int bgl_tensor_info(const bgl_tensor *t, int *kind, int *bits, int *out, int *in, size_t *device_bytes) {
    if (!t) return bgl_fail(BGL_E_ARG, "bgl_tensor_info: NULL tensor");
    if (!t->experts.empty()) {
        if (kind) *kind = 0;
        if (bits) *bits = 0;
        if (out) *out = t->experts[0]->T.N;
        if (in) *in = t->experts[0]->T.K;
        if (device_bytes) { size_t s = 0; for (auto *e : t->experts) s += e->device_bytes; *device_bytes = s; }
        return 0;
    }
    if (kind) *kind = t->T.fmt == BGL_Q4G256SF && t->T.gmul == 1.0f ? BGL_K_Q4G256P : t->T.fmt;
    if (bits) *bits = t->T.bits;
    if (out) *out = t->T.N;
    if (in) *in = t->T.K;
    if (device_bytes) *device_bytes = t->device_bytes;
    return 0;
}

extern "C" int bgl_dequant_dev(bgl_ctx *c, const bgl_tensor *t, int row0, int nrows, float *out_dev) {
    if (!c || !t || !out_dev || !t->experts.empty()) return bgl_fail(BGL_E_ARG, "bgl_dequant_dev: bad argument");
    if (row0 < 0 || nrows <= 0 || row0 + nrows > t->T.N) return bgl_fail(BGL_E_ARG, "bgl_dequant_dev: rows out of range");
    hipLaunchKernelGGL(k_dequant, dim3(nblk((long)nrows * t->T.K)), dim3(256), 0, c->stream, t->T, row0, nrows, out_dev);
    HIPCHK(hipGetLastError());
    return 0;
}

// ------------------------------------------------------------------ activation prep
// g256sf and plain g256 (same device format, gmul = 1) quantize their activations per 256 values
static int act_group(int kind) { return kind == BGL_Q4G256SF || kind == BGL_K_Q4G256P ? 256 : 64; }

// The fp32-activation operands of M prepared columns of length K: k_act_x24 writes level 0 of all
// M columns and then level 1 into each of the three buffers.
void f32_act_ptrs(const void *xw, const void *xs, const void *xsum, int M, int K, const float *x_dev, GemvAct &A) {
    const size_t ng = (size_t)K / 64;
    A.xw = (const int *)xw; A.xs = (const float *)xs; A.xsum = (const int *)xsum;
    A.xw1 = A.xw + (size_t)M * ng * BGL_XD_DW;
    A.xs1 = A.xs + (size_t)M * ng;
    A.xsum1 = A.xsum + (size_t)M * (K / 32) * 4;
    A.xf = x_dev;
    A.gq = 64;
}

int prep_act(bgl_ctx *c, int act, int gq, const float *x_dev, int M, int K, GemvAct &A) {
    memset(&A, 0, sizeof A);
    if (act == BGL_ACT_F32) {
        int ng = K / 64;
        if (dbuf_reserve(c, c->act_w, (size_t)2 * M * ng * 192, false) || dbuf_reserve(c, c->act_s, (size_t)2 * M * ng * 4, false) ||
            dbuf_reserve(c, c->act_sum, (size_t)2 * M * (K / 32) * 16, false))
            return bgl_last_code();
        int tok = prof_begin(c, 0);
        hipLaunchKernelGGL(k_act_x24, dim3(nblk((long)M * ng * 64)), dim3(256), 0, c->stream, x_dev, M, K,
                           (int8_t *)c->act_w.p, (float *)c->act_s.p, (int *)c->act_sum.p);
        prof_end(c, tok);
    } else {
        if (dbuf_reserve(c, c->act_w, (size_t)M * K, false) || dbuf_reserve(c, c->act_s, (size_t)M * (K / gq) * 4, false) ||
            dbuf_reserve(c, c->act_sum, (size_t)M * (K / 64) * 4, false))
            return bgl_last_code();
        int tok = prof_begin(c, 0);
        hipLaunchKernelGGL(k_act_w4a8, dim3(nblk((long)M * (K / gq) * 64)), dim3(256), 0, c->stream, x_dev, M, K, gq,
                           (int8_t *)c->act_w.p, (float *)c->act_s.p, (int *)c->act_sum.p, c->prep_u, c->prep_h);
        prof_end(c, tok);
    }
    HIPCHK(hipGetLastError());
    c->prep_act = act; c->prep_gq = gq; c->prep_M = M; c->prep_K = K; c->prep_x = x_dev;
    c->prep_reuse = false;                 // a GEMV call's own operands: x_dev is the caller's, valid for that call only
    if (act == BGL_ACT_F32) {
        f32_act_ptrs(c->act_w.p, c->act_s.p, c->act_sum.p, M, K, x_dev, A);
    } else {
        A.xw = (const int *)c->act_w.p;
        A.xs = (const float *)c->act_s.p;
        A.xsum = (const int *)c->act_sum.p;
        A.gq = gq;
    }
    return 0;
}

extern "C" int bgl_quant_act_i8_dev(bgl_ctx *c, const float *x_dev, int M, int in, int gsize, int8_t *xq_dev, float *ascale_dev) {
    if (!c || !x_dev || !xq_dev || !ascale_dev || M <= 0) return bgl_fail(BGL_E_ARG, "bgl_quant_act_i8_dev: bad argument");
    if ((gsize != 64 && gsize != 256) || in % gsize) return bgl_fail(BGL_E_ARG, "bgl_quant_act_i8_dev: in=%d gsize=%d", in, gsize);
    if (dbuf_reserve(c, c->act_sum, (size_t)M * (in / 64) * 4, false)) return bgl_last_code();
    hipLaunchKernelGGL(k_act_w4a8, dim3(nblk((long)M * (in / gsize) * 64)), dim3(256), 0, c->stream, x_dev, M, in, gsize, xq_dev,
                       ascale_dev, (int *)c->act_sum.p, (const float *)nullptr, (float *)nullptr);
    HIPCHK(hipGetLastError());
    return 0;
}

// ------------------------------------------------------------------ GEMV planning + launch
// Waves per workgroup: one per work unit up to 16 (BGL_MAX_WAVES overrides the cap).
int pick_waves(bgl_ctx *c, int nunits) {
    int cap = c->max_waves;
    return nunits < cap ? (nunits < 1 ? 1 : nunits) : cap;
}

static void fill_tasks(GemvLaunch &L, int n, const BglDevTensor *Ts, const float *const *bias, float *const *y,
                       const int *ystride, int &blocks) {
    L.ntasks = n;
    blocks = 0;
    for (int i = 0; i < n; i++) {
        GemvTask &t = L.t[i];
        t.T = Ts[i];
        t.y = y[i];
        t.bias = bias ? bias[i] : nullptr;
        t.ystride = ystride ? ystride[i] : Ts[i].N;
        t.blk0 = blocks;
        t.ks = 1;
        t.gpb = Ts[i].nunits;
        t.part = nullptr;
        blocks += Ts[i].ntiles;
    }
}

#define BGL_GEMV_X_LDS_MAX (160 * 1024)
#define BGL_GEMV_X_FUSE_MAX_K 4096            // longer K: one prep kernel beats every workgroup making the digits

// One fp32-activation column through k_gemv_x (bgl_gemv_x.hip): workgroups of TR rows over the whole
// K range, waves taking slots of 64/TR groups in turn, so no launch needs a K split.  A: the prepared
// activation operands, or null to have every workgroup make them from the raw column x_dev.
// Returns 1 when the shape is not taken (the activation records of K would not fit LDS, or a tensor
// spans 2 GiB).
static int run_gemv_x(bgl_ctx *c, int n, const BglDevTensor *Ts, const GemvAct *A, const float *x_dev,
                      const float *const *bias, float *const *y, const int *ystride) {
    GemvLaunch L;
    memset(&L, 0, sizeof L);
    int blocks = 0;
    fill_tasks(L, n, Ts, bias, y, ystride, blocks);
    if (A) L.a = *A;
    L.x = x_dev;
    L.m0 = 0;
    L.mcols = 1;
    L.mtot = 1;
    // Shapes (measured on the cfg1 / cfg3 Q4G32H and qNg64 launches, n = 2..15): making the digits
    // costs every workgroup a pass over K, so those launches keep whole 64-row tiles (>= 128
    // workgroups) with up to 12 waves; with prepared digits the tiles split until >= 256 workgroups,
    // up to 16 waves.
    const bool fused = A == nullptr;
    int TR = 64;
    while (TR > 8 && (long)blocks * (BGL_TILE / TR) < (fused ? 128 : 256)) TR >>= 1;
    if (c->force_tr) TR = c->force_tr;
    const int KQ = BGL_TILE / TR, G = Ts[0].K / 64, S = (G + KQ - 1) / KQ;
    int nw = std::min({S, c->max_waves, fused ? 12 : 16});
    if (c->x_waves) nw = std::min(S, c->x_waves);
    if (bgl_gemv_x_lds(Ts[0].K, TR, nw, fused) > BGL_GEMV_X_LDS_MAX) return 1;
    for (int i = 0; i < n; i++)            // the kernel addresses each tensor through 32-bit buffer offsets
        if ((size_t)Ts[i].ntiles * Ts[i].cpr * 1024 >= (1ull << 31) || (size_t)Ts[i].ntiles * Ts[i].nunits * 512 >= (1ull << 31))
            return 1;
    for (int i = 0; i < n; i++) L.t[i].blk0 *= KQ;
    int tok = prof_begin(c, 1);
    int rc = bgl_launch_gemv_x(L, A == nullptr, blocks * KQ, TR, nw, c->stream);
    prof_end(c, tok);
    if (rc == -2) return bgl_fail(BGL_E_UNSUPPORTED, "kind %d bits %d: no fp32-activation kernel", Ts[0].fmt, Ts[0].bits);
    if (rc) return bgl_fail(BGL_E_ARG, "gemv_x launch: bad shape");
    HIPCHK(hipGetLastError());
    return 0;
}

static bool gemv_x_kind(int fmt) { return fmt == BGL_Q4G64 || fmt == BGL_Q4G32H || fmt == BGL_Q8G64 || fmt == BGL_QNG64; }

int run_gemv(bgl_ctx *c, int n, const BglDevTensor *Ts, int act, const GemvAct &A, int M,
             const float *const *bias, float *const *y, const int *ystride) {
    if (M == 1 && act == BGL_ACT_F32 && !c->no_gemv_x && gemv_x_kind(Ts[0].fmt)) {
        int rc = run_gemv_x(c, n, Ts, &A, nullptr, bias, y, ystride);
        if (rc <= 0) return rc;
    }
    GemvLaunch L;
    memset(&L, 0, sizeof L);
    int blocks = 0;
    fill_tasks(L, n, Ts, bias, y, ystride, blocks);
    L.a = A;
    L.mtot = M;
    // Few tiles and a long K: split K over workgroups (>= 8 units per slice) so the launch keeps
    // enough wavefronts in flight; a second small kernel sums the slices in order.  The extra
    // launch (~2 us) pays only when at most a quarter of the target workgroups exist (measured:
    // 24 and 64 tiles gain 1.4-1.7x; 140 and 224 tiles lose 10-20%).
    int ks = 1;
    if (n == 1 && blocks <= c->min_blocks / 4 && Ts[0].nunits >= 16) {
        ks = (c->min_blocks + blocks - 1) / blocks;
        if (ks > Ts[0].nunits / 8) ks = Ts[0].nunits / 8;
        if (ks < 1) ks = 1;
    }
    if (ks > 1) {
        GemvTask &t = L.t[0];
        t.gpb = (Ts[0].nunits + ks - 1) / ks;
        t.ks = (Ts[0].nunits + t.gpb - 1) / t.gpb;
        if (dbuf_reserve(c, c->part, (size_t)t.ks * M * Ts[0].N * 4, false)) return bgl_last_code();
        t.part = (float *)c->part.p;
        blocks *= t.ks;
    }
    const int nw = pick_waves(c, L.t[0].gpb);
    for (int m0 = 0; m0 < M;) {
        int r = M - m0, MB, mc;
        if (r >= 5) { MB = 8; mc = r < 8 ? r : 8; }
        else if (r >= 2) { MB = 4; mc = r; }
        else { MB = 1; mc = 1; }
        L.m0 = m0;
        L.mcols = mc;
        int tok = prof_begin(c, 1);
        int rc = bgl_launch_gemv(act, MB, L, blocks, nw, c->stream);
        prof_end(c, tok);
        if (rc == -2) return bgl_fail(BGL_E_UNSUPPORTED, "kind %d does not support activation mode %d", Ts[0].fmt, act);
        if (rc) return bgl_fail(BGL_E_ARG, "gemv launch: bad column block");
        HIPCHK(hipGetLastError());
        m0 += mc;
    }
    if (L.t[0].ks > 1) {
        const GemvTask &t = L.t[0];
        int tok = prof_begin(c, 1);
        hipLaunchKernelGGL(k_splitk_reduce, dim3(nblk((long)M * t.T.N)), dim3(256), 0, c->stream, (const float *)t.part, t.ks, M,
                           t.T.N, t.bias, t.y, t.ystride);
        prof_end(c, tok);
        HIPCHK(hipGetLastError());
    }
    return 0;
}

#define BGL_GEMV_Q_LDS_MAX (64 * 1024)          // one column: two workgroups of the largest shapes per CU
#define BGL_Q_PREP_MIN_PASSES 64                // W4A8 calls with this many passes of 256 values per launch quantize up front
#define BGL_GEMV_Q_LDS_MAX_MB (160 * 1024)      // 4 or 8 columns: the codes of every column sit in LDS

static int q_mb(int mc) { return mc <= 1 ? 1 : mc <= 4 ? 4 : 8; }
static size_t q_lds_max(int MB) { return MB == 1 ? BGL_GEMV_Q_LDS_MAX : BGL_GEMV_Q_LDS_MAX_MB; }
// The widest launch (8, 4 or 1 columns) whose LDS fits at 8 rows per workgroup; 0: none does.
static int q_mb_max(int kind, int K) {
    for (int MB : {8, 4, 1})
        if (bgl_gemv_q_lds(kind, K, 8, MB) <= q_lds_max(MB)) return MB;
    return 0;
}

// W4A8 with the quantization fused in, M columns in launches of up to 8 -- fewer where the
// columns' codes would not fit LDS (each launch streams the weights once for its columns; every
// column's arithmetic is the one-column kernel's).
// Launch shape of the matrix-core W4A8 kernel (k_gemv_qm): RB 16-row blocks and S unit slices per
// workgroup.  With the columns quantized in the kernel, the row blocks of one tile share that work
// (4 blocks while that still leaves >= 256 workgroups) and 8 waves split it; with prepared codes a
// workgroup is one block with up to 8 slices.
static void qm_shape(bgl_ctx *c, int nrb, int U, bool prep, int &RB, int &S) {
    RB = prep ? 1 : (nrb / 4 >= 256 ? 4 : nrb / 2 >= 256 ? 2 : 1);
    S = prep ? std::min(U, 16) : RB == 1 ? 12 : 8 / RB;
    const int rb = prep ? c->qm_prb : c->qm_rb, s = prep ? c->qm_ps : c->qm_s;
    if (rb == 1 || rb == 2 || rb == 4) RB = rb;
    if (s > 0) S = std::min(s, 16 / RB);
}

#define QM_MIN_COLS 5

static bool qm_ok(bgl_ctx *c, int kind, int K) {
    if (c->no_qmfma) return false;
    if (kind == BGL_Q4G256SF) return K % 256 == 0;
    return (kind == BGL_Q4G64 || kind == BGL_Q8G64) && K % 64 == 0;
}

static int run_gemv_q(bgl_ctx *c, int n, const BglDevTensor *Ts, const float *x_dev, int M, const float *const *bias,
                      float *const *y) {
    // 5..16 columns: the matrix-core kernel (one MFMA column per activation column), where its
    // terms (and, quantizing in the kernel, the columns' codes) fit LDS.  (Qwen2.5-1.5B g256sf cfg2
    // step: 8 columns 1.239 -> 1.115 ms; at 4 columns the dot4 kernel stays ahead, 0.957 against
    // 0.983 ms.)
    bool qm = M >= QM_MIN_COLS && qm_ok(c, Ts[0].fmt, Ts[0].K);
    if (qm) {
        const int pass16 = std::min(M, 16) * ((Ts[0].K + 255) / 256);
        const bool p16 = c->q_prep == 1 || (c->q_prep < 0 && pass16 >= BGL_Q_PREP_MIN_PASSES);
        const bool fit_nq = bgl_gemv_qm_lds(Ts[0].fmt, Ts[0].K, std::min(M, 16), 1, false) <= BGL_GEMV_Q_LDS_MAX;
        qm = bgl_gemv_qm_lds(Ts[0].fmt, Ts[0].K, std::min(M, 16), 1, true) <= BGL_GEMV_Q_LDS_MAX && (p16 || fit_nq || c->q_prep != 0);
    }
    const int mbq = q_mb_max(Ts[0].fmt, Ts[0].K);            // columns per dot4 launch
    const int mbmax = qm ? 16 : mbq;
    // Several columns over a long K: one k_act_w4a8 launch quantizes them all (the same codes)
    // instead of every workgroup quantizing every column of its launch.  (Measured on Qwen2.5-1.5B
    // g256sf: the down projection, 4 x 35 and 8 x 35 passes per workgroup, 10.95 -> 9.57 and
    // 17.75 -> 11.38 us; for 8 x 6 passes and fewer the extra launch costs more than it saves.)
    GemvAct A;
    memset(&A, 0, sizeof A);
    const int passes = std::min(M, mbmax) * ((Ts[0].K + 255) / 256);
    bool prep = M > 1 && (c->q_prep == 1 || (c->q_prep < 0 && passes >= BGL_Q_PREP_MIN_PASSES));
    if (qm && !prep && bgl_gemv_qm_lds(Ts[0].fmt, Ts[0].K, std::min(M, 16), 1, false) > BGL_GEMV_Q_LDS_MAX) prep = true;
    if (prep) {
        int rc = prep_act(c, BGL_ACT_W4A8, act_group(Ts[0].fmt), x_dev, M, Ts[0].K, A);
        if (rc) return rc;
    }
    for (int m0 = 0; m0 < M;) {
        const bool qml = qm && M - m0 >= QM_MIN_COLS;
        const int mc = std::min(qml ? 16 : mbq, M - m0), MB = q_mb(mc);
        m0 += mc;
        if (qml) {
            GemvLaunch L;
            memset(&L, 0, sizeof L);
            int blocks = 0;
            fill_tasks(L, n, Ts, bias, y, nullptr, blocks);
            L.x = c->prep_h ? c->prep_h : x_dev;
            if (prep) L.a = A;
            L.m0 = m0 - mc;
            L.mcols = mc;
            int RB, S;
            qm_shape(c, blocks * 4, Ts[0].nunits, prep, RB, S);
            while (RB > 1 && bgl_gemv_qm_lds(Ts[0].fmt, Ts[0].K, mc, RB, prep) > BGL_GEMV_Q_LDS_MAX) RB >>= 1;
            for (int i = 0; i < n; i++) L.t[i].blk0 *= 4 / RB;
            int tok = prof_begin(c, 1);
            int rc = bgl_launch_gemv_qm(L, blocks * (4 / RB), RB, S, prep, c->stream);
            prof_end(c, tok);
            if (rc) return bgl_fail(BGL_E_UNSUPPORTED, "matrix-core W4A8 path: kind %d", Ts[0].fmt);
            HIPCHK(hipGetLastError());
            continue;
        }
        GemvLaunch L;
        memset(&L, 0, sizeof L);
        int blocks = 0;
        fill_tasks(L, n, Ts, bias, y, nullptr, blocks);
        L.x = c->prep_h ? c->prep_h : x_dev;     // a SwiGLU column: h, which the prep launch wrote
        if (prep && MB > 1) L.a = A;
        L.m0 = m0 - mc;
        L.mcols = mc;
        // Rows per workgroup: split 64-row tiles until the launch has >= 512 workgroups (8 rows at
        // the least), so the weight stream is spread over every CU.  Waves: ceil(passes / 4), at
        // least 3, since every workgroup quantizes the whole activation; the waves take the weight
        // units in turn (the last ones only quantize when there are fewer units than waves).
        // (Measured on 1536x1536, 2048x1536, 17920x1536 and 1536x8960 g256sf launches at one column:
        // the best shape found for each, or within 0.05 us of it.)
        int TR = 64;
        while (TR > 8 && (long)blocks * (BGL_TILE / TR) < 512) TR >>= 1;
        if (c->force_tr) TR = c->force_tr;
        while (TR > 8 && bgl_gemv_q_lds(Ts[0].fmt, Ts[0].K, TR, MB) > q_lds_max(MB)) TR >>= 1;   // the t[u][row] terms shrink with TR
        const int KQ = BGL_TILE / TR, NP = (Ts[0].K + 255) / 256;
        int nw = std::min(16, std::max(3, (MB * NP + 3) / 4));
        // 8 columns quantized in the kernel by >= 512 workgroups: 4 waves (Qwen2.5-1.5B gate+up,
        // 560 workgroups x 48 passes: 18.2 us with 12 waves, 15.7 with 4; the 256- and 192-
        // workgroup q/k/v and o launches run best with 12)
        if (MB == 8 && !(prep && MB > 1) && (long)blocks * KQ >= 512) nw = std::min(nw, 4);
        if (nw > c->max_waves) nw = c->max_waves;
        // every task block of the launch uses the same TR; remap blk0 to workgroup units
        for (int i = 0; i < n; i++) L.t[i].blk0 *= KQ;
        int tok = prof_begin(c, 1);
        int rc = bgl_launch_gemv_q(L, blocks, TR, nw, MB, c->stream);
        prof_end(c, tok);
        if (rc) return bgl_fail(BGL_E_UNSUPPORTED, "fused W4A8 path: kind %d", Ts[0].fmt);
        HIPCHK(hipGetLastError());
    }
    return 0;
}

// The MLP block's down projection at M > 1 W4A8 columns when its columns are quantized up front:
// that one launch also forms h = SwiGLU(g, u) (k_act_w4a8 with u), writing h, so the block needs
// no SwiGLU launch.  Returns 1 (nothing launched) where the down projection would not quantize up
// front; the caller then runs the SwiGLU itself.
int run_down_swiglu_w4a8(bgl_ctx *c, const BglDevTensor &down, const float *g, const float *u, float *h, int M, float *y) {
    if (c->no_fused || M < 2) return 1;
    const int kind = down.fmt, K = down.K;
    if (kind != BGL_Q4G256SF && kind != BGL_Q4G64 && kind != BGL_Q8G64) return 1;
    const int mbmax = q_mb_max(kind, K);
    if (mbmax < 2) return 1;
    const int passes = std::min(M, mbmax) * ((K + 255) / 256);
    if (!(c->q_prep == 1 || (c->q_prep < 0 && passes >= BGL_Q_PREP_MIN_PASSES))) return 1;
    c->prep_u = u;
    c->prep_h = h;
    const float *nob[1] = {nullptr};
    float *ys[1] = {y};
    const int rc = run_gemv_q(c, 1, &down, g, M, nob, ys);
    c->prep_u = nullptr;
    c->prep_h = nullptr;
    return rc;
}

static bool fused_q_ok(bgl_ctx *c, int kind, int K, int M) {
    (void)M;
    if (c->no_fused) return false;
    if (kind != BGL_Q4G256SF && kind != BGL_Q4G64 && kind != BGL_Q8G64) return false;
    return q_mb_max(kind, K) > 0;
}


extern "C" int bgl_matmul_group_dev(bgl_ctx *c, int n, const bgl_tensor *const *w, int act, const float *x_dev,
                                    const float *const *bias_dev, float *const *y_dev, int M) {
    if (!c || n < 1 || n > BGL_MAX_TASKS || !w || !x_dev || !y_dev || M < 1) return bgl_fail(BGL_E_ARG, "bgl_matmul_group_dev: bad argument");
    if (act != BGL_ACT_F32 && act != BGL_ACT_W4A8) return bgl_fail(BGL_E_ARG, "unknown activation mode %d", act);
    BglDevTensor Ts[BGL_MAX_TASKS];
    for (int i = 0; i < n; i++) {
        if (!w[i] || !w[i]->experts.empty() || !y_dev[i]) return bgl_fail(BGL_E_ARG, "bgl_matmul_group_dev: tensor %d invalid", i);
        Ts[i] = w[i]->T;
        if (Ts[i].K != Ts[0].K || Ts[i].fmt != Ts[0].fmt || Ts[i].bits != Ts[0].bits || Ts[i].gmul != Ts[0].gmul)
            return bgl_fail(BGL_E_ARG, "bgl_matmul_group_dev: fused tensors must share kind, bits and in");
    }
    const int kind = Ts[0].fmt;
    if (kind == BGL_Q4G64A || kind == BGL_F16 || kind == BGL_F32 || kind == BGL_MXFP4)
        return bgl_fail(BGL_E_UNSUPPORTED, "kind %d runs in the MoE gather only (bgl_gather_matvec_dev / bgl_moe_ffn_dev)", kind);
    if (kind == BGL_Q4G256SF && act != BGL_ACT_W4A8)
        return bgl_fail(BGL_E_UNSUPPORTED, "K_Q4G256SF requires W4A8 activations -- no fp32-activation path exists for g256sf");
    if ((kind == BGL_Q4G32H || kind == BGL_QNG64) && act != BGL_ACT_F32)
        return bgl_fail(BGL_E_UNSUPPORTED, "kind %d has fp32-activation kernels only", kind);
    HIPCHK(hipSetDevice(c->device));
    if (act == BGL_ACT_W4A8 && fused_q_ok(c, kind, Ts[0].K, M)) return run_gemv_q(c, n, Ts, x_dev, M, bias_dev, y_dev);
    if (act == BGL_ACT_F32 && M >= BGL_MFMA_MIN_M && !c->no_mfma) {
        bool ok = true;
        for (int i = 0; i < n; i++) ok = ok && bgl_mfma_ok(Ts[i].fmt, Ts[i].bits);
        if (ok) return run_gemm_mfma(c, n, Ts, x_dev, M, bias_dev, y_dev, nullptr);
    }
    // one fp32 column over a short K: the GEMV makes the activation digits itself (no prep launch)
    if (act == BGL_ACT_F32 && M == 1 && !c->no_gemv_x && gemv_x_kind(kind) &&
        (c->x_fuse == 1 || (c->x_fuse < 0 && Ts[0].K <= BGL_GEMV_X_FUSE_MAX_K))) {
        int rc = run_gemv_x(c, n, Ts, nullptr, x_dev, bias_dev, y_dev, nullptr);
        if (rc <= 0) return rc;
    }
    GemvAct A;
    int rc = prep_act(c, act, act_group(kind), x_dev, M, Ts[0].K, A);
    if (rc) return rc;
    return run_gemv(c, n, Ts, act, A, M, bias_dev, y_dev, nullptr);
}

// bgl_matmul_group_dev with every per-call scratch buffer (activation digits and codes, K-split
// partials) carved from this GPU's fixed array instead of the context's allocations: no hipMalloc,
// hipFree or memset.  The context's own scratch and prepared-activation state are left as they
// were.  Every call on one GPU shares the array and leaves its contents behind (no path here
// reads scratch it has not written in the same call); calls that overlap on one GPU -- two
// contexts or streams at once -- race on it.
extern "C" int bgl_matmul_group_noalloc_dev(bgl_ctx *c, int n, const bgl_tensor *const *w, int act, const float *x_dev,
                                            const float *const *bias_dev, float *const *y_dev, int M) {
    if (!c) return bgl_fail(BGL_E_ARG, "bgl_matmul_group_noalloc_dev: NULL context");
    uint8_t *base = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        base = c->device >= 0 && c->device < BGL_MAX_DEVICES ? g_scratch_ptr[c->device] : nullptr;
    }
    if (!base) return bgl_fail(BGL_E_HIP, "bgl_matmul_group_noalloc_dev: no fixed scratch on device %d", c->device);
    const DevBuf aw = c->act_w, as = c->act_s, asum = c->act_sum, part = c->part;
    const int pa = c->prep_act, pg = c->prep_gq, pm = c->prep_M, pk = c->prep_K;
    const float *px = c->prep_x;
    const bool pr = c->prep_reuse;
    const bool prof = c->prof;
    c->act_w = c->act_s = c->act_sum = c->part = DevBuf{};
    c->fixed_base = base; c->fixed_cap = BGL_NOALLOC_SCRATCH_BYTES; c->fixed_used = 0;
    c->prof = false;                        // event brackets would create events
    const int rc = bgl_matmul_group_dev(c, n, w, act, x_dev, bias_dev, y_dev, M);
    c->fixed_base = nullptr; c->fixed_cap = 0; c->fixed_used = 0;
    c->act_w = aw; c->act_s = as; c->act_sum = asum; c->part = part;
    c->prep_act = pa; c->prep_gq = pg; c->prep_M = pm; c->prep_K = pk; c->prep_x = px; c->prep_reuse = pr;
    c->prof = prof;
    return rc;
}

extern "C" int bgl_prep_act_dev(bgl_ctx *c, int act, int kind, const float *x_dev, int M, int in) {
    if (!c || !x_dev || M < 1) return bgl_fail(BGL_E_ARG, "bgl_prep_act_dev: bad argument");
    if (act != BGL_ACT_F32 && act != BGL_ACT_W4A8) return bgl_fail(BGL_E_ARG, "unknown activation mode %d", act);
    const int gq = act_group(kind);
    if (in % 64 || in % gq) return bgl_fail(BGL_E_ARG, "bgl_prep_act_dev: in=%d not a multiple of the group", in);
    HIPCHK(hipSetDevice(c->device));
    GemvAct A;
    const float *src = x_dev;
    if (act == BGL_ACT_F32) {
        // The fp32 GEMVs read the raw columns again for groups holding NaN / +-Inf: keep a copy in the
        // context, so x_dev may be reused or freed once this call is ordered on the stream.
        const size_t xb = (size_t)M * in * sizeof(float);
        if (dbuf_reserve(c, c->prep_xc, xb, false)) return bgl_last_code();
        HIPCHK(hipMemcpyAsync(c->prep_xc.p, x_dev, xb, hipMemcpyDeviceToDevice, c->stream));
        src = (const float *)c->prep_xc.p;
    }
    const int rc = prep_act(c, act, gq, src, M, in, A);
    if (rc) return rc;
    if (act != BGL_ACT_F32) c->prep_x = nullptr;
    c->prep_reuse = true;
    return 0;
}

extern "C" int bgl_matmul_prepped_dev(bgl_ctx *c, const bgl_tensor *w, int act, const float *bias_dev, float *y_dev, int M) {
    if (!c || !w || !y_dev || !w->experts.empty()) return bgl_fail(BGL_E_ARG, "bgl_matmul_prepped_dev: bad argument");
    const BglDevTensor &T = w->T;
    if (T.fmt == BGL_Q4G64A || T.fmt == BGL_F16 || T.fmt == BGL_F32 || T.fmt == BGL_MXFP4)
        return bgl_fail(BGL_E_UNSUPPORTED, "kind %d runs in the MoE gather only", T.fmt);
    const int kind = T.fmt == BGL_Q4G256SF && T.gmul == 1.0f ? BGL_K_Q4G256P : T.fmt;
    if (!c->prep_reuse || c->prep_act != act || c->prep_K != T.K || c->prep_gq != act_group(kind) || M > c->prep_M)
        return bgl_fail(BGL_E_ARG, "bgl_matmul_prepped_dev: no activation prepared by bgl_prep_act_dev matches (act %d, in %d, M %d)",
                        act, T.K, M);
    if (T.fmt == BGL_Q4G256SF && act != BGL_ACT_W4A8)
        return bgl_fail(BGL_E_UNSUPPORTED, "K_Q4G256SF requires W4A8 activations -- no fp32-activation path exists for g256sf");
    HIPCHK(hipSetDevice(c->device));
    GemvAct A;
    memset(&A, 0, sizeof A);
    if (act == BGL_ACT_F32) f32_act_ptrs(c->act_w.p, c->act_s.p, c->act_sum.p, c->prep_M, T.K, c->prep_x, A);
    else { A.xw = (const int *)c->act_w.p; A.xs = (const float *)c->act_s.p; A.xsum = (const int *)c->act_sum.p; A.gq = c->prep_gq; }
    const float *b[1] = {bias_dev};
    float *y[1] = {y_dev};
    return run_gemv(c, 1, &T, act, A, M, b, y, nullptr);
}

extern "C" int bgl_matmul_dev(bgl_ctx *c, const bgl_tensor *w, int act, const float *x_dev, const float *bias_dev,
                              float *y_dev, int M) {
    const float *b[1] = {bias_dev};
    float *y[1] = {y_dev};
    return bgl_matmul_group_dev(c, 1, &w, act, x_dev, b, y, M);
}

// ------------------------------------------------------------------ streaming-read probe
// A plain read of bound tensors' device bytes (chunks, scales, biases): the memory system's floor
// for the bytes a GEMV launch streams, measured beside it.  Grid-stride 16-byte loads, four in
// flight per thread; the xor of everything read is kept alive by an empty asm statement.
typedef unsigned int rp_u32x4 __attribute__((ext_vector_type(4)));
struct ReadSeg {
    const uint8_t *p;
    uint64_t n16;                       // 16-byte words
};
#define BGL_READ_PROBE_MAX_TENSORS 64   // a MoE gather launch's expert tensors (3 segments each)
struct ReadProbe {
    ReadSeg s[3 * BGL_READ_PROBE_MAX_TENSORS];
    int nseg;
};
static_assert(sizeof(ReadProbe) <= 3584, "the read probe's segment list travels as a kernel argument (<= 4 KB)");
__global__ __launch_bounds__(1024) void k_read_probe(ReadProbe P) {
    const uint64_t nt = (uint64_t)gridDim.x * blockDim.x, tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (int k = 0; k < P.nseg; k++) {
        const __attribute__((address_space(1))) rp_u32x4 *q = (const __attribute__((address_space(1))) rp_u32x4 *)P.s[k].p;
        const uint64_t n = P.s[k].n16;
        uint64_t i = tid;
        for (; i + 3 * nt < n; i += 4 * nt) {
            const rp_u32x4 a = q[i], b = q[i + nt], c = q[i + 2 * nt], d = q[i + 3 * nt];
            acc ^= (a.x ^ a.y ^ a.z ^ a.w) ^ (b.x ^ b.y ^ b.z ^ b.w) ^ (c.x ^ c.y ^ c.z ^ c.w) ^ (d.x ^ d.y ^ d.z ^ d.w);
        }
        for (; i < n; i += nt) {
            const rp_u32x4 a = q[i];
            acc ^= a.x ^ a.y ^ a.z ^ a.w;
        }
    }
    asm volatile("" ::"v"(acc));
}

extern "C" int bgl_read_probe_dev(bgl_ctx *c, int n, const bgl_tensor *const *w, int nblocks, int nthreads) {
    if (!c || n < 1 || n > BGL_READ_PROBE_MAX_TENSORS || !w)
        return bgl_fail(BGL_E_ARG, "bgl_read_probe_dev: bad argument (1 <= n <= %d tensors)", BGL_READ_PROBE_MAX_TENSORS);
    if (nblocks <= 0) nblocks = 1024;
    if (nthreads <= 0) nthreads = 256;
    if (nthreads > 1024 || nthreads % 64) return bgl_fail(BGL_E_ARG, "bgl_read_probe_dev: nthreads %d", nthreads);
    ReadProbe P;
    memset(&P, 0, sizeof P);
    for (int i = 0; i < n; i++) {
        if (!w[i] || !w[i]->experts.empty()) return bgl_fail(BGL_E_ARG, "bgl_read_probe_dev: tensor %d invalid", i);
        const BglDevTensor &T = w[i]->T;
        BglDevTensor L;
        size_t b[3];
        device_layout(T.fmt, T.bits, T.N, T.K, L, b);
        const void *ptr[3] = {T.w, T.s0, T.s1};
        for (int k = 0; k < 3; k++)
            if (b[k] && ptr[k]) P.s[P.nseg++] = ReadSeg{(const uint8_t *)ptr[k], (uint64_t)(b[k] / 16)};
    }
    HIPCHK(hipSetDevice(c->device));
    hipLaunchKernelGGL(k_read_probe, dim3(nblocks), dim3(nthreads), 0, c->stream, P);
    HIPCHK(hipGetLastError());
    return 0;
}

// ------------------------------------------------------------------ host-pointer drop-ins
// The device copy of a host weight, bound on first use and cached by its packed pointer.
static int host_tensor(bgl_ctx *c, const bgl_wt &wt, bgl_tensor **res) {
    int rc = check_wt(wt.kind, wt.bits, wt.out, wt.in);
    if (rc) return rc;
    HIPCHK(hipSetDevice(c->device));
    bgl_tensor *t = nullptr;
    {
        std::lock_guard<std::mutex> lk(c->mu);
        auto it = c->host_cache.find(wt.packed);
        if (it != c->host_cache.end()) {
            t = it->second;
            if (t->T.fmt != wt.kind || t->T.N != wt.out || t->T.K != wt.in || (wt.kind == BGL_QNG64 && t->T.bits != wt.bits))
                return bgl_fail(BGL_E_ARG, "cached tensor for %p has a different shape/kind (call bgl_forget first)", wt.packed);
        }
    }
    if (!t) {
        rc = bgl_bind(c, &wt, &t);
        if (rc) return rc;
        std::lock_guard<std::mutex> lk(c->mu);
        c->host_cache[wt.packed] = t;
    }
    *res = t;
    return 0;
}

static int host_call(bgl_ctx *c, const bgl_wt &wt, int act, const float *x, const float *bias, float *y, int M) {
    if (!c || !x || !y || M < 1) return bgl_fail(BGL_E_ARG, "NULL argument");
    bgl_tensor *t = nullptr;
    int rc = host_tensor(c, wt, &t);
    if (rc) return rc;
    size_t xb = (size_t)M * wt.in * 4, yb = (size_t)M * wt.out * 4;
    if (dbuf_reserve(c, c->hx, xb, false) || dbuf_reserve(c, c->hy, yb, false) || dbuf_reserve(c, c->hb, (size_t)wt.out * 4, false))
        return bgl_last_code();
    HIPCHK(hipMemcpyAsync(c->hx.p, x, xb, hipMemcpyHostToDevice, c->stream));
    if (bias) HIPCHK(hipMemcpyAsync(c->hb.p, bias, (size_t)wt.out * 4, hipMemcpyHostToDevice, c->stream));
    rc = bgl_matmul_dev(c, t, act, (const float *)c->hx.p, bias ? (const float *)c->hb.p : nullptr, (float *)c->hy.p, M);
    if (rc) return rc;
    HIPCHK(hipMemcpyAsync(y, c->hy.p, yb, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(hipStreamSynchronize(c->stream));
    return 0;
}

static bgl_wt mkwt(int kind, int bits, int out, int in, const void *packed, const void *scales, const uint8_t *sub) {
    bgl_wt w;
    w.kind = kind; w.bits = bits; w.out = out; w.in = in; w.packed = packed; w.scales = scales; w.sub = sub;
    return w;
}

// Caller-quantized int8 columns (host xq / ascale) -> the W4A8 operands in the context, then the GEMV.
static int host_call_i8(bgl_ctx *c, const bgl_wt &wt, const int8_t *xq, const float *ascale, const float *bias,
                        float *y, int M) {
    if (!c || !xq || !ascale || !y || M < 1 || M > 64) return bgl_fail(BGL_E_ARG, "bad argument (M=%d, 1..64)", M);
    const int gq = wt.kind == BGL_Q4G256SF ? 256 : 64, K = wt.in;
    if (K % gq) return bgl_fail(BGL_E_ARG, "in=%d %% %d != 0", K, gq);
    bgl_tensor *t = nullptr;
    int rc = host_tensor(c, wt, &t);
    if (rc) return rc;
    const size_t qb = (size_t)M * K, ab = (size_t)M * (K / gq) * 4, qpad = (qb + 255) & ~(size_t)255;
    const size_t yb = (size_t)M * wt.out * 4;
    if (dbuf_reserve(c, c->hx, qpad + ab, false) || dbuf_reserve(c, c->hy, yb, false) ||
        dbuf_reserve(c, c->hb, (size_t)wt.out * 4, false) || dbuf_reserve(c, c->act_w, qb, false) ||
        dbuf_reserve(c, c->act_s, ab, false) || dbuf_reserve(c, c->act_sum, (size_t)M * (K / 64) * 4, false))
        return bgl_last_code();
    HIPCHK(hipMemcpyAsync(c->hx.p, xq, qb, hipMemcpyHostToDevice, c->stream));
    HIPCHK(hipMemcpyAsync((char *)c->hx.p + qpad, ascale, ab, hipMemcpyHostToDevice, c->stream));
    if (bias) HIPCHK(hipMemcpyAsync(c->hb.p, bias, (size_t)wt.out * 4, hipMemcpyHostToDevice, c->stream));
    const int split = wt.kind == BGL_Q8G64 ? 0 : 1;     // q4 / g256sf callers pass q4_split_act order
    int tok = prof_begin(c, 0);
    hipLaunchKernelGGL(k_act_import_i8, dim3(nblk((long)M * (K / 64) * 64)), dim3(256), 0, c->stream,
                       (const int8_t *)c->hx.p, (const float *)((char *)c->hx.p + qpad), M, K, gq, split,
                       (int8_t *)c->act_w.p, (float *)c->act_s.p, (int *)c->act_sum.p);
    prof_end(c, tok);
    HIPCHK(hipGetLastError());
    c->prep_act = BGL_ACT_W4A8; c->prep_gq = gq; c->prep_M = M; c->prep_K = K; c->prep_x = nullptr; c->prep_reuse = true;
    rc = bgl_matmul_prepped_dev(c, t, BGL_ACT_W4A8, bias ? (const float *)c->hb.p : nullptr, (float *)c->hy.p, M);
    if (rc) return rc;
    HIPCHK(hipMemcpyAsync(y, c->hy.p, yb, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(hipStreamSynchronize(c->stream));
    return 0;
}

extern "C" int bgl_gemv_q4g64_mt(bgl_ctx *p, const uint8_t *packed, const float *scales, const float *x, const float *bias,
                                 float *y, int out, int in) {
    return host_call(p, mkwt(BGL_Q4G64, 4, out, in, packed, scales, nullptr), BGL_ACT_F32, x, bias, y, 1);
}
extern "C" int bgl_gemv_q4g64_mt_fused(bgl_ctx *p, const uint8_t *packed, const float *scales, const float *x,
                                       const float *bias, float *y, int out, int in) {
    return host_call(p, mkwt(BGL_Q4G64, 4, out, in, packed, scales, nullptr), BGL_ACT_F32, x, bias, y, 1);
}
extern "C" int bgl_gemm_qXg64_sdot_mt(bgl_ctx *p, int bits, const uint8_t *packed, const float *scales, const int8_t *xq,
                                      const float *ascale, const float *bias, float *y, int out, int in, int M) {
    if (bits != 4 && bits != 8) return bgl_fail(BGL_E_ARG, "gemm_qXg64_sdot_mt: bits=%d (4 or 8)", bits);
    return host_call_i8(p, mkwt(bits == 8 ? BGL_Q8G64 : BGL_Q4G64, bits, out, in, packed, scales, nullptr), xq, ascale,
                        bias, y, M);
}
extern "C" int bgl_gemm_q4g256sf_sdot_mt(bgl_ctx *p, const uint8_t *packed, const float *wsuper, const uint8_t *subcode,
                                         const int8_t *xq, const float *ascale, const float *bias, float *y, int out,
                                         int in, int M) {
    return host_call_i8(p, mkwt(BGL_Q4G256SF, 4, out, in, packed, wsuper, subcode), xq, ascale, bias, y, M);
}
extern "C" int bgl_gemv_q4g64_sdot_mt(bgl_ctx *p, const uint8_t *packed, const float *scales, const float *x, const float *bias,
                                      float *y, int out, int in) {
    return host_call(p, mkwt(BGL_Q4G64, 4, out, in, packed, scales, nullptr), BGL_ACT_W4A8, x, bias, y, 1);
}
extern "C" int bgl_gemv_q8g64_mt(bgl_ctx *p, const uint8_t *packed, const float *scales, const float *x, const float *bias,
                                 float *y, int out, int in) {
    return host_call(p, mkwt(BGL_Q8G64, 8, out, in, packed, scales, nullptr), BGL_ACT_F32, x, bias, y, 1);
}
extern "C" int bgl_gemv_q8g64_sdot_mt(bgl_ctx *p, const uint8_t *packed, const float *scales, const float *x, const float *bias,
                                      float *y, int out, int in) {
    return host_call(p, mkwt(BGL_Q8G64, 8, out, in, packed, scales, nullptr), BGL_ACT_W4A8, x, bias, y, 1);
}
extern "C" int bgl_gemm_qXg64_mt(bgl_ctx *p, int bits, const uint8_t *packed, const float *scales, const float *x,
                                 const float *bias, float *y, int out, int in, int M) {
    if (bits != 4 && bits != 8) return bgl_fail(BGL_E_ARG, "gemm_qXg64_mt: bits=%d (4 or 8)", bits);
    return host_call(p, mkwt(bits == 8 ? BGL_Q8G64 : BGL_Q4G64, bits, out, in, packed, scales, nullptr), BGL_ACT_F32, x, bias, y, M);
}
extern "C" int bgl_gemv_q4g256sf_sdot_mt(bgl_ctx *p, const uint8_t *packed, const float *wsuper, const uint8_t *subcode,
                                         const float *x, const float *bias, float *y, int out, int in) {
    return host_call(p, mkwt(BGL_Q4G256SF, 4, out, in, packed, wsuper, subcode), BGL_ACT_W4A8, x, bias, y, 1);
}
extern "C" int bgl_gemm_q4g256sf_mt(bgl_ctx *p, const uint8_t *packed, const float *wsuper, const uint8_t *subcode,
                                    const float *x, const float *bias, float *y, int out, int in, int M) {
    return host_call(p, mkwt(BGL_Q4G256SF, 4, out, in, packed, wsuper, subcode), BGL_ACT_W4A8, x, bias, y, M);
}
extern "C" int bgl_qng64_matvec_f32(bgl_ctx *p, const uint8_t *packed, const float *scales, int n, const float *x,
                                    const float *bias, float *y, int out, int in) {
    return host_call(p, mkwt(BGL_QNG64, n, out, in, packed, scales, nullptr), BGL_ACT_F32, x, bias, y, 1);
}
extern "C" int bgl_qng64_matmul_f32(bgl_ctx *p, const uint8_t *packed, const float *scales, int n, const float *x,
                                    const float *bias, float *y, int out, int in, int M) {
    return host_call(p, mkwt(BGL_QNG64, n, out, in, packed, scales, nullptr), BGL_ACT_F32, x, bias, y, M);
}
extern "C" int bgl_gemv_q4g32h_mt(bgl_ctx *p, const uint8_t *packed, const uint16_t *scales16, const float *x,
                                  const float *bias, float *y, int out, int in) {
    return host_call(p, mkwt(BGL_Q4G32H, 4, out, in, packed, scales16, nullptr), BGL_ACT_F32, x, bias, y, 1);
}
extern "C" int bgl_forget(bgl_ctx *c, const void *packed) {
    if (!c) return bgl_fail(BGL_E_ARG, "bgl_forget: NULL context");
    std::lock_guard<std::mutex> lk(c->mu);
    auto it = c->host_cache.find(packed);
    if (it == c->host_cache.end()) return 0;
    (void)hipStreamSynchronize(c->stream);
    bgl_tensor_free(it->second);
    c->host_cache.erase(it);
    return 0;
}
