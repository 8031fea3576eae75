// bgl_registry.hip -- the name-keyed MoE binding registry behind the bgl_gpu_* entry points: the
// mlx_moe.h boundary (mlx_moe.h:24-125, :255-264, :334) with the reference's argument lists and
// its 1 = ok / 0 = failure convention.  One process-wide registry on device 0 with its own
// stream (MLX binds into one default stream the same way).  Bound tensors are shared between the
// name table and snapshots; a tensor is freed (after a stream sync) when neither holds it.
#include <limits.h>
#include <string.h>

#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "bgl_internal.h"

namespace {

struct Entry {
    std::shared_ptr<bgl_tensor> t;    // expert stack (E >= 1)
    int bits = 0;                     // width as bound: 2..15, 16 or 32 (mixed: the widest cell)
    bool mixed = false;               // mixed per-cell qNg64 (kind 4, no tensor-wide width)
};

// A MoE router: fp32 [E][in] and an optional bias [E], on the device.
struct Router {
    std::shared_ptr<void> w, bias;
    int E = 0, in = 0;
};

struct Registry {
    std::mutex mu;
    bgl_ctx *ctx = nullptr;
    std::unordered_map<std::string, Entry> names;
    std::unordered_map<std::string, Router> routers;
    std::unordered_map<uint64_t, std::pair<std::string, Entry>> snaps;
    uint64_t next_snap = 1;
    int bound = 0;                    // binds performed (mlx_gpu_zerocopy_count's return value)
    size_t bytes_copied = 0, peak = 0;
    int batch = 1, sort_threshold = INT_MAX;
};

// Never destroyed: freeing device memory from a static destructor can outlive the HIP runtime.
Registry &reg() {
    static Registry *r = new Registry();
    return *r;
}

bgl_ctx *reg_ctx(Registry &R) {
    if (!R.ctx && bgl_available() == 1) {
        bgl_ctx *c = nullptr;
        if (bgl_ctx_create(0, nullptr, &c) == 0) R.ctx = c;
    }
    return R.ctx;
}

std::shared_ptr<bgl_tensor> own(bgl_ctx *c, bgl_tensor *t) {
    return std::shared_ptr<bgl_tensor>(t, [c](bgl_tensor *p) {
        if (c) (void)bgl_synchronize(c);
        bgl_tensor_free(p);
    });
}

size_t tensor_bytes(const bgl_tensor *t) {
    size_t b = 0;
    (void)bgl_tensor_info(t, nullptr, nullptr, nullptr, nullptr, &b);
    return b;
}

size_t active_bytes(Registry &R) {
    std::unordered_set<const bgl_tensor *> seen;
    size_t total = 0;
    auto add = [&](const Entry &e) { if (seen.insert(e.t.get()).second) total += tensor_bytes(e.t.get()); };
    for (auto &kv : R.names) add(kv.second);
    for (auto &kv : R.snaps) add(kv.second.second);
    for (auto &kv : R.routers) total += (size_t)kv.second.E * kv.second.in * 4 + (kv.second.bias ? (size_t)kv.second.E * 4 : 0);
    return total;
}

bool qng_planes(int bits) { return bits == 7 || (bits >= 9 && bits <= 15); }
bool bits_ok(int bits) {
    return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8 || qng_planes(bits) || bits == 16 ||
           bits == 32;
}
// mlx_gpu_binding_kind's classes (mlx_moe.h:52-57)
int kind_class(int bits) { return qng_planes(bits) ? 3 : (bits == 16 || bits == 32) ? 2 : 1; }
// ffn_role_kind (mlx_moe.cpp:1522-1526): 0 native quantized, 1 dense, 2 qNg64 planes
int role_class(int bits) { return qng_planes(bits) ? 2 : (bits == 16 || bits == 32) ? 1 : 0; }

// One expert's reference-layout descriptor inside the blob.
bgl_wt expert_desc(const uint8_t *blob, long e, long out, long in, long ng, long packed_off, long scale_off,
                   long bias_off, int bits) {
    bgl_wt w;
    memset(&w, 0, sizeof w);
    w.out = (int)out; w.in = (int)in;
    const size_t rows = (size_t)e * out, sb = (size_t)ng * 4;
    if (bits == 16 || bits == 32) {
        w.kind = bits == 16 ? BGL_K_F16 : BGL_K_F32;
        w.packed = blob + packed_off + rows * in * (bits / 8);
        return w;
    }
    w.scales = blob + scale_off + rows * sb;
    if (bits == 4) {                                   // AF int4 affine: words [E][out][in/8]
        w.kind = BGL_K_Q4G64A; w.bits = 4;
        w.packed = blob + packed_off + rows * (in / 2);
        w.sub = blob + bias_off + rows * sb;
    } else if (bits == 8) {                            // q8g64 raw int8, no bias
        w.kind = BGL_K_Q8G64; w.bits = 8;
        w.packed = blob + packed_off + rows * in;
    } else {                                           // qNg64 planes [E][out][ng*n*8]
        w.kind = BGL_K_QNG64; w.bits = bits;
        w.packed = blob + packed_off + rows * (size_t)ng * bits * 8;
    }
    return w;
}

// Reference-layout byte extents of one E-stacked tensor (for the blob bounds check).
void extents(long E, long out, long in, long ng, int bits, size_t *pb, size_t *sb) {
    const size_t rows = (size_t)E * out;
    *sb = (bits == 16 || bits == 32) ? 0 : rows * ng * 4;
    if (bits == 16 || bits == 32) *pb = rows * in * (bits / 8);
    else if (bits == 4) *pb = rows * in / 2;
    else if (bits == 8) *pb = rows * in;
    else *pb = rows * ng * bits * 8;
}

int bind_stack(Registry &R, const std::vector<bgl_wt> &ws, bgl_tensor **out) {
    std::vector<bgl_tensor *> ts(ws.size(), nullptr);
    int rc = 0;
    for (size_t e = 0; e < ws.size() && !rc; e++) rc = bgl_bind(R.ctx, &ws[e], &ts[e]);
    if (!rc) rc = bgl_experts_from_tensors(R.ctx, (int)ws.size(), ts.data(), out);
    if (rc)
        for (bgl_tensor *t : ts) bgl_tensor_free(t);
    return rc;
}

void put(Registry &R, const std::string &name, bgl_tensor *t, int bits) {
    Entry en;
    en.t = own(R.ctx, t);
    en.bits = bits;
    R.names[name] = en;
    R.bound++;
    R.bytes_copied += tensor_bytes(t);
    const size_t a = active_bytes(R);
    if (a > R.peak) R.peak = a;
}

const Entry *find(Registry &R, const char *name) {
    if (!name) return nullptr;
    auto it = R.names.find(name);
    return it == R.names.end() ? nullptr : &it->second;
}

// Host buffers -> context staging (hx: inputs, hy: outputs).
int stage_in(bgl_ctx *c, const void *const *src, const size_t *bytes, int n, void **dst) {
    size_t total = 0, off[4];
    for (int i = 0; i < n; i++) { off[i] = total; total += (bytes[i] + 255) & ~(size_t)255; }
    if (dbuf_reserve(c, c->hx, total, false)) return BGL_E_NOMEM;
    for (int i = 0; i < n; i++) {
        dst[i] = (char *)c->hx.p + off[i];
        if (hipMemcpyAsync(dst[i], src[i], bytes[i], hipMemcpyHostToDevice, c->stream) != hipSuccess)
            return bgl_fail(BGL_E_HIP, "staging copy failed");
    }
    return 0;
}

int fetch(bgl_ctx *c, void *dst, const void *src, size_t bytes) {
    if (hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
        hipStreamSynchronize(c->stream) != hipSuccess)
        return bgl_fail(BGL_E_HIP, "result copy failed");
    return 0;
}

// y[z] = W_{idx[z]} x[z] through the device gather, host buffers.
int gather_host(bgl_ctx *c, const bgl_tensor *stack, const float *x, int N, const int32_t *idx, float *y) {
    int K = 0, O = 0;
    (void)bgl_tensor_info(stack, nullptr, nullptr, &O, &K, nullptr);
    const void *src[2] = {x, idx};
    const size_t bytes[2] = {(size_t)N * K * 4, (size_t)N * 4};
    void *dst[2];
    int rc = stage_in(c, src, bytes, 2, dst);
    if (rc) return rc;
    if (dbuf_reserve(c, c->hy, (size_t)N * O * 4, false)) return BGL_E_NOMEM;
    rc = bgl_gather_matvec_dev(c, stack, (const float *)dst[0], (const int32_t *)dst[1], N, (float *)c->hy.p);
    if (rc) return rc;
    return fetch(c, y, c->hy.p, (size_t)N * O * 4);
}

}  // namespace

extern "C" int bgl_gpu_available(void) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    return reg_ctx(R) ? 1 : 0;
}

extern "C" bgl_ctx *bgl_gpu_context(void) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    return reg_ctx(R);
}

extern "C" const bgl_tensor *bgl_gpu_lookup(const char *name) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    const Entry *e = find(R, name);
    return e ? e->t.get() : nullptr;
}

extern "C" int bgl_gpu_synchronize(void) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    if (!reg_ctx(R)) return 0;
    return bgl_synchronize(R.ctx) == 0 ? 1 : 0;
}

extern "C" int bgl_gpu_reset_runtime_epoch(void) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    if (!reg_ctx(R)) return 0;
    if (bgl_synchronize(R.ctx) != 0) return 0;
    (void)ctx_scratch(R.ctx, true);
    return 1;
}

extern "C" int bgl_gpu_bind_af(const uint8_t *blob, long blob_bytes, const char *name, long E, long out, long in, long ng,
                               long packed_off, long scale_off, long bias_off, int bits) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    if (!reg_ctx(R)) return 0;
    if (!blob || !name) { bgl_fail(BGL_E_ARG, "bgl_gpu_bind_af: NULL blob or name"); return 0; }
    if (!bits_ok(bits)) { bgl_fail(BGL_E_UNSUPPORTED, "bgl_gpu_bind_af: bits=%d not bindable", bits); return 0; }
    if (E <= 0 || out <= 0 || in <= 0 || E > INT_MAX || out > INT_MAX || in > INT_MAX) {
        bgl_fail(BGL_E_ARG, "bgl_gpu_bind_af: bad shape E=%ld out=%ld in=%ld", E, out, in);
        return 0;
    }
    const bool dense = bits == 16 || bits == 32;
    if (in % 64 || (!dense && ng != in / 64)) {
        bgl_fail(BGL_E_ARG, "bgl_gpu_bind_af: in=%ld, ng=%ld (groups of 64 required)", in, ng);
        return 0;
    }
    if (packed_off < 0 || (!dense && scale_off < 0) || (bits == 4 && bias_off < 0)) {
        bgl_fail(BGL_E_ARG, "bgl_gpu_bind_af: negative offset for a plane this width reads");
        return 0;
    }
    // E * out * in values at most 2^40 (past any device's memory): every extent below then fits 64 bits
    size_t rows = 0, vals = 0;
    if (__builtin_mul_overflow((size_t)E, (size_t)out, &rows) || __builtin_mul_overflow(rows, (size_t)in, &vals) ||
        vals > ((size_t)1 << 40)) {
        bgl_fail(BGL_E_ARG, "bgl_gpu_bind_af: E * out * in (%ld x %ld x %ld) is more than 2^40 values", E, out, in);
        return 0;
    }
    size_t pb, sb;
    extents(E, out, in, ng, bits, &pb, &sb);
    if (blob_bytes > 0) {                  // bounds check when the caller states the blob size
        const size_t lim = (size_t)blob_bytes;
        if ((size_t)packed_off + pb > lim || (sb && (size_t)scale_off + sb > lim) || (bits == 4 && (size_t)bias_off + sb > lim)) {
            bgl_fail(BGL_E_ARG, "bgl_gpu_bind_af: tensor '%s' extends past the blob (%ld bytes)", name, blob_bytes);
            return 0;
        }
    }
    std::vector<bgl_wt> ws;
    for (long e = 0; e < E; e++) ws.push_back(expert_desc(blob, e, out, in, ng, packed_off, scale_off, bias_off, bits));
    bgl_tensor *t = nullptr;
    if (bind_stack(R, ws, &t)) return 0;
    put(R, name, t, bits);
    return 1;
}

extern "C" int bgl_gpu_binding_kind(const char *name, int *bits_out) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    if (bits_out) *bits_out = 0;
    const Entry *e = find(R, name);
    if (!e) return 0;
    if (e->mixed) return 4;           // mlx_moe.cpp:477-481: the width is cell-local, bits_out = 0
    if (bits_out) *bits_out = e->bits;
    return kind_class(e->bits);
}

extern "C" int bgl_gpu_snapshot_binding(const char *name, uint64_t *snapshot_id) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    if (!reg_ctx(R) || !snapshot_id) return 0;
    const Entry *e = find(R, name);
    if (!e) return 0;
    uint64_t id = R.next_snap++;
    if (id == 0) id = R.next_snap++;
    R.snaps[id] = std::make_pair(std::string(name), *e);
    *snapshot_id = id;
    return 1;
}

extern "C" int bgl_gpu_restore_binding_snapshot(uint64_t snapshot_id) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    auto it = R.snaps.find(snapshot_id);
    if (it == R.snaps.end()) return 0;
    R.names[it->second.first] = it->second.second;
    R.bound++;
    return 1;
}

extern "C" int bgl_gpu_drop_binding_snapshot(uint64_t snapshot_id) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    return R.snaps.erase(snapshot_id) ? 1 : 0;
}

extern "C" int bgl_gpu_binding_snapshot_count(void) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    return (int)R.snaps.size();
}

extern "C" int bgl_gpu_zerocopy_count(int *zero_copy, int *copied, size_t *bytes_copied) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    if (zero_copy) *zero_copy = 0;
    if (copied) *copied = R.bound;
    if (bytes_copied) *bytes_copied = R.bytes_copied;
    return R.bound;
}

extern "C" int bgl_gpu_dequant_probe(const char *name, long e, long row, long col0, int ncols, float *out) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    const Entry *en = find(R, name);
    if (!reg_ctx(R) || !en || !out) return 0;
    if (en->mixed) return 0;          // the reference's probe has no mixed arm
    const bgl_tensor *st = en->t.get();
    const long E = (long)st->experts.size();
    int O = 0, K = 0;
    (void)bgl_tensor_info(st, nullptr, nullptr, &O, &K, nullptr);
    if (e < 0 || e >= E || row < 0 || row >= O || ncols <= 0 || col0 < 0 || col0 + ncols > K) return 0;
    bgl_ctx *c = R.ctx;
    if (dbuf_reserve(c, c->hy, (size_t)K * 4, false)) return 0;
    if (bgl_dequant_dev(c, st->experts[e], (int)row, 1, (float *)c->hy.p)) return 0;
    return fetch(c, out, (const float *)c->hy.p + col0, (size_t)ncols * 4) == 0 ? 1 : 0;
}

extern "C" int bgl_gpu_qng64_gather_probe(const uint8_t *planes, long E, long out, long in, long ng, int n, const float *scales,
                                          const float *x, int N, const int32_t *expert_idx, float *out_buf) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    if (!reg_ctx(R) || !planes || !scales || !x || !expert_idx || !out_buf || N < 1) return 0;
    if (E <= 0 || out <= 0 || in <= 0 || in % 64 || ng != in / 64 || n < 2 || n > 15) {
        bgl_fail(BGL_E_ARG, "bgl_gpu_qng64_gather_probe: bad shape or n=%d", n);
        return 0;
    }
    std::vector<bgl_wt> ws;
    for (long e = 0; e < E; e++) {
        bgl_wt w;
        memset(&w, 0, sizeof w);
        w.kind = BGL_K_QNG64; w.bits = n; w.out = (int)out; w.in = (int)in;
        w.packed = planes + (size_t)e * out * ng * n * 8;
        w.scales = scales + (size_t)e * out * ng;
        ws.push_back(w);
    }
    bgl_tensor *t = nullptr;
    if (bind_stack(R, ws, &t)) return 0;
    const int rc = gather_host(R.ctx, t, x, N, expert_idx, out_buf);
    (void)bgl_synchronize(R.ctx);
    bgl_tensor_free(t);
    return rc == 0 ? 1 : 0;
}

extern "C" int bgl_gpu_bind_qng64_dense_probe(const uint8_t *packed, const float *scales, const char *name, long out, long in,
                                              int n) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    if (!reg_ctx(R) || !packed || !scales || !name || out <= 0 || in <= 0 || in % 64) return 0;
    if (n != 2 && n != 3 && n != 5 && n != 6) return 0;       // mlx_moe.cpp:442
    bgl_wt w;
    memset(&w, 0, sizeof w);
    w.kind = BGL_K_QNG64; w.bits = n; w.out = (int)out; w.in = (int)in; w.packed = packed; w.scales = scales;
    std::vector<bgl_wt> ws(1, w);
    bgl_tensor *t = nullptr;
    if (bind_stack(R, ws, &t)) return 0;
    put(R, name, t, n);
    return 1;
}

extern "C" int bgl_gpu_matvec_probe(const char *name, long e, const float *x, float *y) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    const Entry *en = find(R, name);
    if (!reg_ctx(R) || !en || !x || !y) return 0;
    if (e < 0 || e >= (long)en->t->experts.size()) return 0;
    const int32_t idx = (int32_t)e;
    return gather_host(R.ctx, en->t.get(), x, 1, &idx, y) == 0 ? 1 : 0;
}

extern "C" void bgl_gpu_report_memory(size_t *active, size_t *peak, size_t *cache) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    const size_t a = active_bytes(R);
    if (a > R.peak) R.peak = a;
    if (active) *active = a;
    if (peak) *peak = R.peak;
    if (cache) *cache = R.ctx ? ctx_scratch(R.ctx, false) : 0;
}

extern "C" int bgl_gpu_set_batch(int B) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    if (!reg_ctx(R) || B < 1 || B > 64) return 0;
    R.batch = B;
    return 1;
}

extern "C" int bgl_gpu_set_sort_threshold(int threshold) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    if (!reg_ctx(R)) return 0;
    R.sort_threshold = threshold;
    return 1;
}

extern "C" int bgl_gpu_test_ffn_uniform(const char *gate_name, const char *up_name, const char *down_name) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    const Entry *g = find(R, gate_name), *u = find(R, up_name), *d = find(R, down_name);
    if (!g || !u || !d) return -1;
    return (role_class(g->bits) == role_class(u->bits) && role_class(g->bits) == role_class(d->bits)) ? 1 : 0;
}

extern "C" int bgl_gpu_ffn_gather(const char *name, const float *x, int N, const int32_t *expert_idx, float *y) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    const Entry *en = find(R, name);
    if (!reg_ctx(R) || !en || !x || !expert_idx || !y || N < 1) return 0;
    return gather_host(R.ctx, en->t.get(), x, N, expert_idx, y) == 0 ? 1 : 0;
}

extern "C" int bgl_gpu_moe_ffn(const char *gate, const char *up, const char *down, const char *shared_gate,
                               const char *shared_up, const char *shared_down, const float *x, int T,
                               const int32_t *topk_idx, const float *topk_w, int K, float *out) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    const Entry *g = find(R, gate), *u = find(R, up), *d = find(R, down);
    if (!reg_ctx(R) || !g || !u || !d || !x || !topk_idx || !topk_w || !out || T < 1 || K < 1) return 0;
    const bgl_tensor *sh[3] = {nullptr, nullptr, nullptr};
    const char *shn[3] = {shared_gate, shared_up, shared_down};
    for (int i = 0; i < 3; i++) {
        if (!shn[i]) continue;
        const Entry *s = find(R, shn[i]);
        if (!s || s->t->experts.size() != 1) {
            bgl_fail(BGL_E_ARG, "bgl_gpu_moe_ffn: shared tensor '%s' missing or not a single expert", shn[i]);
            return 0;
        }
        sh[i] = s->t->experts[0];
    }
    int H = 0;
    (void)bgl_tensor_info(g->t.get(), nullptr, nullptr, nullptr, &H, nullptr);
    bgl_ctx *c = R.ctx;
    const void *src[3] = {x, topk_idx, topk_w};
    const size_t bytes[3] = {(size_t)T * H * 4, (size_t)T * K * 4, (size_t)T * K * 4};
    void *dst[3];
    if (stage_in(c, src, bytes, 3, dst)) return 0;
    if (dbuf_reserve(c, c->hy, (size_t)T * H * 4, false)) return 0;
    if (bgl_moe_ffn_dev(c, g->t.get(), u->t.get(), d->t.get(), sh[0], sh[1], sh[2], (const float *)dst[0],
                        (const int32_t *)dst[1], (const float *)dst[2], T, K, (float *)c->hy.p))
        return 0;
    return fetch(c, out, c->hy.p, (size_t)T * H * 4) == 0 ? 1 : 0;
}

// ---------------------------------------------------------------- router + whole routed layer
namespace {
std::shared_ptr<void> dev_copy(bgl_ctx *c, const void *src, size_t bytes) {
    void *d = nullptr;
    if (hipMalloc(&d, bytes) != hipSuccess) return nullptr;
    if (hipMemcpyAsync(d, src, bytes, hipMemcpyHostToDevice, c->stream) != hipSuccess || hipStreamSynchronize(c->stream) != hipSuccess) {
        (void)hipFree(d);
        return nullptr;
    }
    return std::shared_ptr<void>(d, [c](void *p) {
        (void)bgl_synchronize(c);
        (void)hipFree(p);
    });
}
}  // namespace

extern "C" int bgl_gpu_bind_router(const char *name, const float *w, const float *bias, long E, long in) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    if (!reg_ctx(R) || !name || !w || E < 1 || E > 256 || in < 4 || in % 4) {
        bgl_fail(BGL_E_ARG, "bgl_gpu_bind_router: bad argument (E=%ld in 1..256, in=%ld a multiple of 4)", E, in);
        return 0;
    }
    Router r;
    r.E = (int)E;
    r.in = (int)in;
    r.w = dev_copy(R.ctx, w, (size_t)E * in * 4);
    if (bias) r.bias = dev_copy(R.ctx, bias, (size_t)E * 4);
    if (!r.w || (bias && !r.bias)) {
        bgl_fail(BGL_E_NOMEM, "bgl_gpu_bind_router: device copy of '%s' failed", name);
        return 0;
    }
    R.routers[name] = r;
    R.bytes_copied += (size_t)E * in * 4;
    R.peak = std::max(R.peak, active_bytes(R));
    return 1;
}

extern "C" int bgl_gpu_moe_layer(const char *router, const char *gate, const char *up, const char *down,
                                 const char *shared_gate, const char *shared_up, const char *shared_down, const float *x,
                                 int T, int K, int renorm, float *out, int32_t *topk_idx, float *topk_w) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    auto rt = router ? R.routers.find(router) : R.routers.end();
    const Entry *g = find(R, gate), *u = find(R, up), *d = find(R, down);
    if (!reg_ctx(R) || rt == R.routers.end() || !g || !u || !d || !x || !out || T < 1 || K < 1) return 0;
    const bgl_tensor *sh[3] = {nullptr, nullptr, nullptr};
    const char *shn[3] = {shared_gate, shared_up, shared_down};
    for (int i = 0; i < 3; i++) {
        if (!shn[i]) continue;
        const Entry *s = find(R, shn[i]);
        if (!s || s->t->experts.size() != 1) {
            bgl_fail(BGL_E_ARG, "bgl_gpu_moe_layer: shared tensor '%s' missing or not a single expert", shn[i]);
            return 0;
        }
        sh[i] = s->t->experts[0];
    }
    int H = 0;
    (void)bgl_tensor_info(g->t.get(), nullptr, nullptr, nullptr, &H, nullptr);
    const Router &r = rt->second;
    if (r.in != H || r.E != (int)g->t->experts.size()) {
        bgl_fail(BGL_E_ARG, "bgl_gpu_moe_layer: router [%d x %d] does not match %zu experts of in=%d", r.E, r.in,
                 g->t->experts.size(), H);
        return 0;
    }
    bgl_ctx *c = R.ctx;
    const void *src[1] = {x};
    const size_t bytes[1] = {(size_t)T * H * 4};
    void *dst[1];
    if (stage_in(c, src, bytes, 1, dst)) return 0;
    if (dbuf_reserve(c, c->hy, (size_t)T * H * 4, false)) return 0;
    if (bgl_moe_layer_dev(c, (const float *)r.w.get(), (const float *)r.bias.get(), renorm, g->t.get(), u->t.get(), d->t.get(),
                          sh[0], sh[1], sh[2], (const float *)dst[0], T, K, (float *)c->hy.p))
        return 0;
    if (fetch(c, out, c->hy.p, (size_t)T * H * 4)) return 0;
    const int32_t *ridx = (const int32_t *)c->moe_route.p;
    if (topk_idx && fetch(c, topk_idx, ridx, (size_t)T * K * 4)) return 0;
    if (topk_w && fetch(c, topk_w, ridx + (size_t)T * K, (size_t)T * K * 4)) return 0;
    return 1;
}

// ---------------------------------------------------------------- mixed per-cell qNg64 (QT-4 probes)
extern "C" int bgl_gpu_bind_qng64_mixed_dense_probe(const uint8_t *planes, long planes_bytes, const uint32_t *offsets,
                                                    const uint8_t *bits, const float *scales, const char *name, long out,
                                                    long in) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    if (!reg_ctx(R) || !name || out <= 0 || out > INT_MAX || in <= 0 || in > INT_MAX) return 0;
    bgl_tensor *t = nullptr, *st = nullptr;
    if (bgl_bind_qng64_mixed(R.ctx, planes, planes_bytes, offsets, bits, scales, (int)out, (int)in, &t)) return 0;
    if (bgl_experts_from_tensors(R.ctx, 1, &t, &st)) {
        bgl_tensor_free(t);
        return 0;
    }
    int W = 0;
    (void)bgl_tensor_info(t, nullptr, &W, nullptr, nullptr, nullptr);
    put(R, name, st, W);
    R.names[name].mixed = true;
    return 1;
}

extern "C" int bgl_gpu_qng64_mixed_dense_probe(const uint8_t *planes, long planes_bytes, const uint32_t *offsets,
                                               const uint8_t *bits, const float *scales, long out, long in, const float *x,
                                               int batch, float *out_buf) {
    Registry &R = reg();
    std::lock_guard<std::mutex> lk(R.mu);
    if (!reg_ctx(R) || !x || !out_buf || batch <= 0 || out <= 0 || out > INT_MAX || in <= 0 || in > INT_MAX) return 0;
    bgl_ctx *c = R.ctx;
    bgl_tensor *t = nullptr;
    if (bgl_bind_qng64_mixed(c, planes, planes_bytes, offsets, bits, scales, (int)out, (int)in, &t)) return 0;
    const void *src[1] = {x};
    const size_t bytes[1] = {(size_t)batch * in * 4};
    void *dst[1];
    int ok = 0;
    if (!stage_in(c, src, bytes, 1, dst) && !dbuf_reserve(c, c->hy, (size_t)batch * out * 4, false) &&
        !bgl_matmul_dev(c, t, BGL_ACT_F32, (const float *)dst[0], nullptr, (float *)c->hy.p, batch))
        ok = fetch(c, out_buf, c->hy.p, (size_t)batch * out * 4) == 0;
    (void)bgl_synchronize(c);
    bgl_tensor_free(t);
    return ok;
}
