// bgl_loader.hip -- the int4-mode weight loader and a cache of the repacked device layout.
//
// bgl_model_load_int4 reads the engine's layout manifest over its weight blob (load_int4,
// qwen_infer.c:554-615): one line per tensor, "name kind doff out in ng soff [soff2]", kinds q4g64,
// q8g64, q4g256sf (8th field: the sub-code offset) and f32.  Every check of the reference loader
// is made before anything is bound, and a failed check loads nothing.  Quantized tensors are bound
// into the tiled device layout; f32 tensors (norms, embeddings) stay in the mapped blob, where the
// engine's CPU code reads them.
//
// The cache (the .beglin pattern of gguf_cache.c) stores the repacked device bytes so a later load
// skips the host->device repack: a header with the blob's and the manifest's size and mtime, the
// device architecture and the device-layout version; a directory; each tensor's three device
// buffers, 64-byte aligned.  A cache whose header does not match is not valid (the caller loads the
// manifest again and rewrites it); a directory that points outside the file is an error.
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/beglin_qgemv.h"
#include "bgl_internal.h"

#define HIPCHK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) return bgl_fail(BGL_E_HIP, "%s: %s", #x, hipGetErrorString(e_)); } while (0)

namespace {

struct Rec {
    std::string name;
    int kind = 0;             // BGL_K_Q4G64 / Q8G64 / Q4G256SF, or 0 for f32
    int out = 0, in = 0, ng = 0;
    long doff = 0, soff = 0, soff2 = 0;
    bgl_tensor *t = nullptr;
    const float *f32 = nullptr;
};

struct Mapping {
    void *p = nullptr;
    size_t bytes = 0;
    ~Mapping() {
        if (p) munmap(p, bytes);
    }
    int open_ro(const char *path, bool nofollow) {
        const int fd = open(path, O_RDONLY | (nofollow ? O_NOFOLLOW : 0));
        if (fd < 0) return bgl_fail(BGL_E_ARG, "cannot open %s", path);
        struct stat st;
        if (fstat(fd, &st) != 0 || st.st_size <= 0) {
            close(fd);
            return bgl_fail(BGL_E_ARG, "%s: empty or unreadable", path);
        }
        bytes = (size_t)st.st_size;
        p = mmap(nullptr, bytes, PROT_READ, MAP_PRIVATE, fd, 0);
        close(fd);
        if (p == MAP_FAILED) {
            p = nullptr;
            return bgl_fail(BGL_E_ARG, "mmap %s failed", path);
        }
        return 0;
    }
};

// load_int4's parse and checks (qwen_infer.c:558-609).  Like the reference's fscanf loop, parsing
// stops at the first line that does not hold the seven leading fields.
int parse_int4(const char *layout, size_t wb, std::vector<Rec> &recs) {
    FILE *f = fopen(layout, "r");
    if (!f) return bgl_fail(BGL_E_ARG, "layout_int4: cannot open %s", layout);
    char nm[96], kind[16];
    long doff, soff;
    int out, in, ng;
    std::unordered_map<std::string, int> seen;
    int rc = 0;
    while (!rc && fscanf(f, "%95s %15s %ld %d %d %d %ld", nm, kind, &doff, &out, &in, &ng, &soff) == 7) {
        if (recs.size() >= 512) { rc = bgl_fail(BGL_E_ARG, ">512 tensors in layout_int4"); break; }
        if (out < 0 || in < 0 || doff < 0) { rc = bgl_fail(BGL_E_ARG, "%s bad dims/off", nm); break; }
        if (seen.count(nm)) { rc = bgl_fail(BGL_E_ARG, "duplicate tensor name in layout: %s", nm); break; }
        seen[nm] = 1;
        Rec r;
        r.name = nm; r.out = out; r.in = in; r.ng = ng; r.doff = doff; r.soff = soff;
        if (!strcmp(kind, "q4g256sf")) {
            long soff2;
            if (fscanf(f, " %ld", &soff2) != 1) { rc = bgl_fail(BGL_E_ARG, "%s q4g256sf missing soff2 (8th field)", nm); break; }
            if (in % 256 != 0) { rc = bgl_fail(BGL_E_ARG, "%s in%%256!=0", nm); break; }
            if (ng != in / 256) { rc = bgl_fail(BGL_E_ARG, "%s ng=%d != in/256=%d", nm, ng, in / 256); break; }
            if (doff % 64 || soff % 64 || soff2 % 64) { rc = bgl_fail(BGL_E_ARG, "%s misaligned", nm); break; }
            const size_t pb = (size_t)out * (in / 2), sb = (size_t)out * ng * 4, cb = (size_t)out * (in / 64);
            if (soff < 0 || soff2 < 0 || (size_t)doff + pb > wb || (size_t)soff + sb > wb || (size_t)soff2 + cb > wb) {
                rc = bgl_fail(BGL_E_ARG, "%s q4g256sf extent past blob (wb=%zu)", nm, wb);
                break;
            }
            r.kind = BGL_K_Q4G256SF; r.soff2 = soff2;
        } else if (!strcmp(kind, "q4g64")) {
            if (in % 64 != 0) { rc = bgl_fail(BGL_E_ARG, "%s in%%64!=0", nm); break; }
            if (ng != in / 64) { rc = bgl_fail(BGL_E_ARG, "%s ng=%d != in/64=%d", nm, ng, in / 64); break; }
            if (doff % 64 || soff % 64) { rc = bgl_fail(BGL_E_ARG, "%s misaligned", nm); break; }
            const size_t pb = (size_t)out * (in / 2), sb = (size_t)out * ng * 4;
            if (soff < 0 || (size_t)doff + pb > wb || (size_t)soff + sb > wb) {
                rc = bgl_fail(BGL_E_ARG, "%s q4 extent past blob (wb=%zu)", nm, wb);
                break;
            }
            r.kind = BGL_K_Q4G64;
        } else if (!strcmp(kind, "q8g64")) {
            if (in % 64 != 0) { rc = bgl_fail(BGL_E_ARG, "%s in%%64!=0", nm); break; }
            if (ng != in / 64) { rc = bgl_fail(BGL_E_ARG, "%s ng=%d != in/64=%d", nm, ng, in / 64); break; }
            const size_t cb = (size_t)out * in, sb = (size_t)out * ng * 4;
            if (soff < 0 || (size_t)doff + cb > wb || (size_t)soff + sb > wb) {
                rc = bgl_fail(BGL_E_ARG, "%s q8 extent past blob (wb=%zu)", nm, wb);
                break;
            }
            r.kind = BGL_K_Q8G64;
        } else if (!strcmp(kind, "f32")) {
            const size_t numel = in > 0 ? (size_t)out * in : (size_t)out;
            if ((size_t)doff + numel * 4 > wb) { rc = bgl_fail(BGL_E_ARG, "%s f32 extent past blob (wb=%zu)", nm, wb); break; }
            r.kind = 0;
        } else {
            rc = bgl_fail(BGL_E_ARG, "%s unknown kind '%s' in %s (recognized: q4g64 q8g64 q4g256sf f32)", nm, kind, layout);
            break;
        }
        recs.push_back(r);
    }
    fclose(f);
    return rc;
}

#define CACHE_MAGIC "BGLDEV01"
#define CACHE_ARCH "gfx950"

struct CacheHeader {
    char magic[8];
    uint64_t blob_size, blob_mtime, layout_size, layout_mtime;
    char arch[16];
    uint32_t layout_version, n;
};

struct CacheEntry {
    char name[96];
    int32_t kind, out, in, ng;             // kind 0: f32 (data stay in the blob at doff)
    int64_t doff;
    BglDevTensor T;                        // pointer fields unused
    uint64_t off[3], len[3];               // device buffers in the file (len 0: absent)
};

bool stat_of(const char *path, uint64_t &size, uint64_t &mtime) {
    struct stat st;
    if (!path || stat(path, &st) != 0) return false;
    size = (uint64_t)st.st_size;
    mtime = (uint64_t)st.st_mtime;
    return true;
}

uint64_t align64(uint64_t x) { return (x + 63) & ~(uint64_t)63; }

}  // namespace

struct bgl_model {
    bgl_ctx *ctx = nullptr;
    std::vector<Rec> recs;
    std::unordered_map<std::string, size_t> by_name;
    Mapping blob;
    ~bgl_model() {
        for (Rec &r : recs)
            if (r.t) bgl_tensor_free(r.t);
    }
};

extern "C" int bgl_int4_layout_check(const char *layout_path, const char *blob_path, int *n_tensors) {
    if (!layout_path || !blob_path) return bgl_fail(BGL_E_ARG, "bgl_int4_layout_check: NULL path");
    uint64_t wb, mt;
    if (!stat_of(blob_path, wb, mt)) return bgl_fail(BGL_E_ARG, "cannot stat %s", blob_path);
    std::vector<Rec> recs;
    int rc = parse_int4(layout_path, (size_t)wb, recs);
    if (rc) return rc;
    if (n_tensors) *n_tensors = (int)recs.size();
    return 0;
}

extern "C" int bgl_model_load_int4(bgl_ctx *c, const char *layout_path, const char *blob_path, bgl_model **out) {
    if (!c || !layout_path || !blob_path || !out) return bgl_fail(BGL_E_ARG, "bgl_model_load_int4: NULL argument");
    *out = nullptr;
    bgl_model *m = new bgl_model();
    m->ctx = c;
    int rc = m->blob.open_ro(blob_path, false);
    if (!rc) rc = parse_int4(layout_path, m->blob.bytes, m->recs);
    const uint8_t *b = (const uint8_t *)m->blob.p;
    for (size_t i = 0; !rc && i < m->recs.size(); i++) {
        Rec &r = m->recs[i];
        m->by_name[r.name] = i;
        if (r.kind == 0) {
            r.f32 = (const float *)(b + r.doff);
            continue;
        }
        bgl_wt w;
        memset(&w, 0, sizeof w);
        w.kind = r.kind; w.bits = r.kind == BGL_K_Q8G64 ? 8 : 4; w.out = r.out; w.in = r.in;
        w.packed = b + r.doff; w.scales = b + r.soff; w.sub = r.kind == BGL_K_Q4G256SF ? b + r.soff2 : nullptr;
        rc = bgl_bind(c, &w, &r.t);
    }
    if (rc) {
        delete m;
        return rc;
    }
    *out = m;
    return 0;
}

extern "C" int bgl_model_count(const bgl_model *m) { return m ? (int)m->recs.size() : 0; }

extern "C" int bgl_model_find(const bgl_model *m, const char *name, int *kind, int *out, int *in, bgl_tensor **t,
                              const float **f32) {
    if (!m || !name) return bgl_fail(BGL_E_ARG, "bgl_model_find: NULL argument");
    auto it = m->by_name.find(name);
    if (it == m->by_name.end()) return bgl_fail(BGL_E_ARG, "bgl_model_find: no tensor '%s'", name);
    const Rec &r = m->recs[it->second];
    if (kind) *kind = r.kind;
    if (out) *out = r.out;
    if (in) *in = r.in;
    if (t) *t = r.t;
    if (f32) *f32 = r.f32;
    return 0;
}

extern "C" int bgl_model_free(bgl_model *m) {
    if (!m) return 0;
    if (m->ctx) (void)bgl_synchronize(m->ctx);
    delete m;
    return 0;
}

extern "C" int bgl_model_save_cache(const bgl_model *m, const char *cache_path, const char *layout_path, const char *blob_path) {
    if (!m || !cache_path) return bgl_fail(BGL_E_ARG, "bgl_model_save_cache: NULL argument");
    CacheHeader h;
    memset(&h, 0, sizeof h);
    memcpy(h.magic, CACHE_MAGIC, 8);
    if (!stat_of(blob_path, h.blob_size, h.blob_mtime) || !stat_of(layout_path, h.layout_size, h.layout_mtime))
        return bgl_fail(BGL_E_ARG, "bgl_model_save_cache: cannot stat the blob or the layout");
    strncpy(h.arch, CACHE_ARCH, sizeof h.arch - 1);
    h.layout_version = BGL_DEVICE_LAYOUT_VERSION;
    h.n = (uint32_t)m->recs.size();
    std::vector<CacheEntry> dir(m->recs.size());
    uint64_t pos = align64(sizeof h + sizeof(CacheEntry) * dir.size());
    for (size_t i = 0; i < m->recs.size(); i++) {
        const Rec &r = m->recs[i];
        CacheEntry &e = dir[i];
        memset(&e, 0, sizeof e);
        strncpy(e.name, r.name.c_str(), sizeof e.name - 1);
        e.kind = r.kind; e.out = r.out; e.in = r.in; e.ng = r.ng; e.doff = r.doff;
        if (!r.t) continue;
        size_t lb[3];
        BglDevTensor T;
        device_layout(r.t->T.fmt, r.t->T.bits, r.t->T.N, r.t->T.K, T, lb);
        e.T = T;
        for (int k = 0; k < 3; k++) {
            e.off[k] = lb[k] ? pos : 0;
            e.len[k] = lb[k];
            pos = align64(pos + lb[k]);
        }
    }
    const int fd = open(cache_path, O_WRONLY | O_CREAT | O_TRUNC | O_NOFOLLOW, 0644);
    if (fd < 0) return bgl_fail(BGL_E_ARG, "bgl_model_save_cache: cannot create %s", cache_path);
    int rc = 0;
    auto put = [&](const void *p, size_t n, uint64_t at) {
        if (!rc && pwrite(fd, p, n, (off_t)at) != (ssize_t)n) rc = bgl_fail(BGL_E_ARG, "bgl_model_save_cache: write failed");
    };
    put(&h, sizeof h, 0);
    put(dir.data(), sizeof(CacheEntry) * dir.size(), sizeof h);
    std::vector<uint8_t> host;
    for (size_t i = 0; !rc && i < m->recs.size(); i++) {
        const Rec &r = m->recs[i];
        if (!r.t) continue;
        const void *src[3] = {r.t->T.w, r.t->T.s0, r.t->T.s1};
        for (int k = 0; k < 3 && !rc; k++) {
            if (!dir[i].len[k]) continue;
            host.resize(dir[i].len[k]);
            if (hipMemcpy(host.data(), src[k], host.size(), hipMemcpyDeviceToHost) != hipSuccess) {
                rc = bgl_fail(BGL_E_HIP, "bgl_model_save_cache: device read of %s", r.name.c_str());
                break;
            }
            put(host.data(), host.size(), dir[i].off[k]);
        }
    }
    if (!rc && ftruncate(fd, (off_t)pos) != 0) rc = bgl_fail(BGL_E_ARG, "bgl_model_save_cache: truncate failed");
    close(fd);
    if (rc) unlink(cache_path);
    return rc;
}

extern "C" int bgl_model_cache_valid(const char *cache_path, const char *layout_path, const char *blob_path) {
    uint64_t bs, bm, ls, lm;
    if (!cache_path || !stat_of(blob_path, bs, bm) || !stat_of(layout_path, ls, lm)) return 0;
    const int fd = open(cache_path, O_RDONLY | O_NOFOLLOW);
    if (fd < 0) return 0;
    CacheHeader h;
    const bool got = pread(fd, &h, sizeof h, 0) == (ssize_t)sizeof h;
    close(fd);
    return got && !memcmp(h.magic, CACHE_MAGIC, 8) && !strncmp(h.arch, CACHE_ARCH, sizeof h.arch) &&
           h.layout_version == BGL_DEVICE_LAYOUT_VERSION && h.blob_size == bs && h.blob_mtime == bm && h.layout_size == ls &&
           h.layout_mtime == lm;
}

extern "C" int bgl_model_load_cache(bgl_ctx *c, const char *cache_path, const char *layout_path, const char *blob_path,
                                    bgl_model **out) {
    if (!c || !cache_path || !out) return bgl_fail(BGL_E_ARG, "bgl_model_load_cache: NULL argument");
    *out = nullptr;
    if (!bgl_model_cache_valid(cache_path, layout_path, blob_path))
        return bgl_fail(BGL_E_ARG, "bgl_model_load_cache: %s is missing or stale for this blob / layout / device", cache_path);
    Mapping cm;
    int rc = cm.open_ro(cache_path, true);
    if (rc) return rc;
    const uint8_t *base = (const uint8_t *)cm.p;
    const CacheHeader &h = *(const CacheHeader *)base;
    if (cm.bytes < sizeof h || h.n > 512 || sizeof h + (uint64_t)h.n * sizeof(CacheEntry) > cm.bytes)
        return bgl_fail(BGL_E_ARG, "bgl_model_load_cache: %s: directory past the end of the file", cache_path);
    const CacheEntry *dir = (const CacheEntry *)(base + sizeof h);
    HIPCHK(hipSetDevice(c->device));
    bgl_model *m = new bgl_model();
    m->ctx = c;
    rc = m->blob.open_ro(blob_path, false);
    for (uint32_t i = 0; !rc && i < h.n; i++) {
        const CacheEntry &e = dir[i];
        Rec r;
        r.name = std::string(e.name, strnlen(e.name, sizeof e.name));
        r.kind = e.kind; r.out = e.out; r.in = e.in; r.ng = e.ng; r.doff = e.doff;
        if (r.name.empty() || m->by_name.count(r.name)) { rc = bgl_fail(BGL_E_ARG, "bgl_model_load_cache: bad entry %u", i); break; }
        if (e.kind == 0) {
            const size_t numel = e.in > 0 ? (size_t)e.out * e.in : (size_t)e.out;
            if (e.doff < 0 || (size_t)e.doff + numel * 4 > m->blob.bytes) { rc = bgl_fail(BGL_E_ARG, "%s f32 extent past blob", e.name); break; }
            r.f32 = (const float *)((const uint8_t *)m->blob.p + e.doff);
        } else {
            size_t lb[3];
            BglDevTensor T;
            if (e.kind != BGL_K_Q4G64 && e.kind != BGL_K_Q8G64 && e.kind != BGL_K_Q4G256SF) { rc = bgl_fail(BGL_E_ARG, "%s: kind %d", e.name, e.kind); break; }
            device_layout(e.kind, e.kind == BGL_K_Q8G64 ? 8 : 4, e.out, e.in, T, lb);
            void *buf[3] = {nullptr, nullptr, nullptr};
            size_t total = 0;
            for (int k = 0; k < 3 && !rc; k++) {
                if (e.len[k] != lb[k] || (lb[k] && (e.off[k] + lb[k] > cm.bytes || e.off[k] < sizeof h))) {
                    rc = bgl_fail(BGL_E_ARG, "bgl_model_load_cache: %s: buffer %d does not match the layout or the file", e.name, k);
                    break;
                }
                if (!lb[k]) continue;
                if (hipMalloc(&buf[k], lb[k]) != hipSuccess) { rc = bgl_fail(BGL_E_NOMEM, "hipMalloc %zu B", lb[k]); break; }
                if (hipMemcpy(buf[k], base + e.off[k], lb[k], hipMemcpyHostToDevice) != hipSuccess) {
                    rc = bgl_fail(BGL_E_HIP, "bgl_model_load_cache: upload of %s", e.name);
                    break;
                }
                total += lb[k];
            }
            if (rc) {
                for (void *p : buf)
                    if (p) (void)hipFree(p);
                break;
            }
            r.t = tensor_from_parts(T, buf[0], buf[1], buf[2], total);
        }
        m->by_name[r.name] = m->recs.size();
        m->recs.push_back(r);
    }
    if (rc) {
        delete m;
        return rc;
    }
    *out = m;
    return 0;
}
