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
#include <ctype.h>
#include <errno.h>
#include <fcntl.h>
#include <limits.h>
#include <stdio.h>
#include <stdlib.h>
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

// ---- manifests
// A manifest is a stream of whitespace-separated tokens holding one record per tensor: a name,
// then fields of fixed meaning.  Line breaks carry no meaning, and a record that runs out of
// tokens, or holds a non-integer where an integer belongs, ends the manifest quietly: the
// engine's fscanf loops stop there too.
class Tokens {
    FILE *f_;
    bool fail_ = false, long_ = false;
public:
    explicit Tokens(FILE *f) : f_(f) {}
    // a token longer than its field allows ended the stream (an error, not a quiet end)
    bool too_long() const { return long_; }
    // the next token into buf (at most cap - 1 characters); false at the end of the stream or
    // when the token is longer
    bool word(char *buf, size_t cap) {
        if (fail_) return false;
        int ch;
        do ch = fgetc(f_); while (ch != EOF && isspace(ch));
        size_t n = 0;
        while (ch != EOF && !isspace(ch)) {
            if (n + 1 >= cap) { fail_ = long_ = true; return false; }
            buf[n++] = (char)ch;
            ch = fgetc(f_);
        }
        buf[n] = 0;
        if (!n) fail_ = true;
        return n > 0;
    }
    bool integer(long &v) {
        char t[32], *end = nullptr;
        if (!word(t, sizeof t)) return false;
        errno = 0;
        v = strtol(t, &end, 10);
        if (*end || errno) { fail_ = true; return false; }
        return true;
    }
};

// The int4-mode manifest (load_int4, qwen_infer.c:551-609): "name kind doff out in ng soff", and
// for q4g256sf an 8th field, the sub-code offset.  What each kind stores, as a table: the codes at
// doff (bytes per value = num / den), fp32 scales [out][ng] at soff for the grouped kinds, u8
// sub-codes [out][in/64] at soff2; `group` values per scale (0: f32, no groups, `in` 0 meaning a
// vector of `out`); the byte alignment every offset must have.
struct Int4Kind {
    const char *tag;
    int kind;                 // BGL_K_*, 0 for f32 (read in place from the blob)
    int group;
    int align;
    int num, den;
    bool sub;
};
const Int4Kind kInt4Kinds[] = {
    {"q4g64", BGL_K_Q4G64, 64, 64, 1, 2, false},
    {"q8g64", BGL_K_Q8G64, 64, 1, 1, 1, false},
    {"q4g256sf", BGL_K_Q4G256SF, 256, 64, 1, 2, true},
    {"f32", 0, 0, 1, 4, 1, false},
};
constexpr int kInt4MaxTensors = 512;

// A plane [off, off + bytes) must lie inside the blob.
int plane_in_blob(const char *layout, const char *nm, const char *what, long off, size_t bytes, size_t wb) {
    if (off < 0) return bgl_fail(BGL_E_ARG, "%s: tensor %s: %s offset %ld is negative", layout, nm, what, off);
    if ((size_t)off > wb || bytes > wb - (size_t)off)
        return bgl_fail(BGL_E_ARG, "%s: tensor %s: %s bytes [%ld, %ld + %zu) reach past the %zu-byte blob", layout, nm, what, off,
                        off, bytes, wb);
    return 0;
}

int parse_int4(const char *layout, size_t wb, std::vector<Rec> &recs) {
    FILE *f = fopen(layout, "r");
    if (!f) return bgl_fail(BGL_E_ARG, "int4 layout %s cannot be opened", layout);
    Tokens tk(f);
    std::unordered_map<std::string, int> seen;
    int rc = 0;
    for (;;) {
        char nm[96], tag[16];
        long doff, out, in, ng, soff;
        if (!tk.word(nm, sizeof nm) || !tk.word(tag, sizeof tag) || !tk.integer(doff) || !tk.integer(out) ||
            !tk.integer(in) || !tk.integer(ng) || !tk.integer(soff)) {
            if (tk.too_long()) rc = bgl_fail(BGL_E_ARG, "%s: record %zu holds a token longer than its field", layout, recs.size() + 1);
            break;
        }
        if (out > INT_MAX || in > INT_MAX || ng > INT_MAX || ng < INT_MIN) break;    // not an int: the record ends here
        if ((int)recs.size() == kInt4MaxTensors) {
            rc = bgl_fail(BGL_E_ARG, "%s: more than %d tensors", layout, kInt4MaxTensors);
            break;
        }
        if (out < 0 || in < 0 || doff < 0) {
            rc = bgl_fail(BGL_E_ARG, "%s: tensor %s: out=%ld in=%ld doff=%ld (none may be negative)", layout, nm, out, in, doff);
            break;
        }
        if (!seen.emplace(nm, 1).second) {
            rc = bgl_fail(BGL_E_ARG, "%s: tensor %s is listed twice", layout, nm);
            break;
        }
        const Int4Kind *k = nullptr;
        for (const Int4Kind &c : kInt4Kinds)
            if (!strcmp(c.tag, tag)) k = &c;
        if (!k) {
            rc = bgl_fail(BGL_E_ARG, "%s: tensor %s has kind \"%s\"; the kinds are q4g64, q8g64, q4g256sf and f32", layout, nm, tag);
            break;
        }
        long soff2 = 0;
        if (k->sub && !tk.integer(soff2)) {
            rc = bgl_fail(BGL_E_ARG, "%s: tensor %s (%s) ends before its sub-code offset, the 8th field", layout, nm, tag);
            break;
        }
        if (k->group) {
            if (in % k->group) {
                rc = bgl_fail(BGL_E_ARG, "%s: tensor %s: in=%ld is not a whole number of %d-value groups", layout, nm, in, k->group);
                break;
            }
            if (ng != in / k->group) {
                rc = bgl_fail(BGL_E_ARG, "%s: tensor %s: ng=%ld, but in / %d = %ld", layout, nm, ng, k->group, in / k->group);
                break;
            }
        }
        if (k->align > 1 && (doff % k->align || soff % k->align || (k->sub && soff2 % k->align))) {
            rc = bgl_fail(BGL_E_ARG, "%s: tensor %s (%s): every offset must be a multiple of %d bytes", layout, nm, tag, k->align);
            break;
        }
        const size_t values = k->group || in > 0 ? (size_t)out * in : (size_t)out;
        if ((rc = plane_in_blob(layout, nm, "code", doff, values * k->num / k->den, wb))) break;
        if (k->group && (rc = plane_in_blob(layout, nm, "scale", soff, (size_t)out * ng * 4, wb))) break;
        if (k->sub && (rc = plane_in_blob(layout, nm, "sub-code", soff2, (size_t)out * (in / 64), wb))) break;
        Rec r;
        r.name = nm; r.kind = k->kind; r.out = (int)out; r.in = (int)in; r.ng = (int)ng;
        r.doff = doff; r.soff = soff; r.soff2 = soff2;
        recs.push_back(r);
    }
    fclose(f);
    return rc;
}

// The AF layout manifest (moe_load_layout_af, qwen_infer.c:2496-2515): "name E out in ng po pb so
// bo" per tensor -- E experts of [out][in] int4 affine weights (nib * scale + bias, groups of 64)
// over one blob: packed nibbles at po (pb bytes, E * out * in / 2 of them read), fp32 scales
// [E][out][ng] at so and biases of the same shape at bo.
struct AfRec {
    std::string name;
    long E, out, in, ng, po, pb, so, bo;
};
constexpr int kAfMaxTensors = 1024;

int parse_af(const char *layout, size_t wb, std::vector<AfRec> &recs) {
    FILE *f = fopen(layout, "r");
    if (!f) return bgl_fail(BGL_E_ARG, "AF layout %s cannot be opened", layout);
    Tokens tk(f);
    std::unordered_map<std::string, int> seen;
    int rc = 0;
    for (;;) {
        char nm[128];
        AfRec r;
        if (!tk.word(nm, sizeof nm) || !tk.integer(r.E) || !tk.integer(r.out) || !tk.integer(r.in) || !tk.integer(r.ng) ||
            !tk.integer(r.po) || !tk.integer(r.pb) || !tk.integer(r.so) || !tk.integer(r.bo)) {
            if (tk.too_long()) rc = bgl_fail(BGL_E_ARG, "%s: record %zu holds a token longer than its field", layout, recs.size() + 1);
            break;
        }
        r.name = nm;
        if ((int)recs.size() == kAfMaxTensors) {
            rc = bgl_fail(BGL_E_ARG, "%s: more than %d tensors", layout, kAfMaxTensors);
            break;
        }
        if (!seen.emplace(nm, 1).second) {
            rc = bgl_fail(BGL_E_ARG, "%s: tensor %s is listed twice", layout, nm);
            break;
        }
        if (r.E < 1 || r.out < 1 || r.in < 64 || r.E > INT_MAX || r.out > INT_MAX || r.in > INT_MAX) {
            rc = bgl_fail(BGL_E_ARG, "%s: tensor %s: E=%ld out=%ld in=%ld (each at least 1, in at least 64)", layout, nm, r.E, r.out, r.in);
            break;
        }
        if (r.in % 64 || r.ng != r.in / 64) {
            rc = bgl_fail(BGL_E_ARG, "%s: tensor %s: in=%ld, ng=%ld; the groups hold 64 values", layout, nm, r.in, r.ng);
            break;
        }
        // E * out * in can exceed 64 bits for fields within int range: such a tensor cannot lie in any blob
        size_t rows = 0, vals = 0;
        if (__builtin_mul_overflow((size_t)r.E, (size_t)r.out, &rows) || __builtin_mul_overflow(rows, (size_t)r.in, &vals) ||
            vals > wb * 2) {
            rc = bgl_fail(BGL_E_ARG, "%s: tensor %s: E * out * in (%ld x %ld x %ld) is more than the blob's %zu bytes hold", layout,
                          nm, r.E, r.out, r.in, wb);
            break;
        }
        const size_t codes = vals / 2, side = rows * (size_t)r.ng * 4;
        if (r.pb < 0 || (size_t)r.pb < codes) {
            rc = bgl_fail(BGL_E_ARG, "%s: tensor %s: pb=%ld is less than its %zu bytes of codes", layout, nm, r.pb, codes);
            break;
        }
        if ((rc = plane_in_blob(layout, nm, "code", r.po, codes, wb)) || (rc = plane_in_blob(layout, nm, "scale", r.so, side, wb)) ||
            (rc = plane_in_blob(layout, nm, "bias", r.bo, side, wb)))
            break;
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
            // the directory's shape is validated like a bind's before it sizes anything
            if ((rc = check_wt(e.kind, e.kind == BGL_K_Q8G64 ? 8 : 4, e.out, e.in))) break;
            if (e.ng != e.in / (e.kind == BGL_K_Q4G256SF ? 256 : 64)) {
                rc = bgl_fail(BGL_E_ARG, "bgl_model_load_cache: %s: ng=%d does not match in=%d", e.name, e.ng, e.in);
                break;
            }
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

extern "C" int bgl_af_layout_check(const char *layout_path, long blob_bytes, int *n_tensors) {
    if (!layout_path || blob_bytes < 0) return bgl_fail(BGL_E_ARG, "bgl_af_layout_check: NULL path or negative blob size");
    std::vector<AfRec> recs;
    int rc = parse_af(layout_path, (size_t)blob_bytes, recs);
    if (rc) return rc;
    if (n_tensors) *n_tensors = (int)recs.size();
    return 0;
}

extern "C" int bgl_gpu_load_layout_af(const char *layout_path, const uint8_t *blob, long blob_bytes) {
    if (!layout_path || !blob || blob_bytes <= 0) {
        bgl_fail(BGL_E_ARG, "bgl_gpu_load_layout_af: NULL path or blob, or blob_bytes <= 0");
        return -1;
    }
    std::vector<AfRec> recs;
    if (parse_af(layout_path, (size_t)blob_bytes, recs)) return -1;
    for (const AfRec &r : recs)
        if (!bgl_gpu_bind_af(blob, blob_bytes, r.name.c_str(), r.E, r.out, r.in, r.ng, r.po, r.so, r.bo, 4)) return -1;
    return (int)recs.size();
}
