// gguf.hip - GGUF model files, their Q8_0 tensors straight to device tiles.
//
// The reader of internal/gguf/gguf.go of github.com/xattribution/gorelaxor:
// versions 2 and 3, the key-value section (every value type, arrays nested
// at most three deep), the tensor table with its checks against crafted
// files (gguf.go:292-354: dimensions and their product within the file,
// offsets that cannot wrap, the alignment key), tensors of F32, F16, BF16
// and Q8_0.  Open (gguf.go:57-113) reads the header in growing pieces and
// refuses tensors whose sizes add up to more than the file; here a tensor's
// bytes are read from the file when it is asked for, so no copy of the
// model stays on the host, and a Q8_0 tensor goes from the file to its
// device tiles (File.Weight + kern.NewQ8 + Pack) in one call.  Error texts
// are the reference's.  Host code only.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "grx_internal.h"

namespace {

enum { kF32 = 0, kF16 = 1, kQ8_0 = 8, kBF16 = 30 };  // gguf.go:21-26
constexpr uint64_t kMaxFile = 4ull << 30;             // gguf.go:55
constexpr uint64_t kMetaMax = 16ull << 20;            // gguf.go:214

// One key's value.  Scalars keep their bits in `raw` (integers zero- or
// sign-extended, float32 / float64 as their bit patterns, bool 0 or 1);
// arrays keep their element type and elements.
struct Val {
    uint32_t t = 0, et = 0;
    uint64_t raw = 0;
    std::string s;
    std::vector<Val> a;
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
};

const char *kShort = "gguf: file is cut short";

// gguf.go:116-212: a cursor over the header bytes whose first error sticks
struct Reader {
    const uint8_t *b;
    size_t n, off = 0;
    std::string err;
    bool ok() const { return err.empty(); }
    const uint8_t *take(uint64_t k) {
        if (!ok()) return nullptr;
        if (k > n - off) {
            err = kShort;
            return nullptr;
        }
        const uint8_t *p = b + off;
        off += (size_t)k;
        return p;
    }
    uint64_t le(int k) {
        const uint8_t *p = take((uint64_t)k);
        uint64_t v = 0;
        if (p)
            for (int i = k - 1; i >= 0; --i) v = v << 8 | p[i];
        return v;
    }
    std::string str() {
        const uint64_t k = le(8);
        if (k > (1u << 30)) {
            err = "gguf: string too long";
            return "";
        }
        const uint8_t *p = take(k);
        return p ? std::string((const char *)p, (size_t)k) : std::string();
    }
    Val value(uint32_t t, int depth) {
        Val v;
        v.t = t;
        switch (t) {
            case 0: v.raw = le(1); break;
            case 1: v.raw = (uint64_t)(int64_t)(int8_t)le(1); break;
            case 2: v.raw = le(2); break;
            case 3: v.raw = (uint64_t)(int64_t)(int16_t)le(2); break;
            case 4: v.raw = le(4); break;
            case 5: v.raw = (uint64_t)(int64_t)(int32_t)le(4); break;
            case 6: v.raw = le(4); break;
            case 7: v.raw = le(1) != 0; break;
            case 8: v.s = str(); break;
            case 9: {
                if (depth > 2) {
                    err = "gguf: arrays nested too deep";
                    return v;
                }
                v.et = (uint32_t)le(4);
                const uint64_t k = le(8);
                // every element takes at least a byte: a count past the
                // bytes left is refused before anything is reserved
                if (k > n - off || k > (1u << 24)) {
                    err = "gguf: array too long";
                    return v;
                }
                v.a.reserve((size_t)std::min<uint64_t>(k, 1024));
                for (uint64_t i = 0; i < k && ok(); ++i) v.a.push_back(value(v.et, depth + 1));
                break;
            }
            case 10: v.raw = le(8); break;
            case 11: v.raw = le(8); break;
            case 12: v.raw = le(8); break;
            default: {
                char m[64];
                snprintf(m, sizeof m, "gguf: unknown value type %u", t);
                err = m;
            }
        }
        return v;
    }
};

bool to_int(const Val &v, int64_t *out) {  // toInt, gguf.go:389-413
    switch (v.t) {
        case 0: case 1: case 2: case 3: case 4: case 5: case 7: case 10: case 11:
            *out = (int64_t)v.raw;
            return true;
    }
    return false;
}

bool to_float(const Val &v, double *out) {  // the number cases of Float and Floats
    if (v.t == 6) {
        float f;
        const uint32_t b = (uint32_t)v.raw;
        memcpy(&f, &b, 4);
        *out = f;
        return true;
    }
    if (v.t == 12) {
        memcpy(out, &v.raw, 8);
        return true;
    }
    int64_t i;
    if (!to_int(v, &i)) return false;
    *out = (double)i;
    return true;
}

std::string fmt(const char *f, const std::string &a, long b = 0) {
    char m[512];
    snprintf(m, sizeof m, f, a.c_str(), b);
    return m;
}

float h2f(uint16_t h) {  // kern.F16ToF32
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16, exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff, b;
    if (exp == 0 && man == 0) {
        b = sign;
    } else if (exp == 0) {
        uint32_t e = 127 - 15 + 1;
        while ((man & 0x400) == 0) {
            man <<= 1;
            --e;
        }
        b = sign | e << 23 | (man & 0x3ff) << 13;
    } else if (exp == 0x1f) {
        b = sign | 0xffu << 23 | man << 13;
    } else {
        b = sign | (exp + 127 - 15) << 23 | man << 13;
    }
    float f;
    memcpy(&f, &b, 4);
    return f;
}

}  // namespace

struct grx_gguf {
    int version = 0;
    std::map<std::string, Val> kv;
    std::vector<std::string> keys;  // sorted, for grx_gguf_key
    std::map<std::string, Tensor> tensors;
    std::vector<std::string> order;  // file order (a repeated name twice)
    uint64_t base = 0, size = 0;
    std::string path;           // Open: tensors read from here
    std::vector<uint8_t> buf;   // Parse: the caller's bytes, copied

    const Val *get(const char *k) const {
        auto it = kv.find(k);
        return it == kv.end() ? nullptr : &it->second;
    }
};

namespace {

// byteSize (gguf.go:356-370)
bool byte_size(const Tensor &t, uint64_t *out, std::string *err) {
    uint64_t n = 1;
    for (uint64_t d : t.dims) n *= d;
    switch (t.type) {
        case kF32: *out = n * 4; return true;
        case kF16: case kBF16: *out = n * 2; return true;
        case kQ8_0:
            if (t.dims.empty() || t.dims[0] % 32 != 0) {
                *err = fmt("gguf: Q8_0 tensor %s rows are not a multiple of 32", t.name);
                return false;
            }
            *out = n / 32 * 34;
            return true;
    }
    *err = fmt("gguf: tensor %s has type %ld, which this reader doesn't handle", t.name, (long)t.type);
    return false;
}

// parseMeta / parseHeader (gguf.go:236-354).  `short_` is set when the
// header ran past b (the caller may read more and try again).
std::string parse_header(const uint8_t *b, size_t n, uint64_t size, bool meta_only, grx_gguf *f, bool *short_) {
    Reader r{b, n};
    *short_ = false;
    const uint8_t *m = r.take(4);
    if (!m || memcmp(m, "GGUF", 4) != 0) return "gguf: not a GGUF file";
    f->version = (int)(uint32_t)r.le(4);
    if (f->version < 2 || f->version > 3) return fmt("gguf: version %s is not supported", std::to_string(f->version));
    const uint64_t nt = r.le(8), nkv = r.le(8);
    if ((!meta_only && nt > (1u << 20)) || nkv > (1u << 20)) return "gguf: header counts out of range";
    for (uint64_t i = 0; i < nkv && r.ok(); ++i) {
        std::string k = r.str();
        const uint32_t t = (uint32_t)r.le(4);
        f->kv[k] = r.value(t, 0);
    }
    if (!meta_only) {
        for (uint64_t i = 0; i < nt && r.ok(); ++i) {
            Tensor t;
            t.name = r.str();
            const uint32_t nd = (uint32_t)r.le(4);
            if (nd > 4) return fmt("gguf: tensor %s has %ld dimensions", t.name, (long)nd);
            // each dimension, and their product, within the file
            uint64_t elems = 1;
            for (uint32_t d = 0; d < nd; ++d) {
                const uint64_t v = r.le(8);
                elems *= v;
                if (v == 0 || v > size || elems > size) return fmt("gguf: tensor %s has an impossible size", t.name);
                t.dims.push_back(v);
            }
            t.type = (uint32_t)r.le(4);
            t.offset = r.le(8);
            f->order.push_back(t.name);
            f->tensors[t.name] = t;
        }
    }
    if (!r.ok()) {
        *short_ = r.err == kShort;
        return r.err;
    }
    for (auto &e : f->kv) f->keys.push_back(e.first);
    if (meta_only) return "";
    uint64_t align = 32;
    if (const Val *a = f->get("general.alignment")) {
        const uint64_t v = a->raw;
        if (a->t != 4 || v < 8 || v > 4096 || (v & (v - 1)) != 0)
            return "gguf: general.alignment must be a power of two from 8 to 4096";
        align = v;
    }
    f->base = (r.off + align - 1) / align * align;
    for (auto &e : f->tensors) {
        const Tensor &t = e.second;
        uint64_t bytes;
        std::string err;
        if (!byte_size(t, &bytes, &err)) return err;
        // in this order, so no sum can wrap around
        if (f->base > size || t.offset > size - f->base || bytes > size - f->base - t.offset)
            return fmt("gguf: tensor %s runs past the end of the file", t.name);
    }
    return "";
}

grx_status gfail(const std::string &m) { return grx_fail(GRX_EINVAL, "%s", m.c_str()); }

const Tensor *find(const grx_gguf *g, const char *name) {
    auto it = g->tensors.find(name);
    return it == g->tensors.end() ? nullptr : &it->second;
}

// the tensor's bytes, from the Parse buffer or read from the Open file
grx_status tensor_bytes(const grx_gguf *g, const Tensor &t, std::vector<uint8_t> *out) {
    uint64_t n;
    std::string err;
    if (!byte_size(t, &n, &err)) return gfail(err);
    out->resize((size_t)n);
    const uint64_t at = g->base + t.offset;
    if (g->path.empty()) {
        if (n) memcpy(out->data(), g->buf.data() + at, (size_t)n);
        return GRX_OK;
    }
    FILE *f = fopen(g->path.c_str(), "rb");
    bool ok = f && fseeko(f, (off_t)at, SEEK_SET) == 0 && (n == 0 || fread(out->data(), 1, (size_t)n, f) == n);
    if (f) fclose(f);
    if (!ok) return gfail(fmt("gguf: reading %s: the file changed or is unreadable", t.name));
    return GRX_OK;
}

// File.Weight's matrix shape (gguf.go:544-558): the rows are the first
// dimension longer than one, the rest flattened into rows
void weight_shape(const Tensor &t, uint64_t *rows, uint64_t *cols) {
    uint64_t c = 1, n = 1;
    for (uint64_t d : t.dims) {
        c = d;
        if (d > 1) break;
    }
    for (uint64_t d : t.dims) n *= d;
    *cols = c;
    *rows = n / std::max<uint64_t>(c, 1);
}

}  // namespace

extern "C" grx_status grx_gguf_parse(const void *b, size_t n, grx_gguf **out) {
    if (!out || (!b && n)) return grx_fail(GRX_EINVAL, "grx_gguf_parse: NULL argument");
    *out = nullptr;
    grx_gguf *g = new grx_gguf();
    bool sh;
    const std::string err = parse_header((const uint8_t *)b, n, n, false, g, &sh);
    if (!err.empty()) {
        delete g;
        return gfail(err);
    }
    g->buf.assign((const uint8_t *)b, (const uint8_t *)b + n);
    g->size = n;
    *out = g;
    return GRX_OK;
}

extern "C" grx_status grx_gguf_open(const char *path, grx_gguf **out) {
    if (!path || !out) return grx_fail(GRX_EINVAL, "grx_gguf_open: NULL argument");
    *out = nullptr;
    FILE *f = fopen(path, "rb");
    if (!f) return grx_fail(GRX_EINVAL, "open %s: no such file or not readable", path);
    struct Closer {
        FILE *f;
        ~Closer() { fclose(f); }
    } closer{f};
    if (fseeko(f, 0, SEEK_END) != 0) return grx_fail(GRX_EINVAL, "gguf: %s: cannot seek", path);
    const uint64_t size = (uint64_t)ftello(f);
    if (size > kMaxFile)
        return grx_fail(GRX_EINVAL, "gguf: %s is %llu MB, more than a model can be", path,
                        (unsigned long long)(size >> 20));
    // the header, read until it's whole (gguf.go:80-93)
    for (uint64_t k = 1 << 20;; k *= 8) {
        const uint64_t want = std::min(k, size);
        std::vector<uint8_t> b((size_t)want);
        if (fseeko(f, 0, SEEK_SET) != 0 || fread(b.data(), 1, (size_t)want, f) != want)
            return grx_fail(GRX_EINVAL, "gguf: %s: read error", path);
        grx_gguf *g = new grx_gguf();
        bool sh;
        const std::string err = parse_header(b.data(), b.size(), size, false, g, &sh);
        if (!err.empty()) {
            delete g;
            if (sh && want < size) continue;
            return gfail(err);
        }
        // tensors that overlap would each cost their full size (gguf.go:94-103)
        uint64_t total = 0;
        for (const std::string &name : g->order) {
            uint64_t n = 0;
            std::string e2;
            byte_size(g->tensors[name], &n, &e2);
            total += n;
        }
        if (total > size) {
            delete g;
            return gfail("gguf: the tensors overlap");
        }
        g->path = path;
        g->size = size;
        *out = g;
        return GRX_OK;
    }
}

extern "C" grx_status grx_gguf_read_meta(const char *path, grx_gguf **out) {
    if (!path || !out) return grx_fail(GRX_EINVAL, "grx_gguf_read_meta: NULL argument");
    *out = nullptr;
    FILE *f = fopen(path, "rb");
    if (!f) return grx_fail(GRX_EINVAL, "open %s: no such file or not readable", path);
    struct Closer {
        FILE *f;
        ~Closer() { fclose(f); }
    } closer{f};
    // ReadMeta (gguf.go:219-234): the start of the file, more only while
    // the settings run on, at most 16 MB
    for (uint64_t k = 256 << 10;; k *= 8) {
        const uint64_t len = std::min(k, kMetaMax);
        std::vector<uint8_t> b((size_t)len);
        if (fseeko(f, 0, SEEK_SET) != 0) return grx_fail(GRX_EINVAL, "gguf: %s: cannot seek", path);
        const size_t got = fread(b.data(), 1, (size_t)len, f);
        grx_gguf *g = new grx_gguf();
        bool sh;
        const std::string err = parse_header(b.data(), got, got, true, g, &sh);
        if (err.empty()) {
            *out = g;
            return GRX_OK;
        }
        delete g;
        if (sh && got == len && len < kMetaMax) continue;
        return gfail(err);
    }
}

extern "C" grx_status grx_gguf_close(grx_gguf *g) {
    delete g;
    return GRX_OK;
}

extern "C" int grx_gguf_version(const grx_gguf *g) { return g ? g->version : 0; }
extern "C" int grx_gguf_n_tensors(const grx_gguf *g) { return g ? (int)g->order.size() : 0; }
extern "C" const char *grx_gguf_tensor_name(const grx_gguf *g, int i) {
    return g && i >= 0 && i < (int)g->order.size() ? g->order[i].c_str() : nullptr;
}
extern "C" int grx_gguf_n_keys(const grx_gguf *g) { return g ? (int)g->keys.size() : 0; }
extern "C" const char *grx_gguf_key(const grx_gguf *g, int i) {
    return g && i >= 0 && i < (int)g->keys.size() ? g->keys[i].c_str() : nullptr;
}
extern "C" int grx_gguf_has(const grx_gguf *g, const char *name) { return g && name && find(g, name) ? 1 : 0; }

extern "C" grx_status grx_gguf_tensor_info(const grx_gguf *g, const char *name, int *type, int *n_dims,
                                           int64_t dims[4]) {
    if (!g || !name) return grx_fail(GRX_EINVAL, "grx_gguf_tensor_info: NULL argument");
    const Tensor *t = find(g, name);
    if (!t) return gfail(fmt("gguf: no tensor %s", name));
    if (type) *type = (int)t->type;
    if (n_dims) *n_dims = (int)t->dims.size();
    if (dims)
        for (int i = 0; i < 4; ++i) dims[i] = i < (int)t->dims.size() ? (int64_t)t->dims[i] : 0;
    return GRX_OK;
}

// File.Int / Float / Bool / String (gguf.go:415-460)
extern "C" int64_t grx_gguf_int(const grx_gguf *g, const char *key, int64_t def) {
    const Val *v = g && key ? g->get(key) : nullptr;
    int64_t i;
    return v && to_int(*v, &i) ? i : def;
}
extern "C" double grx_gguf_float(const grx_gguf *g, const char *key, double def) {
    const Val *v = g && key ? g->get(key) : nullptr;
    double f;
    return v && to_float(*v, &f) ? f : def;
}
extern "C" int grx_gguf_bool(const grx_gguf *g, const char *key, int def) {
    const Val *v = g && key ? g->get(key) : nullptr;
    int64_t i;
    if (v && v->t == 7) return v->raw != 0;
    return v && to_int(*v, &i) ? i != 0 : def;
}
extern "C" const char *grx_gguf_string(const grx_gguf *g, const char *key, const char *def) {
    const Val *v = g && key ? g->get(key) : nullptr;
    return v && v->t == 8 ? v->s.c_str() : def;
}
// Strings / Floats / Ints (gguf.go:462-510): -1 when the key is no array
extern "C" int64_t grx_gguf_array_len(const grx_gguf *g, const char *key) {
    const Val *v = g && key ? g->get(key) : nullptr;
    return v && v->t == 9 ? (int64_t)v->a.size() : -1;
}
extern "C" const char *grx_gguf_array_string(const grx_gguf *g, const char *key, int64_t i) {
    const Val *v = g && key ? g->get(key) : nullptr;
    if (!v || v->t != 9 || i < 0 || i >= (int64_t)v->a.size()) return nullptr;
    return v->a[(size_t)i].t == 8 ? v->a[(size_t)i].s.c_str() : "";
}
extern "C" double grx_gguf_array_float(const grx_gguf *g, const char *key, int64_t i) {
    const Val *v = g && key ? g->get(key) : nullptr;
    double f = 0;
    if (!v || v->t != 9 || i < 0 || i >= (int64_t)v->a.size()) return 0;
    const Val &e = v->a[(size_t)i];
    if (e.t == 6) {  // float32(x) of Floats, widened back
        to_float(e, &f);
        return f;
    }
    if (e.t == 12) {
        to_float(e, &f);
        return (double)(float)f;
    }
    int64_t k;
    return to_int(e, &k) ? (double)(float)k : 0;
}
extern "C" int64_t grx_gguf_array_int(const grx_gguf *g, const char *key, int64_t i) {
    const Val *v = g && key ? g->get(key) : nullptr;
    int64_t k;
    if (!v || v->t != 9 || i < 0 || i >= (int64_t)v->a.size()) return 0;
    return to_int(v->a[(size_t)i], &k) ? k : 0;
}

// File.Float32 (gguf.go:518-542): any tensor widened to float32
extern "C" grx_status grx_gguf_float32(const grx_gguf *g, const char *name, float *out, size_t n) {
    if (!g || !name || (!out && n)) return grx_fail(GRX_EINVAL, "grx_gguf_float32: NULL argument");
    const Tensor *t = find(g, name);
    if (!t) return gfail(fmt("gguf: no tensor %s", name));
    uint64_t elems = 1;
    for (uint64_t d : t->dims) elems *= d;
    if (t->type == kQ8_0) {
        uint64_t rows, cols;
        weight_shape(*t, &rows, &cols);
        if (cols != t->dims[0]) return gfail(fmt("gguf: Q8_0 tensor %s has leading unit dimensions", name));
    }
    if (n < elems) return grx_fail(GRX_ESIZE, "gguf: %s has %llu values, the buffer %zu", name,
                                   (unsigned long long)elems, n);
    std::vector<uint8_t> d;
    grx_status s = tensor_bytes(g, *t, &d);
    if (s != GRX_OK) return s;
    for (uint64_t i = 0; i < elems; ++i) {
        switch (t->type) {
            case kF32: memcpy(&out[i], &d[4 * i], 4); break;
            case kF16: out[i] = h2f((uint16_t)(d[2 * i] | d[2 * i + 1] << 8)); break;
            case kBF16: {
                const uint32_t b = (uint32_t)(d[2 * i] | d[2 * i + 1] << 8) << 16;
                memcpy(&out[i], &b, 4);
                break;
            }
            case kQ8_0: {  // Weight.Float32: f32(d) * q
                const uint8_t *blk = &d[i / 32 * 34];
                out[i] = h2f((uint16_t)(blk[0] | blk[1] << 8)) * (float)(int8_t)blk[2 + i % 32];
                break;
            }
        }
    }
    return GRX_OK;
}

// A tensor's stored bytes and type, for the model loaders in this library.
grx_status grx_gguf_tensor_data(const grx_gguf *g, const char *name, int *type, std::vector<uint8_t> *out) {
    const Tensor *t = find(g, name);
    if (!t) return gfail(fmt("gguf: no tensor %s", name));
    if (type) *type = (int)t->type;
    return tensor_bytes(g, *t, out);
}

// File.Weight's shape (rows, cols) of any tensor
extern "C" grx_status grx_gguf_weight_shape(const grx_gguf *g, const char *name, int64_t *rows, int64_t *cols) {
    if (!g || !name) return grx_fail(GRX_EINVAL, "grx_gguf_weight_shape: NULL argument");
    const Tensor *t = find(g, name);
    if (!t) return gfail(fmt("gguf: no tensor %s", name));
    uint64_t r, c;
    weight_shape(*t, &r, &c);
    if (rows) *rows = (int64_t)r;
    if (cols) *cols = (int64_t)c;
    return GRX_OK;
}

// File.Weight + kern.NewQ8 + Pack: a Q8_0 tensor from the file to its
// device tiles
extern "C" grx_status grx_gguf_weight_q8(grx_ctx *ctx, const grx_gguf *g, const char *name, grx_weight **out) {
    if (!ctx || !g || !name || !out) return grx_fail(GRX_EINVAL, "grx_gguf_weight_q8: NULL argument");
    *out = nullptr;
    const Tensor *t = find(g, name);
    if (!t) return gfail(fmt("gguf: no tensor %s", name));
    uint64_t rows, cols;
    weight_shape(*t, &rows, &cols);
    if (t->type != kQ8_0)
        return gfail(fmt("gguf: tensor %s has type %ld; the device route takes Q8_0", name, (long)t->type));
    if (cols != t->dims[0]) return gfail(fmt("gguf: Q8_0 tensor %s has leading unit dimensions", name));
    if (rows > (1u << 31) - 1 || cols > (1u << 31) - 1)
        return grx_fail(GRX_ESIZE, "gguf: tensor %s is too large", name);
    std::vector<uint8_t> d;
    grx_status s = tensor_bytes(g, *t, &d);
    if (s != GRX_OK) return s;
    return grx_weight_q8_create(ctx, (int)rows, (int)cols, d.data(), d.size(), out);
}
