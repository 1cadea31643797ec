// whisper_load.hip - a whisper.cpp (ggml) model file straight into the
// GPU decoder.
//
// Reads the file as whisper/model.go:109-225 of github.com/xattribution/
// gorelaxor does (magic, hyper-parameters and their checks, mel filters,
// vocabulary, then tensors until the end) and binds the decoder's tensors as
// Model.bind does (model.go:300-404: names, shapes, no unknown or missing
// tensor).  The difference is the reason this file exists: the reference
// widens every matrix to float16 at load (toF16, model.go:420-440), while
// here a Q8_0 matrix goes to the device as it is stored (the ggml block is
// the product's weight format), and a matrix stored another way is widened
// as the reference widens it and then rounded to Q8_0 (kern.ToQ8) for the
// int8 route.  Vectors are widened by the reference's toF32 (model.go:405-
// 418): float32 as stored, anything else through float16.  The encoder's
// tensors are checked and skipped: the decoder takes the encoder output
// from the caller.  Host code only.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "grx_internal.h"

namespace {

constexpr uint32_t kGgmlMagic = 0x67676d6c;  // "ggml", model.go:88
enum { kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ4_1 = 3, kQ5_0 = 6, kQ5_1 = 7, kQ8_0 = 8 };  // model.go:272-280

// typeBytes (model.go:282-294)
bool type_bytes(int t, size_t n, size_t *out) {
    if (t == kF32) return *out = n * 4, true;
    if (t == kF16) return *out = n * 2, true;
    int bs = 0;
    switch (t) {
        case kQ4_0: bs = 18; break;
        case kQ4_1: bs = 20; break;
        case kQ5_0: bs = 22; break;
        case kQ5_1: bs = 24; break;
        case kQ8_0: bs = 34; break;
    }
    if (bs == 0 || n % 32 != 0) return false;
    return *out = n / 32 * bs, true;
}

// half -> float32 (f16tab of whisper/f16.go, the IEEE widening) and float32
// -> half rounded to nearest even (f32toF16, whisper/f16.go:35-71)
float h2f(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16, exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    uint32_t b;
    if (exp == 0) {
        if (man == 0) {
            b = sign;
        } else {  // subnormal: normalize
            int e = -1;
            uint32_t m = man;
            do {
                ++e;
                m <<= 1;
            } while ((m & 0x400) == 0);
            b = sign | (uint32_t)(127 - 15 - e) << 23 | (m & 0x3ff) << 13;
        }
    } else if (exp == 0x1f) {
        b = sign | 0xffu << 23 | man << 13;
    } else {
        b = sign | (exp + 127 - 15) << 23 | man << 13;
    }
    float f;
    memcpy(&f, &b, 4);
    return f;
}

uint16_t f2h(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    const uint16_t sign = (uint16_t)(b >> 16) & 0x8000;
    const int32_t exp = (int32_t)(b >> 23) & 0xff;
    uint32_t man = b & 0x7fffff;
    if (exp == 0xff) return man != 0 ? (sign | 0x7e00) : (sign | 0x7c00);
    const int32_t e = exp - 127 + 15;
    if (e >= 0x1f) return sign | 0x7c00;
    if (e <= 0) {
        if (e < -10) return sign;
        man |= 0x800000;
        const uint32_t shift = (uint32_t)(14 - e);
        uint32_t h = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1) == 1)) h++;
        return sign | (uint16_t)h;
    }
    uint32_t h = (uint32_t)e << 10 | man >> 13;
    const uint32_t rem = man & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1) == 1)) h++;
    return sign | (uint16_t)h;
}

uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | p[1] << 8); }
uint32_t rd32le(const uint8_t *p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }

// dequantBlock (model.go:449-492): one block of 32 values
void dequant_block(int typ, const uint8_t *b, float *out) {
    auto h = [&](int o) { return h2f(rd16(b + o)); };
    switch (typ) {
        case kQ4_0: {
            const float dd = h(0);
            const uint8_t *qs = b + 2;
            for (int j = 0; j < 16; ++j) {
                out[j] = (float)((int)(qs[j] & 0xF) - 8) * dd;
                out[j + 16] = (float)((int)(qs[j] >> 4) - 8) * dd;
            }
            break;
        }
        case kQ4_1: {
            const float dd = h(0), mm = h(2);
            const uint8_t *qs = b + 4;
            for (int j = 0; j < 16; ++j) {
                out[j] = (float)(qs[j] & 0xF) * dd + mm;
                out[j + 16] = (float)(qs[j] >> 4) * dd + mm;
            }
            break;
        }
        case kQ5_0: {
            const float dd = h(0);
            const uint32_t qh = rd32le(b + 2);
            const uint8_t *qs = b + 6;
            for (int j = 0; j < 16; ++j) {
                const uint8_t xh0 = (uint8_t)(((qh >> j) << 4) & 0x10), xh1 = (uint8_t)((qh >> (j + 12)) & 0x10);
                out[j] = (float)((int)((qs[j] & 0xF) | xh0) - 16) * dd;
                out[j + 16] = (float)((int)((qs[j] >> 4) | xh1) - 16) * dd;
            }
            break;
        }
        case kQ5_1: {
            const float dd = h(0), mm = h(2);
            const uint32_t qh = rd32le(b + 4);
            const uint8_t *qs = b + 8;
            for (int j = 0; j < 16; ++j) {
                const uint8_t xh0 = (uint8_t)(((qh >> j) << 4) & 0x10), xh1 = (uint8_t)((qh >> (j + 12)) & 0x10);
                out[j] = (float)((qs[j] & 0xF) | xh0) * dd + mm;
                out[j + 16] = (float)((qs[j] >> 4) | xh1) * dd + mm;
            }
            break;
        }
        case kQ8_0: {
            const float dd = h(0);
            for (int j = 0; j < 32; ++j) out[j] = (float)(int8_t)b[2 + j] * dd;
            break;
        }
    }
}

// toF16 (model.go:420-440) then f16tab: the reference's float16 values of
// any stored tensor, as float32
std::vector<float> widen_via_f16(int typ, const std::vector<uint8_t> &d, size_t n) {
    std::vector<float> out(n);
    if (typ == kF16) {
        for (size_t i = 0; i < n; ++i) out[i] = h2f(rd16(&d[2 * i]));
    } else if (typ == kF32) {
        for (size_t i = 0; i < n; ++i) {
            float f;
            memcpy(&f, &d[4 * i], 4);
            out[i] = h2f(f2h(f));
        }
    } else {
        size_t bs = 0;
        type_bytes(typ, 32, &bs);
        float blk[32];
        for (size_t b = 0; b < n / 32; ++b) {
            dequant_block(typ, &d[b * bs], blk);
            for (int j = 0; j < 32; ++j) out[b * 32 + j] = h2f(f2h(blk[j]));
        }
    }
    return out;
}

// toF32 (model.go:405-418): float32 as stored, else through float16
std::vector<float> to_f32(int typ, const std::vector<uint8_t> &d, size_t n) {
    if (typ != kF32) return widen_via_f16(typ, d, n);
    std::vector<float> out(n);
    memcpy(out.data(), d.data(), n * 4);
    return out;
}

struct File {
    FILE *f = nullptr;
    ~File() {
        if (f) fclose(f);
    }
    bool read(void *p, size_t n) { return n == 0 || fread(p, 1, n, f) == n; }
    bool i32(int32_t *v) {
        uint8_t b[4];
        if (!read(b, 4)) return false;
        *v = (int32_t)rd32le(b);
        return true;
    }
    // read and drop n bytes (a seek would not see a file cut short)
    bool skip(size_t n) {
        uint8_t buf[4096];
        while (n > 0) {
            const size_t c = n < sizeof buf ? n : sizeof buf;
            if (!read(buf, c)) return false;
            n -= c;
        }
        return true;
    }
};

const char *kFormat = "not a Whisper model file in whisper.cpp (ggml) format";

// The tensors Model.bind reads (model.go:360-397): name -> the element count
// and row length (ne[0]) it checks; matrices are `rows x cols` with ne[0] =
// cols.
struct Want {
    std::string name;
    size_t n;
    int ne0;
    bool matrix, decoder;
};

std::vector<Want> wanted(int nv, int actx, int st, int nmels, int alayers, int tctx, int tlayers) {
    std::vector<Want> w;
    auto vec = [&](const std::string &n, size_t c, bool dec) { w.push_back({n, c, (int)c, false, dec}); };
    auto mat = [&](const std::string &n, int rows, int cols, bool dec) {
        w.push_back({n, (size_t)rows * cols, cols, true, dec});
    };
    vec("encoder.positional_embedding", (size_t)actx * st, false);
    mat("encoder.conv1.weight", st, nmels * 3, false);
    vec("encoder.conv1.bias", st, false);
    mat("encoder.conv2.weight", st, st * 3, false);
    vec("encoder.conv2.bias", st, false);
    vec("encoder.ln_post.weight", st, false);
    vec("encoder.ln_post.bias", st, false);
    auto block = [&](const std::string &p, bool dec) {
        vec(p + "attn_ln.weight", st, dec);
        vec(p + "attn_ln.bias", st, dec);
        mat(p + "attn.query.weight", st, st, dec);
        vec(p + "attn.query.bias", st, dec);
        mat(p + "attn.key.weight", st, st, dec);
        mat(p + "attn.value.weight", st, st, dec);
        vec(p + "attn.value.bias", st, dec);
        mat(p + "attn.out.weight", st, st, dec);
        vec(p + "attn.out.bias", st, dec);
        if (dec) {
            vec(p + "cross_attn_ln.weight", st, dec);
            vec(p + "cross_attn_ln.bias", st, dec);
            mat(p + "cross_attn.query.weight", st, st, dec);
            vec(p + "cross_attn.query.bias", st, dec);
            mat(p + "cross_attn.key.weight", st, st, dec);
            mat(p + "cross_attn.value.weight", st, st, dec);
            vec(p + "cross_attn.value.bias", st, dec);
            mat(p + "cross_attn.out.weight", st, st, dec);
            vec(p + "cross_attn.out.bias", st, dec);
        }
        vec(p + "mlp_ln.weight", st, dec);
        vec(p + "mlp_ln.bias", st, dec);
        mat(p + "mlp.0.weight", 4 * st, st, dec);
        vec(p + "mlp.0.bias", 4 * st, dec);
        mat(p + "mlp.2.weight", st, 4 * st, dec);
        vec(p + "mlp.2.bias", st, dec);
    };
    for (int i = 0; i < alayers; ++i) block("encoder.blocks." + std::to_string(i) + ".", false);
    vec("decoder.positional_embedding", (size_t)tctx * st, true);
    mat("decoder.token_embedding.weight", nv, st, true);
    vec("decoder.ln.weight", st, true);
    vec("decoder.ln.bias", st, true);
    for (int i = 0; i < tlayers; ++i) block("decoder.blocks." + std::to_string(i) + ".", true);
    return w;
}

}  // namespace

extern "C" grx_status grx_whisper_load_ggml(grx_ctx *ctx, const char *path, int n_streams,
                                            grx_whisper_hparams *hp_out, grx_whisper **out) {
    if (!ctx || !path || !out) return grx_fail(GRX_EINVAL, "grx_whisper_load_ggml: NULL argument");
    *out = nullptr;
    File fh;
    fh.f = fopen(path, "rb");
    if (!fh.f) return grx_fail(GRX_EINVAL, "%s: cannot open", path);
    int32_t magic;
    if (!fh.i32(&magic) || (uint32_t)magic != kGgmlMagic) return grx_fail(GRX_EINVAL, "%s: %s", path, kFormat);
    int32_t hv[11];
    for (int i = 0; i < 11; ++i)
        if (!fh.i32(&hv[i])) return grx_fail(GRX_EINVAL, "%s: %s", path, kFormat);
    // hparams (model.go:16-20, 126-133)
    const int nv = hv[0], actx = hv[1], ast = hv[2], ahead = hv[3], alay = hv[4];
    const int tctx = hv[5], tst = hv[6], thead = hv[7], tlay = hv[8], nmels = hv[9];
    if (ast != tst || ast <= 0 || ahead <= 0 || ast % ahead != 0 || thead <= 0 || tst % thead != 0 || nmels <= 0 ||
        nmels > 256 || actx != 1500 || nv < 51864 || nv > 60000 || alay <= 0 || alay > 64 || tlay <= 0 || tlay > 64 ||
        tctx <= 0 || tctx > 4096)
        return grx_fail(GRX_ESIZE, "%s: the model's dimensions aren't ones this program knows", path);
    // mel filters (model.go:136-148)
    int32_t nmel, nfft;
    if (!fh.i32(&nmel) || !fh.i32(&nfft) || nmel != nmels || nfft != 201 ||
        !fh.skip((size_t)nmel * nfft * 4))
        return grx_fail(GRX_EINVAL, "%s: %s", path, kFormat);
    // vocabulary (model.go:150-168)
    int32_t nw;
    if (!fh.i32(&nw) || nw <= 0 || nw > nv) return grx_fail(GRX_EINVAL, "%s: %s", path, kFormat);
    for (int i = 0; i < nw; ++i) {
        int32_t l;
        if (!fh.i32(&l) || l < 0 || l > (1 << 16) || !fh.skip((size_t)l))
            return grx_fail(GRX_EINVAL, "%s: %s", path, kFormat);
    }
    const int st = tst;
    grx_whisper_hparams hp = {nv, tctx, st, thead, tlay, actx};
    const std::vector<Want> want = wanted(nv, actx, st, nmels, alay, tctx, tlay);
    std::vector<char> seen(want.size(), 0);  // 0 absent, 1 bound, 2 wrong shape
    std::string unknown;
    grx_whisper *m = nullptr;
    grx_status s = grx_whisper_create_streams(ctx, &hp, n_streams, &m);
    if (s != GRX_OK) return s;
    auto fail = [&](grx_status code, const char *fmt, const char *a, long b = 0) {
        grx_whisper_destroy(m);
        return grx_fail(code, fmt, path, a, b);
    };
    // tensors until the end of the file (model.go:171-219)
    for (;;) {
        uint8_t b4[4];
        const size_t got = fread(b4, 1, 4, fh.f);
        if (got == 0 && feof(fh.f)) break;
        if (got != 4) return fail(GRX_EINVAL, "%s: %s", kFormat);
        const int32_t nd = (int32_t)rd32le(b4);
        int32_t ln, tt;
        if (!fh.i32(&ln) || !fh.i32(&tt) || nd < 1 || nd > 4 || ln <= 0 || ln > 256)
            return fail(GRX_EINVAL, "%s: %s", kFormat);
        int ne[4] = {0, 0, 0, 0};
        size_t n = 1;
        for (int i = 0; i < nd; ++i) {
            int32_t v;
            // a dimension no real model has, or a size that overflows
            if (!fh.i32(&v) || v <= 0 || (size_t)v > (size_t(1) << 31) / n) return fail(GRX_EINVAL, "%s: %s", kFormat);
            ne[i] = v;
            n *= (size_t)v;
        }
        std::string name((size_t)ln, '\0');
        if (!fh.read(&name[0], (size_t)ln)) return fail(GRX_EINVAL, "%s: %s", kFormat);
        size_t size;
        if (!type_bytes(tt, n, &size))
            return fail(GRX_EINVAL, "%s: tensor %s has a weight type (%ld) this program can't read", name.c_str(), tt);
        std::vector<uint8_t> data(size);
        if (!fh.read(data.data(), size)) return fail(GRX_EINVAL, "%s: the model file is cut short%s", "");
        size_t k = 0;
        while (k < want.size() && want[k].name != name) ++k;
        if (k == want.size()) {
            if (unknown.empty()) unknown = name;
            continue;
        }
        const Want &w = want[k];
        // the shape check of bind's get (model.go:303-323); the last tensor
        // of a name counts, as in the reference's map
        seen[k] = n == w.n && (nd != 1 + (int)w.matrix || ne[0] == w.ne0) ? 1 : 2;
        if (seen[k] != 1 || !w.decoder) continue;
        // A vector is what the reference's vec() returns (model.go:325-337):
        // toF32 for a tensor load() widened to float32 (one dimension, a
        // single column, or a positional embedding: model.go:210-214), else
        // its float16 values.  A matrix is Q8_0: as stored, or the
        // reference's float16 values (mat(), model.go:338-351) rounded.
        if (!w.matrix) {
            const bool f32 = nd == 1 || ne[0] == 1 ||
                             (name.size() >= 20 && name.compare(name.size() - 20, 20, "positional_embedding") == 0);
            const std::vector<float> v = f32 ? to_f32(tt, data, n) : widen_via_f16(tt, data, n);
            s = grx_whisper_set_tensor(m, name.c_str(), v.data(), v.size() * 4);
        } else if (tt == kQ8_0) {
            s = grx_whisper_set_tensor(m, name.c_str(), data.data(), data.size());
        } else {
            const std::vector<float> v = widen_via_f16(tt, data, n);
            std::vector<uint8_t> q8(n / 32 * 34);
            s = grx_to_q8(ctx, (int)(n / (size_t)w.ne0), w.ne0, v.data(), q8.data());
            if (s == GRX_OK) s = grx_whisper_set_tensor(m, name.c_str(), q8.data(), q8.size());
        }
        if (s != GRX_OK) {
            grx_whisper_destroy(m);
            return s;
        }
    }
    // bind's errors in its order: the first missing or misshapen tensor,
    // then a tensor it does not know (model.go:398-404)
    for (size_t k = 0; k < want.size(); ++k) {
        if (seen[k] == 0) return fail(GRX_EINVAL, "%s: the model file has no tensor %s", want[k].name.c_str());
        if (seen[k] == 2) return fail(GRX_ESIZE, "%s: tensor %s has the wrong shape", want[k].name.c_str());
    }
    if (!unknown.empty())
        return fail(GRX_EINVAL, "%s: the model file has a tensor this program doesn't know: %s", unknown.c_str());
    if (hp_out) *hp_out = hp;
    *out = m;
    return GRX_OK;
}
