// pocket_load.hip - a Pocket TTS GGUF model file into the GPU flow LM.
//
// The flow-LM part of pockettts.Load (pockettts/model.go:201-250 with the
// loader of model.go:49-125) of github.com/xattribution/gorelaxor: the file
// must name itself a Pocket TTS model and its source; the LM's settings are
// read with the reference's range checks; layers are counted by their
// norm1.weight as the reference counts them and must match the setting; every
// tensor's shape is checked as mat()/vec() check it, with the same texts.
// The transformer matrices go from the file to their device tiles as stored
// (Q8_0, the form pack() gives the int8 kernels, model.go:322-366); the
// input projection and the end-of-speech row are float32 (the converter
// keeps matrices under 64 columns in float32).  When the file holds the flow
// head, it is declared and bound too (settings pockettts.flow.dim,
// flow.depth, decode_steps; matrices as stored).  grx_mimi_load_gguf reads
// the Mimi decoder from the same file; the tokenizer stays with the caller.
// Host code only.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <string>
#include <tuple>
#include <vector>

#include "grx_internal.h"
#include "pocket_internal.h"

namespace {

enum { kF32 = 0, kQ8_0 = 8, kBF16 = 30 };

struct Loader {
    const grx_gguf *f;
    std::string err;
    grx_status code = GRX_OK;

    void fail(grx_status c, const char *fmt, ...) {
        if (!err.empty()) return;
        char b[600];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(b, sizeof b, fmt, ap);
        va_end(ap);
        err = std::string("pockettts: ") + b;
        code = c;
    }
    // num (model.go:90-97)
    int num(const char *key) {
        const int64_t n = grx_gguf_int(f, key, -1);
        if (n < 1 || n > (1 << 16)) {
            fail(GRX_EINVAL, "the setting %s is %lld", key, (long long)n);
            return 1;
        }
        return (int)n;
    }
    int64_t elems(const std::string &name) {
        int nd = 0;
        int64_t dims[4];
        if (grx_gguf_tensor_info(f, name.c_str(), nullptr, &nd, dims) != GRX_OK) return -1;
        int64_t n = 1;
        for (int i = 0; i < nd; ++i) n *= dims[i];
        return n;
    }
    // vec (model.go:76-88): float32 values
    std::vector<float> vec(const std::string &name, int64_t n) {
        std::vector<float> v;
        if (!err.empty()) return v;
        if (elems(name) != n) {
            fail(GRX_EINVAL, "no %lld-value %s", (long long)n, name.c_str());
            return v;
        }
        v.resize((size_t)n);
        if (grx_gguf_float32(f, name.c_str(), v.data(), v.size()) != GRX_OK) fail(GRX_EINVAL, "%s", grx_last_error());
        return v;
    }
    // mat (model.go:61-74): the shape check; `q8` is whether this matrix
    // must be Q8_0 (the transformer's) or is read as float32
    bool mat_shape(const std::string &name, int64_t rows, int64_t cols) {
        if (!err.empty()) return false;
        int64_t r, c;
        if (grx_gguf_weight_shape(f, name.c_str(), &r, &c) != GRX_OK) {
            fail(GRX_EINVAL, "%s", grx_last_error());
            return false;
        }
        if (r != rows || c != cols) {
            fail(GRX_ESIZE, "%s is %lldx%lld, want %lldx%lld", name.c_str(), (long long)r, (long long)c,
                 (long long)rows, (long long)cols);
            return false;
        }
        return true;
    }
};

}  // namespace

extern "C" grx_status grx_pocket_load_gguf(grx_ctx *ctx, const char *path, int max_pos, grx_pocket_hparams *hp_out,
                                           grx_pocket **out) {
    if (!ctx || !path || !out) return grx_fail(GRX_EINVAL, "grx_pocket_load_gguf: NULL argument");
    *out = nullptr;
    grx_gguf *f = nullptr;
    grx_status s = grx_gguf_open(path, &f);
    if (s != GRX_OK) return s;
    struct Closer {
        grx_gguf *f;
        ~Closer() { grx_gguf_close(f); }
    } closer{f};
    const char *arch = grx_gguf_string(f, "general.architecture", "");
    if (std::string(arch) != "pockettts") return grx_fail(GRX_EINVAL, "pockettts: %s isn't a Pocket TTS model", path);
    if (std::string(grx_gguf_string(f, "general.source.sha256", "")).empty())
        return grx_fail(GRX_EINVAL, "pockettts: the file doesn't name its source");
    Loader l{f};
    grx_pocket_hparams hp{};
    hp.ldim = l.num("pockettts.latent_dim");
    hp.d = l.num("pockettts.lm.d_model");
    hp.heads = l.num("pockettts.lm.heads");
    hp.ff = l.num("pockettts.lm.ff");
    hp.period = grx_gguf_float(f, "pockettts.lm.max_period", 1e4);
    hp.max_pos = max_pos;
    // transformer() (model.go:99-125): heads, then layers while norm1 exists
    if (l.err.empty() && (hp.d % hp.heads != 0 || (hp.d / hp.heads) % 2 != 0))
        l.fail(GRX_ESIZE, "%d values don't split into %d heads", hp.d, hp.heads);
    int layers = 0;
    while (grx_gguf_has(f, ("lm.blk." + std::to_string(layers) + ".norm1.weight").c_str())) ++layers;
    if (l.err.empty() && layers == 0) l.fail(GRX_EINVAL, "no %s layers", "lm.blk");
    if (l.err.empty() && layers != l.num("pockettts.lm.layers")) l.fail(GRX_EINVAL, "the flow LM has %d layers", layers);
    hp.n_layer = layers;
    if (!l.err.empty()) return grx_fail(l.code, "%s", l.err.c_str());
    grx_pocket *m = nullptr;
    if ((s = grx_pocket_create(ctx, &hp, &m)) != GRX_OK) return s;
    m->sha = grx_gguf_string(f, "general.source.sha256", "");
    auto done = [&](grx_status st) {
        if (st != GRX_OK) grx_pocket_destroy(m);
        return st;
    };
    auto put_vec = [&](const std::string &name, int64_t n) {
        std::vector<float> v = l.vec(name, n);
        if (!l.err.empty()) return GRX_OK;
        return grx_pocket_set_tensor(m, name.c_str(), v.data(), v.size() * 4);
    };
    // a transformer matrix: Q8_0 rows from the file to the device
    auto put_q8 = [&](const std::string &name, int64_t rows, int64_t cols) {
        if (!l.mat_shape(name, rows, cols)) return GRX_OK;
        int type = -1;
        std::vector<uint8_t> d;
        grx_status st = grx_gguf_tensor_data(f, name.c_str(), &type, &d);
        if (st != GRX_OK) return st;
        if (type != kQ8_0) {
            l.fail(GRX_EINVAL, "%s is type %d; the device flow LM takes Q8_0 transformer weights", name.c_str(), type);
            return GRX_OK;
        }
        return grx_pocket_set_tensor(m, name.c_str(), d.data(), d.size());
    };
    // a small matrix the reference keeps in float32
    auto put_f32mat = [&](const std::string &name, int64_t rows, int64_t cols) {
        if (!l.mat_shape(name, rows, cols)) return GRX_OK;
        int nd, type;
        int64_t dims[4];
        grx_gguf_tensor_info(f, name.c_str(), &type, &nd, dims);
        if (type != kF32 && type != kBF16) {
            l.fail(GRX_EINVAL, "%s is type %d; the device flow LM takes it as float32", name.c_str(), type);
            return GRX_OK;
        }
        std::vector<float> v((size_t)(rows * cols));
        if (grx_gguf_float32(f, name.c_str(), v.data(), v.size()) != GRX_OK) return (grx_status)GRX_EINVAL;
        return grx_pocket_set_tensor(m, name.c_str(), v.data(), v.size() * 4);
    };
    const int64_t d = hp.d, ff = hp.ff, ld = hp.ldim;
    for (int i = 0; i < layers; ++i) {
        const std::string p = "lm.blk." + std::to_string(i) + ".";
        for (const char *n : {"norm1.weight", "norm1.bias", "norm2.weight", "norm2.bias"})
            if ((s = put_vec(p + n, d)) != GRX_OK) return done(s);
        if ((s = put_q8(p + "attn_qkv.weight", 3 * d, d)) != GRX_OK) return done(s);
        if ((s = put_q8(p + "attn_out.weight", d, d)) != GRX_OK) return done(s);
        if ((s = put_q8(p + "ff1.weight", ff, d)) != GRX_OK) return done(s);
        if ((s = put_q8(p + "ff2.weight", d, ff)) != GRX_OK) return done(s);
    }
    if ((s = put_f32mat("lm.input.weight", d, ld)) != GRX_OK) return done(s);
    if ((s = put_vec("lm.bos", ld)) != GRX_OK) return done(s);
    if ((s = put_vec("lm.out_norm.weight", d)) != GRX_OK) return done(s);
    if ((s = put_vec("lm.out_norm.bias", d)) != GRX_OK) return done(s);
    if ((s = put_f32mat("lm.eos.weight", 1, d)) != GRX_OK) return done(s);
    if ((s = put_vec("lm.eos.bias", 1)) != GRX_OK) return done(s);
    // the flow head (model.go:230-247): its settings, then its tensors as
    // stored (Q8_0 or float32 matrices, float32 vectors)
    if (l.err.empty() && grx_gguf_has(f, "flow.cond.weight")) {
        const int fd = l.num("pockettts.flow.dim"), depth = l.num("pockettts.flow.depth");
        const int steps = l.num("pockettts.decode_steps");
        if (l.err.empty() && (s = grx_pocket_flow_init(m, fd, depth, steps)) != GRX_OK) return done(s);
        auto put_any = [&](const std::string &name, int64_t rows, int64_t cols) {
            if (!l.mat_shape(name, rows, cols)) return GRX_OK;
            int type = -1;
            std::vector<uint8_t> d;
            grx_status st = grx_gguf_tensor_data(f, name.c_str(), &type, &d);
            if (st != GRX_OK) return st;
            if (type == kQ8_0) return grx_pocket_set_tensor(m, name.c_str(), d.data(), d.size());
            std::vector<float> v((size_t)(rows * cols));
            if (grx_gguf_float32(f, name.c_str(), v.data(), v.size()) != GRX_OK) return (grx_status)GRX_EINVAL;
            return grx_pocket_set_tensor(m, name.c_str(), v.data(), v.size() * 4);
        };
        const int64_t D = fd;
        for (auto mt : {std::make_tuple("flow.cond", D, d), std::make_tuple("flow.input", D, ld),
                        std::make_tuple("flow.final.ada", 2 * D, D), std::make_tuple("flow.final.out", ld, D)}) {
            const std::string p = std::get<0>(mt);
            if (l.err.empty() && (s = put_any(p + ".weight", std::get<1>(mt), std::get<2>(mt))) != GRX_OK)
                return done(s);
            if ((s = put_vec(p + ".bias", std::get<1>(mt))) != GRX_OK) return done(s);
        }
        for (int i = 0; i < 2; ++i) {
            const std::string p = "flow.time." + std::to_string(i) + ".";
            if ((s = put_vec(p + "freqs", 128)) != GRX_OK) return done(s);
            if (l.err.empty() && (s = put_any(p + "fc1.weight", D, 256)) != GRX_OK) return done(s);
            if ((s = put_vec(p + "fc1.bias", D)) != GRX_OK) return done(s);
            if (l.err.empty() && (s = put_any(p + "fc2.weight", D, D)) != GRX_OK) return done(s);
            if ((s = put_vec(p + "fc2.bias", D)) != GRX_OK) return done(s);
            if ((s = put_vec(p + "norm.alpha", D)) != GRX_OK) return done(s);
        }
        for (int i = 0; i < depth && l.err.empty(); ++i) {
            const std::string p = "flow.res." + std::to_string(i) + ".";
            for (const char *v : {"norm.weight", "norm.bias", "fc1.bias", "fc2.bias"})
                if ((s = put_vec(p + v, D)) != GRX_OK) return done(s);
            if ((s = put_vec(p + "ada.bias", 3 * D)) != GRX_OK) return done(s);
            if (l.err.empty() && (s = put_any(p + "fc1.weight", D, D)) != GRX_OK) return done(s);
            if (l.err.empty() && (s = put_any(p + "fc2.weight", D, D)) != GRX_OK) return done(s);
            if (l.err.empty() && (s = put_any(p + "ada.weight", 3 * D, D)) != GRX_OK) return done(s);
        }
    }
    if (!l.err.empty()) return done(grx_fail(l.code, "%s", l.err.c_str()));
    if (hp_out) *hp_out = hp;
    *out = m;
    return GRX_OK;
}

// The Mimi decoder of a Pocket TTS GGUF file (the Mimi part of
// pockettts.Load, pockettts/model.go:280-308, with its decoder() and
// resBlocks() walks, model.go:128-181): the file's name and source checks,
// the frame size from sample_rate and frame_rate (model.go:208-213), the
// Mimi and SEANet settings with the reference's range checks and texts, the
// transformer's heads and layer count (model.go:103-125), then every tensor
// the decoder reads, its shape checked as mat()/vec() check it, matrices
// as stored (Q8_0 or float32), vectors float32.
extern "C" grx_status grx_mimi_load_gguf(grx_ctx *ctx, const char *path, int max_latents, grx_mimi_hparams *hp_out,
                                         grx_mimi **out) {
    if (!ctx || !path || !out) return grx_fail(GRX_EINVAL, "grx_mimi_load_gguf: NULL argument");
    *out = nullptr;
    grx_gguf *f = nullptr;
    grx_status s = grx_gguf_open(path, &f);
    if (s != GRX_OK) return s;
    struct Closer {
        grx_gguf *f;
        ~Closer() { grx_gguf_close(f); }
    } closer{f};
    const char *arch = grx_gguf_string(f, "general.architecture", "");
    if (std::string(arch) != "pockettts") return grx_fail(GRX_EINVAL, "pockettts: %s isn't a Pocket TTS model", path);
    if (std::string(grx_gguf_string(f, "general.source.sha256", "")).empty())
        return grx_fail(GRX_EINVAL, "pockettts: the file doesn't name its source");
    Loader l{f};
    grx_mimi_hparams hp{};
    hp.ldim = l.num("pockettts.latent_dim");
    const int sr = l.num("pockettts.sample_rate");
    const double fr = grx_gguf_float(f, "pockettts.frame_rate", 0);
    if (fr <= 0 || fmod((double)sr, fr) != 0) l.fail(GRX_EINVAL, "a frame rate of %g", fr);
    const int frame = fr > 0 ? (int)((double)sr / fr) : 0;
    hp.d = l.num("pockettts.mimi.d_model");
    hp.heads = l.num("pockettts.mimi.heads");
    hp.ff = l.num("pockettts.mimi.ff");
    hp.context = l.num("pockettts.mimi.context");
    hp.period = grx_gguf_float(f, "pockettts.mimi.max_period", 1e4);
    hp.upsample = l.num("pockettts.mimi.upsample");
    const int64_t nr = grx_gguf_array_len(f, "pockettts.seanet.ratios");
    std::vector<int> ratios;
    for (int64_t i = 0; i < nr; ++i) ratios.push_back((int)grx_gguf_array_int(f, "pockettts.seanet.ratios", i));
    hp.n_filters = l.num("pockettts.seanet.n_filters");
    const int dim = l.num("pockettts.seanet.dimension");
    hp.kernel_size = l.num("pockettts.seanet.kernel_size");
    hp.residual_kernel_size = l.num("pockettts.seanet.residual_kernel_size");
    hp.last_kernel_size = l.num("pockettts.seanet.last_kernel_size");
    hp.dilation_base = l.num("pockettts.seanet.dilation_base");
    hp.compress = l.num("pockettts.seanet.compress");
    hp.n_residual = l.num("pockettts.seanet.n_residual_layers");
    long long hop = 1;
    for (int r : ratios) {
        if (r < 1 || r > 64) l.fail(GRX_EINVAL, "a SEANet ratio of %d", r);
        hop *= r;
    }
    if (l.err.empty() && (ratios.empty() || dim != hp.d || hop * hp.upsample != frame)) {
        std::string v = "[";
        for (size_t i = 0; i < ratios.size(); ++i) v += (i ? " " : "") + std::to_string(ratios[i]);
        v += "]";
        l.fail(GRX_EINVAL, "SEANet's ratios %s don't make %d-sample frames", v.c_str(), frame);
    }
    if (l.err.empty() && ratios.size() > 8) l.fail(GRX_ESIZE, "%zu SEANet ratios; this decoder takes up to 8", ratios.size());
    hp.n_ratios = (int)ratios.size();
    for (int i = 0; i < hp.n_ratios && i < 8; ++i) hp.ratios[i] = ratios[i];
    // transformer() (model.go:103-125): heads, then layers while norm1 exists
    if (l.err.empty() && (hp.d % hp.heads != 0 || (hp.d / hp.heads) % 2 != 0))
        l.fail(GRX_ESIZE, "%d values don't split into %d heads", hp.d, hp.heads);
    int layers = 0;
    while (grx_gguf_has(f, ("mimi.dec_tf." + std::to_string(layers) + ".norm1.weight").c_str())) ++layers;
    if (l.err.empty() && layers == 0) l.fail(GRX_EINVAL, "no %s layers", "mimi.dec_tf");
    hp.layers = layers;
    hp.max_latents = max_latents;
    if (!l.err.empty()) return grx_fail(l.code, "%s", l.err.c_str());
    grx_mimi *m = nullptr;
    if ((s = grx_mimi_create(ctx, &hp, &m)) != GRX_OK) return s;
    auto done = [&](grx_status st) {
        if (st != GRX_OK) grx_mimi_destroy(m);
        return st;
    };
    auto put_vec = [&](const std::string &name, int64_t n) {
        std::vector<float> v = l.vec(name, n);
        if (!l.err.empty()) return GRX_OK;
        return grx_mimi_set_tensor(m, name.c_str(), v.data(), v.size() * 4);
    };
    // a matrix as the file stores it: Q8_0 rows, or float32 (F32/F16/BF16)
    auto put_mat = [&](const std::string &name, int64_t rows, int64_t cols) {
        if (!l.mat_shape(name, rows, cols)) return GRX_OK;
        int type = -1, nd = 0;
        int64_t dims[4];
        grx_gguf_tensor_info(f, name.c_str(), &type, &nd, dims);
        if (type == kQ8_0) {
            std::vector<uint8_t> d;
            grx_status st = grx_gguf_tensor_data(f, name.c_str(), &type, &d);
            if (st != GRX_OK) return st;
            return grx_mimi_set_tensor(m, name.c_str(), d.data(), d.size());
        }
        std::vector<float> v((size_t)(rows * cols));
        if (grx_gguf_float32(f, name.c_str(), v.data(), v.size()) != GRX_OK) {
            l.fail(GRX_EINVAL, "%s", grx_last_error());
            return GRX_OK;
        }
        return grx_mimi_set_tensor(m, name.c_str(), v.data(), v.size() * 4);
    };
    auto conv = [&](const std::string &name, int cin, int cout, int k) {
        grx_status st = put_mat(name + ".weight", cout, (int64_t)k * cin);
        return st != GRX_OK ? st : put_vec(name + ".bias", cout);
    };
    const int64_t d = hp.d;
    if ((s = put_mat("mimi.quant", d, hp.ldim)) != GRX_OK) return done(s);
    if ((s = put_vec("mimi.up", d * 2 * hp.upsample)) != GRX_OK) return done(s);
    for (int i = 0; i < layers; ++i) {
        const std::string p = "mimi.dec_tf." + std::to_string(i) + ".";
        for (const char *n : {"norm1.weight", "norm1.bias", "norm2.weight", "norm2.bias"})
            if ((s = put_vec(p + n, d)) != GRX_OK) return done(s);
        if ((s = put_mat(p + "attn_qkv.weight", 3 * d, d)) != GRX_OK) return done(s);
        if ((s = put_mat(p + "attn_out.weight", d, d)) != GRX_OK) return done(s);
        if ((s = put_mat(p + "ff1.weight", hp.ff, d)) != GRX_OK) return done(s);
        if ((s = put_mat(p + "ff2.weight", d, hp.ff)) != GRX_OK) return done(s);
        if ((s = put_vec(p + "ls1", d)) != GRX_OK) return done(s);
        if ((s = put_vec(p + "ls2", d)) != GRX_OK) return done(s);
    }
    // decoder() (model.go:163-181): a conv, per ratio a transposed conv and
    // the residual blocks (resBlocks, model.go:140-156), a last conv
    int mult = 1 << hp.n_ratios, idx = 1;
    const int nf = hp.n_filters;
    if ((s = conv("mimi.dec.0", hp.d, mult * nf, hp.kernel_size)) != GRX_OK) return done(s);
    for (int r : ratios) {
        ++idx;
        const std::string tn = "mimi.dec." + std::to_string(idx);
        const int cin = mult * nf, cout = mult * nf / 2;
        if ((s = put_mat(tn + ".weight", (int64_t)2 * r * cout, cin)) != GRX_OK) return done(s);
        if ((s = put_vec(tn + ".bias", cout)) != GRX_OK) return done(s);
        ++idx;
        const int rdim = cout;
        for (int j = 0; j < hp.n_residual; ++j) {
            const std::string p = "mimi.dec." + std::to_string(idx) + ".";
            if ((s = conv(p + "1", rdim, rdim / hp.compress, hp.residual_kernel_size)) != GRX_OK) return done(s);
            if ((s = conv(p + "3", rdim / hp.compress, rdim, 1)) != GRX_OK) return done(s);
            ++idx;
        }
        mult /= 2;
    }
    ++idx;
    if ((s = conv("mimi.dec." + std::to_string(idx), nf, 1, hp.last_kernel_size)) != GRX_OK) return done(s);
    if (!l.err.empty()) return done(grx_fail(l.code, "%s", l.err.c_str()));
    if (hp_out) *hp_out = hp;
    *out = m;
    return GRX_OK;
}
