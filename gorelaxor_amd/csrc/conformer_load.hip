// conformer_load.hip - a FastConformer (parakeet) GGUF model file into the
// GPU encoder.
//
// The encoder part of conformer.Load (conformer/model.go:253-422) of
// github.com/xattribution/gorelaxor: the architecture check, readHParams and
// readEncoder's settings and checks (model.go:163-235, the same texts), then
// loadEncoder's tensors in its order (model.go:358-422; a missing tensor is
// reported as the reference reports the first one it misses, an optional
// bias may be absent).  Linear weights go from the file to their device
// tiles as stored (Q8_0); the pointwise convolutions may be float16 or
// float32 and are rounded by Weight.ToQ8 as the reference rounds them in a
// Q8_0 file; the pre-encoder's conv.3 and conv.6 may be float32, as the
// converter stores them, and keep kern's float route; taps and vectors are
// widened to float32 (File.Float32), and
// the device driver transposes the taps and folds the batch norm.  Where
// the reference would find a tensor that does not fit the settings only
// when the first recording panics ("the model file doesn't fit its own
// settings"), the shapes are checked here at load, with that text.  The
// attention and convolution forms and the streaming settings are read as
// readEncoder and readHParams read them.  The RNN-T/TDT decoder and the
// vocabulary stay with the caller.  Host code only.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <string>
#include <vector>

#include "grx_internal.h"

namespace {

enum { kF32 = 0, kF16 = 1, kQ8_0 = 8, kBF16 = 30 };

struct CLoader {
    grx_ctx *ctx;
    const grx_gguf *f;
    grx_conformer *m = nullptr;
    std::string err;
    grx_status code = GRX_OK;

    bool ok() const { return err.empty(); }
    void fail(grx_status c, const char *fmt, ...) {
        if (!err.empty()) return;
        char b[700];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(b, sizeof b, fmt, ap);
        va_end(ap);
        err = b;
        code = c;
    }
    void misfit(const char *fmt, ...) {
        if (!err.empty()) return;
        char b[600];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(b, sizeof b, fmt, ap);
        va_end(ap);
        fail(GRX_ESIZE, "conformer: the model file doesn't fit its own settings (%s)", b);
    }
    bool present(const std::string &name, bool optional) {
        if (!ok()) return false;
        if (!grx_gguf_has(f, name.c_str())) {
            if (!optional) fail(GRX_EINVAL, "conformer: the model has no %s", name.c_str());
            return false;
        }
        return true;
    }
    void put(const std::string &name, const void *d, size_t n) {
        if (!ok()) return;
        if (grx_conformer_set_tensor(m, name.c_str(), d, n) != GRX_OK) fail(GRX_EINVAL, "%s", grx_last_error());
    }
    int64_t elems(const std::string &name) {
        int nd = 0;
        int64_t dims[4];
        grx_gguf_tensor_info(f, name.c_str(), nullptr, &nd, dims);
        int64_t n = 1;
        for (int i = 0; i < nd; ++i) n *= dims[i];
        return n;
    }
    // vec (model.go:113-128): float32 values, n of them
    void vec(const std::string &name, int64_t n, bool optional = false) {
        if (!present(name, optional)) return;
        const int64_t e = elems(name);
        if (e != n) {
            misfit("%s has %lld values, want %lld", name.c_str(), (long long)e, (long long)n);
            return;
        }
        std::vector<float> v((size_t)n);
        if (grx_gguf_float32(f, name.c_str(), v.data(), v.size()) != GRX_OK) {
            fail(GRX_EINVAL, "%s", grx_last_error());
            return;
        }
        put(name, v.data(), v.size() * 4);
    }
    // mat (model.go:130-146) with the shape the encoder multiplies by.
    // kLinear: Q8_0 only; kPointwise: float16 / float32 too, rounded by
    // Weight.ToQ8; kFloat: float32 too, kept for kern's float route.
    enum Kind { kLinear, kPointwise, kFloat };
    void mat(const std::string &name, int64_t rows, int64_t cols, Kind kind = kLinear) {
        const bool pointwise = kind == kPointwise;
        if (!present(name, false)) return;
        int64_t r, c;
        if (grx_gguf_weight_shape(f, name.c_str(), &r, &c) != GRX_OK) {
            fail(GRX_EINVAL, "%s", grx_last_error());
            return;
        }
        if (r != rows || c != cols) {
            misfit("%s is %lldx%lld, want %lldx%lld", name.c_str(), (long long)r, (long long)c, (long long)rows,
                   (long long)cols);
            return;
        }
        int type = -1;
        std::vector<uint8_t> d;
        if (grx_gguf_tensor_data(f, name.c_str(), &type, &d) != GRX_OK) {
            fail(GRX_EINVAL, "%s", grx_last_error());
            return;
        }
        if (type == kQ8_0 || (pointwise && type == kF16)) {
            put(name, d.data(), d.size());
        } else if (kind == kFloat && (type == kF32 || type == kBF16)) {
            std::vector<float> v((size_t)(rows * cols));
            if (grx_gguf_float32(f, name.c_str(), v.data(), v.size()) != GRX_OK) {
                fail(GRX_EINVAL, "%s", grx_last_error());
                return;
            }
            put(name, v.data(), v.size() * 4);
        } else if (pointwise) {  // float32 or bfloat16 values, rounded here
            std::vector<float> v((size_t)(rows * cols));
            std::vector<uint8_t> q((size_t)(rows * (cols / 32) * 34));
            if (grx_gguf_float32(f, name.c_str(), v.data(), v.size()) != GRX_OK ||
                grx_to_q8(ctx, (int)rows, (int)cols, v.data(), q.data()) != GRX_OK) {
                fail(GRX_EINVAL, "%s", grx_last_error());
                return;
            }
            put(name, q.data(), q.size());
        } else {
            fail(GRX_EINVAL, "conformer: %s is type %d; the device encoder takes Q8_0 linear weights%s", name.c_str(),
                 type, kind == kFloat ? " or float32 ones" : "");
        }
    }
};

}  // namespace

extern "C" grx_status grx_conformer_load_gguf(grx_ctx *ctx, const char *path, grx_conformer_hparams *hp_out,
                                              grx_conformer **out) {
    if (!ctx || !path || !out) return grx_fail(GRX_EINVAL, "grx_conformer_load_gguf: NULL argument");
    *out = nullptr;
    grx_gguf *f = nullptr;
    grx_status s = grx_gguf_open(path, &f);
    if (s != GRX_OK) return s;
    struct Closer {
        grx_gguf *f;
        ~Closer() { grx_gguf_close(f); }
    } closer{f};
    const std::string arch = grx_gguf_string(f, "general.architecture", "");
    if (arch != "parakeet")
        return grx_fail(GRX_EINVAL, "conformer: architecture \"%s\" is not a FastConformer transducer", arch.c_str());
    // readEncoder (model.go:163-190)
    const std::string p = "stt.parakeet.encoder.";
    auto I = [&](const char *k, int64_t def) { return grx_gguf_int(f, (p + k).c_str(), def); };
    const int64_t d = I("d_model", 0), heads = I("n_heads", 0), layers = I("n_layers", 0), dff = I("d_ff", 0);
    const int64_t kernel = I("conv_kernel", 0), subc = I("subsampling_channels", 0), sub = I("subsampling_factor", 8);
    const bool xscaling = grx_gguf_bool(f, (p + "xscaling").c_str(), 0) != 0;
    const std::string style = grx_gguf_string(f, (p + "att_context_style").c_str(), "regular");
    const int64_t att_l = I("att_context_left", -1), att_r = I("att_context_right", -1);
    const int64_t conv_l = I("conv_context_left", -1), conv_r = I("conv_context_right", -1);
    std::string conv_norm = grx_gguf_string(f, (p + "conv_norm_type").c_str(), "batch_norm");
    const bool causal_sub = grx_gguf_bool(f, (p + "causal_downsampling").c_str(), style == "chunked_limited") != 0;
    if (d <= 0 || heads <= 0 || d % heads != 0 || layers <= 0 || kernel <= 0)
        return grx_fail(GRX_EINVAL, "conformer: the model file is missing its encoder settings");
    if (sub != 8) return grx_fail(GRX_EINVAL, "conformer: subsampling %lld is not supported (only 8)", (long long)sub);
    if (conv_norm.empty()) conv_norm = "batch_norm";
    // readHParams' checks of the decoder's settings (model.go:192-235)
    const std::string q = "stt.parakeet.";
    const std::string head = grx_gguf_string(f, (q + "head_kind").c_str(), "rnnt");
    if (head == "tdt") {
        if (grx_gguf_array_len(f, (q + "tdt.durations").c_str()) <= 0)
            return grx_fail(GRX_EINVAL, "conformer: a TDT model needs its durations");
        const int64_t ms = grx_gguf_int(f, (q + "tdt.max_symbols").c_str(), 10);
        if (ms < 1 || ms > 100)
            return grx_fail(GRX_EINVAL, "conformer: tdt.max_symbols %lld is out of range", (long long)ms);
    } else if (head != "rnnt") {
        return grx_fail(GRX_EINVAL, "conformer: \"%s\" models are not supported (only RNN-T and TDT)", head.c_str());
    }
    if (grx_gguf_int(f, (q + "predictor.vocab").c_str(), 0) < 2 || grx_gguf_int(f, (q + "predictor.hidden").c_str(), 0) <= 0 ||
        grx_gguf_int(f, (q + "predictor.n_layers").c_str(), 0) <= 0 || grx_gguf_int(f, (q + "joint.hidden").c_str(), 0) <= 0)
        return grx_fail(GRX_EINVAL, "conformer: the model file is missing its decoder settings");
    if (att_l < -1 || att_r < -1 || conv_l < -1 || conv_r < -1 || att_l > (1 << 20) || att_r > (1 << 20) ||
        conv_l > (1 << 20) || conv_r > (1 << 20))
        return grx_fail(GRX_EINVAL, "conformer: the model file is missing its encoder settings");
    // att_context_size_choices: (left, right) pairs (readHParams, model.go:212-216)
    std::vector<int64_t> choices;
    {
        const int64_t n = grx_gguf_array_len(f, (q + "encoder.att_context_size_choices").c_str());
        if (n >= 2 && n <= 1024)
            for (int64_t i = 0; i < n; ++i)
                choices.push_back(grx_gguf_array_int(f, (q + "encoder.att_context_size_choices").c_str(), i));
        else if (n > 1024)
            return grx_fail(GRX_EINVAL, "conformer: %lld attention context choices", (long long)n / 2);
    }
    if (choices.size() / 2 > 8)
        return grx_fail(GRX_EINVAL, "conformer: %zu attention context choices (this build takes 8)", choices.size() / 2);
    if (conv_norm != "batch_norm" && conv_norm != "layer_norm")
        return grx_fail(GRX_EINVAL, "conformer: conv_norm_type \"%s\" is not supported", conv_norm.c_str());
    const int64_t n_mels = grx_gguf_int(f, "stt.frontend.num_mels", 80);  // melConfig, model.go:237-251
    if (d > (1 << 16) || dff > (1 << 18) || layers > 1024 || kernel > 1024 || subc > (1 << 16) || n_mels < 1 ||
        n_mels > 4096 || heads > 1024)
        return grx_fail(GRX_EINVAL, "conformer: the model file is missing its encoder settings");
    grx_conformer_hparams hp{};
    hp.d = (int)d;
    hp.heads = (int)heads;
    hp.layers = (int)layers;
    hp.dff = (int)dff;
    hp.conv_kernel = (int)kernel;
    hp.sub_channels = (int)subc;
    hp.n_mels = (int)n_mels;
    hp.xscaling = xscaling;
    hp.conv_ln = conv_norm == "layer_norm";
    hp.att_chunked = style == "chunked_limited";  // HParams.Causal (model.go:46)
    hp.att_left = (int)att_l;
    hp.att_right = (int)att_r;
    hp.conv_left = (int)conv_l;
    hp.conv_right = (int)conv_r;
    hp.causal_sub = causal_sub;
    hp.n_context_choices = (int)(choices.size() / 2);
    for (size_t i = 0; i + 1 < choices.size(); i += 2) {
        if (choices[i] < -1 || choices[i] > (1 << 20) || choices[i + 1] < -1 || choices[i + 1] > (1 << 20))
            return grx_fail(GRX_EINVAL, "conformer: attention context choice [%lld, %lld] is out of range",
                            (long long)choices[i], (long long)choices[i + 1]);
        hp.context_choices[i / 2][0] = (int)choices[i];
        hp.context_choices[i / 2][1] = (int)choices[i + 1];
    }
    // the streaming settings (readHParams, model.go:193-196)
    const auto clampi = [](int64_t v) { return (int)std::max<int64_t>(-1, std::min<int64_t>(v, 1 << 20)); };
    hp.pre_encode_cache = clampi(grx_gguf_int(f, (q + "encoder.streaming.pre_encode_cache_size").c_str(), -1));
    hp.drop_extra = clampi(grx_gguf_int(f, (q + "encoder.streaming.drop_extra_pre_encoded").c_str(), -1));
    hp.sampling_frames_first = clampi(grx_gguf_int(f, (q + "encoder.streaming.sampling_frames_first").c_str(), -1));
    CLoader l{ctx, f};
    if ((s = grx_conformer_create(ctx, &hp, &l.m)) != GRX_OK) return s;
    // loadEncoder (model.go:358-422), in its order
    int64_t F = n_mels;  // subOut three times (encoder.go:33-38)
    for (int k = 0; k < 3; ++k) F = causal_sub ? F / 2 + 1 : (F - 1) / 2 + 1;
    const int64_t c = subc;
    const std::string pe = "enc.pre_encode.";
    l.vec(pe + "conv.0.weight", c * 9);
    l.vec(pe + "conv.0.bias", c);
    l.vec(pe + "conv.2.weight", c * 9);
    l.vec(pe + "conv.2.bias", c);
    l.mat(pe + "conv.3.weight", c, c, CLoader::kFloat);
    l.vec(pe + "conv.3.bias", c);
    l.vec(pe + "conv.5.weight", c * 9);
    l.vec(pe + "conv.5.bias", c);
    l.mat(pe + "conv.6.weight", c, c, CLoader::kFloat);
    l.vec(pe + "conv.6.bias", c);
    l.mat(pe + "out.weight", d, c * F);
    l.vec(pe + "out.bias", d);
    for (int i = 0; i < layers && l.ok(); ++i) {
        const std::string b = "enc.blocks." + std::to_string(i) + ".";
        for (const char *n : {"ff1", "ff2"}) {
            l.vec(b + "norm_" + n + ".weight", d);
            l.vec(b + "norm_" + n + ".bias", d);
            l.mat(b + n + ".linear1.weight", dff, d);
            l.vec(b + n + ".linear1.bias", dff, true);
            l.mat(b + n + ".linear2.weight", d, dff);
            l.vec(b + n + ".linear2.bias", d, true);
        }
        l.vec(b + "norm_attn.weight", d);
        l.vec(b + "norm_attn.bias", d);
        for (const char *n : {"linear_q", "linear_k", "linear_v", "linear_out"}) {
            l.mat(b + "attn." + n + ".weight", d, d);
            l.vec(b + "attn." + n + ".bias", d, true);
        }
        l.mat(b + "attn.linear_pos.weight", d, d);
        l.vec(b + "attn.pos_bias_u", d);
        l.vec(b + "attn.pos_bias_v", d);
        l.vec(b + "norm_conv.weight", d);
        l.vec(b + "norm_conv.bias", d);
        l.mat(b + "conv.pointwise1.weight", 2 * d, d, CLoader::kPointwise);
        l.vec(b + "conv.pointwise1.bias", 2 * d, true);
        l.mat(b + "conv.pointwise2.weight", d, d, CLoader::kPointwise);
        l.vec(b + "conv.pointwise2.bias", d, true);
        l.vec(b + "conv.depthwise.weight", d * kernel);
        l.vec(b + "conv.depthwise.bias", d, true);
        l.vec(b + "norm_out.weight", d);
        l.vec(b + "norm_out.bias", d);
        l.vec(b + "conv.bn.weight", d);
        l.vec(b + "conv.bn.bias", d);
        if (!hp.conv_ln) {
            l.vec(b + "conv.bn.running_mean", d);
            l.vec(b + "conv.bn.running_var", d);
        }
    }
    if (!l.ok()) {
        grx_conformer_destroy(l.m);
        return grx_fail(l.code, "%s", l.err.c_str());
    }
    if (hp_out) *hp_out = hp;
    *out = l.m;
    return GRX_OK;
}
