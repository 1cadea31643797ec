// rnnt_load.hip - the transducer head of a FastConformer GGUF file.
//
// conformer/model.go:191-235 (readHParams' decoder settings and checks) and
// :306-315, 337-339 (the decoder tensors fromGGUF reads, in its order; the
// blank id defaulting to the last token) of github.com/xattribution/
// gorelaxor.  Q8_0 matrices go from the file to their device tiles as
// stored; vectors are widened to float32 as gguf.File.Float32 does.
#include <string>
#include <vector>

#include "grx.h"
#include "grx_internal.h"

extern "C" grx_status grx_rnnt_load_gguf(grx_ctx *ctx, const char *path, grx_rnnt_hparams *hp_out, grx_rnnt **out) {
    if (!ctx || !path || !out) return grx_fail(GRX_EINVAL, "grx_rnnt_load_gguf: NULL argument");
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
    const std::string q = "stt.parakeet.";
    auto I = [&](const std::string &k, int64_t def) { return grx_gguf_int(f, (q + k).c_str(), def); };
    const std::string head = grx_gguf_string(f, (q + "head_kind").c_str(), "rnnt");
    grx_rnnt_hparams hp{};
    hp.d = (int)I("encoder.d_model", 0);
    const int64_t H = I("predictor.hidden", 0), L = I("predictor.n_layers", 0), V = I("predictor.vocab", 0);
    const int64_t J = I("joint.hidden", 0);
    const std::string act = grx_gguf_string(f, (q + "joint.activation").c_str(), "relu");
    if (head == "tdt") {
        const int64_t nd = grx_gguf_array_len(f, (q + "tdt.durations").c_str());
        if (nd <= 0) return grx_fail(GRX_EINVAL, "conformer: a TDT model needs its durations");
        const int64_t ms = I("tdt.max_symbols", 10);
        if (ms < 1 || ms > 100)
            return grx_fail(GRX_EINVAL, "conformer: tdt.max_symbols %lld is out of range", (long long)ms);
        if (nd > 16) return grx_fail(GRX_ESIZE, "grx_rnnt_load_gguf: %lld durations (at most 16)", (long long)nd);
        hp.tdt = 1;
        hp.n_durations = (int)nd;
        for (int i = 0; i < nd; ++i) {
            const int64_t v = grx_gguf_array_int(f, (q + "tdt.durations").c_str(), i);
            if (v < 0 || v > (1 << 20)) return grx_fail(GRX_EINVAL, "grx_rnnt_load_gguf: duration %lld", (long long)v);
            hp.durations[i] = (int)v;
        }
        hp.max_symbols = (int)ms;
    } else if (head == "rnnt") {
        hp.max_symbols = 10;
    } else {
        return grx_fail(GRX_EINVAL, "conformer: \"%s\" models are not supported (only RNN-T and TDT)", head.c_str());
    }
    if (V < 2 || H <= 0 || L <= 0 || J <= 0)
        return grx_fail(GRX_EINVAL, "conformer: the model file is missing its decoder settings");
    if (H > (1 << 15) || J > (1 << 15) || L > 64 || V > (1 << 24) || hp.d <= 0 || hp.d > (1 << 16))
        return grx_fail(GRX_EINVAL, "conformer: the model file doesn't fit its own settings (decoder sizes)");
    hp.pred_hidden = (int)H;
    hp.pred_layers = (int)L;
    hp.pred_vocab = (int)V;
    hp.joint_hidden = (int)J;
    hp.joint_act = act == "sigmoid" ? 1 : act == "tanh" ? 2 : 0;  // joint's switch: anything else is ReLU
    const int64_t blank = grx_gguf_int(f, "tokenizer.ggml.blank_token_id", -1);
    if (blank >= V) return grx_fail(GRX_EINVAL, "conformer: the model file doesn't fit its own settings (blank id)");
    hp.blank = (int)blank;
    grx_rnnt *m = nullptr;
    if ((s = grx_rnnt_create(ctx, &hp, &m)) != GRX_OK) return s;
    struct Guard {
        grx_rnnt *m;
        ~Guard() {
            if (m) grx_rnnt_destroy(m);
        }
    } guard{m};
    std::vector<std::string> names = {"pred.embed.weight"};
    for (int i = 0; i < L; ++i)
        for (const char *n : {"Wx", "Wh", "bias"}) names.push_back("pred.lstm." + std::to_string(i) + "." + n);
    for (const char *n : {"joint.enc.weight", "joint.enc.bias", "joint.pred.weight", "joint.pred.bias",
                          "joint.out.weight", "joint.out.bias"})
        names.push_back(n);
    const int nd = hp.tdt ? hp.n_durations : 0;
    for (const std::string &n : names) {
        if (!grx_gguf_has(f, n.c_str())) return grx_fail(GRX_EINVAL, "conformer: the model has no %s", n.c_str());
        const bool mat = n.size() > 7 && (n.compare(n.size() - 7, 7, ".weight") == 0 || n.back() == 'x' ||
                                          n.back() == 'h') && n != "pred.embed.weight";
        if (mat) {
            int64_t r = 0, c = 0;
            if ((s = grx_gguf_weight_shape(f, n.c_str(), &r, &c)) != GRX_OK) return s;
            int64_t wr = 4 * H, wc = H;
            if (n == "joint.enc.weight") wr = J, wc = hp.d;
            else if (n == "joint.pred.weight") wr = J, wc = H;
            else if (n == "joint.out.weight") wr = V + nd, wc = J;
            if (r != wr || c != wc)
                return grx_fail(GRX_EINVAL,
                                "conformer: the model file doesn't fit its own settings (%s is %lldx%lld, not %lldx%lld)",
                                n.c_str(), (long long)r, (long long)c, (long long)wr, (long long)wc);
            int type = -1;
            std::vector<uint8_t> bytes;
            if ((s = grx_gguf_tensor_data(f, n.c_str(), &type, &bytes)) != GRX_OK) return s;
            if (type != 8)
                return grx_fail(GRX_EINVAL, "grx_rnnt_load_gguf: %s is ggml type %d; this build takes Q8_0 matrices",
                                n.c_str(), type);
            if ((s = grx_rnnt_set_tensor(m, n.c_str(), bytes.data(), bytes.size())) != GRX_OK) return s;
        } else {
            int64_t dims[4] = {0, 0, 0, 0};
            int ndim = 0;
            grx_gguf_tensor_info(f, n.c_str(), nullptr, &ndim, dims);
            int64_t count = 1;
            for (int i = 0; i < ndim; ++i) count *= dims[i];
            if (count <= 0 || count > ((int64_t)1 << 31))
                return grx_fail(GRX_EINVAL, "conformer: the model file doesn't fit its own settings (%s)", n.c_str());
            std::vector<float> v((size_t)count);
            if ((s = grx_gguf_float32(f, n.c_str(), v.data(), v.size())) != GRX_OK) return s;
            if ((s = grx_rnnt_set_tensor(m, n.c_str(), v.data(), v.size() * 4)) != GRX_OK) {
                if (s == GRX_ESIZE)
                    return grx_fail(GRX_EINVAL, "conformer: the model file doesn't fit its own settings (%s)",
                                    n.c_str());
                return s;
            }
        }
    }
    if (hp_out) {
        *hp_out = hp;
        if (hp_out->blank < 0) hp_out->blank = (int)V - 1;
    }
    *out = m;
    guard.m = nullptr;
    return GRX_OK;
}
