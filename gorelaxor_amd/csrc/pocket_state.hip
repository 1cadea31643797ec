// pocket_state.hip - the flow LM's transformer state on the device: voices,
// and the copy speaking makes of one.
//
// pockettts keeps a transformer's streaming state as a tstate (pockettts/
// nn.go:113-126: each layer's cache of rotated keys and values, a row per
// position, and the next position).  A Voice is such a state after a voice
// prompt (voice.go:13-24), read from a GGUF file by LoadVoice (voice.go:
// 26-64); speakChunk clones it with room for the chunk (tstate.clone,
// nn.go:128-140; speak.go:117) and runs the text and the frames on the
// clone, so the voice itself never changes.  Here a state lives in device
// memory ([n_layer][positions][d] keys, the same for values); seeding the
// LM copies its rows into the LM's caches (room up to max_pos) and sets the
// position, device to device.  Host code only.
#include <math.h>
#include <stdio.h>

#include <string>
#include <vector>

#include "grx_internal.h"
#include "pocket_internal.h"

struct grx_pocket_state {
    int device = 0;  // a state may outlive the LM and the context it came from
    int n_layer = 0, d = 0, positions = 0;
    float *k = nullptr, *v = nullptr;  // [n_layer][positions][d]
};

namespace {

grx_status state_alloc(grx_ctx *ctx, int n_layer, int d, int positions, grx_pocket_state **out) {
    grx_pocket_state *s = new grx_pocket_state();
    s->device = ctx->device;
    s->n_layer = n_layer;
    s->d = d;
    s->positions = positions;
    const size_t bytes = (size_t)n_layer * positions * d * 4;
    if (bytes > 0) {
        hipError_t e = hipSetDevice(ctx->device);
        if (e == hipSuccess) e = grx_dev_malloc((void **)&s->k, bytes);
        if (e == hipSuccess) e = grx_dev_malloc((void **)&s->v, bytes);
        if (e != hipSuccess) {
            grx_pocket_state_destroy(s);
            return grx_hip_fail(e, "pocket state");
        }
    }
    *out = s;
    return GRX_OK;
}

}  // namespace

extern "C" grx_status grx_pocket_state_create(grx_pocket *m, const float *k, const float *v, int positions,
                                              grx_pocket_state **out) {
    if (!m || !out || (positions > 0 && (!k || !v)))
        return grx_fail(GRX_EINVAL, "grx_pocket_state_create: NULL argument");
    *out = nullptr;
    if (positions < 0) return grx_fail(GRX_EINVAL, "grx_pocket_state_create: %d positions", positions);
    const grx_pocket_hparams &hp = m->hp;
    grx_pocket_state *s = nullptr;
    grx_status st = state_alloc(m->ctx, hp.n_layer, hp.d, positions, &s);
    if (st != GRX_OK) return st;
    const size_t bytes = (size_t)hp.n_layer * positions * hp.d * 4;
    if (bytes > 0) {
        hipError_t e = hipMemcpy(s->k, k, bytes, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(s->v, v, bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            grx_pocket_state_destroy(s);
            return grx_hip_fail(e, "grx_pocket_state_create");
        }
    }
    *out = s;
    return GRX_OK;
}

extern "C" grx_status grx_pocket_state_save(grx_pocket *m, grx_pocket_state **out) {
    if (!m || !out) return grx_fail(GRX_EINVAL, "grx_pocket_state_save: NULL argument");
    *out = nullptr;
    grx_status st = pocket_finalize(m);
    if (st != GRX_OK) return st;
    const grx_pocket_hparams &hp = m->hp;
    const int n = m->pos_host;
    grx_pocket_state *s = nullptr;
    if ((st = state_alloc(m->ctx, hp.n_layer, hp.d, n, &s)) != GRX_OK) return st;
    hipStream_t stream = m->ctx->stream;
    const size_t rows = (size_t)n * hp.d * 4;
    hipError_t e = hipSuccess;
    for (int li = 0; li < hp.n_layer && e == hipSuccess && rows > 0; ++li) {
        e = hipMemcpyAsync(s->k + (size_t)li * n * hp.d, m->L[li].k, rows, hipMemcpyDeviceToDevice, stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(s->v + (size_t)li * n * hp.d, m->L[li].v, rows, hipMemcpyDeviceToDevice, stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) {
        grx_pocket_state_destroy(s);
        return grx_hip_fail(e, "grx_pocket_state_save");
    }
    *out = s;
    return GRX_OK;
}

extern "C" grx_status grx_pocket_set_state(grx_pocket *m, const grx_pocket_state *s) {
    if (!m || !s) return grx_fail(GRX_EINVAL, "grx_pocket_set_state: NULL argument");
    const grx_pocket_hparams &hp = m->hp;
    if (s->n_layer != hp.n_layer || s->d != hp.d)
        return grx_fail(GRX_EINVAL, "grx_pocket_set_state: a state of %d layers of %d values, the LM has %d of %d",
                        s->n_layer, s->d, hp.n_layer, hp.d);
    if (s->device != m->ctx->device)
        return grx_fail(GRX_EINVAL, "grx_pocket_set_state: the state lives on device %d, the LM on %d", s->device,
                        m->ctx->device);
    if (s->positions > hp.max_pos)
        return grx_fail(GRX_ESTATE, "grx_pocket_set_state: %d positions exceed the LM's %d", s->positions, hp.max_pos);
    grx_status st = pocket_finalize(m);
    if (st != GRX_OK) return st;
    hipStream_t stream = m->ctx->stream;
    GRX_HIP(hipSetDevice(m->ctx->device));
    const int n = s->positions;
    const size_t rows = (size_t)n * hp.d * 4;
    for (int li = 0; li < hp.n_layer && rows > 0; ++li) {
        GRX_HIP(hipMemcpyAsync(m->L[li].k, s->k + (size_t)li * n * hp.d, rows, hipMemcpyDeviceToDevice, stream));
        GRX_HIP(hipMemcpyAsync(m->L[li].v, s->v + (size_t)li * n * hp.d, rows, hipMemcpyDeviceToDevice, stream));
    }
    m->pos_host = n;
    GRX_HIP(hipMemcpyAsync(m->pos, &m->pos_host, 4, hipMemcpyHostToDevice, stream));
    GRX_HIP(hipStreamSynchronize(stream));
    return GRX_OK;
}

extern "C" int grx_pocket_state_positions(const grx_pocket_state *s) { return s ? s->positions : 0; }

extern "C" grx_status grx_pocket_state_read(const grx_pocket_state *s, float *k, float *v) {
    if (!s) return grx_fail(GRX_EINVAL, "grx_pocket_state_read: NULL state");
    const size_t bytes = (size_t)s->n_layer * s->positions * s->d * 4;
    if (bytes == 0) return GRX_OK;
    GRX_HIP(hipSetDevice(s->device));
    if (k) GRX_HIP(hipMemcpy(k, s->k, bytes, hipMemcpyDeviceToHost));
    if (v) GRX_HIP(hipMemcpy(v, s->v, bytes, hipMemcpyDeviceToHost));
    return GRX_OK;
}

extern "C" grx_status grx_pocket_state_destroy(grx_pocket_state *s) {
    if (!s) return GRX_OK;
    (void)hipSetDevice(s->device);
    if (s->k) (void)hipFree(s->k);
    if (s->v) (void)hipFree(s->v);
    delete s;
    return GRX_OK;
}

// Model.LoadVoice (pockettts/voice.go:26-64): the file must be a voice
// ("pockettts-voice") made for the LM's model file (its
// pockettts.voice.model.sha256 equal to the model's general.source.sha256),
// hold the LM's layer count and 1..4096 positions, and for each layer in
// order its keys then its values as [positions][d] tensors voice.{i}.k and
// voice.{i}.v (float32, float16 or bfloat16, widened as File.Float32 widens
// them), every value a number.  The first problem is reported, with the
// reference's text.
extern "C" grx_status grx_pocket_load_voice_gguf(grx_pocket *m, const char *path, grx_pocket_state **out) {
    if (!m || !path || !out) return grx_fail(GRX_EINVAL, "grx_pocket_load_voice_gguf: NULL argument");
    *out = nullptr;
    grx_gguf *f = nullptr;
    grx_status st = grx_gguf_open(path, &f);
    if (st != GRX_OK) return st;
    struct Closer {
        grx_gguf *f;
        ~Closer() { grx_gguf_close(f); }
    } closer{f};
    if (std::string(grx_gguf_string(f, "general.architecture", "")) != "pockettts-voice")
        return grx_fail(GRX_EINVAL, "pockettts: %s isn't a Pocket TTS voice", path);
    if (std::string(grx_gguf_string(f, "pockettts.voice.model.sha256", "")) != m->sha)
        return grx_fail(GRX_EINVAL, "pockettts: %s was made for a different model file", path);
    const int64_t nl = grx_gguf_int(f, "pockettts.voice.layers", 0), n = grx_gguf_int(f, "pockettts.voice.positions", 0);
    const int d = m->hp.d;
    if (nl != m->hp.n_layer || n < 1 || n > 4096)
        return grx_fail(GRX_EINVAL, "pockettts: %s holds %lld layers of %lld positions", path, (long long)nl,
                        (long long)n);
    std::vector<float> k((size_t)nl * n * d), v((size_t)nl * n * d);
    for (int i = 0; i < nl; ++i) {
        for (int j = 0; j < 2; ++j) {
            char name[64];
            snprintf(name, sizeof name, "voice.%d.%c", i, "kv"[j]);
            int type = -1, nd = 0;
            int64_t dims[4] = {0, 0, 0, 0};
            if (grx_gguf_tensor_info(f, name, &type, &nd, dims) != GRX_OK || nd != 2 || dims[0] != d || dims[1] != n)
                return grx_fail(GRX_EINVAL, "pockettts: %s has no %lld\xc3\x97%d %s", path, (long long)n, d, name);
            float *dst = (j == 0 ? k.data() : v.data()) + (size_t)i * n * d;
            if ((st = grx_gguf_float32(f, name, dst, (size_t)n * d)) != GRX_OK) return st;
            for (size_t e = 0; e < (size_t)n * d; ++e)
                if (!isfinite(dst[e])) return grx_fail(GRX_EINVAL, "pockettts: %s has values that aren't numbers", path);
        }
    }
    return grx_pocket_state_create(m, k.data(), v.data(), (int)n, out);
}
