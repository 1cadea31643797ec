// pocket_flow.hip - the pocket-TTS flow head on the device.
//
// flowHead.sample and flowHead.net (pockettts/lm.go:107-160 of
// github.com/xattribution/gorelaxor), SimpleMLPAdaLN: from the transformer's
// output c and the frame's noise x0, decode_steps steps of
//   y = cond.c + b;  sy = SiLU(y + tc[s]);  h = input.x + b
//   per residual block: shift|scale|gate = ada.sy + b; n = LN(h)*(1+scale)
//       + shift; m = SiLU(fc1.n + b1); h += gate*(fc2.m + b2)
//   shift|scale = final_ada.sy + b; n = LN(h)*(1+scale) + shift;
//   v = out.n + b;  x += v / steps
// Every product is kern.Linear of one row on a weight that keeps its rows:
// the float route (float_route.hip), Q8_0 or float32 as the file stores the
// matrix.  LayerNorm is pockettts/nn.go:27-49 with eps 1e-6.  The time
// conditions (flowHead.timeConds, lm.go:59-104) are made once, when the head
// is set up: their products on the device, the standard deviation that
// normalizes them on the host in float64 in the reference's order.
// grx_pocket_speak runs a frame of the transformer and the head after it as
// one captured graph, feeding each sampled latent to the next frame.
#include <math.h>

#include <algorithm>

#include "grx_float.h"
#include "grx_ln.h"
#include "pocket_internal.h"

namespace {

constexpr int kFT = 256;

// c and x0 of the frame the transformer step just finished (f = *frame - 1)
__global__ void flow_prep_kernel(const int *__restrict__ frame, const float *__restrict__ out_hist, int d,
                                 const float *__restrict__ noise, int ldim, float *__restrict__ c,
                                 float *__restrict__ cur) {
    const int f = *frame - 1;
    for (int i = threadIdx.x; i < d; i += blockDim.x) c[i] = out_hist[(size_t)f * d + i];
    for (int i = threadIdx.x; i < ldim; i += blockDim.x) cur[i] = noise[(size_t)f * ldim + i];
}

// sy = kern.SiLU(y + tc) over dim entries (siluAVX below dim &^ 7, siluGo past)
__global__ void flow_sy_kernel(const float *__restrict__ y, const float *__restrict__ tc, int dim,
                               float *__restrict__ sy) {
    for (int j = threadIdx.x; j < dim; j += blockDim.x) {
        const float o = __fadd_rn(y[j], tc[j]);
        const float a = __fdiv_rn(o, __fadd_rn(grx_exp8(__fsub_rn(0.f, o)), 1.f));
        const float b = __fdiv_rn(o, __fadd_rn(1.f, grx_expf_go(-o)));
        sy[j] = j < (dim & ~7) ? a : b;
    }
}

// n = layerNorm(h) (float64 statistics; gain and bias when given), then
// n*(1+scale) + shift, one workgroup
__global__ void flow_lnmod_kernel(const float *__restrict__ h, int dim, const float *__restrict__ w,
                                  const float *__restrict__ b, const float *__restrict__ shift,
                                  const float *__restrict__ scale, double eps, float *__restrict__ n) {
    __shared__ double red[48];  // ln_block_reduce
    __shared__ float hl[8192];  // the row (dim <= 8192, checked at set-up)
    const int t = threadIdx.x;
    for (int j = t; j < dim; j += kFT) hl[j] = h[j];
    __syncthreads();
    double mean, inv;
    ln64_stats(hl, dim, eps, red, mean, inv);
    for (int j = t; j < dim; j += kFT) {
        float o = (float)__dmul_rn(__dsub_rn((double)hl[j], mean), inv);
        if (w) o = __fadd_rn(__fmul_rn(o, w[j]), b[j]);
        n[j] = __fadd_rn(__fmul_rn(o, __fadd_rn(1.f, scale[j])), shift[j]);
    }
}

// x += v / steps; on the last step the latent also goes to lat[*frame]
__global__ void flow_update_kernel(float *__restrict__ cur, const float *__restrict__ v, int ldim, float steps,
                                   float *__restrict__ lat, const int *__restrict__ frame) {
    for (int j = threadIdx.x; j < ldim; j += blockDim.x) {
        const float x = __fadd_rn(cur[j], __fdiv_rn(v[j], steps));
        cur[j] = x;
        if (lat) lat[(size_t)*frame * ldim + j] = x;
    }
}

grx_status linear(hipStream_t st, const FlowMat &w, const float *x, const float *bias, float *y,
                  GrxFloatEpi e = GrxFloatEpi()) {
    if (w.q8) return grx_float_gemv_q8(st, w.q8, x, bias, y, e);
    return grx_float_gemv_f32(st, w.f32, w.rows, w.cols, x, bias, y, e);
}

struct Spec {
    std::string name;
    int rows, cols;  // cols 0: a vector of rows values
};

std::vector<Spec> flow_specs(const grx_pocket_hparams &hp, const FlowHead &f) {
    const int D = f.dim;
    std::vector<Spec> s = {{"flow.cond.weight", D, hp.d},    {"flow.cond.bias", D, 0},
                           {"flow.input.weight", D, hp.ldim}, {"flow.input.bias", D, 0}};
    for (int i = 0; i < 2; ++i) {
        const std::string p = "flow.time." + std::to_string(i) + ".";
        for (Spec x : std::vector<Spec>{{"freqs", 128, 0}, {"fc1.weight", D, 256}, {"fc1.bias", D, 0},
                                        {"fc2.weight", D, D}, {"fc2.bias", D, 0}, {"norm.alpha", D, 0}}) {
            x.name = p + x.name;
            s.push_back(x);
        }
    }
    for (int i = 0; i < f.depth; ++i) {
        const std::string p = "flow.res." + std::to_string(i) + ".";
        for (Spec x : std::vector<Spec>{{"norm.weight", D, 0}, {"norm.bias", D, 0}, {"fc1.weight", D, D},
                                        {"fc1.bias", D, 0}, {"fc2.weight", D, D}, {"fc2.bias", D, 0},
                                        {"ada.weight", 3 * D, D}, {"ada.bias", 3 * D, 0}}) {
            x.name = p + x.name;
            s.push_back(x);
        }
    }
    s.push_back({"flow.final.ada.weight", 2 * D, D});
    s.push_back({"flow.final.ada.bias", 2 * D, 0});
    s.push_back({"flow.final.out.weight", hp.ldim, D});
    s.push_back({"flow.final.out.bias", hp.ldim, 0});
    return s;
}

grx_status upload_vec(grx_pocket *m, const std::string &name, float **out) {
    const auto &h = m->host.at(name);
    grx_status s = pocket_alloc(m, h.size(), reinterpret_cast<void **>(out));
    if (s != GRX_OK) return s;
    GRX_HIP(hipMemcpy(*out, h.data(), h.size(), hipMemcpyHostToDevice));
    return GRX_OK;
}

grx_status upload_mat(grx_pocket *m, const std::string &name, int rows, int cols, FlowMat *w) {
    const auto &h = m->host.at(name);
    w->rows = rows;
    w->cols = cols;
    if (h.size() == (size_t)rows * cols * 4) {
        grx_status s = pocket_alloc(m, h.size(), reinterpret_cast<void **>(&w->f32));
        if (s != GRX_OK) return s;
        GRX_HIP(hipMemcpy(w->f32, h.data(), h.size(), hipMemcpyHostToDevice));
        return GRX_OK;
    }
    return grx_weight_q8_create(m->ctx, rows, cols, h.data(), h.size(), &w->q8);
}

template <typename T>
grx_status dev(grx_pocket *m, size_t n, T **out) {
    return pocket_alloc(m, n * sizeof(T), reinterpret_cast<void **>(out));
}

const float *host_f32(const grx_pocket *m, const std::string &name) {
    return reinterpret_cast<const float *>(m->host.at(name).data());
}

// timeEmbed.embed (lm.go:59-87) of time t with embedder e, into out[dim]
grx_status time_embed(grx_pocket *m, int e, float t, FlowMat &fc1, FlowMat &fc2, const float *b1, const float *b2,
                      float *dbuf, float *out) {
    FlowHead &f = m->flow;
    const std::string p = "flow.time." + std::to_string(e) + ".";
    const float *freqs = host_f32(m, p + "freqs"), *alpha = host_f32(m, p + "norm.alpha");
    float in[256];
    for (int i = 0; i < 128; ++i) {
        const double a = (double)(t * freqs[i]);
        in[i] = (float)cos(a);
        in[128 + i] = (float)sin(a);
    }
    hipStream_t st = m->ctx->stream;
    float *din = dbuf, *dh = dbuf + 256, *dy = dbuf + 256 + f.dim;
    GRX_HIP(hipMemcpyAsync(din, in, sizeof in, hipMemcpyHostToDevice, st));
    GrxFloatEpi silu;
    silu.kind = GRX_FEPI_SILU;
    grx_status s = linear(st, fc1, din, b1, dh, silu);
    if (s == GRX_OK) s = linear(st, fc2, dh, b2, dy);
    if (s != GRX_OK) return s;
    GRX_HIP(hipMemcpyAsync(out, dy, (size_t)f.dim * 4, hipMemcpyDeviceToHost, st));
    GRX_HIP(hipStreamSynchronize(st));
    // the normalization by the standard deviation (n - 1), float64 in order
    double sum = 0;
    for (int i = 0; i < f.dim; ++i) sum += (double)out[i];
    const double mean = sum / (double)f.dim;
    double q = 0;
    for (int i = 0; i < f.dim; ++i) q += ((double)out[i] - mean) * ((double)out[i] - mean);
    const float inv = (float)(1 / sqrt(q / (double)(f.dim - 1) + 1e-5));
    for (int i = 0; i < f.dim; ++i) out[i] = out[i] * (alpha[i] * inv);
    return GRX_OK;
}

}  // namespace

bool pocket_flow_tensor(const grx_pocket *m, const std::string &name, size_t *qa, size_t *fb) {
    if (!m->flow.on) return false;
    for (const Spec &x : flow_specs(m->hp, m->flow)) {
        if (x.name != name) continue;
        if (x.cols == 0) {
            *qa = *fb = (size_t)x.rows * 4;
        } else {
            *fb = (size_t)x.rows * x.cols * 4;
            *qa = x.cols % 32 == 0 ? (size_t)x.rows * (x.cols / 32) * 34 : *fb;
        }
        return true;
    }
    return false;
}

// The flow head's weights, and the device allocations from index `mark` of
// the model's list on (those its finalize made), released; its settings
// stay, so a failed finalize can be tried again.
void pocket_flow_release(grx_pocket *m, size_t mark) {
    FlowHead &f = m->flow;
    for (FlowMat *w : {&f.cond, &f.input, &f.final_ada, &f.out}) grx_weight_destroy(w->q8);
    for (FlowRes &r : f.res)
        for (FlowMat *w : {&r.ada, &r.fc1, &r.fc2}) grx_weight_destroy(w->q8);
    for (size_t i = mark; i < m->allocs.size(); ++i) (void)hipFree(m->allocs[i]);
    if (mark < m->allocs.size()) m->allocs.resize(mark);
    FlowHead keep;
    keep.on = f.on;
    keep.dim = f.dim;
    keep.depth = f.depth;
    keep.steps = f.steps;
    f = keep;
}

namespace {

grx_status flow_finalize_tensors(grx_pocket *m);

}  // namespace

grx_status pocket_flow_finalize(grx_pocket *m) {
    if (m->flow.ready) return GRX_OK;
    const size_t mark = m->allocs.size();
    const grx_status s = flow_finalize_tensors(m);
    if (s != GRX_OK) pocket_flow_release(m, mark);
    return s;
}

namespace {

grx_status flow_finalize_tensors(grx_pocket *m) {
    FlowHead &f = m->flow;
    if (!f.on) return grx_fail(GRX_ESTATE, "the flow head is not declared (grx_pocket_flow_init)");
    for (const Spec &x : flow_specs(m->hp, f))
        if (!m->host.count(x.name)) return grx_fail(GRX_ESTATE, "the model file has no tensor %s", x.name.c_str());
    GRX_HIP(hipSetDevice(m->ctx->device));
    const int D = f.dim, d = m->hp.d, ld = m->hp.ldim;
    grx_status s;
    if ((s = upload_mat(m, "flow.cond.weight", D, d, &f.cond)) != GRX_OK) return s;
    if ((s = upload_mat(m, "flow.input.weight", D, ld, &f.input)) != GRX_OK) return s;
    if ((s = upload_mat(m, "flow.final.ada.weight", 2 * D, D, &f.final_ada)) != GRX_OK) return s;
    if ((s = upload_mat(m, "flow.final.out.weight", ld, D, &f.out)) != GRX_OK) return s;
    for (auto v : {std::make_pair("flow.cond.bias", &f.cond_b), std::make_pair("flow.input.bias", &f.input_b),
                   std::make_pair("flow.final.ada.bias", &f.final_ada_b),
                   std::make_pair("flow.final.out.bias", &f.out_b)})
        if ((s = upload_vec(m, v.first, v.second)) != GRX_OK) return s;
    f.res.assign(f.depth, FlowRes());
    for (int i = 0; i < f.depth; ++i) {
        FlowRes &r = f.res[i];
        const std::string p = "flow.res." + std::to_string(i) + ".";
        if ((s = upload_mat(m, p + "ada.weight", 3 * D, D, &r.ada)) != GRX_OK) return s;
        if ((s = upload_mat(m, p + "fc1.weight", D, D, &r.fc1)) != GRX_OK) return s;
        if ((s = upload_mat(m, p + "fc2.weight", D, D, &r.fc2)) != GRX_OK) return s;
        for (auto v : {std::make_pair("norm.weight", &r.norm_w), std::make_pair("norm.bias", &r.norm_b),
                       std::make_pair("ada.bias", &r.ada_b), std::make_pair("fc1.bias", &r.b1),
                       std::make_pair("fc2.bias", &r.b2)})
            if ((s = upload_vec(m, p + v.first, v.second)) != GRX_OK) return s;
    }
    const size_t big = std::max(d, D);
    if ((s = dev(m, (size_t)f.steps * D, &f.tc)) != GRX_OK) return s;
    if ((s = dev(m, (size_t)(m->hp.max_pos + 1) * ld, &f.noise)) != GRX_OK) return s;
    for (float **b : {&f.y, &f.sy, &f.h, &f.n, &f.mm})
        if ((s = dev(m, (size_t)D, b)) != GRX_OK) return s;
    if ((s = dev(m, big + 512 + 2 * (size_t)D, &f.yi)) != GRX_OK) return s;  // c, and time-embedding scratch
    if ((s = dev(m, 3 * (size_t)D, &f.mod)) != GRX_OK) return s;
    if ((s = dev(m, (size_t)ld, &f.cur)) != GRX_OK) return s;
    if ((s = dev(m, (size_t)ld, &f.v)) != GRX_OK) return s;
    // timeConds (lm.go:89-104): the mean of the start and end times' embeddings,
    // from embedders used only here (their weights released on every exit)
    struct TimeMats {
        FlowMat t1[2], t2[2];
        ~TimeMats() {
            for (int e = 0; e < 2; ++e) {
                grx_weight_destroy(t1[e].q8);
                grx_weight_destroy(t2[e].q8);
            }
        }
    } tm;
    FlowMat(&t1)[2] = tm.t1;
    FlowMat(&t2)[2] = tm.t2;
    float *tb1[2], *tb2[2];
    for (int e = 0; e < 2; ++e) {
        const std::string p = "flow.time." + std::to_string(e) + ".";
        if ((s = upload_mat(m, p + "fc1.weight", D, 256, &t1[e])) != GRX_OK) return s;
        if ((s = upload_mat(m, p + "fc2.weight", D, D, &t2[e])) != GRX_OK) return s;
        if ((s = upload_vec(m, p + "fc1.bias", &tb1[e])) != GRX_OK) return s;
        if ((s = upload_vec(m, p + "fc2.bias", &tb2[e])) != GRX_OK) return s;
    }
    std::vector<float> tc((size_t)f.steps * D), a(D), b(D);
    for (int i = 0; i < f.steps && s == GRX_OK; ++i) {
        s = time_embed(m, 0, (float)((double)i / (double)f.steps), t1[0], t2[0], tb1[0], tb2[0], f.yi, a.data());
        if (s == GRX_OK)
            s = time_embed(m, 1, (float)((double)(i + 1) / (double)f.steps), t1[1], t2[1], tb1[1], tb2[1], f.yi,
                           b.data());
        for (int j = 0; j < D && s == GRX_OK; ++j) tc[(size_t)i * D + j] = (a[j] + b[j]) / 2;
    }
    if (s != GRX_OK) return s;
    GRX_HIP(hipMemcpy(f.tc, tc.data(), tc.size() * 4, hipMemcpyHostToDevice));
    for (const Spec &x : flow_specs(m->hp, f)) m->host.erase(x.name);
    f.ready = true;
    return GRX_OK;
}

}  // namespace

// flowHead.sample for the frame the transformer just finished; the latent
// goes to m->lat[*frame]
grx_status pocket_flow_enqueue(grx_pocket *m, hipStream_t st) {
    FlowHead &f = m->flow;
    const int D = f.dim, ld = m->hp.ldim;
    float *c = f.yi;
    flow_prep_kernel<<<1, kFT, 0, st>>>(m->frame, m->out_hist, m->hp.d, f.noise, ld, c, f.cur);
    GRX_LAUNCHED("flow_prep_kernel");
    grx_status s = linear(st, f.cond, c, f.cond_b, f.y);
    if (s != GRX_OK) return s;
    GrxFloatEpi silu, gate;
    silu.kind = GRX_FEPI_SILU;
    gate.kind = GRX_FEPI_GATE;
    for (int step = 0; step < f.steps; ++step) {
        flow_sy_kernel<<<1, kFT, 0, st>>>(f.y, f.tc + (size_t)step * D, D, f.sy);
        GRX_LAUNCHED("flow_sy_kernel");
        if ((s = linear(st, f.input, f.cur, f.input_b, f.h)) != GRX_OK) return s;
        for (FlowRes &r : f.res) {
            if ((s = linear(st, r.ada, f.sy, r.ada_b, f.mod)) != GRX_OK) return s;
            flow_lnmod_kernel<<<1, kFT, 0, st>>>(f.h, D, r.norm_w, r.norm_b, f.mod, f.mod + D, 1e-6, f.n);
            GRX_LAUNCHED("flow_lnmod_kernel");
            if ((s = linear(st, r.fc1, f.n, r.b1, f.mm, silu)) != GRX_OK) return s;
            gate.gate = f.mod + 2 * D;
            if ((s = linear(st, r.fc2, f.mm, r.b2, f.h, gate)) != GRX_OK) return s;
        }
        if ((s = linear(st, f.final_ada, f.sy, f.final_ada_b, f.mod)) != GRX_OK) return s;
        flow_lnmod_kernel<<<1, kFT, 0, st>>>(f.h, D, nullptr, nullptr, f.mod, f.mod + D, 1e-6, f.n);
        GRX_LAUNCHED("flow_lnmod_kernel");
        if ((s = linear(st, f.out, f.n, f.out_b, f.v)) != GRX_OK) return s;
        flow_update_kernel<<<1, 64, 0, st>>>(f.cur, f.v, ld, (float)f.steps, step + 1 == f.steps ? m->lat : nullptr,
                                             m->frame);
        GRX_LAUNCHED("flow_update_kernel");
    }
    return GRX_OK;
}

extern "C" grx_status grx_pocket_flow_init(grx_pocket *m, int dim, int depth, int decode_steps) {
    if (!m) return grx_fail(GRX_EINVAL, "grx_pocket_flow_init: NULL model");
    if (m->flow.on) return grx_fail(GRX_ESTATE, "grx_pocket_flow_init: the flow head is declared already");
    if (dim <= 1 || dim > 8192 || depth < 1 || depth > 64 || decode_steps < 1 || decode_steps > 64)
        return grx_fail(GRX_EINVAL, "grx_pocket_flow_init: dim %d, depth %d, steps %d", dim, depth, decode_steps);
    m->flow.on = true;
    m->flow.dim = dim;
    m->flow.depth = depth;
    m->flow.steps = decode_steps;
    return GRX_OK;
}

extern "C" grx_status grx_pocket_speak(grx_pocket *m, const float *first_latent, const float *noise, int n,
                                       float *latents, float *eos) {
    if (!m || (!noise && n > 0)) return grx_fail(GRX_EINVAL, "grx_pocket_speak: NULL argument");
    grx_status s = pocket_finalize(m);
    if (s == GRX_OK) s = pocket_flow_finalize(m);
    if (s != GRX_OK) return s;
    if (n < 0) return grx_fail(GRX_EINVAL, "grx_pocket_speak: n = %d", n);
    const grx_pocket_hparams &hp = m->hp;
    if (m->pos_host + n > hp.max_pos)
        return grx_fail(GRX_ESTATE, "grx_pocket_speak: %d frames after %d positions exceed %d", n, m->pos_host,
                        hp.max_pos);
    if (n == 0) return GRX_OK;
    hipStream_t st = m->ctx->stream;
    if (!m->lat) {  // latents: frame k reads row k, its flow head writes row k + 1
        if ((s = pocket_alloc(m, (size_t)(hp.max_pos + 1) * hp.ldim * 4, reinterpret_cast<void **>(&m->lat))) !=
            GRX_OK)
            return s;
        m->lat_cap = hp.max_pos;
    }
    GRX_HIP(hipMemcpyAsync(m->lat, first_latent ? first_latent : m->bos, (size_t)hp.ldim * 4,
                           first_latent ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice, st));
    GRX_HIP(hipMemcpyAsync(m->flow.noise, noise, (size_t)n * hp.ldim * 4, hipMemcpyHostToDevice, st));
    GRX_HIP(hipMemsetAsync(m->frame, 0, 4, st));
    const bool eager = grx_tune(GRX_TUNE_NO_GRAPH) == 1;
    auto one = [&]() {
        grx_status cs = pocket_enqueue_frame(m, st, m->lat, m->frame);
        return cs == GRX_OK ? pocket_flow_enqueue(m, st) : cs;
    };
    for (int k = 0; k < n; ++k) {
        if (eager || (!m->speak_exec && k == 0)) {
            if ((s = one()) != GRX_OK) return s;
            if (!eager && !m->speak_exec) {
                GRX_HIP(hipStreamSynchronize(st));
                hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
                if (e == hipSuccess) {
                    grx_status cs = one();
                    hipGraph_t g = nullptr;
                    e = hipStreamEndCapture(st, &g);
                    if (cs == GRX_OK && e == hipSuccess) e = hipGraphInstantiate(&m->speak_exec, g, nullptr, nullptr, 0);
                    if (g) {
                        if (e == hipSuccess && cs == GRX_OK) m->speak_graph = g;
                        else (void)hipGraphDestroy(g);
                    }
                    if (e != hipSuccess || cs != GRX_OK) {
                        (void)hipGetLastError();
                        m->speak_exec = nullptr;
                    }
                }
            }
            continue;
        }
        if (m->speak_exec)
            GRX_HIP(hipGraphLaunch(m->speak_exec, st));
        else if ((s = one()) != GRX_OK)
            return s;
    }
    m->pos_host += n;
    if (latents)
        GRX_HIP(hipMemcpyAsync(latents, m->lat + hp.ldim, (size_t)n * hp.ldim * 4, hipMemcpyDeviceToHost, st));
    if (eos) GRX_HIP(hipMemcpyAsync(eos, m->eos_hist, (size_t)n * 4, hipMemcpyDeviceToHost, st));
    GRX_HIP(hipStreamSynchronize(st));
    return GRX_OK;
}
