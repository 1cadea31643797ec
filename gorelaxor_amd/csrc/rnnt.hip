// rnnt.hip - greedy RNN-T / TDT decoding on the device.
//
// conformer/rnnt.go:46-173 of github.com/xattribution/gorelaxor: the
// prediction network (an LSTM stack over the last emitted token's
// embedding), the joint network (ReLU / sigmoid / tanh of the encoder and
// prediction projections, then the output Linear) and the greedy loop that
// walks the encoder frames, emitting tokens (RNN-T: up to max_symbols per
// frame; TDT: each token or blank also picks how many frames to skip).
//
// Every Linear here has one row of activations except the encoder
// projection, so it takes kern's float route (q8_float_row) with the
// reference's lane chains; the encoder projection of T >= 2 frames takes the
// int8 route (kern.MatMul sends Q8_0 products of m >= 2 rows there), T = 1
// the float route.  The loop is data-dependent (a blank advances the frame,
// a token re-runs the prediction network), so it runs on the device: each
// iteration is L gate launches, one prediction-projection launch (those
// return at once unless the last iteration emitted a token), one joint
// launch and a one-workgroup launch that applies the greedy decision to the
// loop state in device memory.  A captured graph holds kIters iterations;
// the host replays it until the loop reports done, so the host reads the
// loop state once per kIters iterations.  The prediction projection is
// formed only when the prediction changes (the reference recomputes it every
// iteration from the same inputs, to the same values).
#include <string>
#include <vector>

#include "grx.h"
#include "grx_float.h"
#include "grx_internal.h"

namespace {

constexpr int kIters = 16;     // loop iterations per graph replay
constexpr int kMaxDur = 16;    // TDT durations held
constexpr int kMaxDuration = 1 << 20;  // the largest duration (frames) a TDT head may name
constexpr int kExpChunk = 1024;

// The loop state (rnnt.go:134-171) in device memory.
struct RnntCtl {
    int step, iter, newsym, dirty, done, cur, n_out, T, max_iters, frame_offset;
    int last[2];  // DecoderState.last of the two state slots
};

struct RnntHp {
    int H, L, J, V, R, act, tdt, nd, max_symbols, blank;
    int dur[kMaxDur];
};

// ---------------------------------------------------------------- scalar math

// exp of a double by fdlibm's e_exp.c (argument reduction by ln2 in two
// parts, the degree-5 Remez polynomial in r*r, the rational reconstruction),
// every operation rounded on its own, so the CPU oracle's restatement gives
// the same bits.  Within an ulp of the correctly rounded exp.
__device__ inline double fd_exp(double x) {
    const double ln2hi = 6.93147180369123816490e-01, ln2lo = 1.90821492927058770002e-10;
    const double invln2 = 1.44269504088896338700e+00;
    const double P1 = 1.66666666666666019037e-01, P2 = -2.77777777770155933842e-03;
    const double P3 = 6.61375632143793436117e-05, P4 = -1.65339022054652515390e-06;
    const double P5 = 4.13813679705723846039e-08;
    if (x != x) return x;
    if (x > 7.09782712893383973096e+02) return __builtin_inf();
    if (x < -7.45133219101941108420e+02) return 0.0;
    const unsigned hx = (unsigned)(__double_as_longlong(x) >> 32) & 0x7fffffffu;
    const bool neg = x < 0.0;
    double hi = 0.0, lo = 0.0;
    int k = 0;
    if (hx > 0x3fd62e42u) {  // |x| > 0.5 ln2
        if (hx < 0x3ff0a2b2u) {  // |x| < 1.5 ln2
            hi = neg ? __dadd_rn(x, ln2hi) : __dsub_rn(x, ln2hi);
            lo = neg ? -ln2lo : ln2lo;
            k = neg ? -1 : 1;
        } else {
            k = (int)__dadd_rn(__dmul_rn(invln2, x), neg ? -0.5 : 0.5);
            const double t = (double)k;
            hi = __dsub_rn(x, __dmul_rn(t, ln2hi));
            lo = __dmul_rn(t, ln2lo);
        }
        x = __dsub_rn(hi, lo);
    } else if (hx < 0x3e300000u) {  // |x| < 2^-28
        return __dadd_rn(1.0, x);
    }
    const double t = __dmul_rn(x, x);
    double p = __dadd_rn(P4, __dmul_rn(t, P5));
    p = __dadd_rn(P3, __dmul_rn(t, p));
    p = __dadd_rn(P2, __dmul_rn(t, p));
    p = __dadd_rn(P1, __dmul_rn(t, p));
    const double c = __dsub_rn(x, __dmul_rn(t, p));
    if (k == 0) return __dsub_rn(1.0, __dsub_rn(__ddiv_rn(__dmul_rn(x, c), __dsub_rn(c, 2.0)), x));
    const double y = __dsub_rn(1.0, __dsub_rn(__dsub_rn(lo, __ddiv_rn(__dmul_rn(x, c), __dsub_rn(2.0, c))), hi));
    return ldexp(y, k);
}

// tanh32 (rnnt.go:43): float32(math.Tanh(float64(x))), Go's tanh being
// Cephes' (|x| past half of log(2^127): +-1; |x| >= 0.625: 1 - 2/(e^2|x|+1)
// with the sign; else x + x*s*P(s)/Q(s), s = x*x), unfused.
__device__ inline float tanh32(float xf) {
    const double x = (double)xf, z = fabs(x);
    double r;
    if (z > 0.5 * 8.8029691931113054295988e+01) {
        r = x < 0.0 ? -1.0 : 1.0;
    } else if (z >= 0.625) {
        const double s = fd_exp(__dmul_rn(2.0, z));
        r = __dsub_rn(1.0, __ddiv_rn(2.0, __dadd_rn(s, 1.0)));
        if (x < 0.0) r = -r;
    } else {
        if (x == 0.0) return xf;
        const double s = __dmul_rn(x, x);
        double p = __dadd_rn(__dmul_rn(-9.64399179425052238628e-1, s), -9.92877231001918586564e1);
        p = __dadd_rn(__dmul_rn(p, s), -1.61468768441708447952e3);
        double q = __dadd_rn(s, 1.12811678491632931402e2);
        q = __dadd_rn(__dmul_rn(q, s), 2.23548839060100448583e3);
        q = __dadd_rn(__dmul_rn(q, s), 4.84406305325125486048e3);
        r = __dadd_rn(x, __ddiv_rn(__dmul_rn(__dmul_rn(x, s), p), q));
    }
    return (float)r;
}

// sigmoid (conformer/encoder.go:13): 1 / (1 + kern.Expf(-v)).
__device__ __forceinline__ float sigm(float v) { return __fdiv_rn(1.f, __fadd_rn(1.f, grx_expf_go(-v))); }

// The LSTM cell of one layer (rnnt.go:57-64) for all H units into xs, from
// gates = (Wx x + b) + Wh h in gx / gh and the previous cell c0; the new h
// and c also go to hn / cn when those are set.
__device__ inline void lstm_cell(const float *__restrict__ gx, const float *__restrict__ gh,
                                 const float *__restrict__ c0, int H, float *xs, float *hn, float *cn) {
    for (int j = threadIdx.x; j < H; j += blockDim.x) {
        const float i = sigm(__fadd_rn(gx[j], gh[j]));
        const float f = sigm(__fadd_rn(gx[H + j], gh[H + j]));
        const float g = tanh32(__fadd_rn(gx[2 * H + j], gh[2 * H + j]));
        const float o = sigm(__fadd_rn(gx[3 * H + j], gh[3 * H + j]));
        const float c = __fadd_rn(__fmul_rn(f, c0[j]), __fmul_rn(i, g));
        const float h = __fmul_rn(o, tanh32(c));
        xs[j] = h;
        if (hn) {
            hn[j] = h;
            cn[j] = c;
        }
    }
}

// State slots: S[slot] = h[L][H] then c[L][H].
__device__ __forceinline__ float *slot_h(float *S, int slot, int l, const RnntHp &hp) {
    return S + ((size_t)slot * 2 * hp.L + l) * hp.H;
}
__device__ __forceinline__ float *slot_c(float *S, int slot, int l, const RnntHp &hp) {
    return S + ((size_t)slot * 2 * hp.L + hp.L + l) * hp.H;
}

// ---------------------------------------------------------------- kernels

// Layer l's gate products (rnnt.go:53-55): workgroups [0, tiles) form
// Wx x + b into gx, the rest Wh h into gh.  x is the embedding of the last
// token (zeros at the start or after a blank id) for layer 0, else the
// previous layer's new h, formed here from its gates (and stored in the
// next state slot by workgroup 0).
__global__ __launch_bounds__(256) void rnnt_gates_kernel(RnntCtl *ctl, RnntHp hp, int l, const int8_t *wxq,
                                                         const uint16_t *wxd, const int8_t *whq, const uint16_t *whd,
                                                         const float *__restrict__ bias,
                                                         const float *__restrict__ embed, const float *gxp,
                                                         const float *ghp, float *gx, float *gh, float *S) {
    extern __shared__ __align__(16) float xs[];
    if (ctl->done || !ctl->dirty) return;
    const int cur = ctl->cur, H = hp.H, tiles = (4 * H + 63) / 64, nb = H / 32;
    const bool hjob = (int)blockIdx.x >= tiles;
    const int tile = hjob ? blockIdx.x - tiles : blockIdx.x;
    if (hjob) {
        const float *h = slot_h(S, cur, l, hp);
        for (int j = threadIdx.x; j < H; j += blockDim.x) xs[j] = h[j];
    } else if (l == 0) {
        const int last = ctl->last[cur];
        const bool emb = last >= 0 && last != hp.blank;
        for (int j = threadIdx.x; j < H; j += blockDim.x) xs[j] = emb ? embed[(size_t)last * H + j] : 0.f;
    } else {
        const bool w = blockIdx.x == 0;
        lstm_cell(gxp, ghp, slot_c(S, cur, l - 1, hp), H, xs, w ? slot_h(S, 1 - cur, l - 1, hp) : nullptr,
                  w ? slot_c(S, 1 - cur, l - 1, hp) : nullptr);
    }
    __syncthreads();
    int row;
    bool emit;
    const float o = q8_float_row(xs, hjob ? whq : wxq, hjob ? whd : wxd, nb, 4 * H, tile, row, emit);
    if (!emit) return;
    if (hjob)
        gh[row] = o;
    else
        gx[row] = __fadd_rn(o, bias[row]);
}

// The last layer's cell gives the prediction (stored in the next state slot
// by workgroup 0); its joint projection predProj = Wp pred + b (rnnt.go:91).
__global__ __launch_bounds__(256) void rnnt_pred_kernel(RnntCtl *ctl, RnntHp hp, const int8_t *wq, const uint16_t *wd,
                                                        const float *__restrict__ bias, const float *gxp,
                                                        const float *ghp, float *pp, float *S) {
    extern __shared__ __align__(16) float xs[];
    if (ctl->done || !ctl->dirty) return;
    const int cur = ctl->cur, l = hp.L - 1;
    const bool w = blockIdx.x == 0;
    lstm_cell(gxp, ghp, slot_c(S, cur, l, hp), hp.H, xs, w ? slot_h(S, 1 - cur, l, hp) : nullptr,
              w ? slot_c(S, 1 - cur, l, hp) : nullptr);
    __syncthreads();
    int row;
    bool emit;
    const float o = q8_float_row(xs, wq, wd, hp.H / 32, hp.J, blockIdx.x, row, emit);
    if (emit) pp[row] = __fadd_rn(o, bias[row]);
}

struct ArgBest {
    float v;
    int i;
};
__device__ __forceinline__ ArgBest better(ArgBest a, ArgBest b) {
    return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}

// The joint (rnnt.go:90-106) of frame `step`: hidden = act(encProj[step] +
// predProj) in LDS, logits = Wo hidden + b.
__global__ __launch_bounds__(256) void rnnt_joint_kernel(const RnntCtl *ctl, RnntHp hp, const int8_t *wq,
                                                         const uint16_t *wd, const float *__restrict__ bias,
                                                         const float *__restrict__ ep, const float *__restrict__ pp,
                                                         float *logits) {
    extern __shared__ __align__(16) float xs[];
    if (ctl->done) return;
    const int J = hp.J, step = ctl->step;
    const float *e = ep + (size_t)step * J;
    for (int i0 = threadIdx.x; i0 < J; i0 += 8 * (int)blockDim.x) {  // every read in flight first
        float a[8], c[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = i0 + u * (int)blockDim.x;
            a[u] = i < J ? e[i] : 0.f;
            c[u] = i < J ? pp[i] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = i0 + u * (int)blockDim.x;
            if (i >= J) break;
            float v = __fadd_rn(a[u], c[u]);
            if (hp.act == 1)
                v = sigm(v);
            else if (hp.act == 2)
                v = tanh32(v);
            else
                v = v != v ? v : (v > 0.f ? v : 0.f);  // Go's max(v, 0): NaN stays, -0 gives +0
            xs[i] = v;
        }
    }
    __syncthreads();
    int row;
    bool emit;
    const float o = q8_float_row(xs, wq, wd, J / 32, hp.R, blockIdx.x, row, emit);
    if (emit) logits[row] = __fadd_rn(o, bias[row]);
}

// The greedy step (rnnt.go:140-170) in one workgroup: the first maximal
// token, the TDT duration, the softmax probability of an emitted token
// (rnnt.go:78-85), the state swap and the frame advance.
__global__ __launch_bounds__(256) void rnnt_decide_kernel(RnntCtl *ctl, RnntHp hp, const float *__restrict__ logits,
                                                          grx_rnnt_token *tokens) {
    __shared__ double es[kExpChunk];
    __shared__ ArgBest wbest[4];
    if (ctl->done) return;
    const int tid = threadIdx.x, V = hp.V;
    ArgBest b = {-__builtin_inff(), 0x7fffffff};
    for (int i0 = tid; i0 < V; i0 += 8 * (int)blockDim.x) {  // eight reads in flight
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = i0 + u * (int)blockDim.x;
            v[u] = i < V ? logits[i] : -__builtin_inff();
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = i0 + u * (int)blockDim.x;
            if (i < V) b = better(b, ArgBest{v[u], i});
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) b = better(b, ArgBest{__shfl_xor(b.v, off), __shfl_xor(b.i, off)});
    if ((tid & 63) == 0) wbest[tid >> 6] = b;
    __syncthreads();
    b = wbest[0];
    for (int w = 1; w < (int)blockDim.x / 64; ++w) b = better(b, wbest[w]);
    const int tok = b.i == 0x7fffffff ? 0 : b.i;
    const bool blank = tok == hp.blank;
    // softmaxAt's p = float32(e^0 / s), s the float64 sum in token order.  Any
    // order of summing V non-negative terms lands within gamma = (V-1) 2^-53
    // (relative) of the exact sum, so the in-order s lies within 2 gamma of a
    // parallel sum t; if float32(1/s) is the same at both ends of that
    // interval (1/s and its roundings are monotone), it is p.  Otherwise (a
    // float32 rounding boundary inside an interval ~2^-41 wide) the sum is
    // formed in order.
    float p = 0.f;
    if (!blank) {
        const float mx = logits[tok];
        double part = 0.0;
        for (int i0 = tid; i0 < V; i0 += 8 * (int)blockDim.x) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = i0 + u * (int)blockDim.x;
                v[u] = i < V ? logits[i] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (i0 + u * (int)blockDim.x < V) part = __dadd_rn(part, fd_exp((double)__fsub_rn(v[u], mx)));
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) part = __dadd_rn(part, __shfl_xor(part, off));
        if ((tid & 63) == 0) es[tid >> 6] = part;
        __syncthreads();
        double t = es[0];
        for (int w = 1; w < (int)blockDim.x / 64; ++w) t = __dadd_rn(t, es[w]);
        const double delta = (double)(V + 4) * 0x1p-52;
        const float plo = (float)__ddiv_rn(1.0, __dmul_rn(t, 1.0 + delta));
        const float phi = (float)__ddiv_rn(1.0, __dmul_rn(t, 1.0 - delta));
        __syncthreads();
        if (plo == phi) {
            p = plo;
        } else {
            double sq = 0.0;
            for (int c0 = 0; c0 < V; c0 += kExpChunk) {
                const int cn = min(kExpChunk, V - c0);
                for (int i = tid; i < cn; i += blockDim.x) es[i] = fd_exp((double)__fsub_rn(logits[c0 + i], mx));
                __syncthreads();
                if (tid == 0)
                    for (int i = 0; i < cn; ++i) sq = __dadd_rn(sq, es[i]);
                __syncthreads();
            }
            p = (float)__ddiv_rn(fd_exp((double)__fsub_rn(logits[tok], mx)), sq);
        }
    }
    if (tid != 0) return;
    int duration = 1;
    if (hp.tdt) {
        int bd = 0;
        for (int i = 1; i < hp.nd; ++i)
            if (logits[V + i] > logits[V + bd]) bd = i;
        duration = hp.dur[bd];
    }
    int st = ctl->step, ns = ctl->newsym;
    if (!blank) {
        tokens[ctl->n_out] = grx_rnnt_token{tok, ctl->frame_offset + st, duration, p};
        ctl->n_out = ctl->n_out + 1;
        const int nx = 1 - ctl->cur;
        ctl->last[nx] = tok;
        ctl->cur = nx;
    }
    ctl->dirty = blank ? 0 : 1;
    if (!hp.tdt) {
        if (blank) {
            st += 1;
            ns = 0;
        } else if (++ns, hp.max_symbols > 0 && ns >= hp.max_symbols) {
            st += 1;
            ns = 0;
        }
    } else {
        // durations are at most kMaxDuration (checked at create) and st < T
        // here, so the sum cannot overflow; past T the loop is over, so st
        // is kept at T (no frame index past T is ever read)
        st = min(st + duration, ctl->T);
        ++ns;
        if (duration != 0) {
            ns = 0;
        } else if (hp.max_symbols > 0 && ns >= hp.max_symbols) {
            st += 1;
            ns = 0;
        }
    }
    const int it = ctl->iter + 1;
    ctl->step = st;
    ctl->newsym = ns;
    ctl->iter = it;
    ctl->done = (st < ctl->T && it < ctl->max_iters) ? 0 : 1;
}

__global__ void rnnt_ctl_init_kernel(RnntCtl *ctl, int T, int max_iters, int frame_offset, int last) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    RnntCtl c = {};
    c.dirty = 1;
    c.T = T;
    c.max_iters = max_iters;
    c.frame_offset = frame_offset;
    c.last[0] = last;
    c.last[1] = -1;
    *ctl = c;
}

struct Lstm {
    grx_weight *wx = nullptr, *wh = nullptr;
    float *b = nullptr;
};

}  // namespace

// A state keeps what it needs of its decoder (it may outlive it; not its
// context): the decoder's address only identifies it.
struct grx_rnnt_state {
    const grx_rnnt *m;
    grx_ctx *ctx;
    int L, H, V, blank, embed_rows;
    float *hc;  // h[L][H] then c[L][H], device
    int last;
};

struct grx_rnnt {
    grx_ctx *ctx = nullptr;
    grx_rnnt_hparams hp{};
    RnntHp k{};
    bool ready = false;
    std::vector<bool> have;
    float *embed = nullptr;
    int embed_rows = 0;
    std::vector<Lstm> lstm;
    grx_weight *jenc = nullptr, *jpred = nullptr, *jout = nullptr;
    float *jencb = nullptr, *jpredb = nullptr, *joutb = nullptr;
    // work
    RnntCtl *ctl = nullptr, *ctl_host = nullptr;  // ctl_host: pinned
    float *S = nullptr, *gx = nullptr, *gh = nullptr, *pp = nullptr, *logits = nullptr;
    int cap_T = 0;
    float *ep = nullptr, *enc = nullptr, *xs = nullptr;
    int8_t *xq = nullptr;
    grx_rnnt_token *tokens = nullptr;
    hipGraphExec_t exec = nullptr;
    hipGraph_t graph = nullptr;
};

namespace {

// The tensors fromGGUF reads for the decoder (conformer/model.go:306-315).
struct RExpect {
    std::string name;
    int rows, cols;  // cols > 0: a Q8_0 matrix [rows][cols]; 0: a float32 vector of rows values
};

std::vector<RExpect> rexpected(const grx_rnnt_hparams &hp, int embed_rows) {
    const int H = hp.pred_hidden, J = hp.joint_hidden;
    std::vector<RExpect> e;
    e.push_back({"pred.embed.weight", embed_rows * H, 0});
    for (int i = 0; i < hp.pred_layers; ++i) {
        const std::string p = "pred.lstm." + std::to_string(i) + ".";
        e.push_back({p + "Wx", 4 * H, H});
        e.push_back({p + "Wh", 4 * H, H});
        e.push_back({p + "bias", 4 * H, 0});
    }
    e.push_back({"joint.enc.weight", J, hp.d});
    e.push_back({"joint.enc.bias", J, 0});
    e.push_back({"joint.pred.weight", J, H});
    e.push_back({"joint.pred.bias", J, 0});
    e.push_back({"joint.out.weight", hp.pred_vocab + (hp.tdt ? hp.n_durations : 0), J});
    e.push_back({"joint.out.bias", hp.pred_vocab + (hp.tdt ? hp.n_durations : 0), 0});
    return e;
}

grx_status ralloc(grx_rnnt *m, size_t bytes, void **p) {
    GRX_HIP(grx_dev_malloc(p, bytes < 4 ? 4 : bytes));
    (void)m;
    return GRX_OK;
}

grx_status upload_vec(grx_rnnt *m, const void *data, size_t bytes, float **out) {
    grx_status s = ralloc(m, bytes, reinterpret_cast<void **>(out));
    if (s != GRX_OK) return s;
    const hipError_t e = hipMemcpy(*out, data, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(*out);
        *out = nullptr;
        return grx_hip_fail(e, "hipMemcpy");
    }
    return GRX_OK;
}

// Enqueue one loop iteration.
grx_status enqueue_iter(grx_rnnt *m, hipStream_t st) {
    const RnntHp &k = m->k;
    const int H = k.H, L = k.L, tiles4 = (4 * H + 63) / 64;
    for (int l = 0; l < L; ++l) {
        const Lstm &ly = m->lstm[l];
        const float *gxp = l ? m->gx + (size_t)(l - 1) * 4 * H : nullptr;
        const float *ghp = l ? m->gh + (size_t)(l - 1) * 4 * H : nullptr;
        rnnt_gates_kernel<<<2 * tiles4, 256, (size_t)H * 4, st>>>(
            m->ctl, k, l, ly.wx->qs, ly.wx->ds, ly.wh->qs, ly.wh->ds, ly.b, m->embed, gxp, ghp,
            m->gx + (size_t)l * 4 * H, m->gh + (size_t)l * 4 * H, m->S);
        GRX_LAUNCHED("rnnt_gates_kernel");
    }
    rnnt_pred_kernel<<<m->jpred->tiles, 256, (size_t)H * 4, st>>>(m->ctl, k, m->jpred->qs, m->jpred->ds, m->jpredb,
                                                                  m->gx + (size_t)(L - 1) * 4 * H,
                                                                  m->gh + (size_t)(L - 1) * 4 * H, m->pp, m->S);
    GRX_LAUNCHED("rnnt_pred_kernel");
    rnnt_joint_kernel<<<m->jout->tiles, 256, (size_t)k.J * 4, st>>>(m->ctl, k, m->jout->qs, m->jout->ds, m->joutb,
                                                                    m->ep, m->pp, m->logits);
    GRX_LAUNCHED("rnnt_joint_kernel");
    rnnt_decide_kernel<<<1, 256, 0, st>>>(m->ctl, k, m->logits, m->tokens);
    GRX_LAUNCHED("rnnt_decide_kernel");
    return GRX_OK;
}

void free_work(grx_rnnt *m) {
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    m->exec = nullptr;
    m->graph = nullptr;
    for (void *p : {(void *)m->ep, (void *)m->enc, (void *)m->xs, (void *)m->xq, (void *)m->tokens})
        if (p) (void)hipFree(p);
    m->ep = m->enc = m->xs = nullptr;
    m->xq = nullptr;
    m->tokens = nullptr;
    m->cap_T = 0;
}

// Buffers for T frames (grown, never shrunk); the graph captured on them
// is dropped when they move.
grx_status ensure_T(grx_rnnt *m, int T) {
    if (T <= m->cap_T) return GRX_OK;
    free_work(m);
    const int d = m->hp.d, J = m->k.J;
    const size_t iters = (size_t)16 * T + 1024;
    grx_status s;
    if ((s = ralloc(m, (size_t)T * J * 4, reinterpret_cast<void **>(&m->ep))) != GRX_OK) return s;
    if ((s = ralloc(m, (size_t)T * d * 4, reinterpret_cast<void **>(&m->enc))) != GRX_OK) return s;
    if ((s = ralloc(m, (size_t)T * (d / 32) * 4, reinterpret_cast<void **>(&m->xs))) != GRX_OK) return s;
    if ((s = ralloc(m, (size_t)T * d, reinterpret_cast<void **>(&m->xq))) != GRX_OK) return s;
    if ((s = ralloc(m, iters * sizeof(grx_rnnt_token), reinterpret_cast<void **>(&m->tokens))) != GRX_OK)
        return s;
    m->cap_T = T;
    return GRX_OK;
}

// The loop's control and state buffers rfinalize makes, released (after a
// failed finalize the decoder is as before it; grx_rnnt_destroy frees them
// too).
void rrelease(grx_rnnt *m) {
    for (void **p : {(void **)&m->ctl, (void **)&m->S, (void **)&m->gx, (void **)&m->gh, (void **)&m->pp,
                     (void **)&m->logits}) {
        if (*p) (void)hipFree(*p);
        *p = nullptr;
    }
    if (m->ctl_host) (void)hipHostFree(m->ctl_host);
    m->ctl_host = nullptr;
}

grx_status rfinalize_buffers(grx_rnnt *m);

grx_status rfinalize(grx_rnnt *m) {
    const grx_status s = rfinalize_buffers(m);
    if (s != GRX_OK) rrelease(m);
    return s;
}

grx_status rfinalize_buffers(grx_rnnt *m) {
    const grx_rnnt_hparams &hp = m->hp;
    const auto ex = rexpected(hp, m->embed_rows);
    for (size_t i = 0; i < ex.size(); ++i)
        if (!m->have[i]) return grx_fail(GRX_ESTATE, "conformer: the model has no %s", ex[i].name.c_str());
    const int H = hp.pred_hidden, L = hp.pred_layers;
    grx_status s;
    if ((s = ralloc(m, sizeof(RnntCtl), reinterpret_cast<void **>(&m->ctl))) != GRX_OK) return s;
    GRX_HIP(grx_pinned_malloc(reinterpret_cast<void **>(&m->ctl_host), sizeof(RnntCtl)));
    if ((s = ralloc(m, (size_t)2 * 2 * L * H * 4, reinterpret_cast<void **>(&m->S))) != GRX_OK) return s;
    if ((s = ralloc(m, (size_t)L * 4 * H * 4, reinterpret_cast<void **>(&m->gx))) != GRX_OK) return s;
    if ((s = ralloc(m, (size_t)L * 4 * H * 4, reinterpret_cast<void **>(&m->gh))) != GRX_OK) return s;
    if ((s = ralloc(m, (size_t)hp.joint_hidden * 4, reinterpret_cast<void **>(&m->pp))) != GRX_OK) return s;
    if ((s = ralloc(m, (size_t)m->k.R * 4, reinterpret_cast<void **>(&m->logits))) != GRX_OK) return s;
    m->ready = true;
    return GRX_OK;
}

}  // namespace

extern "C" grx_status grx_rnnt_create(grx_ctx *ctx, const grx_rnnt_hparams *hp, grx_rnnt **out) {
    if (!ctx || !hp || !out) return grx_fail(GRX_EINVAL, "grx_rnnt_create: NULL argument");
    *out = nullptr;
    const int H = hp->pred_hidden, J = hp->joint_hidden;
    if (hp->pred_vocab < 2 || H <= 0 || hp->pred_layers <= 0 || J <= 0 || hp->d <= 0)
        return grx_fail(GRX_EINVAL, "conformer: the model file is missing its decoder settings");
    if (H % 32 || J % 32 || hp->d % 32)
        return grx_fail(GRX_ESIZE, "grx_rnnt_create: pred_hidden %d, joint_hidden %d and d %d must be multiples of 32",
                        H, J, hp->d);
    if (H > 32768 || J > 32768 || hp->d > 32768)
        return grx_fail(GRX_ESIZE, "grx_rnnt_create: widths above 32768");
    if (hp->joint_act < 0 || hp->joint_act > 2) return grx_fail(GRX_EINVAL, "grx_rnnt_create: joint_act %d", hp->joint_act);
    if (hp->tdt) {
        if (hp->n_durations <= 0) return grx_fail(GRX_EINVAL, "conformer: a TDT model needs its durations");
        if (hp->n_durations > kMaxDur) return grx_fail(GRX_ESIZE, "grx_rnnt_create: more than %d durations", kMaxDur);
        if (hp->max_symbols < 1 || hp->max_symbols > 100)
            return grx_fail(GRX_EINVAL, "conformer: tdt.max_symbols %d is out of range", hp->max_symbols);
        for (int i = 0; i < hp->n_durations; ++i)
            if (hp->durations[i] < 0 || hp->durations[i] > kMaxDuration)
                return grx_fail(GRX_EINVAL, "grx_rnnt_create: duration %d outside 0..%d", hp->durations[i],
                                kMaxDuration);
    }
    grx_rnnt *m = new grx_rnnt;
    m->ctx = ctx;
    m->hp = *hp;
    if (!hp->tdt) {  // readHParams: RNN-T takes no durations and 10 symbols a frame
        m->hp.n_durations = 0;
        m->hp.max_symbols = 10;
    }
    if (m->hp.blank < 0) m->hp.blank = hp->pred_vocab - 1;
    RnntHp &k = m->k;
    k.H = H;
    k.L = hp->pred_layers;
    k.J = J;
    k.V = hp->pred_vocab;
    k.R = hp->pred_vocab + m->hp.n_durations;
    k.act = hp->joint_act;
    k.tdt = hp->tdt ? 1 : 0;
    k.nd = m->hp.n_durations;
    k.max_symbols = m->hp.max_symbols;
    k.blank = m->hp.blank;
    for (int i = 0; i < k.nd; ++i) k.dur[i] = hp->durations[i];
    // the embedding rows a token can index: every id below pred_vocab but blank
    m->embed_rows = m->hp.blank == hp->pred_vocab - 1 ? hp->pred_vocab - 1 : hp->pred_vocab;
    m->lstm.resize(hp->pred_layers);
    m->have.assign(rexpected(m->hp, m->embed_rows).size(), false);
    *out = m;
    return GRX_OK;
}

extern "C" grx_status grx_rnnt_destroy(grx_rnnt *m) {
    if (!m) return GRX_OK;
    (void)hipSetDevice(m->ctx->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    free_work(m);
    for (Lstm &l : m->lstm) {
        grx_weight_destroy(l.wx);
        grx_weight_destroy(l.wh);
        if (l.b) (void)hipFree(l.b);
    }
    grx_weight_destroy(m->jenc);
    grx_weight_destroy(m->jpred);
    grx_weight_destroy(m->jout);
    for (void *p : {(void *)m->embed, (void *)m->jencb, (void *)m->jpredb, (void *)m->joutb})
        if (p) (void)hipFree(p);
    rrelease(m);
    delete m;
    return GRX_OK;
}

extern "C" grx_status grx_rnnt_set_tensor(grx_rnnt *m, const char *name, const void *data, size_t nbytes) {
    if (!m || !name || (!data && nbytes)) return grx_fail(GRX_EINVAL, "grx_rnnt_set_tensor: NULL argument");
    if (m->ready) return grx_fail(GRX_ESTATE, "grx_rnnt_set_tensor: the decoder is in use already");
    const auto ex = rexpected(m->hp, m->embed_rows);
    size_t i = 0;
    while (i < ex.size() && ex[i].name != name) ++i;
    if (i == ex.size()) return grx_fail(GRX_EINVAL, "grx_rnnt_set_tensor: unknown tensor %s", name);
    if (m->have[i]) return grx_fail(GRX_ESTATE, "grx_rnnt_set_tensor: %s given twice", name);
    const RExpect &e = ex[i];
    const std::string n = name;
    grx_status s;
    if (e.cols > 0) {
        const size_t want = (size_t)e.rows * (e.cols / 32) * 34;
        if (nbytes != want)
            return grx_fail(GRX_ESIZE, "grx_rnnt_set_tensor: %s holds %zu bytes, a Q8_0 [%d][%d] matrix is %zu", name,
                            nbytes, e.rows, e.cols, want);
        grx_weight *w = nullptr;
        if ((s = grx_weight_q8_create(m->ctx, e.rows, e.cols, static_cast<const uint8_t *>(data), nbytes, &w)) !=
            GRX_OK)
            return s;
        if (n == "joint.enc.weight") m->jenc = w;
        else if (n == "joint.pred.weight") m->jpred = w;
        else if (n == "joint.out.weight") m->jout = w;
        else {
            const int l = atoi(name + 10);  // "pred.lstm.<l>."
            (n.back() == 'x' ? m->lstm[l].wx : m->lstm[l].wh) = w;
        }
    } else {
        size_t want = (size_t)e.rows * 4;
        if (n == "pred.embed.weight") {
            // more rows than the ids reach are allowed (the converter keeps NeMo's padding row)
            const size_t row = (size_t)m->hp.pred_hidden * 4;
            if (nbytes < want || nbytes % row)
                return grx_fail(GRX_ESIZE, "grx_rnnt_set_tensor: %s holds %zu bytes, at least %d rows of %d wanted", name,
                                nbytes, m->embed_rows, m->hp.pred_hidden);
            want = nbytes;
        }
        if (nbytes != want)
            return grx_fail(GRX_ESIZE, "grx_rnnt_set_tensor: %s holds %zu bytes, %zu wanted", name, nbytes, want);
        float *p = nullptr;
        GRX_HIP(hipSetDevice(m->ctx->device));
        if ((s = upload_vec(m, data, nbytes, &p)) != GRX_OK) return s;
        if (n == "pred.embed.weight") m->embed = p;
        else if (n == "joint.enc.bias") m->jencb = p;
        else if (n == "joint.pred.bias") m->jpredb = p;
        else if (n == "joint.out.bias") m->joutb = p;
        else m->lstm[atoi(name + 10)].b = p;
    }
    m->have[i] = true;
    for (bool h : m->have)
        if (!h) return GRX_OK;
    return rfinalize(m);
}

extern "C" grx_status grx_rnnt_state_create(grx_rnnt *m, grx_rnnt_state **out) {
    if (!m || !out) return grx_fail(GRX_EINVAL, "grx_rnnt_state_create: NULL argument");
    *out = nullptr;
    GRX_HIP(hipSetDevice(m->ctx->device));
    const size_t bytes = (size_t)2 * m->k.L * m->k.H * 4;
    grx_rnnt_state *s = new grx_rnnt_state{m, m->ctx, m->k.L, m->k.H, m->k.V, m->k.blank, m->embed_rows, nullptr, -1};
    hipError_t e = grx_dev_malloc(reinterpret_cast<void **>(&s->hc), bytes);
    if (e == hipSuccess) e = hipMemset(s->hc, 0, bytes);
    if (e != hipSuccess) {
        if (s->hc) (void)hipFree(s->hc);
        delete s;
        return grx_hip_fail(e, "grx_rnnt_state_create");
    }
    *out = s;
    return GRX_OK;
}

extern "C" grx_status grx_rnnt_state_destroy(grx_rnnt_state *s) {
    if (!s) return GRX_OK;
    (void)hipSetDevice(s->ctx->device);
    (void)hipFree(s->hc);
    delete s;
    return GRX_OK;
}

extern "C" grx_status grx_rnnt_state_read(const grx_rnnt_state *s, float *h, float *c, int *last) {
    if (!s) return grx_fail(GRX_EINVAL, "grx_rnnt_state_read: NULL state");
    const size_t n = (size_t)s->L * s->H * 4;
    GRX_HIP(hipSetDevice(s->ctx->device));
    GRX_HIP(hipStreamSynchronize(s->ctx->stream));
    if (h) GRX_HIP(hipMemcpy(h, s->hc, n, hipMemcpyDeviceToHost));
    if (c) GRX_HIP(hipMemcpy(c, reinterpret_cast<const char *>(s->hc) + n, n, hipMemcpyDeviceToHost));
    if (last) *last = s->last;
    return GRX_OK;
}

extern "C" grx_status grx_rnnt_state_write(grx_rnnt_state *s, const float *h, const float *c, int last) {
    if (!s || !h || !c) return grx_fail(GRX_EINVAL, "grx_rnnt_state_write: NULL argument");
    if (last < -1 || last >= s->V) return grx_fail(GRX_EINVAL, "grx_rnnt_state_write: last token %d", last);
    if (last >= 0 && last != s->blank && last >= s->embed_rows)
        return grx_fail(GRX_EINVAL, "grx_rnnt_state_write: last token %d has no embedding row", last);
    const size_t n = (size_t)s->L * s->H * 4;
    GRX_HIP(hipSetDevice(s->ctx->device));
    GRX_HIP(hipStreamSynchronize(s->ctx->stream));
    GRX_HIP(hipMemcpy(s->hc, h, n, hipMemcpyHostToDevice));
    GRX_HIP(hipMemcpy(reinterpret_cast<char *>(s->hc) + n, c, n, hipMemcpyHostToDevice));
    s->last = last;
    return GRX_OK;
}

extern "C" grx_status grx_rnnt_decode(grx_rnnt *m, const float *enc, int T, int enc_on_device, grx_rnnt_state *st,
                                      int frame_offset, grx_rnnt_token *out, int cap, int *n_out) {
    if (!m || (!enc && T > 0) || !n_out || (!out && cap > 0) || T < 0 || cap < 0)
        return grx_fail(GRX_EINVAL, "grx_rnnt_decode: NULL argument or negative size");
    if (!m->ready) {
        // the last tensor's set-up may have failed (out of memory): try again
        for (bool h : m->have)
            if (!h) return grx_fail(GRX_ESTATE, "grx_rnnt_decode: the decoder's tensors are not all set");
        grx_status fs = rfinalize(m);
        if (fs != GRX_OK) return fs;
    }
    if (st && (st->m != m || st->L != m->k.L || st->H != m->k.H))
        return grx_fail(GRX_EINVAL, "grx_rnnt_decode: the state belongs to another decoder");
    *n_out = 0;
    if (T == 0) return GRX_OK;
    if (T > (1 << 24)) return grx_fail(GRX_ESIZE, "grx_rnnt_decode: %d frames", T);
    GRX_HIP(hipSetDevice(m->ctx->device));
    hipStream_t s0 = m->ctx->stream;
    grx_status s;
    if ((s = ensure_T(m, T)) != GRX_OK) return s;
    const int d = m->hp.d, J = m->k.J, max_iters = 16 * T + 1024;
    const float *x = enc;
    if (!enc_on_device) {
        GRX_HIP(hipMemcpyAsync(m->enc, enc, (size_t)T * d * 4, hipMemcpyHostToDevice, s0));
        x = m->enc;
    }
    // encProj = enc Wencᵀ + b (rnnt.go:126-128)
    if (T == 1) {
        if ((s = grx_float_gemv_q8(s0, m->jenc, x, m->jencb, m->ep)) != GRX_OK) return s;
    } else {
        if ((s = grx_quant_act_dev(m->ctx, m->xq, m->xs, x, d, T, d)) != GRX_OK) return s;
        if ((s = grx_gemm_q8_launch(s0, m->jenc, m->xq, m->xs, T, m->jencb, m->ep, J)) != GRX_OK) return s;
    }
    const size_t hcb = (size_t)2 * m->k.L * m->k.H * 4;
    if (st)
        GRX_HIP(hipMemcpyAsync(m->S, st->hc, hcb, hipMemcpyDeviceToDevice, s0));
    else
        GRX_HIP(hipMemsetAsync(m->S, 0, hcb, s0));
    rnnt_ctl_init_kernel<<<1, 64, 0, s0>>>(m->ctl, T, max_iters, frame_offset, st ? st->last : -1);
    GRX_LAUNCHED("rnnt_ctl_init_kernel");
    const bool eager = grx_tune(GRX_TUNE_NO_GRAPH) == 1;
    if (!eager && !m->exec) {
        GRX_HIP(hipStreamSynchronize(s0));
        hipError_t e = hipStreamBeginCapture(s0, hipStreamCaptureModeThreadLocal);
        if (e == hipSuccess) {
            grx_status cs = GRX_OK;
            for (int i = 0; i < kIters && cs == GRX_OK; ++i) cs = enqueue_iter(m, s0);
            hipGraph_t g = nullptr;
            e = hipStreamEndCapture(s0, &g);
            if (cs == GRX_OK && e == hipSuccess) e = hipGraphInstantiate(&m->exec, g, nullptr, nullptr, 0);
            if (g) {
                if (e == hipSuccess && cs == GRX_OK) m->graph = g;
                else (void)hipGraphDestroy(g);
            }
            if (e != hipSuccess || cs != GRX_OK) {
                (void)hipGetLastError();
                m->exec = nullptr;
            }
        }
    }
    // every iteration that is not done advances iter, so the loop is done
    // after max_iters iterations at the latest
    const int rounds = (max_iters + kIters - 1) / kIters;
    bool done = false;
    for (int r = 0; r < rounds && !done; ++r) {
        if (m->exec && !eager) {
            GRX_HIP(hipGraphLaunch(m->exec, s0));
        } else {
            for (int i = 0; i < kIters; ++i)
                if ((s = enqueue_iter(m, s0)) != GRX_OK) return s;
        }
        GRX_HIP(hipMemcpyAsync(m->ctl_host, m->ctl, sizeof(RnntCtl), hipMemcpyDeviceToHost, s0));
        GRX_HIP(hipStreamSynchronize(s0));
        done = m->ctl_host->done != 0;
    }
    if (!done) return grx_fail(GRX_ESTATE, "grx_rnnt_decode: the loop did not end after %d iterations", max_iters);
    const RnntCtl c = *m->ctl_host;
    if (st) {
        GRX_HIP(hipMemcpyAsync(st->hc, m->S + (size_t)c.cur * 2 * m->k.L * m->k.H, hcb, hipMemcpyDeviceToDevice, s0));
        st->last = c.last[c.cur];
    }
    const int n = c.n_out;
    if (n > 0 && cap > 0)
        GRX_HIP(hipMemcpyAsync(out, m->tokens, (size_t)(n < cap ? n : cap) * sizeof(grx_rnnt_token),
                               hipMemcpyDeviceToHost, s0));
    GRX_HIP(hipStreamSynchronize(s0));
    *n_out = n;
    if (n > cap) return grx_fail(GRX_ESIZE, "grx_rnnt_decode: %d tokens for room of %d", n, cap);
    return GRX_OK;
}
