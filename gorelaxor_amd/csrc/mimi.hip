// mimi.hip - pocket-TTS's Mimi decoder (latents to 24 kHz audio) on one GPU.
//
// mimiDecoder.decode of pockettts/mimi.go:122-152 (github.com/xattribution/
// gorelaxor): the latent's projection to d channels, the depthwise
// transposed upsampling with the overlap carried to the next call, the
// context-limited transformer with layer scales (nn.go:142-254), then
// runSea (mimi.go:62-108) over SEANet's decoder: causal convolutions as
// im2col + Linear with their past rows carried (nn.go:272-296), transposed
// convolutions as Linear + overlap-add with the partial carried (nn.go:
// 308-327), residual blocks, ELU (nn.go:51-64).  Each Linear takes kern.
// MatMul's route for its weight's type: Q8_0 the int8 route (the rows
// rounded to Q8_0, then the matrix-core product), float32 the float route
// (k6x16 / gemvRows); every float step keeps the reference's order, so the
// samples are bit-identical to the CPU oracle's.
//
// One decode call is about 60 launches per latent: the stream's state
// (caches, carried rows, position) lives in device memory, the position
// also on the host, which passes each call's positions and rotary angles.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "grx_float.h"
#include "grx_internal.h"
#include "grx_ln.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxPast = 64;  // carried rows of one convolution
constexpr size_t kMaxAttnLds = 128 * 1024;  // a head's value rows and one query's scores

// ---------------------------------------------------------------- kernels

// ELU of element i of an n-value buffer (nn.go:51-64): t = min(v, 0)
// through ExpSub(t, 0) over chunks of 512 values (EXP8 below the chunk's
// whole groups of eight, expf past them), then max(v, 0) + (t - 1).
__device__ __forceinline__ float elu_at(float v, size_t i, size_t n) {
    const size_t c0 = i / 512 * 512;
    const size_t cl = n - c0 < 512 ? n - c0 : 512;
    const float t = __fsub_rn(v < 0.f ? v : 0.f, 0.f);
    const float e = (i - c0) < (cl & ~(size_t)7) ? grx_exp8(t) : grx_expf_go(t);
    return __fadd_rn(v > 0.f ? v : 0.f, __fsub_rn(e, 1.f));
}

__global__ void elu_kernel(float *__restrict__ x, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = elu_at(x[i], i, n);
}

// The depthwise ConvTranspose1d of decode (mimi.go:130-146) for n latent
// rows z [n][C] (taps up [C][2S]): row i of the full output is 0 plus, for
// t ascending, z[t][c] * up[c][i - tS]; the first S rows then add the
// carried part, rows [0, nS) go to x and rows [nS, nS+S) become the new
// carried part.  The thread of row i < S also ends row nS + i, after it
// has read the old part.
__global__ void mimi_up_kernel(const float *__restrict__ z, const float *__restrict__ up, int n, int S, int C,
                               float *__restrict__ part, float *__restrict__ x) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)n * S * C) return;
    const int i = (int)(idx / C), c = (int)(idx % C), K = 2 * S;
    auto row = [&](int r) {
        float f = 0.f;
        const int t1 = min(n - 1, r / S);
        for (int t = max(0, (r - K + S) / S); t <= t1; ++t) {
            const int j = r - t * S;
            if (j >= 0 && j < K) f = __fadd_rn(f, __fmul_rn(z[(size_t)t * C + c], up[(size_t)c * K + j]));
        }
        return f;
    };
    float f = row(i);
    if (i < S) {
        f = __fadd_rn(f, part[(size_t)i * C + c]);
        part[(size_t)i * C + c] = row(n * S + i);
    }
    x[(size_t)i * C + c] = f;
}

// pockettts' float64 LayerNorm (nn.go:27-49, eps 1e-5) of rows of n
// values, one workgroup per row: h = f32((v - mean) * inv) * w + b.
__global__ __launch_bounds__(kThreads) void ln64_rows_kernel(const float *__restrict__ x, int n,
                                                             const float *__restrict__ w, const float *__restrict__ b,
                                                             float *__restrict__ y) {
    extern __shared__ __align__(16) float row[];
    __shared__ double red[48];
    const float *xr = x + (size_t)blockIdx.x * n;
    for (int i = threadIdx.x; i < n; i += blockDim.x) row[i] = xr[i];
    __syncthreads();
    double mean, inv;
    ln64_stats(row, n, 1e-5, red, mean, inv);
    float *yr = y + (size_t)blockIdx.x * n;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float o = (float)__dmul_rn(__dsub_rn((double)row[i], mean), inv);
        yr[i] = __fadd_rn(__fmul_rn(o, w[i]), b[i]);
    }
}

// applyRope (nn.go:80-93) of q and k of T rows of qkv [T][3d] at the
// call's positions (cos/sin [T][hd/2] from the host: f32(cos(f64(f_i *
// f32(pos))))), q in place; k (rotated) and v into the ring slots
// (pos0 + r) % cap.
__global__ void mimi_rope_ring_kernel(float *__restrict__ qkv, int T, int d, int hd, const float *__restrict__ cs,
                                      const float *__restrict__ sn, float *__restrict__ kr, float *__restrict__ vr,
                                      int cap, const long long *__restrict__ posd) {
    const long long pos0 = *posd;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int half = hd / 2, pairs = d / 2;
    if (idx >= (size_t)T * pairs) return;
    const int r = (int)(idx / pairs), p = (int)(idx % pairs), h = p / half, i = p % half;
    const float c = cs[(size_t)r * half + i], s = sn[(size_t)r * half + i];
    float *row = qkv + (size_t)r * 3 * d;
    const int j = h * hd + 2 * i;
    const size_t slot = (size_t)((pos0 + r) % cap) * d;
    {
        const float re = row[j], im = row[j + 1];
        row[j] = __fsub_rn(__fmul_rn(re, c), __fmul_rn(im, s));
        row[j + 1] = __fadd_rn(__fmul_rn(re, s), __fmul_rn(im, c));
    }
    {
        const float re = row[d + j], im = row[d + j + 1];
        kr[slot + j] = __fsub_rn(__fmul_rn(re, c), __fmul_rn(im, s));
        kr[slot + j + 1] = __fadd_rn(__fmul_rn(re, s), __fmul_rn(im, c));
    }
    vr[slot + j] = row[2 * d + j];
    vr[slot + j + 1] = row[2 * d + j + 1];
}

// attend (nn.go:200-254) for T rows after pos0 positions, one workgroup per
// (head, query row): query p sees keys max(lo0, p - context + 1) .. p, lo0 =
// max(0, pos0 - context + 1); the row's scores over its window by
// MatMulF32's route for T rows (outside the window they are 0 after the
// softmax, as the reference clears them), scaled and softmaxed (expSub's
// order, block_softmax); then T < 4: AddScaled over the nk = pos0 + T - lo0
// keys in order, zero weights skipped; else the product of the row with the
// values by the same route, over all nk keys.  The head's value rows are
// staged in LDS ([nk][hd]), keys read from the ring.
__global__ __launch_bounds__(kThreads) void mimi_attn_kernel(const float *__restrict__ qkv, const float *__restrict__ kr,
                                                             const float *__restrict__ vr, int cap,
                                                             const long long *__restrict__ posd, int T, int d, int hd,
                                                             int context, float scale, float *__restrict__ att) {
    extern __shared__ __align__(16) float sm[];
    const long long pos0 = *posd;
    const int h = blockIdx.x, r = blockIdx.y, tid = threadIdx.x;
    const long long lo0 = pos0 - context + 1 > 0 ? pos0 - context + 1 : 0;
    const int nk = (int)(pos0 + T - lo0);
    const long long p = pos0 + r;
    const long long lo = p - context + 1 > lo0 ? p - context + 1 : lo0;
    const int off = (int)(lo - lo0), ns = (int)(p + 1 - lo);
    float *V = sm;            // [nk][hd]
    float *s = V + nk * hd;   // [nk]
    float *q = s + nk;        // [hd]
    float *part = q + hd;     // block_softmax's 32
    for (int i = tid; i < hd; i += blockDim.x) q[i] = qkv[(size_t)r * 3 * d + h * hd + i];
    for (int i = tid; i < nk * hd; i += blockDim.x) {
        const int j = i / hd, e = i % hd;
        V[i] = vr[(size_t)((lo0 + j) % cap) * d + h * hd + e];
    }
    __syncthreads();
    for (int j = tid; j < nk; j += blockDim.x) {
        float v = 0.f;
        if (j >= off && j < off + ns)
            v = __fmul_rn(matmul_f32_one(q, kr + (size_t)((lo0 + j) % cap) * d + h * hd, 1, hd, r, T, j, nk), scale);
        s[j] = v;
    }
    __syncthreads();
    block_softmax(s + off, ns, part);
    const int h8 = hd & ~7;
    for (int e = tid; e < hd; e += blockDim.x) {
        float o;
        if (T < 4) {
            o = 0.f;
            for (int j = 0; j < nk; ++j) {
                const float w = s[j];
                if (w == 0.f) continue;
                const float v = V[(size_t)j * hd + e];
                o = e < h8 ? __fmaf_rn(w, v, o) : __fadd_rn(o, __fmul_rn(w, v));
            }
        } else {
            o = matmul_f32_one(s, V + e, hd, nk, r, T, e, hd);
        }
        att[(size_t)r * d + h * hd + e] = o;
    }
}

// addScaled (nn.go:185-196): x += s[i % d] * y (unfused), or x += y
__global__ void add_scaled_kernel(float *__restrict__ x, const float *__restrict__ y, const float *__restrict__ s,
                                  int d, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    x[i] = s != nullptr ? __fadd_rn(x[i], __fmul_rn(s[i % d], y[i])) : __fadd_rn(x[i], y[i]);
}

// kern.GELU over n values (geluVec: the assembly form below n &^ 7)
__global__ void gelu_kernel(float *__restrict__ x, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = grx_gelu_at(x[i], (int)i, (int)n);
}

// conv.run's im2col (nn.go:283-290): buf = the P carried rows then T rows
// of x (ELU'd first when elu: runSea's in-place ELU, nn.go/mimi.go:67-69,
// or the residual block's copy), col row t, tap j = buf row t*stride + j*dil.
__global__ void im2col_kernel(const float *__restrict__ prev, const float *__restrict__ x, int T, int cin, int k,
                              int stride, int dil, int P, int elu, float *__restrict__ col) {
    const int To = T / stride, cols = k * cin;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)To * cols) return;
    const int t = (int)(idx / cols), q = (int)(idx % cols), j = q / cin, e = q % cin;
    const int br = t * stride + j * dil;
    float v;
    if (br < P) {
        v = prev[(size_t)br * cin + e];
    } else {
        const size_t xi = (size_t)(br - P) * cin + e;
        v = elu ? elu_at(x[xi], xi, (size_t)T * cin) : x[xi];
    }
    col[idx] = v;
}

// The carried rows after a conv call: the last P rows of buf (nn.go:293),
// one thread per channel, rows in increasing order (a row moved within prev
// is read before it is overwritten).
__global__ void conv_past_kernel(float *__restrict__ prev, const float *__restrict__ x, int T, int cin, int P,
                                 int elu) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= cin) return;
    for (int i = 0; i < P; ++i) {
        const int br = T + i;  // buf row
        float v;
        if (br < P) {
            v = prev[(size_t)br * cin + e];
        } else {
            const size_t xi = (size_t)(br - P) * cin + e;
            v = elu ? elu_at(x[xi], xi, (size_t)T * cin) : x[xi];
        }
        prev[(size_t)i * cin + e] = v;
    }
}

// convtr.run's overlap-add (nn.go:314-326) of z [T][k*co]: row i starts at
// the bias, adds z[t][(i - tS)*co + e] for t ascending, then the first
// k - S rows add the carried partial; rows [0, TS) go to y, rows [TS,
// TS + k - S) minus the bias become the new partial.  The thread of row
// i < k - S also ends row TS + i after reading the old partial.
__global__ void convtr_overlap_kernel(const float *__restrict__ z, const float *__restrict__ b, int T, int S, int K,
                                      int co, float *__restrict__ partial, float *__restrict__ y) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)T * S * co) return;
    const int i = (int)(idx / co), e = (int)(idx % co), PT = K - S;
    auto row = [&](int r) {
        float f = b[e];
        const int t1 = min(T - 1, r / S);
        for (int t = max(0, (r - K + S) / S); t <= t1; ++t) {
            const int j = r - t * S;
            if (j >= 0 && j < K) f = __fadd_rn(f, z[((size_t)t * K + j) * co + e]);
        }
        return f;
    };
    float f = row(i);
    if (i < PT) {
        f = __fadd_rn(f, partial[(size_t)i * co + e]);
        partial[(size_t)i * co + e] = __fsub_rn(row(T * S + i), b[e]);
    }
    y[idx] = f;
}

// ---------------------------------------------------------------- host side

struct MLin {
    int n = 0, k = 0;
    grx_weight *q = nullptr;  // Q8_0: the int8 route
    float *f = nullptr;       // float32 [n][k]: the float route
    float *b = nullptr;       // [n] or none
    bool have_w = false, have_b = false;
};

struct MConv {
    int cin = 0, cout = 0, k = 0, stride = 1, dil = 1, past = 0;
    MLin w;
    float *prev = nullptr;  // [past][cin]
};

struct MConvTr {
    int cin = 0, cout = 0, k = 0, stride = 1;
    MLin w;                    // no bias in the product
    float *b = nullptr;        // [cout]
    float *partial = nullptr;  // [k - stride][cout]
};

struct MStep {
    int kind = 0, elu = 0;  // 0 conv, 1 transposed conv, 2 residual block
    std::string name;
    MConv c, a, bb;
    MConvTr t;
};

struct MLayer {
    float *n1w = nullptr, *n1b = nullptr, *n2w = nullptr, *n2b = nullptr, *ls1 = nullptr, *ls2 = nullptr;
    MLin qkv, out, ff1, ff2;
    float *kr = nullptr, *vr = nullptr;  // rings [cap][d]
};

// A tensor the model expects: its name, where it goes, and its shape
// (rows x cols for matrices, n for vectors).
struct MExpect {
    std::string name;
    MLin *lin = nullptr;   // matrix
    float **vec = nullptr; // vector
    int rows = 0, cols = 0;
    bool bias = false;     // a Linear's bias (lin set)
};

}  // namespace

struct grx_mimi {
    grx_ctx *ctx = nullptr;
    grx_mimi_hparams hp{};
    int hd = 0, tmax = 0, cap = 0, spl = 0;
    std::vector<MLayer> layers;
    std::vector<MStep> steps;
    MLin quant;
    float *up = nullptr;
    std::vector<MExpect> expect;
    std::vector<bool> have;
    bool complete = false;  // every tensor given
    bool ready = false;     // and the state and work buffers made
    hipEvent_t rope_copied = nullptr;  // the last call's copy of rope_host
    std::vector<void *> allocs;
    // state: the position (the host's copy forms the rotary angles, the
    // device's is what the kernels read, so a captured call replays)
    long long pos = 0;
    long long *posd = nullptr;
    float *up_part = nullptr;
    // the captured call: one graph for the last (latents, input, output)
    hipGraphExec_t exec = nullptr;
    int g_n = 0;
    const float *g_lat = nullptr;
    float *g_out = nullptr;
    bool no_graph = false;  // capture refused once: launch kernel by kernel
    // work
    float *x = nullptr, *y = nullptr, *h = nullptr, *o = nullptr, *col = nullptr, *z = nullptr;
    float *qkv = nullptr, *att = nullptr, *f = nullptr, *lat = nullptr, *out = nullptr;
    int8_t *xq = nullptr;
    float *xs = nullptr;
    float *rope = nullptr;        // device cos [tmax][hd/2] then sin
    float *rope_host = nullptr;   // pinned
    std::vector<float> freqs;
    size_t act_floats = 0, col_floats = 0, z_floats = 0, h_floats = 0, q_bytes = 0, attn_lds = 0;
};

namespace {

// LDS of the attention kernel: a head's value rows over the ring's
// positions, one query's scores, the query, block_softmax's 32 floats
size_t attn_lds(const grx_mimi_hparams &hp) {
    const size_t cap = (size_t)hp.context + (size_t)hp.max_latents * hp.upsample - 1, hd = hp.d / hp.heads;
    return (cap * hd + cap + hd + 32) * 4;
}

grx_status malloc_dev(grx_mimi *m, size_t bytes, void **out) {
    *out = nullptr;
    const hipError_t e = grx_dev_malloc(out, bytes ? bytes : 4);
    if (e != hipSuccess) return grx_hip_fail(e, "hipMalloc");
    m->allocs.push_back(*out);
    return GRX_OK;
}

template <typename T>
grx_status malloc_t(grx_mimi *m, size_t count, T **out) {
    return malloc_dev(m, count * sizeof(T), reinterpret_cast<void **>(out));
}

void release(grx_mimi *m) {
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    m->exec = nullptr;
    for (void *p : m->allocs) (void)hipFree(p);
    m->allocs.clear();
    if (m->rope_host) (void)hipHostFree(m->rope_host);
    m->rope_host = nullptr;
    if (m->rope_copied) (void)hipEventDestroy(m->rope_copied);
    m->rope_copied = nullptr;
    for (MLayer &L : m->layers)
        for (MLin *w : {&L.qkv, &L.out, &L.ff1, &L.ff2})
            if (w->q) {
                grx_weight_destroy(w->q);
                w->q = nullptr;
            }
    for (MStep &s : m->steps)
        for (MLin *w : {&s.c.w, &s.a.w, &s.bb.w, &s.t.w})
            if (w->q) {
                grx_weight_destroy(w->q);
                w->q = nullptr;
            }
    if (m->quant.q) {
        grx_weight_destroy(m->quant.q);
        m->quant.q = nullptr;
    }
}

void gridn(size_t n, unsigned *blocks) { *blocks = (unsigned)((n + kThreads - 1) / kThreads); }

// kern.Linear(y, x, rows, w, bias) by the weight's route; ADD (Q8_0 only):
// y += the product (kern.Add of it, the residual's sum).
grx_status lin(grx_mimi *m, hipStream_t st, const MLin &w, const float *x, int rows, float *y, bool add = false) {
    if (rows == 0) return GRX_OK;
    if (w.q && rows % 8 == 0 && rows <= 64 && w.k <= 1280) {
        // a few groups of 8 rows in one several-row GEMV launch that rounds
        // its rows in its own prologue (quantU8, the same arithmetic as the
        // rounding launch it replaces)
        GemvArgs a = {};
        a.qs = w.q->qs;
        a.ds = w.q->ds;
        a.rows = w.q->rows;
        a.nb = w.q->nb;
        a.x = x;
        a.lda = w.k;
        a.bias = w.b;
        a.y = y;
        a.ldc = w.n;
        a.resid = y;
        a.ldr = w.n;
        a.cacheable = 1;
        a.chunks = rows / 8;
        return grx_gemv_launch(st, 8, GRX_PRO_QUANT, add ? GRX_EPI_RESID : GRX_EPI_STORE, a, 0);
    }
    if (w.q) {
        grx_status s = grx_quant_rows(st, x, w.k, rows, w.k, m->xq, m->xs);
        if (s != GRX_OK) return s;
        GemmOut o;
        o.y = y;
        o.ldc = w.n;
        o.epi = add ? GRX_GEMM_ADD : GRX_GEMM_STORE;
        return grx_gemm_q8_launch_ex(st, w.q, m->xq, m->xs, rows, w.b, o);
    }
    if (add) return grx_fail(GRX_EINVAL, "grx_mimi: a float32 residual product adds separately");
    return grx_float_rows_f32(st, x, w.f, w.b, y, 1, rows, w.n, w.k);
}

grx_status conv_run(grx_mimi *m, hipStream_t st, MConv &c, const float *x, int T, int elu, float *y) {
    unsigned blocks;
    if (c.k == 1 && c.stride == 1) {
        if (elu) return grx_fail(GRX_EINVAL, "grx_mimi: ELU before a 1x1 convolution");
        return lin(m, st, c.w, x, T, y);
    }
    const int To = T / c.stride;
    gridn((size_t)To * c.k * c.cin, &blocks);
    im2col_kernel<<<blocks, kThreads, 0, st>>>(c.prev, x, T, c.cin, c.k, c.stride, c.dil, c.past, elu, m->col);
    GRX_LAUNCHED("im2col_kernel");
    gridn((size_t)c.cin, &blocks);
    conv_past_kernel<<<blocks, kThreads, 0, st>>>(c.prev, x, T, c.cin, c.past, elu);
    GRX_LAUNCHED("conv_past_kernel");
    return lin(m, st, c.w, m->col, To, y);
}

// decode (mimi.go:122-152) of n latents at lat (device) into out (device)
// The call's rotary angles (nn.go:83-86), as the oracle forms them, into
// the pinned staging buffer (host work, before the call's kernels): it is
// rewritten once the previous call's copy of it is done.
grx_status rope_angles(grx_mimi *m, int T) {
    const int half = m->hd / 2;
    GRX_HIP(hipEventSynchronize(m->rope_copied));
    for (int r = 0; r < T; ++r) {
        const float p = (float)(m->pos + r);
        for (int i = 0; i < half; ++i) {
            const double a = (double)(m->freqs[i] * p);
            m->rope_host[(size_t)r * half + i] = (float)cos(a);
            m->rope_host[(size_t)(m->tmax + r) * half + i] = (float)sin(a);
        }
    }
    return GRX_OK;
}

__global__ void mimi_pos_kernel(long long *posd, int T) { *posd += T; }

// The call's device work, in stream order (captured into a graph, or
// launched kernel by kernel): the angles' copy, the kernels, and the
// device position moved on by the call's rows.
grx_status enqueue_decode(grx_mimi *m, hipStream_t st, const float *lat, int n, float *out) {
    const grx_mimi_hparams &hp = m->hp;
    const int d = hp.d, S = hp.upsample, T = n * S, hd = m->hd, half = hd / 2;
    unsigned blocks;
    grx_status s;
    GRX_HIP(hipMemcpyAsync(m->rope, m->rope_host, (size_t)2 * m->tmax * half * 4, hipMemcpyHostToDevice, st));
    // latent projection (kern.Linear, no bias), then the upsampling
    if ((s = lin(m, st, m->quant, lat, n, m->z)) != GRX_OK) return s;
    gridn((size_t)T * d, &blocks);
    mimi_up_kernel<<<blocks, kThreads, 0, st>>>(m->z, m->up, n, S, d, m->up_part, m->x);
    GRX_LAUNCHED("mimi_up_kernel");
    const float scale = (float)(1.0 / sqrt((double)hd));
    for (MLayer &L : m->layers) {
        ln64_rows_kernel<<<T, kThreads, (size_t)d * 4, st>>>(m->x, d, L.n1w, L.n1b, m->h);
        GRX_LAUNCHED("ln64_rows_kernel");
        if ((s = lin(m, st, L.qkv, m->h, T, m->qkv)) != GRX_OK) return s;
        gridn((size_t)T * d / 2, &blocks);
        mimi_rope_ring_kernel<<<blocks, kThreads, 0, st>>>(m->qkv, T, d, hd, m->rope, m->rope + (size_t)m->tmax * half,
                                                           L.kr, L.vr, m->cap, m->posd);
        GRX_LAUNCHED("mimi_rope_ring_kernel");
        mimi_attn_kernel<<<dim3(hp.heads, T), kThreads, m->attn_lds, st>>>(m->qkv, L.kr, L.vr, m->cap, m->posd, T, d,
                                                                          hd, hp.context, scale, m->att);
        GRX_LAUNCHED("mimi_attn_kernel");
        if ((s = lin(m, st, L.out, m->att, T, m->h)) != GRX_OK) return s;
        gridn((size_t)T * d, &blocks);
        add_scaled_kernel<<<blocks, kThreads, 0, st>>>(m->x, m->h, L.ls1, d, (size_t)T * d);
        GRX_LAUNCHED("add_scaled_kernel");
        ln64_rows_kernel<<<T, kThreads, (size_t)d * 4, st>>>(m->x, d, L.n2w, L.n2b, m->h);
        GRX_LAUNCHED("ln64_rows_kernel");
        if ((s = lin(m, st, L.ff1, m->h, T, m->f)) != GRX_OK) return s;
        gridn((size_t)T * hp.ff, &blocks);
        gelu_kernel<<<blocks, kThreads, 0, st>>>(m->f, (size_t)T * hp.ff);
        GRX_LAUNCHED("gelu_kernel");
        if ((s = lin(m, st, L.ff2, m->f, T, m->h)) != GRX_OK) return s;
        gridn((size_t)T * d, &blocks);
        add_scaled_kernel<<<blocks, kThreads, 0, st>>>(m->x, m->h, L.ls2, d, (size_t)T * d);
        GRX_LAUNCHED("add_scaled_kernel");
    }
    mimi_pos_kernel<<<1, 1, 0, st>>>(m->posd, T);
    GRX_LAUNCHED("mimi_pos_kernel");
    // SEANet (runSea, mimi.go:62-108): x and y alternate as the rows
    float *cur = m->x, *nxt = m->y;
    int R = T;
    for (size_t si = 0; si < m->steps.size(); ++si) {
        MStep &q = m->steps[si];
        const bool last = si + 1 == m->steps.size();
        float *dst = last ? out : nxt;
        if (q.kind == 0) {
            if ((s = conv_run(m, st, q.c, cur, R, q.elu, dst)) != GRX_OK) return s;
            R /= q.c.stride;
            std::swap(cur, nxt);
        } else if (q.kind == 1) {
            MConvTr &t = q.t;
            if (q.elu) {
                gridn((size_t)R * t.cin, &blocks);
                elu_kernel<<<blocks, kThreads, 0, st>>>(cur, (size_t)R * t.cin);
                GRX_LAUNCHED("elu_kernel");
            }
            if ((s = lin(m, st, t.w, cur, R, m->z)) != GRX_OK) return s;
            gridn((size_t)R * t.stride * t.cout, &blocks);
            convtr_overlap_kernel<<<blocks, kThreads, 0, st>>>(m->z, t.b, R, t.stride, t.k, t.cout, t.partial, dst);
            GRX_LAUNCHED("convtr_overlap_kernel");
            R *= t.stride;
            std::swap(cur, nxt);
        } else {
            // v = ELU(copy of x) inside the first conv's im2col; h = ELU(a(v));
            // x += b(h)
            if ((s = conv_run(m, st, q.a, cur, R, 1, m->h)) != GRX_OK) return s;
            gridn((size_t)R * q.a.cout, &blocks);
            elu_kernel<<<blocks, kThreads, 0, st>>>(m->h, (size_t)R * q.a.cout);
            GRX_LAUNCHED("elu_kernel");
            if (q.bb.w.q) {
                if ((s = lin(m, st, q.bb.w, m->h, R, cur, true)) != GRX_OK) return s;
            } else {
                if ((s = lin(m, st, q.bb.w, m->h, R, m->o)) != GRX_OK) return s;
                gridn((size_t)R * q.bb.cout, &blocks);
                add_scaled_kernel<<<blocks, kThreads, 0, st>>>(cur, m->o, nullptr, 1, (size_t)R * q.bb.cout);
                GRX_LAUNCHED("add_scaled_kernel");
            }
            if (last) GRX_HIP(hipMemcpyAsync(out, cur, (size_t)R * q.bb.cout * 4, hipMemcpyDeviceToDevice, st));
        }
    }
    return GRX_OK;
}

// The tensors of the model (pockettts/model.go:105-181, 306-308) and the
// buffers a decode of max_latents needs.
grx_status build_plan(grx_mimi *m) {
    const grx_mimi_hparams &hp = m->hp;
    const int d = hp.d;
    auto mat = [&](const std::string &name, MLin *w, int rows, int cols) {
        w->n = rows;
        w->k = cols;
        m->expect.push_back({name, w, nullptr, rows, cols, false});
    };
    auto bias = [&](const std::string &name, MLin *w, int n) { m->expect.push_back({name, w, nullptr, n, 0, true}); };
    auto vec = [&](const std::string &name, float **p, int n) { m->expect.push_back({name, nullptr, p, n, 0, false}); };
    mat("mimi.quant", &m->quant, d, hp.ldim);
    vec("mimi.up", &m->up, d * 2 * hp.upsample);
    m->layers.resize(hp.layers);
    for (int i = 0; i < hp.layers; ++i) {
        const std::string p = "mimi.dec_tf." + std::to_string(i) + ".";
        MLayer &L = m->layers[i];
        vec(p + "norm1.weight", &L.n1w, d);
        vec(p + "norm1.bias", &L.n1b, d);
        vec(p + "norm2.weight", &L.n2w, d);
        vec(p + "norm2.bias", &L.n2b, d);
        mat(p + "attn_qkv.weight", &L.qkv, 3 * d, d);
        mat(p + "attn_out.weight", &L.out, d, d);
        mat(p + "ff1.weight", &L.ff1, hp.ff, d);
        mat(p + "ff2.weight", &L.ff2, d, hp.ff);
        vec(p + "ls1", &L.ls1, d);
        vec(p + "ls2", &L.ls2, d);
    }
    // SEANetDecoder (model.go:163-181)
    int mult = 1 << hp.n_ratios, idx = 1;
    m->steps.reserve((size_t)hp.n_ratios * (hp.n_residual + 1) + 2);
    auto conv = [&](MConv &c, const std::string &name, int cin, int cout, int k, int stride, int dil) {
        c.cin = cin, c.cout = cout, c.k = k, c.stride = stride, c.dil = dil;
        c.past = (k - 1) * dil + 1 - stride;
        mat(name + ".weight", &c.w, cout, k * cin);
        bias(name + ".bias", &c.w, cout);
    };
    {
        MStep s;
        s.kind = 0;
        m->steps.push_back(s);
        conv(m->steps.back().c, "mimi.dec.0", d, mult * hp.n_filters, hp.kernel_size, 1, 1);
    }
    for (int ri = 0; ri < hp.n_ratios; ++ri) {
        const int r = hp.ratios[ri];
        ++idx;
        MStep s;
        s.kind = 1;
        s.elu = 1;
        m->steps.push_back(s);
        MConvTr &t = m->steps.back().t;
        t.cin = mult * hp.n_filters, t.cout = mult * hp.n_filters / 2, t.k = 2 * r, t.stride = r;
        const std::string tn = "mimi.dec." + std::to_string(idx);
        mat(tn + ".weight", &t.w, t.k * t.cout, t.cin);
        vec(tn + ".bias", &t.b, t.cout);
        ++idx;
        const int dim = mult * hp.n_filters / 2;
        int dl = 1;
        for (int j = 0; j < hp.n_residual; ++j) {
            MStep rs;
            rs.kind = 2;
            m->steps.push_back(rs);
            MStep &b = m->steps.back();
            const std::string p = "mimi.dec." + std::to_string(idx) + ".";
            conv(b.a, p + "1", dim, dim / hp.compress, hp.residual_kernel_size, 1, dl);
            conv(b.bb, p + "3", dim / hp.compress, dim, 1, 1, 1);
            dl *= hp.dilation_base;
            ++idx;
        }
        mult /= 2;
    }
    ++idx;
    {
        MStep s;
        s.kind = 0;
        s.elu = 1;
        m->steps.push_back(s);
        conv(m->steps.back().c, "mimi.dec." + std::to_string(idx), hp.n_filters, 1, hp.last_kernel_size, 1, 1);
    }
    m->have.assign(m->expect.size(), false);
    // buffer sizes over the stages of a decode of max_latents
    const int T = hp.max_latents * hp.upsample;
    m->tmax = T;
    size_t act = (size_t)T * d, col = 0, z = (size_t)hp.max_latents * d, h = (size_t)T * d;
    size_t kmax = std::max(std::max(d, hp.ff), hp.ldim);
    int R = T, C = d;
    for (const MStep &s : m->steps) {
        if (s.kind == 0) {
            col = std::max(col, (size_t)(R / s.c.stride) * s.c.k * s.c.cin);
            kmax = std::max(kmax, (size_t)s.c.k * s.c.cin);
            R /= s.c.stride;
            C = s.c.cout;
        } else if (s.kind == 1) {
            z = std::max(z, (size_t)R * s.t.k * s.t.cout);
            kmax = std::max(kmax, (size_t)s.t.cin);
            R *= s.t.stride;
            C = s.t.cout;
        } else {
            col = std::max(col, (size_t)R * s.a.k * s.a.cin);
            h = std::max(h, (size_t)R * s.a.cout);
            kmax = std::max(kmax, (size_t)s.a.k * s.a.cin);
        }
        act = std::max(act, (size_t)R * C);
    }
    m->act_floats = act;
    m->col_floats = col;
    m->z_floats = z;
    m->h_floats = h;
    size_t rows = (size_t)T;
    R = T;
    for (const MStep &s : m->steps) {  // the most rows any product rounds
        if (s.kind == 1) R *= s.t.stride;
        rows = std::max(rows, (size_t)R);
    }
    m->q_bytes = rows * kmax;
    m->spl = R;  // rows of one channel per max_latents; per latent below
    m->spl = hp.upsample;
    for (int ri = 0; ri < hp.n_ratios; ++ri) m->spl *= hp.ratios[ri];
    return GRX_OK;
}

grx_status alloc_state(grx_mimi *m) {
    const grx_mimi_hparams &hp = m->hp;
    const int d = hp.d, half = m->hd / 2;
    grx_status s;
    m->cap = hp.context + m->tmax - 1;
    m->attn_lds = attn_lds(hp);
    if (m->attn_lds > 64 * 1024)
        GRX_HIP(hipFuncSetAttribute((const void *)mimi_attn_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)m->attn_lds));
    for (MLayer &L : m->layers) {
        if ((s = malloc_t(m, (size_t)m->cap * d, &L.kr)) != GRX_OK) return s;
        if ((s = malloc_t(m, (size_t)m->cap * d, &L.vr)) != GRX_OK) return s;
    }
    if ((s = malloc_t(m, (size_t)hp.upsample * d, &m->up_part)) != GRX_OK) return s;
    if ((s = malloc_t(m, 1, &m->posd)) != GRX_OK) return s;
    for (MStep &q : m->steps) {
        for (MConv *c : {&q.c, &q.a, &q.bb})
            if (c->k > 0 && c->past > 0 && (s = malloc_t(m, (size_t)c->past * c->cin, &c->prev)) != GRX_OK) return s;
        if (q.kind == 1 && (s = malloc_t(m, (size_t)(q.t.k - q.t.stride) * q.t.cout, &q.t.partial)) != GRX_OK)
            return s;
    }
    if ((s = malloc_t(m, m->act_floats, &m->x)) != GRX_OK) return s;
    if ((s = malloc_t(m, m->act_floats, &m->y)) != GRX_OK) return s;
    if ((s = malloc_t(m, m->h_floats, &m->h)) != GRX_OK) return s;
    if ((s = malloc_t(m, m->act_floats, &m->o)) != GRX_OK) return s;
    if ((s = malloc_t(m, std::max(m->col_floats, (size_t)1), &m->col)) != GRX_OK) return s;
    if ((s = malloc_t(m, m->z_floats, &m->z)) != GRX_OK) return s;
    if ((s = malloc_t(m, (size_t)m->tmax * 3 * d, &m->qkv)) != GRX_OK) return s;
    if ((s = malloc_t(m, (size_t)m->tmax * d, &m->att)) != GRX_OK) return s;
    if ((s = malloc_t(m, (size_t)m->tmax * hp.ff, &m->f)) != GRX_OK) return s;
    if ((s = malloc_t(m, m->q_bytes, &m->xq)) != GRX_OK) return s;
    if ((s = malloc_t(m, m->q_bytes / GRX_QK + 1, &m->xs)) != GRX_OK) return s;
    if ((s = malloc_t(m, (size_t)2 * m->tmax * half, &m->rope)) != GRX_OK) return s;
    if ((s = malloc_t(m, (size_t)hp.max_latents * hp.ldim, &m->lat)) != GRX_OK) return s;
    if ((s = malloc_t(m, (size_t)hp.max_latents * m->spl, &m->out)) != GRX_OK) return s;
    hipError_t e = grx_pinned_malloc(reinterpret_cast<void **>(&m->rope_host), (size_t)2 * m->tmax * half * 4);
    if (e != hipSuccess) return grx_hip_fail(e, "hipHostMalloc");
    if ((e = hipEventCreateWithFlags(&m->rope_copied, hipEventDisableTiming)) != hipSuccess)
        return grx_hip_fail(e, "hipEventCreate");
    return GRX_OK;
}

grx_status zero_state(grx_mimi *m) {
    hipStream_t st = m->ctx->stream;
    const grx_mimi_hparams &hp = m->hp;
    m->pos = 0;
    GRX_HIP(hipMemsetAsync(m->posd, 0, sizeof(long long), st));
    GRX_HIP(hipMemsetAsync(m->up_part, 0, (size_t)hp.upsample * hp.d * 4, st));
    for (MStep &q : m->steps) {
        for (MConv *c : {&q.c, &q.a, &q.bb})
            if (c->prev) GRX_HIP(hipMemsetAsync(c->prev, 0, (size_t)c->past * c->cin * 4, st));
        if (q.t.partial) GRX_HIP(hipMemsetAsync(q.t.partial, 0, (size_t)(q.t.k - q.t.stride) * q.t.cout * 4, st));
    }
    return GRX_OK;
}

grx_status finalize(grx_mimi *m) {
    grx_status s = alloc_state(m);
    if (s == GRX_OK) s = zero_state(m);
    if (s == GRX_OK) {
        const hipError_t e = hipStreamSynchronize(m->ctx->stream);
        if (e != hipSuccess) s = grx_hip_fail(e, "hipStreamSynchronize");
    }
    if (s != GRX_OK) {
        // back to "every tensor given, nothing allocated": the state's and
        // the work buffers are freed, the weights kept
        std::vector<void *> keep;
        for (void *p : m->allocs) {
            bool weight = false;
            for (const MExpect &e : m->expect)
                if ((e.vec && *e.vec == p) || (e.lin && (e.lin->f == p || e.lin->b == p))) weight = true;
            if (weight) keep.push_back(p);
            else (void)hipFree(p);
        }
        m->allocs = keep;
        if (m->rope_host) (void)hipHostFree(m->rope_host);
        m->rope_host = nullptr;
        if (m->rope_copied) (void)hipEventDestroy(m->rope_copied);
        m->rope_copied = nullptr;
        for (MLayer &L : m->layers) L.kr = L.vr = nullptr;
        for (MStep &q : m->steps) {
            q.c.prev = q.a.prev = q.bb.prev = nullptr;
            q.t.partial = nullptr;
        }
        m->up_part = m->x = m->y = m->h = m->o = m->col = m->z = m->qkv = m->att = m->f = nullptr;
        m->lat = m->out = m->rope = m->xs = nullptr;
        m->xq = nullptr;
        return s;
    }
    m->ready = true;
    return GRX_OK;
}

grx_status check_hp(const grx_mimi_hparams *hp) {
    if (hp->d <= 0 || hp->heads <= 0 || hp->d % hp->heads != 0 || (hp->d / hp->heads) % 2 != 0)
        return grx_fail(GRX_EINVAL, "grx_mimi_create: %d values don't split into %d heads", hp->d, hp->heads);
    if (hp->ff <= 0 || hp->layers < 0 || hp->context < 1 || hp->ldim <= 0 || hp->upsample < 1 || hp->max_latents < 1)
        return grx_fail(GRX_EINVAL, "grx_mimi_create: bad sizes (ff %d, layers %d, context %d, ldim %d, upsample %d, "
                                    "max_latents %d)", hp->ff, hp->layers, hp->context, hp->ldim, hp->upsample,
                        hp->max_latents);
    if (attn_lds(*hp) > kMaxAttnLds)
        return grx_fail(GRX_EINVAL, "grx_mimi_create: %d positions of context and %d latents a call need %zu bytes of "
                                    "LDS (at most %zu)", hp->context, hp->max_latents, attn_lds(*hp), kMaxAttnLds);
    if (hp->n_ratios < 1 || hp->n_ratios > 8)
        return grx_fail(GRX_EINVAL, "grx_mimi_create: %d SEANet ratios", hp->n_ratios);
    for (int i = 0; i < hp->n_ratios; ++i)
        if (hp->ratios[i] < 1 || hp->ratios[i] > 64)
            return grx_fail(GRX_EINVAL, "grx_mimi_create: a SEANet ratio of %d", hp->ratios[i]);
    if (hp->n_filters < 1 || hp->kernel_size < 1 || hp->residual_kernel_size < 1 || hp->last_kernel_size < 1 ||
        hp->dilation_base < 1 || hp->compress < 1 || hp->n_residual < 0)
        return grx_fail(GRX_EINVAL, "grx_mimi_create: bad SEANet settings");
    // the first conv maps d channels (SEANet's dimension is the transformer's)
    long long dil = 1;
    for (int j = 1; j < hp->n_residual; ++j) dil *= hp->dilation_base;
    if ((hp->residual_kernel_size - 1) * dil > kMaxPast || hp->kernel_size - 1 > kMaxPast ||
        hp->last_kernel_size - 1 > kMaxPast)
        return grx_fail(GRX_EINVAL, "grx_mimi_create: a convolution carries more than %d rows", kMaxPast);
    for (int i = 0; i < hp->n_ratios; ++i) {
        const int c = (hp->n_filters << (hp->n_ratios - i)) / 2;
        if (c % hp->compress != 0) return grx_fail(GRX_EINVAL, "grx_mimi_create: %d channels by compress %d", c,
                                                   hp->compress);
    }
    return GRX_OK;
}

}  // namespace

extern "C" grx_status grx_mimi_create(grx_ctx *ctx, const grx_mimi_hparams *hp, grx_mimi **out) {
    if (!ctx || !hp || !out) return grx_fail(GRX_EINVAL, "grx_mimi_create: NULL argument");
    *out = nullptr;
    grx_status s = check_hp(hp);
    if (s != GRX_OK) return s;
    GRX_HIP(hipSetDevice(ctx->device));
    grx_mimi *m = new grx_mimi;
    m->ctx = ctx;
    m->hp = *hp;
    m->hd = hp->d / hp->heads;
    m->freqs.resize(m->hd / 2);
    {  // ropeFreqs (nn.go:69-76)
        const float c = (float)(-log(hp->period) * 2.0 / (double)m->hd);
        for (int i = 0; i < m->hd / 2; ++i) m->freqs[i] = (float)exp((double)((float)i * c));
    }
    build_plan(m);
    *out = m;
    return GRX_OK;
}

extern "C" grx_status grx_mimi_destroy(grx_mimi *m) {
    if (!m) return GRX_OK;
    (void)hipSetDevice(m->ctx->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    release(m);
    delete m;
    return GRX_OK;
}

extern "C" grx_status grx_mimi_set_tensor(grx_mimi *m, const char *name, const void *data, size_t nbytes) {
    if (!m || !name || (!data && nbytes)) return grx_fail(GRX_EINVAL, "grx_mimi_set_tensor: NULL argument");
    if (m->complete) return grx_fail(GRX_ESTATE, "grx_mimi_set_tensor: the decoder is complete already");
    size_t i = 0;
    while (i < m->expect.size() && m->expect[i].name != name) ++i;
    if (i == m->expect.size()) return grx_fail(GRX_EINVAL, "grx_mimi_set_tensor: unknown tensor %s", name);
    if (m->have[i]) return grx_fail(GRX_ESTATE, "grx_mimi_set_tensor: %s given twice", name);
    MExpect &e = m->expect[i];
    GRX_HIP(hipSetDevice(m->ctx->device));
    grx_status s;
    auto upload = [&](float **p, size_t bytes) -> grx_status {
        grx_status r = malloc_dev(m, bytes, reinterpret_cast<void **>(p));
        if (r != GRX_OK) return r;
        const hipError_t he = hipMemcpy(*p, data, bytes, hipMemcpyHostToDevice);
        return he == hipSuccess ? GRX_OK : grx_hip_fail(he, "hipMemcpy");
    };
    if (e.lin && !e.bias) {
        const size_t f32 = (size_t)e.rows * e.cols * 4, q8 = (size_t)e.rows * (e.cols / GRX_QK) * 34;
        if (e.cols % GRX_QK == 0 && nbytes == q8) {
            if ((s = grx_weight_q8_create(m->ctx, e.rows, e.cols, static_cast<const uint8_t *>(data), nbytes,
                                          &e.lin->q)) != GRX_OK)
                return s;
        } else if (nbytes == f32) {
            if ((s = upload(&e.lin->f, f32)) != GRX_OK) return s;
        } else {
            return grx_fail(GRX_ESIZE, "grx_mimi_set_tensor: %s holds %zu bytes, a [%d][%d] matrix is %zu (float32)%s",
                            name, nbytes, e.rows, e.cols, f32, e.cols % GRX_QK == 0 ? " or Q8_0" : "");
        }
        e.lin->have_w = true;
    } else {
        const size_t want = (size_t)e.rows * 4;
        if (nbytes != want)
            return grx_fail(GRX_ESIZE, "grx_mimi_set_tensor: %s holds %zu bytes, %zu wanted", name, nbytes, want);
        if ((s = upload(e.bias ? &e.lin->b : e.vec, want)) != GRX_OK) return s;
    }
    m->have[i] = true;
    for (bool h : m->have)
        if (!h) return GRX_OK;
    m->complete = true;
    return finalize(m);
}

// The decoder's state and work buffers, made once every tensor is given (a
// failed attempt is retried by the next call).
static grx_status ensure_ready(grx_mimi *m, const char *fn) {
    if (m->ready) return GRX_OK;
    if (!m->complete) return grx_fail(GRX_ESTATE, "%s: the decoder is missing tensors", fn);
    return finalize(m);
}

extern "C" grx_status grx_mimi_reset(grx_mimi *m) {
    if (!m) return grx_fail(GRX_EINVAL, "grx_mimi_reset: NULL decoder");
    GRX_HIP(hipSetDevice(m->ctx->device));
    grx_status s = ensure_ready(m, "grx_mimi_reset");
    return s != GRX_OK ? s : zero_state(m);
}

extern "C" int grx_mimi_samples_per_latent(const grx_mimi *m) { return m ? m->spl : 0; }

static grx_status decode_check(grx_mimi *m, const float *lat, int n, float *out, const char *fn) {
    if (!m || (n > 0 && (!lat || !out))) return grx_fail(GRX_EINVAL, "%s: NULL argument", fn);
    if (n < 0 || n > m->hp.max_latents)
        return grx_fail(GRX_ESIZE, "%s: %d latents, at most %d per call", fn, n, m->hp.max_latents);
    GRX_HIP(hipSetDevice(m->ctx->device));
    return ensure_ready(m, fn);
}

// One decode call: the angles on the host, then the call's device work as
// one captured graph (made again when the latent count or the buffers
// change; kernel by kernel with GRX_NO_GRAPH=1 or if capture is refused),
// then the host's position.
static grx_status run_decode(grx_mimi *m, hipStream_t st, const float *lat, int n, float *out) {
    grx_status s = rope_angles(m, n * m->hp.upsample);
    if (s != GRX_OK) return s;
    if (grx_tune(GRX_TUNE_NO_GRAPH) == 1 || m->no_graph) {
        if ((s = enqueue_decode(m, st, lat, n, out)) != GRX_OK) return s;
    } else {
        if (!m->exec || m->g_n != n || m->g_lat != lat || m->g_out != out) {
            if (m->exec) GRX_HIP(hipGraphExecDestroy(m->exec));
            m->exec = nullptr;
            hipGraph_t g = nullptr;
            hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
            if (e == hipSuccess) {
                const grx_status cs = enqueue_decode(m, st, lat, n, out);
                e = hipStreamEndCapture(st, &g);
                if (cs == GRX_OK && e == hipSuccess) e = hipGraphInstantiate(&m->exec, g, nullptr, nullptr, 0);
                if (g) (void)hipGraphDestroy(g);
                if (cs != GRX_OK) return cs;
            }
            if (e != hipSuccess || !m->exec) {  // capture refused: kernel by kernel from now on
                (void)hipGetLastError();
                m->exec = nullptr;
                m->no_graph = true;
                if ((s = enqueue_decode(m, st, lat, n, out)) != GRX_OK) return s;
                GRX_HIP(hipEventRecord(m->rope_copied, st));
                m->pos += (long long)n * m->hp.upsample;
                return GRX_OK;
            }
            m->g_n = n;
            m->g_lat = lat;
            m->g_out = out;
        }
        GRX_HIP(hipGraphLaunch(m->exec, st));
    }
    GRX_HIP(hipEventRecord(m->rope_copied, st));
    m->pos += (long long)n * m->hp.upsample;
    return GRX_OK;
}

extern "C" grx_status grx_mimi_decode_dev(grx_mimi *m, const float *lat, int n, float *out) {
    grx_status s = decode_check(m, lat, n, out, "grx_mimi_decode_dev");
    if (s != GRX_OK || n == 0) return s;
    return run_decode(m, m->ctx->stream, lat, n, out);
}

extern "C" grx_status grx_mimi_decode(grx_mimi *m, const float *lat, int n, float *out) {
    grx_status s = decode_check(m, lat, n, out, "grx_mimi_decode");
    if (s != GRX_OK || n == 0) return s;
    hipStream_t st = m->ctx->stream;
    GRX_HIP(hipMemcpyAsync(m->lat, lat, (size_t)n * m->hp.ldim * 4, hipMemcpyHostToDevice, st));
    if ((s = run_decode(m, st, m->lat, n, m->out)) != GRX_OK) return s;
    GRX_HIP(hipMemcpyAsync(out, m->out, (size_t)n * m->spl * 4, hipMemcpyDeviceToHost, st));
    GRX_HIP(hipStreamSynchronize(st));
    return GRX_OK;
}
