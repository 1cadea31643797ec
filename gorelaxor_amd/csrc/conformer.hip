// conformer.hip - the FastConformer encoder forward (conformer/encoder.go of
// github.com/xattribution/gorelaxor) with Q8_0 weights on one GPU, for a
// batch of utterances of the same frame count.
//
// Every Linear is the int8 route (conformer/model.go:348-356 packs and drops
// the rows of every encoder weight) on the matrix cores (q8_gemm.hip), its
// activations rounded to Q8_0 by the kernel that produces them: the
// LayerNorms, the pre-encoder convolutions, the attention output and the
// depthwise convolution round their rows as they write them, and the first
// feed-forward product rounds its SiLU output in its epilogue.  Residual
// updates happen in the product epilogues.  Everything else - the
// relative-position attention in the float route of MatMulF32, the GLU, the
// depthwise convolution with its folded batch norm - is one kernel each and
// restates the reference's order of operations, so every utterance's output
// is bit-identical to the CPU restatement of encoder.go.
//
// Rows are [utterance][frame][channel]; the whole encode is one HIP graph
// per (batch, frames) shape.
#include <cmath>
#include <cstring>
#include <functional>
#include <map>
#include <string>
#include <vector>

#include "grx_float.h"
#include "grx_internal.h"
#include "grx_ln.h"

namespace {

constexpr int kRowThreads = 256;
constexpr int kAttnQ = 32;        // queries per attention block (encoder.go:211)
constexpr int kAttnThreads = 512;
constexpr int kAttnLdsThreads = 1024;

// encoder.go:33-38 (subOut): a causal pre-encoder pads two before and one
// after, the centred one one on each side; and the valid length after s
// halvings.
__host__ __device__ inline int sub_out(int n, int causal) { return causal ? n / 2 + 1 : (n - 1) / 2 + 1; }
__host__ __device__ inline int stage_len(int valid, int s, int causal) {
    int L = valid;
    for (int i = 0; i < s; ++i) L = sub_out(L, causal);
    return L;
}

// A query's keys [lo, hi), per offlineKeys (encoder.go:196-212) cut at the
// valid length L (encoder.go:465-472), or for a streaming chunk per
// stream.go:273-287.  Queries go in blocks of bl rows, each block's keys
// the union of its rows' ranges.
enum { kKeysAll = 0, kKeysChunked = 1, kKeysWindow = 2, kKeysStream = 3 };
struct AttnKeys {
    int mode, bl;
    int chunk, lchunks;  // chunked and streaming: rows per chunk, chunks of left context
    int left, right;     // window limits; streaming: the left context (rows a stream keeps)
};
// q: the query's key index (a streaming chunk's queries follow its c
// cached keys); T: the keys; L: the valid rows (queries past them see no
// key).  The streaming form is the closed form of the reference's two
// loops: the keys of whole chunks (NeMo's cache slots, key 0 in slot
// left - c) from lchunks chunks before the query's through its own.
__device__ inline void attn_keys(const AttnKeys &k, int q, int T, int L, int c, int &lo, int &hi) {
    if (k.mode == kKeysStream) {
        if (q - c >= L) {
            lo = hi = 0;
            return;
        }
        const int slot0 = k.left - c, qc = (slot0 + q) / k.chunk;
        lo = max(0, (qc - k.lchunks) * k.chunk - slot0);
        hi = min(c + L, (qc + 1) * k.chunk - slot0);
        return;
    }
    if (q >= L) {
        lo = hi = 0;
        return;
    }
    int l = 0, h = T;
    if (k.mode == kKeysChunked) {
        const int cq = q / k.chunk;
        l = max(0, (cq - k.lchunks) * k.chunk);
        h = min(T, (cq + 1) * k.chunk);
    } else if (k.mode == kKeysWindow) {
        l = max(0, q - k.left);
        h = min(T, q + k.right + 1);
    }
    lo = l;
    hi = min(h, L);
}

// Where the attention finds its rows.  Queries of utterance b: q + (b*T +
// t)*ldq.  Keys: K at kv + kvb*b + key*ldkv, V vo floats further; a stream's
// keys start at its ring's head (ctl[1] rows in).  Position rows: pp, rows
// ldp apart, row 0 for relative position Tk-1 (offline), or for maxfirst
// in a streaming table (the rows for Tk-1 found from ctl[0]).
struct AttnIO {
    const float *q;
    int ldq;
    const float *kv;
    int ldkv, vo;
    size_t kvb;
    const float *pp;
    int ldp, maxfirst;
    const int *lens;  // valid rows per utterance
    const int *ctl;   // streaming: [0] cached keys c, [1] ring head; null offline
    int T;            // queries per utterance
};

// Go's builtin max for float32 (NaN wins, +0 over -0).
__device__ inline float go_max(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a == b) return signbit(a) ? b : a;
    return a > b ? a : b;
}

// ---------------------------------------------------------------- pre-encoder

// conv0 then the first depthwise convolution (encoder.go:141-150) in one
// pass: the conv0 outputs a depthwise output needs (3x3 positions, maskRows
// and ReLU applied) are recomputed from the log-mel values instead of being
// written out, which at 256 channels would be 64x the mel's size.  One
// workgroup of c threads (a channel each) per output frame row (b, t2),
// walking its F2 positions with the channel's taps in registers; the mel
// rows 4*t2-3 .. 4*t2+3 (zero outside the plane and past the valid frames)
// are staged in LDS.  Output rows past the stage's valid length are zeroed,
// and each position's c values rounded to Q8_0 for the pointwise Linear
// (or, for a float32 pointwise weight, stored as they are in xf).
// conv0's arithmetic: from the bias, AddScaled of the nonzero taps in order
// (fma for channels of whole groups of eight); the depthwise: from the bias,
// w*x unfused over the taps in range.
__global__ void sub_conv01_kernel(const float *__restrict__ mel, int frames, int nm, const int *__restrict__ valid,
                                  int causal, const float *__restrict__ w0, const float *__restrict__ b0,
                                  const float *__restrict__ w2, const float *__restrict__ b2, int c, int T1, int F1,
                                  int T2, int F2, int8_t *__restrict__ xq, float *__restrict__ xs,
                                  float *__restrict__ xf) {
    extern __shared__ float patch[];  // [7][4*F2 + 3], column q = mel column q - 3*pl
    const int ch = threadIdx.x, t2 = blockIdx.x % T2, b = blockIdx.x / T2;
    const int W = 4 * F2 + 3, pl = causal ? 2 : 1;  // the padding before
    const int vb = valid[b], tv = min(frames, vb);
    const int L1 = stage_len(vb, 1, causal), L2 = stage_len(vb, 2, causal);
    for (int e = ch; e < 7 * W; e += blockDim.x) {
        const int r = e / W, q = e % W, ti = 4 * t2 - 3 * pl + r, fi = q - 3 * pl;
        patch[e] = (ti >= 0 && ti < tv && fi >= 0 && fi < nm) ? mel[((size_t)b * nm + fi) * frames + ti] : 0.f;
    }
    __syncthreads();
    float w0v[9], w2v[9];
#pragma unroll
    for (int j = 0; j < 9; ++j) {
        w0v[j] = w0[j * c + ch];
        w2v[j] = w2[j * c + ch];
    }
    const float bias0 = b0[ch], bias2 = b2[ch];
    const bool fm = ch < (c & ~7);
    // the conv0 outputs of column kf = 2 of a position are column kf = 0 of
    // the next one (conv0 position 2 f2 + 2 - pl): carried, not formed twice
    float carry[3] = {0.f, 0.f, 0.f};
    for (int f2 = 0; f2 < F2; ++f2) {
        float o = 0.f;
        if (t2 < L2) {
            // the 7x7 mel values of this position: patch columns 4f2 .. 4f2+6,
            // rows and columns 4t2-3pl.., 4f2-3pl.. of the plane (columns 0
            // and 1 feed only column kf = 0, carried past the first position)
            float pv[7][7];
#pragma unroll
            for (int r = 0; r < 7; ++r)
#pragma unroll
                for (int q = 2; q < 7; ++q) pv[r][q] = patch[r * W + 4 * f2 + q];
            if (f2 == 0) {
#pragma unroll
                for (int r = 0; r < 7; ++r)
#pragma unroll
                    for (int q = 0; q < 2; ++q) pv[r][q] = patch[r * W + q];
            }
            o = bias2;
            float next[3];
#pragma unroll
            for (int j2 = 0; j2 < 9; ++j2) {
                const int kt = j2 / 3, kf = j2 % 3;
                const int ti = 2 * t2 + kt - pl, fi = 2 * f2 + kf - pl;  // conv0 output position
                const bool in = !(ti < 0 || ti >= T1 || fi < 0 || fi >= F1);
                float x = 0.f;
                if (kf == 0 && f2 > 0) {
                    x = carry[kt];
                } else if (in && ti < L1) {
                    float a = bias0;
#pragma unroll
                    for (int j = 0; j < 9; ++j) {
                        // mel (2ti + j/3 - pl, 2fi + j%3 - pl) = pv[2kt + j/3][2kf + j%3]; zero taps
                        // are skipped (a select, not a branch)
                        const float v = pv[2 * kt + j / 3][2 * kf + j % 3];
                        const float t = fm ? __fmaf_rn(v, w0v[j], a) : __fadd_rn(a, __fmul_rn(v, w0v[j]));
                        a = v != 0.f ? t : a;
                    }
                    x = a < 0.f ? 0.f : a;
                }
                if (kf == 2) next[kt] = x;
                if (!in) continue;
                o = __fadd_rn(o, __fmul_rn(w2v[j2], x));
            }
#pragma unroll
            for (int kt = 0; kt < 3; ++kt) carry[kt] = next[kt];
        }
        const size_t p = ((size_t)b * T2 + t2) * F2 + f2;
        if (xf)
            xf[p * c + ch] = o;
        else
            quant32_store(o, xq + p * c + ch, xs + p * (c / 32) + ch / 32, ch & 31);
    }
}

// dwConv2 (encoder.go:80-110) at halving s (input [b][T][F][c], one
// workgroup of c threads per output position), rows from the stage's valid
// length on zeroed, rounded to Q8_0 for the pointwise Linear that follows
// (row (b, t1, f1) of c values), or stored as they are in xf for a float32
// pointwise weight.  RELU_IN: the input is the previous
// pointwise output, read through maskRows and ReLU (encoder.go:152-153).
template <bool RELU_IN>
__global__ void sub_dwconv_kernel(const float *__restrict__ in, int T, int F, int c, const int *__restrict__ valid,
                                  int causal, int s, const float *__restrict__ w, const float *__restrict__ bias,
                                  int T1, int F1, int8_t *__restrict__ xq, float *__restrict__ xs,
                                  float *__restrict__ xf) {
    const int p = blockIdx.x, ch = threadIdx.x;
    const int f1 = p % F1, t1 = (p / F1) % T1, b = p / (F1 * T1);
    const int vb = valid[b], pl = causal ? 2 : 1;
    const int Lin = stage_len(vb, s - 1, causal), Lout = stage_len(vb, s, causal);
    float o = 0.f;
    if (t1 < Lout) {
        float xv[9], wv[9];
        bool ok[9];
#pragma unroll
        for (int j = 0; j < 9; ++j) {
            const int ti = 2 * t1 + j / 3 - pl, fi = 2 * f1 + j % 3 - pl;
            ok[j] = ti >= 0 && ti < T && fi >= 0 && fi < F;  // taps outside the plane are skipped
            // the load is issued at a clamped address and the value chosen
            // afterwards, so the nine loads stay in flight together
            const int tc = min(max(ti, 0), T - 1), fc = min(max(fi, 0), F - 1);
            float x = in[(((size_t)b * T + tc) * F + fc) * c + ch];
            x = ok[j] ? x : 0.f;
            if constexpr (RELU_IN) x = ti < Lin ? (x < 0.f ? 0.f : x) : 0.f;
            xv[j] = x;
            wv[j] = w[j * c + ch];
        }
        o = bias[ch];
#pragma unroll
        for (int j = 0; j < 9; ++j)
            if (ok[j]) o = __fadd_rn(o, __fmul_rn(wv[j], xv[j]));
    }
    if (xf)
        xf[(size_t)p * c + ch] = o;
    else
        quant32_store(o, xq + (size_t)p * c + ch, xs + (size_t)p * (c / 32) + ch / 32, ch & 31);
}

// The last pointwise output through maskRows and ReLU, flattened [t][c*F+f]
// (encoder.go:158-166) and rounded to Q8_0 for the output Linear: one
// workgroup per kept (utterance, frame): frames drop.. of each utterance's
// T (a streaming chunk's first rows are dropped, stream.go:255-258), Tp of
// them, to rows b*Tp + t - drop.
__global__ void sub_flatten_kernel(const float *__restrict__ y, int T, int F, int c, const int *__restrict__ valid,
                                   int causal, int drop, int Tp, int8_t *__restrict__ xq, float *__restrict__ xs) {
    const int row = blockIdx.x, b = row / Tp, t = row % Tp + drop;
    const int L = stage_len(valid[b], 3, causal);
    const int K = c * F;
    const size_t src = (size_t)b * T + t;
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
        const int ch = i / F, f = i % F;
        const float v = y[(src * F + f) * c + ch];
        const float r = t < L ? (v < 0.f ? 0.f : v) : 0.f;
        quant32_store(r, xq + (size_t)row * K + i, xs + (size_t)row * (K / 32) + i / 32, i & 31);
    }
}

// ---------------------------------------------------------------- LayerNorm rows

// kern.LayerNorm of one row (internal/kern/mathx.go:55-75) held in LDS:
// float64 sums with the reference's results (ln32_stats), mean and inv
// rounded to float32, y = (v-mean)*inv*w + b rounded step by step.  The
// caller has the whole row in LDS (a barrier after writing it).
__device__ void ln_row(float *v, int n, const float *w, const float *bb, double *red) {
    const int tid = threadIdx.x;
    float mean, inv;
    ln32_stats(v, n, red, mean, inv);
    for (int i = tid; i < n; i += blockDim.x) {
        float t = __fsub_rn(v[i], mean);
        t = __fmul_rn(t, inv);
        t = __fmul_rn(t, w[i]);
        v[i] = __fadd_rn(t, bb[i]);
    }
    __syncthreads();
}

// ln_rows_kernel's work with one wave per row (no workgroup barrier): the
// row as NP float4 pieces per lane (piece P = 64 j + lane, n <= 256 NP),
// kern.LayerNorm by wave_ln32 (DPP sums with the in-order check), and the
// rounding of each 32-value block (8 pieces in 8 consecutive lanes) by
// xor-shuffle maxima.
template <bool OUT, bool Q, int NP>
__global__ __launch_bounds__(64) void ln_rows_wave_kernel(float *__restrict__ x, int n, const float *__restrict__ w1,
                                                          const float *__restrict__ b1, const float *__restrict__ w2,
                                                          const float *__restrict__ b2, int8_t *__restrict__ xq,
                                                          float *__restrict__ xs) {
    const int r = blockIdx.x, lane = threadIdx.x, npc = n / 4;
    float4 *x4 = reinterpret_cast<float4 *>(x + (size_t)r * n);
    float4 xv[NP], wv[NP], bv[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const int P = min(j * 64 + lane, npc - 1);
        xv[j] = x4[P];
        wv[j] = reinterpret_cast<const float4 *>(w1)[P];
        bv[j] = reinterpret_cast<const float4 *>(b1)[P];
    }
    wave_ln32<NP>(xv, wv, bv, npc, lane);
    if constexpr (OUT) {
#pragma unroll
        for (int j = 0; j < NP; ++j)
            if (j * 64 + lane < npc) x4[j * 64 + lane] = xv[j];
        if constexpr (Q) {
#pragma unroll
            for (int j = 0; j < NP; ++j) {
                const int P = min(j * 64 + lane, npc - 1);
                wv[j] = reinterpret_cast<const float4 *>(w2)[P];
                bv[j] = reinterpret_cast<const float4 *>(b2)[P];
            }
            wave_ln32<NP>(xv, wv, bv, npc, lane);
        }
    }
    if constexpr (Q) {
        // quantU8 of block b = pieces 8b..8b+7 (n % 32 == 0)
#pragma unroll
        for (int j = 0; j < NP; ++j) {
            const float4 v = xv[j];
            float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
            for (int o = 4; o > 0; o >>= 1) {
                const float t = __shfl_xor(amax, o, 8);
                amax = t > amax ? t : amax;
            }
            const int P = j * 64 + lane;
            if (P >= npc) continue;
            const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
            auto q1 = [&](float f) {
                float t = rintf(__fmul_rn(f, id));
                t = fminf(fmaxf(t, -128.0f), 127.0f);
                return (uint32_t)(uint8_t)(int8_t)(int)t;
            };
            const uint32_t pk = q1(v.x) | q1(v.y) << 8 | q1(v.z) << 16 | q1(v.w) << 24;
            *reinterpret_cast<uint32_t *>(xq + (size_t)r * n + 4 * P) = pk;
            if ((P & 7) == 0) xs[(size_t)r * (n / 32) + P / 8] = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
        }
    }
}

// One workgroup per row of x [rows][n].  OUT: x = LN(x; w1, b1) written
// back first (a block's norm_out, encoder.go:426).  Q: the row (after OUT,
// LN(x; w2, b2)) rounded to Q8_0 into xq [rows][n], xs [rows][n/32].
template <bool OUT, bool Q>
__global__ __launch_bounds__(kRowThreads) void ln_rows_kernel(float *__restrict__ x, int n,
                                                              const float *__restrict__ w1,
                                                              const float *__restrict__ b1,
                                                              const float *__restrict__ w2,
                                                              const float *__restrict__ b2,
                                                              int8_t *__restrict__ xq, float *__restrict__ xs) {
    extern __shared__ __align__(16) float row[];
    __shared__ double red[48];  // ln_block_reduce
    const int r = blockIdx.x, tid = threadIdx.x;
    float *xr = x + (size_t)r * n;
    for (int i = tid; i < n / 4; i += blockDim.x)  // n % 32 == 0
        reinterpret_cast<float4 *>(row)[i] = reinterpret_cast<const float4 *>(xr)[i];
    __syncthreads();
    ln_row(row, n, w1, b1, red);
    if constexpr (OUT) {
        for (int i = tid; i < n; i += blockDim.x) xr[i] = row[i];
        if constexpr (Q) ln_row(row, n, w2, b2, red);
    }
    if constexpr (Q) {
        // n % 32 == 0 and the stride is a multiple of 32: whole blocks per 32 lanes
        for (int i = tid; i < n; i += blockDim.x)
            quant32_store(row[i], xq + (size_t)r * n + i, xs + (size_t)r * (n / 32) + i / 32, i & 31);
    }
}

// ---------------------------------------------------------------- attention

// The keys [k0, k1) of a block of queries q0..q1-1 (key indices qoff+q):
// the union of its rows' ranges (encoder.go:285-289).
// The union of the ranges of block rows q0..q1-1: the rows that see keys
// are a prefix of the block (those before the valid length), whose ranges'
// ends never decrease with the row, so the first gives the start and the
// last the end; a row that sees none counts as [0, 0), as a loop over the
// rows taking min(lo) and max(hi) from k0 = Tk, k1 = 0 would have it.
__device__ inline void block_keys(const AttnKeys &ak, int q0, int q1, int qoff, int Tk, int L, int c, int &k0,
                                  int &k1) {
    const int lim = (ak.mode == kKeysStream ? c + L : L) - qoff;  // rows q < lim see keys
    const int qv = min(q1, max(q0, lim));
    k0 = Tk;
    k1 = 0;
    if (qv > q0) {
        int lo, hi;
        attn_keys(ak, qoff + q0, Tk, L, c, lo, hi);
        k0 = lo;
        attn_keys(ak, qoff + qv - 1, Tk, L, c, lo, hi);
        k1 = hi;
    }
    if (qv < q1) {
        k0 = min(k0, 0);
        k1 = max(k1, 0);
    }
}

// A stream's cached keys and ring head (0 offline), the keys' first row
// and the position rows for relative position Tk-1.
struct AttnRows {
    int c, Tk;
    const float *kv, *pp;
};
__device__ inline AttnRows attn_rows(const AttnIO &io, int b) {
    AttnRows r;
    r.c = io.ctl ? io.ctl[0] : 0;
    const int head = io.ctl ? io.ctl[1] : 0;
    r.Tk = r.c + io.T;
    r.kv = io.kv + io.kvb * b + (size_t)head * io.ldkv;
    r.pp = io.ctl ? io.pp + (size_t)(io.maxfirst - (r.Tk - 1)) * io.ldp : io.pp;
    return r;
}

// Relative-position multi-head self-attention (encoder.go:259-330) of one
// (utterance, head, block of bl queries): the block's keys [k0, k1) (the
// union of its rows' ranges), qu = q + pos_u and qv = q + pos_v in float32;
// scores = MatMulF32(qu, k) and bd = MatMulF32(qv, pp rows jlo..), each in
// the route MatMulF32 takes for nq rows; row i adds bd shifted by nq-1-i,
// scales, keeps its own keys [lo, hi) (-inf outside), softmax by
// ExpSub/Scale; the output MatMulF32(p, v^T) is rounded to Q8_0 per 32
// values of the head's slice for the out Linear.
__global__ __launch_bounds__(kAttnThreads) void conf_attn_kernel(const AttnIO io, const AttnKeys ak,
                                                                 const float *__restrict__ pos_u,
                                                                 const float *__restrict__ pos_v, int D, int hd,
                                                                 float scale, int8_t *__restrict__ xq,
                                                                 float *__restrict__ xs) {
    extern __shared__ float sm[];
    const int blk = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, nt = blockDim.x;
    const int T = io.T, L = io.lens[b];
    const AttnRows ar = attn_rows(io, b);
    const int c = ar.c, Tk = ar.Tk, qoff = Tk - T;
    const int q0 = blk * ak.bl, q1 = min(T, q0 + ak.bl), nq = q1 - q0;
    int k0, k1;
    block_keys(ak, q0, q1, qoff, Tk, L, c, k0, k1);
    const int nk = k1 - k0;
    const float *qb = io.q + (size_t)b * T * io.ldq;
    const int nqb = hd / 32;
    if (nk <= 0) {  // encoder.go:290-293: the block's output rows are zero
        for (int g = tid >> 5; g < nq * nqb; g += nt >> 5) {
            const int i = g / nqb, bb = g % nqb;
            const size_t row = (size_t)b * T + q0 + i;
            quant32_store(0.f, xq + row * D + h * hd + bb * 32 + (tid & 31), xs + row * (D / 32) + (h * hd) / 32 + bb,
                          tid & 31);
        }
        return;
    }
    const int np = nq + nk - 1, jlo = Tk - 1 - (qoff + q1 - 1) + k0;
    const int sq = hd + 1, sS = nk | 1, sB = np | 1;
    float *qu = sm, *qv = sm + kAttnQ * sq, *S = qv + kAttnQ * sq, *BD = S + kAttnQ * sS;
    float *rmx = BD + kAttnQ * sB, *rinv = rmx + kAttnQ;
    const float *kb = ar.kv + (size_t)k0 * io.ldkv;
    for (int e = tid; e < nq * hd; e += nt) {
        const int i = e / hd, j = e % hd;
        const float q = qb[(size_t)(q0 + i) * io.ldq + h * hd + j];
        qu[i * sq + j] = __fadd_rn(q, pos_u[h * hd + j]);
        qv[i * sq + j] = __fadd_rn(q, pos_v[h * hd + j]);
    }
    __syncthreads();
    for (int e = tid; e < nq * nk; e += nt) {
        const int i = e % nq, kk = e / nq;
        S[i * sS + kk] = matmul_f32_one(qu + i * sq, kb + (size_t)kk * io.ldkv + h * hd, 1, hd, i, nq, kk, nk);
    }
    for (int e = tid; e < nq * np; e += nt) {
        const int i = e % nq, jj = e / nq;
        BD[i * sB + jj] =
            matmul_f32_one(qv + i * sq, ar.pp + (size_t)(jlo + jj) * io.ldp + h * hd, 1, hd, i, nq, jj, np);
    }
    __syncthreads();
    // the scores of row i: (s + bd[i][nq-1-i+kk]) * scale inside [lo, hi),
    // -inf outside; the row maximum by one wave per row
    const int lane = tid & 63, wave = tid >> 6, nw = nt >> 6;
    for (int i = wave; i < nq; i += nw) {
        int lo, hi;
        attn_keys(ak, qoff + q0 + i, Tk, L, c, lo, hi);
        float mx = -__builtin_inff();
        for (int kk = lane; kk < nk; kk += 64) {
            const int kx = k0 + kk;
            float v;
            if (kx < lo || kx >= hi) {
                v = -__builtin_inff();
            } else {
                v = __fmul_rn(__fadd_rn(S[i * sS + kk], BD[i * sB + nq - 1 - i + kk]), scale);
                mx = go_max(mx, v);
            }
            S[i * sS + kk] = v;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = go_max(mx, __shfl_xor(mx, o));
        if (lane == 0) rmx[i] = mx;
    }
    __syncthreads();
    // ExpSub: EXP8 below nk &^ 7, the scalar expf past it; rows whose
    // maximum is -inf are cleared instead (encoder.go:312-315)
    const int n8 = nk & ~7;
    for (int e = tid; e < nq * nk; e += nt) {
        const int i = e / nk, kk = e % nk;
        const float mx = rmx[i];
        float &v = S[i * sS + kk];
        if (mx == -__builtin_inff())
            v = 0.f;
        else {
            const float d = __fsub_rn(v, mx);
            v = kk < n8 ? grx_exp8(d) : grx_expf_go(d);
        }
    }
    __syncthreads();
    // the eight lane sums of expSubAVX, HSUM, plus the tail's own sum; one
    // wave per row, lanes 0..7 a lane sum each, lane 8 the tail
    for (int i = wave; i < nq; i += nw) {
        float acc = 0.f;
        if (lane < 8) {
            for (int kk = lane; kk < n8; kk += 8) acc = __fadd_rn(acc, S[i * sS + kk]);
        } else if (lane == 8) {
            for (int kk = n8; kk < nk; ++kk) acc = __fadd_rn(acc, S[i * sS + kk]);
        }
        float a8[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) a8[l] = __shfl(acc, l);
        const float tail = __shfl(acc, 8);
        if (lane == 0) {
            const float sa = n8 > 0 ? hsum8(a8) : 0.f;
            rinv[i] = __fdiv_rn(1.0f, __fadd_rn(sa, tail));
        }
    }
    __syncthreads();
    for (int e = tid; e < nq * nk; e += nt) {
        const int i = e / nk, kk = e % nk;
        if (rmx[i] != -__builtin_inff()) S[i * sS + kk] = __fmul_rn(S[i * sS + kk], rinv[i]);
    }
    __syncthreads();
    // out = MatMulF32(p, v^T): m = nq, n = hd, k = nk; v^T's row e is the
    // value column e (elements ldkv apart)
    float *O = qu;  // [nq][sq], qu is no longer needed
    for (int e = tid; e < nq * hd; e += nt) {
        const int i = e % nq, ee = e / nq;
        O[i * sq + ee] = matmul_f32_one(S + i * sS, kb + io.vo + h * hd + ee, io.ldkv, nk, i, nq, ee, hd);
    }
    __syncthreads();
    for (int g = tid >> 5; g < nq * nqb; g += nt >> 5) {
        const int i = g / nqb, bb = g % nqb, e = tid & 31;
        const size_t row = (size_t)b * T + q0 + i;
        quant32_store(O[i * sq + bb * 32 + e], xq + row * D + h * hd + bb * 32 + e,
                      xs + row * (D / 32) + (h * hd) / 32 + bb, e);
    }
}

// rows x cols floats (cols % 4 == 0, source rows 16-byte aligned) from
// global memory (rows ssrc floats apart) into LDS (rows sdst apart), every
// thread keeping four 16-byte loads in flight.
// One float4 into LDS at d: a 16-byte store when the rows are 16-byte
// aligned (stride a multiple of four floats), else four 4-byte ones.
__device__ __forceinline__ void put_f4(float *d, bool a16, const float4 &v) {
    if (a16) {
        *reinterpret_cast<float4 *>(d) = v;
    } else {
        d[0] = v.x;
        d[1] = v.y;
        d[2] = v.z;
        d[3] = v.w;
    }
}

// f(row, col) with row(e), col(e) the row and float4 column of element e
// of rows of cols/4 float4s: a shift and a mask where that is a power of
// two (the usual head widths), else a division (the choice is uniform, so
// only one form runs).
template <class F>
__device__ __forceinline__ void by_rows(int cols, F f) {
    const int c4 = cols >> 2;
    if ((c4 & (c4 - 1)) == 0) {
        const int sh = __builtin_ctz(c4);
        f([=](int e) { return e >> sh; }, [=](int e) { return e & (c4 - 1); });
    } else {
        f([=](int e) { return e / c4; }, [=](int e) { return e % c4; });
    }
}

__device__ __forceinline__ void stage_f4(float *dst, int sdst, const float *src, size_t ssrc, int rows, int cols) {
    const int n = rows * (cols >> 2), nt = blockDim.x;
    const bool a16 = (sdst & 3) == 0;
    by_rows(cols, [&](auto row, auto col) {
        for (int e0 = threadIdx.x; e0 < n; e0 += 4 * nt) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {  // clamped: the four loads stay in flight together
                const int e = min(e0 + u * nt, n - 1);
                v[u] = *reinterpret_cast<const float4 *>(src + (size_t)row(e) * ssrc + 4 * col(e));
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int e = e0 + u * nt;
                if (e < n) put_f4(dst + row(e) * sdst + 4 * col(e), a16, v[u]);
            }
        }
    });
}

// stage_f4 in two halves: the loads of the first U float4s a thread takes
// (issued early, held in registers while other work runs), then their
// stores and the rest of the rows.
template <int U>
__device__ __forceinline__ void stage_pre(float4 (&v)[U], const float *src, size_t ssrc, int rows, int cols) {
    const int n = rows * (cols >> 2), nt = blockDim.x;
    by_rows(cols, [&](auto row, auto col) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int e = min((int)threadIdx.x + u * nt, n - 1);
            v[u] = *reinterpret_cast<const float4 *>(src + (size_t)row(e) * ssrc + 4 * col(e));
        }
    });
}
template <int U>
__device__ __forceinline__ void stage_post(float *dst, int sdst, const float4 (&v)[U], const float *src, size_t ssrc,
                                           int rows, int cols) {
    const int n = rows * (cols >> 2), nt = blockDim.x;
    const bool a16 = (sdst & 3) == 0;
    by_rows(cols, [&](auto row, auto col) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int e = threadIdx.x + u * nt;
            if (e < n) put_f4(dst + row(e) * sdst + 4 * col(e), a16, v[u]);
        }
        for (int e = threadIdx.x + U * nt; e < n; e += nt)
            put_f4(dst + row(e) * sdst + 4 * col(e), a16,
                   *reinterpret_cast<const float4 *>(src + (size_t)row(e) * ssrc + 4 * col(e)));
    });
}

// MatMulF32's 6x16 panel route (kernels_amd64.s:5-88) for R rows a_j
// (16-byte aligned, rows sa floats apart) against one operand b, reading
// four k at a time with 16-byte LDS reads: out_j = sum over k chunks of 256
// of (fma chain over the chunk, in k order), each chunk's chain added to
// the running result from 0.  BS: b is 16-byte aligned and contiguous (one
// 16-byte read per four k), else its elements are sb apart (four reads).
// A tail of k % 4 (a chunk's end) reads one element at a time.
template <int R, bool BS>
__device__ __forceinline__ void panel_v4(const float *a, int sa, const float *b, size_t sb, int k, float out[R]) {
    float c[R];
#pragma unroll
    for (int j = 0; j < R; ++j) c[j] = 0.f;
    for (int k0 = 0; k0 < k; k0 += 256) {
        const int kn = min(256, k - k0), k4 = kn & ~3;
        float acc[R];
#pragma unroll
        for (int j = 0; j < R; ++j) acc[j] = 0.f;
        auto step = [&](int kk) {
            float4 bv;
            if constexpr (BS) {
                bv = *reinterpret_cast<const float4 *>(b + k0 + kk);
            } else {
                bv.x = b[(size_t)(k0 + kk) * sb];
                bv.y = b[(size_t)(k0 + kk + 1) * sb];
                bv.z = b[(size_t)(k0 + kk + 2) * sb];
                bv.w = b[(size_t)(k0 + kk + 3) * sb];
            }
#pragma unroll
            for (int j = 0; j < R; ++j) {
                const float4 av = *reinterpret_cast<const float4 *>(a + (size_t)j * sa + k0 + kk);
                acc[j] = __fmaf_rn(av.x, bv.x, acc[j]);
                acc[j] = __fmaf_rn(av.y, bv.y, acc[j]);
                acc[j] = __fmaf_rn(av.z, bv.z, acc[j]);
                acc[j] = __fmaf_rn(av.w, bv.w, acc[j]);
            }
        };
        // (one chain: eight steps' reads in flight; four chains: two, for
        // the registers)
        if constexpr (R == 1) {
#pragma unroll 8
            for (int kk = 0; kk < k4; kk += 4) step(kk);
        } else {
#pragma unroll 2
            for (int kk = 0; kk < k4; kk += 4) step(kk);
        }
        for (int kk = k4; kk < kn; ++kk) {
            const float bx = BS ? b[k0 + kk] : b[(size_t)(k0 + kk) * sb];
#pragma unroll
            for (int j = 0; j < R; ++j) acc[j] = __fmaf_rn(a[(size_t)j * sa + k0 + kk], bx, acc[j]);
        }
#pragma unroll
        for (int j = 0; j < R; ++j) c[j] = __fadd_rn(acc[j], c[j]);
    }
#pragma unroll
    for (int j = 0; j < R; ++j) out[j] = c[j];
}

// One output of MatMulF32 (matmul_f32_one's routes) with a 16-byte aligned
// a: the panel route through panel_v4, the gemvRows route as before.
template <bool BS>
__device__ __forceinline__ float matmul_f32_one_v4(const float *a, const float *b, size_t sb, int k, int r, int m, int j,
                                                   int n) {
    if (m > 16 && r < m / 6 * 6) {
        float o[1];
        panel_v4<1, BS>(a, 0, b, sb, k, o);
        return o[0];
    }
    return matmul_f32_one(a, b, sb, k, r, m, j, n);
}

// Four outputs of MatMulF32's 6x16 panel route (kernels_amd64.s:5-88) at
// once: out_j = sum over k chunks of 256 of (fma chain over the chunk),
// each chunk's chain added to the running result; a(j, k) and b(j, k) give
// output j's operands.  The four chains are independent, so their loads
// and FMAs interleave.
template <class FA, class FB>
__device__ __forceinline__ void packed4(const FA &a, const FB &b, int k, float out[4]) {
    float c[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < k; k0 += 256) {
        const int kn = min(256, k - k0);
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
        for (int kk = 0; kk < kn; ++kk) {
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = __fmaf_rn(a(j, k0 + kk), b(j, k0 + kk), acc[j]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) c[j] = __fadd_rn(acc[j], c[j]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = c[j];
}

// The same attention with the head's keys, the rows of the position table
// the block uses and the values staged in LDS, for RQ of the block's query
// rows per workgroup (rows r0.. of block blk; the route of each product is
// still chosen by the row's index in its block and by the block's full
// column counts).  Only the band of bd that the rows use is computed:
// bd[i][nq-1-i+kk] for the nk keys.
// The (piece, head, utterance) of a workgroup of a (pieces, heads, B)
// launch such that one head's workgroups share an XCD: workgroup L of the
// launch runs on XCD L % 8, so XCD x takes the x-th eighth of the list in
// (utterance, head, piece) order, and a head's keys, position rows and
// values come into that XCD's L2 once rather than into all eight.
__device__ __forceinline__ void attn_wg_xcd(int &px, int &h, int &b) {
    const int nx = gridDim.x, ny = gridDim.y, n = nx * ny * gridDim.z;
    const int l = blockIdx.x + nx * (blockIdx.y + ny * blockIdx.z);
    const int w = n % 8 == 0 ? (l % 8) * (n / 8) + l / 8 : l;
    px = w % nx;
    h = (w / nx) % ny;
    b = w / (nx * ny);
}

// G8: blocks of at most 16 rows (every output on the gemvRows route) whose
// scores and outputs fit one round of 8-lane groups (one row of up to 128
// keys and 128 values: a streaming chunk step of one row), each output by
// a group of 8 lanes (dot8_s: the same sums in the same order; the
// single-thread chains measured 1.9 us for a row's 71 scores, the groups
// 0.8); the host picks it.
template <int RQ, bool G8 = false>
__global__ __launch_bounds__(kAttnLdsThreads) void conf_attn_lds_kernel(const AttnIO io, const AttnKeys ak,
                                                                        const float *__restrict__ pos_u,
                                                                        const float *__restrict__ pos_v, int D,
                                                                        int hd, float scale,
                                                                        int8_t *__restrict__ xq,
                                                                        float *__restrict__ xs) {
    extern __shared__ __align__(16) float sm[];
    const int pieces = (ak.bl + RQ - 1) / RQ;
    int px, h, b;
    attn_wg_xcd(px, h, b);
    const int blk = px / pieces, r0 = (px % pieces) * RQ;
    const int tid = threadIdx.x, nt = blockDim.x;
    const int T = io.T;
    const int q0 = blk * ak.bl, q1 = min(T, q0 + ak.bl), nq = q1 - q0;
    if (r0 >= nq) return;
    const int nr = min(RQ, nq - r0);  // rows r0 .. r0+nr-1 of the block
    // the query rows' loads first: they wait for nothing (the keys' rows
    // wait for the stream's ring head)
    const float *qb = io.q + (size_t)b * T * io.ldq;
    const float *qsrc = qb + (size_t)(q0 + r0) * io.ldq + h * hd;
    float4 qv4[1];
    stage_pre(qv4, qsrc, io.ldq, nr, hd);
    const int L = io.lens[b];
    const AttnRows ar = attn_rows(io, b);
    const int c = ar.c, Tk = ar.Tk, qoff = Tk - T;
    int k0, k1;
    block_keys(ak, q0, q1, qoff, Tk, L, c, k0, k1);
    const int nk = k1 - k0;
    const int nqb = hd / 32;
    if (nk <= 0) {
        for (int g = tid >> 5; g < nr * nqb; g += nt >> 5) {
            const int i = g / nqb, bb = g % nqb;
            const size_t row = (size_t)b * T + q0 + r0 + i;
            quant32_store(0.f, xq + row * D + h * hd + bb * 32 + (tid & 31), xs + row * (D / 32) + (h * hd) / 32 + bb,
                          tid & 31);
        }
        return;
    }
    const int np = nq + nk - 1, jlo = Tk - 1 - (qoff + q1 - 1) + k0;
    // rows below pf (index in the block) take the panel route: whole groups
    // of four of them run four chains per thread; every other output (the
    // gemvRows rows, a last partial group) is a task of its own
    // (a workgroup with fewer groups than it has threads for one chain
    // each runs every output as a task of its own: four times the chains at
    // once, the same bits)
    const int pf = nq > 16 ? nq / 6 * 6 : 0;
    const int pr = r0 < pf ? min(nr, pf - r0) : 0, ng0 = pr / 4;
    const int ng = 4 * ng0 * nk > nt ? ng0 : 0, r1 = 4 * ng;
    // on the panel route (blocks of more than 16 rows) with groups, or with
    // more single-chain tasks than threads, rows 16-byte aligned: the chains
    // read four floats at once, sq = hd + 4 spreading a row per lane's 16-byte
    // reads over the banks; otherwise (the gemvRows route, or a task per
    // thread, measured faster so) one float at a time, spread by an odd stride
    const bool v4 = nq > 16 && (ng > 0 || nr * nk > nt);
    const int sq = v4 ? hd + 4 : hd + 1, sS = v4 ? (nk + 3) & ~3 : nk | 1;
    float *qu = sm, *qv = qu + RQ * sq, *S = qv + RQ * sq, *BD = S + RQ * sS, *rmx = BD + RQ * sS,
          *rinv = rmx + RQ, *st = rinv + RQ;
    const float *kb = ar.kv + (size_t)k0 * io.ldkv;
    // position rows jlo + nq-1-(r0+i) + kk: from pb = jlo + nq-1-(r0+nr-1) on, nk + nr - 1 of them
    const int pb = jlo + nq - 1 - (r0 + nr - 1), npr = nk + nr - 1;
    const float *pp = ar.pp + (size_t)pb * io.ldp + h * hd, *vp = kb + io.vo + h * hd;
    // the keys k0.. of the head (rows sq apart in LDS), and the position
    // rows' and the values' loads, all in flight with the query rows' (the
    // position rows and values go to LDS once the keys, then the position
    // rows, are done with)
    constexpr int kPre = 5;
    float4 kv4[4], pv[kPre], vv[kPre];
    stage_pre(kv4, kb + h * hd, io.ldkv, nk, hd);
    stage_pre(pv, pp, io.ldp, npr, hd);
    stage_pre(vv, vp, io.ldkv, nk, hd);
    stage_post(qu, sq, qv4, qsrc, io.ldq, nr, hd);
    stage_post(st, sq, kv4, kb + h * hd, io.ldkv, nk, hd);
    __syncthreads();
    for (int e = tid; e < nr * hd; e += nt) {
        const int i = e / hd, j = e % hd;
        const float q = qu[i * sq + j];
        qu[i * sq + j] = __fadd_rn(q, pos_u[h * hd + j]);
        qv[i * sq + j] = __fadd_rn(q, pos_v[h * hd + j]);
    }
    __syncthreads();
    const int grp = tid >> 3, gq = tid & 7, ngrp = nt >> 3;
    if constexpr (G8) {
        for (int e = grp; e < nr * nk; e += ngrp) {
            const int i = e / nk, kk = e % nk;
            const float v = dot8_s(qu + i * sq, st + kk * sq, 1, hd, kk < (nk & ~3), gq);
            if (gq == 0) S[i * sS + kk] = v;
        }
    }
    for (int e = tid; !G8 && e < ng * nk + (nr - r1) * nk; e += nt) {
        if (e < ng * nk) {
            const int i0 = 4 * (e / nk), kk = e % nk;
            float o[4];
            panel_v4<4, true>(qu + i0 * sq, sq, st + kk * sq, 1, hd, o);
#pragma unroll
            for (int j = 0; j < 4; ++j) S[(i0 + j) * sS + kk] = o[j];
        } else {
            const int e2 = e - ng * nk, i = r1 + e2 / nk, kk = e2 % nk;
            S[i * sS + kk] = v4 ? matmul_f32_one_v4<true>(qu + i * sq, st + kk * sq, 1, hd, r0 + i, nq, kk, nk)
                                : matmul_f32_one(qu + i * sq, st + kk * sq, 1, hd, r0 + i, nq, kk, nk);
        }
    }
    __syncthreads();
    stage_post(st, sq, pv, pp, io.ldp, npr, hd);
    __syncthreads();
    // bd[i][kk] uses position row (nr-1-i) + kk of the staged ones: rows
    // i0+j with keys kd+j share row nr-1-i0+kd, so a thread takes such a
    // diagonal of four (kd in [0, nk-4]); the three outputs per row each
    // group's diagonals miss, and every output of the other rows, are tasks
    // of their own
    const int nd = nk >= 4 ? nk - 3 : 0, gd = nd > 0 ? ng : 0, rs = nd > 0 ? r1 : 0;
    const int n_diag = gd * nd, n_left = gd * 12, n_rest = (nr - rs) * nk;
    if constexpr (G8) {
        for (int e = grp; e < nr * nk; e += ngrp) {
            const int i = e / nk, kj = e % nk, jj = nq - 1 - (r0 + i) + kj;
            const float v = dot8_s(qv + i * sq, st + (nr - 1 - i + kj) * sq, 1, hd, jj < (np & ~3), gq);
            if (gq == 0) BD[i * sS + kj] = v;
        }
    }
    for (int e = tid; !G8 && e < n_diag + n_left + n_rest; e += nt) {
        int i, kj;
        if (e < n_diag) {
            const int i0 = 4 * (e / nd), kd = e % nd;
            float o[4];
            panel_v4<4, true>(qv + i0 * sq, sq, st + (nr - 1 - i0 + kd) * sq, 1, hd, o);
#pragma unroll
            for (int j = 0; j < 4; ++j) BD[(i0 + j) * sS + kd + j] = o[j];
            continue;
        } else if (e < n_diag + n_left) {
            const int e2 = e - n_diag, q = e2 % 12, j = q / 3, t = q % 3;
            i = 4 * (e2 / 12) + j;
            kj = t < j ? t : nk - 3 + t;
        } else {
            const int e2 = e - n_diag - n_left;
            i = rs + e2 / nk;
            kj = e2 % nk;
        }
        const int jj = nq - 1 - (r0 + i) + kj;  // column of bd in the block's product
        const float *bq = qv + i * sq, *bpr = st + (nr - 1 - i + kj) * sq;
        BD[i * sS + kj] = v4 ? matmul_f32_one_v4<true>(bq, bpr, 1, hd, r0 + i, nq, jj, np)
                             : matmul_f32_one(bq, bpr, 1, hd, r0 + i, nq, jj, np);
    }
    __syncthreads();
    // values of the head (rows sv apart: hd, or hd + 1 where 8 lanes read
    // one column's rows) while the rows are scored
    const int sv = G8 ? hd + 1 : hd;
    stage_post(st, sv, vv, vp, io.ldkv, nk, hd);
    const int lane = tid & 63, wave = tid >> 6, nw = nt >> 6;
    for (int i = wave; i < nr; i += nw) {
        int lo, hi;
        attn_keys(ak, qoff + q0 + r0 + i, Tk, L, c, lo, hi);
        float mx = -__builtin_inff();
        for (int kk = lane; kk < nk; kk += 64) {
            const int kx = k0 + kk;
            float v;
            if (kx < lo || kx >= hi) {
                v = -__builtin_inff();
            } else {
                v = __fmul_rn(__fadd_rn(S[i * sS + kk], BD[i * sS + kk]), scale);
                mx = go_max(mx, v);
            }
            S[i * sS + kk] = v;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = go_max(mx, __shfl_xor(mx, o));
        if (lane == 0) rmx[i] = mx;
    }
    __syncthreads();
    const int n8 = nk & ~7;
    for (int e = tid; e < nr * nk; e += nt) {
        const int i = e / nk, kk = e % nk;
        const float mx = rmx[i];
        float &v = S[i * sS + kk];
        if (mx == -__builtin_inff())
            v = 0.f;
        else {
            const float d = __fsub_rn(v, mx);
            v = kk < n8 ? grx_exp8(d) : grx_expf_go(d);
        }
    }
    __syncthreads();
    for (int i = wave; i < nr; i += nw) {
        float acc = 0.f;
        if (lane < 8) {  // (unrolled: the reads go out ahead of the sum's chain)
#pragma unroll 8
            for (int kk = lane; kk < n8; kk += 8) acc = __fadd_rn(acc, S[i * sS + kk]);
        } else if (lane == 8) {
#pragma unroll 8
            for (int kk = n8; kk < nk; ++kk) acc = __fadd_rn(acc, S[i * sS + kk]);
        }
        float a8[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) a8[l] = __shfl(acc, l);
        const float tail = __shfl(acc, 8);
        if (lane == 0) {
            const float sa = n8 > 0 ? hsum8(a8) : 0.f;
            rinv[i] = __fdiv_rn(1.0f, __fadd_rn(sa, tail));
        }
    }
    __syncthreads();
    for (int e = tid; e < nr * nk; e += nt) {
        const int i = e / nk, kk = e % nk;
        if (rmx[i] != -__builtin_inff()) S[i * sS + kk] = __fmul_rn(S[i * sS + kk], rinv[i]);
    }
    __syncthreads();
    float *O = qu;  // [nr][sq]
    if constexpr (G8) {
        for (int e = grp; e < nr * hd; e += ngrp) {
            const int i = e / hd, ee = e % hd;
            const float v = dot8_s(S + i * sS, st + ee, sv, nk, ee < (hd & ~3), gq);
            if (gq == 0) O[i * sq + ee] = v;
        }
    }
    for (int e = tid; !G8 && e < ng * hd + (nr - r1) * hd; e += nt) {
        if (e < ng * hd) {
            const int i0 = 4 * (e / hd), ee = e % hd;
            float o[4];
            panel_v4<4, false>(S + i0 * sS, sS, st + ee, hd, nk, o);
#pragma unroll
            for (int j = 0; j < 4; ++j) O[(i0 + j) * sq + ee] = o[j];
        } else {
            const int e2 = e - ng * hd, i = r1 + e2 / hd, ee = e2 % hd;
            O[i * sq + ee] = v4 ? matmul_f32_one_v4<false>(S + i * sS, st + ee, hd, nk, r0 + i, nq, ee, hd)
                                : matmul_f32_one(S + i * sS, st + ee, hd, nk, r0 + i, nq, ee, hd);
        }
    }
    __syncthreads();
    for (int g = tid >> 5; g < nr * nqb; g += nt >> 5) {
        const int i = g / nqb, bb = g % nqb, e = tid & 31;
        const size_t row = (size_t)b * T + q0 + r0 + i;
        quant32_store(O[i * sq + bb * 32 + e], xq + row * D + h * hd + bb * 32 + e,
                      xs + row * (D / 32) + (h * hd) / 32 + bb, e);
    }
}

size_t attn_lds_smem_floats(int T, int hd, int rq) {
    const int nk = T, sq = hd + 4, sS = (nk + 3) & ~3;
    const size_t stage = std::max((size_t)(nk + rq - 1) * sq, (size_t)nk * hd);
    return (size_t)2 * rq * sq + (size_t)2 * rq * sS + 2 * rq + stage;
}

size_t attn_smem_floats(int T, int hd) {
    const int nk = T, np = kAttnQ + T - 1;
    return (size_t)2 * kAttnQ * (hd + 1) + (size_t)kAttnQ * (nk | 1) + (size_t)kAttnQ * (np | 1) + 2 * kAttnQ;
}

// ---------------------------------------------------------------- convolution module

// Products of this many rows or fewer (one or two 16-row groups) may take
// the blocks' LayerNorms in their prologues (CONF_FUSE=3; by default only
// one-row products do).
constexpr int kFuseLnRows = 32;

// GLU of the pointwise output (encoder.go:350-361) by grx_glu_pair, the
// output's rows paired as grx_glu_row lays them out, rows at or past the
// utterance's valid rows lens[b] zeroed.
__global__ void conf_glu_kernel(const float *__restrict__ a, int R, int T, int D, const int *__restrict__ lens,
                                float *__restrict__ g) {
    const size_t total = (size_t)R * D;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int c = (int)(idx % D);
        const int row = (int)(idx / D), t = row % T, b = row / T;
        float v = 0.f;
        if (t < lens[b]) {
            const float *ar = a + (size_t)row * 2 * D;
            v = grx_glu_pair(ar[grx_glu_row(c, false)], ar[grx_glu_row(c, true)]);
        }
        g[idx] = v;
    }
}

// The gated frames before a call's first one (encoder.go:372-377): a
// stream's frames in a ring of cap >= padL + chunk rows per stream, frame
// ti of this call at slot (ctl[2] + ti) mod cap (so the call's own frames
// never overwrite the padL before them), or none (offline: those taps are
// skipped).
struct ConvPrev {
    const float *ring;  // [B][cap][D], or null
    int cap;
    const int *ctl;
};
// Frame ti < 0 of utterance b, or null when there is none.
__device__ inline const float *conv_prev_row(const ConvPrev &cp, int b, int ti, int padL, int D) {
    if (cp.ring == nullptr || ti < -padL) return nullptr;
    const int slot = (cp.ctl[2] + cp.cap + ti) % cp.cap;
    return cp.ring + ((size_t)b * cp.cap + slot) * D;
}

// The depthwise convolution (encoder.go:362-385: from the bias, w*x unfused
// over the taps in range, tap j at frame t + j - padL, in order), the folded
// batch norm r*s + b (unfused) or the LayerNorm (LN), SiLU of the AVX route,
// rounded to Q8_0 for pointwise2.  One workgroup per row; a thread takes
// four channels (blockDim apart) at a time with every tap's loads of the
// four in flight together.
template <bool LN>
__global__ __launch_bounds__(kRowThreads) void conf_dwconv_kernel(const float *__restrict__ g, int T, int D, int K,
                                                                  int padL, const ConvPrev cp,
                                                                  const float *__restrict__ w,
                                                                  const float *__restrict__ dwb,
                                                                  const float *__restrict__ cn_w,
                                                                  const float *__restrict__ cn_b,
                                                                  int8_t *__restrict__ xq, float *__restrict__ xs) {
    extern __shared__ __align__(16) float row[];
    __shared__ double red[48];  // ln_block_reduce
    const int r = blockIdx.x, t = r % T, b = r / T, tid = threadIdx.x;
    const float *gb = g + (size_t)b * T * D;
    const int nt = blockDim.x;
    for (int c0 = tid; c0 < D; c0 += 4 * nt) {
        float o[4];
        int cc[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            cc[q] = min(c0 + q * nt, D - 1);  // clamped: loads stay in bounds, results unused
            o[q] = dwb != nullptr ? dwb[cc[q]] : 0.f;
        }
        for (int j0 = 0; j0 < K; j0 += 8) {
            float xv[4][8], wv[4][8];
            bool ok[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int j = j0 + u, ti = t + j - padL;
                const float *pr = ti < 0 ? conv_prev_row(cp, b, ti, padL, D) : nullptr;
                // taps outside the frames (and before a stream's cache) are skipped
                ok[u] = j < K && ((ti >= 0 && ti < T) || pr != nullptr);
                // clamped addresses keep every load in flight together
                const float *xr = pr != nullptr ? pr : gb + (size_t)min(max(ti, 0), T - 1) * D;
                const float *wr = w + (size_t)min(j, K - 1) * D;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    xv[q][u] = xr[cc[q]];
                    wv[q][u] = wr[cc[q]];
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (ok[u]) o[q] = __fadd_rn(o[q], __fmul_rn(wv[q][u], xv[q][u]));
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int c = c0 + q * nt;
            if (c >= D) break;
            float v = o[q];
            if constexpr (!LN) v = __fadd_rn(__fmul_rn(v, cn_w[c]), cn_b[c]);
            row[c] = v;
        }
    }
    __syncthreads();
    if constexpr (LN) ln_row(row, D, cn_w, cn_b, red);
    for (int c = tid; c < D; c += blockDim.x) {
        const float v = row[c];
        const float s = __fdiv_rn(v, __fadd_rn(grx_exp8(__fsub_rn(0.0f, v)), 1.0f));
        quant32_store(s, xq + (size_t)r * D + c, xs + (size_t)r * (D / 32) + c / 32, c & 31);
    }
}

// The same depthwise convolution, folded batch norm, SiLU and rounding for
// kDwRows consecutive frames x 64 channels per workgroup of four waves: the
// channels' window of kDwRows + K - 1 gated frames and their K taps are
// staged in LDS once (instead of K reads per output frame), then wave w
// runs frames 4w .. 4w+3 side by side, lane = channel, taps in order for
// each frame.  grid (ceil(T/kDwRows), D/64, B).
constexpr int kDwRows = 16;
__global__ __launch_bounds__(256) void conf_dwconv_win_kernel(const float *__restrict__ g, int T, int D, int K,
                                                              int padL, const ConvPrev cp,
                                                              const float *__restrict__ w,
                                                              const float *__restrict__ dwb,
                                                              const float *__restrict__ cn_w,
                                                              const float *__restrict__ cn_b,
                                                              int8_t *__restrict__ xq, float *__restrict__ xs) {
    extern __shared__ float win[];  // [kDwRows + K - 1][64] frames, then [K][64] taps
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.x * kDwRows, c0 = blockIdx.y * 64, b = blockIdx.z, c = c0 + lane;
    const int nrow = min(kDwRows, T - t0), wr = nrow + K - 1;
    float *wl = win + (kDwRows + K - 1) * 64;
    const float *gb = g + (size_t)b * T * D + c0;
    const int n = (wr + K) * 64;
    const int lo_t = cp.ring != nullptr ? -padL : 0;  // the first frame a tap may read
    for (int e0 = tid; e0 < n; e0 += 8 * 256) {
        // every load issued at a clamped address, the value chosen after,
        // so the eight stay in flight together
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = min(e0 + u * 256, n - 1), r = e >> 6, l = e & 63, ti = t0 - padL + r;
            const float *pr = (r < wr && ti < 0) ? conv_prev_row(cp, b, ti, padL, D) : nullptr;
            const float *src = r < wr ? (pr != nullptr ? pr + c0 + l : gb + (size_t)min(max(ti, 0), T - 1) * D + l)
                                      : w + (size_t)min(r - wr, K - 1) * D + c0 + l;
            v[u] = *src;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = e0 + u * 256, r = e >> 6, l = e & 63, ti = t0 - padL + r;
            if (e < n) {
                if (r < wr)
                    win[e] = (ti >= lo_t && ti < T) ? v[u] : 0.f;
                else
                    wl[(r - wr) * 64 + l] = v[u];
            }
        }
    }
    __syncthreads();
    float o[4];
    const float b0 = dwb != nullptr ? dwb[c] : 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = b0;
    const int r0 = 4 * wave;
    for (int j = 0; j < K; ++j) {
        const float wj = wl[j * 64 + lane];
        float xv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) xv[r] = win[(r0 + r + j) * 64 + lane];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int ti = t0 + r0 + r + j - padL;  // taps outside the frames are skipped
            const float t = __fadd_rn(o[r], __fmul_rn(wj, xv[r]));
            o[r] = (r0 + r < nrow && ti >= lo_t && ti < T) ? t : o[r];
        }
    }
    const float sw = cn_w[c], sb = cn_b[c];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        if (r0 + r < nrow) {  // uniform across the wave
            const float a = __fadd_rn(__fmul_rn(o[r], sw), sb);
            const float sl = __fdiv_rn(a, __fadd_rn(grx_exp8(__fsub_rn(0.0f, a)), 1.0f));
            const size_t row = (size_t)b * T + t0 + r0 + r;
            quant32_store(sl, xq + row * D + c, xs + row * (D / 32) + c / 32, c & 31);
        }
    }
}

// The same depthwise convolution, folded batch norm, SiLU and rounding with
// one wave per frame and 64 channels (lane = channel): the K gated values
// its taps read and the K taps are loaded at once through buffer resources
// (rows clamped into the buffers; a clamped row's value is never used), then
// one chain over the taps in range.  The range is the same for the whole
// wave, so a skipped tap costs no vector work.  grid (T, D/64, B), one wave
// per workgroup.
constexpr int kDwLaneK = 32;  // the largest kernel the registers hold
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dw_rsrc(const float *p, uint32_t n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p), (short)0, (int)n, 0x00020000);
}
template <bool RING>
__global__ __launch_bounds__(64) void conf_dwconv_lane_kernel(const float *__restrict__ g, int T, int D, int K,
                                                              int padL, const ConvPrev cp,
                                                              const float *__restrict__ w,
                                                              const float *__restrict__ dwb,
                                                              const float *__restrict__ cn_w,
                                                              const float *__restrict__ cn_b,
                                                              int8_t *__restrict__ xq, float *__restrict__ xs) {
    const int lane = threadIdx.x, t = blockIdx.x, c = blockIdx.y * 64 + lane, b = blockIdx.z;
    const int lo_t = RING ? -padL : 0;                     // the first frame a tap may read
    const int f0 = t - padL;                               // the frame tap 0 reads
    const int jlo = max(0, lo_t - f0), jhi = min(K, T - f0);  // the taps in range
    const __amdgpu_buffer_rsrc_t gr = dw_rsrc(g + (size_t)b * T * D, (uint32_t)T * D * 4);
    const __amdgpu_buffer_rsrc_t wr = dw_rsrc(w, (uint32_t)K * D * 4);
    // (no branches among the loads: every one is issued before any is used)
    float xv[kDwLaneK], wv[kDwLaneK];
    const int head = RING ? cp.ctl[2] : 0;                 // the call's first frame's slot
#pragma unroll
    for (int j = 0; j < kDwLaneK; ++j) {
        const int ti = f0 + j;
        const int tc = min(max(ti, 0), T - 1), jc = min(j, K - 1);
        if constexpr (RING) {
            // frames before the call from the stream's ring
            const int slot = (head + cp.cap + max(ti, -padL)) % cp.cap;
            const float *row = ti < 0 ? cp.ring + ((size_t)b * cp.cap + slot) * D : g + ((size_t)b * T + tc) * D;
            xv[j] = row[c];
        } else {
            xv[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(gr, (tc * D + c) * 4, 0, 0));
        }
        wv[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(wr, (jc * D + c) * 4, 0, 0));
    }
    float o = dwb != nullptr ? dwb[c] : 0.f;
#pragma unroll
    for (int j = 0; j < kDwLaneK; ++j)
        if (j >= jlo && j < jhi) o = __fadd_rn(o, __fmul_rn(wv[j], xv[j]));
    const float a = __fadd_rn(__fmul_rn(o, cn_w[c]), cn_b[c]);
    const float sl = __fdiv_rn(a, __fadd_rn(grx_exp8(__fsub_rn(0.0f, a)), 1.0f));
    const size_t row = (size_t)b * T + t;
    quant32_store(sl, xq + row * D + c, xs + row * (D / 32) + c / 32, c & 31);
}

// The depthwise convolution with its LayerNorm (a causal streaming model's
// conv_ln), rows of at most 1024 channels (D % 32 == 0) and kernels of at
// most 16 taps: one workgroup per row, thread = four channels (a float4
// piece: a row's loads are a quarter of the instructions one channel a
// thread takes, which bound a lone workgroup's load time), every tap's
// loads issued at once (the call's earlier frames from the stream's ring)
// and one chain per channel over the taps in range, as
// conf_dwconv_lane_kernel; the row's values to LDS, then every wave takes
// the row's mean and inv (wave_ln32_stats: kern.LayerNorm,
// internal/kern/mathx.go:55-75) and ends its own pieces: the
// normalization, SiLU and the rounding (8 pieces in 8 lanes a block).
template <int KM>
__global__ __launch_bounds__(256) void conf_dwconv_ln_kernel(const float *__restrict__ g, int T, int D, int K,
                                                             int padL, const ConvPrev cp,
                                                             const float *__restrict__ w,
                                                             const float *__restrict__ dwb,
                                                             const float *__restrict__ cn_w,
                                                             const float *__restrict__ cn_b,
                                                             int8_t *__restrict__ xq, float *__restrict__ xs) {
    __shared__ __align__(16) float rowv[1024];
    const int r = blockIdx.x, t = r % T, b = r / T, tid = threadIdx.x;
    const int npc = D / 4, P = min(tid, npc - 1);           // this thread's piece (clamped: loads stay in bounds)
    const bool ring = cp.ring != nullptr;
    const int lo_t = ring ? -padL : 0;                      // the first frame a tap may read
    const int f0 = t - padL;                                // the frame tap 0 reads
    const int jlo = max(0, lo_t - f0), jhi = min(K, T - f0);  // the taps in range
    const int head = ring ? cp.ctl[2] : 0;                  // the call's first frame's slot
    float4 xv[KM], wv[KM];
#pragma unroll
    for (int j = 0; j < KM; ++j) {
        const int ti = f0 + j;
        const int tc = min(max(ti, 0), T - 1), jc = min(j, K - 1);
        const float *src = (ring && ti < 0)
                               ? cp.ring + ((size_t)b * cp.cap + (head + cp.cap + max(ti, -padL)) % cp.cap) * D
                               : g + ((size_t)b * T + tc) * D;
        xv[j] = reinterpret_cast<const float4 *>(src)[P];
        wv[j] = reinterpret_cast<const float4 *>(w + (size_t)jc * D)[P];
    }
    const float4 gw = reinterpret_cast<const float4 *>(cn_w)[P], gb = reinterpret_cast<const float4 *>(cn_b)[P];
    float4 o = dwb != nullptr ? reinterpret_cast<const float4 *>(dwb)[P] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < KM; ++j) {
        if (j >= jlo && j < jhi) {
            o.x = __fadd_rn(o.x, __fmul_rn(wv[j].x, xv[j].x));
            o.y = __fadd_rn(o.y, __fmul_rn(wv[j].y, xv[j].y));
            o.z = __fadd_rn(o.z, __fmul_rn(wv[j].z, xv[j].z));
            o.w = __fadd_rn(o.w, __fmul_rn(wv[j].w, xv[j].w));
        }
    }
    if (tid < npc) reinterpret_cast<float4 *>(rowv)[tid] = o;
    __syncthreads();
    constexpr int NP = 4;
    const int lane = tid & 63;
    float4 v4[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) v4[j] = reinterpret_cast<const float4 *>(rowv)[min(j * 64 + lane, npc - 1)];
    float mean, inv;
    wave_ln32_stats<NP>(v4, npc, lane, mean, inv);
    auto end = [&](float v, float wg, float bg) {
        float a = __fsub_rn(v, mean);
        a = __fmul_rn(a, inv);
        a = __fmul_rn(a, wg);
        a = __fadd_rn(a, bg);
        return __fdiv_rn(a, __fadd_rn(grx_exp8(__fsub_rn(0.0f, a)), 1.0f));
    };
    const float4 v = make_float4(end(o.x, gw.x, gb.x), end(o.y, gw.y, gb.y), end(o.z, gw.z, gb.z),
                                 end(o.w, gw.w, gb.w));
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
    for (int s = 4; s > 0; s >>= 1) {
        const float tt = __shfl_xor(amax, s, 8);
        amax = tt > amax ? tt : amax;
    }
    if (tid >= npc) return;
    const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    auto q1 = [&](float x) {
        float q = rintf(__fmul_rn(x, id));
        q = fminf(fmaxf(q, -128.0f), 127.0f);
        return (uint32_t)(uint8_t)(int8_t)(int)q;
    };
    *reinterpret_cast<uint32_t *>(xq + (size_t)r * D + 4 * tid) = q1(v.x) | q1(v.y) << 8 | q1(v.z) << 16 | q1(v.w) << 24;
    if ((tid & 7) == 0) xs[(size_t)r * (D / 32) + tid / 8] = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
}

// ---------------------------------------------------------------- stream caches

// A chunk's key and value rows (the K and V thirds of the q|k|v product,
// rows [B][T][3D]) into each stream's ring of cap rows: chunk row i to slot
// (head + c + i) % cap, written twice (slot and slot + cap), so that any cap
// consecutive slots from the head read as one run of rows.  ctl: [0] the
// cached keys c, [1] the head.
__global__ void kv_ring_append_kernel(const float *__restrict__ qkv, int B, int T, int D, float *__restrict__ ring,
                                      int cap, const int *__restrict__ ctl) {
    const int c = ctl[0], head = ctl[1];
    const size_t total = (size_t)B * T * 2 * D;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int col = (int)(idx % (2 * D));
        const size_t rt = idx / (2 * D);
        const int i = (int)(rt % T), b = (int)(rt / T);
        const float v = qkv[rt * 3 * D + D + col];
        const int slot = (head + c + i) % cap;
        float *rb = ring + (size_t)b * 2 * cap * 2 * D;
        rb[(size_t)slot * 2 * D + col] = v;
        rb[(size_t)(slot + cap) * 2 * D + col] = v;
    }
}

// The chunk's gated frames into each stream's convolution ring
// (stream.go:302-305 keeps the last padL of them): frame i to slot (ctl[2]
// + i) % cap, over frames older than the padL before the chunk.
__global__ void conv_ring_append_kernel(const float *__restrict__ g, int B, int T, int D, float *__restrict__ ring,
                                        int cap, const int *__restrict__ ctl) {
    const int head = ctl[2];
    const size_t total = (size_t)B * T * D;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int col = (int)(idx % D);
        const size_t rt = idx / D;
        const int i = (int)(rt % T), b = (int)(rt / T);
        const int slot = (head + i) % cap;
        ring[((size_t)b * cap + slot) * D + col] = g[rt * D + col];
    }
}

}  // namespace

// ---------------------------------------------------------------- host side

struct CFF {
    float *norm_w = nullptr, *norm_b = nullptr, *b1 = nullptr, *b2 = nullptr;
    grx_weight *w1 = nullptr, *w2 = nullptr;
};

struct CBlock {
    CFF ff1, ff2;
    float *norm_attn_w, *norm_attn_b, *qkv_b, *out_b, *pos_u, *pos_v;
    float *norm_conv_w, *norm_conv_b, *pw1_b, *pw2_b, *dw, *dw_b, *cn_w, *cn_b, *norm_out_w, *norm_out_b;
    grx_weight *qkv = nullptr, *out = nullptr, *pw1 = nullptr, *pw2 = nullptr;
};

struct grx_conformer {
    grx_ctx *ctx = nullptr;
    grx_conformer_hparams hp{};
    std::map<std::string, std::vector<uint8_t>> host;
    bool ready = false;
    std::vector<void *> allocs;        // weights and constants
    std::vector<void *> work;          // shape-dependent buffers
    // pre-encoder
    float *w0, *b0, *w2, *b2, *w5, *b5, *b3, *b6, *outb;
    grx_weight *w3 = nullptr, *w6 = nullptr, *wout = nullptr;
    float *w3f = nullptr, *w6f = nullptr;  // conv.3 / conv.6 stored float32: the float route
    std::vector<CBlock> blk;
    grx_weight *pos_all = nullptr;  // every block's linear_pos, [layers*d][d]
    // shape-dependent state
    int B = 0, frames = 0, T = 0;
    int attn_rq = 0;         // query rows per staged attention workgroup (0: unstaged kernel)
    bool dw_win = false;     // the windowed depthwise kernel runs (its LDS was granted)
    size_t attn_smem = 0;
    float *mel = nullptr, *sub0 = nullptr, *suby = nullptr, *x = nullptr, *qkv = nullptr, *pp = nullptr;
    float *subx = nullptr;  // float input of a float32 pointwise Linear
    float *x2 = nullptr;  // the residual rows' second buffer (blocks with fused LayerNorms alternate)
    float *conv = nullptr, *glu = nullptr, *pos = nullptr;
    int8_t *xq = nullptr, *fq = nullptr, *pos_q = nullptr;  // fq: the rounded SiLU output of W1
    float *xs = nullptr, *fs = nullptr, *pos_s = nullptr;
    int *valid = nullptr;       // [B] mel frames, then [B] encoder rows of each utterance
    int *valid_host = nullptr;  // pinned, the same 2B values
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace {

struct CExpect {
    std::string name;
    size_t bytes;
    bool optional;
};

size_t q8b(size_t rows, size_t cols) { return rows * (cols / 32) * 34; }

int sub_F(const grx_conformer_hparams &hp) { return stage_len(hp.n_mels, 3, hp.causal_sub); }

// The tensors loadEncoder reads (conformer/model.go:370-422), with sizes.
std::vector<CExpect> cexpected(const grx_conformer_hparams &hp) {
    const size_t d = hp.d, c = hp.sub_channels, ff = hp.dff, K = hp.conv_kernel;
    const size_t cF = c * sub_F(hp);
    std::vector<CExpect> e;
    const std::string pe = "enc.pre_encode.";
    for (const char *n : {"conv.0", "conv.2", "conv.5"}) {
        e.push_back({pe + n + ".weight", c * 9 * 4, false});
        e.push_back({pe + n + ".bias", c * 4, false});
    }
    for (const char *n : {"conv.3", "conv.6"}) {
        e.push_back({pe + n + ".weight", 0, false});  // Q8_0, or float32: checked at finalize
        e.push_back({pe + n + ".bias", c * 4, false});
    }
    e.push_back({pe + "out.weight", q8b(d, cF), false});
    e.push_back({pe + "out.bias", d * 4, false});
    for (int i = 0; i < hp.layers; ++i) {
        const std::string p = "enc.blocks." + std::to_string(i) + ".";
        for (const char *f : {"ff1", "ff2"}) {
            e.push_back({p + "norm_" + f + ".weight", d * 4, false});
            e.push_back({p + "norm_" + f + ".bias", d * 4, false});
            e.push_back({p + f + ".linear1.weight", q8b(ff, d), false});
            e.push_back({p + f + ".linear1.bias", ff * 4, true});
            e.push_back({p + f + ".linear2.weight", q8b(d, ff), false});
            e.push_back({p + f + ".linear2.bias", d * 4, true});
        }
        for (const char *n : {"norm_attn", "norm_conv", "norm_out"}) {
            e.push_back({p + n + ".weight", d * 4, false});
            e.push_back({p + n + ".bias", d * 4, false});
        }
        for (const char *n : {"linear_q", "linear_k", "linear_v", "linear_out"}) {
            e.push_back({p + "attn." + n + ".weight", q8b(d, d), false});
            e.push_back({p + "attn." + n + ".bias", d * 4, true});
        }
        e.push_back({p + "attn.linear_pos.weight", q8b(d, d), false});
        e.push_back({p + "attn.pos_bias_u", d * 4, false});
        e.push_back({p + "attn.pos_bias_v", d * 4, false});
        // the pointwise convolutions: Q8_0, or float16 rounded at load
        e.push_back({p + "conv.pointwise1.weight", 0, false});
        e.push_back({p + "conv.pointwise1.bias", 2 * d * 4, true});
        e.push_back({p + "conv.pointwise2.weight", 0, false});
        e.push_back({p + "conv.pointwise2.bias", d * 4, true});
        e.push_back({p + "conv.depthwise.weight", d * K * 4, false});
        e.push_back({p + "conv.depthwise.bias", d * 4, true});
        e.push_back({p + "conv.bn.weight", d * 4, false});
        e.push_back({p + "conv.bn.bias", d * 4, false});
        e.push_back({p + "conv.bn.running_mean", d * 4, hp.conv_ln != 0});
        e.push_back({p + "conv.bn.running_var", d * 4, hp.conv_ln != 0});
    }
    return e;
}

grx_status calloc_dev(std::vector<void *> &list, size_t bytes, void **out) {
    void *p = nullptr;
    GRX_HIP(grx_dev_malloc(&p, bytes > 0 ? bytes : 16));
    list.push_back(p);
    *out = p;
    return GRX_OK;
}

template <typename T>
grx_status calloc_t(std::vector<void *> &list, size_t count, T **out) {
    return calloc_dev(list, count * sizeof(T), reinterpret_cast<void **>(out));
}

grx_status upload(grx_conformer *m, const void *data, size_t bytes, float **out) {
    grx_status s = calloc_t(m->allocs, bytes / 4, out);
    if (s != GRX_OK) return s;
    GRX_HIP(hipMemcpy(*out, data, bytes, hipMemcpyHostToDevice));
    return GRX_OK;
}

// A named float vector (nullptr when optional and absent).
grx_status cvec(grx_conformer *m, const std::string &name, float **out) {
    *out = nullptr;
    auto it = m->host.find(name);
    if (it == m->host.end()) return GRX_OK;
    return upload(m, it->second.data(), it->second.size(), out);
}

// transposeTaps (conformer/model.go:147-159): [c][taps] to [taps][c].
std::vector<float> transpose_taps(const std::vector<uint8_t> &raw, int c, int taps) {
    const float *w = reinterpret_cast<const float *>(raw.data());
    std::vector<float> out((size_t)c * taps);
    for (int i = 0; i < c; ++i)
        for (int j = 0; j < taps; ++j) out[(size_t)j * c + i] = w[(size_t)i * taps + j];
    return out;
}

// IEEE half to float, exactly.
float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    int e = (h >> 10) & 0x1f;
    uint32_t f = h & 0x3ff, bits;
    if (e == 0x1f) {
        bits = sign | 0x7f800000u | (f << 13);
    } else if (e == 0) {
        if (f == 0) {
            bits = sign;
        } else {
            e = 1;
            while (!(f & 0x400)) {
                f <<= 1;
                --e;
            }
            f &= 0x3ff;
            bits = sign | ((uint32_t)(e + 112) << 23) | (f << 13);
        }
    } else {
        bits = sign | ((uint32_t)(e + 112) << 23) | (f << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

// Rows of a pointwise1 weight (2d rows of `bytes` each) or bias (4
// bytes) reordered into the GLU's pairs: row grx_glu_row(c, false) is row
// c (channel c's a-row), grx_glu_row(c, true) row d + c (its b-row).  The
// products of each row are unchanged (the same blocks in the same order).
std::vector<uint8_t> glu_pair_rows(const uint8_t *src, int d, size_t bytes) {
    std::vector<uint8_t> out((size_t)2 * d * bytes);
    for (int c = 0; c < d; ++c) {
        memcpy(out.data() + (size_t)grx_glu_row(c, false) * bytes, src + (size_t)c * bytes, bytes);
        memcpy(out.data() + (size_t)grx_glu_row(c, true) * bytes, src + (size_t)(d + c) * bytes, bytes);
    }
    return out;
}

// A pointwise-convolution weight: Q8_0 rows as they are, or float16
// widened and rounded by Weight.ToQ8 (conformer/model.go:397-402); glu:
// pointwise1's rows paired for the GLU (glu_pair_rows).
grx_status pointwise_weight(grx_conformer *m, const std::string &name, int rows, int cols, bool glu,
                            grx_weight **out) {
    const auto &raw = m->host.at(name);
    const size_t n = (size_t)rows * cols;
    std::vector<uint8_t> q;
    if (raw.size() == q8b(rows, cols)) {
        q.assign(raw.begin(), raw.end());
    } else {
        if (raw.size() != n * 2)
            return grx_fail(GRX_ESIZE, "tensor %s is neither Q8_0 nor float16 %dx%d", name.c_str(), rows, cols);
        std::vector<float> v(n);
        const uint16_t *h = reinterpret_cast<const uint16_t *>(raw.data());
        for (size_t i = 0; i < n; ++i) v[i] = half_to_float(h[i]);
        q.resize(q8b(rows, cols));
        grx_status s = grx_to_q8(m->ctx, rows, cols, v.data(), q.data());
        if (s != GRX_OK) return s;
    }
    if (glu) q = glu_pair_rows(q.data(), rows / 2, q8b(1, cols));
    return grx_weight_q8_create(m->ctx, rows, cols, q.data(), q.size(), out);
}

// What cfinalize made (the device weights and constants), released: after a
// failed finalize the model is as before it (its host tensors kept), and
// grx_conformer_destroy releases a finished one.
void crelease(grx_conformer *m) {
    for (void *p : m->allocs) (void)hipFree(p);
    m->allocs.clear();
    for (grx_weight **w : {&m->w3, &m->w6, &m->wout, &m->pos_all}) {
        grx_weight_destroy(*w);
        *w = nullptr;
    }
    m->w3f = m->w6f = nullptr;
    for (CBlock &B : m->blk)
        for (grx_weight *w : {B.ff1.w1, B.ff1.w2, B.ff2.w1, B.ff2.w2, B.qkv, B.out, B.pw1, B.pw2}) grx_weight_destroy(w);
    m->blk.clear();
}

grx_status cfinalize_tensors(grx_conformer *m);

grx_status cfinalize(grx_conformer *m) {
    if (m->ready) return GRX_OK;
    const grx_status s = cfinalize_tensors(m);
    if (s != GRX_OK) crelease(m);
    return s;
}

grx_status cfinalize_tensors(grx_conformer *m) {
    const grx_conformer_hparams &hp = m->hp;
    for (const CExpect &e : cexpected(hp))
        if (!e.optional && !m->host.count(e.name)) return grx_fail(GRX_ESTATE, "the model has no tensor %s", e.name.c_str());
    GRX_HIP(hipSetDevice(m->ctx->device));
    grx_status s;
    const int d = hp.d, c = hp.sub_channels, cF = c * sub_F(hp), K = hp.conv_kernel;
    const std::string pe = "enc.pre_encode.";
    {
        struct {
            const char *n;
            float **w, **b;
        } taps[] = {{"conv.0", &m->w0, &m->b0}, {"conv.2", &m->w2, &m->b2}, {"conv.5", &m->w5, &m->b5}};
        for (auto &t : taps) {
            std::vector<float> tw = transpose_taps(m->host.at(pe + t.n + ".weight"), c, 9);
            if ((s = upload(m, tw.data(), tw.size() * 4, t.w)) != GRX_OK) return s;
            if ((s = cvec(m, pe + t.n + ".bias", t.b)) != GRX_OK) return s;
        }
    }
    auto mat = [&](const std::string &n, int rows, int cols, grx_weight **w) {
        const auto &t = m->host.at(n);
        return grx_weight_q8_create(m->ctx, rows, cols, t.data(), t.size(), w);
    };
    // conv.3 / conv.6: Q8_0 rows (the int8 route), or float32 values as the
    // reference's converter stores them (the float route)
    for (auto pw : {std::make_pair("conv.3.weight", &m->w3), std::make_pair("conv.6.weight", &m->w6)}) {
        const std::string n = pe + pw.first;
        const auto &t = m->host.at(n);
        if (t.size() == (size_t)c * c * 4) {
            float **dst = pw.second == &m->w3 ? &m->w3f : &m->w6f;
            if ((s = upload(m, t.data(), t.size(), dst)) != GRX_OK) return s;
        } else if (t.size() == q8b(c, c)) {
            if ((s = mat(n, c, c, pw.second)) != GRX_OK) return s;
        } else {
            return grx_fail(GRX_ESIZE, "tensor %s is neither Q8_0 nor float32 %dx%d", n.c_str(), c, c);
        }
    }
    if ((s = mat(pe + "out.weight", d, cF, &m->wout)) != GRX_OK) return s;
    if ((s = cvec(m, pe + "conv.3.bias", &m->b3)) != GRX_OK) return s;
    if ((s = cvec(m, pe + "conv.6.bias", &m->b6)) != GRX_OK) return s;
    if ((s = cvec(m, pe + "out.bias", &m->outb)) != GRX_OK) return s;
    m->blk.assign(hp.layers, CBlock());
    std::vector<uint8_t> pos_cat;
    for (int i = 0; i < hp.layers; ++i) {
        CBlock &B = m->blk[i];
        const std::string p = "enc.blocks." + std::to_string(i) + ".";
        for (int f = 0; f < 2; ++f) {
            CFF &F = f == 0 ? B.ff1 : B.ff2;
            const std::string n = f == 0 ? "ff1" : "ff2";
            if ((s = cvec(m, p + "norm_" + n + ".weight", &F.norm_w)) != GRX_OK) return s;
            if ((s = cvec(m, p + "norm_" + n + ".bias", &F.norm_b)) != GRX_OK) return s;
            if ((s = mat(p + n + ".linear1.weight", hp.dff, d, &F.w1)) != GRX_OK) return s;
            if ((s = mat(p + n + ".linear2.weight", d, hp.dff, &F.w2)) != GRX_OK) return s;
            if ((s = cvec(m, p + n + ".linear1.bias", &F.b1)) != GRX_OK) return s;
            if ((s = cvec(m, p + n + ".linear2.bias", &F.b2)) != GRX_OK) return s;
        }
        {  // q, k and v share their input: one weight of 3d rows, missing biases 0
            std::vector<uint8_t> cat;
            std::vector<float> bias(3 * (size_t)d, 0.0f);
            int j = 0;
            for (const char *n : {"linear_q", "linear_k", "linear_v"}) {
                const auto &t = m->host.at(p + "attn." + n + ".weight");
                cat.insert(cat.end(), t.begin(), t.end());
                auto it = m->host.find(p + "attn." + n + ".bias");
                if (it != m->host.end()) memcpy(bias.data() + (size_t)j * d, it->second.data(), (size_t)d * 4);
                ++j;
            }
            if ((s = grx_weight_q8_create(m->ctx, 3 * d, d, cat.data(), cat.size(), &B.qkv)) != GRX_OK) return s;
            if ((s = upload(m, bias.data(), bias.size() * 4, &B.qkv_b)) != GRX_OK) return s;
        }
        {
            const auto &t = m->host.at(p + "attn.linear_pos.weight");
            pos_cat.insert(pos_cat.end(), t.begin(), t.end());
        }
        if ((s = mat(p + "attn.linear_out.weight", d, d, &B.out)) != GRX_OK) return s;
        if ((s = pointwise_weight(m, p + "conv.pointwise1.weight", 2 * d, d, true, &B.pw1)) != GRX_OK) return s;
        if ((s = pointwise_weight(m, p + "conv.pointwise2.weight", d, d, false, &B.pw2)) != GRX_OK) return s;
        B.pw1_b = nullptr;
        if (auto it = m->host.find(p + "conv.pointwise1.bias"); it != m->host.end()) {  // optional
            const std::vector<uint8_t> pb = glu_pair_rows(it->second.data(), d, sizeof(float));
            if ((s = upload(m, pb.data(), pb.size(), &B.pw1_b)) != GRX_OK) return s;
        }
        struct {
            const char *n;
            float **v;
        } vecs[] = {{"norm_attn.weight", &B.norm_attn_w}, {"norm_attn.bias", &B.norm_attn_b},
                    {"attn.linear_out.bias", &B.out_b},   {"attn.pos_bias_u", &B.pos_u},
                    {"attn.pos_bias_v", &B.pos_v},        {"norm_conv.weight", &B.norm_conv_w},
                    {"norm_conv.bias", &B.norm_conv_b},   {"conv.pointwise2.bias", &B.pw2_b},
                    {"conv.depthwise.bias", &B.dw_b},
                    {"norm_out.weight", &B.norm_out_w},   {"norm_out.bias", &B.norm_out_b}};
        for (auto &v : vecs)
            if ((s = cvec(m, p + v.n, v.v)) != GRX_OK) return s;
        {
            std::vector<float> tw = transpose_taps(m->host.at(p + "conv.depthwise.weight"), d, K);
            if ((s = upload(m, tw.data(), tw.size() * 4, &B.dw)) != GRX_OK) return s;
        }
        const float *gw = reinterpret_cast<const float *>(m->host.at(p + "conv.bn.weight").data());
        const float *gb = reinterpret_cast<const float *>(m->host.at(p + "conv.bn.bias").data());
        if (hp.conv_ln) {
            if ((s = upload(m, gw, (size_t)d * 4, &B.cn_w)) != GRX_OK) return s;
            if ((s = upload(m, gb, (size_t)d * 4, &B.cn_b)) != GRX_OK) return s;
        } else {  // conformer/model.go:408-418: the batch norm folded to scale and bias
            const float *mean = reinterpret_cast<const float *>(m->host.at(p + "conv.bn.running_mean").data());
            const float *vr = reinterpret_cast<const float *>(m->host.at(p + "conv.bn.running_var").data());
            std::vector<float> sw(d), sb(d);
            for (int j = 0; j < d; ++j) {
                const float sj = (float)((double)gw[j] / std::sqrt((double)vr[j] + 1e-5));
                sw[j] = sj;
                const float ms = mean[j] * sj;
                sb[j] = gb[j] - ms;
            }
            if ((s = upload(m, sw.data(), (size_t)d * 4, &B.cn_w)) != GRX_OK) return s;
            if ((s = upload(m, sb.data(), (size_t)d * 4, &B.cn_b)) != GRX_OK) return s;
        }
    }
    if ((s = grx_weight_q8_create(m->ctx, hp.layers * d, d, pos_cat.data(), pos_cat.size(), &m->pos_all)) != GRX_OK)
        return s;
    m->host.clear();
    m->ready = true;
    return GRX_OK;
}

void free_work(grx_conformer *m) {
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    m->exec = nullptr;
    m->graph = nullptr;
    for (void *p : m->work) (void)hipFree(p);
    m->work.clear();
    if (m->valid_host) (void)hipHostFree(m->valid_host);
    m->valid_host = nullptr;
    m->B = m->frames = m->T = 0;
}

// relPosRange (encoder.go:183-191): count rows for relative positions
// first, first-1, ...; relPosEmb(n) is first = n-1, count = 2n-1.
std::vector<float> rel_pos(int first, int count, int d) {
    std::vector<float> out((size_t)count * d);
    for (int i = 0; i < count; ++i) {
        const double pos = (double)(first - i);
        float *row = out.data() + (size_t)i * d;
        for (int j = 0; j < d; j += 2) {
            const float div = (float)std::exp((double)j * -(std::log(10000.0) / (double)d));
            const double a = (double)((float)pos * div);
            row[j] = (float)std::sin(a);
            if (j + 1 < d) row[j + 1] = (float)std::cos(a);
        }
    }
    return out;
}

// offlineKeys (encoder.go:196-212) for T encoder frames.
AttnKeys offline_keys(const grx_conformer_hparams &hp, int T) {
    AttnKeys k{};
    const int al = hp.att_left, ar = hp.att_right;
    if (hp.att_chunked && al >= 0 && ar >= 0) {
        k.mode = kKeysChunked;
        k.chunk = ar + 1;
        k.lchunks = al / k.chunk;
        k.bl = k.chunk;
    } else if (al >= 0 && ar >= 0 && T - 1 > std::min(al, ar)) {
        k.mode = kKeysWindow;
        k.left = al;
        k.right = ar;
        k.bl = 16;
    } else {
        k.mode = kKeysAll;
        k.bl = kAttnQ;
    }
    return k;
}

// convPadLeft (encoder.go:399-404).
int pad_left(const grx_conformer_hparams &hp) {
    return hp.conv_left >= 0 && hp.conv_right >= 0 ? hp.conv_left : (hp.conv_kernel - 1) / 2;
}

// Which attention kernel runs and its LDS: the staged kernel takes 4 query
// rows per workgroup for few workgroups, 8 or 16 for more; past what LDS holds
// the unstaged kernel runs.  nk: the most keys a block sees.
grx_status attn_pick(int B, int heads, int nblk, int bl, int nk, int hd, int *rq, size_t *smem) {
    // (batch 1 at T = 126: 128 workgroups of 8 rows; 4 rows each measured
    // 4.32 -> 4.20 ms an encode, the streaming chunks 3.28 -> 3.20 ms)
    const long n8 = (long)B * heads * nblk * ((bl + 7) / 8);
    *rq = n8 < 256 ? 4 : n8 < 1024 ? 8 : 16;
    // a row a workgroup on 8-lane groups where a block has at most 16 rows,
    // a row's scores and outputs fit one round of the groups, and the
    // workgroups number at most 256 (a streaming chunk step of 14 rows, one
    // stream: 2.48 -> 2.38 ms against 4 rows a workgroup; of one row 1.75 ->
    // 1.72, the smaller LDS)
    if (bl <= 16 && (long)B * heads * nblk * bl <= 256 && std::max(nk, hd) * 8 <= kAttnLdsThreads) *rq = 1;
    if (grx_tune(GRX_TUNE_CONF_ATTN_RQ) >= 0) *rq = grx_tune(GRX_TUNE_CONF_ATTN_RQ);  // 0 (unstaged), 1, 4, 8 or 16, for tests
    if (*rq != 0 && *rq != 1 && *rq != 4 && *rq != 8 && *rq != 16) *rq = 8;
    if (*rq == 1 && !(bl <= 16 && std::max(nk, hd) * 8 <= kAttnLdsThreads)) *rq = 4;
    const size_t staged = attn_lds_smem_floats(nk, hd, *rq) * 4;
    const size_t sq = hd + 1;
    const void *fn = *rq == 1   ? (const void *)conf_attn_lds_kernel<1, true>
                     : *rq == 4 ? (const void *)conf_attn_lds_kernel<4>
                     : *rq == 8 ? (const void *)conf_attn_lds_kernel<8>
                                : (const void *)conf_attn_lds_kernel<16>;
    if (*rq != 0 && staged <= 160 * 1024 &&
        (staged <= 64 * 1024 ||
         (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)staged) == hipSuccess &&
          (*rq != 4 || hipFuncSetAttribute((const void *)conf_attn_lds_kernel<4, true>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)staged) == hipSuccess)))) {
        *smem = staged;
        return GRX_OK;
    }
    (void)hipGetLastError();
    *rq = 0;
    const size_t np = kAttnQ + nk - 1;
    const size_t need = ((size_t)2 * kAttnQ * sq + (size_t)kAttnQ * (nk | 1) + (size_t)kAttnQ * (np | 1) + 2 * kAttnQ) * 4;
    if (need > 160 * 1024 ||
        (need > 64 * 1024 && hipFuncSetAttribute((const void *)conf_attn_kernel,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)need) != hipSuccess))
        return grx_fail(GRX_ESIZE, "%d keys per query block are more than the attention kernel holds", nk);
    *smem = need;
    return GRX_OK;
}

// Whether the windowed depthwise kernel runs (its LDS granted).
bool dw_win_ok(const grx_conformer_hparams &hp) {
    const size_t need = (size_t)(kDwRows + 2 * hp.conv_kernel - 1) * 64 * 4;
    const bool ok = hp.d % 64 == 0 && !hp.conv_ln && need <= 160 * 1024 &&
                    (need <= 64 * 1024 || hipFuncSetAttribute((const void *)conf_dwconv_win_kernel,
                                                              hipFuncAttributeMaxDynamicSharedMemorySize,
                                                              (int)need) == hipSuccess);
    (void)hipGetLastError();
    return ok;
}

// The working buffers of B utterances of `frames` mel frames whose
// pre-encoder gives T rows each, Tp kept (the blocks' rows).
struct CBuf {
    float *mel = nullptr, *sub0 = nullptr, *suby = nullptr, *subx = nullptr, *x = nullptr, *x2 = nullptr;
    float *qkv = nullptr;
    float *conv = nullptr, *glu = nullptr;
    int8_t *xq = nullptr, *fq = nullptr;
    float *xs = nullptr, *fs = nullptr;
};
grx_status cbuf_alloc(const grx_conformer *m, std::vector<void *> &w, int B, int frames, int Tp, CBuf *b) {
    const grx_conformer_hparams &hp = m->hp;
    const int d = hp.d, c = hp.sub_channels, nm = hp.n_mels, cs = hp.causal_sub;
    const int T2 = stage_len(frames, 2, cs), F2 = stage_len(nm, 2, cs), T = stage_len(frames, 3, cs),
              F3 = stage_len(nm, 3, cs);
    const size_t R = (size_t)B * Tp;
    grx_status s;
    if ((s = calloc_t(w, (size_t)B * nm * frames, &b->mel)) != GRX_OK) return s;
    if ((s = calloc_t(w, (size_t)B * T * F3 * c, &b->sub0)) != GRX_OK) return s;
    if ((s = calloc_t(w, (size_t)B * T2 * F2 * c, &b->suby)) != GRX_OK) return s;
    if ((m->w3f || m->w6f) && (s = calloc_t(w, (size_t)B * T2 * F2 * c, &b->subx)) != GRX_OK) return s;
    // rounded activations: the largest row set of any product
    const size_t qn = std::max({(size_t)B * T2 * F2 * c, R * (size_t)c * F3, R * (size_t)hp.dff, R * 2 * (size_t)d});
    if ((s = calloc_t(w, qn, &b->xq)) != GRX_OK) return s;
    if ((s = calloc_t(w, qn / 32, &b->xs)) != GRX_OK) return s;
    if ((s = calloc_t(w, R * hp.dff, &b->fq)) != GRX_OK) return s;
    if ((s = calloc_t(w, R * hp.dff / 32, &b->fs)) != GRX_OK) return s;
    if ((s = calloc_t(w, R * d, &b->x)) != GRX_OK) return s;
    if ((s = calloc_t(w, R * d, &b->x2)) != GRX_OK) return s;
    if ((s = calloc_t(w, R * 3 * d, &b->qkv)) != GRX_OK) return s;
    if ((s = calloc_t(w, R * 2 * d, &b->conv)) != GRX_OK) return s;
    if ((s = calloc_t(w, R * d, &b->glu)) != GRX_OK) return s;
    return GRX_OK;
}

// Buffers for B utterances of `frames` mel frames, the position table of
// their T and its rounding.
grx_status cshape(grx_conformer *m, int B, int frames) {
    if (m->B == B && m->frames == frames) return GRX_OK;
    free_work(m);
    const grx_conformer_hparams &hp = m->hp;
    const int d = hp.d, T = stage_len(frames, 3, hp.causal_sub);
    {
        const AttnKeys k = offline_keys(hp, T);
        grx_status s = attn_pick(B, hp.heads, (T + k.bl - 1) / k.bl, k.bl, T, d / hp.heads, &m->attn_rq, &m->attn_smem);
        if (s != GRX_OK) return s;
    }
    m->dw_win = dw_win_ok(hp);
    grx_status s;
    auto &w = m->work;
    CBuf b;
    if ((s = cbuf_alloc(m, w, B, frames, T, &b)) != GRX_OK) return s;
    m->mel = b.mel, m->sub0 = b.sub0, m->suby = b.suby, m->subx = b.subx, m->x = b.x, m->x2 = b.x2, m->qkv = b.qkv;
    m->conv = b.conv, m->glu = b.glu, m->xq = b.xq, m->xs = b.xs, m->fq = b.fq, m->fs = b.fs;
    if ((s = calloc_t(w, (size_t)(2 * T - 1) * hp.layers * d, &m->pp)) != GRX_OK) return s;
    if ((s = calloc_t(w, (size_t)(2 * T - 1) * d, &m->pos)) != GRX_OK) return s;
    if ((s = calloc_t(w, (size_t)(2 * T - 1) * d, &m->pos_q)) != GRX_OK) return s;
    if ((s = calloc_t(w, (size_t)(2 * T - 1) * d / 32, &m->pos_s)) != GRX_OK) return s;
    if ((s = calloc_t(w, 2 * (size_t)B, &m->valid)) != GRX_OK) return s;
    GRX_HIP(grx_pinned_malloc((void **)&m->valid_host, 2 * (size_t)B * sizeof(int)));
    std::vector<float> pos = rel_pos(T - 1, 2 * T - 1, d);
    GRX_HIP(hipMemcpy(m->pos, pos.data(), pos.size() * 4, hipMemcpyHostToDevice));
    if ((s = grx_quant_act_dev(m->ctx, m->pos_q, m->pos_s, m->pos, d, 2 * T - 1, d)) != GRX_OK) return s;
    GRX_HIP(hipStreamSynchronize(m->ctx->stream));
    m->B = B;
    m->frames = frames;
    m->T = T;
    return GRX_OK;
}

unsigned grid_for(size_t n) { return (unsigned)std::min<size_t>((n + 255) / 256, 1u << 20); }

// The rows' LayerNorm (and rounding) by ln_rows_wave_kernel where a wave
// holds the row (n % 32 == 0, n <= 1280), else ln_rows_kernel.
template <bool OUT, bool Q>
grx_status ln_rows_launch(hipStream_t st, int R, float *x, int n, const float *w1, const float *b1, const float *w2,
                          const float *b2, int8_t *xq, float *xs) {
    if (n % 32 == 0 && n <= 1280) {
        if (n <= 512)
            ln_rows_wave_kernel<OUT, Q, 2><<<R, 64, 0, st>>>(x, n, w1, b1, w2, b2, xq, xs);
        else if (n <= 1024)
            ln_rows_wave_kernel<OUT, Q, 4><<<R, 64, 0, st>>>(x, n, w1, b1, w2, b2, xq, xs);
        else
            ln_rows_wave_kernel<OUT, Q, 5><<<R, 64, 0, st>>>(x, n, w1, b1, w2, b2, xq, xs);
        GRX_LAUNCHED("ln_rows_wave_kernel");
        return GRX_OK;
    }
    ln_rows_kernel<OUT, Q><<<R, kRowThreads, (size_t)n * 4, st>>>(x, n, w1, b1, w2, b2, xq, xs);
    GRX_LAUNCHED("ln_rows_kernel");
    return GRX_OK;
}

// One run of the encoder over B utterances (or streams' chunks): the
// pre-encoder on `frames` mel frames (T rows each, the first `drop` cut,
// Tp kept), xscale, then every block.
struct CRun {
    int B, frames, T, Tp, drop;
    CBuf b;
    const int *valid, *lens;  // device: mel frames and encoder rows per utterance
    // the attention: key form, position rows, kernel
    AttnKeys keys;
    const float *pp;
    int maxfirst;
    const int *ctl;  // streaming: c, ring heads (device); null offline
    int attn_rq;
    int attn_keys;  // the most keys a block's queries see
    size_t attn_smem;
    bool dw_win;
    // streaming caches per layer (null offline)
    float *kv_ring;
    size_t kv_ring_layer;
    int cap;
    float *conv_ring;
    size_t conv_ring_layer;
    int conv_cap;
};

grx_status enqueue_run(grx_conformer *m, const CRun &r, hipStream_t st) {
    const grx_conformer_hparams &hp = m->hp;
    const int B = r.B, frames = r.frames, d = hp.d, c = hp.sub_channels, nm = hp.n_mels, T = r.T, Tp = r.Tp;
    const int cs = hp.causal_sub, padL = pad_left(hp);
    const int T1 = stage_len(frames, 1, cs), F1 = stage_len(nm, 1, cs), T2 = stage_len(frames, 2, cs),
              F2 = stage_len(nm, 2, cs), F3 = stage_len(nm, 3, cs);
    const int R = B * Tp, hd = d / hp.heads;
    const CBuf &bf = r.b;
    grx_status s;
    // pre-encoder (encoder.go:123-167)
    sub_conv01_kernel<<<B * T2, c, (size_t)7 * (4 * F2 + 3) * 4, st>>>(bf.mel, frames, nm, r.valid, cs, m->w0, m->b0,
                                                                      m->w2, m->b2, c, T1, F1, T2, F2, bf.xq, bf.xs,
                                                                      m->w3f ? bf.subx : nullptr);
    GRX_LAUNCHED("sub_conv01_kernel");
    if (m->w3f) {
        if ((s = grx_float_rows_f32(st, bf.subx, m->w3f, m->b3, bf.suby, B, T2 * F2, c, c)) != GRX_OK) return s;
    } else if ((s = grx_gemm_q8_launch(st, m->w3, bf.xq, bf.xs, B * T2 * F2, m->b3, bf.suby, c)) != GRX_OK) {
        return s;
    }
    sub_dwconv_kernel<true><<<B * T * F3, c, 0, st>>>(bf.suby, T2, F2, c, r.valid, cs, 3, m->w5, m->b5, T, F3, bf.xq,
                                                      bf.xs, m->w6f ? bf.subx : nullptr);
    GRX_LAUNCHED("sub_dwconv_kernel");
    if (m->w6f) {
        if ((s = grx_float_rows_f32(st, bf.subx, m->w6f, m->b6, bf.sub0, B, T * F3, c, c)) != GRX_OK) return s;
    } else if ((s = grx_gemm_q8_launch(st, m->w6, bf.xq, bf.xs, B * T * F3, m->b6, bf.sub0, c)) != GRX_OK) {
        return s;
    }
    sub_flatten_kernel<<<R, 256, 0, st>>>(bf.sub0, T, F3, c, r.valid, cs, r.drop, Tp, bf.xq, bf.xs);
    GRX_LAUNCHED("sub_flatten_kernel");
    const size_t row_smem = (size_t)d * 4;
    const float scale = (float)(1.0 / std::sqrt((double)hd));
    const int nblk = (Tp + r.keys.bl - 1) / r.keys.bl;
    // Which products take their LayerNorm, the GLU and the caches' copies
    // into their own launch (decided once: every block has the same shapes).
    // The LayerNorms by default only for one row (the one-row GEMV's
    // prologue: a streaming chunk step at right context 0, 2.31 -> 2.02 ms);
    // on the K-split kernel each workgroup normalizes its 16-row group
    // itself, which measured slower than the LayerNorm launches at 14 and
    // 16 rows (2.61 -> 2.76 ms a chunk step at right context 13), so there
    // only when CONF_FUSE=3 asks.
    const CBlock &B0 = m->blk[0];
    auto probe = [&](const grx_weight *w, int epi, bool ln, bool ln2, bool ring) {
        GemmOut o;
        o.epi = epi;
        o.y = bf.qkv;
        o.ldc = w->rows;
        o.lens = r.lens;
        o.T = Tp;
        if (ln) {
            o.x = bf.x;
            o.lda = d;
            o.ln_w = B0.norm_attn_w;
            o.ln_b = B0.norm_attn_b;
            if (ln2) {
                o.ln_w2 = B0.norm_attn_w;
                o.ln_b2 = B0.norm_attn_b;
                o.x_out = bf.x2;
            }
        }
        if (ring) {
            o.ring.p = bf.glu;
            o.ring.ctl = r.ctl;
        }
        return grx_gemm_q8_fuses(w, R, o);
    };
    const bool kv_ring = r.kv_ring != nullptr, cv_ring = r.conv_ring != nullptr && padL > 0;
    // the attention's 8-lane groups: blocks of up to 16 rows whose
    // workgroups' scores (rows x the most keys a block sees) and outputs
    // (rows x head width) fit one round of the workgroup's groups
    const int attn_rows_wg = std::min(r.attn_rq, r.keys.bl), attn_keys_max = r.attn_keys;
    const bool attn_g8 = grx_tune(GRX_TUNE_CONF_ATTN_G8) != 0 && r.keys.bl <= 16 &&
                         attn_rows_wg * std::max(attn_keys_max, hd) * 8 <= kAttnLdsThreads;
    // threads of the row-a-workgroup launch (its loops go by the block's
    // size, staging what the registers do not hold straight from memory)
    const int attn_thr = grx_tune(GRX_TUNE_CONF_ATTN_THREADS);
    const int attn1_threads = attn_thr == 256 || attn_thr == 512 ? attn_thr : kAttnLdsThreads;
    const int fz = grx_tune(GRX_TUNE_CONF_FUSE);  // 0 none, 3 LayerNorm prologues on up to 32 rows
    const bool fuse_ln = R <= kFuseLnRows && fz != 0 && (fz == 3 || R == 1) && bf.x2 != nullptr &&
                         probe(B0.qkv, GRX_GEMM_STORE, true, false, kv_ring) &&
                         probe(B0.pw1, GRX_GEMM_GLU, true, false, cv_ring) &&
                         probe(B0.ff1.w1, GRX_GEMM_SILU_Q, true, true, false) &&
                         probe(B0.ff2.w1, GRX_GEMM_SILU_Q, true, false, false);
    const bool fuse_glu = fz != 0 && probe(B0.pw1, GRX_GEMM_GLU, fuse_ln, false, cv_ring);
    const bool fuse_kv = kv_ring && fz != 0 &&
                         probe(B0.qkv, GRX_GEMM_STORE, fuse_ln, false, true);
    // the residual rows: with the LayerNorms fused, each block from the
    // second on continues in the other buffer (its first product stores the
    // previous norm_out there), chosen so that the last block ends in bf.x
    float *x = fuse_ln && (hp.layers - 1) % 2 != 0 ? bf.x2 : bf.x;
    auto other = [&](float *p) { return p == bf.x ? bf.x2 : bf.x; };
    {  // output Linear, then xscale (encoder.go:445-451; stream.go:259)
        GemmOut o;
        o.y = x;
        o.ldc = d;
        if (hp.xscaling) {
            o.epi = GRX_GEMM_SCALE;
            o.scale = (float)std::sqrt((double)d);
        }
        if ((s = grx_gemm_q8_launch_ex(st, m->wout, bf.xq, bf.xs, R, m->outb, o)) != GRX_OK) return s;
    }
    // the first block's feed-forward LayerNorm
    if (!fuse_ln && (s = ln_rows_launch<false, true>(st, R, x, d, B0.ff1.norm_w, B0.ff1.norm_b, nullptr, nullptr,
                                                     bf.xq, bf.xs)) != GRX_OK)
        return s;
    // a product's fused LayerNorm of the residual rows (ln2: the previous
    // block's norm_out first, kept in the other buffer, which the block
    // then continues in)
    auto with_ln = [&](GemmOut &o, const float *w1, const float *b1, const float *w2, const float *b2) {
        if (!fuse_ln) return;
        o.x = x;
        o.lda = d;
        o.ln_w = w1;
        o.ln_b = b1;
        if (w2 != nullptr) {
            o.ln_w2 = w2;
            o.ln_b2 = b2;
            o.x_out = other(x);
        }
    };
    for (int i = 0; i < hp.layers; ++i) {
        const CBlock &Bk = m->blk[i];
        // x += 0.5 * W2 . SiLU(W1 . LN(x)) (encoder.go:244-251); LN(x) is in
        // xq, or made by W1's prologue (the first feed-forward of a block
        // after the first: the previous block's norm_out, then its own LN)
        auto ff_pair = [&](const CFF &F, const CBlock *prev) -> grx_status {
            GemmOut o1;
            o1.epi = GRX_GEMM_SILU_Q;
            o1.yq = bf.fq;
            o1.ys = bf.fs;
            if (prev != nullptr)
                with_ln(o1, prev->norm_out_w, prev->norm_out_b, F.norm_w, F.norm_b);
            else
                with_ln(o1, F.norm_w, F.norm_b, nullptr, nullptr);
            grx_status q = grx_gemm_q8_launch_ex(st, F.w1, bf.xq, bf.xs, R, F.b1, o1);
            if (q != GRX_OK) return q;
            if (o1.x_out != nullptr) x = o1.x_out;
            GemmOut o2;
            o2.y = x;
            o2.ldc = d;
            o2.epi = GRX_GEMM_AXPY_HALF;
            return grx_gemm_q8_launch_ex(st, F.w2, bf.fq, bf.fs, R, F.b2, o2);
        };
        if ((s = ff_pair(Bk.ff1, fuse_ln && i > 0 ? &m->blk[i - 1] : nullptr)) != GRX_OK) return s;
        // attention (encoder.go:259-330)
        if (!fuse_ln && (s = ln_rows_launch<false, true>(st, R, x, d, Bk.norm_attn_w, Bk.norm_attn_b, nullptr, nullptr,
                                                         bf.xq, bf.xs)) != GRX_OK)
            return s;
        float *ring = r.kv_ring ? r.kv_ring + r.kv_ring_layer * i : nullptr;
        {
            GemmOut o;
            o.y = bf.qkv;
            o.ldc = 3 * d;
            with_ln(o, Bk.norm_attn_w, Bk.norm_attn_b, nullptr, nullptr);
            if (fuse_kv) {
                // the chunk's keys and values (columns d..3d) into the
                // stream's ring as well: row i to slot (head + c + i) % cap
                // and + cap (kv_ring_append_kernel's layout)
                o.ring.p = ring;
                o.ring.bstride = (size_t)2 * r.cap * 2 * d;
                o.ring.width = 2 * d;
                o.ring.col0 = d;
                o.ring.cap = r.cap;
                o.ring.twice = 1;
                o.ring.T = Tp;
                o.ring.ctl = r.ctl;
                o.ring.c0 = 0;
                o.ring.c1 = 1;
            }
            if ((s = grx_gemm_q8_launch_ex(st, Bk.qkv, bf.xq, bf.xs, R, Bk.qkv_b, o)) != GRX_OK) return s;
        }
        AttnIO io{};
        io.q = bf.qkv;
        io.ldq = 3 * d;
        io.lens = r.lens;
        io.T = Tp;
        if (ring) {
            // the chunk's keys and values join the stream's ring, which then
            // holds every key of the chunk's queries
            if (!fuse_kv) {
                kv_ring_append_kernel<<<grid_for((size_t)R * 2 * d), 256, 0, st>>>(bf.qkv, B, Tp, d, ring, r.cap,
                                                                                   r.ctl);
                GRX_LAUNCHED("kv_ring_append_kernel");
            }
            io.kv = ring;
            io.ldkv = 2 * d;
            io.vo = d;
            io.kvb = (size_t)2 * r.cap * 2 * d;
            io.pp = r.pp + (size_t)i * d;
            io.ldp = hp.layers * d;
            io.maxfirst = r.maxfirst;
            io.ctl = r.ctl;
        } else {
            io.kv = bf.qkv + d;
            io.ldkv = 3 * d;
            io.vo = d;
            io.kvb = (size_t)Tp * 3 * d;
            io.pp = r.pp + (size_t)i * d;
            io.ldp = hp.layers * d;
        }
        if (r.attn_rq == 1)
            conf_attn_lds_kernel<1, true><<<dim3(nblk * r.keys.bl, hp.heads, B), attn1_threads, r.attn_smem, st>>>(
                io, r.keys, Bk.pos_u, Bk.pos_v, d, hd, scale, bf.xq, bf.xs);
        else if (r.attn_rq == 4 && attn_g8)
            conf_attn_lds_kernel<4, true><<<dim3(nblk * ((r.keys.bl + 3) / 4), hp.heads, B), kAttnLdsThreads,
                                            r.attn_smem, st>>>(io, r.keys, Bk.pos_u, Bk.pos_v, d, hd, scale, bf.xq,
                                                               bf.xs);
        else if (r.attn_rq == 4)
            conf_attn_lds_kernel<4><<<dim3(nblk * ((r.keys.bl + 3) / 4), hp.heads, B), kAttnLdsThreads, r.attn_smem,
                                      st>>>(io, r.keys, Bk.pos_u, Bk.pos_v, d, hd, scale, bf.xq, bf.xs);
        else if (r.attn_rq == 8)
            conf_attn_lds_kernel<8><<<dim3(nblk * ((r.keys.bl + 7) / 8), hp.heads, B), kAttnLdsThreads, r.attn_smem,
                                      st>>>(io, r.keys, Bk.pos_u, Bk.pos_v, d, hd, scale, bf.xq, bf.xs);
        else if (r.attn_rq == 16)
            conf_attn_lds_kernel<16><<<dim3(nblk * ((r.keys.bl + 15) / 16), hp.heads, B), kAttnLdsThreads,
                                       r.attn_smem, st>>>(io, r.keys, Bk.pos_u, Bk.pos_v, d, hd, scale, bf.xq, bf.xs);
        else
            conf_attn_kernel<<<dim3(nblk, hp.heads, B), kAttnThreads, r.attn_smem, st>>>(io, r.keys, Bk.pos_u,
                                                                                         Bk.pos_v, d, hd, scale,
                                                                                         bf.xq, bf.xs);
        GRX_LAUNCHED("conf_attn_kernel");
        {
            GemmOut o;
            o.y = x;
            o.ldc = d;
            o.epi = GRX_GEMM_ADD;
            if ((s = grx_gemm_q8_launch_ex(st, Bk.out, bf.xq, bf.xs, R, Bk.out_b, o)) != GRX_OK) return s;
        }
        // convolution module (encoder.go:343-397)
        if (!fuse_ln && (s = ln_rows_launch<false, true>(st, R, x, d, Bk.norm_conv_w, Bk.norm_conv_b, nullptr, nullptr,
                                                         bf.xq, bf.xs)) != GRX_OK)
            return s;
        ConvPrev cp{};
        if (cv_ring) {
            cp.ring = r.conv_ring + r.conv_ring_layer * i;
            cp.cap = r.conv_cap;
            cp.ctl = r.ctl;
        }
        // pointwise1 (its rows paired for the GLU), the GLU (rows past an
        // utterance's valid rows zeroed), and the chunk's gated frames into
        // the stream's convolution ring: frame i to slot (ctl[2] + i) % cap
        if (fuse_glu) {
            GemmOut o;
            o.epi = GRX_GEMM_GLU;
            o.y = bf.glu;
            o.ldc = d;
            o.lens = r.lens;
            o.T = Tp;
            with_ln(o, Bk.norm_conv_w, Bk.norm_conv_b, nullptr, nullptr);
            if (cv_ring) {
                o.ring.p = const_cast<float *>(cp.ring);
                o.ring.bstride = (size_t)cp.cap * d;
                o.ring.width = d;
                o.ring.cap = cp.cap;
                o.ring.T = Tp;
                o.ring.ctl = r.ctl;
                o.ring.c0 = 2;
            }
            if ((s = grx_gemm_q8_launch_ex(st, Bk.pw1, bf.xq, bf.xs, R, Bk.pw1_b, o)) != GRX_OK) return s;
        } else {
            if ((s = grx_gemm_q8_launch(st, Bk.pw1, bf.xq, bf.xs, R, Bk.pw1_b, bf.conv, 2 * d)) != GRX_OK) return s;
            conf_glu_kernel<<<grid_for((size_t)R * d), 256, 0, st>>>(bf.conv, R, Tp, d, r.lens, bf.glu);
            GRX_LAUNCHED("conf_glu_kernel");
            if (cp.ring) {
                conv_ring_append_kernel<<<grid_for((size_t)R * d), 256, 0, st>>>(bf.glu, B, Tp, d,
                                                                                  const_cast<float *>(cp.ring),
                                                                                  cp.cap, r.ctl);
                GRX_LAUNCHED("conv_ring_append_kernel");
            }
        }
        // the depthwise kernel: 0 a workgroup per row, 1 LDS windows, 2 a
        // wave per frame (measured at the parakeet shape: 5.2 us against 10.6
        // for 126 rows, 25.5 against 22.8 for 2016, where the windows' reuse
        // of each loaded frame pays)
        const bool dw_lane = d % 64 == 0 && hp.conv_kernel <= kDwLaneK && !hp.conv_ln;
        int dw = grx_tune(GRX_TUNE_CONF_DW);
        if (dw < 0 || dw > 2) dw = dw_lane && R <= 1024 ? 2 : 1;
        if (dw == 2 && !dw_lane) dw = 1;
        if (dw == 1 && !r.dw_win) dw = 0;
        // with the LayerNorm: a row per workgroup of float4 pieces where
        // the row has at most 1024 channels and the kernel at most 16 taps
        // (one row at d 1024: 5.4 us a launch, against 11.0 for the row per
        // workgroup with workgroup-wide reductions), else that kernel
        const bool dw_ln4 = d <= 1024 && hp.conv_kernel <= 16 && grx_tune(GRX_TUNE_CONF_DW) != 0;
        const int dw_ln_threads = 64 * grx_ceil_div(d / 4, 64);
        if (hp.conv_ln && dw_ln4 && hp.conv_kernel <= 12)
            conf_dwconv_ln_kernel<12><<<R, dw_ln_threads, 0, st>>>(bf.glu, Tp, d, hp.conv_kernel, padL, cp, Bk.dw,
                                                                   Bk.dw_b, Bk.cn_w, Bk.cn_b, bf.xq, bf.xs);
        else if (hp.conv_ln && dw_ln4)
            conf_dwconv_ln_kernel<16><<<R, dw_ln_threads, 0, st>>>(bf.glu, Tp, d, hp.conv_kernel, padL, cp, Bk.dw,
                                                                   Bk.dw_b, Bk.cn_w, Bk.cn_b, bf.xq, bf.xs);
        else if (hp.conv_ln)
            conf_dwconv_kernel<true><<<R, kRowThreads, row_smem, st>>>(bf.glu, Tp, d, hp.conv_kernel, padL, cp, Bk.dw,
                                                                       Bk.dw_b, Bk.cn_w, Bk.cn_b, bf.xq, bf.xs);
        else if (dw == 2 && cp.ring != nullptr)
            conf_dwconv_lane_kernel<true><<<dim3(Tp, d / 64, B), 64, 0, st>>>(
                bf.glu, Tp, d, hp.conv_kernel, padL, cp, Bk.dw, Bk.dw_b, Bk.cn_w, Bk.cn_b, bf.xq, bf.xs);
        else if (dw == 2)
            conf_dwconv_lane_kernel<false><<<dim3(Tp, d / 64, B), 64, 0, st>>>(
                bf.glu, Tp, d, hp.conv_kernel, padL, cp, Bk.dw, Bk.dw_b, Bk.cn_w, Bk.cn_b, bf.xq, bf.xs);
        else if (dw == 1)
            conf_dwconv_win_kernel<<<dim3((Tp + kDwRows - 1) / kDwRows, d / 64, B), 256,
                                     (size_t)(kDwRows + 2 * hp.conv_kernel - 1) * 64 * 4, st>>>(
                bf.glu, Tp, d, hp.conv_kernel, padL, cp, Bk.dw, Bk.dw_b, Bk.cn_w, Bk.cn_b, bf.xq, bf.xs);
        else
            conf_dwconv_kernel<false><<<R, kRowThreads, row_smem, st>>>(bf.glu, Tp, d, hp.conv_kernel, padL, cp,
                                                                        Bk.dw, Bk.dw_b, Bk.cn_w, Bk.cn_b, bf.xq,
                                                                        bf.xs);
        GRX_LAUNCHED("conf_dwconv_kernel");
        {
            GemmOut o;
            o.y = x;
            o.ldc = d;
            o.epi = GRX_GEMM_ADD;
            if ((s = grx_gemm_q8_launch_ex(st, Bk.pw2, bf.xq, bf.xs, R, Bk.pw2_b, o)) != GRX_OK) return s;
        }
        // second feed-forward, then norm_out (and the next block's first
        // LayerNorm; fused: the next block's first product does both)
        if (!fuse_ln && (s = ln_rows_launch<false, true>(st, R, x, d, Bk.ff2.norm_w, Bk.ff2.norm_b, nullptr, nullptr,
                                                         bf.xq, bf.xs)) != GRX_OK)
            return s;
        if ((s = ff_pair(Bk.ff2, nullptr)) != GRX_OK) return s;
        if (i + 1 < hp.layers) {
            if (!fuse_ln) {
                const CFF &N = m->blk[i + 1].ff1;
                if ((s = ln_rows_launch<true, true>(st, R, x, d, Bk.norm_out_w, Bk.norm_out_b, N.norm_w, N.norm_b,
                                                    bf.xq, bf.xs)) != GRX_OK)
                    return s;
            }
        } else {
            if ((s = ln_rows_launch<true, false>(st, R, x, d, Bk.norm_out_w, Bk.norm_out_b, nullptr, nullptr, nullptr,
                                                 nullptr)) != GRX_OK)
                return s;
        }
    }
    if (x != bf.x) return grx_fail(GRX_EINVAL, "conformer: the blocks ended in the wrong buffer");
    return GRX_OK;
}

// The whole offline encode (encoder.go:432-489) of m->B utterances from
// m->mel into m->x, enqueued on the stream: every block's position
// projection first (pp [2T-1][layers*d]), then the run.
grx_status enqueue_encode(grx_conformer *m, hipStream_t st) {
    const grx_conformer_hparams &hp = m->hp;
    const int T = m->T;
    grx_status s = grx_gemm_q8_launch(st, m->pos_all, m->pos_q, m->pos_s, 2 * T - 1, nullptr, m->pp, hp.layers * hp.d);
    if (s != GRX_OK) return s;
    CRun r{};
    r.B = m->B;
    r.frames = m->frames;
    r.T = r.Tp = T;
    r.b.mel = m->mel, r.b.sub0 = m->sub0, r.b.suby = m->suby, r.b.subx = m->subx, r.b.x = m->x, r.b.x2 = m->x2;
    r.b.qkv = m->qkv;
    r.b.conv = m->conv, r.b.glu = m->glu, r.b.xq = m->xq, r.b.xs = m->xs, r.b.fq = m->fq, r.b.fs = m->fs;
    r.valid = m->valid;
    r.lens = m->valid + m->B;
    r.keys = offline_keys(hp, T);
    r.pp = m->pp;
    r.attn_rq = m->attn_rq;
    r.attn_keys = T;
    r.attn_smem = m->attn_smem;
    r.dw_win = m->dw_win;
    return enqueue_run(m, r, st);
}

grx_status run_graph(hipStream_t st, hipGraph_t *graph, hipGraphExec_t *exec,
                     const std::function<grx_status(hipStream_t)> &enqueue) {
    if (grx_tune(GRX_TUNE_NO_GRAPH) == 1) return enqueue(st);
    if (!*exec) {
        GRX_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        grx_status s = enqueue(st);
        hipGraph_t g = nullptr;
        hipError_t e = hipStreamEndCapture(st, &g);
        if (s != GRX_OK) {
            if (g) (void)hipGraphDestroy(g);
            return s;
        }
        if (e != hipSuccess) return grx_fail(GRX_EDEVICE, "graph capture: %s", hipGetErrorString(e));
        *graph = g;
        GRX_HIP(hipGraphInstantiate(exec, g, nullptr, nullptr, 0));
    }
    GRX_HIP(hipGraphLaunch(*exec, st));
    return GRX_OK;
}

grx_status run_encode(grx_conformer *m) {
    return run_graph(m->ctx->stream, &m->graph, &m->exec, [m](hipStream_t st) { return enqueue_encode(m, st); });
}

grx_status check_valid(const grx_conformer *m, const int *valid, int batch, int frames) {
    (void)m;
    for (int b = 0; b < batch; ++b)
        if (valid[b] < 1 || valid[b] > frames)
            return grx_fail(GRX_EINVAL, "utterance %d: valid frames %d outside [1, %d]", b, valid[b], frames);
    return GRX_OK;
}

// The encoder rows of an utterance of `valid` frames out of T (encoder.go:166).
int enc_rows(const grx_conformer_hparams &hp, int valid, int T) {
    return std::max(0, std::min(stage_len(valid, 3, hp.causal_sub), T));
}

grx_status encode_common(grx_conformer *m, const float *mel, int batch, int frames, const int *valid,
                         hipMemcpyKind kind) {
    grx_status s;
    if ((s = check_valid(m, valid, batch, frames)) != GRX_OK) return s;
    GRX_HIP(hipSetDevice(m->ctx->device));
    if ((s = cfinalize(m)) != GRX_OK) return s;
    if ((s = cshape(m, batch, frames)) != GRX_OK) return s;
    hipStream_t st = m->ctx->stream;
    const size_t mel_n = (size_t)batch * m->hp.n_mels * frames;
    for (int b = 0; b < batch; ++b) {
        m->valid_host[b] = valid[b];
        m->valid_host[batch + b] = enc_rows(m->hp, valid[b], m->T);
    }
    GRX_HIP(hipMemcpyAsync(m->valid, m->valid_host, 2 * (size_t)batch * sizeof(int), hipMemcpyHostToDevice, st));
    GRX_HIP(hipMemcpyAsync(m->mel, mel, mel_n * 4, kind, st));
    return run_encode(m);
}

}  // namespace

// ---------------------------------------------------------------- streams

struct grx_conformer_stream {
    grx_conformer *m = nullptr;
    int B = 0;
    grx_conformer_stream_geom g{};
    int cap = 0, padL = 0, maxfirst = 0;
    int conv_cap = 0;  // rows of a stream's convolution ring: padL + chunk
    bool dw_win = false;
    int steps = 0;                          // chunks done
    int kv_len = 0, kv_head = 0, conv_head = 0;
    std::vector<void *> allocs;
    float *kv_ring = nullptr;    // [layers][B][2*cap][2d]: keys | values
    float *conv_ring = nullptr;  // [layers][B][conv_cap][d]
    float *pp = nullptr;         // [left+2*chunk-1][layers*d]: positions maxfirst down, projected
    int *ctl = nullptr;          // device [4 + 2B]: c, kv head, conv head, 0, mel frames[B], rows[B]
    int *ctl_host = nullptr;     // pinned
    // working buffers, for chunks of up to buf_frames mel frames
    int buf_frames = 0;
    std::vector<void *> work;
    CBuf b;
    struct Shape {
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        int attn_rq = 0;
        size_t attn_smem = 0;
    };
    std::map<std::pair<int, int>, Shape> shapes;  // by (frames, first)
};

namespace {

void stream_free_work(grx_conformer_stream *s) {
    for (auto &kv : s->shapes) {
        if (kv.second.exec) (void)hipGraphExecDestroy(kv.second.exec);
        if (kv.second.graph) (void)hipGraphDestroy(kv.second.graph);
    }
    s->shapes.clear();
    for (void *p : s->work) (void)hipFree(p);
    s->work.clear();
    s->b = CBuf();
    s->buf_frames = 0;
}

// newGeom (stream.go:23-69).
grx_status stream_geom(const grx_conformer_hparams &hp, int right, grx_conformer_stream_geom *g) {
    if (!hp.att_chunked) return grx_fail(GRX_EINVAL, "conformer: this model can't stream");
    int left = -1;
    for (int i = 0; i < hp.n_context_choices; ++i)
        if (hp.context_choices[i][1] == right) left = hp.context_choices[i][0];
    if (hp.n_context_choices == 0 && right == hp.att_right) left = hp.att_left;
    if (left < 0 || right < 0)
        return grx_fail(GRX_EINVAL, "conformer: the model wasn't trained for a right context of %d", right);
    const int sub = 8;
    const int cache = hp.pre_encode_cache < 0 ? sub + 1 : hp.pre_encode_cache;
    const int drop = hp.drop_extra < 0 ? 1 + (cache - 1) / sub : hp.drop_extra;
    const int first = hp.sampling_frames_first < 0 ? 1 : hp.sampling_frames_first;
    g->right = right;
    g->chunk = right + 1;
    g->left = left;
    g->left_chunks = left / g->chunk;
    g->mel_first = first + sub * right;
    g->mel_next = sub * g->chunk;
    g->mel_cache = cache;
    g->drop = drop;
    g->sample_first = first;
    return GRX_OK;
}

grx_status stream_bufs(grx_conformer_stream *s, int frames) {
    if (frames <= s->buf_frames) return GRX_OK;
    stream_free_work(s);
    const int T = stage_len(frames, 3, s->m->hp.causal_sub);
    grx_status r = cbuf_alloc(s->m, s->work, s->B, frames, T, &s->b);
    if (r != GRX_OK) return r;
    s->buf_frames = frames;
    return GRX_OK;
}

// One chunk: the pre-encoder over it, its first rows dropped unless it is
// the stream's first, then the blocks with the caches (stream.go:249-307).
grx_status stream_run(grx_conformer_stream *s, const float *mel, int nf, const int *length, hipMemcpyKind kind,
                      int *Tp_out) {
    grx_conformer *m = s->m;
    const grx_conformer_hparams &hp = m->hp;
    const int B = s->B, first = s->steps == 0;
    const int T = stage_len(nf, 3, hp.causal_sub), drop = first ? 0 : std::min(s->g.drop, T);
    const int Tp = T - drop;
    *Tp_out = Tp;
    if (Tp <= 0) return GRX_OK;  // stream.go:262-264: no rows, nothing changes
    if (Tp > s->g.chunk)
        return grx_fail(GRX_ESIZE, "a chunk of %d mel frames gives %d encoder rows, more than the stream's %d", nf, Tp,
                        s->g.chunk);
    grx_status r;
    if ((r = stream_bufs(s, nf)) != GRX_OK) return r;
    auto key = std::make_pair(nf, first);
    auto it = s->shapes.find(key);
    if (it == s->shapes.end()) {
        grx_conformer_stream::Shape sh;
        // LDS for the most keys a chunk's queries see: the full left
        // context and the chunk's own rows
        if ((r = attn_pick(B, hp.heads, 1, Tp, s->g.left + Tp, hp.d / hp.heads, &sh.attn_rq, &sh.attn_smem)) !=
            GRX_OK)
            return r;
        it = s->shapes.emplace(key, sh).first;
    }
    hipStream_t st = m->ctx->stream;
    s->ctl_host[0] = s->kv_len;
    s->ctl_host[1] = s->kv_head;
    s->ctl_host[2] = s->conv_head;
    s->ctl_host[3] = 0;
    for (int b = 0; b < B; ++b) {
        int L = stage_len(length[b], 3, hp.causal_sub);  // subsample's L, then the drop (stream.go:253-260)
        L = std::max(0, std::min(L, T));
        L = std::max(0, L - drop);
        s->ctl_host[4 + b] = length[b];
        s->ctl_host[4 + B + b] = std::min(L, Tp);
    }
    GRX_HIP(hipMemcpyAsync(s->ctl, s->ctl_host, (size_t)(4 + 2 * B) * sizeof(int), hipMemcpyHostToDevice, st));
    GRX_HIP(hipMemcpyAsync(s->b.mel, mel, (size_t)B * hp.n_mels * nf * 4, kind, st));
    grx_conformer_stream::Shape &sh = it->second;
    CRun run{};
    run.B = B;
    run.frames = nf;
    run.T = T;
    run.Tp = Tp;
    run.drop = drop;
    run.b = s->b;
    run.valid = s->ctl + 4;
    run.lens = s->ctl + 4 + B;
    run.keys.mode = kKeysStream;
    run.keys.bl = Tp;  // stream.go:272: one block of the chunk's rows
    run.keys.chunk = s->g.chunk;
    run.keys.lchunks = s->g.left_chunks;
    run.keys.left = s->g.left;
    run.pp = s->pp;
    run.maxfirst = s->maxfirst;
    run.ctl = s->ctl;
    run.attn_rq = sh.attn_rq;
    run.attn_keys = s->g.left + Tp;
    run.attn_smem = sh.attn_smem;
    run.dw_win = s->dw_win;
    run.kv_ring = s->kv_ring;
    run.kv_ring_layer = (size_t)B * 2 * s->cap * 2 * hp.d;
    run.cap = s->cap;
    run.conv_ring = s->padL > 0 ? s->conv_ring : nullptr;
    run.conv_ring_layer = (size_t)B * s->conv_cap * hp.d;
    run.conv_cap = s->conv_cap;
    if ((r = run_graph(st, &sh.graph, &sh.exec, [m, run](hipStream_t q) { return enqueue_run(m, run, q); })) != GRX_OK)
        return r;
    // the caches after the chunk (stream.go:296-306)
    const int Tk = s->kv_len + Tp, keep = std::min(Tk, s->g.left);
    s->kv_head = (s->kv_head + Tk - keep) % s->cap;
    s->kv_len = keep;
    if (s->padL > 0) s->conv_head = (s->conv_head + Tp) % s->conv_cap;
    s->steps++;
    return GRX_OK;
}

grx_status stream_step(grx_conformer_stream *s, const float *mel, int nf, const int *length, float *out, int *lens,
                       hipMemcpyKind in, hipMemcpyKind outk) {
    if (!s || !mel || !length || !out) return grx_fail(GRX_EINVAL, "grx_conformer_stream_step: NULL argument");
    if (nf < 1) return grx_fail(GRX_EINVAL, "grx_conformer_stream_step: %d frames", nf);
    for (int b = 0; b < s->B; ++b)
        if (length[b] < 1 || length[b] > nf)
            return grx_fail(GRX_EINVAL, "stream %d: length %d outside [1, %d]", b, length[b], nf);
    GRX_HIP(hipSetDevice(s->m->ctx->device));
    int Tp = 0;
    grx_status r = stream_run(s, mel, nf, length, in, &Tp);
    if (r != GRX_OK) return r;
    const int d = s->m->hp.d, B = s->B, chunk = s->g.chunk;
    hipStream_t st = s->m->ctx->stream;
    if (Tp > 0) {
        GRX_HIP(hipMemcpy2DAsync(out, (size_t)chunk * d * 4, s->b.x, (size_t)Tp * d * 4, (size_t)Tp * d * 4, B, outk,
                                 st));
    }
    // the pinned control values are read by the copy above: wait before reuse
    GRX_HIP(hipStreamSynchronize(st));
    if (lens)
        for (int b = 0; b < B; ++b) lens[b] = Tp > 0 ? s->ctl_host[4 + B + b] : 0;
    return GRX_OK;
}

}  // namespace

extern "C" grx_status grx_conformer_stream_create(grx_conformer *m, int right, int batch, grx_conformer_stream **out) {
    if (!m || !out) return grx_fail(GRX_EINVAL, "grx_conformer_stream_create: NULL argument");
    *out = nullptr;
    if (batch < 1 || batch > 4096) return grx_fail(GRX_EINVAL, "grx_conformer_stream_create: batch %d", batch);
    grx_conformer_stream_geom g;
    grx_status r;
    if ((r = stream_geom(m->hp, right, &g)) != GRX_OK) return r;
    if (g.chunk > kAttnQ)
        return grx_fail(GRX_ESIZE, "a chunk of %d rows is more than the attention kernels take (%d)", g.chunk, kAttnQ);
    GRX_HIP(hipSetDevice(m->ctx->device));
    if ((r = cfinalize(m)) != GRX_OK) return r;
    const grx_conformer_hparams &hp = m->hp;
    grx_conformer_stream *s = new grx_conformer_stream();
    s->m = m;
    s->B = batch;
    s->g = g;
    s->cap = g.left + g.chunk;
    s->padL = pad_left(hp);
    s->conv_cap = s->padL + g.chunk;
    s->maxfirst = g.left + g.chunk - 1;
    s->dw_win = dw_win_ok(hp);
    auto fail = [&](grx_status e) {
        grx_conformer_stream_destroy(s);
        return e;
    };
    // working buffers for the longest chunk that gives at most one chunk of
    // rows after the drop, so that no step allocates (or recaptures a
    // shape's graph for new buffers)
    {
        int nf = 1;
        while (stage_len(nf + 1, 3, hp.causal_sub) - g.drop <= g.chunk) ++nf;
        if ((r = stream_bufs(s, std::max(nf, g.mel_first))) != GRX_OK) return fail(r);
    }
    const int d = hp.d, count = g.left + 2 * g.chunk - 1;
    if ((r = calloc_t(s->allocs, (size_t)hp.layers * batch * 2 * s->cap * 2 * d, &s->kv_ring)) != GRX_OK) return fail(r);
    if ((r = calloc_t(s->allocs, (size_t)hp.layers * batch * s->conv_cap * d, &s->conv_ring)) != GRX_OK)
        return fail(r);
    if ((r = calloc_t(s->allocs, (size_t)count * hp.layers * d, &s->pp)) != GRX_OK) return fail(r);
    if ((r = calloc_t(s->allocs, (size_t)4 + 2 * batch, &s->ctl)) != GRX_OK) return fail(r);
    if (grx_pinned_malloc((void **)&s->ctl_host, (size_t)(4 + 2 * batch) * sizeof(int)) != hipSuccess) {
        (void)hipGetLastError();
        s->ctl_host = nullptr;
        return fail(grx_fail(GRX_ENOMEM, "grx_conformer_stream_create: pinned memory"));
    }
    // newEncState: zero convolution caches (newEncState, stream.go:80-88),
    // and the projected positions left+chunk-1 .. -(chunk-1) of every layer
    if (hipMemset(s->conv_ring, 0, (size_t)hp.layers * batch * s->conv_cap * d * 4) != hipSuccess)
        return fail(grx_hip_fail(hipGetLastError(), "hipMemset"));
    {
        std::vector<float> pos = rel_pos(s->maxfirst, count, d);
        float *dpos = nullptr, *dps = nullptr;
        int8_t *dpq = nullptr;
        std::vector<void *> tmp;
        auto done = [&](grx_status e) {
            for (void *p : tmp) (void)hipFree(p);
            return e;
        };
        if ((r = calloc_t(tmp, pos.size(), &dpos)) != GRX_OK || (r = calloc_t(tmp, pos.size(), &dpq)) != GRX_OK ||
            (r = calloc_t(tmp, pos.size() / 32, &dps)) != GRX_OK)
            return fail(done(r));
        if (hipMemcpy(dpos, pos.data(), pos.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
            return fail(done(grx_hip_fail(hipGetLastError(), "hipMemcpy")));
        if ((r = grx_quant_act_dev(m->ctx, dpq, dps, dpos, d, count, d)) != GRX_OK ||
            (r = grx_gemm_q8_launch(m->ctx->stream, m->pos_all, dpq, dps, count, nullptr, s->pp, hp.layers * d)) !=
                GRX_OK)
            return fail(done(r));
        if (hipStreamSynchronize(m->ctx->stream) != hipSuccess)
            return fail(done(grx_hip_fail(hipGetLastError(), "hipStreamSynchronize")));
        done(GRX_OK);
    }
    *out = s;
    return GRX_OK;
}

extern "C" grx_status grx_conformer_stream_destroy(grx_conformer_stream *s) {
    if (!s) return GRX_OK;
    GRX_HIP(hipSetDevice(s->m->ctx->device));
    stream_free_work(s);
    for (void *p : s->allocs) (void)hipFree(p);
    if (s->ctl_host) (void)hipHostFree(s->ctl_host);
    delete s;
    return GRX_OK;
}

extern "C" grx_status grx_conformer_stream_geometry(const grx_conformer_stream *s, grx_conformer_stream_geom *g) {
    if (!s || !g) return grx_fail(GRX_EINVAL, "grx_conformer_stream_geometry: NULL argument");
    *g = s->g;
    return GRX_OK;
}

extern "C" grx_status grx_conformer_stream_step(grx_conformer_stream *s, const float *mel, int nf, const int *length,
                                                float *out, int *lens) {
    return stream_step(s, mel, nf, length, out, lens, hipMemcpyHostToDevice, hipMemcpyDeviceToHost);
}

extern "C" grx_status grx_conformer_stream_step_dev(grx_conformer_stream *s, const float *mel, int nf,
                                                    const int *length, float *out, int *lens) {
    return stream_step(s, mel, nf, length, out, lens, hipMemcpyDeviceToDevice, hipMemcpyDeviceToDevice);
}

// ---------------------------------------------------------------- the model

extern "C" grx_status grx_conformer_create(grx_ctx *ctx, const grx_conformer_hparams *hp, grx_conformer **out) {
    if (!ctx || !hp || !out) return grx_fail(GRX_EINVAL, "grx_conformer_create: NULL argument");
    *out = nullptr;
    if (hp->d <= 0 || hp->heads <= 0 || hp->layers <= 0 || hp->dff <= 0 || hp->conv_kernel <= 0 ||
        hp->sub_channels <= 0 || hp->n_mels <= 0)
        return grx_fail(GRX_EINVAL, "grx_conformer_create: every size must be positive");
    if (hp->d % 32 != 0 || hp->dff % 32 != 0 || hp->d % hp->heads != 0 || (hp->d / hp->heads) % 32 != 0)
        return grx_fail(GRX_ESIZE, "d %d, dff %d, heads %d: sizes must split into 32-value blocks per head", hp->d,
                        hp->dff, hp->heads);
    if (hp->sub_channels % 32 != 0 || hp->sub_channels > 1024 || hp->d > 8192)
        return grx_fail(GRX_ESIZE, "sub_channels %d (a multiple of 32 up to 1024) or d %d unsupported",
                        hp->sub_channels, hp->d);
    if (hp->att_left < -1 || hp->att_right < -1 || hp->conv_left < -1 || hp->conv_right < -1)
        return grx_fail(GRX_EINVAL, "grx_conformer_create: a context limit below -1");
    const bool conv_padded = hp->conv_left >= 0 && hp->conv_right >= 0;
    if (conv_padded ? hp->conv_left + hp->conv_right + 1 != hp->conv_kernel : hp->conv_kernel % 2 != 1)
        return grx_fail(GRX_ESIZE, "convolution padding %d + %d does not fit kernel %d", hp->conv_left,
                        hp->conv_right, hp->conv_kernel);
    if (hp->att_chunked && hp->att_left >= 0 && hp->att_right >= 0 && hp->att_right + 1 > kAttnQ)
        return grx_fail(GRX_ESIZE, "chunks of %d rows are more than the attention kernels take (%d)",
                        hp->att_right + 1, kAttnQ);
    if (hp->n_context_choices < 0 || hp->n_context_choices > 8)
        return grx_fail(GRX_EINVAL, "grx_conformer_create: %d context choices (at most 8)", hp->n_context_choices);
    for (int i = 0; i < hp->n_context_choices; ++i)
        if (hp->context_choices[i][0] < -1 || hp->context_choices[i][1] < -1 ||
            hp->context_choices[i][1] + 1 > kAttnQ)
            return grx_fail(GRX_EINVAL, "context choice [%d, %d] unsupported", hp->context_choices[i][0],
                            hp->context_choices[i][1]);
    if ((hp->sub_channels * sub_F(*hp)) % 32 != 0)
        return grx_fail(GRX_ESIZE, "the pre-encoder output (%d values) is not whole Q8_0 blocks",
                        hp->sub_channels * sub_F(*hp));
    grx_conformer *m = new grx_conformer();
    m->ctx = ctx;
    m->hp = *hp;
    *out = m;
    return GRX_OK;
}

extern "C" grx_status grx_conformer_destroy(grx_conformer *m) {
    if (!m) return GRX_OK;
    GRX_HIP(hipSetDevice(m->ctx->device));
    free_work(m);
    crelease(m);
    delete m;
    return GRX_OK;
}

extern "C" grx_status grx_conformer_set_tensor(grx_conformer *m, const char *name, const void *data, size_t nbytes) {
    if (!m || !name || (!data && nbytes)) return grx_fail(GRX_EINVAL, "grx_conformer_set_tensor: NULL argument");
    if (m->ready) return grx_fail(GRX_ESTATE, "grx_conformer_set_tensor: the model is in use already");
    for (const CExpect &e : cexpected(m->hp)) {
        if (e.name != name) continue;
        if (e.bytes != 0 && nbytes != e.bytes)
            return grx_fail(GRX_ESIZE, "tensor %s has the wrong shape (%zu bytes, want %zu)", name, nbytes, e.bytes);
        const uint8_t *p = static_cast<const uint8_t *>(data);
        m->host[name] = std::vector<uint8_t>(p, p + nbytes);
        return GRX_OK;
    }
    return grx_fail(GRX_EINVAL, "the model has a tensor this program doesn't know: %s", name);
}

extern "C" int grx_conformer_frames_out(const grx_conformer *m, int frames) {
    return frames < 1 ? 0 : stage_len(frames, 3, m ? m->hp.causal_sub : 0);
}

extern "C" grx_status grx_conformer_encode_dev(grx_conformer *m, const float *mel, int batch, int frames,
                                               const int *valid, float *out) {
    if (!m || !mel || !valid || !out) return grx_fail(GRX_EINVAL, "grx_conformer_encode_dev: NULL argument");
    if (batch < 1 || frames < 1) return grx_fail(GRX_EINVAL, "grx_conformer_encode_dev: batch %d, frames %d", batch, frames);
    grx_status s;
    if ((s = encode_common(m, mel, batch, frames, valid, hipMemcpyDeviceToDevice)) != GRX_OK) return s;
    hipStream_t st = m->ctx->stream;
    GRX_HIP(hipMemcpyAsync(out, m->x, (size_t)batch * m->T * m->hp.d * 4, hipMemcpyDeviceToDevice, st));
    // the pinned valid lengths are read by the copy above: wait before reuse
    GRX_HIP(hipStreamSynchronize(st));
    return GRX_OK;
}

extern "C" grx_status grx_conformer_encode(grx_conformer *m, const float *mel, int batch, int frames, const int *valid,
                                           float *out, int *lens) {
    if (!m || !mel || !valid || !out) return grx_fail(GRX_EINVAL, "grx_conformer_encode: NULL argument");
    if (batch < 1 || frames < 1) return grx_fail(GRX_EINVAL, "grx_conformer_encode: batch %d, frames %d", batch, frames);
    grx_status s;
    if ((s = encode_common(m, mel, batch, frames, valid, hipMemcpyHostToDevice)) != GRX_OK) return s;
    hipStream_t st = m->ctx->stream;
    GRX_HIP(hipMemcpyAsync(out, m->x, (size_t)batch * m->T * m->hp.d * 4, hipMemcpyDeviceToHost, st));
    GRX_HIP(hipStreamSynchronize(st));
    if (lens)
        for (int b = 0; b < batch; ++b) lens[b] = enc_rows(m->hp, valid[b], m->T);
    return GRX_OK;
}
