// pocket_step.hip - the pocket-TTS flow-LM transformer (the "LM step") on
// one GPU.
//
// The graph is flowLM.text/run/step of pockettts/lm.go:164-195 over
// transformer.forward and attend (pockettts/nn.go:142-254) of
// github.com/xattribution/gorelaxor: float64 LayerNorm, q|k|v (Q8_0, int8
// route, as pockettts/model.go:331-366 packs and drops these weights),
// rotary q and k, causal attention over the cache, out projection, GELU
// feed-forward; no context limit, no layer scales.  Every float step keeps
// the reference's order (the float route of MatMulF32 for the scores and
// values, expSub for the softmax, AddScaled for T < 4), so the frame outputs
// and end-of-speech logits are bit-identical to the CPU oracle's.
//
// A frame is 32 launches: the input projection of the latent, per layer
// [LN -> q|k|v + RoPE + cache] [attention, one workgroup per head, output
// rounded to Q8_0] [out + residual] [LN -> ff1 -> GELU, rounded] [ff2 +
// residual], and [out_norm, end-of-speech logit, position and frame + 1].
// Position and frame index live in device memory: a run of teacher-forced
// frames is one captured graph replayed per frame.  The text prefix (T rows
// at once) goes through the same products in launches of up to 8 rows and
// its own attention kernel, which follows MatMulF32's route for T rows.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "grx_float.h"
#include "grx_internal.h"
#include "grx_ln.h"
#include "pocket_internal.h"

namespace {

constexpr int kThreads = 256;

// x = input . latent (lm.go:188-190): an F32 [d][ldim] weight on the float
// route with one row, gemvRows (gemm.go:195-259): dotF32x4 for whole groups
// of four outputs, dotF32Go for the rest.
__global__ void input_kernel(const float *__restrict__ w, const float *__restrict__ lat_base,
                             const int *__restrict__ frame, int d, int ldim, float *__restrict__ x) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= d) return;
    const float *lat = lat_base + (frame != nullptr ? (size_t)(*frame) * ldim : 0);
    const float *wr = w + (size_t)j * ldim;
    x[j] = j < (d & ~3) ? dot_x4(lat, wr, ldim) : dot_go(lat, wr, ldim);
}

// Frame attention for heads of 64 over n <= kStepN keys, without divergent
// branches (the arithmetic of attn_step_kernel's general body below): thread
// j holds key row j (zeros past n, never used), its score (dotF32x4 below
// n &^ 3, dotF32Go past it, times the scale), the maximum by DPP and one
// barrier, EXP8 or expf, each wave's own 1 / sum (expSub's eight lane sums,
// HSUM, the tail), then w_j and value row j into LDS (w = 0 past n); wave
// 0's lane d runs AddScaled's chain o = fma(w_j, v_j[d], o) in key order,
// zero weights skipped.
constexpr int kStepHd = 64, kStepN = 512, kStepLd = kStepHd + 4, kStepThreads = kStepN;
// chain-major exps kStepCs floats apart: the eight chains' 16-byte reads
// fall in distinct banks
constexpr int kStepCs = kStepN / 8 + 4;
// LDS floats: value rows [kStepN][kStepLd], chain-major exps, exps by key,
// weights, reductions, dummy slots
constexpr size_t kStepLds = (size_t)kStepN * kStepLd + 8 * (size_t)kStepCs + 2 * (size_t)kStepN + 16 + 8;

template <bool QOUT>
__device__ __forceinline__ void attn_step_small(float *sm, const float *q, const float *kc, const float *vc, int n,
                                                int d, float scale, float *att, int8_t *att_q, float *att_s) {
    constexpr int HD = kStepHd, RC = kStepN, LD = kStepLd;
    float *vl = sm, *ch = vl + RC * LD, *pl = ch + 8 * kStepCs, *pw = pl + RC, *red = pw + RC, *dummy = red + 16;
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool live = tid < n;
    const int j = min(tid, n - 1);
    const float4 *kr = reinterpret_cast<const float4 *>(kc + (size_t)j * d + h * HD);
    const float4 *vr = reinterpret_cast<const float4 *>(vc + (size_t)j * d + h * HD);
    float4 kv[HD / 4], vv[HD / 4];
    if (live) {  // lanes past n load nothing (many lanes loading one repeated row measured far slower)
#pragma unroll
        for (int i = 0; i < HD / 4; ++i) kv[i] = kr[i];
#pragma unroll
        for (int i = 0; i < HD / 4; ++i) vv[i] = vr[i];
    } else {
#pragma unroll
        for (int i = 0; i < HD / 4; ++i) kv[i] = vv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float4 *qh = reinterpret_cast<const float4 *>(q + h * HD);
    // dot4f32avx's row (eight-lane accumulators A, B over steps of 16) and
    // dotF32Go's four running sums, both from the same products' operands
    float A[8], B[8], s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
    for (int l = 0; l < 8; ++l) A[l] = B[l] = 0.f;
#pragma unroll
    for (int i = 0; i < HD / 4; ++i) {
        const float4 a = qh[i], b = kv[i];
        const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = 4 * i + e, l = c & 15;
            if (l < 8)
                A[l] = __fmaf_rn(av[e], bv[e], A[l]);
            else
                B[l - 8] = __fmaf_rn(av[e], bv[e], B[l - 8]);
        }
        s0 = __fadd_rn(s0, __fmul_rn(a.x, b.x));
        s1 = __fadd_rn(s1, __fmul_rn(a.y, b.y));
        s2 = __fadd_rn(s2, __fmul_rn(a.z, b.z));
        s3 = __fadd_rn(s3, __fmul_rn(a.w, b.w));
    }
    float S[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) S[l] = __fadd_rn(A[l], B[l]);
    const float x4 = hsum8(S);
    const float go = __fadd_rn(__fadd_rn(__fadd_rn(s0, s1), s2), s3);
    const float score = __fmul_rn(tid < (n & ~3) ? x4 : go, scale);
    float mx = wave_max(live ? score : -__builtin_inff());
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < kStepThreads / 64; ++w) mx = red[w] > mx ? red[w] : mx;
    const int n8 = n & ~7;
    const float dd = __fsub_rn(score, mx);
    const float e8 = grx_exp8(dd), eg = grx_expf_go(dd);
    const float e = tid < n8 ? e8 : eg;
    *(tid < n8 ? ch + (tid & 7) * kStepCs + (tid >> 3) : dummy) = e;
    *(live ? pl + tid : dummy + 1) = e;
    __syncthreads();
    const float inv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(softmax_inv(ch, kStepCs, pl + n8, n)), 0));
    const float wj = live ? __fmul_rn(e, inv) : 0.f;
    pw[tid] = wj;
    // a key of weight zero is skipped: its value row goes in as zeros, so
    // the chain's fma(0, 0, o) leaves o as it is (o starts at +0 and exact
    // cancellation rounds to +0, so o is never -0) whatever the row held
    float4 *vw = reinterpret_cast<float4 *>(vl + tid * LD);
    const bool zr = wj == 0.f;
#pragma unroll
    for (int i = 0; i < HD / 4; ++i) {  // (per component: the row stays in registers)
        const float a = vv[i].x, b = vv[i].y, c = vv[i].z, e4 = vv[i].w;
        vw[i] = make_float4(zr ? 0.f : a, zr ? 0.f : b, zr ? 0.f : c, zr ? 0.f : e4);
    }
    __syncthreads();
    if (wave == 0) {
        float o = 0.f;
        const int n32 = (n + 31) & ~31;
        for (int j0 = 0; j0 < n32; j0 += 32) {
            float w[32], v[32];
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                const float4 t = *reinterpret_cast<const float4 *>(pw + j0 + i);
                w[i] = t.x;
                w[i + 1] = t.y;
                w[i + 2] = t.z;
                w[i + 3] = t.w;
            }
#pragma unroll
            for (int i = 0; i < 32; ++i) v[i] = vl[(j0 + i) * LD + lane];
#pragma unroll
            for (int i = 0; i < 32; ++i) o = __fmaf_rn(w[i], v[i], o);
        }
        att[h * HD + lane] = o;
        if constexpr (QOUT) quant32_store(o, att_q + h * HD + lane, att_s + (h * HD + lane) / 32, lane & 31);
    }
}

// attend for one query row (T = 1, nn.go:200-244), one workgroup per head:
// scores of the pos+1 keys by MatMulF32's one-row route (dotF32x4 per group
// of four keys, dotF32Go for the rest), times 1/sqrt(hd), softmax by expSub,
// then out += w_j * v_j with AddScaled in key order, zero weights skipped
// (axpyAVX's fma below hd &^ 7, axpyGo past it).  With QOUT the head's
// outputs are also rounded to Q8_0.
template <bool QOUT>
__global__ __launch_bounds__(kStepThreads) void attn_step_kernel(const float *__restrict__ q, const float *__restrict__ kc,
                                                            const float *__restrict__ vc, const int *__restrict__ pos,
                                                            int d, int hd, float scale, int rc, float *__restrict__ att,
                                                            int8_t *__restrict__ att_q, float *__restrict__ att_s) {
    extern __shared__ __align__(16) float sm[];
    const int h = blockIdx.x, n = *pos + 1, tid = threadIdx.x;
    if (hd == kStepHd && n <= kStepN) {
        attn_step_small<QOUT>(sm, q, kc, vc, n, d, scale, att, att_q, att_s);
        return;
    }
    float *part = sm, *s = sm + 32, *vl = sm + 32 + ((n + 3) & ~3);
    const float *qh = q + h * hd;
    const int n4 = n & ~3;
    for (int j = tid; j < n; j += blockDim.x) {
        const float *kj = kc + (size_t)j * d + h * hd;
        s[j] = __fmul_rn(j < n4 ? dot_x4(qh, kj, hd) : dot_go(qh, kj, hd), scale);
    }
    __syncthreads();
    block_softmax(s, n, part);
    // the values, rc rows at a time through LDS, summed in key order
    const int h8 = hd & ~7;
    float o = 0.f;
    for (int r0 = 0; r0 < n; r0 += rc) {
        const int rows = min(rc, n - r0);
        stage_rows(vl, vc + h * hd, d, r0, rows, hd);
        __syncthreads();
        // keys of weight 0 are skipped (a select, so the loads of the
        // unrolled loop issue together ahead of the dependent chain)
        if (tid < h8) {
#pragma unroll 16
            for (int j = 0; j < rows; ++j) {
                const float w = s[r0 + j], t = __fmaf_rn(w, vl[j * hd + tid], o);
                o = w == 0.f ? o : t;
            }
        } else if (tid < hd) {
#pragma unroll 16
            for (int j = 0; j < rows; ++j) {
                const float w = s[r0 + j], t = __fadd_rn(o, __fmul_rn(w, vl[j * hd + tid]));
                o = w == 0.f ? o : t;
            }
        }
        __syncthreads();
    }
    if (tid < hd) {
        att[h * hd + tid] = o;
        if constexpr (QOUT) quant32_store(o, att_q + h * hd + tid, att_s + (h * hd + tid) / 32, tid & 31);
    }
}

// One output of ws.matmul's float route for row r of m rows (gemm.go:116-
// 184): rows in whole groups of six (m > 16) take k6x16avx's chain, fma over
// k in chunks of 256 added to C from 0; other rows take gemvRows (dotF32x4
// for whole groups of four columns, dotF32Go for the rest).  a_r and b_j are
// k long with element strides sa and sb.
__device__ float route_dot(const float *a, int sa, const float *b, int sb, int k, int r, int m, int j, int n) {
    const bool packed = m > 16 && r < m / 6 * 6;
    if (packed) {
        float c = 0.f;
        for (int k0 = 0; k0 < k; k0 += 256) {
            const int kn = min(256, k - k0);
            float acc = 0.f;
            for (int kk = 0; kk < kn; ++kk) acc = __fmaf_rn(a[(size_t)(k0 + kk) * sa], b[(size_t)(k0 + kk) * sb], acc);
            c = __fadd_rn(acc, c);
        }
        return c;
    }
    // gemvRows: the element strides are 1 on this route's operands
    return j < (n & ~3) ? dot_x4(a, b, k) : dot_go(a, b, k);
}

// route_dot with the second operand's elements sb apart on both routes.
__device__ float route_dot_s(const float *a, const float *b, size_t sb, int k, int r, int m, int j, int n) {
    if (m > 16 && r < m / 6 * 6) return route_dot(a, 1, b, (int)sb, k, r, m, j, n);
    return j < (n & ~3) ? dot_x4_s(a, b, sb, k) : dot_go_s(a, b, sb, k);
}

// seq_softmax(s, n) with the 64 lanes of one wave (every lane calls it):
// the maximum as its loop finds it (the first s[j] greater than the running
// maximum from -inf: among equal values, +0 and -0 included, the lowest
// index) by a reduction over (value, index), the exps in parallel, the
// eight chains below n & ~7 summed in order by lanes 0-7 and the tail by
// lane 8, then 1 / (HSUM + tail) and the scaled values in parallel.
__device__ void wave_seq_softmax(float *s, int n) {
    const int lane = threadIdx.x & 63;
    float mx = -__builtin_inff();
    int mi = 0x7fffffff;
    for (int j = lane; j < n; j += 64)
        if (s[j] > mx) {
            mx = s[j];
            mi = j;
        }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(mx, o);
        const int oi = __shfl_xor(mi, o);
        const bool take = ov > mx || (ov == mx && oi < mi);
        mx = take ? ov : mx;
        mi = take ? oi : mi;
    }
    const int n8 = n & ~7;
    for (int j = lane; j < n; j += 64) {
        const float dd = __fsub_rn(s[j], mx);
        s[j] = j < n8 ? grx_exp8(dd) : grx_expf_go(dd);
    }
    __syncthreads();
    float acc = 0.f;
    if (lane < 8) {
        for (int j = lane; j < n8; j += 8) acc = __fadd_rn(acc, s[j]);
    } else if (lane == 8) {
        for (int j = n8; j < n; ++j) acc = __fadd_rn(acc, s[j]);
    }
    float a8[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) a8[l] = __shfl(acc, l);
    const float t = __shfl(acc, 8);
    const float sa = n8 > 0 ? hsum8(a8) : 0.f;
    const float inv = __fdiv_rn(1.0f, __fadd_rn(sa, t));
    for (int j = lane; j < n; j += 64) s[j] = __fmul_rn(s[j], inv);
}

// attend for T rows after pos0 cached positions (nn.go:200-254), one
// workgroup (a wave) per (row r = blockIdx.x, head h = blockIdx.y): thread
// j takes the scores of keys j, j + 64, ... by MatMulF32's route for T
// rows into LDS, the wave the row's scale and causal softmax
// (wave_seq_softmax; zeros past the row's position), then thread e output
// e: T < 4 AddScaled in key order, else the product with value column e by
// the same route.  With `staged` (heads of 64) the head's key rows (65
// floats apart) and value rows are first copied to LDS, 64 rows at a time
// with every lane's 16-byte loads in flight at once, and read from there;
// else they are read in place (value column e's elements d apart).  LDS:
// the row's pos0 + T scores (rounded up to 4 floats), then if staged the
// keys and the values.
__global__ __launch_bounds__(64) void attn_prefix_kernel(const float *__restrict__ q, const float *__restrict__ kc,
                                                         const float *__restrict__ vc, int pos0, int T, int d, int hd,
                                                         float scale, float *__restrict__ att, int staged) {
    extern __shared__ float row[];
    const int r = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, nk = pos0 + T, p = pos0 + r;
    const float *qr = q + (size_t)r * 3 * d + h * hd;
    float *kl = row + ((nk + 3) & ~3), *vl = kl + (size_t)nk * 65;
    if (staged) {
        // rows c0 + 4u + tid / 16 of each run of 64, float4 tid % 16
        for (int c0 = 0; c0 < nk; c0 += 64) {
            float4 kr[16], vr[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const size_t j = (size_t)min(c0 + 4 * u + (tid >> 4), nk - 1);
                kr[u] = reinterpret_cast<const float4 *>(kc + j * d + h * 64)[tid & 15];
                vr[u] = reinterpret_cast<const float4 *>(vc + j * d + h * 64)[tid & 15];
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int j = c0 + 4 * u + (tid >> 4), e = 4 * (tid & 15);
                if (j < nk) {
                    float *kd = kl + j * 65 + e;
                    kd[0] = kr[u].x;
                    kd[1] = kr[u].y;
                    kd[2] = kr[u].z;
                    kd[3] = kr[u].w;
                    reinterpret_cast<float4 *>(vl + j * 64)[tid & 15] = vr[u];
                }
            }
        }
        __syncthreads();
    }
    for (int j = tid; j < nk; j += 64) {
        const float v = staged ? route_dot(qr, 1, kl + j * 65, 1, hd, r, T, j, nk)
                               : route_dot(qr, 1, kc + (size_t)j * d + h * hd, 1, hd, r, T, j, nk);
        row[j] = j <= p ? __fmul_rn(v, scale) : 0.f;
    }
    __syncthreads();
    wave_seq_softmax(row, p + 1);
    __syncthreads();
    const int h8 = hd & ~7;
    for (int e = tid; e < hd; e += 64) {
        // value j of column e at vcol[j * vs]
        const float *vcol = staged ? vl + e : vc + h * hd + e;
        const size_t vs = staged ? (size_t)64 : (size_t)d;
        float o;
        if (T < 4) {
            o = 0.f;
            for (int j = 0; j < nk; ++j) {
                const float w = row[j];
                if (w == 0.f) continue;
                const float v = vcol[j * vs];
                o = e < h8 ? __fmaf_rn(w, v, o) : __fadd_rn(o, __fmul_rn(w, v));
            }
        } else {
            o = route_dot_s(row, vcol, vs, nk, r, T, e, hd);
        }
        att[(size_t)r * d + h * hd + e] = o;
    }
}

// End of a frame (lm.go:168-169, 191-194): out_norm (float64 LayerNorm of
// the last row), eos = dotF32Go(out, w) + b, recorded at the frame index;
// then position and frame move on (advance 0: neither moves).
__global__ __launch_bounds__(kThreads) void finish_kernel(const float *__restrict__ x, int d, const float *__restrict__ nw,
                                                          const float *__restrict__ nb, const float *__restrict__ ew,
                                                          float eb, int *__restrict__ pos, int *__restrict__ frame,
                                                          int advance, float *__restrict__ out_hist,
                                                          float *__restrict__ eos_hist) {
    __shared__ double red[48];  // ln_block_reduce
    __shared__ float ov[8192], ewl[8192], part4[4];
    const int tid = threadIdx.x;
    // the row in LDS (ewl, until the eos weights replace it below)
    for (int i = tid; i < d; i += blockDim.x) ewl[i] = x[i];
    __syncthreads();
    double mean, inv;
    ln64_stats(ewl, d, 1e-5, red, mean, inv);
    const int f = frame != nullptr ? *frame : 0;
    float *out = out_hist + (size_t)f * d;
    for (int i = tid; i < d; i += blockDim.x) {
        float o = (float)(((double)ewl[i] - mean) * inv);
        o = __fadd_rn(__fmul_rn(o, nw[i]), nb[i]);
        out[i] = o;
        ov[i] = o;
        ewl[i] = ew[i];
    }
    __syncthreads();
    // dotF32Go (gemm.go:294-308): running sum t over elements t, t+4, ...
    // below d &^ 3 (the tail into sum 0), each on its own thread
    if (tid < 4) {
        const int d4 = d & ~3;
        float acc = 0.f;
#pragma unroll 16
        for (int i = tid; i < d4; i += 4) acc = __fadd_rn(acc, __fmul_rn(ov[i], ewl[i]));
        if (tid == 0)
            for (int i = d4; i < d; ++i) acc = __fadd_rn(acc, __fmul_rn(ov[i], ewl[i]));
        part4[tid] = acc;
    }
    __syncthreads();
    if (tid == 0) {
        const float dg = __fadd_rn(__fadd_rn(__fadd_rn(part4[0], part4[1]), part4[2]), part4[3]);
        eos_hist[f] = __fadd_rn(dg, eb);
        if (advance) {
            *pos = *pos + 1;
            if (frame != nullptr) *frame = f + 1;
        }
    }
}

}  // namespace

// ---------------------------------------------------------------- host side

namespace {

struct PExpect {
    std::string name;
    size_t bytes;
};

std::vector<PExpect> pexpected(const grx_pocket_hparams &hp) {
    const size_t d = hp.d, ff = hp.ff;
    auto q8 = [](size_t rows, size_t cols) { return rows * (cols / 32) * 34; };
    std::vector<PExpect> e;
    for (int i = 0; i < hp.n_layer; ++i) {
        const std::string p = "lm.blk." + std::to_string(i) + ".";
        for (const char *n : {"norm1.weight", "norm1.bias", "norm2.weight", "norm2.bias"}) e.push_back({p + n, d * 4});
        e.push_back({p + "attn_qkv.weight", q8(3 * d, d)});
        e.push_back({p + "attn_out.weight", q8(d, d)});
        e.push_back({p + "ff1.weight", q8(ff, d)});
        e.push_back({p + "ff2.weight", q8(d, ff)});
    }
    e.push_back({"lm.input.weight", d * hp.ldim * 4});
    e.push_back({"lm.bos", (size_t)hp.ldim * 4});
    e.push_back({"lm.out_norm.weight", d * 4});
    e.push_back({"lm.out_norm.bias", d * 4});
    e.push_back({"lm.eos.weight", d * 4});
    e.push_back({"lm.eos.bias", 4});
    return e;
}

grx_status palloc(grx_pocket *m, size_t bytes, void **out) {
    void *p = nullptr;
    GRX_HIP(grx_dev_malloc(&p, bytes > 0 ? bytes : 16));
    m->allocs.push_back(p);
    *out = p;
    return GRX_OK;
}

template <typename T>
grx_status palloc_t(grx_pocket *m, size_t count, T **out) {
    return palloc(m, count * sizeof(T), reinterpret_cast<void **>(out));
}

grx_status pupload(grx_pocket *m, const std::string &name, float **out) {
    const auto &h = m->host.at(name);
    grx_status s = palloc(m, h.size(), reinterpret_cast<void **>(out));
    if (s != GRX_OK) return s;
    GRX_HIP(hipMemcpy(*out, h.data(), h.size(), hipMemcpyHostToDevice));
    return GRX_OK;
}

// cos/sin of every position's pair angles (nn.go:69-93): f_i =
// f32(exp(f64(f32(i) * f32(-ln(period)*2/hd)))), angle f64(f_i * f32(pos)),
// kept as f32.  Computed once on the host.
void rope_table(const grx_pocket_hparams &hp, std::vector<float> &cs, std::vector<float> &sn) {
    const int hd = hp.d / hp.heads, half = hd / 2;
    const float c = (float)(-log(hp.period) * 2.0 / (double)hd);
    std::vector<float> f(half);
    for (int i = 0; i < half; ++i) {
        const float t = (float)i * c;
        f[i] = (float)exp((double)t);
    }
    cs.resize((size_t)hp.max_pos * half);
    sn.resize((size_t)hp.max_pos * half);
    for (int p = 0; p < hp.max_pos; ++p)
        for (int i = 0; i < half; ++i) {
            const float fp = f[i] * (float)p;
            const double a = (double)fp;
            cs[(size_t)p * half + i] = (float)cos(a);
            sn[(size_t)p * half + i] = (float)sin(a);
        }
}

// What pfinalize made (and, with it, anything allocated later: the flow
// head's buffers, the latents), released; the flow head's weights are
// released by pocket_flow_release.  After a failed finalize the model is
// as before it (its host tensors kept).
void prelease(grx_pocket *m) {
    for (PLayer &L : m->L)
        for (grx_weight *w : {L.qkv, L.out, L.ff1, L.ff2}) grx_weight_destroy(w);
    m->L.clear();
    for (void *p : m->allocs) (void)hipFree(p);
    m->allocs.clear();
    m->lat = nullptr;
}

grx_status pfinalize_tensors(grx_pocket *m);

grx_status pfinalize(grx_pocket *m) {
    if (m->ready) return GRX_OK;
    const grx_status s = pfinalize_tensors(m);
    if (s != GRX_OK) prelease(m);
    return s;
}

grx_status pfinalize_tensors(grx_pocket *m) {
    const grx_pocket_hparams &hp = m->hp;
    for (const PExpect &e : pexpected(hp))
        if (!m->host.count(e.name)) return grx_fail(GRX_ESTATE, "the model file has no tensor %s", e.name.c_str());
    GRX_HIP(hipSetDevice(m->ctx->device));
    grx_status s;
    const size_t d = hp.d, ff = hp.ff, mp = hp.max_pos;
    m->L.assign(hp.n_layer, PLayer());
    for (int i = 0; i < hp.n_layer; ++i) {
        PLayer &L = m->L[i];
        const std::string p = "lm.blk." + std::to_string(i) + ".";
        auto mat = [&](const char *n, int rows, int cols, grx_weight **w) {
            const auto &t = m->host.at(p + n);
            return grx_weight_q8_create(m->ctx, rows, cols, t.data(), t.size(), w);
        };
        if ((s = mat("attn_qkv.weight", 3 * hp.d, hp.d, &L.qkv)) != GRX_OK) return s;
        if ((s = mat("attn_out.weight", hp.d, hp.d, &L.out)) != GRX_OK) return s;
        if ((s = mat("ff1.weight", hp.ff, hp.d, &L.ff1)) != GRX_OK) return s;
        if ((s = mat("ff2.weight", hp.d, hp.ff, &L.ff2)) != GRX_OK) return s;
        if ((s = pupload(m, p + "norm1.weight", &L.n1w)) != GRX_OK) return s;
        if ((s = pupload(m, p + "norm1.bias", &L.n1b)) != GRX_OK) return s;
        if ((s = pupload(m, p + "norm2.weight", &L.n2w)) != GRX_OK) return s;
        if ((s = pupload(m, p + "norm2.bias", &L.n2b)) != GRX_OK) return s;
        if ((s = palloc_t(m, mp * d, &L.k)) != GRX_OK) return s;
        if ((s = palloc_t(m, mp * d, &L.v)) != GRX_OK) return s;
        GRX_HIP(hipMemset(L.k, 0, mp * d * 4));
        GRX_HIP(hipMemset(L.v, 0, mp * d * 4));
    }
    if ((s = pupload(m, "lm.input.weight", &m->input)) != GRX_OK) return s;
    if ((s = pupload(m, "lm.bos", &m->bos)) != GRX_OK) return s;
    if ((s = pupload(m, "lm.out_norm.weight", &m->onw)) != GRX_OK) return s;
    if ((s = pupload(m, "lm.out_norm.bias", &m->onb)) != GRX_OK) return s;
    if ((s = pupload(m, "lm.eos.weight", &m->eosw)) != GRX_OK) return s;
    memcpy(&m->eosb, m->host.at("lm.eos.bias").data(), 4);
    std::vector<float> cs, sn;
    rope_table(hp, cs, sn);
    if ((s = palloc_t(m, cs.size(), &m->rope_cos)) != GRX_OK) return s;
    if ((s = palloc_t(m, sn.size(), &m->rope_sin)) != GRX_OK) return s;
    GRX_HIP(hipMemcpy(m->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    GRX_HIP(hipMemcpy(m->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    if ((s = palloc_t(m, mp * d, &m->x)) != GRX_OK) return s;
    if ((s = palloc_t(m, mp * 3 * d, &m->q)) != GRX_OK) return s;  // q rows 3d apart
    if ((s = palloc_t(m, mp * d, &m->att)) != GRX_OK) return s;
    if ((s = palloc_t(m, mp * ff, &m->ff)) != GRX_OK) return s;
    if ((s = palloc_t(m, mp * d, &m->att_q)) != GRX_OK) return s;
    if ((s = palloc_t(m, mp * d / 32, &m->att_s)) != GRX_OK) return s;
    if ((s = palloc_t(m, mp * ff, &m->ff_q)) != GRX_OK) return s;
    if ((s = palloc_t(m, mp * ff / 32, &m->ff_s)) != GRX_OK) return s;
    if ((s = palloc_t(m, mp * d, &m->out_hist)) != GRX_OK) return s;
    if ((s = palloc_t(m, mp, &m->eos_hist)) != GRX_OK) return s;
    if ((s = palloc_t(m, 1, &m->pos)) != GRX_OK) return s;
    if ((s = palloc_t(m, 1, &m->frame)) != GRX_OK) return s;
    GRX_HIP(hipMemset(m->pos, 0, 4));
    GRX_HIP(hipMemset(m->frame, 0, 4));
    // the transformer's host copies go; the flow head's stay until its own set-up
    for (const PExpect &e : pexpected(hp)) m->host.erase(e.name);
    m->ready = true;
    return GRX_OK;
}

GemvArgs pargs(const grx_weight *w) {
    GemvArgs a = {};
    a.qs = w->qs;
    a.ds = w->ds;
    a.rows = w->rows;
    a.nb = w->nb;
    a.cacheable = 1;
    a.ln_eps = 1e-5;
    return a;
}

// transformer.forward of rows r0..r0+mm-1 of x (nn.go:151-179) for one
// layer's products; attention is separate.  ph: 0 = LN -> q|k|v, 1 = out +
// residual, 2 = LN -> ff1 -> GELU, 3 = ff2 + residual.
grx_status layer_product(grx_pocket *m, hipStream_t st, PLayer &L, int ph, int r0, int mm, bool qatt,
                         int chunks = 1) {
    const int d = m->hp.d, ff = m->hp.ff;
    GemvArgs a;
    auto launch = [&](int pro, int epi) {
        a.chunks = chunks;
        return grx_gemv_launch(st, mm, pro, epi, a, 0);
    };
    switch (ph) {
        case 0:
            a = pargs(L.qkv);
            a.x = m->x + (size_t)r0 * d;
            a.lda = d;
            a.ln_w = L.n1w;
            a.ln_b = L.n1b;
            a.y = m->q + (size_t)r0 * 3 * d;  // q rows 3d apart, as the reference's qkv rows
            a.ldc = 3 * d;
            a.seg = d;
            a.kc = L.k;
            a.vc = L.v;
            a.pos = m->pos;
            a.pos_add = r0;
            a.rope_cos = m->rope_cos;
            a.rope_sin = m->rope_sin;
            a.rope_half = d / m->hp.heads / 2;
            return launch(GRX_PRO_LN64, GRX_EPI_QKV_ROPE);
        case 1:
            a = pargs(L.out);
            a.x = m->att + (size_t)r0 * d;
            a.lda = d;
            a.xq = m->att_q + (size_t)r0 * d;
            a.xs = m->att_s + (size_t)r0 * d / 32;
            a.y = m->x + (size_t)r0 * d;
            a.ldc = d;
            a.resid = m->x + (size_t)r0 * d;
            a.ldr = d;
            return launch(qatt ? GRX_PRO_PREQ : GRX_PRO_QUANT, GRX_EPI_RESID);
        case 2:
            a = pargs(L.ff1);
            a.x = m->x + (size_t)r0 * d;
            a.lda = d;
            a.ln_w = L.n2w;
            a.ln_b = L.n2b;
            a.y = m->ff + (size_t)r0 * ff;
            a.ldc = ff;
            a.yq = m->ff_q + (size_t)r0 * ff;
            a.ys = m->ff_s + (size_t)r0 * ff / 32;
            return launch(GRX_PRO_LN64, GRX_EPI_GELU_Q);
        default:
            a = pargs(L.ff2);
            a.xq = m->ff_q + (size_t)r0 * ff;
            a.xs = m->ff_s + (size_t)r0 * ff / 32;
            a.y = m->x + (size_t)r0 * d;
            a.ldc = d;
            a.resid = m->x + (size_t)r0 * d;
            a.ldr = d;
            return launch(GRX_PRO_PREQ, GRX_EPI_RESID);
    }
}

// One frame (T = 1) from the latent at lat_base[*frame] (frame may be null:
// lat_base itself), on stream st.
grx_status enqueue_frame(grx_pocket *m, hipStream_t st, const float *lat_base, const int *frame) {
    const grx_pocket_hparams &hp = m->hp;
    const int d = hp.d, hd = d / hp.heads;
    const bool qatt = hd % 32 == 0;
    const float scale = (float)(1.0 / sqrt((double)hd));
    grx_status s;
    input_kernel<<<grx_ceil_div(d, kThreads), kThreads, 0, st>>>(m->input, lat_base, frame, d, hp.ldim, m->x);
    GRX_LAUNCHED("input_kernel");
    // LDS: 32 + max_pos scores, then value rows in chunks within 48 KiB; or
    // the branch-free body's (heads of 64, up to kStepN keys), 512 threads
    const int rc = max(1, min(hp.max_pos, (48 * 1024) / (hd * 4)));
    size_t smem = (32 + (((size_t)hp.max_pos + 3) & ~(size_t)3) + (size_t)rc * hd) * 4;
    if (hd == kStepHd) {
        smem = std::max(smem, kStepLds * 4);
        static bool raised = false;  // set by the eager frame that precedes any capture
        if (!raised) {
            raised = true;
            GRX_HIP(hipFuncSetAttribute((const void *)attn_step_kernel<true>,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)(kStepLds * 4)));
            GRX_HIP(hipFuncSetAttribute((const void *)attn_step_kernel<false>,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)(kStepLds * 4)));
        }
    }
    for (int li = 0; li < hp.n_layer; ++li) {
        PLayer &L = m->L[li];
        if ((s = layer_product(m, st, L, 0, 0, 1, qatt)) != GRX_OK) return s;
        if (qatt)
            attn_step_kernel<true><<<hp.heads, kStepThreads, smem, st>>>(m->q, L.k, L.v, m->pos, d, hd, scale, rc,
                                                                         m->att, m->att_q, m->att_s);
        else
            attn_step_kernel<false><<<hp.heads, kStepThreads, smem, st>>>(m->q, L.k, L.v, m->pos, d, hd, scale, rc,
                                                                          m->att, nullptr, nullptr);
        GRX_LAUNCHED("attn_step_kernel");
        for (int ph = 1; ph < 4; ++ph)
            if ((s = layer_product(m, st, L, ph, 0, 1, qatt)) != GRX_OK) return s;
    }
    finish_kernel<<<1, kThreads, 0, st>>>(m->x, d, m->onw, m->onb, m->eosw, m->eosb, m->pos, m->frame, 1,
                                          m->out_hist, m->eos_hist);
    GRX_LAUNCHED("finish_kernel");
    return GRX_OK;
}

}  // namespace

grx_status pocket_finalize(grx_pocket *m) { return pfinalize(m); }
grx_status pocket_enqueue_frame(grx_pocket *m, hipStream_t st, const float *lat_base, const int *frame) {
    return enqueue_frame(m, st, lat_base, frame);
}
grx_status pocket_alloc(grx_pocket *m, size_t bytes, void **out) { return palloc(m, bytes, out); }

extern "C" grx_status grx_pocket_create(grx_ctx *ctx, const grx_pocket_hparams *hp, grx_pocket **out) {
    if (!ctx || !hp || !out) return grx_fail(GRX_EINVAL, "grx_pocket_create: NULL argument");
    *out = nullptr;
    if (hp->d <= 0 || hp->heads <= 0 || hp->ff <= 0 || hp->n_layer <= 0 || hp->max_pos <= 0 || hp->ldim <= 0 ||
        !(hp->period > 0))
        return grx_fail(GRX_EINVAL, "grx_pocket_create: every size must be positive");
    if (hp->d % 32 != 0 || hp->ff % 32 != 0 || hp->d % hp->heads != 0 || (hp->d / hp->heads) % 2 != 0)
        return grx_fail(GRX_ESIZE, "%d values don't split into %d heads", hp->d, hp->heads);
    if (hp->d > 8192 || (size_t)hp->max_pos * hp->max_pos * 4 > 64 * 1024 * 1024)
        return grx_fail(GRX_ESIZE, "grx_pocket_create: d %d or max_pos %d too large", hp->d, hp->max_pos);
    grx_pocket *m = new grx_pocket();
    m->ctx = ctx;
    m->hp = *hp;
    *out = m;
    return GRX_OK;
}

extern "C" grx_status grx_pocket_destroy(grx_pocket *m) {
    if (!m) return GRX_OK;
    GRX_HIP(hipSetDevice(m->ctx->device));
    GRX_HIP(hipStreamSynchronize(m->ctx->stream));
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    if (m->speak_exec) (void)hipGraphExecDestroy(m->speak_exec);
    if (m->speak_graph) (void)hipGraphDestroy(m->speak_graph);
    pocket_flow_release(m, m->allocs.size());
    prelease(m);
    delete m;
    return GRX_OK;
}

extern "C" grx_status grx_pocket_set_tensor(grx_pocket *m, const char *name, const void *data, size_t nbytes) {
    if (!m || !name || (!data && nbytes)) return grx_fail(GRX_EINVAL, "grx_pocket_set_tensor: NULL argument");
    const uint8_t *p = static_cast<const uint8_t *>(data);
    size_t qa = 0, fb = 0;  // the flow head's tensors, once declared
    if (pocket_flow_tensor(m, name, &qa, &fb)) {
        if (nbytes != qa && nbytes != fb)
            return grx_fail(GRX_ESIZE, "tensor %s has the wrong shape (%zu bytes, want %zu or %zu)", name, nbytes, qa,
                            fb);
        if (m->flow.ready) return grx_fail(GRX_ESTATE, "grx_pocket_set_tensor: the flow head is in use already");
        m->host[name].assign(p, p + nbytes);
        return GRX_OK;
    }
    for (const PExpect &e : pexpected(m->hp)) {
        if (e.name != name) continue;
        if (m->ready) return grx_fail(GRX_ESTATE, "grx_pocket_set_tensor: the model is in use already");
        if (nbytes != e.bytes)
            return grx_fail(GRX_ESIZE, "tensor %s has the wrong shape (%zu bytes, want %zu)", name, nbytes, e.bytes);
        m->host[name].assign(p, p + nbytes);
        return GRX_OK;
    }
    return grx_fail(GRX_EINVAL, "the model file has a tensor this program doesn't know: %s", name);
}

extern "C" grx_status grx_pocket_reset(grx_pocket *m) {
    if (!m) return grx_fail(GRX_EINVAL, "grx_pocket_reset: NULL model");
    if (m->ready) GRX_HIP(hipMemsetAsync(m->pos, 0, 4, m->ctx->stream));
    m->pos_host = 0;
    return GRX_OK;
}

extern "C" int grx_pocket_pos(const grx_pocket *m) { return m ? m->pos_host : 0; }

extern "C" grx_status grx_pocket_run(grx_pocket *m, const float *x, int T, float *out) {
    if (!m || (!x && T > 0)) return grx_fail(GRX_EINVAL, "grx_pocket_run: NULL argument");
    grx_status s = pfinalize(m);
    if (s != GRX_OK) return s;
    if (T <= 0) return grx_fail(GRX_EINVAL, "grx_pocket_run: T = %d", T);
    if (m->pos_host + T > m->hp.max_pos)
        return grx_fail(GRX_ESTATE, "grx_pocket_run: %d rows after %d positions exceed %d", T, m->pos_host,
                        m->hp.max_pos);
    const grx_pocket_hparams &hp = m->hp;
    const int d = hp.d, hd = d / hp.heads, pos0 = m->pos_host;
    const bool qatt = hd % 32 == 0;
    hipStream_t st = m->ctx->stream;
    GRX_HIP(hipMemcpyAsync(m->x, x, (size_t)T * d * 4, hipMemcpyHostToDevice, st));
    const float scale = (float)(1.0 / sqrt((double)hd));
    // rows in groups of 8 (every whole group in one launch), then 4, 2 and 1
    auto rows_of = [&](int left) { return left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1; };
    for (int li = 0; li < hp.n_layer; ++li) {
        PLayer &L = m->L[li];
        for (int r0 = 0; r0 < T;) {
            const int mm = rows_of(T - r0), nc = mm == 8 ? (T - r0) / 8 : 1;
            if ((s = layer_product(m, st, L, 0, r0, mm, qatt, nc)) != GRX_OK) return s;
            r0 += mm * nc;
        }
        {
            // heads of 64: keys and values through LDS while they fit in 64 KiB
            const size_t nk = (size_t)pos0 + T, rowb = ((nk + 3) & ~(size_t)3) * 4, kvb = nk * 129 * 4;
            const int staged = hd == 64 && rowb + kvb <= 64 * 1024;
            attn_prefix_kernel<<<dim3(T, hp.heads), 64, rowb + (staged ? kvb : 0), st>>>(
                m->q, L.k, L.v, pos0, T, d, hd, scale, m->att, staged);
        }
        GRX_LAUNCHED("attn_prefix_kernel");
        // the prefix's attention rows are rounded in the out product's prologue
        for (int ph = 1; ph < 4; ++ph)
            for (int r0 = 0; r0 < T;) {
                const int mm = rows_of(T - r0), nc = mm == 8 ? (T - r0) / 8 : 1;
                if ((s = layer_product(m, st, L, ph, r0, mm, ph == 1 ? false : qatt, nc)) != GRX_OK) return s;
                r0 += mm * nc;
            }
    }
    // out_norm of the last row into the history slot of frame 0 (not kept)
    finish_kernel<<<1, kThreads, 0, st>>>(m->x + (size_t)(T - 1) * d, d, m->onw, m->onb, m->eosw, m->eosb, m->pos,
                                          nullptr, 0, m->out_hist, m->eos_hist);
    GRX_LAUNCHED("finish_kernel");
    m->pos_host += T;
    GRX_HIP(hipMemcpyAsync(m->pos, &m->pos_host, 4, hipMemcpyHostToDevice, st));
    if (out) GRX_HIP(hipMemcpyAsync(out, m->out_hist, (size_t)d * 4, hipMemcpyDeviceToHost, st));
    GRX_HIP(hipStreamSynchronize(st));
    return GRX_OK;
}

extern "C" grx_status grx_pocket_frames(grx_pocket *m, const float *latents, int n, float *outs, float *eos) {
    if (!m) return grx_fail(GRX_EINVAL, "grx_pocket_frames: NULL model");
    grx_status s = pfinalize(m);
    if (s != GRX_OK) return s;
    if (n < 0) return grx_fail(GRX_EINVAL, "grx_pocket_frames: n = %d", n);
    if (m->pos_host + n > m->hp.max_pos)
        return grx_fail(GRX_ESTATE, "grx_pocket_frames: %d frames after %d positions exceed %d", n, m->pos_host,
                        m->hp.max_pos);
    if (n == 0) return GRX_OK;
    const grx_pocket_hparams &hp = m->hp;
    hipStream_t st = m->ctx->stream;
    if (n > m->lat_cap) {
        if (m->lat) {
            GRX_HIP(hipStreamSynchronize(st));
            GRX_HIP(hipFree(m->lat));
            for (auto &p : m->allocs)
                if (p == m->lat) p = nullptr;
            if (m->exec) {
                (void)hipGraphExecDestroy(m->exec);
                (void)hipGraphDestroy(m->graph);
                m->exec = nullptr;
                m->graph = nullptr;
            }
        }
        GRX_HIP(grx_dev_malloc((void **)&m->lat, (size_t)(hp.max_pos + 1) * hp.ldim * 4));  // + the row a flow head writes last
        m->allocs.push_back(m->lat);
        m->lat_cap = hp.max_pos;
    }
    // frame k's latent at lat[k]; latents NULL: the bos input for every frame
    if (latents)
        GRX_HIP(hipMemcpyAsync(m->lat, latents, (size_t)n * hp.ldim * 4, hipMemcpyHostToDevice, st));
    else
        for (int k = 0; k < n; ++k)
            GRX_HIP(hipMemcpyAsync(m->lat + (size_t)k * hp.ldim, m->bos, (size_t)hp.ldim * 4, hipMemcpyDeviceToDevice,
                                   st));
    GRX_HIP(hipMemsetAsync(m->frame, 0, 4, st));
    const bool eager = grx_tune(GRX_TUNE_NO_GRAPH) == 1;
    for (int k = 0; k < n; ++k) {
        if (eager || (!m->exec && k == 0)) {
            if ((s = enqueue_frame(m, st, m->lat, m->frame)) != GRX_OK) return s;
            if (!eager && !m->exec) {
                // capture the frame once the eager one has set every attribute
                GRX_HIP(hipStreamSynchronize(st));
                hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
                if (e == hipSuccess) {
                    grx_status cs = enqueue_frame(m, st, m->lat, m->frame);
                    hipGraph_t g = nullptr;
                    e = hipStreamEndCapture(st, &g);
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
            continue;
        }
        if (m->exec)
            GRX_HIP(hipGraphLaunch(m->exec, st));
        else if ((s = enqueue_frame(m, st, m->lat, m->frame)) != GRX_OK)
            return s;
    }
    m->pos_host += n;
    if (outs) GRX_HIP(hipMemcpyAsync(outs, m->out_hist, (size_t)n * hp.d * 4, hipMemcpyDeviceToHost, st));
    if (eos) GRX_HIP(hipMemcpyAsync(eos, m->eos_hist, (size_t)n * 4, hipMemcpyDeviceToHost, st));
    GRX_HIP(hipStreamSynchronize(st));
    return GRX_OK;
}
