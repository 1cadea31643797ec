// whisper_step.hip - a whisper-shaped text decoder step on one GPU.
//
// The graph is Model.decode of whisper/decoder.go:33-140 (github.com/
// xattribution/gorelaxor) with every matrix a Q8_0 weight on the int8 route
// of q8_gemv.hip; the vector kernels below restate the reference's float
// arithmetic in its own order, so a step's logits are bit-identical to the
// CPU oracle's and the greedy tokens are the same.
//
// One step is, per layer:
//   [LN -> q|k|v GEMV, k and v written into the cache at pos]  (one launch;
//    layer 0 builds the embedding row in the same prologue)
//   [self-attention over pos+1 cached keys, one workgroup per head, output
//    rounded to Q8_0]  [out GEMV + residual]
//   [LN -> cross query GEMV] [cross scores] [softmax + weighted values,
//    rounded to Q8_0]  [cross out GEMV + residual]
//   [LN -> fc1 GEMV -> GELU, rounded to Q8_0] [fc2 GEMV + residual]
// then [LN -> logits GEMV -> argmax; the last workgroup writes the token and
// moves the position on].  Token and position live in device memory, so the
// step is captured once into a HIP graph and replayed; greedy decoding never
// returns to the host.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "grx_float.h"
#include "grx_internal.h"
#include "q8_gemv_impl.h"

namespace {

constexpr int kAttnThreads = 256;

// ---------------------------------------------------------------- kernels

constexpr int kBatchV = 96;  // the same for the cross values' longer chains (one batch at 1500 keys)

// Self-attention workgroups are 256 threads; heads of 64 over at most
// kSmallN positions take the branch-free body, others the general one.
constexpr int kSmallHd = 64, kSmallN = 256, kSmallPld = kSmallHd + 4;
// chain-major exps kSmallCs floats apart (distinct banks for the eight chains)
constexpr int kSmallCs = kSmallN / 8 + 4;
// LDS floats of the branch-free body: products [kSmallN][kSmallPld] (rows 68
// floats apart: 16-byte writes of 16 lanes fall in distinct banks), chain-
// major exps, exps by position, reductions, a dummy slot
constexpr size_t kSmallLds = (size_t)kSmallN * kSmallPld + 8 * kSmallCs + kSmallN + 16 + 4;

// Causal self-attention of one head over n <= kSmallN positions, head_dim
// 64, with no divergent branches: thread j holds K and V row j in registers
// (zeros past n, never used), its score (dotF32Go),
// the maximum by DPP and
// one barrier, its exp (chain-major and by position in LDS), every wave's own
// 1 / sum (softmax_inv), then its products p_j * v_j[d] into LDS (zeros past
// n); wave 0's lane d sums them in position order (whole groups of 32).
template <bool QOUT>
__device__ __forceinline__ void self_attn_small(float *sm, const float *q, const float4 (&kv)[kSmallHd / 4],
                                                const float4 (&vv)[kSmallHd / 4], int n, float sc, float *att,
                                                int8_t *att_q, float *att_s) {
    constexpr int HD = kSmallHd, RC = kSmallN, PLD = kSmallPld;
    float *prod = sm, *ch = prod + RC * PLD, *pl = ch + 8 * kSmallCs, *red = pl + RC, *dummy = red + 16;
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool live = tid < n;
    // dotF32Go (gemm.go:294-308): four running sums over the float4 pieces
    const float4 *qh = reinterpret_cast<const float4 *>(q + h * HD);
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
    for (int i = 0; i < HD / 4; ++i) {
        const float4 a = qh[i], b = kv[i];
        s0 = __fadd_rn(s0, __fmul_rn(a.x, b.x));
        s1 = __fadd_rn(s1, __fmul_rn(a.y, b.y));
        s2 = __fadd_rn(s2, __fmul_rn(a.z, b.z));
        s3 = __fadd_rn(s3, __fmul_rn(a.w, b.w));
    }
    const float score = __fmul_rn(__fadd_rn(__fadd_rn(__fadd_rn(s0, s1), s2), s3), sc);
    float mx = wave_max(live ? score : -__builtin_inff());
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const int n8 = n & ~7;
    const float d = __fsub_rn(score, mx);
    // both forms, then the reference's (EXP8 below n8, expf past it): no branch
    const float e8 = grx_exp8(d), eg = grx_expf_go(d);
    const float e = tid < n8 ? e8 : eg;
    *(tid < n8 ? ch + (tid & 7) * kSmallCs + (tid >> 3) : dummy) = e;
    *(live ? pl + tid : dummy + 1) = e;
    __syncthreads();
    const float inv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(softmax_inv(ch, kSmallCs, pl + n8, n)), 0));
    const float pj = __fmul_rn(e, inv);
    float4 *pr = reinterpret_cast<float4 *>(prod + tid * PLD);
#pragma unroll
    for (int i = 0; i < HD / 4; ++i) {
        const float4 v = vv[i];
        pr[i] = live ? make_float4(__fmul_rn(pj, v.x), __fmul_rn(pj, v.y), __fmul_rn(pj, v.z), __fmul_rn(pj, v.w))
                     : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    if (wave == 0) {
        float o = 0.f;
        const int n32 = (n + 31) & ~31;
        for (int j0 = 0; j0 < n32; j0 += 32) {
            float t[32];
#pragma unroll
            for (int i = 0; i < 32; ++i) t[i] = prod[(j0 + i) * PLD + lane];
#pragma unroll
            for (int i = 0; i < 32; ++i) o = __fadd_rn(o, t[i]);
        }
        att[h * HD + lane] = o;
        if constexpr (QOUT) quant32_store(o, att_q + h * HD + lane, att_s + (h * HD + lane) / 32, lane & 31);
    }
}

// Causal self-attention of one head (blockIdx.x) of one stream (blockIdx.y,
// its cache kv_stream floats after the previous stream's) over the pos+1
// cached positions (decoder.go:70-87): scores dotF32Go(q, k_j)*sc, softmax, and
// out[d] += p_j * v_j[d] in position order, unfused.  With QOUT (head_dim a
// multiple of 32) the head's outputs are also rounded to Q8_0 for the out
// projection.  Heads of 64 over at most kSmallN positions take the
// branch-free body above (the choice is uniform: n is read on the device).
template <bool QOUT>
__global__ __launch_bounds__(kAttnThreads) void self_attn_kernel(
    const float *__restrict__ q, const float *__restrict__ kc, const float *__restrict__ vc,
    const int *__restrict__ pos, int st, int hd, float sc, int rc, size_t kv_stream, float *__restrict__ att,
    int8_t *__restrict__ att_q, float *__restrict__ att_s, int ctx_rows) {
    extern __shared__ __align__(16) float sm[];
    const int h = blockIdx.x, tid = threadIdx.x, sm_ = blockIdx.y;  // head, stream
    const int n = *pos + 1;
    if (hd == kSmallHd && n <= kSmallN) {
        // thread j's K and V row j (many lanes loading one repeated row
        // measured far slower than leaving them out)
        const int j = min(min(tid, n - 1), ctx_rows - 1);
        const float4 *kr = reinterpret_cast<const float4 *>(kc + sm_ * kv_stream + (size_t)j * st + h * kSmallHd);
        const float4 *vr = reinterpret_cast<const float4 *>(vc + sm_ * kv_stream + (size_t)j * st + h * kSmallHd);
        float4 kv[kSmallHd / 4], vv[kSmallHd / 4];
        if (tid < n) {  // lanes past n load nothing
#pragma unroll
            for (int i = 0; i < kSmallHd / 4; ++i) kv[i] = kr[i];
#pragma unroll
            for (int i = 0; i < kSmallHd / 4; ++i) vv[i] = vr[i];
        } else {
#pragma unroll
            for (int i = 0; i < kSmallHd / 4; ++i) kv[i] = vv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        self_attn_small<QOUT>(sm, q + (size_t)sm_ * st, kv, vv, n, sc, att + (size_t)sm_ * st,
                              QOUT ? att_q + (size_t)sm_ * st : nullptr,
                              QOUT ? att_s + (size_t)sm_ * (st / 32) : nullptr);
        return;
    }
    float *part = sm, *s = sm + 32, *vl = sm + 32 + ((n + 3) & ~3);
    q += (size_t)sm_ * st;
    kc += sm_ * kv_stream;
    vc += sm_ * kv_stream;
    att += (size_t)sm_ * st;
    if constexpr (QOUT) {
        att_q += (size_t)sm_ * st;
        att_s += (size_t)sm_ * (st / 32);
    }
    const float *qh = q + h * hd;
    for (int j = tid; j < n; j += blockDim.x) s[j] = __fmul_rn(dot_go(qh, kc + (size_t)j * st + h * hd, hd), sc);
    __syncthreads();
    block_softmax(s, n, part);
    // the values, rc rows at a time through LDS, summed in position order
    float o = 0.f;
    for (int r0 = 0; r0 < n; r0 += rc) {
        const int rows = min(rc, n - r0);
        stage_rows(vl, vc + h * hd, st, r0, rows, hd);
        __syncthreads();
        if (tid < hd) {
#pragma unroll 16
            for (int j = 0; j < rows; ++j) o = __fadd_rn(o, __fmul_rn(s[r0 + j], vl[j * hd + tid]));
        }
        __syncthreads();
    }
    if (tid < hd) {
        att[h * hd + tid] = o;
        if constexpr (QOUT) quant32_store(o, att_q + h * hd + tid, att_s + (h * hd + tid) / 32, tid & 31);
    }
}

// Cross-attention scores of one head for a run of keys of stream blockIdx.z
// (its cross keys x_stream floats after the previous stream's) (decoder.go:94-108):
// dotF32x4 for the keys in whole groups of four, dotF32Go for the rest.
__global__ __launch_bounds__(64) void cross_scores_kernel(
    const float *__restrict__ q, const float *__restrict__ ck, int nctx, int hd, int st, size_t x_stream,
    float *__restrict__ scores) {
    const int h = blockIdx.x, j = blockIdx.y * blockDim.x + threadIdx.x, sm_ = blockIdx.z;  // stream sm_
    if (j >= nctx) return;
    q += (size_t)sm_ * st;
    ck += sm_ * x_stream;
    scores += (size_t)sm_ * (st / hd) * nctx;
    const float *qh = q + h * hd;
    const float *kj = ck + ((size_t)h * nctx + j) * hd;
    scores[(size_t)h * nctx + j] = j < (nctx & ~3) ? dot_x4(qh, kj, hd) : dot_go(qh, kj, hd);
}

// Row stride (floats) of the key rows staged by cross_scores64_kernel: a
// lane's 16-byte reads of its own row land in distinct banks.
constexpr int kXKeyLd = 68;

// cross_scores_kernel for heads of 64 values: the run's 64 key rows are
// staged through LDS with 16-byte loads, 16 lanes to a row (whole cache
// lines per load, where a lane reading its own row touches 64 lines), and
// lane j then takes key j's dotF32x4 / dotF32Go from LDS in the same order.
// Keys past nctx repeat the last one and are not written.
__global__ __launch_bounds__(64) void cross_scores64_kernel(const float *__restrict__ q,
                                                            const float *__restrict__ ck, int nctx, int st,
                                                            size_t x_stream, float *__restrict__ scores) {
    constexpr int HD = 64;
    __shared__ __align__(16) float lk[64 * kXKeyLd];
    const int h = blockIdx.x, lane = threadIdx.x, sm_ = blockIdx.z, j0 = blockIdx.y * 64;
    const float4 *kb = reinterpret_cast<const float4 *>(ck + sm_ * x_stream + (size_t)h * nctx * HD);
    float4 kv[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {  // piece 64u + lane: row (64u + lane) / 16, float4 lane % 16
        const int r = 4 * u + (lane >> 4), key = min(j0 + r, nctx - 1);
        kv[u] = kb[(size_t)key * (HD / 4) + (lane & 15)];
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) reinterpret_cast<float4 *>(lk + (4 * u + (lane >> 4)) * kXKeyLd)[lane & 15] = kv[u];
    __syncthreads();
    const int j = j0 + lane;
    if (j >= nctx) return;
    const float *qh = q + (size_t)sm_ * st + h * HD;
    const float *kr = lk + lane * kXKeyLd;
    scores[((size_t)sm_ * (st / HD) + h) * nctx + j] = j < (nctx & ~3) ? dot_x4(qh, kr, HD) : dot_go(qh, kr, HD);
}

// softmax of one head's scores (decoder.go:109) and its weighted values
// (decoder.go:110-118): out[d] = dotF32x4(p, Vt[d]) for d in groups of four
// (dotF32Go for a last partial group).  Each workgroup serves DG values of
// d of one head, 16 lanes per d: lane l (l < 8) runs the lane-l chain of the
// assembly's first accumulator, lane 8+l that of the second, in step order,
// the values fetched a batch of steps at a time; the tail past n &^ 15 is one
// lane's dotF32Go.  Every workgroup of a head computes the same softmax into
// its LDS.  With QOUT (DG == 32) the 32 outputs are rounded to Q8_0.
// blockIdx.z is the stream (its cross values x_stream floats after the
// previous stream's).
template <bool QOUT>
__global__ __launch_bounds__(512) void cross_values_kernel(const float *__restrict__ scores,
                                                          const float *__restrict__ cv, int nctx, int hd, int dg,
                                                          int st, size_t x_stream, float *__restrict__ att,
                                                          int8_t *__restrict__ att_q, float *__restrict__ att_s) {
    extern __shared__ float sm[];
    float *part = sm, *outv = sm + 32, *s = sm + 64;
    const int h = blockIdx.x, tid = threadIdx.x, sm_ = blockIdx.z;  // head, stream
    scores += (size_t)sm_ * (st / hd) * nctx;
    cv += sm_ * x_stream;
    att += (size_t)sm_ * st;
    if constexpr (QOUT) {
        att_q += (size_t)sm_ * st;
        att_s += (size_t)sm_ * (st / 32);
    }
    const float *row = scores + (size_t)h * nctx;
    for (int j = tid; j < nctx; j += blockDim.x) s[j] = row[j];
    __syncthreads();
    block_softmax(s, nctx, part);
    const int dl = tid >> 4, c = tid & 15;
    const int d = blockIdx.y * dg + dl;
    if (d < hd) {
        const float *vd = cv + ((size_t)h * hd + d) * nctx;
        float o;
        if (d >= (hd & ~3)) {  // a last partial group of d: dotF32Go
            o = dot_go(s, vd, nctx);
        } else {
            const int kk = nctx & ~15, steps = kk >> 4;
            float acc = 0.f;
            for (int t0 = 0; t0 < steps; t0 += kBatchV) {
                float vv[kBatchV];
#pragma unroll
                for (int u = 0; u < kBatchV; ++u) vv[u] = t0 + u < steps ? vd[16 * (t0 + u) + c] : 0.f;
#pragma unroll
                for (int u = 0; u < kBatchV; ++u)
                    if (t0 + u < steps) acc = __fmaf_rn(s[16 * (t0 + u) + c], vv[u], acc);
            }
            // S_l = A_l + B_l, then HSUM (kernels_amd64.s:194-202)
            const float other = __shfl_xor(acc, 8, 16);
            const float S = __fadd_rn(c < 8 ? acc : other, c < 8 ? other : acc);
            const float h4 = __fadd_rn(S, __shfl_xor(S, 4, 16));
            const float h01 = __fadd_rn(h4, __shfl_xor(h4, 1, 16));
            const float h23 = __shfl_xor(h01, 2, 16);
            o = kk > 0 ? __fadd_rn(h01, h23) : 0.f;
            if (c == 0 && kk < nctx) o = __fadd_rn(o, dot_go(s + kk, vd + kk, nctx - kk));
        }
        if (c == 0) {
            att[h * hd + d] = o;
            if (QOUT) outv[dl] = o;
        }
    }
    if constexpr (QOUT) {
        __syncthreads();
        if (tid < 32) {
            const int dd = blockIdx.y * 32 + tid;
            quant32_store(outv[tid], att_q + h * hd + dd, att_s + (h * hd + dd) / 32, tid);
        }
    }
}

// dotF32Go (gemm.go:294-308) of at most 15 values, r of them, without
// branches (clamped reads, selected sums).
__device__ __forceinline__ float dot_go15(const float *x, const float *y, int r) {
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    const int last = max(r - 1, 0);
#pragma unroll
    for (int i = 0; i < 12; i += 4) {
        const bool ok = i + 4 <= r;
        const float f0 = __fadd_rn(s0, __fmul_rn(x[min(i, last)], y[min(i, last)]));
        const float f1 = __fadd_rn(s1, __fmul_rn(x[min(i + 1, last)], y[min(i + 1, last)]));
        const float f2 = __fadd_rn(s2, __fmul_rn(x[min(i + 2, last)], y[min(i + 2, last)]));
        const float f3 = __fadd_rn(s3, __fmul_rn(x[min(i + 3, last)], y[min(i + 3, last)]));
        s0 = ok ? f0 : s0;
        s1 = ok ? f1 : s1;
        s2 = ok ? f2 : s2;
        s3 = ok ? f3 : s3;
    }
    const int r4 = r & ~3;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const float f = __fadd_rn(s0, __fmul_rn(x[min(r4 + i, last)], y[min(r4 + i, last)]));
        s0 = i < (r & 3) ? f : s0;
    }
    return __fadd_rn(__fadd_rn(__fadd_rn(s0, s1), s2), s3);
}

// Cross values without divergent branches, for nctx <= kFastCtx and head_dim
// a multiple of 4: the same softmax and dotF32x4 chains as
// cross_values_kernel, 32 values of d per workgroup of 512 threads.  Each
// lane's 96 values of V are loaded before the scores; each thread holds 3
// scores, the exps below n8 go to a chain-major copy for the eight sums
// (softmax_inv), and the probabilities to LDS for the chains.
constexpr int kFastCtx = 3 * 512;
template <bool QOUT>
__global__ __launch_bounds__(512) void cross_values_fast_kernel(const float *__restrict__ scores,
                                                                const float *__restrict__ cv, int nctx, int hd,
                                                                int st, size_t x_stream, float *__restrict__ att,
                                                                int8_t *__restrict__ att_q, float *__restrict__ att_s) {
    constexpr int NT = 512, PER = kFastCtx / NT, CS = kFastCtx / 8 + 32, KB = 96;
    __shared__ __align__(16) float ch[8 * CS + 8];
    __shared__ __align__(16) float p[kFastCtx + 16];
    __shared__ float red[32], outv[32];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, sm_ = blockIdx.z;
    scores += ((size_t)sm_ * (st / hd) + h) * nctx;
    cv += sm_ * x_stream;
    att += (size_t)sm_ * st;
    const int dl = tid >> 4, c = tid & 15, d = blockIdx.y * 32 + dl;
    const int kk = nctx & ~15, steps = kk >> 4;
    const float *vd = cv + ((size_t)h * hd + min(d, hd - 1)) * nctx;
    float vv[KB];
#pragma unroll
    for (int u = 0; u < KB; ++u) vv[u] = vd[min(16 * u + c, nctx - 1)];
    float sv[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) sv[u] = scores[min(tid + u * NT, nctx - 1)];
    float mx = sv[0];
#pragma unroll
    for (int u = 1; u < PER; ++u) mx = sv[u] > mx ? sv[u] : mx;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float t = __shfl_xor(mx, o);
        mx = t > mx ? t : mx;
    }
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) mx = red[w] > mx ? red[w] : mx;
    const int n8 = nctx & ~7;
    float e[PER];
    float *dummy = ch + 8 * CS;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const int j = tid + u * NT;
        const float dd = __fsub_rn(sv[u], mx);
        e[u] = j < n8 ? grx_exp8(dd) : grx_expf_go(dd);
        *(j < n8 ? ch + (j & 7) * CS + (j >> 3) : dummy) = e[u];
        *(j < nctx ? p + j : dummy + 1) = e[u];
    }
    __syncthreads();
    if (wave == 0) {
        const float inv = softmax_inv(ch, CS, p + n8, nctx);
        if (lane == 0) red[8] = inv;
    }
    __syncthreads();
    const float inv = red[8];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const int j = tid + u * NT;
        *(j < nctx ? p + j : dummy + 2) = __fmul_rn(e[u], inv);
    }
    __syncthreads();
    // dot4f32avx's lane chains over whole steps of 16, then HSUM
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < KB; ++u) {
        const float f = __fmaf_rn(p[16 * u + c], vv[u], acc);
        acc = u < steps ? f : acc;
    }
    const float other = __shfl_xor(acc, 8, 16);
    const float S = __fadd_rn(c < 8 ? acc : other, c < 8 ? other : acc);
    const float h4 = __fadd_rn(S, __shfl_xor(S, 4, 16));
    const float h01 = __fadd_rn(h4, __shfl_xor(h4, 1, 16));
    const float h23 = __shfl_xor(h01, 2, 16);
    float o = kk > 0 ? __fadd_rn(h01, h23) : 0.f;
    if (kk < nctx) o = __fadd_rn(o, dot_go15(p + kk, vd + kk, nctx - kk));
    if (c == 0) {
        if (d < hd) att[h * hd + d] = o;
        outv[dl] = o;
    }
    if constexpr (QOUT) {
        __syncthreads();
        if (tid < 32) {
            att_q += (size_t)sm_ * st;
            att_s += (size_t)sm_ * (st / 32);
            const int dd = blockIdx.y * 32 + tid;
            quant32_store(outv[tid], att_q + h * hd + dd, att_s + (h * hd + dd) / 32, tid);
        }
    }
}

// dotF32Go (gemm.go:294-308) of r < 16 values, x in LDS and y in registers,
// static indices only: whole groups of four into four running sums, the
// rest into the first, then ((s0 + s1) + s2) + s3.
__device__ __forceinline__ float dot_go15_reg(const float *x, const float (&y)[16], int r) {
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    const int r4 = r & ~3;
#pragma unroll
    for (int i = 0; i < 12; i += 4) {
        const bool ok = i + 4 <= r;
        const float f0 = __fadd_rn(s0, __fmul_rn(x[i], y[i]));
        const float f1 = __fadd_rn(s1, __fmul_rn(x[i + 1], y[i + 1]));
        const float f2 = __fadd_rn(s2, __fmul_rn(x[i + 2], y[i + 2]));
        const float f3 = __fadd_rn(s3, __fmul_rn(x[i + 3], y[i + 3]));
        s0 = ok ? f0 : s0;
        s1 = ok ? f1 : s1;
        s2 = ok ? f2 : s2;
        s3 = ok ? f3 : s3;
    }
#pragma unroll
    for (int i = 0; i < 15; ++i) {
        const float f = __fadd_rn(s0, __fmul_rn(x[i], y[i]));
        s0 = i >= r4 && i < r ? f : s0;
    }
    return __fadd_rn(__fadd_rn(__fadd_rn(s0, s1), s2), s3);
}

// Cross values for kWaveOut outputs d of one head of one stream, four waves
// (nctx <= kWaveCtx, head_dim % kWaveOut == 0): the head's softmax
// (decoder.go:109, block_softmax's order: expSubAVX below nctx &^ 7 with
// eight lane sums, expSubGo past it, 1 / sum, scale), then, as
// cross_values_fast_kernel, out[d] = dotF32x4(p, Vt[d]) with 16 lanes per d
// (lane c runs the chain of steps 16u + c), HSUM, dotF32Go for the tail.
// Every workgroup of a head redoes its softmax (6 exps per thread; each
// wave takes 1 / sum itself), so a head's values spread over
// hd / kWaveOut CUs.  The outputs are left in float32 (the next product
// rounds them).
constexpr int kWaveCtx = 1536, kWaveOut = 16;

__global__ __launch_bounds__(256) void cross_values_wave_kernel(const float *__restrict__ scores,
                                                                const float *__restrict__ cv, int nctx, int hd,
                                                                int st, size_t x_stream, float *__restrict__ att) {
    constexpr int NT = 256, PER = kWaveCtx / NT, CS = kWaveCtx / 8 + 4, G = 16, KB = kWaveCtx / 16;
    constexpr int R = KB + 4;  // row of pt: lane c's steps, 16-byte aligned
    __shared__ __align__(16) float ch[8 * CS + 8];  // exps below n8, chain-major (+ dummy slots)
    __shared__ __align__(16) float pt[16 * R];      // p[16u + c] at pt[c * R + u], u < steps
    __shared__ float tl[16], p2[16], red[4];        // exps past n8; p past 16 * steps
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, sm_ = blockIdx.z;
    scores += ((size_t)sm_ * (st / hd) + h) * nctx;
    att += (size_t)sm_ * st;
    const int dl = tid >> 4, c = tid & 15, d = blockIdx.y * kWaveOut + dl;
    const int kk = nctx & ~15, steps = kk >> 4, nfull = steps / G, ng = (steps + G - 1) / G;
    // values: one uniform base, 32-bit offsets
    const float *__restrict__ vb = cv + sm_ * x_stream + ((size_t)h * hd + blockIdx.y * kWaveOut) * nctx;
    // the scores first (loads return in order: the softmax waits for
    // nothing issued after them), then every value of this thread's chain,
    // in flight during the softmax
    float sv[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) sv[u] = scores[min(tid + NT * u, nctx - 1)];
    const int n8 = nctx & ~7, jt = n8 + tid;  // threads tid < nctx - n8 take the tail
    const float st_ = scores[min(jt, nctx - 1)];
    float vv[KB], vt[16];
#pragma unroll
    for (int u = 0; u < KB; ++u) vv[u] = vb[dl * nctx + min(16 * u + c, max(kk - 1, 0))];
    // the values past 16 * steps (dotF32Go's tail), ahead of need
#pragma unroll
    for (int i = 0; i < 16; ++i) vt[i] = vb[dl * nctx + min(kk + i, nctx - 1)];
    float mx = sv[0];
#pragma unroll
    for (int u = 1; u < PER; ++u) mx = sv[u] > mx ? sv[u] : mx;
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // EXP8 below n8 (branch-free), expf (scalar form) for the tail n8..nctx-1
    float e[PER];
    float *dummy = ch + 8 * CS;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const int jj = tid + NT * u;
        e[u] = grx_exp8(__fsub_rn(sv[u], mx));
        *(jj < n8 ? ch + (jj & 7) * CS + (jj >> 3) : dummy) = e[u];
    }
    const bool tail = jt < nctx;
    const float et = grx_expf_go(__fsub_rn(st_, mx));
    *(tail ? tl + tid : dummy + 1) = et;
    __syncthreads();
    const float inv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(softmax_inv(ch, CS, tl, nctx)), 0));
    // p = e * inv: below 16 * steps lane-major, past it in p2
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const int jj = tid + NT * u;
        const float pv = __fmul_rn(e[u], inv);
        *(jj < kk ? pt + (jj & 15) * R + (jj >> 4) : jj < n8 ? p2 + (jj - kk) : dummy + 2) = pv;
    }
    *(tail ? p2 + (jt - kk) : dummy + 3) = __fmul_rn(et, inv);
    __syncthreads();
    // dot4f32avx's lane chains over whole steps of 16
    const float4 *pr = reinterpret_cast<const float4 *>(pt + c * R);
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < KB / G; ++g) {
        if (g >= ng) break;  // uniform
        float4 pp[G / 4];
#pragma unroll
        for (int i = 0; i < G / 4; ++i) pp[i] = pr[(G / 4) * g + i];
        if (g < nfull) {
#pragma unroll
            for (int i = 0; i < G / 4; ++i) {
                acc = __fmaf_rn(pp[i].x, vv[G * g + 4 * i], acc);
                acc = __fmaf_rn(pp[i].y, vv[G * g + 4 * i + 1], acc);
                acc = __fmaf_rn(pp[i].z, vv[G * g + 4 * i + 2], acc);
                acc = __fmaf_rn(pp[i].w, vv[G * g + 4 * i + 3], acc);
            }
        } else {
            const int left = steps - G * g;
#pragma unroll
            for (int i = 0; i < G / 4; ++i) {
                float f = __fmaf_rn(pp[i].x, vv[G * g + 4 * i], acc);
                acc = 4 * i < left ? f : acc;
                f = __fmaf_rn(pp[i].y, vv[G * g + 4 * i + 1], acc);
                acc = 4 * i + 1 < left ? f : acc;
                f = __fmaf_rn(pp[i].z, vv[G * g + 4 * i + 2], acc);
                acc = 4 * i + 2 < left ? f : acc;
                f = __fmaf_rn(pp[i].w, vv[G * g + 4 * i + 3], acc);
                acc = 4 * i + 3 < left ? f : acc;
            }
        }
    }
    const float other = __shfl_xor(acc, 8, 16);
    const float S = __fadd_rn(c < 8 ? acc : other, c < 8 ? other : acc);
    const float h4 = __fadd_rn(S, __shfl_xor(S, 4, 16));
    const float h01 = __fadd_rn(h4, __shfl_xor(h4, 1, 16));
    const float h23 = __shfl_xor(h01, 2, 16);
    float o = kk > 0 ? __fadd_rn(h01, h23) : 0.f;
    if (kk < nctx) o = __fadd_rn(o, dot_go15_reg(p2, vt, nctx - kk));
    if (c == 0) att[h * hd + d] = o;
}

// ---------------------------------------------------------------- q|k|v + self-attention

// One stream's self-attention for head h (blockIdx.x), heads of 64, in one
// launch (decoder.go:60-87): the head's q, k and v (three 64-row tiles of
// the fused q|k|v weight on the int8 route: the LayerNorm'd row, or layer
// 0's embedding row, built by wave 0 as the products' prologue builds it,
// each output's fold in block order), k and v into the cache at pos, then
// the causal attention over pos+1 positions with self_attn_kernel's
// arithmetic (dotF32Go scores times sc, block_softmax's EXP8/expf split and
// sums, out[d] += p_j * v_j[d] in position order, unfused), the output
// rounded to Q8_0.  A decode step is a chain of dependent launches, each
// with a fixed cost of several microseconds, so the head's product and its
// attention share one; the cached keys and values of the first kQaChunk
// positions are loaded before the product starts, their latency hidden
// behind it.  Positions go to four threads each (a quarter of the head's 64
// dims): dotF32Go's four running sums pass from lane to lane, quarter by
// quarter in piece order, so every sum adds in the reference's order.
constexpr int kQaPf = 3;        // (tile, block) pairs per wave whose loads precede the prologue
constexpr int kQaChunk = 256;   // positions per pass (four threads each)
constexpr int kQaMaxN = 1024;   // longest context the kernel takes
constexpr int kQaPld = 68;      // floats between rows of products (16-byte writes in distinct banks)
constexpr int kQaCs = kQaMaxN / 8 + 4;

struct QaLds {
    size_t xs, q, red, s, pj, ch, big, total;
};
__host__ __device__ inline QaLds qkv_attn_lds(int nb) {
    QaLds o;
    const size_t K = (size_t)nb * GRX_QK;
    o.xs = (K + 15) & ~(size_t)15;
    o.q = o.xs + (((size_t)nb * 4 + 15) & ~(size_t)15);
    o.red = o.q + 3 * 64 * 4;
    o.s = o.red + 32 * 4;
    o.pj = o.s + (kQaMaxN + 8) * 4;
    o.ch = o.pj + (kQaMaxN + 8) * 4;
    o.big = o.ch + (8 * kQaCs + 16) * 4;
    const size_t lp = (size_t)3 * nb * 64 * 4, prod = (size_t)kQaChunk * kQaPld * 4;
    o.total = o.big + (lp > prod ? lp : prod);
    return o;
}

// 16 bytes at byte offset off of a buffer resource; offsets past its size
// read zeros and touch no memory (no branch, so the loads' wait counts stay
// exact)
typedef float grx_v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 rsrc_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const grx_v4f v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_float4(v.x, v.y, v.z, v.w);
}
// A buffer resource over the first n bytes at p (raw: no stride, no swizzle)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const float *p, uint32_t n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p), (short)0, (int)n, 0x00020000);
}

// row shift by one lane within rows of 16 (lane l receives lane l-1's value)
__device__ __forceinline__ float shr1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xf, 0xf, false));
}

template <int NP, int PRO>
__global__ __launch_bounds__(1024) void qkv_attn_kernel(const GemvArgs a, float sc, int ctx_rows,
                                                        float *__restrict__ att, int8_t *__restrict__ att_q,
                                                        float *__restrict__ att_s) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int W = 16;
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int st = a.seg, nb = a.nb, tpm = st >> 6;  // tiles per q, k or v matrix
    const int pos = *a.pos, n = pos + 1;
    const QaLds L = qkv_attn_lds(nb);
    int8_t *lxq = reinterpret_cast<int8_t *>(smem);
    float *lxs = reinterpret_cast<float *>(smem + L.xs);
    float *lq = reinterpret_cast<float *>(smem + L.q), *lk = lq + 64, *lv = lk + 64;
    float *red = reinterpret_cast<float *>(smem + L.red);
    float *sl = reinterpret_cast<float *>(smem + L.s), *pjl = reinterpret_cast<float *>(smem + L.pj);
    float *ch = reinterpret_cast<float *>(smem + L.ch), *dummy = ch + 8 * kQaCs;
    float *lp = reinterpret_cast<float *>(smem + L.big), *prod = lp;

    // ---- loads that wait for nothing: this wave's first (tile, block)
    // pairs.  The cached key and value quarters of positions 0..255
    // (thread t: position t / 4, quarter t % 4) go out once the row is
    // built (keys) and once the blocks' products are formed (values): issued
    // with the weights they would hold up the row the prologue waits for.
    // They read through buffer resources of pos rows: rows from pos on read
    // zeros without a memory access (row pos comes from LDS).
    const int p = tid >> 2, c = tid & 3;
    const int np = 3 * nb, ne = wave < np ? (np - wave + W - 1) / W : 0;
    const int4 *__restrict__ wq = reinterpret_cast<const int4 *>(a.qs);
    auto load_pair = [&](int e, int4 &w0, int4 &w1, uint32_t &dh) {
        const int u = e / nb, b = e - u * nb;
        const size_t blk = (size_t)(u * tpm + h) * nb + b;
        w0 = wq[blk * 128 + lane];
        w1 = wq[blk * 128 + 64 + lane];
        dh = a.ds[blk * 64 + lane];
    };
    int4 pw[2 * kQaPf];
    uint32_t pd[kQaPf];
    const int npf = min(kQaPf, ne);
    float4 kq[4], vq[4];
    const __amdgpu_buffer_rsrc_t krs = rsrc_of(a.kc, (uint32_t)pos * st * 4), vrs = rsrc_of(a.vc, (uint32_t)pos * st * 4);
    const uint32_t qoff = (uint32_t)(h * 64 + 16 * c) * 4;  // this thread's quarter within a row
    auto early = [&] {
#pragma unroll
        for (int u = 0; u < kQaPf; ++u)
            if (u < npf) load_pair(wave + u * W, pw[2 * u], pw[2 * u + 1], pd[u]);
    };
    if (wave != 0) early();
    float bias = 0.0f;
    if (wave < 3 && a.bias != nullptr) bias = a.bias[wave * st + h * 64 + lane];

    // ---- prologue (wave 0): the row, rounded to Q8_0, into LDS
    if (wave == 0) wave_row_prologue<NP, PRO>(a, 0, lxq, lxs, lane, h, early);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) kq[i] = rsrc_load4(krs, (uint32_t)p * st * 4 + qoff + 16 * i);

    // ---- block products of pair e = u * nb + b into lp [3 * nb][64]
    auto dots = [&](int e, const int4 &w0, const int4 &w1, uint32_t dh) {
        const int b = e - (e / nb) * nb;
        const int4 *pa = reinterpret_cast<const int4 *>(lxq + (size_t)b * GRX_QK);
        const int s = sdot8(w0, w1, pa[0], pa[1]);
        lp[(size_t)e * 64 + lane] = __fmul_rn((float)s, grx_f16_to_f32((uint16_t)dh));
    };
#pragma unroll
    for (int u = 0; u < kQaPf; ++u)
        if (u < npf) dots(wave + u * W, pw[2 * u], pw[2 * u + 1], pd[u]);
    for (int u0 = kQaPf; u0 < ne; u0 += kQaPf) {
        int4 w[2 * kQaPf];
        uint32_t dh[kQaPf];
        const int nv = min(kQaPf, ne - u0);
#pragma unroll
        for (int u = 0; u < kQaPf; ++u)
            if (u < nv) load_pair(wave + (u0 + u) * W, w[2 * u], w[2 * u + 1], dh[u]);
#pragma unroll
        for (int u = 0; u < kQaPf; ++u)
            if (u < nv) dots(wave + (u0 + u) * W, w[2 * u], w[2 * u + 1], dh[u]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) vq[i] = rsrc_load4(vrs, (uint32_t)p * st * 4 + qoff + 16 * i);
    __syncthreads();

    // ---- waves 0, 1, 2 fold q, k, v: c = fma(p_b, da_b, c) in block order
    if (wave < 3) {
        float acc = bias;
        const float *lpu = lp + (size_t)wave * nb * 64;
        int b = 0;
        for (; b + 8 <= nb; b += 8) {
            float t[8], s8[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                t[u] = lpu[(size_t)(b + u) * 64 + lane];
                s8[u] = lxs[b + u];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = __fmaf_rn(t[u], s8[u], acc);
        }
        for (; b < nb; ++b) acc = __fmaf_rn(lpu[(size_t)b * 64 + lane], lxs[b], acc);
        lq[wave * 64 + lane] = acc;  // lq, lk, lv
        if (wave == 1) a.kc[(size_t)pos * st + h * 64 + lane] = acc;
        if (wave == 2) a.vc[(size_t)pos * st + h * 64 + lane] = acc;
    }
    __syncthreads();

    // ---- scores of positions 0..n-1 (dotF32Go, gemm.go:294-308, times sc)
    float4 qv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[i] = reinterpret_cast<const float4 *>(lq + 16 * c)[i];
    const int nch = (n + kQaChunk - 1) / kQaChunk;
    for (int k = 0; k < nch; ++k) {
        const int j = k * kQaChunk + p;
        float4 kk[4];
        if (k == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) kk[i] = kq[i];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) kk[i] = rsrc_load4(krs, (uint32_t)j * st * 4 + qoff + 16 * i);
        }
        if (j == pos) {
#pragma unroll
            for (int i = 0; i < 4; ++i) kk[i] = reinterpret_cast<const float4 *>(lk + 16 * c)[i];
        }
        // quarter r extends the four sums quarter r-1 left (lane c's are
        // right once lane c-1's have arrived, after round c)
        float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (r > 0) {
                s0 = shr1(s0);
                s1 = shr1(s1);
                s2 = shr1(s2);
                s3 = shr1(s3);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s0 = __fadd_rn(s0, __fmul_rn(qv[i].x, kk[i].x));
                s1 = __fadd_rn(s1, __fmul_rn(qv[i].y, kk[i].y));
                s2 = __fadd_rn(s2, __fmul_rn(qv[i].z, kk[i].z));
                s3 = __fadd_rn(s3, __fmul_rn(qv[i].w, kk[i].w));
            }
        }
        if (c == 3 && j < n) sl[j] = __fmul_rn(__fadd_rn(__fadd_rn(__fadd_rn(s0, s1), s2), s3), sc);
    }
    __syncthreads();
    // ---- softmax (mathx.go:78-90 as block_softmax forms it): thread t
    // owns position t; waves with no position below n wait at the barriers
    // (the serial sums run faster without them on the same SIMDs)
    const bool live = tid < n, wlive = wave * 64 < n;
    const float sv = live ? sl[tid] : -__builtin_inff();
    float e = 0.0f;
    if (wlive) {
        const float m = wave_max(sv);
        if (lane == 0) red[wave] = m;
    }
    __syncthreads();
    if (wlive) {
        const int nw = (n + 63) >> 6;
        float mx = red[0];
        for (int w = 1; w < nw; ++w) mx = red[w] > mx ? red[w] : mx;
        const int n8 = n & ~7;
        const float d = __fsub_rn(sv, mx);
        const float e8 = grx_exp8(d), eg = grx_expf_go(d);
        e = tid < n8 ? e8 : eg;
        *(tid < n8 ? ch + (tid & 7) * kQaCs + (tid >> 3) : dummy) = e;
        *(live ? sl + tid : dummy + 1) = e;
    }
    __syncthreads();
    if (wave == 0) {
        const float inv = softmax_inv(ch, kQaCs, sl + (n & ~7), n);
        if (lane == 0) red[16] = inv;
    }
    __syncthreads();
    if (live) pjl[tid] = __fmul_rn(e, red[16]);
    __syncthreads();

    // ---- out[d] += p_j * v_j[d] in position order: each pass's products
    // into LDS (zeros past n), wave 0's lane d adds them in order
    float o = 0.f;
    for (int k = 0; k < nch; ++k) {
        const int j = k * kQaChunk + p;
        float4 vv[4];
        if (k == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) vv[i] = vq[i];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) vv[i] = rsrc_load4(vrs, (uint32_t)j * st * 4 + qoff + 16 * i);
        }
        if (j == pos) {
#pragma unroll
            for (int i = 0; i < 4; ++i) vv[i] = reinterpret_cast<const float4 *>(lv + 16 * c)[i];
        }
        const bool lj = j < n;
        const float pj = pjl[lj ? j : 0];
        float4 *pr = reinterpret_cast<float4 *>(prod + (size_t)p * kQaPld + 16 * c);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = vv[i];
            pr[i] = lj ? make_float4(__fmul_rn(pj, v.x), __fmul_rn(pj, v.y), __fmul_rn(pj, v.z), __fmul_rn(pj, v.w))
                       : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        __syncthreads();
        if (wave == 0) {
            const int rows = min(kQaChunk, n - k * kQaChunk), r32 = (rows + 31) & ~31;
            for (int j0 = 0; j0 < r32; j0 += 32) {
                float t[32];
#pragma unroll
                for (int i = 0; i < 32; ++i) t[i] = prod[(size_t)(j0 + i) * kQaPld + lane];
#pragma unroll
                for (int i = 0; i < 32; ++i) o = __fadd_rn(o, t[i]);
            }
        }
        __syncthreads();
    }
    if (wave == 0) {
        att[h * 64 + lane] = o;
        quant32_store(o, att_q + h * 64 + lane, att_s + (h * 64 + lane) / 32, lane & 31);
    }
}

// cross K (scaled) [h][t][d] and V [h][d][t] from K, V [t][h*hd+d]
// (whisper/encoder.go:131-142).
__global__ void cross_layout_kernel(const float *__restrict__ k, const float *__restrict__ v, int nctx, int st,
                                    int hd, float tsc, float *__restrict__ ck, float *__restrict__ cv) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)nctx * st) return;
    const int t = (int)(i / st), c = (int)(i % st);
    const int h = c / hd, d = c % hd;
    ck[((size_t)h * nctx + t) * hd + d] = __fmul_rn(k[i], tsc);
    cv[((size_t)h * hd + d) * nctx + t] = v[i];
}

}  // namespace

// ---------------------------------------------------------------- host side

struct WLayer {
    grx_weight *qkv = nullptr, *o = nullptr, *xq = nullptr, *xk = nullptr, *xv = nullptr, *xo = nullptr;
    grx_weight *fc1 = nullptr, *fc2 = nullptr;
    float *attn_ln_w, *attn_ln_b, *x_ln_w, *x_ln_b, *mlp_ln_w, *mlp_ln_b;
    float *qkv_b, *o_b, *xq_b, *xv_b, *xo_b, *fc1_b, *fc2_b;
    float *cross_k, *cross_v, *self_k, *self_v;
};

struct grx_whisper {
    grx_ctx *ctx = nullptr;
    grx_whisper_hparams hp{};
    int S = 1;  // streams decoded side by side (rows of every product)
    std::vector<bool> have_xs;  // cross K/V set, per stream
    std::map<std::string, std::vector<uint8_t>> host;  // set_tensor copies, until finalize
    bool ready = false, have_cross = false;
    std::vector<WLayer> L;
    grx_weight *tok_emb = nullptr;
    std::vector<void *> allocs;  // every device buffer below
    float *dec_pos = nullptr, *dec_ln_w = nullptr, *dec_ln_b = nullptr;
    float *x = nullptr, *q = nullptr, *att = nullptr, *ff = nullptr, *logits = nullptr, *scores = nullptr;
    int8_t *att_q = nullptr, *ff_q = nullptr;  // Q8_0 copies for the next product
    int8_t *ln_q = nullptr;                    // several streams: LayerNorm rows rounded once per product
    float *ln_s = nullptr;
    float *att_s = nullptr, *ff_s = nullptr;
    unsigned long long *amax = nullptr;
    unsigned long long *keys = nullptr;  // argmax keys, [vocabulary tiles][streams]
    unsigned int *counter = nullptr;
    int *tok = nullptr, *pos = nullptr, *hist = nullptr;
    float *xenc = nullptr, *xk_tmp = nullptr, *xv_tmp = nullptr;  // cross K/V precompute staging
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int pos_host = 0;
    // the decode loop with the token rules (grx_whisper_rules_loop)
    float *samp_g = nullptr;            // the sampler's terms, 2 x 64k floats
    int *samp_sup = nullptr;            // the suppress list
    int samp_sup_cap = 0;
    GrxLoopDev *loop_st = nullptr;      // the sequence and the loop counter
    grx_whisper_token *loop_rec = nullptr;  // [n_text_ctx] the tokens sampled
    float *loop_rs = nullptr;           // [n_text_ctx] draws
};

namespace {

struct Expect {
    std::string name;
    size_t bytes;
};

// Every decoder tensor Model.bind reads (whisper/model.go:376-401), with its size.
std::vector<Expect> expected(const grx_whisper_hparams &hp) {
    const size_t st = hp.n_state;
    auto q8 = [](size_t rows, size_t cols) { return rows * (cols / 32) * 34; };
    std::vector<Expect> e;
    e.push_back({"decoder.positional_embedding", (size_t)hp.n_text_ctx * st * 4});
    e.push_back({"decoder.token_embedding.weight", q8(hp.n_vocab, st)});
    e.push_back({"decoder.ln.weight", st * 4});
    e.push_back({"decoder.ln.bias", st * 4});
    for (int i = 0; i < hp.n_layer; ++i) {
        const std::string p = "decoder.blocks." + std::to_string(i) + ".";
        for (const char *ln : {"attn_ln", "cross_attn_ln", "mlp_ln"}) {
            e.push_back({p + ln + ".weight", st * 4});
            e.push_back({p + ln + ".bias", st * 4});
        }
        for (const char *a : {"attn", "cross_attn"}) {
            for (const char *w : {"query", "key", "value", "out"}) e.push_back({p + a + "." + w + ".weight", q8(st, st)});
            for (const char *b : {"query", "value", "out"}) e.push_back({p + a + "." + b + ".bias", st * 4});
        }
        e.push_back({p + "mlp.0.weight", q8(4 * st, st)});
        e.push_back({p + "mlp.0.bias", 4 * st * 4});
        e.push_back({p + "mlp.2.weight", q8(st, 4 * st)});
        e.push_back({p + "mlp.2.bias", st * 4});
    }
    return e;
}

grx_status dev_alloc(grx_whisper *m, size_t bytes, void **out) {
    void *p = nullptr;
    GRX_HIP(grx_dev_malloc(&p, bytes > 0 ? bytes : 16));
    m->allocs.push_back(p);
    *out = p;
    return GRX_OK;
}

template <typename T>
grx_status dev_alloc_t(grx_whisper *m, size_t count, T **out) {
    return dev_alloc(m, count * sizeof(T), reinterpret_cast<void **>(out));
}

grx_status upload_vec(grx_whisper *m, const std::string &name, float **out) {
    const auto &h = m->host.at(name);
    grx_status s = dev_alloc(m, h.size(), reinterpret_cast<void **>(out));
    if (s != GRX_OK) return s;
    GRX_HIP(hipMemcpy(*out, h.data(), h.size(), hipMemcpyHostToDevice));
    return GRX_OK;
}

// What finalize made (weights, constants and step buffers), released: after
// a failed finalize the model is as before it (its host tensors kept), and
// grx_whisper_destroy releases a finished one.
void wrelease(grx_whisper *m) {
    for (WLayer &L : m->L)
        for (grx_weight *w : {L.qkv, L.o, L.xq, L.xk, L.xv, L.xo, L.fc1, L.fc2}) grx_weight_destroy(w);
    m->L.clear();
    grx_weight_destroy(m->tok_emb);
    m->tok_emb = nullptr;
    for (void *p : m->allocs) (void)hipFree(p);
    m->allocs.clear();
}

grx_status finalize_tensors(grx_whisper *m);

grx_status finalize(grx_whisper *m) {
    if (m->ready) return GRX_OK;
    const grx_status s = finalize_tensors(m);
    if (s != GRX_OK) wrelease(m);
    return s;
}

grx_status finalize_tensors(grx_whisper *m) {
    const grx_whisper_hparams &hp = m->hp;
    for (const Expect &e : expected(hp))
        if (!m->host.count(e.name)) return grx_fail(GRX_ESTATE, "the model file has no tensor %s", e.name.c_str());
    grx_status s;
    const int st = hp.n_state, hd = st / hp.n_head;
    GRX_HIP(hipSetDevice(m->ctx->device));
    {
        const auto &t = m->host.at("decoder.token_embedding.weight");
        if ((s = grx_weight_q8_create(m->ctx, hp.n_vocab, st, t.data(), t.size(), &m->tok_emb)) != GRX_OK) return s;
    }
    if ((s = upload_vec(m, "decoder.positional_embedding", &m->dec_pos)) != GRX_OK) return s;
    if ((s = upload_vec(m, "decoder.ln.weight", &m->dec_ln_w)) != GRX_OK) return s;
    if ((s = upload_vec(m, "decoder.ln.bias", &m->dec_ln_b)) != GRX_OK) return s;
    m->L.assign(hp.n_layer, WLayer());
    for (int i = 0; i < hp.n_layer; ++i) {
        WLayer &L = m->L[i];
        const std::string p = "decoder.blocks." + std::to_string(i) + ".";
        auto mat = [&](const std::string &n, int rows, int cols, grx_weight **w) {
            const auto &t = m->host.at(p + n);
            return grx_weight_q8_create(m->ctx, rows, cols, t.data(), t.size(), w);
        };
        // q, k and v share their input: one weight of 3*st rows, one launch.
        {
            std::vector<uint8_t> cat;
            for (const char *w : {"attn.query.weight", "attn.key.weight", "attn.value.weight"}) {
                const auto &t = m->host.at(p + w);
                cat.insert(cat.end(), t.begin(), t.end());
            }
            if ((s = grx_weight_q8_create(m->ctx, 3 * st, st, cat.data(), cat.size(), &L.qkv)) != GRX_OK) return s;
            std::vector<float> b(3 * st, 0.0f);  // the key has no bias (decoder.go:65)
            memcpy(b.data(), m->host.at(p + "attn.query.bias").data(), st * 4);
            memcpy(b.data() + 2 * st, m->host.at(p + "attn.value.bias").data(), st * 4);
            if ((s = dev_alloc_t(m, 3 * st, &L.qkv_b)) != GRX_OK) return s;
            GRX_HIP(hipMemcpy(L.qkv_b, b.data(), b.size() * 4, hipMemcpyHostToDevice));
        }
        if ((s = mat("attn.out.weight", st, st, &L.o)) != GRX_OK) return s;
        if ((s = mat("cross_attn.query.weight", st, st, &L.xq)) != GRX_OK) return s;
        if ((s = mat("cross_attn.key.weight", st, st, &L.xk)) != GRX_OK) return s;
        if ((s = mat("cross_attn.value.weight", st, st, &L.xv)) != GRX_OK) return s;
        if ((s = mat("cross_attn.out.weight", st, st, &L.xo)) != GRX_OK) return s;
        if ((s = mat("mlp.0.weight", 4 * st, st, &L.fc1)) != GRX_OK) return s;
        if ((s = mat("mlp.2.weight", st, 4 * st, &L.fc2)) != GRX_OK) return s;
        struct {
            const char *n;
            float **d;
        } vecs[] = {{"attn_ln.weight", &L.attn_ln_w},       {"attn_ln.bias", &L.attn_ln_b},
                    {"cross_attn_ln.weight", &L.x_ln_w},    {"cross_attn_ln.bias", &L.x_ln_b},
                    {"mlp_ln.weight", &L.mlp_ln_w},         {"mlp_ln.bias", &L.mlp_ln_b},
                    {"attn.out.bias", &L.o_b},              {"cross_attn.query.bias", &L.xq_b},
                    {"cross_attn.value.bias", &L.xv_b},     {"cross_attn.out.bias", &L.xo_b},
                    {"mlp.0.bias", &L.fc1_b},               {"mlp.2.bias", &L.fc2_b}};
        for (auto &v : vecs)
            if ((s = upload_vec(m, p + v.n, v.d)) != GRX_OK) return s;
        const size_t cross = (size_t)m->S * hp.n_audio_ctx * st, self = (size_t)m->S * hp.n_text_ctx * st;
        if ((s = dev_alloc_t(m, cross, &L.cross_k)) != GRX_OK) return s;
        if ((s = dev_alloc_t(m, cross, &L.cross_v)) != GRX_OK) return s;
        if ((s = dev_alloc_t(m, self, &L.self_k)) != GRX_OK) return s;
        if ((s = dev_alloc_t(m, self, &L.self_v)) != GRX_OK) return s;
        GRX_HIP(hipMemset(L.self_k, 0, self * 4));
        GRX_HIP(hipMemset(L.self_v, 0, self * 4));
    }
    const size_t S = m->S;
    if ((s = dev_alloc_t(m, S * st, &m->x)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, S * st, &m->q)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, S * st, &m->att)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, S * 4 * (size_t)st, &m->ff)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, S * hp.n_vocab, &m->logits)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, S * hp.n_head * hp.n_audio_ctx, &m->scores)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, S * st, &m->att_q)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, S * st, &m->ln_q)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, S * st / 32, &m->ln_s)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, S * st / 32, &m->att_s)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, S * 4 * (size_t)st, &m->ff_q)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, S * 4 * (size_t)st / 32, &m->ff_s)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, 1, &m->counter)) != GRX_OK) return s;
    GRX_HIP(hipMemset(m->counter, 0, 4));
    if ((s = dev_alloc_t(m, S, &m->amax)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, (size_t)grx_ceil_div(hp.n_vocab, 64) * S, &m->keys)) != GRX_OK) return s;
    GRX_HIP(hipMemset(m->amax, 0, 8 * S));
    if ((s = dev_alloc_t(m, S, &m->tok)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, 1, &m->pos)) != GRX_OK) return s;
    if ((s = dev_alloc_t(m, S * hp.n_text_ctx, &m->hist)) != GRX_OK) return s;
    GRX_HIP(hipMemset(m->pos, 0, 4));
    GRX_HIP(hipMemset(m->tok, 0, 4 * S));
    m->host.clear();
    m->ready = true;
    (void)hd;
    return GRX_OK;
}

// The decode step's products read their weights with ordinary loads: the
// step's 52 MB of weights stay in the 256 MB Infinity Cache from token to token.
GemvArgs gemv_args(const grx_weight *w) {
    GemvArgs a = {};
    a.qs = w->qs;
    a.ds = w->ds;
    a.rows = w->rows;
    a.nb = w->nb;
    a.cacheable = 1;
    return a;
}

// A kernel choice tuned to 0 (for comparisons in tests).
bool tuned_off(int id) { return grx_tune(id) == 0; }

// One stream's fused q|k|v + self-attention of every head (qkv_attn_kernel).
template <int NP, int PRO>
grx_status launch_qkv_attn(hipStream_t stream, const GemvArgs &a, int nh, float sc, int ctx_rows, grx_whisper *m) {
    static bool raised = false;  // set by the eager step that precedes any capture
    if (!raised) {
        raised = true;
        GRX_HIP(hipFuncSetAttribute((const void *)qkv_attn_kernel<NP, PRO>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    160 * 1024));
    }
    qkv_attn_kernel<NP, PRO><<<nh, 1024, qkv_attn_lds(a.nb).total, stream>>>(a, sc, ctx_rows, m->att, m->att_q,
                                                                               m->att_s);
    GRX_LAUNCHED("qkv_attn_kernel");
    return GRX_OK;
}

// The launches of one decode step on stream st.
grx_status enqueue_step(grx_whisper *m, hipStream_t stream) {
    const grx_whisper_hparams &hp = m->hp;
    const int st = hp.n_state, nh = hp.n_head, hd = st / nh, nctx = hp.n_audio_ctx;
    const float sc = (float)(1.0 / sqrt((double)hd));
    const bool qatt = hd % 32 == 0;  // attention outputs are whole Q8_0 blocks per head
    grx_status s;
    const int rc = std::max(1, std::min(hp.n_text_ctx, (48 * 1024) / (hd * 4)));
    size_t attn_smem = (32 + (((size_t)hp.n_text_ctx + 3) & ~(size_t)3) + (size_t)rc * hd) * 4;
    if (hd == kSmallHd) {
        attn_smem = std::max(attn_smem, kSmallLds * 4);
        static bool raised = false;  // set by the eager step that precedes any capture
        if (!raised) {
            raised = true;
            GRX_HIP(hipFuncSetAttribute((const void *)self_attn_kernel<true>,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)(kSmallLds * 4)));
            GRX_HIP(hipFuncSetAttribute((const void *)self_attn_kernel<false>,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)(kSmallLds * 4)));
        }
    }
    const size_t val_smem = (64 + (size_t)nctx) * 4;
    const int dg = qatt ? 32 : 4;
    const int S = m->S;  // rows of every product: one per stream
    const size_t kv_stream = (size_t)hp.n_text_ctx * st, x_stream = (size_t)nctx * st;
    // streams at one position: each row its own token, cache and record
    auto gemv_args = [&](const grx_weight *w) {
        GemvArgs a = ::gemv_args(w);
        a.streams = S > 1;
        a.kv_stream = kv_stream;
        a.hist_stream = hp.n_text_ctx;
        return a;
    };
    // Several streams: the product's prologue builds each stream's row with
    // one wave per row (rows up to 1280 values); wider rows are LayerNorm'd
    // and rounded once by a row kernel and read pre-rounded
    // (GRX_FUSE_LN=0 takes that route for every width).
    const bool sep = S > 1 && (st > 1280 || tuned_off(GRX_TUNE_FUSE_LN));
    auto ln_rows = [&](const float *w, const float *b, GemvArgs &a) {
        a.xq = m->ln_q;
        a.xs = m->ln_s;
        return grx_ln_quant_rows(stream, m->x, st, S, st, w, b, m->ln_q, m->ln_s);
    };
    // one stream, heads of 64: each head's q|k|v product and its attention
    // in one launch (rows up to 512 values: wider rows' prologue registers
    // do not fit beside the prefetched keys and values; contexts up to
    // kQaMaxN)
    const bool fused_attn = S == 1 && hd == 64 && st % 64 == 0 && st <= 512 && hp.n_text_ctx <= kQaMaxN &&
                            !tuned_off(GRX_TUNE_FUSE_SELF_ATTN);
    for (int li = 0; li < hp.n_layer; ++li) {
        WLayer &L = m->L[li];
        if (fused_attn) {
            GemvArgs a = gemv_args(L.qkv);
            a.x = m->x;
            a.lda = st;
            a.ln_w = L.attn_ln_w;
            a.ln_b = L.attn_ln_b;
            a.bias = L.qkv_b;
            a.seg = st;
            a.kc = L.self_k;
            a.vc = L.self_v;
            a.pos = m->pos;
            if (li == 0) {
                a.tok = m->tok;
                a.emb_qs = m->tok_emb->qs;
                a.emb_ds = m->tok_emb->ds;
                a.pos_emb = m->dec_pos;
                a.x_out = m->x;
            }
            s = li == 0 ? launch_qkv_attn<2, GRX_PRO_EMBED_LN>(stream, a, nh, sc, hp.n_text_ctx, m)
                        : launch_qkv_attn<2, GRX_PRO_LN>(stream, a, nh, sc, hp.n_text_ctx, m);
            if (s != GRX_OK) return s;
        } else {  // LN -> q | k | v, k and v into the cache at pos; layer 0 embeds first
            GemvArgs a = gemv_args(L.qkv);
            a.x = m->x;
            a.lda = st;
            a.ln_w = L.attn_ln_w;
            a.ln_b = L.attn_ln_b;
            a.y = m->q;
            a.ldc = st;
            a.bias = L.qkv_b;
            a.seg = st;
            a.kc = L.self_k;
            a.vc = L.self_v;
            a.pos = m->pos;
            int pro = GRX_PRO_LN;
            if (li == 0) {
                pro = GRX_PRO_EMBED_LN;
                a.tok = m->tok;
                a.emb_qs = m->tok_emb->qs;
                a.emb_ds = m->tok_emb->ds;
                a.pos_emb = m->dec_pos;
                a.x_out = m->x;
            }
            if (sep) {
                pro = GRX_PRO_PREQ;
                a.xq = m->ln_q;
                a.xs = m->ln_s;
                s = li == 0 ? grx_embed_ln_quant_rows(stream, m->tok, m->pos, m->tok_emb, m->dec_pos, m->x, S,
                                                      L.attn_ln_w, L.attn_ln_b, m->ln_q, m->ln_s)
                            : grx_ln_quant_rows(stream, m->x, st, S, st, L.attn_ln_w, L.attn_ln_b, m->ln_q, m->ln_s);
                if (s != GRX_OK) return s;
            }
            if ((s = grx_gemv_launch(stream, S, pro, GRX_EPI_QKV, a, 0)) != GRX_OK) return s;
            if (qatt)
                self_attn_kernel<true><<<dim3(nh, S), kAttnThreads, attn_smem, stream>>>(
                    m->q, L.self_k, L.self_v, m->pos, st, hd, sc, rc, kv_stream, m->att, m->att_q, m->att_s,
                    hp.n_text_ctx);
            else
                self_attn_kernel<false><<<dim3(nh, S), kAttnThreads, attn_smem, stream>>>(
                    m->q, L.self_k, L.self_v, m->pos, st, hd, sc, rc, kv_stream, m->att, nullptr, nullptr,
                    hp.n_text_ctx);
            GRX_LAUNCHED("self_attn_kernel");
        }
        auto out_proj = [&](grx_weight *w, const float *b, bool rounded) {  // x += att . W^T + b
            if (S > 1 && w->nb <= 128) {
                // several streams: the K-split matrix-core product, its
                // blocks over ~10 waves per 16-column tile (the GEMV puts a
                // 1280-row product on 20 workgroups)
                if (!rounded && (s = grx_quant_rows(stream, m->att, st, S, st, m->att_q, m->att_s)) != GRX_OK)
                    return s;
                GemmOut o;
                o.y = m->x;
                o.ldc = st;
                o.epi = GRX_GEMM_ADD;
                return grx_gemm_q8_launch_ex(stream, w, m->att_q, m->att_s, S, b, o);
            }
            GemvArgs a = gemv_args(w);
            a.x = m->att;
            a.lda = st;
            a.xq = m->att_q;
            a.xs = m->att_s;
            a.y = m->x;
            a.ldc = st;
            a.bias = b;
            a.resid = m->x;
            a.ldr = st;
            return grx_gemv_launch(stream, S, rounded ? GRX_PRO_PREQ : GRX_PRO_QUANT, GRX_EPI_RESID, a, 0);
        };
        if ((s = out_proj(L.o, L.o_b, qatt)) != GRX_OK) return s;
        // one stream, heads of 64: the cross query's tile of each head is
        // computed inside the scores kernel (one launch instead of two)
        const bool fused_scores = S == 1 && hd == 64 && st >= 512 && st <= 1280 && !tuned_off(GRX_TUNE_FUSE_XSCORES);
        if (fused_scores) {
            GemvArgs a = gemv_args(L.xq);
            a.x = m->x;
            a.lda = st;
            a.ln_w = L.x_ln_w;
            a.ln_b = L.x_ln_b;
            a.bias = L.xq_b;
            a.xk = L.cross_k;
            a.nctx = nctx;
            a.scores = m->scores;
            if ((s = grx_gemv_launch(stream, 1, GRX_PRO_LN, GRX_EPI_XSCORES, a, 16)) != GRX_OK) return s;
        } else {  // LN -> cross query
            GemvArgs a = gemv_args(L.xq);
            a.x = m->x;
            a.lda = st;
            a.ln_w = L.x_ln_w;
            a.ln_b = L.x_ln_b;
            a.y = m->q;
            a.ldc = st;
            a.bias = L.xq_b;
            if (sep && (s = ln_rows(L.x_ln_w, L.x_ln_b, a)) != GRX_OK) return s;
            if ((s = grx_gemv_launch(stream, S, sep ? GRX_PRO_PREQ : GRX_PRO_LN, GRX_EPI_STORE, a, 0)) != GRX_OK)
                return s;
            if (hd == 64) {
                cross_scores64_kernel<<<dim3(nh, grx_ceil_div(nctx, 64), S), 64, 0, stream>>>(
                    m->q, L.cross_k, nctx, st, x_stream, m->scores);
            } else {
                cross_scores_kernel<<<dim3(nh, grx_ceil_div(nctx, 64), S), 64, 0, stream>>>(
                    m->q, L.cross_k, nctx, hd, st, x_stream, m->scores);
            }
            GRX_LAUNCHED("cross_scores_kernel");
        }
        // workgroups over 16 outputs each, float32 out (the cross-out product
        // rounds its rows in its prologue; several streams: a wave per row)
        const bool wave_values = nctx <= kWaveCtx && hd % kWaveOut == 0 && (S == 1 || st <= 1280) &&
                                 !tuned_off(GRX_TUNE_WAVE_VALUES);
        if (wave_values) {
            cross_values_wave_kernel<<<dim3(nh, hd / kWaveOut, S), 256, 0, stream>>>(m->scores, L.cross_v, nctx,
                                                                                     hd, st, x_stream, m->att);
        } else if (nctx <= kFastCtx && hd % 4 == 0) {
            if (qatt)
                cross_values_fast_kernel<true><<<dim3(nh, grx_ceil_div(hd, 32), S), 512, 0, stream>>>(
                    m->scores, L.cross_v, nctx, hd, st, x_stream, m->att, m->att_q, m->att_s);
            else
                cross_values_fast_kernel<false><<<dim3(nh, grx_ceil_div(hd, 32), S), 512, 0, stream>>>(
                    m->scores, L.cross_v, nctx, hd, st, x_stream, m->att, nullptr, nullptr);
        } else if (qatt) {
            cross_values_kernel<true><<<dim3(nh, grx_ceil_div(hd, dg), S), dg * 16, val_smem, stream>>>(
                m->scores, L.cross_v, nctx, hd, dg, st, x_stream, m->att, m->att_q, m->att_s);
        } else {
            cross_values_kernel<false><<<dim3(nh, grx_ceil_div(hd, dg), S), dg * 16, val_smem, stream>>>(
                m->scores, L.cross_v, nctx, hd, dg, st, x_stream, m->att, nullptr, nullptr);
        }
        GRX_LAUNCHED("cross_values_kernel");
        if ((s = out_proj(L.xo, L.xo_b, qatt && !wave_values)) != GRX_OK) return s;
        {  // LN -> fc1 -> GELU, rounded to Q8_0 for fc2
            GemvArgs a = gemv_args(L.fc1);
            a.x = m->x;
            a.lda = st;
            a.ln_w = L.mlp_ln_w;
            a.ln_b = L.mlp_ln_b;
            a.y = m->ff;
            a.ldc = 4 * st;
            a.bias = L.fc1_b;
            a.yq = m->ff_q;
            a.ys = m->ff_s;
            if (sep && (s = ln_rows(L.mlp_ln_w, L.mlp_ln_b, a)) != GRX_OK) return s;
            if ((s = grx_gemv_launch(stream, S, sep ? GRX_PRO_PREQ : GRX_PRO_LN, GRX_EPI_GELU_Q, a, 0)) != GRX_OK)
                return s;
        }
        if (S > 1) {  // x += ff . Wfc2^T + b, several streams: the K-split product, the chain carried in q
            GemmOut o;
            o.y = m->x;
            o.ldc = st;
            o.epi = GRX_GEMM_ADD;
            o.carry = m->q;
            if ((s = grx_gemm_q8_launch_ex(stream, L.fc2, m->ff_q, m->ff_s, S, L.fc2_b, o)) != GRX_OK) return s;
        } else {  // x += ff . Wfc2^T + b
            GemvArgs a = gemv_args(L.fc2);
            a.xq = m->ff_q;
            a.xs = m->ff_s;
            a.y = m->x;
            a.ldc = st;
            a.bias = L.fc2_b;
            a.resid = m->x;
            a.ldr = st;
            if ((s = grx_gemv_launch(stream, S, GRX_PRO_PREQ, GRX_EPI_RESID, a, 0)) != GRX_OK) return s;
        }
    }
    {  // LN -> logits = tokEmb . h -> argmax; the last workgroup ends the step
        GemvArgs a = gemv_args(m->tok_emb);
        a.cacheable = 0;  // 26.5 MB streamed once per step: non-temporal loads
        a.x = m->x;
        a.lda = st;
        a.ln_w = m->dec_ln_w;
        a.ln_b = m->dec_ln_b;
        a.y = m->logits;
        a.ldc = hp.n_vocab;
        // per-workgroup argmax keys and a one-workgroup end of step (no
        // contended atomics); ARGMAX_ATOMIC tuned to 1 takes the atomic form
        const bool atomic_form = grx_tune(GRX_TUNE_ARGMAX_ATOMIC) == 1;
        a.amax = m->amax;
        if (atomic_form)
            a.counter = m->counter;
        else
            a.keys = m->keys;
        a.tok_w = m->tok;
        a.pos = m->pos;
        a.pos_w = m->pos;
        a.hist = m->hist;
        if (sep && (s = ln_rows(m->dec_ln_w, m->dec_ln_b, a)) != GRX_OK) return s;
        if ((s = grx_gemv_launch(stream, S, sep ? GRX_PRO_PREQ : GRX_PRO_LN, GRX_EPI_ARGMAX, a, 0)) != GRX_OK)
            return s;
    }
    return GRX_OK;
}

// One step: the captured graph, or (GRX_NO_GRAPH=1, or capture refused)
// the same launches directly.
grx_status run_step(grx_whisper *m) {
    hipStream_t stream = m->ctx->stream;
    if (grx_tune(GRX_TUNE_NO_GRAPH) == 1) return enqueue_step(m, stream);
    if (!m->exec) {
        // an eager step first sets every kernel's attributes outside capture;
        // its effect is undone by the caller's bookkeeping (it runs the step
        // it was asked to run)
        grx_status s = enqueue_step(m, stream);
        if (s != GRX_OK) return s;
        GRX_HIP(hipStreamSynchronize(stream));
        hipError_t e = hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal);
        if (e == hipSuccess) {
            s = enqueue_step(m, stream);
            hipGraph_t g = nullptr;
            e = hipStreamEndCapture(stream, &g);
            if (s == GRX_OK && e == hipSuccess) e = hipGraphInstantiate(&m->exec, g, nullptr, nullptr, 0);
            if (g) {
                if (e == hipSuccess) m->graph = g;
                else (void)hipGraphDestroy(g);
            }
        }
        if (e != hipSuccess || s != GRX_OK) {
            (void)hipGetLastError();
            m->exec = nullptr;
        }
        return GRX_OK;
    }
    GRX_HIP(hipGraphLaunch(m->exec, stream));
    return GRX_OK;
}

}  // namespace

extern "C" grx_status grx_whisper_create(grx_ctx *ctx, const grx_whisper_hparams *hp, grx_whisper **out) {
    return grx_whisper_create_streams(ctx, hp, 1, out);
}

extern "C" grx_status grx_whisper_create_streams(grx_ctx *ctx, const grx_whisper_hparams *hp, int n_streams,
                                                 grx_whisper **out) {
    if (!ctx || !hp || !out) return grx_fail(GRX_EINVAL, "grx_whisper_create: NULL argument");
    *out = nullptr;
    if (n_streams != 1 && n_streams != 2 && n_streams != 4 && n_streams != 8)
        return grx_fail(GRX_EINVAL, "grx_whisper_create_streams: %d streams (1, 2, 4 or 8)", n_streams);
    if (hp->n_vocab <= 0 || hp->n_text_ctx <= 0 || hp->n_state <= 0 || hp->n_head <= 0 || hp->n_layer <= 0 ||
        hp->n_audio_ctx <= 0)
        return grx_fail(GRX_EINVAL, "grx_whisper_create: every size must be positive");
    if (hp->n_state % 32 != 0 || hp->n_state % hp->n_head != 0)
        return grx_fail(GRX_ESIZE, "grx_whisper_create: n_state %d must be a multiple of 32 and of n_head %d",
                        hp->n_state, hp->n_head);
    grx_whisper *m = new grx_whisper();
    m->ctx = ctx;
    m->hp = *hp;
    m->S = n_streams;
    m->have_xs.assign(n_streams, false);
    *out = m;
    return GRX_OK;
}

extern "C" int grx_whisper_streams(const grx_whisper *m) { return m ? m->S : 0; }

extern "C" grx_status grx_whisper_destroy(grx_whisper *m) {
    if (!m) return GRX_OK;
    GRX_HIP(hipSetDevice(m->ctx->device));
    GRX_HIP(hipStreamSynchronize(m->ctx->stream));
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    wrelease(m);
    delete m;
    return GRX_OK;
}

extern "C" grx_status grx_whisper_set_tensor(grx_whisper *m, const char *name, const void *data, size_t nbytes) {
    if (!m || !name || (!data && nbytes)) return grx_fail(GRX_EINVAL, "grx_whisper_set_tensor: NULL argument");
    if (m->ready) return grx_fail(GRX_ESTATE, "grx_whisper_set_tensor: the model is in use already");
    for (const Expect &e : expected(m->hp)) {
        if (e.name != name) continue;
        if (nbytes != e.bytes)
            return grx_fail(GRX_ESIZE, "tensor %s has the wrong shape (%zu bytes, want %zu)", name, nbytes, e.bytes);
        const uint8_t *p = static_cast<const uint8_t *>(data);
        m->host[name].assign(p, p + nbytes);
        return GRX_OK;
    }
    return grx_fail(GRX_EINVAL, "the model file has a tensor this program doesn't know: %s", name);
}

extern "C" grx_status grx_whisper_set_encoder_output(grx_whisper *m, const float *enc, int n_audio_ctx) {
    return grx_whisper_set_encoder_output_stream(m, 0, enc, n_audio_ctx);
}

extern "C" grx_status grx_whisper_set_encoder_output_stream(grx_whisper *m, int stream_ix, const float *enc,
                                                            int n_audio_ctx) {
    if (!m || !enc) return grx_fail(GRX_EINVAL, "grx_whisper_set_encoder_output: NULL argument");
    if (stream_ix < 0 || stream_ix >= m->S)
        return grx_fail(GRX_EINVAL, "grx_whisper_set_encoder_output: stream %d of %d", stream_ix, m->S);
    if (n_audio_ctx != m->hp.n_audio_ctx)
        return grx_fail(GRX_ESIZE, "grx_whisper_set_encoder_output: %d positions, the model has %d", n_audio_ctx,
                        m->hp.n_audio_ctx);
    grx_status s = finalize(m);
    if (s != GRX_OK) return s;
    const int st = m->hp.n_state, nctx = n_audio_ctx, hd = st / m->hp.n_head;
    const size_t n = (size_t)nctx * st;
    // staging for every later window too; each buffer on its own, so that
    // a call that failed half-way allocates only what is still missing
    for (float **b : {&m->xenc, &m->xk_tmp, &m->xv_tmp})
        if (*b == nullptr && (s = dev_alloc_t(m, n, b)) != GRX_OK) return s;
    float *denc = m->xenc, *dk = m->xk_tmp, *dv = m->xv_tmp;
    hipStream_t stream = m->ctx->stream;
    GRX_HIP(hipMemcpyAsync(denc, enc, n * 4, hipMemcpyHostToDevice, stream));
    const float tsc = (float)(1.0 / sqrt((double)hd));
    for (int li = 0; li < m->hp.n_layer && s == GRX_OK; ++li) {
        WLayer &L = m->L[li];
        s = grx_matmul_q8_dev(m->ctx, dk, st, denc, st, nctx, L.xk, nullptr);
        if (s == GRX_OK) s = grx_matmul_q8_dev(m->ctx, dv, st, denc, st, nctx, L.xv, L.xv_b);
        if (s == GRX_OK) {
            cross_layout_kernel<<<(int)((n + 255) / 256), 256, 0, stream>>>(dk, dv, nctx, st, hd, tsc,
                                                                           L.cross_k + stream_ix * n,
                                                                           L.cross_v + stream_ix * n);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) s = grx_hip_fail(e, "cross_layout_kernel");
        }
    }
    hipError_t e = hipStreamSynchronize(stream);
    if (s != GRX_OK) return s;
    if (e != hipSuccess) return grx_hip_fail(e, "grx_whisper_set_encoder_output");
    m->have_xs[stream_ix] = true;
    m->have_cross = std::all_of(m->have_xs.begin(), m->have_xs.end(), [](bool b) { return b; });
    return GRX_OK;
}

extern "C" grx_status grx_whisper_reset(grx_whisper *m) {
    if (!m) return grx_fail(GRX_EINVAL, "grx_whisper_reset: NULL model");
    if (m->ready) GRX_HIP(hipMemsetAsync(m->pos, 0, 4, m->ctx->stream));
    m->pos_host = 0;
    return GRX_OK;
}

extern "C" int grx_whisper_pos(const grx_whisper *m) { return m ? m->pos_host : 0; }

static grx_status check_ready(grx_whisper *m, const char *fn) {
    if (!m) return grx_fail(GRX_EINVAL, "%s: NULL model", fn);
    grx_status s = finalize(m);
    if (s != GRX_OK) return s;
    if (!m->have_cross) return grx_fail(GRX_ESTATE, "%s: no encoder output set", fn);
    return GRX_OK;
}

extern "C" grx_status grx_whisper_sample(grx_whisper *m, int stream, const grx_whisper_rules *rules,
                                         const grx_whisper_seq *seq, float temp, float r, grx_whisper_token *out) {
    if (!m) return grx_fail(GRX_EINVAL, "grx_whisper_sample: NULL model");
    if (stream < 0 || stream >= m->S) return grx_fail(GRX_EINVAL, "grx_whisper_sample: stream %d of %d", stream, m->S);
    if (!m->logits) return grx_fail(GRX_ESTATE, "grx_whisper_sample: nothing decoded yet");
    return grx_sample_run(m->ctx, m->logits + (size_t)stream * m->hp.n_vocab, nullptr, m->hp.n_vocab, rules, seq,
                          temp, r, out);
}

extern "C" grx_status grx_whisper_decode(grx_whisper *m, const int32_t *tokens, int n, float *logits, int32_t *next) {
    grx_status s = check_ready(m, "grx_whisper_decode");
    if (s != GRX_OK) return s;
    if (m->S != 1) return grx_fail(GRX_ESTATE, "grx_whisper_decode: %d streams: use grx_whisper_greedy_streams", m->S);
    if (n < 0 || (n > 0 && !tokens)) return grx_fail(GRX_EINVAL, "grx_whisper_decode: bad tokens");
    if (m->pos_host + n > m->hp.n_text_ctx)
        return grx_fail(GRX_ESTATE, "grx_whisper_decode: %d tokens after %d positions exceed the context of %d", n,
                        m->pos_host, m->hp.n_text_ctx);
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= m->hp.n_vocab)
            return grx_fail(GRX_EINVAL, "grx_whisper_decode: token %d out of the vocabulary", tokens[i]);
    hipStream_t stream = m->ctx->stream;
    for (int i = 0; i < n; ++i) {
        GRX_HIP(hipMemcpyAsync(m->tok, tokens + i, 4, hipMemcpyHostToDevice, stream));
        if ((s = run_step(m)) != GRX_OK) return s;
        m->pos_host++;
    }
    if (n > 0 && logits)
        GRX_HIP(hipMemcpyAsync(logits, m->logits, (size_t)m->hp.n_vocab * 4, hipMemcpyDeviceToHost, stream));
    if (n > 0 && next) GRX_HIP(hipMemcpyAsync(next, m->tok, 4, hipMemcpyDeviceToHost, stream));
    GRX_HIP(hipStreamSynchronize(stream));
    return GRX_OK;
}

extern "C" grx_status grx_whisper_greedy(grx_whisper *m, const int32_t *prompt, int n_prompt, int n_steps,
                                         int32_t *out) {
    grx_status s = check_ready(m, "grx_whisper_greedy");
    if (s != GRX_OK) return s;
    if (m->S != 1) return grx_fail(GRX_ESTATE, "grx_whisper_greedy: %d streams: use grx_whisper_greedy_streams", m->S);
    if (n_prompt <= 0 || n_steps < 0 || !prompt || !out)
        return grx_fail(GRX_EINVAL, "grx_whisper_greedy: bad arguments");
    if (n_prompt + n_steps > m->hp.n_text_ctx)
        return grx_fail(GRX_ESTATE, "grx_whisper_greedy: %d prompt tokens and %d steps exceed the context of %d",
                        n_prompt, n_steps, m->hp.n_text_ctx);
    if ((s = grx_whisper_reset(m)) != GRX_OK) return s;
    if ((s = grx_whisper_decode(m, prompt, n_prompt, nullptr, nullptr)) != GRX_OK) return s;
    hipStream_t stream = m->ctx->stream;
    for (int i = 0; i < n_steps; ++i) {
        if ((s = run_step(m)) != GRX_OK) return s;
        m->pos_host++;
    }
    GRX_HIP(hipMemcpyAsync(out, m->hist + (n_prompt - 1), (size_t)(n_steps + 1) * 4, hipMemcpyDeviceToHost, stream));
    GRX_HIP(hipStreamSynchronize(stream));
    return GRX_OK;
}

extern "C" grx_status grx_whisper_greedy_streams(grx_whisper *m, const int32_t *prompts, int n_prompt, int n_steps,
                                                 int32_t *out) {
    grx_status s = check_ready(m, "grx_whisper_greedy_streams");
    if (s != GRX_OK) return s;
    const int S = m->S;
    if (n_prompt <= 0 || n_steps < 0 || !prompts || !out)
        return grx_fail(GRX_EINVAL, "grx_whisper_greedy_streams: bad arguments");
    if (n_prompt + n_steps > m->hp.n_text_ctx)
        return grx_fail(GRX_ESTATE, "grx_whisper_greedy_streams: %d prompt tokens and %d steps exceed the context of %d",
                        n_prompt, n_steps, m->hp.n_text_ctx);
    for (int i = 0; i < S * n_prompt; ++i)
        if (prompts[i] < 0 || prompts[i] >= m->hp.n_vocab)
            return grx_fail(GRX_EINVAL, "grx_whisper_greedy_streams: token %d out of the vocabulary", prompts[i]);
    if ((s = grx_whisper_reset(m)) != GRX_OK) return s;
    hipStream_t stream = m->ctx->stream;
    // the prompt position by position, every stream's token uploaded first
    std::vector<int32_t> col(S);
    for (int i = 0; i < n_prompt; ++i) {
        for (int k = 0; k < S; ++k) col[k] = prompts[(size_t)k * n_prompt + i];
        GRX_HIP(hipMemcpyAsync(m->tok, col.data(), (size_t)S * 4, hipMemcpyHostToDevice, stream));
        if ((s = run_step(m)) != GRX_OK) return s;
        m->pos_host++;
        GRX_HIP(hipStreamSynchronize(stream));  // col is reused
    }
    for (int i = 0; i < n_steps; ++i) {
        if ((s = run_step(m)) != GRX_OK) return s;
        m->pos_host++;
    }
    for (int k = 0; k < S; ++k)
        GRX_HIP(hipMemcpyAsync(out + (size_t)k * (n_steps + 1), m->hist + (size_t)k * m->hp.n_text_ctx + (n_prompt - 1),
                               (size_t)(n_steps + 1) * 4, hipMemcpyDeviceToHost, stream));
    GRX_HIP(hipStreamSynchronize(stream));
    return GRX_OK;
}

// kvCache.copyFrom (whisper/decoder.go:22-28) between the streams of one
// decoder: stream dst's self-attention keys and values take stream src's
// rows for the positions filled so far, its next token and its token record
// src's.  Cross keys and values stay (grx_whisper_share_encoder_output).
extern "C" grx_status grx_whisper_stream_copy(grx_whisper *m, int dst, int src) {
    if (!m) return grx_fail(GRX_EINVAL, "grx_whisper_stream_copy: NULL model");
    if (dst < 0 || dst >= m->S || src < 0 || src >= m->S)
        return grx_fail(GRX_EINVAL, "grx_whisper_stream_copy: streams %d, %d of %d", dst, src, m->S);
    grx_status s = finalize(m);
    if (s != GRX_OK) return s;
    if (dst == src) return GRX_OK;
    const grx_whisper_hparams &hp = m->hp;
    const size_t kv_stream = (size_t)hp.n_text_ctx * hp.n_state, rows = (size_t)m->pos_host * hp.n_state * 4;
    hipStream_t stream = m->ctx->stream;
    GRX_HIP(hipSetDevice(m->ctx->device));
    for (int li = 0; li < hp.n_layer && rows > 0; ++li) {
        WLayer &L = m->L[li];
        GRX_HIP(hipMemcpyAsync(L.self_k + dst * kv_stream, L.self_k + src * kv_stream, rows, hipMemcpyDeviceToDevice,
                               stream));
        GRX_HIP(hipMemcpyAsync(L.self_v + dst * kv_stream, L.self_v + src * kv_stream, rows, hipMemcpyDeviceToDevice,
                               stream));
    }
    GRX_HIP(hipMemcpyAsync(m->tok + dst, m->tok + src, 4, hipMemcpyDeviceToDevice, stream));
    GRX_HIP(hipMemcpyAsync(m->hist + (size_t)dst * hp.n_text_ctx, m->hist + (size_t)src * hp.n_text_ctx,
                           (size_t)hp.n_text_ctx * 4, hipMemcpyDeviceToDevice, stream));
    GRX_HIP(hipStreamSynchronize(stream));
    return GRX_OK;
}

// Stream dst takes stream src's cross-attention keys and values: streams
// decoding one window (transcribe.go:170-204, bestOf sequences) share its
// encoder output without a second projection (a device copy).
extern "C" grx_status grx_whisper_share_encoder_output(grx_whisper *m, int dst, int src) {
    if (!m) return grx_fail(GRX_EINVAL, "grx_whisper_share_encoder_output: NULL model");
    if (dst < 0 || dst >= m->S || src < 0 || src >= m->S)
        return grx_fail(GRX_EINVAL, "grx_whisper_share_encoder_output: streams %d, %d of %d", dst, src, m->S);
    if (!m->ready || !m->have_xs[src])
        return grx_fail(GRX_ESTATE, "grx_whisper_share_encoder_output: stream %d has no encoder output", src);
    if (dst == src) return GRX_OK;
    const grx_whisper_hparams &hp = m->hp;
    const size_t n = (size_t)hp.n_audio_ctx * hp.n_state;
    hipStream_t stream = m->ctx->stream;
    GRX_HIP(hipSetDevice(m->ctx->device));
    for (int li = 0; li < hp.n_layer; ++li) {
        WLayer &L = m->L[li];
        GRX_HIP(hipMemcpyAsync(L.cross_k + dst * n, L.cross_k + src * n, n * 4, hipMemcpyDeviceToDevice, stream));
        GRX_HIP(hipMemcpyAsync(L.cross_v + dst * n, L.cross_v + src * n, n * 4, hipMemcpyDeviceToDevice, stream));
    }
    GRX_HIP(hipStreamSynchronize(stream));
    m->have_xs[dst] = true;
    m->have_cross = std::all_of(m->have_xs.begin(), m->have_xs.end(), [](bool b) { return b; });
    return GRX_OK;
}

// n_steps greedy steps of every stream from the current position, each
// stream fed the token its last step chose (the loop of transcribe.go:
// 207-260 with plain argmax, continued); out [n_streams][n_steps] receives
// the tokens chosen.
extern "C" grx_status grx_whisper_steps(grx_whisper *m, int n_steps, int32_t *out) {
    grx_status s = check_ready(m, "grx_whisper_steps");
    if (s != GRX_OK) return s;
    if (n_steps < 0 || (n_steps > 0 && !out)) return grx_fail(GRX_EINVAL, "grx_whisper_steps: bad arguments");
    if (n_steps > 0 && m->pos_host == 0)
        return grx_fail(GRX_ESTATE, "grx_whisper_steps: nothing decoded yet (no token to feed)");
    if (m->pos_host + n_steps > m->hp.n_text_ctx)
        return grx_fail(GRX_ESTATE, "grx_whisper_steps: %d steps after %d positions exceed the context of %d", n_steps,
                        m->pos_host, m->hp.n_text_ctx);
    const int p0 = m->pos_host;
    for (int i = 0; i < n_steps; ++i) {
        if ((s = run_step(m)) != GRX_OK) return s;
        m->pos_host++;
    }
    hipStream_t stream = m->ctx->stream;
    for (int k = 0; k < m->S && n_steps > 0; ++k)
        GRX_HIP(hipMemcpyAsync(out + (size_t)k * n_steps, m->hist + (size_t)k * m->hp.n_text_ctx + p0,
                               (size_t)n_steps * 4, hipMemcpyDeviceToHost, stream));
    GRX_HIP(hipStreamSynchronize(stream));
    return GRX_OK;
}

// The logits of stream `stream`'s last step (n_vocab floats) into host memory.
extern "C" grx_status grx_whisper_logits(grx_whisper *m, int stream_ix, float *out) {
    if (!m || !out) return grx_fail(GRX_EINVAL, "grx_whisper_logits: NULL argument");
    if (stream_ix < 0 || stream_ix >= m->S)
        return grx_fail(GRX_EINVAL, "grx_whisper_logits: stream %d of %d", stream_ix, m->S);
    if (!m->logits || m->pos_host == 0) return grx_fail(GRX_ESTATE, "grx_whisper_logits: nothing decoded yet");
    GRX_HIP(hipSetDevice(m->ctx->device));
    GRX_HIP(hipMemcpyAsync(out, m->logits + (size_t)stream_ix * m->hp.n_vocab, (size_t)m->hp.n_vocab * 4,
                           hipMemcpyDeviceToHost, m->ctx->stream));
    GRX_HIP(hipStreamSynchronize(m->ctx->stream));
    return GRX_OK;
}

// The loop of one window (whisper/transcribe.go:207-260) for one sequence,
// on the device: after the prompt (decoded by the caller: its logits are
// the last step's), each iteration runs process + sample (transcribe.go:
// 370-494) on the last logits with the sequence state held in device
// memory, applies the loop's timestamp, end and stuck rules (transcribe.go:
// 211-237), and feeds the token to the next decode step.  The host enqueues
// sixteen iterations at a time and reads the state back between them, so
// the only round trips are those checks; a sequence that is done or failed
// makes the later samplers of its batch return at once (their decode steps
// run on unused tokens, and the position moves past them).
extern "C" grx_status grx_whisper_rules_loop(grx_whisper *m, const grx_whisper_rules *rules,
                                             const grx_whisper_loop *lp, grx_whisper_token *out,
                                             grx_whisper_loop_result *res) {
    grx_status s = check_ready(m, "grx_whisper_rules_loop");
    if (s != GRX_OK) return s;
    if (!rules || !lp || !out || !res) return grx_fail(GRX_EINVAL, "grx_whisper_rules_loop: NULL argument");
    if (m->S != 1) return grx_fail(GRX_ESTATE, "grx_whisper_rules_loop: %d streams (one sequence only)", m->S);
    if (m->pos_host == 0) return grx_fail(GRX_ESTATE, "grx_whisper_rules_loop: no prompt decoded");
    if (lp->n_max < 0 || m->pos_host + lp->n_max > m->hp.n_text_ctx)
        return grx_fail(GRX_ESTATE, "grx_whisper_rules_loop: %d iterations after %d positions exceed the context of %d",
                        lp->n_max, m->pos_host, m->hp.n_text_ctx);
    if (lp->temp > 0.f && lp->n_max > 0 && !lp->r)
        return grx_fail(GRX_EINVAL, "grx_whisper_rules_loop: a temperature above 0 needs n_max draws");
    const grx_whisper_seq none{};
    GrxSampleArgs a;
    if ((s = grx_sample_args(rules, &none, m->hp.n_vocab, lp->temp, 0.f, &a)) != GRX_OK) return s;
    const int ctxn = m->hp.n_text_ctx;
    if (!m->samp_g && (s = dev_alloc_t(m, (size_t)2 * 65536, &m->samp_g)) != GRX_OK) return s;
    if (!m->loop_st && (s = dev_alloc_t(m, 1, &m->loop_st)) != GRX_OK) return s;
    if (!m->loop_rec && (s = dev_alloc_t(m, (size_t)ctxn, &m->loop_rec)) != GRX_OK) return s;
    if (!m->loop_rs && (s = dev_alloc_t(m, (size_t)ctxn, &m->loop_rs)) != GRX_OK) return s;
    if (rules->n_suppress > m->samp_sup_cap) {
        if ((s = dev_alloc_t(m, (size_t)rules->n_suppress, &m->samp_sup)) != GRX_OK) return s;
        m->samp_sup_cap = rules->n_suppress;
    }
    hipStream_t stream = m->ctx->stream;
    GRX_HIP(hipSetDevice(m->ctx->device));
    if (rules->n_suppress > 0)
        GRX_HIP(hipMemcpyAsync(m->samp_sup, rules->suppress, (size_t)rules->n_suppress * 4, hipMemcpyHostToDevice,
                               stream));
    GrxLoopDev st0{};
    st0.seek_delta = lp->win_frames;  // a fresh seq (transcribe.go:201)
    GRX_HIP(hipMemcpyAsync(m->loop_st, &st0, sizeof st0, hipMemcpyHostToDevice, stream));
    if (lp->temp > 0.f && lp->n_max > 0)
        GRX_HIP(hipMemcpyAsync(m->loop_rs, lp->r, (size_t)lp->n_max * 4, hipMemcpyHostToDevice, stream));
    GrxLoopArgs la;
    la.st = m->loop_st;
    la.tok_w = m->tok;
    la.rec = m->loop_rec;
    la.rs = lp->temp > 0.f ? m->loop_rs : nullptr;
    la.seek = lp->seek;
    la.seek_end = lp->seek_end;
    la.delta_min = lp->delta_min;
    la.win_frames = lp->win_frames;
    la.n_max = lp->n_max;
    GrxLoopDev st{};
    GRX_HIP(hipStreamSynchronize(stream));  // st0 and the draws are read from host memory
    for (int it = 0; it < lp->n_max;) {
        const int chunk = std::min(16, lp->n_max - it);
        for (int k = 0; k < chunk; ++k) {
            if ((s = grx_sample_launch(stream, m->logits, a, m->samp_sup, m->samp_g, nullptr, la)) != GRX_OK) return s;
            if ((s = run_step(m)) != GRX_OK) return s;
            m->pos_host++;
        }
        it += chunk;
        GRX_HIP(hipMemcpyAsync(&st, m->loop_st, sizeof st, hipMemcpyDeviceToHost, stream));
        GRX_HIP(hipStreamSynchronize(stream));
        if (st.done || st.failed) break;
    }
    if (lp->n_max == 0) st = st0;
    if (st.i > 0) GRX_HIP(hipMemcpy(out, m->loop_rec, (size_t)st.i * sizeof(grx_whisper_token), hipMemcpyDeviceToHost));
    res->n_tokens = st.i;
    res->done = st.done;
    res->failed = st.failed;
    res->result_len = st.result_len;
    res->seek_delta = st.seek_delta;
    res->has_ts = st.has_ts;
    return GRX_OK;
}
