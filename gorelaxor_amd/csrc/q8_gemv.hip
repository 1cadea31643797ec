// q8_gemv.hip - the Q8_0 int8 product for few activation rows (m <= 8 per
// launch): the decode-time GEMV and the skinny GEMM of batched streams.
//
// Restates the int8 route of kern.MatMul (internal/kern/kern.go:185-196 ->
// matmulQ8Int, q8int.go:148-223 of github.com/xattribution/gorelaxor) with
// the per-output arithmetic of the VNNI tile kernel (vnni_amd64.s:58-69):
//     c = bias (or 0);  for b in 0..nb-1:  c = fma(f32(s_b) * dw_b, da_b, c)
// where s_b is the int32 dot of block b's rounded activations and weights.
//
// MI355X design: a workgroup owns one tile of 64 weight rows; lane l of
// every wave owns row 64*tile+l.  The tile's blocks are split among W waves
// (W = 1 for tall matrices, more for short ones so that a 512-row matrix
// still spreads over many CUs).  Per block a lane issues two 16-byte loads
// (one 1 KiB coalesced transaction per wave each) plus one 2-byte scale load,
// eight v_dot4_i32_i8 against the activation block, one convert and one
// multiply.  With W = 1 the lane also runs the ordered fma chain as it goes;
// with W > 1 the products f32(s_b)*dw_b go to LDS and wave 0 runs the chain
// in block order afterwards, so the result is the same bit for bit.
// One-row products of short weights run on slices of the tiles instead
// (q8_gemv1n.hip).
#include <mutex>

#include "q8_gemv_impl.h"

namespace {

// ---------------------------------------------------------------- kernel

// The arguments of this workgroup's group of M rows (blockIdx.z) when one
// launch runs several (GemvArgs::chunks).
template <int M>
__device__ __forceinline__ GemvArgs chunk_args(const GemvArgs &a0) {
    GemvArgs a = a0;
    const int g = blockIdx.z;
    if (g > 0) {
        const size_t r = (size_t)g * M, K = (size_t)a.nb * GRX_QK;
        if (a.x) a.x += r * a.lda;
        if (a.xq) a.xq += r * K;
        if (a.xs) a.xs += r * a.nb;
        if (a.y) a.y += r * a.ldc;
        if (a.resid) a.resid += r * a.ldr;
        if (a.yq) a.yq += r * a.rows;
        if (a.ys) a.ys += r * (a.rows >> 5);
        a.pos_add += (int)r;
    }
    return a;
}

template <int M, int W, int PRO, int EPI>
__global__ __launch_bounds__(64 * W) void gemv_q8_kernel(const GemvArgs a0) {
    const GemvArgs a = chunk_args<M>(a0);
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: loops stay scalar
    const int tile = blockIdx.x;
    const int nb = a.nb, K = nb * GRX_QK;
    const int row = tile * 64 + lane;
    const int pos0 = (EPI == GRX_EPI_QKV || EPI == GRX_EPI_QKV_ROPE) ? *a.pos : 0;

    // LDS, each region 16-byte aligned (gemv_smem):
    //   [lxq M*K int8][lxs M*nb f32][lp M*(nb or kRound)*64 f32 if W>1, and
    //   in the same bytes lf M*K f32 if LN: lf is done with before lp is
    //   written][red]
    // activations in LDS: rounded here, or (several rows, up to kStageMax
    // bytes of them) copied from HBM; several pre-rounded rows keep their
    // scales in LDS either way
    // compile-time, so the activation reads are LDS reads, not flat ones
    // (the host keeps M * K within kStageMax for pre-rounded rows)
    constexpr bool LQ = PRO != GRX_PRO_PREQ || M > 1;
    constexpr bool LS = PRO != GRX_PRO_PREQ || M > 1;
    const size_t o_xs = LQ ? (size_t)M * K : 0;
    const size_t o_p = o_xs + (LS ? (((size_t)M * nb * 4 + 15) & ~(size_t)15) : 0);
    constexpr bool RND = M > 1 && W > 1;
    const size_t n_p = W > 1 ? (size_t)M * (RND ? kRound : nb) * 64 * 4 : 0;
    const size_t n_f = PRO >= GRX_PRO_LN ? (size_t)M * K * 4 : 0;
    const size_t o_f = o_p;
    const size_t o_r = o_p + (n_p > n_f ? n_p : n_f);
    int8_t *lxq = reinterpret_cast<int8_t *>(smem);
    float *lxs = reinterpret_cast<float *>(smem + o_xs);
    float *lp = reinterpret_cast<float *>(smem + o_p);
    float *lf = reinterpret_cast<float *>(smem + o_f);
    double *red = reinterpret_cast<double *>(smem + o_r);

    // ---- prologue: the activation rows, rounded, in LDS (or left in HBM)
    if constexpr (PRO == GRX_PRO_PREQ && M > 1) {
        // several pre-rounded rows: copied to LDS once (16-byte pieces), so
        // the blocks' dots and the folds read LDS instead of HBM
        if (LQ) {
            const int n16 = M * K / 16;
            for (int i = tid; i < n16; i += 64 * W)
                reinterpret_cast<int4 *>(lxq)[i] = reinterpret_cast<const int4 *>(a.xq)[i];
        }
        for (int i = tid; i < M * nb; i += 64 * W) lxs[i] = a.xs[i];
        __syncthreads();
    }
    // several rows of up to 1280 values and a wave for each: wave m builds
    // row m with the one-wave prologue (no workgroup reductions)
    constexpr bool WROW = PRO != GRX_PRO_PREQ && M > 1 && W >= M;
    const bool wrow = WROW && K <= kRowPieces * 256;
    if (wrow) {
        if constexpr (WROW) {
            if (wave < M) wave_row_prologue<kRowPieces, PRO>(a, wave, lxq, lxs, lane, tile, [] {});
            __syncthreads();
        }
    } else if constexpr (PRO == GRX_PRO_QUANT) {
        quant_into_lds<M>(a.x, a.lda, nb, lxq, lxs, tid, 64 * W);
        __syncthreads();
    } else if constexpr (PRO == GRX_PRO_LN || PRO == GRX_PRO_EMBED_LN) {
        // layerNorm (internal/kern/mathx.go:55-75) of each row, then quantU8.
        for (int m = 0; m < M; ++m) {
            const float *xr = a.x + (size_t)m * a.lda;
            float *fr = lf + (size_t)m * K;
            if constexpr (PRO == GRX_PRO_EMBED_LN) {
                // the row is tokEmb.row(tok) + decPos[pos] (whisper/decoder.go:42-46),
                // built by every workgroup; tile 0 stores it for the residual
                const int t = a.tok[m], p = *a.pos + a.pos_add + (a.streams ? 0 : m);
                const int etile = t >> 6, elane = t & 63;
                for (int i = tid; i < K; i += 64 * W) {
                    const int b = i >> 5, h = (i >> 4) & 1, e = i & 15;
                    const int8_t q = a.emb_qs[(((size_t)etile * nb + b) * 2 + h) * 1024 + elane * 16 + e];
                    const float d = grx_f16_to_f32(a.emb_ds[((size_t)etile * nb + b) * 64 + elane]);
                    const float v = __fadd_rn(__fmul_rn((float)q, d), a.pos_emb[(size_t)p * K + i]);
                    fr[i] = v;
                    if (tile == 0) a.x_out[(size_t)m * a.lda + i] = v;
                }
            } else {
                for (int i = tid; i < K; i += 64 * W) fr[i] = xr[i];
            }
            __syncthreads();  // the row, built by every thread, is read by all of them
            float mean, inv;
            ln32_stats(fr, K, red, mean, inv);
            for (int i = tid; i < K; i += 64 * W) {
                float t = __fsub_rn(fr[i], mean);
                t = __fmul_rn(t, inv);
                t = __fmul_rn(t, a.ln_w[i]);
                fr[i] = __fadd_rn(t, a.ln_b[i]);
            }
        }
        __syncthreads();
        quant_into_lds<M>(lf, K, nb, lxq, lxs, tid, 64 * W);
        __syncthreads();
    } else if constexpr (PRO == GRX_PRO_LN64) {
        // layerNorm of pockettts/nn.go:27-49: statistics and the normalized
        // value in float64, the gain and bias (when given) in float32.
        for (int m = 0; m < M; ++m) {
            const float *xr = a.x + (size_t)m * a.lda;
            float *fr = lf + (size_t)m * K;
            for (int i = tid; i < K; i += 64 * W) fr[i] = xr[i];
            __syncthreads();
            double mean, inv;
            ln64_stats(fr, K, a.ln_eps, red, mean, inv);
            for (int i = tid; i < K; i += 64 * W) {
                float o = (float)(((double)fr[i] - mean) * inv);
                if (a.ln_w != nullptr) o = __fadd_rn(__fmul_rn(o, a.ln_w[i]), a.ln_b[i]);
                fr[i] = o;
            }
        }
        __syncthreads();
        quant_into_lds<M>(lf, K, nb, lxq, lxs, tid, 64 * W);
        __syncthreads();
    }

    auto act = [&](int m, int b, int4 &a0, int4 &a1) {
        const int4 *p;
        if (!LQ)
            p = reinterpret_cast<const int4 *>(a.xq + (size_t)m * K + b * GRX_QK);
        else
            p = reinterpret_cast<const int4 *>(lxq + (size_t)m * K + b * GRX_QK);
        a0 = p[0];
        a1 = p[1];
    };
    auto act_scale = [&](int m, int b) -> float {
        if constexpr (!LS)
            return a.xs[(size_t)m * nb + b];
        else
            return lxs[m * nb + b];
    };

    // ---- main loop: this wave's run of blocks
    const int b0 = (wave * nb) / W, b1 = ((wave + 1) * nb) / W;
    const int4 *__restrict__ wq = reinterpret_cast<const int4 *>(a.qs) + (size_t)tile * nb * 128;
    const uint16_t *__restrict__ wd = a.ds + (size_t)tile * nb * 64;

    float acc[M];
    if constexpr (W == 1) {
        const float bv = (a.bias != nullptr && row < a.rows) ? a.bias[row] : 0.0f;
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] = bv;
    }

    // U blocks: all loads issued first, then the dots in block order.
    // Partial products go to lp at block b - rb (rows ld apart).
    auto run = [&](auto u_tag, int bb, int rb, int ldp) {
        constexpr int U = decltype(u_tag)::value;
        int4 w[2 * U];
        uint32_t dh[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (a.cacheable) {
                w[2 * u] = wq[(size_t)(bb + u) * 128 + lane];
                w[2 * u + 1] = wq[(size_t)(bb + u) * 128 + 64 + lane];
                dh[u] = wd[(size_t)(bb + u) * 64 + lane];
            } else {
                w[2 * u] = wload(wq + (size_t)(bb + u) * 128 + lane);
                w[2 * u + 1] = wload(wq + (size_t)(bb + u) * 128 + 64 + lane);
                dh[u] = wload(wd + (size_t)(bb + u) * 64 + lane);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int b = bb + u;
            const float dw = grx_f16_to_f32((uint16_t)dh[u]);
#pragma unroll
            for (int m = 0; m < M; ++m) {
                int4 a0, a1;
                act(m, b, a0, a1);
                const int s = sdot8(w[2 * u], w[2 * u + 1], a0, a1);
                const float pv = __fmul_rn((float)s, dw);
                if constexpr (W == 1)
                    acc[m] = __fmaf_rn(pv, act_scale(m, b), acc[m]);
                else
                    lp[((size_t)m * ldp + (b - rb)) * 64 + lane] = pv;
            }
        }
    };
    if constexpr (RND) {
        // rounds of kRound blocks, kRound / W per wave; wave w folds the rows
        // m = w, w + W, ... over the round in block order.  The next round's
        // weights are loaded before this round's products and fold.
        constexpr int BR = kRound / W > 0 ? kRound / W : 1;
        constexpr int R = BR * W;
        const float bv = (a.bias != nullptr && row < a.rows) ? a.bias[row] : 0.0f;
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] = bv;
        int4 wa[2 * BR], wb[2 * BR];
        uint32_t da[BR], db[BR];
        // this wave's blocks of the round at r0 (past nb: the last block again)
        auto ld = [&](int4 *w, uint32_t *dh, int r0) {
#pragma unroll
            for (int u = 0; u < BR; ++u) {
                const int b = min(r0 + wave * BR + u, nb - 1);
                if (a.cacheable) {
                    w[2 * u] = wq[(size_t)b * 128 + lane];
                    w[2 * u + 1] = wq[(size_t)b * 128 + 64 + lane];
                    dh[u] = wd[(size_t)b * 64 + lane];
                } else {
                    w[2 * u] = wload(wq + (size_t)b * 128 + lane);
                    w[2 * u + 1] = wload(wq + (size_t)b * 128 + 64 + lane);
                    dh[u] = wload(wd + (size_t)b * 64 + lane);
                }
            }
        };
        auto round = [&](const int4 *w, const uint32_t *dh, int r0) {
#pragma unroll
            for (int u = 0; u < BR; ++u) {
                const int b = r0 + wave * BR + u;
                if (b < nb) {  // uniform
                    const float dw = grx_f16_to_f32((uint16_t)dh[u]);
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        int4 a0, a1;
                        act(m, b, a0, a1);
                        const int sd = sdot8(w[2 * u], w[2 * u + 1], a0, a1);
                        lp[((size_t)m * R + (b - r0)) * 64 + lane] = __fmul_rn((float)sd, dw);
                    }
                }
            }
            __syncthreads();
            const int re = min(r0 + R, nb);
#pragma unroll
            for (int m = 0; m < M; ++m) {
                if (m % W != wave) continue;  // uniform across the wave
                if (re - r0 == R) {
                    float t[R], sc[R];
#pragma unroll
                    for (int k = 0; k < R; ++k) {
                        t[k] = lp[((size_t)m * R + k) * 64 + lane];
                        sc[k] = act_scale(m, r0 + k);
                    }
#pragma unroll
                    for (int k = 0; k < R; ++k) acc[m] = __fmaf_rn(t[k], sc[k], acc[m]);
                } else {
                    for (int b = r0; b < re; ++b)
                        acc[m] = __fmaf_rn(lp[((size_t)m * R + (b - r0)) * 64 + lane], act_scale(m, b), acc[m]);
                }
            }
            __syncthreads();
        };
        // loads are issued unconditionally (past nb they repeat the last
        // block): the number in flight is then fixed, so waiting for one
        // round's weights never waits for the next round's
        ld(wa, da, 0);
        for (int r0 = 0; r0 < nb; r0 += 2 * R) {
            ld(wb, db, r0 + R);
            round(wa, da, r0);
            if (r0 + R >= nb) break;
            ld(wa, da, r0 + 2 * R);
            round(wb, db, r0 + R);
        }
    } else {
        int bb = b0;
        for (; bb + BU <= b1; bb += BU) run(std::integral_constant<int, BU>{}, bb, 0, nb);
        for (; bb < b1; ++bb) run(std::integral_constant<int, 1>{}, bb, 0, nb);
    }

    if constexpr (W > 1 && !RND) {
        __syncthreads();
        if (wave != 0) return;
        const float bv = (a.bias != nullptr && row < a.rows) ? a.bias[row] : 0.0f;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float c = bv;
            for (int b = 0; b < nb; ++b) c = __fmaf_rn(lp[((size_t)m * nb + b) * 64 + lane], act_scale(m, b), c);
            acc[m] = c;
        }
    }

    // ---- epilogue: row m is ended by wave 0 (one wave, or after the fold
    // above), or by wave m % W when rows were folded round by round
    gemv_epilogue<M, W, RND, EPI>(a, acc, row, lane, wave, pos0);
}

// Several activation rows (M = 2..8: a batch of streams, a short prompt) on
// the matrix cores, with the multi-row GEMV's prologues and epilogues.  A
// workgroup owns 16*NS weight rows (a quarter or half of a 64-row tile, so a
// 1280-row product runs on 80 workgroups instead of 20) and its W waves
// split the blocks, KB each: wave m builds activation row m with the
// one-wave prologue, its weights' loads issued behind the row's (rounded
// rows in LDS, 16 bytes apart beyond K so the fragment reads of 16 rows fall
// in different banks), takes its blocks' int32 dots with
// v_mfma_i32_16x16x32_i8
// (weights as A, activation rows as B: a lane holds four consecutive weight
// rows of one activation row) and forms t = f32(s) * dw; the ordered chain
// c = fma(t, da, c) from the bias then runs wave after wave through LDS, so
// every output sees the blocks in order, as in gemv_q8_kernel.  The last
// wave hands its outputs, through LDS, to the lanes of their rows and ends
// them with gemv_epilogue.
template <int M, int PRO, int EPI, int NS, int KB>
__global__ __launch_bounds__(512) void gemv_q8_mx_kernel(const GemvArgs a0) {
    const GemvArgs a = chunk_args<M>(a0);
    static_assert(M >= 2 && M <= 8, "2 to 8 activation rows");
    static_assert(KB % 4 == 0, "blocks per wave in whole groups of four");
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = a.nb, K = nb * GRX_QK, ldq = K + 16;
    const int WK = (nb + KB - 1) / KB;  // waves with blocks (the workgroup has max(WK, M))
    // LDS: lxq [M][ldq] int8 | lxs [M][nb] f32 | cx [2][NS*4][64] f32 | ot [M][16*NS] f32
    int8_t *lxq = reinterpret_cast<int8_t *>(smem);
    float *lxs = reinterpret_cast<float *>(smem + (((size_t)M * ldq + 15) & ~(size_t)15));
    float *cx = lxs + (((size_t)M * nb + 3) & ~(size_t)3);
    float *ot = cx + 2 * NS * 4 * 64;
    const int g = blockIdx.x;
    const int n0 = g * 16 * NS, tile = n0 >> 6, sub = n0 & 63;
    const int pos0 = (EPI == GRX_EPI_QKV || EPI == GRX_EPI_QKV_ROPE) ? *a.pos : 0;
    const int li = lane & 15, lk = lane >> 4;

    // the weights of the wave's blocks, issued behind its activation row's
    // loads (they complete in order: the row does not wait for them)
    const int b0 = wave * KB, nbw = min(KB, nb - b0);
    const int8_t *wq = reinterpret_cast<const int8_t *>(a.qs) + (size_t)tile * nb * 2048;
    const char *wd = reinterpret_cast<const char *>(a.ds + (size_t)tile * nb * 64);
    const unsigned qoff = (unsigned)((lk >> 1) * 1024 + (sub + li) * 16 + 8 * (lk & 1));
    const unsigned doff = (unsigned)(sub + 4 * lk);
    long bv[KB][NS];
    uint2 dq[KB][NS];
    auto load_weights = [&] {
        if (wave >= WK) return;
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const unsigned b = (unsigned)min(b0 + u, nb - 1);
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                bv[u][s] = *reinterpret_cast<const long *>(wq + (qoff + b * 2048 + s * 256));
                dq[u][s] = *reinterpret_cast<const uint2 *>(wd + 2 * (doff + b * 64 + 16 * s));
            }
        }
    };

    // ---- prologue: the M rounded rows in LDS, row m built by wave m
    if constexpr (PRO == GRX_PRO_PREQ) {
        load_weights();
        const int n16 = K / 16;
        for (int i = threadIdx.x; i < M * n16; i += blockDim.x) {
            const int m = i / n16, j = i % n16;
            reinterpret_cast<int4 *>(lxq + (size_t)m * ldq)[j] = reinterpret_cast<const int4 *>(a.xq + (size_t)m * K)[j];
        }
        for (int i = threadIdx.x; i < M * nb; i += blockDim.x) lxs[i] = a.xs[i];
    } else {
        if (wave < M)
            wave_row_prologue<kRowPieces, PRO>(a, wave, lxq, lxs, lane, g, load_weights, ldq);
        else
            load_weights();
    }
    __syncthreads();
    if (wave >= WK) {
        // no blocks: through the chain's barriers only
        for (int p = 0; p + 1 < WK; ++p) __syncthreads();
        return;
    }

    // the block dots (weight rows 4*lk+r of each 16, activation row li) and
    // their scaled forms t = f32(s) * dw; rows past M read row M-1 and are
    // never stored
    const int ar = min(li, M - 1);
    float t[KB][NS][4];
#pragma unroll
    for (int u = 0; u < KB; ++u) {
        const int b = min(b0 + u, nb - 1);
        const long av = *reinterpret_cast<const long *>(lxq + (size_t)ar * ldq + b * GRX_QK + 8 * lk);
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            grx_v4i d = {0, 0, 0, 0};
            d = __builtin_amdgcn_mfma_i32_16x16x32_i8(bv[u][s], av, d, 0, 0, 0);
            const uint32_t h[2] = {dq[u][s].x, dq[u][s].y};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float dw = grx_f16_to_f32((uint16_t)(h[r >> 1] >> (16 * (r & 1))));
                t[u][s][r] = __fmul_rn((float)d[r], dw);
            }
        }
    }

    // the ordered chain, one wave after another
    float c[NS][4];
    for (int p = 0; p < WK; ++p) {
        if (wave == p) {
            if (p == 0) {
#pragma unroll
                for (int s = 0; s < NS; ++s)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int n = n0 + 16 * s + 4 * lk + r;
                        c[s][r] = (a.bias != nullptr && n < a.rows) ? a.bias[n] : 0.0f;
                    }
            } else {
#pragma unroll
                for (int s = 0; s < NS; ++s)
#pragma unroll
                    for (int r = 0; r < 4; ++r) c[s][r] = cx[(((p - 1) & 1) * NS * 4 + 4 * s + r) * 64 + lane];
            }
#pragma unroll
            for (int u = 0; u < KB; ++u) {
                if (u < nbw) {
                    const float da = lxs[ar * nb + b0 + u];
#pragma unroll
                    for (int s = 0; s < NS; ++s)
#pragma unroll
                        for (int r = 0; r < 4; ++r) c[s][r] = __fmaf_rn(t[u][s][r], da, c[s][r]);
                }
            }
            if (p + 1 < WK) {
#pragma unroll
                for (int s = 0; s < NS; ++s)
#pragma unroll
                    for (int r = 0; r < 4; ++r) cx[((p & 1) * NS * 4 + 4 * s + r) * 64 + lane] = c[s][r];
            }
        }
        if (p + 1 < WK) __syncthreads();
    }
    if (wave != WK - 1) return;

    // ---- epilogue: output row n0+lane of activation row m in lane `lane`
    constexpr int NR = 16 * NS;
    if (li < M) {
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r) ot[li * NR + 16 * s + 4 * lk + r] = c[s][r];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = lane < NR ? ot[m * NR + lane] : 0.0f;
    const int row = lane < NR ? n0 + lane : a.rows;
    gemv_epilogue<M, 1, false, EPI>(a, acc, row, lane, 0, pos0);
}

// LDS of gemv_q8_mx_kernel.
size_t gemv_mx_smem(int M, int NS, int nb) {
    const size_t K = (size_t)nb * GRX_QK;
    return ((M * (K + 16) + 15) & ~(size_t)15) + (((size_t)M * nb + 3) & ~(size_t)3) * 4 + 2 * NS * 4 * 64 * 4 +
           (size_t)M * 16 * NS * 4;
}

// The product of ONE activation row (decode steps): q8_gemv's tile scheme
// with the latency of a single row in mind.
//  - every wave issues its first kPrefetch blocks' weight loads (and wave 0
//    the bias and residual) before anything waits;
//  - the activation row is built by wave 0 alone (LayerNorm and rounding
//    with cross-lane DPP sums, the row as NP float4 pieces per lane, piece
//    P = 64 j + lane), so the prologue has no workgroup barrier; the other
//    waves wait once, at the barrier that publishes the rounded row;
//  - the remaining blocks go in batches of BU with every load in flight,
//    a last partial batch included (indices clamped, duplicates discarded);
//  - with several waves, wave 0 folds the tile's block products in block
//    order, 8 LDS reads in flight at a time.
// The arithmetic per output is the same as gemv_q8_kernel's (bit for bit).
template <int W, int NP, int PRO, int EPI>
__global__ __launch_bounds__(64 * W) void gemv1_kernel(const GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = blockIdx.x;
    const int nb = a.nb, K = nb * GRX_QK;
    const int row = tile * 64 + lane;
    constexpr bool PQ = PRO == GRX_PRO_PREQ;
    // the rounded row in LDS when the prologue builds it; pre-rounded rows
    // are read from HBM by each wave (a copy to LDS measured slower)
    constexpr bool LQ = !PQ;
    // LDS: [lxq K int8][lxs nb f32][lp nb*64 f32 if W > 1][lk 64*kKeyLd f32 if XSCORES]
    const size_t o_xs = LQ ? (size_t)K : 0;
    const size_t o_p = o_xs + (LQ ? (((size_t)nb * 4 + 15) & ~(size_t)15) : 0);
    int8_t *lxq = reinterpret_cast<int8_t *>(smem);
    float *lxs = reinterpret_cast<float *>(smem + o_xs);
    float *lp = reinterpret_cast<float *>(smem + o_p);
    float *lk = reinterpret_cast<float *>(smem + o_p + (W > 1 ? (size_t)nb * 64 * 4 : 0));

    const int b0 = (wave * nb) / W, b1 = ((wave + 1) * nb) / W;
    const int4 *__restrict__ wq = reinterpret_cast<const int4 *>(a.qs) + (size_t)tile * nb * 128;
    const uint16_t *__restrict__ wd = a.ds + (size_t)tile * nb * 64;
    auto load_block = [&](int b, int4 &w0, int4 &w1, uint32_t &dh) {
        if (a.cacheable) {
            w0 = wq[(size_t)b * 128 + lane];
            w1 = wq[(size_t)b * 128 + 64 + lane];
            dh = wd[(size_t)b * 64 + lane];
        } else {
            w0 = wload(wq + (size_t)b * 128 + lane);
            w1 = wload(wq + (size_t)b * 128 + 64 + lane);
            dh = wload(wd + (size_t)b * 64 + lane);
        }
    };
    auto act = [&](int b, int4 &a0, int4 &a1) {
        const int4 *p = reinterpret_cast<const int4 *>((LQ ? lxq : a.xq) + (size_t)b * GRX_QK);
        a0 = p[0];
        a1 = p[1];
    };
    auto act_scale = [&](int b) -> float { return LQ ? lxs[b] : a.xs[b]; };

    // ---- loads that wait for nothing: the first npf blocks (1, 2 or
    // PF; up to PF - 1 repeats of the last).  With 16 waves a wave owns at
    // most 2 blocks of rows up to 1024 values; two more would only cost
    // registers (a lane has 128 at 16 waves).
    constexpr int PF = LQ ? (W >= 16 ? 2 : kPrefetch) : 0;
    int4 pw[2 * (PF > 0 ? PF : 1)];
    uint32_t pd[PF > 0 ? PF : 1];
    const int npf = PF > 0 ? min(PF, b1 - b0) : 0;
    auto prefetch = [&] {
        if constexpr (PF > 0) {
            const int nl = npf <= 2 ? npf : PF;
#pragma unroll
            for (int u = 0; u < PF; ++u)
                if (u < nl) load_block(b0 + min(u, npf - 1), pw[2 * u], pw[2 * u + 1], pd[u]);
        }
    };
    // wave 0 issues them behind its prologue's loads (below)
    if (PQ || wave != 0) prefetch();
    float bias = 0.0f, resid = 0.0f;
    if (wave == 0 && row < a.rows) {
        if (a.bias != nullptr) bias = a.bias[row];
        if constexpr (EPI == GRX_EPI_RESID) resid = a.resid[row];
    }
    // the cache position of the QKV epilogues, read now rather than at the end
    const int pos0 = (EPI == GRX_EPI_QKV || EPI == GRX_EPI_QKV_ROPE) ? *a.pos : 0;

    if constexpr (EPI == GRX_EPI_XSCORES) {
        // waves 1..4 stage the 64 key rows of this run (rows past nctx
        // repeat the last), kKeyLd floats apart, while wave 0 builds the row
        static_assert(W >= 5, "XSCORES stages keys with waves 1..4");
        if (wave >= 1 && wave <= 4) {
            const float4 *kb = reinterpret_cast<const float4 *>(a.xk + (size_t)tile * a.nctx * 64);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int piece = (wave - 1) * 256 + u * 64 + lane;  // 16 pieces per key row
                const int r = piece >> 4, c4 = piece & 15;
                const int key = min((int)blockIdx.y * 64 + r, a.nctx - 1);
                reinterpret_cast<float4 *>(lk + r * kKeyLd)[c4] = kb[(size_t)key * 16 + c4];
            }
        }
    }
    // ---- prologue (wave 0): the activation row, rounded to Q8_0, into LDS
    if constexpr (!PQ) {
        if (wave == 0) wave_row_prologue<NP, PRO>(a, 0, lxq, lxs, lane, tile, prefetch);
        __syncthreads();
    }

    // ---- this wave's blocks: the prefetched ones, then batches of BU
    float acc = bias;
    // U blocks from bb on, nv of them real (the rest repeat block bb+nv-1)
    auto dots = [&](auto u_tag, const int4 *w, const uint32_t *dh, int bb, int nv) {
        constexpr int U = decltype(u_tag)::value;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int b = bb + min(u, nv - 1);
            int4 a0, a1;
            act(b, a0, a1);
            const int s = sdot8(w[2 * u], w[2 * u + 1], a0, a1);
            const float pv = __fmul_rn((float)s, grx_f16_to_f32((uint16_t)dh[u]));
            if constexpr (W == 1) {
                const float f = __fmaf_rn(pv, act_scale(b), acc);
                acc = u < nv ? f : acc;
            } else {
                lp[(size_t)b * 64 + lane] = pv;  // a repeated block writes its own value again
            }
        }
    };
    auto batch = [&](auto u_tag, int bb, int nv) {
        constexpr int U = decltype(u_tag)::value;
        int4 w[2 * U];
        uint32_t dh[U];
#pragma unroll
        for (int u = 0; u < U; ++u) load_block(bb + min(u, nv - 1), w[2 * u], w[2 * u + 1], dh[u]);
        dots(u_tag, w, dh, bb, nv);
    };
    // a last partial batch of nv blocks: the smallest of 1, 2, 4, BU that holds them
    auto tail = [&](int bb, int nv) {
        if (nv == 1)
            batch(std::integral_constant<int, 1>{}, bb, 1);
        else if (nv == 2)
            batch(std::integral_constant<int, 2>{}, bb, 2);
        else if (nv <= 4)
            batch(std::integral_constant<int, 4>{}, bb, nv);
        else
            batch(std::integral_constant<int, BU>{}, bb, nv);
    };
    int bb = b0;
    if constexpr (PF > 0) {
        if (npf == 1)
            dots(std::integral_constant<int, 1>{}, pw, pd, b0, 1);
        else if (npf == 2)
            dots(std::integral_constant<int, 2>{}, pw, pd, b0, 2);
        else
            dots(std::integral_constant<int, PF>{}, pw, pd, b0, npf);
        bb += npf;
    }
    for (; bb + BU <= b1; bb += BU) batch(std::integral_constant<int, BU>{}, bb, BU);
    if (bb < b1) tail(bb, b1 - bb);

    if constexpr (W > 1) {
        __syncthreads();
        if (wave != 0) return;
        // the ordered chain c = fma(p_b, da_b, c) in block order
        int b = 0;
        for (; b + 8 <= nb; b += 8) {
            float t[8], sc[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                t[u] = lp[(size_t)(b + u) * 64 + lane];
                sc[u] = act_scale(b + u);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = __fmaf_rn(t[u], sc[u], acc);
        }
        for (; b < nb; ++b) acc = __fmaf_rn(lp[(size_t)b * 64 + lane], act_scale(b), acc);
    }

    // ---- epilogue (wave 0)
    if constexpr (EPI == GRX_EPI_XSCORES) {
        // cross scores (whisper/decoder.go:94-108) of key j = 64*run + lane:
        // dotF32x4 (dot4f32avx, kernels_amd64.s:156-204) for keys in whole
        // groups of four, dotF32Go for the rest; q (this tile's 64 outputs)
        // broadcast from the lanes
        const int key = (int)blockIdx.y * 64 + lane;
        const float4 *kr = reinterpret_cast<const float4 *>(lk + lane * kKeyLd);
        float A[8], B[8], s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
        for (int l = 0; l < 8; ++l) A[l] = B[l] = 0.f;
#pragma unroll
        for (int c = 0; c < 64; c += 16) {
            float kv[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 t = kr[c / 4 + i];
                kv[4 * i] = t.x;
                kv[4 * i + 1] = t.y;
                kv[4 * i + 2] = t.z;
                kv[4 * i + 3] = t.w;
            }
#pragma unroll
            for (int l = 0; l < 16; ++l) {
                const float qd = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), c + l));
                if (l < 8)
                    A[l] = __fmaf_rn(qd, kv[l], A[l]);
                else
                    B[l - 8] = __fmaf_rn(qd, kv[l], B[l - 8]);
                const float pr = __fmul_rn(qd, kv[l]);
                if ((l & 3) == 0) s0 = __fadd_rn(s0, pr);
                if ((l & 3) == 1) s1 = __fadd_rn(s1, pr);
                if ((l & 3) == 2) s2 = __fadd_rn(s2, pr);
                if ((l & 3) == 3) s3 = __fadd_rn(s3, pr);
            }
        }
        float S[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) S[l] = __fadd_rn(A[l], B[l]);
        const float h0 = __fadd_rn(S[0], S[4]), h1 = __fadd_rn(S[1], S[5]);
        const float h2 = __fadd_rn(S[2], S[6]), h3 = __fadd_rn(S[3], S[7]);
        const float x4 = __fadd_rn(__fadd_rn(h0, h1), __fadd_rn(h2, h3));
        const float go = __fadd_rn(__fadd_rn(__fadd_rn(s0, s1), s2), s3);
        if (key < a.nctx) a.scores[(size_t)tile * a.nctx + key] = key < (a.nctx & ~3) ? x4 : go;
    } else if constexpr (EPI == GRX_EPI_RESID) {
        if (row < a.rows) a.y[row] = __fadd_rn(resid, acc);
    } else if constexpr (EPI == GRX_EPI_STORE) {
        if (row < a.rows) {
            a.y[row] = acc;
            if (a.ring.p != nullptr && row >= a.ring.col0)
                ring_put(a.ring, ring_row(a.ring, ring_head(a.ring), 0), row - a.ring.col0, acc);
        }
    } else {
        const float accm[1] = {acc};
        gemv_epilogue<1, W, false, EPI>(a, accm, row, lane, wave, pos0);
    }
}

// One-row products take gemv1_kernel unless GEMV1 is tuned to 0 (the
// general kernel, for comparisons) or the row is too wide for its prologue.
bool gemv1_fits(int pro, int nb) {
    if (grx_tune(GRX_TUNE_GEMV1) == 0) return false;
    return pro == GRX_PRO_PREQ || nb * GRX_QK <= kRowPieces * 256;
}

size_t gemv1_smem(int W, int pro, int nb, int epi = GRX_EPI_STORE) {
    size_t n = 0;
    if (pro != GRX_PRO_PREQ) n += (size_t)nb * GRX_QK + (((size_t)nb * 4 + 15) & ~(size_t)15);
    if (W > 1) n += (size_t)nb * 64 * 4;
    if (epi == GRX_EPI_XSCORES) n += (size_t)64 * kKeyLd * 4;
    return n;
}

// End of a decode step from per-workgroup argmax keys (keys [nslots][M]):
// row m's token is the first index of its largest value (the maximum key),
// recorded at the position (streams: in stream m's record), then the
// position moves on (streams: by one; one stream's rows: by M).
__global__ __launch_bounds__(256) void argmax_finish_kernel(const unsigned long long *__restrict__ keys, int nslots,
                                                            int M, int *__restrict__ tok_w, int *__restrict__ hist,
                                                            int *__restrict__ pos, int streams, int hist_stream) {
    __shared__ unsigned long long best[4][8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // every row's keys of four slots a thread in flight at once
    constexpr int U = 4;
    unsigned long long k[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int t0 = tid; t0 < nslots; t0 += U * 256) {
        unsigned long long v[U][8];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                const int t = t0 + 256 * u;
                v[u][m] = (m < M && t < nslots) ? keys[(size_t)t * M + m] : 0ull;
            }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int m = 0; m < 8; ++m) k[m] = v[u][m] > k[m] ? v[u][m] : k[m];
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        if (m >= M) break;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long w = __shfl_xor(k[m], o);
            k[m] = w > k[m] ? w : k[m];
        }
        if (lane == 0) best[wave][m] = k[m];
    }
    __syncthreads();
    if (tid < M) {
        unsigned long long k = 0;
        for (int w = 0; w < (int)(blockDim.x >> 6); ++w) k = best[w][tid] > k ? best[w][tid] : k;
        const int p0 = *pos;
        const int t = (int)(0xffffffffu - (uint32_t)(k & 0xffffffffull));
        tok_w[tid] = t;
        if (streams)
            hist[(size_t)tid * hist_stream + p0] = t;
        else
            hist[p0 + tid] = t;
    }
    __syncthreads();
    if (tid == 0) *pos = *pos + (streams ? 1 : M);
}

// One thread per block: quantU8 of m rows (q8int.go:88-105), signed.
__global__ void quant_act_kernel(const float *__restrict__ x, int lda, int m, int nb,
                                 int8_t *__restrict__ q, float *__restrict__ sc) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= m * nb) return;
    const int r = i / nb, b = i - r * nb;
    const float *src = x + (size_t)r * lda + b * GRX_QK;
    float v[GRX_QK];
#pragma unroll
    for (int j = 0; j < GRX_QK; ++j) v[j] = src[j];
    int8_t qq[GRX_QK];
    sc[i] = grx_quant_block(v, qq);
    int8_t *d = q + (size_t)r * nb * GRX_QK + b * GRX_QK;
#pragma unroll
    for (int j = 0; j < GRX_QK; ++j) d[j] = qq[j];
}

// s[m][rows][nb]: one thread per (activation row, weight row, block).
__global__ void block_dots_kernel(const int8_t *__restrict__ qs, int rows, int nb,
                                  const int8_t *__restrict__ q, int m, int32_t *__restrict__ s) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)m * rows * nb) return;
    const int b = (int)(i % nb);
    const int row = (int)((i / nb) % rows);
    const int r = (int)(i / ((size_t)nb * rows));
    const int tile = row >> 6, lane = row & 63;
    const int4 *wq = reinterpret_cast<const int4 *>(qs) + ((size_t)tile * nb + b) * 128;
    const int4 w0 = wq[lane], w1 = wq[64 + lane];
    const int4 *ap = reinterpret_cast<const int4 *>(q + (size_t)r * nb * GRX_QK + b * GRX_QK);
    s[i] = sdot8(w0, w1, ap[0], ap[1]);
}

size_t gemv_smem(int M, int W, int pro, int nb) {
    const size_t K = (size_t)nb * GRX_QK;
    size_t n = 0;
    if (pro != GRX_PRO_PREQ || M > 1) n += M * K;
    if (pro != GRX_PRO_PREQ || M > 1) n += ((size_t)M * nb * 4 + 15) & ~(size_t)15;
    const size_t n_p = W > 1 ? (size_t)M * (M > 1 ? kRound : nb) * 64 * 4 : 0;
    const size_t n_f = pro >= GRX_PRO_LN ? (size_t)M * K * 4 : 0;
    n += n_p > n_f ? n_p : n_f;  // the two share their bytes
    if (pro >= GRX_PRO_LN) n += 3 * 16 * sizeof(double);  // ln_block_reduce
    return n;
}

template <int M, int W, int PRO, int EPI>
hipError_t launch_one(hipStream_t st, const GemvArgs &a, int tiles) {
    const size_t smem = gemv_smem(M, W, PRO, a.nb);
    if (smem > 64 * 1024) {
        static bool raised = false;
        if (!raised) {
            raised = true;
            (void)hipFuncSetAttribute((const void *)gemv_q8_kernel<M, W, PRO, EPI>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        }
    }
    gemv_q8_kernel<M, W, PRO, EPI><<<dim3(tiles, 1, a.chunks > 1 ? a.chunks : 1), 64 * W, smem, st>>>(a);
    return hipGetLastError();
}

template <int M, int PRO, int EPI>
hipError_t launch_w(hipStream_t st, const GemvArgs &a, int tiles, int W) {
    switch (W) {
        case 1: return launch_one<M, 1, PRO, EPI>(st, a, tiles);
        case 2: return launch_one<M, 2, PRO, EPI>(st, a, tiles);
        case 4: return launch_one<M, 4, PRO, EPI>(st, a, tiles);
        case 8: return launch_one<M, 8, PRO, EPI>(st, a, tiles);
        default: return launch_one<M, 16, PRO, EPI>(st, a, tiles);
    }
}

template <int W, int NP, int PRO, int EPI>
hipError_t launch1_one(hipStream_t st, const GemvArgs &a, int tiles) {
    const size_t smem = gemv1_smem(W, PRO, a.nb, EPI);
    if (smem > 64 * 1024) {
        static bool raised = false;
        if (!raised) {
            raised = true;
            (void)hipFuncSetAttribute((const void *)gemv1_kernel<W, NP, PRO, EPI>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        }
    }
    const dim3 grid(tiles, EPI == GRX_EPI_XSCORES ? grx_ceil_div(a.nctx, 64) : 1);
    gemv1_kernel<W, NP, PRO, EPI><<<grid, 64 * W, smem, st>>>(a);
    return hipGetLastError();
}

// One-row launches: pre-rounded rows on 1..16 waves; rows rounded in the
// prologue on 1, 4, 8 or 16 waves with 2, 4 or 5 pieces per lane.
template <int PRO, int EPI>
hipError_t launch1_one_w(hipStream_t st, const GemvArgs &a, int tiles, int W) {
    while (W > 1 && W > a.nb) W >>= 1;  // every wave owns a block
    if constexpr (PRO == GRX_PRO_PREQ) {
        switch (W) {
            case 1: return launch1_one<1, 1, PRO, EPI>(st, a, tiles);
            case 2: return launch1_one<2, 1, PRO, EPI>(st, a, tiles);
            case 4: return launch1_one<4, 1, PRO, EPI>(st, a, tiles);
            case 8: return launch1_one<8, 1, PRO, EPI>(st, a, tiles);
            default: return launch1_one<16, 1, PRO, EPI>(st, a, tiles);
        }
    } else {
        const int pieces = a.nb * GRX_QK / 4;  // float4 pieces of the row
        const int np = pieces <= 128 ? 2 : pieces <= 256 ? 4 : 5;
        const int w = W >= 16 ? 16 : W >= 8 ? 8 : W >= 4 ? 4 : 1;
        auto go = [&](auto np_tag) -> hipError_t {
            constexpr int NP = decltype(np_tag)::value;
            if constexpr (EPI == GRX_EPI_XSCORES) {
                return launch1_one<16, NP, PRO, EPI>(st, a, tiles);
            } else {
                if (w == 1) return launch1_one<1, NP, PRO, EPI>(st, a, tiles);
                if (w == 4) return launch1_one<4, NP, PRO, EPI>(st, a, tiles);
                if (w == 8) return launch1_one<8, NP, PRO, EPI>(st, a, tiles);
                return launch1_one<16, NP, PRO, EPI>(st, a, tiles);
            }
        };
        if (np == 2) return go(std::integral_constant<int, 2>{});
        if (np == 4) return go(std::integral_constant<int, 4>{});
        return go(std::integral_constant<int, 5>{});
    }
}

// The one-row kernel on whole tiles, or on slices (gemv1n_kernel) where
// those pay and no ring copy is asked for.
template <int PRO, int EPI>
hipError_t launch1(hipStream_t st, const GemvArgs &a, int tiles, int W) {
    if constexpr (EPI != GRX_EPI_ARGMAX && EPI != GRX_EPI_XSCORES) {
        const int r = grx_gemv1_rows(tiles, PRO, EPI);
        if (r < 64 && a.ring.p == nullptr) return grx_gemv1n_launch(st, a, tiles, r, PRO, EPI);
    }
    return launch1_one_w<PRO, EPI>(st, a, tiles, W);
}

template <int M, int PRO, int EPI, int NS, int KB>
hipError_t launch_mx_one(hipStream_t st, const GemvArgs &a) {
    const size_t smem = gemv_mx_smem(M, NS, a.nb);
    const int groups = grx_ceil_div(a.rows, 16 * NS), WK = grx_ceil_div(a.nb, KB), W = WK > M ? WK : M;
    gemv_q8_mx_kernel<M, PRO, EPI, NS, KB><<<dim3(groups, 1, a.chunks > 1 ? a.chunks : 1), 64 * W, smem, st>>>(a);
    return hipGetLastError();
}

// Whether gemv_q8_mx_kernel takes M rows of this product: 4 or 8 rows, at
// most 8 waves of 8 blocks (16 with 16-row tiles), a one-wave prologue (rows
// of at most 1280 values), its LDS within 64 KiB, an epilogue it ends (not
// the fused cross scores, not the float64 LayerNorm's registers), and not
// switched off (GEMV_MX = 0).  Measured slower and left on gemv_q8_kernel:
// the rounded GELU output (its 32-row blocks on 32-row workgroups: 8 x 5120
// x 1280 14.5 us against 13.5) and the argmax over the vocabulary (16-row
// groups each staging the 8 rows: 8 x 51866 x 1280 30.4 us plus a row
// kernel and 4x the key slots, against 34 us in all).
bool mx_takes(int m, int pro, int epi, int nb) {
    if (grx_tune(GRX_TUNE_GEMV_MX) == 0) return false;
    if (m != 4 && m != 8) return false;
    if (nb < 1 || nb > 8 * 16) return false;
    if (pro != GRX_PRO_PREQ && nb * GRX_QK > kRowPieces * 256) return false;
    if (pro == GRX_PRO_LN64 || epi == GRX_EPI_ARGMAX || epi == GRX_EPI_XSCORES || epi == GRX_EPI_QKV_ROPE ||
        epi == GRX_EPI_GELU_Q)
        return false;
    return gemv_mx_smem(m, 1, nb) <= 64 * 1024;
}

// 8 blocks a wave up to 64 blocks, 16 past that
template <int M, int PRO, int EPI>
hipError_t launch_mx(hipStream_t st, const GemvArgs &a) {
    if (a.nb > 64) return launch_mx_one<M, PRO, EPI, 1, 16>(st, a);
    return launch_mx_one<M, PRO, EPI, 1, 8>(st, a);
}

template <int PRO, int EPI>
hipError_t launch_m(hipStream_t st, int m, const GemvArgs &a, int tiles, int W) {
    if (m == 1 && gemv1_fits(PRO, a.nb)) return launch1<PRO, EPI>(st, a, tiles, W);
    if constexpr (PRO != GRX_PRO_LN64 && EPI != GRX_EPI_ARGMAX && EPI != GRX_EPI_XSCORES &&
                  EPI != GRX_EPI_QKV_ROPE && EPI != GRX_EPI_GELU_Q) {
        if (mx_takes(m, PRO, EPI, a.nb)) return m == 4 ? launch_mx<4, PRO, EPI>(st, a) : launch_mx<8, PRO, EPI>(st, a);
    }
    switch (m) {
        case 1: return launch_w<1, PRO, EPI>(st, a, tiles, W);
        case 2: return launch_w<2, PRO, EPI>(st, a, tiles, W);
        case 4: return launch_w<4, PRO, EPI>(st, a, tiles, W);
        default: return launch_w<8, PRO, EPI>(st, a, tiles, W);
    }
}

}  // namespace

// Waves per tile: enough tiles x waves to cover the CUs, never more waves
// than blocks, and the workgroup's LDS within 64 KiB.
// GEMV_WAVES (1, 2, 4, 8 or 16) forces the choice, for tests.
int grx_gemv_pick_waves(int tiles, int nb, int m, int pro) {
    {
        const int w = grx_tune(GRX_TUNE_GEMV_WAVES);
        if (w == 1 || w == 2 || w == 4 || w == 8 || w == 16) return w;
    }
    const size_t lim = m > 1 ? kMultiLds : 64 * 1024;
    int W = 1;
    while (W < 16 && tiles * W < 2048 && 2 * W <= nb && gemv_smem(m, 2 * W, pro, nb) <= lim) W *= 2;
    // several rows fold in rounds, one wave per row: at least m waves
    if (m > 1 && W > 1 && W < m && gemv_smem(m, m, pro, nb) <= lim) W = m;
    // the float64 LayerNorm prologue (its bound check included) and the
    // two LayerNorms of LN2 need more than the 128 registers a lane has at
    // 16 waves; 8 waves measured the same as 16 for these products
    if ((pro == GRX_PRO_LN64 || pro == GRX_PRO_LN2) && W > 8) W = 8;
    return W;
}

// m must be 1, 2, 4 or 8; pro/epi one of the supported pairs below.
grx_status grx_gemv_launch(hipStream_t st, int m, int pro, int epi, const GemvArgs &a, int waves) {
    const int tiles = grx_ceil_div(a.rows, 64);
    if (tiles == 0 || m == 0) return GRX_OK;
    if (m > 1 && pro == GRX_PRO_PREQ && (size_t)m * a.nb * GRX_QK > kStageMax)
        return grx_fail(GRX_ESIZE, "grx: %d pre-rounded rows of %d values exceed %zu bytes of LDS", m,
                        a.nb * GRX_QK, kStageMax);
    if (a.chunks > 1 && (m < 2 || m > 8 || epi == GRX_EPI_ARGMAX || epi == GRX_EPI_XSCORES || a.streams ||
                         a.chunks > 65535))
        return grx_fail(GRX_EINVAL, "grx: %d groups of %d rows in one launch are not supported here", a.chunks, m);
    const int W = waves > 0 ? waves : grx_gemv_pick_waves(tiles, a.nb, m, pro);
    hipError_t e = hipErrorInvalidValue;
    if (pro == GRX_PRO_PREQ && epi == GRX_EPI_STORE) e = launch_m<GRX_PRO_PREQ, GRX_EPI_STORE>(st, m, a, tiles, W);
    else if (pro == GRX_PRO_QUANT && epi == GRX_EPI_STORE) e = launch_m<GRX_PRO_QUANT, GRX_EPI_STORE>(st, m, a, tiles, W);
    else if (pro == GRX_PRO_QUANT && epi == GRX_EPI_RESID) e = launch_m<GRX_PRO_QUANT, GRX_EPI_RESID>(st, m, a, tiles, W);
    else if (pro == GRX_PRO_LN && epi == GRX_EPI_STORE) e = launch_m<GRX_PRO_LN, GRX_EPI_STORE>(st, m, a, tiles, W);
    else if (pro == GRX_PRO_LN && epi == GRX_EPI_GELU) e = launch_m<GRX_PRO_LN, GRX_EPI_GELU>(st, m, a, tiles, W);
    else if (pro == GRX_PRO_LN && epi == GRX_EPI_QKV) e = launch_m<GRX_PRO_LN, GRX_EPI_QKV>(st, m, a, tiles, W);
    else if (pro == GRX_PRO_LN && epi == GRX_EPI_ARGMAX) e = launch_m<GRX_PRO_LN, GRX_EPI_ARGMAX>(st, m, a, tiles, W);
    else if (pro == GRX_PRO_LN && epi == GRX_EPI_GELU_Q) e = launch_m<GRX_PRO_LN, GRX_EPI_GELU_Q>(st, m, a, tiles, W);
    else if (pro == GRX_PRO_LN && epi == GRX_EPI_XSCORES) {
        // one row, 64-row tiles = heads of 64, 16 waves (keys staged by waves 1..4)
        if (m != 1 || a.nb < 16 || !gemv1_fits(pro, a.nb))
            return grx_fail(GRX_EINVAL, "grx: cross scores epilogue needs one row of 512..1280 values");
        e = launch1<GRX_PRO_LN, GRX_EPI_XSCORES>(st, a, tiles, 16);
    }
    else if (pro == GRX_PRO_EMBED_LN && epi == GRX_EPI_QKV) e = launch_m<GRX_PRO_EMBED_LN, GRX_EPI_QKV>(st, m, a, tiles, W);
    else if (pro == GRX_PRO_PREQ && epi == GRX_EPI_RESID) e = launch_m<GRX_PRO_PREQ, GRX_EPI_RESID>(st, m, a, tiles, W);
    else if (pro == GRX_PRO_PREQ && epi == GRX_EPI_QKV) e = launch_m<GRX_PRO_PREQ, GRX_EPI_QKV>(st, m, a, tiles, W);
    else if (pro == GRX_PRO_PREQ && epi == GRX_EPI_GELU_Q) e = launch_m<GRX_PRO_PREQ, GRX_EPI_GELU_Q>(st, m, a, tiles, W);
    else if (pro == GRX_PRO_PREQ && epi == GRX_EPI_ARGMAX) e = launch_m<GRX_PRO_PREQ, GRX_EPI_ARGMAX>(st, m, a, tiles, W);
    else if (pro == GRX_PRO_LN64 && epi == GRX_EPI_QKV_ROPE) e = launch_m<GRX_PRO_LN64, GRX_EPI_QKV_ROPE>(st, m, a, tiles, W);
    else if (pro == GRX_PRO_LN64 && epi == GRX_EPI_GELU_Q) e = launch_m<GRX_PRO_LN64, GRX_EPI_GELU_Q>(st, m, a, tiles, W);
    else if (m == 1 && ((pro == GRX_PRO_PREQ && epi == GRX_EPI_GLU) ||
                        ((pro == GRX_PRO_LN || pro == GRX_PRO_LN2) && (epi == GRX_EPI_SILU_Q || epi == GRX_EPI_GLU)) ||
                        (pro == GRX_PRO_LN2 && epi == GRX_EPI_STORE))) {
        // one row with a fused LayerNorm prologue and the matrix-core
        // product's epilogues, or a pre-rounded row into the GLU (a streaming
        // conformer's one-row chunk), on whole 64-row tiles (GLU pairs rows
        // 16 apart within 32)
        if (!gemv1_fits(pro, a.nb) || a.rows % GRX_QK != 0)
            return grx_fail(GRX_EINVAL, "grx: prologue %d epilogue %d needs one row of at most %d values and rows %% 32 == 0",
                            pro, epi, kRowPieces * 256);
        if (epi == GRX_EPI_GLU && a.lens == nullptr)
            return grx_fail(GRX_EINVAL, "grx: the GLU epilogue needs the valid rows");
        if (pro == GRX_PRO_PREQ)
            e = launch1_one_w<GRX_PRO_PREQ, GRX_EPI_GLU>(st, a, tiles, W);
        else if (pro == GRX_PRO_LN)
            e = epi == GRX_EPI_SILU_Q ? launch1_one_w<GRX_PRO_LN, GRX_EPI_SILU_Q>(st, a, tiles, W)
                                      : launch1_one_w<GRX_PRO_LN, GRX_EPI_GLU>(st, a, tiles, W);
        else
            e = epi == GRX_EPI_SILU_Q ? launch1_one_w<GRX_PRO_LN2, GRX_EPI_SILU_Q>(st, a, tiles, W)
                : epi == GRX_EPI_GLU  ? launch1_one_w<GRX_PRO_LN2, GRX_EPI_GLU>(st, a, tiles, W)
                                      : launch1_one_w<GRX_PRO_LN2, GRX_EPI_STORE>(st, a, tiles, W);
    }
    else if (pro == GRX_PRO_PREQ && (epi == GRX_EPI_AXPY_HALF || epi == GRX_EPI_SILU_Q)) {
        // one pre-rounded row (the matrix-core product's one-row epilogues)
        if (m != 1 || !gemv1_fits(pro, a.nb))
            return grx_fail(GRX_EINVAL, "grx: epilogue %d takes one pre-rounded row on the one-row kernel", epi);
        if (epi == GRX_EPI_SILU_Q && a.rows % GRX_QK != 0)
            return grx_fail(GRX_ESIZE, "rounded product output needs rows %% 32 == 0 (rows %d)", a.rows);
        e = epi == GRX_EPI_AXPY_HALF ? launch1<GRX_PRO_PREQ, GRX_EPI_AXPY_HALF>(st, a, tiles, W)
                                     : launch1<GRX_PRO_PREQ, GRX_EPI_SILU_Q>(st, a, tiles, W);
    }
    else return grx_fail(GRX_EINVAL, "grx: no GEMV variant for prologue %d epilogue %d", pro, epi);
    if (e != hipSuccess) return grx_hip_fail(e, "gemv_q8_kernel");
    if (epi == GRX_EPI_ARGMAX && a.keys != nullptr) {
        argmax_finish_kernel<<<1, 256, 0, st>>>(a.keys, tiles, m, a.tok_w, a.hist, a.pos_w, a.streams,
                                                a.hist_stream);
        GRX_LAUNCHED("argmax_finish_kernel");
    }
    return GRX_OK;
}

// ---------------------------------------------------------------- C ABI

static grx_status check_mm(const char *fn, grx_ctx *ctx, const void *dst, int ldc, const void *x,
                           int lda, int m, const grx_weight *w) {
    if (!ctx || !w) return grx_fail(GRX_EINVAL, "%s: NULL context or weight", fn);
    if (m < 0) return grx_fail(GRX_EINVAL, "%s: m = %d", fn, m);
    if (m > 0 && w->rows > 0 && (!dst || !x)) return grx_fail(GRX_EINVAL, "%s: NULL buffer", fn);
    if (m > 0 && w->rows > 0 && (ldc < w->rows || lda < w->cols))
        return grx_fail(GRX_EINVAL, "%s: ldc %d < %d or lda %d < %d", fn, ldc, w->rows, lda, w->cols);
    if (ctx->device != w->device) return grx_fail(GRX_EINVAL, "%s: weight lives on device %d, context on %d", fn, w->device, ctx->device);
    return GRX_OK;
}

int grx_gemm_min_m(void) {
    const int v = grx_tune(GRX_TUNE_GEMM_MIN_M);
    return v > 0 ? v : 16;
}

// Many rows on the matrix cores; few rows in GEMV launches of 8, 4, 2 and 1.
static grx_status gemv_rows_preq(hipStream_t st, float *dst, int ldc, const int8_t *q, const float *sc,
                                 int m, const grx_weight *w, const float *bias) {
    const int K = w->cols, nb = w->nb;
    if (m >= grx_gemm_min_m() && nb > 0) return grx_gemm_q8_launch(st, w, q, sc, m, bias, dst, ldc);
    int i = 0;
    while (i < m) {
        const int left = m - i;
        int mm = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
        while (mm > 1 && (size_t)mm * K > kStageMax) mm >>= 1;  // rows staged in LDS
        GemvArgs a = {};
        a.qs = w->qs;
        a.ds = w->ds;
        a.rows = w->rows;
        a.nb = nb;
        a.xq = q + (size_t)i * K;
        a.xs = sc + (size_t)i * nb;
        a.y = dst + (size_t)i * ldc;
        a.ldc = ldc;
        a.bias = bias;
        grx_status s = grx_gemv_launch(st, mm, GRX_PRO_PREQ, GRX_EPI_STORE, a, 0);
        if (s != GRX_OK) return s;
        i += mm;
    }
    return GRX_OK;
}

grx_status grx_quant_rows(hipStream_t st, const float *x, int lda, int m, int k, int8_t *q, float *sc) {
    const int nb = k / GRX_QK;
    if (m * nb == 0) return GRX_OK;
    quant_act_kernel<<<grx_ceil_div(m * nb, 256), 256, 0, st>>>(x, lda, m, nb, q, sc);
    GRX_LAUNCHED("quant_act_kernel");
    return GRX_OK;
}

extern "C" grx_status grx_quant_act_dev(grx_ctx *ctx, int8_t *q, float *sc, const float *x, int lda,
                                        int m, int k) {
    if (!ctx) return grx_fail(GRX_EINVAL, "grx_quant_act_dev: NULL context");
    if (m < 0 || k < 0 || lda < k) return grx_fail(GRX_EINVAL, "grx_quant_act_dev: bad shape");
    if (k % GRX_QK != 0) return grx_fail(GRX_ESIZE, "grx_quant_act_dev: k %d is not a multiple of 32", k);
    const int nb = k / GRX_QK;
    if (m * nb == 0) return GRX_OK;
    if (!q || !sc || !x) return grx_fail(GRX_EINVAL, "grx_quant_act_dev: NULL buffer");
    GRX_HIP(hipSetDevice(ctx->device));
    quant_act_kernel<<<grx_ceil_div(m * nb, 256), 256, 0, ctx->stream>>>(x, lda, m, nb, q, sc);
    GRX_LAUNCHED("quant_act_kernel");
    return GRX_OK;
}

extern "C" grx_status grx_matmul_q8_prequant_dev(grx_ctx *ctx, float *dst, int ldc, const int8_t *q,
                                                 const float *sc, int m, const grx_weight *w,
                                                 const float *bias) {
    grx_status s = check_mm("grx_matmul_q8_prequant_dev", ctx, dst, ldc, q, w ? w->cols : 0, m, w);
    if (s != GRX_OK) return s;
    if (m == 0 || w->rows == 0) return GRX_OK;
    if (!sc && w->cols > 0) return grx_fail(GRX_EINVAL, "grx_matmul_q8_prequant_dev: NULL scales");
    GRX_HIP(hipSetDevice(ctx->device));
    return gemv_rows_preq(ctx->stream, dst, ldc, q, sc, m, w, bias);
}

// Few rows (below the matrix cores' threshold) whose rounded values fit the
// products' LDS: each GEMV launch rounds its rows in its own prologue
// (quantU8, q8int.go:88-105, the same arithmetic as grx_quant_act_dev), so
// a row costs one launch and no scratch.
static grx_status gemv_rows_quant(hipStream_t st, float *dst, int ldc, const float *x, int lda, int m,
                                  const grx_weight *w, const float *bias) {
    const int K = w->cols;
    int i = 0;
    while (i < m) {
        const int left = m - i;
        int mm = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
        while (mm > 1 && (size_t)mm * K > kStageMax) mm >>= 1;
        GemvArgs a = {};
        a.qs = w->qs;
        a.ds = w->ds;
        a.rows = w->rows;
        a.nb = w->nb;
        a.x = x + (size_t)i * lda;
        a.lda = lda;
        a.y = dst + (size_t)i * ldc;
        a.ldc = ldc;
        a.bias = bias;
        grx_status s = grx_gemv_launch(st, mm, GRX_PRO_QUANT, GRX_EPI_STORE, a, 0);
        if (s != GRX_OK) return s;
        i += mm;
    }
    return GRX_OK;
}

extern "C" grx_status grx_matmul_q8_dev(grx_ctx *ctx, float *dst, int ldc, const float *x, int lda, int m,
                                        const grx_weight *w, const float *bias) {
    grx_status s = check_mm("grx_matmul_q8_dev", ctx, dst, ldc, x, lda, m, w);
    if (s != GRX_OK) return s;
    if (m == 0 || w->rows == 0) return GRX_OK;
    GRX_HIP(hipSetDevice(ctx->device));
    const int K = w->cols, nb = w->nb;
    if (nb > 0 && m < grx_gemm_min_m() && (size_t)K <= kStageMax)
        return gemv_rows_quant(ctx->stream, dst, ldc, x, lda, m, w, bias);
    void *buf;
    const size_t qbytes = ((size_t)m * K + 255) & ~(size_t)255;
    s = grx_ctx_scratch(ctx, qbytes + (size_t)m * nb * 4 + 16, &buf);
    if (s != GRX_OK) return s;
    int8_t *q = (int8_t *)buf;
    float *sc = (float *)((char *)buf + qbytes);
    s = grx_quant_act_dev(ctx, q, sc, x, lda, m, K);
    if (s != GRX_OK) return s;
    return grx_matmul_q8_prequant_dev(ctx, dst, ldc, q, sc, m, w, bias);
}

// ---------------------------------------------------------------- allocation-free product

// Device scratch of grx_matmul_q8_dev_noalloc: the last call's rounded
// activations, int8 [m][K] (256-byte aligned), then float32 scales
// [m][K/32].  Each GPU holds its own copy for the life of the process, and
// every call on a GPU shares it: calls that overlap on one GPU (two
// streams, or two threads) race for it.  Nothing in it needs to start at
// zero: each call writes every byte it reads.
constexpr size_t kNoAllocScratch = (size_t)4 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratch];

// The device address of `scratch` on each device (the array's name is a
// host-side stand-in, not a device address), looked up once per device.
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices];
static hipError_t g_scratch_err[kMaxDevices];

// Called by grx_ctx_create with `device` current.
void grx_noalloc_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[device] != nullptr) return;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_err[device] = e;
    if (e == hipSuccess) g_scratch_ptr[device] = p;
}

extern "C" grx_status grx_matmul_q8_dev_noalloc(grx_ctx *ctx, float *dst, int ldc, const float *x, int lda, int m,
                                                const grx_weight *w, const float *bias) {
    grx_status s = check_mm("grx_matmul_q8_dev_noalloc", ctx, dst, ldc, x, lda, m, w);
    if (s != GRX_OK) return s;
    if (m == 0 || w->rows == 0) return GRX_OK;
    const int K = w->cols, nb = w->nb;
    // few rows: each GEMV launch rounds its rows in its own prologue, so
    // the scratch is not touched (one launch per group of rows, as
    // grx_matmul_q8_dev takes them)
    if (nb > 0 && m < grx_gemm_min_m() && (size_t)K <= kStageMax) {
        GRX_HIP(hipSetDevice(ctx->device));
        return gemv_rows_quant(ctx->stream, dst, ldc, x, lda, m, w, bias);
    }
    const size_t qbytes = ((size_t)m * K + 255) & ~(size_t)255;
    const size_t need = qbytes + (size_t)m * nb * 4;
    if (need > kNoAllocScratch)
        return grx_fail(GRX_ESIZE,
                        "grx_matmul_q8_dev_noalloc: %d rows of %d values need %zu bytes of scratch, above its "
                        "%zu (call grx_matmul_q8_dev, or split the rows)",
                        m, K, need, kNoAllocScratch);
    void *base;
    {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        if (ctx->device >= kMaxDevices) return grx_fail(GRX_EINVAL, "grx_matmul_q8_dev_noalloc: device %d", ctx->device);
        base = g_scratch_ptr[ctx->device];
        if (base == nullptr)
            return grx_hip_fail(g_scratch_err[ctx->device] != hipSuccess ? g_scratch_err[ctx->device] : hipErrorNotReady,
                                "hipGetSymbolAddress(scratch)");
    }
    GRX_HIP(hipSetDevice(ctx->device));
    int8_t *q = static_cast<int8_t *>(base);
    float *sc = reinterpret_cast<float *>(static_cast<char *>(base) + qbytes);
    s = grx_quant_act_dev(ctx, q, sc, x, lda, m, K);
    if (s != GRX_OK) return s;
    return grx_matmul_q8_prequant_dev(ctx, dst, ldc, q, sc, m, w, bias);
}

extern "C" grx_status grx_matmul_q8(grx_ctx *ctx, float *dst, int ldc, const float *x, int lda, int m,
                                    const grx_weight *w, const float *bias) {
    grx_status s = check_mm("grx_matmul_q8", ctx, dst, ldc, x, lda, m, w);
    if (s != GRX_OK) return s;
    if (m == 0 || w->rows == 0) return GRX_OK;
    GRX_HIP(hipSetDevice(ctx->device));
    const int K = w->cols, N = w->rows, nb = w->nb;
    // device staging: [x m*K][y m*N][bias N][q m*K][sc m*nb]
    auto al = [](size_t n) { return (n + 255) & ~(size_t)255; };
    const size_t xb = al((size_t)m * K * 4), yb = al((size_t)m * N * 4), bb = al((size_t)N * 4);
    const size_t qb = al((size_t)m * K), sb = al((size_t)m * nb * 4 + 4);
    void *buf;
    s = grx_ctx_scratch(ctx, xb + yb + bb + qb + sb, &buf);
    if (s != GRX_OK) return s;
    char *p = (char *)buf;
    float *dx = (float *)p, *dy = (float *)(p + xb), *db = (float *)(p + xb + yb);
    int8_t *dq = (int8_t *)(p + xb + yb + bb);
    float *dsc = (float *)(p + xb + yb + bb + qb);
    if (K > 0)
        GRX_HIP(hipMemcpy2DAsync(dx, (size_t)K * 4, x, (size_t)lda * 4, (size_t)K * 4, m, hipMemcpyHostToDevice,
                                 ctx->stream));
    if (bias) GRX_HIP(hipMemcpyAsync(db, bias, (size_t)N * 4, hipMemcpyHostToDevice, ctx->stream));
    if (K > 0) {
        s = grx_quant_act_dev(ctx, dq, dsc, dx, K, m, K);
        if (s != GRX_OK) return s;
    }
    s = grx_matmul_q8_prequant_dev(ctx, dy, N, dq, dsc, m, w, bias ? db : nullptr);
    if (s != GRX_OK) return s;
    GRX_HIP(hipMemcpy2DAsync(dst, (size_t)ldc * 4, dy, (size_t)N * 4, (size_t)N * 4, m, hipMemcpyDeviceToHost,
                             ctx->stream));
    GRX_HIP(hipStreamSynchronize(ctx->stream));
    return GRX_OK;
}

extern "C" grx_status grx_linear_q8(grx_ctx *ctx, float *dst, const float *x, int m, const grx_weight *w,
                                    const float *bias) {
    if (!w) return grx_fail(GRX_EINVAL, "grx_linear_q8: NULL weight");
    return grx_matmul_q8(ctx, dst, w->rows, x, w->cols, m, w, bias);
}

namespace {
__global__ void vec_kernel(int fn, float *__restrict__ y, const float *__restrict__ x, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    y[i] = fn == GRX_VEC_EXPF ? grx_expf_go(v) : fn == GRX_VEC_EXP8 ? grx_exp8(v) : grx_gelu_at(v, i, n);
}
}  // namespace

extern "C" grx_status grx_vec_dev(grx_ctx *ctx, int fn, float *y, const float *x, int n) {
    if (!ctx) return grx_fail(GRX_EINVAL, "grx_vec_dev: NULL context");
    if (fn < GRX_VEC_EXPF || fn > GRX_VEC_GELU) return grx_fail(GRX_EINVAL, "grx_vec_dev: function %d", fn);
    if (n < 0) return grx_fail(GRX_EINVAL, "grx_vec_dev: n = %d", n);
    if (n == 0) return GRX_OK;
    if (!y || !x) return grx_fail(GRX_EINVAL, "grx_vec_dev: NULL buffer");
    GRX_HIP(hipSetDevice(ctx->device));
    vec_kernel<<<grx_ceil_div(n, 256), 256, 0, ctx->stream>>>(fn, y, x, n);
    GRX_LAUNCHED("vec_kernel");
    return GRX_OK;
}

extern "C" grx_status grx_block_dots_dev(grx_ctx *ctx, int32_t *s, const int8_t *q, int m, const grx_weight *w) {
    if (!ctx || !w) return grx_fail(GRX_EINVAL, "grx_block_dots_dev: NULL context or weight");
    if (m < 0) return grx_fail(GRX_EINVAL, "grx_block_dots_dev: m = %d", m);
    const size_t n = (size_t)m * w->rows * w->nb;
    if (n == 0) return GRX_OK;
    if (!s || !q) return grx_fail(GRX_EINVAL, "grx_block_dots_dev: NULL buffer");
    GRX_HIP(hipSetDevice(ctx->device));
    block_dots_kernel<<<(int)((n + 255) / 256), 256, 0, ctx->stream>>>(w->qs, w->rows, w->nb, q, m, s);
    GRX_LAUNCHED("block_dots_kernel");
    return GRX_OK;
}
