// q8_gemv1n.hip - the Q8_0 product of one activation row on slices of the
// weight's 64-row tiles, for the decode steps' short products.
//
// Same arithmetic as q8_gemv.hip (the int8 route of kern.MatMul,
// internal/kern/kern.go:185-196 -> matmulQ8Int, q8int.go:148-223, with the
// VNNI tile kernel's per-output fold, vnni_amd64.s:58-69); only the mapping
// of rows and blocks onto workgroups differs.
#include "q8_gemv_impl.h"

namespace {

// The product of ONE activation row on slices of R = 2^lr rows of the
// 64-row tiles (R = 8, 16 or 32), so that a 512-row product runs on 64
// workgroups instead of 8: a decode step's products are latency-bound, and a
// single CU pulls ~20 bytes a cycle, so a 64-row tile of a 2048-wide weight
// (139 KB) on one CU takes ~3 us where eight CUs take a fraction of that.
//  - lane l holds row r0 + (l % R) of the slice and block slot l / R: a
//    wave's iteration covers G = 64 / R consecutive blocks, each lane's two
//    16-byte loads falling in G contiguous runs of 16 R bytes of the tile;
//  - block group n (G blocks) belongs to wave n % W; every wave issues its
//    first kPrefetchN iterations' loads before anything waits (wave 0
//    behind its prologue's row loads), the rest in pairs;
//  - the per-block products f32(s_b) * dw_b go to LDS [nb][R] and wave 0's
//    lanes l < R run the ordered chain c = fma(p_b, da_b, c) from the bias
//    in block order, as gemv1_kernel does (the same bits);
//  - workgroup g runs on XCD g % 8, and the 64 / R slices of one tile are
//    numbered onto one XCD, so the tile's scale lines are fetched into one
//    L2 once.
// W = blockDim.x / 64 is read at run time (one instantiation per prologue
// and epilogue); at most 16 waves, 8 for the float64 LayerNorm prologue
// (its registers do not fit the 128 a lane has at 16 waves).  Not for the
// argmax and cross-scores epilogues (whole tiles); the rounded epilogues
// (GELU_Q, SILU_Q) need R >= 32 (a Q8_0 block of outputs in one workgroup).
constexpr int kPrefetchN = 2;
constexpr int kNoRow = 0x3fffffff;  // a row index past every product: lanes l >= R store nothing

template <int NP, int PRO, int EPI>
__global__ __launch_bounds__(PRO == GRX_PRO_LN64 ? 512 : 1024) void gemv1n_kernel(const GemvArgs a, int lr) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int W = blockDim.x >> 6;
    const int R = 1 << lr, G = 64 >> lr, S = G;  // rows, block slots per wave, slices per tile
    const int g = blockIdx.x, xcd = g & 7, q = g >> 3;
    const int tile = (q / S) * 8 + xcd, slice = q % S;
    if (tile * 64 >= a.rows) return;  // the whole workgroup: no barrier is reached
    const int nb = a.nb, K = nb * GRX_QK;
    const int i = lane & (R - 1), j = lane >> lr;
    const int row = tile * 64 + slice * R + i;
    constexpr bool PQ = PRO == GRX_PRO_PREQ;
    constexpr bool LQ = !PQ;
    // LDS: [lxq K int8][lxs nb f32][lp nb*R f32]
    const size_t o_xs = LQ ? (size_t)K : 0;
    const size_t o_p = o_xs + (LQ ? (((size_t)nb * 4 + 15) & ~(size_t)15) : 0);
    int8_t *lxq = reinterpret_cast<int8_t *>(smem);
    float *lxs = reinterpret_cast<float *>(smem + o_xs);
    float *lp = reinterpret_cast<float *>(smem + o_p);

    const int4 *__restrict__ wq = reinterpret_cast<const int4 *>(a.qs) + (size_t)tile * nb * 128 + slice * R + i;
    const uint16_t *__restrict__ wd = a.ds + (size_t)tile * nb * 64 + slice * R + i;
    auto load_block = [&](int b, int4 &w0, int4 &w1, uint32_t &dh) {
        if (a.cacheable) {
            w0 = wq[(size_t)b * 128];
            w1 = wq[(size_t)b * 128 + 64];
            dh = wd[(size_t)b * 64];
        } else {
            w0 = wload(wq + (size_t)b * 128);
            w1 = wload(wq + (size_t)b * 128 + 64);
            dh = wload(wd + (size_t)b * 64);
        }
    };
    // iteration t of this wave: block group t*W + wave, lane's block j of it
    const int ng = (nb + G - 1) / G;
    const int nit = wave < ng ? (ng - wave + W - 1) / W : 0;
    auto blk_raw = [&](int t) { return (t * W + wave) * G + j; };
    auto blk = [&](int t) { return min(blk_raw(t), nb - 1); };

    int4 pw[2 * kPrefetchN];
    uint32_t pd[kPrefetchN];
    const int npf = min(kPrefetchN, nit);
    auto prefetch = [&] {
#pragma unroll
        for (int u = 0; u < kPrefetchN; ++u)
            if (u < npf) load_block(blk(u), pw[2 * u], pw[2 * u + 1], pd[u]);
    };
    if (PQ || wave != 0) prefetch();
    float bias = 0.0f, resid = 0.0f;
    if (wave == 0 && row < a.rows) {
        if (a.bias != nullptr) bias = a.bias[row];
        if constexpr (EPI == GRX_EPI_RESID) resid = a.resid[row];
    }
    const int pos0 = (EPI == GRX_EPI_QKV || EPI == GRX_EPI_QKV_ROPE) ? *a.pos : 0;

    if constexpr (!PQ) {
        // tile argument 0 only for workgroup 0: the embedding row is stored once
        if (wave == 0) wave_row_prologue<NP, PRO>(a, 0, lxq, lxs, lane, g == 0 ? 0 : 1, prefetch);
        __syncthreads();
    }
    auto dots = [&](int t, const int4 &w0, const int4 &w1, uint32_t dh) {
        const int b = blk(t);
        const int4 *p = reinterpret_cast<const int4 *>((LQ ? lxq : a.xq) + (size_t)b * GRX_QK);
        const int4 a0 = p[0], a1 = p[1];
        const int s = sdot8(w0, w1, a0, a1);
        const float pv = __fmul_rn((float)s, grx_f16_to_f32((uint16_t)dh));
        if (blk_raw(t) < nb) lp[(size_t)b * R + i] = pv;
    };
#pragma unroll
    for (int u = 0; u < kPrefetchN; ++u)
        if (u < npf) dots(u, pw[2 * u], pw[2 * u + 1], pd[u]);
    for (int t = kPrefetchN; t < nit; t += kPrefetchN) {
        int4 w[2 * kPrefetchN];
        uint32_t dh[kPrefetchN];
        const int nv = min(kPrefetchN, nit - t);
#pragma unroll
        for (int u = 0; u < kPrefetchN; ++u)
            if (u < nv) load_block(blk(t + u), w[2 * u], w[2 * u + 1], dh[u]);
#pragma unroll
        for (int u = 0; u < kPrefetchN; ++u)
            if (u < nv) dots(t + u, w[2 * u], w[2 * u + 1], dh[u]);
    }
    __syncthreads();
    if (wave != 0) return;
    // the ordered chain c = fma(p_b, da_b, c) in block order (lanes l >= R
    // repeat lane l % R's chain and store nothing)
    auto act_scale = [&](int b) -> float { return LQ ? lxs[b] : a.xs[b]; };
    float acc = bias;
    int b = 0;
    for (; b + 8 <= nb; b += 8) {
        float t[8], sc[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            t[u] = lp[(size_t)(b + u) * R + i];
            sc[u] = act_scale(b + u);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = __fmaf_rn(t[u], sc[u], acc);
    }
    for (; b < nb; ++b) acc = __fmaf_rn(lp[(size_t)b * R + i], act_scale(b), acc);

    const int orow = lane < R ? row : kNoRow;
    if constexpr (EPI == GRX_EPI_RESID) {
        if (orow < a.rows) a.y[orow] = __fadd_rn(resid, acc);
    } else if constexpr (EPI == GRX_EPI_STORE) {
        if (orow < a.rows) a.y[orow] = acc;
    } else {
        const float accm[1] = {acc};
        gemv_epilogue<1, 1, false, EPI>(a, accm, orow, lane, 0, pos0);
    }
}

size_t gemv1n_smem(int lr, int pro, int nb) {
    size_t n = 0;
    if (pro != GRX_PRO_PREQ) n += (size_t)nb * GRX_QK + (((size_t)nb * 4 + 15) & ~(size_t)15);
    n += (size_t)nb * ((size_t)1 << lr) * 4;
    return n;
}

}  // namespace

// Rows per workgroup of a one-row product: 64 (gemv1_kernel) or a slice of
// 8, 16 or 32 (gemv1n_kernel), so the product covers ~64-256 workgroups.
// Slices pay for pre-rounded rows (a 512 x 2048 product with a residual:
// 4.13 -> 3.72 us); rows rounded or LayerNorm'd in the prologue measured
// faster on whole tiles (LN, fc1, GELU: 4.50 us against 5.10 on 32-row
// slices), so they keep them.  GEMV1_ROWS (8, 16, 32 or 64) forces the
// choice, for tests and profiles.
int grx_gemv1_rows(int tiles, int pro, int epi) {
    if (epi == GRX_EPI_ARGMAX || epi == GRX_EPI_XSCORES) return 64;
    const int t = grx_tune(GRX_TUNE_GEMV1_ROWS);
    int r = (t == 8 || t == 16 || t == 32 || t == 64) ? t
            : pro != GRX_PRO_PREQ                       ? 64
            : tiles <= 32                               ? 8
            : tiles <= 64                               ? 16
            : tiles <= 128                              ? 32
                                                        : 64;
    if ((epi == GRX_EPI_GELU_Q || epi == GRX_EPI_SILU_Q) && r < 32) r = 32;
    return r;
}

// Waves of a narrow-tile product: one iteration per wave where 16 waves
// hold every block group (GEMV_WAVES forces 1..16).
static int gemv1n_waves(int nb, int lr) {
    const int w = grx_tune(GRX_TUNE_GEMV_WAVES);
    if (w == 1 || w == 2 || w == 4 || w == 8 || w == 16) return w;
    const int ng = grx_ceil_div(nb, 64 >> lr);
    int W = 1;
    while (W < 16 && W < ng) W *= 2;
    return W;
}

namespace {

template <int NP, int PRO, int EPI>
hipError_t launch1n_one(hipStream_t st, const GemvArgs &a, int tiles, int lr) {
    const size_t smem = gemv1n_smem(lr, PRO, a.nb);
    if (smem > 64 * 1024) {
        static bool raised = false;
        if (!raised) {
            raised = true;
            (void)hipFuncSetAttribute((const void *)gemv1n_kernel<NP, PRO, EPI>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        }
    }
    const int S = 64 >> lr, groups = grx_ceil_div(tiles, 8) * 8 * S;
    int W = gemv1n_waves(a.nb, lr);
    if (PRO == GRX_PRO_LN64 && W > 8) W = 8;
    gemv1n_kernel<NP, PRO, EPI><<<groups, 64 * W, smem, st>>>(a, lr);
    return hipGetLastError();
}


template <int PRO, int EPI>
hipError_t launch_np(hipStream_t st, const GemvArgs &a, int tiles, int lr) {
    if constexpr (PRO == GRX_PRO_PREQ) {
        return launch1n_one<1, PRO, EPI>(st, a, tiles, lr);
    } else {
        const int pieces = a.nb * GRX_QK / 4;  // float4 pieces of the row
        if (pieces <= 128) return launch1n_one<2, PRO, EPI>(st, a, tiles, lr);
        if (pieces <= 256) return launch1n_one<4, PRO, EPI>(st, a, tiles, lr);
        return launch1n_one<5, PRO, EPI>(st, a, tiles, lr);
    }
}

}  // namespace

hipError_t grx_gemv1n_launch(hipStream_t st, const GemvArgs &a, int tiles, int rows, int pro, int epi) {
    const int lr = rows == 8 ? 3 : rows == 16 ? 4 : 5;
#define GRX_N(P, E) \
    if (pro == P && epi == E) return launch_np<P, E>(st, a, tiles, lr)
    GRX_N(GRX_PRO_PREQ, GRX_EPI_STORE);
    GRX_N(GRX_PRO_QUANT, GRX_EPI_STORE);
    GRX_N(GRX_PRO_QUANT, GRX_EPI_RESID);
    GRX_N(GRX_PRO_LN, GRX_EPI_STORE);
    GRX_N(GRX_PRO_LN, GRX_EPI_GELU);
    GRX_N(GRX_PRO_LN, GRX_EPI_QKV);
    GRX_N(GRX_PRO_LN, GRX_EPI_GELU_Q);
    GRX_N(GRX_PRO_EMBED_LN, GRX_EPI_QKV);
    GRX_N(GRX_PRO_PREQ, GRX_EPI_RESID);
    GRX_N(GRX_PRO_PREQ, GRX_EPI_QKV);
    GRX_N(GRX_PRO_PREQ, GRX_EPI_GELU_Q);
    GRX_N(GRX_PRO_LN64, GRX_EPI_QKV_ROPE);
    GRX_N(GRX_PRO_LN64, GRX_EPI_GELU_Q);
    GRX_N(GRX_PRO_PREQ, GRX_EPI_AXPY_HALF);
    GRX_N(GRX_PRO_PREQ, GRX_EPI_SILU_Q);
#undef GRX_N
    return hipErrorInvalidValue;
}
