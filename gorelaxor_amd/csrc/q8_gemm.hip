// q8_gemm.hip - the Q8_0 int8 product for many activation rows (encoder and
// prefill batches, the cross-attention key/value precompute) on the matrix
// cores.
//
// Same arithmetic as q8_gemv.hip, per output (the VNNI kernel's order,
// internal/kern/vnni_amd64.s:58-69 of github.com/xattribution/gorelaxor):
//     c = bias (or 0);  for b in 0..nb-1:  c = fma(f32(s_b) * dw_b, da_b, c)
// Here s_b, the int32 dot of one 32-value block, comes from one
// v_mfma_i32_16x16x32_i8 per 16x16 output tile: its K of 32 is exactly one
// Q8_0 block, so every block's sum stays separate (the K = 64 form would add
// two blocks together before their scales apply).  The lane then folds its
// four int32 results into its four running outputs in block order, so the
// result is bit-identical to the GEMV and to the reference.
//
// A wave computes 16 activation rows x 64 weight rows (one weight tile, four
// MFMAs sharing the A fragment); a workgroup of four waves covers 64 x 64.
// Per block a lane loads 8 bytes of A, 4 x 8 bytes of B (the weight tile
// layout keeps each row's 32 bytes in two 16-byte halves), four weight scales
// and four activation scales.  The per-output fold (convert, multiply, fma:
// 3 VALU ops per output per block) is the bound, not the MFMA: exact
// per-block scaling costs that much vector work per 32 multiply-adds.
#include <type_traits>

#include "grx_internal.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGemmBU = 2;  // blocks whose loads are issued before use

// What the epilogue does with each finished output c (GemmOut::epi):
//   STORE      y = c
//   ADD        y = y + c                      (kern.Add of the product)
//   AXPY_HALF  y = fma(0.5, c, y)             (AddScaled(y, c, 0.5), whole groups of 8)
//   SCALE      y = c * scale
//   SILU_Q     SiLU(c) of the AVX route (c / (EXP8(0 - c) + 1)), rounded to
//              Q8_0 per 32 outputs into yq [m][rows], ys [m][rows/32]
template <int EPI>
__global__ __launch_bounds__(256) void gemm_q8_mfma_kernel(const int8_t *__restrict__ qs,
                                                           const uint16_t *__restrict__ ds, int rows, int nb,
                                                           const int8_t *__restrict__ xq,
                                                           const float *__restrict__ xs, int m,
                                                           const float *__restrict__ bias, float *__restrict__ y,
                                                           int ldc, float scale, int8_t *__restrict__ yq,
                                                           float *__restrict__ ys) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tile = blockIdx.y;                     // weight rows 64*tile ..
    const int m0 = blockIdx.x * 64 + wave * 16;      // activation rows m0 .. m0+15
    const int K = nb * GRX_QK;
    const int li = lane & 15, lk = lane >> 4;        // fragment row/column, k group of 8

    // A fragment: row m0+li, bytes 8*lk..8*lk+7 of each block
    const int arow = m0 + li;
    const bool arow_ok = arow < m;
    const int8_t *ap = xq + (size_t)(arow_ok ? arow : 0) * K + 8 * lk;
    // B fragments: weight row 16*s+li of the tile, bytes 8*lk..: half lk/2, offset 8*(lk&1)
    const int8_t *bp = qs + (size_t)tile * nb * 2048 + (lk >> 1) * 1024 + li * 16 + 8 * (lk & 1);
    const uint16_t *dp = ds + (size_t)tile * nb * 64 + li;
    // D layout: lane holds column li, rows 4*lk + r
    int drow[4];
    bool drow_ok[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        drow[r] = m0 + 4 * lk + r;
        drow_ok[r] = drow[r] < m;
    }
    const float *sp[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) sp[r] = xs + (size_t)(drow_ok[r] ? drow[r] : 0) * nb;

    float c[4][4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int n = tile * 64 + 16 * s + li;
        const float bv = (bias != nullptr && n < rows) ? bias[n] : 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) c[s][r] = bv;
    }

    auto fold = [&](auto u_tag, int b0) {
        constexpr int U = decltype(u_tag)::value;
        long av[U], bv[U][4];
        uint32_t dh[U][4];
        float da[U][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int b = b0 + u;
            av[u] = arow_ok ? *reinterpret_cast<const long *>(ap + (size_t)b * GRX_QK) : 0l;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                bv[u][s] = *reinterpret_cast<const long *>(bp + (size_t)b * 2048 + s * 256);
                dh[u][s] = dp[(size_t)b * 64 + 16 * s];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) da[u][r] = sp[r][b];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                v4i d = {0, 0, 0, 0};
                d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[u], bv[u][s], d, 0, 0, 0);
                const float dw = grx_f16_to_f32((uint16_t)dh[u][s]);
#pragma unroll
                for (int r = 0; r < 4; ++r) c[s][r] = __fmaf_rn(__fmul_rn((float)d[r], dw), da[u][r], c[s][r]);
            }
        }
    };
    int b = 0;
    for (; b + kGemmBU <= nb; b += kGemmBU) fold(std::integral_constant<int, kGemmBU>{}, b);
    for (; b < nb; ++b) fold(std::integral_constant<int, 1>{}, b);

    if constexpr (EPI == GRX_GEMM_SILU_Q) {
        // The 64 columns of the tile are two Q8_0 blocks: block j holds
        // columns 16*(2j) + li and 16*(2j+1) + li of the 16 lanes sharing lk,
        // so a row's block maximum is four xor-shuffles within those lanes.
        const int nr = rows / GRX_QK;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n0 = tile * 64 + 32 * j;
            const bool col_ok = n0 < rows;  // rows % 32 == 0: whole blocks
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float x = c[2 * j + h][r];
                    v[h] = __fdiv_rn(x, __fadd_rn(grx_exp8(__fsub_rn(0.0f, x)), 1.0f));
                }
                const float a0 = fabsf(v[0]), a1 = fabsf(v[1]);
                float amax = a0 > 0.0f ? a0 : 0.0f;
                amax = a1 > amax ? a1 : amax;
#pragma unroll
                for (int o = 8; o > 0; o >>= 1) {
                    const float t = __shfl_xor(amax, o, 16);
                    amax = t > amax ? t : amax;
                }
                const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
                if (col_ok && drow_ok[r]) {
                    int8_t *qrow = yq + (size_t)drow[r] * rows + n0;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        float q = rintf(__fmul_rn(v[h], id));
                        q = fminf(fmaxf(q, -128.0f), 127.0f);
                        qrow[16 * h + li] = (int8_t)(int)q;
                    }
                    if (li == 0) ys[(size_t)drow[r] * nr + n0 / GRX_QK] = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
                }
            }
        }
    } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int n = tile * 64 + 16 * s + li;
            if (n >= rows) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (!drow_ok[r]) continue;
                float *yp = y + (size_t)drow[r] * ldc + n;
                if constexpr (EPI == GRX_GEMM_STORE) *yp = c[s][r];
                if constexpr (EPI == GRX_GEMM_ADD) *yp = __fadd_rn(*yp, c[s][r]);
                if constexpr (EPI == GRX_GEMM_AXPY_HALF) *yp = __fmaf_rn(0.5f, c[s][r], *yp);
                if constexpr (EPI == GRX_GEMM_SCALE) *yp = __fmul_rn(c[s][r], scale);
            }
        }
    }
}

}  // namespace

grx_status grx_gemm_q8_launch_ex(hipStream_t st, const grx_weight *w, const int8_t *xq, const float *xs, int m,
                                 const float *bias, const GemmOut &o) {
    if (m <= 0 || w->rows == 0) return GRX_OK;
    if (o.epi == GRX_GEMM_SILU_Q && w->rows % GRX_QK != 0)
        return grx_fail(GRX_ESIZE, "rounded product output needs rows %% 32 == 0 (rows %d)", w->rows);
    dim3 grid(grx_ceil_div(m, 64), w->tiles);
#define GRX_GEMM_CASE(E)                                                                                    \
    case E:                                                                                                 \
        gemm_q8_mfma_kernel<E><<<grid, 256, 0, st>>>(w->qs, w->ds, w->rows, w->nb, xq, xs, m, bias, o.y, o.ldc, \
                                                     o.scale, o.yq, o.ys);                                  \
        break;
    switch (o.epi) {
        GRX_GEMM_CASE(GRX_GEMM_STORE)
        GRX_GEMM_CASE(GRX_GEMM_ADD)
        GRX_GEMM_CASE(GRX_GEMM_AXPY_HALF)
        GRX_GEMM_CASE(GRX_GEMM_SCALE)
        GRX_GEMM_CASE(GRX_GEMM_SILU_Q)
        default:
            return grx_fail(GRX_EINVAL, "unknown product epilogue %d", o.epi);
    }
#undef GRX_GEMM_CASE
    GRX_LAUNCHED("gemm_q8_mfma_kernel");
    return GRX_OK;
}

// m rows of pre-rounded activations (xq [m][K], xs [m][K/32]) times the
// weight, into y (rows ldc apart), plus bias.
grx_status grx_gemm_q8_launch(hipStream_t st, const grx_weight *w, const int8_t *xq, const float *xs, int m,
                              const float *bias, float *y, int ldc) {
    GemmOut o;
    o.y = y;
    o.ldc = ldc;
    return grx_gemm_q8_launch_ex(st, w, xq, xs, m, bias, o);
}
