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

__global__ __launch_bounds__(256) void gemm_q8_mfma_kernel(const int8_t *__restrict__ qs,
                                                           const uint16_t *__restrict__ ds, int rows, int nb,
                                                           const int8_t *__restrict__ xq,
                                                           const float *__restrict__ xs, int m,
                                                           const float *__restrict__ bias, float *__restrict__ y,
                                                           int ldc) {
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

#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int n = tile * 64 + 16 * s + li;
        if (n >= rows) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (drow_ok[r]) y[(size_t)drow[r] * ldc + n] = c[s][r];
    }
}

}  // namespace

// m rows of pre-rounded activations (xq [m][K], xs [m][K/32]) times the
// weight, into y (rows ldc apart), plus bias.
grx_status grx_gemm_q8_launch(hipStream_t st, const grx_weight *w, const int8_t *xq, const float *xs, int m,
                              const float *bias, float *y, int ldc) {
    if (m <= 0 || w->rows == 0) return GRX_OK;
    dim3 grid(grx_ceil_div(m, 64), w->tiles);
    gemm_q8_mfma_kernel<<<grid, 256, 0, st>>>(w->qs, w->ds, w->rows, w->nb, xq, xs, m, bias, y, ldc);
    GRX_LAUNCHED("gemm_q8_mfma_kernel");
    return GRX_OK;
}
