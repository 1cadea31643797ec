// layernorm.hip - the path's two LayerNorms as a parity-check entry point
// (grx_layernorm_dev), through the same device code the model kernels use:
//   - the workgroup form (ln32_stats / ln64_stats over a row in LDS or
//     global memory): the conformer's rows, the several-row products'
//     prologues, the pocket frame end and the flow head;
//   - the one-wave form (wave_ln32 / wave_ln64 over a row held as float4
//     pieces in registers): the one-row products' prologues.
// kern form: internal/kern/mathx.go:55-75; float64 form: pockettts/nn.go:
// 27-49 (github.com/xattribution/gorelaxor).  GRX_LN_TREE_ONLY keeps the
// parallel sums' results even where they could round differently from the
// reference's in-order sums, so tests can show which rows need the in-order
// pass.
#include "grx_internal.h"
#include "grx_ln.h"

namespace {

constexpr int kBlock = 256;
constexpr int kWavePieces = 5;  // rows up to 1280 values, as the one-row products

template <int FORM, bool CHECK>
__global__ __launch_bounds__(kBlock) void ln_block_kernel(const float *__restrict__ x, int n,
                                                          const float *__restrict__ w, const float *__restrict__ b,
                                                          double eps, float *__restrict__ y) {
    extern __shared__ __align__(16) float row[];
    __shared__ double red[48];  // ln_block_reduce
    const float *xr = x + (size_t)blockIdx.x * n;
    float *yr = y + (size_t)blockIdx.x * n;
    for (int i = threadIdx.x; i < n; i += blockDim.x) row[i] = xr[i];
    __syncthreads();
    if constexpr (FORM == GRX_LN_KERN) {
        float mean, inv;
        ln32_stats<CHECK>(row, n, red, mean, inv);
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            float t = __fsub_rn(row[i], mean);
            t = __fmul_rn(t, inv);
            t = __fmul_rn(t, w[i]);
            yr[i] = __fadd_rn(t, b[i]);
        }
    } else {
        double mean, inv;
        ln64_stats<CHECK>(row, n, eps, red, mean, inv);
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            float o = (float)__dmul_rn(__dsub_rn((double)row[i], mean), inv);
            if (w != nullptr) o = __fadd_rn(__fmul_rn(o, w[i]), b[i]);
            yr[i] = o;
        }
    }
}

template <int FORM, bool CHECK>
__global__ __launch_bounds__(64) void ln_wave_kernel(const float *__restrict__ x, int n, const float *__restrict__ w,
                                                     const float *__restrict__ b, double eps,
                                                     float *__restrict__ y) {
    constexpr int NP = kWavePieces;
    const int lane = threadIdx.x, npc = n / 4;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)blockIdx.x * n);
    float4 *y4 = reinterpret_cast<float4 *>(y + (size_t)blockIdx.x * n);
    float4 xv[NP], wv[NP], bv[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const int P = min(j * 64 + lane, npc - 1);
        xv[j] = x4[P];
        if (w != nullptr) {
            wv[j] = reinterpret_cast<const float4 *>(w)[P];
            bv[j] = reinterpret_cast<const float4 *>(b)[P];
        }
    }
    if constexpr (FORM == GRX_LN_KERN)
        wave_ln32<NP, CHECK>(xv, wv, bv, npc, lane);
    else
        wave_ln64<NP, CHECK>(xv, wv, bv, w != nullptr, npc, lane, eps, [&](float4 (&v)[NP]) {
#pragma unroll
            for (int j = 0; j < NP; ++j) v[j] = x4[min(j * 64 + lane, npc - 1)];
        });
#pragma unroll
    for (int j = 0; j < NP; ++j)
        if (j * 64 + lane < npc) y4[j * 64 + lane] = xv[j];
}

template <int FORM, bool CHECK>
void launch(int impl, hipStream_t st, float *y, const float *x, int rows, int n, const float *w, const float *b,
            double eps) {
    if (impl == GRX_LN_BLOCK)
        ln_block_kernel<FORM, CHECK><<<rows, kBlock, (size_t)n * 4, st>>>(x, n, w, b, eps, y);
    else
        ln_wave_kernel<FORM, CHECK><<<rows, 64, 0, st>>>(x, n, w, b, eps, y);
}

}  // namespace

extern "C" grx_status grx_layernorm_dev(grx_ctx *ctx, int form, int impl, int flags, float *y, const float *x,
                                        int rows, int n, const float *w, const float *b, double eps) {
    if (!ctx) return grx_fail(GRX_EINVAL, "grx_layernorm_dev: NULL context");
    if (form != GRX_LN_KERN && form != GRX_LN_F64) return grx_fail(GRX_EINVAL, "grx_layernorm_dev: form %d", form);
    if (impl != GRX_LN_BLOCK && impl != GRX_LN_WAVE) return grx_fail(GRX_EINVAL, "grx_layernorm_dev: impl %d", impl);
    if (flags & ~GRX_LN_TREE_ONLY) return grx_fail(GRX_EINVAL, "grx_layernorm_dev: flags %#x", flags);
    if (rows < 0 || n < 0) return grx_fail(GRX_EINVAL, "grx_layernorm_dev: rows %d, n %d", rows, n);
    if (rows == 0 || n == 0) return GRX_OK;
    if (!y || !x) return grx_fail(GRX_EINVAL, "grx_layernorm_dev: NULL buffer");
    if ((w == nullptr) != (b == nullptr)) return grx_fail(GRX_EINVAL, "grx_layernorm_dev: w and b go together");
    if (form == GRX_LN_KERN && w == nullptr) return grx_fail(GRX_EINVAL, "grx_layernorm_dev: kern's form needs w and b");
    if (impl == GRX_LN_BLOCK && n > 8192) return grx_fail(GRX_ESIZE, "grx_layernorm_dev: n %d above 8192", n);
    if (impl == GRX_LN_WAVE && (n % 4 != 0 || n > 64 * 4 * kWavePieces))
        return grx_fail(GRX_ESIZE, "grx_layernorm_dev: the one-wave form takes n %% 4 == 0, n <= %d (n = %d)",
                        64 * 4 * kWavePieces, n);
    GRX_HIP(hipSetDevice(ctx->device));
    const bool tree = (flags & GRX_LN_TREE_ONLY) != 0;
    if (form == GRX_LN_KERN) {
        if (tree)
            launch<GRX_LN_KERN, false>(impl, ctx->stream, y, x, rows, n, w, b, eps);
        else
            launch<GRX_LN_KERN, true>(impl, ctx->stream, y, x, rows, n, w, b, eps);
    } else {
        if (tree)
            launch<GRX_LN_F64, false>(impl, ctx->stream, y, x, rows, n, w, b, eps);
        else
            launch<GRX_LN_F64, true>(impl, ctx->stream, y, x, rows, n, w, b, eps);
    }
    GRX_LAUNCHED("grx_layernorm_dev");
    return GRX_OK;
}
