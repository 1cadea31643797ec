// float_route.hip - kern.MatMul's float route for one row of activations.
//
// internal/kern/kern.go:185-196 of github.com/xattribution/gorelaxor sends a
// product to the float route when the weight keeps its rows and there is
// one row of activations (m = 1 < intMinM), or when the weight is float32:
// gemvRows (gemm.go:195-259) runs the weight's rows in groups of four with
// the assembly kernels and the last partial group with the Go ones, then
// adds the bias:
//   Q8_0  rows in whole groups of four: dot4q8avx (kernels_amd64.s:340-400):
//         per block, eight lanes l: t = w[l]*x[l], then three fmas with the
//         next 24 values, acc[l] = fma(t, d, acc[l]); HSUM at the end.
//         Other rows: dotQ8Go (kern.go:248-266): per block four running sums,
//         s += d*(a0+a1+a2+a3).
//   F32   rows in whole groups of four: dotF32x4 (dot4f32avx over k &^ 15,
//         dotF32Go over the rest); other rows dotF32Go.
// One thread per output row; the Q8_0 weight is the one packed for the int8
// route (grx_weight tiles), so one weight serves both routes.  x is staged
// in LDS and read by every lane at the same address (a broadcast).
#include "grx_float.h"
#include "grx_internal.h"

namespace {

constexpr int kFloatWaves = 4;  // tiles of 64 rows per workgroup

// What happens to output row `row` of n after the bias (GrxFloatEpi):
// stored, stored through kern.SiLU (siluAVX's x/(EXP8(0-x)+1) for the rows
// below n &^ 7, siluGo's x/(1+expf(-x)) past them, kernels_amd64.go:241-250),
// or added to h as h += gate*o (unfused).
__device__ __forceinline__ void float_epilogue(const GrxFloatEpi &e, float o, int row, int n, float *y) {
    if (e.kind == GRX_FEPI_SILU) {
        const float a = __fdiv_rn(o, __fadd_rn(grx_exp8(__fsub_rn(0.f, o)), 1.f));
        const float b = __fdiv_rn(o, __fadd_rn(1.f, grx_expf_go(-o)));
        y[row] = row < (n & ~7) ? a : b;
    } else if (e.kind == GRX_FEPI_GATE) {
        y[row] = __fadd_rn(y[row], __fmul_rn(e.gate[row], o));
    } else {
        y[row] = o;
    }
}

__global__ __launch_bounds__(64 * kFloatWaves) void q8_float_gemv_kernel(const float *__restrict__ x, int k,
                                                                          const int8_t *__restrict__ qs,
                                                                          const uint16_t *__restrict__ ds, int nb,
                                                                          int n, const float *__restrict__ bias,
                                                                          float *__restrict__ y, GrxFloatEpi e) {
    extern __shared__ __align__(16) float xs[];
    for (int i = threadIdx.x; i < k; i += blockDim.x) xs[i] = x[i];
    __syncthreads();
    const int lane = threadIdx.x & 63, tile = blockIdx.x * kFloatWaves + (threadIdx.x >> 6);
    const int row = tile * 64 + lane;
    if (row >= n) return;
    const bool avx = row < (n & ~3);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float s = 0.f;
    const int8_t *qt = qs + (size_t)tile * nb * 2 * 64 * 16 + (size_t)lane * 16;
    const uint16_t *dt = ds + (size_t)tile * nb * 64 + lane;
    for (int b = 0; b < nb; ++b) {
        const int4 h0 = *reinterpret_cast<const int4 *>(qt + (size_t)(2 * b) * 64 * 16);
        const int4 h1 = *reinterpret_cast<const int4 *>(qt + (size_t)(2 * b + 1) * 64 * 16);
        const float d = grx_f16_to_f32(dt[(size_t)b * 64]);
        int8_t w[32];
        *reinterpret_cast<int4 *>(w) = h0;
        *reinterpret_cast<int4 *>(w + 16) = h1;
        const float *xb = xs + b * 32;
        if (avx) {
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                float t = __fmul_rn((float)w[l], xb[l]);
                t = __fmaf_rn((float)w[8 + l], xb[8 + l], t);
                t = __fmaf_rn((float)w[16 + l], xb[16 + l], t);
                t = __fmaf_rn((float)w[24 + l], xb[24 + l], t);
                acc[l] = __fmaf_rn(t, d, acc[l]);
            }
        } else {
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                a0 = __fadd_rn(a0, __fmul_rn(xb[i], (float)w[i]));
                a1 = __fadd_rn(a1, __fmul_rn(xb[i + 1], (float)w[i + 1]));
                a2 = __fadd_rn(a2, __fmul_rn(xb[i + 2], (float)w[i + 2]));
                a3 = __fadd_rn(a3, __fmul_rn(xb[i + 3], (float)w[i + 3]));
            }
            s = __fadd_rn(s, __fmul_rn(d, __fadd_rn(__fadd_rn(__fadd_rn(a0, a1), a2), a3)));
        }
    }
    float o = avx ? hsum8(acc) : s;
    if (bias) o = __fadd_rn(o, bias[row]);
    float_epilogue(e, o, row, n, y);
}

__global__ __launch_bounds__(256) void f32_gemv_kernel(const float *__restrict__ x, int k,
                                                       const float *__restrict__ w, int n,
                                                       const float *__restrict__ bias, float *__restrict__ y,
                                                       GrxFloatEpi e) {
    extern __shared__ __align__(16) float xs[];
    for (int i = threadIdx.x; i < k; i += blockDim.x) xs[i] = x[i];
    __syncthreads();
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= n) return;
    const float *wr = w + (size_t)row * k;
    float o = row < (n & ~3) ? dot_x4(xs, wr, k) : dot_go(xs, wr, k);
    if (bias) o = __fadd_rn(o, bias[row]);
    float_epilogue(e, o, row, n, y);
}

constexpr int kMaxK = 32768;

}  // namespace

grx_status grx_float_gemv_q8(hipStream_t st, const grx_weight *w, const float *x, const float *bias, float *y,
                             GrxFloatEpi e) {
    if (w->cols > kMaxK) return grx_fail(GRX_ESIZE, "float route: %d columns (at most %d)", w->cols, kMaxK);
    if (w->rows == 0) return GRX_OK;
    const int blocks = grx_ceil_div(w->tiles, kFloatWaves);
    q8_float_gemv_kernel<<<blocks, 64 * kFloatWaves, (size_t)w->cols * 4, st>>>(x, w->cols, w->qs, w->ds, w->nb,
                                                                                 w->rows, bias, y, e);
    GRX_LAUNCHED("q8_float_gemv_kernel");
    return GRX_OK;
}

grx_status grx_float_gemv_f32(hipStream_t st, const float *w, int n, int k, const float *x, const float *bias,
                              float *y, GrxFloatEpi e) {
    if (k > kMaxK) return grx_fail(GRX_ESIZE, "float route: %d columns (at most %d)", k, kMaxK);
    if (n == 0) return GRX_OK;
    f32_gemv_kernel<<<grx_ceil_div(n, 256), 256, (size_t)k * 4, st>>>(x, k, w, n, bias, y, e);
    GRX_LAUNCHED("f32_gemv_kernel");
    return GRX_OK;
}

// kern.Linear of one row through the float route, host buffers: the
// weight keeps its rows (no DropRows), so m = 1 takes gemvRows.
extern "C" grx_status grx_linear_q8_float(grx_ctx *ctx, float *dst, const float *x, const grx_weight *w,
                                          const float *bias) {
    if (!ctx || !dst || !x || !w) return grx_fail(GRX_EINVAL, "grx_linear_q8_float: NULL argument");
    const size_t xb = (size_t)w->cols * 4, yb = (size_t)w->rows * 4, bb = bias ? yb : 0;
    void *buf;
    grx_status s = grx_ctx_scratch(ctx, xb + yb + bb + 768, &buf);
    if (s != GRX_OK) return s;
    char *p = static_cast<char *>(buf);
    float *dx = reinterpret_cast<float *>(p), *dy = reinterpret_cast<float *>(p + (xb + 255) / 256 * 256);
    float *dbias = bias ? reinterpret_cast<float *>(p + (xb + 255) / 256 * 256 + (yb + 255) / 256 * 256) : nullptr;
    GRX_HIP(hipSetDevice(ctx->device));
    GRX_HIP(hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, ctx->stream));
    if (bias) GRX_HIP(hipMemcpyAsync(dbias, bias, bb, hipMemcpyHostToDevice, ctx->stream));
    if ((s = grx_float_gemv_q8(ctx->stream, w, dx, dbias, dy)) != GRX_OK) return s;
    GRX_HIP(hipMemcpyAsync(dst, dy, yb, hipMemcpyDeviceToHost, ctx->stream));
    GRX_HIP(hipStreamSynchronize(ctx->stream));
    return GRX_OK;
}

// The same for a float32 weight (rows x cols, row-major) in host memory.
extern "C" grx_status grx_linear_f32(grx_ctx *ctx, float *dst, const float *x, const float *w, int rows, int cols,
                                     const float *bias) {
    if (!ctx || !dst || !x || (!w && rows * cols > 0) || rows < 0 || cols < 0)
        return grx_fail(GRX_EINVAL, "grx_linear_f32: NULL argument or negative size");
    const size_t wb = (size_t)rows * cols * 4, xb = (size_t)cols * 4, yb = (size_t)rows * 4, bb = bias ? yb : 0;
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    void *buf;
    grx_status s = grx_ctx_scratch(ctx, up(wb) + up(xb) + up(yb) + up(bb) + 256, &buf);
    if (s != GRX_OK) return s;
    char *p = static_cast<char *>(buf);
    float *dw = reinterpret_cast<float *>(p), *dx = reinterpret_cast<float *>(p + up(wb));
    float *dy = reinterpret_cast<float *>(p + up(wb) + up(xb));
    float *dbias = bias ? reinterpret_cast<float *>(p + up(wb) + up(xb) + up(yb)) : nullptr;
    GRX_HIP(hipSetDevice(ctx->device));
    GRX_HIP(hipMemcpyAsync(dw, w, wb, hipMemcpyHostToDevice, ctx->stream));
    GRX_HIP(hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, ctx->stream));
    if (bias) GRX_HIP(hipMemcpyAsync(dbias, bias, bb, hipMemcpyHostToDevice, ctx->stream));
    if ((s = grx_float_gemv_f32(ctx->stream, dw, rows, cols, dx, dbias, dy)) != GRX_OK) return s;
    GRX_HIP(hipMemcpyAsync(dst, dy, yb, hipMemcpyDeviceToHost, ctx->stream));
    GRX_HIP(hipStreamSynchronize(ctx->stream));
    return GRX_OK;
}
