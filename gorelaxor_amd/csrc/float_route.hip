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
// Several threads per output row, each keeping whole lane chains of the
// reference's assembly; the Q8_0 weight is the one packed for the int8
// route (grx_weight tiles), so one weight serves both routes.  x is staged
// in LDS.
#include "grx_float.h"
#include "grx_internal.h"

namespace {

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

// x into LDS: every thread's reads issued before its stores
__device__ __forceinline__ void stage_x(const float *__restrict__ x, int k, float *xs) {
    const int t = threadIdx.x, nt = blockDim.x;
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int i = t + u * nt;
        v[u] = i < k ? x[i] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int i = t + u * nt;
        if (i < k) xs[i] = v[u];
    }
    for (int i = t + 8 * nt; i < k; i += nt) xs[i] = x[i];
    __syncthreads();
}

// Q8_0: the rows of one tile per workgroup (q8_float_row).
__global__ __launch_bounds__(256) void q8_float_gemv_kernel(const float *__restrict__ x, int k,
                                                            const int8_t *__restrict__ qs,
                                                            const uint16_t *__restrict__ ds, int nb, int n,
                                                            const float *__restrict__ bias, float *__restrict__ y,
                                                            GrxFloatEpi e) {
    extern __shared__ __align__(16) float xs[];
    stage_x(x, k, xs);
    int row;
    bool emit;
    float o = q8_float_row(xs, qs, ds, nb, n, blockIdx.x, row, emit);
    if (!emit) return;
    if (bias) o = __fadd_rn(o, bias[row]);
    float_epilogue(e, o, row, n, y);
}

// float32: eight threads per row; thread l keeps dot4f32avx's two chains
// A[l] and B[l] (16 values a step), S[l] = A[l]+B[l], and the HSUM is formed
// across the eight as (h0+h1)+(h2+h3), h_l = S[l]+S[l+4]; thread 0 adds
// dotF32Go over k past k &^ 15.  Rows past n &^ 3 take dotF32Go in thread 0.
__global__ __launch_bounds__(256) void f32_gemv_kernel(const float *__restrict__ x, int k,
                                                       const float *__restrict__ w, int n,
                                                       const float *__restrict__ bias, float *__restrict__ y,
                                                       GrxFloatEpi e) {
    extern __shared__ __align__(16) float xs[];
    stage_x(x, k, xs);
    const int row = blockIdx.x * 32 + (threadIdx.x >> 3), l = threadIdx.x & 7;
    const bool live = row < n, avx = row < (n & ~3);
    const float *wr = w + (size_t)row * k;
    const int kk = k & ~15;
    float A = 0.f, B = 0.f;
    if (live && avx) {
#pragma unroll 4
        for (int c = 0; c < kk; c += 16) {
            A = __fmaf_rn(xs[c + l], wr[c + l], A);
            B = __fmaf_rn(xs[c + 8 + l], wr[c + 8 + l], B);
        }
    }
    const float S = __fadd_rn(A, B);
    const float hl = __fadd_rn(S, __shfl_down(S, 4, 8));
    const float h1 = __shfl_down(hl, 1, 8), h2 = __shfl_down(hl, 2, 8), h3 = __shfl_down(hl, 3, 8);
    if (!live || l != 0) return;
    float o;
    if (avx) {
        o = kk > 0 ? __fadd_rn(__fadd_rn(hl, h1), __fadd_rn(h2, h3)) : 0.f;
        if (kk < k) o = __fadd_rn(o, dot_go(xs + kk, wr + kk, k - kk));
    } else {
        o = dot_go(xs, wr, k);
    }
    if (bias) o = __fadd_rn(o, bias[row]);
    float_epilogue(e, o, row, n, y);
}

constexpr int kMaxK = 32768;

}  // namespace

grx_status grx_float_gemv_q8(hipStream_t st, const grx_weight *w, const float *x, const float *bias, float *y,
                             GrxFloatEpi e) {
    if (w->cols > kMaxK) return grx_fail(GRX_ESIZE, "float route: %d columns (at most %d)", w->cols, kMaxK);
    if (w->rows == 0) return GRX_OK;
    q8_float_gemv_kernel<<<w->tiles, 256, (size_t)w->cols * 4, st>>>(x, w->cols, w->qs, w->ds, w->nb, w->rows, bias,
                                                                      y, e);
    GRX_LAUNCHED("q8_float_gemv_kernel");
    return GRX_OK;
}

grx_status grx_float_gemv_f32(hipStream_t st, const float *w, int n, int k, const float *x, const float *bias,
                              float *y, GrxFloatEpi e) {
    if (k > kMaxK) return grx_fail(GRX_ESIZE, "float route: %d columns (at most %d)", k, kMaxK);
    if (n == 0) return GRX_OK;
    f32_gemv_kernel<<<grx_ceil_div(n, 32), 256, (size_t)k * 4, st>>>(x, k, w, n, bias, y, e);
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
