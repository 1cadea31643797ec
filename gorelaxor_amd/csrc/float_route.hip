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

// kern.Linear of a float32 weight (kern.go:185-201 -> ws.matmul,
// gemm.go:116-185) applied to each of B groups of `per` rows: with more than
// 16 rows, the rows in whole groups of six take k6x16 (kernels_amd64.s:5-88):
// from the bias (0 without one), each chunk of 256 k's fma chain (from zero)
// is added in.  This kernel computes that form for every row, 64 rows x 64
// columns per workgroup, 4 x 4 outputs per thread, 32 k's of x and w staged
// in LDS per pass (k's past the end staged as zeros: fma(0, 0, acc) leaves a
// chain that started at +0 unchanged); the rows the reference sends to
// gemvRows are rewritten afterwards by f32_rows_gemv_kernel.
constexpr int kPwT = 64, kPwK = 32;
__global__ __launch_bounds__(256) void f32_rows_k6x16_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                             const float *__restrict__ bias, float *__restrict__ y,
                                                             int rows, int n, int k) {
    __shared__ __align__(16) float as[kPwK][kPwT + 4];
    __shared__ __align__(16) float ws[kPwK][kPwT + 4];
    const int tid = threadIdx.x, tr = tid / 16, tc = tid % 16;
    const int r0 = blockIdx.y * kPwT, c0 = blockIdx.x * kPwT;
    float acc[4][4], out[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int col = c0 + tc * 4 + j;
        const float bj = (bias != nullptr && col < n) ? bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[i][j] = bj;
            acc[i][j] = 0.f;
        }
    }
    for (int k0 = 0; k0 < k; k0 += kPwK) {
        for (int e = tid; e < kPwT * kPwK; e += 256) {
            const int rr = e / kPwK, kk = e % kPwK, gr = r0 + rr, gc = c0 + rr;
            const bool kin = k0 + kk < k;
            as[kk][rr] = (gr < rows && kin) ? x[(size_t)gr * k + k0 + kk] : 0.f;
            ws[kk][rr] = (gc < n && kin) ? w[(size_t)gc * k + k0 + kk] : 0.f;
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < kPwK; ++kk) {
            const float4 a = *reinterpret_cast<const float4 *>(&as[kk][tr * 4]);
            const float4 b = *reinterpret_cast<const float4 *>(&ws[kk][tc * 4]);
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __fmaf_rn(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
        if ((k0 + kPwK) % 256 == 0 || k0 + kPwK >= k) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    out[i][j] = __fadd_rn(acc[i][j], out[i][j]);
                    acc[i][j] = 0.f;
                }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = r0 + tr * 4 + i;
        if (row >= rows) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = c0 + tc * 4 + j;
            if (col < n) y[(size_t)row * n + col] = out[i][j];
        }
    }
}

// The k6x16 form of the rows below lo of each group, one thread per output
// (for narrow outputs, where the 64 x 64 tiles would idle): from the bias,
// each chunk of 256 k's fma chain added in.
__global__ void f32_rows_k6x16_one_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                          const float *__restrict__ bias, float *__restrict__ y, int B, int per,
                                          int lo, int n, int k) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)B * lo * n) return;
    const int j = (int)(i % n);
    const size_t rr = i / n, row = rr / lo * per + rr % lo;
    const float *a = x + row * k, *b = w + (size_t)j * k;
    float c = bias != nullptr ? bias[j] : 0.f;
    for (int k0 = 0; k0 < k; k0 += 256) {
        const int kn = min(256, k - k0);
        float acc = 0.f;
#pragma unroll 8
        for (int kk = 0; kk < kn; ++kk) acc = __fmaf_rn(a[k0 + kk], b[k0 + kk], acc);
        c = __fadd_rn(acc, c);
    }
    y[row * n + j] = c;
}

// The rows of each group that ws.matmul sends to gemvRows (gemm.go:
// 182-184, 195-259): rows lo..per-1 of every group (all of them when
// per <= 16): dotF32x4 for whole groups of four columns, dotF32Go for the
// rest, then the bias added (none without one).  One thread per output.
__global__ void f32_rows_gemv_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                     const float *__restrict__ bias, float *__restrict__ y, int B, int per, int lo,
                                     int n, int k) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x, tail = (size_t)(per - lo);
    if (i >= (size_t)B * tail * n) return;
    const int j = (int)(i % n);
    const size_t rr = i / n, row = rr / tail * per + lo + rr % tail;
    const float *xr = x + row * k, *wj = w + (size_t)j * k;
    const float o = j < (n & ~3) ? dot_x4_s(xr, wj, 1, k) : dot_go_s(xr, wj, 1, k);
    y[row * n + j] = bias != nullptr ? __fadd_rn(o, bias[j]) : o;
}


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

// kern.Linear of a float32 weight w [n][k] over B groups of `per` rows of x
// [B*per][k] into y [B*per][n] (bias nullable): the k6x16 form for every
// row when a group has more than 16, then the gemvRows rows rewritten.
grx_status grx_float_rows_f32(hipStream_t st, const float *x, const float *w, const float *bias, float *y, int B,
                              int per, int n, int k) {
    const int rows = B * per, lo = per > 16 ? per / 6 * 6 : 0;
    if (rows == 0 || n == 0) return GRX_OK;
    if (lo > 0 && n < kPwT) {  // narrow outputs: a thread per output
        const size_t cnt = (size_t)B * lo * n;
        f32_rows_k6x16_one_kernel<<<(unsigned)((cnt + 255) / 256), 256, 0, st>>>(x, w, bias, y, B, per, lo, n, k);
        GRX_LAUNCHED("f32_rows_k6x16_one_kernel");
    } else if (lo > 0) {
        f32_rows_k6x16_kernel<<<dim3((n + kPwT - 1) / kPwT, (rows + kPwT - 1) / kPwT), 256, 0, st>>>(x, w, bias, y,
                                                                                                     rows, n, k);
        GRX_LAUNCHED("f32_rows_k6x16_kernel");
    }
    const size_t tail = (size_t)B * (per - lo) * n;
    if (tail > 0) {
        f32_rows_gemv_kernel<<<(unsigned)((tail + 255) / 256), 256, 0, st>>>(x, w, bias, y, B, per, lo, n, k);
        GRX_LAUNCHED("f32_rows_gemv_kernel");
    }
    return GRX_OK;
}
