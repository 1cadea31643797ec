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

// Q8_0: four threads per row (64 rows a workgroup); thread j keeps the
// reference's lane chains j and j+4 of dot4q8avx, so no chain changes order,
// and the HSUM is formed across the four as (h0+h1)+(h2+h3), h_j =
// acc[j]+acc[j+4].  Rows of the last partial group of four take dotQ8Go in
// their thread 0.  Blocks are read four at a time.
__global__ __launch_bounds__(256) void q8_float_gemv_kernel(const float *__restrict__ x, int k,
                                                            const int8_t *__restrict__ qs,
                                                            const uint16_t *__restrict__ ds, int nb, int n,
                                                            const float *__restrict__ bias, float *__restrict__ y,
                                                            GrxFloatEpi e) {
    extern __shared__ __align__(16) float xs[];
    stage_x(x, k, xs);
    const int tile = blockIdx.x, rl = threadIdx.x >> 2, j = threadIdx.x & 3;
    const int row = tile * 64 + rl;
    const bool live = row < n, avx = row < (n & ~3);
    const int8_t *qt = qs + (size_t)tile * nb * 2 * 64 * 16 + (size_t)rl * 16;
    const uint16_t *dt = ds + (size_t)tile * nb * 64 + rl;
    auto ld = [&](int b, int4 &h0, int4 &h1, uint16_t &d) {
        h0 = *reinterpret_cast<const int4 *>(qt + (size_t)(2 * b) * 64 * 16);
        h1 = *reinterpret_cast<const int4 *>(qt + (size_t)(2 * b + 1) * 64 * 16);
        d = dt[(size_t)b * 64];
    };
    float a0 = 0.f, a1 = 0.f, s = 0.f;
    if (live && avx) {
        // the reference's lane chains j and j+4 of one block
        // value i of the block is byte i%4 of dword i/4; chain l = j + 4c
        // reads values l, 8+l, 16+l, 24+l: byte j of dwords c, 2+c, 4+c, 6+c
        const unsigned sh = 24u - 8u * (unsigned)j;
        auto val = [&](int dw) { return (float)((int)((unsigned)dw << sh) >> 24); };
        auto fold = [&](int b, const int4 &h0, const int4 &h1, uint16_t dh) {
            const float d = grx_f16_to_f32(dh);
            const float *xb = xs + b * 32;
            const int dws[2][4] = {{h0.x, h0.z, h1.x, h1.z}, {h0.y, h0.w, h1.y, h1.w}};
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int l = j + 4 * c;
                float t = __fmul_rn(val(dws[c][0]), xb[l]);
                t = __fmaf_rn(val(dws[c][1]), xb[8 + l], t);
                t = __fmaf_rn(val(dws[c][2]), xb[16 + l], t);
                t = __fmaf_rn(val(dws[c][3]), xb[24 + l], t);
                if (c == 0) a0 = __fmaf_rn(t, d, a0);
                else a1 = __fmaf_rn(t, d, a1);
            }
        };
        // groups of four blocks, the next group read (at a clamped index,
        // unconditionally) while this one is folded
        const int ng = nb / 4;
        int4 c0[4], c1[4];
        uint16_t cd[4];
        if (ng > 0) {
#pragma unroll
            for (int u = 0; u < 4; ++u) ld(u, c0[u], c1[u], cd[u]);
        }
        for (int g = 0; g < ng; ++g) {
            const int gn = min(g + 1, ng - 1);
            int4 n0[4], n1[4];
            uint16_t nd[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) ld(4 * gn + u, n0[u], n1[u], nd[u]);
#pragma unroll
            for (int u = 0; u < 4; ++u) fold(4 * g + u, c0[u], c1[u], cd[u]);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                c0[u] = n0[u];
                c1[u] = n1[u];
                cd[u] = nd[u];
            }
        }
        for (int b = 4 * ng; b < nb; ++b) {
            int4 h0, h1;
            uint16_t dh;
            ld(b, h0, h1, dh);
            fold(b, h0, h1, dh);
        }
    } else if (live && j == 0) {  // dotQ8Go (kern.go:248-266)
        for (int b = 0; b < nb; ++b) {
            int4 h0, h1;
            uint16_t dh;
            ld(b, h0, h1, dh);
            int8_t w[32];
            *reinterpret_cast<int4 *>(w) = h0;
            *reinterpret_cast<int4 *>(w + 16) = h1;
            const float d = grx_f16_to_f32(dh);
            const float *xb = xs + b * 32;
            float q0 = 0.f, q1 = 0.f, q2 = 0.f, q3 = 0.f;
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                q0 = __fadd_rn(q0, __fmul_rn(xb[i], (float)w[i]));
                q1 = __fadd_rn(q1, __fmul_rn(xb[i + 1], (float)w[i + 1]));
                q2 = __fadd_rn(q2, __fmul_rn(xb[i + 2], (float)w[i + 2]));
                q3 = __fadd_rn(q3, __fmul_rn(xb[i + 3], (float)w[i + 3]));
            }
            s = __fadd_rn(s, __fmul_rn(d, __fadd_rn(__fadd_rn(__fadd_rn(q0, q1), q2), q3)));
        }
    }
    // HSUM over the row's four threads: h_j = acc[j] + acc[j+4], then (h0+h1)+(h2+h3)
    const float h = __fadd_rn(a0, a1);
    const float h1 = __shfl_down(h, 1, 4), h23 = __fadd_rn(__shfl_down(h, 2, 4), __shfl_down(h, 3, 4));
    if (!live || j != 0) return;
    float o = avx ? __fadd_rn(__fadd_rn(h, h1), h23) : s;
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
