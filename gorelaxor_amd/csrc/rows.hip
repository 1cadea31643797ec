// rows.hip - row kernels shared by the decoders: LayerNorm of activation
// rows rounded to Q8_0 for the next product, and the whisper decoder's
// token + position embedding in front of it.  One workgroup per row.
#include "grx_internal.h"
#include "grx_ln.h"

namespace {

constexpr int kThreads = 256;

// kern.LayerNorm of one row held in LDS (internal/kern/mathx.go:55-75):
// float64 sums with the reference's results (ln32_stats), mean and inv
// rounded to float32, y = (v-mean)*inv*w + b rounded step by step.  The
// caller has the whole row in LDS (a barrier after writing it).
__device__ void ln_lds_row(float *v, int n, const float *w, const float *bb, double *red) {
    const int tid = threadIdx.x;
    float mean, inv;
    ln32_stats(v, n, red, mean, inv);
    for (int i = tid; i < n; i += blockDim.x) {
        float t = __fsub_rn(v[i], mean);
        t = __fmul_rn(t, inv);
        t = __fmul_rn(t, w[i]);
        v[i] = __fadd_rn(t, bb[i]);
    }
    __syncthreads();
}

// quantU8 (internal/kern/q8int.go:88-105) of the row in LDS, 32 lanes per
// block, signed values and float32 scales.
__device__ void quant_lds_row(const float *v, int n, int8_t *q, float *sc) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) {  // n % 32 == 0, blockDim % 32 == 0
        const float x = v[i];
        const float av = fabsf(x);
        float amax = av > 0.0f ? av : 0.0f;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) {
            const float t = __shfl_xor(amax, o, 32);
            amax = t > amax ? t : amax;
        }
        const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
        float r = rintf(__fmul_rn(x, id));
        r = fminf(fmaxf(r, -128.0f), 127.0f);
        q[i] = (int8_t)(int)r;
        if ((i & 31) == 0) sc[i / 32] = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
    }
}

// Row r of x [rows][ldx]: LayerNorm (w, b), rounded into xq [rows][n],
// xs [rows][n/32].
__global__ __launch_bounds__(kThreads) void ln_quant_rows_kernel(const float *__restrict__ x, int ldx, int n,
                                                                 const float *__restrict__ w,
                                                                 const float *__restrict__ b, int8_t *__restrict__ xq,
                                                                 float *__restrict__ xs) {
    extern __shared__ __align__(16) float row[];
    __shared__ double red[48];  // ln_block_reduce
    const int r = blockIdx.x;
    const float *xr = x + (size_t)r * ldx;
    if ((n & 3) == 0 && (ldx & 3) == 0) {  // 16-byte loads, all in flight together
        for (int i = threadIdx.x; i < n / 4; i += blockDim.x)
            reinterpret_cast<float4 *>(row)[i] = reinterpret_cast<const float4 *>(xr)[i];
    } else {
        for (int i = threadIdx.x; i < n; i += blockDim.x) row[i] = xr[i];
    }
    __syncthreads();
    ln_lds_row(row, n, w, b, red);
    quant_lds_row(row, n, xq + (size_t)r * n, xs + (size_t)r * (n / 32));
}

// Row r = stream r: x[r] = tokEmb.row(tok[r]) + decPos[*pos] (whisper/
// decoder.go:42-46; the embedding row widened from its Q8_0 tile layout,
// d*q then + pos unfused), stored as the residual stream, then LayerNorm
// and rounding as above.
__global__ __launch_bounds__(kThreads) void embed_ln_quant_kernel(
    const int *__restrict__ tok, const int *__restrict__ pos, const int8_t *__restrict__ emb_qs,
    const uint16_t *__restrict__ emb_ds, int nb, const float *__restrict__ pos_emb, float *__restrict__ x,
    const float *__restrict__ w, const float *__restrict__ b, int8_t *__restrict__ xq, float *__restrict__ xs) {
    extern __shared__ __align__(16) float row[];
    __shared__ double red[48];  // ln_block_reduce
    const int r = blockIdx.x, n = nb * GRX_QK;
    const int t = tok[r], p = *pos;
    const int etile = t >> 6, elane = t & 63;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int bk = i >> 5, h = (i >> 4) & 1, e = i & 15;
        const int8_t q = emb_qs[(((size_t)etile * nb + bk) * 2 + h) * 1024 + elane * 16 + e];
        const float d = grx_f16_to_f32(emb_ds[((size_t)etile * nb + bk) * 64 + elane]);
        const float v = __fadd_rn(__fmul_rn((float)q, d), pos_emb[(size_t)p * n + i]);
        row[i] = v;
        x[(size_t)r * n + i] = v;
    }
    __syncthreads();
    ln_lds_row(row, n, w, b, red);
    quant_lds_row(row, n, xq + (size_t)r * n, xs + (size_t)r * (n / 32));
}

}  // namespace

grx_status grx_ln_quant_rows(hipStream_t st, const float *x, int ldx, int rows, int n, const float *w,
                             const float *b, int8_t *xq, float *xs) {
    if (rows <= 0) return GRX_OK;
    ln_quant_rows_kernel<<<rows, kThreads, (size_t)n * 4, st>>>(x, ldx, n, w, b, xq, xs);
    GRX_LAUNCHED("ln_quant_rows_kernel");
    return GRX_OK;
}

grx_status grx_embed_ln_quant_rows(hipStream_t st, const int *tok, const int *pos, const grx_weight *emb,
                                   const float *pos_emb, float *x, int rows, const float *w, const float *b,
                                   int8_t *xq, float *xs) {
    if (rows <= 0) return GRX_OK;
    embed_ln_quant_kernel<<<rows, kThreads, (size_t)emb->nb * GRX_QK * 4, st>>>(tok, pos, emb->qs, emb->ds, emb->nb,
                                                                              pos_emb, x, w, b, xq, xs);
    GRX_LAUNCHED("embed_ln_quant_kernel");
    return GRX_OK;
}
