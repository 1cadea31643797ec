/*
 * grx_oracle.c - CPU restatement of gorelaxor's Q8_0 hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker the HIP product is compared
 * against.  Loaded by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg; the product never calls it.
 *
 * Citations are file:line in the reference Go module
 * github.com/xattribution/gorelaxor.  Built with -ffp-contract=off: every
 * fmaf() below stands for a VFMADD/VFNMADD in the reference assembly, and
 * every other product and sum is rounded on its own, as the reference's
 * Go code (GOAMD64=v1, which fuses nothing) and non-FMA instructions do.
 */
#include "grx_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static inline float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* ------------------------------------------------------------------ */
/* half precision                                                      */
/* ------------------------------------------------------------------ */

/* internal/kern/f16.go:14-33 (f16toF32): exact widening, subnormals kept. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1f;
    uint32_t man = (uint32_t)h & 0x3ff;
    if (exp == 0 && man == 0) return bits_f32(sign);
    if (exp == 0) { /* subnormal */
        uint32_t e = 127 - 15 + 1;
        while ((man & 0x400) == 0) {
            man <<= 1;
            e--;
        }
        man &= 0x3ff;
        return bits_f32(sign | e << 23 | man << 13);
    }
    if (exp == 0x1f) return bits_f32(sign | 0xffu << 23 | man << 13);
    return bits_f32(sign | (exp + 127 - 15) << 23 | man << 13);
}

/* internal/kern/f16.go:36-71 (f32toF16): round to nearest, ties to even. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t b = f32_bits(f);
    uint16_t sign = (uint16_t)(b >> 16) & 0x8000;
    int32_t exp = (int32_t)(b >> 23) & 0xff;
    uint32_t man = b & 0x7fffff;
    if (exp == 0xff) return man != 0 ? (sign | 0x7e00) : (sign | 0x7c00);
    int32_t e = exp - 127 + 15;
    if (e >= 0x1f) return sign | 0x7c00;
    if (e <= 0) {
        if (e < -10) return sign;
        man |= 0x800000;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t h = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1) == 1)) h++;
        return sign | (uint16_t)h;
    }
    uint32_t h = (uint32_t)e << 10 | man >> 13;
    uint32_t rem = man & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1) == 1)) h++;
    return sign | (uint16_t)h;
}

/* internal/kern/f16.go:6-12 (f16tab): every half widened, built once. */
static float g_f16tab[65536];
static pthread_once_t g_f16once = PTHREAD_ONCE_INIT;
static void f16tab_init(void) {
    for (uint32_t i = 0; i < 65536; i++) g_f16tab[i] = orc_f16_to_f32((uint16_t)i);
}
static inline const float *f16tab(void) {
    pthread_once(&g_f16once, f16tab_init);
    return g_f16tab;
}
static inline uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | p[1] << 8); }

/* ------------------------------------------------------------------ */
/* Q8_0 weights                                                        */
/* ------------------------------------------------------------------ */

/* kern_test.go:10-28 (quantQ8) and kern.go:149-164 (ToQ8): per block,
 * d = amax/127 in float32, id = 1/d (0 for d == 0), the scale stored as
 * f32toF16(d), each value int8(math.Round(float64(x*id))) - rounding half
 * away from zero. */
void orc_quant_q8(const float *v, size_t nvals, uint8_t *out) {
    for (size_t b = 0; b + ORC_QK <= nvals; b += ORC_QK) {
        float amax = 0;
        for (int i = 0; i < ORC_QK; i++) {
            float a = fabsf(v[b + i]);
            amax = a > amax ? a : amax;
        }
        float d = amax / 127.0f;
        float id = 0;
        if (d != 0) id = 1.0f / d;
        uint16_t h = orc_f32_to_f16(d);
        uint8_t *blk = out + (b / ORC_QK) * ORC_Q8_BYTES;
        blk[0] = (uint8_t)(h & 0xff);
        blk[1] = (uint8_t)(h >> 8);
        for (int i = 0; i < ORC_QK; i++) {
            float p = v[b + i] * id;
            blk[2 + i] = (uint8_t)(int8_t)round((double)p);
        }
    }
}

/* kern.go:235-246 (dequantQ8Go) = kernels_amd64.s:402-437 (dequantq8avx):
 * out[i] = f16(d) * int8(q[i]), exact in float32. */
void orc_dequant_q8(float *dst, const uint8_t *q, int nb) {
    const float *t = f16tab();
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = q + (size_t)b * ORC_Q8_BYTES;
        float d = t[le16(blk)];
        for (int i = 0; i < ORC_QK; i++) dst[b * ORC_QK + i] = d * (float)(int8_t)blk[2 + i];
    }
}

/* ------------------------------------------------------------------ */
/* activations                                                         */
/* ------------------------------------------------------------------ */

/* q8int.go:88-105 (quantU8Go), the same arithmetic as vnni_amd64.s:194-256
 * (quantU8avx) for finite inputs: sc = amax*f32(1/127) (0x3c010204),
 * id = 127/amax (0 when amax == 0), q = clamp(rne(x*id), -128, 127) + 128. */
void orc_quant_u8(uint8_t *dst, float *sc, const float *x, int nb) {
    const float inv127 = bits_f32(0x3c010204u);
    for (int b = 0; b < nb; b++) {
        const float *xs = x + b * ORC_QK;
        float amax = 0;
        for (int i = 0; i < ORC_QK; i++) {
            float a = fabsf(xs[i]);
            amax = a > amax ? a : amax;
        }
        sc[b] = amax * inv127;
        float id = 0;
        if (amax != 0) id = 127.0f / amax;
        for (int i = 0; i < ORC_QK; i++) {
            float p = xs[i] * id;
            int32_t q = (int32_t)rint((double)p);
            if (q > 127) q = 127;
            if (q < -128) q = -128;
            dst[b * ORC_QK + i] = (uint8_t)(q + 128);
        }
    }
}

/* The same rounding with the signed value stored directly: the unsigned
 * byte minus 128 (what the GPU keeps, since v_dot4_i32_i8 is signed). */
void orc_quant_act_i8(int8_t *dst, float *sc, const float *x, int nb) {
    uint8_t *u = (uint8_t *)malloc((size_t)nb * ORC_QK + 1);
    orc_quant_u8(u, sc, x, nb);
    for (int i = 0; i < nb * ORC_QK; i++) dst[i] = (int8_t)((int)u[i] - 128);
    free(u);
}

/* ------------------------------------------------------------------ */
/* int8 products                                                       */
/* ------------------------------------------------------------------ */

/* One block's int32 dot: vnni_amd64.s:34-69 computes Σ ua·w − 128·Σw with
 * ua = qa+128, which is Σ qa·w exactly (q8int.go:108-125 likewise). */
static inline int32_t block_dot(const int8_t *qa, const int8_t *w) {
    int32_t s = 0;
    for (int i = 0; i < ORC_QK; i++) s += (int32_t)qa[i] * (int32_t)w[i];
    return s;
}

/* s[(i*n + j)*nb + b] = the int32 dot of activation row i's block b with
 * weight row j's block b. */
void orc_block_dots(int32_t *s, const int8_t *qa, int m, const uint8_t *wq, int n, int k) {
    int nb = k / ORC_QK;
    size_t ld = (size_t)nb * ORC_Q8_BYTES;
    for (int i = 0; i < m; i++)
        for (int j = 0; j < n; j++)
            for (int b = 0; b < nb; b++)
                s[((size_t)i * n + j) * nb + b] =
                    block_dot(qa + (size_t)i * k + b * ORC_QK,
                              (const int8_t *)(wq + j * ld + (size_t)b * ORC_Q8_BYTES + 2));
}

/* Per-output finalize shared by the two entry points below.
 * EVEX/VEX order (vnni_amd64.s:58-69 FIN, driven block by block from the
 * bias by q8int.go:175-222): c = fma(f32(s)*dw, da, c).
 * Go twin order (q8int.go:121, intGo): c += f32(s)*dw*da, unfused. */
static void matmul_q8_int_core(float *c, int ldc, const int8_t *qa, const float *sa, int m,
                               const uint8_t *wq, int n, int k, const float *bias, int evex) {
    const float *t = f16tab();
    int nb = k / ORC_QK;
    size_t ld = (size_t)nb * ORC_Q8_BYTES;
    for (int i = 0; i < m; i++) {
        const int8_t *ar = qa + (size_t)i * k;
        const float *as = sa + (size_t)i * nb;
        for (int j = 0; j < n; j++) {
            const uint8_t *wr = wq + j * ld;
            float acc = bias ? bias[j] : 0.0f;
            for (int b = 0; b < nb; b++) {
                const uint8_t *blk = wr + (size_t)b * ORC_Q8_BYTES;
                int32_t s = block_dot(ar + b * ORC_QK, (const int8_t *)(blk + 2));
                float dw = t[le16(blk)];
                float p = (float)s * dw;
                if (evex) {
                    acc = fmaf(p, as[b], acc);
                } else {
                    float q = p * as[b];
                    acc = acc + q;
                }
            }
            c[(size_t)i * ldc + j] = acc;
        }
    }
}

/* Another implementation of the EVEX-order product for the graphs below
 * (orc_set_q8_product): the benchmark's CPU baselines route every product
 * of a graph through the VNNI restatement of the reference's kernel
 * (oracle/grx_vnni.cc, bit-equal to this one) at many threads.  NULL: this
 * file's scalar form. */
static orc_q8_product_fn g_q8_product = NULL;
void orc_set_q8_product(orc_q8_product_fn fn) { g_q8_product = fn; }

/* q8int.go:148-223 (matmulQ8Int): quantize each row of a (quantU8), set C
 * to the bias (or zero), then accumulate block by block.  Every output is
 * owned by one task, so its value does not depend on the thread split. */
void orc_matmul_q8_int(float *c, int ldc, const float *a, int lda, int m, const uint8_t *wq,
                       int n, int k, const float *bias, int evex) {
    if (m == 0 || n == 0) return; /* kern.go:186-188 */
    if (g_q8_product != NULL && evex) {
        g_q8_product(c, ldc, a, lda, m, wq, n, k, bias);
        return;
    }
    int nb = k / ORC_QK;
    int8_t *qa = (int8_t *)malloc((size_t)m * k + 1);
    float *sa = (float *)malloc(((size_t)m * nb + 1) * sizeof(float));
    for (int i = 0; i < m; i++)
        orc_quant_act_i8(qa + (size_t)i * k, sa + (size_t)i * nb, a + (size_t)i * lda, nb);
    matmul_q8_int_core(c, ldc, qa, sa, m, wq, n, k, bias, evex);
    free(qa);
    free(sa);
}

/* The int8 product from activations already rounded (EVEX order). */
void orc_matmul_q8_int_prequant(float *c, int ldc, const int8_t *qa, const float *sa, int m,
                                const uint8_t *wq, int n, int k, const float *bias) {
    if (m == 0 || n == 0) return;
    matmul_q8_int_core(c, ldc, qa, sa, m, wq, n, k, bias, 1);
}

/* ------------------------------------------------------------------ */
/* float dot products                                                  */
/* ------------------------------------------------------------------ */

/* kernels_amd64.s:90-95 (HSUM): lanes l and l+4 added, then two HADDPS. */
static inline float hsum8(const float a[8]) {
    float h0 = a[0] + a[4], h1 = a[1] + a[5], h2 = a[2] + a[6], h3 = a[3] + a[7];
    return (h0 + h1) + (h2 + h3);
}

/* gemm.go:294-308 (dotF32Go): four running sums, unfused, then summed
 * left to right. */
float orc_dot_f32_go(const float *x, const float *y, int n) {
    float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    int i = 0;
    for (; i + 4 <= n; i += 4) {
        float p0 = x[i] * y[i], p1 = x[i + 1] * y[i + 1];
        float p2 = x[i + 2] * y[i + 2], p3 = x[i + 3] * y[i + 3];
        s0 = s0 + p0;
        s1 = s1 + p1;
        s2 = s2 + p2;
        s3 = s3 + p3;
    }
    for (; i < n; i++) {
        float p = x[i] * y[i];
        s0 = s0 + p;
    }
    return ((s0 + s1) + s2) + s3;
}

/* kernels_amd64.s:156-204 (dot4f32avx) for one row: two 8-lane FMA
 * accumulators over 16-value steps, added, then HSUM.  kk % 16 == 0. */
static float dot_f32_avx_row(const float *x, const float *w, int kk) {
    float A[8] = {0}, B[8] = {0};
    for (int c = 0; c < kk; c += 16)
        for (int l = 0; l < 8; l++) {
            A[l] = fmaf(x[c + l], w[c + l], A[l]);
            B[l] = fmaf(x[c + 8 + l], w[c + 8 + l], B[l]);
        }
    float S[8];
    for (int l = 0; l < 8; l++) S[l] = A[l] + B[l];
    return hsum8(S);
}

/* kernels_amd64.go:75-95 (dotF32x4): the assembly over k &^ 15 values,
 * then dotF32Go over the rest, added on. */
void orc_dot_f32_x4(const float *x, const float *w, int ld, int k, float out[4]) {
    int kk = k & ~15;
    for (int r = 0; r < 4; r++) out[r] = kk > 0 ? dot_f32_avx_row(x, w + (size_t)r * ld, kk) : 0.0f;
    if (kk < k)
        for (int r = 0; r < 4; r++)
            out[r] = out[r] + orc_dot_f32_go(x + kk, w + (size_t)r * ld + kk, k - kk);
}

/* kernels_amd64.s:340-400 (dot4q8avx) for one row: per block an 8-lane
 * product of the first 8 values, three FMAs for the next 24, then
 * acc = fma(t, d, acc); HSUM at the end. */
static float dot_q8_avx_row(const float *x, const uint8_t *q, int nb) {
    const float *tab = f16tab();
    float acc[8] = {0};
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = q + (size_t)b * ORC_Q8_BYTES;
        const int8_t *w = (const int8_t *)(blk + 2);
        const float *xs = x + b * ORC_QK;
        float d = tab[le16(blk)];
        for (int l = 0; l < 8; l++) {
            float t = (float)w[l] * xs[l];
            t = fmaf((float)w[8 + l], xs[8 + l], t);
            t = fmaf((float)w[16 + l], xs[16 + l], t);
            t = fmaf((float)w[24 + l], xs[24 + l], t);
            acc[l] = fmaf(t, d, acc[l]);
        }
    }
    return hsum8(acc);
}

/* kern.go:248-266 (dotQ8Go): four running sums per block, unfused, then
 * s += d*(a0+a1+a2+a3). */
static float dot_q8_go(const float *x, const uint8_t *q, int nb) {
    const float *tab = f16tab();
    float s = 0;
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = q + (size_t)b * ORC_Q8_BYTES;
        const int8_t *w = (const int8_t *)(blk + 2);
        const float *xs = x + b * ORC_QK;
        float d = tab[le16(blk)];
        float a0 = 0, a1 = 0, a2 = 0, a3 = 0;
        for (int i = 0; i < ORC_QK; i += 4) {
            a0 = a0 + xs[i] * (float)w[i];
            a1 = a1 + xs[i + 1] * (float)w[i + 1];
            a2 = a2 + xs[i + 2] * (float)w[i + 2];
            a3 = a3 + xs[i + 3] * (float)w[i + 3];
        }
        s = s + d * (((a0 + a1) + a2) + a3);
    }
    return s;
}

/* The float route of kern.MatMul for Q8_0 weights (kern.go:193-194 ->
 * gemm.go:116-119 -> gemvRows gemm.go:195-259), m <= 16 only: one row of
 * activations reads the Q8_0 rows directly (dot4q8avx, four rows a group,
 * dotQ8Go for a last partial group); several rows widen each group of four
 * once and use dotF32x4; the bias is added afterwards. */
void orc_matmul_q8_float(float *c, int ldc, const float *a, int lda, int m, const uint8_t *wq,
                         int n, int k, const float *bias) {
    if (m == 0 || n == 0) return;
    int nb = k / ORC_QK;
    size_t ld = (size_t)nb * ORC_Q8_BYTES;
    float *wide = (float *)malloc((size_t)4 * k * sizeof(float) + 4);
    for (int j = 0; j < n; j += 4) {
        if (m > 1 && j + 4 <= n) {
            for (int r = 0; r < 4; r++) orc_dequant_q8(wide + (size_t)r * k, wq + (j + r) * ld, nb);
            for (int i = 0; i < m; i++) {
                float out[4];
                orc_dot_f32_x4(a + (size_t)i * lda, wide, k, k, out);
                float *y = c + (size_t)i * ldc;
                for (int r = 0; r < 4; r++) y[j + r] = out[r];
                if (bias)
                    for (int r = 0; r < 4; r++) y[j + r] = y[j + r] + bias[j + r];
            }
            continue;
        }
        for (int i = 0; i < m; i++) {
            const float *x = a + (size_t)i * lda;
            float *y = c + (size_t)i * ldc;
            if (j + 4 <= n) {
                for (int r = 0; r < 4; r++)
                    y[j + r] = nb > 0 ? dot_q8_avx_row(x, wq + (j + r) * ld, nb)
                                      : dot_q8_go(x, wq + (j + r) * ld, nb);
            } else {
                for (int jj = j; jj < n; jj++) y[jj] = dot_q8_go(x, wq + jj * ld, nb);
            }
            if (bias)
                for (int jj = j; jj < j + 4 && jj < n; jj++) y[jj] = y[jj] + bias[jj];
        }
    }
    free(wide);
}

/* ------------------------------------------------------------------ */
/* exp, softmax, activations                                           */
/* ------------------------------------------------------------------ */

#define C_LOG2E 0x3fb8aa3bu  /* f32(1.4426950408889634) */
#define C_LN2HI 0x3f317200u  /* 0.693145751953125 */
#define C_LN2LO 0x35bfbe8eu  /* f32(1.428606765330187e-06) */
#define C_P720 0x3ab60b61u   /* f32(1/720) */
#define C_P120 0x3c088889u   /* f32(1/120) */
#define C_P24 0x3d2aaaabu    /* f32(1/24) */
#define C_P6 0x3e2aaaabu     /* f32(1/6) */

/* mathx.go:7-33 (expf): n = floor(x*log2e + 0.5), two-part ln2 reduction,
 * degree-6 Taylor polynomial, all unfused. */
float orc_expf(float x) {
    if (x < -87) return 0;
    if (x > 88) return INFINITY;
    float t = x * bits_f32(C_LOG2E);
    t = t + 0.5f;
    int32_t ni = (int32_t)t;
    if ((float)ni > t) ni--;
    float n = (float)ni;
    float r = x - n * bits_f32(C_LN2HI);
    r = r - n * bits_f32(C_LN2LO);
    float p = bits_f32(C_P720) * r;
    p = p + bits_f32(C_P120);
    p = p * r;
    p = p + bits_f32(C_P24);
    p = p * r;
    p = p + bits_f32(C_P6);
    p = p * r;
    p = p + 0.5f;
    p = p * r;
    p = p + 1.0f;
    p = p * r;
    p = p + 1.0f;
    if (ni < -126) {
        float v = p * bits_f32((uint32_t)(ni + 127 + 64) << 23);
        return v * bits_f32(0x1f800000u); /* 2^-64 */
    }
    return p * bits_f32((uint32_t)(ni + 127) << 23);
}

/* kernels_amd64.s:236-258 (EXP8) for one lane: x clamped to [-87, 88],
 * n = rne(x*log2e), r by two fused reductions, Horner by FMA, times 2^n. */
float orc_exp8(float x) {
    x = x > -87.0f ? x : -87.0f;
    x = x < 88.0f ? x : 88.0f;
    float n = rintf(x * bits_f32(C_LOG2E));
    float r = fmaf(-n, bits_f32(C_LN2HI), x);
    r = fmaf(-n, bits_f32(C_LN2LO), r);
    float p = bits_f32(C_P720);
    p = fmaf(p, r, bits_f32(C_P120));
    p = fmaf(p, r, bits_f32(C_P24));
    p = fmaf(p, r, bits_f32(C_P6));
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int32_t ni = (int32_t)n;
    return p * bits_f32((uint32_t)(ni + 127) << 23);
}

/* kernels_amd64.go:107-117 (expSub): expSubAVX (kernels_amd64.s:271-297)
 * over the first n &^ 7 values - eight lane sums, then HSUM - plus
 * expSubGo (mathx.go:92-100) over the rest, its own sum added last. */
float orc_expsub(float *x, int n, float mx) {
    int n8 = n & ~7;
    float s = 0;
    if (n8 > 0) {
        float acc[8] = {0};
        for (int i = 0; i < n8; i += 8)
            for (int l = 0; l < 8; l++) {
                float e = orc_exp8(x[i + l] - mx);
                x[i + l] = e;
                acc[l] = acc[l] + e;
            }
        s = hsum8(acc);
    }
    float t = 0;
    for (int i = n8; i < n; i++) {
        float e = orc_expf(x[i] - mx);
        x[i] = e;
        t = t + e;
    }
    return s + t;
}

/* mathx.go:78-90 (softmax). */
void orc_softmax(float *x, int n) {
    float mx = -INFINITY;
    for (int i = 0; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float s = orc_expsub(x, n, mx);
    float inv = 1.0f / s;
    for (int i = 0; i < n; i++) x[i] = x[i] * inv;
}

/* kernels_amd64.s:299-338 (geluAVX) for one lane. */
static float gelu_avx1(float v) {
    float u = v * v;
    u = fmaf(bits_f32(0x3d372713u), u, 1.0f); /* 0.044715 */
    u = u * v;
    u = u * bits_f32(0x3f4c422au); /* sqrt(2/pi) */
    u = u < 9.0f ? u : 9.0f;
    u = u > -9.0f ? u : -9.0f;
    float e = orc_exp8(u + u);
    e = e + 1.0f;
    float t = 2.0f / e;
    t = 1.0f - t;
    t = 1.0f + t;
    t = t * v;
    return t * 0.5f;
}

/* mathx.go:36-52 (gelu), the scalar form. */
static float gelu_go1(float v) {
    const float c = bits_f32(0x3f4c422au);
    float u = c * v;
    float w = bits_f32(0x3d372713u) * v;
    w = w * v;
    w = 1.0f + w;
    u = u * w;
    float t;
    if (u > 9)
        t = 1;
    else if (u < -9)
        t = -1;
    else {
        float e = orc_expf(2.0f * u);
        t = 1.0f - 2.0f / (e + 1.0f);
    }
    float h = 0.5f * v;
    return h * (1.0f + t);
}

/* kernels_amd64.go:119-129 (geluVec): assembly over n &^ 7, Go for the rest. */
void orc_gelu_vec(float *x, int n) {
    int n8 = n & ~7;
    for (int i = 0; i < n8; i++) x[i] = gelu_avx1(x[i]);
    for (int i = n8; i < n; i++) x[i] = gelu_go1(x[i]);
}

/* kernels_amd64.go:241-250 (siluVec): siluAVX (kernels_amd64.s:439-460)
 * x/(exp8(0-x)+1) over n &^ 7, siluGo x/(1+expf(-x)) for the rest. */
void orc_silu_vec(float *x, int n) {
    int n8 = n & ~7;
    for (int i = 0; i < n8; i++) {
        float v = x[i];
        float e = orc_exp8(0.0f - v);
        x[i] = v / (e + 1.0f);
    }
    for (int i = n8; i < n; i++) {
        float v = x[i];
        x[i] = v / (1.0f + orc_expf(-v));
    }
}

/* kernels_amd64.go:252-262 (axpy): axpyAVX dst = fma(s, src, dst) over
 * n &^ 7, axpyGo dst += s*src unfused for the rest. */
void orc_axpy(float *dst, const float *src, int n, float s) {
    int n8 = n & ~7;
    for (int i = 0; i < n8; i++) dst[i] = fmaf(s, src[i], dst[i]);
    for (int i = n8; i < n; i++) dst[i] = dst[i] + s * src[i];
}

/* mathx.go:55-75 (layerNorm, also whisper/mathx.go:55-75): the mean of
 * float64 sums rounded to float32, the variance of float64(v-mean) in
 * float64, inv = f32(1/sqrt(var+1e-5)), y = (v-mean)*inv*w + b in float32. */
void orc_layernorm(float *dst, const float *src, int rows, int n, const float *w, const float *b) {
    for (int r = 0; r < rows; r++) {
        const float *x = src + (size_t)r * n;
        float *y = dst + (size_t)r * n;
        double sum = 0;
        for (int i = 0; i < n; i++) sum += (double)x[i];
        float mean = (float)(sum / (double)n);
        double vs = 0;
        for (int i = 0; i < n; i++) {
            double d = (double)(x[i] - mean);
            vs += d * d;
        }
        float inv = (float)(1.0 / sqrt(vs / (double)n + 1e-5));
        for (int i = 0; i < n; i++) {
            float t = x[i] - mean;
            t = t * inv;
            t = t * w[i];
            y[i] = t + b[i];
        }
    }
}

/* pockettts/nn.go:27-49 (layerNorm with eps): statistics and the
 * normalized value in float64, gain and bias (optional) in float32. */
void orc_layernorm_f64(float *dst, const float *src, int rows, int n, const float *w,
                       const float *b, double eps) {
    for (int r = 0; r < rows; r++) {
        const float *x = src + (size_t)r * n;
        float *y = dst + (size_t)r * n;
        double s = 0;
        for (int i = 0; i < n; i++) s += (double)x[i];
        double mean = s / (double)n;
        double q = 0;
        for (int i = 0; i < n; i++) {
            double d = (double)x[i] - mean;
            q += d * d;
        }
        double inv = 1.0 / sqrt(q / (double)n + eps);
        for (int i = 0; i < n; i++) {
            float o = (float)(((double)x[i] - mean) * inv);
            if (w) {
                o = o * w[i];
                o = o + b[i];
            }
            y[i] = o;
        }
    }
}

/* whisper/transcribe.go:459-464 (sample at temperature 0): the first
 * index of the largest value. */
int orc_argmax(const float *x, int n) {
    int id = 0;
    for (int i = 0; i < n; i++)
        if (x[i] > x[id]) id = i;
    return id;
}

/* ------------------------------------------------------------------ */
/* whisper-shaped decoder                                              */
/* ------------------------------------------------------------------ */

/* whisper/encoder.go:120-143: per decoder layer, K = enc·Wxkᵀ scaled by
 * f32(1/sqrt(head_dim)) and stored [h][t][d]; V = enc·Wxvᵀ + b stored
 * transposed [h][d][t].  Products take the int8 route. */
void orc_whisper_cross_kv(orc_whisper *m, const float *enc) {
    int st = m->n_state, nctx = m->n_audio_ctx, nh = m->n_head, hd = st / nh;
    float tsc = (float)(1.0 / sqrt((double)hd));
    float *k = (float *)malloc((size_t)nctx * st * sizeof(float));
    float *v = (float *)malloc((size_t)nctx * st * sizeof(float));
    for (int li = 0; li < m->n_layer; li++) {
        orc_whisper_layer *L = &m->layers[li];
        orc_matmul_q8_int(k, st, enc, st, nctx, L->xk, st, st, NULL, 1);
        orc_matmul_q8_int(v, st, enc, st, nctx, L->xv, st, st, L->xv_b, 1);
        for (int h = 0; h < nh; h++) {
            float *kd = L->cross_k + (size_t)h * nctx * hd;
            float *vd = L->cross_v + (size_t)h * nctx * hd;
            for (int t = 0; t < nctx; t++)
                for (int d = 0; d < hd; d++) {
                    kd[(size_t)t * hd + d] = k[(size_t)t * st + h * hd + d] * tsc;
                    vd[(size_t)d * nctx + t] = v[(size_t)t * st + h * hd + d];
                }
        }
    }
    free(k);
    free(v);
}

static void add_to(float *dst, const float *src, int n) {
    for (int i = 0; i < n; i++) dst[i] = dst[i] + src[i];
}

/* whisper/decoder.go:33-140 (Model.decode) with every matrix a Q8_0
 * weight on the int8 route: tokens placed after the cache's positions,
 * the logits of the last one written to `logits`.  Returns 0, or -1 when
 * the tokens do not fit the context (decoder.go:38-40). */
int orc_whisper_decode(orc_whisper *m, const int *tokens, int nt, float *logits) {
    int st = m->n_state, nh = m->n_head, hd = st / nh, nctx = m->n_audio_ctx;
    int pos0 = m->n;
    if (pos0 + nt > m->n_text_ctx) return -1;
    int nb = st / ORC_QK;
    size_t ld = (size_t)nb * ORC_Q8_BYTES;
    float sc = (float)(1.0 / sqrt((double)hd));
    float *x = (float *)malloc((size_t)nt * st * sizeof(float));
    float *cur = (float *)malloc((size_t)nt * st * sizeof(float));
    float *q = (float *)malloc((size_t)nt * st * sizeof(float));
    float *att = (float *)malloc((size_t)nt * st * sizeof(float));
    float *ff = (float *)malloc((size_t)nt * 4 * st * sizeof(float));
    float *kn = (float *)malloc((size_t)nt * st * sizeof(float));
    float *vn = (float *)malloc((size_t)nt * st * sizeof(float));
    int sw = nctx > pos0 + nt ? nctx : pos0 + nt;
    float *s = (float *)malloc((size_t)sw * sizeof(float));

    for (int i = 0; i < nt; i++) { /* decoder.go:42-46 */
        orc_dequant_q8(x + (size_t)i * st, m->tok_emb + (size_t)tokens[i] * ld, nb);
        add_to(x + (size_t)i * st, m->dec_pos + (size_t)(pos0 + i) * st, st);
    }
    for (int li = 0; li < m->n_layer; li++) {
        orc_whisper_layer *L = &m->layers[li];
        /* self-attention, causal (decoder.go:62-89) */
        orc_layernorm(cur, x, nt, st, L->attn_ln_w, L->attn_ln_b);
        orc_matmul_q8_int(q, st, cur, st, nt, L->q, st, st, L->q_b, 1);
        orc_matmul_q8_int(kn, st, cur, st, nt, L->k, st, st, NULL, 1);
        orc_matmul_q8_int(vn, st, cur, st, nt, L->v, st, st, L->v_b, 1);
        memcpy(L->self_k + (size_t)pos0 * st, kn, (size_t)nt * st * sizeof(float));
        memcpy(L->self_v + (size_t)pos0 * st, vn, (size_t)nt * st * sizeof(float));
        for (int i = 0; i < nt; i++)
            for (int h = 0; h < nh; h++) {
                int n = pos0 + i + 1;
                const float *qi = q + (size_t)i * st + h * hd;
                for (int j = 0; j < n; j++)
                    s[j] = orc_dot_f32_go(qi, L->self_k + (size_t)j * st + h * hd, hd) * sc;
                orc_softmax(s, n);
                float *out = att + (size_t)i * st + h * hd;
                for (int d = 0; d < hd; d++) out[d] = 0;
                for (int j = 0; j < n; j++) {
                    const float *vj = L->self_v + (size_t)j * st + h * hd;
                    float p = s[j];
                    for (int d = 0; d < hd; d++) out[d] = out[d] + p * vj[d];
                }
            }
        orc_matmul_q8_int(cur, st, att, st, nt, L->o, st, st, L->o_b, 1);
        add_to(x, cur, nt * st);

        /* cross-attention over the encoded audio (decoder.go:92-121) */
        orc_layernorm(cur, x, nt, st, L->x_ln_w, L->x_ln_b);
        orc_matmul_q8_int(q, st, cur, st, nt, L->xq, st, st, L->xq_b, 1);
        for (int i = 0; i < nt; i++)
            for (int h = 0; h < nh; h++) {
                const float *kd = L->cross_k + (size_t)h * nctx * hd;
                const float *vd = L->cross_v + (size_t)h * nctx * hd;
                const float *qi = q + (size_t)i * st + h * hd;
                float o4[4];
                int j = 0;
                for (; j + 4 <= nctx; j += 4) {
                    orc_dot_f32_x4(qi, kd + (size_t)j * hd, hd, hd, o4);
                    memcpy(s + j, o4, sizeof o4);
                }
                for (; j < nctx; j++) s[j] = orc_dot_f32_go(qi, kd + (size_t)j * hd, hd);
                orc_softmax(s, nctx);
                float *out = att + (size_t)i * st + h * hd;
                int d = 0;
                for (; d + 4 <= hd; d += 4) {
                    orc_dot_f32_x4(s, vd + (size_t)d * nctx, nctx, nctx, o4);
                    memcpy(out + d, o4, sizeof o4);
                }
                for (; d < hd; d++) out[d] = orc_dot_f32_go(s, vd + (size_t)d * nctx, nctx);
            }
        orc_matmul_q8_int(cur, st, att, st, nt, L->xo, st, st, L->xo_b, 1);
        add_to(x, cur, nt * st);

        /* feed-forward (decoder.go:124-128); parGelu (encoder.go:147-151)
         * runs geluVec over chunks of 1<<14 values */
        orc_layernorm(cur, x, nt, st, L->mlp_ln_w, L->mlp_ln_b);
        orc_matmul_q8_int(ff, 4 * st, cur, st, nt, L->fc1, 4 * st, st, L->fc1_b, 1);
        for (int o = 0; o < nt * 4 * st; o += 1 << 14) {
            int len = nt * 4 * st - o;
            if (len > 1 << 14) len = 1 << 14;
            orc_gelu_vec(ff + o, len);
        }
        orc_matmul_q8_int(cur, st, ff, 4 * st, nt, L->fc2, st, 4 * st, L->fc2_b, 1);
        add_to(x, cur, nt * st);
    }
    m->n = pos0 + nt;
    if (logits) { /* decoder.go:131-138, the last position only */
        float *row = (float *)malloc((size_t)st * sizeof(float));
        orc_layernorm(row, x + (size_t)(nt - 1) * st, 1, st, m->dec_ln_w, m->dec_ln_b);
        orc_matmul_q8_int(logits, m->n_vocab, row, st, 1, m->tok_emb, m->n_vocab, st, NULL, 1);
        free(row);
    }
    free(x);
    free(cur);
    free(q);
    free(att);
    free(ff);
    free(kn);
    free(vn);
    free(s);
    return 0;
}

/* whisper/transcribe.go:207-260 reduced to plain greedy decoding: the
 * prompt in one call, then n_steps single-token calls, each fed the
 * previous argmax.  out_tokens receives n_steps+1 ids. */
void orc_whisper_greedy(orc_whisper *m, const int *prompt, int n_prompt, int n_steps,
                        int *out_tokens) {
    float *lg = (float *)malloc((size_t)m->n_vocab * sizeof(float));
    m->n = 0;
    orc_whisper_decode(m, prompt, n_prompt, lg);
    int tok = orc_argmax(lg, m->n_vocab);
    out_tokens[0] = tok;
    for (int i = 0; i < n_steps; i++) {
        orc_whisper_decode(m, &tok, 1, lg);
        tok = orc_argmax(lg, m->n_vocab);
        out_tokens[i + 1] = tok;
    }
    free(lg);
}

/* ------------------------------------------------------------------ */
/* float route of ws.matmul (gemm.go:116-259) with float32 B           */
/* ------------------------------------------------------------------ */

/* k6x16avx (kernels_amd64.s:5-88) for one output: acc = fma(a_k, b_k, acc)
 * over k in order, then added to C (VADDPS). */
static float k6x16_one(const float *a, const float *b, int ldb_col_stride, int k) {
    float acc = 0.0f;
    for (int kk = 0; kk < k; kk++) acc = fmaf(a[kk], b[(size_t)kk * ldb_col_stride], acc);
    return acc;
}

/* gemvRows (gemm.go:195-259) for one row of A against float32 rows of B:
 * dotF32x4 for whole groups of four columns, dotF32Go for the rest, bias
 * added afterwards. */
static void gemv_f32_row(float *y, const float *x, const float *b, int ldb, int n, int k, const float *bias) {
    for (int j = 0; j < n; j += 4) {
        if (j + 4 <= n) {
            float out[4];
            orc_dot_f32_x4(x, b + (size_t)j * ldb, ldb, k, out);
            for (int r = 0; r < 4; r++) y[j + r] = out[r];
        } else {
            for (int jj = j; jj < n; jj++) y[jj] = orc_dot_f32_go(x, b + (size_t)jj * ldb, k);
        }
        if (bias)
            for (int jj = j; jj < j + 4 && jj < n; jj++) y[jj] = y[jj] + bias[jj];
    }
}

/* ws.matmul with float32 B (MatMulF32, kern.go:205-212, and Linear of an F32
 * weight): C[m][n] = A[m][k] . B[n][k]^T + bias.  m <= 16: gemvRows.  m > 16:
 * the rows in whole groups of six take k6x16avx over k in chunks of 256 from
 * C = bias (or 0) (gemm.go:121-180); the last m % 6 rows take gemv. */
void orc_matmul_f32(float *c, int ldc, const float *a, int lda, const float *b, int ldb, int m, int n,
                    int k, const float *bias) {
    if (m == 0 || n == 0) return;
    if (m <= 16) {
        for (int i = 0; i < m; i++) gemv_f32_row(c + (size_t)i * ldc, a + (size_t)i * lda, b, ldb, n, k, bias);
        return;
    }
    int mfull = m / 6 * 6;
    /* the packed panel holds B's column j as [kk][j]; element (kk, j) is b[j*ldb + kk] */
    for (int i = 0; i < mfull; i++) {
        float *ci = c + (size_t)i * ldc;
        for (int j = 0; j < n; j++) ci[j] = bias ? bias[j] : 0.0f;
        for (int k0 = 0; k0 < k; k0 += 256) {
            int kn = k - k0 < 256 ? k - k0 : 256;
            for (int j = 0; j < n; j++) {
                float acc = k6x16_one(a + (size_t)i * lda + k0, b + (size_t)j * ldb + k0, 1, kn);
                ci[j] = acc + ci[j];
            }
        }
    }
    for (int i = mfull; i < m; i++) gemv_f32_row(c + (size_t)i * ldc, a + (size_t)i * lda, b, ldb, n, k, bias);
}

/* ------------------------------------------------------------------ */
/* pocket-TTS flow-LM transformer                                      */
/* ------------------------------------------------------------------ */

/* pockettts/nn.go:69-76 (ropeFreqs): f_i = f32(exp(f32(i) * c)),
 * c = f32(-ln(period) * 2 / head_dim). */
void orc_rope_freqs(float *f, int head_dim, double period) {
    float c = (float)(-log(period) * 2.0 / (double)head_dim);
    for (int i = 0; i < head_dim / 2; i++) {
        float t = (float)i * c;
        f[i] = (float)exp((double)t);
    }
}

/* pockettts/nn.go:80-93 (applyRope): pair i of every head rotated by the
 * angle f64(f_i * pos) with f32(cos), f32(sin), unfused. */
void orc_apply_rope(float *x, int heads, const float *freqs, int half, int pos) {
    int hd = half * 2;
    float p = (float)pos;
    for (int i = 0; i < half; i++) {
        float fp = freqs[i] * p;
        double a = (double)fp;
        float c = (float)cos(a), s = (float)sin(a);
        for (int h = 0; h < heads; h++) {
            int j = h * hd + 2 * i;
            float r = x[j], im = x[j + 1];
            float rc = r * c, is = im * s, rs = r * s, ic = im * c;
            x[j] = rc - is;
            x[j + 1] = rs + ic;
        }
    }
}

/* pockettts/nn.go:200-254 (attend) with no context limit: per head, the
 * scores of the T queries against every cached key (MatMulF32), scaled,
 * softmax over the causal range (ExpSub, Scale), the rest cleared; then for
 * T < 4 the values summed by AddScaled in key order (zero weights skipped),
 * else MatMulF32 against the transposed values. */
static void ptts_attend(orc_ptts *m, float *out, const float *qkv, int T, const orc_ptts_layer *L, int pos0) {
    int d = m->d, hd = d / m->heads;
    float scale = (float)(1.0 / sqrt((double)hd));
    int nk = pos0 + T;
    float *sc = (float *)malloc((size_t)T * nk * sizeof(float));
    float *vt = (float *)malloc((size_t)hd * nk * sizeof(float));
    for (int h = 0; h < m->heads; h++) {
        orc_matmul_f32(sc, nk, qkv + h * hd, 3 * d, L->k + h * hd, d, T, nk, hd, NULL);
        for (int r = 0; r < T; r++) {
            int p = pos0 + r;
            float *row = sc + (size_t)r * nk;
            float mx = -INFINITY;
            for (int j = 0; j <= p; j++) {
                row[j] = row[j] * scale;
                mx = row[j] > mx ? row[j] : mx;
            }
            float sum = orc_expsub(row, p + 1, mx);
            float inv = 1.0f / sum;
            for (int j = 0; j <= p; j++) row[j] = row[j] * inv;
            for (int j = p + 1; j < nk; j++) row[j] = 0;
        }
        if (T < 4) {
            for (int r = 0; r < T; r++) {
                float *o = out + (size_t)r * d + h * hd;
                for (int e = 0; e < hd; e++) o[e] = 0;
                const float *row = sc + (size_t)r * nk;
                for (int j = 0; j < nk; j++)
                    if (row[j] != 0) orc_axpy(o, L->v + (size_t)j * d + h * hd, hd, row[j]);
            }
            continue;
        }
        for (int j = 0; j < nk; j++)
            for (int e = 0; e < hd; e++) vt[(size_t)e * nk + j] = L->v[(size_t)j * d + h * hd + e];
        orc_matmul_f32(out + h * hd, d, sc, nk, vt, nk, T, hd, nk, NULL);
    }
    free(sc);
    free(vt);
}

/* pockettts/nn.go:142-182 (transformer.forward), no context limit and no
 * layer scales (the flow LM's): T rows of x in place after m->pos. */
int orc_ptts_forward(orc_ptts *m, float *x, int T) {
    int d = m->d, ff = m->ff, hd = d / m->heads;
    if (m->pos + T > m->max_pos) return -1;
    float *h = (float *)malloc((size_t)T * d * sizeof(float));
    float *qkv = (float *)malloc((size_t)T * 3 * d * sizeof(float));
    float *att = (float *)malloc((size_t)T * d * sizeof(float));
    float *f = (float *)malloc((size_t)T * ff * sizeof(float));
    for (int li = 0; li < m->n_layer; li++) {
        orc_ptts_layer *L = &m->layers[li];
        orc_layernorm_f64(h, x, T, d, L->norm1_w, L->norm1_b, 1e-5);
        orc_matmul_q8_int(qkv, 3 * d, h, d, T, L->qkv, 3 * d, d, NULL, 1);
        for (int r = 0; r < T; r++) {
            float *row = qkv + (size_t)r * 3 * d;
            orc_apply_rope(row, m->heads, m->freqs, hd / 2, m->pos + r);
            orc_apply_rope(row + d, m->heads, m->freqs, hd / 2, m->pos + r);
        }
        for (int r = 0; r < T; r++) {
            memcpy(L->k + (size_t)(m->pos + r) * d, qkv + (size_t)r * 3 * d + d, (size_t)d * sizeof(float));
            memcpy(L->v + (size_t)(m->pos + r) * d, qkv + (size_t)r * 3 * d + 2 * d, (size_t)d * sizeof(float));
        }
        ptts_attend(m, att, qkv, T, L, m->pos);
        orc_matmul_q8_int(h, d, att, d, T, L->out, d, d, NULL, 1);
        add_to(x, h, T * d);
        orc_layernorm_f64(h, x, T, d, L->norm2_w, L->norm2_b, 1e-5);
        orc_matmul_q8_int(f, ff, h, d, T, L->ff1, ff, d, NULL, 1);
        orc_gelu_vec(f, T * ff);
        orc_matmul_q8_int(h, d, f, ff, T, L->ff2, d, ff, NULL, 1);
        add_to(x, h, T * d);
    }
    m->pos += T;
    free(h);
    free(qkv);
    free(att);
    free(f);
    return 0;
}

/* pockettts/lm.go:164-170 (flowLM.run): forward, then out_norm of the last
 * row (float64 LayerNorm, eps 1e-5). */
int orc_ptts_run(orc_ptts *m, float *x, int T, float *out) {
    if (orc_ptts_forward(m, x, T) != 0) return -1;
    orc_layernorm_f64(out, x + (size_t)(T - 1) * m->d, 1, m->d, m->out_w, m->out_b, 1e-5);
    return 0;
}

/* pockettts/lm.go:185-195 (flowLM.step): x = input . latent (bos when
 * latent is NULL; an F32 weight on the float route), run, and the
 * end-of-speech logit eos . out + b (a one-row F32 product: dotF32Go). */
int orc_ptts_step(orc_ptts *m, const float *latent, float *out, float *eos) {
    float *x = (float *)malloc((size_t)m->d * sizeof(float));
    orc_matmul_f32(x, m->d, latent ? latent : m->bos, m->ldim, m->input, m->ldim, 1, m->d, m->ldim, NULL);
    int rc = orc_ptts_run(m, x, 1, out);
    if (rc == 0) {
        float e;
        orc_matmul_f32(&e, 1, out, m->d, m->eos_w, m->d, 1, 1, m->d, NULL);
        *eos = e + m->eos_b;
    }
    free(x);
    return rc;
}
