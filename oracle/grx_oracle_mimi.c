/* grx_oracle_mimi.c - CPU oracle of pocket-TTS's Mimi decoder (test
 * infrastructure only: never linked into the product).
 *
 * Restates, from github.com/xattribution/gorelaxor:
 *   mimiDecoder.decode  pockettts/mimi.go:122-152   latent projection, the
 *                                                   depthwise transposed
 *                                                   upsampling with its
 *                                                   carried overlap, the
 *                                                   transformer, SEANet
 *   runSea              pockettts/mimi.go:62-108    conv / convtr / residual
 *                                                   steps, ELU before a step
 *   conv.run            pockettts/nn.go:272-296     causal Conv1d as im2col +
 *                                                   Linear, past rows carried
 *   convtr.run          pockettts/nn.go:308-327     ConvTranspose1d as Linear +
 *                                                   overlap-add, partial carried
 *   elu                 pockettts/nn.go:51-64       min(v,0) through ExpSub(.,0)
 *                                                   per 512 values, then
 *                                                   max(v,0) + (e - 1)
 *   transformer.forward pockettts/nn.go:142-182     with a context limit and
 *   attend              pockettts/nn.go:200-254     layer scales (addScaled,
 *                                                   nn.go:185-196)
 * Every Linear takes kern.MatMul's route for its weight's type: the int8
 * route for Q8_0 (pockettts/model.go:331-366 packs and drops them), the
 * float route of MatMulF32 for float32 weights. */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "grx_oracle.h"

/* kern.Linear(y, x, m, w, bias) by the weight's type */
static void mlin(float *y, const float *x, int m, const orc_mlin *w) {
    if (w->wq)
        orc_matmul_q8_int(y, w->n, x, w->k, m, w->wq, w->n, w->k, w->b, 1);
    else
        orc_matmul_f32(y, w->n, x, w->k, w->wf, w->k, m, w->n, w->k, w->b);
}

/* nn.go:51-64: per chunk of 512 values, t = min(v, 0) through
 * ExpSub(t, 0) (EXP8 over the chunk's whole groups of eight, expf past
 * them), then v = max(v, 0) + (t - 1). */
void orc_elu(float *x, size_t n) {
    float t[512];
    for (size_t o = 0; o < n; o += 512) {
        int c = n - o < 512 ? (int)(n - o) : 512;
        for (int i = 0; i < c; i++) t[i] = x[o + i] < 0.0f ? x[o + i] : 0.0f;
        orc_expsub(t, c, 0.0f);
        for (int i = 0; i < c; i++) {
            float v = x[o + i];
            x[o + i] = (v > 0.0f ? v : 0.0f) + (t[i] - 1.0f);
        }
    }
}

int orc_mconv_past(const orc_mconv *c) { return (c->k - 1) * c->dil + 1 - c->stride; }

/* nn.go:272-296: T rows of x after the P rows prev holds (P = past()),
 * im2col rows t taking rows t*stride + j*dil, one Linear, prev updated;
 * T/stride rows into y.  k = 1 and stride 1: the Linear alone. */
static void mconv_run(const orc_mconv *c, float *y, float *prev, const float *x, int T) {
    int cin = c->cin, P = orc_mconv_past(c), To = T / c->stride;
    if (c->k == 1 && c->stride == 1) {
        mlin(y, x, T, &c->w);
        return;
    }
    float *buf = (float *)malloc((size_t)(P + T) * cin * sizeof(float));
    memcpy(buf, prev, (size_t)P * cin * sizeof(float));
    memcpy(buf + (size_t)P * cin, x, (size_t)T * cin * sizeof(float));
    int cols = c->k * cin;
    float *col = (float *)malloc((size_t)To * cols * sizeof(float));
    for (int t = 0; t < To; t++)
        for (int j = 0; j < c->k; j++)
            memcpy(col + (size_t)t * cols + (size_t)j * cin, buf + (size_t)(t * c->stride + j * c->dil) * cin,
                   (size_t)cin * sizeof(float));
    mlin(y, col, To, &c->w);
    memcpy(prev, buf + (size_t)T * cin, (size_t)P * cin * sizeof(float));
    free(buf);
    free(col);
}

/* nn.go:308-327: z = x . W (no bias), full rows from the bias, each input
 * row's k taps added in (t, then j, order), the carried partial added to
 * the first k - stride rows, the new partial = the last k - stride rows
 * minus the bias; T*stride rows into y. */
static void mconvtr_run(const orc_mconvtr *c, float *y, float *partial, const float *x, int T) {
    int co = c->cout, S = c->stride, K = c->k;
    float *z = (float *)malloc((size_t)T * K * co * sizeof(float));
    orc_mlin w = c->w;
    w.b = NULL;
    mlin(z, x, T, &w);
    int L = (T - 1) * S + K;
    float *full = (float *)malloc((size_t)L * co * sizeof(float));
    for (int i = 0; i < L; i++) memcpy(full + (size_t)i * co, c->w.b, (size_t)co * sizeof(float));
    for (int t = 0; t < T; t++)
        for (int j = 0; j < K; j++) {
            float *f = full + (size_t)(t * S + j) * co;
            const float *zz = z + ((size_t)t * K + j) * co;
            for (int e = 0; e < co; e++) f[e] = f[e] + zz[e];
        }
    int PT = K - S;
    for (int i = 0; i < PT * co; i++) full[i] = full[i] + partial[i];
    const float *tail = full + (size_t)(L - PT) * co;
    for (int i = 0; i < PT * co; i++) partial[i] = tail[i] - c->w.b[i % co];
    memcpy(y, full, (size_t)T * S * co * sizeof(float));
    free(z);
    free(full);
}

/* attend with a context limit (nn.go:200-254): each query p sees the keys
 * max(lo0, p - context + 1) .. p, lo0 = max(0, pos0 - context + 1) (no
 * limit: 0); the cache here keeps every row, which gives the same keys as
 * the reference's trimmed one. */
static void mimi_attend(const orc_mimi *m, float *out, const float *qkv, int T, const float *kc, const float *vc,
                        int pos0) {
    int d = m->d, hd = d / m->heads;
    float scale = (float)(1.0 / sqrt((double)hd));
    int lo0 = 0;
    if (m->context > 0 && pos0 - m->context + 1 > lo0) lo0 = pos0 - m->context + 1;
    int nk = pos0 + T - lo0;
    float *sc = (float *)malloc((size_t)T * nk * sizeof(float));
    float *vt = (float *)malloc((size_t)hd * nk * sizeof(float));
    for (int h = 0; h < m->heads; h++) {
        orc_matmul_f32(sc, nk, qkv + h * hd, 3 * d, kc + (size_t)lo0 * d + h * hd, d, T, nk, hd, NULL);
        for (int r = 0; r < T; r++) {
            int p = pos0 + r;
            int lo = lo0;
            if (m->context > 0 && p - m->context + 1 > lo) lo = p - m->context + 1;
            float *row = sc + (size_t)r * nk;
            float *s = row + (lo - lo0);
            int ns = p + 1 - lo;
            float mx = -INFINITY;
            for (int j = 0; j < ns; j++) {
                s[j] = s[j] * scale;
                mx = s[j] > mx ? s[j] : mx;
            }
            float inv = 1.0f / orc_expsub(s, ns, mx);
            for (int j = 0; j < ns; j++) s[j] = s[j] * inv;
            for (int j = 0; j < lo - lo0; j++) row[j] = 0;
            for (int j = p + 1 - lo0; j < nk; j++) row[j] = 0;
        }
        if (T < 4) {
            for (int r = 0; r < T; r++) {
                float *o = out + (size_t)r * d + h * hd;
                for (int e = 0; e < hd; e++) o[e] = 0;
                const float *row = sc + (size_t)r * nk;
                for (int j = 0; j < nk; j++)
                    if (row[j] != 0) orc_axpy(o, vc + (size_t)(lo0 + j) * d + h * hd, hd, row[j]);
            }
            continue;
        }
        for (int j = 0; j < nk; j++)
            for (int e = 0; e < hd; e++) vt[(size_t)e * nk + j] = vc[(size_t)(lo0 + j) * d + h * hd + e];
        orc_matmul_f32(out + h * hd, d, sc, nk, vt, nk, T, hd, nk, NULL);
    }
    free(sc);
    free(vt);
}

/* nn.go:185-196 (addScaled): x += s[i % n] * y, or kern.Add without s */
static void add_scaled(float *x, const float *y, const float *s, int n, size_t len) {
    for (size_t i = 0; i < len; i++) x[i] = s ? x[i] + s[i % n] * y[i] : x[i] + y[i];
}

/* nn.go:142-182 with the context limit and layer scales */
static int mimi_forward(const orc_mimi *m, orc_mimi_state *st, float *x, int T) {
    int d = m->d, ff = m->ff, hd = d / m->heads;
    if (st->pos + T > st->max_pos) return -1;
    float *h = (float *)malloc((size_t)T * d * sizeof(float));
    float *qkv = (float *)malloc((size_t)T * 3 * d * sizeof(float));
    float *att = (float *)malloc((size_t)T * d * sizeof(float));
    float *f = (float *)malloc((size_t)T * ff * sizeof(float));
    for (int li = 0; li < m->n_layer; li++) {
        const orc_mimi_layer *L = &m->layers[li];
        orc_layernorm_f64(h, x, T, d, L->norm1_w, L->norm1_b, 1e-5);
        mlin(qkv, h, T, &L->qkv);
        for (int r = 0; r < T; r++) {
            float *row = qkv + (size_t)r * 3 * d;
            orc_apply_rope(row, m->heads, m->freqs, hd / 2, st->pos + r);
            orc_apply_rope(row + d, m->heads, m->freqs, hd / 2, st->pos + r);
        }
        float *kc = st->k[li], *vc = st->v[li];
        for (int r = 0; r < T; r++) {
            memcpy(kc + (size_t)(st->pos + r) * d, qkv + (size_t)r * 3 * d + d, (size_t)d * sizeof(float));
            memcpy(vc + (size_t)(st->pos + r) * d, qkv + (size_t)r * 3 * d + 2 * d, (size_t)d * sizeof(float));
        }
        mimi_attend(m, att, qkv, T, kc, vc, st->pos);
        mlin(h, att, T, &L->out);
        add_scaled(x, h, L->ls1, d, (size_t)T * d);
        orc_layernorm_f64(h, x, T, d, L->norm2_w, L->norm2_b, 1e-5);
        mlin(f, h, T, &L->ff1);
        orc_gelu_vec(f, T * ff);
        mlin(h, f, T, &L->ff2);
        add_scaled(x, h, L->ls2, d, (size_t)T * d);
    }
    st->pos += T;
    free(h);
    free(qkv);
    free(att);
    free(f);
    return 0;
}

orc_mimi_state *orc_mimi_state_new(const orc_mimi *m, int max_pos) {
    orc_mimi_state *s = (orc_mimi_state *)calloc(1, sizeof *s);
    s->max_pos = max_pos;
    s->k = (float **)calloc((size_t)m->n_layer, sizeof(float *));
    s->v = (float **)calloc((size_t)m->n_layer, sizeof(float *));
    for (int i = 0; i < m->n_layer; i++) {
        s->k[i] = (float *)calloc((size_t)max_pos * m->d, sizeof(float));
        s->v[i] = (float *)calloc((size_t)max_pos * m->d, sizeof(float));
    }
    s->up_part = (float *)calloc((size_t)m->up_s * m->d, sizeof(float));
    /* newSeaState (mimi.go:44-60): one carried buffer per conv, convtr, and
     * two per residual block */
    int n = 0;
    for (int i = 0; i < m->n_steps; i++) n += m->steps[i].kind == 2 ? 2 : 1;
    s->n_prev = n;
    s->prev = (float **)calloc((size_t)n, sizeof(float *));
    int p = 0;
    for (int i = 0; i < m->n_steps; i++) {
        const orc_sea_step *q = &m->steps[i];
        if (q->kind == 0) {
            s->prev[p++] = (float *)calloc((size_t)(orc_mconv_past(&q->c) + 1) * q->c.cin, sizeof(float));
        } else if (q->kind == 1) {
            s->prev[p++] = (float *)calloc((size_t)(q->t.k - q->t.stride) * q->t.cout + 1, sizeof(float));
        } else {
            s->prev[p++] = (float *)calloc((size_t)(orc_mconv_past(&q->a) + 1) * q->a.cin, sizeof(float));
            s->prev[p++] = (float *)calloc((size_t)(orc_mconv_past(&q->b) + 1) * q->b.cin, sizeof(float));
        }
    }
    return s;
}

void orc_mimi_state_free(const orc_mimi *m, orc_mimi_state *s) {
    if (!s) return;
    for (int i = 0; i < m->n_layer; i++) {
        free(s->k[i]);
        free(s->v[i]);
    }
    free(s->k);
    free(s->v);
    free(s->up_part);
    for (int i = 0; i < s->n_prev; i++) free(s->prev[i]);
    free(s->prev);
    free(s);
}

/* mimi.go:62-108 (runSea) over T rows of C values; returns the output row
 * count, the rows in *out (malloc'd; the caller frees it). */
static int run_sea(const orc_mimi *m, orc_mimi_state *st, float *x, int T, int C, float **out) {
    int pi = 0;
    float *cur = (float *)malloc((size_t)T * C * sizeof(float));
    memcpy(cur, x, (size_t)T * C * sizeof(float));
    for (int i = 0; i < m->n_steps; i++) {
        const orc_sea_step *q = &m->steps[i];
        if (q->elu) orc_elu(cur, (size_t)T * C);
        if (q->kind == 0) {
            int To = T / q->c.stride;
            float *y = (float *)malloc((size_t)To * q->c.cout * sizeof(float));
            mconv_run(&q->c, y, st->prev[pi++], cur, T);
            free(cur);
            cur = y;
            T = To;
            C = q->c.cout;
        } else if (q->kind == 1) {
            int To = T * q->t.stride;
            float *y = (float *)malloc((size_t)To * q->t.cout * sizeof(float));
            mconvtr_run(&q->t, y, st->prev[pi++], cur, T);
            free(cur);
            cur = y;
            T = To;
            C = q->t.cout;
        } else {
            size_t n = (size_t)T * C;
            float *v = (float *)malloc(n * sizeof(float));
            memcpy(v, cur, n * sizeof(float));
            orc_elu(v, n);
            float *h = (float *)malloc((size_t)T * q->a.cout * sizeof(float));
            mconv_run(&q->a, h, st->prev[pi], v, T);
            orc_elu(h, (size_t)T * q->a.cout);
            float *o = (float *)malloc(n * sizeof(float));
            mconv_run(&q->b, o, st->prev[pi + 1], h, T);
            for (size_t e = 0; e < n; e++) cur[e] = cur[e] + o[e];
            pi += 2;
            free(v);
            free(h);
            free(o);
        }
    }
    *out = cur;
    return T;
}

/* mimi.go:122-152: n latents (already scaled back by the flow LM's mean
 * and std) to n * up_s * hop samples in out. */
int orc_mimi_decode(const orc_mimi *m, orc_mimi_state *st, const float *lat, int n, float *out, int *n_out) {
    int C = m->d, S = m->up_s, K = 2 * S;
    float *z = (float *)malloc((size_t)n * C * sizeof(float));
    mlin(z, lat, n, &m->quant);
    int L = (n - 1) * S + K;
    float *full = (float *)calloc((size_t)L * C, sizeof(float));
    for (int t = 0; t < n; t++)
        for (int c = 0; c < C; c++) {
            const float *w = m->up + (size_t)c * K;
            float v = z[(size_t)t * C + c];
            for (int j = 0; j < K; j++) {
                float *f = full + (size_t)(t * S + j) * C + c;
                *f = *f + v * w[j];
            }
        }
    for (int i = 0; i < S * C; i++) full[i] = full[i] + st->up_part[i];
    memcpy(st->up_part, full + (size_t)(L - S) * C, (size_t)S * C * sizeof(float));
    int T = n * S;
    int rc = mimi_forward(m, st, full, T);
    if (rc == 0) {
        float *y;
        int To = run_sea(m, st, full, T, C, &y);
        memcpy(out, y, (size_t)To * sizeof(float));  /* one channel */
        *n_out = To;
        free(y);
    }
    free(z);
    free(full);
    return rc;
}
