/*
 * grx_oracle_conformer.c - CPU restatement of gorelaxor's FastConformer
 * encoder forward (package conformer) with Q8_0 weights.
 *
 * TEST INFRASTRUCTURE ONLY (see grx_oracle.h): the checker for the HIP
 * encoder, never called by the product.
 *
 * The offline (whole-recording) encoder of conformer/encoder.go with the
 * settings of a non-streaming FastConformer: pre-encoder padding 1 on each
 * side, full attention in query blocks of 32, a centred depthwise
 * convolution.  Every Linear takes the int8 route (conformer/model.go:
 * 348-356 packs and drops the rows of every encoder weight).  Vector
 * kernels follow the AVX assembly a VNNI host runs for whole groups of
 * eight and the Go twin for the rest, as kernels_amd64.go dispatches them.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "grx_oracle.h"

/* Go's builtin max for float32 (NaN wins, +0 over -0). */
static inline float go_max(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a == b) return signbit(a) ? b : a;
    return a > b ? a : b;
}

/* reluVec (kernels_amd64.go:263-273): VMAXPS returns x unless 0 is larger;
 * reluGo zeroes v < 0.  Both keep -0 and NaN. */
static void relu_vec(float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (x[i] < 0.0f) x[i] = 0.0f;
}

/* kern.Add (mathx.go:102-107). */
static void add_vec(float *dst, const float *src, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = dst[i] + src[i];
}

static void axpy_big(float *dst, const float *src, size_t n, float s) {
    /* axpy over a whole buffer: the AVX part covers n &^ 7 of it */
    size_t n8 = n & ~(size_t)7;
    for (size_t i = 0; i < n8; i++) dst[i] = fmaf(s, src[i], dst[i]);
    for (size_t i = n8; i < n; i++) dst[i] = dst[i] + s * src[i];
}

static void silu_big(float *x, size_t n) {
    size_t n8 = n & ~(size_t)7;
    for (size_t i = 0; i < n8; i++) {
        float v = x[i];
        float e = orc_exp8(0.0f - v);
        x[i] = v / (e + 1.0f);
    }
    for (size_t i = n8; i < n; i++) {
        float v = x[i];
        x[i] = v / (1.0f + orc_expf(-v));
    }
}

static void linear(float *y, const float *x, int m, const uint8_t *w, int n, int k, const float *bias) {
    if (m > 0) orc_matmul_q8_int(y, n, x, k, m, w, n, k, bias, 1);
}

/* kern.Linear of a float32 weight (kern.go:185-201): ws.matmul, gemm.go:116-185 */
static void linear_f32(float *y, const float *x, int m, const float *w, int n, int k, const float *bias) {
    if (m > 0) orc_matmul_f32(y, n, x, k, w, k, m, n, k, bias);
}

/* encoder.go:33-38 (subOut): causal models pad two before and one after,
 * the others one on each side. */
static inline int sub_out(int n, int causal) { return causal ? n / 2 + 1 : (n - 1) / 2 + 1; }

/* encoder.go:171-191 (relPosEmb, relPosRange): rows for relative positions
 * n-1 down to -(n-1); div_j = f32(exp(j * -(ln(10000)/d))), angle =
 * f64(f32(pos) * div_j), even columns f32(sin), odd f32(cos). */
void orc_conf_rel_pos(float *out, int n, int d) {
    int count = 2 * n - 1;
    for (int i = 0; i < count; i++) {
        double pos = (double)(n - 1 - i);
        float *row = out + (size_t)i * d;
        for (int j = 0; j < d; j += 2) {
            float div = (float)exp((double)j * -(log(10000.0) / (double)d));
            double a = (double)((float)pos * div);
            row[j] = (float)sin(a);
            if (j + 1 < d) row[j + 1] = (float)cos(a);
        }
    }
}

/* conformer/model.go:405-419: batch norm folded to a scale and a bias,
 * s = f32(f64(gamma) / sqrt(f64(var) + 1e-5)), b = beta - mean*s. */
void orc_conf_bn_fold(const float *gw, const float *gb, const float *mean, const float *var, int d, float *s,
                      float *b) {
    for (int j = 0; j < d; j++) {
        float sj = (float)((double)gw[j] / sqrt((double)var[j] + 1e-5));
        s[j] = sj;
        float ms = mean[j] * sj;
        b[j] = gb[j] - ms;
    }
}

/* encoder.go:41-77 (conv0): one plane [T][F] to c channels [T1][F1][c];
 * each output starts from the bias and takes AddScaled of the nine taps in
 * order, taps equal to 0 skipped. */
static float *conv0(const float *in, int T, int F, const float *w, const float *b, int c, int causal, int *T1o,
                    int *F1o) {
    int T1 = sub_out(T, causal), F1 = sub_out(F, causal), pl = causal ? 2 : 1;
    float *out = (float *)malloc((size_t)T1 * F1 * c * sizeof(float));
    for (int t = 0; t < T1; t++)
        for (int f = 0; f < F1; f++) {
            float taps[9];
            for (int kt = 0; kt < 3; kt++)
                for (int kf = 0; kf < 3; kf++) {
                    int ti = 2 * t + kt - pl, fi = 2 * f + kf - pl;
                    taps[kt * 3 + kf] = (ti >= 0 && ti < T && fi >= 0 && fi < F) ? in[(size_t)ti * F + fi] : 0.0f;
                }
            float *o = out + ((size_t)t * F1 + f) * c;
            memcpy(o, b, (size_t)c * sizeof(float));
            for (int j = 0; j < 9; j++)
                if (taps[j] != 0.0f) orc_axpy(o, w + (size_t)j * c, c, taps[j]);
        }
    *T1o = T1;
    *F1o = F1;
    return out;
}

/* encoder.go:80-110 (dwConv2): depthwise 3x3 stride 2 on [T][F][c]; each
 * output starts from the bias and adds w*x (unfused) over the taps in
 * range, in order. */
static float *dw_conv2(const float *in, int T, int F, int c, const float *w, const float *b, int causal, int *T1o,
                       int *F1o) {
    int T1 = sub_out(T, causal), F1 = sub_out(F, causal), pl = causal ? 2 : 1;
    float *out = (float *)malloc((size_t)T1 * F1 * c * sizeof(float));
    for (int t = 0; t < T1; t++)
        for (int f = 0; f < F1; f++) {
            float *o = out + ((size_t)t * F1 + f) * c;
            memcpy(o, b, (size_t)c * sizeof(float));
            for (int kt = 0; kt < 3; kt++) {
                int ti = 2 * t + kt - pl;
                if (ti < 0 || ti >= T) continue;
                for (int kf = 0; kf < 3; kf++) {
                    int fi = 2 * f + kf - pl;
                    if (fi < 0 || fi >= F) continue;
                    const float *x = in + ((size_t)ti * F + fi) * c;
                    const float *wk = w + (size_t)(kt * 3 + kf) * c;
                    for (int i = 0; i < c; i++) o[i] = o[i] + wk[i] * x[i];
                }
            }
        }
    *T1o = T1;
    *F1o = F1;
    return out;
}

/* encoder.go:114-118 (maskRows). */
static void mask_rows(float *x, int rows, int valid, size_t width) {
    if (valid < rows) {
        int v = valid > 0 ? valid : 0;
        memset(x + (size_t)v * width, 0, (size_t)(rows - v) * width * sizeof(float));
    }
}

/* encoder.go:123-167 (subsample): log-mel [mels][frames] (the first valid
 * frames real) through conv0, ReLU, depthwise, pointwise, ReLU, depthwise,
 * pointwise, ReLU (rows past the valid length zeroed before each step),
 * flattened to [t][c*F+f] and the output Linear: out [T][d]. */
int orc_conf_subsample(const orc_conformer *m, const float *mel, int frames, int valid, float *out, int *T_out,
                       int *L_out) {
    int nm = m->n_mels, c = m->sub_channels;
    float *in = (float *)calloc((size_t)frames * nm, sizeof(float));
    int tv = frames < valid ? frames : valid;
    for (int f = 0; f < nm; f++)
        for (int t = 0; t < tv; t++) in[(size_t)t * nm + f] = mel[(size_t)f * frames + t];
    int T, F, L = valid, cs = m->causal_sub;
    float *x = conv0(in, frames, nm, m->w0, m->b0, c, cs, &T, &F);
    free(in);
    L = sub_out(L, cs);
    mask_rows(x, T, L, (size_t)F * c);
    relu_vec(x, (size_t)T * F * c);
    int T2, F2;
    float *x2 = dw_conv2(x, T, F, c, m->w2, m->b2, cs, &T2, &F2);
    free(x);
    T = T2, F = F2;
    L = sub_out(L, cs);
    mask_rows(x2, T, L, (size_t)F * c);
    float *y = (float *)malloc((size_t)T * F * c * sizeof(float));
    if (m->w3f)
        linear_f32(y, x2, T * F, m->w3f, c, c, m->b3);
    else
        linear(y, x2, T * F, m->w3, c, c, m->b3);
    free(x2);
    mask_rows(y, T, L, (size_t)F * c);
    relu_vec(y, (size_t)T * F * c);
    float *x3 = dw_conv2(y, T, F, c, m->w5, m->b5, cs, &T2, &F2);
    free(y);
    T = T2, F = F2;
    L = sub_out(L, cs);
    mask_rows(x3, T, L, (size_t)F * c);
    y = (float *)malloc((size_t)T * F * c * sizeof(float));
    if (m->w6f)
        linear_f32(y, x3, T * F, m->w6f, c, c, m->b6);
    else
        linear(y, x3, T * F, m->w6, c, c, m->b6);
    free(x3);
    mask_rows(y, T, L, (size_t)F * c);
    relu_vec(y, (size_t)T * F * c);
    float *flat = (float *)malloc((size_t)T * c * F * sizeof(float));
    for (int t = 0; t < T; t++)
        for (int f = 0; f < F; f++)
            for (int ch = 0; ch < c; ch++) flat[(size_t)t * c * F + (size_t)ch * F + f] = y[((size_t)t * F + f) * c + ch];
    free(y);
    linear(out, flat, T, m->out, m->d, c * F, m->out_b);
    free(flat);
    *T_out = T;
    *L_out = L < 0 ? 0 : (L < T ? L : T);
    return 0;
}

/* encoder.go:244-251 (feedForward): x += 0.5 * W2 . SiLU(W1 . LN(x)). */
static void feed_forward(const orc_conformer *m, const orc_conf_ff *w, float *x, int T, float *ln, float *ff,
                         float *tmp) {
    int d = m->d, dff = m->dff;
    orc_layernorm(ln, x, T, d, w->norm_w, w->norm_b);
    linear(ff, ln, T, w->w1, dff, d, w->b1);
    silu_big(ff, (size_t)T * dff);
    linear(tmp, ff, T, w->w2, d, dff, w->b2);
    axpy_big(x, tmp, (size_t)T * d, 0.5f);
}

/* keyRange (encoder.go:193-212) cut at the valid length L (encoder.go:
 * 465-472), and a streaming chunk's keys (stream.go:273-287, its two loops
 * as written). */
void orc_conf_key_range(const orc_keys *k, int q, int *lo, int *hi) {
    if (k->mode == ORC_KEYS_STREAM) {
        if (q - k->c >= k->L) {
            *lo = *hi = 0;
            return;
        }
        int qc = (k->slot0 + q) / k->chunk;
        int l = 0;
        while (l < k->c + k->Tc && qc - (k->slot0 + l) / k->chunk > k->left_chunks) l++;
        int h = k->c + k->L;
        while (h > l && (k->slot0 + h - 1) / k->chunk > qc) h--;
        *lo = l;
        *hi = h;
        return;
    }
    if (q >= k->L) {
        *lo = *hi = 0;
        return;
    }
    int l = 0, h = k->T;
    if (k->mode == ORC_KEYS_CHUNKED) {
        int c = q / k->chunk;
        l = (c - k->left_chunks) * k->chunk;
        l = l > 0 ? l : 0;
        h = (c + 1) * k->chunk;
        h = h < k->T ? h : k->T;
    } else if (k->mode == ORC_KEYS_WINDOW) {
        l = q - k->left > 0 ? q - k->left : 0;
        h = q + k->right + 1 < k->T ? q + k->right + 1 : k->T;
    }
    *lo = l;
    *hi = h < k->L ? h : k->L;
}

/* offlineKeys (encoder.go:196-212): chunked limited context for a
 * streaming model with both limits (blocks of one chunk), a window for a
 * regular one whose limits are shorter than the recording (blocks of 16),
 * else every key (blocks of 32). */
int orc_conf_offline_keys(const orc_conformer *m, int T, int L, orc_keys *k) {
    memset(k, 0, sizeof(*k));
    k->T = T;
    k->L = L;
    int al = m->att_left, ar = m->att_right;
    int mn = al < ar ? al : ar;
    if (m->att_style == 1 && al >= 0 && ar >= 0) {
        k->mode = ORC_KEYS_CHUNKED;
        k->chunk = ar + 1;
        k->left_chunks = al / k->chunk;
        return k->chunk;
    }
    if (al >= 0 && ar >= 0 && T - 1 > mn) {
        k->mode = ORC_KEYS_WINDOW;
        k->left = al;
        k->right = ar;
        return 16;
    }
    k->mode = ORC_KEYS_ALL;
    return 32;
}

/* convPadLeft (encoder.go:399-404). */
int orc_conf_pad_left(const orc_conformer *m) {
    if (m->conv_left >= 0 && m->conv_right >= 0) return m->conv_left;
    return (m->conv_kernel - 1) / 2;
}

/* encoder.go:259-330 (attention): queries are the T normalized rows ln,
 * keys and values come from the Tk rows kv (the queries' own rows last, so
 * query i is key Tk-T+i); pp holds the projected position rows for
 * relative positions Tk-1 down to -(T-1).  Queries go in blocks of bl, each
 * block's keys the union of its rows' ranges. */
static void attention(const orc_conformer *m, const orc_conf_block *b, float *x, const float *ln, const float *kv,
                      int T, int Tk, const float *pp, const orc_keys *keys, int bl) {
    int D = m->d, H = m->heads, hd = D / H;
    size_t TD = (size_t)T * D, KD = (size_t)Tk * D;
    float *q = (float *)malloc(TD * sizeof(float)), *k = (float *)malloc(KD * sizeof(float));
    float *v = (float *)malloc(KD * sizeof(float)), *qu = (float *)malloc(TD * sizeof(float));
    float *qv = (float *)malloc(TD * sizeof(float)), *vt = (float *)malloc(KD * sizeof(float));
    float *glu = (float *)malloc(TD * sizeof(float)), *att = (float *)malloc(TD * sizeof(float));
    linear(q, ln, T, b->q, D, D, b->q_b);
    linear(k, kv, Tk, b->k, D, D, b->k_b);
    linear(v, kv, Tk, b->v, D, D, b->v_b);
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++)
            for (int j = 0; j < hd; j++) {
                size_t o = (size_t)t * D + h * hd + j;
                qu[o] = q[o] + b->pos_u[h * hd + j];
                qv[o] = q[o] + b->pos_v[h * hd + j];
            }
    for (int t = 0; t < Tk; t++)
        for (int c = 0; c < D; c++) vt[(size_t)c * Tk + t] = v[(size_t)t * D + c];
    const float scale = (float)(1.0 / sqrt((double)hd));
    const int nblk = (T + bl - 1) / bl, qoff = Tk - T;
    for (int h = 0; h < H; h++)
        for (int blk = 0; blk < nblk; blk++) {
            int q0 = blk * bl, q1 = (blk + 1) * bl < T ? (blk + 1) * bl : T, nq = q1 - q0;
            int k0 = Tk, k1 = 0;
            for (int qq = q0; qq < q1; qq++) {
                int lo, hi;
                orc_conf_key_range(keys, qoff + qq, &lo, &hi);
                k0 = lo < k0 ? lo : k0;
                k1 = hi > k1 ? hi : k1;
            }
            int nk = k1 - k0;
            if (nk <= 0) {
                for (int i = q0; i < q1; i++) memset(glu + (size_t)i * D + h * hd, 0, (size_t)hd * sizeof(float));
                continue;
            }
            int np = nq + nk - 1;
            int jlo = Tk - 1 - (qoff + q1 - 1) + k0;
            float *sc = (float *)malloc((size_t)nq * nk * sizeof(float));
            float *bd = (float *)malloc((size_t)nq * np * sizeof(float));
            orc_matmul_f32(sc, nk, qu + (size_t)q0 * D + h * hd, D, k + (size_t)k0 * D + h * hd, D, nq, nk, hd, NULL);
            orc_matmul_f32(bd, np, qv + (size_t)q0 * D + h * hd, D, pp + (size_t)jlo * D + h * hd, D, nq, np, hd,
                           NULL);
            for (int i = 0; i < nq; i++) {
                float *row = sc + (size_t)i * nk;
                const float *brow = bd + (size_t)i * np + (nq - 1 - i);
                int lo, hi;
                orc_conf_key_range(keys, qoff + q0 + i, &lo, &hi);
                float mx = -INFINITY;
                for (int kk = 0; kk < nk; kk++) {
                    int kx = k0 + kk;
                    if (kx < lo || kx >= hi) {
                        row[kk] = -INFINITY;
                        continue;
                    }
                    float s = (row[kk] + brow[kk]) * scale;
                    row[kk] = s;
                    mx = go_max(mx, s);
                }
                if (isinf(mx) && mx < 0) {
                    memset(row, 0, (size_t)nk * sizeof(float));
                    continue;
                }
                float sum = orc_expsub(row, nk, mx);
                float inv = 1.0f / sum;
                for (int kk = 0; kk < nk; kk++) row[kk] = row[kk] * inv;
            }
            orc_matmul_f32(glu + (size_t)q0 * D + h * hd, D, sc, nk, vt + (size_t)h * hd * Tk + k0, Tk, nq, hd, nk,
                           NULL);
            free(sc);
            free(bd);
        }
    linear(att, glu, T, b->out, D, D, b->out_b);
    add_vec(x, att, TD);
    free(q), free(k), free(v), free(qu), free(qv), free(vt), free(glu), free(att);
}

/* encoder.go:343-397 (convModule): pointwise to 2D, GLU a*sigmoid(b)
 * (sigmoid = 1/(1+expf(-v)), rows from valid on zeroed), depthwise taps at
 * t+j-padL from the bias (unfused w*x sums in tap order; taps before the
 * first frame read prev, the padL gated frames before it, or are skipped
 * when there is none), the folded batch norm (r*s + b, unfused) or a
 * LayerNorm, SiLU, pointwise back to D, added to x.  The gated frames are
 * left in glu_out [T][D] when it is given. */
static void conv_module(const orc_conformer *m, const orc_conf_block *b, float *x, const float *ln, int T, int valid,
                        int padL, const float *prev, float *glu_out) {
    int D = m->d, K = m->conv_kernel;
    size_t TD = (size_t)T * D;
    float *conv = (float *)malloc(2 * TD * sizeof(float));
    float *glu = (float *)malloc(TD * sizeof(float)), *dw = (float *)malloc(TD * sizeof(float));
    linear(conv, ln, T, b->pw1, 2 * D, D, b->pw1_b);
    for (int t = 0; t < T; t++) {
        const float *a = conv + (size_t)t * 2 * D;
        float *g = glu + (size_t)t * D;
        if (t >= valid) {
            memset(g, 0, (size_t)D * sizeof(float));
            continue;
        }
        for (int c = 0; c < D; c++) {
            float sg = 1.0f / (1.0f + orc_expf(-a[D + c]));
            g[c] = a[c] * sg;
        }
    }
    for (int t = 0; t < T; t++) {
        float *o = dw + (size_t)t * D;
        if (b->dw_b)
            memcpy(o, b->dw_b, (size_t)D * sizeof(float));
        else
            memset(o, 0, (size_t)D * sizeof(float));
        for (int j = 0; j < K; j++) {
            int ti = t + j - padL;
            const float *src;
            if (ti >= 0 && ti < T)
                src = glu + (size_t)ti * D;
            else if (ti < 0 && prev != NULL && padL + ti >= 0)
                src = prev + (size_t)(padL + ti) * D;
            else
                continue;
            const float *w = b->dw + (size_t)j * D;
            for (int c = 0; c < D; c++) o[c] = o[c] + w[c] * src[c];
        }
    }
    if (m->conv_ln) {
        orc_layernorm(dw, dw, T, D, b->cn_w, b->cn_b);
    } else {
        for (int t = 0; t < T; t++) {
            float *r = dw + (size_t)t * D;
            for (int c = 0; c < D; c++) {
                float p = r[c] * b->cn_w[c];
                r[c] = p + b->cn_b[c];
            }
        }
    }
    silu_big(dw, TD);
    linear(conv, dw, T, b->pw2, D, D, b->pw2_b);
    add_vec(x, conv, TD);
    if (glu_out) memcpy(glu_out, glu, TD * sizeof(float));
    free(conv), free(glu), free(dw);
}

/* encoder.go:411-429 (runBlock): kv_before holds c earlier normalized
 * attention inputs (streaming; none offline), conv_prev the gated frames
 * before this call's first frame (NULL offline).  kv_out (when given)
 * receives the c + T key rows, glu_out the gated frames. */
static void run_block(const orc_conformer *m, int i, float *x, int T, int L, const float *pp, const float *kv_before,
                      int c, const float *conv_prev, const orc_keys *keys, int bl, float *kv_out, float *glu_out) {
    const orc_conf_block *b = &m->blocks[i];
    int D = m->d;
    size_t TD = (size_t)T * D;
    float *ln = (float *)malloc(TD * sizeof(float));
    float *ff = (float *)malloc((size_t)T * m->dff * sizeof(float));
    float *tmp = (float *)malloc(TD * sizeof(float));
    float *kv = (float *)malloc((size_t)(c + T) * D * sizeof(float));
    feed_forward(m, &b->ff1, x, T, ln, ff, tmp);
    orc_layernorm(ln, x, T, D, b->norm_attn_w, b->norm_attn_b);
    if (c > 0) memcpy(kv, kv_before, (size_t)c * D * sizeof(float));
    memcpy(kv + (size_t)c * D, ln, TD * sizeof(float));
    attention(m, b, x, ln, kv, T, c + T, pp, keys, bl);
    orc_layernorm(ln, x, T, D, b->norm_conv_w, b->norm_conv_b);
    conv_module(m, b, x, ln, T, L, orc_conf_pad_left(m), conv_prev, glu_out);
    feed_forward(m, &b->ff2, x, T, ln, ff, tmp);
    orc_layernorm(x, x, T, D, b->norm_out_w, b->norm_out_b);
    if (kv_out) memcpy(kv_out, kv, (size_t)(c + T) * D * sizeof(float));
    free(ln), free(ff), free(tmp), free(kv);
}

/* One block offline (encoder.go:474-486): its position projection pp =
 * pos . Wpos^T (pos: relPosEmb(T)), the offline keys, runBlock. */
int orc_conf_block_run(const orc_conformer *m, int i, float *x, int T, int L, const float *pos) {
    int D = m->d, np = 2 * T - 1;
    float *pp = (float *)malloc((size_t)np * D * sizeof(float));
    linear(pp, pos, np, m->blocks[i].pos, D, D, NULL);
    orc_keys keys;
    int bl = orc_conf_offline_keys(m, T, L, &keys);
    run_block(m, i, x, T, L, pp, NULL, 0, NULL, &keys, bl, NULL, NULL);
    free(pp);
    return 0;
}

/* encoder.go:432-489 (encode, xscale, encodeEmbeddings) for layers
 * [0, n_layers): the pre-encoder, x *= f32(sqrt(d)) when the model scales,
 * the relative position table, each block.  out receives all T rows (the
 * first L are the result); T and L are returned. */
int orc_conformer_encode(const orc_conformer *m, const float *mel, int frames, int valid, int n_layers, float *out,
                         int *T_out, int *L_out) {
    int T, L;
    if (frames < 1) return -1;
    orc_conf_subsample(m, mel, frames, valid, out, &T, &L);
    int D = m->d;
    if (m->xscaling) {
        float s = (float)sqrt((double)D);
        for (size_t i = 0; i < (size_t)T * D; i++) out[i] = out[i] * s;
    }
    float *pos = (float *)malloc((size_t)(2 * T - 1) * D * sizeof(float));
    orc_conf_rel_pos(pos, T, D);
    for (int i = 0; i < n_layers && i < m->layers; i++) orc_conf_block_run(m, i, out, T, L, pos);
    free(pos);
    *T_out = T;
    *L_out = L;
    return 0;
}

/* relPosRange (encoder.go:183-191): count rows for positions first,
 * first-1, ... */
static void rel_pos_range(float *out, int first, int count, int d) {
    for (int i = 0; i < count; i++) {
        double pos = (double)(first - i);
        float *row = out + (size_t)i * d;
        for (int j = 0; j < d; j += 2) {
            float div = (float)exp((double)j * -(log(10000.0) / (double)d));
            double a = (double)((float)pos * div);
            row[j] = (float)sin(a);
            if (j + 1 < d) row[j + 1] = (float)cos(a);
        }
    }
}

/* newGeom's chunking and position tables (stream.go:23-69) for a right
 * context and the left context the model pairs with it, and newEncState
 * (stream.go:80-88): empty attention caches, zero convolution caches. */
orc_conf_stream *orc_conf_stream_new(const orc_conformer *m, int right, int left, int drop) {
    orc_conf_stream *s = (orc_conf_stream *)calloc(1, sizeof(orc_conf_stream));
    int D = m->d, padL = orc_conf_pad_left(m);
    s->right = right;
    s->chunk = right + 1;
    s->left = left;
    s->left_chunks = left / s->chunk;
    s->drop = drop;
    int first = left + s->chunk - 1, count = left + 2 * s->chunk - 1;
    float *pos = (float *)malloc((size_t)count * D * sizeof(float));
    rel_pos_range(pos, first, count, D);
    s->kv = (float **)calloc((size_t)m->layers, sizeof(float *));
    s->conv = (float **)calloc((size_t)m->layers, sizeof(float *));
    s->pos_proj = (float **)calloc((size_t)m->layers, sizeof(float *));
    for (int i = 0; i < m->layers; i++) {
        s->kv[i] = (float *)calloc((size_t)(left > 0 ? left : 1) * D, sizeof(float));
        s->conv[i] = (float *)calloc((size_t)(padL > 0 ? padL : 1) * D, sizeof(float));
        s->pos_proj[i] = (float *)malloc((size_t)count * D * sizeof(float));
        linear(s->pos_proj[i], pos, count, m->blocks[i].pos, D, D, NULL);
    }
    free(pos);
    return s;
}

void orc_conf_stream_free(const orc_conformer *m, orc_conf_stream *s) {
    if (!s) return;
    for (int i = 0; i < m->layers; i++) free(s->kv[i]), free(s->conv[i]), free(s->pos_proj[i]);
    free(s->kv), free(s->conv), free(s->pos_proj);
    free(s);
}

/* streamStep (stream.go:241-245) and streamEncode (stream.go:249-307): the
 * pre-encoder over the chunk, the first drop rows cut from every chunk but
 * the first, xscale, then each block with the stream's caches: keys are
 * the cached rows and the chunk's own, limited per NeMo's fixed-size cache
 * slots; afterwards each layer keeps its last `left` key rows and its last
 * padL gated frames. */
int orc_conf_stream_step(const orc_conformer *m, orc_conf_stream *s, const float *mel, int nf, int length, int first,
                         float *out, int *L_out) {
    int D = m->d, T, L;
    *L_out = 0;
    if (nf < 1) return 0;
    int Tfull = nf;
    for (int k = 0; k < 3; k++) Tfull = sub_out(Tfull, m->causal_sub);
    float *xs = (float *)malloc((size_t)Tfull * D * sizeof(float));
    orc_conf_subsample(m, mel, nf, length, xs, &T, &L);
    float *x = xs;
    if (!first) {
        int dr = s->drop < T ? s->drop : T;
        x = xs + (size_t)dr * D;
        T = T - s->drop > 0 ? T - s->drop : 0;
        L = L - s->drop > 0 ? L - s->drop : 0;
    }
    L = L < T ? L : T;
    if (T <= 0) {
        free(xs);
        return 0;
    }
    int c = s->kv_len, Tk = c + T, maxFirst = s->left + s->chunk - 1, padL = orc_conf_pad_left(m);
    if (Tk - 1 > maxFirst) {
        free(xs);
        return -1; /* the position table ends at left+chunk-1 */
    }
    if (m->xscaling) {
        float sc = (float)sqrt((double)D);
        for (size_t i = 0; i < (size_t)T * D; i++) x[i] = x[i] * sc;
    }
    orc_keys keys;
    memset(&keys, 0, sizeof(keys));
    keys.mode = ORC_KEYS_STREAM;
    keys.L = L;
    keys.chunk = s->chunk;
    keys.left_chunks = s->left_chunks;
    keys.c = c;
    keys.slot0 = s->left - c;
    keys.Tc = T;
    float *kv = (float *)malloc((size_t)Tk * D * sizeof(float));
    float *glu = (float *)malloc((size_t)T * D * sizeof(float));
    float *all = (float *)malloc((size_t)(padL + T) * D * sizeof(float));
    for (int i = 0; i < m->layers; i++) {
        const float *pp = s->pos_proj[i] + (size_t)(maxFirst - (Tk - 1)) * D;
        run_block(m, i, x, T, L, pp, s->kv[i], c, s->conv[i], &keys, T, kv, glu);
        int keep = Tk < s->left ? Tk : s->left;
        if (keep > 0) memcpy(s->kv[i], kv + (size_t)(Tk - keep) * D, (size_t)keep * D * sizeof(float));
        if (padL > 0) {
            memcpy(all, s->conv[i], (size_t)padL * D * sizeof(float));
            memcpy(all + (size_t)padL * D, glu, (size_t)T * D * sizeof(float));
            memcpy(s->conv[i], all + (size_t)T * D, (size_t)padL * D * sizeof(float));
        }
    }
    s->kv_len = Tk < s->left ? Tk : s->left;
    memcpy(out, x, (size_t)L * D * sizeof(float));
    *L_out = L;
    free(kv), free(glu), free(all), free(xs);
    return 0;
}
