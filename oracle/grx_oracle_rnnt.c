/* CPU oracle (test infrastructure): greedy RNN-T / TDT decoding,
 * conformer/rnnt.go:46-173 of github.com/xattribution/gorelaxor, in the
 * reference's order of operations.  Linears of one activation row take
 * kern's float route (gemvRows with dot4q8avx / dotQ8Go), the encoder
 * projection of T >= 2 rows the int8 route (kern.go:189-192). */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "grx_oracle.h"

/* fdlibm e_exp.c: the double exp the decoder's tanh and softmax use here,
 * each operation rounded on its own (built with -ffp-contract=off). */
double orc_fd_exp(double x) {
    const double ln2hi = 6.93147180369123816490e-01, ln2lo = 1.90821492927058770002e-10;
    const double invln2 = 1.44269504088896338700e+00;
    const double P1 = 1.66666666666666019037e-01, P2 = -2.77777777770155933842e-03;
    const double P3 = 6.61375632143793436117e-05, P4 = -1.65339022054652515390e-06;
    const double P5 = 4.13813679705723846039e-08;
    if (x != x) return x;
    if (x > 7.09782712893383973096e+02) return INFINITY;
    if (x < -7.45133219101941108420e+02) return 0.0;
    uint64_t bits;
    memcpy(&bits, &x, 8);
    uint32_t hx = (uint32_t)(bits >> 32) & 0x7fffffffu;
    int neg = x < 0.0;
    double hi = 0.0, lo = 0.0;
    int k = 0;
    if (hx > 0x3fd62e42u) {
        if (hx < 0x3ff0a2b2u) {
            hi = neg ? x + ln2hi : x - ln2hi;
            lo = neg ? -ln2lo : ln2lo;
            k = neg ? -1 : 1;
        } else {
            k = (int)(invln2 * x + (neg ? -0.5 : 0.5));
            double t = (double)k;
            hi = x - t * ln2hi;
            lo = t * ln2lo;
        }
        x = hi - lo;
    } else if (hx < 0x3e300000u) {
        return 1.0 + x;
    }
    double t = x * x;
    double c = x - t * (P1 + t * (P2 + t * (P3 + t * (P4 + t * P5))));
    if (k == 0) return 1.0 - ((x * c) / (c - 2.0) - x);
    double y = 1.0 - ((lo - (x * c) / (2.0 - c)) - hi);
    return ldexp(y, k);
}

/* rnnt.go:43 (tanh32): float32(math.Tanh(float64(x))); Go's tanh is
 * Cephes': +-1 past half of log(2^127), 1 - 2/(e^(2|x|)+1) from 0.625 on,
 * the rational form x + x*s*P(s)/Q(s) below. */
float orc_tanh32(float xf) {
    double x = (double)xf, z = fabs(x), r;
    if (z > 0.5 * 8.8029691931113054295988e+01) {
        r = x < 0.0 ? -1.0 : 1.0;
    } else if (z >= 0.625) {
        double s = orc_fd_exp(2.0 * z);
        r = 1.0 - 2.0 / (s + 1.0);
        if (x < 0.0) r = -r;
    } else {
        if (x == 0.0) return xf;
        double s = x * x;
        double p = (-9.64399179425052238628e-1 * s + -9.92877231001918586564e1) * s + -1.61468768441708447952e3;
        double q = ((s + 1.12811678491632931402e2) * s + 2.23548839060100448583e3) * s + 4.84406305325125486048e3;
        r = x + x * s * p / q;
    }
    return (float)r;
}

/* conformer/encoder.go:13 */
static float sigm(float v) { return 1.0f / (1.0f + orc_expf(-v)); }

static void linear1(float *y, const float *x, const uint8_t *w, int n, int k, const float *bias) {
    orc_matmul_q8_float(y, n, x, k, 1, w, n, k, bias);
}

/* rnnt.go:47-68 (predict): from state (h, c, last) into (hn, cn); returns
 * the top layer's h (inside hn). */
static const float *predict(const orc_rnnt *m, const float *h, const float *c, int last, float *hn, float *cn,
                            float *gates, float *tmp, float *x0) {
    int H = m->H;
    memset(x0, 0, (size_t)H * 4);
    if (last >= 0 && last != m->blank) memcpy(x0, m->embed + (size_t)last * H, (size_t)H * 4);
    const float *x = x0;
    for (int l = 0; l < m->L; l++) {
        linear1(gates, x, m->wx[l], 4 * H, H, m->b[l]);
        linear1(tmp, h + (size_t)l * H, m->wh[l], 4 * H, H, NULL);
        for (int j = 0; j < 4 * H; j++) gates[j] = gates[j] + tmp[j];
        float *ho = hn + (size_t)l * H, *co = cn + (size_t)l * H;
        const float *ci = c + (size_t)l * H;
        for (int j = 0; j < H; j++) {
            float i = sigm(gates[j]);
            float f = sigm(gates[H + j]);
            float g = orc_tanh32(gates[2 * H + j]);
            float o = sigm(gates[3 * H + j]);
            co[j] = f * ci[j] + i * g;
            ho[j] = o * orc_tanh32(co[j]);
        }
        x = ho;
    }
    return x;
}

static int argmax(const float *v, int n) {
    int best = 0;
    for (int i = 0; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

/* rnnt.go:78-85 (softmaxAt) */
static float softmax_at(const float *v, int n, int i) {
    float mx = v[argmax(v, n)];
    double s = 0.0;
    for (int j = 0; j < n; j++) s += orc_fd_exp((double)(v[j] - mx));
    return (float)(orc_fd_exp((double)(v[i] - mx)) / s);
}

/* rnnt.go:111-173 (Decode). h, c ([L][H]) and *last hold the state on entry
 * and on return.  Returns the number of tokens (at most cap are written). */
int orc_rnnt_decode(const orc_rnnt *m, const float *enc, int T, float *h, float *c, int *last, int frame_offset,
                    orc_rnnt_token *out, int cap) {
    if (T == 0) return 0;
    const int H = m->H, L = m->L, J = m->J, V = m->V, R = m->V + (m->tdt ? m->nd : 0);
    float *ep = malloc((size_t)T * J * 4);
    if (T == 1)
        orc_matmul_q8_float(ep, J, enc, m->d, 1, m->jenc, J, m->d, m->jencb);
    else
        orc_matmul_q8_int(ep, J, enc, m->d, T, m->jenc, J, m->d, m->jencb, 1);
    size_t sb = (size_t)L * H;
    float *st = malloc(sb * 4 * 4); /* two slots of h then c */
    float *hs[2] = {st, st + 2 * sb}, *cs[2] = {st + sb, st + 3 * sb};
    int lastv[2] = {*last, -1};
    memcpy(hs[0], h, sb * 4);
    memcpy(cs[0], c, sb * 4);
    memset(hs[1], 0, sb * 4);
    memset(cs[1], 0, sb * 4);
    int cur = 0;
    float *gates = malloc((size_t)4 * H * 4), *tmp = malloc((size_t)4 * H * 4), *x0 = malloc((size_t)H * 4);
    float *hidden = malloc((size_t)J * 4), *pp = malloc((size_t)J * 4), *logits = malloc((size_t)R * 4);
    const float *pred = NULL;
    int dirty = 1, step = 0, newsym = 0, n = 0;
    long max_iters = 16L * T + 1024;
    for (long iter = 0; step < T && iter < max_iters; iter++) {
        if (dirty) {
            pred = predict(m, hs[cur], cs[cur], lastv[cur], hs[1 - cur], cs[1 - cur], gates, tmp, x0);
            dirty = 0;
        }
        /* joint (rnnt.go:90-106) */
        linear1(pp, pred, m->jpred, J, H, m->jpredb);
        const float *e = ep + (size_t)step * J;
        for (int i = 0; i < J; i++) {
            float v = e[i] + pp[i];
            if (m->act == 1) v = sigm(v);
            else if (m->act == 2) v = orc_tanh32(v);
            else v = v != v ? v : (v > 0.0f ? v : 0.0f);
            hidden[i] = v;
        }
        linear1(logits, hidden, m->jout, R, J, m->joutb);
        int tok = argmax(logits, V);
        int blank = tok == m->blank;
        int duration = 1;
        if (m->tdt) duration = m->dur[argmax(logits + V, m->nd)];
        if (!blank) {
            if (n < cap) {
                out[n].id = tok;
                out[n].frame = frame_offset + step;
                out[n].duration = duration;
                out[n].p = softmax_at(logits, V, tok);
            }
            n++;
            lastv[1 - cur] = tok;
            cur = 1 - cur;
            dirty = 1;
        }
        if (!m->tdt) {
            if (blank) {
                step++;
                newsym = 0;
            } else if (++newsym, m->max_symbols > 0 && newsym >= m->max_symbols) {
                step++;
                newsym = 0;
            }
            continue;
        }
        step += duration;
        newsym++;
        if (duration != 0) {
            newsym = 0;
        } else if (m->max_symbols > 0 && newsym >= m->max_symbols) {
            step++;
            newsym = 0;
        }
    }
    memcpy(h, hs[cur], sb * 4);
    memcpy(c, cs[cur], sb * 4);
    *last = lastv[cur];
    free(ep);
    free(st);
    free(gates);
    free(tmp);
    free(x0);
    free(hidden);
    free(pp);
    free(logits);
    return n;
}
