/* CPU oracle (test infrastructure only) of whisper's token rules and sampler:
 * session.process and session.sample, whisper/transcribe.go:370-494, with
 * logSoftmax (:495-515) and softmaxInf (:517-536), restated line by line in
 * plain sequential C: every sum left to right in float32, every product,
 * quotient and difference rounded on its own.  The log of a sum is
 * float32(log(double)), as the reference forms it with math.Log. */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "grx_oracle.h"

static void log_softmax(float *dst, const float *x, int n) {
    float mx = -INFINITY;
    for (int i = 0; i < n; i++) mx = x[i] > mx ? x[i] : mx;
    float s = 0.0f;
    for (int i = 0; i < n; i++)
        if (x[i] > -INFINITY) s = s + orc_expf(x[i] - mx);
    float ls = (float)log((double)s) + mx;
    for (int i = 0; i < n; i++) dst[i] = x[i] > -INFINITY ? x[i] - ls : -INFINITY;
}

static void softmax_inf(float *x, int n) {
    float mx = -INFINITY;
    for (int i = 0; i < n; i++) mx = x[i] > mx ? x[i] : mx;
    float s = 0.0f;
    for (int i = 0; i < n; i++) {
        if (x[i] > -INFINITY) {
            float e = orc_expf(x[i] - mx);
            x[i] = e;
            s = s + e;
        } else {
            x[i] = 0.0f;
        }
    }
    for (int i = 0; i < n; i++) x[i] = x[i] / s;
}

void orc_whisper_sample(const float *logits, int n, const orc_whisper_rules *v, const orc_whisper_seq *q,
                        float temp, float r, orc_whisper_token *out) {
    float *lg = (float *)malloc((size_t)n * sizeof(float));
    float *lp = (float *)malloc((size_t)n * sizeof(float));
    memcpy(lg, logits, (size_t)n * sizeof(float));
    /* process() */
    if (temp > 0)
        for (int i = 0; i < n; i++) lg[i] = lg[i] / temp;
    int initial = q->n_tokens == 0;
    if (initial) {
        lg[v->eot] = -INFINITY;
        if (v->space >= 0) lg[v->space] = -INFINITY;
    }
    lg[v->no_timestamps] = -INFINITY;
    lg[v->sot] = lg[v->nosp] = lg[v->solm] = -INFINITY;
    lg[v->translate] = lg[v->transcribe] = lg[v->prev] = -INFINITY;
    for (int i = 0; i < v->n_lang; i++) lg[v->sot + 1 + i] = -INFINITY;
    for (int k = 0; k < v->n_suppress; k++) lg[v->suppress[k]] = -INFINITY;
    int nt = q->n_tokens;
    int last = nt > 0 && q->last >= v->beg;
    int penult = nt < 2 || q->penult >= v->beg;
    if (last) {
        if (penult)
            for (int i = v->beg; i < n; i++) lg[i] = -INFINITY;
        else
            for (int i = 0; i < v->eot; i++) lg[i] = -INFINITY;
    }
    if (initial) {
        double prec = 30.0 / (double)v->n_audio_ctx;
        int tid0 = (int)round(v->max_initial_ts / prec);
        for (int i = v->beg + tid0 + 1; i < n; i++) lg[i] = -INFINITY;
    }
    if (q->has_ts)
        for (int i = v->beg; i < v->beg + q->seek_delta / 2 && i < n; i++) lg[i] = -INFINITY;
    log_softmax(lp, lg, n);
    float ts_max = -INFINITY;
    for (int i = v->beg; i < n; i++) ts_max = lp[i] > ts_max ? lp[i] : ts_max;
    out->force_ts = 0;
    if (ts_max > -INFINITY) {
        float sum = 0.0f;
        for (int i = v->beg; i < n; i++)
            if (lp[i] > -INFINITY) sum = sum + orc_expf(lp[i] - ts_max);
        float ts_lp = (float)log((double)sum) + ts_max;
        float text_max = -INFINITY;
        for (int i = 0; i < v->beg; i++) text_max = lp[i] > text_max ? lp[i] : text_max;
        if (ts_lp > text_max) {
            for (int i = 0; i < v->beg; i++) lg[i] = lp[i] = -INFINITY;
            out->force_ts = 1;
        }
    }
    float *p = lg; /* copy(q.probs, lg); softmaxInf(q.probs) */
    softmax_inf(p, n);
    /* sample() */
    int id = 0;
    if (temp == 0) {
        for (int i = 0; i < n; i++)
            if (p[i] > p[id]) id = i;
    } else {
        float acc = 0.0f;
        id = -1;
        for (int i = 0; i < n; i++) {
            acc = acc + p[i];
            if (r < acc) {
                id = i;
                break;
            }
        }
        if (id < 0)
            for (int i = 0; i < n; i++)
                if (p[i] > 0) id = i;
    }
    int tid = v->beg;
    for (int i = v->beg; i < n; i++)
        if (p[i] > p[tid]) tid = i;
    if (id >= v->beg) tid = id;
    out->id = id;
    out->tid = tid;
    out->p = p[id];
    out->plog = lp[id];
    free(lg);
    free(lp);
}
