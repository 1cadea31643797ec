/*
 * grx_oracle.h - CPU restatement of gorelaxor's Q8_0 hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * product is compared against; it is linked or loaded only by tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py.  The
 * product (gorelaxor_amd/libgrx.so) never calls into it.
 *
 * Every function restates one reference function, in the same arithmetic
 * order, and cites it as file:line of the reference Go module
 * github.com/xattribution/gorelaxor.  Where the reference has both a Go
 * twin and an AVX2/VNNI assembly kernel, the restatement follows the
 * kernel a VNNI host actually runs (the assembly), and says so.
 *
 * Floating point: the library is built with -ffp-contract=off; every fused
 * multiply-add below is an explicit fmaf() matching a VFMADD in the
 * reference assembly, and every other product is rounded on its own, as
 * Go (GOAMD64=v1, no fusion) and the non-FMA instructions round it.
 */
#ifndef GRX_ORACLE_H
#define GRX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK 32
#define ORC_Q8_BYTES 34

/* ---- half precision (internal/kern/f16.go) ---- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

/* ---- weight rounding (kern.go ToQ8, kern_test.go quantQ8) ---- */
void orc_quant_q8(const float *v, size_t nvals, uint8_t *out);
void orc_dequant_q8(float *dst, const uint8_t *q, int nb);

/* ---- activation rounding (q8int.go quantU8Go / vnni_amd64.s quantU8avx) ---- */
void orc_quant_u8(uint8_t *dst, float *sc, const float *x, int nb);
void orc_quant_act_i8(int8_t *dst, float *sc, const float *x, int nb);

/* ---- int8 products ---- */
void orc_block_dots(int32_t *s, const int8_t *qa, int m, const uint8_t *wq, int n, int k);
typedef void (*orc_q8_product_fn)(float *c, int ldc, const float *a, int lda, int m, const uint8_t *wq, int n,
                                  int k, const float *bias);
void orc_set_q8_product(orc_q8_product_fn fn);
void orc_matmul_q8_int(float *c, int ldc, const float *a, int lda, int m,
                       const uint8_t *wq, int n, int k, const float *bias, int evex);
void orc_matmul_q8_int_prequant(float *c, int ldc, const int8_t *qa, const float *sa, int m,
                                const uint8_t *wq, int n, int k, const float *bias);
void orc_matmul_q8_float(float *c, int ldc, const float *a, int lda, int m,
                         const uint8_t *wq, int n, int k, const float *bias);

/* ---- float kernels (mathx.go, kernels_amd64.s) ---- */
float orc_expf(float x);
float orc_exp8(float x);
float orc_expsub(float *x, int n, float mx);
void orc_softmax(float *x, int n);
void orc_gelu_vec(float *x, int n);
void orc_silu_vec(float *x, int n);
void orc_axpy(float *dst, const float *src, int n, float s);
void orc_layernorm(float *dst, const float *src, int rows, int n, const float *w, const float *b);
void orc_layernorm_f64(float *dst, const float *src, int rows, int n, const float *w,
                       const float *b, double eps);
float orc_dot_f32_go(const float *x, const float *y, int n);
void orc_dot_f32_x4(const float *x, const float *w, int ld, int k, float out[4]);
int orc_argmax(const float *x, int n);

/* ---- whisper-shaped decoder with Q8_0 weights (whisper/decoder.go) ---- */
typedef struct {
    const float *attn_ln_w, *attn_ln_b;
    const uint8_t *q, *k, *v, *o;
    const float *q_b, *v_b, *o_b;
    const float *x_ln_w, *x_ln_b;
    const uint8_t *xq, *xk, *xv, *xo;
    const float *xq_b, *xv_b, *xo_b;
    const float *mlp_ln_w, *mlp_ln_b;
    const uint8_t *fc1, *fc2;
    const float *fc1_b, *fc2_b;
    float *cross_k; /* [head][audio_ctx][head_dim], keys pre-scaled */
    float *cross_v; /* [head][head_dim][audio_ctx] */
    float *self_k;  /* [text_ctx][state] */
    float *self_v;  /* [text_ctx][state] */
} orc_whisper_layer;

typedef struct {
    int n_vocab, n_text_ctx, n_state, n_head, n_layer, n_audio_ctx;
    const uint8_t *tok_emb; /* Q8_0 [n_vocab][n_state] */
    const float *dec_pos;   /* [n_text_ctx][n_state] */
    const float *dec_ln_w, *dec_ln_b;
    orc_whisper_layer *layers;
    int n; /* positions filled in the self-attention caches */
} orc_whisper;

void orc_whisper_cross_kv(orc_whisper *m, const float *enc);
int orc_whisper_decode(orc_whisper *m, const int *tokens, int nt, float *logits);
void orc_whisper_greedy(orc_whisper *m, const int *prompt, int n_prompt, int n_steps,
                        int *out_tokens);

/* ---- float products of the reference's float route (gemm.go) ---- */
void orc_matmul_f32(float *c, int ldc, const float *a, int lda, const float *b, int ldb, int m, int n,
                    int k, const float *bias);

/* ---- pocket-TTS flow-LM transformer (pockettts/nn.go, lm.go) ---- */
void orc_rope_freqs(float *f, int head_dim, double period);
void orc_apply_rope(float *x, int heads, const float *freqs, int half, int pos);

typedef struct {
    const float *norm1_w, *norm1_b, *norm2_w, *norm2_b;
    const uint8_t *qkv, *out, *ff1, *ff2; /* Q8_0 rows: [3d][d], [d][d], [ff][d], [d][ff] */
    float *k, *v;                         /* caches [max_pos][d] */
} orc_ptts_layer;

typedef struct {
    int d, heads, ff, n_layer, max_pos, ldim;
    const float *freqs;   /* head_dim/2 rotary frequencies */
    orc_ptts_layer *layers;
    const float *input;   /* [d][ldim] float32 */
    const float *bos;     /* [ldim] */
    const float *out_w, *out_b;
    const float *eos_w;   /* [d] float32 */
    float eos_b;
    int pos;
} orc_ptts;

int orc_ptts_forward(orc_ptts *m, float *x, int T);
int orc_ptts_run(orc_ptts *m, float *x, int T, float *out);
int orc_ptts_step(orc_ptts *m, const float *latent, float *out, float *eos);

/* ---- pocket-TTS's Mimi decoder (pockettts/mimi.go, nn.go) ---- */
typedef struct {
    int n, k;            /* rows (outputs) and columns (inputs) */
    const uint8_t *wq;   /* Q8_0 rows, or NULL */
    const float *wf;     /* float32 rows when wq is NULL */
    const float *b;      /* [n] or NULL */
} orc_mlin;
typedef struct {
    int cin, cout, k, stride, dil;
    orc_mlin w;          /* [cout][k*cin] */
} orc_mconv;
typedef struct {
    int cin, cout, k, stride;
    orc_mlin w;          /* [k*cout][cin]; w.b is the [cout] bias */
} orc_mconvtr;
typedef struct {
    int kind;            /* 0 conv, 1 transposed conv, 2 residual block */
    int elu;             /* ELU before the step */
    orc_mconv c;         /* kind 0 */
    orc_mconvtr t;       /* kind 1 */
    orc_mconv a, b;      /* kind 2: a (kernel resK, dilation) then b (1x1) */
} orc_sea_step;
typedef struct {
    const float *norm1_w, *norm1_b, *norm2_w, *norm2_b;
    orc_mlin qkv, out, ff1, ff2;
    const float *ls1, *ls2; /* layer scales [d], or NULL */
} orc_mimi_layer;
typedef struct {
    int d, heads, ff, n_layer, context, ldim, up_s;
    const float *freqs;     /* head_dim/2 rotary frequencies */
    orc_mimi_layer *layers;
    orc_mlin quant;         /* [d][ldim], no bias */
    const float *up;        /* [d][2*up_s] depthwise taps */
    int n_steps;
    orc_sea_step *steps;
} orc_mimi;
typedef struct {
    int pos, max_pos;
    float **k, **v;         /* per layer [max_pos][d] */
    float *up_part;         /* [up_s][d] */
    int n_prev;
    float **prev;           /* each conv's past rows, each convtr's partial */
} orc_mimi_state;
void orc_elu(float *x, size_t n);
int orc_mconv_past(const orc_mconv *c);
orc_mimi_state *orc_mimi_state_new(const orc_mimi *m, int max_pos);
void orc_mimi_state_free(const orc_mimi *m, orc_mimi_state *s);
int orc_mimi_decode(const orc_mimi *m, orc_mimi_state *st, const float *lat, int n, float *out, int *n_out);

/* ---- FastConformer encoder with Q8_0 weights (conformer/encoder.go) ---- */
typedef struct {
    const float *norm_w, *norm_b;
    const uint8_t *w1, *w2; /* Q8_0 rows: [dff][d], [d][dff] */
    const float *b1, *b2;   /* may be NULL */
} orc_conf_ff;

typedef struct {
    orc_conf_ff ff1, ff2;
    const float *norm_attn_w, *norm_attn_b;
    const uint8_t *q, *k, *v, *out, *pos; /* Q8_0 [d][d] */
    const float *q_b, *k_b, *v_b, *out_b; /* may be NULL */
    const float *pos_u, *pos_v;           /* [heads][head_dim] */
    const float *norm_conv_w, *norm_conv_b;
    const uint8_t *pw1, *pw2; /* Q8_0 [2d][d], [d][d] */
    const float *pw1_b, *pw2_b;
    const float *dw;   /* depthwise taps, [kernel][d] */
    const float *dw_b; /* may be NULL */
    const float *cn_w, *cn_b; /* folded batch norm, or the LayerNorm's gain and bias */
    const float *norm_out_w, *norm_out_b;
} orc_conf_block;

typedef struct {
    int d, heads, layers, dff, conv_kernel, sub_channels, n_mels, xscaling, conv_ln;
    const float *w0, *b0, *w2, *b2, *w5, *b5; /* pre-encoder 3x3 taps, [9][c] */
    const uint8_t *w3, *w6, *out;             /* Q8_0 [c][c], [c][c], [d][c*F] */
    const float *b3, *b6, *out_b;
    orc_conf_block *blocks;
    /* conv.3 / conv.6 as float32 [c][c] (the reference's converter keeps
     * them float32): when set, Linear takes the float route, not w3 / w6 */
    const float *w3f, *w6f;
    /* HParams' attention and convolution forms (conformer/model.go:15-44):
     * causal_sub pads the pre-encoder two before and one after; att_style 1
     * is "chunked_limited" (cache-aware streaming), 0 "regular"; att_left,
     * att_right, conv_left, conv_right as the file gives them (-1: none) */
    int causal_sub, att_style, att_left, att_right, conv_left, conv_right;
} orc_conformer;

/* One query's keys [lo, hi) (keyRange, conformer/encoder.go:193-212, cut at
 * the valid length as encodeEmbeddings does, :465-472; a streaming chunk's
 * keys as streamEncode builds them, stream.go:273-287). */
enum { ORC_KEYS_ALL = 0, ORC_KEYS_CHUNKED = 1, ORC_KEYS_WINDOW = 2, ORC_KEYS_STREAM = 3 };
typedef struct {
    int mode;
    int T, L;               /* keys (offline: = queries) and the valid length */
    int chunk, left_chunks; /* CHUNKED, STREAM */
    int left, right;        /* WINDOW */
    int c, slot0, Tc;       /* STREAM: cached keys, the cache slot of key 0, the chunk's rows */
} orc_keys;
void orc_conf_key_range(const orc_keys *k, int q, int *lo, int *hi);
/* offlineKeys (encoder.go:196-212) for T frames of which L are valid: the
 * key form and the query block length. */
int orc_conf_offline_keys(const orc_conformer *m, int T, int L, orc_keys *k);
int orc_conf_pad_left(const orc_conformer *m);

/* Cache-aware streaming (conformer/stream.go:23-88, 241-307): the geometry
 * for one right context and one stream's caches. */
typedef struct {
    int right, chunk, left, left_chunks, drop;
    int kv_len;
    float **kv;       /* per layer: up to left rows of normalized attention input */
    float **conv;     /* per layer: the last pad_left gated frames */
    float **pos_proj; /* per layer: positions left+chunk-1 down to -(chunk-1), projected */
} orc_conf_stream;
orc_conf_stream *orc_conf_stream_new(const orc_conformer *m, int right, int left, int drop);
void orc_conf_stream_free(const orc_conformer *m, orc_conf_stream *s);
/* streamStep: one chunk's log-mel [mels][nf] (cache frames first), length
 * of them real; out receives the chunk's encoder rows (at most nf rows),
 * *L_out how many.  -1 when the chunk has more rows than the geometry. */
int orc_conf_stream_step(const orc_conformer *m, orc_conf_stream *s, const float *mel, int nf, int length, int first,
                         float *out, int *L_out);

void orc_conf_rel_pos(float *out, int n, int d);
void orc_conf_bn_fold(const float *gw, const float *gb, const float *mean, const float *var, int d, float *s,
                      float *b);
int orc_conf_subsample(const orc_conformer *m, const float *mel, int frames, int valid, float *out, int *T_out,
                       int *L_out);
int orc_conf_block_run(const orc_conformer *m, int i, float *x, int T, int L, const float *pos);
int orc_conformer_encode(const orc_conformer *m, const float *mel, int frames, int valid, int n_layers, float *out,
                         int *T_out, int *L_out);

/* ---- whisper's token rules and sampler (whisper/transcribe.go:370-536) ---- */
typedef struct {
    int eot, sot, translate, transcribe, solm, prev, nosp, no_timestamps, beg;
    int n_lang, space;
    const int *suppress;
    int n_suppress;
    int n_audio_ctx;
    double max_initial_ts;
} orc_whisper_rules;
typedef struct {
    int n_tokens, last, penult, has_ts, seek_delta;
} orc_whisper_seq;
typedef struct {
    int id, tid;
    float p, plog;
    int force_ts;
} orc_whisper_token;
void orc_whisper_sample(const float *logits, int n, const orc_whisper_rules *v, const orc_whisper_seq *q,
                        float temp, float r, orc_whisper_token *out);

/* ---- RNN-T / TDT greedy decoding (conformer/rnnt.go) ---- */
typedef struct {
    int d, H, L, V, J, act, tdt, nd, dur[16], max_symbols, blank;
    const float *embed;
    const uint8_t *const *wx, *const *wh; /* Q8_0 [4H][H] per layer */
    const float *const *b;                /* [4H] per layer */
    const uint8_t *jenc, *jpred, *jout;
    const float *jencb, *jpredb, *joutb;
} orc_rnnt;
typedef struct {
    int id, frame, duration;
    float p;
} orc_rnnt_token;
double orc_fd_exp(double x);
float orc_tanh32(float x);
int orc_rnnt_decode(const orc_rnnt *m, const float *enc, int T, float *h, float *c, int *last, int frame_offset,
                    orc_rnnt_token *out, int cap);

#ifdef __cplusplus
}
#endif
#endif
