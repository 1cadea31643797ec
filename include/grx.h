/*
 * grx.h - C ABI of the MI355X (gfx950) Q8_0 product library, libgrx.so.
 *
 * It replaces the Q8_0 branch of gorelaxor's operator seam, package
 * internal/kern (github.com/xattribution/gorelaxor), for callers that hold a
 * GPU.  Each entry point names the reference function it stands in for as
 * file:line of that module.  Plain C types only: no HIP or torch types cross
 * this boundary, so a cgo, ctypes or FFI binding needs nothing but this file.
 *
 * Conventions
 *  - Every call returns a grx_status; 0 is success.  On failure,
 *    grx_last_error() returns a message for the calling thread.  Nothing
 *    throws across the boundary.
 *  - Matrices are row-major.  A weight is `rows` outputs by `cols` inputs
 *    (kern.Weight, internal/kern/kern.go:38-50); `cols` is a multiple of 32.
 *  - Entry points without the _dev suffix take host pointers and return
 *    when the result is in host memory.  _dev entry points take device
 *    pointers (HBM) and only enqueue work on the context's stream; call
 *    grx_ctx_sync() before reading the results.
 *  - Threading: a grx_weight is immutable after creation and may be used
 *    from any number of contexts and threads at once.  A grx_ctx owns one
 *    HIP stream and its scratch buffers: use one context per thread.
 */
#ifndef GRX_H
#define GRX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    GRX_OK = 0,
    GRX_EINVAL = -1,   /* a null pointer, negative size or stride too small */
    GRX_ESIZE = -2,    /* a buffer too short for the shape, or cols % 32 != 0 */
    GRX_EDEVICE = -3,  /* a HIP runtime error (message has the HIP text) */
    GRX_ENOMEM = -4,   /* device memory exhausted */
    GRX_ESTATE = -5,   /* call out of order (e.g. decoding past the context) */
    GRX_ENODEV = -6    /* no gfx950 device visible */
} grx_status;

typedef struct grx_ctx grx_ctx;
typedef struct grx_weight grx_weight;

/* Library */
int grx_version(void);
const char *grx_last_error(void);
/* Number of visible devices; 0 when there is no GPU (never an error). */
int grx_device_count(void);

/* Context: a device and one stream.  No reference counterpart: the
 * reference runs on the calling goroutine (internal/kern/gemm.go:52-108). */
grx_status grx_ctx_create(int device, grx_ctx **out);
grx_status grx_ctx_destroy(grx_ctx *ctx);
grx_status grx_ctx_sync(grx_ctx *ctx);
/* The context's hipStream_t, as an opaque pointer, for callers that order
 * their own device work with it. */
void *grx_ctx_stream(grx_ctx *ctx);

/* ---- Q8_0 weights ---- */

/* kern.NewQ8 + Weight.Pack + Weight.DropRows (internal/kern/kern.go:76-103,
 * q8int.go:35-64): check the shape, copy `rows` ggml Q8_0 rows (cols/32
 * blocks of 34 bytes: a little-endian float16 scale, then 32 int8 values)
 * to the device and repack them once into the HBM tile layout the GEMV
 * streams.  The host buffer may be freed on return.  Errors as NewQ8:
 * GRX_ESIZE when cols % 32 != 0 or nbytes < rows*cols/32*34. */
grx_status grx_weight_q8_create(grx_ctx *ctx, int rows, int cols, const uint8_t *q8,
                                size_t nbytes, grx_weight **out);
grx_status grx_weight_destroy(grx_weight *w);
/* Weight.Rows / Weight.Cols (kern.go:42). */
int grx_weight_rows(const grx_weight *w);
int grx_weight_cols(const grx_weight *w);
/* Weight.Bytes (kern.go:172-179): device bytes the weight holds. */
size_t grx_weight_bytes(const grx_weight *w);
/* Weight.Row (kern.go:115-122, q8int.go:66-78): widen row j to float32,
 * exactly. */
grx_status grx_weight_row(grx_ctx *ctx, const grx_weight *w, int j, float *dst);
/* Weight.Float32 (kern.go:124-134): the whole matrix widened, rows*cols. */
grx_status grx_weight_float32(grx_ctx *ctx, const grx_weight *w, float *dst);

/* Weight.ToQ8 (kern.go:136-170) on the device: round rows*cols float32
 * values (cols % 32 == 0) to ggml Q8_0 bytes, rows*cols/32*34 of them,
 * each block's scale amax/127 and each value rounded half away from zero. */
grx_status grx_to_q8(grx_ctx *ctx, int rows, int cols, const float *v, uint8_t *q8_out);

/* ---- products ---- */

/* kern.MatMul (internal/kern/kern.go:183-196) on the int8 route of
 * matmulQ8Int (q8int.go:148-223): dst[m][ldc] = x[m][lda] . W^T + bias.
 * Each row of x is rounded to Q8_0 per 32 values (quantU8,
 * q8int.go:88-105); each output starts from the bias (or 0) and takes
 * c = fma(f32(s_b)*dw_b, da_b, c) block by block in order, as the VNNI
 * kernel does (vnni_amd64.s:58-69), so results are bit-identical to it.
 * bias may be NULL.  m == 0 is a no-op (kern.go:186-188). */
grx_status grx_matmul_q8(grx_ctx *ctx, float *dst, int ldc, const float *x, int lda, int m,
                         const grx_weight *w, const float *bias);
/* kern.Linear (kern.go:198-201): MatMul with ldc = rows, lda = cols. */
grx_status grx_linear_q8(grx_ctx *ctx, float *dst, const float *x, int m, const grx_weight *w,
                         const float *bias);
/* grx_matmul_q8 on device pointers, enqueued on the context's stream. */
grx_status grx_matmul_q8_dev(grx_ctx *ctx, float *dst, int ldc, const float *x, int lda, int m,
                             const grx_weight *w, const float *bias);

/* grx_matmul_q8_dev without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Fewer rows than the matrix-core threshold (16) are rounded
 * inside the product's own launches and need no memory beyond x and dst;
 * for more rows the rounded activations go to a fixed device array of the
 * library (4 MiB per GPU, held until the process ends) instead of the
 * context's scratch: m * cols + m * cols/32 * 4 bytes (plus alignment to
 * 256) must fit, else GRX_ESIZE.  Every call on a GPU shares that array:
 * calls that overlap on one GPU (other streams or threads) race.  Results
 * are those of grx_matmul_q8_dev, bit for bit. */
grx_status grx_matmul_q8_dev_noalloc(grx_ctx *ctx, float *dst, int ldc, const float *x, int lda, int m,
                                     const grx_weight *w, const float *bias);

/* quantU8 (internal/kern/q8int.go:86-105, vnni_amd64.s:194-256) on device
 * pointers: round m rows of k float32 values (k % 32 == 0, rows lda apart)
 * to signed int8 q[m][k] (the reference's unsigned byte minus 128) and one
 * float32 scale per 32 values, sc[m][k/32]. */
grx_status grx_quant_act_dev(grx_ctx *ctx, int8_t *q, float *sc, const float *x, int lda, int m,
                             int k);
/* The int8 product from activations rounded already (grx_quant_act_dev's
 * output), device pointers.  The per-block int32 dots and the finalize are
 * those of grx_matmul_q8. */
grx_status grx_matmul_q8_prequant_dev(grx_ctx *ctx, float *dst, int ldc, const int8_t *q,
                                      const float *sc, int m, const grx_weight *w,
                                      const float *bias);
/* The per-block int32 dot products s[m][rows][cols/32] of rounded
 * activations with the weight (q8tile's int32 sums, vnni_amd64.s:34-54
 * minus the 128*sum(w) offset), device pointers.  For parity checks. */
grx_status grx_block_dots_dev(grx_ctx *ctx, int32_t *s, const int8_t *q, int m,
                              const grx_weight *w);
/* The elementwise float kernels of the path on n values, device pointers
 * (y may equal x), exactly as the decode and encode kernels evaluate them.
 * For parity checks:
 *   GRX_VEC_EXPF  expf, the scalar form (whisper/mathx.go:7-33)
 *   GRX_VEC_EXP8  EXP8, one lane of the vector form (kernels_amd64.s:236-258)
 *   GRX_VEC_GELU  geluVec over the n values (kernels_amd64.go:119-129: the
 *                 assembly form below n &^ 7, gelu (mathx.go:36-52) past it) */
enum { GRX_VEC_EXPF = 0, GRX_VEC_EXP8 = 1, GRX_VEC_GELU = 2 };
grx_status grx_vec_dev(grx_ctx *ctx, int fn, float *y, const float *x, int n);

/* The path's two LayerNorms on `rows` rows of n float32 values, device
 * pointers, exactly as the decode and encode kernels evaluate them.  For
 * parity checks.
 *   form GRX_LN_KERN  kern's layerNorm (internal/kern/mathx.go:55-75):
 *                     float64 sums, mean and inv rounded to float32,
 *                     eps 1e-5; w and b required
 *   form GRX_LN_F64   pockettts' layerNorm (pockettts/nn.go:27-49): mean
 *                     and inv in float64, each output rounded to float32,
 *                     then * w + b when given (both or neither); eps given
 *   impl GRX_LN_BLOCK a workgroup per row, the row in LDS (the encoder's
 *                     rows, several-row products, the frame end, the flow
 *                     head); n <= 8192
 *   impl GRX_LN_WAVE  one wave per row, the row in registers (the one-row
 *                     products' prologues); n % 4 == 0, n <= 1280
 * The sums are formed in parallel, and again in the reference's order for
 * the rows where the parallel sums could round to other float32 results.
 * flags GRX_LN_TREE_ONLY skips that second pass (tests use it to show
 * which rows need it); products never set it. */
enum { GRX_LN_KERN = 0, GRX_LN_F64 = 1 };
enum { GRX_LN_BLOCK = 0, GRX_LN_WAVE = 1 };
enum { GRX_LN_TREE_ONLY = 1 };
grx_status grx_layernorm_dev(grx_ctx *ctx, int form, int impl, int flags, float *y, const float *x, int rows, int n,
                             const float *w, const float *b, double eps);

/* kern.Linear of ONE row through the float route (kern.go:185-196 ->
 * gemvRows, gemm.go:195-259): what the reference does for m = 1 when the
 * weight keeps its rows (no DropRows) - dot4q8avx for rows in whole groups
 * of four, dotQ8Go for the rest, then the bias - instead of the int8 route
 * that grx_linear_q8 takes.  Host buffers. */
grx_status grx_linear_q8_float(grx_ctx *ctx, float *dst, const float *x, const grx_weight *w, const float *bias);
/* The same for a float32 weight (rows x cols, row-major, host memory):
 * dotF32x4 for rows in whole groups of four, dotF32Go for the rest. */
grx_status grx_linear_f32(grx_ctx *ctx, float *dst, const float *x, const float *w, int rows, int cols,
                          const float *bias);

/* ---- whisper-shaped text decoder with Q8_0 weights ---- */

/* The decoder graph of whisper/decoder.go:33-140 with every matrix a Q8_0
 * weight on the int8 route above, kept on one GPU: the self-attention KV
 * cache, the cross-attention keys and values, the token and the position
 * live in HBM, and one decode step is a fixed sequence of launches
 * (replayed from a HIP graph) that ends in the argmax of the logits. */
typedef struct {
    int n_vocab, n_text_ctx, n_state, n_head, n_layer, n_audio_ctx; /* whisper/model.go:16-21 */
} grx_whisper_hparams;

typedef struct grx_whisper grx_whisper;

grx_status grx_whisper_create(grx_ctx *ctx, const grx_whisper_hparams *hp, grx_whisper **out);
grx_status grx_whisper_destroy(grx_whisper *m);
/* Model.bind (whisper/model.go:300-404) for the decoder's tensors, by the
 * ggml names ("decoder.token_embedding.weight", "decoder.blocks.0.attn.
 * query.weight", ...): matrices as ggml Q8_0 rows, vectors as float32.
 * Shapes are checked; all tensors must be set before the first decode. */
grx_status grx_whisper_set_tensor(grx_whisper *m, const char *name, const void *data, size_t nbytes);
/* The cross-attention keys and values of every layer from the encoder
 * output, n_audio_ctx x n_state float32 on the host (whisper/encoder.go:
 * 120-143): K scaled by 1/sqrt(head_dim) and kept [head][t][d], V kept
 * transposed [head][d][t]. */
grx_status grx_whisper_set_encoder_output(grx_whisper *m, const float *enc, int n_audio_ctx);
/* Empty the self-attention cache (kvCache.n = 0, decoder.go:7-11). */
grx_status grx_whisper_reset(grx_whisper *m);
/* Positions filled in the self-attention cache. */
int grx_whisper_pos(const grx_whisper *m);
/* Model.decode (decoder.go:33-140) of n tokens after the cached positions;
 * the logits of the last one go to `logits` (n_vocab floats, may be NULL)
 * and their argmax - the first index of the largest value, as the greedy
 * sampler takes it (whisper/transcribe.go:459-464) - to *next (may be
 * NULL).  GRX_ESTATE when the tokens do not fit n_text_ctx. */
grx_status grx_whisper_decode(grx_whisper *m, const int32_t *tokens, int n, float *logits, int32_t *next);
/* Greedy decoding on the device (the loop of whisper/transcribe.go:207-260
 * with plain argmax): the prompt, then n_steps single-token steps each fed
 * the previous argmax, with no host round trip in between.  out receives
 * n_steps+1 token ids: the argmax after the prompt, then one per step. */
grx_status grx_whisper_greedy(grx_whisper *m, const int32_t *prompt, int n_prompt, int n_steps,
                              int32_t *out);

/* Several independent decodes side by side: n_streams (1, 2, 4 or 8)
 * whisper sessions, each its own encoder output, KV cache and token loop
 * (whisper/transcribe.go:207-260 run once per stream), sharing the weights
 * and stepping together, so every product takes n_streams rows at once.
 * Each stream's tokens are the ones its own decode gives.  No reference
 * counterpart: the reference decodes one session at a time. */
grx_status grx_whisper_create_streams(grx_ctx *ctx, const grx_whisper_hparams *hp, int n_streams,
                                      grx_whisper **out);
int grx_whisper_streams(const grx_whisper *m);
/* grx_whisper_set_encoder_output for one stream (0 .. n_streams-1); every
 * stream needs one before decoding. */
grx_status grx_whisper_set_encoder_output_stream(grx_whisper *m, int stream, const float *enc, int n_audio_ctx);
/* grx_whisper_greedy for every stream: prompts [n_streams][n_prompt],
 * out [n_streams][n_steps+1].  (grx_whisper_decode and grx_whisper_greedy
 * serve one stream and return GRX_ESTATE for more.) */
grx_status grx_whisper_greedy_streams(grx_whisper *m, const int32_t *prompts, int n_prompt, int n_steps,
                                      int32_t *out);

/* kvCache.copyFrom (whisper/decoder.go:22-28) between streams of one
 * decoder: stream dst's self-attention cache takes stream src's rows for
 * the positions filled so far, and dst's next token and token record
 * become src's.  transcribe.go:196-204 decodes a window's prompt once and
 * copies that cache to each bestOf sequence; here those sequences are the
 * streams.  Cross keys and values are not copied. */
grx_status grx_whisper_stream_copy(grx_whisper *m, int dst, int src);
/* Stream dst takes stream src's cross-attention keys and values (streams
 * decoding one window share its encoder output; a device copy, no second
 * projection).  GRX_ESTATE when src has none. */
grx_status grx_whisper_share_encoder_output(grx_whisper *m, int dst, int src);
/* n_steps greedy steps of every stream from the current position, each
 * stream fed the token its last step chose (the loop of
 * whisper/transcribe.go:207-260 with plain argmax, continued after a
 * decode, a greedy run or a stream copy); out [n_streams][n_steps]
 * receives the tokens chosen. */
grx_status grx_whisper_steps(grx_whisper *m, int n_steps, int32_t *out);
/* The logits of stream `stream`'s last step (n_vocab floats, host). */
grx_status grx_whisper_logits(grx_whisper *m, int stream, float *out);

/* A whisper.cpp (ggml) model file straight into a decoder of n_streams
 * streams (1, 2, 4 or 8): replaces whisper.Load (whisper/model.go:93-225)
 * and Model.bind (model.go:300-404) for the decoder.  The file is read and
 * checked as the reference reads it (magic, dimensions, mel filters,
 * vocabulary, tensors until the end; the same error texts, prefixed with
 * the path), but a Q8_0 matrix goes to the device as stored instead of
 * being widened to float16; other matrix types are widened as the
 * reference widens them and rounded to Q8_0.  The encoder's tensors are
 * checked and skipped.  *hp_out (may be NULL) receives the decoder's
 * dimensions. */
grx_status grx_whisper_load_ggml(grx_ctx *ctx, const char *path, int n_streams, grx_whisper_hparams *hp_out,
                                 grx_whisper **out);

/* ---- whisper's token rules and sampler (whisper/transcribe.go:370-494) ---- */

/* The vocabulary's special tokens (whisper/vocab.go:18-45) and the rules'
 * settings. */
typedef struct {
    int eot, sot, translate, transcribe, solm, prev, nosp, no_timestamps, beg;
    int n_lang;               /* language tokens after sot */
    int space;                /* the id of " ", or -1 when the vocabulary has none */
    const int32_t *suppress;  /* vocab.suppressed(), host memory */
    int n_suppress;
    int n_audio_ctx;          /* the model's, for the initial timestamp limit */
    double max_initial_ts;    /* seconds (maxInitialTS, 1.0) */
} grx_whisper_rules;
/* What the rules read of a sequence (seq of transcribe.go:100-115). */
typedef struct {
    int n_tokens;        /* len(q.tokens): tokens sampled in this window */
    int last, penult;    /* the last two of them (read only when present) */
    int has_ts;          /* q.hasTS */
    int seek_delta;      /* q.seekDelta */
} grx_whisper_seq;
/* tok of transcribe.go (id, best timestamp, probability, log probability);
 * force_ts: timestamps together outweighed every text token. */
typedef struct {
    int id, tid;
    float p, plog;
    int force_ts;
} grx_whisper_token;
/* session.process + session.sample over n logits in host memory: the
 * temperature, the suppression and timestamp rules, logSoftmax, softmaxInf,
 * then the argmax (temp 0) or the draw against r (s.rng.Float32(), drawn
 * by the caller).  Bit-identical to the reference's float32 arithmetic,
 * its left-to-right sums included. */
grx_status grx_whisper_sample_logits(grx_ctx *ctx, const float *logits, int n, const grx_whisper_rules *rules,
                                     const grx_whisper_seq *seq, float temp, float r, grx_whisper_token *out);
/* The same over the logits of stream `stream`'s last decode, which stay on
 * the device. */
grx_status grx_whisper_sample(grx_whisper *m, int stream, const grx_whisper_rules *rules,
                              const grx_whisper_seq *seq, float temp, float r, grx_whisper_token *out);

/* One window's decode loop (whisper/transcribe.go:207-260) on the device
 * for one sequence: the window's place in the audio (mel frames of 10 ms),
 * the loop's limits, the temperature and its draws. */
typedef struct {
    int seek, seek_end;  /* the window's first frame; the audio's end */
    int delta_min;       /* deltaMin (transcribe.go:38): frames left that count as the end */
    int win_frames;      /* frames in a window (3000): a fresh seq's seekDelta */
    int n_max;           /* iterations at most (nMax = n_text_ctx/2 - 4) */
    float temp;          /* 0: the most likely token; above 0: draws */
    const float *r;      /* temp > 0: n_max draws s.rng.Float32(), in order (host) */
} grx_whisper_loop;
/* What the loop left of the seq (transcribe.go:100-115). */
typedef struct {
    int n_tokens;    /* tokens sampled, in out */
    int done, failed;
    int result_len, seek_delta, has_ts;
} grx_whisper_loop_result;
/* The loop after a prompt decoded with grx_whisper_decode (its logits are
 * where the step left them): each iteration applies process + sample
 * (transcribe.go:370-494) with the sequence state kept on the device, then
 * the loop's rules - a timestamp moves seekDelta and the result length or
 * fails the sequence when it goes back; the end token, or a timestamp that
 * reaches the audio's end, finishes it; the last iteration fails a
 * sequence stuck repeating itself - and feeds the token to the next decode
 * step, with no host round trip in between (the state is read back every
 * sixteen iterations).  out receives each token (n_max of them at most);
 * *res the sequence's state.  One stream. */
grx_status grx_whisper_rules_loop(grx_whisper *m, const grx_whisper_rules *rules, const grx_whisper_loop *loop,
                                  grx_whisper_token *out, grx_whisper_loop_result *res);

/* ---- GGUF model files (internal/gguf/gguf.go) ---- */

/* A GGUF file (versions 2 and 3; tensors F32, F16, BF16, Q8_0) with the
 * reference's checks against crafted files and its error texts.  Host
 * only: these calls need no GPU, except grx_gguf_weight_q8. */
typedef struct grx_gguf grx_gguf;
/* gguf.Open (gguf.go:57-113): the header and tensor table; a tensor's bytes
 * are read from the file when asked for.  Tensors whose sizes add up to
 * more than the file are refused. */
grx_status grx_gguf_open(const char *path, grx_gguf **out);
/* gguf.Parse (gguf.go:277-289) of a file held in memory (copied). */
grx_status grx_gguf_parse(const void *bytes, size_t n, grx_gguf **out);
/* gguf.ReadMeta (gguf.go:219-234): the settings only, no tensor table. */
grx_status grx_gguf_read_meta(const char *path, grx_gguf **out);
grx_status grx_gguf_close(grx_gguf *g);
int grx_gguf_version(const grx_gguf *g);
/* File.Names (file order) and File.Keys (sorted). */
int grx_gguf_n_tensors(const grx_gguf *g);
const char *grx_gguf_tensor_name(const grx_gguf *g, int i);
int grx_gguf_n_keys(const grx_gguf *g);
const char *grx_gguf_key(const grx_gguf *g, int i);
/* File.Has */
int grx_gguf_has(const grx_gguf *g, const char *name);
/* A tensor's type and dimensions (dims[0] the row length); unused dims 0. */
grx_status grx_gguf_tensor_info(const grx_gguf *g, const char *name, int *type, int *n_dims, int64_t dims[4]);
/* File.Int / Float / Bool / String (gguf.go:415-460): def when missing or
 * of another kind.  Strings live as long as the file handle. */
int64_t grx_gguf_int(const grx_gguf *g, const char *key, int64_t def);
double grx_gguf_float(const grx_gguf *g, const char *key, double def);
int grx_gguf_bool(const grx_gguf *g, const char *key, int def);
const char *grx_gguf_string(const grx_gguf *g, const char *key, const char *def);
/* File.Strings / Floats / Ints (gguf.go:462-510) element by element:
 * grx_gguf_array_len is -1 when the key holds no array; an element of
 * another kind reads as "" or 0, as there. */
int64_t grx_gguf_array_len(const grx_gguf *g, const char *key);
const char *grx_gguf_array_string(const grx_gguf *g, const char *key, int64_t i);
double grx_gguf_array_float(const grx_gguf *g, const char *key, int64_t i);
int64_t grx_gguf_array_int(const grx_gguf *g, const char *key, int64_t i);
/* File.Float32 (gguf.go:518-542): n >= the tensor's values. */
grx_status grx_gguf_float32(const grx_gguf *g, const char *name, float *out, size_t n);
/* File.Weight's matrix shape (gguf.go:544-558): cols is the first
 * dimension longer than one, the rest flattened into rows. */
grx_status grx_gguf_weight_shape(const grx_gguf *g, const char *name, int64_t *rows, int64_t *cols);
/* File.Weight + kern.NewQ8 + Pack (gguf.go:544-581, kern.go:41-93): a Q8_0
 * tensor from the file to its device tiles, with no host copy kept. */
grx_status grx_gguf_weight_q8(grx_ctx *ctx, const grx_gguf *g, const char *name, grx_weight **out);

/* ---- pocket-TTS flow-LM transformer with Q8_0 weights ---- */

/* flowLM of pockettts/lm.go:164-195 over transformer.forward and attend of
 * pockettts/nn.go:142-254 (float64 LayerNorm, rotary q and k with period
 * `period`, causal attention, tanh-GELU feed-forward, no context limit),
 * its transformer matrices Q8_0 on the int8 route as pockettts/model.go:
 * 331-366 packs them.  The KV caches, position and frame index stay in HBM. */
typedef struct {
    int d, heads, ff, n_layer, max_pos, ldim;
    double period;
} grx_pocket_hparams;

typedef struct grx_pocket grx_pocket;

grx_status grx_pocket_create(grx_ctx *ctx, const grx_pocket_hparams *hp, grx_pocket **out);
grx_status grx_pocket_destroy(grx_pocket *m);
/* The flow LM's tensors by the names pockettts/model.go reads ("lm.blk.0.
 * attn_qkv.weight", "lm.input.weight", "lm.bos", "lm.out_norm.weight",
 * "lm.eos.weight", ...): transformer matrices as ggml Q8_0 rows, the rest
 * float32; shapes checked. */
grx_status grx_pocket_set_tensor(grx_pocket *m, const char *name, const void *data, size_t nbytes);
/* The flow LM of a Pocket TTS GGUF file (pockettts.Load, pockettts/model.go:
 * 201-250, its loader model.go:49-125): the file's name and source checks,
 * the LM settings (latent_dim, lm.d_model, lm.heads, lm.ff, lm.layers,
 * lm.max_period) with the reference's range checks, layers counted as the
 * reference counts them, every tensor's shape checked with the reference's
 * texts; the transformer's Q8_0 matrices go from the file to the device as
 * stored.  max_pos bounds the KV caches.  *hp_out (may be NULL) receives
 * the dimensions.  The flow head, Mimi and the tokenizer are not read. */
grx_status grx_pocket_load_gguf(grx_ctx *ctx, const char *path, int max_pos, grx_pocket_hparams *hp_out,
                                grx_pocket **out);
/* Declare the flow head (SimpleMLPAdaLN, pockettts/lm.go:27-160): its width
 * (pockettts.flow.dim), residual blocks (pockettts.flow.depth) and LSD steps
 * per latent (pockettts.decode_steps).  Its tensors then bind by their
 * names ("flow.cond.weight", "flow.res.0.ada.weight", "flow.time.1.freqs",
 * "flow.final.out.weight", ...): matrices as ggml Q8_0 rows or float32
 * (as the file stores them; each takes kern's float route, as the
 * reference's unpacked weights do), vectors float32. */
grx_status grx_pocket_flow_init(grx_pocket *m, int dim, int depth, int decode_steps);
/* The frame loop of speakChunk (pockettts/speak.go:146-176) on the device:
 * n frames, each a transformer step (flowLM.step, fed the previous frame's
 * latent; the first frame is fed first_latent, or bos when NULL) and the
 * flow head's sample from its output and noise[k] (ldim values per frame,
 * drawn and scaled by the caller as speakChunk does), one captured graph a
 * frame.  latents [n][ldim] receives each sampled latent (before the
 * mean/std scaling), eos [n] the end-of-speech logits; either may be NULL.
 * The caller applies the end-of-speech rule. */
grx_status grx_pocket_speak(grx_pocket *m, const float *first_latent, const float *noise, int n, float *latents,
                            float *eos);
/* Empty the caches (position 0). */
grx_status grx_pocket_reset(grx_pocket *m);
int grx_pocket_pos(const grx_pocket *m);
/* flowLM.run (lm.go:164-170) of T rows of transformer input (the text
 * prefix's embeddings, host float32 [T][d]) after the cached positions;
 * out (d floats, may be NULL) receives out_norm of the last row. */
grx_status grx_pocket_run(grx_pocket *m, const float *x, int T, float *out);
/* n flowLM.step calls (lm.go:185-195) on the device, frame k fed latents[k]
 * (host float32 [n][ldim]; NULL: the bos input every frame), no host round
 * trip in between: outs (n x d, may be NULL) receives each frame's out_norm
 * output and eos (n, may be NULL) its end-of-speech logit. */
grx_status grx_pocket_frames(grx_pocket *m, const float *latents, int n, float *outs, float *eos);

/* The flow LM's transformer state (tstate, pockettts/nn.go:113-126): each
 * layer's rotated keys and values for `positions` positions, held in device
 * memory on the LM's device.  A Voice (pockettts/voice.go:13-24) is such a
 * state.  A state does not change when the LM runs on from it, so one
 * voice seeds any number of chunks, as speakChunk's clone does. */
typedef struct grx_pocket_state grx_pocket_state;
/* A state from host keys and values k, v [n_layer][positions][d] (the LM's
 * layer count and width), as a Voice holds them. */
grx_status grx_pocket_state_create(grx_pocket *m, const float *k, const float *v, int positions,
                                   grx_pocket_state **out);
/* Model.LoadVoice (pockettts/voice.go:26-64): a voice GGUF file made for the
 * model file the LM was loaded from (grx_pocket_load_gguf; its
 * general.source.sha256), with the reference's checks in its order and its
 * texts: architecture "pockettts-voice", the model's hash, the LM's layer
 * count and 1..4096 positions, tensors voice.{i}.k and voice.{i}.v of
 * [positions][d] (float32, float16 or bfloat16, widened to float32), every
 * value a number. */
grx_status grx_pocket_load_voice_gguf(grx_pocket *m, const char *path, grx_pocket_state **out);
/* The LM's current state (its positions so far), copied into a new state
 * on the device. */
grx_status grx_pocket_state_save(grx_pocket *m, grx_pocket_state **out);
/* tstate.clone (nn.go:128-140) into the LM, as speakChunk seeds a chunk
 * from its voice (speak.go:117): the LM's caches take the state's
 * positions and its next position becomes the state's count; the state
 * is unchanged.  The LM's max_pos bounds the room left for the text and
 * the frames (GRX_ESTATE when the state alone exceeds it; GRX_EINVAL for
 * another layer count, width or device). */
grx_status grx_pocket_set_state(grx_pocket *m, const grx_pocket_state *s);
int grx_pocket_state_positions(const grx_pocket_state *s);
/* Host copies of the state's keys and values, [n_layer][positions][d]
 * floats each (either may be NULL). */
grx_status grx_pocket_state_read(const grx_pocket_state *s, float *k, float *v);
grx_status grx_pocket_state_destroy(grx_pocket_state *s);

/* ---- pocket-TTS's Mimi decoder (latents to audio) ---- */

/* mimiDecoder of pockettts/mimi.go:23-152 (its settings as pockettts.Load
 * reads them, pockettts/model.go:280-308): a latent's 1x1 projection to
 * d channels, the depthwise transposed upsampling by `upsample` with its
 * overlap carried to the next call, the context-limited transformer with
 * layer scales (pockettts/nn.go:142-254), then SEANet's decoder (a conv,
 * per ratio ELU + transposed conv + residual blocks, ELU + a last conv to
 * one channel; model.go:163-181).  Every Linear takes kern.MatMul's route
 * for its weight: Q8_0 matrices the int8 route (model.go:331-366 packs
 * them), float32 ones the float route.  max_latents bounds the latents one
 * decode call takes. */
typedef struct {
    int d, heads, ff, layers, context, ldim, upsample;
    double period;
    int n_ratios;
    int ratios[8];
    int n_filters, kernel_size, residual_kernel_size, last_kernel_size, dilation_base, compress, n_residual;
    int max_latents;
} grx_mimi_hparams;

typedef struct grx_mimi grx_mimi;

grx_status grx_mimi_create(grx_ctx *ctx, const grx_mimi_hparams *hp, grx_mimi **out);
grx_status grx_mimi_destroy(grx_mimi *m);
/* The decoder's tensors by the names pockettts/model.go reads ("mimi.quant",
 * "mimi.up", "mimi.dec_tf.0.attn_qkv.weight", "mimi.dec_tf.0.ls1",
 * "mimi.dec.2.weight", "mimi.dec.3.1.bias", ...): a matrix as ggml Q8_0
 * rows or float32 (told apart by nbytes, as a GGUF file types them),
 * vectors float32; shapes checked.  The last one given completes the
 * model. */
grx_status grx_mimi_set_tensor(grx_mimi *m, const char *name, const void *data, size_t nbytes);
/* A fresh decState (mimi.go:112-119): empty caches, position 0, no carried
 * rows. */
grx_status grx_mimi_reset(grx_mimi *m);
/* mimiDecoder.decode (mimi.go:122-152): n latents (host float32 [n][ldim],
 * already scaled back by the flow LM's mean and std) to
 * n * samples_per_latent samples in out (host), continuing the stream.
 * The speak loop's fade-in of the first frame (speak.go:180-184) is the
 * caller's.  GRX_ESIZE past max_latents. */
grx_status grx_mimi_decode(grx_mimi *m, const float *lat, int n, float *out);
/* The same with device buffers, enqueued on the context's stream. */
grx_status grx_mimi_decode_dev(grx_mimi *m, const float *lat, int n, float *out);
/* upsample x the product of the ratios (1920 at the english_2026-09
 * settings); 0 for NULL. */
int grx_mimi_samples_per_latent(const grx_mimi *m);
/* The Mimi decoder of a Pocket TTS GGUF file (the Mimi part of
 * pockettts.Load, pockettts/model.go:201-213 and 280-308, with decoder()
 * and resBlocks(), model.go:140-181): the file's name and source checks, the
 * frame size from pockettts.sample_rate / frame_rate, the settings
 * pockettts.mimi.{d_model, heads, ff, context, max_period, upsample} and
 * pockettts.seanet.{ratios, n_filters, dimension, kernel_size,
 * residual_kernel_size, last_kernel_size, dilation_base, compress,
 * n_residual_layers} with the reference's range checks and texts ("a SEANet
 * ratio of %d", "SEANet's ratios %v don't make %d-sample frames"), the
 * transformer's layers counted by their norm1.weight, and every tensor's
 * shape checked as mat()/vec() check it; matrices go to the device as
 * stored (Q8_0 or float32).  max_latents bounds the latents one decode call
 * takes; *hp_out (may be NULL) receives the settings. */
grx_status grx_mimi_load_gguf(grx_ctx *ctx, const char *path, int max_latents, grx_mimi_hparams *hp_out,
                              grx_mimi **out);

/* ---- FastConformer encoder with Q8_0 weights ---- */

/* Model.encode (conformer/encoder.go:432-489) of a FastConformer (HParams
 * of conformer/model.go:15-44, subsampling 8): the depthwise-striding
 * pre-encoder (encoder.go:123-167, causal or centred), xscale, and `layers`
 * Conformer blocks (encoder.go:411-429) with the attention limits of
 * offlineKeys (encoder.go:196-212) and the depthwise convolution's padding,
 * every Linear a Q8_0 weight on the int8 route as conformer/model.go:
 * 348-356 packs them.  A batch of utterances of the same frame count runs
 * at once; each utterance's output is the one it gets alone.  A
 * cache-aware ("chunked_limited") model also streams
 * (grx_conformer_stream_*). */
typedef struct {
    int d, heads, layers, dff, conv_kernel, sub_channels, n_mels;
    int xscaling; /* nonzero: x *= sqrt(d) after the pre-encoder (HParams.XScaling) */
    int conv_ln;  /* nonzero: conv_norm_type "layer_norm", else folded batch norm */
    /* The attention and convolution forms.  att_chunked nonzero:
     * AttStyle "chunked_limited", else "regular"; att_left, att_right:
     * the attention context (-1: no limit); conv_left, conv_right: the
     * depthwise convolution's padding (both -1: centred, else they add up
     * to conv_kernel - 1); causal_sub nonzero: the causal pre-encoder.
     * Every field is read: -1 where the model has no limit. */
    int att_chunked, att_left, att_right, conv_left, conv_right, causal_sub;
    /* Streaming settings (conformer/stream.go:23-69): the trained (left,
     * right) context pairs (att_context_size_choices) and the pre-encoder
     * cache, the rows it drops and the first chunk's sampling frames (-1:
     * NeMo's 9, 2 and 1). */
    int n_context_choices;
    int context_choices[8][2];
    int pre_encode_cache, drop_extra, sampling_frames_first;
} grx_conformer_hparams;

typedef struct grx_conformer grx_conformer;

grx_status grx_conformer_create(grx_ctx *ctx, const grx_conformer_hparams *hp, grx_conformer **out);
grx_status grx_conformer_destroy(grx_conformer *m);
/* loadEncoder (conformer/model.go:370-422) by the names it reads
 * ("enc.pre_encode.conv.0.weight", "enc.blocks.0.ff1.linear1.weight",
 * "enc.blocks.0.conv.bn.running_var", ...): Linear weights as ggml Q8_0 rows
 * (the pointwise convolutions may be float16 instead and are rounded by
 * Weight.ToQ8 at load, model.go:397-402; the pre-encoder's conv.3 and
 * conv.6 may be float32 and then take kern's float route), convolution taps
 * [c][taps] and vectors as float32.  Optional biases may be left out.
 * Shapes checked. */
grx_status grx_conformer_set_tensor(grx_conformer *m, const char *name, const void *data, size_t nbytes);
/* The encoder of a FastConformer GGUF file (conformer.Load, conformer/
 * model.go:163-422): the architecture check, the encoder and decoder
 * settings with the reference's checks and texts, then loadEncoder's
 * tensors in its order (the first missing one reported as there, optional
 * biases may be absent).  Linear weights go from the file to the device as
 * stored (Q8_0); pointwise convolutions may be float16 or float32 (rounded
 * by Weight.ToQ8); the pre-encoder's conv.3 / conv.6 may be float32 (the
 * float route, as converted files hold them).  Tensors that do not fit the
 * settings fail here ("the model file doesn't fit its own settings").
 * The attention and convolution forms and the streaming settings are
 * read as readEncoder and readHParams read them (att_context_size_choices
 * beyond 8 pairs are refused).  *hp_out (may be NULL) receives the
 * settings. */
grx_status grx_conformer_load_gguf(grx_ctx *ctx, const char *path, grx_conformer_hparams *hp_out,
                                   grx_conformer **out);
/* Encoder frames T for `frames` mel frames (three halvings, encoder.go:33-38,
 * causal ones for a causal pre-encoder). */
int grx_conformer_frames_out(const grx_conformer *m, int frames);
/* Model.encode of `batch` utterances: mel is [batch][n_mels][frames] float32
 * on the host (Mel.Compute's layout), valid[b] the real frames of each
 * (Mel.Valid, 1..frames).  out receives [batch][T][d]: of utterance b the
 * first lens[b] rows are the encoder output (encoder.go:488), the rest what
 * the computation leaves there.  lens may be NULL. */
grx_status grx_conformer_encode(grx_conformer *m, const float *mel, int batch, int frames, const int *valid,
                                float *out, int *lens);
/* The same with mel and out in device memory (valid on the host); returns
 * when the output is written. */
grx_status grx_conformer_encode_dev(grx_conformer *m, const float *mel, int batch, int frames, const int *valid,
                                    float *out);

/* ---- Cache-aware streaming of a FastConformer encoder ---- */

/* newGeom and newEncState (conformer/stream.go:23-88): `batch` streams
 * stepped together, with right context `right` (one of the model's
 * trained choices; the left context is the one trained with it).  Each
 * stream keeps, per layer, its last `left` attention key and value rows
 * and its last conv_left gated frames in device memory. */
typedef struct grx_conformer_stream grx_conformer_stream;
typedef struct {
    int right, chunk, left, left_chunks; /* encoder rows; chunk = right + 1 */
    int mel_first, mel_next;             /* mel frames of the first chunk and of the later ones */
    int mel_cache, drop;                 /* frames before each later chunk, and the encoder rows they give */
    int sample_first;                    /* the fewest frames a first chunk may have */
} grx_conformer_stream_geom;
grx_status grx_conformer_stream_create(grx_conformer *m, int right, int batch, grx_conformer_stream **out);
grx_status grx_conformer_stream_destroy(grx_conformer_stream *s);
grx_status grx_conformer_stream_geometry(const grx_conformer_stream *s, grx_conformer_stream_geom *g);
/* streamStep (stream.go:241-307) of one chunk per stream: mel is
 * [batch][n_mels][nf] float32 on the host (the cache frames first, as the
 * chunker cuts them), length[b] the real frames of each (1..nf).  The
 * first call is each stream's first chunk.  out receives [batch][chunk][d]:
 * stream b's first lens[b] rows are its encoder rows for the chunk (lens
 * may be NULL).  A chunk whose rows after the drop exceed one chunk is an
 * error; one that gives no rows leaves the streams unchanged. */
grx_status grx_conformer_stream_step(grx_conformer_stream *s, const float *mel, int nf, const int *length, float *out,
                                     int *lens);
/* The same with mel and out in device memory (length and lens on the
 * host); returns when the output is written. */
grx_status grx_conformer_stream_step_dev(grx_conformer_stream *s, const float *mel, int nf, const int *length,
                                         float *out, int *lens);

/* ---- RNN-T / TDT greedy decoder (prediction network and joint) ---- */

/* The transducer head of conformer/model.go:306-315 and the HParams it
 * reads (model.go:191-235): pred_hidden, pred_layers, pred_vocab (tokens
 * plus blank), joint_hidden, joint_act (0 "relu", 1 "sigmoid", 2 "tanh"),
 * tdt (nonzero: "tdt", with n_durations durations and max_symbols; RNN-T
 * takes no durations and 10 symbols a frame), blank (-1: pred_vocab - 1)
 * and d, the encoder width.  Widths are multiples of 32. */
typedef struct {
    int d, pred_hidden, pred_layers, pred_vocab, joint_hidden, joint_act;
    int tdt, n_durations, durations[16], max_symbols, blank;
} grx_rnnt_hparams;

/* Token (conformer/rnnt.go:10-15). */
typedef struct {
    int id, frame, duration;
    float p;
} grx_rnnt_token;

typedef struct grx_rnnt grx_rnnt;
/* DecoderState (rnnt.go:19-23): the LSTM's h and c per layer and the last
 * emitted token, in device memory. */
typedef struct grx_rnnt_state grx_rnnt_state;

grx_status grx_rnnt_create(grx_ctx *ctx, const grx_rnnt_hparams *hp, grx_rnnt **out);
grx_status grx_rnnt_destroy(grx_rnnt *m);
/* fromGGUF's decoder tensors by name (model.go:306-315): "pred.embed.weight"
 * (float32 [rows][pred_hidden], every id but blank has a row),
 * "pred.lstm.<i>.Wx" / ".Wh" (Q8_0 [4H][H]), "pred.lstm.<i>.bias" (float32,
 * the two NeMo biases summed), "joint.enc.weight" (Q8_0 [J][d]),
 * "joint.pred.weight" (Q8_0 [J][H]), "joint.out.weight" (Q8_0 [pred_vocab +
 * durations][J]) and their float32 biases.  The decoder is ready when all
 * are set. */
grx_status grx_rnnt_set_tensor(grx_rnnt *m, const char *name, const void *data, size_t nbytes);
/* The transducer head of a FastConformer GGUF file (conformer/model.go:
 * 191-235, 306-315, 337-339): readHParams' decoder settings with its checks
 * and texts, then the decoder tensors in fromGGUF's order (the first
 * missing one reported as there); Q8_0 matrices go to the device as stored
 * (other matrix types are refused), vectors are widened to float32.
 * Tensors that do not fit the settings fail ("the model file doesn't fit
 * its own settings").  *hp_out (may be NULL) receives the settings, blank
 * resolved. */
grx_status grx_rnnt_load_gguf(grx_ctx *ctx, const char *path, grx_rnnt_hparams *hp_out, grx_rnnt **out);
/* Model.NewDecoderState (rnnt.go:26-33): zeros, last = -1.  A state may
 * outlive its decoder, not the decoder's context. */
grx_status grx_rnnt_state_create(grx_rnnt *m, grx_rnnt_state **out);
grx_status grx_rnnt_state_destroy(grx_rnnt_state *s);
/* The state's h and c ([layers][pred_hidden] each, either may be NULL) and
 * last token, to the host / from the host. */
grx_status grx_rnnt_state_read(const grx_rnnt_state *s, float *h, float *c, int *last);
grx_status grx_rnnt_state_write(grx_rnnt_state *s, const float *h, const float *c, int last);
/* Model.Decode (rnnt.go:111-173): greedy RNN-T or TDT decoding of encoder
 * output enc [T][d] (host memory, or device memory when enc_on_device),
 * continuing from st and leaving the final state there (st NULL: start
 * fresh, no state kept); token frames are offset by frame_offset.  The
 * tokens go to out (room for cap; 16*T + 1024 always suffices) and their
 * number to *n_out; more than cap is GRX_ESIZE, with the first cap
 * written.  Each token's id, frame, duration and float32 probability are
 * the reference's. */
grx_status grx_rnnt_decode(grx_rnnt *m, const float *enc, int T, int enc_on_device, grx_rnnt_state *st,
                           int frame_offset, grx_rnnt_token *out, int cap, int *n_out);

/* ---- Fault injection, for tests of the cleanup paths ---- */

/* No counterpart in the reference (its tests reach its error paths through
 * panics turned into errors, conformer/robust_test.go:16-27, model.go:
 * 282-289).  For callers that test how the library fails: the n-th device
 * or pinned allocation from now on (n = 0: the next one) fails as out of
 * memory, so the call that makes it returns GRX_ENOMEM; the allocations
 * after it succeed again.  n < 0 disarms it.  Process-wide; not for use
 * while other threads call the library. */
void grx_debug_fail_alloc_after(long long n);
/* Allocations left before the injected failure, -1 when none is armed (the
 * failing one taken, or disarmed). */
long long grx_debug_alloc_countdown(void);

/* ---- Kernel choices, for tests and profiles ---- */

/* Stands in for the reference's test-only kernel switch setInt
 * (internal/kern/kernels_amd64.go:190-200), which picks which int8 kernel
 * later products take.  Overrides one of the library's kernel choices
 * by name: GEMM_MIN_M, GEMM_KERNEL, GEMM_NS, GEMM_KB, GEMV_WAVES, GEMV1,
 * CONF_ATTN_RQ, FUSE_LN, FUSE_XSCORES, WAVE_VALUES, ARGMAX_ATOMIC,
 * NO_GRAPH, GEMM_STAGE_A, GEMV_MX, GEMV1_ROWS, FUSE_SELF_ATTN; value -1
 * gives the choice back to the library.  The environment variable
 * GRX_<name>, read once, sets the starting value.  Every choice gives the
 * same results bit for bit.  Process-wide; a model whose HIP graph is
 * already captured keeps the kernels it captured.  GRX_EINVAL for an
 * unknown name. */
grx_status grx_debug_tune(const char *name, int value);

#ifdef __cplusplus
}
#endif
#endif
