// grx_internal.h - shared declarations of libgrx.so (gfx950 only).
//
// Device helpers here restate, lane by lane, the arithmetic of the
// reference's kernels (github.com/xattribution/gorelaxor, cited file:line);
// they are written with explicit __fmul_rn/__fadd_rn/__fmaf_rn so that the
// compiler can neither fuse nor reorder them, and the library is built with
// -ffp-contract=off on top.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/grx.h"

// ---------------------------------------------------------------- host side

struct grx_ctx {
    int device;
    hipStream_t stream;
    void *scratch;        // device scratch for host-pointer calls, grown on demand
    size_t scratch_bytes;
};

// Q8_0 weight in HBM, packed once (grx_weight_q8_create).  Layout, for
// tiles of 64 rows (row r = 64*tile + lane):
//   qs: int8  [tiles][nb][2][64][16]  the 16 values 16h..16h+15 of block b
//   ds: f16   [tiles][nb][64]         the scale of block b
// Exactly 34 bytes per 32 weights (plus zero rows to a whole last tile).
// A wave owns a tile: lane l reads row 64*tile+l, each of its 16-byte value
// loads is one 1 KiB coalesced transaction for the wave and its scale load
// one 128-byte transaction.
struct grx_weight {
    int rows, cols, nb, tiles, device;
    int8_t *qs;
    uint16_t *ds;
    size_t bytes;
};

grx_status grx_fail(grx_status s, const char *fmt, ...);

// float_route.hip: kern.MatMul's float route for one row of activations
// (device buffers), for a Q8_0 weight that keeps its rows and for float32
enum { GRX_FEPI_STORE = 0, GRX_FEPI_SILU = 1, GRX_FEPI_GATE = 2 };
struct GrxFloatEpi {
    int kind = GRX_FEPI_STORE;
    const float *gate = nullptr;  // GATE: y[row] += gate[row] * (product + bias)
};
grx_status grx_float_gemv_q8(hipStream_t st, const grx_weight *w, const float *x, const float *bias, float *y,
                             GrxFloatEpi e = GrxFloatEpi());
grx_status grx_float_gemv_f32(hipStream_t st, const float *w, int n, int k, const float *x, const float *bias,
                              float *y, GrxFloatEpi e = GrxFloatEpi());
// kern.Linear of a float32 weight [n][k] over B groups of `per` rows (the
// k6x16 form for rows in whole groups of six when a group has more than 16,
// gemvRows for the rest); bias nullable.
grx_status grx_float_rows_f32(hipStream_t st, const float *x, const float *w, const float *bias, float *y, int B,
                              int per, int n, int k);
// quantU8 of m rows of k values (k % 32 == 0, rows lda apart) into q [m][k]
// and sc [m][k/32]
grx_status grx_quant_rows(hipStream_t st, const float *x, int lda, int m, int k, int8_t *q, float *sc);

// whisper_sample.hip: one row of logits through whisper's token rules and
// sampler (the public grx_whisper_rules / grx_whisper_seq, resolved)
struct GrxSampleArgs {
    int n, eot, sot, not_, nosp, solm, translate, transcribe, prev, beg, n_lang, space, tid0;
    int initial, last, penult, has_ts, seek_delta, n_suppress;
    float temp, r;
};
struct GrxSampleOut {
    int id, tid;
    float p, plog;
    int force_ts, n_terms;
};
// The decode loop of one window (transcribe.go:207-237) on the device: the
// sequence the rules read (seq of transcribe.go:100-115) and the loop's
// counter, read by the sampler before it samples and updated after.
struct GrxLoopDev {
    int i;  // iterations done
    int n_tokens, last, penult;
    int has_ts, seek_delta, result_len;
    int done, failed;
};
struct GrxLoopArgs {
    GrxLoopDev *st;          // nullptr: one sample from the arguments as given
    int *tok_w;              // the decoder's next token
    grx_whisper_token *rec;  // [n_max] each iteration's token
    const float *rs;         // [n_max] draws (temperature above 0), or nullptr
    int seek, seek_end, delta_min, win_frames, n_max;
};
#ifdef __cplusplus
// scratch: 2 x 65536 floats; out may be NULL in loop form
grx_status grx_sample_launch(hipStream_t st, const float *logits, const GrxSampleArgs &a, const int *suppress,
                             float *scratch, GrxSampleOut *out, const GrxLoopArgs &la = GrxLoopArgs{});
// the rules and sequence state in kernel form (checks the token ids)
grx_status grx_sample_args(const grx_whisper_rules *rules, const grx_whisper_seq *seq, int n, float temp, float r,
                           GrxSampleArgs *a);
// runs the sampler on device logits (or host ones, copied first) and
// returns the token (synchronous)
grx_status grx_sample_run(grx_ctx *ctx, const float *dev_logits, const float *host_logits, int n,
                          const grx_whisper_rules *rules, const grx_whisper_seq *seq, float temp, float r,
                          grx_whisper_token *out);
#endif

#ifdef __cplusplus
#include <vector>
// gguf.hip: a tensor's stored bytes and its ggml type code
grx_status grx_gguf_tensor_data(const grx_gguf *g, const char *name, int *type, std::vector<uint8_t> *out);
#endif
grx_status grx_hip_fail(hipError_t e, const char *what);

// Kernel choices that tests and profiles override (grx_debug_tune; the
// GRX_* environment variable of the same name, read once when the library
// first asks, sets the starting value).  -1 means "the library's own choice".
enum {
    GRX_TUNE_GEMM_MIN_M,      // fewest rows that take the matrix-core product
    GRX_TUNE_GEMM_KERNEL,     // 1 the whole-K register kernel, 2 the K-split one, 3 the LDS-staged one
    GRX_TUNE_GEMM_NS,         // 16-column tiles per wave of the register kernels: 1, 2 or 4
    GRX_TUNE_GEMM_KB,         // blocks per wave of the K-split kernel: 4, 8 or 16
    GRX_TUNE_GEMV_WAVES,      // waves per tile of the GEMV: 1, 2, 4, 8 or 16
    GRX_TUNE_GEMV1,           // 0: one-row products on the general GEMV kernel
    GRX_TUNE_CONF_ATTN_RQ,    // conformer attention: 0 unstaged, 8 or 16 query rows per workgroup
    GRX_TUNE_FUSE_LN,         // 0: batched decoder LayerNorm rows in their own launch
    GRX_TUNE_FUSE_XSCORES,    // 0: whisper cross scores without the fused query product
    GRX_TUNE_WAVE_VALUES,     // 0: whisper cross values on the wide-workgroup kernel
    GRX_TUNE_ARGMAX_ATOMIC,   // 1: the decoders' argmax through a contended atomic
    GRX_TUNE_NO_GRAPH,        // 1: model loops launch kernel by kernel (no HIP graphs)
    GRX_TUNE_GEMM_STAGE_A,    // 0: the K-split kernel reads activations straight from memory, 1: through LDS
    GRX_TUNE_GEMV_MX,         // 0: several-row GEMVs on the dot-product kernel, not the matrix-core one
    GRX_TUNE_GEMV1_ROWS,      // rows per workgroup of one-row products: 8, 16, 32 (slices) or 64 (whole tiles)
    GRX_TUNE_FUSE_SELF_ATTN,  // 0: whisper's q|k|v product and self-attention in launches of their own
    GRX_TUNE_CONF_DW,         // conformer depthwise convolution: 0 a workgroup per row, 1 windows in LDS,
                              // 2 a wave per frame
    GRX_TUNE_CONF_FUSE,       // 0: conformer LayerNorms, GLU and cache copies in launches of their own,
                              // 3: LayerNorms in the prologues of products of up to 32 rows too
                              // (default: of one-row products only)
    GRX_TUNE_CONF_ATTN_G8,    // 0: the conformer attention's few-row outputs one a thread, not 8 lanes each
    GRX_TUNE_CONF_ATTN_THREADS,  // 256 or 512: threads of the conformer attention's row-a-workgroup launch
    GRX_TUNE_COUNT
};
int grx_tune(int id);
// Every device and pinned allocation of the library: hipMalloc and
// hipHostMalloc, or the out-of-memory failure grx_debug_fail_alloc_after
// injects.
hipError_t grx_dev_malloc(void **p, size_t bytes);
hipError_t grx_pinned_malloc(void **p, size_t bytes);
// q8_gemv.hip: looks up grx_matmul_q8_dev_noalloc's device scratch on the
// current device, once (grx_ctx_create calls it)
void grx_noalloc_setup(int device);
grx_status grx_ctx_scratch(grx_ctx *ctx, size_t bytes, void **out);

#define GRX_HIP(expr)                                                       \
    do {                                                                    \
        hipError_t e_ = (expr);                                             \
        if (e_ != hipSuccess) return grx_hip_fail(e_, #expr);               \
    } while (0)

#define GRX_LAUNCHED(what)                                                  \
    do {                                                                    \
        hipError_t e_ = hipGetLastError();                                  \
        if (e_ != hipSuccess) return grx_hip_fail(e_, what);                \
    } while (0)

static inline int grx_ceil_div(int a, int b) { return (a + b - 1) / b; }

// ------------------------------------------------------------ device side

#define GRX_QK 32

__device__ __forceinline__ float grx_bits_f32(uint32_t u) { return __uint_as_float(u); }

// f16 -> f32, exact incl. subnormals (internal/kern/f16.go:14-33); the
// kernels run with f16 denormals kept (denorm mode 3), so the hardware
// conversion is exact.
__device__ __forceinline__ float grx_f16_to_f32(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

// f32 -> f16 round to nearest even with the reference's NaN and overflow
// results (internal/kern/f16.go:36-71), in integer arithmetic.
__device__ __forceinline__ uint16_t grx_f32_to_f16(float f) {
    uint32_t b = __float_as_uint(f);
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

// quantU8 for one block of 32 values (internal/kern/q8int.go:88-105,
// vnni_amd64.s:194-256): sc = amax*f32(1/127), id = 127/amax (0 for an
// all-zero block), q = clamp(rne(x*id), -128, 127), kept signed.
__device__ __forceinline__ float grx_quant_block(const float *x, int8_t *q) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < GRX_QK; ++i) {
        float a = fabsf(x[i]);
        amax = a > amax ? a : amax;
    }
    const float sc = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
    const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
#pragma unroll
    for (int i = 0; i < GRX_QK; ++i) {
        float r = rintf(__fmul_rn(x[i], id));
        r = fminf(fmaxf(r, -128.0f), 127.0f);
        q[i] = (int8_t)(int)r;
    }
    return sc;
}

// EXP8 of internal/kern/kernels_amd64.s:236-258, one lane.
__device__ __forceinline__ float grx_exp8(float x) {
    x = x > -87.0f ? x : -87.0f;
    x = x < 88.0f ? x : 88.0f;
    const float n = rintf(__fmul_rn(x, grx_bits_f32(0x3fb8aa3bu)));
    float r = __fmaf_rn(-n, grx_bits_f32(0x3f317200u), x);
    r = __fmaf_rn(-n, grx_bits_f32(0x35bfbe8eu), r);
    float p = grx_bits_f32(0x3ab60b61u);
    p = __fmaf_rn(p, r, grx_bits_f32(0x3c088889u));
    p = __fmaf_rn(p, r, grx_bits_f32(0x3d2aaaabu));
    p = __fmaf_rn(p, r, grx_bits_f32(0x3e2aaaabu));
    p = __fmaf_rn(p, r, 0.5f);
    p = __fmaf_rn(p, r, 1.0f);
    p = __fmaf_rn(p, r, 1.0f);
    const int ni = (int)n;
    return __fmul_rn(p, grx_bits_f32((uint32_t)(ni + 127) << 23));
}

// expf of internal/kern/mathx.go:7-33 (the scalar form), unfused, without
// branches: every case is computed and the reference's one selected (a
// divergent branch costs more than the few extra operations).  t is kept
// within +-256 before its conversion, which changes nothing for
// -87 <= x <= 88 (t in [-125, 127.5]); outside that range the result is
// the reference's 0 or +Inf.
__device__ __forceinline__ float grx_expf_go(float x) {
    float t = __fmul_rn(x, grx_bits_f32(0x3fb8aa3bu));
    t = __fadd_rn(t, 0.5f);
    const float tc = fminf(fmaxf(t, -256.0f), 256.0f);
    int ni = (int)tc;
    ni -= (float)ni > tc ? 1 : 0;  // floor
    const float n = (float)ni;
    float r = __fsub_rn(x, __fmul_rn(n, grx_bits_f32(0x3f317200u)));
    r = __fsub_rn(r, __fmul_rn(n, grx_bits_f32(0x35bfbe8eu)));
    float p = __fmul_rn(grx_bits_f32(0x3ab60b61u), r);
    p = __fadd_rn(p, grx_bits_f32(0x3c088889u));
    p = __fadd_rn(__fmul_rn(p, r), grx_bits_f32(0x3d2aaaabu));
    p = __fadd_rn(__fmul_rn(p, r), grx_bits_f32(0x3e2aaaabu));
    p = __fadd_rn(__fmul_rn(p, r), 0.5f);
    p = __fadd_rn(__fmul_rn(p, r), 1.0f);
    p = __fadd_rn(__fmul_rn(p, r), 1.0f);
    // ni < -126: p * 2^(ni+64) * 2^-64
    const float small = __fmul_rn(__fmul_rn(p, grx_bits_f32((uint32_t)(ni + 127 + 64) << 23)),
                                  grx_bits_f32(0x1f800000u));
    const float big = __fmul_rn(p, grx_bits_f32((uint32_t)(ni + 127) << 23));
    float e = ni < -126 ? small : big;
    e = x < -87.0f ? 0.0f : e;
    return x > 88.0f ? __builtin_inff() : e;
}

// geluAVX of internal/kern/kernels_amd64.s:299-338, one lane.
__device__ __forceinline__ float grx_gelu_avx(float v) {
    float u = __fmul_rn(v, v);
    u = __fmaf_rn(grx_bits_f32(0x3d372713u), u, 1.0f);
    u = __fmul_rn(u, v);
    u = __fmul_rn(u, grx_bits_f32(0x3f4c422au));
    u = u < 9.0f ? u : 9.0f;
    u = u > -9.0f ? u : -9.0f;
    float e = grx_exp8(__fadd_rn(u, u));
    e = __fadd_rn(e, 1.0f);
    float t = __fdiv_rn(2.0f, e);
    t = __fsub_rn(1.0f, t);
    t = __fadd_rn(1.0f, t);
    t = __fmul_rn(t, v);
    return __fmul_rn(t, 0.5f);
}

// gelu of internal/kern/mathx.go:36-52 (the scalar form, used past the last
// whole group of eight).
__device__ __forceinline__ float grx_gelu_go(float v) {
    float u = __fmul_rn(grx_bits_f32(0x3f4c422au), v);
    float w = __fmul_rn(grx_bits_f32(0x3d372713u), v);
    w = __fadd_rn(1.0f, __fmul_rn(w, v));
    u = __fmul_rn(u, w);
    // tanh(u) = 1 - 2/(e^{2u}+1), or +-1 past +-9; computed, then selected
    float t = __fsub_rn(1.0f, __fdiv_rn(2.0f, __fadd_rn(grx_expf_go(__fmul_rn(2.0f, u)), 1.0f)));
    t = u < -9.0f ? -1.0f : t;
    t = u > 9.0f ? 1.0f : t;
    return __fmul_rn(__fmul_rn(0.5f, v), __fadd_rn(1.0f, t));
}

// geluVec over an array of n values (kernels_amd64.go:119-129): element i
// takes the assembly form below n &^ 7, the scalar form past it.
__device__ __forceinline__ float grx_gelu_at(float v, int i, int n) {
    return i < (n & ~7) ? grx_gelu_avx(v) : grx_gelu_go(v);
}

// Launch helpers of the product kernels (q8_gemv.hip).
enum { GRX_PRO_PREQ = 0, GRX_PRO_QUANT = 1, GRX_PRO_LN = 2, GRX_PRO_EMBED_LN = 3, GRX_PRO_LN64 = 4,
       GRX_PRO_LN2 = 5 };  // LN2: LayerNorm (ln_w, ln_b) stored to x_out, then LayerNorm (ln_w2, ln_b2)
enum {
    GRX_EPI_STORE = 0,   // y = c
    GRX_EPI_RESID = 1,   // y = resid + c
    GRX_EPI_GELU = 2,    // y = geluVec(c) over the flat output
    GRX_EPI_QKV = 3,     // rows split in three: q, then K and V caches at *pos
    GRX_EPI_ARGMAX = 4,  // y = c (optional) and the first index of the maximum
    GRX_EPI_GELU_Q = 5,  // y = geluVec(c), and y rounded to Q8_0 into yq/ys
    GRX_EPI_QKV_ROPE = 6, // as QKV, with q and k rotated by the cos/sin table at pos
    GRX_EPI_XSCORES = 7,  // one row, tile = one head of 64: the head's cross-attention
                          // scores over a run of 64 keys (blockIdx.y) instead of y
    GRX_EPI_AXPY_HALF = 8,  // y = fma(0.5, c, resid) (a macaron feed-forward's residual)
    GRX_EPI_SILU_Q = 9,     // SiLU of c rounded to Q8_0 into yq/ys only (whole 32-row blocks)
    GRX_EPI_GLU = 10        // rows paired as a GLU: y[ch] = a * sigmoid(b) (grx_glu_pair)
};

// A copy of a product's outputs into per-stream rings of rows (a streaming
// encoder's caches): activation row r is row t = r % T of stream b = r / T,
// and goes to slot (ctl[c0] + ctl[c1] + t) % cap (c1 < 0: no second term)
// of stream b's ring (bstride floats apart, rows of width floats); output
// column n >= col0 lands in column n - col0.  twice: also to slot + cap (a
// ring read as one run of rows from any slot).
struct RingCopy {
    float *p = nullptr;
    size_t bstride = 0;
    int width = 0, col0 = 0, cap = 1, twice = 0, T = 1;
    const int *ctl = nullptr;
    int c0 = 0, c1 = -1;
};
__device__ __forceinline__ float *ring_row(const RingCopy &r, int head, int arow) {
    const int b = arow / r.T, t = arow - b * r.T;
    return r.p + (size_t)b * r.bstride + (size_t)((head + t) % r.cap) * r.width;
}
__device__ __forceinline__ int ring_head(const RingCopy &r) {
    return r.ctl[r.c0] + (r.c1 >= 0 ? r.ctl[r.c1] : 0);
}
__device__ __forceinline__ void ring_put(const RingCopy &r, float *row, int col, float v) {
    row[col] = v;
    if (r.twice) row[(size_t)r.cap * r.width + col] = v;
}

// The convolution module's GLU (conformer/encoder.go:350-361) on a product
// whose 2d output rows are stored paired: in each group of 32 rows, rows
// 0..15 are a-rows of channels 16g..16g+15 and rows 16..31 their b-rows
// (channel c's a-row is row c, its b-row row d + c, of the weight as
// stored in the file).  g = a * sigmoid(b), sigmoid(v) = 1/(1 + expf(-v))
// with the scalar expf; rows at or past the utterance's valid rows are 0.
__host__ __device__ __forceinline__ int grx_glu_row(int ch, bool b) { return 32 * (ch >> 4) + (ch & 15) + (b ? 16 : 0); }
__device__ __forceinline__ float grx_glu_pair(float a, float b) {
    const float sg = __fdiv_rn(1.0f, __fadd_rn(1.0f, grx_expf_go(-b)));
    return __fmul_rn(a, sg);
}

struct GemvArgs {
    const int8_t *qs;
    const uint16_t *ds;
    int rows, nb;
    // activations: PREQ reads xq/xs; QUANT and LN read x (lda apart)
    const int8_t *xq;
    const float *xs;
    const float *x;
    int lda;
    const float *ln_w, *ln_b;
    // output
    float *y;
    int ldc;
    const float *bias;
    const float *resid;
    int ldr;
    // QKV: rows [0,seg) -> y, [seg,2seg) -> kc[(pos+m)*seg], [2seg,3seg) -> vc
    int seg;
    float *kc, *vc;
    const int *pos;
    // ARGMAX: one 64-bit key per activation row; with counter set, the last
    // workgroup writes tok_w[m], hist[pos+m] and pos_w = pos+M
    unsigned long long *amax;
    unsigned int *counter;
    int *tok_w, *pos_w, *hist;
    // EMBED_LN: x rows from token embeddings (the tile layout of a weight)
    // plus positional rows, stored to x_out by tile 0
    const int *tok;
    const int8_t *emb_qs;
    const uint16_t *emb_ds;
    const float *pos_emb;
    float *x_out;
    // GELU_Q: the output rounded to Q8_0 (int8 [M][rows], f32 [M][rows/32])
    int8_t *yq;
    float *ys;
    // ordinary (cache-retained) weight loads instead of non-temporal ones
    int cacheable;
    // QKV_ROPE: cos/sin of every position's pair angles, [max_pos][half],
    // half = head_dim/2 (pairs are adjacent rows of a head)
    const float *rope_cos, *rope_sin;
    int rope_half;
    // LN64: the normalization's epsilon
    double ln_eps;
    // added to *pos for the rows of this launch (QKV, QKV_ROPE, EMBED_LN)
    int pos_add;
    // nonzero: the M rows are independent streams at one position (each
    // with its own token, KV cache kv_stream floats after the previous
    // stream's, and argmax record hist_stream ints apart) instead of
    // consecutive positions of one stream
    int streams;
    size_t kv_stream;
    int hist_stream;
    // ARGMAX with key slots: each workgroup writes its rows' best keys to
    // keys[tile][M] and a one-workgroup kernel ends the step (no counter)
    unsigned long long *keys;
    // XSCORES: pre-scaled cross keys [heads][nctx][64], scores [heads][nctx]
    const float *xk;
    int nctx;
    float *scores;
    // chunks > 1 (M of 2..8 rows, not ARGMAX, XSCORES nor streams): one
    // launch runs that many consecutive groups of M rows, group g
    // (blockIdx.z) with x, xq/xs, y, resid and yq/ys M*g rows on and
    // pos_add M*g larger
    int chunks;
    // LN2: the second LayerNorm's gain and bias
    const float *ln_w2, *ln_b2;
    // STORE and GLU: outputs also copied into rings (ring.p set)
    RingCopy ring;
    // GLU: valid rows per stream (rows of a stream T apart in the launch)
    const int *lens;
    int T;
};

grx_status grx_gemv_launch(hipStream_t st, int m, int pro, int epi, const GemvArgs &a,
                           int waves_hint);
// The many-row product on the matrix cores (q8_gemm.hip), same results.
grx_status grx_gemm_q8_launch(hipStream_t st, const grx_weight *w, const int8_t *xq, const float *xs, int m,
                              const float *bias, float *y, int ldc);
// Row kernels (rows.hip): LayerNorm + rounding to Q8_0 of `rows` rows of n
// values (x rows ldx apart) into xq [rows][n], xs [rows][n/32]; and the
// whisper decoder's embedding rows (token tok[r], position *pos) written to
// x [rows][n] before the same.
grx_status grx_ln_quant_rows(hipStream_t st, const float *x, int ldx, int rows, int n, const float *w,
                             const float *b, int8_t *xq, float *xs);
grx_status grx_embed_ln_quant_rows(hipStream_t st, const int *tok, const int *pos, const grx_weight *emb,
                                   const float *pos_emb, float *x, int rows, const float *w, const float *b,
                                   int8_t *xq, float *xs);

// Epilogues of the matrix-core product (q8_gemm.hip).
enum { GRX_GEMM_STORE = 0, GRX_GEMM_ADD = 1, GRX_GEMM_AXPY_HALF = 2, GRX_GEMM_SCALE = 3, GRX_GEMM_SILU_Q = 4,
       GRX_GEMM_GLU = 5 };
struct GemmOut {
    float *y = nullptr;  // [m][ldc] (STORE writes it, ADD/AXPY_HALF update it)
    int ldc = 0;
    int epi = GRX_GEMM_STORE;
    float scale = 1.0f;     // SCALE
    int8_t *yq = nullptr;   // SILU_Q: [m][rows] int8
    float *ys = nullptr;    //         [m][rows/32] scales
    // [m][rows] floats the K-split product may use to carry each output's
    // ordered chain from one run of blocks to the next when the weight has
    // more blocks than one workgroup holds (few rows only); NULL: none
    float *carry = nullptr;
    // GLU (weight rows paired as grx_glu_row lays them out): y [m][ldc]
    // holds rows/2 channels; rows of stream b = r / T at or past lens[b]
    // are zeroed
    const int *lens = nullptr;
    int T = 1;
    // STORE and GLU: outputs also copied into rings
    RingCopy ring;
    // A fused prologue instead of pre-rounded activations: x [m][lda]
    // LayerNorm'd (ln_w, ln_b) and rounded in the product; with ln_w2 set,
    // the first LayerNorm is stored to x_out [m][lda] and a second (ln_w2,
    // ln_b2) is rounded.  x_out must not alias x.  Only where
    // grx_gemm_q8_fuses says so (xq/xs then unused).
    const float *x = nullptr;
    int lda = 0;
    const float *ln_w = nullptr, *ln_b = nullptr, *ln_w2 = nullptr, *ln_b2 = nullptr;
    float *x_out = nullptr;
};
// Whether the product of m rows takes o's fused parts (prologue, GLU, ring
// copy) on the kernel it would run: the one-row GEMV, or the K-split kernel
// with staged activations in one run of blocks (a prologue: rows of at most
// 1024 values, at most two 16-row groups).
bool grx_gemm_q8_fuses(const grx_weight *w, int m, const GemmOut &o);
grx_status grx_gemm_q8_launch_ex(hipStream_t st, const grx_weight *w, const int8_t *xq, const float *xs, int m,
                                 const float *bias, const GemmOut &o);
// Fewest activation rows that take the matrix-core product (GRX_GEMM_MIN_M
// overrides it, for tests).
int grx_gemm_min_m(void);
int grx_gemv_pick_waves(int tiles, int nb, int m, int pro);
