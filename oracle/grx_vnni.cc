// grx_vnni.cc - the reference's CPU int8 product (Q8_0 weights, activations
// rounded to Q8_0) restated with x86 intrinsics, as the CPU baseline of the
// benchmark.  Test and benchmark infrastructure, never the product.
//
// Restates, from github.com/xattribution/gorelaxor:
//   packQ8Panels    internal/kern/q8int.go:35-64   16-row panels of 640-byte
//                                                  blocks: [8][16][4] int8,
//                                                  [16] f32 scales, [16] i32
//                                                  128 * sum(w)
//   quantU8avx      internal/kern/vnni_amd64.s:180-256
//   q8tileEVEX/VEX  internal/kern/vnni_amd64.s:1-178  6 x 16 tiles, twelve
//                                                  vpdpbusd accumulators,
//                                                  c = fma(f32(s - 128 sum w)
//                                                  * dw, da, c) per block
//   matmulQ8Int     internal/kern/q8int.go:148-223 quantization over rows,
//                                                  tasks = groups of 8 row
//                                                  tiles x runs of panels
//   parallel/tasks  internal/kern/gemm.go:52-108   (a persistent pool of
//                                                  threads and an atomic
//                                                  task counter here)
// The EVEX form needs AVX512-VNNI with AVX512-VL, the VEX form AVX-VNNI;
// both give the same bits, which equal the oracle's orc_matmul_q8_int.
//
// Also the reference's own whisper decode on the CPU, for timing only (its
// whisper package keeps every matrix as float16 and has no int8 route):
//   decode          whisper/decoder.go:33-140     one step over the token(s),
//                                                 self- and cross-attention
//   gemv, parallel  whisper/gemm.go:223-256,52-108 four rows per task
//   dot4f16avx      whisper/kernels_amd64.s:97-154 F16C widening, two
//                                                 accumulator sets per row
//   dot4f32avx      whisper/kernels_amd64.s:156-204 cross-attention rows
//   expSubAVX       internal/kern/kernels_amd64.s:236-297 (EXP8 per 8 lanes)
//   geluAVX         internal/kern/kernels_amd64.s:299-338
// Its outputs are not compared with anything: the weights are float16, not
// the Q8_0 the product path runs.
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace {

constexpr int kQK = 32, kPanelCols = 16, kTileRows = 6, kBlockBytes = 640, kQ8Bytes = 34;

float f16_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else {  // subnormal: normalize
            int ee = -1;
            uint32_t mm = m;
            do {
                ++ee;
                mm <<= 1;
            } while ((mm & 0x400) == 0);
            bits = s | ((uint32_t)(127 - 15 - ee) << 23) | ((mm & 0x3ff) << 13);
        }
    } else if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else {
        bits = s | ((e + 127 - 15) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// ---------------------------------------------------------------- rounding

// quantU8avx: per block of 32 values, amax by vmaxps, sc = amax * 1/127
// (the float 0x3c010204), id = 127 / amax (0 for a zero block), the values
// times id rounded to even by vcvtps2dq, saturated by the packs, plus 128.
__attribute__((target("avx2"))) void quant_u8(uint8_t *dst, float *sc, const float *x, int nb) {
    const __m256 absmask = _mm256_castsi256_ps(_mm256_set1_epi32(0x7fffffff));
    const __m256i perm = _mm256_setr_epi32(0, 4, 1, 5, 2, 6, 3, 7);
    const __m256i sign = _mm256_set1_epi32((int)0x80808080u);
    float inv127;
    const uint32_t ib = 0x3c010204u;
    memcpy(&inv127, &ib, 4);
    for (int b = 0; b < nb; ++b) {
        const float *xs = x + (size_t)b * kQK;
        __m256 v0 = _mm256_loadu_ps(xs), v1 = _mm256_loadu_ps(xs + 8), v2 = _mm256_loadu_ps(xs + 16),
               v3 = _mm256_loadu_ps(xs + 24);
        __m256 m = _mm256_max_ps(_mm256_max_ps(_mm256_and_ps(v0, absmask), _mm256_and_ps(v1, absmask)),
                                 _mm256_max_ps(_mm256_and_ps(v2, absmask), _mm256_and_ps(v3, absmask)));
        __m128 h = _mm_max_ps(_mm256_castps256_ps128(m), _mm256_extractf128_ps(m, 1));
        h = _mm_max_ps(h, _mm_movehl_ps(h, h));
        h = _mm_max_ss(h, _mm_shuffle_ps(h, h, 1));
        const float amax = _mm_cvtss_f32(h);
        sc[b] = amax * inv127;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        const __m256 vid = _mm256_set1_ps(id);
        const __m256i q0 = _mm256_cvtps_epi32(_mm256_mul_ps(v0, vid)), q1 = _mm256_cvtps_epi32(_mm256_mul_ps(v1, vid)),
                      q2 = _mm256_cvtps_epi32(_mm256_mul_ps(v2, vid)), q3 = _mm256_cvtps_epi32(_mm256_mul_ps(v3, vid));
        __m256i p = _mm256_packs_epi16(_mm256_packs_epi32(q0, q1), _mm256_packs_epi32(q2, q3));
        p = _mm256_permutevar8x32_epi32(p, perm);
        _mm256_storeu_si256(reinterpret_cast<__m256i *>(dst + (size_t)b * kQK), _mm256_xor_si256(p, sign));
    }
}

// ---------------------------------------------------------------- the tile

// C[6][16] += sum over blocks of da[r][b] * dw[c][b] * (sum ua*w - 128 sum w):
// per 4-value group, the panel's two 32-byte rows against each tile row's
// broadcast four activation bytes (twelve vpdpbusd accumulators); per
// block, FIN: minus 128 sum w, to float, times dw, then c = fma(., da, c).
// DPBUSD names the encoding; each form is compiled for its own ISA only.
#define GRX_Q8TILE(NAME, TARGET, DPBUSD)                                                                    \
    __attribute__((target(TARGET))) void NAME(int nb, const uint8_t *a, int lda, const float *as,           \
                                              const uint8_t *w, float *c, int ldc) {                         \
        for (int b = 0; b < nb; ++b) {                                                                      \
            const uint8_t *blk = w + (size_t)b * kBlockBytes;                                               \
            __m256i acc[kTileRows][2];                                                                      \
            for (int r = 0; r < kTileRows; ++r) acc[r][0] = acc[r][1] = _mm256_setzero_si256();             \
            for (int g = 0; g < kQK / 4; ++g) {                                                             \
                const __m256i w0 = _mm256_loadu_si256(reinterpret_cast<const __m256i *>(blk + g * 64));     \
                const __m256i w1 = _mm256_loadu_si256(reinterpret_cast<const __m256i *>(blk + g * 64 + 32)); \
                for (int r = 0; r < kTileRows; ++r) {                                                       \
                    int32_t four;                                                                           \
                    memcpy(&four, a + (size_t)r * lda + (size_t)b * kQK + 4 * g, 4);                        \
                    const __m256i ab = _mm256_set1_epi32(four);                                             \
                    acc[r][0] = DPBUSD(acc[r][0], ab, w0);                                                  \
                    acc[r][1] = DPBUSD(acc[r][1], ab, w1);                                                  \
                }                                                                                           \
            }                                                                                               \
            const __m256i off0 = _mm256_loadu_si256(reinterpret_cast<const __m256i *>(blk + 576));          \
            const __m256i off1 = _mm256_loadu_si256(reinterpret_cast<const __m256i *>(blk + 608));          \
            const __m256 dw0 = _mm256_loadu_ps(reinterpret_cast<const float *>(blk + 512));                 \
            const __m256 dw1 = _mm256_loadu_ps(reinterpret_cast<const float *>(blk + 544));                 \
            for (int r = 0; r < kTileRows; ++r) {                                                           \
                const __m256 t0 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_sub_epi32(acc[r][0], off0)), dw0); \
                const __m256 t1 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_sub_epi32(acc[r][1], off1)), dw1); \
                const __m256 da = _mm256_set1_ps(as[(size_t)r * nb + b]);                                   \
                float *cr = c + (size_t)r * ldc;                                                            \
                _mm256_storeu_ps(cr, _mm256_fmadd_ps(t0, da, _mm256_loadu_ps(cr)));                         \
                _mm256_storeu_ps(cr + 8, _mm256_fmadd_ps(t1, da, _mm256_loadu_ps(cr + 8)));                 \
            }                                                                                               \
        }                                                                                                   \
    }
GRX_Q8TILE(q8tile_evex, "avx2,fma,avx512vnni,avx512vl", _mm256_dpbusd_epi32)
GRX_Q8TILE(q8tile_vex, "avx2,fma,avxvnni", _mm256_dpbusd_avx_epi32)
#undef GRX_Q8TILE

// ---------------------------------------------------------------- threads

// A persistent pool: run(n, fn) calls fn(0..n-1), task indices taken from
// an atomic counter by the calling thread and the pool's threads.  Idle
// threads spin a few microseconds before they sleep on the condition
// variable, and the caller spins for the last tasks before it waits: a
// woken sleeper costs several microseconds, while the reference's
// goroutines are handed their tasks by spinning schedulers.
struct Pool {
    std::vector<std::thread> th;
    std::mutex mu;
    std::condition_variable cv, done_cv;
    std::function<void(int)> fn;
    std::atomic<int> next{0};
    int n = 0, gen = 0, busy = 0;
    bool stop = false;
    // copies of gen and busy read without the lock, only to end a spin
    std::atomic<int> gen_a{0}, busy_a{0};
    std::atomic<bool> stop_a{false};
    static constexpr int kSpin = 2000;

    explicit Pool(int threads) {
        for (int i = 1; i < threads; ++i) th.emplace_back([this] { loop(); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> lk(mu);
            stop = true;
            stop_a.store(true);
        }
        cv.notify_all();
        for (auto &t : th) t.join();
    }
    void drain() {
        for (;;) {
            const int i = next.fetch_add(1);
            if (i >= n) return;
            fn(i);
        }
    }
    void loop() {
        int seen = 0;
        for (;;) {
            for (int i = 0; i < kSpin && gen_a.load(std::memory_order_acquire) == seen && !stop_a.load(); ++i)
                _mm_pause();
            {
                std::unique_lock<std::mutex> lk(mu);
                cv.wait(lk, [&] { return stop || gen != seen; });
                if (stop) return;
                seen = gen;
                ++busy;
                busy_a.store(busy);
            }
            drain();
            {
                std::lock_guard<std::mutex> lk(mu);
                busy_a.store(--busy);
                if (busy == 0) done_cv.notify_all();
            }
        }
    }
    void run(int count, const std::function<void(int)> &f) {
        if (th.empty() || count <= 1) {
            for (int i = 0; i < count; ++i) f(i);
            return;
        }
        {
            std::lock_guard<std::mutex> lk(mu);
            fn = f;
            n = count;
            next.store(0);
            ++gen;
            gen_a.store(gen, std::memory_order_release);
        }
        cv.notify_all();
        drain();
        for (int i = 0; i < kSpin && busy_a.load() != 0; ++i) _mm_pause();
        std::unique_lock<std::mutex> lk(mu);
        done_cv.wait(lk, [&] { return busy == 0 && next.load() >= n; });
    }
};

Pool *g_pool = nullptr;
int g_threads = 0;

Pool &pool(int threads) {
    if (g_pool == nullptr || g_threads != threads) {
        delete g_pool;
        g_pool = new Pool(threads);
        g_threads = threads;
    }
    return *g_pool;
}

// ---------------------------------------------------------------- whisper F16

// dot4f16avx: out[r] = sum x[i] * w[r*ld+i], k a multiple of 16; per row two
// accumulators (values 0-7 and 8-15 of each 16), added, then summed across.
__attribute__((target("avx2,fma,f16c"))) void dot4_f16(const float *x, const uint16_t *w, size_t ld, int k,
                                                       float out[4]) {
    __m256 a[4], b[4];
    for (int r = 0; r < 4; ++r) a[r] = b[r] = _mm256_setzero_ps();
    for (int i = 0; i + 16 <= k; i += 16) {
        const __m256 x0 = _mm256_loadu_ps(x + i), x1 = _mm256_loadu_ps(x + i + 8);
        for (int r = 0; r < 4; ++r) {
            const uint16_t *wr = w + r * ld + i;
            a[r] = _mm256_fmadd_ps(x0, _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i *>(wr))), a[r]);
            b[r] = _mm256_fmadd_ps(x1, _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i *>(wr + 8))),
                                   b[r]);
        }
    }
    for (int r = 0; r < 4; ++r) {
        const __m256 v = _mm256_add_ps(a[r], b[r]);
        __m128 h = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
        h = _mm_hadd_ps(h, h);
        h = _mm_hadd_ps(h, h);
        out[r] = _mm_cvtss_f32(h);
    }
}

// dotF16Go for rows past the last whole group of four (and k past 16s).
float dot_f16_go(const float *x, const uint16_t *w, int k) {
    float s = 0.0f;
    for (int i = 0; i < k; ++i) s += x[i] * f16_to_f32(w[i]);
    return s;
}

// dot4f32avx: the same over float32 rows (k a multiple of 16 here).
__attribute__((target("avx2,fma"))) void dot4_f32(const float *x, const float *w, size_t ld, int k, float out[4]) {
    __m256 a[4], b[4];
    for (int r = 0; r < 4; ++r) a[r] = b[r] = _mm256_setzero_ps();
    int i = 0;
    for (; i + 16 <= k; i += 16) {
        const __m256 x0 = _mm256_loadu_ps(x + i), x1 = _mm256_loadu_ps(x + i + 8);
        for (int r = 0; r < 4; ++r) {
            a[r] = _mm256_fmadd_ps(x0, _mm256_loadu_ps(w + r * ld + i), a[r]);
            b[r] = _mm256_fmadd_ps(x1, _mm256_loadu_ps(w + r * ld + i + 8), b[r]);
        }
    }
    for (int r = 0; r < 4; ++r) {
        const __m256 v = _mm256_add_ps(a[r], b[r]);
        __m128 h = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
        h = _mm_hadd_ps(h, h);
        h = _mm_hadd_ps(h, h);
        float t = _mm_cvtss_f32(h);
        for (int j = i; j < k; ++j) t += x[j] * w[r * ld + j];
        out[r] = t;
    }
}

float dot_f32_go(const float *x, const float *y, int n) {
    float s = 0.0f;
    for (int i = 0; i < n; ++i) s += x[i] * y[i];
    return s;
}

// EXP8 on eight lanes (the same polynomial as the int8 path's SiLU).
__attribute__((target("avx2,fma"))) __m256 exp8(__m256 x) {
    x = _mm256_min_ps(_mm256_max_ps(x, _mm256_set1_ps(-87.0f)), _mm256_set1_ps(88.0f));
    const __m256 n = _mm256_round_ps(_mm256_mul_ps(x, _mm256_set1_ps(1.44269504f)), _MM_FROUND_TO_NEAREST_INT);
    __m256 r = _mm256_fnmadd_ps(n, _mm256_set1_ps(0.693359375f), x);
    r = _mm256_fnmadd_ps(n, _mm256_set1_ps(-2.12194440e-4f), r);
    __m256 p = _mm256_set1_ps(1.3888949e-3f);
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(8.3333338e-3f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(4.1666668e-2f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.6666667e-1f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0.5f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
    const __m256i e = _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(n), _mm256_set1_epi32(127)), 23);
    return _mm256_mul_ps(p, _mm256_castsi256_ps(e));
}

// softmax: max, e^(x - max) with their sum (expSubAVX over groups of
// eight, the scalar form past them), then times 1/sum.
__attribute__((target("avx2,fma"))) void softmax(float *x, int n) {
    float mx = -INFINITY;
    for (int i = 0; i < n; ++i) mx = x[i] > mx ? x[i] : mx;
    const int n8 = n & ~7;
    __m256 acc = _mm256_setzero_ps();
    const __m256 vm = _mm256_set1_ps(mx);
    for (int i = 0; i < n8; i += 8) {
        const __m256 e = exp8(_mm256_sub_ps(_mm256_loadu_ps(x + i), vm));
        _mm256_storeu_ps(x + i, e);
        acc = _mm256_add_ps(acc, e);
    }
    __m128 h = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    h = _mm_hadd_ps(h, h);
    h = _mm_hadd_ps(h, h);
    float s = _mm_cvtss_f32(h);
    for (int i = n8; i < n; ++i) {
        x[i] = expf(x[i] - mx);
        s += x[i];
    }
    const float inv = 1.0f / s;
    for (int i = 0; i < n; ++i) x[i] *= inv;
}

// geluAVX over groups of eight, the scalar form past them.
__attribute__((target("avx2,fma"))) void gelu(float *x, int n) {
    const int n8 = n & ~7;
    for (int i = 0; i < n8; i += 8) {
        const __m256 v = _mm256_loadu_ps(x + i);
        __m256 u = _mm256_fmadd_ps(_mm256_set1_ps(0.044715f), _mm256_mul_ps(v, v), _mm256_set1_ps(1.0f));
        u = _mm256_mul_ps(_mm256_mul_ps(u, v), _mm256_set1_ps(0.7978845608f));
        u = _mm256_min_ps(_mm256_max_ps(u, _mm256_set1_ps(-9.0f)), _mm256_set1_ps(9.0f));
        const __m256 e = _mm256_add_ps(exp8(_mm256_add_ps(u, u)), _mm256_set1_ps(1.0f));
        __m256 t = _mm256_sub_ps(_mm256_set1_ps(1.0f), _mm256_div_ps(_mm256_set1_ps(2.0f), e));
        t = _mm256_mul_ps(_mm256_mul_ps(_mm256_add_ps(_mm256_set1_ps(1.0f), t), v), _mm256_set1_ps(0.5f));
        _mm256_storeu_ps(x + i, t);
    }
    for (int i = n8; i < n; ++i) {
        const float v = x[i], u = 0.7978845608f * v * (1.0f + 0.044715f * v * v);
        const float t = u > 9.0f ? 1.0f : u < -9.0f ? -1.0f : 1.0f - 2.0f / (expf(2.0f * u) + 1.0f);
        x[i] = 0.5f * v * (1.0f + t);
    }
}

void layer_norm(float *y, const float *x, int n, const float *w, const float *b) {
    double sum = 0;
    for (int i = 0; i < n; ++i) sum += x[i];
    const float mean = (float)(sum / n);
    double vs = 0;
    for (int i = 0; i < n; ++i) {
        const double d = (double)(x[i] - mean);
        vs += d * d;
    }
    const float inv = (float)(1.0 / sqrt(vs / n + 1e-5));
    for (int i = 0; i < n; ++i) y[i] = (x[i] - mean) * inv * w[i] + b[i];
}

// gemv: y[n] = W[n][k] . x + bias, (n+3)/4 tasks of four rows over the
// pool (one thread below 2^16 multiply-adds), contiguous task ranges.
void gemv_f16(float *y, const float *x, const uint16_t *w, int n, int k, const float *bias, int threads) {
    const int groups = (n + 3) / 4;
    const int tt = (long)n * k < (1 << 16) ? 1 : threads;
    auto part = [&](int lo, int hi) {
        float out[4];
        for (int g = lo; g < hi; ++g) {
            const int j = 4 * g;
            if (j + 4 <= n) {
                const int kk = k & ~15;
                if (kk > 0) dot4_f16(x, w + (size_t)j * k, k, kk, out);
                else out[0] = out[1] = out[2] = out[3] = 0.0f;
                for (int r = 0; r < 4; ++r) {
                    if (kk < k) out[r] += dot_f16_go(x + kk, w + (size_t)(j + r) * k + kk, k - kk);
                    y[j + r] = out[r];
                }
            } else {
                for (int jj = j; jj < n; ++jj) y[jj] = dot_f16_go(x, w + (size_t)jj * k, k);
            }
            if (bias)
                for (int jj = j; jj < std::min(j + 4, n); ++jj) y[jj] += bias[jj];
        }
    };
    if (tt <= 1) {
        part(0, groups);
        return;
    }
    const int parts = std::min(tt, groups);
    pool(tt).run(parts, [&](int t) { part(groups * t / parts, groups * (t + 1) / parts); });
}

}  // namespace

extern "C" {

// The reference's whisper decoder with float16 matrices (whisper/decoder.go).
typedef struct {
    const float *attn_ln_w, *attn_ln_b;
    const uint16_t *q, *k, *v, *o;
    const float *q_b, *v_b, *o_b;
    const float *x_ln_w, *x_ln_b;
    const uint16_t *xq, *xo;
    const float *xq_b, *xo_b;
    const float *mlp_ln_w, *mlp_ln_b;
    const uint16_t *fc1, *fc2;
    const float *fc1_b, *fc2_b;
    const float *cross_k; /* [head][audio_ctx][head_dim] */
    const float *cross_v; /* [head][head_dim][audio_ctx] */
    float *self_k, *self_v; /* [text_ctx][state] */
} f16w_layer;

typedef struct {
    int n_vocab, n_text_ctx, n_state, n_head, n_layer, n_audio_ctx;
    const uint16_t *tok_emb; /* [n_vocab][n_state] */
    const float *dec_pos, *dec_ln_w, *dec_ln_b;
    f16w_layer *layers;
    int n;
} f16w_model;

// One decode call over nt < 6 tokens (rows through gemv one at a time, as
// matmul does below its 6-row tile); logits of the last token.
int f16w_decode(f16w_model *m, const int *tokens, int nt, float *logits, int threads) {
    const int st = m->n_state, nh = m->n_head, hd = st / nh, nctx = m->n_audio_ctx, pos0 = m->n;
    if (nt < 1 || nt >= kTileRows || pos0 + nt > m->n_text_ctx) return -1;
    if (threads < 1) threads = 1;
    std::vector<float> x((size_t)nt * st), cur((size_t)nt * st), q((size_t)nt * st), att((size_t)nt * st),
        ff((size_t)nt * 4 * st), sbuf((size_t)nt * nh * std::max(nctx, pos0 + nt));
    const int sw = std::max(nctx, pos0 + nt);
    const float sc = (float)(1.0 / sqrt((double)hd));
    for (int i = 0; i < nt; ++i)
        for (int j = 0; j < st; ++j)
            x[(size_t)i * st + j] = f16_to_f32(m->tok_emb[(size_t)tokens[i] * st + j]) + m->dec_pos[(size_t)(pos0 + i) * st + j];
    auto lin = [&](float *y, int ldy, const float *a, int lda, int n, int k, const uint16_t *w, const float *b) {
        for (int i = 0; i < nt; ++i) gemv_f16(y + (size_t)i * ldy, a + (size_t)i * lda, w, n, k, b, threads);
    };
    auto jobs = [&](const std::function<void(int)> &fn) {
        if (threads <= 1) {
            for (int j = 0; j < nt * nh; ++j) fn(j);
        } else {
            pool(threads).run(nt * nh, fn);
        }
    };
    for (int li = 0; li < m->n_layer; ++li) {
        const f16w_layer &L = m->layers[li];
        for (int i = 0; i < nt; ++i) layer_norm(&cur[(size_t)i * st], &x[(size_t)i * st], st, L.attn_ln_w, L.attn_ln_b);
        lin(q.data(), st, cur.data(), st, st, st, L.q, L.q_b);
        lin(L.self_k + (size_t)pos0 * st, st, cur.data(), st, st, st, L.k, nullptr);
        lin(L.self_v + (size_t)pos0 * st, st, cur.data(), st, st, st, L.v, L.v_b);
        jobs([&](int job) {
            const int i = job / nh, h = job % nh, n = pos0 + i + 1;
            float *s = &sbuf[(size_t)job * sw];
            const float *qi = &q[(size_t)i * st + h * hd];
            for (int j = 0; j < n; ++j) s[j] = dot_f32_go(qi, L.self_k + (size_t)j * st + h * hd, hd) * sc;
            softmax(s, n);
            float *out = &att[(size_t)i * st + h * hd];
            for (int d = 0; d < hd; ++d) out[d] = 0.0f;
            for (int j = 0; j < n; ++j) {
                const float *vj = L.self_v + (size_t)j * st + h * hd;
                for (int d = 0; d < hd; ++d) out[d] += s[j] * vj[d];
            }
        });
        lin(cur.data(), st, att.data(), st, st, st, L.o, L.o_b);
        for (size_t t = 0; t < x.size(); ++t) x[t] += cur[t];
        for (int i = 0; i < nt; ++i) layer_norm(&cur[(size_t)i * st], &x[(size_t)i * st], st, L.x_ln_w, L.x_ln_b);
        lin(q.data(), st, cur.data(), st, st, st, L.xq, L.xq_b);
        jobs([&](int job) {
            const int i = job / nh, h = job % nh;
            const float *kd = L.cross_k + (size_t)h * nctx * hd, *vd = L.cross_v + (size_t)h * nctx * hd;
            const float *qi = &q[(size_t)i * st + h * hd];
            float *s = &sbuf[(size_t)job * sw];
            float o4[4];
            int j = 0;
            for (; j + 4 <= nctx; j += 4) {
                dot4_f32(qi, kd + (size_t)j * hd, hd, hd, o4);
                for (int r = 0; r < 4; ++r) s[j + r] = o4[r];
            }
            for (; j < nctx; ++j) s[j] = dot_f32_go(qi, kd + (size_t)j * hd, hd);
            softmax(s, nctx);
            float *out = &att[(size_t)i * st + h * hd];
            int d = 0;
            for (; d + 4 <= hd; d += 4) {
                dot4_f32(s, vd + (size_t)d * nctx, nctx, nctx, o4);
                for (int r = 0; r < 4; ++r) out[d + r] = o4[r];
            }
            for (; d < hd; ++d) out[d] = dot_f32_go(s, vd + (size_t)d * nctx, nctx);
        });
        lin(cur.data(), st, att.data(), st, st, st, L.xo, L.xo_b);
        for (size_t t = 0; t < x.size(); ++t) x[t] += cur[t];
        for (int i = 0; i < nt; ++i) layer_norm(&cur[(size_t)i * st], &x[(size_t)i * st], st, L.mlp_ln_w, L.mlp_ln_b);
        lin(ff.data(), 4 * st, cur.data(), st, 4 * st, st, L.fc1, L.fc1_b);
        gelu(ff.data(), nt * 4 * st);
        lin(cur.data(), st, ff.data(), 4 * st, st, 4 * st, L.fc2, L.fc2_b);
        for (size_t t = 0; t < x.size(); ++t) x[t] += cur[t];
    }
    m->n = pos0 + nt;
    std::vector<float> row(st);
    layer_norm(row.data(), &x[(size_t)(nt - 1) * st], st, m->dec_ln_w, m->dec_ln_b);
    gemv_f16(logits, row.data(), m->tok_emb, m->n_vocab, st, nullptr, threads);
    return 0;
}


// 2: the EVEX form (AVX512-VNNI + AVX512-VL), 1: the VEX form (AVX-VNNI),
// 0: neither (the baseline cannot run here).
int vnni_kind(void) {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512vl")) return 2;
    if (__builtin_cpu_supports("avxvnni")) return 1;
    return 0;
}

size_t vnni_panel_bytes(int n, int k) {
    return (size_t)((n + kPanelCols - 1) / kPanelCols) * (k / kQK) * kBlockBytes;
}

// packQ8Panels of n Q8_0 rows of k values (ggml blocks) into out.
void vnni_pack(const uint8_t *q, int n, int k, uint8_t *out) {
    const int nb = k / kQK, np = (n + kPanelCols - 1) / kPanelCols;
    const size_t ld = (size_t)nb * kQ8Bytes;
    memset(out, 0, vnni_panel_bytes(n, k));
    for (int pi = 0; pi < np; ++pi)
        for (int b = 0; b < nb; ++b) {
            uint8_t *dst = out + ((size_t)pi * nb + b) * kBlockBytes;
            for (int j = 0; j < kPanelCols; ++j) {
                const int col = pi * kPanelCols + j;
                if (col >= n) continue;
                const uint8_t *blk = q + (size_t)col * ld + (size_t)b * kQ8Bytes;
                int32_t s = 0;
                for (int g = 0; g < kQK / 4; ++g) {
                    memcpy(dst + g * 64 + j * 4, blk + 2 + 4 * g, 4);
                    for (int i = 0; i < 4; ++i) s += (int8_t)blk[2 + 4 * g + i];
                }
                const float d = f16_to_f32((uint16_t)(blk[0] | blk[1] << 8));
                const int32_t off = 128 * s;
                memcpy(dst + 512 + j * 4, &d, 4);
                memcpy(dst + 576 + j * 4, &off, 4);
            }
        }
}

// matmulQ8Int: c[m][ldc] = a[m][lda] . W^T + bias with W as panels (n
// rows of k).  qa / sc: scratch of ceil(m/6)*6*k bytes and as many * k/32
// floats.  threads: the reference's `threads` argument.  Returns -1 when
// the processor has no VNNI.
int vnni_matmul(float *c, int ldc, const float *a, int lda, int m, const uint8_t *panels, int n, int k,
                const float *bias, int threads, uint8_t *qa, float *sc) {
    const int kind = vnni_kind();
    if (kind == 0) return -1;
    const int nb = k / kQK, np = (n + kPanelCols - 1) / kPanelCols;
    const int mp = (m + kTileRows - 1) / kTileRows * kTileRows;
    if (threads < 1) threads = 1;
    const int qt = (long)m * k < (1 << 15) ? 1 : threads;
    auto quant_rows = [&](int lo, int hi) {
        for (int i = lo; i < hi; ++i) quant_u8(qa + (size_t)i * k, sc + (size_t)i * nb, a + (size_t)i * lda, nb);
    };
    if (qt <= 1 || m <= 1) {
        quant_rows(0, m);
    } else {  // parallel(m, qt, ...): contiguous row ranges
        const int parts = std::min(qt, m);
        pool(threads).run(parts, [&](int t) { quant_rows(m * t / parts, m * (t + 1) / parts); });
    }
    memset(qa + (size_t)m * k, 128, (size_t)(mp - m) * k);
    memset(sc + (size_t)m * nb, 0, (size_t)(mp - m) * nb * sizeof(float));
    for (int i = 0; i < m; ++i) {
        float *ci = c + (size_t)i * ldc;
        if (bias)
            memcpy(ci, bias, (size_t)n * 4);
        else
            memset(ci, 0, (size_t)n * 4);
    }
    const int tiles = mp / kTileRows, group = 8;
    const int rowGroups = (tiles + group - 1) / group;
    int chunks = 1;
    if (threads > 1) chunks = std::min(np, std::max(1, (4 * threads + rowGroups - 1) / rowGroups));
    int tt = threads;
    if ((long)m * n * k < (1 << 18)) tt = 1;
    auto task = [&](int t) {
        const int g = t / chunks, ch = t % chunks;
        const int t0 = g * group, t1 = std::min((g + 1) * group, tiles);
        const int p0 = np * ch / chunks, p1 = np * (ch + 1) / chunks;
        float tile[kTileRows * kPanelCols];
        for (int p = p0; p < p1; ++p) {
            const uint8_t *wp = panels + (size_t)p * nb * kBlockBytes;
            const int col = p * kPanelCols, cols = std::min(kPanelCols, n - col);
            for (int ti = t0; ti < t1; ++ti) {
                const int r0 = ti * kTileRows, rows = std::min(kTileRows, m - r0);
                const uint8_t *ar = qa + (size_t)r0 * k;
                const float *as = sc + (size_t)r0 * nb;
                if (rows == kTileRows && cols == kPanelCols) {
                    if (kind == 2)
                        q8tile_evex(nb, ar, k, as, wp, c + (size_t)r0 * ldc + col, ldc);
                    else
                        q8tile_vex(nb, ar, k, as, wp, c + (size_t)r0 * ldc + col, ldc);
                    continue;
                }
                memset(tile, 0, sizeof tile);
                for (int r = 0; r < rows; ++r)
                    memcpy(tile + r * kPanelCols, c + (size_t)(r0 + r) * ldc + col, (size_t)cols * 4);
                if (kind == 2)
                    q8tile_evex(nb, ar, k, as, wp, tile, kPanelCols);
                else
                    q8tile_vex(nb, ar, k, as, wp, tile, kPanelCols);
                for (int r = 0; r < rows; ++r)
                    memcpy(c + (size_t)(r0 + r) * ldc + col, tile + r * kPanelCols, (size_t)cols * 4);
            }
        }
    };
    const int ntasks = rowGroups * chunks;
    if (tt <= 1)
        for (int t = 0; t < ntasks; ++t) task(t);
    else
        pool(tt).run(ntasks, task);
    return 0;
}

// kern.MatMul on the int8 route for the oracle's graphs (the hook
// orc_set_q8_product installs): matmulQ8Int over panels packed once per
// weight on first use, as Weight.Pack does lazily (q8int.go:81-84), at
// vnni_set_threads threads.  A weight is known by its ggml bytes' address,
// shape and a sample of its bytes (vnni_forget drops every packed weight).
namespace {
struct Packed {
    int n = 0, k = 0;
    uint64_t tag = 0;
    std::vector<uint8_t> panels;
};
std::mutex g_pack_mu;
std::vector<std::pair<const uint8_t *, Packed>> g_packed;
std::atomic<int> g_product_threads{1};
uint64_t bytes_tag(const uint8_t *q, size_t nbytes) {
    uint64_t h = 1469598103934665603ull;
    const size_t step = nbytes / 61 + 1;
    for (size_t i = 0; i < nbytes; i += step) h = (h ^ q[i]) * 1099511628211ull;
    return h ^ q[nbytes - 1];
}
}  // namespace

void vnni_set_threads(int threads) { g_product_threads.store(threads < 1 ? 1 : threads); }

void vnni_forget(void) {
    std::lock_guard<std::mutex> lk(g_pack_mu);
    g_packed.clear();
}

void vnni_q8_product(float *c, int ldc, const float *a, int lda, int m, const uint8_t *wq, int n, int k,
                     const float *bias) {
    if (m == 0 || n == 0) return;
    const size_t nbytes = (size_t)n * (k / kQK) * kQ8Bytes;
    const uint64_t tag = bytes_tag(wq, nbytes);
    const uint8_t *panels = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_pack_mu);
        for (auto &e : g_packed)
            if (e.first == wq && e.second.n == n && e.second.k == k && e.second.tag == tag) panels = e.second.panels.data();
        if (panels == nullptr) {
            Packed p;
            p.n = n;
            p.k = k;
            p.tag = tag;
            p.panels.resize(vnni_panel_bytes(n, k));
            vnni_pack(wq, n, k, p.panels.data());
            g_packed.emplace_back(wq, std::move(p));
            panels = g_packed.back().second.panels.data();
        }
    }
    const int mp = (m + kTileRows - 1) / kTileRows * kTileRows;
    thread_local std::vector<uint8_t> qa;
    thread_local std::vector<float> sc;
    if (qa.size() < (size_t)mp * k) qa.resize((size_t)mp * k);
    if (sc.size() < (size_t)mp * (k / kQK)) sc.resize((size_t)mp * (k / kQK));
    vnni_matmul(c, ldc, a, lda, m, panels, n, k, bias, g_product_threads.load(), qa.data(), sc.data());
}

// The benchmark's CPU loop: reps passes over `count` matrices (panels
// panel_stride bytes apart), one matmulQ8Int of the single row x each, as a
// caller of kern.MatMul issues them; y receives each matrix's n outputs.
int vnni_ring(float *y, const float *x, const uint8_t *panels, size_t panel_stride, int count, int n, int k,
              int threads, int reps, uint8_t *qa, float *sc) {
    for (int r = 0; r < reps; ++r)
        for (int i = 0; i < count; ++i) {
            const int rc = vnni_matmul(y + (size_t)i * n, n, x, k, 1, panels + (size_t)i * panel_stride, n, k,
                                       nullptr, threads, qa, sc);
            if (rc != 0) return rc;
        }
    return 0;
}

}  // extern "C"
