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
#include <immintrin.h>
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
// an atomic counter by the calling thread and the pool's threads.
struct Pool {
    std::vector<std::thread> th;
    std::mutex mu;
    std::condition_variable cv, done_cv;
    std::function<void(int)> fn;
    std::atomic<int> next{0};
    int n = 0, gen = 0, busy = 0;
    bool stop = false;

    explicit Pool(int threads) {
        for (int i = 1; i < threads; ++i) th.emplace_back([this] { loop(); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> lk(mu);
            stop = true;
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
            {
                std::unique_lock<std::mutex> lk(mu);
                cv.wait(lk, [&] { return stop || gen != seen; });
                if (stop) return;
                seen = gen;
                ++busy;
            }
            drain();
            {
                std::lock_guard<std::mutex> lk(mu);
                if (--busy == 0) done_cv.notify_all();
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
        }
        cv.notify_all();
        drain();
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

}  // namespace

extern "C" {

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
