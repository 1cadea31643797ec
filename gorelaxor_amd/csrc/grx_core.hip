// grx_core.hip - library state, errors, contexts and Q8_0 weights.
//
// Stands in for kern.Weight and its constructors (internal/kern/kern.go:38-179,
// q8int.go:15-84 of github.com/xattribution/gorelaxor): a weight is copied to
// HBM once and repacked into the tile layout of grx_internal.h.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <stdlib.h>

#include <atomic>
#include <mutex>
#include <string>

#include "grx_internal.h"

static thread_local std::string g_last_error;

// Allocations left before an injected out-of-memory failure (-1: none).
static std::atomic<long long> g_alloc_countdown{-1};

// Whether this allocation is the one grx_debug_fail_alloc_after named; the
// countdown then stops, so later allocations (the cleanup's) succeed.
static bool alloc_injected_failure() {
    long long c = g_alloc_countdown.load();
    while (c >= 0)
        if (g_alloc_countdown.compare_exchange_weak(c, c - 1)) return c == 0;
    return false;
}

hipError_t grx_dev_malloc(void **p, size_t bytes) {
    *p = nullptr;
    if (alloc_injected_failure()) return hipErrorOutOfMemory;
    return hipMalloc(p, bytes);
}

hipError_t grx_pinned_malloc(void **p, size_t bytes) {
    *p = nullptr;
    if (alloc_injected_failure()) return hipErrorOutOfMemory;
    return hipHostMalloc(p, bytes, hipHostMallocDefault);
}

extern "C" void grx_debug_fail_alloc_after(long long n) { g_alloc_countdown.store(n < 0 ? -1 : n); }

extern "C" long long grx_debug_alloc_countdown(void) { return g_alloc_countdown.load(); }

// The kernel-choice table: names (the GRX_* environment variables without
// their prefix) in the order of the GRX_TUNE_* ids.
static const char *const kTuneNames[GRX_TUNE_COUNT] = {
    "GEMM_MIN_M", "GEMM_KERNEL", "GEMM_NS",    "GEMM_KB",     "GEMV_WAVES",    "GEMV1",
    "CONF_ATTN_RQ", "FUSE_LN",   "FUSE_XSCORES", "WAVE_VALUES", "ARGMAX_ATOMIC", "NO_GRAPH",
    "GEMM_STAGE_A", "GEMV_MX", "GEMV1_ROWS", "FUSE_SELF_ATTN", "CONF_DW", "CONF_FUSE", "CONF_ATTN_G8",
    "CONF_ATTN_THREADS"};
static std::atomic<int> g_tune[GRX_TUNE_COUNT];
static std::once_flag g_tune_once;

static void tune_init() {
    for (int i = 0; i < GRX_TUNE_COUNT; ++i) {
        const std::string env = std::string("GRX_") + kTuneNames[i];
        const char *v = getenv(env.c_str());
        g_tune[i].store(v && v[0] ? atoi(v) : -1);
    }
}

int grx_tune(int id) {
    std::call_once(g_tune_once, tune_init);
    return (id >= 0 && id < GRX_TUNE_COUNT) ? g_tune[id].load(std::memory_order_relaxed) : -1;
}

extern "C" grx_status grx_debug_tune(const char *name, int value) {
    std::call_once(g_tune_once, tune_init);
    if (name != nullptr)
        for (int i = 0; i < GRX_TUNE_COUNT; ++i)
            if (strcmp(name, kTuneNames[i]) == 0) {
                g_tune[i].store(value < 0 ? -1 : value);
                return GRX_OK;
            }
    return grx_fail(GRX_EINVAL, "grx_debug_tune: no setting named %s", name ? name : "(null)");
}

grx_status grx_fail(grx_status s, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return s;
}

grx_status grx_hip_fail(hipError_t e, const char *what) {
    return grx_fail(e == hipErrorOutOfMemory ? GRX_ENOMEM : GRX_EDEVICE, "grx: %s: %s", what,
                    hipGetErrorString(e));
}

extern "C" int grx_version(void) { return 1; }

extern "C" const char *grx_last_error(void) { return g_last_error.c_str(); }

extern "C" int grx_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

// ------------------------------------------------------------ contexts

extern "C" grx_status grx_ctx_create(int device, grx_ctx **out) {
    if (!out) return grx_fail(GRX_EINVAL, "grx_ctx_create: out is NULL");
    *out = nullptr;
    int n = grx_device_count();
    if (n == 0) return grx_fail(GRX_ENODEV, "grx_ctx_create: no GPU is visible");
    if (device < 0 || device >= n)
        return grx_fail(GRX_EINVAL, "grx_ctx_create: device %d of %d", device, n);
    hipDeviceProp_t prop;
    GRX_HIP(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return grx_fail(GRX_ENODEV, "grx_ctx_create: device %d is %s, this library is built for gfx950",
                        device, prop.gcnArchName);
    GRX_HIP(hipSetDevice(device));
    grx_ctx *c = new grx_ctx();
    c->device = device;
    // a blocking stream: ordered with the legacy default stream other HIP users
    // (torch's default stream among them) enqueue on
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamDefault);
    if (e != hipSuccess) {
        delete c;
        return grx_hip_fail(e, "hipStreamCreateWithFlags");
    }
    grx_noalloc_setup(device);  // grx_matmul_q8_dev_noalloc's scratch address on this device
    *out = c;
    return GRX_OK;
}

extern "C" grx_status grx_ctx_destroy(grx_ctx *ctx) {
    if (!ctx) return GRX_OK;
    GRX_HIP(hipSetDevice(ctx->device));
    GRX_HIP(hipStreamSynchronize(ctx->stream));
    if (ctx->scratch) GRX_HIP(hipFree(ctx->scratch));
    GRX_HIP(hipStreamDestroy(ctx->stream));
    delete ctx;
    return GRX_OK;
}

extern "C" grx_status grx_ctx_sync(grx_ctx *ctx) {
    if (!ctx) return grx_fail(GRX_EINVAL, "grx_ctx_sync: ctx is NULL");
    GRX_HIP(hipStreamSynchronize(ctx->stream));
    return GRX_OK;
}

extern "C" void *grx_ctx_stream(grx_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

grx_status grx_ctx_scratch(grx_ctx *ctx, size_t bytes, void **out) {
    if (bytes > ctx->scratch_bytes) {
        GRX_HIP(hipStreamSynchronize(ctx->stream));
        if (ctx->scratch) GRX_HIP(hipFree(ctx->scratch));
        ctx->scratch = nullptr;
        ctx->scratch_bytes = 0;
        size_t want = bytes + bytes / 4 + 4096;
        GRX_HIP(grx_dev_malloc(&ctx->scratch, want));
        ctx->scratch_bytes = want;
    }
    *out = ctx->scratch;
    return GRX_OK;
}

// ------------------------------------------------------------ weights

// One thread per (tile, block, lane): moves the 32 values and the scale of
// block b of row 64*tile+lane from the ggml row layout (34-byte blocks) into
// the tile layout; rows past the matrix and blocks past nb are zero.
__global__ void grx_pack_q8_kernel(const uint8_t *__restrict__ raw, int rows, int nb,
                                   int8_t *__restrict__ qs, uint16_t *__restrict__ ds) {
    const int lane = threadIdx.x;
    const int b = blockIdx.x % nb;
    const int tile = blockIdx.x / nb;
    const int row = tile * 64 + lane;
    uint16_t scale = 0;
    int4 v0 = make_int4(0, 0, 0, 0), v1 = make_int4(0, 0, 0, 0);
    if (row < rows) {
        const uint8_t *src = raw + ((size_t)row * nb + b) * 34;
        scale = (uint16_t)(src[0] | (src[1] << 8));
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            w[i] = (uint32_t)src[2 + 4 * i] | (uint32_t)src[3 + 4 * i] << 8 |
                   (uint32_t)src[4 + 4 * i] << 16 | (uint32_t)src[5 + 4 * i] << 24;
        v0 = make_int4((int)w[0], (int)w[1], (int)w[2], (int)w[3]);
        v1 = make_int4((int)w[4], (int)w[5], (int)w[6], (int)w[7]);
    }
    int4 *dst = reinterpret_cast<int4 *>(qs) + ((size_t)tile * nb + b) * 128;
    dst[lane] = v0;
    dst[64 + lane] = v1;
    ds[((size_t)tile * nb + b) * 64 + lane] = scale;
}

extern "C" grx_status grx_weight_q8_create(grx_ctx *ctx, int rows, int cols, const uint8_t *q8,
                                           size_t nbytes, grx_weight **out) {
    if (!ctx || !out) return grx_fail(GRX_EINVAL, "grx_weight_q8_create: NULL argument");
    *out = nullptr;
    if (rows < 0 || cols < 0) return grx_fail(GRX_EINVAL, "grx_weight_q8_create: negative size");
    if (cols % GRX_QK != 0)
        return grx_fail(GRX_ESIZE, "kern: Q8_0 rows must be a multiple of 32 values");
    const size_t need = (size_t)rows * (size_t)(cols / GRX_QK) * 34;
    if (nbytes < need || (need > 0 && !q8))
        return grx_fail(GRX_ESIZE, "kern: %zu bytes for a %dx%d Q8_0 matrix", nbytes, rows, cols);
    GRX_HIP(hipSetDevice(ctx->device));
    grx_weight *w = new grx_weight();
    w->rows = rows;
    w->cols = cols;
    w->nb = cols / GRX_QK;
    w->tiles = grx_ceil_div(rows, 64);
    w->device = ctx->device;
    const size_t qbytes = (size_t)w->tiles * 64 * (size_t)w->nb * 32;
    const size_t dbytes = (size_t)w->tiles * 64 * (size_t)w->nb * 2;
    w->bytes = qbytes + dbytes;
    hipError_t e = hipSuccess;
    void *raw = nullptr;
    if (w->bytes > 0) {
        e = grx_dev_malloc((void **)&w->qs, qbytes > 0 ? qbytes : 16);
        if (e == hipSuccess) e = grx_dev_malloc((void **)&w->ds, dbytes > 0 ? dbytes : 16);
        if (e == hipSuccess && need > 0) e = grx_dev_malloc(&raw, need);
        if (e == hipSuccess && need > 0)
            e = hipMemcpyAsync(raw, q8, need, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess && w->tiles > 0 && w->nb > 0) {
            grx_pack_q8_kernel<<<w->tiles * w->nb, 64, 0, ctx->stream>>>(
                (const uint8_t *)raw, rows, w->nb, w->qs, w->ds);
            e = hipGetLastError();
        }
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    }
    if (raw) (void)hipFree(raw);
    if (e != hipSuccess) {
        if (w->qs) (void)hipFree(w->qs);
        if (w->ds) (void)hipFree(w->ds);
        delete w;
        return grx_hip_fail(e, "grx_weight_q8_create");
    }
    *out = w;
    return GRX_OK;
}

extern "C" grx_status grx_weight_destroy(grx_weight *w) {
    if (!w) return GRX_OK;
    GRX_HIP(hipSetDevice(w->device));
    if (w->qs) GRX_HIP(hipFree(w->qs));
    if (w->ds) GRX_HIP(hipFree(w->ds));
    delete w;
    return GRX_OK;
}

extern "C" int grx_weight_rows(const grx_weight *w) { return w ? w->rows : 0; }
extern "C" int grx_weight_cols(const grx_weight *w) { return w ? w->cols : 0; }
extern "C" size_t grx_weight_bytes(const grx_weight *w) { return w ? w->bytes : 0; }

// q8Panels.row (internal/kern/q8int.go:66-78): float32(int8(v)) * d, exact.
__global__ void grx_rows_f32_kernel(const int8_t *__restrict__ qs, const uint16_t *__restrict__ ds,
                                    int nb, int row0, int nrows, float *__restrict__ out) {
    const int cols = nb * GRX_QK;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)nrows * cols) return;
    const int row = row0 + (int)(i / cols);
    const int c = (int)(i % cols);
    const int tile = row >> 6, lane = row & 63, b = c >> 5, h = (c >> 4) & 1, e = c & 15;
    const int8_t q = qs[(((size_t)tile * nb + b) * 2 + h) * 1024 + lane * 16 + e];
    const float d = grx_f16_to_f32(ds[((size_t)tile * nb + b) * 64 + lane]);
    out[i] = __fmul_rn((float)q, d);
}

static grx_status rows_f32(grx_ctx *ctx, const grx_weight *w, int row0, int nrows, float *dst) {
    if (!ctx || !w || !dst) return grx_fail(GRX_EINVAL, "grx_weight_row: NULL argument");
    if (row0 < 0 || row0 + nrows > w->rows)
        return grx_fail(GRX_EINVAL, "grx_weight_row: row %d of %d", row0, w->rows);
    const size_t n = (size_t)nrows * w->cols;
    if (n == 0) return GRX_OK;
    GRX_HIP(hipSetDevice(ctx->device));
    void *buf;
    grx_status s = grx_ctx_scratch(ctx, n * sizeof(float), &buf);
    if (s != GRX_OK) return s;
    const int threads = 256;
    const int blocks = (int)((n + threads - 1) / threads);
    grx_rows_f32_kernel<<<blocks, threads, 0, ctx->stream>>>(w->qs, w->ds, w->nb, row0, nrows,
                                                            (float *)buf);
    GRX_LAUNCHED("grx_rows_f32_kernel");
    GRX_HIP(hipMemcpyAsync(dst, buf, n * sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
    GRX_HIP(hipStreamSynchronize(ctx->stream));
    return GRX_OK;
}

extern "C" grx_status grx_weight_row(grx_ctx *ctx, const grx_weight *w, int j, float *dst) {
    return rows_f32(ctx, w, j, 1, dst);
}

extern "C" grx_status grx_weight_float32(grx_ctx *ctx, const grx_weight *w, float *dst) {
    if (!w) return grx_fail(GRX_EINVAL, "grx_weight_float32: NULL weight");
    return rows_f32(ctx, w, 0, w->rows, dst);
}

// Weight.ToQ8 (internal/kern/kern.go:149-164), one thread per block:
// d = amax/127, id = 1/d (0 when d == 0), scale f32toF16(d), values
// int8(round half away from zero of x*id).
__global__ void grx_to_q8_kernel(const float *__restrict__ v, size_t nblocks, uint8_t *__restrict__ out) {
    const size_t blk = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= nblocks) return;
    const float *xs = v + blk * GRX_QK;
    float amax = 0.0f;
    for (int i = 0; i < GRX_QK; ++i) {
        float a = fabsf(xs[i]);
        amax = a > amax ? a : amax;
    }
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint8_t *o = out + blk * 34;
    const uint16_t h = grx_f32_to_f16(d);
    o[0] = (uint8_t)(h & 0xff);
    o[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < GRX_QK; ++i) o[2 + i] = (uint8_t)(int8_t)(int)roundf(__fmul_rn(xs[i], id));
}

extern "C" grx_status grx_to_q8(grx_ctx *ctx, int rows, int cols, const float *v, uint8_t *q8_out) {
    if (!ctx || (!v && rows * cols > 0) || (!q8_out && rows * cols > 0))
        return grx_fail(GRX_EINVAL, "grx_to_q8: NULL argument");
    if (rows < 0 || cols < 0) return grx_fail(GRX_EINVAL, "grx_to_q8: negative size");
    if (cols % GRX_QK != 0) return grx_fail(GRX_ESIZE, "grx_to_q8: cols %d is not a multiple of 32", cols);
    const size_t n = (size_t)rows * cols, nblocks = n / GRX_QK, obytes = nblocks * 34;
    if (n == 0) return GRX_OK;
    GRX_HIP(hipSetDevice(ctx->device));
    const size_t vbytes = (n * sizeof(float) + 255) & ~(size_t)255;
    void *buf;
    grx_status s = grx_ctx_scratch(ctx, vbytes + obytes, &buf);
    if (s != GRX_OK) return s;
    float *dv = (float *)buf;
    uint8_t *dq = (uint8_t *)buf + vbytes;
    GRX_HIP(hipMemcpyAsync(dv, v, n * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
    grx_to_q8_kernel<<<(int)((nblocks + 255) / 256), 256, 0, ctx->stream>>>(dv, nblocks, dq);
    GRX_LAUNCHED("grx_to_q8_kernel");
    GRX_HIP(hipMemcpyAsync(q8_out, dq, obytes, hipMemcpyDeviceToHost, ctx->stream));
    GRX_HIP(hipStreamSynchronize(ctx->stream));
    return GRX_OK;
}
