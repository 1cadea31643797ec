// grx_ln.h - LayerNorm statistics formed in parallel that give the results
// of the reference's left-to-right sums.
//
// Both LayerNorms of the reference sum float64 terms in index order: the
// row's values, then the squared deviations from the mean.
//   kern form  (internal/kern/mathx.go:55-75): mean and inv rounded to
//              float32, y = (v - mean) * inv * w + b in float32;
//   float64 form (pockettts/nn.go:27-49): mean and inv kept in float64,
//              each output float32((v - mean) * inv), then * w + b.
// The kernels sum in a tree (shuffles, DPP), which can round differently.
//  - The values' sum is usually exact in any order: the values are float32,
//    so every partial sum is a multiple of the smallest unit in the last
//    place among them, 2^emin (that of the smallest nonzero |v|), and no
//    larger than n max|v|; when n max|v| < 2^(53+emin) every partial sum
//    is a float64 and no addition rounds.
//  - Otherwise, and for the squared deviations, a sum of n terms formed in
//    order lies within gamma_{n-1} sum|terms| of the exact sum, and one
//    formed by a tree at most D additions deep within gamma_D sum|terms|
//    (gamma_k = k u / (1 - k u), u = 2^-53); ln_slack bounds their gap with
//    room for the roundings of the bound itself.  Each float32 result the
//    reference derives from a sum is a monotone function of it as IEEE
//    arithmetic evaluates it (division, sqrt and conversion round
//    correctly), so when it gives the same float32 bits at both ends of the
//    interval, that is the reference's result.
// When a float32 rounding boundary falls inside (for n = 1024 values drawn
// from N(0,1): about one row in 10^5 for the kern form, a few in 10^3 for
// the float64 form, whose n outputs each round to float32), the sums are
// formed again in index order.
#pragma once

#include "grx_internal.h"

constexpr double kLnU = 0x1p-53;

// |in-order sum - tree sum| for n terms whose magnitudes add up to a, the
// tree at most depth additions deep
__device__ __forceinline__ double ln_slack(int n, int depth, double a) {
    return __dmul_rn(__dmul_rn(__dadd_rn((double)(n + depth), 8.0), kLnU * 1.001), a);
}
__device__ __forceinline__ bool ln_same(float x, float y) { return __float_as_uint(x) == __float_as_uint(y); }

// The exponent of the unit in the last place of a float32 (127 for zero,
// which constrains nothing).
__device__ __forceinline__ int ln_ulp_exp(float v) {
    const uint32_t b = __float_as_uint(v) & 0x7fffffffu;
    return b == 0 ? 127 : max((int)(b >> 23), 1) - 150;
}
// Is every partial sum of n float32 values of magnitude at most mx, the
// smallest nonzero of them mn (+inf if none), a float64?  Then every order
// of summing them gives the exact sum.  a = n mx bounds sum|v| (exactly:
// n <= 2^24 and mx a float32).
__device__ __forceinline__ bool ln_sum_exact(double a, float mn) {
    return !(mn < __builtin_inff()) || a < ldexp(1.0, 53 + ln_ulp_exp(mn));
}
// the per-value part of those: the largest |v| and the smallest nonzero |v|
__device__ __forceinline__ void ln_mag(float v, float &mx, float &mn) {
    const float av = fabsf(v);
    mx = fmaxf(mx, av);
    mn = fminf(mn, av > 0.0f ? av : __builtin_inff());
}

// ---- kern form (mathx.go:63, 69)
__device__ __forceinline__ float ln32_mean(double s, int n) { return (float)(s / (double)n); }
// s: the tree sum of the values, a >= the sum of their magnitudes
__device__ __forceinline__ bool ln32_mean_sure(double s, double a, int n, int depth) {
    const double e = ln_slack(n, depth, a);
    return ln_same(ln32_mean(__dsub_rn(s, e), n), ln32_mean(__dadd_rn(s, e), n));
}
// The relative half-width of the interval holding 1/sqrt(x'/n + eps) as
// IEEE arithmetic evaluates it, around that value at x, for every x'
// within r (x + n eps) of x: (1 -+ r)^(-1/2) lies within r/2 (1 + 5r) of 1
// for r <= 1/2, and each evaluation rounds four times (division, sum,
// sqrt, division), the interval's ends twice more.  Past r = 1/2 the width
// is infinite (the caller then sums in order).
__device__ __forceinline__ double ln_inv_width(double r) {
    if (!(r <= 0.5)) return __builtin_inf();
    return __dadd_rn(__dmul_rn(__dmul_rn(0.5, r), __dadd_rn(1.0, __dmul_rn(5.0, r))), 10.5 * kLnU);
}
// vs: the tree sum of the (non-negative) squared deviations, inv_d =
// 1 / sqrt(vs / n + 1e-5) in float64: does float32(inv_d) hold for every
// order of the sum?  The orders' gap is ln_slack(n, depth, vs) <=
// ln_slack(n, depth, 1) (vs + n 1e-5).
__device__ __forceinline__ bool ln32_inv_sure(double inv_d, int n, int depth) {
    const double w = ln_inv_width(ln_slack(n, depth, 1.0));
    return ln_same((float)__dmul_rn(inv_d, __dsub_rn(1.0, w)), (float)__dmul_rn(inv_d, __dadd_rn(1.0, w)));
}
// the variance term of one value (mathx.go:65-66)
__device__ __forceinline__ double ln32_sq(float v, float mean) {
    const double d = (double)__fsub_rn(v, mean);
    return __dmul_rn(d, d);
}

// ---- float64 form (nn.go:33-44)
__device__ __forceinline__ double ln64_inv(double q, int n, double eps) { return 1.0 / sqrt(q / (double)n + eps); }
__device__ __forceinline__ double ln64_sq(float v, double mean) {
    const double d = __dsub_rn((double)v, mean);
    return __dmul_rn(d, d);
}
// Where the in-order mean and inv can lie, given the tree's: |mean_r - mean|
// <= em and inv_r in [ilo, ihi]; c1 + c2 |v - mean| bounds |x_r - x| for an
// output x = (v - mean) * inv (as computed) against the reference's x_r.
struct Ln64Bound {
    double c1, c2;
};
// mean = s / n from the tree sum s, inv = 1 / sqrt(q / n + eps) from the
// tree sum q of the squared deviations from mean, a >= sum |v|;
// exact: s is the exact sum (so the in-order mean is the same double).
__device__ __forceinline__ Ln64Bound ln64_bound(double mean, double inv, double a, double q, int n, int depth,
                                               bool exact, double eps) {
    const double am = fabs(mean), dn = (double)n;
    double es = 0.0, em = 0.0;
    if (!exact) {
        // |mean_r - mean|: the sums' gap over n, and both divisions'
        // roundings
        es = ln_slack(n, depth, a);
        em = __dadd_rn(__dmul_rn(es / dn, 1.001), __dmul_rn(3.0 * kLnU, am));
    }
    // |q_r - q|: both sums' orders and their terms' roundings, plus the
    // change of sum (v - m)^2 as m moves by em, 2 em |sum v - n m| + n em^2
    const double shift = __dadd_rn(__dmul_rn(2.0 * em, __dadd_rn(es, __dmul_rn(dn * kLnU * 1.001, am))),
                                   __dmul_rn(dn, __dmul_rn(em, em)));
    // that gap over q + n eps: ln_slack(n, depth, q) <= ln_slack(n, depth,
    // 1) (q + n eps); the shift (zero when s is exact) over it in float64
    double r = ln_slack(n, depth, 1.0);
    if (!exact) r = __dadd_rn(r, shift / __dadd_rn(q, __dmul_rn(dn, eps)));
    // |inv_r - inv| <= w inv
    const double w = ln_inv_width(__dmul_rn(r, 1.01)), ihi = __dmul_rn(inv, __dadd_rn(1.0, w));
    // |fl(v - m_r) - fl(v - m)| <= em + 2u|v - m| (+ second order), times
    // ihi; |d| w inv from inv; 2u|x| from the two products' roundings and
    // 2u|x| more for forming x -+ the bound (|x| <= |d| ihi)
    Ln64Bound b;
    b.c1 = __dmul_rn(__dmul_rn(em, ihi), 1.0102);
    b.c2 = __dmul_rn(__dadd_rn(__dmul_rn(w, inv), __dmul_rn(8.1 * kLnU, ihi)), 1.01);
    return b;
}
// Is float32(x), x = d * inv as computed here (d = v - mean), also the
// reference's float32((v - mean_r) * inv_r)?
__device__ __forceinline__ bool ln64_out_sure(double d, double x, const Ln64Bound &b) {
    const double del = __dadd_rn(b.c1, __dmul_rn(fabs(d), b.c2));
    return ln_same((float)__dsub_rn(x, del), (float)__dadd_rn(x, del));
}

// ---------------------------------------------------------------- cross-lane sums

// Cross-lane moves within rows of 16 lanes (DPP; every lane active): the
// quad permutations [1,0,3,2] and [2,3,0,1], the mirror of each 8 and of
// each 16 lanes.  Sums and maxima built from them hold the same value in
// every lane of the group (a + b == b + a).
constexpr int kDppXor1 = 0xb1, kDppXor2 = 0x4e, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xf, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xf, 0xf, false);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ double readlane_f64(double v, int l) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
// The wave's float64 sum, the same in every lane: rows of 16 by DPP, then
// (row0 + row1) + (row2 + row3).
__device__ __forceinline__ double wave_sum_f64(double v) {
    v = __dadd_rn(v, dpp_f64<kDppXor1>(v));
    v = __dadd_rn(v, dpp_f64<kDppXor2>(v));
    v = __dadd_rn(v, dpp_f64<kDppHalfMirror>(v));
    v = __dadd_rn(v, dpp_f64<kDppMirror>(v));
    return __dadd_rn(__dadd_rn(readlane_f64(v, 0), readlane_f64(v, 16)),
                     __dadd_rn(readlane_f64(v, 32), readlane_f64(v, 48)));
}
// The wave's float32 maximum and minimum, the same in every lane
__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, dpp_f32<kDppXor1>(v));
    v = fmaxf(v, dpp_f32<kDppXor2>(v));
    v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f32<kDppMirror>(v));
    return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)),
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16))),
                 fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)),
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48))));
}
__device__ __forceinline__ float wave_min_f32(float v) {
    v = fminf(v, dpp_f32<kDppXor1>(v));
    v = fminf(v, dpp_f32<kDppXor2>(v));
    v = fminf(v, dpp_f32<kDppHalfMirror>(v));
    v = fminf(v, dpp_f32<kDppMirror>(v));
    return fminf(fminf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)),
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16))),
                 fminf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)),
                       __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48))));
}
// ---------------------------------------------------------------- rows in memory

// In-order float64 sum of term(v[i]), i = 0..n-1 (the reference's loop),
// formed by every thread that calls it (the same value in all of them); v
// is in LDS or global memory.
template <typename F>
__device__ __forceinline__ double ln_serial_sum(const float *v, int n, F term) {
    double s = 0.0;
    int i = 0;
    for (; i + 8 <= n; i += 8) {
        float t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t[u] = v[i + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) s = __dadd_rn(s, term(t[u]));
    }
    for (; i < n; ++i) s = __dadd_rn(s, term(v[i]));
    return s;
}

// A per-thread float64 partial summed over the workgroup, and a float32
// maximum and minimum taken, the same values in every thread: each wave's
// by DPP, then the waves in order.  red: 48 doubles of LDS; blockDim.x a
// multiple of 64, <= 1024.
__device__ __forceinline__ void ln_block_reduce(double &x, float &mx, float &mn, double *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    x = wave_sum_f64(x);
    mx = wave_max_f32(mx);
    mn = wave_min_f32(mn);
    __syncthreads();  // red may still be read by a previous call
    if (lane == 0) {
        red[wave] = x;
        red[16 + wave] = (double)mx;
        red[32 + wave] = (double)mn;
    }
    __syncthreads();
    double sx = 0.0;
    float a = 0.0f, b = __builtin_inff();
    for (int w = 0; w < nw; ++w) {
        sx = __dadd_rn(sx, red[w]);
        a = fmaxf(a, (float)red[16 + w]);
        b = fminf(b, (float)red[32 + w]);
    }
    x = sx;
    mx = a;
    mn = b;
}
// A per-thread float64 partial summed over the workgroup as above
__device__ __forceinline__ double ln_block_sum(double x, double *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    x = wave_sum_f64(x);
    __syncthreads();  // red may still be read by a previous call
    if (lane == 0) red[wave] = x;
    __syncthreads();
    double sx = 0.0;
    for (int w = 0; w < nw; ++w) sx = __dadd_rn(sx, red[w]);
    return sx;
}
// additions on the longest path of ln_block_reduce's tree over n terms
__device__ __forceinline__ int ln_block_depth(int n) {
    return ((n + (int)blockDim.x - 1) / (int)blockDim.x) + 6 + ((int)blockDim.x >> 6);
}

// The values' sum s, a = n max|v| (>= sum |v|) and whether s is exact,
// over the workgroup.
__device__ __forceinline__ void ln_block_values(const float *v, int n, double *red, double &s, double &a,
                                                bool &exact) {
    s = 0.0;
    float mx = 0.0f, mn = __builtin_inff();
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float x = v[i];
        s = __dadd_rn(s, (double)x);
        ln_mag(x, mx, mn);
    }
    ln_block_reduce(s, mx, mn, red);
    a = __dmul_rn((double)n, (double)mx);
    exact = ln_sum_exact(a, mn);
}

// kern.LayerNorm's mean and inv (mathx.go:59-69) of the row v[0..n), LDS
// or global memory, called by every thread of the workgroup once the whole
// row is in place (the in-order pass reads all of it).  CHECK false
// keeps the tree sums whatever they give (for tests that show the
// in-order pass is needed).
template <bool CHECK = true>
__device__ __forceinline__ void ln32_stats(const float *v, int n, double *red, float &mean, float &inv) {
    const int depth = ln_block_depth(n);
    double s, a;
    bool exact;
    ln_block_values(v, n, red, s, a, exact);
    if (CHECK && !exact && !ln32_mean_sure(s, a, n, depth))
        s = ln_serial_sum(v, n, [](float x) { return (double)x; });
    const float m = ln32_mean(s, n);
    double q = 0.0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) q = __dadd_rn(q, ln32_sq(v[i], m));
    q = ln_block_sum(q, red);
    double inv_d = 1.0 / sqrt(q / (double)n + 1e-5);
    if (CHECK && !ln32_inv_sure(inv_d, n, depth)) {
        q = ln_serial_sum(v, n, [m](float x) { return ln32_sq(x, m); });
        inv_d = 1.0 / sqrt(q / (double)n + 1e-5);
    }
    mean = m;
    inv = (float)inv_d;
    __syncthreads();  // every read of the row is done: the caller may write it in place
}

// pockettts layerNorm's mean and inv (nn.go:32-40) of the row v[0..n), as
// ln32_stats; each output's float32 rounding is checked too.
template <bool CHECK = true>
__device__ __forceinline__ void ln64_stats(const float *v, int n, double eps, double *red, double &mean, double &inv) {
    const int depth = ln_block_depth(n);
    double s, a;
    bool exact;
    ln_block_values(v, n, red, s, a, exact);
    double m = s / (double)n;
    double q = 0.0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) q = __dadd_rn(q, ln64_sq(v[i], m));
    q = ln_block_sum(q, red);
    double iv = ln64_inv(q, n, eps);
    if (CHECK) {
        const Ln64Bound b = ln64_bound(m, iv, a, q, n, depth, exact, eps);
        int unsure = 0;
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            const double d = __dsub_rn((double)v[i], m);
            if (!ln64_out_sure(d, __dmul_rn(d, iv), b)) unsure = 1;
        }
        if (__syncthreads_or(unsure)) {
            if (!exact) m = ln_serial_sum(v, n, [](float x) { return (double)x; }) / (double)n;
            iv = ln64_inv(ln_serial_sum(v, n, [m](float x) { return ln64_sq(x, m); }), n, eps);
        }
    }
    mean = m;
    inv = iv;
    __syncthreads();  // every read of the row is done: the caller may write it in place
}

// ---------------------------------------------------------------- rows in one wave

// A row of K values held by one wave as NP float4 pieces per lane: value i
// is component i % 4 of piece P = i / 4, which lane P % 64 holds in
// xv[P / 64] (pieces at or past npc = K / 4 are not part of the row).

// In-order float64 sum of term(value i), i = 0..K-1, the same in every lane.
template <int NP, typename F>
__device__ __forceinline__ double wave_serial_sum(const float4 (&xv)[NP], int npc, F term) {
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        const int lanes = min(64, npc - 64 * j);
        for (int l = 0; l < lanes; ++l) {
            s = __dadd_rn(s, term(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(xv[j].x), l))));
            s = __dadd_rn(s, term(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(xv[j].y), l))));
            s = __dadd_rn(s, term(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(xv[j].z), l))));
            s = __dadd_rn(s, term(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(xv[j].w), l))));
        }
    }
    return s;
}

template <int NP, typename F>
__device__ __forceinline__ void wave_partial(const float4 (&xv)[NP], int npc, int lane, double &s, F term) {
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        if (j * 64 + lane < npc) {
            s = __dadd_rn(s, term(xv[j].x));
            s = __dadd_rn(s, term(xv[j].y));
            s = __dadd_rn(s, term(xv[j].z));
            s = __dadd_rn(s, term(xv[j].w));
        }
    }
}
// additions on the longest path of the wave's tree: a lane's pieces, the
// DPP steps and the two final sums
__device__ __forceinline__ int ln_wave_depth(int npc) { return 4 * ((npc + 63) / 64) + 6; }

// The values' sum s, a = K max|v| (>= sum |v|) and whether s is exact.
template <int NP>
__device__ __forceinline__ void ln_wave_values(const float4 (&xv)[NP], int npc, int lane, double &s, double &a,
                                               bool &exact) {
    s = 0.0;
    float mx = 0.0f, mn = __builtin_inff();
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        if (j * 64 + lane < npc) {
            s = __dadd_rn(s, (double)xv[j].x);
            s = __dadd_rn(s, (double)xv[j].y);
            s = __dadd_rn(s, (double)xv[j].z);
            s = __dadd_rn(s, (double)xv[j].w);
            ln_mag(xv[j].x, mx, mn);
            ln_mag(xv[j].y, mx, mn);
            ln_mag(xv[j].z, mx, mn);
            ln_mag(xv[j].w, mx, mn);
        }
    }
    s = wave_sum_f64(s);
    mx = wave_max_f32(mx);
    mn = wave_min_f32(mn);
    a = __dmul_rn((double)(4 * npc), (double)mx);
    exact = ln_sum_exact(a, mn);
}

// kern.LayerNorm's mean and inv (mathx.go:59-69) of the wave's row, the
// same in every lane.
template <int NP, bool CHECK = true>
__device__ __forceinline__ void wave_ln32_stats(const float4 (&xv)[NP], int npc, int lane, float &mean_out,
                                               float &inv_out) {
    const int K = 4 * npc, depth = ln_wave_depth(npc);
    double s, a;
    bool exact;
    ln_wave_values(xv, npc, lane, s, a, exact);
    if (CHECK && !exact && !ln32_mean_sure(s, a, K, depth))
        s = wave_serial_sum(xv, npc, [](float v) { return (double)v; });
    const float mean = ln32_mean(s, K);
    double vs = 0.0;
    wave_partial(xv, npc, lane, vs, [mean](float v) { return ln32_sq(v, mean); });
    vs = wave_sum_f64(vs);
    double inv_d = 1.0 / sqrt(vs / (double)K + 1e-5);
    if (CHECK && !ln32_inv_sure(inv_d, K, depth)) {
        vs = wave_serial_sum(xv, npc, [mean](float v) { return ln32_sq(v, mean); });
        inv_d = 1.0 / sqrt(vs / (double)K + 1e-5);
    }
    mean_out = mean;
    inv_out = (float)inv_d;
}

// kern.LayerNorm (mathx.go:55-75) of the wave's row in place: xv[j] =
// (v - mean) * inv * w + b, rounded step by step.
template <int NP, bool CHECK = true>
__device__ __forceinline__ void wave_ln32(float4 (&xv)[NP], const float4 (&wv)[NP], const float4 (&bv)[NP], int npc,
                                         int lane) {
    float mean, inv;
    wave_ln32_stats<NP, CHECK>(xv, npc, lane, mean, inv);
    auto nrm = [&](float v, float w, float b) {
        float t = __fsub_rn(v, mean);
        t = __fmul_rn(t, inv);
        t = __fmul_rn(t, w);
        return __fadd_rn(t, b);
    };
#pragma unroll
    for (int j = 0; j < NP; ++j) {
        xv[j].x = nrm(xv[j].x, wv[j].x, bv[j].x);
        xv[j].y = nrm(xv[j].y, wv[j].y, bv[j].y);
        xv[j].z = nrm(xv[j].z, wv[j].z, bv[j].z);
        xv[j].w = nrm(xv[j].w, wv[j].w, bv[j].w);
    }
}

// pockettts layerNorm (nn.go:27-49) of the wave's row in place: float32
// of (v - mean) * inv in float64, then * w + b when gb.  The outputs
// replace the values as they are checked (no float64 copy of the row stays
// live); when a row needs the in-order pass, reload(xv) brings the values
// back first.
template <int NP, bool CHECK = true, typename Reload>
__device__ __forceinline__ void wave_ln64(float4 (&xv)[NP], const float4 (&wv)[NP], const float4 (&bv)[NP], bool gb,
                                         int npc, int lane, double eps, Reload reload) {
    const int K = 4 * npc, depth = ln_wave_depth(npc);
    double s, a;
    bool exact;
    ln_wave_values(xv, npc, lane, s, a, exact);
    double mean = s / (double)K;
    double q = 0.0;
    wave_partial(xv, npc, lane, q, [mean](float v) { return ln64_sq(v, mean); });
    q = wave_sum_f64(q);
    double inv = ln64_inv(q, K, eps);
    auto out = [&](float &v) { v = (float)__dmul_rn(__dsub_rn((double)v, mean), inv); };
    if (CHECK) {
        const Ln64Bound b = ln64_bound(mean, inv, a, q, K, depth, exact, eps);
        bool sure = true;
        auto one = [&](float &v) {
            const double d = __dsub_rn((double)v, mean), x = __dmul_rn(d, inv);
            sure &= ln64_out_sure(d, x, b);
            v = (float)x;
        };
#pragma unroll
        for (int j = 0; j < NP; ++j) {
            if (j * 64 + lane < npc) {
                one(xv[j].x);
                one(xv[j].y);
                one(xv[j].z);
                one(xv[j].w);
            }
        }
        if (__ballot(!sure) != 0) {
            reload(xv);
            if (!exact) mean = wave_serial_sum(xv, npc, [](float v) { return (double)v; }) / (double)K;
            inv = ln64_inv(wave_serial_sum(xv, npc, [mean](float v) { return ln64_sq(v, mean); }), K, eps);
#pragma unroll
            for (int j = 0; j < NP; ++j) {
                out(xv[j].x);
                out(xv[j].y);
                out(xv[j].z);
                out(xv[j].w);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < NP; ++j) {
            out(xv[j].x);
            out(xv[j].y);
            out(xv[j].z);
            out(xv[j].w);
        }
    }
    if (gb) {
#pragma unroll
        for (int j = 0; j < NP; ++j) {
            xv[j].x = __fadd_rn(__fmul_rn(xv[j].x, wv[j].x), bv[j].x);
            xv[j].y = __fadd_rn(__fmul_rn(xv[j].y, wv[j].y), bv[j].y);
            xv[j].z = __fadd_rn(__fmul_rn(xv[j].z, wv[j].z), bv[j].z);
            xv[j].w = __fadd_rn(__fmul_rn(xv[j].w, wv[j].w), bv[j].w);
        }
    }
}
