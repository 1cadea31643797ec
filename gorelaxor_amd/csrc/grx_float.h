// grx_float.h - the reference's float-kernel orders as device functions.
//
// Each function restates one float kernel of github.com/xattribution/gorelaxor
// (cited file:line) in its exact order of operations, so that the decoder
// kernels built from them give bit-identical results to the CPU oracle.
#pragma once

#include "grx_internal.h"

// dotF32Go (internal/kern/gemm.go:294-308): four running sums, unfused.
__device__ __forceinline__ float dot_go(const float *x, const float *y, int n) {
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    int i = 0;
    for (; i + 4 <= n; i += 4) {
        s0 = __fadd_rn(s0, __fmul_rn(x[i], y[i]));
        s1 = __fadd_rn(s1, __fmul_rn(x[i + 1], y[i + 1]));
        s2 = __fadd_rn(s2, __fmul_rn(x[i + 2], y[i + 2]));
        s3 = __fadd_rn(s3, __fmul_rn(x[i + 3], y[i + 3]));
    }
    for (; i < n; i++) s0 = __fadd_rn(s0, __fmul_rn(x[i], y[i]));
    return __fadd_rn(__fadd_rn(__fadd_rn(s0, s1), s2), s3);
}

// HSUM of kernels_amd64.s:90-95 over eight lane values.
__device__ __forceinline__ float hsum8(const float *a) {
    const float h0 = __fadd_rn(a[0], a[4]), h1 = __fadd_rn(a[1], a[5]);
    const float h2 = __fadd_rn(a[2], a[6]), h3 = __fadd_rn(a[3], a[7]);
    return __fadd_rn(__fadd_rn(h0, h1), __fadd_rn(h2, h3));
}

// One row of dot4f32avx (kernels_amd64.s:156-204), kk % 16 == 0.
__device__ __forceinline__ float dot_avx(const float *x, const float *w, int kk) {
    float A[8], B[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) A[l] = B[l] = 0.f;
    for (int c = 0; c < kk; c += 16) {
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            A[l] = __fmaf_rn(x[c + l], w[c + l], A[l]);
            B[l] = __fmaf_rn(x[c + 8 + l], w[c + 8 + l], B[l]);
        }
    }
    float S[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) S[l] = __fadd_rn(A[l], B[l]);
    return hsum8(S);
}

// dotF32x4 (kernels_amd64.go:75-95) for one row: assembly over k &^ 15,
// dotF32Go over the rest added on.
__device__ __forceinline__ float dot_x4(const float *x, const float *w, int k) {
    const int kk = k & ~15;
    float o = kk > 0 ? dot_avx(x, w, kk) : 0.f;
    if (kk < k) o = __fadd_rn(o, dot_go(x + kk, w + kk, k - kk));
    return o;
}

// One Q8_0 weight row of the float route per four threads (256 threads = 64
// rows of tile `tile`), x in LDS.  Thread j keeps the reference's lane chains j
// and j+4 of dot4q8avx, so no chain changes order, and the HSUM is formed
// across the four as (h0+h1)+(h2+h3), h_j = acc[j]+acc[j+4].  Rows of the last
// partial group of four take dotQ8Go, its block sums spread over the four
// threads and chained in thread 0.  Blocks are read four
// at a time.  Returns the product (no bias) with emit set in thread 0 of a
// live row; every thread of the workgroup must call it (shuffles).
__device__ __forceinline__ float q8_float_row(const float *xs, const int8_t *__restrict__ qs,
                                              const uint16_t *__restrict__ ds, int nb, int n, int tile, int &row,
                                              bool &emit) {
    const int rl = threadIdx.x >> 2, j = threadIdx.x & 3;
    row = tile * 64 + rl;
    const bool live = row < n, avx = row < (n & ~3);
    const int8_t *qt = qs + (size_t)tile * nb * 2 * 64 * 16 + (size_t)rl * 16;
    const uint16_t *dt = ds + (size_t)tile * nb * 64 + rl;
    auto ld = [&](int b, int4 &h0, int4 &h1, uint16_t &d) {
        h0 = *reinterpret_cast<const int4 *>(qt + (size_t)(2 * b) * 64 * 16);
        h1 = *reinterpret_cast<const int4 *>(qt + (size_t)(2 * b + 1) * 64 * 16);
        d = dt[(size_t)b * 64];
    };
    float a0 = 0.f, a1 = 0.f, s = 0.f;
    if (live && avx) {
        // the reference's lane chains j and j+4 of one block
        // value i of the block is byte i%4 of dword i/4; chain l = j + 4c
        // reads values l, 8+l, 16+l, 24+l: byte j of dwords c, 2+c, 4+c, 6+c
        const unsigned sh = 24u - 8u * (unsigned)j;
        auto val = [&](int dw) { return (float)((int)((unsigned)dw << sh) >> 24); };
        auto fold = [&](int b, const int4 &h0, const int4 &h1, uint16_t dh) {
            const float d = grx_f16_to_f32(dh);
            const float *xb = xs + b * 32;
            const int dws[2][4] = {{h0.x, h0.z, h1.x, h1.z}, {h0.y, h0.w, h1.y, h1.w}};
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int l = j + 4 * c;
                float t = __fmul_rn(val(dws[c][0]), xb[l]);
                t = __fmaf_rn(val(dws[c][1]), xb[8 + l], t);
                t = __fmaf_rn(val(dws[c][2]), xb[16 + l], t);
                t = __fmaf_rn(val(dws[c][3]), xb[24 + l], t);
                if (c == 0) a0 = __fmaf_rn(t, d, a0);
                else a1 = __fmaf_rn(t, d, a1);
            }
        };
        // groups of four blocks, the next group read (at a clamped index,
        // unconditionally) while this one is folded
        const int ng = nb / 4;
        int4 c0[4], c1[4];
        uint16_t cd[4];
        if (ng > 0) {
#pragma unroll
            for (int u = 0; u < 4; ++u) ld(u, c0[u], c1[u], cd[u]);
        }
        for (int g = 0; g < ng; ++g) {
            const int gn = min(g + 1, ng - 1);
            int4 n0[4], n1[4];
            uint16_t nd[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) ld(4 * gn + u, n0[u], n1[u], nd[u]);
#pragma unroll
            for (int u = 0; u < 4; ++u) fold(4 * g + u, c0[u], c1[u], cd[u]);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                c0[u] = n0[u];
                c1[u] = n1[u];
                cd[u] = nd[u];
            }
        }
        for (int b = 4 * ng; b < nb; ++b) {
            int4 h0, h1;
            uint16_t dh;
            ld(b, h0, h1, dh);
            fold(b, h0, h1, dh);
        }
    } else if (live) {
        // dotQ8Go (kern.go:248-266): per block four running sums and
        // t = d*(((q0+q1)+q2)+q3), added to s in block order.  The blocks'
        // t are independent: thread j forms those of blocks 4g+j, and
        // thread 0 adds each group's four in order.
        auto blk = [&](int b, const int4 &h0, const int4 &h1, uint16_t dh) {
            int8_t w[32];
            *reinterpret_cast<int4 *>(w) = h0;
            *reinterpret_cast<int4 *>(w + 16) = h1;
            const float d = grx_f16_to_f32(dh);
            const float *xb = xs + b * 32;
            float q0 = 0.f, q1 = 0.f, q2 = 0.f, q3 = 0.f;
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                q0 = __fadd_rn(q0, __fmul_rn(xb[i], (float)w[i]));
                q1 = __fadd_rn(q1, __fmul_rn(xb[i + 1], (float)w[i + 1]));
                q2 = __fadd_rn(q2, __fmul_rn(xb[i + 2], (float)w[i + 2]));
                q3 = __fadd_rn(q3, __fmul_rn(xb[i + 3], (float)w[i + 3]));
            }
            return __fmul_rn(d, __fadd_rn(__fadd_rn(__fadd_rn(q0, q1), q2), q3));
        };
        const int ngrp = (nb + 3) / 4;
        for (int g0 = 0; g0 < ngrp; g0 += 4) {  // four groups' reads in flight (indexes clamped into range)
            int4 a0[4], a1[4];
            uint16_t ad[4];
            float t[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) ld(min((g0 + u) * 4 + j, nb - 1), a0[u], a1[u], ad[u]);
#pragma unroll
            for (int u = 0; u < 4; ++u) t[u] = blk(min((g0 + u) * 4 + j, nb - 1), a0[u], a1[u], ad[u]);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int gb = (g0 + u) * 4;
                const float t1 = __shfl_down(t[u], 1, 4), t2 = __shfl_down(t[u], 2, 4), t3 = __shfl_down(t[u], 3, 4);
                if (j == 0) {
                    if (gb < nb) s = __fadd_rn(s, t[u]);
                    if (gb + 1 < nb) s = __fadd_rn(s, t1);
                    if (gb + 2 < nb) s = __fadd_rn(s, t2);
                    if (gb + 3 < nb) s = __fadd_rn(s, t3);
                }
            }
        }
    }
    // HSUM over the row's four threads: h_j = acc[j] + acc[j+4], then (h0+h1)+(h2+h3)
    const float h = __fadd_rn(a0, a1);
    const float h1 = __shfl_down(h, 1, 4), h23 = __fadd_rn(__shfl_down(h, 2, 4), __shfl_down(h, 3, 4));
    emit = live && j == 0;
    return avx ? __fadd_rn(__fadd_rn(h, h1), h23) : s;
}

// softmax (internal/kern/mathx.go:78-90) of s[0..n) in LDS by one block:
// max, e = EXP8(v-max) below n &^ 7 and expf past it, the eight lane sums
// of expSubAVX + HSUM, plus the tail's own sum, then v *= 1/sum.
__device__ inline void block_softmax(float *s, int n, float *part) {
    const int tid = threadIdx.x, nt = blockDim.x;
    float mx = -__builtin_inff();
    for (int j = tid; j < n; j += nt) mx = s[j] > mx ? s[j] : mx;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v = __shfl_xor(mx, o);
        mx = v > mx ? v : mx;
    }
    if ((tid & 63) == 0) part[16 + (tid >> 6)] = mx;
    __syncthreads();
    mx = -__builtin_inff();
    for (int w = 0; w < (nt + 63) / 64; ++w) mx = part[16 + w] > mx ? part[16 + w] : mx;
    const int n8 = n & ~7;
    for (int j = tid; j < n; j += nt) {
        const float d = __fsub_rn(s[j], mx);
        s[j] = j < n8 ? grx_exp8(d) : grx_expf_go(d);
    }
    __syncthreads();
    if (tid < 8) {
        float acc = 0.f;
#pragma unroll 16
        for (int j = tid; j < n8; j += 8) acc = __fadd_rn(acc, s[j]);
        part[tid] = acc;
    } else if (tid == 8) {
        float t = 0.f;
        for (int j = n8; j < n; ++j) t = __fadd_rn(t, s[j]);
        part[8] = t;
    }
    __syncthreads();
    const float sa = n8 > 0 ? hsum8(part) : 0.f;
    const float inv = __fdiv_rn(1.0f, __fadd_rn(sa, part[8]));
    for (int j = tid; j < n; j += nt) s[j] = __fmul_rn(s[j], inv);
    __syncthreads();
}

// A DPP move within rows of 16 lanes (every lane active).
template <int CTRL>
__device__ __forceinline__ float dpp_max_step(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// The largest value of the wave, in every lane (DPP within rows of 16, then
// the four rows).
__device__ __forceinline__ float wave_max(float m) {
    float t = dpp_max_step<0xb1>(m);
    m = t > m ? t : m;
    t = dpp_max_step<0x4e>(m);
    m = t > m ? t : m;
    t = dpp_max_step<0x141>(m);
    m = t > m ? t : m;
    t = dpp_max_step<0x140>(m);
    m = t > m ? t : m;
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 48));
    const float ab = b > a ? b : a, cd = d > c ? d : c;
    return cd > ab ? cd : ab;
}

// The softmax sums of block_softmax (mathx.go:78-90) for wave 0, from the
// exps below n8 stored chain-major (chain c = j % 8 at ch[c*cs + j/8],
// cs % 4 == 0) and the tail's exps tl[0..n-n8): lane 0 gets
// 1 / (HSUM(eight chains) + tail).  Branch-free: whole runs of 32 steps,
// then a last run under selects.
__device__ __forceinline__ float softmax_inv(const float *ch, int cs, const float *tl, int n) {
    const int lane = threadIdx.x & 63, c = lane & 7, n8 = n & ~7, nt = n - n8, N = n8 >> 3;
    const float4 *cr = reinterpret_cast<const float4 *>(ch + c * cs);
    float acc = 0.f;
    int g0 = 0;
    for (; g0 + 32 <= N; g0 += 32) {
        float4 t[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) t[g] = cr[(g0 >> 2) + g];
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            acc = __fadd_rn(acc, t[g].x);
            acc = __fadd_rn(acc, t[g].y);
            acc = __fadd_rn(acc, t[g].z);
            acc = __fadd_rn(acc, t[g].w);
        }
    }
    if (g0 < N) {
        float4 t[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) t[g] = cr[min((g0 >> 2) + g, (N - 1) >> 2)];
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const int m = g0 + 4 * g;
            float f;
            f = __fadd_rn(acc, t[g].x);
            acc = m + 0 < N ? f : acc;
            f = __fadd_rn(acc, t[g].y);
            acc = m + 1 < N ? f : acc;
            f = __fadd_rn(acc, t[g].z);
            acc = m + 2 < N ? f : acc;
            f = __fadd_rn(acc, t[g].w);
            acc = m + 3 < N ? f : acc;
        }
    }
    float tt = 0.f;
#pragma unroll
    for (int i = 0; i < 7; ++i) {
        const float f = __fadd_rn(tt, tl[min(i, max(nt - 1, 0))]);
        tt = i < nt ? f : tt;
    }
    const float p0 = __shfl(acc, 0), p1 = __shfl(acc, 1), p2 = __shfl(acc, 2), p3 = __shfl(acc, 3);
    const float p4 = __shfl(acc, 4), p5 = __shfl(acc, 5), p6 = __shfl(acc, 6), p7 = __shfl(acc, 7);
    const float sa = n8 > 0 ? __fadd_rn(__fadd_rn(__fadd_rn(p0, p4), __fadd_rn(p1, p5)),
                                        __fadd_rn(__fadd_rn(p2, p6), __fadd_rn(p3, p7)))
                            : 0.f;
    return __fdiv_rn(1.0f, __fadd_rn(sa, tt));
}

// Round the values held by 32 consecutive lanes (one Q8_0 block) for the
// next product: quantU8 (internal/kern/q8int.go:88-105) with the block's
// largest magnitude from xor-shuffles.  Every lane of the 32 must call it.
__device__ __forceinline__ void quant32_store(float v, int8_t *q, float *sc, int lane32) {
    const float av = fabsf(v);
    float amax = av > 0.0f ? av : 0.0f;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) {
        const float t = __shfl_xor(amax, o, 32);
        amax = t > amax ? t : amax;
    }
    const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    float r = rintf(__fmul_rn(v, id));
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    *q = (int8_t)(int)r;
    if (lane32 == 0) *sc = __fmul_rn(amax, grx_bits_f32(0x3c010204u));
}


// softmax of s[0..n) by one thread (the same arithmetic as block_softmax):
// expSub's eight lane sums over n &^ 7, HSUM, the tail's own sum.
__device__ inline void seq_softmax(float *s, int n) {
    float mx = -__builtin_inff();
    for (int j = 0; j < n; ++j) mx = s[j] > mx ? s[j] : mx;
    const int n8 = n & ~7;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < n8; ++j) {
        const float e = grx_exp8(__fsub_rn(s[j], mx));
        s[j] = e;
        acc[j & 7] = __fadd_rn(acc[j & 7], e);
    }
    float t = 0.f;
    for (int j = n8; j < n; ++j) {
        const float e = grx_expf_go(__fsub_rn(s[j], mx));
        s[j] = e;
        t = __fadd_rn(t, e);
    }
    const float sa = n8 > 0 ? hsum8(acc) : 0.f;
    const float inv = __fdiv_rn(1.0f, __fadd_rn(sa, t));
    for (int j = 0; j < n; ++j) s[j] = __fmul_rn(s[j], inv);
}

// dot4f32avx (kernels_amd64.s:156-204) of one row on 16 lanes of a wave
// (c = lane & 15): lane l < 8 runs chain A_l over elements 16i + l, lane 8+l
// chain B_l over 16i + 8 + l; then S_l = A_l + B_l and HSUM by shuffles
// within the 16 lanes.  Every lane of the 16 must call it with the same
// row; the sum is returned in lane c == 0.  kk % 16 == 0.
__device__ __forceinline__ float dot_avx16(const float *x, const float *w, int kk, int c) {
    float acc = 0.f;
    for (int i = c; i < kk; i += 16) acc = __fmaf_rn(x[i], w[i], acc);
    const float other = __shfl_xor(acc, 8, 16);
    const float S = __fadd_rn(c < 8 ? acc : other, c < 8 ? other : acc);
    const float h4 = __fadd_rn(S, __shfl_xor(S, 4, 16));
    const float h01 = __fadd_rn(h4, __shfl_xor(h4, 1, 16));
    const float h23 = __shfl_xor(h01, 2, 16);
    return kk > 0 ? __fadd_rn(h01, h23) : 0.f;
}

// dotF32Go (gemm.go:294-308) of one row on 4 lanes (c = lane & 3): lane c
// keeps running sum s_c over elements c, c+4, ... below n &^ 3, lane 0 also
// the tail; then ((s0 + s1) + s2) + s3 by shuffles.  Every lane of the 4
// must call it; the sum is returned in lane c == 0.
__device__ __forceinline__ float dot_go4(const float *x, const float *y, int n, int c) {
    const int n4 = n & ~3;
    float acc = 0.f;
    for (int i = c; i < n4; i += 4) acc = __fadd_rn(acc, __fmul_rn(x[i], y[i]));
    if (c == 0)
        for (int i = n4; i < n; ++i) acc = __fadd_rn(acc, __fmul_rn(x[i], y[i]));
    const float s1 = __shfl_xor(acc, 1, 4);
    const float s2 = __shfl_xor(acc, 2, 4);
    const float s3 = __shfl_xor(acc, 3, 4);
    return __fadd_rn(__fadd_rn(__fadd_rn(acc, s1), s2), s3);
}

// Rows [r0, r0+rows) of one head's cached values (rows `ld` floats apart,
// the head's hd values at `base`) into LDS vl[rows][hd], every thread
// keeping eight loads in flight (16-byte loads when hd % 4 == 0).
__device__ __forceinline__ void stage_rows(float *vl, const float *base, size_t ld, int r0, int rows, int hd) {
    const int nt = blockDim.x, tid = threadIdx.x;
    constexpr int kF = 8;
    if ((hd & 3) == 0 && (ld & 3) == 0) {
        const int h4 = hd >> 2, n4 = rows * h4;
        for (int i0 = tid; i0 < n4; i0 += kF * nt) {
            float4 v[kF];
#pragma unroll
            for (int u = 0; u < kF; ++u) {  // clamped: the loads stay in flight together
                const int i = min(i0 + u * nt, n4 - 1);
                v[u] = *reinterpret_cast<const float4 *>(base + (size_t)(r0 + i / h4) * ld + 4 * (i % h4));
            }
#pragma unroll
            for (int u = 0; u < kF; ++u) {
                const int i = i0 + u * nt;
                if (i < n4) *reinterpret_cast<float4 *>(vl + 4 * i) = v[u];
            }
        }
    } else {
        const int n = rows * hd;
        for (int i0 = tid; i0 < n; i0 += kF * nt) {
            float v[kF];
#pragma unroll
            for (int u = 0; u < kF; ++u) {
                const int i = min(i0 + u * nt, n - 1);
                v[u] = base[(size_t)(r0 + i / hd) * ld + i % hd];
            }
#pragma unroll
            for (int u = 0; u < kF; ++u) {
                const int i = i0 + u * nt;
                if (i < n) vl[i] = v[u];
            }
        }
    }
}

// dotF32Go, dot4f32avx and dotF32x4 with the second operand's elements sb
// apart (the first's contiguous): the same orders as dot_go, dot_avx, dot_x4.
__device__ __forceinline__ float dot_go_s(const float *x, const float *y, size_t sb, int n) {
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    int i = 0;
#pragma unroll 4
    for (; i + 4 <= n; i += 4) {
        s0 = __fadd_rn(s0, __fmul_rn(x[i], y[i * sb]));
        s1 = __fadd_rn(s1, __fmul_rn(x[i + 1], y[(i + 1) * sb]));
        s2 = __fadd_rn(s2, __fmul_rn(x[i + 2], y[(i + 2) * sb]));
        s3 = __fadd_rn(s3, __fmul_rn(x[i + 3], y[(i + 3) * sb]));
    }
    for (; i < n; i++) s0 = __fadd_rn(s0, __fmul_rn(x[i], y[i * sb]));
    return __fadd_rn(__fadd_rn(__fadd_rn(s0, s1), s2), s3);
}

__device__ __forceinline__ float dot_avx_s(const float *x, const float *w, size_t sb, int kk) {
    float A[8], B[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) A[l] = B[l] = 0.f;
    for (int c = 0; c < kk; c += 16) {
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            A[l] = __fmaf_rn(x[c + l], w[(c + l) * sb], A[l]);
            B[l] = __fmaf_rn(x[c + 8 + l], w[(c + 8 + l) * sb], B[l]);
        }
    }
    float S[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) S[l] = __fadd_rn(A[l], B[l]);
    return hsum8(S);
}

__device__ __forceinline__ float dot_x4_s(const float *x, const float *w, size_t sb, int k) {
    const int kk = k & ~15;
    float o = kk > 0 ? dot_avx_s(x, w, sb, kk) : 0.f;
    if (kk < k) o = __fadd_rn(o, dot_go_s(x + kk, w + kk * sb, sb, k - kk));
    return o;
}

// dot_x4_s (x4) or dot_go_s of one output by a group of 8 lanes (lane q
// of the group; all 8 call it together): lane q runs dot4f32avx's
// accumulators A[q] and B[q] (elements c+q and c+8+q of each 16, in order)
// and S[q] = A[q] + B[q], the group's shuffles add the S as hsum8 does
// ((S0+S4 + S1+S5) + (S2+S6 + S3+S7)); lanes 0..3 run dotF32Go's four sums
// over the tail (the whole row without x4), the rest into the first.  The
// result is lane 0's.
__device__ __forceinline__ float dot8_s(const float *x, const float *w, size_t sb, int k, bool x4, int q) {
    float o = 0.f;
    int kk = 0;
    if (x4) {
        kk = k & ~15;
        float A = 0.f, B = 0.f;
        for (int c = 0; c < kk; c += 16) {
            A = __fmaf_rn(x[c + q], w[(size_t)(c + q) * sb], A);
            B = __fmaf_rn(x[c + 8 + q], w[(size_t)(c + 8 + q) * sb], B);
        }
        float t = __fadd_rn(A, B);                   // S[q]
        t = __fadd_rn(t, __shfl_down(t, 4, 8));      // S[q] + S[q+4]
        t = __fadd_rn(t, __shfl_down(t, 1, 8));      // q = 0: h0 + h1, q = 2: h2 + h3
        t = __fadd_rn(t, __shfl_down(t, 2, 8));      // q = 0: the sum
        o = kk > 0 ? t : 0.f;
        if (kk == k) return o;
    }
    const int n = k - kk, n4 = n & ~3;
    const float *xt = x + kk, *wt = w + (size_t)kk * sb;
    float s = 0.f;
    if (q < 4) {
        for (int i = q; i < n4; i += 4) s = __fadd_rn(s, __fmul_rn(xt[i], wt[(size_t)i * sb]));
        if (q == 0)
            for (int i = n4; i < n; ++i) s = __fadd_rn(s, __fmul_rn(xt[i], wt[(size_t)i * sb]));
    }
    const float s1 = __shfl_down(s, 1, 8), s2 = __shfl_down(s, 2, 8), s3 = __shfl_down(s, 3, 8);
    const float go = __fadd_rn(__fadd_rn(__fadd_rn(s, s1), s2), s3);
    return x4 ? __fadd_rn(o, go) : go;
}

// One output (row r of m, column j of n) of MatMulF32 (internal/kern/
// kern.go:205-212 over gemm.go:116-259) with no bias: for m > 16 the rows in
// whole groups of six take k6x16avx (kernels_amd64.s:5-88: acc = fma(a, b,
// acc) over k in chunks of 256, each chunk's acc added to C from 0), the
// other rows gemvRows (dotF32x4 for whole groups of four columns, dotF32Go
// for the rest).  a is contiguous; b's elements are sb apart.
__device__ __forceinline__ float matmul_f32_one(const float *a, const float *b, size_t sb, int k, int r, int m, int j,
                                                int n) {
    if (m > 16 && r < m / 6 * 6) {
        float c = 0.f;
        for (int k0 = 0; k0 < k; k0 += 256) {
            const int kn = min(256, k - k0);
            float acc = 0.f;
#pragma unroll 16
            for (int kk = 0; kk < kn; ++kk) acc = __fmaf_rn(a[k0 + kk], b[(size_t)(k0 + kk) * sb], acc);
            c = __fadd_rn(acc, c);
        }
        return c;
    }
    return j < (n & ~3) ? dot_x4_s(a, b, sb, k) : dot_go_s(a, b, sb, k);
}
